"""Oracle codecs: IEEE half conversion (raw_kv_store.cpp:33-95) and the ggml
q8_0 / q4_0 block formats (llama-kvmem-stagein.cu:133-234)."""
import numpy as np
import pytest

import oracle as O


def test_f16_to_f32_exhaustive():
    o = O.lib()
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([o.oracle_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_round_nearest_even():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000).astype(np.float32),
        # exact halfway points between adjacent halves (ties to even), normal and subnormal
        (np.arange(0, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24),
        (np.arange(1024, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf, -np.inf, 5.96e-8, 2.98e-8, 2.99e-8],
                 dtype=np.float32)])
    got = O.f32_to_f16(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def _rand_q8_blocks(rng, nblk):
    b = np.zeros((nblk, 34), dtype=np.uint8)
    q = rng.integers(-127, 128, size=(nblk, 32)).astype(np.int8)
    q[np.arange(nblk), rng.integers(0, 32, nblk)] = rng.choice([-127, 127], nblk)   # max |q| = 127
    d = (rng.uniform(1e-3, 2.0, nblk)).astype(np.float16)
    b[:, 0:2] = d.view(np.uint8).reshape(nblk, 2)
    b[:, 2:] = q.view(np.uint8)
    return b


def test_q8_0_round_trip_bytes():
    """quant(dequant(b)) == b for blocks whose max |q| is 127: d' = 127 d / 127 = d exactly."""
    rng = np.random.default_rng(2)
    b = _rand_q8_blocks(rng, 4096)
    x = O.dequant(O.T_Q8_0, b.reshape(-1), 4096 * 32)
    assert np.array_equal(O.quant(O.T_Q8_0, x), b.reshape(-1))


def test_q4_0_round_trip_bytes():
    """A q4_0 block holding nibble 0 (value -8 d) has vmax = -8 d, so d' = d and every
    nibble is recovered by (int)(x / d + 8.5)."""
    rng = np.random.default_rng(3)
    n = 4096
    nib = rng.integers(0, 16, size=(n, 32))
    nib[np.arange(n), rng.integers(0, 32, n)] = 0
    d = rng.uniform(1e-3, 2.0, n).astype(np.float16)
    b = np.zeros((n, 18), dtype=np.uint8)
    b[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    b[:, 2:] = (nib[:, :16] | (nib[:, 16:] << 4)).astype(np.uint8)
    x = O.dequant(O.T_Q4_0, b.reshape(-1), n * 32)
    # element j of the block is nibble j (low) / j-16 (high) of byte j % 16
    assert np.array_equal(x.reshape(n, 32), ((nib - 8) * d.astype(np.float32)[:, None]).astype(np.float32))
    assert np.array_equal(O.quant(O.T_Q4_0, x), b.reshape(-1))


def test_q8_0_known_answers():
    x = np.zeros(64, dtype=np.float32)
    x[:32] = np.linspace(-1.0, 1.0, 32, dtype=np.float32)
    b = O.quant(O.T_Q8_0, x).reshape(2, 34)
    d = b[0, :2].view(np.float16)[0]
    assert d == np.float16(1.0 / 127.0)
    q = b[0, 2:].view(np.int8)
    assert q[0] == -127 and q[31] == 127
    # roundf ties away from zero: 0.5 * id rounds to +-1 when x*id is exactly +-0.5
    y = np.zeros(32, dtype=np.float32)
    y[0], y[1], y[2] = 127.0, 0.5, -0.5
    q2 = O.quant(O.T_Q8_0, y)[2:].view(np.int8)
    assert q2[0] == 127 and q2[1] == 1 and q2[2] == -1
    # an all-zero block has d = 0 and zero quants
    assert np.all(b[1] == 0)


def test_q4_0_known_answers():
    x = np.zeros(32, dtype=np.float32)
    x[3] = -4.0                     # largest magnitude: d = -4 / -8 = 0.5, id = 2, nibble 0
    x[4] = 3.0                      # (int)(3 * 2 + 8.5) = 14
    x[20] = 2.0                     # (int)(2 * 2 + 8.5) = 12, high nibble of byte 4
    b = O.quant(O.T_Q4_0, x)
    assert b[:2].view(np.float16)[0] == np.float16(0.5)
    q = b[2:]
    assert q[3] & 15 == 0 and q[4] & 15 == 14 and q[4] >> 4 == 12
    assert q[0] & 15 == 8           # zero -> nibble 8
    z = O.quant(O.T_Q4_0, np.zeros(32, np.float32))
    # vmax = 0 gives d = 0 / -8 = -0.0 (fp16 0x8000); every nibble is (int)(0 + 8.5) = 8
    assert z[:2].view(np.uint16)[0] == 0x8000 and np.all(z[2:] == 0x88)


def test_row_bytes():
    o = O.lib()
    assert o.oracle_row_bytes(O.T_Q8_0, 1024) == 1088
    assert o.oracle_row_bytes(O.T_Q4_0, 1024) == 576
    assert o.oracle_row_bytes(O.T_F16, 128) == 256
