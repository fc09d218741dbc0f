"""Oracle RoPE (rope.cpp:8-45), Walsh-Hadamard (llama-kvmem-stagein.cu:105-131)
and the fused K stage-in chain (stagein.cu:731-786)."""
import numpy as np
import pytest
import scipy.linalg

import oracle as O


def test_rope_pos0_identity_kat():
    """raw_kv_store_test.cpp:239-254: position 0 is the identity, position 1 is not."""
    theta = O.rope_theta(10000.0, 1.0, 4)
    src = np.array([1.0, 0.0, 1.0, 0.0], dtype=np.float32)
    assert np.array_equal(O.rope_neox(src, 1, 4, 4, 0, theta), src)
    out = O.rope_neox(src, 1, 4, 4, 1, theta)
    assert abs(out[0] - src[0]) > 1e-6 or abs(out[2] - src[2]) > 1e-6


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs the reference sources)")
@pytest.mark.parametrize("pos0", [0, 1, 977, 131072, 262000])
def test_rope_matches_reference_rope_neox_apply(pos0):
    """Against the reference's own host RoPE (libm cosf/sinf of the same fp32 angle):
    equal up to the last-ulp difference between cosf and cos-in-double."""
    rng = np.random.default_rng(pos0)
    n_head, d, n_rot = 4, 256, 64
    x = rng.standard_normal((16, n_head, d)).astype(np.float32)
    theta = O.rope_theta(1e7, 1.0, n_rot)
    ours = O.rope_neox(x, n_head, d, n_rot, pos0, theta)
    ref = O.ref_rope_neox(x, n_head, d, n_rot, 1e7, 1.0, pos0)
    assert np.array_equal(ours[..., n_rot:], x[..., n_rot:])          # pass-through dims
    np.testing.assert_allclose(ours, ref, rtol=0, atol=4e-6 * np.abs(x).max())


def test_rope_theta_formula():
    theta = O.rope_theta(1e7, 0.5, 64)
    i = np.arange(32, dtype=np.float32)
    want = (np.float32(1e7) ** (np.float32(-2.0) * i / np.float32(64))).astype(np.float32) * np.float32(0.5)
    np.testing.assert_allclose(theta, want, rtol=2e-7)
    assert theta[0] == np.float32(0.5)


def test_rope_rotation_properties():
    rng = np.random.default_rng(5)
    n_head, d, n_rot = 2, 128, 64
    x = rng.standard_normal((8, n_head, d)).astype(np.float32)
    theta = O.rope_theta(1e4, 1.0, n_rot)
    y = O.rope_neox(x, n_head, d, n_rot, 100, theta)
    h = n_rot // 2
    # each (i, i + n_rot/2) pair keeps its norm
    np.testing.assert_allclose(x[..., :h] ** 2 + x[..., h:n_rot] ** 2, y[..., :h] ** 2 + y[..., h:n_rot] ** 2,
                               rtol=1e-5, atol=1e-6)
    # float64 evaluation of the textbook rotation at positions 100 + t
    t = np.arange(8)[:, None, None] + 100
    ang = (t.astype(np.float32) * theta[None, None, :]).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    x0, x1 = x[..., :h].astype(np.float64), x[..., h:n_rot].astype(np.float64)
    np.testing.assert_allclose(y[..., :h], x0 * c - x1 * s, atol=1e-5)
    np.testing.assert_allclose(y[..., h:n_rot], x0 * s + x1 * c, atol=1e-5)
    # rotating by a then b equals rotating by a + b (up to rounding)
    z = O.rope_neox(O.rope_neox(x[:1], n_head, d, n_rot, 7, theta), n_head, d, n_rot, 30, theta)
    np.testing.assert_allclose(z, O.rope_neox(x[:1], n_head, d, n_rot, 37, theta), atol=2e-5)


@pytest.mark.parametrize("n", [64, 128, 256])
def test_fwht_is_normalised_hadamard(n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal((5, n)).astype(np.float32)
    H = scipy.linalg.hadamard(n).astype(np.float64) / np.sqrt(n)
    np.testing.assert_allclose(O.fwht(x, n), x.astype(np.float64) @ H.T, atol=2e-5)
    np.testing.assert_allclose(O.fwht(O.fwht(x, n), n), x, atol=2e-5)        # H^2 = I
    ones = np.ones(n, np.float32)
    e = O.fwht(ones, n)
    assert e[0] == np.float32(np.sqrt(n)) and np.all(e[1:] == 0)


def test_hadamard_width_rule():
    o = O.lib()
    assert [o.oracle_hadamard_nrot_k(d) for d in (64, 128, 192, 256, 320, 384)] == [64, 128, 64, 256, 64, 128]
    assert o.oracle_attn_rot_on(O.T_Q8_0, 256) == 1 and o.oracle_attn_rot_on(O.T_F16, 256) == 0
    assert o.oracle_attn_rot_on(O.T_Q8_0, 96) == 0


def _packed_k(rng, nt, n_head, d):
    x = rng.standard_normal((nt, n_head * d)).astype(np.float32)
    return O.quant(O.T_Q8_0, x.reshape(-1))


def test_stagein_identity_round_trip():
    """One token at position 0 with the Hadamard step off is the identity on q8_0
    blocks whose max |q| is 127 (quant(dequant(b)) == b)."""
    rng = np.random.default_rng(6)
    blocks = np.zeros((32, 34), np.uint8)
    q = rng.integers(-127, 128, (32, 32)).astype(np.int8)
    q[:, 0] = 127
    blocks[:, :2] = rng.uniform(0.01, 1, 32).astype(np.float16).view(np.uint8).reshape(32, 2)
    blocks[:, 2:] = q.view(np.uint8)
    packed = blocks.reshape(-1)                    # 1 token x 4 heads x 256 dims
    theta = O.rope_theta(1e7, 1.0, 64)
    assert np.array_equal(O.stagein_k(packed, 1, 4, 256, 64, 0, 0, theta), packed)


def test_stagein_chain_order():
    """stagein = quant(fwht(rope(dequant))) in this order; swapping RoPE and the
    Hadamard step gives different bytes."""
    rng = np.random.default_rng(7)
    nt, n_head, d, n_rot = 3, 4, 256, 64
    packed = _packed_k(rng, nt, n_head, d)
    theta = O.rope_theta(1e7, 1.0, n_rot)
    got = O.stagein_k(packed, nt, n_head, d, n_rot, 256, 1000, theta)
    f = O.dequant(O.T_Q8_0, packed, nt * n_head * d)
    want = O.quant(O.T_Q8_0, O.fwht(O.rope_neox(f, n_head, d, n_rot, 1000, theta), 256))
    assert np.array_equal(got, want)
    swapped = O.quant(O.T_Q8_0, O.rope_neox(O.fwht(f, 256), n_head, d, n_rot, 1000, theta))
    assert not np.array_equal(got, swapped)


def test_stagein_inverts_up_to_quantisation():
    """Dequant, inverse Hadamard (H itself) and RoPE at -pos recover the raw K
    within the two q8_0 roundings."""
    rng = np.random.default_rng(8)
    nt, n_head, d, n_rot, pos0 = 4, 4, 256, 64, 5000
    x = rng.standard_normal((nt, n_head * d)).astype(np.float32)
    packed = O.quant(O.T_Q8_0, x.reshape(-1))
    theta = O.rope_theta(1e7, 1.0, n_rot)
    staged = O.stagein_k(packed, nt, n_head, d, n_rot, 256, pos0, theta)
    y = O.fwht(O.dequant(O.T_Q8_0, staged, x.size), 256).reshape(nt, n_head, d)
    back = np.stack([O.rope_neox(y[t:t + 1], n_head, d, n_rot, -(pos0 + t), theta)[0] for t in range(nt)])
    ref = O.dequant(O.T_Q8_0, packed, x.size).reshape(nt, n_head, d)
    assert np.abs(back - ref).max() < 0.05


def test_stagein_q4_0_identity_and_inverse():
    """The q4_0 K chain (dequant_q4_0 -> RoPE -> FWHT -> quant_q4_0): one token
    at position 0 with the Hadamard step off gives back q4_0 blocks whose
    largest-magnitude quant is -8 (nibble 0) unchanged, since quant_q4_0 of
    their dequantised values reproduces them; and dequant, inverse Hadamard
    and RoPE at -pos recover the raw K within the two q4_0 roundings."""
    rng = np.random.default_rng(16)
    blocks = np.zeros((32, 18), np.uint8)
    nib = rng.integers(1, 16, (32, 32))                 # quants -7 .. 7 ...
    nib[:, 5] = 0                                      # ... and one -8 (vmax = -8 d)
    blocks[:, :2] = rng.uniform(0.01, 1, 32).astype(np.float16).view(np.uint8).reshape(32, 2)
    blocks[:, 2:] = (nib[:, :16] | (nib[:, 16:] << 4)).astype(np.uint8)
    packed = blocks.reshape(-1)                        # 1 token x 4 heads x 256 dims
    theta = O.rope_theta(1e7, 1.0, 64)
    assert np.array_equal(O.stagein_k(packed, 1, 4, 256, 64, 0, 0, theta, k_type=O.T_Q4_0), packed)
    nt, n_head, d, n_rot, pos0 = 4, 4, 256, 64, 3000
    x = rng.standard_normal((nt, n_head * d)).astype(np.float32)
    p4 = O.quant(O.T_Q4_0, x.reshape(-1))
    staged = O.stagein_k(p4, nt, n_head, d, n_rot, 256, pos0, theta, k_type=O.T_Q4_0)
    f = O.dequant(O.T_Q4_0, p4, x.size)
    assert np.array_equal(staged, O.quant(O.T_Q4_0, O.fwht(O.rope_neox(f, n_head, d, n_rot, pos0, theta), 256)))
    y = O.fwht(O.dequant(O.T_Q4_0, staged, x.size), 256).reshape(nt, n_head, d)
    back = np.stack([O.rope_neox(y[t:t + 1], n_head, d, n_rot, -(pos0 + t), theta)[0] for t in range(nt)])
    ref = f.reshape(nt, n_head, d)
    assert np.abs(back - ref).max() < 0.6 and np.abs(back - ref).mean() < 0.15
