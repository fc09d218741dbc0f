"""GPU row codecs and the tiled window against the oracle (bit-exact)."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import dev, host, rand_rows
from kvmem_amd import api, _lib as L

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ty", [L.T_Q8_0, L.T_Q4_0, L.T_F16])
def test_quantize_rows_bit_exact(kvm_state, ty):
    rng = np.random.default_rng(ty)
    x = (rng.standard_normal((300, 256)) * np.float32(10.0) ** rng.integers(-3, 3, (300, 1))).astype(np.float32)
    x[0] = 0.0
    x[1, :32] = 0.5 * np.arange(32)          # exact halfway products
    got = host(api.quantize_rows(kvm_state, ty, dev(x)))
    if ty == L.T_F16:
        want = x.astype(np.float16).view(np.uint8).reshape(300, -1)
    else:
        want = O.quant(ty, x.reshape(-1)).reshape(300, -1)
    assert np.array_equal(got, want)
    back = host(api.dequantize_rows(kvm_state, ty, dev(got), 256))
    if ty == L.T_F16:
        assert np.array_equal(back, want.view(np.float16).astype(np.float32).reshape(300, 256))
    else:
        assert np.array_equal(back.reshape(-1), O.dequant(ty, want.reshape(-1), x.size))


@pytest.mark.parametrize("kt,vt,d", [(L.T_Q8_0, L.T_Q4_0, 256), (L.T_Q8_0, L.T_Q4_0, 128),
                                     (L.T_F16, L.T_F16, 128), (L.T_Q4_0, L.T_Q4_0, 256),
                                     (L.T_Q4_0, L.T_Q4_0, 128)])
def test_window_import_export_round_trip(kvm_state, kt, vt, d):
    rng = np.random.default_rng(d + kt)
    H, n_cells = 4, 512
    w = api.KVWindow(kvm_state, n_cells, H, d, 128, kt, vt)
    kr, vr = rand_rows(rng, n_cells, H, d, kt, vt)
    w.import_rows(0, dev(kr), dev(vr), dev(np.arange(n_cells, dtype=np.int32)))
    # overwrite a range that starts and ends inside tiles; the rest must keep its bytes
    kr2, vr2 = rand_rows(rng, 77, H, d, kt, vt)
    w.import_rows(101, dev(kr2), dev(vr2))
    kr[101:178], vr[101:178] = kr2, vr2
    ek, ev = w.export_rows(0, n_cells)
    assert np.array_equal(host(ek), kr)
    assert np.array_equal(host(ev), vr)
    assert np.array_equal(host(w.cell_pos), np.arange(n_cells))
    w.reset()
    assert np.all(host(w.cell_pos) == -1) and np.all(host(w.slot_block) == -1)


def test_d2d_batched(kvm_state):
    import ctypes as C
    a = torch.arange(1 << 16, dtype=torch.uint8, device="cuda")
    b = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    srcs = (C.c_void_p * 3)(a.data_ptr(), a.data_ptr() + 100, a.data_ptr() + 4096)
    dsts = (C.c_void_p * 3)(b.data_ptr() + 50000, b.data_ptr() + 7, b.data_ptr() + 60000)
    ns = (C.c_size_t * 3)(4096, 33, 1024)
    kvm_state.check(kvm_state.lib.kvm_d2d_batched(kvm_state.h, srcs, dsts, ns, 3))
    torch.cuda.synchronize()
    ah, bh = host(a), host(b)
    assert np.array_equal(bh[50000:54096], ah[:4096])
    assert np.array_equal(bh[7:40], ah[100:133])
    assert np.array_equal(bh[60000:61024], ah[4096:5120])


def test_d2d_batched_alignments_and_sizes(kvm_state):
    """kvm_d2d_batched (kvmem_d2d_batched, llama-kvmem-stagein.cu:236-261) over
    every alignment of source and destination modulo 16, sizes from 0 to past
    several 16 KiB chunks, and a block-sized move (128 rows of 1,088 bytes);
    bytes outside the destinations stay untouched."""
    import ctypes as C
    rng = np.random.default_rng(52)
    a = torch.from_numpy(rng.integers(0, 256, 1 << 21, dtype=np.uint8)).cuda()
    b = torch.zeros(1 << 21, dtype=torch.uint8, device="cuda")
    ops, pos = [], 0
    sizes = [0, 1, 15, 16, 17, 63, 64, 1000, 16383, 16384, 16385, 50001, 128 * 1088]
    for k in range(48):
        n = sizes[k % len(sizes)]
        so, do = int(rng.integers(0, 1 << 20)), pos + (k * 7) % 16
        ops.append((so, do, n))
        pos = do + n + 64
    assert pos < b.numel()
    srcs = (C.c_void_p * len(ops))(*[a.data_ptr() + so for so, _, _ in ops])
    dsts = (C.c_void_p * len(ops))(*[b.data_ptr() + do for _, do, _ in ops])
    ns = (C.c_size_t * len(ops))(*[n for _, _, n in ops])
    kvm_state.check(kvm_state.lib.kvm_d2d_batched(kvm_state.h, srcs, dsts, ns, len(ops)))
    torch.cuda.synchronize()
    ah, bh = host(a), host(b)
    want = np.zeros_like(bh)
    for so, do, n in ops:
        want[do:do + n] = ah[so:so + n]
    assert np.array_equal(bh, want)
