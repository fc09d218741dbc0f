"""Host history from the reference's raw-store session snapshot
(RawKvStore::snapshot_write, raw_kv_store.cpp:1225-1247): the reference's own
store writes the snapshot (oracle/_ref), the library's reader
(kvm_snapshot_read_layer) hands back every layer's rows, token counts and
mean-K sums, and refuses the inputs the reference reader refuses.  Host-side
parsing only: no GPU is needed."""
import numpy as np
import pytest

import oracle as O
from kvmem_amd import api

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs the reference sources)")

N_LAYER, H, D, BT = 2, 2, 128, 128
E = H * D
K_ROW, V_ROW = E // 32 * 34, E // 32 * 18          # q8_0 K row, q4_0 V row


def _store(seed, n_tokens, chunk):
    rng = np.random.default_rng(seed)
    k_rows = rng.integers(0, 256, (N_LAYER, n_tokens, K_ROW), dtype=np.uint8)
    v_rows = rng.integers(0, 256, (N_LAYER, n_tokens, V_ROW), dtype=np.uint8)
    k_f32 = rng.standard_normal((N_LAYER, n_tokens, E)).astype(np.float32)
    snap = O.ref_raw_snapshot(k_rows, k_f32, v_rows, E, E, BT, chunk)
    return snap, k_rows, v_rows, k_f32


@needs_ref
@pytest.mark.parametrize("n_tokens,chunk", [(3 * BT + 77, 50), (2 * BT, BT), (5, 3)])
def test_snapshot_layers_match_the_store(n_tokens, chunk):
    snap, k_rows, v_rows, k_f32 = _store(n_tokens, n_tokens, chunk)
    info, layers = api.read_snapshot(snap)
    nb = (n_tokens + BT - 1) // BT
    assert (info["n_layer"], info["n_embd_k"], info["n_embd_v"], info["block_tokens"]) == (N_LAYER, E, E, BT)
    assert (info["k_row_bytes"], info["v_gpu_row_bytes"], info["n_blocks"]) == (K_ROW, V_ROW, nb)
    want_nt = np.array([min(BT, n_tokens - b * BT) for b in range(nb)], np.uint32)
    for il, ly in enumerate(layers):
        assert np.array_equal(ly["k_rows"][:n_tokens], k_rows[il])
        assert np.array_equal(ly["v_rows"][:n_tokens], v_rows[il])
        assert not ly["k_rows"][n_tokens:].any() and not ly["v_rows"][n_tokens:].any()
        assert np.array_equal(ly["n_tokens"], want_nt)
        assert np.array_equal(ly["mean_tokens"], want_nt)
        # the store's mean-K sums: ordered fp32 sums in token order (raw_kv_store.cpp:215-234),
        # the same the reference's mean_k divides (987-1054)
        for b in range(nb):
            acc = np.zeros(E, np.float32)
            for t in range(b * BT, b * BT + int(want_nt[b])):
                acc = acc + k_f32[il, t]
            assert np.array_equal(ly["k_sum"][b], acc), (il, b)
            mean = ly["k_sum"][b] * (np.float32(1.0) / np.float32(want_nt[b]))
            assert np.array_equal(mean, O.ref_mean_k(k_f32[il, b * BT:b * BT + int(want_nt[b])], BT, chunk)[0])


@needs_ref
def test_snapshot_reader_refuses_what_the_reference_refuses():
    snap, *_ = _store(9, BT + 10, 64)
    api.read_snapshot(snap)                                          # intact: reads
    bad = bytearray(snap)
    bad[0] ^= 1
    with pytest.raises(RuntimeError):                                # magic
        api.read_snapshot(bytes(bad))
    with pytest.raises(RuntimeError):                                # truncated
        api.read_snapshot(snap[:len(snap) - 5])
    with pytest.raises(RuntimeError):                                # more blocks than allowed
        api.read_snapshot(snap, max_blocks=1)
    bad = bytearray(snap)
    hdr = 4 + 4 * 4 + 3 * 8 + 8                                      # header, then the block's section length
    bad[hdr + 8:hdr + 12] = np.uint32(BT + 1).tobytes()              # first layer's n_tokens above the block
    with pytest.raises(RuntimeError):
        api.read_snapshot(bytes(bad))
    bad = bytearray(snap)
    bad[hdr:hdr + 8] = np.uint64(np.frombuffer(snap[hdr:hdr + 8], np.uint64)[0] + 1).tobytes()
    with pytest.raises(RuntimeError):                                # section length disagrees
        api.read_snapshot(bytes(bad))
