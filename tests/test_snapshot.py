"""Host history from the reference's raw-store session snapshot
(RawKvStore::snapshot_write, raw_kv_store.cpp:1225-1247): the reference's own
store writes the snapshot (oracle/_ref), the library's reader
(kvm_snapshot_read_layer) hands back every layer's rows, token counts and
mean-K sums, and refuses the inputs the reference reader refuses.  Host-side
parsing only: no GPU is needed."""
import numpy as np
import pytest

import oracle as O
from gpu_util import golden_snapshot
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
    # a store of max_blocks blocks reads a snapshot of max_blocks + 1 (the partly
    # filled tail block) and refuses more (raw_kv_store.cpp:1255-1256)
    api.read_snapshot(snap, max_blocks=1)
    with pytest.raises(RuntimeError):
        api.read_snapshot(snap, max_blocks=0)
    bad = bytearray(snap)
    hdr = 4 + 4 * 4 + 3 * 8 + 8                                      # header, then the block's section length
    bad[hdr + 8:hdr + 12] = np.uint32(BT + 1).tobytes()              # first layer's n_tokens above the block
    with pytest.raises(RuntimeError):
        api.read_snapshot(bytes(bad))
    bad = bytearray(snap)
    bad[hdr:hdr + 8] = np.uint64(np.frombuffer(snap[hdr:hdr + 8], np.uint64)[0] + 1).tobytes()
    with pytest.raises(RuntimeError):                                # section length disagrees
        api.read_snapshot(bytes(bad))


def _header(n_layer, n_embd_k, n_embd_v, bt, k_row, k_gpu_row, v_gpu_row, n_blocks):
    return (np.array([0x31564b52, n_layer, n_embd_k, n_embd_v, bt], np.uint32).tobytes() +
            np.array([k_row, k_gpu_row, v_gpu_row, n_blocks], np.uint64).tobytes())


def test_snapshot_reader_bounds_a_crafted_header():
    """Header fields whose products would wrap 64 bits are refused before any
    buffer is sized or written (block_tokens 1, k_row_bytes 2^63, 2 blocks:
    2 * 1 * 2^63 wraps to 0)."""
    lib = api.L.load()
    body = b"\0" * 64
    for hdr in (_header(1, 256, 256, 1, 1 << 63, 0, 0, 2),            # K row wider than fp32
                _header(1, 256, 256, 1 << 20, 512, 0, 0, 2),          # block of 2^20 rows
                _header(1, 1 << 30, 256, 128, 0, 0, 0, 2),            # n_embd_k past 2^20
                _header(1, 256, 256, 128, 512, 0, 1 << 62, 2)):       # V row wider than fp32
        buf = np.frombuffer(hdr + body, np.uint8)
        info = api.L.SnapshotInfo()
        assert lib.kvm_snapshot_info_read(None, buf.ctypes.data, buf.size, api.C.byref(info)) == api.L.KVM_EINVAL
        with pytest.raises(RuntimeError):
            api.read_snapshot(bytes(buf))


def test_snapshot_reader_expects_the_store_geometry():
    """With the store's configuration the reader refuses a snapshot of another
    geometry, as SnapshotReader::expect does (raw_kv_store.cpp:1251-1254)."""
    snap, meta, kr, vr, _ = golden_snapshot("snap_stagein")
    E = meta["n_head_kv"] * meta["head_dim"]
    want = dict(n_layer=1, n_embd_k=E, n_embd_v=E, block_tokens=meta["block_tokens"], k_row_bytes=E // 32 * 34,
                k_gpu_row_bytes=0, v_gpu_row_bytes=E // 32 * 18)
    api.read_snapshot(snap, expect=want)
    for field, value in (("n_layer", 2), ("block_tokens", 64), ("k_row_bytes", 0), ("v_gpu_row_bytes", 0)):
        with pytest.raises(RuntimeError):
            api.read_snapshot(snap, expect=dict(want, **{field: value}))


@pytest.mark.parametrize("name", ["snap_stagein", "snap_score"])
def test_committed_snapshots_read_back(name):
    """The committed snapshots (written by the reference's RawKvStore, see
    tests/golden/make_snapshots.py) hand back the rows the store was filled with
    and its ordered fp32 block sums, with no reference build present."""
    snap, meta, kr, vr, kf = golden_snapshot(name)
    info, layers = api.read_snapshot(snap)
    bt, n = meta["block_tokens"], kr.shape[1]
    assert info["n_blocks"] == meta["n_blocks"] and info["block_tokens"] == bt
    ly = layers[0]
    assert np.array_equal(ly["k_rows"][:n], kr[0]) and np.array_equal(ly["v_rows"][:n], vr[0])
    sums, mt = O.meank_sums(kf[0], bt)
    assert np.array_equal(ly["k_sum"].view(np.uint32), sums.view(np.uint32))
    assert np.array_equal(ly["mean_tokens"], mt) and np.array_equal(ly["n_tokens"], mt)
