"""GPU stage-in (pinned host history -> tiled window with RoPE re-applied at the
window position, Walsh-Hadamard and q8_0 requantisation) against the oracle,
byte for byte."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import dev, golden_snapshot, host, rand_rows
from kvmem_amd import api, _lib as L

pytestmark = pytest.mark.gpu


def _history(seed, n_tokens, H=4, D=256):
    rng = np.random.default_rng(seed)
    kr, vr = rand_rows(rng, n_tokens, H, D, L.T_Q8_0, L.T_Q4_0)
    return api.History(kr, vr), kr, vr


@pytest.mark.parametrize("D,n_rot,hadamard,freq_base", [
    (256, 64, -1, 1e7), (256, 64, 0, 1e7), (256, 128, 128, 1e4), (256, 32, -1, 1e4), (256, 256, 256, 1e4),
    (128, 64, -1, 1e7), (128, 128, 128, 1e4), (128, 32, 0, 1e7),
    # RoPE pairs not one dim bit >= 4 apart (n_half 12, 8): the one-row-per-wave path
    (256, 24, -1, 1e7), (256, 16, 64, 1e7),
    # 16-lane rows with a Hadamard width below the head (64: its pre-scale 1/8 rides on the block scale)
    (256, 64, 64, 1e7)])
def test_stagein_selection_bytes(kvm_state, D, n_rot, hadamard, freq_base):
    H, bt = 4, 128
    n_blocks = 40
    n_hist = n_blocks * bt - 50                     # last block is partial (78 tokens)
    hist, kr, vr = _history(n_rot + hadamard, n_hist, H, D)
    w = api.KVWindow(kvm_state, 16 * bt, H, D, bt)
    rng = np.random.default_rng(5)
    s = rng.standard_normal(n_blocks)
    s[n_blocks - 1] = 10.0                          # select the partial block too
    nt = np.array([min(bt, n_hist - b * bt) for b in range(n_blocks)], np.int32)
    sel = api.select_topk(kvm_state, dev(s), dev(nt), 12, 1, 0, None, window=w)
    api.stagein_selection(kvm_state, hist, w, sel, n_rot, freq_base, 1.0, hadamard)
    res = sel.result()
    assert res["status"] == 0 and len(res["ids"]) == 12 and list(res["stage_slots"]) == list(range(12))
    nrot = D if hadamard == -1 else hadamard
    theta = O.rope_theta(freq_base, 1.0, n_rot)
    ek, ev = w.export_rows(0, 12 * bt)
    ek, ev = host(ek), host(ev)
    cp = host(w.cell_pos)
    for k, (bid, base) in enumerate(zip(res["ids"], res["to_base"])):
        n = int(nt[bid])
        packed = kr[bid * bt:bid * bt + n]
        want = O.stagein_k(packed.reshape(-1), n, H, D, n_rot, nrot, int(base), theta).reshape(n, -1)
        assert np.array_equal(ek[k * bt:k * bt + n], want), (k, bid)
        assert np.array_equal(ev[k * bt:k * bt + n], vr[bid * bt:bid * bt + n])
        assert np.array_equal(cp[k * bt:k * bt + n], np.arange(base, base + n))
        assert np.all(cp[k * bt + n:(k + 1) * bt] == -1)
    assert list(host(w.slot_block)[:12]) == list(res["ids"])
    assert list(host(w.slot_base)[:12]) == list(res["to_base"])
    # the same retrieval again stages nothing
    sel2 = api.select_topk(kvm_state, dev(s), dev(nt), 12, 1, 0, None, window=w)
    assert len(sel2.result()["stage_slots"]) == 0


def test_stagein_from_reference_snapshot(kvm_state):
    """The host history format end to end: a session snapshot written by the
    reference's RawKvStore holding q8_0 K / q4_0 V rows (tests/golden/
    snap_stagein.bin.gz), read by kvm_snapshot_read_layer into the history; the
    stage-in of a selection from it equals the oracle's bytes for the original
    rows."""
    snap, meta, kr, vr, _ = golden_snapshot("snap_stagein")
    H, D, bt, n_blocks = meta["n_head_kv"], meta["head_dim"], meta["block_tokens"], meta["n_blocks"]
    kr, vr = kr[0], vr[0]
    n_hist = kr.shape[0]
    info, layers = api.read_snapshot(snap)
    assert info["n_blocks"] == n_blocks
    assert np.array_equal(layers[0]["k_rows"][:n_hist], kr) and np.array_equal(layers[0]["v_rows"][:n_hist], vr)
    hist = api.History(layers[0]["k_rows"][:n_hist], layers[0]["v_rows"][:n_hist])
    w = api.KVWindow(kvm_state, 4 * bt, H, D, bt)
    s = np.random.default_rng(7).standard_normal(n_blocks)
    s[n_blocks - 1] = 10.0                          # the partial last block too
    nt = layers[0]["n_tokens"].astype(np.int32)
    sel = api.select_topk(kvm_state, dev(s), dev(nt), 4, 1, 0, None, window=w)
    api.stagein_selection(kvm_state, hist, w, sel, 64, 1e7)
    res = sel.result()
    assert res["status"] == 0 and n_blocks - 1 in res["ids"]
    theta = O.rope_theta(1e7, 1.0, 64)
    ek, ev = w.export_rows(0, 4 * bt)
    ek, ev = host(ek), host(ev)
    for k, (bid, base) in enumerate(zip(res["ids"], res["to_base"])):
        n = int(nt[bid])
        want = O.stagein_k(kr[bid * bt:bid * bt + n].reshape(-1), n, H, D, 64, 256, int(base), theta).reshape(n, -1)
        assert np.array_equal(ek[k * bt:k * bt + n], want), (k, bid)
        assert np.array_equal(ev[k * bt:k * bt + n], vr[bid * bt:bid * bt + n])


def test_stagein_reselect_moves_only_changed_slots(kvm_state):
    H, D, bt, n_blocks = 4, 256, 128, 30
    hist, kr, vr = _history(9, n_blocks * bt, H, D)
    w = api.KVWindow(kvm_state, 8 * bt, H, D, bt)
    nt = dev(np.full(n_blocks, bt, np.int32))
    s = np.zeros(n_blocks)
    s[[3, 7, 20]] = [3, 2, 1]
    sel = api.select_topk(kvm_state, dev(s), nt, 4, 1, 0, None, window=w)
    api.stagein_selection(kvm_state, hist, w, sel, 64, 1e7)
    s[3], s[25] = 0, 5                               # block 3 leaves, block 25 enters; later slots shift
    sel = api.select_topk(kvm_state, dev(s), nt, 4, 1, 0, None, window=w)
    res = sel.result()
    assert list(res["ids"]) == [0, 7, 20, 25]
    assert list(res["stage_slots"]) == [1, 2, 3]     # slot 0 (sink at base 0) stays
    api.stagein_selection(kvm_state, hist, w, sel, 64, 1e7)
    ek, _ = w.export_rows(0, 4 * bt)
    theta = O.rope_theta(1e7, 1.0, 64)
    for k, bid in enumerate(res["ids"]):
        want = O.stagein_k(kr[bid * bt:(bid + 1) * bt].reshape(-1), bt, H, D, 64, 256, k * bt, theta)
        assert np.array_equal(host(ek)[k * bt:(k + 1) * bt].reshape(-1), want)


def test_stagein_lanes_match_single_lane(kvm_state):
    """Three lanes (different kv-head counts, histories, budgets and a partial
    last block) staged in one launch leave every window, cell position and slot
    map byte-equal to single-lane stage-ins, and lane 0 equal to the oracle."""
    D, bt = 256, 128
    cases = [(4, 40, 12, 16), (2, 25, 6, 8), (4, 60, 16, 20)]      # (H, n_blocks, budget, window slots)
    lanes, single, ref = [], [], []
    for i, (H, n_blocks, budget, slots) in enumerate(cases):
        n_hist = n_blocks * bt - (37 if i == 2 else 0)
        hist, kr, vr = _history(30 + i, n_hist, H, D)
        rng = np.random.default_rng(40 + i)
        s = rng.standard_normal(n_blocks)
        s[n_blocks - 1] = 10.0
        nt = dev(np.array([min(bt, n_hist - b * bt) for b in range(n_blocks)], np.int32))
        pair = []
        for _ in range(2):
            w = api.KVWindow(kvm_state, slots * bt, H, D, bt)
            sel = api.select_topk(kvm_state, dev(s), nt, budget, 1, 0, None, window=w)
            pair.append((hist, w, sel))
        lanes.append(pair[0])
        single.append(pair[1])
        ref.append((kr, vr, nt, H))
    api.stagein_selection_lanes(kvm_state, lanes, 64, 1e7)
    for h1, w1, sel1 in single:
        api.stagein_selection(kvm_state, h1, w1, sel1, 64, 1e7)
    for (_, w, sel), (_, w1, sel1) in zip(lanes, single):
        for name in ("k", "v", "cell_pos", "slot_block", "slot_base"):
            assert torch.equal(getattr(w, name), getattr(w1, name)), name
        assert sel.result()["status"] == 0
    kr, vr, nt, H = ref[0]
    _, w, sel = lanes[0]
    res = sel.result()
    theta = O.rope_theta(1e7, 1.0, 64)
    ek, ev = w.export_rows(0, len(res["ids"]) * bt)
    for k, (bid, base) in enumerate(zip(res["ids"], res["to_base"])):
        want = O.stagein_k(kr[bid * bt:(bid + 1) * bt].reshape(-1), bt, H, D, 64, 256, int(base), theta)
        assert np.array_equal(host(ek)[k * bt:(k + 1) * bt].reshape(-1), want), k
        assert np.array_equal(host(ev)[k * bt:(k + 1) * bt], vr[bid * bt:(bid + 1) * bt])
    # bad lane sets are refused before any launch
    with pytest.raises(L.KvmError):
        api.stagein_selection_lanes(kvm_state, [lanes[0]] * 9, 64, 1e7)            # more than 8 lanes
    w128 = api.KVWindow(kvm_state, 256, 4, 128, 128)
    sel128 = api.SelectionBuffers(kvm_state, 2, 2)
    with pytest.raises(L.KvmError):
        api.stagein_selection_lanes(kvm_state, [lanes[0], (lanes[0][0], w128, sel128)], 64, 1e7)


@pytest.mark.parametrize("kt", [L.T_Q8_0, L.T_Q4_0], ids=["q8_0", "q4_0"])
def test_enqueue_flush_api(kvm_state, kt):
    """Reference-shaped item API (llama-kvmem-stagein.h:36-46) at arbitrary
    cells, q8_0 and q4_0 K rows; rows of another type than the window's are
    refused."""
    H, D = 4, 256
    rng = np.random.default_rng(10)
    w = api.KVWindow(kvm_state, 512, H, D, 128, kt, L.T_Q4_0)
    kr, vr = rand_rows(rng, 100, H, D, kt, L.T_Q4_0)
    theta = O.rope_theta(1e7, 1.0, 64)
    lib = kvm_state.lib
    items = [(0, 30, 500), (30, 70, 7)]             # (row0, n, pos0)
    cells = [3, 200]
    for (r0, n, pos0), c0 in zip(items, cells):
        kb = np.ascontiguousarray(kr[r0:r0 + n])
        vb = np.ascontiguousarray(vr[r0:r0 + n])
        kvm_state.check(lib.kvm_stagein_enqueue_k(kvm_state.h, kt, kb.ctypes.data_as(C.c_void_p), kb.nbytes,
                                                  C.byref(w.c), c0, n, H * D, 256, H, D, 64, pos0,
                                                  theta.ctypes.data_as(C.c_void_p), 32))
        kvm_state.check(lib.kvm_stagein_enqueue_v(kvm_state.h, vb.ctypes.data_as(C.c_void_p), vb.nbytes,
                                                  C.byref(w.c), c0, n))
    other = L.T_Q4_0 if kt == L.T_Q8_0 else L.T_Q8_0
    kb = np.ascontiguousarray(kr[:4])
    assert lib.kvm_stagein_enqueue_k(kvm_state.h, other, kb.ctypes.data_as(C.c_void_p), kb.nbytes, C.byref(w.c), 0, 4,
                                     H * D, 256, H, D, 64, 0, theta.ctypes.data_as(C.c_void_p), 32) == L.KVM_EUNSUPPORTED
    kvm_state.check(lib.kvm_stagein_flush(kvm_state.h))
    ek, ev = w.export_rows(0, 512)
    ek, ev = host(ek), host(ev)
    cp = host(w.cell_pos)
    for (r0, n, pos0), c0 in zip(items, cells):
        want = O.stagein_k(kr[r0:r0 + n].reshape(-1), n, H, D, 64, 256, pos0, theta, k_type=kt).reshape(n, -1)
        assert np.array_equal(ek[c0:c0 + n], want)
        assert np.array_equal(ev[c0:c0 + n], vr[r0:r0 + n])
        assert np.array_equal(cp[c0:c0 + n], np.arange(pos0, pos0 + n))


def test_enqueue_flush_mixed_hadamard_widths(kvm_state):
    """Items of Hadamard width 256, 128 and 0 queued into one flush are each
    rotated with their own 1/sqrt(width) scale."""
    H, D = 4, 256
    rng = np.random.default_rng(12)
    w = api.KVWindow(kvm_state, 512, H, D, 128)
    kr, _ = rand_rows(rng, 120, H, D, L.T_Q8_0, L.T_Q4_0)
    theta = O.rope_theta(1e7, 1.0, 64)
    lib = kvm_state.lib
    items = [(0, 40, 900, 256, 0), (40, 50, 11, 128, 100), (90, 30, 300, 0, 300)]   # (row0, n, pos0, width, cell0)
    for r0, n, pos0, nrot, c0 in items:
        kb = np.ascontiguousarray(kr[r0:r0 + n])
        kvm_state.check(lib.kvm_stagein_enqueue_k(kvm_state.h, L.T_Q8_0, kb.ctypes.data_as(C.c_void_p), kb.nbytes,
                                                  C.byref(w.c), c0, n, H * D, nrot, H, D, 64, pos0,
                                                  theta.ctypes.data_as(C.c_void_p), 32))
    kvm_state.check(lib.kvm_stagein_flush(kvm_state.h))
    ek, _ = w.export_rows(0, 512)
    ek = host(ek)
    for r0, n, pos0, nrot, c0 in items:
        want = O.stagein_k(kr[r0:r0 + n].reshape(-1), n, H, D, 64, nrot, pos0, theta).reshape(n, -1)
        assert np.array_equal(ek[c0:c0 + n], want), nrot


def test_stagein_rejects_bad_arguments(kvm_state):
    w = api.KVWindow(kvm_state, 256, 4, 256, 128)
    hist, _, _ = _history(11, 256)
    sel = api.SelectionBuffers(kvm_state, 2, 2)
    with pytest.raises(L.KvmError):
        api.stagein_selection(kvm_state, hist, w, sel, 7, 1e7)      # n_rot not a multiple of 8
    wf = api.KVWindow(kvm_state, 256, 4, 128, 128, L.T_F16, L.T_F16)
    with pytest.raises(L.KvmError):
        api.stagein_selection(kvm_state, hist, wf, sel, 64, 1e7)    # re-RoPE stage-in needs q8_0 K


def test_stagein_plan_that_does_not_fit_stages_nothing(kvm_state):
    """A selection larger than the window's slots (status 2) stages nothing:
    window bytes, cell positions and slot map are left as they were."""
    H, D, bt = 4, 256, 128
    hist, _, _ = _history(13, 20 * bt, H, D)
    w = api.KVWindow(kvm_state, 4 * bt, H, D, bt)              # 4 slots
    s = np.random.default_rng(2).standard_normal(20)
    sel = api.select_topk(kvm_state, dev(s), dev(np.full(20, bt, np.int32)), 8, 1, 0, None, window=w)
    assert sel.result()["status"] == 2
    before = [t.clone() for t in (w.k, w.v, w.cell_pos, w.slot_block, w.slot_base)]
    api.stagein_selection(kvm_state, hist, w, sel, 64, 1e7)
    torch.cuda.synchronize()
    for b, a in zip(before, (w.k, w.v, w.cell_pos, w.slot_block, w.slot_base)):
        assert torch.equal(a, b)


def test_stagein_block_outside_history(kvm_state):
    """A selected block past the end of the pinned history is skipped and
    flagged (status bit 4); the other blocks are staged byte for byte and the
    skipped slot keeps no live cells, also when it held another block before
    the reselect: its cells are emptied and its slot map entry cleared, so the
    next plan restages it."""
    H, D, bt = 4, 256, 128
    hist, kr, _ = _history(14, 10 * bt, H, D)                   # 10 blocks of history
    w = api.KVWindow(kvm_state, 8 * bt, H, D, bt)
    nt = dev(np.full(14, bt, np.int32))
    theta = O.rope_theta(1e7, 1.0, 64)
    s = np.zeros(14)
    s[[3, 9, 6]] = [3.0, 2.0, 1.0]
    sel = api.select_topk(kvm_state, dev(s), nt, 4, 1, 0, None, window=w)
    api.stagein_selection(kvm_state, hist, w, sel, 64, 1e7)
    assert list(sel.result()["ids"]) == [0, 3, 6, 9] and sel.result()["status"] == 0
    assert np.all(host(w.cell_pos)[3 * bt:4 * bt] >= 0)             # slot 3 holds block 9
    s[9], s[12] = 0.0, 2.0                                          # block 12 is past the history
    sel = api.select_topk(kvm_state, dev(s), nt, 4, 1, 0, None, window=w)
    assert list(sel.result()["ids"]) == [0, 3, 6, 12] and list(sel.result()["stage_slots"]) == [3]
    api.stagein_selection(kvm_state, hist, w, sel, 64, 1e7)
    assert sel.result()["status"] & 4
    ek, _ = w.export_rows(0, 3 * bt)
    for k, bid in enumerate([0, 3, 6]):
        want = O.stagein_k(kr[bid * bt:(bid + 1) * bt].reshape(-1), bt, H, D, 64, 256, k * bt, theta)
        assert np.array_equal(host(ek)[k * bt:(k + 1) * bt].reshape(-1), want), k
    assert np.all(host(w.cell_pos)[3 * bt:4 * bt] == -1)
    assert host(w.slot_block)[3] == -1 and host(w.slot_base)[3] == -1
    # the same selection again still plans slot 3 (its entry no longer claims block 12)
    sel = api.select_topk(kvm_state, dev(s), nt, 4, 1, 0, None, window=w)
    assert list(sel.result()["stage_slots"]) == [3]
    # and a selection of blocks in the history stages it byte for byte
    s[12], s[8] = 0.0, 2.0
    sel = api.select_topk(kvm_state, dev(s), nt, 4, 1, 0, None, window=w)
    api.stagein_selection(kvm_state, hist, w, sel, 64, 1e7)
    assert list(sel.result()["ids"]) == [0, 3, 6, 8] and sel.result()["status"] == 0
    ek, _ = w.export_rows(3 * bt, bt)
    want = O.stagein_k(kr[8 * bt:9 * bt].reshape(-1), bt, H, D, 64, 256, 3 * bt, theta)
    assert np.array_equal(host(ek).reshape(-1), want)
    assert np.array_equal(host(w.cell_pos)[3 * bt:4 * bt], np.arange(3 * bt, 4 * bt))


def test_select_topk_over_no_blocks(kvm_state):
    """A selection over an empty store (no scores, no token counts) selects
    nothing and stages nothing; the kernel reads a stand-in, not address 0."""
    w = api.KVWindow(kvm_state, 4 * 128, 4, 256, 128)
    empty = torch.empty(0, dtype=torch.float64, device="cuda")
    sel = api.select_topk(kvm_state, empty, torch.empty(0, dtype=torch.int32, device="cuda"), 4, 1, 0, None,
                          window=w)
    r = sel.result()
    assert len(r["ids"]) == 0 and r["total"] == 0 and len(r["stage_slots"]) == 0 and r["status"] == 0


def _retrieval(st, seed, n_blocks, H, D, n_head, bt=128):
    rng = np.random.default_rng(seed)
    ix = api.MeanKIndex(st, 1, n_blocks, H, D, bt)
    ix.set_block_sums(dev((rng.standard_normal((1, n_blocks, H * D)) * 128).astype(np.float32)))
    ix.mean_tokens[:, :n_blocks] = 128
    ix.present[:n_blocks] = 1
    qa = api.QueryAcc(st, 1, n_head, D)
    qa.q_sum.copy_(dev(rng.standard_normal((1, n_head * D)).astype(np.float32)))
    qa.q_count.copy_(dev(np.array([1], np.int32)))
    return ix, qa, rng


def _same_selection_and_window(sa, wa, sb, wb):
    ra, rb = sa.result(), sb.result()
    for key in ("ids", "to_base", "stage_slots"):
        assert np.array_equal(ra[key], rb[key]), key
    assert ra["total"] == rb["total"] and ra["status"] == rb["status"] == 0
    for name in ("k", "v", "cell_pos", "slot_block", "slot_base"):
        assert torch.equal(getattr(wa, name), getattr(wb, name)), name
    return ra


@pytest.mark.parametrize("H,n_head", [(4, 24), (5, 10)])
def test_score_topk_stagein_matches_two_calls(kvm_state, H, n_head):
    """The one-call retrieval + stage-in (at 4 and 5 kv heads) against
    kvm_score_topk + kvm_stagein_selection on a second window:
    a fresh window (full plan), a changed query (some slots restaged) and the
    same query again (empty plan) give equal selections and equal windows."""
    D, bt, n_blocks, budget, slots = 256, 128, 40, 12, 16
    ix, qa, rng = _retrieval(kvm_state, 60 + H, n_blocks, H, D, n_head)
    n_hist = n_blocks * bt - 30                                 # last block partial
    hist, kr, _ = _history(70 + H, n_hist, H, D)
    nt = dev(np.array([min(bt, n_hist - b * bt) for b in range(n_blocks)], np.int32))
    wa, wb = (api.KVWindow(kvm_state, slots * bt, H, D, bt) for _ in range(2))
    sa, sb = (api.SelectionBuffers(kvm_state, n_blocks, budget) for _ in range(2))
    staged = []
    for step in range(3):
        if step == 1:
            qa.q_sum.add_(dev((rng.standard_normal((1, n_head * D)) * 0.7).astype(np.float32)))
        api.score_topk_stagein(kvm_state, ix, qa, n_blocks, nt, budget, 1, 0, wa, sa, hist, 64, 1e7)
        api.score_topk(kvm_state, ix, qa, n_blocks, nt, budget, 1, 0, None, wb, sb)
        api.stagein_selection(kvm_state, hist, wb, sb, 64, 1e7)
        staged.append(len(_same_selection_and_window(sa, wa, sb, wb)["stage_slots"]))
    assert staged[0] == budget and 0 < staged[1] < budget and staged[2] == 0, staged
    res = sa.result()
    k = 5
    bid, base = int(res["ids"][k]), int(res["to_base"][k])
    theta = O.rope_theta(1e7, 1.0, 64)
    ek, _ = wa.export_rows(k * bt, bt)
    want = O.stagein_k(kr[bid * bt:(bid + 1) * bt].reshape(-1), bt, H, D, 64, 256, base, theta)
    assert np.array_equal(host(ek).reshape(-1), want)


def test_score_topk_stagein_lanes_matches_two_calls(kvm_state):
    """Three lanes (different histories and index sizes) in one fused launch
    pair against kvm_score_topk_lanes + kvm_stagein_selection_lanes."""
    H, D, n_head, bt, budget, slots = 4, 256, 24, 128, 10, 12
    fused, two = [], []
    for i, n_blocks in enumerate((20, 33, 48)):
        ix, qa, _ = _retrieval(kvm_state, 80 + i, n_blocks, H, D, n_head)
        hist, _, _ = _history(90 + i, n_blocks * bt, H, D)
        nt = dev(np.full(n_blocks, bt, np.int32))
        for group in (fused, two):
            group.append(dict(index=ix, query=qa, n_blocks=n_blocks, n_tokens=nt, budget_blocks=budget,
                              sink_blocks=1, window=api.KVWindow(kvm_state, slots * bt, H, D, bt),
                              sel=api.SelectionBuffers(kvm_state, n_blocks, budget), history=hist))
    for step in range(2):
        api.prepare_score_topk_stagein_lanes(kvm_state, fused, 64, 1e7)()
        api.score_topk_lanes(kvm_state, two)
        api.stagein_selection_lanes(kvm_state, [(ln["history"], ln["window"], ln["sel"]) for ln in two], 64, 1e7)
        for a, b in zip(fused, two):
            r = _same_selection_and_window(a["sel"], a["window"], b["sel"], b["window"])
            assert len(r["stage_slots"]) == (budget if step == 0 else 0)


@pytest.mark.parametrize("D,n_rot,hadamard", [(256, 64, -1), (256, 128, 0), (128, 32, -1), (256, 24, -1),
                                              (128, 16, 64), (256, 64, 128), (256, 64, 64)])
def test_stagein_selection_bytes_q4_0_k(kvm_state, D, n_rot, hadamard):
    """A q4_0 K cache: the history's raw K rows are q4_0 and the stage-in
    requantises to q4_0 (quant_q4_0, llama-kvmem-stagein.cu:201-234, in the
    chain of :731-786); the window holds them as q8_0 tile quants and exports
    the q4_0 rows the oracle's chain produces, byte for byte.  RoPE pairs 12 or
    8 dims apart (n_rot 24, 16) take the one-row-per-wave requantiser, the
    others the 16-lane one."""
    H, bt, n_blocks = 4, 128, 30
    n_hist = n_blocks * bt - 70
    rng = np.random.default_rng(D + n_rot)
    kr, vr = rand_rows(rng, n_hist, H, D, L.T_Q4_0, L.T_Q4_0)
    hist = api.History(kr, vr)
    w = api.KVWindow(kvm_state, 12 * bt, H, D, bt, L.T_Q4_0, L.T_Q4_0)
    s = rng.standard_normal(n_blocks)
    s[n_blocks - 1] = 10.0
    nt = np.array([min(bt, n_hist - b * bt) for b in range(n_blocks)], np.int32)
    sel = api.select_topk(kvm_state, dev(s), dev(nt), 10, 1, 0, None, window=w)
    api.stagein_selection(kvm_state, hist, w, sel, n_rot, 1e7, 1.0, hadamard)
    res = sel.result()
    assert res["status"] == 0 and len(res["ids"]) == 10
    nrot = D if hadamard == -1 else hadamard
    theta = O.rope_theta(1e7, 1.0, n_rot)
    ek, ev = w.export_rows(0, 10 * bt)
    ek, ev = host(ek), host(ev)
    for k, (bid, base) in enumerate(zip(res["ids"], res["to_base"])):
        n = int(nt[bid])
        want = O.stagein_k(kr[bid * bt:bid * bt + n].reshape(-1), n, H, D, n_rot, nrot, int(base), theta,
                           k_type=O.T_Q4_0).reshape(n, -1)
        assert np.array_equal(ek[k * bt:k * bt + n], want), (k, bid)
        assert np.array_equal(ev[k * bt:k * bt + n], vr[bid * bt:bid * bt + n])


