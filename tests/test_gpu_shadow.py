"""Re-basing resident blocks from the window's HBM shadow.

A window with a K shadow keeps the raw (unrotated) q8_0 or q4_0 K rows of every
staged cell.  When a new plan moves a full block that the window already holds to
another slot (its window position changes), the stage-in re-rotates it from
that shadow and moves its V tiles within HBM; only blocks new to the window are
read from the host history.  Before each plan the tests poison the host rows of
every full block the window holds (and restore them after the plan's stage-in),
so any host read of such a block shows up, and compare
the whole window (K, V, positions, slot map) with a fresh stage-in of the same
plan from the clean history into a window without a shadow, byte for byte."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import dev, host, rand_rows
from kvmem_amd import api, _lib as L

pytestmark = pytest.mark.gpu

H, D, BT = 4, 256, 128
V_ROW = H * D // 32 * 18


def _k_row(kt):
    return H * D // 32 * (18 if kt == L.T_Q4_0 else 34)


def _histories(seed, n_tok, kt=L.T_Q8_0):
    rng = np.random.default_rng(seed)
    kr, vr = rand_rows(rng, n_tok, H, D, kt, L.T_Q4_0)
    return api.History(kr, vr), api.History(kr, vr), kr, vr, rng


def _poison(hist, blocks, rng):
    """Overwrite the host K and V rows of `blocks` (full blocks) with random bytes."""
    torch.cuda.synchronize()
    k = hist.kbuf.u8.reshape(hist.n_tokens, -1)
    v = hist.vbuf.u8.reshape(hist.n_tokens, V_ROW)
    for b in blocks:
        k[b * BT:(b + 1) * BT] = rng.integers(0, 256, (BT, k.shape[1]), dtype=np.uint8)
        v[b * BT:(b + 1) * BT] = rng.integers(0, 256, (BT, V_ROW), dtype=np.uint8)


def _restore(hist, blocks, kr, vr):
    """Put the clean rows of `blocks` back once the stage-in has run."""
    torch.cuda.synchronize()
    k = hist.kbuf.u8.reshape(hist.n_tokens, -1)
    v = hist.vbuf.u8.reshape(hist.n_tokens, V_ROW)
    for b in blocks:
        k[b * BT:(b + 1) * BT] = kr[b * BT:(b + 1) * BT]
        v[b * BT:(b + 1) * BT] = vr[b * BT:(b + 1) * BT]


def _resident_full(w, nt):
    """The full blocks the window holds: a stage-in must not read their host rows."""
    return sorted({int(b) for b in host(w.slot_block) if 0 <= int(b) < len(nt) and nt[int(b)] == BT})


def _same_window(wa, wb, n_used):
    for name in ("cell_pos", "slot_block", "slot_base"):
        assert torch.equal(getattr(wa, name), getattr(wb, name)), name
    ka, va = wa.export_rows(0, n_used)
    kb, vb = wb.export_rows(0, n_used)
    assert torch.equal(ka, kb) and torch.equal(va, vb)
    assert torch.equal(wa.k, wb.k) and torch.equal(wa.v, wb.v)


def _check_shadow(w, kr, res, nt):
    """The shadow holds each occupied slot's raw K rows and their count."""
    sh = host(w.k_shadow).reshape(w.n_cells, _k_row(w.k_type))
    rows = host(w.shadow_rows)
    for k, b in enumerate(res["ids"]):
        n = int(nt[b])
        assert rows[k] == n, (k, b)
        assert np.array_equal(sh[k * BT:k * BT + n], kr[b * BT:b * BT + n]), (k, b)


def _fresh(st, hist, s, nt, budget, slots, kt=L.T_Q8_0):
    w = api.KVWindow(st, slots * BT, H, D, BT, kt, L.T_Q4_0)
    sel = api.select_topk(st, dev(s), dev(nt), budget, 1, 0, None, window=w)
    api.stagein_selection(st, hist, w, sel, 64, 1e7)
    return w, sel.result()


@pytest.mark.parametrize("kt", [L.T_Q8_0, L.T_Q4_0], ids=["q8_0", "q4_0"])
def test_moved_blocks_restage_from_shadow(kvm_state, kt):
    """select_topk + stagein_selection (the gather launch, then the stage-in
    launch), over q8_0 and q4_0 K caches.  Plan 1 stages 12 of 40 blocks (the last, partly filled block
    among them).  Plan 2 drops an early block and adds a later one, so the
    blocks between shift down a slot; plan 3 adds an early block and drops a
    late one, so blocks shift up.  Moved full blocks name their old slot in
    stage_src and are not read from the host; the partly filled block and new
    blocks are (stage_src -1)."""
    st = kvm_state
    n_blocks, budget, slots = 40, 12, 16
    n_tok = n_blocks * BT - 30
    hp, hc, kr, vr, rng = _histories(0x5AD0, n_tok, kt)
    nt = np.array([min(BT, n_tok - b * BT) for b in range(n_blocks)], np.int32)
    w = api.KVWindow(st, slots * BT, H, D, BT, kt, L.T_Q4_0, shadow=True)
    assert w.k_shadow.numel() == slots * BT * _k_row(kt)
    s = rng.standard_normal(n_blocks)
    s[n_blocks - 1] = 10.0
    prev = None
    for step in range(4):
        if step == 1:
            ids = sorted(int(b) for b in prev["ids"])
            s[ids[2]] = -100.0                                    # an early block leaves
            s[next(b for b in range(ids[-2], n_blocks) if b not in ids)] = 100.0
        elif step == 2:
            ids = sorted(int(b) for b in prev["ids"])
            s[next(b for b in range(1, n_blocks) if b not in ids)] = 100.0    # the earliest free block joins
            s[ids[-3]] = -100.0
        old_block = host(w.slot_block).copy()
        held = _resident_full(w, nt)
        _poison(hp, held, rng)
        sel = api.select_topk(st, dev(s), dev(nt), budget, 1, 0, None, window=w)
        api.stagein_selection(st, hp, w, sel, 64, 1e7)
        _restore(hp, held, kr, vr)
        res = sel.result()
        assert res["status"] == 0
        ref_w, ref = _fresh(st, hc, s, nt, budget, slots, kt)
        assert np.array_equal(res["ids"], ref["ids"]) and np.array_equal(res["to_base"], ref["to_base"])
        _same_window(w, ref_w, budget * BT)
        _check_shadow(w, kr, res, nt)
        # stage_src: the old slot of each moved full block, else -1
        n_moved = 0
        for slot, src in zip(res["stage_slots"], res["stage_src"]):
            b = int(res["ids"][slot])
            held = np.nonzero(old_block == b)[0]
            if nt[b] == BT and len(held):
                assert src == held[0], (step, slot, b)
                n_moved += 1
            else:
                assert src == -1, (step, slot, b)
        if step == 0:
            assert len(res["stage_slots"]) == budget and n_moved == 0
        elif step in (1, 2):
            assert n_moved > 0 and len(res["stage_slots"]) > n_moved, (step, n_moved)
        else:
            assert len(res["stage_slots"]) == 0
        prev = res
    # the oracle on one moved block of the last plan that changed the window
    k = budget // 2
    b, base = int(res["ids"][k]), int(res["to_base"][k])
    ek, ev = w.export_rows(k * BT, BT)
    want = O.stagein_k(kr[b * BT:(b + 1) * BT].reshape(-1), BT, H, D, 64, 256, base, O.rope_theta(1e7, 1.0, 64),
                       k_type=kt)
    assert np.array_equal(host(ek).reshape(-1), want) and np.array_equal(host(ev), vr[b * BT:(b + 1) * BT])


def _retrieval(st, seed, n_blocks, n_head):
    rng = np.random.default_rng(seed)
    ix = api.MeanKIndex(st, 1, n_blocks, H, D, BT)
    ix.set_block_sums(dev((rng.standard_normal((1, n_blocks, H * D)) * 128).astype(np.float32)))
    ix.mean_tokens[:, :n_blocks] = BT
    ix.present[:n_blocks] = 1
    qa = api.QueryAcc(st, 1, n_head, D)
    qa.q_sum.copy_(dev(rng.standard_normal((1, n_head * D)).astype(np.float32)))
    qa.q_count.copy_(dev(np.array([1], np.int32)))
    return ix, qa, rng


@pytest.mark.parametrize("n_lanes", [1, 3])
def test_fused_retrieval_restages_from_shadow(kvm_state, n_lanes):
    """kvm_score_topk_stagein(_lanes), one and three lanes.  Queries drift over six steps; each lane's
    window (with a shadow, the host rows of the blocks it holds poisoned during
    each plan) equals kvm_score_topk + kvm_stagein_selection from the clean
    history into a window without a shadow."""
    st = kvm_state
    n_head, budget, slots = 24, 16, 20
    lanes, refs = [], []
    for i in range(n_lanes):
        n_blocks = 48 + 7 * i
        ix, qa, rng = _retrieval(st, 0x5AD1 + i, n_blocks, n_head)
        hp, hc, kr, vr, _ = _histories(0x5AE0 + i, n_blocks * BT)
        nt = dev(np.full(n_blocks, BT, np.int32))
        lanes.append(dict(index=ix, query=qa, n_blocks=n_blocks, n_tokens=nt, budget_blocks=budget, sink_blocks=1,
                          window=api.KVWindow(st, slots * BT, H, D, BT, shadow=True),
                          sel=api.SelectionBuffers(st, n_blocks, budget), history=hp))
        refs.append(dict(hc=hc, kr=kr, vr=vr, rng=rng, nt=np.full(n_blocks, BT, np.int32),
                         window=api.KVWindow(st, slots * BT, H, D, BT),
                         sel=api.SelectionBuffers(st, n_blocks, budget)))
    moved_total = 0
    for step in range(6):
        for ln, rf in zip(lanes, refs):
            if step:
                ln["query"].q_sum.add_(dev((rf["rng"].standard_normal((1, n_head * D)) * 0.5).astype(np.float32)))
        held = [_resident_full(ln["window"], rf["nt"]) for ln, rf in zip(lanes, refs)]
        for ln, rf, hb in zip(lanes, refs, held):
            _poison(ln["history"], hb, rf["rng"])
        if n_lanes == 1:
            ln = lanes[0]
            api.score_topk_stagein(st, ln["index"], ln["query"], ln["n_blocks"], ln["n_tokens"], budget, 1, 0,
                                   ln["window"], ln["sel"], ln["history"], 64, 1e7)
        else:
            api.prepare_score_topk_stagein_lanes(st, lanes, 64, 1e7)()
        for ln, rf, hb in zip(lanes, refs, held):
            _restore(ln["history"], hb, rf["kr"], rf["vr"])
        for ln, rf in zip(lanes, refs):
            api.score_topk(st, ln["index"], ln["query"], ln["n_blocks"], ln["n_tokens"], budget, 1, 0, None,
                           rf["window"], rf["sel"])
            api.stagein_selection(st, rf["hc"], rf["window"], rf["sel"], 64, 1e7)
            ra, rb = ln["sel"].result(), rf["sel"].result()
            for key in ("ids", "to_base", "stage_slots"):
                assert np.array_equal(ra[key], rb[key]), (step, key)
            _same_window(ln["window"], rf["window"], budget * BT)
            moved_total += int((ra["stage_src"] >= 0).sum())
    assert moved_total > 0


def test_import_voids_the_slot_shadow(kvm_state):
    """Rows imported into a slot's cells (a new token's K/V, a slot copied in
    from the host) are not in the shadow: the slot's shadow count drops to 0
    and a later move of its block reads the host history."""
    st = kvm_state
    n_blocks, budget, slots = 16, 6, 8
    hp, _, kr, vr, rng = _histories(0x5AF0, n_blocks * BT)
    nt = np.full(n_blocks, BT, np.int32)
    w = api.KVWindow(st, slots * BT, H, D, BT, shadow=True)
    s = np.arange(n_blocks, dtype=np.float64)
    s[[1, 2, 3]] = 100.0
    sel = api.select_topk(st, dev(s), dev(nt), budget, 1, 0, None, window=w)
    api.stagein_selection(st, hp, w, sel, 64, 1e7)
    r1 = sel.result()
    assert list(host(w.shadow_rows)[:budget]) == [BT] * budget
    assert list(r1["ids"]) == [0, 1, 2, 3, 14, 15]
    # a row re-imported into slot 2 (block 2) voids that slot's shadow only
    ek, ev = w.export_rows(2 * BT + 5, 1)
    w.import_rows(2 * BT + 5, ek, ev)
    rows = host(w.shadow_rows)
    assert rows[2] == 0 and all(rows[k] == BT for k in range(budget) if k != 2)
    # block 1 leaves and block 13 joins: blocks 2 and 3 move down one slot
    s[1] = -100.0
    sel = api.select_topk(st, dev(s), dev(nt), budget, 1, 0, None, window=w)
    r2 = sel.result()
    assert list(r2["ids"]) == [0, 2, 3, 13, 14, 15]
    src = dict(zip(r2["stage_slots"].tolist(), r2["stage_src"].tolist()))
    assert src == {1: -1, 2: 3, 3: -1}        # block 2 from the host (its shadow was voided), 13 is new
    api.stagein_selection(st, hp, w, sel, 64, 1e7)
    ref_w, ref = _fresh(st, hp, s, nt, budget, slots)
    _same_window(w, ref_w, budget * BT)
    # a window reset empties the shadow counts
    w.reset()
    assert not host(w.shadow_rows).any()


def test_shadow_geometry_is_checked(kvm_state):
    """A shadow needs its row counts (and the other way round) and a q8_0 or
    q4_0 K cache; a q4_0 shadow holds 18-byte blocks."""
    w = api.KVWindow(kvm_state, 256, H, D, BT, shadow=True)
    lib = kvm_state.lib
    import ctypes as C
    c = L.Window.from_buffer_copy(w.c)
    c.shadow_rows = None
    assert lib.kvm_window_check(C.byref(c)) == L.KVM_EINVAL
    c = L.Window.from_buffer_copy(w.c)
    c.k_shadow = None
    assert lib.kvm_window_check(C.byref(c)) == L.KVM_EINVAL
    wf = api.KVWindow(kvm_state, 256, H, 128, BT, L.T_F16, L.T_F16)
    assert lib.kvm_window_shadow_bytes(C.byref(wf.c)) == 0
    w4 = api.KVWindow(kvm_state, 256, H, D, BT, L.T_Q4_0, L.T_Q4_0, shadow=True)
    assert w4.k_shadow.numel() == 256 * H * (D // 32) * 18
    with pytest.raises(L.KvmError):
        api.KVWindow(kvm_state, 256, H, 128, BT, L.T_F16, L.T_F16, shadow=True)


@pytest.mark.parametrize("kt", [L.T_Q8_0, L.T_Q4_0], ids=["q8_0", "q4_0"])
def test_churn_over_a_128_block_window(kvm_state, kt):
    """The decode workload's window shape: 128 blocks of 128 tokens from a
    512-block history (q8_0 or q4_0 K).  Each step drops the second-earliest block and adds one
    past the last, or the reverse, so 126 blocks move a slot (504 staging items,
    the stage-in's gather barrier over its full grid); the window equals a fresh
    stage-in of the plan from the clean history."""
    st = kvm_state
    n_blocks, nsel = 512, 128
    hp, hc, kr, vr, rng = _histories(0x5B00, n_blocks * BT, kt)
    nt = np.full(n_blocks, BT, np.int32)
    sa = np.concatenate([[0], np.sort(rng.choice(np.arange(1, n_blocks - 1), nsel - 1, replace=False))])
    late = next(b for b in range(n_blocks - 1, 0, -1) if b not in set(sa))
    sb = np.sort(np.concatenate([np.setdiff1d(sa, [sa[1]]), [late]]))
    w = api.KVWindow(st, nsel * BT, H, D, BT, kt, L.T_Q4_0, shadow=True)
    for step, chosen in enumerate((sa, sb, sa, sb)):
        s = np.zeros(n_blocks)
        s[chosen] = 1.0
        held = _resident_full(w, nt)
        _poison(hp, held, rng)
        sel = api.select_topk(st, dev(s), dev(nt), nsel, 1, 0, None, window=w)
        api.stagein_selection(st, hp, w, sel, 64, 1e7)
        _restore(hp, held, kr, vr)
        res = sel.result()
        assert res["status"] == 0 and np.array_equal(res["ids"], chosen), step
        n_moved = int((res["stage_src"] >= 0).sum())
        assert (len(res["stage_slots"]), n_moved) == ((nsel, 0) if step == 0 else (nsel - 1, nsel - 2)), step
        ref_w, _ = _fresh(st, hc, s, nt, nsel, nsel, kt)
        _same_window(w, ref_w, nsel * BT)
