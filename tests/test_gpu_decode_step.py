"""kvm_score_topk_stagein_fa_decode(_lanes): a whole decode step in two
launches (the scoring grid, then one launch whose selector workgroup picks the
blocks while the attention workgroups attend, stage a non-empty plan and attend
again) against the same step as separate calls on a second window:
kvm_score_topk, kvm_stagein_selection, kvm_fa_decode.  Selections equal
(scores, ids, layout, stage plan), windows equal byte for byte, attention
outputs bit-equal where both split the keys alike (KVM_FA_SPLITS), else within
the attention tolerance; one output also against the oracle."""
import ctypes as C

import numpy as np
import pytest
import torch

from gpu_util import check_attention, dev, host, rand_rows
from kvmem_amd import api, _lib as L
import oracle as O

pytestmark = pytest.mark.gpu

H, G, D, BT = 4, 6, 256, 128
K_ROW, V_ROW = H * D // 32 * 34, H * D // 32 * 18


def _lane(st, seed, n_blocks, budget, slots, n_tok_q=4, terms=False, kt=L.T_Q8_0):
    rng = np.random.default_rng(seed)
    n_hist = n_blocks * BT - 40                         # the last block partly filled
    kr, vr = rand_rows(rng, n_hist, H, D, kt, L.T_Q4_0)
    ix = api.MeanKIndex(st, 1, n_blocks, H, D, BT, norms=terms)
    ix.add(0, 0, dev(rng.standard_normal((n_hist, H * D)).astype(np.float32)))
    qa = api.QueryAcc(st, 1, H * G, D, n_head_kv=H if terms else 0)
    qa.reset()
    qa.add(0, dev(rng.standard_normal((4, H * G * D)).astype(np.float32)))
    nt = dev(np.array([min(BT, n_hist - b * BT) for b in range(n_blocks)], np.int32))
    mk = lambda sh: dict(window=api.KVWindow(st, slots * BT, H, D, BT, kt, L.T_Q4_0, shadow=sh),
                         sel=api.SelectionBuffers(st, n_blocks, budget), history=api.History(kr, vr))
    return dict(rng=rng, kr=kr, vr=vr, kt=kt, ix=ix, qa=qa, nt=nt, n_blocks=n_blocks, budget=budget, n_hist=n_hist,
                q_pos=dev(np.arange(budget * BT - max(n_tok_q, 1), budget * BT, dtype=np.int32)), n_tok_q=n_tok_q,
                a=mk(True), b=mk(False))


def _step_dict(ln):
    a = ln["a"]
    return dict(index=ln["ix"], query=ln["qa"], n_blocks=ln["n_blocks"], n_tokens=ln["nt"],
                budget_blocks=ln["budget"], sink_blocks=1, recent_blocks=0, window=a["window"], sel=a["sel"],
                history=a["history"], q=ln["q"], q_pos=ln["q_pos"], out=ln["out"])


def _resident_full(w, nt_host):
    return sorted({int(b) for b in host(w.slot_block) if 0 <= int(b) < len(nt_host) and nt_host[int(b)] == BT})


def _set_rows(hist, blocks, rows_k, rows_v):
    torch.cuda.synchronize()
    k = hist.kbuf.u8.reshape(hist.n_tokens, -1)
    v = hist.vbuf.u8.reshape(hist.n_tokens, V_ROW)
    for b in blocks:
        k[b * BT:(b + 1) * BT] = rows_k(b)
        v[b * BT:(b + 1) * BT] = rows_v(b)


def _reference_step(st, ln):
    b = ln["b"]
    api.score_topk(st, ln["ix"], ln["qa"], ln["n_blocks"], ln["nt"], ln["budget"], 1, 0, None, b["window"], b["sel"])
    api.stagein_selection(st, b["history"], b["window"], b["sel"], 64, 1e7)
    return api.fa_decode(st, b["window"], ln["q"], ln["q_pos"], H * G, D ** -0.5)


def _compare(ln, ref, bit_equal, tag):
    ra, rb = ln["a"]["sel"].result(), ln["b"]["sel"].result()
    assert ra["status"] == rb["status"] == 0, tag
    assert ra["total"] == rb["total"], tag
    for key in ("ids", "to_base", "stage_slots"):
        assert np.array_equal(ra[key], rb[key]), (tag, key)
    n = ln["n_blocks"]
    assert torch.equal(ln["a"]["sel"].scores[:n], ln["b"]["sel"].scores[:n]), tag
    for name in ("k", "v", "cell_pos", "slot_block", "slot_base"):
        assert torch.equal(getattr(ln["a"]["window"], name), getattr(ln["b"]["window"], name)), (tag, name)
    if bit_equal:
        assert torch.equal(ln["out"], ref), tag
    else:
        check_attention(host(ln["out"]), host(ref))
    return int((ra["stage_src"] >= 0).sum())


@pytest.mark.parametrize("n_lanes,splits,terms,kt", [(1, None, False, L.T_Q8_0), (1, 32, True, L.T_Q8_0),
                                                    (3, None, True, L.T_Q8_0), (1, 32, True, L.T_Q4_0)],
                         ids=["q8_0", "q8_0-32-splits-terms", "q8_0-3-lanes-terms", "q4_0-32-splits-terms"])
def test_decode_step_matches_separate_calls(kvm_state, monkeypatch, n_lanes, splits, terms, kt):
    """Queries drift over six steps, so plans restage and move blocks within
    windows that carry a K shadow (the host rows of the full blocks a window
    holds are poisoned while its step runs: a moved block must come from the
    shadow).  splits: both attention paths take that many key splits, so the
    outputs are bit-equal (the same code over the same bytes); otherwise the
    step's launch takes one split fewer per head than kvm_fa_decode (the
    selectors' column) and the outputs agree within the attention tolerance.
    terms: the query accumulators carry the scorer's query terms, refreshed
    after each drift of the sums, and the indexes the blocks' terms.  kt: the K cache type (q4_0: the selecting
    launch stages the q4_0 rows with the one-row-per-wave requantiser, the
    separate calls with the 16-lane one)."""
    if splits:
        monkeypatch.setenv("KVM_FA_SPLITS", str(splits))
    st = kvm_state
    lanes = [_lane(st, 0x5D00 + i, 40 + 6 * i, 12, 16, terms=terms, kt=kt) for i in range(n_lanes)]
    moved = staged = 0
    for step in range(6):
        for ln in lanes:
            if step:
                ln["qa"].q_sum.add_(dev((ln["rng"].standard_normal((1, H * G * D)) * 0.6).astype(np.float32)))
                if terms:
                    ln["qa"].refresh()
            ln["q"] = dev(ln["rng"].standard_normal((ln["n_tok_q"], H * G, D)).astype(np.float32)).to(torch.bfloat16)
            ln["out"] = torch.empty((ln["n_tok_q"], H * G, D), dtype=torch.float32, device="cuda")
        nts = [host(ln["nt"]) for ln in lanes]
        held = [_resident_full(ln["a"]["window"], nt) for ln, nt in zip(lanes, nts)]
        for ln, hb in zip(lanes, held):
            _set_rows(ln["a"]["history"], hb, lambda b, r=ln["rng"], kw=ln["kr"].shape[1]: r.integers(0, 256, (BT, kw), dtype=np.uint8),
                      lambda b, r=ln["rng"]: r.integers(0, 256, (BT, V_ROW), dtype=np.uint8))
        if n_lanes == 1:
            d = _step_dict(lanes[0])
            api.decode_step(st, d["index"], d["query"], d["n_blocks"], d["n_tokens"], d["budget_blocks"], 1, 0,
                            d["window"], d["sel"], d["history"], d["q"], d["q_pos"], H * G, D ** -0.5, 64, 1e7,
                            out=d["out"])
        else:
            api.prepare_decode_step_lanes(st, [_step_dict(ln) for ln in lanes], H * G, D ** -0.5, 64, 1e7)()
        for ln, hb in zip(lanes, held):
            _set_rows(ln["a"]["history"], hb, lambda b, ln=ln: ln["kr"][b * BT:(b + 1) * BT],
                      lambda b, ln=ln: ln["vr"][b * BT:(b + 1) * BT])
        for i, ln in enumerate(lanes):
            ref = _reference_step(st, ln)
            torch.cuda.synchronize()
            staged += len(ln["a"]["sel"].result()["stage_slots"])
            moved += _compare(ln, ref, splits is not None, (step, i))
    assert moved > 0 and staged > moved
    # the oracle on the last step of lane 0 (ggml semantics over the window's bytes)
    ln = lanes[0]
    w = ln["b"]["window"]
    ek, ev = w.export_rows(0, w.n_cells)
    ref = O.fa_ggml(kt, O.T_Q4_0, ln["q"].float().cpu().numpy(), host(ek), host(ev), host(w.cell_pos),
                    host(ln["q_pos"]), H * G, H, D, D ** -0.5)
    check_attention(host(ln["out"]), ref)


def test_select_step_from_caller_scores_matches_separate_calls(kvm_state, monkeypatch):
    """kvm_select_topk_stagein_fa_decode (caller scores, one launch) against
    kvm_select_topk + kvm_stagein_fa_decode on a second window, over steps
    whose scores change (plans restage and move blocks within a shadowed
    window) and one whose scores repeat (an empty plan): selections, windows
    and outputs equal (both attention paths take 32 splits)."""
    monkeypatch.setenv("KVM_FA_SPLITS", "32")
    st = kvm_state
    ln = _lane(st, 0x5E1, 40, 12, 16)
    rng = ln["rng"]
    scores = None
    for step in range(5):
        if step != 3:
            scores = dev(rng.standard_normal(ln["n_blocks"]))
        ln["q"] = dev(rng.standard_normal((ln["n_tok_q"], H * G, D)).astype(np.float32)).to(torch.bfloat16)
        ln["out"] = torch.empty((ln["n_tok_q"], H * G, D), dtype=torch.float32, device="cuda")
        a, b = ln["a"], ln["b"]
        api.prepare_select_decode_step(st, scores, ln["nt"], ln["budget"], 1, 0, a["window"], a["sel"],
                                       a["history"], ln["q"], ln["q_pos"], H * G, D ** -0.5, ln["out"], 64, 1e7)()
        api.select_topk(st, scores, ln["nt"], ln["budget"], 1, 0, None, b["window"], b["sel"])
        ref = api.stagein_fa_decode(st, b["history"], b["sel"], b["window"], ln["q"], ln["q_pos"], H * G,
                                    D ** -0.5, 64, 1e7)
        torch.cuda.synchronize()
        _compare(ln, ref, True, step)
        if step == 3:
            assert len(a["sel"].result()["stage_slots"]) == 0
    assert st.status() == 0


def test_decode_step_steady_state(kvm_state, monkeypatch):
    """The same query accumulator twice: the second step's plan is empty (the
    attention workgroups keep their first pass), its selection and window equal
    the first's and its output equals kvm_fa_decode's over the window."""
    monkeypatch.setenv("KVM_FA_SPLITS", "48")
    st = kvm_state
    ln = _lane(st, 0x5D10, 32, 10, 12)
    ln["q"] = dev(ln["rng"].standard_normal((4, H * G, D)).astype(np.float32))
    ln["out"] = torch.empty((4, H * G, D), dtype=torch.float32, device="cuda")
    d = _step_dict(ln)
    step = api.prepare_decode_step(st, d["index"], d["query"], d["n_blocks"], d["n_tokens"], d["budget_blocks"], 1, 0,
                                   d["window"], d["sel"], d["history"], d["q"], d["q_pos"], H * G, D ** -0.5,
                                   d["out"], 64, 1e7)
    step()
    torch.cuda.synchronize()
    first = ln["a"]["sel"].result()
    assert len(first["stage_slots"]) > 0
    k0 = ln["a"]["window"].k.clone()
    ln["out"].zero_()
    step()
    torch.cuda.synchronize()
    second = ln["a"]["sel"].result()
    assert len(second["stage_slots"]) == 0 and second["status"] == 0
    assert np.array_equal(first["ids"], second["ids"]) and np.array_equal(first["to_base"], second["to_base"])
    assert torch.equal(ln["a"]["window"].k, k0)
    ref = api.fa_decode(st, ln["a"]["window"], ln["q"], ln["q_pos"], H * G, D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(ln["out"], ref)


@pytest.mark.parametrize("n_layer,splits", [(3, None), (14, 8)], ids=["3-layers", "14-layers-8-splits"])
def test_decode_step_scores_every_layer(kvm_state, monkeypatch, n_layer, splits):
    """Indexes and accumulators of several layers that carry their terms, one
    layer without query rows (the top-k skips it, averaging the others in
    layer order): over three steps whose last layer's query drifts, the step
    equals the separate calls (scores bit for bit; outputs bit-equal under a
    common split count)."""
    if splits:
        monkeypatch.setenv("KVM_FA_SPLITS", str(splits))
    st = kvm_state
    ln = _lane(st, 0x5D50 + n_layer, 40, 12, 16, terms=True)
    rng = ln["rng"]
    ix = api.MeanKIndex(st, n_layer, ln["n_blocks"], H, D, BT, norms=True)
    for il in range(n_layer):
        ix.add(il, 0, dev(rng.standard_normal((ln["n_hist"], H * D)).astype(np.float32)))
    qa = api.QueryAcc(st, n_layer, H * G, D, n_head_kv=H)
    qa.reset()
    for il in range(n_layer):
        if il != 1:
            qa.add(il, dev(rng.standard_normal((4, H * G * D)).astype(np.float32)))
    ln["ix"], ln["qa"] = ix, qa
    for step in range(3):
        if step:
            qa.q_sum[2].add_(dev((rng.standard_normal(H * G * D) * 0.8).astype(np.float32)))
            qa.refresh()
        ln["q"] = dev(rng.standard_normal((4, H * G, D)).astype(np.float32)).to(torch.bfloat16)
        ln["out"] = torch.empty((4, H * G, D), dtype=torch.float32, device="cuda")
        d = _step_dict(ln)
        api.decode_step(st, d["index"], d["query"], d["n_blocks"], d["n_tokens"], d["budget_blocks"], 1, 0,
                        d["window"], d["sel"], d["history"], d["q"], d["q_pos"], H * G, D ** -0.5, 64, 1e7,
                        out=d["out"])
        ref = _reference_step(st, ln)
        torch.cuda.synchronize()
        _compare(ln, ref, splits is not None, step)
    assert st.status() == 0


def test_decode_step_three_launch_path(kvm_state):
    """A step with a lane that has no query token takes the three-launch path
    (kvm_score_topk + kvm_stagein_fa_decode) with the same results: the other
    lane's selection, window and output as the separate calls give them, the
    empty lane's plan staged and its output untouched."""
    st = kvm_state
    lanes = [_lane(st, 0x5D20 + i, 24, 8, 10, n_tok_q=(4, 0)[i]) for i in range(2)]
    for ln in lanes:
        ln["q"] = dev(ln["rng"].standard_normal((max(ln["n_tok_q"], 1), H * G, D)).astype(np.float32))
        ln["q"] = ln["q"][:ln["n_tok_q"]] if ln["n_tok_q"] else ln["q"]
        ln["out"] = torch.full((max(ln["n_tok_q"], 1), H * G, D), 7.0, dtype=torch.float32, device="cuda")
    steps = [_step_dict(ln) for ln in lanes]
    n = len(steps)
    arr, hists, fl = (L.RetrievalLane * n)(), (C.POINTER(L.History) * n)(), (L.Lane * n)()
    keep = []
    for i, (ln, d) in enumerate(zip(lanes, steps)):
        p = L.SelectParams(d["n_blocks"], d["budget_blocks"], 1, 0, None, 0, d["n_tokens"].data_ptr())
        keep.append(p)
        arr[i] = L.RetrievalLane(C.pointer(d["index"].c), C.pointer(d["query"].c), C.pointer(p),
                                 C.pointer(d["window"].c), C.pointer(d["sel"].c))
        hists[i] = C.pointer(d["history"].c)
        fl[i] = L.Lane(C.pointer(d["window"].c), d["q"].data_ptr(), d["q_pos"].data_ptr(), d["out"].data_ptr(),
                       ln["n_tok_q"])
    st.check(st.lib.kvm_score_topk_stagein_fa_decode_lanes(st.h, arr, hists, fl, n, C.byref(L.RopeParams(64, 1e7, 1.0, -1)),
                                                           L.T_F32, H * G, D ** -0.5))
    torch.cuda.synchronize()
    ref = _reference_step(st, lanes[0])
    torch.cuda.synchronize()
    _compare(lanes[0], ref, False, "lane 0")
    ln = lanes[1]
    b = ln["b"]
    api.score_topk(st, ln["ix"], ln["qa"], ln["n_blocks"], ln["nt"], ln["budget"], 1, 0, None, b["window"], b["sel"])
    api.stagein_selection(st, b["history"], b["window"], b["sel"], 64, 1e7)
    torch.cuda.synchronize()
    for name in ("k", "v", "cell_pos", "slot_block", "slot_base"):
        assert torch.equal(getattr(ln["a"]["window"], name), getattr(b["window"], name)), name
    assert bool((ln["out"] == 7.0).all())


def test_decode_step_bad_arguments(kvm_state):
    """A lane that selects for one window and attends another is refused
    before anything is launched."""
    st = kvm_state
    ln = _lane(st, 0x5D30, 16, 6, 8)
    q = dev(ln["rng"].standard_normal((4, H * G, D)).astype(np.float32))
    out = torch.empty((4, H * G, D), dtype=torch.float32, device="cuda")
    p = L.SelectParams(ln["n_blocks"], ln["budget"], 1, 0, None, 0, ln["nt"].data_ptr())
    a, b = ln["a"], ln["b"]
    arr = (L.RetrievalLane * 1)(L.RetrievalLane(C.pointer(ln["ix"].c), C.pointer(ln["qa"].c), C.pointer(p),
                                                C.pointer(a["window"].c), C.pointer(a["sel"].c)))
    hists = (C.POINTER(L.History) * 1)(C.pointer(a["history"].c))
    fl = (L.Lane * 1)(L.Lane(C.pointer(b["window"].c), q.data_ptr(), ln["q_pos"].data_ptr(), out.data_ptr(), 4))
    info0 = a["sel"].info.clone()
    rc = st.lib.kvm_score_topk_stagein_fa_decode_lanes(st.h, arr, hists, fl, 1, C.byref(L.RopeParams(64, 1e7, 1.0, -1)),
                                                       L.T_F32, H * G, D ** -0.5)
    assert rc == L.KVM_EINVAL
    torch.cuda.synchronize()
    assert torch.equal(a["sel"].info, info0)


def _rows(rng, n, h, d):
    """Valid q8_0 K / q4_0 V rows without an fp32 source: fp16 scales in
    [2^-8, 2^-4), random quants."""
    nb = h * d // 32
    k = np.zeros((n, nb, 34), np.uint8)
    k[:, :, :2] = (rng.uniform(2 ** -8, 2 ** -4, (n, nb)).astype(np.float16)).view(np.uint8).reshape(n, nb, 2)
    k[:, :, 2:] = rng.integers(-127, 128, (n, nb, 32), dtype=np.int8).view(np.uint8)
    v = np.zeros((n, nb, 18), np.uint8)
    v[:, :, :2] = (rng.uniform(2 ** -6, 2 ** -2, (n, nb)).astype(np.float16)).view(np.uint8).reshape(n, nb, 2)
    v[:, :, 2:] = rng.integers(0, 256, (n, nb, 16), dtype=np.uint8)
    return k.reshape(n, -1), v.reshape(n, -1)


def _small_lane(st, seed, n_blocks, bt, budget, slots, h=1, g=8, d=128):
    rng = np.random.default_rng(seed)
    n_hist = n_blocks * bt
    kr, vr = _rows(rng, n_hist, h, d)
    ix = api.MeanKIndex(st, 1, n_blocks, h, d, bt)
    ix.set_block_sums(dev(rng.standard_normal((1, n_blocks, h * d)).astype(np.float32)))
    ix.mean_tokens[:, :n_blocks] = bt
    ix.present[:n_blocks] = 1
    qa = api.QueryAcc(st, 1, h * g, d)
    qa.reset()
    qa.add(0, dev(rng.standard_normal((2, h * g * d)).astype(np.float32)))
    nt = dev(np.full(n_blocks, bt, np.int32))
    mk = lambda: dict(window=api.KVWindow(st, slots * bt, h, d, bt), sel=api.SelectionBuffers(st, n_blocks, budget),
                      history=api.History(kr, vr))
    q = dev(rng.standard_normal((1, h * g, d)).astype(np.float32))
    q_pos = dev(np.array([budget * bt - 1], np.int32))
    return dict(rng=rng, ix=ix, qa=qa, nt=nt, n_blocks=n_blocks, bt=bt, budget=budget, h=h, g=g, d=d, q=q,
                q_pos=q_pos, a=mk(), b=mk())


def _check_small(st, ln, sink, recent, mandatory=None):
    h, g, d = ln["h"], ln["g"], ln["d"]
    a, b = ln["a"], ln["b"]
    out = api.decode_step(st, ln["ix"], ln["qa"], ln["n_blocks"], ln["nt"], ln["budget"], sink, recent,
                          a["window"], a["sel"], a["history"], ln["q"], ln["q_pos"], h * g, d ** -0.5, 64, 1e7,
                          mandatory=mandatory)
    api.score_topk(st, ln["ix"], ln["qa"], ln["n_blocks"], ln["nt"], ln["budget"], sink, recent, mandatory,
                   b["window"], b["sel"])
    api.stagein_selection(st, b["history"], b["window"], b["sel"], 64, 1e7)
    ref = api.fa_decode(st, b["window"], ln["q"], ln["q_pos"], h * g, d ** -0.5)
    torch.cuda.synchronize()
    ra, rb = a["sel"].result(), b["sel"].result()
    assert ra["status"] == rb["status"] == 0
    for key in ("ids", "to_base", "stage_slots"):
        assert np.array_equal(ra[key], rb[key]), key
    assert torch.equal(a["sel"].scores[:ln["n_blocks"]], b["sel"].scores[:ln["n_blocks"]])
    for name in ("k", "v", "cell_pos", "slot_block", "slot_base"):
        assert torch.equal(getattr(a["window"], name), getattr(b["window"], name)), name
    check_attention(host(out), host(ref))
    return ra


@pytest.mark.parametrize("n_blocks", [4096, 4097])
def test_decode_step_at_the_selector_capacity(kvm_state, n_blocks):
    """4,096 blocks (the selector workgroup's capacity: eight keys per thread)
    take the two-launch step, one block more the three-launch path; 1,100
    selected blocks in 1,100 slots (past the 1,024 slot-map entries the
    selector keeps in LDS), over two steps whose query drifts.  Both equal the
    separate calls (scores, selection, window bytes, attention)."""
    st = kvm_state
    ln = _small_lane(st, 0x5D40 + n_blocks, n_blocks, 64, 1100, 1100)
    r = _check_small(st, ln, 1, 0)
    assert len(r["ids"]) == 1100 and r["ids"][0] == 0 and len(r["stage_slots"]) == 1100
    ln["qa"].q_sum.add_(dev((ln["rng"].standard_normal((1, ln["h"] * ln["g"] * ln["d"])) * 0.5).astype(np.float32)))
    r = _check_small(st, ln, 1, 0)
    assert 0 < len(r["stage_slots"]) < 1100


def test_decode_step_mandatory_and_recent(kvm_state):
    """Mandatory ids (newest last, trimmed by the budget newest first) and a
    recent tail go through the selector's serial pass as through the top-k
    kernel's."""
    ln = _small_lane(kvm_state, 0x5D50, 300, 64, 10, 12)
    mand = dev(np.array([7, 250, 31, 123, 250], np.int32))
    r = _check_small(kvm_state, ln, 2, 3, mandatory=mand)
    ids = set(r["ids"].tolist())
    assert {0, 1, 297, 298, 299, 7, 31, 123, 250} <= ids


def test_decode_step_lane_without_blocks(kvm_state):
    """A lane whose history holds no block yet selects nothing, stages nothing
    and attends over what its window holds, beside a lane that retrieves."""
    st = kvm_state
    H1, G1, D1, bt = 1, 8, 128, 64
    full = _small_lane(st, 0x5D60, 40, bt, 8, 10)
    empty = _small_lane(st, 0x5D61, 1, bt, 8, 10)
    lanes = []
    for ln, nb in ((full, 40), (empty, 0)):
        ln["out"] = torch.empty((1, H1 * G1, D1), dtype=torch.float32, device="cuda")
        lanes.append(dict(index=ln["ix"], query=ln["qa"], n_blocks=nb, n_tokens=ln["nt"], budget_blocks=8,
                          sink_blocks=1, recent_blocks=0, window=ln["a"]["window"], sel=ln["a"]["sel"],
                          history=ln["a"]["history"], q=ln["q"], q_pos=ln["q_pos"], out=ln["out"]))
    api.prepare_decode_step_lanes(st, lanes, H1 * G1, D1 ** -0.5, 64, 1e7)()
    torch.cuda.synchronize()
    r = empty["a"]["sel"].result()
    assert r["status"] == 0 and len(r["ids"]) == 0 and len(r["stage_slots"]) == 0
    # nothing staged: every cell of the empty lane's window is still empty, so
    # its token sees no cell and gets zeros
    assert bool((empty["a"]["window"].cell_pos == -1).all())
    assert bool((empty["out"] == 0).all())
    b = full["b"]
    api.score_topk(st, full["ix"], full["qa"], 40, full["nt"], 8, 1, 0, None, b["window"], b["sel"])
    api.stagein_selection(st, b["history"], b["window"], b["sel"], 64, 1e7)
    ref = api.fa_decode(st, b["window"], full["q"], full["q_pos"], H1 * G1, D1 ** -0.5)
    torch.cuda.synchronize()
    assert np.array_equal(full["a"]["sel"].result()["ids"], b["sel"].result()["ids"])
    assert torch.equal(full["a"]["window"].k, b["window"].k)
    check_attention(host(full["out"]), host(ref))


def test_decode_step_four_lanes_full_windows(kvm_state):
    """The four-lane decode shape through the two-launch step: four lanes with
    32,768-cell windows (24 q / 4 kv heads, head_dim 256, one bf16 token each)
    selecting 128 blocks from histories of 160-400 blocks; the same step as
    three launches on second windows gives the same selections and window
    bytes, outputs within the attention tolerance (other key splits), and
    lane 0 agrees with the oracle."""
    st = kvm_state
    cells, budget = 32768, 128
    lanes, ref_lanes, fa_ref, keep = [], [], [], []
    for i, nb in enumerate((160, 240, 320, 400)):
        rng = np.random.default_rng(0x5D70 + i)
        kr, vr = _rows(rng, nb * BT, H, D)
        ix = api.MeanKIndex(st, 1, nb, H, D, BT)
        ix.set_block_sums(dev(rng.standard_normal((1, nb, H * D)).astype(np.float32)))
        ix.mean_tokens[:, :nb] = BT
        ix.present[:nb] = 1
        qa = api.QueryAcc(st, 1, H * G, D)
        qa.reset()
        qa.add(0, dev(rng.standard_normal((1, H * G * D)).astype(np.float32)))
        nt = dev(np.full(nb, BT, np.int32))
        q = dev(rng.standard_normal((1, H * G, D)).astype(np.float32)).to(torch.bfloat16)
        q_pos = dev(np.array([budget * BT - 1], np.int32))
        sides = []
        for _ in range(2):
            sides.append(dict(window=api.KVWindow(st, cells, H, D, BT), sel=api.SelectionBuffers(st, nb, budget),
                              history=api.History(kr, vr),
                              out=torch.empty((1, H * G, D), dtype=torch.float32, device="cuda")))
        a, b = sides
        base = dict(index=ix, query=qa, n_blocks=nb, n_tokens=nt, budget_blocks=budget, sink_blocks=1,
                    recent_blocks=0, q=q, q_pos=q_pos)
        lanes.append(dict(base, window=a["window"], sel=a["sel"], history=a["history"], out=a["out"]))
        ref_lanes.append(dict(base, window=b["window"], sel=b["sel"], history=b["history"], out=b["out"]))
        fa_ref.append(dict(history=b["history"], sel=b["sel"], window=b["window"], q=q, q_pos=q_pos, out=b["out"]))
        keep.append((kr, vr))
    api.prepare_decode_step_lanes(st, lanes, H * G, D ** -0.5, 64, 1e7)()
    api.prepare_score_topk_lanes(st, ref_lanes)()
    api.prepare_stagein_fa_decode_lanes(st, fa_ref, H * G, D ** -0.5, 64, 1e7)()
    torch.cuda.synchronize()
    for i, (la, lb) in enumerate(zip(lanes, ref_lanes)):
        ra, rb = la["sel"].result(), lb["sel"].result()
        assert ra["status"] == rb["status"] == 0, i
        assert len(ra["ids"]) == budget and len(ra["stage_slots"]) == budget, i
        for key in ("ids", "to_base", "stage_slots"):
            assert np.array_equal(ra[key], rb[key]), (i, key)
        for name in ("k", "v", "cell_pos", "slot_block", "slot_base"):
            assert torch.equal(getattr(la["window"], name), getattr(lb["window"], name)), (i, name)
        check_attention(host(la["out"]), host(lb["out"]))
    w = lanes[0]["window"]
    ek, ev = w.export_rows(0, budget * BT)
    ref = O.fa_ggml(O.T_Q8_0, O.T_Q4_0, lanes[0]["q"].float().cpu().numpy(), host(ek), host(ev),
                    host(w.cell_pos)[:budget * BT], host(lanes[0]["q_pos"]), H * G, H, D, D ** -0.5)
    check_attention(host(lanes[0]["out"]), ref)


def test_decode_step_q4_0_k_window(kvm_state):
    """The whole step over a q4_0 K cache (history rows and window in q4_0):
    kvm_score_topk_stagein_fa_decode runs it as the two-launch step (the
    selecting launch stages the q4_0 rows); the staged blocks equal the
    oracle's q4_0 stage-in and the output the ggml
    attention over the window it leaves (a q4_0 K cache: Q quantised to q8_0,
    vec_dot_q4_0_q8_0)."""
    st = kvm_state
    rng = np.random.default_rng(0x44)
    n_blocks, budget = 24, 8
    n_hist = n_blocks * BT
    kr, vr = rand_rows(rng, n_hist, H, D, L.T_Q4_0, L.T_Q4_0)
    ix = api.MeanKIndex(st, 1, n_blocks, H, D, BT)
    ix.add(0, 0, dev(rng.standard_normal((n_hist, H * D)).astype(np.float32)))
    qa = api.QueryAcc(st, 1, H * G, D)
    qa.reset()
    qa.add(0, dev(rng.standard_normal((4, H * G * D)).astype(np.float32)))
    nt = dev(np.full(n_blocks, BT, np.int32))
    w = api.KVWindow(st, budget * BT, H, D, BT, L.T_Q4_0, L.T_Q4_0)
    sel = api.SelectionBuffers(st, n_blocks, budget)
    q = dev(rng.standard_normal((4, H * G, D)).astype(np.float32)).to(torch.bfloat16)
    q_pos = dev(np.arange(budget * BT - 4, budget * BT, dtype=np.int32))
    out = api.decode_step(st, ix, qa, n_blocks, nt, budget, 1, 0, w, sel, api.History(kr, vr), q, q_pos, H * G,
                          D ** -0.5, 64, 1e7)
    st.sync()
    res = sel.result()
    assert res["status"] == 0 and len(res["ids"]) == budget
    theta = O.rope_theta(1e7, 1.0, 64)
    ek, ev = w.export_rows(0, budget * BT)
    ek, ev = host(ek), host(ev)
    for k in (0, 3, budget - 1):
        bid, base = int(res["ids"][k]), int(res["to_base"][k])
        want = O.stagein_k(kr[bid * BT:(bid + 1) * BT].reshape(-1), BT, H, D, 64, 256, base, theta,
                           k_type=O.T_Q4_0).reshape(BT, -1)
        assert np.array_equal(ek[k * BT:(k + 1) * BT], want), k
    ref = O.fa_ggml(O.T_Q4_0, O.T_Q4_0, q.float().cpu().numpy(), ek, ev, host(w.cell_pos), host(q_pos), H * G, H, D,
                    D ** -0.5)
    check_attention(host(out), ref)
