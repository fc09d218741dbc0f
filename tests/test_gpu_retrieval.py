"""GPU retrieval: query accumulator, mean-K sums, scoring (bit-exact), top-k and
window layout against the oracle and the reference's top-k known answers."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import dev, golden_snapshot, host
from kvmem_amd import api, _lib as L

pytestmark = pytest.mark.gpu


def test_query_add_bit_exact(kvm_state):
    rng = np.random.default_rng(1)
    qa = api.QueryAcc(kvm_state, 2, 24, 256)
    qa.reset()
    rows0 = rng.standard_normal((4, 24 * 256)).astype(np.float32)
    rows1 = (rng.standard_normal((3, 24 * 256)) * 1e4).astype(np.float32)
    qa.add(0, dev(rows0))
    qa.add(1, dev(rows1[:1]))
    qa.add(1, dev(rows1[1:]))
    want0 = np.zeros(24 * 256, np.float32)
    for r in rows0:
        want0 = (want0 + r).astype(np.float32)
    want1 = np.zeros(24 * 256, np.float32)
    for r in rows1:
        want1 = (want1 + r).astype(np.float32)
    got = host(qa.q_sum)
    assert np.array_equal(got[0].view(np.uint32), want0.view(np.uint32))
    assert np.array_equal(got[1].view(np.uint32), want1.view(np.uint32))
    assert list(host(qa.q_count)) == [4, 3]


def test_meank_add_bit_exact(kvm_state):
    rng = np.random.default_rng(2)
    n, e, bt = 700, 512, 128
    k = rng.standard_normal((n, e)).astype(np.float32)
    k[::7] *= 1e6
    ix = api.MeanKIndex(kvm_state, 1, 8, 2, 256, bt)
    pos = 0
    for chunk in (5, 200, 11, 300, 184):
        ix.add(0, pos, dev(k[pos:pos + chunk]))
        pos += chunk
    sums, mt = O.meank_sums(k, bt, chunk=None)
    got = host(ix.block_sums())[0]                   # [blocks][e]
    assert np.array_equal(got[:6].view(np.uint32), sums.view(np.uint32))
    assert list(host(ix.mean_tokens)[0][:6]) == list(mt)
    assert list(host(ix.present)[:7]) == [1, 1, 1, 1, 1, 1, 0]


def _build_index(st, k_sum, mt, n_blocks_cap, H, D, bt=128, norms=False):
    """norms: the index carries the blocks' nk, formed by kvm_meank_refresh
    after the direct writes."""
    L_, nb, e = k_sum.shape
    ix = api.MeanKIndex(st, L_, n_blocks_cap, H, D, bt, norms=norms)
    ix.set_block_sums(dev(np.ascontiguousarray(k_sum)))
    ix.mean_tokens[:, :nb] = dev(mt.astype(np.int32))
    ix.present[:nb] = 1
    if norms:
        ix.refresh()
    return ix


def _case(seed, n_blocks, n_layer=1, n_head=24, H=4, D=256, planted=16):
    rng = np.random.default_rng(seed)
    k_sum = (rng.standard_normal((n_layer, n_blocks, H * D)) * 128).astype(np.float32)
    mt = np.full((n_layer, n_blocks), 128, np.uint32)
    mt[:, -1] = 77
    ids = rng.choice(np.arange(1, n_blocks), planted, replace=False)
    g = n_head // H
    q = np.zeros((n_layer, n_head * D), np.float32)
    inv = np.float32(1.0) / mt.astype(np.float32)
    for il in range(n_layer):
        for b in ids:
            mean = k_sum[il, b] * inv[il, b]
            for h in range(n_head):
                q[il, h * D:(h + 1) * D] += mean[(h // g) * D:(h // g + 1) * D]
    q += (rng.standard_normal(q.shape) * 0.1).astype(np.float32)
    return q, np.full(n_layer, 4, np.uint32), k_sum, mt, ids


@pytest.mark.parametrize("n_blocks,n_layer,n_head,H,D", [(2048, 1, 24, 4, 256), (128, 1, 8, 2, 128),
                                                       (300, 3, 24, 4, 256), (5000, 1, 24, 4, 256),
                                                       # 8-block workgroups with full (8 kv heads), split
                                                       # (16) and partly filled (3, 1) head chunks; 5000
                                                       # blocks at 4 kv heads take 16-block workgroups
                                                       (700, 2, 8, 8, 128), (260, 1, 32, 16, 128),
                                                       (500, 1, 12, 3, 128), (333, 1, 3, 1, 256)])
@pytest.mark.parametrize("terms", ["none", "q", "qk"], ids=["q_sum", "q_terms", "q_k_terms"])
def test_score_topk_bit_exact(kvm_state, n_blocks, n_layer, n_head, H, D, terms):
    """terms: q, the accumulator carries the query terms (formed by
    kvm_query_refresh after the direct writes) and the scorer reads them; qk,
    the index carries the blocks' nk too (kvm_meank_refresh)."""
    q, qc, k_sum, mt, planted = _case(n_blocks + n_layer, n_blocks, n_layer, n_head, H, D)
    ix = _build_index(kvm_state, k_sum, mt, n_blocks + 5, H, D, norms=terms == "qk")
    qa = api.QueryAcc(kvm_state, n_layer, n_head, D, n_head_kv=H if terms != "none" else 0)
    qa.q_sum.copy_(dev(q))
    qa.q_count.copy_(dev(qc.astype(np.int32)))
    if terms != "none":
        qa.refresh()
    n_tokens = np.full(n_blocks, 128, np.int32)
    n_tokens[-1] = 77
    budget = 128 if n_blocks > 128 else 32
    sel = api.score_topk(kvm_state, ix, qa, n_blocks, dev(n_tokens), budget, sink_blocks=1)
    res = sel.result()
    want_scores = O.score_retrieval(q, qc, k_sum, mt, n_head, H, D)
    got_scores = host(sel.scores)[:n_blocks]
    assert np.array_equal(got_scores.view(np.uint64), want_scores.view(np.uint64))
    want_ids = O.pick_topk(want_scores, budget, 1, 0)
    assert np.array_equal(res["ids"], want_ids)
    assert set(planted) <= set(res["ids"])
    to_base, _, total = O.window_layout(want_ids, n_tokens.astype(np.uint32), 128, len(want_ids))
    assert np.array_equal(res["to_base"], to_base) and res["total"] == total and res["status"] == 0


@pytest.mark.parametrize("terms", ["none", "q", "qk"], ids=["q_sum", "q_terms", "q_k_terms"])
def test_score_bit_exact_where_every_term_matters(kvm_state, terms):
    """The closed-form pin's inputs (norms near 1e-6 so the epsilon and invq
    count, g = 3, three layers with query counts 5, 0, 2, a block without K in
    one layer): the GPU scores equal the oracle's bit for bit, with the query
    terms formed by the scorer or carried by the accumulator."""
    from scoring_cases import tiny_norm_case
    n_head, H, D = 6, 2, 128
    q, qc, k_sum, mt = tiny_norm_case(41, n_head=n_head, H=H, d=D)
    n_layer, n_blocks = mt.shape
    ix = _build_index(kvm_state, k_sum, mt, n_blocks + 3, H, D, norms=terms == "qk")
    qa = api.QueryAcc(kvm_state, n_layer, n_head, D, n_head_kv=H if terms != "none" else 0)
    qa.q_sum.copy_(dev(q))
    qa.q_count.copy_(dev(qc.astype(np.int32)))
    if terms != "none":
        qa.refresh()
    sel = api.score_topk(kvm_state, ix, qa, n_blocks, dev(np.full(n_blocks, 128, np.int32)), 4, sink_blocks=1)
    sel.result()
    want = O.score_retrieval(q, qc, k_sum, mt, n_head, H, D)
    assert np.array_equal(host(sel.scores)[:n_blocks].view(np.uint64), want.view(np.uint64))


def test_query_terms_follow_reset_and_adds(kvm_state):
    """The accumulator's query terms are kept current by reset, add and
    add_view (no refresh): after each, the scores equal the oracle's on the
    accumulated sums bit for bit, and equal those of an accumulator without
    terms.  An index with another kv-head count is refused."""
    n_blocks, n_layer, n_head, H, D = 300, 2, 12, 3, 128
    q, _, k_sum, mt, _ = _case(77, n_blocks, n_layer, n_head, H, D)
    ix = _build_index(kvm_state, k_sum, mt, n_blocks, H, D)
    qa = api.QueryAcc(kvm_state, n_layer, n_head, D, n_head_kv=H)
    plain = api.QueryAcc(kvm_state, n_layer, n_head, D)
    rng = np.random.default_rng(5)
    n_tokens = dev(np.full(n_blocks, 128, np.int32))

    def check():
        a = api.score_topk(kvm_state, ix, qa, n_blocks, n_tokens, 32, sink_blocks=1)
        b = api.score_topk(kvm_state, ix, plain, n_blocks, n_tokens, 32, sink_blocks=1)
        qs, qc = host(plain.q_sum), host(plain.q_count).astype(np.uint32)
        want = O.score_retrieval(qs, qc, k_sum, mt, n_head, H, D)
        got = host(a.scores)[:n_blocks]
        assert np.array_equal(got.view(np.uint64), want.view(np.uint64))
        assert np.array_equal(got.view(np.uint64), host(b.scores)[:n_blocks].view(np.uint64))

    for acc in (qa, plain):
        acc.reset()
    rows = (q[0] + rng.standard_normal((3, n_head * D)) * 0.2).astype(np.float32)
    for acc in (qa, plain):
        acc.add(0, dev(rows))
    check()                                   # layer 1 has no queries yet
    rows1 = torch.from_numpy((q[1] + rng.standard_normal((5, n_head * D)) * 0.2).astype(np.float32))
    view = dev(rows1.numpy()).view(5, n_head, D).to(torch.bfloat16)
    keep = np.array([1, 0, 1, 1, 0], np.uint8)
    for acc in (qa, plain):
        acc.add_view(1, view, keep)
    check()
    for acc in (qa, plain):
        acc.reset()
        acc.add(1, dev(rows[:1]))
    check()
    assert not host(qa.q_vec)[0].any() and not host(qa.q_norm)[0].any()
    wrong = api.QueryAcc(kvm_state, n_layer, n_head, D, n_head_kv=1)
    with pytest.raises(RuntimeError):
        api.score_topk(kvm_state, ix, wrong, n_blocks, n_tokens, 32, sink_blocks=1)


def test_index_terms_follow_adds_and_flushes(kvm_state):
    """The index's block terms (nk) are kept current by kvm_meank_add (whole
    and partial blocks), the decode running sum's flush and refresh: after
    each, the scores equal the oracle's on the index's sums bit for bit, and
    those of an index without the terms.  The query accumulator carries its
    terms too."""
    n_layer, n_head, H, D, bt = 2, 12, 3, 128, 128
    n_blocks = 20
    rng = np.random.default_rng(8)
    ixs = [api.MeanKIndex(kvm_state, n_layer, n_blocks, H, D, bt, norms=nm) for nm in (True, False)]
    qa = api.QueryAcc(kvm_state, n_layer, n_head, D, n_head_kv=H)
    qa.reset()
    for il in range(n_layer):
        qa.add(il, dev(rng.standard_normal((3, n_head * D)).astype(np.float32)))
    n_tokens = dev(np.full(n_blocks, bt, np.int32))

    def check(n_used):
        outs = [api.score_topk(kvm_state, ix, qa, n_used, n_tokens[:n_used].contiguous(), 4, sink_blocks=1)
                for ix in ixs]
        ks = host(ixs[1].block_sums())[:, :n_used]
        mt = host(ixs[1].mean_tokens)[:, :n_used].astype(np.uint32)
        want = O.score_retrieval(host(qa.q_sum), host(qa.q_count).astype(np.uint32), ks, mt, n_head, H, D)
        got = host(outs[0].scores)[:n_used]
        assert np.array_equal(got.view(np.uint64), want.view(np.uint64))
        assert np.array_equal(got.view(np.uint64), host(outs[1].scores)[:n_used].view(np.uint64))

    rows = (rng.standard_normal((n_layer, 9 * bt + 50, H * D)) * 3).astype(np.float32)
    for il in range(n_layer):
        for ix in ixs:
            ix.add(il, 0, dev(rows[il, :5 * bt + 17]))          # 5 full blocks and part of a sixth
    check(6)
    for il in range(n_layer):
        for ix in ixs:
            ix.add(il, 5 * bt + 17, dev(rows[il, 5 * bt + 17:9 * bt + 50]))   # the sixth completed, up to 10
    check(10)
    # the decode running sum flushed into block 10
    dec = dev(rng.standard_normal((40, H * D)).astype(np.float32))
    for ix in ixs:
        ix.acc_zero(1)
        ix.acc_add(1, dec.view(40, H, D), 0, 40)
        ix.acc_flush(1, 10 * bt, 40)
    check(11)
    # direct writes, then refresh
    for ix in ixs:
        ix.k_sum.mul_(0.5)
        if ix.k_norm is not None:
            ix.refresh()
    check(11)


@pytest.mark.parametrize("terms", [False, True], ids=["q_sum", "q_terms"])
def test_score_topk_lanes_match_single_lane(kvm_state, terms):
    """Four lanes of different sizes (multi-lane decode) in one launch sequence:
    every lane's scores, ids, layout and stage plan equal the oracle's and a
    single-lane call's.  Without the terms the four-lane grid (1,024
    workgroups) takes the scorer whose chains form their products, a single
    lane the one with product rows in LDS; with them (query and index terms)
    both take the one with the 9 rows of dot products and qv squares."""
    H, n_head, D = 4, 24, 256
    lanes, single, cases = [], [], []
    for i, n_blocks in enumerate((512, 1024, 1536, 2048)):
        q, qc, k_sum, mt, planted = _case(200 + i, n_blocks, 1, n_head, H, D)
        ix = _build_index(kvm_state, k_sum, mt, n_blocks, H, D, norms=terms)
        qa = api.QueryAcc(kvm_state, 1, n_head, D, n_head_kv=H if terms else 0)
        qa.q_sum.copy_(dev(q))
        qa.q_count.copy_(dev(qc.astype(np.int32)))
        if terms:
            qa.refresh()
        n_tokens = dev(np.full(n_blocks, 128, np.int32))
        w = api.KVWindow(kvm_state, 128 * 128, H, D, 128)
        sel = api.SelectionBuffers(kvm_state, n_blocks, 128)
        lanes.append(dict(index=ix, query=qa, n_blocks=n_blocks, n_tokens=n_tokens, budget_blocks=128,
                          sink_blocks=1, window=w, sel=sel))
        w1 = api.KVWindow(kvm_state, 128 * 128, H, D, 128)
        single.append(api.score_topk(kvm_state, ix, qa, n_blocks, n_tokens, 128, 1, 0, None, w1))
        cases.append((q, qc, k_sum, mt, planted))
    api.score_topk_lanes(kvm_state, lanes)
    for ln, one, (q, qc, k_sum, mt, planted) in zip(lanes, single, cases):
        r, r1 = ln["sel"].result(), one.result()
        for key in ("ids", "to_base", "stage_slots"):
            assert np.array_equal(r[key], r1[key]), key
        assert r["total"] == r1["total"] and r["status"] == r1["status"] == 0
        want = O.score_retrieval(q, qc, k_sum, mt, n_head, H, D)
        got = host(ln["sel"].scores)[:ln["n_blocks"]]
        assert np.array_equal(got.view(np.uint64), want.view(np.uint64))
        assert np.array_equal(r["ids"], O.pick_topk(want, 128, 1, 0))
        assert set(planted) <= set(r["ids"])


@pytest.mark.parametrize("H,n_head,D,terms", [(2, 8, 128, False), (1, 3, 256, False), (2, 8, 128, True)])
def test_score_topk_lanes_wide_grids(kvm_state, H, n_head, D, terms):
    """Four lanes of 8192 blocks (the top-k maximum) at 2 or 1 kv heads: a
    grid of 4,096 workgroups (8-block tiles), past what the CUs hold with
    product rows in LDS, so the chains form their products; every lane's
    scores are bit-exact and its ids equal the oracle's (terms: with the query
    terms carried by the accumulators)."""
    n_blocks, lanes, cases = 8192, [], []
    for i in range(4):
        q, qc, k_sum, mt, _ = _case(300 + i, n_blocks, 1, n_head, H, D)
        ix = _build_index(kvm_state, k_sum, mt, n_blocks, H, D)
        qa = api.QueryAcc(kvm_state, 1, n_head, D, n_head_kv=H if terms else 0)
        qa.q_sum.copy_(dev(q))
        qa.q_count.copy_(dev(qc.astype(np.int32)))
        if terms:
            qa.refresh()
        lanes.append(dict(index=ix, query=qa, n_blocks=n_blocks, n_tokens=dev(np.full(n_blocks, 128, np.int32)),
                          budget_blocks=128, sink_blocks=1, window=api.KVWindow(kvm_state, 128 * 128, H, D, 128),
                          sel=api.SelectionBuffers(kvm_state, n_blocks, 128)))
        cases.append((q, qc, k_sum, mt))
    api.score_topk_lanes(kvm_state, lanes)
    for ln, (q, qc, k_sum, mt) in zip(lanes, cases):
        r = ln["sel"].result()
        assert r["status"] == 0
        want = O.score_retrieval(q, qc, k_sum, mt, n_head, H, D)
        got = host(ln["sel"].scores)[:n_blocks]
        assert np.array_equal(got.view(np.uint64), want.view(np.uint64))
        assert np.array_equal(r["ids"], O.pick_topk(want, 128, 1, 0))
        # (no planted-block check: with 8192 blocks and 128- or 256-dim heads some
        # random blocks outscore a planted one; the oracle's selection is the check)


def test_score_topk_from_reference_snapshot(kvm_state):
    """The mean-K index read out of a raw-store snapshot the reference's RawKvStore
    wrote (tests/golden/snap_score.bin.gz: block sums and token counts the store
    accumulated) scores and selects exactly as the oracle does on the same sums."""
    snap, meta, _, _, kf = golden_snapshot("snap_score")
    H, D, bt, n_blocks = meta["n_head_kv"], meta["head_dim"], meta["block_tokens"], meta["n_blocks"]
    n_head = 6 * H
    info, layers = api.read_snapshot(snap)
    k_sum, mt = layers[0]["k_sum"][None], layers[0]["mean_tokens"][None]
    # the store's sums are the ordered fp32 sums of the rows it was filled with
    want_sums, want_mt = O.meank_sums(kf[0], bt)
    assert np.array_equal(k_sum[0], want_sums) and np.array_equal(mt[0], want_mt)
    ix = _build_index(kvm_state, k_sum, mt, n_blocks, H, D)
    rng = np.random.default_rng(88)
    planted = rng.choice(np.arange(1, n_blocks), 12, replace=False)
    g = n_head // H
    q = np.zeros((1, n_head * D), np.float32)
    for b in planted:
        mean = k_sum[0, b] * (np.float32(1.0) / np.float32(mt[0, b]))
        for h in range(n_head):
            q[0, h * D:(h + 1) * D] += mean[(h // g) * D:(h // g + 1) * D]
    q += (rng.standard_normal(q.shape) * 0.1).astype(np.float32)
    qc = np.array([4], np.uint32)
    qa = api.QueryAcc(kvm_state, 1, n_head, D)
    qa.q_sum.copy_(dev(q))
    qa.q_count.copy_(dev(qc.astype(np.int32)))
    nt = dev(layers[0]["n_tokens"].astype(np.int32))
    sel = api.score_topk(kvm_state, ix, qa, n_blocks, nt, 32, 1, 0, None, api.KVWindow(kvm_state, 32 * bt, H, D, bt))
    want = O.score_retrieval(q, qc, k_sum, mt, n_head, H, D)
    assert np.array_equal(host(sel.scores)[:n_blocks].view(np.uint64), want.view(np.uint64))
    assert np.array_equal(sel.result()["ids"], O.pick_topk(want, 32, 1, 0))
    assert set(planted) <= set(sel.result()["ids"])


KATS = [
    # (scores, budget, sink, recent, mandatory, expected) -- kvmem_store_test.cpp
    ({5: 100.0, 6: 90.0, 3: 10.0}, 4, 1, 1, [], [0, 5, 6, 9]),
    ({3: 80.0, 5: 100.0, 6: 90.0, 9: -100.0}, 4, 1, 0, [], [0, 3, 5, 6]),
    ({2: 100.0, 3: 90.0, 4: 80.0, 8: -10.0, 9: -20.0}, 4, 1, 0, [8, 9], [0, 2, 8, 9]),
    ({}, 4, 2, 3, [0, 0, 5], [0, 1, 5, 9]),
    ({}, 4, 1, 2, [1, 2, 3, 4], [0, 2, 3, 4]),
    ({}, 4, 1, 0, [], [0, 7, 8, 9]),
    ({}, 100, 1, 0, [], list(range(10))),
]


@pytest.mark.parametrize("kat", range(len(KATS)))
def test_select_topk_reference_kats(kvm_state, kat):
    sc, budget, sink, recent, mand, want = KATS[kat]
    s = np.zeros(10)
    for i, v in sc.items():
        s[i] = v
    nt = dev(np.full(10, 128, np.int32))
    m = dev(np.array(mand, np.int32)) if mand else None
    res = api.select_topk(kvm_state, dev(s), nt, budget, sink, recent, m).result()
    assert list(res["ids"]) == want


def _scores(rng, trial, n):
    """Score sets for the selection: integers (long ties: the radix select),
    normals (the one-pass histogram, threshold bin ranked exactly), normals
    rounded to 2 decimals (equal keys inside the ranked bin: ties by id) and
    normals with infinities (not finite: the radix select)."""
    kind = trial % 4
    if kind == 0:
        return rng.integers(-3, 4, n).astype(np.float64)
    s = rng.standard_normal(n)
    if kind == 2:
        s = np.round(s, 2)
    if kind == 3:
        s[rng.choice(n, min(n, 3), replace=False)] = [np.inf, -np.inf, np.inf][:min(n, 3)]
    return s


def test_select_topk_random_vs_oracle(kvm_state):
    rng = np.random.default_rng(3)
    for trial in range(60):
        n = int(rng.integers(1, 8192))
        budget = int(rng.integers(0, min(n + 3, 600)))
        sink, recent = int(rng.integers(0, 4)), int(rng.integers(0, 4))
        s = _scores(rng, trial, n)
        mand = rng.integers(0, n, int(rng.integers(0, 6))).astype(np.int32)
        nt = np.full(n, 128, np.int32)
        res = api.select_topk(kvm_state, dev(s), dev(nt), budget, sink, recent,
                              dev(mand) if mand.size else None).result()
        want = O.pick_topk(s, budget, sink, recent, list(mand))
        assert np.array_equal(res["ids"], want), trial


def test_stage_plan_against_slot_map(kvm_state):
    w = api.KVWindow(kvm_state, 1024, 4, 256, 128)           # 8 slots
    s = np.zeros(20)
    s[[4, 9, 13]] = [3.0, 2.0, 1.0]
    nt = dev(np.full(20, 128, np.int32))
    # slots hold (block, base): slot 0 = (0, 0) matches, slot 1 = (4, 999) wrong base
    w.slot_block[:2] = dev(np.array([0, 4], np.int32))
    w.slot_base[:2] = dev(np.array([0, 999], np.int32))
    res = api.select_topk(kvm_state, dev(s), nt, 4, 1, 0, None, window=w).result()
    assert list(res["ids"]) == [0, 4, 9, 13]
    assert list(res["stage_slots"]) == [1, 2, 3]


def test_select_topk_maximum_size(kvm_state):
    """n = 8192 blocks (the most the selection takes) with long ties, distinct
    scores and infinities, each against the oracle; one block more is refused."""
    rng = np.random.default_rng(12)
    n = 8192
    nt = dev(np.full(n, 128, np.int32))
    for kind, budget in ((0, 700), (1, 700), (3, 4096), (2, 8192)):
        s = _scores(rng, kind, n)
        res = api.select_topk(kvm_state, dev(s), nt, budget, 1, 2).result()
        assert np.array_equal(res["ids"], O.pick_topk(s, budget, 1, 2)), (kind, budget)
    with pytest.raises(L.KvmError):
        api.select_topk(kvm_state, dev(np.zeros(n + 1)), dev(np.full(n + 1, 128, np.int32)), 8, 1, 0)


def test_topk_with_mandatory_blocks_from_row_ranges(kvm_state):
    """The turn's mandatory spans and force_pos become block ids on the host
    (kvm_retrieval_mandatory, llama-memory-kvmem.cpp:4306-4325) and the GPU
    top-k keeps them within the budget, newest first, exactly as the oracle's
    pick_topk_ungrouped restatement does; the query span stands in when the
    turn has no explicit spans."""
    rng = np.random.default_rng(17)
    bt, n_blocks, budget = 128, 300, 24
    nt = np.full(n_blocks, bt, np.int64)
    nt[-1] = 61
    total = int(nt.sum())
    scores = rng.standard_normal(n_blocks)
    cases = [([(1000, 1900), (30000, 30100)], -1, 0, 5000),     # explicit spans + force_pos
             (None, 36000, 0, -1),                               # query span to the store's end
             ([(0, total)], -1, 0, 100),                         # every block mandatory: trimmed to the budget
             ([], 36000, 0, total - 1)]                          # explicit, empty spans: force_pos alone
    for spans, qb, qe, fp in cases:
        mand = api.retrieval_mandatory(nt, spans, qb, qe, fp)
        want = O.pick_topk(scores, budget, 1, 2, mandatory=mand)
        sel = api.select_topk(kvm_state, dev(scores), dev(nt.astype(np.int32)), budget, 1, 2,
                              mandatory=dev(mand.astype(np.int32)))
        r = sel.result()
        assert r["status"] == 0 and np.array_equal(r["ids"], want), (spans, qb, fp)
        kept = set(r["ids"].tolist())
        if len(set(mand.tolist())) + 3 <= budget:
            assert set(mand.tolist()) <= kept
