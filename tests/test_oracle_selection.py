"""Oracle mean-K (raw_kv_store.cpp:215-234, 987-1006), scoring
(llama-memory-kvmem.cpp:4149-4196), top-k (kvmem_store.cpp:482-623) and the
window layout (kvmem_store.cpp:758-882, llama-memory-kvmem.cpp:1958-1993)."""
import numpy as np
import pytest

import oracle as O

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs the reference sources)")


# ---------------------------------------------------------------- top-k KATs
def test_topk_budget_sink_recent_kat():
    """kvmem_store_test.cpp:284-314 (recent kept, hottest middle blocks)."""
    s = np.zeros(10)
    s[5], s[6], s[3] = 100.0, 90.0, 10.0
    sel = O.pick_topk(s, 4, sink_blocks=1, recent_blocks=1)
    assert list(sel) == [0, 5, 6, 9]


def test_topk_zero_recent_kat():
    """kvmem_store_test.cpp:316-339."""
    s = np.zeros(10)
    s[3], s[5], s[6], s[9] = 80.0, 100.0, 90.0, -100.0
    assert list(O.pick_topk(s, 4, 1, 0)) == [0, 3, 5, 6]


def test_topk_mandatory_inside_budget_kat():
    """kvmem_store_test.cpp:433-456."""
    s = np.zeros(10)
    s[2], s[3], s[4], s[8], s[9] = 100.0, 90.0, 80.0, -10.0, -20.0
    assert list(O.pick_topk(s, 4, 1, 0, mandatory=[8, 9])) == [0, 2, 8, 9]


def test_topk_mandatory_dedup_and_recent_best_effort_kat():
    """kvmem_store_test.cpp:458-475."""
    assert list(O.pick_topk(np.zeros(10), 4, 2, 3, mandatory=[0, 0, 5])) == [0, 1, 5, 9]


def test_topk_mandatory_overflow_trims_oldest_kat():
    """kvmem_store_test.cpp:477-504: sink {0} + mandatory {1,2,3,4} > budget 4 keeps the newest."""
    assert list(O.pick_topk(np.zeros(10), 4, 1, 2, mandatory=[1, 2, 3, 4])) == [0, 2, 3, 4]


def test_topk_all_fit_and_empty_kat():
    """kvmem_store_test.cpp:763-781."""
    assert list(O.pick_topk(np.zeros(3), 100)) == [0, 1, 2]
    assert list(O.pick_topk(np.zeros(0), 4)) == []
    assert list(O.pick_topk(np.zeros(5), 0)) == [0, 1, 2, 3, 4]        # budget 0 selects all


def test_topk_ties_prefer_newest():
    """Equal scores fall back to the higher block id (kvmem_store.cpp:604-609)."""
    assert list(O.pick_topk(np.zeros(10), 4, 1, 0)) == [0, 7, 8, 9]
    s = np.zeros(10)
    s[2] = -0.0
    s[3] = 0.0
    assert list(O.pick_topk(s, 3, 1, 0)) == [0, 8, 9]


def test_topk_brute_force_small():
    rng = np.random.default_rng(11)
    for trial in range(300):
        n = int(rng.integers(1, 14))
        budget = int(rng.integers(0, n + 2))
        sink, recent = int(rng.integers(0, 3)), int(rng.integers(0, 3))
        s = rng.integers(-3, 4, n).astype(np.float64)           # many ties
        mand = list(rng.integers(0, n + 1, int(rng.integers(0, 3))))
        sel = O.pick_topk(s, budget, sink, recent, mand)
        if budget == 0 or n <= budget:
            assert list(sel) == list(range(n))
            continue
        kept = []
        for i in range(min(sink, n)):
            if len(kept) < budget and i not in kept:
                kept.append(i)
        for m in reversed(mand):
            if len(kept) < budget and m < n and m not in kept:
                kept.append(m)
        for i in range(min(recent, n)):
            if len(kept) < budget and n - 1 - i not in kept:
                kept.append(n - 1 - i)
        rest = sorted((i for i in range(n) if i not in kept), key=lambda i: (-s[i], -i))
        kept += rest[:budget - len(kept)]
        assert list(sel) == sorted(kept), (trial, n, budget, sink, recent, mand)


@needs_ref
def test_topk_matches_reference_library():
    rng = np.random.default_rng(12)
    for trial in range(200):
        n = int(rng.integers(1, 3000))
        bt = 128
        total = n * bt - int(rng.integers(0, bt))
        budget = int(rng.integers(0, n + 10))
        sink, recent = int(rng.integers(0, 4)), int(rng.integers(0, 4))
        if trial % 3 == 0:
            s = rng.integers(-2, 3, n).astype(np.float64)
        else:
            s = rng.standard_normal(n)
        mand = list(rng.integers(0, n, int(rng.integers(0, 5))))
        got = O.pick_topk(s, budget, sink, recent, mand)
        want = O.ref_pick_topk(total, bt, budget * bt, sink, recent, s, mand)
        assert np.array_equal(got, want), trial


# ---------------------------------------------------------------- window layout
def test_window_layout_closed_form():
    n_tokens = np.full(100, 128, np.uint32)
    n_tokens[-1] = 40
    sel = np.array([0, 3, 10, 99], np.uint32)
    to_base, cell_pos, total = O.window_layout(sel, n_tokens, 128, 6)
    assert list(to_base) == [0, 128, 256, 384] and total == 424
    assert np.array_equal(cell_pos[:384], np.arange(384))
    assert np.array_equal(cell_pos[384:424], np.arange(384, 424))
    assert np.all(cell_pos[424:] == -1)


@needs_ref
def test_window_layout_matches_set_selection():
    """to_base of every remap equals the reference's set_selection, also after a
    reselection (baked positions then come from the previous window)."""
    rng = np.random.default_rng(13)
    for trial in range(100):
        n = int(rng.integers(2, 400))
        total_tokens = n * 128 - int(rng.integers(0, 128))
        steps = [np.sort(rng.choice(n, int(rng.integers(1, n + 1)), replace=False)) for _ in range(2)]
        ref = O.ref_set_selection_seq(total_tokens, 128, steps)
        n_tokens = np.array([min(128, total_tokens - 128 * b) for b in range(n)], np.uint32)
        to_base, _, total = O.window_layout(steps[-1], n_tokens, 128, n)
        assert np.array_equal(ref["remaps"]["block_id"], steps[-1])
        assert np.array_equal(ref["remaps"]["to_base"], to_base)
        assert ref["total"] == total


@needs_ref
def test_selection_remap_kat_via_reference():
    """kvmem_store_test.cpp:53-110 through the reference library: from/to bases and skips."""
    r = O.ref_set_selection_seq(128 * 5, 128, [[4, 0, 2]])
    rm = r["remaps"]
    assert list(rm["block_id"]) == [0, 2, 4] and list(rm["to_base"]) == [0, 128, 256]
    assert list(rm["from_base"]) == [0, 256, 512] and list(rm["skip"]) == [1, 0, 0]
    assert list(r["stage_out"]) == [1, 3] and r["total"] == 384
    r2 = O.ref_set_selection_seq(128 * 5, 128, [[4, 0, 2], [0, 2, 3]])
    assert list(r2["stage_in"]) == [3] and list(r2["stage_out"]) == [4]
    assert list(r2["remaps"]["skip"]) == [1, 1, 0] and r2["remaps"]["from_base"][2] == 384


# ---------------------------------------------------------------- mean-K
def _kat_input(n, e):
    vals = np.array([1e7, .125, -1e7, .3, -7.1, .001, 9.7], dtype=np.float32)
    t = np.arange(n)[:, None]
    d = np.arange(e)[None, :]
    return vals[(t + d) % 7]


@pytest.mark.parametrize("bt", [32, 128])
def test_meank_cancellation_kat(bt):
    """raw_kv_store_test.cpp:26-94: ordered fp32 sum times 1/n, compared with memcmp,
    on values that cancel, written in uneven 11-token batches."""
    e = 1024
    n = 2 * bt + 7
    k = _kat_input(n, e)
    sums, mt = O.meank_sums(k, bt, chunk=11)
    for b in range(len(mt)):
        rows = k[b * bt:min(n, (b + 1) * bt)]
        exp = np.zeros(e, np.float32)
        for r in rows:
            exp = (exp + r).astype(np.float32)
        inv = np.float32(1.0) / np.float32(len(rows))
        out = np.zeros(e, np.float32)
        O.lib().oracle_meank_normalize(O._p(sums[b]), int(mt[b]), O._p(out), e)
        assert mt[b] == len(rows)
        assert np.array_equal(out.view(np.uint32), (exp * inv).astype(np.float32).view(np.uint32))


@needs_ref
@pytest.mark.parametrize("chunk", [1, 11, 128, 1000])
def test_meank_matches_reference_library(chunk):
    rng = np.random.default_rng(chunk)
    k = rng.standard_normal((700, 256)).astype(np.float32)
    k[::5] *= 1e5
    sums, mt = O.meank_sums(k, 128, chunk=chunk)
    ref = O.ref_mean_k(k, 128, chunk)
    for b in range(len(mt)):
        out = np.zeros(256, np.float32)
        O.lib().oracle_meank_normalize(O._p(sums[b]), int(mt[b]), O._p(out), 256)
        assert np.array_equal(out.view(np.uint32), ref[b].view(np.uint32))


# ---------------------------------------------------------------- scoring
def _scoring_case(seed, n_blocks=64, n_layer=1, n_head=24, n_head_kv=4, d=256, planted=(5, 17, 40)):
    rng = np.random.default_rng(seed)
    k_sum = rng.standard_normal((n_layer, n_blocks, n_head_kv * d)).astype(np.float32) * 128
    mt = np.full((n_layer, n_blocks), 128, np.uint32)
    mean = k_sum / np.float32(128)
    g = n_head // n_head_kv
    q = np.zeros((n_layer, n_head * d), np.float32)
    for il in range(n_layer):
        for h in range(n_head):
            q[il, h * d:(h + 1) * d] = sum(mean[il, b, (h // g) * d:(h // g + 1) * d] for b in planted)
    q += rng.standard_normal(q.shape).astype(np.float32) * 0.1
    return q, np.full(n_layer, 4, np.uint32), k_sum, mt


def _score_f32_loop(q_sum, q_count, k_sum, mt, n_head, H, d, b):
    """The reference loop with numpy float32 scalars: same operation order."""
    f = np.float32
    g = n_head // H
    acc, nlay = 0.0, 0
    for il in range(len(q_count)):
        if q_count[il] == 0:
            continue
        inv = f(1.0) / f(mt[il, b]) if mt[il, b] else None
        mk = (k_sum[il, b] * inv).astype(np.float32) if inv is not None else np.zeros(H * d, np.float32)
        layer = 0.0
        invq = f(1.0) / f(int(q_count[il]) * max(1, g))
        for h in range(H):
            qh = np.zeros(d, np.float32)
            for gi in range(g):
                qh = (qh + q_sum[il, (h * g + gi) * d:(h * g + gi + 1) * d]).astype(np.float32)
            dot = nq = nk = f(0.0)
            kh = mk[h * d:(h + 1) * d]
            for j in range(d):
                qv = f(qh[j] * invq)
                dot = f(dot + f(qv * kh[j]))
                nq = f(nq + f(qv * qv))
                nk = f(nk + f(kh[j] * kh[j]))
            layer += float(f(dot / f(f(np.sqrt(nq)) * f(np.sqrt(nk)) + f(1e-6))))
        acc += layer / H
        nlay += 1
    return acc / nlay if nlay else 0.0


def test_score_bit_exact_against_float32_loop():
    q, qc, ks, mt = _scoring_case(21, n_blocks=6, n_layer=2, n_head=8, n_head_kv=2, d=64, planted=(1,))
    qc[1] = 3
    s = O.score_retrieval(q, qc, ks, mt, 8, 2, 64)
    for b in range(6):
        assert s[b] == _score_f32_loop(q, qc, ks, mt, 8, 2, 64, b)


def test_score_properties():
    q, qc, ks, mt = _scoring_case(22)
    s = O.score_retrieval(q, qc, ks, mt, 24, 4, 256)
    assert np.all(np.abs(s) <= 1.0)
    assert set(np.argsort(-s)[:3]) == {5, 17, 40}
    # float64 evaluation of the same cosine average
    g = 6
    mean = ks[0].astype(np.float64) / 128.0
    for b in (0, 5, 33):
        cs = []
        for h in range(4):
            qh = q[0].reshape(24, 256)[h * g:(h + 1) * g].astype(np.float64).sum(0) / (4 * g)
            kh = mean[b, h * 256:(h + 1) * 256]
            cs.append(qh @ kh / (np.linalg.norm(qh) * np.linalg.norm(kh) + 1e-6))
        assert abs(s[b] - np.mean(cs)) < 1e-5
    # moving one query head into another kv group changes the scores (GQA grouping matters)
    q2 = q.copy().reshape(1, 24, 256)
    q2[0, [0, 6]] = q2[0, [6, 0]]
    q2[0, 0] += 5.0
    assert not np.array_equal(O.score_retrieval(q2.reshape(1, -1), qc, ks, mt, 24, 4, 256), s)


def test_score_missing_blocks_and_layers():
    q, qc, ks, mt = _scoring_case(23, n_blocks=8, n_layer=2, planted=(1, 5))
    present = np.ones(8, np.uint8)
    present[3] = 0
    mt[1, 4] = 0                                       # layer 1 of block 4 has no K
    qc[0] = 0                                          # layer 0 has no query
    s = O.score_retrieval(q, qc, ks, mt, 24, 4, 256, present=present)
    assert s[3] == 0.0 and s[4] == 0.0                 # missing block; zero mean-K -> cosine 0
    assert np.all(s[[0, 1, 2, 5, 6, 7]] != 0.0)
    qc[:] = 0
    assert np.all(O.score_retrieval(q, qc, ks, mt, 24, 4, 256, present=present) == 0.0)


# ------------------------------------------ scoring pinned by the closed form
def test_score_closed_form_where_every_term_matters():
    """Norms near 1e-6 (the epsilon weighs like them), g = 3, three layers
    with query counts 5, 0 and 2, token counts 1..128 and a block without K in
    one layer: the oracle equals the float64 closed form within 2e-5, and each
    plausible mistake (invq without g, the epsilon inside the square root or
    missing or in the numerator, interleaved query heads, a layer average
    weighted by q_count or counting the layer without queries) moves some
    score by more than 50 times that."""
    from scoring_cases import VARIANTS, score_f64, tiny_norm_case
    n_head, H, d = 6, 2, 128
    q, qc, ks, mt = tiny_norm_case(41, n_head=n_head, H=H, d=d)
    got = O.score_retrieval(q, qc, ks, mt, n_head, H, d)
    want = score_f64(q, qc, ks, mt, n_head, H, d)
    tol = 2e-5
    assert np.max(np.abs(got - want)) < tol, np.max(np.abs(got - want))
    assert np.ptp(want) > 0.1                          # the cosines are not all alike
    for v in VARIANTS:
        wrong = score_f64(q, qc, ks, mt, n_head, H, d, variant=v)
        assert np.max(np.abs(wrong - want)) > 50 * tol, v
    # a block whose mean-K is missing in one layer still averages that layer's zero
    only = score_f64(q, qc[:1], ks[:1], mt[:1], n_head, H, d)
    assert abs(got[3] - only[3] / 2) < tol            # layers 0 and 2 count, layer 2 gives 0 for block 3


def test_score_closed_form_on_ordinary_magnitudes_with_unequal_counts():
    """The same closed form at the scale of real activations (norms ~1..100,
    where the epsilon is negligible), four layers with query counts 1, 7, 0, 3."""
    from scoring_cases import score_f64
    rng = np.random.default_rng(42)
    n_head, H, d, nb, nl = 8, 2, 64, 9, 4
    ks = (rng.standard_normal((nl, nb, H * d)) * 40).astype(np.float32)
    mt = rng.integers(1, 129, (nl, nb)).astype(np.uint32)
    q = (rng.standard_normal((nl, n_head * d)) * 3).astype(np.float32)
    qc = np.array([1, 7, 0, 3], np.uint32)
    got = O.score_retrieval(q, qc, ks, mt, n_head, H, d)
    assert np.max(np.abs(got - score_f64(q, qc, ks, mt, n_head, H, d))) < 1e-5
    for v in ("interleaved_heads", "all_layers"):
        assert np.max(np.abs(score_f64(q, qc, ks, mt, n_head, H, d, variant=v) - got)) > 1e-3, v
