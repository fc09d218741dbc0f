"""The reference's CPU-runnable case at its stated size, end to end on the GPU:
one attention layer with 8 query heads over 2 kv heads, head_dim 128, an fp16
K/V history of 16,384 tokens in 128-token blocks with Q/K/V ~ N(0,1), the
query built from the mean keys of 4 planted blocks plus N(0, 0.1) noise, a
4,096-token budget (32 blocks including 1 sink) plus a 512-token generation
reserve, one decode token.  The selection is checked bit for bit against the
oracle (scores, ids, window layout; the planted blocks among the ids); the
fp16 window is filled the way the reference's product stage-in fills an fp16
cache (the rows copied unchanged, each cell keeping its original position);
the attention is checked against the float64 softmax over the same cells."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import check_attention, dev, host
from kvmem_amd import api, _lib as L

pytestmark = pytest.mark.gpu

H_Q, H, D, BT = 8, 2, 128, 128
N_TOK, BUDGET, GEN = 16384, 4096, 512


def test_fp16_16k_history_end_to_end(kvm_state):
    st = kvm_state
    rng = np.random.default_rng(0xC0FFEE01)
    n_blocks = N_TOK // BT
    k = rng.standard_normal((N_TOK, H * D)).astype(np.float32)
    v = rng.standard_normal((N_TOK, H * D)).astype(np.float32)
    k16 = k.astype(np.float16)
    v16 = v.astype(np.float16)
    kr = k16.view(np.uint8).reshape(N_TOK, -1)
    vr = v16.view(np.uint8).reshape(N_TOK, -1)
    # mean-K index over the history's K (fp32 sums of the rows as captured)
    ix = api.MeanKIndex(st, 1, n_blocks, H, D, BT)
    ix.add(0, 0, dev(k))
    sums, mt = O.meank_sums(k, BT)
    planted = rng.choice(np.arange(1, n_blocks), 4, replace=False)
    mean = sums / mt[:, None].astype(np.float32)
    g = H_Q // H
    qrow = np.zeros((1, H_Q * D), np.float32)
    for hq in range(H_Q):
        hk = hq // g
        qrow[0, hq * D:(hq + 1) * D] = mean[planted][:, hk * D:(hk + 1) * D].sum(0)
    qrow += (rng.standard_normal(qrow.shape) * 0.1).astype(np.float32)
    qa = api.QueryAcc(st, 1, H_Q, D)
    qa.reset()
    qa.add(0, dev(qrow))
    n_slots = (BUDGET + GEN) // BT
    w = api.KVWindow(st, n_slots * BT, H, D, BT, L.T_F16, L.T_F16)
    n_tokens = dev(np.full(n_blocks, BT, np.int32))
    sel = api.score_topk(st, ix, qa, n_blocks, n_tokens, BUDGET // BT, 1, 0, None, w)
    res = sel.result()
    want_scores = O.score_retrieval(qrow, np.array([1], np.uint32), sums[None], mt[None], H_Q, H, D)
    assert np.array_equal(host(sel.scores).view(np.uint64), want_scores.view(np.uint64))
    want_ids = O.pick_topk(want_scores, BUDGET // BT, 1, 0)
    assert np.array_equal(res["ids"], want_ids) and want_ids[0] == 0
    assert set(planted.tolist()) <= set(res["ids"].tolist())
    to_base, _, total = O.window_layout(want_ids.astype(np.uint32), np.full(n_blocks, BT, np.uint32), BT, n_slots)
    assert np.array_equal(res["to_base"], to_base) and res["total"] == total == BUDGET
    # slot k takes the k-th selected block, rows unchanged at their original positions
    for kk, b in enumerate(res["ids"]):
        rows = slice(int(b) * BT, (int(b) + 1) * BT)
        w.import_rows(kk * BT, dev(kr[rows]), dev(vr[rows]), dev(np.arange(rows.start, rows.stop, dtype=np.int32)))
    # the decode token's own K/V row in the first generation cell, at position N_TOK
    kt = rng.standard_normal((1, H * D)).astype(np.float16)
    vt = rng.standard_normal((1, H * D)).astype(np.float16)
    w.import_rows(BUDGET, dev(kt.view(np.uint8).reshape(1, -1)), dev(vt.view(np.uint8).reshape(1, -1)),
                  dev(np.array([N_TOK], np.int32)))
    q = rng.standard_normal((1, H_Q, D)).astype(np.float32)
    q_pos = np.array([N_TOK], np.int32)
    out = host(api.fa_decode(st, w, dev(q), dev(q_pos), H_Q, D ** -0.5))
    ek, ev = w.export_rows(0, w.n_cells)
    cp = host(w.cell_pos)
    assert (cp >= 0).sum() == BUDGET + 1
    qh = q.astype(np.float16).astype(np.float32)          # ggml rounds Q to fp16 for an f16 K
    ref = O.fa_f64(L.T_F16, L.T_F16, qh, host(ek), host(ev), cp, q_pos, H_Q, H, D, D ** -0.5)
    check_attention(out, ref)
