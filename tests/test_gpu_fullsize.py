"""Parity at the workloads' full sizes, through the C ABI, against the oracle:

* stage-in of 128 distinct 128-token blocks drawn from a 2,048-block
  (262,144-token) pinned history into a 16,384-cell window, every K and V byte;
* chunked prefill of a 2,048-token bf16 chunk over a 34,816-cell window
  (32,768 window cells + the chunk's own), sampled tokens over all 24 heads
  against the float64 softmax on the kernel's f16 operands;
* four conversation lanes of 32,768-cell windows in one decode launch, one bf16
  token each, every lane against the ggml-semantics oracle.
"""
import os

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import check_attention, dev, host
from kvmem_amd import api, workload as W, _lib as L

pytestmark = pytest.mark.gpu

H, G, D, BT = 4, 6, 256, 128
K_ROW, V_ROW = H * D // 32 * 34, H * D // 32 * 18
THREADS = min(16, os.cpu_count() or 1)


def _random_rows(rng, n, row, bsz):
    """n ggml rows of random quants with finite fp16 block scales in [2^-9, 2^-2)."""
    rows = rng.integers(0, 256, (n, row), dtype=np.uint8)
    nb = row // bsz
    d = rng.uniform(2.0 ** -9, 2.0 ** -2, (n, nb)).astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    rows.reshape(n, nb, bsz)[..., :2] = d
    return rows


def test_stagein_128_blocks_from_256k_history(kvm_state):
    """128 blocks at uniform-random original positions in a 262,144-token
    history, re-RoPE'd (64 dims, theta 1e7) to window positions 128 k, FWHT 256,
    q8_0 requantised; V moved unchanged.  Every byte equals the oracle's."""
    n_tok = 262144
    n_blocks = n_tok // BT
    rng = np.random.default_rng(0xC0FFEE03)
    kr = _random_rows(rng, n_tok, K_ROW, 34)
    vr = _random_rows(rng, n_tok, V_ROW, 18)
    chosen = np.sort(W.distinct_ids(0xC0FFEE03, 0, 128, 0, n_blocks))
    # the chosen blocks hold real q8_0 rows of N(0,1) keys
    for b in chosen:
        kr[b * BT:(b + 1) * BT] = O.quant(O.T_Q8_0, rng.standard_normal(BT * H * D).astype(np.float32)).reshape(BT, -1)
    hist = api.History(kr, vr)
    scores = np.zeros(n_blocks)
    scores[chosen] = 1.0
    w = api.KVWindow(kvm_state, 128 * BT, H, D, BT)
    sel = api.select_topk(kvm_state, dev(scores), dev(np.full(n_blocks, BT, np.int32)), 128, 0, 0, None, window=w)
    api.stagein_selection(kvm_state, hist, w, sel, 64, 1e7)
    res = sel.result()
    assert res["status"] == 0 and np.array_equal(res["ids"], chosen)
    assert np.array_equal(res["to_base"], np.arange(0, 128 * BT, BT)) and len(res["stage_slots"]) == 128
    ek, ev = w.export_rows(0, 128 * BT)
    ek, ev = host(ek), host(ev)
    theta = O.rope_theta(1e7, 1.0, 64)
    for k, b in enumerate(chosen):
        want = O.stagein_k(kr[b * BT:(b + 1) * BT].reshape(-1), BT, H, D, 64, 256, k * BT, theta)
        assert np.array_equal(ek[k * BT:(k + 1) * BT].reshape(-1), want), (k, b)
        assert np.array_equal(ev[k * BT:(k + 1) * BT], vr[b * BT:(b + 1) * BT]), (k, b)
    assert np.array_equal(host(w.cell_pos), np.arange(128 * BT))
    assert np.array_equal(host(w.slot_block), chosen) and np.array_equal(host(w.slot_base), res["to_base"])


def test_prefill_2048_chunk_over_34816_cells(kvm_state):
    """A 2,048-token bf16 query chunk at positions 32768..34815, causal, over a
    32,768-cell q8_0/q4_0 window plus the chunk's own quantised cells; 24 q heads
    over 4 kv heads.  Sampled tokens (first, tile and split boundaries, middle,
    last), all 24 heads, against the float64 softmax over the f16 operands the
    MFMA path multiplies (K, V dequantised and rounded to f16; bf16 Q is exact
    in f16 here): max |err| <= 2e-3 and <= 1e-3 max |ref|."""
    chunk, win = 2048, 32768
    n = win + chunk
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0xC0FFEE04)
    w = api.KVWindow(kvm_state, n, H, D, BT)
    for c0 in range(0, n, 8192):
        m = min(8192, n - c0)
        k = api.quantize_rows(kvm_state, L.T_Q8_0, torch.randn((m, H * D), generator=gen, device="cuda"))
        v = api.quantize_rows(kvm_state, L.T_Q4_0, torch.randn((m, H * D), generator=gen, device="cuda"))
        w.import_rows(c0, k, v, torch.arange(c0, c0 + m, dtype=torch.int32, device="cuda"))
    q = torch.randn((chunk, H * G, D), generator=gen, device="cuda").to(torch.bfloat16)
    q_pos = torch.arange(win, n, dtype=torch.int32, device="cuda")
    out = host(api.fa_prefill(kvm_state, w, q, q_pos, H * G, D ** -0.5))
    ek, ev = w.export_rows(0, n)
    ek, ev = host(ek), host(ev)
    kh = O.dequant(O.T_Q8_0, ek.reshape(-1), n * H * D).astype(np.float16).view(np.uint8).reshape(n, -1)
    vh = O.dequant(O.T_Q4_0, ev.reshape(-1), n * H * D).astype(np.float16).view(np.uint8).reshape(n, -1)
    toks = np.array([0, 1, 63, 64, 127, 128, 1023, 1024, 1535, 2046, 2047])
    qf = q.float().cpu().numpy()[toks]
    assert np.array_equal(qf.astype(np.float16).astype(np.float32), qf)
    ref = O.fa_f64(O.T_F16, O.T_F16, qf, kh, vh, host(w.cell_pos), host(q_pos)[toks], H * G, H, D, D ** -0.5,
                   n_threads=THREADS)
    check_attention(out[toks], ref)
    assert np.isfinite(out).all()


def test_fa_decode_four_lanes_32k(kvm_state):
    """Four 32,768-cell q8_0/q4_0 windows in one kvm_fa_decode_lanes launch, one
    bf16 token per lane, 24 q heads over 4 kv heads: a full window, one with
    scattered empty cells, a half-filled one and one whose token sits in the
    middle (later cells are masked).  Each lane against the ggml-semantics
    oracle."""
    n = 32768
    rng = np.random.default_rng(0xC0FFEE05)
    windows, qs, qps, refs_in = [], [], [], []
    for lane in range(4):
        kr = O.quant(O.T_Q8_0, rng.standard_normal(n * H * D).astype(np.float32)).reshape(n, -1)
        vr = O.quant(O.T_Q4_0, rng.standard_normal(n * H * D).astype(np.float32)).reshape(n, -1)
        cp = np.arange(n, dtype=np.int32)
        qpos = n - 1
        if lane == 1:
            cp[rng.choice(n, 3000, replace=False)] = -1
        elif lane == 2:
            cp[n // 2:] = -1
            qpos = n // 2 - 1
        elif lane == 3:
            qpos = 20000
        w = api.KVWindow(kvm_state, n, H, D, BT)
        w.import_rows(0, dev(kr), dev(vr), dev(cp))
        qt = torch.from_numpy(rng.standard_normal((1, H * G, D)).astype(np.float32)).to(torch.bfloat16)
        windows.append(w)
        qs.append(qt.cuda())
        qps.append(dev(np.array([qpos], np.int32)))
        refs_in.append((qt.float().numpy(), kr, vr, cp, np.array([qpos], np.int32)))
    outs = api.fa_decode_lanes(kvm_state, windows, qs, qps, H * G, D ** -0.5)
    for lane, (o, (q, kr, vr, cp, qp)) in enumerate(zip(outs, refs_in)):
        ref = O.fa_ggml(O.T_Q8_0, O.T_Q4_0, q, kr, vr, cp, qp, H * G, H, D, D ** -0.5, n_threads=THREADS)
        check_attention(host(o), ref)
