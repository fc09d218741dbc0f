"""GPU flash attention over the window against the ggml-semantics oracle
(tolerance 2e-3 max-abs and 1e-3 relative to max |ref|) and the float64 anchor."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import check_attention, dev, host, rand_rows
from kvmem_amd import api, _lib as L

pytestmark = pytest.mark.gpu


def _window(st, rng, n_cells, H, D, kt, vt, live=None, holes=0, kscale=1.0):
    w = api.KVWindow(st, n_cells, H, D, 128, kt, vt)
    kr, vr = rand_rows(rng, n_cells, H, D, kt, vt, kscale)
    cp = np.arange(n_cells, dtype=np.int32)
    if live is not None:
        cp[live:] = -1
    if holes:
        cp[rng.choice(n_cells, holes, replace=False)] = -1
    w.import_rows(0, dev(kr), dev(vr), dev(cp))
    return w, kr, vr, cp


CASES = [
    # n_cells, H, G, D, tokens, kt, vt, kscale
    (4096, 4, 6, 256, 4, L.T_Q8_0, L.T_Q4_0, 1.0),      # MTP3 verify, 24 rows per kv head
    (4096, 4, 6, 256, 1, L.T_Q8_0, L.T_Q4_0, 1.0),      # single decode token
    (2048, 2, 4, 128, 1, L.T_F16, L.T_F16, 1.0),        # fp16 cache, head_dim 128
    (2048, 2, 4, 128, 3, L.T_Q8_0, L.T_Q4_0, 3.0),      # peaked softmax
    (1024, 4, 8, 256, 4, L.T_F16, L.T_F16, 2.0),        # 32 rows per kv head
    (4096, 4, 6, 256, 4, L.T_Q4_0, L.T_Q4_0, 1.0),      # q4_0 K cache (held as q8_0 quants)
    (2048, 2, 4, 128, 1, L.T_Q4_0, L.T_Q4_0, 3.0),
]


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("qdt", ["f32", "bf16"])
def test_fa_decode_parity(kvm_state, case, qdt):
    n_cells, H, G, D, T, kt, vt, ks = CASES[case]
    rng = np.random.default_rng(case)
    w, kr, vr, cp = _window(kvm_state, rng, n_cells, H, D, kt, vt, live=n_cells - 100, holes=50, kscale=ks)
    q = rng.standard_normal((T, H * G, D)).astype(np.float32)
    if qdt == "bf16":
        qt = torch.from_numpy(q).to(torch.bfloat16)
        q = qt.float().numpy()
        qd = qt.cuda()
    else:
        qd = dev(q)
    qp = np.arange(n_cells - 100 - T, n_cells - 100, dtype=np.int32)
    scale = 1.0 / np.sqrt(D)
    out = host(api.fa_decode(kvm_state, w, qd, dev(qp), H * G, scale))
    ref = O.fa_ggml(kt, vt, q, kr, vr, cp, qp, H * G, H, D, scale)
    if kt in (L.T_Q8_0, L.T_Q4_0):
        check_attention(out, ref)
        f64 = O.fa_f64(kt, vt, q, kr, vr, cp, qp, H * G, H, D, scale)
        assert np.abs(out - f64).max() <= 3e-2 * np.abs(f64).max()      # Q -> q8_0 as in ggml
    else:
        # ggml-CPU accumulates f16 V in an fp16 vector (ggml_vec_mad_f16), itself off
        # the exact result by more than the stated tolerance; the GPU accumulates in
        # fp32 and is held to the tolerance against the float64 softmax over the same
        # fp16 Q (ggml rounds Q to fp16 for an f16 K).
        qh = q.astype(np.float16).astype(np.float32)
        f64 = O.fa_f64(kt, vt, qh, kr, vr, cp, qp, H * G, H, D, scale)
        check_attention(out, f64)
        assert np.abs(out - ref).max() <= 2e-2 * np.abs(ref).max()


@pytest.mark.parametrize("T", [4, 1])
def test_fa_decode_full_window(kvm_state, T):
    """The decode workload at its real shape: a 32,768-cell q8_0/q4_0 window,
    24 query heads over 4 kv heads, head_dim 256, bf16 query; 4 tokens (24 rows
    per kv head: one full row tile and one packed) or 1 token (6 rows: one
    packed tile), with empty cells spread through the window."""
    rng = np.random.default_rng(40 + T)
    H, G, D, n = 4, 6, 256, 32768
    w, kr, vr, cp = _window(kvm_state, rng, n, H, D, L.T_Q8_0, L.T_Q4_0, holes=300)
    qt = torch.from_numpy(rng.standard_normal((T, H * G, D)).astype(np.float32)).to(torch.bfloat16)
    q = qt.float().numpy()
    qp = np.arange(n - T, n, dtype=np.int32)
    out = host(api.fa_decode(kvm_state, w, qt.cuda(), dev(qp), H * G, D ** -0.5))
    ref = O.fa_ggml(L.T_Q8_0, L.T_Q4_0, q, kr, vr, cp, qp, H * G, H, D, D ** -0.5)
    check_attention(out, ref)


def test_fa_decode_masks_and_empty_rows(kvm_state):
    rng = np.random.default_rng(7)
    H, G, D, n = 4, 6, 256, 1024
    w, kr, vr, cp = _window(kvm_state, rng, n, H, D, L.T_Q8_0, L.T_Q4_0)
    q = rng.standard_normal((4, H * G, D)).astype(np.float32)
    qp = np.array([-1, 0, 500, 1023], np.int32)          # token 0 sees nothing, token 1 sees cell 0
    out = host(api.fa_decode(kvm_state, w, dev(q), dev(qp), H * G, 0.0625))
    assert np.all(out[0] == 0)
    V = O.dequant(O.T_Q4_0, vr[0].reshape(-1), H * D).reshape(H, D)
    for h in range(H * G):
        np.testing.assert_allclose(out[1, h], V[h // G], rtol=2e-3, atol=2e-3)
    ref = O.fa_ggml(L.T_Q8_0, L.T_Q4_0, q, kr, vr, cp, qp, H * G, H, D, 0.0625)
    check_attention(out, ref)


def _v_rows(vt, vr, n, H, D):
    if vt == L.T_F16:
        return np.ascontiguousarray(vr).view(np.float16).astype(np.float32).reshape(n, H, D)
    return O.dequant(vt, np.ascontiguousarray(vr).reshape(-1), n * H * D).reshape(n, H, D)


@pytest.mark.parametrize("kt,vt", [(L.T_Q8_0, L.T_Q4_0), (L.T_F16, L.T_F16)])
@pytest.mark.parametrize("T", [4, 1])
def test_fa_decode_closed_forms(kvm_state, kt, vt, T):
    """Two cases the mathematics fixes without an attention oracle: identical
    keys (every visible score equals the maximum, P = 1, the output is the mean
    of the visible V rows) and a single visible key (the output is that cell's
    V row); V rows from the dequantiser."""
    rng = np.random.default_rng(31 + T)
    H, G, D, n = 4, 6, 256, 2048
    w, kr, vr, cp = _window(kvm_state, rng, n, H, D, kt, vt)
    kr[:] = kr[0]                                           # identical keys
    w.import_rows(0, dev(kr), dev(vr), dev(cp))
    q = rng.standard_normal((T, H * G, D)).astype(np.float32)
    qp = np.array([0, 7, 1000, n - 1][-T:], np.int32)       # token t sees cells 0..qp[t]
    out = host(api.fa_decode(kvm_state, w, dev(q), dev(qp), H * G, D ** -0.5))
    V = _v_rows(vt, vr, n, H, D)
    for t, p in enumerate(qp):
        want = V[:p + 1].astype(np.float64).mean(0)
        for h in range(H * G):
            np.testing.assert_allclose(out[t, h], want[h // G], rtol=0, atol=1e-5, err_msg=str((t, h)))
    # one visible cell (mid-tile), the rest empty; a token before it sees nothing
    w, kr, vr, cp = _window(kvm_state, rng, n, H, D, kt, vt)
    cp[:] = -1
    cp[777] = 5
    w.import_rows(0, dev(kr), dev(vr), dev(cp))
    qp = np.array([5, 4, 100, 2000][-T:], np.int32)
    out = host(api.fa_decode(kvm_state, w, dev(q), dev(qp), H * G, D ** -0.5))
    V = _v_rows(vt, vr, n, H, D)
    for t, p in enumerate(qp):
        for h in range(H * G):
            want = V[777, h // G] if p >= 5 else np.zeros(D, np.float32)
            np.testing.assert_allclose(out[t, h], want, rtol=0, atol=1e-6, err_msg=str((t, h)))


def test_fa_decode_lanes_match_single_lane(kvm_state):
    rng = np.random.default_rng(8)
    H, G, D = 4, 6, 256
    ws, qs, qps, refs = [], [], [], []
    for i, n in enumerate((1024, 2048, 3072, 4096)):
        w, kr, vr, cp = _window(kvm_state, rng, n, H, D, L.T_Q8_0, L.T_Q4_0)
        q = rng.standard_normal((1, H * G, D)).astype(np.float32)
        qp = np.array([n - 1], np.int32)
        ws.append(w)
        qs.append(dev(q))
        qps.append(dev(qp))
        refs.append(host(api.fa_decode(kvm_state, w, dev(q), dev(qp), H * G, 0.0625)))
    outs = api.fa_decode_lanes(kvm_state, ws, qs, qps, H * G, 0.0625)
    for o, r in zip(outs, refs):
        # the fused launch splits the keys differently, so P is rounded to fp16
        # against different running maxima: equal to well inside the tolerance
        np.testing.assert_allclose(host(o), r, rtol=1e-3, atol=1e-4)


def _f16_rows(ty, rows, n_cells, H, D):
    """Rows dequantised and rounded to fp16: the operands the prefill MFMA kernel
    multiplies (ggml's GPU backends convert a quantised cache to f16 for
    multi-token attention the same way)."""
    x = O.dequant(ty, np.ascontiguousarray(rows).reshape(-1), n_cells * H * D) if ty != L.T_F16 else \
        np.ascontiguousarray(rows).view(np.float16).astype(np.float32).reshape(-1)
    return x.astype(np.float16).view(np.uint8).reshape(n_cells, -1)


def _prefill_check(out, q, kr, vr, cp, pos, H, G, D, kt, vt, scale):
    n = kr.shape[0]
    qh = q.astype(np.float16).astype(np.float32)
    ref16 = O.fa_f64(L.T_F16, L.T_F16, qh, _f16_rows(kt, kr, n, H, D), _f16_rows(vt, vr, n, H, D), cp, pos,
                     H * G, H, D, scale)
    err = check_attention(out, ref16)
    if kt in (L.T_Q8_0, L.T_Q4_0):
        # ggml-CPU rounds Q to q8_0 for a q8_0 or q4_0 K: a coarser computation of the same op
        ref = O.fa_ggml(kt, vt, q, kr, vr, cp, pos, H * G, H, D, scale)
        assert np.abs(out - ref).max() <= 3e-2 * np.abs(ref).max()
    return err


def test_fa_prefill_chunked_causal(kvm_state):
    rng = np.random.default_rng(9)
    H, G, D, n_win, T = 4, 6, 256, 2048, 40
    w, kr, vr, cp = _window(kvm_state, rng, n_win + 128, H, D, L.T_Q8_0, L.T_Q4_0, live=n_win)
    kc, vc = rand_rows(rng, T, H, D, L.T_Q8_0, L.T_Q4_0)
    pos = np.arange(n_win, n_win + T, dtype=np.int32)
    w.import_rows(n_win, dev(kc), dev(vc), dev(pos))           # the chunk's own K/V
    kr[n_win:n_win + T], vr[n_win:n_win + T] = kc, vc
    cp[n_win:n_win + T] = pos
    q = rng.standard_normal((T, H * G, D)).astype(np.float32)
    out = host(api.fa_prefill(kvm_state, w, dev(q), dev(pos), H * G, 0.0625))
    _prefill_check(out, q, kr, vr, cp, pos, H, G, D, L.T_Q8_0, L.T_Q4_0, 0.0625)


PREFILL_CASES = [
    # n_cells, H, G, D, tokens, kt, vt, holes, empty cell range, splits (None = auto), q dtype
    (2048, 4, 6, 256, 48, L.T_Q8_0, L.T_Q4_0, 40, None, None, "bf16"),
    (1024, 2, 4, 128, 64, L.T_F16, L.T_F16, 0, None, 1, "f32"),
    (4096, 4, 6, 256, 30, L.T_Q8_0, L.T_Q4_0, 7, (1024, 2048), 3, "f32"),   # whole empty tiles
    (2048, 1, 8, 256, 20, L.T_Q8_0, L.T_Q4_0, 0, None, 8, "bf16"),
    (2048, 4, 6, 256, 48, L.T_Q4_0, L.T_Q4_0, 40, None, None, "bf16"),
]


@pytest.mark.parametrize("case", range(len(PREFILL_CASES)))
def test_fa_prefill_mfma(kvm_state, case, monkeypatch):
    n_cells, H, G, D, T, kt, vt, holes, empty, splits, qdt = PREFILL_CASES[case]
    if splits is not None:
        monkeypatch.setenv("KVM_PF_SPLITS", str(splits))
    rng = np.random.default_rng(100 + case)
    w, kr, vr, cp = _window(kvm_state, rng, n_cells, H, D, kt, vt, holes=holes)
    if empty is not None:
        cp[empty[0]:empty[1]] = -1
        w.import_rows(0, dev(kr), dev(vr), dev(cp))
    # the chunk occupies the last T cells at positions n_cells - T .. n_cells - 1:
    # causal inside the chunk, the whole earlier window visible
    pos = np.arange(n_cells - T, n_cells, dtype=np.int32)
    cp[n_cells - T:] = pos
    w.import_rows(0, dev(kr), dev(vr), dev(cp))
    q = rng.standard_normal((T, H * G, D)).astype(np.float32)
    if qdt == "bf16":
        qt = torch.from_numpy(q).to(torch.bfloat16)
        q = qt.float().numpy()
        qd = qt.cuda()
    else:
        qd = dev(q)
    scale = 1.0 / np.sqrt(D)
    out = host(api.fa_prefill(kvm_state, w, qd, dev(pos), H * G, scale))
    _prefill_check(out, q, kr, vr, cp, pos, H, G, D, kt, vt, scale)


@pytest.mark.parametrize("kt,vt", [(L.T_Q8_0, L.T_Q4_0), (L.T_F16, L.T_F16)])
def test_fa_prefill_identical_keys(kvm_state, kt, vt):
    """Identical keys on the MFMA prefill path: every visible score equals the
    row maximum, P = 1, so each token's output is the mean of the fp16 V
    operands over the cells it sees (causal by position, holes skipped)."""
    rng = np.random.default_rng(41)
    H, G, D, n, T = 4, 6, 256, 1536, 96
    w, kr, vr, cp = _window(kvm_state, rng, n, H, D, kt, vt, holes=30)
    kr[:] = kr[0]
    pos = np.arange(n - T, n, dtype=np.int32)
    cp[n - T:] = pos
    w.import_rows(0, dev(kr), dev(vr), dev(cp))
    q = rng.standard_normal((T, H * G, D)).astype(np.float32)
    out = host(api.fa_prefill(kvm_state, w, dev(q), dev(pos), H * G, D ** -0.5))
    V = _f16_rows(vt, vr, n, H, D).view(np.float16).astype(np.float64).reshape(n, H, D)
    for t in range(0, T, 7):
        vis = (cp >= 0) & (cp <= pos[t])
        want = V[vis].mean(0)
        for h in range(H * G):
            np.testing.assert_allclose(out[t, h], want[h // G], rtol=0, atol=1e-5, err_msg=str((t, h)))


def test_fa_prefill_blind_rows_and_single_key(kvm_state):
    """A token that sees no cell gets zeros; a token that sees exactly one cell
    gets that cell's V row."""
    rng = np.random.default_rng(11)
    H, G, D, n = 2, 6, 256, 1024
    w, kr, vr, cp = _window(kvm_state, rng, n, H, D, L.T_Q8_0, L.T_Q4_0)
    T = 12
    pos = np.full(T, 700, np.int32)
    pos[0], pos[1] = -1, 0
    q = rng.standard_normal((T, H * G, D)).astype(np.float32)
    out = host(api.fa_prefill(kvm_state, w, dev(q), dev(pos), H * G, 0.0625))
    assert np.all(out[0] == 0)
    V = _f16_rows(L.T_Q4_0, vr[:1], 1, H, D).view(np.float16).astype(np.float32).reshape(H, D)
    for h in range(H * G):
        np.testing.assert_allclose(out[1, h], V[h // G], rtol=1e-3, atol=1e-3)
    _prefill_check(out, q, kr, vr, cp, pos, H, G, D, L.T_Q8_0, L.T_Q4_0, 0.0625)


def test_fa_prefill_splits_agree(kvm_state, monkeypatch):
    rng = np.random.default_rng(12)
    H, G, D, n, T = 4, 6, 256, 4096, 64
    w, kr, vr, cp = _window(kvm_state, rng, n, H, D, L.T_Q8_0, L.T_Q4_0)
    pos = np.arange(n - T, n, dtype=np.int32)
    q = dev(rng.standard_normal((T, H * G, D)).astype(np.float32))
    outs = []
    for s in (1, 2, 5):
        monkeypatch.setenv("KVM_PF_SPLITS", str(s))
        outs.append(host(api.fa_prefill(kvm_state, w, q, dev(pos), H * G, 0.0625)))
    for o in outs[1:]:
        # P is rounded to fp16 against each split's own running maxima
        np.testing.assert_allclose(o, outs[0], rtol=1e-3, atol=1e-4)


def test_fa_decode_rejects_wide_batches(kvm_state):
    rng = np.random.default_rng(10)
    w, *_ = _window(kvm_state, rng, 256, 4, 256, L.T_Q8_0, L.T_Q4_0)
    q = dev(np.zeros((6, 24, 256), np.float32))
    with pytest.raises(L.KvmError):
        api.fa_decode(kvm_state, w, q, dev(np.zeros(6, np.int32)), 24, 0.0625)
