"""Flash-attention oracles: ggml-CPU semantics (oracle_fa_ggml) and the float64
textbook softmax (oracle_fa_f64).  ggml itself is not in the reference tree, so
ggml-level parity is pinned only through these special cases and the f64 anchor."""
import numpy as np
import pytest

import oracle as O


def _case(seed, n_cells, n_tokens, n_head, n_head_kv, d, kt=O.T_Q8_0, vt=O.T_Q4_0):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((n_cells, n_head_kv * d)).astype(np.float32)
    v = rng.standard_normal((n_cells, n_head_kv * d)).astype(np.float32)
    q = rng.standard_normal((n_tokens, n_head, d)).astype(np.float32)

    def enc(ty, x):
        if ty == O.T_F16:
            return x.astype(np.float16).view(np.uint8).reshape(n_cells, -1)
        return O.quant(ty, x.reshape(-1)).reshape(n_cells, -1)
    return q, enc(kt, k), enc(vt, v)


def _deq(ty, rows, n):
    if ty == O.T_F16:
        return rows.view(np.float16).astype(np.float32).reshape(rows.shape[0], -1)
    return O.dequant(ty, rows.reshape(-1), rows.shape[0] * n).reshape(rows.shape[0], n)


def test_textbook_brute_force():
    q, kr, vr = _case(1, 37, 2, 4, 2, 128)
    cp = np.arange(37, dtype=np.int32)
    cp[5] = -1
    qp = np.array([30, 36], np.int32)
    got = O.fa_f64(O.T_Q8_0, O.T_Q4_0, q, kr, vr, cp, qp, 4, 2, 128, 0.0884)
    K, V = _deq(O.T_Q8_0, kr, 256).reshape(37, 2, 128), _deq(O.T_Q4_0, vr, 256).reshape(37, 2, 128)
    for t in range(2):
        for h in range(4):
            vis = (cp >= 0) & (cp <= qp[t])
            s = K[vis, h // 2].astype(np.float64) @ q[t, h].astype(np.float64) * 0.0884
            p = np.exp(s - s.max())
            np.testing.assert_allclose(got[t, h], p @ V[vis, h // 2] / p.sum(), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("kt,vt", [(O.T_Q8_0, O.T_Q4_0), (O.T_F16, O.T_F16)])
def test_special_cases(kt, vt):
    n_cells, d = 64, 128
    q, kr, vr = _case(2, n_cells, 1, 2, 1, d, kt, vt)
    V = _deq(vt, vr, d)
    # a single visible key returns its V row
    cp = np.full(n_cells, -1, np.int32)
    cp[17] = 3
    for fn in (O.fa_ggml, O.fa_f64):
        out = fn(kt, vt, q, kr, vr, cp, np.array([10], np.int32), 2, 1, d, 0.1)
        np.testing.assert_allclose(out[0, 0], V[17], rtol=1e-6, atol=1e-6)
    # no visible key gives zeros
    out = O.fa_ggml(kt, vt, q, kr, vr, cp, np.array([2], np.int32), 2, 1, d, 0.1)
    assert np.all(out == 0)
    # identical keys give the mean of V
    kr2 = np.repeat(kr[:1], n_cells, axis=0)
    out = O.fa_ggml(kt, vt, q, kr2, vr, None, np.array([n_cells], np.int32), 2, 1, d, 0.1)
    np.testing.assert_allclose(out[0, 0], V.mean(0), atol=2e-3 if vt == O.T_F16 else 1e-5)


def test_ggml_semantics_vs_textbook_q8_q4():
    """ggml quantises Q to q8_0 for a q8_0 K: its output departs from the f64 anchor
    by the Q quantisation error only (well under 1 % relative here), while rounding
    Q to q8_0 before the f64 oracle closes the gap to fp32 rounding."""
    q, kr, vr = _case(3, 2048, 4, 24, 4, 256)
    cp = np.arange(2048, dtype=np.int32)
    qp = np.array([2044, 2045, 2046, 2047], np.int32)
    g = O.fa_ggml(O.T_Q8_0, O.T_Q4_0, q, kr, vr, cp, qp, 24, 4, 256, 1 / 16)
    f = O.fa_f64(O.T_Q8_0, O.T_Q4_0, q, kr, vr, cp, qp, 24, 4, 256, 1 / 16)
    rel = np.abs(g - f).max() / np.abs(f).max()
    assert rel < 2e-2
    qq = O.dequant(O.T_Q8_0, O.quant(O.T_Q8_0, q.reshape(-1)), q.size).reshape(q.shape)
    f2 = O.fa_f64(O.T_Q8_0, O.T_Q4_0, qq, kr, vr, cp, qp, 24, 4, 256, 1 / 16)
    assert np.abs(g - f2).max() / np.abs(f2).max() < 1e-5


def test_ggml_semantics_vs_textbook_f16():
    q, kr, vr = _case(4, 4608, 1, 8, 2, 128, O.T_F16, O.T_F16)
    qp = np.array([4607], np.int32)
    g = O.fa_ggml(O.T_F16, O.T_F16, q, kr, vr, None, qp, 8, 2, 128, 128 ** -0.5)
    qh = q.astype(np.float16).astype(np.float32)
    f = O.fa_f64(O.T_F16, O.T_F16, qh, kr, vr, None, qp, 8, 2, 128, 128 ** -0.5)
    # ggml accumulates V*p in an fp16 vector: error at the fp16 level of the accumulator
    assert np.abs(g - f).max() < 2e-3


def _q4_as_q8(rows4, n_per_row):
    """q4_0 rows -> the q8_0 rows of the same values (quant = nibble - 8, same scale)."""
    nb = n_per_row // 32
    r4 = rows4.reshape(rows4.shape[0], nb, 18)
    out = np.zeros((rows4.shape[0], nb, 34), np.uint8)
    out[:, :, :2] = r4[:, :, :2]
    lo = (r4[:, :, 2:] & 15).astype(np.int16) - 8
    hi = (r4[:, :, 2:] >> 4).astype(np.int16) - 8
    out[:, :, 2:18] = lo.astype(np.int8).view(np.uint8)
    out[:, :, 18:34] = hi.astype(np.int8).view(np.uint8)
    return out.reshape(rows4.shape[0], -1)


def test_q4_0_keys_are_q8_0_keys_of_the_same_values():
    """A q4_0 K cache (ggml's vec_dot_q4_0_q8_0: low nibbles against query quants
    0-15, high nibbles against 16-31, minus 8) attends exactly as the q8_0 cache
    holding the same values, up to the order of the two scale products
    (sumi * d_k * d_q against sumi * (d_k * d_q)); a swapped nibble half or a
    missing -8 would move every score.  Against the float64 anchor (unquantised
    Q) the gap is the query's q8_0 rounding, as for a q8_0 cache."""
    n_cells, d, H, n_head = 200, 128, 2, 6
    q, k4, vr = _case(9, n_cells, 3, n_head, H, d, O.T_Q4_0, O.T_Q4_0)
    k8 = _q4_as_q8(k4, H * d)
    assert np.array_equal(_deq(O.T_Q4_0, k4, H * d), _deq(O.T_Q8_0, k8, H * d))
    cp = np.arange(n_cells, dtype=np.int32)
    qp = np.array([60, 150, 199], np.int32)
    a = O.fa_ggml(O.T_Q4_0, O.T_Q4_0, q, k4, vr, cp, qp, n_head, H, d, d ** -0.5)
    b = O.fa_ggml(O.T_Q8_0, O.T_Q4_0, q, k8, vr, cp, qp, n_head, H, d, d ** -0.5)
    np.testing.assert_allclose(a, b, rtol=0, atol=2e-6)
    ref = O.fa_f64(O.T_Q4_0, O.T_Q4_0, q, k4, vr, cp, qp, n_head, H, d, d ** -0.5)
    ref8 = O.fa_f64(O.T_Q8_0, O.T_Q4_0, q, k8, vr, cp, qp, n_head, H, d, d ** -0.5)
    assert np.max(np.abs(ref - ref8)) < 1e-12
    assert np.max(np.abs(a - ref)) / np.max(np.abs(ref)) < 2e-2
    # the wrong nibble order is far outside that
    k4s = k4.reshape(n_cells, -1, 18).copy()
    k4s[:, :, 2:] = ((k4s[:, :, 2:] & 15) << 4) | (k4s[:, :, 2:] >> 4)
    c = O.fa_ggml(O.T_Q4_0, O.T_Q4_0, q, k4s.reshape(n_cells, -1), vr, cp, qp, n_head, H, d, d ** -0.5)
    assert np.max(np.abs(c - a)) > 1e-2
