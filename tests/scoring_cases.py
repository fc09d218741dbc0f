"""Scoring inputs where the cosine's epsilon, the query scale invq =
1 / (q_count * g), the query-head grouping and the layer average all change
the answer, and a float64 evaluation of score_retrieval's closed form
(llama-memory-kvmem.cpp:4149-4196) with deliberate variants of each term.

The norms are chosen so that sqrt(nq) * sqrt(nk) is about 1e-6: the 1e-6 in
the denominator then weighs as much as the norms, so scaling q (a wrong invq)
or moving the epsilon changes every cosine by a large fraction, although a
cosine without the epsilon would not see a scale at all."""
import numpy as np


def tiny_norm_case(seed, n_blocks=12, n_layer=3, n_head=6, H=2, d=128, q_count=(5, 0, 2)):
    rng = np.random.default_rng(seed)
    g = n_head // H
    mt = rng.choice([1, 7, 33, 128], (n_layer, n_blocks)).astype(np.uint32)
    mt[-1, 3] = 0                                   # no K for block 3 in the last layer
    # kh = k_sum / mt with |kh| per (block, head) between 2e-4 and 4e-3
    kdir = rng.standard_normal((n_layer, n_blocks, H, d))
    kdir /= np.linalg.norm(kdir, axis=-1, keepdims=True)
    knorm = np.exp(rng.uniform(np.log(2e-4), np.log(4e-3), (n_layer, n_blocks, H, 1)))
    k_sum = (kdir * knorm * np.maximum(mt, 1)[:, :, None, None]).reshape(n_layer, n_blocks, H * d)
    # query rows: a planted block's direction plus noise; the group's mean has
    # |qv| near 5e-4
    q = rng.standard_normal((n_layer, n_head, d)) * 0.4
    for il in range(n_layer):
        for h in range(n_head):
            q[il, h] += kdir[il, 5, h // g] * 1.0
    qc = np.asarray(q_count, np.uint32)
    for il in range(n_layer):
        scale = 5e-4 * max(int(qc[il]), 1) * g / np.sqrt(g * d * 0.16 + g * g)
        q[il] *= scale
    return (q.reshape(n_layer, n_head * d).astype(np.float32), qc, k_sum.astype(np.float32), mt)


def score_f64(q_sum, q_count, k_sum, mt, n_head, H, d, variant=None):
    """score_retrieval in float64; variant names one plausible mistake:
    'invq_no_g' (1/q_count), 'eps_in_sqrt' (sqrt(nq nk + eps)), 'no_eps',
    'eps_in_num' ((dot + eps) / (|q||k| + eps)), 'interleaved_heads' (query
    head h + H*i in kv group h), 'layers_weighted' (layers weighted by
    q_count), 'all_layers' (layers without a query count in the average)."""
    q_sum = np.asarray(q_sum, np.float64)
    k_sum = np.asarray(k_sum, np.float64)
    n_layer, n_blocks = mt.shape
    g = n_head // H
    out = np.zeros(n_blocks)
    for b in range(n_blocks):
        layers, weights = [], []
        for il in range(n_layer):
            if q_count[il] == 0:
                if variant == "all_layers":
                    layers.append(0.0)
                    weights.append(1.0)
                continue
            kh_all = k_sum[il, b] / mt[il, b] if mt[il, b] else np.zeros(H * d)
            rows = q_sum[il].reshape(n_head, d)
            cs = []
            for h in range(H):
                grp = rows[h::H] if variant == "interleaved_heads" else rows[h * g:(h + 1) * g]
                qv = grp.sum(0) / (q_count[il] * (1 if variant == "invq_no_g" else g))
                kh = kh_all[h * d:(h + 1) * d]
                dot, nq, nk = qv @ kh, qv @ qv, kh @ kh
                if variant == "eps_in_sqrt":
                    cs.append(dot / np.sqrt(nq * nk + 1e-6))
                elif variant == "no_eps":
                    cs.append(dot / (np.sqrt(nq) * np.sqrt(nk)) if nk > 0 else 0.0)
                elif variant == "eps_in_num":
                    cs.append((dot + 1e-6) / (np.sqrt(nq) * np.sqrt(nk) + 1e-6))
                else:
                    cs.append(dot / (np.sqrt(nq) * np.sqrt(nk) + 1e-6))
            layers.append(np.mean(cs))
            weights.append(float(q_count[il]) if variant == "layers_weighted" else 1.0)
        out[b] = np.average(layers, weights=weights) if layers else 0.0
    return out


VARIANTS = ("invq_no_g", "eps_in_sqrt", "no_eps", "eps_in_num", "interleaved_heads", "layers_weighted",
            "all_layers")
