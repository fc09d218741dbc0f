/*
 * kvm_oracle.c -- CPU restatement of the KVMem retrieval + attention hot path.
 * TEST INFRASTRUCTURE ONLY (see kvm_oracle.h).  Built with -ffp-contract=off so
 * that every a*b+c is two IEEE roundings, as in the reference's host C++.
 */
#include "kvm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------- */
/* half precision (raw_kv_store.cpp:33-95): IEEE binary16, round to nearest   */
/* even, gradual underflow, NaN kept quiet.                                   */
/* ------------------------------------------------------------------------- */
uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t aexp = (x >> 23) & 0xffu;
    uint32_t mant = x & 0x7fffffu;
    if (aexp == 0xffu) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
    if ((x & 0x7fffffffu) == 0) return (uint16_t)sign;
    int e = (int)aexp - 127 + 15;               /* biased half exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {                                /* half subnormal or zero */
        if (e < -10) return (uint16_t)sign;
        mant |= 0x800000u;
        const uint32_t shift = (uint32_t)(14 - e);
        uint32_t h = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* may carry into inf */
    return (uint16_t)(sign | h);
}

float oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t out;
    if (e == 0) {
        if (m == 0) {
            out = sign;
        } else {                                  /* normalise the subnormal */
            int ee = 1;
            while (!(m & 0x400u)) { m <<= 1; ee--; }
            m &= 0x3ffu;
            out = sign | ((uint32_t)(ee + 127 - 15) << 23) | (m << 13);
        }
    } else if (e == 31) {
        out = sign | 0x7f800000u | (m << 13);
    } else {
        out = sign | ((e + 127 - 15) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &out, 4);
    return f;
}

/* ------------------------------------------------------------------------- */
/* ggml block codecs (llama-kvmem-stagein.cu:133-234; same formulas as ggml's */
/* quantize_row_q8_0_ref / quantize_row_q4_0_ref).                            */
/* ------------------------------------------------------------------------- */
static inline void put_f16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
static inline uint16_t get_f16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

void oracle_quant_q8_0(const float *x, uint8_t *y, int64_t n) {
    for (int64_t b = 0; b < n / 32; ++b) {
        const float *src = x + b * 32;
        uint8_t *blk = y + b * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(src[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        put_f16(blk, oracle_f32_to_f16(d));
        for (int j = 0; j < 32; ++j) blk[2 + j] = (uint8_t)(int8_t)roundf(src[j] * id);
    }
}

void oracle_dequant_q8_0(const uint8_t *x, float *y, int64_t n) {
    for (int64_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = x + b * 34;
        const float d = oracle_f16_to_f32(get_f16(blk));
        for (int j = 0; j < 32; ++j) y[b * 32 + j] = (float)(int8_t)blk[2 + j] * d;
    }
}

void oracle_quant_q4_0(const float *x, uint8_t *y, int64_t n) {
    for (int64_t b = 0; b < n / 32; ++b) {
        const float *src = x + b * 32;
        uint8_t *blk = y + b * 18;
        float amax = 0.0f, vmax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            if (amax < fabsf(src[j])) { amax = fabsf(src[j]); vmax = src[j]; }
        }
        const float d = vmax / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        put_f16(blk, oracle_f32_to_f16(d));
        for (int j = 0; j < 16; ++j) {
            int x0 = (int)(src[j] * id + 8.5f);
            int x1 = (int)(src[j + 16] * id + 8.5f);
            if (x0 > 15) x0 = 15;
            if (x1 > 15) x1 = 15;
            blk[2 + j] = (uint8_t)((x0 & 15) | ((x1 & 15) << 4));
        }
    }
}

void oracle_dequant_q4_0(const uint8_t *x, float *y, int64_t n) {
    for (int64_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = x + b * 18;
        const float d = oracle_f16_to_f32(get_f16(blk));
        for (int j = 0; j < 16; ++j) {
            y[b * 32 + j] = (float)((blk[2 + j] & 0x0f) - 8) * d;
            y[b * 32 + j + 16] = (float)((blk[2 + j] >> 4) - 8) * d;
        }
    }
}

int64_t oracle_row_bytes(int type, int64_t n) {
    switch (type) {
        case ORACLE_T_F32: return n * 4;
        case ORACLE_T_F16: return n * 2;
        case ORACLE_T_Q8_0: return n / 32 * 34;
        case ORACLE_T_Q4_0: return n / 32 * 18;
        default: return -1;
    }
}

static void to_float_row(int type, const uint8_t *src, float *dst, int64_t n) {
    switch (type) {
        case ORACLE_T_F32: memcpy(dst, src, (size_t)n * 4); break;
        case ORACLE_T_F16:
            for (int64_t i = 0; i < n; ++i) dst[i] = oracle_f16_to_f32(get_f16(src + 2 * i));
            break;
        case ORACLE_T_Q8_0: oracle_dequant_q8_0(src, dst, n); break;
        case ORACLE_T_Q4_0: oracle_dequant_q4_0(src, dst, n); break;
        default: memset(dst, 0, (size_t)n * 4); break;
    }
}

void oracle_quant_q8_0_rows(const float *x, uint8_t *y, int64_t n_rows, int64_t n_per_row) {
    for (int64_t r = 0; r < n_rows; ++r)
        oracle_quant_q8_0(x + r * n_per_row, y + r * (n_per_row / 32 * 34), n_per_row);
}

/* ------------------------------------------------------------------------- */
/* NeoX RoPE.  theta_i = powf(base, -2i/n_rot) * scale (rope.cpp:19-22).      */
/* The reference computes sin/cos with libm (host) or the device sincosf      */
/* (stagein.cu:171); neither is reproducible bit-for-bit on another device,   */
/* so both sides use cos/sin of the fp32 angle evaluated in double and        */
/* rounded once to fp32.  Rotation order stagein.cu:172-175 / rope.cpp:34-37. */
/* ------------------------------------------------------------------------- */
void oracle_rope_theta(float freq_base, float freq_scale, int n_rot, float *theta) {
    for (int i = 0; i < n_rot / 2; ++i) {
        float t = powf(freq_base, -2.0f * (float)i / (float)n_rot);
        theta[i] = t * freq_scale;
    }
}

void oracle_rope_cs(const float *theta, int n_half, int32_t pos, float *c, float *s) {
    const float p = (float)pos;
    for (int i = 0; i < n_half; ++i) {
        const float ang = p * theta[i];
        c[i] = (float)cos((double)ang);
        s[i] = (float)sin((double)ang);
    }
}

void oracle_rope_neox(float *x, int64_t n_tokens, int n_head, int head_dim, int n_rot,
                      int32_t pos0, const float *theta) {
    const int half = n_rot / 2;
    float *c = (float *)malloc(sizeof(float) * (size_t)half);
    float *s = (float *)malloc(sizeof(float) * (size_t)half);
    for (int64_t t = 0; t < n_tokens; ++t) {
        oracle_rope_cs(theta, half, pos0 + (int32_t)t, c, s);
        for (int h = 0; h < n_head; ++h) {
            float *row = x + (t * n_head + h) * head_dim;
            for (int i = 0; i < half; ++i) {
                const float x0 = row[i], x1 = row[i + half];
                row[i] = x0 * c[i] - x1 * s[i];
                row[i + half] = x0 * s[i] + x1 * c[i];
            }
        }
    }
    free(c);
    free(s);
}

/* ------------------------------------------------------------------------- */
/* Normalised Walsh-Hadamard transform of each n-wide row: pre-scale by       */
/* 1/sqrt(n), then radix-2 butterflies with h = 1, 2, ..., n/2               */
/* (stagein.cu:105-131 with scale from :594).                                 */
/* ------------------------------------------------------------------------- */
void oracle_fwht(float *x, int64_t n_rows, int n) {
    const float scale = 1.0f / sqrtf((float)n);
    for (int64_t r = 0; r < n_rows; ++r) {
        float *row = x + r * n;
        for (int i = 0; i < n; ++i) row[i] = row[i] * scale;
        for (int h = 1; h < n; h *= 2) {
            for (int i = 0; i < n; i += 2 * h) {
                for (int j = 0; j < h; ++j) {
                    const float a = row[i + j], b = row[i + j + h];
                    row[i + j] = a + b;
                    row[i + j + h] = a - b;
                }
            }
        }
    }
}

int oracle_hadamard_nrot_k(int head_dim) {
    int nrot = 64;
    do { nrot *= 2; } while (head_dim % nrot == 0);
    return nrot / 2;
}

int oracle_attn_rot_on(int type, int head_dim) {
    const int quantized = type == ORACLE_T_Q8_0 || type == ORACLE_T_Q4_0;
    return quantized && head_dim >= 64 && head_dim % 64 == 0;
}

void oracle_stagein_k_type(int k_type, const uint8_t *packed, uint8_t *out, int64_t nt, int n_head,
                           int head_dim, int n_rot, int nrot, int32_t pos0, const float *theta) {
    const int64_t n_embd = (int64_t)n_head * head_dim;
    float *f = (float *)malloc(sizeof(float) * (size_t)(nt * n_embd));
    if (k_type == ORACLE_T_Q4_0) oracle_dequant_q4_0(packed, f, nt * n_embd);
    else oracle_dequant_q8_0(packed, f, nt * n_embd);
    oracle_rope_neox(f, nt, n_head, head_dim, n_rot, pos0, theta);
    if (nrot > 0) oracle_fwht(f, nt * (n_embd / nrot), nrot);
    if (k_type == ORACLE_T_Q4_0) oracle_quant_q4_0(f, out, nt * n_embd);
    else oracle_quant_q8_0(f, out, nt * n_embd);
    free(f);
}

void oracle_stagein_k(const uint8_t *packed, uint8_t *out, int64_t nt, int n_head,
                      int head_dim, int n_rot, int nrot, int32_t pos0, const float *theta) {
    oracle_stagein_k_type(ORACLE_T_Q8_0, packed, out, nt, n_head, head_dim, n_rot, nrot, pos0, theta);
}

/* ------------------------------------------------------------------------- */
/* Mean-K authority: ordered fp32 sum (raw_kv_store.cpp:215-234), then one    */
/* reciprocal and a multiply (raw_kv_store.cpp:996-1006).                     */
/* ------------------------------------------------------------------------- */
void oracle_meank_add(float *k_sum, uint32_t *mean_tokens, const float *k, uint32_t off,
                      uint32_t take, int n_embd) {
    if (!k || take == 0 || n_embd == 0) return;
    if (off == 0) memset(k_sum, 0, sizeof(float) * (size_t)n_embd);
    for (uint32_t t = 0; t < take; ++t) {
        const float *row = k + (size_t)t * (size_t)n_embd;
        for (int d = 0; d < n_embd; ++d) k_sum[d] += row[d];
    }
    const uint32_t end = off + take;
    *mean_tokens = off == 0 ? take : (*mean_tokens > end ? *mean_tokens : end);
}

void oracle_meank_normalize(const float *k_sum, uint32_t mean_tokens, float *out, int n_embd) {
    if (mean_tokens == 0) {
        memset(out, 0, sizeof(float) * (size_t)n_embd);
        return;
    }
    const float inv = 1.0f / (float)mean_tokens;
    for (int d = 0; d < n_embd; ++d) out[d] = k_sum[d] * inv;
}

/* ------------------------------------------------------------------------- */
/* score_retrieval (llama-memory-kvmem.cpp:4149-4196).  Per block, per layer   */
/* with queries, per kv head: the grouped query sum qh, scaled by            */
/* invq = 1/(q_count*g), and the block's mean K give a cosine computed with   */
/* three sequential fp32 sums; the cosines are averaged in double.            */
/* ------------------------------------------------------------------------- */
static double score_block(int b, int n_blocks, int n_layer, int n_head, int n_head_kv,
                          int head_dim, const float *q_sum, const uint32_t *q_count,
                          const float *k_sum, const uint32_t *mean_tokens, float *mk,
                          float *qh) {
    const int n_embd_k = n_head_kv * head_dim;
    const uint32_t g = n_head_kv == 0 ? 1u : (uint32_t)(n_head / n_head_kv);
    const uint32_t g1 = g > 1u ? g : 1u;
    double acc = 0.0;
    uint32_t nlay = 0;
    for (int il = 0; il < n_layer; ++il) {
        if (q_count[il] == 0) continue;
        oracle_meank_normalize(k_sum + ((size_t)il * n_blocks + b) * n_embd_k,
                               mean_tokens[(size_t)il * n_blocks + b], mk, n_embd_k);
        double layer = 0.0;
        const float invq = 1.0f / (float)(q_count[il] * g1);
        for (int h = 0; h < n_head_kv; ++h) {
            for (int d = 0; d < head_dim; ++d) qh[d] = 0.0f;
            for (uint32_t gi = 0; gi < g; ++gi) {
                const uint32_t qi = (uint32_t)h * g + gi;
                if (qi >= (uint32_t)n_head) break;
                const float *q = q_sum + (size_t)il * n_head * head_dim + (size_t)qi * head_dim;
                for (int d = 0; d < head_dim; ++d) qh[d] += q[d];
            }
            const float *kh = mk + (size_t)h * head_dim;
            float dot = 0.0f, nq = 0.0f, nk = 0.0f;
            for (int d = 0; d < head_dim; ++d) {
                const float qv = qh[d] * invq;
                dot += qv * kh[d];
                nq += qv * qv;
                nk += kh[d] * kh[d];
            }
            const float cosv = dot / (sqrtf(nq) * sqrtf(nk) + 1e-6f);
            layer += (double)cosv;
        }
        acc += layer / (double)(n_head_kv > 1 ? n_head_kv : 1);
        nlay++;
    }
    return nlay ? acc / (double)nlay : 0.0;
}

void oracle_score_retrieval(int n_blocks, int n_layer, int n_head, int n_head_kv, int head_dim,
                            const float *q_sum, const uint32_t *q_count, const float *k_sum,
                            const uint32_t *mean_tokens, const uint8_t *present,
                            double *scores, int n_threads) {
    (void)n_threads;
#ifdef _OPENMP
#pragma omp parallel num_threads(n_threads > 0 ? n_threads : 1)
#endif
    {
        float *mk = (float *)malloc(sizeof(float) * (size_t)n_head_kv * head_dim);
        float *qh = (float *)malloc(sizeof(float) * (size_t)head_dim);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int b = 0; b < n_blocks; ++b) {
            scores[b] = (present && !present[b]) ? 0.0
                : score_block(b, n_blocks, n_layer, n_head, n_head_kv, head_dim, q_sum,
                              q_count, k_sum, mean_tokens, mk, qh);
        }
        free(mk);
        free(qh);
    }
}

/* ------------------------------------------------------------------------- */
/* pick_topk_ungrouped, TopK policy (kvmem_store.cpp:482-623): sink prefix,   */
/* mandatory ids newest-first (from the end of the list), recent tail, then   */
/* the best remaining blocks under the strict order (score desc, id desc).    */
/* nth_element selects the same set as a full sort under a strict total      */
/* order, which is what this restatement uses.                               */
/* ------------------------------------------------------------------------- */
static const double *g_cmp_scores;
static int cmp_better(const void *pa, const void *pb) {
    const uint32_t a = *(const uint32_t *)pa, b = *(const uint32_t *)pb;
    const double sa = g_cmp_scores[a], sb = g_cmp_scores[b];
    if (sa != sb) return sa > sb ? -1 : 1;
    return a > b ? -1 : (a < b ? 1 : 0);
}

uint32_t oracle_pick_topk(uint32_t n, const double *scores, uint32_t budget_blocks,
                          uint32_t sink_blocks, uint32_t recent_blocks,
                          const uint32_t *mandatory, uint32_t n_mandatory, uint32_t *out) {
    if (n == 0) return 0;
    if (budget_blocks == 0 || n <= budget_blocks) {
        for (uint32_t i = 0; i < n; ++i) out[i] = i;
        return n;
    }
    const uint32_t budget = budget_blocks;
    const uint32_t sink = sink_blocks < n ? sink_blocks : n;
    const uint32_t recent = recent_blocks < n ? recent_blocks : n;
    uint8_t *kept = (uint8_t *)calloc(n, 1);
    uint32_t count = 0;
#define KEEP(id_) do { uint32_t id__ = (id_); if (id__ < n && !kept[id__]) { kept[id__] = 1; ++count; } } while (0)
    for (uint32_t i = 0; i < sink && count < budget; ++i) KEEP(i);
    for (uint32_t i = n_mandatory; i > 0 && count < budget; --i) KEEP(mandatory[i - 1]);
    for (uint32_t i = 0; i < recent && count < budget; ++i) KEEP(n - 1 - i);
    if (count < budget) {
        uint32_t *cand = (uint32_t *)malloc(sizeof(uint32_t) * n);
        uint32_t nc = 0;
        for (uint32_t i = 0; i < n; ++i) if (!kept[i]) cand[nc++] = i;
        const uint32_t need = budget - count < nc ? budget - count : nc;
        g_cmp_scores = scores;
        qsort(cand, nc, sizeof(uint32_t), cmp_better);
        for (uint32_t i = 0; i < need; ++i) KEEP(cand[i]);
        free(cand);
    }
#undef KEEP
    uint32_t m = 0;
    for (uint32_t i = 0; i < n; ++i) if (kept[i]) out[m++] = i;
    free(kept);
    return m;
}

/* ------------------------------------------------------------------------- */
/* Window layout: set_selection packs the selected blocks in ascending id     */
/* order, to_base = sum of n_tokens of the blocks before it                   */
/* (kvmem_store.cpp:797-880); layout_gpu_slots_by_orig_pos gives slot k to    */
/* the k-th block in original-position order after reset_slots' LIFO list     */
/* (llama-memory-kvmem.cpp:1958-1993, 1018-1024).  Cell c of slot k holds     */
/* window position to_base_k + (c - k*bt) for c - k*bt < n_tokens_k.          */
/* ------------------------------------------------------------------------- */
uint32_t oracle_window_layout(const uint32_t *sel, uint32_t n_sel, const uint32_t *n_tokens,
                              uint32_t block_tokens, uint32_t n_slots, int32_t *to_base,
                              int32_t *cell_pos) {
    for (uint64_t c = 0; c < (uint64_t)n_slots * block_tokens; ++c) cell_pos[c] = -1;
    uint32_t pos = 0;
    for (uint32_t k = 0; k < n_sel; ++k) {
        to_base[k] = (int32_t)pos;
        const uint32_t nt = n_tokens[sel[k]];
        if (k < n_slots)
            for (uint32_t t = 0; t < nt; ++t)
                cell_pos[(uint64_t)k * block_tokens + t] = (int32_t)(pos + t);
        pos += nt;
    }
    return pos;
}

/* ------------------------------------------------------------------------- */
/* Mandatory blocks of a retrieval (llama-memory-kvmem.cpp:4306-4325): the     */
/* ranges are the explicit mandatory spans when explicit_spans (even none),    */
/* else the query span                                                          */
/* [query_begin, query_end > 0 ? query_end : total) when query_begin >= 0;     */
/* every block overlapping a range, once, in block order; then the block       */
/* containing force_pos (KvMemStore::block_id_containing, kvmem_store.cpp:     */
/* 158-177) when force_pos >= 0 and inside the store, appended even if listed. */
/* Block b covers [sum_{i<b} n_tokens_i, + n_tokens_b).  Returns the count.    */
/* ------------------------------------------------------------------------- */
uint32_t oracle_retrieval_mandatory(const uint32_t *n_tokens, uint32_t n_blocks, const int32_t *ranges,
                                    uint32_t n_ranges, int explicit_spans, int32_t query_begin,
                                    int32_t query_end, int32_t force_pos, uint32_t *out) {
    int64_t total = 0;
    for (uint32_t b = 0; b < n_blocks; ++b) total += n_tokens[b];
    int32_t qr[2];
    const int32_t *rg = ranges;
    uint32_t nr = explicit_spans ? n_ranges : 0u;
    if (!explicit_spans && query_begin >= 0) {
        qr[0] = query_begin;
        qr[1] = query_end > 0 ? query_end : (int32_t)total;
        rg = qr;
        nr = 1;
    }
    uint32_t n = 0;
    int64_t start = 0;
    for (uint32_t b = 0; b < n_blocks; ++b) {
        const int64_t end = start + n_tokens[b];
        for (uint32_t r = 0; r < nr; ++r) {
            if (end > rg[2 * r] && start < rg[2 * r + 1]) {
                out[n++] = b;
                break;
            }
        }
        start = end;
    }
    if (force_pos >= 0 && force_pos < total) {
        start = 0;
        for (uint32_t b = 0; b < n_blocks; ++b) {
            if (force_pos >= start && force_pos < start + n_tokens[b]) {
                out[n++] = b;
                break;
            }
            start += n_tokens[b];
        }
    }
    return n;
}

/* ------------------------------------------------------------------------- */
/* Flash attention, ggml-CPU semantics (ggml-cpu/ops.cpp,                      */
/* ggml_compute_forward_flash_attn_ext_f16_one_chunk, called from build_attn,  */
/* patches/0002-attn-qk-capture-hook.patch:225 with kq_scale 1/sqrt(d) :256):  */
/*  - Q is converted to K's vec_dot type: fp16 for f16 K (RNE), q8_0 for q8_0  */
/*    K (quantize_row_q8_0);                                                  */
/*  - s = vec_dot(K row, Q) * scale; f16 dot sums fp32 products in double,     */
/*    q8_0 dot sums (float)sumi * (dk*dq) over 32-blocks in fp32;              */
/*  - masked cells are skipped; online softmax with M, S and expf;            */
/*  - f16 V accumulates in an fp16 vector (ggml_vec_mad_f16 / scale_f16),      */
/*    other V types are dequantised to fp32 and accumulated in fp32;           */
/*  - out = VKQ * (1/S); S == 0 (no visible key) gives zeros.                 */
/* ------------------------------------------------------------------------- */
static inline int visible(const int32_t *cell_pos, const int32_t *q_pos, int t, int c) {
    const int32_t p = cell_pos ? cell_pos[c] : c;
    return p >= 0 && p <= q_pos[t];
}

int oracle_fa_ggml(int k_type, int v_type, const float *q, const void *k, const void *v,
                   const int32_t *cell_pos, const int32_t *q_pos, int n_tokens, int n_head,
                   int n_head_kv, int head_dim, int n_cells, float scale, float *out,
                   int n_threads) {
    if (k_type != ORACLE_T_F16 && k_type != ORACLE_T_Q8_0 && k_type != ORACLE_T_Q4_0) return -1;
    if (v_type != ORACLE_T_F16 && v_type != ORACLE_T_Q4_0 && v_type != ORACLE_T_Q8_0) return -1;
    if (n_head_kv <= 0 || n_head % n_head_kv) return -1;
    const int g = n_head / n_head_kv;
    const int64_t krow = oracle_row_bytes(k_type, head_dim);
    const int64_t vrow = oracle_row_bytes(v_type, head_dim);
    const uint8_t *K = (const uint8_t *)k, *V = (const uint8_t *)v;
    const int n_rows = n_tokens * n_head;
    (void)n_threads;
#ifdef _OPENMP
#pragma omp parallel num_threads(n_threads > 0 ? n_threads : 1)
#endif
    {
        float *vkq = (float *)malloc(sizeof(float) * (size_t)head_dim);
        float *v32 = (float *)malloc(sizeof(float) * (size_t)head_dim);
        uint16_t *vkq16 = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)head_dim);
        uint8_t *qq = (uint8_t *)malloc((size_t)head_dim * 2 + 64);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int r = 0; r < n_rows; ++r) {
            const int t = r / n_head, h = r % n_head, hk = h / g;
            const float *pq = q + (size_t)r * head_dim;
            if (k_type != ORACLE_T_F16) oracle_quant_q8_0(pq, qq, head_dim);   /* the vec_dot type of q8_0 and q4_0 */
            else for (int d = 0; d < head_dim; ++d) put_f16(qq + 2 * d, oracle_f32_to_f16(pq[d]));
            float S = 0.0f, M = -INFINITY;
            memset(vkq, 0, sizeof(float) * (size_t)head_dim);
            memset(vkq16, 0, sizeof(uint16_t) * (size_t)head_dim);
            for (int c = 0; c < n_cells; ++c) {
                if (!visible(cell_pos, q_pos, t, c)) continue;
                const uint8_t *kr = K + ((int64_t)c * n_head_kv + hk) * krow;
                float s;
                if (k_type == ORACLE_T_Q8_0) {
                    float sumf = 0.0f;
                    for (int b = 0; b < head_dim / 32; ++b) {
                        const uint8_t *xb = kr + b * 34, *yb = qq + b * 34;
                        int sumi = 0;
                        for (int j = 0; j < 32; ++j)
                            sumi += (int)(int8_t)xb[2 + j] * (int)(int8_t)yb[2 + j];
                        sumf += (float)sumi * (oracle_f16_to_f32(get_f16(xb)) *
                                               oracle_f16_to_f32(get_f16(yb)));
                    }
                    s = sumf;
                } else if (k_type == ORACLE_T_Q4_0) {
                    /* ggml's vec_dot_q4_0_q8_0: low nibbles (minus 8) against
                     * query quants 0-15, high nibbles against 16-31, then
                     * sumi * d_k * d_q left to right */
                    float sumf = 0.0f;
                    for (int b = 0; b < head_dim / 32; ++b) {
                        const uint8_t *xb = kr + b * 18, *yb = qq + b * 34;
                        int sumi0 = 0, sumi1 = 0;
                        for (int j = 0; j < 16; ++j) {
                            sumi0 += ((int)(xb[2 + j] & 15) - 8) * (int)(int8_t)yb[2 + j];
                            sumi1 += ((int)(xb[2 + j] >> 4) - 8) * (int)(int8_t)yb[2 + j + 16];
                        }
                        sumf += (float)(sumi0 + sumi1) * oracle_f16_to_f32(get_f16(xb)) *
                                oracle_f16_to_f32(get_f16(yb));
                    }
                    s = sumf;
                } else {
                    double sumf = 0.0;
                    for (int d = 0; d < head_dim; ++d)
                        sumf += (double)(oracle_f16_to_f32(get_f16(kr + 2 * d)) *
                                         oracle_f16_to_f32(get_f16(qq + 2 * d)));
                    s = (float)sumf;
                }
                s = s * scale;
                const float Mold = M;
                float ms = 1.0f, vs = 1.0f;
                const uint8_t *vr = V + ((int64_t)c * n_head_kv + hk) * vrow;
                if (v_type == ORACLE_T_F16) {
                    if (s > M) {
                        M = s;
                        ms = expf(Mold - M);
                        for (int d = 0; d < head_dim; ++d)
                            vkq16[d] = oracle_f32_to_f16(oracle_f16_to_f32(vkq16[d]) * ms);
                    } else {
                        vs = expf(s - M);
                    }
                    for (int d = 0; d < head_dim; ++d)
                        vkq16[d] = oracle_f32_to_f16(oracle_f16_to_f32(vkq16[d]) +
                                                     oracle_f16_to_f32(get_f16(vr + 2 * d)) * vs);
                } else {
                    if (s > M) {
                        M = s;
                        ms = expf(Mold - M);
                        for (int d = 0; d < head_dim; ++d) vkq[d] *= ms;
                    } else {
                        vs = expf(s - M);
                    }
                    to_float_row(v_type, vr, v32, head_dim);
                    for (int d = 0; d < head_dim; ++d) vkq[d] += v32[d] * vs;
                }
                S = S * ms + vs;
            }
            if (v_type == ORACLE_T_F16)
                for (int d = 0; d < head_dim; ++d) vkq[d] = oracle_f16_to_f32(vkq16[d]);
            const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
            float *po = out + (size_t)r * head_dim;
            for (int d = 0; d < head_dim; ++d) po[d] = vkq[d] * S_inv;
        }
        free(vkq);
        free(v32);
        free(vkq16);
        free(qq);
    }
    return 0;
}

int oracle_fa_f64(int k_type, int v_type, const float *q, const void *k, const void *v,
                  const int32_t *cell_pos, const int32_t *q_pos, int n_tokens, int n_head,
                  int n_head_kv, int head_dim, int n_cells, double scale, double *out,
                  int n_threads) {
    if (n_head_kv <= 0 || n_head % n_head_kv) return -1;
    const int g = n_head / n_head_kv;
    const int64_t krow = oracle_row_bytes(k_type, head_dim);
    const int64_t vrow = oracle_row_bytes(v_type, head_dim);
    if (krow < 0 || vrow < 0) return -1;
    const uint8_t *K = (const uint8_t *)k, *V = (const uint8_t *)v;
    const int n_rows = n_tokens * n_head;
    (void)n_threads;
#ifdef _OPENMP
#pragma omp parallel num_threads(n_threads > 0 ? n_threads : 1)
#endif
    {
        float *kf = (float *)malloc(sizeof(float) * (size_t)head_dim);
        float *vf = (float *)malloc(sizeof(float) * (size_t)head_dim);
        double *sc = (double *)malloc(sizeof(double) * (size_t)(n_cells > 0 ? n_cells : 1));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int r = 0; r < n_rows; ++r) {
            const int t = r / n_head, h = r % n_head, hk = h / g;
            const float *pq = q + (size_t)r * head_dim;
            double mx = -INFINITY;
            for (int c = 0; c < n_cells; ++c) {
                sc[c] = -INFINITY;
                if (!visible(cell_pos, q_pos, t, c)) continue;
                to_float_row(k_type, K + ((int64_t)c * n_head_kv + hk) * krow, kf, head_dim);
                double dot = 0.0;
                for (int d = 0; d < head_dim; ++d) dot += (double)pq[d] * (double)kf[d];
                sc[c] = dot * scale;
                if (sc[c] > mx) mx = sc[c];
            }
            double *po = out + (size_t)r * head_dim;
            for (int d = 0; d < head_dim; ++d) po[d] = 0.0;
            if (mx == -INFINITY) continue;
            double l = 0.0;
            for (int c = 0; c < n_cells; ++c) {
                if (sc[c] == -INFINITY) continue;
                const double p = exp(sc[c] - mx);
                l += p;
                to_float_row(v_type, V + ((int64_t)c * n_head_kv + hk) * vrow, vf, head_dim);
                for (int d = 0; d < head_dim; ++d) po[d] += p * (double)vf[d];
            }
            for (int d = 0; d < head_dim; ++d) po[d] /= l;
        }
        free(kf);
        free(vf);
        free(sc);
    }
    return 0;
}
