// kvm_retrieval.hip -- capture-side index upkeep (query accumulator, mean-K sums)
// and the retrieval step: score_retrieval + top-k + chronological window layout.
//
// Bit-exactness: the scorer restates llama-memory-kvmem.cpp:4149-4196 with the
// same fp32 operation order, each operation one IEEE rounding (this file is
// compiled with -ffp-contract=off and correctly rounded `/` and sqrtf), and the
// per-head/per-layer accumulation in double in the same order.
#include "kvm_internal.h"

// ---------------------------------------------------------------------------
// Query accumulator (llama-memory-kvmem.cpp:3300-3315, 3417-3433)
// ---------------------------------------------------------------------------
__global__ void k_query_add(float *q_sum, uint32_t *q_count, uint32_t n_embd, const float *rows,
                            uint32_t n_rows) {
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j < n_embd) {
        float s = q_sum[j];
        for (uint32_t r = 0; r < n_rows; ++r) s = kvm_fadd(s, rows[(uint64_t)r * n_embd + j]);
        q_sum[j] = s;
    }
    if (j == 0) q_count[0] += n_rows;
}

__global__ void k_zero_f32(float *p, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}
__global__ void k_zero_u32(uint32_t *p, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

extern "C" int kvm_query_reset(kvm_state *st, const kvm_query_acc *acc) {
    if (!st || !acc || !acc->q_sum || !acc->q_count) return kvm_fail(st, KVM_EINVAL, "query_reset: args");
    KVM_HIP(st, hipSetDevice(st->device));
    const uint64_t n = (uint64_t)acc->n_layer * acc->n_head * acc->head_dim;
    if (n) hipLaunchKernelGGL(k_zero_f32, dim3(kvm_cdiv(n, 256)), dim3(256), 0, st->stream, acc->q_sum, n);
    if (acc->n_layer)
        hipLaunchKernelGGL(k_zero_u32, dim3(kvm_cdiv(acc->n_layer, 256)), dim3(256), 0, st->stream,
                           acc->q_count, (uint64_t)acc->n_layer);
    KVM_LAUNCH_CHECK(st, "query_reset");
    return KVM_OK;
}

extern "C" int kvm_query_add(kvm_state *st, const kvm_query_acc *acc, uint32_t il,
                             const float *q_rows, uint32_t n_rows) {
    if (!st || !acc || !acc->q_sum || !acc->q_count || !q_rows) return kvm_fail(st, KVM_EINVAL, "query_add: args");
    if (il >= acc->n_layer) return kvm_fail(st, KVM_ERANGE, "query_add: layer %u >= %u", il, acc->n_layer);
    if (n_rows == 0) return KVM_OK;
    KVM_HIP(st, hipSetDevice(st->device));
    const uint32_t n_embd = acc->n_head * acc->head_dim;
    hipLaunchKernelGGL(k_query_add, dim3(kvm_cdiv(n_embd, 256)), dim3(256), 0, st->stream,
                       acc->q_sum + (uint64_t)il * n_embd, acc->q_count + il, n_embd, q_rows, n_rows);
    KVM_LAUNCH_CHECK(st, "query_add");
    return KVM_OK;
}

// ---------------------------------------------------------------------------
// Mean-K sums (RawKvStore::write_layer_mean_k / add_mean_f32,
// raw_kv_store.cpp:215-234, 685-705).  Device layout of the index:
// k_sum[il][e][block] (embedding-major, blocks fastest) so the scorer's lanes
// (one block each) read consecutive addresses.
// ---------------------------------------------------------------------------
__global__ void k_meank_add(float *k_sum, uint32_t *mean_tokens, uint8_t *present, uint32_t cap,
                            uint32_t n_embd, uint32_t bt, uint32_t pos0, uint32_t n,
                            const float *rows) {
    const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t ci = blockIdx.y;                  // chunk = one block's share
    const uint32_t bid = pos0 / bt + ci;
    const uint32_t start = ci == 0 ? pos0 : bid * bt;
    const uint32_t end_blk = (bid + 1) * bt;
    const uint32_t end = pos0 + n < end_blk ? pos0 + n : end_blk;
    if (bid >= cap || start >= end) return;
    const uint32_t off = start - bid * bt, take = end - start;
    if (e < n_embd) {
        float *p = k_sum + (uint64_t)e * cap + bid;
        float s = off == 0 ? 0.0f : *p;
        for (uint32_t t = start; t < end; ++t) s = kvm_fadd(s, rows[(uint64_t)(t - pos0) * n_embd + e]);
        *p = s;
    }
    if (e == 0) {
        const uint32_t mt = mean_tokens[bid];
        mean_tokens[bid] = off == 0 ? take : (mt > off + take ? mt : off + take);
        if (present) present[bid] = 1;
    }
}

extern "C" int kvm_meank_add(kvm_state *st, const kvm_meank_index *ix, uint32_t il, uint32_t pos0,
                             uint32_t n, const float *k_rows) {
    if (!st || !ix || !ix->k_sum || !ix->mean_tokens || !k_rows || ix->block_tokens == 0)
        return kvm_fail(st, KVM_EINVAL, "meank_add: args");
    if (il >= ix->n_layer) return kvm_fail(st, KVM_ERANGE, "meank_add: layer %u", il);
    if (n == 0) return KVM_OK;
    const uint32_t bt = ix->block_tokens;
    const uint32_t last = (pos0 + n - 1) / bt;
    if (last >= ix->n_blocks) return kvm_fail(st, KVM_ERANGE, "meank_add: block %u >= capacity %u", last, ix->n_blocks);
    KVM_HIP(st, hipSetDevice(st->device));
    const uint32_t n_embd = ix->n_head_kv * ix->head_dim;
    const uint32_t n_chunks = last - pos0 / bt + 1;
    hipLaunchKernelGGL(k_meank_add, dim3(kvm_cdiv(n_embd, 256), n_chunks), dim3(256), 0, st->stream,
                       ix->k_sum + (uint64_t)il * n_embd * ix->n_blocks,
                       ix->mean_tokens + (uint64_t)il * ix->n_blocks, ix->present, ix->n_blocks, n_embd,
                       bt, pos0, n, k_rows);
    KVM_LAUNCH_CHECK(st, "meank_add");
    return KVM_OK;
}

// ---------------------------------------------------------------------------
// Scoring.  Workgroup = n_head_kv waves; wave h scores kv head h of 64
// consecutive blocks (lane = block).  The per-(layer, head) query vector
// qv = qh * invq and its sequential norm nq do not depend on the block and are
// built once per workgroup in LDS with the reference's operation order.
// ---------------------------------------------------------------------------
struct score_args {
    const float *q_sum;
    const uint32_t *q_count;
    const float *k_sum;
    const uint32_t *mean_tokens;
    const uint8_t *present;
    double *scores;
    uint32_t n_blocks, cap, n_layer, n_head, H;
};

template <int D, int CH, int MAXT>
__global__ void __launch_bounds__(MAXT) k_score(score_args a) {
    extern __shared__ float s_qv[];                  // [n_layer][H*D] then nq[n_layer][H]
    const uint32_t HD = a.H * D;
    float *s_nq = s_qv + (size_t)a.n_layer * HD;
    __shared__ float s_cos[16][64];
    const uint32_t tid = threadIdx.x, nthr = blockDim.x;
    const uint32_t g = a.H == 0 ? 1u : a.n_head / a.H;
    const uint32_t g1 = g > 1u ? g : 1u;
    for (uint32_t idx = tid; idx < a.n_layer * HD; idx += nthr) {
        const uint32_t il = idx / HD, h = (idx % HD) / D, d = idx % D;
        float qh = 0.0f;
        for (uint32_t gi = 0; gi < g; ++gi) {
            const uint32_t qi = h * g + gi;
            if (qi >= a.n_head) break;
            qh = kvm_fadd(qh, a.q_sum[(uint64_t)il * a.n_head * D + (uint64_t)qi * D + d]);
        }
        const float invq = kvm_fdiv(1.0f, (float)(a.q_count[il] * g1));
        s_qv[idx] = kvm_fmul(qh, invq);
    }
    __syncthreads();
    for (uint32_t idx = tid; idx < a.n_layer * a.H; idx += nthr) {
        const float *qv = s_qv + (size_t)(idx / a.H) * HD + (size_t)(idx % a.H) * D;
        float nq = 0.0f;
        for (uint32_t d = 0; d < D; ++d) nq = kvm_fadd(nq, kvm_fmul(qv[d], qv[d]));
        s_nq[idx] = nq;
    }
    __syncthreads();

    const uint32_t h = tid >> 6, lane = tid & 63;
    const uint32_t b = blockIdx.x * 64 + lane;
    const bool valid = b < a.n_blocks;
    double acc = 0.0;
    uint32_t nlay = 0;
    for (uint32_t il = 0; il < a.n_layer; ++il) {
        if (a.q_count[il] == 0) continue;             // uniform across the workgroup
        float c = 0.0f;
        if (valid) {
            const uint32_t mt = a.mean_tokens[(uint64_t)il * a.cap + b];
            const float inv = mt ? kvm_fdiv(1.0f, (float)mt) : 0.0f;
            const float *ks = a.k_sum + (uint64_t)il * HD * a.cap + (uint64_t)h * D * a.cap + b;
            // Issue CH dims of the column at once (one coalesced 256-byte access
            // per dim across the wave) before the sequential fp32 chain over them,
            // so the index streams with CH loads in flight per lane.
            const float *qv = s_qv + (size_t)il * HD + (size_t)h * D;
            float dot = 0.0f, nk = 0.0f;
            for (uint32_t c0 = 0; c0 < (uint32_t)D; c0 += CH) {
                float kraw[CH];
#pragma unroll
                for (uint32_t d = 0; d < (uint32_t)CH; ++d)
                    kraw[d] = __builtin_nontemporal_load(ks + (uint64_t)(c0 + d) * a.cap);
#pragma unroll
                for (uint32_t d = 0; d < (uint32_t)CH; ++d) {
                    const float kh = mt ? kvm_fmul(kraw[d], inv) : 0.0f;
                    dot = kvm_fadd(dot, kvm_fmul(qv[c0 + d], kh));
                    nk = kvm_fadd(nk, kvm_fmul(kh, kh));
                }
            }
            const float den = kvm_fadd(kvm_fmul(kvm_fsqrt(s_nq[il * a.H + h]), kvm_fsqrt(nk)), 1e-6f);
            c = kvm_fdiv(dot, den);
        }
        s_cos[h][lane] = c;
        __syncthreads();
        if (h == 0 && valid) {
            double layer = 0.0;
            for (uint32_t hh = 0; hh < a.H; ++hh) layer += (double)s_cos[hh][lane];
            acc += layer / (double)(a.H > 1 ? a.H : 1);
            nlay++;
        }
        __syncthreads();
    }
    if (h == 0 && valid) {
        double sc = nlay ? acc / (double)nlay : 0.0;
        if (a.present && !a.present[b]) sc = 0.0;
        a.scores[b] = sc;
    }
}

// ---------------------------------------------------------------------------
// Top-k + layout: one workgroup of 1024 threads.
// ---------------------------------------------------------------------------
struct topk_args {
    const double *scores;
    const uint32_t *n_tokens;
    const uint32_t *mandatory;
    const uint32_t *slot_block;
    const int32_t *slot_base;
    uint32_t *ids;
    int32_t *to_base;
    uint32_t *stage_slots;
    uint32_t *info;
    uint32_t n, budget, sink, recent, n_mand, n_slots, cap;
};

// order-preserving map of a double to uint64 (-0.0 folded onto +0.0, so the
// two compare equal as in the reference's `sa != sb` test)
__device__ inline uint64_t ord_key(double x) {
    if (x == 0.0) x = 0.0;
    const uint64_t u = (uint64_t)__double_as_longlong(x);
    return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

// exclusive prefix sum over the workgroup; returns the total through *total
__device__ uint32_t block_scan(uint32_t v, uint32_t *s_tmp, uint32_t *total) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, nw = blockDim.x >> 6;
    uint32_t x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(x, o, 64);
        if (lane >= (uint32_t)o) x += y;
    }
    if (lane == 63) s_tmp[wid] = x;
    __syncthreads();
    if (tid == 0) {
        uint32_t run = 0;
        for (uint32_t w = 0; w < nw; ++w) {
            const uint32_t t = s_tmp[w];
            s_tmp[w] = run;
            run += t;
        }
        s_tmp[nw] = run;
    }
    __syncthreads();
    const uint32_t res = x - v + s_tmp[wid];
    *total = s_tmp[nw];
    __syncthreads();
    return res;
}

// Selection of the `need` best candidates under the strict order
// (score desc, block id desc): an 8-pass MSB-first radix select over the
// order-preserving 64-bit keys finds the need-th largest key T; keys above T
// are taken, and among keys equal to T the highest block ids.
__global__ void __launch_bounds__(1024) k_topk(topk_args a) {
    __shared__ uint64_t s_key[KVM_MAX_TOPK_BLOCKS];
    __shared__ uint8_t s_kept[KVM_MAX_TOPK_BLOCKS];
    __shared__ uint32_t s_hist[256];
    __shared__ uint32_t s_tmp[32];
    __shared__ uint32_t s_count, s_k;
    __shared__ uint64_t s_prefix;
    const uint32_t tid = threadIdx.x, nthr = blockDim.x, n = a.n;
    const bool all = a.budget == 0 || n <= a.budget;
    for (uint32_t i = tid; i < n; i += nthr) s_kept[i] = all ? 1 : 0;
    __syncthreads();
    if (!all) {
        // sink prefix, mandatory ids newest first, recent tail (kvmem_store.cpp:520-545)
        if (tid == 0) {
            uint32_t count = 0;
            const uint32_t sink = a.sink < n ? a.sink : n, recent = a.recent < n ? a.recent : n;
            for (uint32_t i = 0; i < sink && count < a.budget; ++i)
                if (!s_kept[i]) { s_kept[i] = 1; ++count; }
            for (uint32_t i = a.n_mand; i > 0 && count < a.budget; --i) {
                const uint32_t id = a.mandatory[i - 1];
                if (id < n && !s_kept[id]) { s_kept[id] = 1; ++count; }
            }
            for (uint32_t i = 0; i < recent && count < a.budget; ++i) {
                const uint32_t id = n - 1 - i;
                if (!s_kept[id]) { s_kept[id] = 1; ++count; }
            }
            s_count = count;
        }
        __syncthreads();
        const uint32_t count = s_count;
        if (count < a.budget) {
            uint32_t nc_local = 0;
            for (uint32_t i = tid; i < n; i += nthr) {
                s_key[i] = ord_key(a.scores[i]);
                nc_local += !s_kept[i];
            }
            uint32_t ncand;
            (void)block_scan(nc_local, s_tmp, &ncand);
            const uint32_t need = a.budget - count < ncand ? a.budget - count : ncand;
            if (tid == 0) { s_prefix = 0; s_k = need; }
            uint64_t mask = 0;
            for (int shift = 56; shift >= 0 && need; shift -= 8) {
                if (tid < 256) s_hist[tid] = 0;
                __syncthreads();
                const uint64_t prefix = s_prefix;
                for (uint32_t i = tid; i < n; i += nthr)
                    if (!s_kept[i] && (s_key[i] & mask) == prefix)
                        atomicAdd(&s_hist[(uint32_t)(s_key[i] >> shift) & 255u], 1u);
                __syncthreads();
                if (tid < 64) {
                    // lane l owns bins 255-4l .. 252-4l (descending)
                    uint32_t c[4], tot = 0;
#pragma unroll
                    for (int j = 0; j < 4; ++j) { c[j] = s_hist[255 - 4 * tid - j]; tot += c[j]; }
                    uint32_t incl = tot;
#pragma unroll
                    for (int o = 1; o < 64; o <<= 1) {
                        const uint32_t y = __shfl_up(incl, o, 64);
                        if (tid >= (uint32_t)o) incl += y;
                    }
                    uint32_t run = incl - tot;           // keys in higher bins
                    const uint32_t k = s_k;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if (run < k && k <= run + c[j]) {
                            s_prefix = prefix | ((uint64_t)(255 - 4 * tid - j) << shift);
                            s_k = k - run;
                        }
                        run += c[j];
                    }
                }
                mask |= (uint64_t)0xff << shift;
                __syncthreads();
            }
            // keys above T are selected; among keys equal to T the s_k highest ids
            const uint64_t T = s_prefix;
            const uint32_t ktie = s_k;
            const uint32_t per = (n + nthr - 1) / nthr;
            const uint32_t i0 = tid * per, i1 = i0 + per < n ? i0 + per : n;
            uint32_t ties = 0;
            for (uint32_t i = i0; i < i1; ++i) ties += !s_kept[i] && s_key[i] == T;
            uint32_t n_ties;
            uint32_t before = block_scan(ties, s_tmp, &n_ties);
            for (uint32_t i = i0; i < i1 && need; ++i) {
                if (s_kept[i]) continue;
                if (s_key[i] > T) {
                    s_kept[i] = 2;
                } else if (s_key[i] == T) {
                    if (n_ties - 1 - before < ktie) s_kept[i] = 2;     // rank by descending id
                    ++before;
                }
            }
            __syncthreads();
        }
    }
    // ascending compaction of the kept flags
    const uint32_t per = (n + nthr - 1) / nthr;
    const uint32_t i0 = tid * per, i1 = i0 + per < n ? i0 + per : n;
    uint32_t local = 0;
    for (uint32_t i = i0; i < i1; ++i) local += s_kept[i] != 0;
    uint32_t n_sel;
    uint32_t rank = block_scan(local, s_tmp, &n_sel);
    const bool fits = n_sel <= a.cap;
    if (fits)
        for (uint32_t i = i0; i < i1; ++i)
            if (s_kept[i]) a.ids[rank++] = i;
    __syncthreads();
    // window positions: to_base[k] = sum of n_tokens of the selected blocks before k
    const uint32_t per2 = (n_sel + nthr - 1) / nthr;
    const uint32_t k0 = tid * per2, k1 = fits ? (k0 + per2 < n_sel ? k0 + per2 : n_sel) : k0;
    uint32_t tok = 0;
    for (uint32_t k = k0; k < k1; ++k) tok += a.n_tokens[a.ids[k]];
    uint32_t total;
    uint32_t base = block_scan(tok, s_tmp, &total);
    for (uint32_t k = k0; k < k1; ++k) {
        a.to_base[k] = (int32_t)base;
        base += a.n_tokens[a.ids[k]];
    }
    __syncthreads();
    // slots whose (block, base) differ from the new layout
    uint32_t need_local = 0;
    const uint32_t ns = fits ? (n_sel < a.n_slots ? n_sel : a.n_slots) : 0;
    const uint32_t per3 = (ns + nthr - 1) / nthr;
    const uint32_t s0 = tid * per3, s1 = s0 + per3 < ns ? s0 + per3 : ns;
    for (uint32_t s = s0; s < s1; ++s)
        need_local += !a.slot_block || a.slot_block[s] != a.ids[s] || a.slot_base[s] != a.to_base[s];
    uint32_t n_stage;
    uint32_t pos = block_scan(need_local, s_tmp, &n_stage);
    for (uint32_t s = s0; s < s1; ++s)
        if (!a.slot_block || a.slot_block[s] != a.ids[s] || a.slot_base[s] != a.to_base[s])
            a.stage_slots[pos++] = s;
    if (tid == 0) {
        a.info[0] = n_sel;
        a.info[1] = total;
        a.info[2] = n_stage;
        a.info[3] = fits ? (n_sel <= a.n_slots || a.n_slots == 0 ? 0u : 2u) : 1u;
    }
}

static int launch_topk(kvm_state *st, const double *scores, const kvm_select_params *p,
                       const kvm_window *w, const kvm_selection *out) {
    if (w && (kvm_window_check(w) || !w->slot_block || !w->slot_base))
        return kvm_fail(st, KVM_EINVAL, "topk: bad window or window without slot map");
    topk_args ta{scores, p->n_tokens, p->mandatory,
                 w ? w->slot_block : nullptr, w ? w->slot_base : nullptr,
                 out->ids, out->to_base, out->stage_slots, out->info,
                 p->n_blocks, p->budget_blocks, p->sink_blocks, p->recent_blocks, p->n_mandatory,
                 w ? w->n_cells / w->block_tokens : 0u, out->cap};
    hipLaunchKernelGGL(k_topk, dim3(1), dim3(1024), 0, st->stream, ta);
    KVM_LAUNCH_CHECK(st, "topk");
    return KVM_OK;
}

static int check_select(kvm_state *st, const kvm_select_params *p, const kvm_selection *out) {
    if (!p || !out) return kvm_fail(st, KVM_EINVAL, "select: null argument");
    if (!p->n_tokens || !out->ids || !out->to_base || !out->stage_slots || !out->info)
        return kvm_fail(st, KVM_EINVAL, "select: null buffer");
    if (p->n_blocks > KVM_MAX_TOPK_BLOCKS) return kvm_fail(st, KVM_ERANGE, "select: n_blocks %u > %u", p->n_blocks, KVM_MAX_TOPK_BLOCKS);
    const uint32_t want = p->budget_blocks == 0 || p->n_blocks <= p->budget_blocks ? p->n_blocks : p->budget_blocks;
    if (want > out->cap) return kvm_fail(st, KVM_ERANGE, "select: selection capacity %u < %u", out->cap, want);
    if (p->n_mandatory && !p->mandatory) return kvm_fail(st, KVM_EINVAL, "select: mandatory list missing");
    return KVM_OK;
}

extern "C" int kvm_select_topk(kvm_state *st, const double *scores, const kvm_select_params *p,
                               const kvm_window *w, const kvm_selection *out) {
    if (!st) return KVM_EINVAL;
    int rc = check_select(st, p, out);
    if (rc) return rc;
    if (p->n_blocks && !scores) return kvm_fail(st, KVM_EINVAL, "select_topk: null scores");
    KVM_HIP(st, hipSetDevice(st->device));
    return launch_topk(st, scores, p, w, out);
}

extern "C" int kvm_score_topk(kvm_state *st, const kvm_meank_index *ix, const kvm_query_acc *q,
                              const kvm_select_params *p, const kvm_window *w,
                              const kvm_selection *out) {
    if (!st) return KVM_EINVAL;
    if (!ix || !q) return kvm_fail(st, KVM_EINVAL, "score_topk: null argument");
    int rc = check_select(st, p, out);
    if (rc) return rc;
    if (!ix->k_sum || !ix->mean_tokens || !q->q_sum || !q->q_count || !out->scores)
        return kvm_fail(st, KVM_EINVAL, "score_topk: null buffer");
    if (p->n_blocks > ix->n_blocks) return kvm_fail(st, KVM_ERANGE, "score_topk: n_blocks %u > index capacity %u", p->n_blocks, ix->n_blocks);
    if (q->n_layer != ix->n_layer || q->head_dim != ix->head_dim) return kvm_fail(st, KVM_EINVAL, "score_topk: query/index shape mismatch");
    if (ix->head_dim != 128 && ix->head_dim != 256) return kvm_fail(st, KVM_EUNSUPPORTED, "score_topk: head_dim %u", ix->head_dim);
    if (ix->n_head_kv == 0 || ix->n_head_kv > 16 || q->n_head % ix->n_head_kv)
        return kvm_fail(st, KVM_EUNSUPPORTED, "score_topk: n_head %u / n_head_kv %u", q->n_head, ix->n_head_kv);
    const size_t lds = ((size_t)ix->n_layer * ix->n_head_kv * ix->head_dim + (size_t)ix->n_layer * ix->n_head_kv) * 4;
    if (lds > 120 * 1024) return kvm_fail(st, KVM_ERANGE, "score_topk: %u layers x %u heads x %u dims exceeds LDS", ix->n_layer, ix->n_head_kv, ix->head_dim);
    KVM_HIP(st, hipSetDevice(st->device));
    if (p->n_blocks) {
        score_args sa{q->q_sum, q->q_count, ix->k_sum, ix->mean_tokens, ix->present, out->scores,
                      p->n_blocks, ix->n_blocks, ix->n_layer, q->n_head, ix->n_head_kv};
        // up to 4 kv heads: 256 threads, 128 dims in flight per lane; more heads
        // (up to 16 waves) keep 32 in flight within the smaller register budget
        const bool small = ix->n_head_kv <= 4;
        const void *fn = ix->head_dim == 256 ? (small ? (const void *)k_score<256, 128, 256> : (const void *)k_score<256, 32, 1024>)
                                              : (small ? (const void *)k_score<128, 128, 256> : (const void *)k_score<128, 32, 1024>);
        if (lds > 64 * 1024)
            KVM_HIP(st, hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        const dim3 grid(kvm_cdiv(p->n_blocks, 64)), block(64 * ix->n_head_kv);
        if (ix->head_dim == 256) {
            if (small) hipLaunchKernelGGL((k_score<256, 128, 256>), grid, block, lds, st->stream, sa);
            else hipLaunchKernelGGL((k_score<256, 32, 1024>), grid, block, lds, st->stream, sa);
        } else {
            if (small) hipLaunchKernelGGL((k_score<128, 128, 256>), grid, block, lds, st->stream, sa);
            else hipLaunchKernelGGL((k_score<128, 32, 1024>), grid, block, lds, st->stream, sa);
        }
        KVM_LAUNCH_CHECK(st, "score");
    }
    return launch_topk(st, out->scores, p, w, out);
}
