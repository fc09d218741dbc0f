// kvm_retrieval.hip -- capture-side index upkeep (query accumulator, mean-K sums)
// and the retrieval step: score_retrieval + top-k + chronological window layout.
//
// Bit-exactness: the scorer restates llama-memory-kvmem.cpp:4149-4196 with the
// same fp32 operation order, each operation one IEEE rounding (this file is
// compiled with -ffp-contract=off and correctly rounded `/` and sqrtf), and the
// per-head/per-layer accumulation in double in the same order.
#include "kvm_score_dev.h"
#include "kvm_stagein_dev.h"
#include "kvm_topk_dev.h"

// Captured views (view_args, kvm_internal.h) enter every sum converted exactly
// to fp32, as the reference's token-major flattening does
// (bytes_to_f32_token_major, llama-memory-kvmem.cpp:3317-3341; the f16 K
// branch, 3405-3410, converts the same way).
//
// Rows of one query-accumulation launch: their keep flags travel as a bitmask
// in the kernel arguments.
#define KVM_QVIEW_ROWS 2048u

// ---------------------------------------------------------------------------
// Query accumulator (llama-memory-kvmem.cpp:3300-3315 reset, 3417-3433 /
// 3470-3483 add): q_sum[il][e] += row[e] for the kept rows in token order,
// q_count[il] += kept rows.
// ---------------------------------------------------------------------------
struct qview_args {
    view_args v;
    float *q_sum;
    uint32_t *q_count;
    uint32_t n_embd, t0, n_rows, n_kept;
    uint32_t keep[KVM_QVIEW_ROWS / 32];     // bit r: row t0 + r is added (all set without a mask)
};

__global__ void k_query_add(qview_args a) {
    const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e < a.n_embd) {
        float s = a.q_sum[e];
        for (uint32_t r = 0; r < a.n_rows; ++r)
            if (a.keep[r >> 5] >> (r & 31) & 1u) s = kvm_fadd(s, view_load(a.v, a.t0 + r, e));
        a.q_sum[e] = s;
    }
    if (e == 0) a.q_count[0] += a.n_kept;
}

__global__ void k_zero_f32(float *p, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}
__global__ void k_zero_u32(uint32_t *p, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// The query terms of score_retrieval (llama-memory-kvmem.cpp:4167-4185) for
// one (layer, kv head) per workgroup of 64 threads: lane l forms qv of dims l,
// l + 64, ... (the group's rows added in row order from 0.0f, times 1 / (q_count
// g)), then lane 0 sums qv^2 over the dims in order from LDS.  The same
// operations as the scorer's own formation, so the scores do not change.
template <int D>
__global__ void __launch_bounds__(64) k_query_terms(const float *q_sum, const uint32_t *q_count, float *q_vec,
                                                    float *q_norm, uint32_t il0, uint32_t n_head, uint32_t H) {
    const uint32_t il = il0 + blockIdx.x, h = blockIdx.y, l = threadIdx.x, g = n_head / H;
    __shared__ float s_sq[D];
    const uint32_t qc = q_count[il];
    const float invq = kvm_recip_or0((float)(qc * (g > 1u ? g : 1u)));
    const float *qrow = q_sum + ((uint64_t)il * n_head + (uint64_t)h * g) * D;
    float *out = q_vec + ((uint64_t)il * H + h) * D;
    for (uint32_t d = l; d < (uint32_t)D; d += 64u) {
        float qh = 0.0f;
        for (uint32_t gi = 0; gi < g; ++gi) qh = kvm_fadd(qh, qrow[(uint64_t)gi * D + d]);
        const float qv = kvm_fmul(qh, invq);
        out[d] = qv;
        s_sq[d] = kvm_fmul(qv, qv);
    }
    __syncthreads();
    if (l == 0) {
        float nq = 0.0f;
        for (uint32_t d = 0; d < (uint32_t)D; ++d) nq = kvm_fadd(nq, s_sq[d]);
        q_norm[(uint64_t)il * H + h] = nq;
    }
}

// An accumulator that carries the query terms: their buffers and grouping.
static int query_terms_check(kvm_state *st, const kvm_query_acc *acc, const char *who) {
    if (!acc->q_vec) return KVM_OK;
    if (!acc->q_norm || acc->n_head_kv == 0 || acc->n_head % acc->n_head_kv)
        return kvm_fail(st, KVM_EINVAL, "%s: q_vec needs q_norm and n_head_kv dividing n_head (%u / %u)", who,
                        acc->n_head, acc->n_head_kv);
    if (acc->head_dim != 128 && acc->head_dim != 256)
        return kvm_fail(st, KVM_EUNSUPPORTED, "%s: query terms at head_dim %u", who, acc->head_dim);
    return KVM_OK;
}

// Forms the terms of layers [il0, il0 + n) on the state's stream.
static int query_terms_launch(kvm_state *st, const kvm_query_acc *acc, uint32_t il0, uint32_t n) {
    if (!acc->q_vec || n == 0) return KVM_OK;
    const dim3 grid(n, acc->n_head_kv);
    if (acc->head_dim == 256)
        hipLaunchKernelGGL(k_query_terms<256>, grid, dim3(64), 0, st->stream, acc->q_sum, acc->q_count, acc->q_vec,
                           acc->q_norm, il0, acc->n_head, acc->n_head_kv);
    else
        hipLaunchKernelGGL(k_query_terms<128>, grid, dim3(64), 0, st->stream, acc->q_sum, acc->q_count, acc->q_vec,
                           acc->q_norm, il0, acc->n_head, acc->n_head_kv);
    KVM_LAUNCH_CHECK(st, "query_terms");
    return KVM_OK;
}

extern "C" int kvm_query_reset(kvm_state *st, const kvm_query_acc *acc) {
    if (!st || !acc || !acc->q_sum || !acc->q_count) return kvm_fail(st, KVM_EINVAL, "query_reset: args");
    int rc = query_terms_check(st, acc, "query_reset");
    if (rc) return rc;
    KVM_HIP(st, hipSetDevice(st->device));
    const uint64_t n = (uint64_t)acc->n_layer * acc->n_head * acc->head_dim;
    if (n) hipLaunchKernelGGL(k_zero_f32, dim3(kvm_cdiv(n, 256)), dim3(256), 0, st->stream, acc->q_sum, n);
    if (acc->n_layer)
        hipLaunchKernelGGL(k_zero_u32, dim3(kvm_cdiv(acc->n_layer, 256)), dim3(256), 0, st->stream,
                           acc->q_count, (uint64_t)acc->n_layer);
    if (acc->q_vec) {
        // the terms of an empty accumulator: qv = 0 * (1 / 0 -> 0), nq = 0
        const uint64_t nv = (uint64_t)acc->n_layer * acc->n_head_kv * acc->head_dim;
        const uint64_t nn = (uint64_t)acc->n_layer * acc->n_head_kv;
        if (nv) hipLaunchKernelGGL(k_zero_f32, dim3(kvm_cdiv(nv, 256)), dim3(256), 0, st->stream, acc->q_vec, nv);
        if (nn) hipLaunchKernelGGL(k_zero_f32, dim3(kvm_cdiv(nn, 256)), dim3(256), 0, st->stream, acc->q_norm, nn);
    }
    KVM_LAUNCH_CHECK(st, "query_reset");
    return KVM_OK;
}

extern "C" int kvm_query_refresh(kvm_state *st, const kvm_query_acc *acc) {
    if (!st || !acc || !acc->q_sum || !acc->q_count) return kvm_fail(st, KVM_EINVAL, "query_refresh: args");
    int rc = query_terms_check(st, acc, "query_refresh");
    if (rc) return rc;
    KVM_HIP(st, hipSetDevice(st->device));
    return query_terms_launch(st, acc, 0, acc->n_layer);
}

extern "C" int kvm_query_add_view(kvm_state *st, const kvm_query_acc *acc, uint32_t il, const kvm_view *q,
                                  const uint8_t *keep) {
    if (!st || !acc || !acc->q_sum || !acc->q_count) return kvm_fail(st, KVM_EINVAL, "query_add: args");
    if (il >= acc->n_layer) return kvm_fail(st, KVM_ERANGE, "query_add: layer %u >= %u", il, acc->n_layer);
    const uint32_t n_embd = acc->n_head * acc->head_dim;
    int rc = query_terms_check(st, acc, "query_add");
    if (rc) return rc;
    rc = view_check(st, q, n_embd, "query_add");
    if (rc) return rc;
    KVM_HIP(st, hipSetDevice(st->device));
    bool added = false;
    for (uint64_t t0 = 0; t0 < (uint64_t)q->ne2; t0 += KVM_QVIEW_ROWS) {
        qview_args a{};
        a.v = view_of(q);
        a.q_sum = acc->q_sum + (uint64_t)il * n_embd;
        a.q_count = acc->q_count + il;
        a.n_embd = n_embd;
        a.t0 = (uint32_t)t0;
        a.n_rows = (uint32_t)((uint64_t)q->ne2 - t0 < KVM_QVIEW_ROWS ? (uint64_t)q->ne2 - t0 : KVM_QVIEW_ROWS);
        for (uint32_t r = 0; r < a.n_rows; ++r)
            if (!keep || keep[t0 + r]) {
                a.keep[r >> 5] |= 1u << (r & 31);
                ++a.n_kept;
            }
        if (a.n_kept == 0) continue;
        hipLaunchKernelGGL(k_query_add, dim3(kvm_cdiv(n_embd, 256)), dim3(256), 0, st->stream, a);
        KVM_LAUNCH_CHECK(st, "query_add");
        added = true;
    }
    return added ? query_terms_launch(st, acc, il, 1) : KVM_OK;
}

extern "C" int kvm_query_add(kvm_state *st, const kvm_query_acc *acc, uint32_t il,
                             const float *q_rows, uint32_t n_rows) {
    if (!st || !acc || !q_rows) return kvm_fail(st, KVM_EINVAL, "query_add: args");
    const int64_t n_embd = (int64_t)acc->n_head * acc->head_dim;
    const kvm_view v{q_rows, KVM_TYPE_F32, (int64_t)acc->head_dim, (int64_t)acc->n_head, (int64_t)n_rows,
                     4, (size_t)acc->head_dim * 4, (size_t)n_embd * 4};
    return n_rows ? kvm_query_add_view(st, acc, il, &v, nullptr) : KVM_OK;
}

// ---------------------------------------------------------------------------
// Mean-K sums (RawKvStore::write_layer_mean_k / add_mean_f32,
// raw_kv_store.cpp:215-234, 685-705).  Device layout of the index:
// k_sum[il][tile][e][8] with tile = block / 8 (KVM_MEANK_TILE blocks, the
// embedding index e fastest after the block-in-tile): a tile's sums for all
// heads are one contiguous slab, which the scorer streams whole.
// ---------------------------------------------------------------------------
__host__ __device__ inline uint64_t kvm_meank_off(uint32_t n_embd, uint32_t e, uint32_t b) {
    return ((uint64_t)(b / KVM_MEANK_TILE) * n_embd + e) * KVM_MEANK_TILE + b % KVM_MEANK_TILE;
}

extern "C" size_t kvm_meank_k_sum_floats(const kvm_meank_index *ix) {
    if (!ix) return 0;
    const size_t tiles = (ix->n_blocks + KVM_MEANK_TILE - 1) / KVM_MEANK_TILE;
    return (size_t)ix->n_layer * tiles * KVM_MEANK_TILE * ix->n_head_kv * ix->head_dim;
}

// One block's share (chunk ci of the positions pos0 .. pos0+n-1) per
// blockIdx.y; the view's token pos - pos0 + tok0 holds position pos.
__global__ void k_meank_add(float *k_sum, uint32_t *mean_tokens, uint8_t *present, uint32_t cap,
                            uint32_t n_embd, uint32_t bt, uint32_t pos0, uint32_t n, view_args v, uint32_t tok0) {
    const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t ci = blockIdx.y;                  // chunk = one block's share
    const uint32_t bid = pos0 / bt + ci;
    const uint32_t start = ci == 0 ? pos0 : bid * bt;
    const uint32_t end_blk = (bid + 1) * bt;
    const uint32_t end = pos0 + n < end_blk ? pos0 + n : end_blk;
    if (bid >= cap || start >= end) return;
    const uint32_t off = start - bid * bt, take = end - start;
    if (e < n_embd) {
        float *p = k_sum + kvm_meank_off(n_embd, e, bid);
        float s = off == 0 ? 0.0f : *p;
        for (uint32_t t = start; t < end; ++t) s = kvm_fadd(s, view_load(v, t - pos0 + tok0, e));
        *p = s;
    }
    if (e == 0) {
        const uint32_t mt = mean_tokens[bid];
        mean_tokens[bid] = off == 0 ? take : (mt > off + take ? mt : off + take);
        if (present) present[bid] = 1;
    }
}

static int meank_check(kvm_state *st, const kvm_meank_index *ix, uint32_t il, const char *what) {
    if (!st || !ix || !ix->k_sum || !ix->mean_tokens || ix->block_tokens == 0)
        return kvm_fail(st, KVM_EINVAL, "%s: args", what);
    if (il >= ix->n_layer) return kvm_fail(st, KVM_ERANGE, "%s: layer %u", what, il);
    return KVM_OK;
}

static uint64_t meank_layer_floats(const kvm_meank_index *ix) {
    return (uint64_t)kvm_cdiv(ix->n_blocks, KVM_MEANK_TILE) * KVM_MEANK_TILE * ix->n_head_kv * ix->head_dim;
}

// The index's block terms (k_norm) of blocks b0 .. b0 + gridDim.x - 1, kv head
// blockIdx.y, layer il0 + blockIdx.z, one wave each: lane l forms kh of dims
// l, l + 64, ... as the scorer does (k_sum * (1 / mean_tokens), 0 without
// tokens), then lane 0 sums kh^2 over the dims in order from LDS.
template <int D>
__global__ void __launch_bounds__(64) k_meank_terms(const float *k_sum, const uint32_t *mean_tokens, float *k_norm,
                                                    uint64_t layer_floats, uint32_t cap, uint32_t H, uint32_t il0,
                                                    uint32_t b0) {
    const uint32_t b = b0 + blockIdx.x, h = blockIdx.y, il = il0 + blockIdx.z, l = threadIdx.x, n_embd = H * D;
    __shared__ float s_sq[D];
    const uint32_t mt = mean_tokens[(uint64_t)il * cap + b];
    const float inv = kvm_recip_or0((float)mt);
    const uint32_t keep = mt ? 0xffffffffu : 0u;
    const float *ks = k_sum + (uint64_t)il * layer_floats;
    for (uint32_t d = l; d < (uint32_t)D; d += 64u) {
        const float kh = __uint_as_float(__float_as_uint(kvm_fmul(ks[kvm_meank_off(n_embd, h * D + d, b)], inv)) & keep);
        s_sq[d] = kvm_fmul(kh, kh);
    }
    __syncthreads();
    if (l == 0) {
        float nk = 0.0f;
        for (uint32_t d = 0; d < (uint32_t)D; ++d) nk = kvm_fadd(nk, s_sq[d]);
        k_norm[((uint64_t)il * H + h) * cap + b] = nk;
    }
}

// Forms k_norm of layers [il0, il0 + n_lay) and blocks [b0, b1) on the state's stream.
static int meank_terms_launch(kvm_state *st, const kvm_meank_index *ix, uint32_t il0, uint32_t n_lay, uint32_t b0,
                              uint32_t b1) {
    if (!ix->k_norm || n_lay == 0 || b1 <= b0) return KVM_OK;
    const dim3 grid(b1 - b0, ix->n_head_kv, n_lay);
    if (ix->head_dim == 256)
        hipLaunchKernelGGL(k_meank_terms<256>, grid, dim3(64), 0, st->stream, ix->k_sum, ix->mean_tokens, ix->k_norm,
                           meank_layer_floats(ix), ix->n_blocks, ix->n_head_kv, il0, b0);
    else
        hipLaunchKernelGGL(k_meank_terms<128>, grid, dim3(64), 0, st->stream, ix->k_sum, ix->mean_tokens, ix->k_norm,
                           meank_layer_floats(ix), ix->n_blocks, ix->n_head_kv, il0, b0);
    KVM_LAUNCH_CHECK(st, "meank_terms");
    return KVM_OK;
}

static int meank_terms_check(kvm_state *st, const kvm_meank_index *ix, const char *what) {
    if (ix->k_norm && ix->head_dim != 128 && ix->head_dim != 256)
        return kvm_fail(st, KVM_EUNSUPPORTED, "%s: block terms at head_dim %u", what, ix->head_dim);
    return KVM_OK;
}

extern "C" int kvm_meank_refresh(kvm_state *st, const kvm_meank_index *ix) {
    if (!st || !ix || !ix->k_sum || !ix->mean_tokens) return kvm_fail(st, KVM_EINVAL, "meank_refresh: args");
    int rc = meank_terms_check(st, ix, "meank_refresh");
    if (rc) return rc;
    KVM_HIP(st, hipSetDevice(st->device));
    return meank_terms_launch(st, ix, 0, ix->n_layer, 0, ix->n_blocks);
}

// write_layer_mean_k from view tokens tok0 .. tok0+n-1 at positions pos0 ..
static int meank_add_view(kvm_state *st, const kvm_meank_index *ix, uint32_t il, uint32_t pos0, const kvm_view *k,
                          uint32_t tok0, uint32_t n) {
    int rc = meank_check(st, ix, il, "meank_add");
    if (rc) return rc;
    rc = meank_terms_check(st, ix, "meank_add");
    if (rc) return rc;
    const uint32_t n_embd = ix->n_head_kv * ix->head_dim;
    rc = view_check(st, k, n_embd, "meank_add");
    if (rc) return rc;
    if (n == 0) return KVM_OK;
    if ((uint64_t)tok0 + n > (uint64_t)k->ne2) return kvm_fail(st, KVM_ERANGE, "meank_add: tokens past the view");
    const uint32_t bt = ix->block_tokens;
    const uint64_t last = ((uint64_t)pos0 + n - 1) / bt;
    if (last >= ix->n_blocks) return kvm_fail(st, KVM_ERANGE, "meank_add: block %llu >= capacity %u",
                                              (unsigned long long)last, ix->n_blocks);
    KVM_HIP(st, hipSetDevice(st->device));
    const uint32_t n_chunks = (uint32_t)(last - pos0 / bt + 1);
    hipLaunchKernelGGL(k_meank_add, dim3(kvm_cdiv(n_embd, 256), n_chunks), dim3(256), 0, st->stream,
                       ix->k_sum + (uint64_t)il * meank_layer_floats(ix),
                       ix->mean_tokens + (uint64_t)il * ix->n_blocks, ix->present, ix->n_blocks, n_embd,
                       bt, pos0, n, view_of(k), tok0);
    KVM_LAUNCH_CHECK(st, "meank_add");
    return meank_terms_launch(st, ix, il, 1, pos0 / bt, (uint32_t)last + 1);
}

extern "C" int kvm_meank_add_view(kvm_state *st, const kvm_meank_index *ix, uint32_t il, uint32_t pos0,
                                  const kvm_view *k) {
    if (!k) return kvm_fail(st, KVM_EINVAL, "meank_add: null view");
    return meank_add_view(st, ix, il, pos0, k, 0, k->ne2 > 0 ? (uint32_t)k->ne2 : 0u);
}

extern "C" int kvm_meank_add(kvm_state *st, const kvm_meank_index *ix, uint32_t il, uint32_t pos0,
                             uint32_t n, const float *k_rows) {
    if (!ix || !k_rows) return kvm_fail(st, KVM_EINVAL, "meank_add: args");
    const int64_t n_embd = (int64_t)ix->n_head_kv * ix->head_dim;
    const kvm_view v{k_rows, KVM_TYPE_F32, (int64_t)ix->head_dim, (int64_t)ix->n_head_kv, (int64_t)n,
                     4, (size_t)ix->head_dim * 4, (size_t)n_embd * 4};
    return meank_add_view(st, ix, il, pos0, &v, 0, n);
}

// ---------------------------------------------------------------------------
// Decode running sum (kvmem_meank_zero / _add, llama-kvmem-stagein.cu:
// 1066-1097; meank_add_* 270-320) and its flush into the index
// (RawKvStore::write_layer_mean_sum, raw_kv_store.cpp:707-731, as
// decode_mean_flush applies it, llama-memory-kvmem.cpp:3939-3993).
// ---------------------------------------------------------------------------
__global__ void k_meank_acc_add(float *acc, uint32_t n_embd, view_args v, uint32_t tok0, uint32_t n_keep) {
    const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_embd) return;
    float s = acc[e];
    for (uint32_t t = 0; t < n_keep; ++t) s = kvm_fadd(s, view_load(v, tok0 + t, e));
    acc[e] = s;
}

// k_sum of block pos0 / bt: zeroed when the range starts the block, then
// += acc[e]; mean_tokens as write_layer_mean_sum sets it.
__global__ void k_meank_acc_flush(float *k_sum, uint32_t *mean_tokens, uint8_t *present, const float *acc,
                                  uint32_t n_embd, uint32_t bid, uint32_t off, uint32_t take) {
    const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e < n_embd) {
        float *p = k_sum + kvm_meank_off(n_embd, e, bid);
        *p = kvm_fadd(off == 0 ? 0.0f : *p, acc[e]);
    }
    if (e == 0) {
        const uint32_t mt = mean_tokens[bid];
        mean_tokens[bid] = off == 0 ? take : (mt > off + take ? mt : off + take);
        if (present) present[bid] = 1;
    }
}

extern "C" int kvm_meank_acc_zero(kvm_state *st, const kvm_meank_index *ix, uint32_t il) {
    int rc = meank_check(st, ix, il, "meank_acc_zero");
    if (rc) return rc;
    if (!ix->acc) return kvm_fail(st, KVM_EINVAL, "meank_acc_zero: index without a running sum");
    const uint32_t n_embd = ix->n_head_kv * ix->head_dim;
    KVM_HIP(st, hipSetDevice(st->device));
    hipLaunchKernelGGL(k_zero_f32, dim3(kvm_cdiv(n_embd, 256)), dim3(256), 0, st->stream,
                       ix->acc + (uint64_t)il * n_embd, (uint64_t)n_embd);
    KVM_LAUNCH_CHECK(st, "meank_acc_zero");
    return KVM_OK;
}

extern "C" int kvm_meank_acc_add(kvm_state *st, const kvm_meank_index *ix, uint32_t il, const kvm_view *k,
                                 uint32_t tok0, uint32_t n_keep) {
    int rc = meank_check(st, ix, il, "meank_acc_add");
    if (rc) return rc;
    if (!ix->acc) return kvm_fail(st, KVM_EINVAL, "meank_acc_add: index without a running sum");
    const uint32_t n_embd = ix->n_head_kv * ix->head_dim;
    rc = view_check(st, k, n_embd, "meank_acc_add");
    if (rc) return rc;
    if (n_keep == 0) return KVM_OK;
    if ((uint64_t)tok0 + n_keep > (uint64_t)k->ne2) return kvm_fail(st, KVM_ERANGE, "meank_acc_add: tokens past the view");
    KVM_HIP(st, hipSetDevice(st->device));
    hipLaunchKernelGGL(k_meank_acc_add, dim3(kvm_cdiv(n_embd, 256)), dim3(256), 0, st->stream,
                       ix->acc + (uint64_t)il * n_embd, n_embd, view_of(k), tok0, n_keep);
    KVM_LAUNCH_CHECK(st, "meank_acc_add");
    return KVM_OK;
}

extern "C" int kvm_meank_acc_flush(kvm_state *st, const kvm_meank_index *ix, uint32_t il, uint32_t pos0,
                                   uint32_t n) {
    int rc = meank_check(st, ix, il, "meank_acc_flush");
    if (rc) return rc;
    if (!ix->acc) return kvm_fail(st, KVM_EINVAL, "meank_acc_flush: index without a running sum");
    rc = meank_terms_check(st, ix, "meank_acc_flush");
    if (rc) return rc;
    if (n == 0) return KVM_OK;
    const uint32_t bt = ix->block_tokens, bid = pos0 / bt, off = pos0 % bt;
    const uint32_t take = n < bt - off ? n : bt - off;
    if (bid >= ix->n_blocks) return kvm_fail(st, KVM_ERANGE, "meank_acc_flush: block %u >= capacity %u", bid, ix->n_blocks);
    const uint32_t n_embd = ix->n_head_kv * ix->head_dim;
    KVM_HIP(st, hipSetDevice(st->device));
    hipLaunchKernelGGL(k_meank_acc_flush, dim3(kvm_cdiv(n_embd, 256)), dim3(256), 0, st->stream,
                       ix->k_sum + (uint64_t)il * meank_layer_floats(ix),
                       ix->mean_tokens + (uint64_t)il * ix->n_blocks, ix->present,
                       ix->acc + (uint64_t)il * n_embd, n_embd, bid, off, take);
    KVM_LAUNCH_CHECK(st, "meank_acc_flush");
    return meank_terms_launch(st, ix, il, 1, bid, bid + 1);
}

// ---------------------------------------------------------------------------
// Scoring (kvm_score_dev.h).  Workgroup = (8-block tile, layer, lane), four
// waves, one kv head per wave (heads w, w + 4, ... for more than four): the
// wave's reads (the head's 8 KB slab of the tile, its query group's rows, the
// token counts) are issued first, then every lane forms the products of its 4
// dims and 17 lanes sum one product row each in the reference's order (dot of
// blocks 0-7, their nk, and nq), without a workgroup barrier; one barrier
// before wave 0 sums each block's cosines over the heads in double in head
// order and writes the layer's contribution layer / H to [layer][block],
// which the top-k averages over layers.
// ---------------------------------------------------------------------------
// Independent retrievals (conversation lanes) in one launch: lane = blockIdx.z.
struct score_lanes {
    score_args lane[KVM_RET_LANES];
};

template <int D, bool QV, int LAY>
__global__ void __launch_bounds__(256) k_score(score_lanes sl) {
    // one copy of the lane's arguments: its scalar loads are issued together
    // ahead of the first branch, not one round trip per field
    const score_args a = sl.lane[blockIdx.z];
    if constexpr (QV) asm volatile("" ::"s"(a.q_vec), "s"(a.q_norm), "s"(a.q_count), "s"(a.k_sum), "s"(a.mean_tokens));
    else asm volatile("" ::"s"(a.q_sum), "s"(a.q_count), "s"(a.k_sum), "s"(a.mean_tokens));
    if constexpr (LAY == KVM_SL_NK) asm volatile("" ::"s"(a.k_norm));
    const uint32_t tile = blockIdx.x, il = blockIdx.y;
    if (tile >= a.n_tiles_used || il >= a.n_layer) return;
    __shared__ __align__(16) score_wg_lds<D, 4, LAY> L;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t g = a.g, qc = a.q_count[il];
    score_regs r;
    if ((uint32_t)w < a.H) score_tile_load<D, QV, LAY>(a, il, tile, (uint32_t)w, g, r);
    if (qc == 0) return;                 // a layer without queries: skipped by the reduction
    for (uint32_t hh = (uint32_t)w; hh < a.H; hh += 4u) {
        if (hh != (uint32_t)w) score_tile_load<D, QV, LAY>(a, il, tile, hh, g, r);
        score_tile_compute<D, QV, LAY>(a, il, hh, qc, g, r, L.w[w], L.cos[hh]);
    }
    __syncthreads();
    if (w == 0) score_tile_store(a, il, tile, L.cos);
}

// ---------------------------------------------------------------------------
// Top-k + layout (kvm_topk_dev.h): one workgroup of 1,024 threads per lane, up
// to KVM_MAX_TOPK_BLOCKS blocks and the first 2,048 slots of the slot map in LDS.
// ---------------------------------------------------------------------------
#define KVM_TOPK_THREADS 1024
typedef topk_lds<KVM_TOPK_THREADS, KVM_MAX_TOPK_BLOCKS, 2048> topk_lds_1k;
__global__ void __launch_bounds__(KVM_TOPK_THREADS) k_topk(topk_lanes tl) {
    const topk_args a = tl.lane[blockIdx.x];     // one copy out of the argument segment
    __shared__ topk_lds_1k T;
    topk_body(a, T);
}

static int make_topk(kvm_state *st, const double *scores, const double *layer_score,
                     const kvm_meank_index *ix, const kvm_query_acc *q, const kvm_select_params *p,
                     const kvm_window *w, const kvm_selection *out, topk_args *ta) {
    if (w && (kvm_window_check(w) || !w->slot_block || !w->slot_base))
        return kvm_fail(st, KVM_EINVAL, "topk: bad window or window without slot map");
    const uint32_t *ntok = p->n_tokens;
    if (p->n_blocks == 0) {
        // The kernel's first phase loads element 0 of the score and token-count
        // arrays unconditionally (its values are unused when there is no block);
        // a selection over no blocks may pass NULL or empty arrays, so those
        // loads read the state's workspace instead.
        void *z = kvm_workspace(st, 64);
        if (!z) return kvm_fail(st, KVM_ENOMEM, "topk: workspace");
        scores = (const double *)z;
        layer_score = nullptr;
        ntok = (const uint32_t *)z;
        ix = nullptr;
    }
    *ta = topk_args{scores, layer_score, q ? q->q_count : nullptr, ix ? ix->present : nullptr, out->scores,
                    ntok, p->mandatory,
                    w ? w->slot_block : nullptr, w ? w->slot_base : nullptr,
                    out->ids, out->to_base, out->stage_slots, out->info,
                    p->n_blocks, p->budget_blocks, p->sink_blocks, p->recent_blocks, p->n_mandatory,
                    w ? w->n_cells / w->block_tokens : 0u, out->cap,
                    ix ? ix->n_layer : 0u, ix ? ix->n_blocks : 0u,
                    w ? w->shadow_rows : nullptr, w ? out->stage_src : nullptr, w ? w->block_tokens : 0u,
                    w ? w->pending_rows : nullptr, w ? out->stage_out : nullptr};
    return KVM_OK;
}

int kvm_topk_launch(kvm_state *st, const topk_lanes &tl, uint32_t n_lanes) {
    hipLaunchKernelGGL(k_topk, dim3(n_lanes), dim3(KVM_TOPK_THREADS), 0, st->stream, tl);
    KVM_LAUNCH_CHECK(st, "topk");
    return KVM_OK;
}

static int check_select(kvm_state *st, const kvm_select_params *p, const kvm_selection *out) {
    if (!p || !out) return kvm_fail(st, KVM_EINVAL, "select: null argument");
    if ((p->n_blocks && !p->n_tokens) || !out->ids || !out->to_base || !out->stage_slots || !out->info)
        return kvm_fail(st, KVM_EINVAL, "select: null buffer");
    if (p->n_blocks > KVM_MAX_TOPK_BLOCKS) return kvm_fail(st, KVM_ERANGE, "select: n_blocks %u > %u", p->n_blocks, KVM_MAX_TOPK_BLOCKS);
    const uint32_t want = p->budget_blocks == 0 || p->n_blocks <= p->budget_blocks ? p->n_blocks : p->budget_blocks;
    if (want > out->cap) return kvm_fail(st, KVM_ERANGE, "select: selection capacity %u < %u", out->cap, want);
    if (p->n_mandatory && !p->mandatory) return kvm_fail(st, KVM_EINVAL, "select: mandatory list missing");
    return KVM_OK;
}

int kvm_select_prepare(kvm_state *st, const double *scores, const kvm_select_params *p, const kvm_window *w,
                       const kvm_selection *out, topk_args *ta) {
    if (!st) return KVM_EINVAL;
    int rc = check_select(st, p, out);
    if (rc) return rc;
    if (p->n_blocks && !scores) return kvm_fail(st, KVM_EINVAL, "select_topk: null scores");
    KVM_HIP(st, hipSetDevice(st->device));
    return make_topk(st, scores, nullptr, nullptr, nullptr, p, w, out, ta);
}

extern "C" int kvm_select_topk(kvm_state *st, const double *scores, const kvm_select_params *p,
                               const kvm_window *w, const kvm_selection *out) {
    topk_lanes tl{};
    const int rc = kvm_select_prepare(st, scores, p, w, out, &tl.lane[0]);
    if (rc) return rc;
    return kvm_topk_launch(st, tl, 1);
}

static int check_score(kvm_state *st, const kvm_retrieval_lane &r, uint32_t i) {
    const kvm_meank_index *ix = r.ix;
    const kvm_query_acc *q = r.q;
    const kvm_select_params *p = r.p;
    if (!ix || !q) return kvm_fail(st, KVM_EINVAL, "score_topk: lane %u: null argument", i);
    int rc = check_select(st, p, r.out);
    if (rc) return rc;
    if (!ix->k_sum || !ix->mean_tokens || !q->q_sum || !q->q_count || !r.out->scores)
        return kvm_fail(st, KVM_EINVAL, "score_topk: lane %u: null buffer", i);
    if (p->n_blocks > ix->n_blocks) return kvm_fail(st, KVM_ERANGE, "score_topk: n_blocks %u > index capacity %u", p->n_blocks, ix->n_blocks);
    if (q->n_layer != ix->n_layer || q->head_dim != ix->head_dim) return kvm_fail(st, KVM_EINVAL, "score_topk: query/index shape mismatch");
    if (ix->head_dim != 128 && ix->head_dim != 256) return kvm_fail(st, KVM_EUNSUPPORTED, "score_topk: head_dim %u", ix->head_dim);
    if (ix->n_head_kv == 0 || ix->n_head_kv > KVM_SCORE_HMAX || q->n_head % ix->n_head_kv ||
        q->n_head / ix->n_head_kv > KVM_SCORE_GMAX)
        return kvm_fail(st, KVM_EUNSUPPORTED, "score_topk: n_head %u / n_head_kv %u (at most %d kv heads, groups of at most %d)",
                        q->n_head, ix->n_head_kv, KVM_SCORE_HMAX, KVM_SCORE_GMAX);
    if (q->q_vec && (!q->q_norm || q->n_head_kv != ix->n_head_kv))
        return kvm_fail(st, KVM_EINVAL, "score_topk: lane %u: query terms for %u kv heads, index has %u", i,
                        q->n_head_kv, ix->n_head_kv);
    return KVM_OK;
}

// Checks every lane's retrieval and fills its top-k arguments; the lanes'
// per-layer score contributions go to the state's workspace.  Nothing is
// launched.
int kvm_retrieval_prepare(kvm_state *st, const kvm_retrieval_lane *lanes, uint32_t n_lanes, topk_lanes *tl) {
    if (!st) return KVM_EINVAL;
    if (!lanes || n_lanes == 0) return kvm_fail(st, KVM_EINVAL, "score_topk: no lanes");
    if (n_lanes > KVM_RET_LANES) return kvm_fail(st, KVM_ERANGE, "score_topk: %u lanes > %d", n_lanes, KVM_RET_LANES);
    size_t ls_total = 0;
    for (uint32_t i = 0; i < n_lanes; ++i) {
        int rc = check_score(st, lanes[i], i);
        if (rc) return rc;
        if (lanes[i].ix->head_dim != lanes[0].ix->head_dim)
            return kvm_fail(st, KVM_EINVAL, "score_topk: lanes differ in head_dim");
        ls_total += (size_t)lanes[i].ix->n_layer * lanes[i].ix->n_blocks;
    }
    KVM_HIP(st, hipSetDevice(st->device));
    // (at least 64 bytes: a lane without blocks reads 64 bytes of it, see make_topk)
    double *ls = (double *)kvm_workspace(st, ls_total * sizeof(double) + 64);
    if (!ls) return kvm_fail(st, KVM_ENOMEM, "score_topk: workspace");
    *tl = topk_lanes{};
    size_t off = 0;
    for (uint32_t i = 0; i < n_lanes; ++i) {
        const kvm_retrieval_lane &r = lanes[i];
        const kvm_meank_index *ix = r.ix;
        // a lane without blocks reduces nothing: top-k reads its own (empty) score array
        int rc = r.p->n_blocks ? make_topk(st, nullptr, ls + off, ix, r.q, r.p, r.w, r.out, &tl->lane[i])
                               : make_topk(st, r.out->scores, nullptr, nullptr, nullptr, r.p, r.w, r.out, &tl->lane[i]);
        if (rc) return rc;
        off += (size_t)ix->n_layer * ix->n_blocks;
    }
    return KVM_OK;
}

// The scoring grid of prepared lanes: every lane's layer contributions into
// the buffer its top-k arguments read.
void kvm_retrieval_score_args(const kvm_retrieval_lane *lanes, uint32_t n_lanes, const topk_lanes &tl,
                              score_args *out) {
    for (uint32_t i = 0; i < n_lanes; ++i) {
        const kvm_retrieval_lane &r = lanes[i];
        const kvm_meank_index *ix = r.ix;
        const uint32_t used = r.p->n_blocks ? kvm_cdiv(r.p->n_blocks, KVM_MEANK_TILE) : 0u;
        out[i] = score_args{r.q->q_sum, r.q->q_count, ix->k_sum, ix->mean_tokens, (double *)tl.lane[i].layer_score,
                            r.p->n_blocks, ix->n_blocks, kvm_cdiv(ix->n_blocks, KVM_MEANK_TILE), ix->n_layer,
                            r.q->n_head, ix->n_head_kv, used, r.q->n_head / ix->n_head_kv, r.q->q_vec, r.q->q_norm,
                            ix->k_norm};
    }
}

int kvm_retrieval_score(kvm_state *st, const kvm_retrieval_lane *lanes, uint32_t n_lanes, const topk_lanes &tl) {
    score_lanes sl{};
    kvm_retrieval_score_args(lanes, n_lanes, tl, sl.lane);
    uint32_t max_tiles = 0, max_layer = 0;
    for (uint32_t i = 0; i < n_lanes; ++i) {
        max_tiles = sl.lane[i].n_tiles_used > max_tiles ? sl.lane[i].n_tiles_used : max_tiles;
        max_layer = sl.lane[i].n_layer > max_layer ? sl.lane[i].n_layer : max_layer;
    }
    if (max_tiles == 0) return KVM_OK;
    // the accumulators' formed query terms when every lane has them, the
    // indexes' block terms likewise
    bool qv = true, nk = true;
    for (uint32_t i = 0; i < n_lanes; ++i) {
        qv = qv && sl.lane[i].q_vec;
        nk = nk && sl.lane[i].k_norm;
    }
    KVM_HIP(st, hipSetDevice(st->device));
    const dim3 grid(max_tiles, max_layer, n_lanes), block(256);
    // product rows in LDS (the shorter chains) while the grid fits the CUs at
    // once with them; past that the chains form their products (half the LDS,
    // twice the workgroups per CU)
    const uint64_t n_wg = (uint64_t)max_tiles * max_layer * n_lanes;
    const bool wide = lanes[0].ix->head_dim == 256;
    const size_t lds_rows = wide ? sizeof(score_wg_lds<256, 4, KVM_SL_ROWS>) : sizeof(score_wg_lds<128, 4, KVM_SL_ROWS>);
    const int lay = nk ? KVM_SL_NK : n_wg > (uint64_t)st->n_cu * (KVM_LDS_PER_CU / lds_rows) ? KVM_SL_OTF : KVM_SL_ROWS;
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, block, 0, st->stream, sl); };
    auto pick = [&](auto d, auto q) {
        constexpr int DD = decltype(d)::value;
        constexpr bool QQ = decltype(q)::value;
        if (lay == KVM_SL_NK) go(k_score<DD, QQ, KVM_SL_NK>);
        else if (lay == KVM_SL_OTF) go(k_score<DD, QQ, KVM_SL_OTF>);
        else go(k_score<DD, QQ, KVM_SL_ROWS>);
    };
    if (wide) {
        if (qv) pick(std::integral_constant<int, 256>{}, std::true_type{});
        else pick(std::integral_constant<int, 256>{}, std::false_type{});
    } else {
        if (qv) pick(std::integral_constant<int, 128>{}, std::true_type{});
        else pick(std::integral_constant<int, 128>{}, std::false_type{});
    }
    KVM_LAUNCH_CHECK(st, "score");
    return KVM_OK;
}

// Scoring grid + top-k for every lane.
static int score_topk_impl(kvm_state *st, const kvm_retrieval_lane *lanes, uint32_t n_lanes) {
    topk_lanes tl;
    int rc = kvm_retrieval_prepare(st, lanes, n_lanes, &tl);
    if (rc) return rc;
    rc = kvm_retrieval_score(st, lanes, n_lanes, tl);
    if (rc) return rc;
    return kvm_topk_launch(st, tl, n_lanes);
}

extern "C" int kvm_score_topk_lanes(kvm_state *st, const kvm_retrieval_lane *lanes, uint32_t n_lanes) {
    return score_topk_impl(st, lanes, n_lanes);
}

extern "C" int kvm_score_topk_stagein_lanes(kvm_state *st, const kvm_retrieval_lane *lanes,
                                            const kvm_history *const *hist, uint32_t n_lanes,
                                            const kvm_rope_params *rope) {
    if (!st) return KVM_EINVAL;
    if (!lanes || !hist || n_lanes == 0) return kvm_fail(st, KVM_EINVAL, "score_topk_stagein: no lanes");
    if (n_lanes > KVM_RET_LANES) return kvm_fail(st, KVM_ERANGE, "score_topk_stagein: %u lanes > %d", n_lanes, KVM_RET_LANES);
    kvm_stagein_lane sg[KVM_RET_LANES];
    for (uint32_t i = 0; i < n_lanes; ++i) sg[i] = kvm_stagein_lane{hist[i], lanes[i].w, lanes[i].out};
    // the stage-in arguments are checked before anything is launched
    stage_lanes stl;
    uint32_t max_items = 0;
    size_t lds = 0;
    int rc = kvm_stage_prepare(st, sg, n_lanes, rope, &stl, &max_items, &lds);
    if (rc) return rc;
    rc = score_topk_impl(st, lanes, n_lanes);
    if (rc) return rc;
    return kvm_stage_launch(st, stl, n_lanes, max_items, lds, lanes[0].w->head_dim);
}

extern "C" int kvm_score_topk_stagein(kvm_state *st, const kvm_meank_index *ix, const kvm_query_acc *q,
                                      const kvm_select_params *p, const kvm_window *w,
                                      const kvm_selection *out, const kvm_history *h,
                                      const kvm_rope_params *rope) {
    const kvm_retrieval_lane lane{ix, q, p, w, out};
    return kvm_score_topk_stagein_lanes(st, &lane, &h, 1, rope);
}

extern "C" int kvm_score_topk(kvm_state *st, const kvm_meank_index *ix, const kvm_query_acc *q,
                              const kvm_select_params *p, const kvm_window *w,
                              const kvm_selection *out) {
    const kvm_retrieval_lane lane{ix, q, p, w, out};
    return kvm_score_topk_lanes(st, &lane, 1);
}
