// kvm_retrieval.hip -- capture-side index upkeep (query accumulator, mean-K sums)
// and the retrieval step: score_retrieval + top-k + chronological window layout.
//
// Bit-exactness: the scorer restates llama-memory-kvmem.cpp:4149-4196 with the
// same fp32 operation order, each operation one IEEE rounding (this file is
// compiled with -ffp-contract=off and correctly rounded `/` and sqrtf), and the
// per-head/per-layer accumulation in double in the same order.
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

extern "C" int kvm_query_add_view(kvm_state *st, const kvm_query_acc *acc, uint32_t il, const kvm_view *q,
                                  const uint8_t *keep) {
    if (!st || !acc || !acc->q_sum || !acc->q_count) return kvm_fail(st, KVM_EINVAL, "query_add: args");
    if (il >= acc->n_layer) return kvm_fail(st, KVM_ERANGE, "query_add: layer %u >= %u", il, acc->n_layer);
    const uint32_t n_embd = acc->n_head * acc->head_dim;
    int rc = view_check(st, q, n_embd, "query_add");
    if (rc) return rc;
    KVM_HIP(st, hipSetDevice(st->device));
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
    }
    return KVM_OK;
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
#define KVM_MEANK_TILE 8u

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

// write_layer_mean_k from view tokens tok0 .. tok0+n-1 at positions pos0 ..
static int meank_add_view(kvm_state *st, const kvm_meank_index *ix, uint32_t il, uint32_t pos0, const kvm_view *k,
                          uint32_t tok0, uint32_t n) {
    int rc = meank_check(st, ix, il, "meank_add");
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
    return KVM_OK;
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
    return KVM_OK;
}

// ---------------------------------------------------------------------------
// Scoring.  Workgroup = (8-block tile t, layer il), four waves; chain lane
// (hh, bi) = 8*hh + bi owns block 8t + bi under head 8c + hh of head chunk c
// (up to 8 heads per chunk).  Per chunk:
//   1. the tile's slab of mean-K sums (8 blocks x the chunk's heads x D,
//      contiguous) is loaded in one round trip, turned into
//      kh = k_sum * (1/mean_tokens) (+0.0 for a block without tokens, the
//      reference's zeroed mean) and written to LDS as [dim][lane], while each
//      wave builds qv = qh * invq of two of the chunk's heads;
//   2. wave 0 runs the sequential fp32 dot chains, wave 1 the nk chains and
//      wave 2 the block-independent nq chains (lane hh), in the reference's
//      operation order;
//   3. wave 0 forms the cosines.
// Lanes bi of wave 0 then sum each block's cosines over the heads in double
// in head order and write the layer's contribution layer/H to a workspace
// [layer][block] that the top-k kernel averages over layers.
// ---------------------------------------------------------------------------
struct score_args {
    const float *q_sum;
    const uint32_t *q_count;
    const float *k_sum;
    const uint32_t *mean_tokens;
    double *layer_score;    // [n_layer][cap]
    uint32_t n_blocks, cap, n_tiles, n_layer, n_head, H;
    uint32_t n_tiles_used;  // tiles holding the first n_blocks blocks
};

#define KVM_SCORE_GMAX 16   // largest query group (n_head / n_head_kv)
#define KVM_SCORE_HMAX 16   // largest n_head_kv

// One head chunk of NT consecutive tiles (HC = 8 / NT heads, so NT tiles x HC
// heads x 8 blocks = 64 (tile, head, block) rows): the chunk's slabs (every
// load issued first) go into LDS as kh, row (t HC + head) 8 + block, then one
// wave per chain (dot, nk, nq) walks the dims in order.  UPB = 16-byte slab
// units per thread and 32-dim batch (1 for a single tile of <= 4 heads).
template <int D, int UPB, int NT>
__device__ __forceinline__ void score_chunk(const score_args &a, uint32_t il, uint32_t tile0, uint32_t c,
                                            uint32_t nh, uint32_t g, uint32_t qc, float (*s_k)[D + 4],
                                            float (*s_qv)[D + 4], float *s_nq, float *s_nk,
                                            float (*s_cos)[KVM_MEANK_TILE * 8], float *dot_out) {
    constexpr uint32_t TW = KVM_MEANK_TILE, HC = 8 / NT, NBAT = D / 32;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t HD = a.H * D;
    // ---- all loads first: query gathers, token counts, slab batches.  Query
    // item u = tid + 256x is (head u / (D/4), dims 4(u % (D/4)) .. +3); its
    // group's rows come in 16 bytes at a time.
    constexpr uint32_t NQI = (HC * (D / 4) + 255) / 256;
    kvm_f32x4 qg[NQI][8];
#pragma unroll
    for (uint32_t x = 0; x < NQI; ++x) {
        const uint32_t u = tid + 256u * x, hl = u / (D / 4), d4 = u % (D / 4);
        const uint32_t h = c * HC + (hl < nh ? hl : 0u);
#pragma unroll
        for (int gi = 0; gi < 8; ++gi) {
            const uint32_t gc = (uint32_t)gi < g ? (uint32_t)gi : 0u;
            qg[x][gi] = *(const kvm_f32x4 *)&a.q_sum[((uint64_t)il * a.n_head + h * g + gc) * D + 4 * d4];
        }
    }
    const uint32_t quad = tid % (TW / 4);
    // unit tid + 256x of batch k: hu = unit/64 = (tile t, head) = (hu / HC, hu % HC)
    // (wave-uniform), dim 32k + (unit%64)/2, blocks 4 quad .. +3
    const kvm_f32x4 *slab[UPB];
    uint32_t mt4[UPB][4];
    bool unit_live[UPB];
#pragma unroll
    for (int x = 0; x < UPB; ++x) {
        const uint32_t hu = (tid >> 6) + 4u * x, t = hu / HC, head = hu % HC;
        const uint32_t tile = tile0 + t < a.n_tiles_used ? tile0 + t : a.n_tiles_used - 1;
        unit_live[x] = head < nh;
        slab[x] = (const kvm_f32x4 *)(a.k_sum + (((uint64_t)il * a.n_tiles + tile) * HD +
                                                 ((uint64_t)c * HC + (head < nh ? head : 0u)) * D) * TW);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t b = tile * TW + 4 * quad + j;
            mt4[x][j] = a.mean_tokens[(uint64_t)il * a.cap + (b < a.n_blocks ? b : a.n_blocks - 1)];
        }
    }
    kvm_f32x4 kv[NBAT][UPB];
#pragma unroll
    for (uint32_t k = 0; k < NBAT; ++k)
#pragma unroll
        for (int x = 0; x < UPB; ++x) {
            const uint32_t r = (tid % 64) / 2;
            kv[k][x] = __builtin_nontemporal_load(slab[x] + (32 * k + r) * (TW / 4) + quad);
        }
    if (qc == 0) return;                 // layer without queries: skipped by the reduction
    // ---- qv of the chunk's heads (the group's q rows summed in order, scaled)
    const float invq = kvm_fdiv(1.0f, (float)(qc * (g > 1u ? g : 1u)));
#pragma unroll
    for (uint32_t x = 0; x < NQI; ++x) {
        const uint32_t u = tid + 256u * x, hl = u / (D / 4), d4 = u % (D / 4);
        if (hl < nh) {
            const uint32_t h = c * HC + hl;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float qh = 0.0f;
#pragma unroll
                for (int gi = 0; gi < 8; ++gi)
                    if ((uint32_t)gi < g) qh = kvm_fadd(qh, qg[x][gi][e]);
                for (uint32_t g0 = 8; g0 < g; ++g0)              // groups above 8 (rare)
                    qh = kvm_fadd(qh, a.q_sum[((uint64_t)il * a.n_head + h * g + g0) * D + 4 * d4 + e]);
                s_qv[hl][4 * d4 + e] = kvm_fmul(qh, invq);
            }
        }
    }
    float inv4[UPB][4];
    uint32_t keep4[UPB][4];
#pragma unroll
    for (int x = 0; x < UPB; ++x)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            inv4[x][j] = mt4[x][j] ? kvm_fdiv(1.0f, (float)mt4[x][j]) : 0.0f;
            keep4[x][j] = mt4[x][j] ? 0xffffffffu : 0u;
        }
    // ---- kh for all dims into LDS (one barrier), then the chains run straight
    // through the D dims in the reference's order
    const uint32_t hh = (lane / TW) % HC, tl = lane / (TW * HC);   // the chain's head and tile
    const float *qrow = s_qv[hh < nh ? hh : 0u];
    const float *nqrow = s_qv[lane < nh ? lane : 0u];
    float chain = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < NBAT; ++k) {
#pragma unroll
        for (int x = 0; x < UPB; ++x) {
            const uint32_t u = tid + 256u * x, hu = u / 64, r = (u % 64) / 2;
            if (unit_live[x]) {
                float4 kh;
                kh.x = __uint_as_float(__float_as_uint(kvm_fmul(kv[k][x][0], inv4[x][0])) & keep4[x][0]);
                kh.y = __uint_as_float(__float_as_uint(kvm_fmul(kv[k][x][1], inv4[x][1])) & keep4[x][1]);
                kh.z = __uint_as_float(__float_as_uint(kvm_fmul(kv[k][x][2], inv4[x][2])) & keep4[x][2]);
                kh.w = __uint_as_float(__float_as_uint(kvm_fmul(kv[k][x][3], inv4[x][3])) & keep4[x][3]);
                float *col = &s_k[hu * TW + 4 * quad][32 * k + r];
                col[0] = kh.x;
                col[D + 4] = kh.y;
                col[2 * (D + 4)] = kh.z;
                col[3 * (D + 4)] = kh.w;
            }
        }
    }
    KVM_LDS_BARRIER();
    // Each chain reads 32 dims ahead (16-byte LDS reads into a second register
    // buffer, kept ahead of the arithmetic by a scheduling barrier), so the
    // dependent adds never wait on LDS.
    const float *krow = s_k[lane];
    constexpr int CH = 8;                // float4 per 32-dim chunk
    auto chain_over = [&](auto &&ld, auto &&step) {
        float4 buf[2][2][CH];
        ld(buf[0], 0);
#pragma unroll
        for (int c = 0; c < D / (4 * CH); ++c) {
            if (c + 1 < D / (4 * CH)) ld(buf[(c + 1) & 1], c + 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < CH; ++j) step(buf[c & 1][0][j], buf[c & 1][1][j]);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    if (w == 0) {
        chain_over([&](float4 (&b)[2][CH], int c) {
#pragma unroll
                       for (int j = 0; j < CH; ++j) {
                           b[0][j] = *(const float4 *)&qrow[4 * (CH * c + j)];
                           b[1][j] = *(const float4 *)&krow[4 * (CH * c + j)];
                       }
                   },
                   [&](const float4 &q4, const float4 &k4) {
                       chain = kvm_fadd(chain, kvm_fmul(q4.x, k4.x));
                       chain = kvm_fadd(chain, kvm_fmul(q4.y, k4.y));
                       chain = kvm_fadd(chain, kvm_fmul(q4.z, k4.z));
                       chain = kvm_fadd(chain, kvm_fmul(q4.w, k4.w));
                   });
    } else if (w == 1) {
        chain_over([&](float4 (&b)[2][CH], int c) {
#pragma unroll
                       for (int j = 0; j < CH; ++j) b[1][j] = *(const float4 *)&krow[4 * (CH * c + j)];
                   },
                   [&](const float4 &, const float4 &k4) {
                       chain = kvm_fadd(chain, kvm_fmul(k4.x, k4.x));
                       chain = kvm_fadd(chain, kvm_fmul(k4.y, k4.y));
                       chain = kvm_fadd(chain, kvm_fmul(k4.z, k4.z));
                       chain = kvm_fadd(chain, kvm_fmul(k4.w, k4.w));
                   });
    } else if (w == 2) {
        chain_over([&](float4 (&b)[2][CH], int c) {
#pragma unroll
                       for (int j = 0; j < CH; ++j) b[0][j] = *(const float4 *)&nqrow[4 * (CH * c + j)];
                   },
                   [&](const float4 &q4, const float4 &) {
                       chain = kvm_fadd(chain, kvm_fmul(q4.x, q4.x));
                       chain = kvm_fadd(chain, kvm_fmul(q4.y, q4.y));
                       chain = kvm_fadd(chain, kvm_fmul(q4.z, q4.z));
                       chain = kvm_fadd(chain, kvm_fmul(q4.w, q4.w));
                   });
    }
    if (w == 1) s_nk[lane] = chain;
    if (w == 2 && lane < nh) s_nq[lane] = chain;
    KVM_LDS_BARRIER();
    // ---- cosines of the chunk
    const uint32_t bi = lane % TW, b = (tile0 + tl) * TW + bi;
    if (w == 0 && hh < nh && b < a.n_blocks) {
        const float den = kvm_fadd(kvm_fmul(kvm_fsqrt(s_nq[hh]), kvm_fsqrt(s_nk[lane])), 1e-6f);
        s_cos[c * HC + hh][tl * TW + bi] = kvm_fdiv(chain, den);
    }
    *dot_out = chain;
    KVM_LDS_BARRIER();                   // chunk c's LDS reads done before chunk c+1 writes
}

// Independent retrievals (conversation lanes) in one launch: lane = blockIdx.z.
struct score_lanes {
    score_args lane[KVM_RET_LANES];
};

// Workgroup = NT consecutive tiles of one layer: NT = 8 / HC tiles for head
// chunks of HC heads, so that a chunk fills the 64 chain lanes (NT = 2 at 4 kv
// heads: 16 blocks per workgroup).
template <int D, int NT>
__global__ void __launch_bounds__(256) k_score(score_lanes sl) {
    const score_args &a = sl.lane[blockIdx.z];
    if (blockIdx.x * NT >= a.n_tiles_used || blockIdx.y >= a.n_layer) return;
    constexpr uint32_t TW = KVM_MEANK_TILE;       // blocks per tile
    constexpr uint32_t HC = 8 / NT;               // heads per chunk
    __shared__ __align__(16) float s_k[64][D + 4];   // kh as [lane][dim], rows padded against bank conflicts
    __shared__ __align__(16) float s_qv[HC][D + 4];
    __shared__ float s_nq[HC];
    __shared__ float s_nk[64];
    __shared__ float s_cos[KVM_SCORE_HMAX][TW * 8];
    const uint32_t tile = blockIdx.x * NT, il = blockIdx.y;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t qc = a.q_count[il];
    const uint32_t g = a.n_head / a.H;
    for (uint32_t c = 0; c * HC < a.H; ++c) {
        const uint32_t nh = a.H - c * HC < HC ? a.H - c * HC : HC;
        float dot;
        if (NT == 1 && nh <= 4) score_chunk<D, 1, NT>(a, il, tile, c, nh, g, qc, s_k, s_qv, s_nq, s_nk, s_cos, &dot);
        else score_chunk<D, 2, NT>(a, il, tile, c, nh, g, qc, s_k, s_qv, s_nq, s_nk, s_cos, &dot);
        if (qc == 0) return;
    }
    if (w == 0 && lane < TW * NT && tile * TW + lane < a.n_blocks) {
        double layer = 0.0;
        for (uint32_t h = 0; h < a.H; ++h) layer += (double)s_cos[h][lane];
        a.layer_score[(uint64_t)il * a.cap + tile * TW + lane] = layer / (double)(a.H > 1 ? a.H : 1);
    }
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
                    w ? w->shadow_rows : nullptr, w ? out->stage_src : nullptr, w ? w->block_tokens : 0u};
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

extern "C" int kvm_select_topk(kvm_state *st, const double *scores, const kvm_select_params *p,
                               const kvm_window *w, const kvm_selection *out) {
    if (!st) return KVM_EINVAL;
    int rc = check_select(st, p, out);
    if (rc) return rc;
    if (p->n_blocks && !scores) return kvm_fail(st, KVM_EINVAL, "select_topk: null scores");
    KVM_HIP(st, hipSetDevice(st->device));
    topk_lanes tl{};
    rc = make_topk(st, scores, nullptr, nullptr, nullptr, p, w, out, &tl.lane[0]);
    if (rc) return rc;
    return kvm_topk_launch(st, tl, 1);
}

template <int NT>
static void launch_score(bool d256, dim3 grid, dim3 block, hipStream_t stream, const score_lanes &sl) {
    if (d256) hipLaunchKernelGGL((k_score<256, NT>), grid, block, 0, stream, sl);
    else hipLaunchKernelGGL((k_score<128, NT>), grid, block, 0, stream, sl);
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
int kvm_retrieval_score(kvm_state *st, const kvm_retrieval_lane *lanes, uint32_t n_lanes, const topk_lanes &tl) {
    score_lanes sl{};
    uint32_t max_tiles = 0, max_layer = 0;
    for (uint32_t i = 0; i < n_lanes; ++i) {
        const kvm_retrieval_lane &r = lanes[i];
        const kvm_meank_index *ix = r.ix;
        const uint32_t used = r.p->n_blocks ? kvm_cdiv(r.p->n_blocks, KVM_MEANK_TILE) : 0u;
        sl.lane[i] = score_args{r.q->q_sum, r.q->q_count, ix->k_sum, ix->mean_tokens, (double *)tl.lane[i].layer_score,
                                r.p->n_blocks, ix->n_blocks, kvm_cdiv(ix->n_blocks, KVM_MEANK_TILE), ix->n_layer,
                                r.q->n_head, ix->n_head_kv, used};
        max_tiles = used > max_tiles ? used : max_tiles;
        max_layer = ix->n_layer > max_layer ? ix->n_layer : max_layer;
    }
    if (max_tiles == 0) return KVM_OK;
    KVM_HIP(st, hipSetDevice(st->device));
    // tiles per workgroup: head chunks of HC = 8 / NT heads fill the 64 chain
    // lanes; lanes with different kv-head counts share the largest chunk
    uint32_t max_h = 0;
    for (uint32_t i = 0; i < n_lanes; ++i) max_h = lanes[i].ix->n_head_kv > max_h ? lanes[i].ix->n_head_kv : max_h;
    int nt = max_h > 4 ? 1 : max_h > 2 ? 2 : max_h == 2 ? 4 : 8;
    // fewer tiles per workgroup (some chain lanes idle) while the scoring
    // workgroups still all run at once, two per CU: one memory round trip and
    // one chain per workgroup either way, so more of them finish sooner (a
    // 256K-token lane at 4 kv heads: 256 workgroups of 8 blocks score and
    // select in 15.8 us against 16.8 with 128 of 16)
    while (nt > 1) {
        uint64_t wgs = 0;
        for (uint32_t i = 0; i < n_lanes; ++i) {
            const uint32_t used = lanes[i].p->n_blocks ? kvm_cdiv(lanes[i].p->n_blocks, KVM_MEANK_TILE) : 0u;
            wgs += (uint64_t)kvm_cdiv(used, (uint32_t)nt / 2) * lanes[i].ix->n_layer;
        }
        if (wgs > 2ull * st->n_cu) break;
        nt /= 2;
    }
    const dim3 grid(kvm_cdiv(max_tiles, (uint32_t)nt), max_layer, n_lanes), block(256);
    const bool d256 = lanes[0].ix->head_dim == 256;
    switch (nt) {
    case 1: launch_score<1>(d256, grid, block, st->stream, sl); break;
    case 2: launch_score<2>(d256, grid, block, st->stream, sl); break;
    case 4: launch_score<4>(d256, grid, block, st->stream, sl); break;
    default: launch_score<8>(d256, grid, block, st->stream, sl); break;
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
