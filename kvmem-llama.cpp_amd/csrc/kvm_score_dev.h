// kvm_score_dev.h -- the retrieval scorer's device side shared by the scoring
// grid (k_score, kvm_retrieval.hip) and the decode step's selecting attention
// launch (kvm_fa_decode.hip), whose attention workgroups score one 8-block
// tile of the mean-K index each before their first key tile.
//
// score_retrieval (llama-memory-kvmem.cpp:4149-4196) per (layer, block, kv head):
//   qv[d] = (sum over the group's query rows of q_sum, in row order) * invq,
//           invq = 1 / (q_count * g)
//   kh[d] = k_sum[d] * (1 / mean_tokens)   (+0 for a block without tokens)
//   dot = sum qv kh, nq = sum qv qv, nk = sum kh kh   (sequential fp32 chains)
//   cos = dot / (sqrt(nq) sqrt(nk) + 1e-6f)
// and per (layer, block): the cosines summed in double in head order, / H.
// Every fp32 operation is one IEEE rounding (kvm_fadd / kvm_fmul / kvm_fdiv,
// correctly rounded sqrtf), as on the host.
#pragma once
#include "kvm_internal.h"

// Mean-K index tiles: KVM_MEANK_TILE blocks, embedding-major inside a tile.
#define KVM_MEANK_TILE 8u
#define KVM_SCORE_GMAX 16   // largest query group (n_head / n_head_kv)
#define KVM_SCORE_HMAX 16   // largest n_head_kv

struct score_args {
    const float *q_sum;
    const uint32_t *q_count;
    const float *k_sum;
    const uint32_t *mean_tokens;
    double *layer_score;    // [n_layer][cap]
    uint32_t n_blocks, cap, n_tiles, n_layer, n_head, H;
    uint32_t n_tiles_used;  // tiles holding the first n_blocks blocks
    uint32_t g;             // query heads per kv head, n_head / H
    const float *q_vec;     // [n_layer][H][D]: qv formed with the sums, or null
    const float *q_norm;    // [n_layer][H]: nq beside it
    const float *k_norm;    // [n_layer][H][cap]: the blocks' nk formed with the index, or null
};

// Device-coherent 64-bit store / load of a layer contribution written and read
// by different workgroups of one launch (agent scope: the reader may sit on
// another XCD, whose L2 holds no copy or a stale one).
__device__ __forceinline__ void kvm_st_f64_dev(double *p, double v) {
    __hip_atomic_store((uint64_t *)p, (uint64_t)__double_as_longlong(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ double kvm_ld_f64_dev(const double *p) {
    return __longlong_as_double(
        (long long)__hip_atomic_load((const uint64_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// LDS of one wave's (tile, head) pass, rows of D floats padded against bank
// conflicts, by layout:
//   KVM_SL_ROWS  the 17 product rows (dot products of blocks 0-7, their kh
//                squares, qv squares);
//   KVM_SL_OTF   qv and the kh of blocks 0-7, the chains forming their
//                products on the fly (about half the LDS);
//   KVM_SL_NK    the index carries the blocks' nk: 9 product rows (the dot
//                products, qv squares).
#define KVM_SL_ROWS 0
#define KVM_SL_OTF 1
#define KVM_SL_NK 2
template <int D, int LAY>
struct score_wave_lds {
    float p[LAY == KVM_SL_NK ? 9 : 17][D + 4];
};
template <int D>
struct score_wave_lds<D, KVM_SL_OTF> {
    float qv[D + 4];
    float kh[KVM_MEANK_TILE][D + 4];
};
// The scoring workgroup's LDS: one region per scoring wave, the cosines of
// every head and the count of heads done.
template <int D, int NW, int LAY>
struct score_wg_lds {
    score_wave_lds<D, LAY> w[NW];
    float cos[KVM_SCORE_HMAX][KVM_MEANK_TILE];
    uint32_t heads_done;
};

// The global reads of one wave's (layer il, tile, kv head h) pass: lane
// l < D/4 holds dims 4l..4l+3 of the tile's 8 blocks (8 x 16 B of the slab:
// blocks 0-3 then 4-7 of each dim) and of the group's first 8 query rows
// (clamped: a load under a branch would be waited for at the branch's join),
// or with QV of the head's qv row and its nq, and the 8 token counts.  Issued
// early, they overlap other round trips.
struct score_regs {
    kvm_f32x4 kv[8];
    kvm_f32x4 qg[8];
    uint32_t mt[KVM_MEANK_TILE];
    float nq, nk;
};
template <int D, bool QV, int LAY>
__device__ __forceinline__ void score_tile_load(const score_args &a, uint32_t il, uint32_t tile, uint32_t h, uint32_t g,
                                                score_regs &r) {
    constexpr uint32_t TW = KVM_MEANK_TILE, NL = D / 4;
    const uint32_t l = threadIdx.x & 63u, lc = l < NL ? l : 0u;
    const uint64_t HD = (uint64_t)a.H * D;
    const kvm_f32x4 *slab = (const kvm_f32x4 *)(a.k_sum + (((uint64_t)il * a.n_tiles + tile) * HD + (uint64_t)h * D) * TW);
#pragma unroll
    for (int j = 0; j < 8; ++j) r.kv[j] = slab[lc * 8u + j];
    if constexpr (QV) {
        r.qg[0] = *(const kvm_f32x4 *)(a.q_vec + ((uint64_t)il * a.H + h) * D + 4u * lc);
        r.nq = a.q_norm[(uint64_t)il * a.H + h];
    } else {
        const float *qrow = a.q_sum + ((uint64_t)il * a.n_head + (uint64_t)h * g) * D + 4u * lc;
#pragma unroll
        for (uint32_t gi = 0; gi < 8; ++gi) r.qg[gi] = *(const kvm_f32x4 *)(qrow + (uint64_t)(gi < g ? gi : 0u) * D);
    }
#pragma unroll
    for (uint32_t bi = 0; bi < TW; ++bi) {
        const uint32_t b = tile * TW + bi;
        r.mt[bi] = a.mean_tokens[(uint64_t)il * a.cap + (b < a.n_blocks ? b : a.n_blocks - 1)];
    }
    if constexpr (LAY == KVM_SL_NK) {
        // lane c < 8: nk of block 8 tile + c (clamped, as the counts)
        const uint32_t b = tile * TW + (l & 7u);
        r.nk = a.k_norm[((uint64_t)il * a.H + h) * a.cap + (b < a.n_blocks ? b : a.n_blocks - 1)];
    }
}

// One wave scores the pass whose reads `r` holds, without any workgroup
// barrier (the other waves of its workgroup may be in a barrier sequence of
// their own): every lane forms qv and kh of its 4 dims and the products
// qv kh (8 blocks), kh kh (8 blocks) and qv qv, each one IEEE rounding, into
// the wave's LDS rows (read back by the same wave only); lane c < 17 then runs
// chain c over d in order (the reference's dot of block c, nk of block c - 8,
// nq: the product of each step is the same float, and the additions the same
// sequence), and lanes 0-7 form the cosines into cos_h[0..7].  LAY (the LDS
// layouts above): KVM_SL_OTF stores qv and kh instead and each chain forms
// its products as it goes (the same floats); KVM_SL_NK takes nk from the
// index (formed once per change of a block's sum, the same operations), so
// only the dot rows and qv squares are formed: chain 8 is nq.  qc =
// q_count[il] > 0.  With QV, qv and nq come formed (the same operations, done
// once per change of the query sums).
template <int D, bool QV, int LAY>
__device__ __forceinline__ void score_tile_compute(const score_args &a, uint32_t il, uint32_t h, uint32_t qc,
                                                   uint32_t g, const score_regs &r, score_wave_lds<D, LAY> &L,
                                                   float *cos_h) {
    constexpr bool OTF = LAY == KVM_SL_OTF, NK = LAY == KVM_SL_NK;
    constexpr uint32_t RQ = NK ? 8u : 16u;          // the row of the qv squares
    constexpr uint32_t TW = KVM_MEANK_TILE, NL = D / 4;
    const uint32_t l = threadIdx.x & 63u;
    if (l < NL) {
        float qv[4];
        if constexpr (QV) {
#pragma unroll
            for (int e = 0; e < 4; ++e) qv[e] = r.qg[0][e];
        } else {
            const float invq = kvm_recip_or0((float)(qc * (g > 1u ? g : 1u)));   // = 1.0f / x, IEEE
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float qh = 0.0f;
#pragma unroll
                for (uint32_t gi = 0; gi < 8; ++gi)
                    if (gi < g) qh = kvm_fadd(qh, r.qg[gi][e]);
                if (g > 8u) {                                // groups above 8 (rare)
                    const float *qrow = a.q_sum + ((uint64_t)il * a.n_head + (uint64_t)h * g) * D + 4u * l;
                    for (uint32_t gi = 8; gi < g; ++gi) qh = kvm_fadd(qh, qrow[(uint64_t)gi * D + e]);
                }
                qv[e] = kvm_fmul(qh, invq);
            }
            if constexpr (!OTF)
                *(kvm_f32x4 *)&L.p[RQ][4u * l] = kvm_f32x4{kvm_fmul(qv[0], qv[0]), kvm_fmul(qv[1], qv[1]),
                                                           kvm_fmul(qv[2], qv[2]), kvm_fmul(qv[3], qv[3])};
        }
        if constexpr (OTF) *(kvm_f32x4 *)&L.qv[4u * l] = kvm_f32x4{qv[0], qv[1], qv[2], qv[3]};
#pragma unroll
        for (uint32_t bi = 0; bi < TW; ++bi) {
            const float inv = kvm_recip_or0((float)r.mt[bi]);
            const uint32_t keep = r.mt[bi] ? 0xffffffffu : 0u;
            const uint32_t hi = bi >= 4u ? 1u : 0u, e = bi & 3u;
            float k4[4];
#pragma unroll
            for (int dd = 0; dd < 4; ++dd)
                k4[dd] = __uint_as_float(__float_as_uint(kvm_fmul(r.kv[2 * dd + hi][e], inv)) & keep);
            if constexpr (OTF) {
                *(kvm_f32x4 *)&L.kh[bi][4u * l] = kvm_f32x4{k4[0], k4[1], k4[2], k4[3]};
            } else {
                *(kvm_f32x4 *)&L.p[bi][4u * l] = kvm_f32x4{kvm_fmul(qv[0], k4[0]), kvm_fmul(qv[1], k4[1]),
                                                           kvm_fmul(qv[2], k4[2]), kvm_fmul(qv[3], k4[3])};
                if constexpr (!NK)
                    *(kvm_f32x4 *)&L.p[8 + bi][4u * l] = kvm_f32x4{kvm_fmul(k4[0], k4[0]), kvm_fmul(k4[1], k4[1]),
                                                                   kvm_fmul(k4[2], k4[2]), kvm_fmul(k4[3], k4[3])};
            }
        }
    }
    // the wave's LDS writes are done before its reads (LDS operations of one
    // wave complete in order; the fence keeps the compiler from moving them)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    // ---- chains: lane c <= RQ runs chain c (lanes past RQ repeat chain RQ,
    // unused; with QV chain RQ is not used).  The adds of one chain are
    // dependent, so the chain runs at the VALU's dependent-issue rate only if
    // its operands are in registers ahead of it: LOOK chunks of 16 dims (of
    // both factors, 8 dims, with OTF) are in flight, the LDS latency being
    // longer than one chunk's adds.
    float chain = 0.0f;
    const uint32_t c = l <= RQ ? l : RQ;
    if constexpr (!OTF) {
        const float *row = L.p[c];
        constexpr int CH = 4;                // float4 per 16-dim chunk
        constexpr int NC = D / (4 * CH);     // chunks
        constexpr int LOOK = 3;              // chunks in flight (12 LDS reads: under lgkmcnt's 15)
        kvm_f32x4 buf[LOOK][CH];
        auto ld = [&](kvm_f32x4 (&x)[CH], int k) {
#pragma unroll
            for (int j = 0; j < CH; ++j) x[j] = *(const kvm_f32x4 *)&row[4 * (CH * k + j)];
        };
        auto add = [&](const kvm_f32x4 (&x)[CH]) {
#pragma unroll
            for (int j = 0; j < CH; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) chain = kvm_fadd(chain, x[j][e]);
        };
#pragma unroll
        for (int k = 0; k < LOOK; ++k) ld(buf[k], k);
#pragma unroll
        for (int k = 0; k < NC; ++k) {
            __builtin_amdgcn_sched_barrier(0);
            add(buf[k % LOOK]);
            __builtin_amdgcn_sched_barrier(0);
            if (k + LOOK < NC) ld(buf[k % LOOK], k + LOOK);
        }
    } else {
        const float *fa = c < 8u || c == 16u ? L.qv : L.kh[c - 8u];
        const float *fb = c < 8u ? L.kh[c] : (c < 16u ? L.kh[c - 8u] : L.qv);
        constexpr int CH = 2;                // float4 per 8-dim chunk
        constexpr int NC = D / (4 * CH);     // chunks
        constexpr int LOOK = 3;              // chunks in flight (12 LDS reads)
        kvm_f32x4 bufa[LOOK][CH], bufb[LOOK][CH];
        auto ld = [&](kvm_f32x4 (&x)[CH], kvm_f32x4 (&y)[CH], int k) {
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                x[j] = *(const kvm_f32x4 *)&fa[4 * (CH * k + j)];
                y[j] = *(const kvm_f32x4 *)&fb[4 * (CH * k + j)];
            }
        };
        auto add = [&](const kvm_f32x4 (&x)[CH], const kvm_f32x4 (&y)[CH]) {
#pragma unroll
            for (int j = 0; j < CH; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) chain = kvm_fadd(chain, kvm_fmul(x[j][e], y[j][e]));
        };
#pragma unroll
        for (int k = 0; k < LOOK; ++k) ld(bufa[k], bufb[k], k);
#pragma unroll
        for (int k = 0; k < NC; ++k) {
            __builtin_amdgcn_sched_barrier(0);
            add(bufa[k % LOOK], bufb[k % LOOK]);
            __builtin_amdgcn_sched_barrier(0);
            if (k + LOOK < NC) ld(bufa[k % LOOK], bufb[k % LOOK], k + LOOK);
        }
    }
    // (the chain counts as live on every lane: where only lanes 0-7 use theirs,
    // the compiler otherwise runs the chain under a narrowed exec mask and
    // takes three times the registers)
    asm volatile("" : "+v"(chain));
    // ---- cosines of blocks 0-7 (every lane takes part in the shuffles)
    const float nk = NK ? r.nk : __shfl(chain, (int)((l & 7u) + 8u), 64);
    const float nq = QV ? r.nq : __shfl(chain, (int)RQ, 64);
    if (l < TW) {
        const float den = kvm_fadd(kvm_fmul(kvm_fsqrt(nq), kvm_fsqrt(nk)), 1e-6f);
        cos_h[l] = kvm_fdiv(chain, den);
    }
}

// The layer contribution of the tile's blocks from the cosines of all H
// heads (lanes 0-7): sum in double in head order, / H, stored device-coherently.
__device__ __forceinline__ void score_tile_store(const score_args &a, uint32_t il, uint32_t tile,
                                                 const float (*cos)[KVM_MEANK_TILE]) {
    const uint32_t l = threadIdx.x & 63u, b = tile * KVM_MEANK_TILE + l;
    if (l < KVM_MEANK_TILE && b < a.n_blocks) {
        double layer = 0.0;
        for (uint32_t hh = 0; hh < a.H; ++hh) layer += (double)cos[hh][l];
        kvm_st_f64_dev(a.layer_score + (uint64_t)il * a.cap + b, layer / (double)(a.H > 1 ? a.H : 1));
    }
}
