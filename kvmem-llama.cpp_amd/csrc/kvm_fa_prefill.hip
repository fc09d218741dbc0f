// kvm_fa_prefill.hip -- flash attention for long query chunks (chunked prefill,
// long MTP verify) on the matrix cores.
//
// The op is ggml_flash_attn_ext as build_attn calls it
// (patches/0002-attn-qk-capture-hook.patch:225, kq_scale at :256), causal over
// the window plus the chunk's own cells: a cell is visible to a query token iff
// it is live (pos >= 0) and its original position is <= the token's
// (patches/0003-kv-cache-skip-hole-purge.patch:78-90).  For a quantised cache
// and a multi-token query, ggml's GPU backends convert K and V to f16 and run
// an f16 matrix-core kernel; this file does the same with CDNA4 MFMA.
//
// Launch 1, k_pf_stage: per (kv head, 64-cell tile) the q8_0 K / q4_0 V (or
// f16 / f16) tile becomes f16 MFMA operand tiles in the workspace, and tile
// 0..n of the window gets a (min pos, max pos, live cells) summary.
//   K f16 tile: [sub 4][kstep D/32][lane 64][8 halves], lane 16g+m = key
//               16*sub+m, dims 32*kstep+8g..+7 (the A operand of S^T = K Q^T).
//   V f16 tile: [dim tile D/16][kstep 2][lane 64][8 halves], lane 16g+m = dim
//               16*dt+m; half j = 4h+r is key 32*kstep + 16h + 4g + r.  That
//               key order is the order in which S^T's accumulator holds the
//               scores (key 4g+r of each 16-key sub tile), so P goes from the
//               S^T accumulator into the B operand of O^T = V^T P^T without a
//               cross-lane exchange.
// Launch 2, k_pf_attn: one workgroup per (128 query rows, kv head, key split);
// a row is (token, query head of the group), so the 6 query heads of a kv
// head share every K/V tile.  8 waves x 16 rows (two waves per SIMD).  K/V tiles are copied from
// global memory straight into LDS (double buffered, one barrier per tile); the
// tiles of the workgroup's key range that some row can see are listed in LDS
// once at the start.  Q stays in registers as f16 B
// operands; O^T (16 rows x D per wave) lives in the accumulators.  Online softmax in the
// log2 domain with a lazy running maximum (rescale only when a row max grows
// by more than 2^8).  Tiles no row of the workgroup can see are skipped;
// tiles every row sees in full skip the mask.
// Launch 3 (key splits > 1), k_pf_combine: merges the split partials.
#include "kvm_internal.h"

#include <climits>

#define KVM_PF_ROWS 128          // query rows per workgroup
#define KVM_PF_MAX_SPLITS 8
#define KVM_PF_LAZY 8.0f         // log2 growth of a row max tolerated before a rescale
#define KVM_PF_LIST 8192         // most tiles one key split may hold

typedef __attribute__((address_space(3))) void *kvm_lds_ptr;

extern "C" int kvm_fa_prefill_chunked(kvm_state *st, const kvm_window *w, const void *q, int q_type,
                                      const int32_t *q_pos, uint32_t n_tokens, uint32_t n_head,
                                      float scale, float *out);

struct pf_stage_args {
    const uint8_t *k, *v;        // window K / V tiles
    const int32_t *cell_pos;
    _Float16 *kh, *vh;           // f16 operand tiles [H][n_tiles][64 * D]
    int32_t *info;               // [n_tiles][4]: min live pos, max live pos, live cells, 0
    uint32_t n_tiles;
    int k_q8, v_q4;
};

__device__ inline float q8_val(uint32_t w, int byte) {
    return (float)(int8_t)(uint8_t)(w >> (8 * byte));
}
__device__ inline float q4_val(uint32_t w, uint32_t j) {
    return (float)((int)((w >> kvm_vq_nib_shift(j)) & 15u) - 8);
}

template <int D>
__global__ void __launch_bounds__(256) k_pf_stage(pf_stage_args a) {
    constexpr int NB = D / 32;
    const uint32_t t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const uint64_t tile = (uint64_t)h * a.n_tiles + t;
    _Float16 *kh = a.kh + tile * 64 * D;
    _Float16 *vh = a.vh + tile * 64 * D;
    if (a.k_q8) {
        // unit = the 16 quant bytes of (sub s, block pair p, lane 16g+m): key
        // 16s+m, blocks 2p and 2p+1, dims 8g..8g+7 of each
        const uint8_t *kt = a.k + tile * kvm_ktile_bytes(KVM_TYPE_Q8_0, D);
        for (uint32_t u = tid; u < 4u * (NB / 2) * 64u; u += 256) {
            const uint32_t ln = u & 63u, sp = u >> 6, s = sp / (NB / 2), p = sp % (NB / 2), m = ln & 15u;
            const kvm_u32x4 qw = *(const kvm_u32x4 *)(kt + (u << 4));
            const float d0 = kvm_h2f(*(const uint16_t *)(kt + kvm_kd_off(D, 16 * s + m, 2 * p)));
            const float d1 = kvm_h2f(*(const uint16_t *)(kt + kvm_kd_off(D, 16 * s + m, 2 * p + 1)));
            kvm_f16x8 o0, o1;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                o0[j] = (_Float16)(q8_val(qw[j >> 2], j & 3) * d0);
                o1[j] = (_Float16)(q8_val(qw[2 + (j >> 2)], j & 3) * d1);
            }
            *(kvm_f16x8 *)(kh + ((s * NB + 2 * p) * 64 + ln) * 8) = o0;
            *(kvm_f16x8 *)(kh + ((s * NB + 2 * p + 1) * 64 + ln) * 8) = o1;
        }
    } else {
        // the f16 window tile already has the operand layout
        const kvm_u32x4 *src = (const kvm_u32x4 *)(a.k + tile * kvm_ktile_bytes(KVM_TYPE_F16, D));
        for (uint32_t i = tid; i < 64u * D / 8; i += 256) ((kvm_u32x4 *)kh)[i] = src[i];
    }
    // V: unit = (dim tile dt, kstep ks, pair gp, dim m).  Its two source words
    // hold keys 32ks + 8gp + j (h = 0) and 32ks + 16 + 8gp + j (h = 1), j < 8;
    // keys j < 4 go to operand lane group 2gp, keys j >= 4 to group 2gp + 1.
    for (uint32_t u = tid; u < 4u * D; u += 256) {
        const uint32_t m = u & 15u, gp = (u >> 4) & 1u, ks = (u >> 5) & 1u, dt = u >> 6;
        const uint32_t d = 16 * dt + m;
        float va[8], vb[8];
        if (a.v_q4) {
            const uint8_t *vt = a.v + tile * kvm_vtile_bytes(KVM_TYPE_Q4_0, D);
            const uint32_t wa = *(const uint32_t *)(vt + kvm_vq_word(d, gp, ks));
            const uint32_t wb = *(const uint32_t *)(vt + kvm_vq_word(d, 2 + gp, ks));
            const uint16_t *sa = (const uint16_t *)(vt + kvm_vd_off(D, 32 * ks + 8 * gp, d >> 5));
            const uint16_t *sb = (const uint16_t *)(vt + kvm_vd_off(D, 32 * ks + 16 + 8 * gp, d >> 5));
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                va[j] = q4_val(wa, j) * kvm_h2f(sa[j]);
                vb[j] = q4_val(wb, j) * kvm_h2f(sb[j]);
            }
        } else {
            const _Float16 *vt = (const _Float16 *)(a.v + tile * kvm_vtile_bytes(KVM_TYPE_F16, D));
            const kvm_f16x8 ha = *(const kvm_f16x8 *)(vt + kvm_vh_idx(32 * ks + 8 * gp, d));
            const kvm_f16x8 hb = *(const kvm_f16x8 *)(vt + kvm_vh_idx(32 * ks + 16 + 8 * gp, d));
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                va[j] = (float)ha[j];
                vb[j] = (float)hb[j];
            }
        }
        kvm_f16x8 lo, hi;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            lo[r] = (_Float16)va[r];
            lo[4 + r] = (_Float16)vb[r];
            hi[r] = (_Float16)va[4 + r];
            hi[4 + r] = (_Float16)vb[4 + r];
        }
        *(kvm_f16x8 *)(vh + ((dt * 2 + ks) * 64 + 16 * (2 * gp) + m) * 8) = lo;
        *(kvm_f16x8 *)(vh + ((dt * 2 + ks) * 64 + 16 * (2 * gp + 1) + m) * 8) = hi;
    }
    if (h == 0 && tid < 64) {
        const int32_t p = a.cell_pos[(uint64_t)t * 64 + tid];
        int32_t mn = p >= 0 ? p : INT_MAX, mx = p >= 0 ? p : INT_MIN, n = p >= 0;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            mn = min(mn, __shfl_xor(mn, o, 64));
            mx = max(mx, __shfl_xor(mx, o, 64));
            n += __shfl_xor(n, o, 64);
        }
        if (tid == 0) {
            int32_t *f = a.info + (uint64_t)t * 4;
            f[0] = mn;
            f[1] = mx;
            f[2] = n;
            f[3] = 0;
        }
    }
}

struct pf_args {
    const _Float16 *kh, *vh;
    const int32_t *info, *cell_pos;
    const void *q;
    const int32_t *q_pos;
    float *out;                  // [token][n_head][D] fp32
    float *ws_o;                 // split partials [split][H][rows_pad][D]
    float *ws_ml;                // [split][H][rows_pad][2]: scaled max, sum
    uint32_t n_tiles, H, G, n_head, n_rows, rows_pad, n_splits, n_row_tiles;
    float c;                     // kq_scale * log2(e)
    int q_bf16;
};

template <int D, int RT>
__global__ void __launch_bounds__(64 * (8 / RT)) k_pf_attn(pf_args a) {
    // LDS operand rings: K runs KR-1 k-steps ahead of its MFMAs, V VR-1
    // operands ahead (the first ones in flight during the softmax), so the
    // LDS latency hides behind matrix-core work instead of a wait per MFMA
    constexpr int KR = 3, VR = 6;
    constexpr int NW = 8 / RT;                            // waves; NW x RT x 16 = 128 rows
    constexpr int KS = D / 32, DT = D / 16;
    constexpr uint32_t TILE_H = 64u * D;                  // halves per K (or V) tile
    __shared__ __align__(16) _Float16 s_kv[2][2 * TILE_H];   // [buffer][K tile | V tile]
    __shared__ __align__(16) int32_t s_cp[2][64];           // the tiles' cell positions
    __shared__ uint16_t s_list[KVM_PF_LIST];
    __shared__ int32_t s_mm[2][NW];
    __shared__ uint32_t s_wsum[NW];
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 4, m = l & 15;

    // Workgroup -> (row tile, kv head, split).  Consecutive hardware workgroup
    // ids go round robin over the 8 XCDs; regroup them so one XCD runs
    // consecutive row tiles of the same (head, split), which share their K/V
    // tiles in that XCD's L2.
    const uint32_t n_wg = gridDim.x;
    uint32_t wg = blockIdx.x;
    if ((n_wg & 7u) == 0) wg = (wg & 7u) * (n_wg >> 3) + (wg >> 3);
    const uint32_t rt_i = wg % a.n_row_tiles, hs = wg / a.n_row_tiles;
    const uint32_t h = hs % a.H, split = hs / a.H;
    const uint32_t r0 = rt_i * KVM_PF_ROWS;

    // ---- rows of this lane: r0 + 16 RT w + 16 rt + m
    int32_t qpos[RT];
    uint32_t rows[RT];
    int32_t mn = INT_MAX, mx = INT_MIN;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        rows[rt] = r0 + 16 * RT * w + 16 * rt + m;
        const bool live = rows[rt] < a.n_rows;
        qpos[rt] = live ? a.q_pos[rows[rt] / a.G] : INT_MIN;
        if (live) {
            mn = min(mn, qpos[rt]);
            mx = max(mx, qpos[rt]);
        }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        mn = min(mn, __shfl_xor(mn, o, 64));
        mx = max(mx, __shfl_xor(mx, o, 64));
    }
    if (l == 0) {
        s_mm[0][w] = mn;
        s_mm[1][w] = mx;
    }

    // ---- Q rows as f16 B operands: lane (g, m) holds Q[row m][32ks + 8g .. +7]
    kvm_f16x8 qop[RT][KS];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const bool live = rows[rt] < a.n_rows;
        const uint32_t row = live ? rows[rt] : 0;
        const uint64_t base = ((uint64_t)(row / a.G) * a.n_head + h * a.G + row % a.G) * D + 8 * g;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            kvm_f16x8 v;
            if (a.q_bf16) {
                const kvm_u32x4 raw = *(const kvm_u32x4 *)((const uint16_t *)a.q + base + 32 * ks);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    v[2 * j] = (_Float16)__uint_as_float(raw[j] << 16);
                    v[2 * j + 1] = (_Float16)__uint_as_float(raw[j] & 0xffff0000u);
                }
            } else {
                const kvm_f32x4 x0 = *(const kvm_f32x4 *)((const float *)a.q + base + 32 * ks);
                const kvm_f32x4 x1 = *(const kvm_f32x4 *)((const float *)a.q + base + 32 * ks + 4);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    v[j] = (_Float16)x0[j];
                    v[4 + j] = (_Float16)x1[j];
                }
            }
            if (!live) v = kvm_f16x8{};
            qop[rt][ks] = v;
        }
    }
    __syncthreads();
    int32_t wg_min = s_mm[0][0], wg_max = s_mm[1][0];
#pragma unroll
    for (int i = 1; i < NW; ++i) {
        wg_min = min(wg_min, s_mm[0][i]);
        wg_max = max(wg_max, s_mm[1][i]);
    }

    // ---- this split's tiles.  A list in LDS holds the tiles some row here can
    // see (tile - t_begin, bit 15 = every cell live and visible to every row,
    // so no mask), built once by a block-wide scan.
    const uint32_t tps = (a.n_tiles + a.n_splits - 1) / a.n_splits;
    const uint32_t t_begin = split * tps < a.n_tiles ? split * tps : a.n_tiles;
    const uint32_t t_end = t_begin + tps < a.n_tiles ? t_begin + tps : a.n_tiles;
    uint32_t n_live = 0;
    for (uint32_t t0 = t_begin; t0 < t_end; t0 += 64 * NW) {
        const uint32_t t = t0 + tid;
        uint32_t live = 0, full = 0;
        if (t < t_end) {
            const kvm_i32x4 f = *(const kvm_i32x4 *)(a.info + (uint64_t)t * 4);
            live = f[2] != 0 && f[0] <= wg_max;
            full = f[2] == 64 && f[1] <= wg_min;
        }
        const uint32_t incl = kvm_wave_incl_scan(live);
        if (l == 63) s_wsum[w] = incl;
        __syncthreads();
        uint32_t before = n_live, total = 0;
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            before += i < w ? s_wsum[i] : 0u;
            total += s_wsum[i];
        }
        if (live) s_list[before + incl - 1] = (uint16_t)((t - t_begin) | (full << 15));
        n_live += total;
        __syncthreads();
    }

    // Tile copies go global -> LDS directly (global_load_lds_dwordx4: lane l
    // writes 16 bytes at M0 + offset + 16 l), issued from asm so the compiler
    // adds no wait for them; the loop waits for them itself before each
    // barrier.  The asm restores M0, which the compiler reserves.  Wave w copies
    // bytes [CW w, CW (w+1)) of the tile's K and of its V: CW / 1 KB copies per
    // part under one M0 value, the immediate offset moving the global and the
    // LDS address alike.  Wave 0 also copies the tile's 64 cell positions.
    constexpr uint32_t CW = TILE_H * 2 / NW;             // bytes of one K (or V) tile per wave
    static_assert(CW == 4096 || CW == 2048, "copy layout");
    const uint32_t lds_kv = (uint32_t)(uintptr_t)(kvm_lds_ptr)&s_kv[0][0];
    const uint32_t lds_cp = (uint32_t)(uintptr_t)(kvm_lds_ptr)&s_cp[0][0];
    const uint32_t loff = 16u * l;                       // this lane's bytes in a 1 KB copy
    const uint32_t wofs = __builtin_amdgcn_readfirstlane(CW * w);
    const uint8_t *k_head = (const uint8_t *)(a.kh + (uint64_t)h * a.n_tiles * TILE_H) + wofs;
    const uint8_t *v_head = (const uint8_t *)(a.vh + (uint64_t)h * a.n_tiles * TILE_H) + wofs;
    auto dma_tile = [&](uint32_t t, int buf) {
        t = __builtin_amdgcn_readfirstlane(t);
        const uint8_t *kb = k_head + (uint64_t)t * (TILE_H * 2);
        const uint8_t *vb = v_head + (uint64_t)t * (TILE_H * 2);
        const uint32_t dk = lds_kv + (uint32_t)buf * (2 * TILE_H * 2) + wofs;
        const uint32_t dv = dk + TILE_H * 2;
        uint32_t m0_saved;
        if constexpr (CW == 4096) {
            asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\t"
                         "global_load_lds_dwordx4 %1, %4\n\t"
                         "global_load_lds_dwordx4 %1, %4 offset:1024\n\t"
                         "global_load_lds_dwordx4 %1, %4 offset:2048\n\t"
                         "global_load_lds_dwordx4 %1, %4 offset:3072\n\t"
                         "s_mov_b32 m0, %3\n\ts_nop 0\n\t"
                         "global_load_lds_dwordx4 %1, %5\n\t"
                         "global_load_lds_dwordx4 %1, %5 offset:1024\n\t"
                         "global_load_lds_dwordx4 %1, %5 offset:2048\n\t"
                         "global_load_lds_dwordx4 %1, %5 offset:3072\n\t"
                         "s_mov_b32 m0, %0"
                         : "=&s"(m0_saved) : "v"(loff), "s"(dk), "s"(dv), "s"(kb), "s"(vb) : "memory");
        } else {
            asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\t"
                         "global_load_lds_dwordx4 %1, %4\n\t"
                         "global_load_lds_dwordx4 %1, %4 offset:1024\n\t"
                         "s_mov_b32 m0, %3\n\ts_nop 0\n\t"
                         "global_load_lds_dwordx4 %1, %5\n\t"
                         "global_load_lds_dwordx4 %1, %5 offset:1024\n\t"
                         "s_mov_b32 m0, %0"
                         : "=&s"(m0_saved) : "v"(loff), "s"(dk), "s"(dv), "s"(kb), "s"(vb) : "memory");
        }
        if (w == 0) {
            const int32_t *src = a.cell_pos + (uint64_t)t * 64;
            const uint32_t dst = lds_cp + (uint32_t)buf * 256;
            asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, %3\n\ts_mov_b32 m0, %0"
                         : "=&s"(m0_saved) : "v"(4u * l), "s"(dst), "s"(src) : "memory");
        }
    };

    kvm_f32x4 O[RT][DT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) O[rt][dt] = kvm_f32x4{0.f, 0.f, 0.f, 0.f};
    float ms[RT], lp[RT];                   // running max of each row (times c), lane's share of its sum
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        ms[rt] = -INFINITY;
        lp[rt] = 0.0f;
    }
    const float c = a.c;

    // list entries k and k+1 are in registers at the top of tile k; entry k+2
    // is read during tile k
    uint32_t e_cur = n_live > 0 ? s_list[0] : 0u, e_nxt = n_live > 1 ? s_list[1] : e_cur;
    if (n_live > 0) dma_tile(t_begin + (e_cur & 0x7fffu), 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (uint32_t k = 0; k < n_live; ++k) {
        const int b = k & 1;
        const uint32_t e = __builtin_amdgcn_readfirstlane(e_cur);
        const uint32_t en = __builtin_amdgcn_readfirstlane(e_nxt);
        e_cur = en;
        e_nxt = s_list[k + 2 < n_live ? k + 2 : n_live - 1];
        dma_tile(t_begin + (en & 0x7fffu), b ^ 1);        // next tile, in flight during this one
        const bool masked = (e >> 15) == 0;
        const _Float16 *sk = s_kv[b];
        const _Float16 *sv = s_kv[b] + TILE_H;

        // S^T = K Q^T: sub tile s holds keys 16s + 4g + r of row m
        kvm_f32x4 S[4][RT];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) S[s][rt] = kvm_f32x4{0.f, 0.f, 0.f, 0.f};
        // K operands run KR-1 k-steps ahead of their MFMAs (a register ring)
        kvm_f16x8 kr[KR][4];
#pragma unroll
        for (int p = 0; p < KR - 1; ++p)
#pragma unroll
            for (int s = 0; s < 4; ++s) kr[p][s] = *(const kvm_f16x8 *)(sk + ((s * KS + p) * 64 + l) * 8);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            if (ks + KR - 1 < KS) {
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    kr[(ks + KR - 1) % KR][s] = *(const kvm_f16x8 *)(sk + ((s * KS + ks + KR - 1) * 64 + l) * 8);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
                    S[s][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kr[ks % KR][s], qop[rt][ks], S[s][rt], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        // the first V operands, in flight during the softmax
        kvm_f16x8 vr[VR];
#pragma unroll
        for (int i = 0; i < VR - 1; ++i) vr[i] = *(const kvm_f16x8 *)(sv + (((i % DT) * 2 + i / DT) * 64 + l) * 8);
        if (masked) {
            asm volatile("" ::: "memory");                // keep the mask on this (rare) path
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const kvm_i32x4 cp = *(const kvm_i32x4 *)&s_cp[b][16 * s + 4 * g];
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (!(cp[r] >= 0 && cp[r] <= qpos[rt])) S[s][rt][r] = -INFINITY;
            }
        }
        // online softmax per row
        float tmax[RT];
        bool up[RT], any = false;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            float x = S[0][rt][0];
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int r = 0; r < 4; ++r) x = fmaxf(x, S[s][rt][r]);
            x = kvm_max_xor32(kvm_max_xor16(x));
            tmax[rt] = x;
            up[rt] = fmaf(x, c, -ms[rt]) > KVM_PF_LAZY;   // false for a row with nothing visible yet
            any = any || up[rt];
        }
        if (__builtin_amdgcn_ballot_w64(any) != 0) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const float mnew = up[rt] ? tmax[rt] * c : ms[rt];
                const float alpha = up[rt] ? __builtin_amdgcn_exp2f(ms[rt] - mnew) : 1.0f;
                ms[rt] = mnew;
                lp[rt] *= alpha;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) O[rt][dt] *= alpha;
            }
        }
        kvm_f16x8 pB[RT][2];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const float msr = ms[rt] == -INFINITY ? 0.0f : ms[rt];
            float sum = 0.0f;
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    // the row sum takes p before its rounding to the fp16 operand:
                    // within 2^-11 of it per element
                    const float p = __builtin_amdgcn_exp2f(fmaf(S[s][rt][r], c, -msr));
                    pB[rt][s >> 1][4 * (s & 1) + r] = (_Float16)p;
                    sum += p;
                }
            lp[rt] += sum;
        }
        // O^T += V^T P^T
        // operand i = (kk, dt) = (i / DT, i % DT); the ring stays VR-1 ahead
#pragma unroll
        for (int i = 0; i < 2 * DT; ++i) {
            const int kk = i / DT, dt = i % DT, n = i + VR - 1;
            if (n < 2 * DT) vr[n % VR] = *(const kvm_f16x8 *)(sv + (((n % DT) * 2 + n / DT) * 64 + l) * 8);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
                O[rt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vr[i % VR], pB[rt][kk], O[rt][dt], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the next tile's copies
        __syncthreads();
    }

    // ---- results
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        float lr = lp[rt];
        lr = kvm_add_xor32(kvm_add_xor16(lr));
        const uint32_t row = rows[rt];
        if (row >= a.n_rows) continue;
        if (a.n_splits == 1) {
            const float inv = lr > 0.0f ? 1.0f / lr : 0.0f;
            float *o = a.out + ((uint64_t)(row / a.G) * a.n_head + h * a.G + row % a.G) * D + 4 * g;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) *(kvm_f32x4 *)(o + 16 * dt) = O[rt][dt] * inv;
        } else {
            const uint64_t pr = ((uint64_t)split * a.H + h) * a.rows_pad + row;
            float *o = a.ws_o + pr * D + 4 * g;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) *(kvm_f32x4 *)(o + 16 * dt) = O[rt][dt];
            if (g == 0) {
                a.ws_ml[pr * 2] = ms[rt];
                a.ws_ml[pr * 2 + 1] = lr;
            }
        }
    }
}

// Merge the key splits of each (kv head, row): one thread per 4 dims.
template <int D>
__global__ void __launch_bounds__(256) k_pf_combine(pf_args a) {
    constexpr int TPR = D / 4;                            // threads per row
    const uint32_t row = blockIdx.x * (256 / TPR) + threadIdx.x / TPR, h = blockIdx.y;
    if (row >= a.n_rows) return;
    const uint32_t d4 = (threadIdx.x % TPR) * 4;
    float M = -INFINITY;
    for (uint32_t s = 0; s < a.n_splits; ++s)
        M = fmaxf(M, a.ws_ml[(((uint64_t)s * a.H + h) * a.rows_pad + row) * 2]);
    kvm_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    float L = 0.0f;
    if (M != -INFINITY) {
        for (uint32_t s = 0; s < a.n_splits; ++s) {
            const uint64_t pr = ((uint64_t)s * a.H + h) * a.rows_pad + row;
            const float ms = a.ws_ml[pr * 2];
            const float wgt = ms == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ms - M);
            L += a.ws_ml[pr * 2 + 1] * wgt;
            acc += *(const kvm_f32x4 *)(a.ws_o + pr * D + d4) * wgt;
        }
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    *(kvm_f32x4 *)(a.out + ((uint64_t)(row / a.G) * a.n_head + h * a.G + row % a.G) * D + d4) = acc * inv;
}

// Key splits: the fewest that keep the whole device busy, for one resident
// workgroup per CU (the double-buffered K/V tiles take 128 KB of LDS at D 256).
// KVM_PF_SPLITS in the environment fixes the count.
static uint32_t pf_choose_splits(uint32_t n_units, uint32_t n_tiles, int n_cu) {
    if (const char *e = getenv("KVM_PF_SPLITS")) {
        const int v = atoi(e);
        if (v >= 1 && v <= KVM_PF_MAX_SPLITS) return (uint32_t)v < n_tiles ? (uint32_t)v : n_tiles;
    }
    uint32_t best = 1;
    double best_t = 1e30;
    for (uint32_t s = 1; s <= KVM_PF_MAX_SPLITS && s <= n_tiles; ++s) {
        const uint32_t rounds = (n_units * s + n_cu - 1) / n_cu;
        const double t = (double)rounds / s + (s > 1 ? 0.02 : 0.0);   // combine pass
        if (t < best_t - 1e-9) {
            best_t = t;
            best = s;
        }
    }
    return best;
}

template <int D>
static void pf_launch(const pf_args &a, const pf_stage_args &sa, hipStream_t stream) {
    hipLaunchKernelGGL(k_pf_stage<D>, dim3(sa.n_tiles, a.H), dim3(256), 0, stream, sa);
    // 8 waves of 16 rows: two waves per SIMD, so one wave's softmax overlaps
    // the other's matrix-core work
    hipLaunchKernelGGL((k_pf_attn<D, 1>), dim3(a.n_row_tiles * a.H * a.n_splits), dim3(512), 0, stream, a);
    if (a.n_splits > 1)
        hipLaunchKernelGGL(k_pf_combine<D>, dim3(kvm_cdiv(a.n_rows, 256 / (D / 4)), a.H), dim3(256), 0, stream, a);
}

extern "C" int kvm_fa_prefill(kvm_state *st, const kvm_window *w, const void *q, int q_type,
                              const int32_t *q_pos, uint32_t n_tokens, uint32_t n_head, float scale,
                              float *out) {
    if (!st || !w || !q || !q_pos || !out) return kvm_fail(st, KVM_EINVAL, "fa_prefill: null argument");
    int rc = kvm_window_check(w);
    if (rc) return kvm_fail(st, rc, "fa_prefill: bad window");
    if (q_type != KVM_TYPE_F32 && q_type != KVM_TYPE_BF16) return kvm_fail(st, KVM_EUNSUPPORTED, "fa_prefill: q type %d", q_type);
    if (!w->n_head_kv || n_head % w->n_head_kv) return kvm_fail(st, KVM_EINVAL, "fa_prefill: head counts");
    if (n_tokens == 0) return KVM_OK;
    const uint32_t G = n_head / w->n_head_kv;
    // Up to 32 rows per kv head the decode kernel's tile fits the whole query.
    if ((uint64_t)n_tokens * G <= 32) return kvm_fa_prefill_chunked(st, w, q, q_type, q_pos, n_tokens, n_head, scale, out);

    const uint32_t D = w->head_dim, H = w->n_head_kv, n_tiles = w->n_cells / KVM_TILE_CELLS;
    const uint64_t n_rows = (uint64_t)n_tokens * G;
    if (n_rows > (1u << 30)) return kvm_fail(st, KVM_ERANGE, "fa_prefill: %u tokens", n_tokens);
    int n_cu = 256;
    if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, st->device) != hipSuccess || n_cu <= 0) n_cu = 256;

    pf_args a{};
    a.n_tiles = n_tiles;
    a.H = H;
    a.G = G;
    a.n_head = n_head;
    a.n_rows = (uint32_t)n_rows;
    a.n_row_tiles = (uint32_t)kvm_cdiv(n_rows, KVM_PF_ROWS);
    a.rows_pad = a.n_row_tiles * KVM_PF_ROWS;
    a.n_splits = pf_choose_splits(a.n_row_tiles * H, n_tiles, n_cu);
    while (kvm_cdiv(n_tiles, a.n_splits) > KVM_PF_LIST) ++a.n_splits;   // a split's tile list fits LDS
    a.c = scale * 1.4426950408889634f;
    a.q_bf16 = q_type == KVM_TYPE_BF16;
    a.q = q;
    a.q_pos = q_pos;
    a.out = out;
    a.cell_pos = w->cell_pos;

    // workspace: f16 K and V operand tiles, tile summaries, split partials
    const size_t kv_bytes = (size_t)H * n_tiles * 64 * D * 2;
    const size_t info_bytes = (size_t)n_tiles * 16;
    const size_t part_o = a.n_splits > 1 ? (size_t)a.n_splits * H * a.rows_pad * D * 4 : 0;
    const size_t part_ml = a.n_splits > 1 ? (size_t)a.n_splits * H * a.rows_pad * 2 * 4 : 0;
    auto up256 = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t total = 2 * up256(kv_bytes) + up256(info_bytes) + up256(part_o) + up256(part_ml);
    uint8_t *ws = (uint8_t *)kvm_workspace(st, total);
    if (!ws) return kvm_fail(st, KVM_ENOMEM, "fa_prefill: workspace of %zu bytes", total);
    pf_stage_args sa{};
    sa.k = (const uint8_t *)w->k;
    sa.v = (const uint8_t *)w->v;
    sa.cell_pos = w->cell_pos;
    sa.kh = (_Float16 *)ws;
    sa.vh = (_Float16 *)(ws + up256(kv_bytes));
    sa.info = (int32_t *)(ws + 2 * up256(kv_bytes));
    sa.n_tiles = n_tiles;
    sa.k_q8 = kvm_k_quant(w->k_type);
    sa.v_q4 = w->v_type == KVM_TYPE_Q4_0;
    a.kh = sa.kh;
    a.vh = sa.vh;
    a.info = sa.info;
    a.ws_o = (float *)(ws + 2 * up256(kv_bytes) + up256(info_bytes));
    a.ws_ml = (float *)(ws + 2 * up256(kv_bytes) + up256(info_bytes) + up256(part_o));

    KVM_HIP(st, hipSetDevice(st->device));
    if (D == 256) pf_launch<256>(a, sa, st->stream);
    else pf_launch<128>(a, sa, st->stream);
    KVM_LAUNCH_CHECK(st, "fa_prefill");
    return KVM_OK;
}
