// kvm_stagein_dev.h -- device side of the stage-in, shared by the stage-in
// kernel and the decode attention kernel that stages its lanes' plans.
//
// K: dequant q8_0 -> NeoX RoPE at the window position -> normalised
// Walsh-Hadamard -> q8_0, the order of llama-kvmem-stagein.cu:731-786, fused in
// one pass with the row held in registers (one wave per (token, head) row,
// lane L owning dims DPL*L .. DPL*L+DPL-1).  Every operation is an explicitly
// rounded IEEE op, so the output bytes equal the host restatement's.
// V: q4_0 bytes are moved unchanged into the tiled layout (stagein.cu:733-744).
#pragma once
#include "kvm_internal.h"

#include <type_traits>

struct rope_ctx {
    const float2 *tab;     // [n_pos][n_half] (cos, sin)
    uint32_t n_half;       // n_rot / 2
    uint32_t n_pos;
    int32_t nrot;          // Hadamard width, 0 = off
    float hscale;          // 1 / sqrtf(nrot), computed on the host as the reference does
};

// NR (token, head) rows of D dims, interleaved so that their dependent shuffle
// chains overlap: row r's src = NB q8_0 blocks (34 B each; q4: q4_0 blocks of
// 18 B, requantised with quant_q4_0's arithmetic, llama-kvmem-stagein.cu:201-234,
// and held as q8_0 tile quants, the nibble minus 8) readable by every lane,
// requantised into K tile kt[r] at cell c[r] (0..63); cs[r] = the (cos, sin)
// row of its window position, [n_half] (global memory or LDS).  Rows with
// live[r] false are computed on their (valid) inputs but not written.  KQ:
// KVM_KQ_Q8 / KVM_KQ_Q4 fix the K type at compile time (the other's code left
// out), KVM_KQ_ANY takes it from q4_arg.
#define KVM_KQ_Q8 0
#define KVM_KQ_Q4 1
#define KVM_KQ_ANY 2
template <int D, int NR, int KQ = KVM_KQ_ANY>
__device__ inline void stage_k_rows(const uint8_t *const (&src)[NR], uint8_t *const (&kt)[NR],
                                    const uint32_t (&c)[NR], const float2 *const (&cs_pos)[NR],
                                    const bool (&live)[NR], const rope_ctx &rc, bool q4_arg = false) {
    const bool q4 = KQ == KVM_KQ_ANY ? q4_arg : KQ == KVM_KQ_Q4;
    constexpr int DPL = D / 64;
    const int L = threadIdx.x & 63;
    const int d0 = DPL * L;
    const int b = d0 >> 5, e = d0 & 31;
    float x[NR][DPL];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        if (!q4) {
            const uint8_t *blk = src[r] + b * 34;
            const float dsc = kvm_h2f((uint16_t)(blk[0] | (blk[1] << 8)));
#pragma unroll
            for (int i = 0; i < DPL; ++i) x[r][i] = kvm_fmul((float)(int8_t)blk[2 + e + i], dsc);
        } else {
            // dims 0-15 of a block are the low nibbles of its 16 bytes, 16-31 the
            // high ones (a lane's DPL dims sit in one half)
            const uint8_t *blk = src[r] + b * 18;
            const float dsc = kvm_h2f((uint16_t)(blk[0] | (blk[1] << 8)));
            const int sh = e >= 16 ? 4 : 0, j0 = e & 15;
#pragma unroll
            for (int i = 0; i < DPL; ++i) x[r][i] = kvm_fmul((float)((int)((blk[2 + j0 + i] >> sh) & 15) - 8), dsc);
        }
    }

    // NeoX RoPE: dims i and i + n_half rotate together for i < n_half.
    const int nh = (int)rc.n_half;
    if (nh > 0) {
        const int pl = nh / DPL;                       // lane distance of the partner
        const bool lo = d0 < nh, hi = d0 >= nh && d0 < 2 * nh;
        // each lane reads its partner only: lane + pl below n_half, lane - pl
        // above (lanes past 2 n_half read a value they do not use)
        const int pa = ((lo ? L + pl : L - pl) & 63) << 2;
        float y[NR][DPL];
#pragma unroll
        for (int r = 0; r < NR; ++r)
#pragma unroll
            for (int i = 0; i < DPL; ++i)
                y[r][i] = __int_as_float(__builtin_amdgcn_ds_bpermute(pa, __float_as_int(x[r][i])));
        // x0' = x0 c - x1 s below n_half, x1' = x0 s + x1 c above, both as
        // RN(RN(x c) + RN(y s')) with s' = -s below (the same roundings, no
        // branch); lanes past 2 n_half read row entry 0 and keep x
        const bool act = lo || hi;
        const int ci = lo ? d0 : hi ? d0 - nh : 0;
        const uint32_t sm = lo ? 0x80000000u : 0u;
        // every table entry loaded before the first product (source order is
        // what the compiler keeps where registers are scarce)
        float2 t[NR][DPL];
#pragma unroll
        for (int r = 0; r < NR; ++r)
#pragma unroll
            for (int i = 0; i < DPL; ++i) t[r][i] = cs_pos[r][ci + (act ? i : 0)];
#pragma unroll
        for (int r = 0; r < NR; ++r)
#pragma unroll
            for (int i = 0; i < DPL; ++i) {
                const float v = kvm_fadd(kvm_fmul(x[r][i], t[r][i].x),
                                         kvm_fmul(y[r][i], __uint_as_float(__float_as_uint(t[r][i].y) ^ sm)));
                x[r][i] = act ? v : x[r][i];
            }
    }

    // normalised Walsh-Hadamard over nrot-wide chunks: pre-scale, then
    // butterflies h = 1, 2, ..., nrot/2 (stagein.cu:105-131)
    if (rc.nrot > 0) {
#pragma unroll
        for (int r = 0; r < NR; ++r)
#pragma unroll
            for (int i = 0; i < DPL; ++i) x[r][i] = kvm_fmul(x[r][i], rc.hscale);
#pragma unroll
        for (int h = 1; h < DPL; h <<= 1)
#pragma unroll
            for (int r = 0; r < NR; ++r)
#pragma unroll
                for (int i = 0; i < DPL; ++i) {
                    if (!(i & h)) {
                        const float a = x[r][i], bb = x[r][i + h];
                        x[r][i] = kvm_fadd(a, bb);
                        x[r][i + h] = kvm_fsub(a, bb);
                    }
                }
        // across lanes, with the partner's value o: a lane whose bit lx is
        // clear needs x + o, its partner o - x.  Both compute fma(o, +-1, x),
        // the same single rounding, the partner getting -(o - x): its register
        // holds the value negated from then on.  A lane's sign is the parity of
        // its bits below lx; that holds for its partner too, so every stage
        // reads like the first, and x is the fma's addend, updated in place.
        for (int h = DPL; h < rc.nrot; h <<= 1) {
            const int lx = h / DPL;
            const int pa = (L ^ lx) << 2;
            const float sg = (L & lx) == 0 ? 1.0f : -1.0f;
            // all of the stage's shuffles in flight before its first fma
            float o[NR][DPL];
#pragma unroll
            for (int r = 0; r < NR; ++r)
#pragma unroll
                for (int i = 0; i < DPL; ++i)
                    o[r][i] = __int_as_float(__builtin_amdgcn_ds_bpermute(pa, __float_as_int(x[r][i])));
#pragma unroll
            for (int r = 0; r < NR; ++r)
#pragma unroll
                for (int i = 0; i < DPL; ++i) x[r][i] = __builtin_fmaf(o[r][i], sg, x[r][i]);
        }
    }
    // the sign the lane's registers carry (bit 31), undone by the requantiser's
    // 1/d (|x| is unaffected, and x * -id is -x * id exactly)
    const uint32_t xs = rc.nrot > DPL && (__popc((uint32_t)L & (uint32_t)(rc.nrot / DPL - 1)) & 1) ? 0x80000000u : 0u;

    // q8_0 requantisation of each 32-dim block (32/DPL lanes per block); q4:
    // quant_q4_0's, vmax = the first value of largest magnitude in dim order
    // (lanes in dim order, the lower lanes' value kept on a tie) with its true
    // sign, d = vmax / -8 (vmax * -0.125 exactly), id = d ? 1/d : 0, quant =
    // min(15, (int)(x id + 8.5)) - 8
    const uint32_t lq = kvm_kq_off(D, 0, d0);
    float amax[NR], vmax[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        amax[r] = 0.0f;
        vmax[r] = 0.0f;
        if (!q4) {
#pragma unroll
            for (int i = 0; i < DPL; ++i) amax[r] = fmaxf(amax[r], fabsf(x[r][i]));
        } else {
#pragma unroll
            for (int i = 0; i < DPL; ++i) {
                const float av = fabsf(x[r][i]);
                if (amax[r] < av) {
                    amax[r] = av;
                    vmax[r] = x[r][i];
                }
            }
            vmax[r] = __uint_as_float(__float_as_uint(vmax[r]) ^ xs);
        }
    }
#pragma unroll
    for (int o = 1; o < 32 / DPL; o <<= 1)
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const float ap = __shfl_xor(amax[r], o, 64);
            if (!q4) {
                amax[r] = fmaxf(amax[r], ap);
            } else {
                const float vp = __shfl_xor(vmax[r], o, 64);
                const bool lower = (L & o) == 0;                 // this lane's dims come first
                const float a_f = lower ? amax[r] : ap, v_f = lower ? vmax[r] : vp;
                const float a_s = lower ? ap : amax[r], v_s = lower ? vp : vmax[r];
                const bool take_s = a_f < a_s;
                amax[r] = take_s ? a_s : a_f;
                vmax[r] = take_s ? v_s : v_f;
            }
        }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const float d = q4 ? kvm_fmul(vmax[r], -0.125f) : kvm_div127(amax[r]);
        const float id = __uint_as_float(__float_as_uint(kvm_recip_or0(d)) ^ xs);
        // the lane's DPL quants are consecutive in the tile (8-byte runs of one
        // block and lane group): one store of DPL bytes, aligned to DPL
        uint32_t qw = 0;
#pragma unroll
        for (int i = 0; i < DPL; ++i) {
            int qi;
            if (!q4) {
                qi = kvm_round_away(kvm_fmul(x[r][i], id));
            } else {
                qi = (int)kvm_fadd(kvm_fmul(x[r][i], id), 8.5f);
                qi = (qi > 15 ? 15 : qi) - 8;
            }
            qw |= (uint32_t)(uint8_t)(int8_t)qi << (8 * i);
        }
        if (!live[r]) continue;
        // tile offsets split into the row's cell part and the lane's dim part
        uint8_t *row = kt[r] + kvm_kq_off(D, c[r], 0);
        uint8_t *qd = row + lq;
        if constexpr (DPL == 4) *(uint32_t *)qd = qw;
        else if constexpr (DPL == 2) *(uint16_t *)qd = (uint16_t)qw;
        else *qd = (uint8_t)qw;
        if (e == 0) *(uint16_t *)(kt[r] + kvm_kd_off(D, c[r], 0) + 32u * b) = kvm_f2h(d);
    }
}

// One row (stage_k_rows of one; q4: src holds q4_0 blocks).
template <int D>
__device__ inline void stage_k_row(const uint8_t *src, uint8_t *kt, uint32_t c, const float2 *cs_pos,
                                   const rope_ctx &rc, bool q4 = false) {
    const uint8_t *const s1[1] = {src};
    uint8_t *const k1[1] = {kt};
    const uint32_t c1[1] = {c};
    const float2 *const t1[1] = {cs_pos};
    const bool l1[1] = {true};
    stage_k_rows<D, 1>(s1, k1, c1, t1, l1, rc, q4);
}

// The same K rows with LG = D / 16 lanes per (token, head) row, 64 / LG rows
// per wave.  Lane l of a row's group holds the 16 consecutive dims 16 m ..
// 16 m + 15, where the bits of m (dim bits 4 and up) are the lane's
// coordinates c4, c5, ... in a basis of lane patterns that one DPP move
// exchanges within the group: dim bit 4 <-> lane xor 1 and bit 5 <-> xor 2
// (quad permutes), bit 6 <-> xor 8 (the 16-lane row rotated by 8; D = 128:
// xor 7, the half-row mirror), bit 7 <-> xor 15 (the row mirror).  Two dims
// that differ in one bit >= 4 then sit in lanes one DPP move apart, so the
// Walsh-Hadamard stages above 8 and the RoPE pairs (n_half a power of two
// >= 16) exchange values without an LDS round trip; dim bits 0-3 stay in the
// lane's registers.  The arithmetic is stage_k_rows' (the same IEEE
// operations in the same order, the same sign carried through the lane
// stages), so the bytes are the same.
template <int D>
__device__ __forceinline__ uint32_t k16_m(uint32_t l) {
    const uint32_t top = (l >> 2) & 1u;
    if constexpr (D == 256) {
        const uint32_t lp = l ^ (top * 15u);
        return (lp & 1u) | (lp & 2u) | (((lp >> 3) & 1u) << 2) | (top << 3);
    } else {
        const uint32_t lp = l ^ (top * 7u);
        return (lp & 1u) | (lp & 2u) | (top << 2);
    }
}
template <int D, int BIT>
__device__ __forceinline__ float k16_swap(float v) {
    static_assert(BIT >= 4 && BIT <= (D == 256 ? 7 : 6), "dim bit held across lanes");
    constexpr int ctrl = BIT == 4 ? 0xB1 : BIT == 5 ? 0x4E : BIT == 6 ? (D == 256 ? 0x128 : 0x141) : 0x140;
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, false));
}
// Whether stage_k_row16 serves this RoPE width (n_half a power of two of
// 16 .. D / 2); others take stage_k_rows.
template <int D>
__host__ __device__ inline bool k16_ok(uint32_t n_half) {
    return n_half >= 16 && n_half <= (uint32_t)D / 2 && (n_half & (n_half - 1)) == 0;
}
// One row per lane group: src = the row's NB q8_0 blocks (34 B each, 2-byte
// aligned; q4: q4_0 blocks of 18 B, requantised to q4_0 with quant_q4_0's
// arithmetic, llama-kvmem-stagein.cu:201-234, and held as q8_0 tile quants,
// the nibble minus 8), requantised into K tile kt at cell c; cs = the (cos,
// sin) row of its window position; l = the lane within the group; live false:
// computed, not written.  Every lane of the wave takes part (the DPP moves).
template <int D>
__device__ __forceinline__ void stage_k_row16(const uint8_t *src, uint8_t *kt, uint32_t c, const float2 *cs, bool live,
                                              uint32_t l, const rope_ctx &rc, bool q4 = false) {
    const uint32_t m = k16_m<D>(l), b = m >> 1, d0 = 16u * m;
    // a power-of-two Hadamard pre-scale (a width that is a power of 4) rides
    // on the block scale: every value it reaches before the butterflies is
    // then scaled by it exactly (no product comes near the subnormals)
    const bool hs2 = (__float_as_uint(rc.hscale) & 0x807fffffu) == 0u;
    const float hs = hs2 ? rc.hscale : 1.0f;
    float x[16];
    if (!q4) {
        const uint8_t *blk = src + b * 34u;
        const float dsc = kvm_fmul(kvm_h2f(*(const uint16_t *)blk), hs);
        const uint16_t *q = (const uint16_t *)(blk + 2u + 16u * (m & 1u));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t w = q[i];
            x[2 * i] = kvm_fmul((float)(int8_t)(uint8_t)w, dsc);
            x[2 * i + 1] = kvm_fmul((float)(int8_t)(uint8_t)(w >> 8), dsc);
        }
    } else {
        // dims 0-15 of a block are the low nibbles of its 16 bytes, 16-31 the high
        const uint8_t *blk = src + b * 18u;
        const float dsc = kvm_fmul(kvm_h2f(*(const uint16_t *)blk), hs);
        const uint16_t *q = (const uint16_t *)(blk + 2u);
        const uint32_t sh = 4u * (m & 1u);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t w = q[i];
            x[2 * i] = kvm_fmul((float)((int)((w >> sh) & 15u) - 8), dsc);
            x[2 * i + 1] = kvm_fmul((float)((int)((w >> (8u + sh)) & 15u) - 8), dsc);
        }
    }
    // NeoX RoPE: dims i and i + n_half (one dim bit, log2 n_half >= 4, apart)
    const uint32_t nh = rc.n_half;
    {
        float y[16];
        switch (nh) {
        case 16:
#pragma unroll
            for (int i = 0; i < 16; ++i) y[i] = k16_swap<D, 4>(x[i]);
            break;
        case 32:
#pragma unroll
            for (int i = 0; i < 16; ++i) y[i] = k16_swap<D, 5>(x[i]);
            break;
        case 64:
#pragma unroll
            for (int i = 0; i < 16; ++i) y[i] = k16_swap<D, 6>(x[i]);
            break;
        default:
#pragma unroll
            for (int i = 0; i < 16; ++i) y[i] = k16_swap<D, D == 256 ? 7 : 6>(x[i]);
            break;
        }
        // x0' = x0 c - x1 s below n_half, x1' = x0 s + x1 c above, as
        // RN(RN(x c) + RN(y s')) with s' = -s below; lanes past 2 n_half keep x
        const bool lo = d0 < nh, act = d0 < 2u * nh;
        const float2 *t = cs + (act ? (d0 & (nh - 1u)) : 0u);
        const uint32_t sm = lo ? 0x80000000u : 0u;
        float2 tv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) tv[i] = t[act ? i : 0];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float v = kvm_fadd(kvm_fmul(x[i], tv[i].x), kvm_fmul(y[i], __uint_as_float(__float_as_uint(tv[i].y) ^ sm)));
            x[i] = act ? v : x[i];
        }
    }
    // normalised Walsh-Hadamard over nrot-wide chunks: pre-scale, butterflies
    // h = 1, 2, 4, 8 in the lane, then one DPP exchange per dim bit 4 .. log2
    // nrot - 1 with the lane's sign carried as in stage_k_rows
    uint32_t xs = 0;
    if (rc.nrot > 0) {
        if (!hs2) {
#pragma unroll
            for (int i = 0; i < 16; ++i) x[i] = kvm_fmul(x[i], rc.hscale);
        }
#pragma unroll
        for (int h = 1; h < 16; h <<= 1)
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (!(i & h)) {
                    const float a = x[i], bb = x[i + h];
                    x[i] = kvm_fadd(a, bb);
                    x[i + h] = kvm_fsub(a, bb);
                }
        auto stage = [&](auto bit_c) {
            constexpr int BIT = decltype(bit_c)::value;
            const uint32_t ck = (m >> (BIT - 4)) & 1u;
            const float sg = ck ? -1.0f : 1.0f;
            xs ^= ck;
            float o[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) o[i] = k16_swap<D, BIT>(x[i]);
#pragma unroll
            for (int i = 0; i < 16; ++i) x[i] = __builtin_fmaf(o[i], sg, x[i]);
        };
        if (rc.nrot > 16) stage(std::integral_constant<int, 4>{});
        if (rc.nrot > 32) stage(std::integral_constant<int, 5>{});
        if (rc.nrot > 64) stage(std::integral_constant<int, 6>{});
        if constexpr (D == 256)
            if (rc.nrot > 128) stage(std::integral_constant<int, 7>{});
    }
    // requantisation: a 32-dim block is the lane and its dim bit 4 partner
    uint32_t qw[4];
    float d;
    if (!q4) {
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(x[i]));
        amax = fmaxf(amax, k16_swap<D, 4>(amax));
        d = kvm_div127(amax);
        const float id = __uint_as_float(__float_as_uint(kvm_recip_or0(d)) ^ (xs << 31));
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            qw[k] = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) qw[k] |= (uint32_t)(uint8_t)kvm_round_away(kvm_fmul(x[4 * k + i], id)) << (8 * i);
        }
    } else {
        // quant_q4_0: vmax = the first value of largest magnitude in dim order
        // (the lane with dims 0-15 of the block comes first), with its true
        // sign (the lane's registers carry xs); d = vmax / -8 (vmax * -0.125
        // exactly), id = d ? 1/d : 0, quant = min(15, (int)(x id + 8.5)) - 8
        float am = 0.0f, vm = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float a = fabsf(x[i]);
            if (am < a) { am = a; vm = x[i]; }
        }
        vm = __uint_as_float(__float_as_uint(vm) ^ (xs << 31));
        const float am_p = k16_swap<D, 4>(am), vm_p = k16_swap<D, 4>(vm);
        const bool first = (m & 1u) == 0u;
        const float am_f = first ? am : am_p, vm_f = first ? vm : vm_p;
        const float am_s = first ? am_p : am, vm_s = first ? vm_p : vm;
        const float vmax = am_f < am_s ? vm_s : vm_f;
        d = kvm_fmul(vmax, -0.125f);
        const float id = __uint_as_float(__float_as_uint(kvm_recip_or0(d)) ^ (xs << 31));
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            qw[k] = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int xi = (int)kvm_fadd(kvm_fmul(x[4 * k + i], id), 8.5f);
                xi = xi > 15 ? 15 : xi;
                qw[k] |= (uint32_t)(uint8_t)(int8_t)(xi - 8) << (8 * i);
            }
        }
    }
    if (!live) return;
    // two 8-byte runs of the tile (dims 16m .. +7 and 16m + 8 .. +15)
    *(kvm_u32x2 *)(kt + kvm_kq_off(D, c, d0)) = kvm_u32x2{qw[0], qw[1]};
    *(kvm_u32x2 *)(kt + kvm_kq_off(D, c, d0 + 8u)) = kvm_u32x2{qw[2], qw[3]};
    if ((m & 1u) == 0) *(uint16_t *)(kt + kvm_kd_off(D, c, b)) = kvm_f2h(d);
}

// ---------------------------------------------------------------------------
// Selection-driven stage-in: workgroup = (staged slot, 64-cell tile of it).
// ---------------------------------------------------------------------------
struct stage_args {
    const uint8_t *hk, *hv;          // pinned host rows
    uint32_t h_tokens;
    uint8_t *wk, *wv;
    int32_t *cell_pos;
    uint32_t *slot_block;
    int32_t *slot_base;
    uint32_t n_tiles, H, bt, n_slots;
    const uint32_t *ids;
    const int32_t *to_base;
    const uint32_t *stage_slots;
    uint32_t *info;
    rope_ctx rc;
    // HBM re-basing of resident blocks (all null without a shadow): the raw K
    // rows of every staged cell, per plan entry the slot its block held before
    // the plan (-1: from the host), and per plan entry a staging region of
    // bt K rows then bt V rows that the gather fills before any slot is written
    uint8_t *k_shadow;
    uint32_t *shadow_rows;
    const int32_t *stage_src;
    uint8_t *moves;
    uint32_t *sync;                  // the lane's barrier words (kvm_state::stage_sync)
    uint32_t *status;                // the state's sticky wait status (KVM_WAIT_STAGE when a barrier gives up)
    uint32_t spin;                   // polls of a barrier wait before it gives up (0: at once)
    uint32_t k_q4;                   // q4_0 K: history rows of 18-byte blocks, requantised to q4_0
};

// dst[i] = src[i] for 16-byte units i = tid, tid + nth, ... < n (n >= 1, the
// ranges disjoint): eight loads in flight before their stores (a load-store
// pair per step would wait for each load in turn); loads past n re-read n - 1.
// The loads (LD_DEV) or the stores (ST_DEV) device-coherent (kvm_ld16_dev /
// kvm_st16_dev): the move staging is written before a lane barrier and read
// after it by other workgroups.
template <bool LD_DEV, bool ST_DEV>
__device__ inline void copy16_dev(uint8_t *dst, const uint8_t *src, uint32_t n, uint32_t tid, uint32_t nth) {
    constexpr uint32_t B = 8;
    const __amdgpu_buffer_rsrc_t rs = kvm_rsrc(src), rd = kvm_rsrc(dst);
    for (uint32_t i0 = tid; i0 < n; i0 += B * nth) {
        kvm_u32x4 r[B];
#pragma unroll
        for (uint32_t j = 0; j < B; ++j) {
            const uint32_t i = i0 + j * nth, ic = i < n ? i : n - 1;
            r[j] = LD_DEV ? kvm_ld16_dev(rs, 16u * ic) : *(const kvm_u32x4 *)(src + 16u * ic);
        }
#pragma unroll
        for (uint32_t j = 0; j < B; ++j) {
            const uint32_t i = i0 + j * nth;
            if (i < n) {
                if (ST_DEV) kvm_st16_dev(rd, 16u * i, r[j]);
                else *(kvm_u32x4 *)(dst + 16u * i) = r[j];
            }
        }
    }
}

// The LDS fill of an item whose rows were gathered into the staging region
// sb by other workgroups before the lane's barrier (device-coherent loads): nk
// 16-byte units of K rows from sb + koff to dk, then nv units of V rows from
// sb + voff to dv, and nt units of (cos, sin) rows, the first TB per thread
// held in registers while the rows stream.
__device__ inline void stage_fill_dev(uint8_t *dk, uint8_t *dv, const uint8_t *sb, uint32_t koff, uint32_t nk,
                                      uint32_t voff, uint32_t nv, uint8_t *dt, const uint8_t *__restrict__ stab,
                                      uint32_t nt, uint32_t tid, uint32_t nth) {
    constexpr uint32_t B = 8, TB = 4;
    kvm_u32x4 tr[TB];
    if (nt) {
#pragma unroll
        for (uint32_t j = 0; j < TB; ++j) {
            const uint32_t i = tid + j * nth, ic = i < nt ? i : nt - 1;
            tr[j] = *(const kvm_u32x4 *)(stab + 16u * ic);
        }
    }
    const __amdgpu_buffer_rsrc_t rs = kvm_rsrc(sb);
    const uint32_t n = nk + nv;
    for (uint32_t i0 = tid; i0 < n; i0 += B * nth) {
        kvm_u32x4 r[B];
#pragma unroll
        for (uint32_t j = 0; j < B; ++j) {
            const uint32_t i = i0 + j * nth, ic = i < n ? i : n - 1;
            r[j] = kvm_ld16_dev(rs, ic < nk ? koff + 16u * ic : voff + 16u * (ic - nk));
        }
#pragma unroll
        for (uint32_t j = 0; j < B; ++j) {
            const uint32_t i = i0 + j * nth;
            if (i < n) *(kvm_u32x4 *)(i < nk ? dk + 16u * i : dv + 16u * (i - nk)) = r[j];
        }
    }
    if (nt) {
#pragma unroll
        for (uint32_t j = 0; j < TB; ++j) {
            const uint32_t i = tid + j * nth;
            if (i < nt) *(kvm_u32x4 *)(dt + 16u * i) = tr[j];
        }
        for (uint32_t i = tid + TB * nth; i < nt; i += nth) *(kvm_u32x4 *)(dt + 16u * i) = *(const kvm_u32x4 *)(stab + 16u * i);
    }
}

// An item's LDS fill: n0, n1, n2 16-byte units from s0, s1, s2 to d0, d1, d2,
// as one stream of loads, eight in flight per thread before their stores.
__device__ inline void stage_fill(uint8_t *d0, const uint8_t *__restrict__ s0, uint32_t n0, uint8_t *d1,
                                  const uint8_t *__restrict__ s1, uint32_t n1, uint8_t *d2,
                                  const uint8_t *__restrict__ s2, uint32_t n2, uint32_t tid, uint32_t nth) {
    constexpr uint32_t B = 8;
    const uint32_t n01 = n0 + n1, n = n01 + n2;
    for (uint32_t i0 = tid; i0 < n; i0 += B * nth) {
        uint4 r[B];
#pragma unroll
        for (uint32_t j = 0; j < B; ++j) {
            const uint32_t i = i0 + j * nth, ic = i < n ? i : n - 1;
            const uint8_t *p = ic < n0 ? s0 + 16u * ic : ic < n01 ? s1 + 16u * (ic - n0) : s2 + 16u * (ic - n01);
            r[j] = *(const uint4 *)p;
        }
#pragma unroll
        for (uint32_t j = 0; j < B; ++j) {
            const uint32_t i = i0 + j * nth;
            if (i < n) {
                uint8_t *p = i < n0 ? d0 + 16u * i : i < n01 ? d1 + 16u * (i - n0) : d2 + 16u * (i - n01);
                *(uint4 *)p = r[j];
            }
        }
    }
}

// Row bytes of the history / shadow: q8_0 (or q4_0) K and q4_0 V, all kv heads.
__host__ __device__ inline uint32_t stage_kblk(const stage_args &a) { return a.k_q4 ? 18u : 34u; }
__host__ __device__ inline uint32_t stage_row_k(const stage_args &a, uint32_t D) { return a.H * (D / 32) * stage_kblk(a); }
__host__ __device__ inline uint32_t stage_row_v(const stage_args &a, uint32_t D) { return a.H * (D / 32) * 18; }
// Whether a plan that moves blocks also gathers its host entries' rows into
// the staging (16-byte units: rows and history 16-byte aligned), so that every
// item reads HBM after the barrier and a block's rows cross the host link
// spread over all of the lane's workgroups instead of one per item.
template <int D>
__device__ inline bool stage_host_via(const stage_args &a) {
    return a.moves && ((stage_row_k(a, D) | stage_row_v(a, D)) & 15u) == 0 &&
           (((uintptr_t)a.hk | (uintptr_t)a.hv) & 15u) == 0;
}

// One entry's gather (the same copies) by one workgroup with ordinary stores,
// for a launch whose gather barrier writes back and invalidates the caches.
template <int D>
__device__ inline void stage_gather_entry(const stage_args &a, uint32_t si, uint32_t tid, uint32_t nth) {
    const int32_t src = a.stage_src[si];
    if (src < 0) return;
    const uint32_t rowK = stage_row_k(a, D), rowV = stage_row_v(a, D);
    uint8_t *dk = a.moves + (uint64_t)si * a.bt * (rowK + rowV);
    copy16_dev<false, false>(dk, a.k_shadow + (uint64_t)src * a.bt * rowK, a.bt * rowK / 16, tid, nth);
    const uint32_t vtile = kvm_vtile_bytes(KVM_TYPE_Q4_0, D), tps = a.bt / 64, per = vtile / 16;
    uint8_t *dv = dk + (uint64_t)a.bt * rowK;
    for (uint32_t h = 0; h < a.H; ++h)     // a slot's tiles of one head are consecutive
        copy16_dev<false, false>(dv + (uint64_t)h * tps * vtile,
                                 a.wv + ((uint64_t)h * a.n_tiles + (uint64_t)src * tps) * vtile, tps * per, tid, nth);
}

// Gather of the plan entries whose blocks move within the window (stage_src[si]
// = src >= 0) into their staging regions: entry si's bt raw K rows from the
// shadow of slot src, then the slot's V tiles, [head][tile of the slot].
// Slots start on tile boundaries (block_tokens % 64 == 0), so a V tile's bytes
// do not depend on where the slot lies and move as they are.  Only full blocks
// move (the top-k stages partly filled ones from the host).  With host_via
// (stage_host_via) an entry staged from the host gathers its rows too: its
// K rows, then its V rows (row format), the block's tokens only.  The n_ent
// entries' staging regions are one run of 16-byte units, split evenly over the
// lane's G workgroups: workgroup x copies units [U x / G, U (x+1) / G), each
// piece one contiguous copy (K rows of one entry, one head's tiles, or an
// entry's V rows).
template <int D>
__device__ inline void stage_gather_split(const stage_args &a, uint32_t n_ent, uint32_t x, uint32_t G, uint32_t tid,
                                          uint32_t nth, bool host_via) {
    const uint32_t rowK = stage_row_k(a, D), rowV = stage_row_v(a, D);
    const uint32_t vtile = kvm_vtile_bytes(KVM_TYPE_Q4_0, D), tps = a.bt / 64, per = vtile / 16;
    const uint64_t KU = (uint64_t)a.bt * rowK / 16, HU = (uint64_t)tps * per, EU = KU + a.H * HU;
    const uint64_t U = (uint64_t)n_ent * EU, u0 = U * x / G, u1 = U * (x + 1) / G;
    for (uint64_t si = u0 / EU; si < n_ent && si * EU < u1; ++si) {
        const int32_t src = a.stage_src[si];
        const uint64_t e0 = si * EU;
        const uint64_t lo = (u0 > e0 ? u0 : e0) - e0, hi = (u1 < e0 + EU ? u1 : e0 + EU) - e0;
        uint8_t *dk = a.moves + si * a.bt * (rowK + rowV);
        if (src < 0) {
            if (!host_via) continue;
            const uint64_t first = (uint64_t)a.ids[a.stage_slots[si]] * a.bt;
            if (first >= a.h_tokens) continue;                 // not staged (stagein_item reports it)
            const uint64_t nt = a.h_tokens - first < a.bt ? a.h_tokens - first : a.bt;
            const uint64_t k1 = nt * rowK / 16, v1 = KU + nt * rowV / 16;
            if (lo < k1)
                copy16_dev<false, true>(dk + 16 * lo, a.hk + first * rowK + 16 * lo, (uint32_t)((hi < k1 ? hi : k1) - lo),
                                        tid, nth);
            const uint64_t c0 = lo > KU ? lo : KU, c1 = hi < v1 ? hi : v1;
            if (c0 < c1)
                copy16_dev<false, true>(dk + (uint64_t)a.bt * rowK + 16 * (c0 - KU), a.hv + first * rowV + 16 * (c0 - KU),
                                        (uint32_t)(c1 - c0), tid, nth);
            continue;
        }
        if (lo < KU) {
            const uint64_t k1 = hi < KU ? hi : KU;
            copy16_dev<false, true>(dk + 16 * lo, a.k_shadow + (uint64_t)src * a.bt * rowK + 16 * lo, (uint32_t)(k1 - lo),
                                    tid, nth);
        }
        for (uint32_t h = 0; h < a.H; ++h) {           // a slot's tiles of one head are consecutive
            const uint64_t h0 = KU + h * HU, h1 = h0 + HU;
            const uint64_t c0 = lo > h0 ? lo : h0, c1 = hi < h1 ? hi : h1;
            if (c0 >= c1) continue;
            copy16_dev<false, true>(dk + (uint64_t)a.bt * rowK + (uint64_t)h * tps * vtile + 16 * (c0 - h0),
                                    a.wv + ((uint64_t)h * a.n_tiles + (uint64_t)src * tps) * vtile + 16 * (c0 - h0),
                                    (uint32_t)(c1 - c0), tid, nth);
        }
    }
}

// One (plan entry, IT-token run) item, staged by a workgroup of NTH threads
// through the LDS rows buffer s_rows (IT * n_head_kv * (D/32) * 52 bytes).  An
// item of 32 tokens fills one key half (ks) of a 64-cell window tile.
template <int D, int NTH, int IT = 64, bool FAST = true, int KQ = KVM_KQ_ANY>
__device__ __forceinline__ void stagein_item(const stage_args &a, uint8_t *s_rows, uint32_t si, uint32_t tt,
                                             bool host_via = false) {
    static_assert(IT == 64 || IT == 32, "stage-in item size");
    constexpr uint32_t NB = D / 32;
    const uint32_t slot = a.stage_slots[si];
    const uint32_t id = a.ids[slot];
    const int32_t base = a.to_base[slot];
    // history blocks are consecutive block_tokens-sized runs (register_append,
    // kvmem_store.cpp:179-205): block id covers [id*bt, min((id+1)*bt, h_tokens))
    const uint64_t first = (uint64_t)id * a.bt;
    const uint32_t tid = threadIdx.x;
    const int32_t src = a.moves ? a.stage_src[si] : -1;          // >= 0: rows from the gathered staging
    if (src < 0 && first >= a.h_tokens) {
        // a block outside the history is not staged: report it, and empty the
        // slot's cells of this item (and, once, its slot map entry) so attention
        // never reads what the slot held before and the next plan restages it
        if (tid == 0) atomicOr(&a.info[3], 4u);
        if (tid < IT) a.cell_pos[slot * a.bt + tt * IT + tid] = -1;
        if (tt == 0 && tid == 0) {
            a.slot_block[slot] = 0xffffffffu;
            a.slot_base[slot] = -1;
            if (a.shadow_rows) a.shadow_rows[slot] = 0u;
        }
        return;
    }
    const uint32_t nt = src >= 0 ? a.bt : (a.h_tokens - first < a.bt ? (uint32_t)(a.h_tokens - first) : a.bt);
    const uint32_t t0 = tt * IT;
    const uint32_t count = nt > t0 ? (nt - t0 < IT ? nt - t0 : IT) : 0;
    const uint64_t htok0 = first + t0;
    const uint32_t kb = stage_kblk(a), rowK = a.H * NB * kb, rowV = a.H * NB * 18;
    // LDS: the item's K rows, V rows, and the (cos, sin) rows of its positions
    uint8_t *lk = s_rows, *lv = s_rows + IT * rowK;
    float2 *lt = (float2 *)(s_rows + IT * (rowK + rowV));
    // bulk copy of `count` consecutive token rows of K and V (contiguous in host
    // memory, or in the entry's staging region for a block moving in HBM)
    const uint8_t *mk = src >= 0 ? a.moves + (uint64_t)si * a.bt * (rowK + rowV) : nullptr;
    const uint8_t *gk = src >= 0 ? mk + (uint64_t)t0 * rowK : a.hk + htok0 * rowK;
    const uint8_t *gv = src >= 0 ? mk : a.hv + htok0 * rowV;
    // a moved block's V comes as whole tiles (below), not as rows
    const uint32_t nk = count * rowK, nv = src >= 0 ? 0u : count * rowV;
    // the table rows are contiguous ([position][n_half] float2, n_half a multiple of 4)
    const uint32_t nh = a.rc.n_half, ntab = count * nh * 8;
    const uint8_t *gt = (const uint8_t *)(a.rc.tab + (uint64_t)(base + (int32_t)t0) * nh);
    const bool al16 = (((uintptr_t)gk | (uintptr_t)gv | rowK | rowV) & 15u) == 0;
    if (FAST && src >= 0) {
        // rows gathered by other workgroups before the lane's barrier (the
        // staging and the table are 16-byte aligned: rowK is a multiple of 16)
        stage_fill_dev(lk, lv, mk, t0 * rowK, nk / 16, 0, 0, (uint8_t *)lt, gt, ntab / 16, tid, NTH);
    } else if (FAST && host_via) {
        // a host entry's rows, gathered into its staging region: K rows, then V rows
        const uint8_t *hb = a.moves + (uint64_t)si * a.bt * (rowK + rowV);
        stage_fill_dev(lk, lv, hb, t0 * rowK, nk / 16, a.bt * rowK + t0 * rowV, nv / 16, (uint8_t *)lt, gt, ntab / 16,
                       tid, NTH);
    } else if (al16) {
        stage_fill(lk, gk, nk / 16, lv, gv, nv / 16, (uint8_t *)lt, gt, ntab / 16, tid, NTH);
    } else {
        stage_fill(lk, gk, 0, lv, gv, 0, (uint8_t *)lt, gt, ntab / 16, tid, NTH);
        for (uint32_t i = tid; i < nk; i += NTH) lk[i] = gk[i];
        for (uint32_t i = tid; i < nv; i += NTH) lv[i] = gv[i];
    }
    __syncthreads();
    // the raw K rows of the staged cells into the shadow (read when the block
    // is later re-based within the window)
    if (a.k_shadow) {
        // 16-byte aligned: the item starts at a multiple of 32 rows, of an even size
        uint8_t *sk = a.k_shadow + ((uint64_t)slot * a.bt + t0) * rowK;
        for (uint32_t i = tid; i < nk / 16; i += NTH) ((uint4 *)sk)[i] = ((const uint4 *)lk)[i];
        for (uint32_t i = nk / 16 * 16 + tid; i < nk; i += NTH) sk[i] = lk[i];
    }

    const uint32_t tile = (slot * a.bt + t0) / 64, c0 = t0 % 64;   // c0: the item's first cell in the tile
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6), nrow = count * a.H;
    constexpr uint32_t W = NTH / 64, NR = 4;
    uint8_t *const ktile = a.wk + (uint64_t)tile * kvm_ktile_bytes(KVM_TYPE_Q8_0, D);
    if (FAST && k16_ok<D>(nh)) {
        // K rows: a wave takes RW rows (cell j, head h) at a time, one per lane group
        constexpr uint32_t LG = D / 16, RW = 64 / LG;
        const uint32_t lane = tid & 63u, grp = lane / LG, l = lane % LG;
        // row r = (cell j, head h), advanced by W RW rows a step without a division
        const uint32_t H = a.H, dj = W * RW / H, dh = W * RW % H;
        uint32_t j = (wave * RW + grp) / H, h = (wave * RW + grp) % H;
        uint32_t j0 = wave * RW / H, h0 = wave * RW % H;            // row r0
        for (uint32_t r0 = wave * RW; r0 < nrow; r0 += W * RW) {
            const bool live = r0 + grp < nrow;                         // past the rows: recompute r0, unwritten
            const uint32_t jj = live ? j : j0, hh = live ? h : h0;
            stage_k_row16<D>(lk + jj * rowK + hh * NB * kb, ktile + (uint64_t)hh * a.n_tiles * kvm_ktile_bytes(KVM_TYPE_Q8_0, D),
                             c0 + jj, lt + jj * nh, live, l, a.rc, a.k_q4 != 0);
            j += dj;
            h += dh;
            if (h >= H) {
                h -= H;
                ++j;
            }
            j0 += dj;
            h0 += dh;
            if (h0 >= H) {
                h0 -= H;
                ++j0;
            }
        }
    } else
    // K rows: wave w takes rows (cell j, head h) = r, r + NTH/64, ..., four at a time
    for (uint32_t r0 = wave; r0 < nrow; r0 += NR * W) {
        const uint8_t *src[NR];
        uint8_t *kt[NR];
        uint32_t cc[NR];
        const float2 *cs[NR];
        bool live[NR];
#pragma unroll
        for (uint32_t k = 0; k < NR; ++k) {
            const uint32_t r = r0 + k * W < nrow ? r0 + k * W : r0;    // past the rows: recompute r0, unwritten
            const uint32_t j = r / a.H, h = r % a.H;
            src[k] = lk + j * rowK + h * NB * kb;
            kt[k] = a.wk + ((uint64_t)h * a.n_tiles + tile) * kvm_ktile_bytes(KVM_TYPE_Q8_0, D);
            cc[k] = c0 + j;
            cs[k] = lt + j * nh;
            live[k] = r0 + k * W < nrow;
        }
        stage_k_rows<D, NR, KQ>(src, kt, cc, cs, live, a.rc, a.k_q4 != 0);
    }
    const uint32_t vtile = kvm_vtile_bytes(KVM_TYPE_Q4_0, D);
    if (src >= 0) {
        // a moved block's V: its gathered tiles, whole, by the first item of each
        // tile (an item of 32 tokens fills half a tile; the other half's item
        // skips V, its bytes come with this copy)
        if (c0 == 0) {
            const uint32_t per = vtile / 16;
            const uint8_t *mv = gv + (uint64_t)a.bt * rowK + (uint64_t)(t0 / 64) * vtile;
            for (uint32_t h = 0; h < a.H; ++h)
                copy16_dev<FAST, false>(a.wv + ((uint64_t)h * a.n_tiles + tile) * vtile, mv + (uint64_t)h * (a.bt / 64) * vtile,
                                        per, tid, NTH);
        }
    } else {
        // V nibbles: destination-driven, one 32-bit word (8 keys of one dim) per
        // step; the 8 byte reads of a word are unconditional (keys past the
        // item's rows read row 0 and are zeroed), so they are all in flight
        // together, and two words per thread per round
        constexpr uint32_t NKS = IT / 32;    // key halves of the tile this item fills
        constexpr uint32_t NW = (uint32_t)D * 4 * NKS;   // words per head
        auto word_at = [&](uint32_t wi) {
            const uint32_t h = wi / NW, r = wi % NW;
            const uint32_t X = r / NKS, ks = NKS == 2 ? (r & 1u) : c0 / 32;
            const uint32_t dd = (X >> 6) * 16 + (X & 15u), gg = (X & 63u) >> 4;
            const uint32_t b = dd / 32, e = dd % 32;
            const uint32_t byte = 2 + (e & 15u), shift = e < 16 ? 0u : 4u;
            uint32_t nb8[8];
#pragma unroll
            for (uint32_t j = 0; j < 8; ++j) {
                const uint32_t cj = 32 * ks + 8 * gg + j - c0;    // key within the item
                nb8[j] = lv[(cj < count ? cj : 0u) * rowV + h * NB * 18 + b * 18 + byte];
            }
            uint32_t word = 0;
#pragma unroll
            for (uint32_t j = 0; j < 8; ++j) {
                const uint32_t cj = 32 * ks + 8 * gg + j - c0;
                const uint32_t nib = cj < count ? (nb8[j] >> shift) & 15u : 0u;
                word |= nib << kvm_vq_nib_shift(j);
            }
            *(uint32_t *)(a.wv + ((uint64_t)h * a.n_tiles + tile) * vtile + kvm_vq_word(dd, gg, ks)) = word;
        };
        for (uint32_t wi = tid; wi < a.H * NW; wi += 2 * NTH) {
            word_at(wi);
            if (wi + NTH < a.H * NW) word_at(wi + NTH);
        }
        for (uint32_t si2 = tid; si2 < a.H * IT * NB; si2 += NTH) {
            const uint32_t h = si2 / (IT * NB), cj = (si2 / NB) % IT, b = si2 % NB;
            uint8_t *sd = a.wv + ((uint64_t)h * a.n_tiles + tile) * vtile + kvm_vd_off(D, c0 + cj, b);
            if (cj < count) {
                const uint8_t *blk = lv + cj * rowV + h * NB * 18 + b * 18;
                sd[0] = blk[0];
                sd[1] = blk[1];
            } else {
                sd[0] = 0;
                sd[1] = 0;
            }
        }
    }
    if (tid < IT) a.cell_pos[slot * a.bt + t0 + tid] = tid < count ? base + (int32_t)(t0 + tid) : -1;
    if (tt == 0 && tid == 0) {
        a.slot_block[slot] = id;
        a.slot_base[slot] = base;
        if (a.shadow_rows) a.shadow_rows[slot] = nt;
    }
}

// ---------------------------------------------------------------------------
// A lane's plan staged by G workgroups x = 0 .. G-1 of one launch
// ---------------------------------------------------------------------------
// A wait at a lane barrier polls at most `spin` times (s_sleep rounds of ~64
// cycles, about 0.1 s by default): every workgroup of the launch is resident
// (the grids never exceed what the CUs hold at once) and arrives without
// waiting on anything, so the wait ends unless workgroups cannot be scheduled;
// past the limit the selection's status says so (info[3] bit 16, and the
// state's status word KVM_WAIT_STAGE) and the workgroups empty their items'
// cells instead.

__device__ __forceinline__ uint32_t sync_load(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void sync_store(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool sync_wait(const uint32_t *p, uint32_t v, uint32_t spin) {
    for (uint32_t it = 0;; ++it) {
        if (it >= spin) return false;
        if (sync_load(p) == v) return true;
        __builtin_amdgcn_s_sleep(1);
    }
}

// Entries of the lane's plan to stage: none when the plan does not fit (status
// bits 0, over capacity, and 1, more blocks than slots) or was refused (bit 2:
// it would overwrite a slot's unharvested rows).
__device__ inline uint32_t stage_entries(const stage_args &a) {
    return (a.info[3] & 7u) != 0 ? 0u : a.info[2];
}

// Barrier of a lane's G workgroups (NTH threads each) at value v, through the
// lane's sync words (kvm_state::stage_sync): [0] the epoch, [1] the go flag,
// [2] the failure flag, [64 + x] workgroup x's arrival.  Every workgroup reads
// the epoch e before its first arrival of the launch and the launch's barriers
// take values e + 1, e + 2, ...; workgroup 0 stores the last one as the epoch
// (`last`) once every workgroup has arrived there, so no flag of an earlier
// launch (at most e) passes for one of this launch, also when the launch is
// replayed from a captured graph.  Every thread's writes before the barrier
// are acknowledged before the arrival; with `fences` they are also written
// back from the writer's L2 (release) and the caches are invalidated after the
// go flag (acquire, by one wave: the invalidation covers the CU's and the XCD's
// caches for every wave after the workgroup barrier).  Without `fences` the
// data crossing the barrier must be written and read device-coherently
// (kvm_st16_dev / kvm_ld16_dev).  False: the wait timed out.
template <int NTH>
__device__ bool lane_barrier(uint32_t *sync, uint32_t *status, uint32_t spin, uint32_t v, uint32_t x, uint32_t G,
                             bool last, bool fences) {
    __shared__ uint32_t s_ok;
    const uint32_t tid = threadIdx.x;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
        if (fences) __threadfence();
        sync_store(sync + 64 + x, v);
    }
    uint32_t ok = 1;
    if (x == 0) {
        for (uint32_t t = tid; t < G; t += NTH) ok &= sync_wait(sync + 64 + t, v, spin) ? 1u : 0u;
        ok = __syncthreads_and(ok);
        if (tid == 0) {
            if (!ok) sync_store(sync + 2, v);
            if (last) sync_store(sync, v);
            __threadfence();
            sync_store(sync + 1, v);
        }
    } else if (tid == 0) {
        ok = sync_wait(sync + 1, v, spin) && sync_load(sync + 2) != v;
        s_ok = ok;
    }
    if (fences && tid == 0) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    if (x != 0) ok = s_ok;
    if (!ok && tid == 0) atomicOr(status, (uint32_t)KVM_WAIT_STAGE);
    return ok != 0;
}

// An item whose plan could not be carried out: its cells are emptied and,
// once, its slot's map entry and shadow count, so attention never reads what
// the slot held before and the next plan restages it.
template <int IT>
__device__ void stage_void_item(const stage_args &a, uint32_t si, uint32_t tt) {
    const uint32_t slot = a.stage_slots[si], tid = threadIdx.x;
    if (tid < IT) a.cell_pos[slot * a.bt + tt * IT + tid] = -1;
    if (tt == 0 && tid == 0) {
        a.slot_block[slot] = 0xffffffffu;
        a.slot_base[slot] = -1;
        if (a.shadow_rows) a.shadow_rows[slot] = 0u;
        atomicOr(&a.info[3], 16u);
    }
}

// The lane's n_ent plan entries staged by workgroup x of G: the gather of the
// moving entries (x, x + G, ...) and a barrier at value v when any entry moves
// within the window, then items x, x + G, ... of IT tokens.  `last`: the
// gather barrier is the launch's last on these sync words.  No barrier
// follows the items.
template <int D, int NTH, int IT, bool FAST = true, int KQ = KVM_KQ_ANY>
__device__ void stage_plan(const stage_args &a, uint8_t *s_rows, uint32_t n_ent, uint32_t x, uint32_t G,
                           uint32_t v, bool last) {
    const uint32_t tps = a.bt / IT, n_items = n_ent * tps;
    bool ok = true, host_via = false;
    if (a.moves) {
        uint32_t any = 0;
        for (uint32_t si = threadIdx.x; si < n_ent; si += NTH) any |= a.stage_src[si] >= 0 ? 1u : 0u;
        if (__syncthreads_or(any)) {
            if (FAST) {
                host_via = stage_host_via<D>(a);
                stage_gather_split<D>(a, n_ent, x, G, threadIdx.x, NTH, host_via);
            } else {
                for (uint32_t si = x; si < n_ent; si += G) stage_gather_entry<D>(a, si, threadIdx.x, NTH);
            }
            ok = lane_barrier<NTH>(a.sync, a.status, a.spin, v, x, G, last, !FAST);
        }
    }
    for (uint32_t item = x; item < n_items; item += G) {
        if (ok) stagein_item<D, NTH, IT, FAST, KQ>(a, s_rows, item / tps, item % tps, host_via);
        else stage_void_item<IT>(a, item / tps, item % tps);
        __syncthreads();                 // LDS rows of this item read before the next overwrites them
    }
}

// Every lane's plan in one launch (blockIdx.y = lane): the lanes' windows,
// histories and plans are independent, so the workgroups of one lane never touch
// another lane's memory.
#define KVM_STAGEIN_LANES 8
struct stage_lanes {
    stage_args lane[KVM_STAGEIN_LANES];
};

// Checks every lane and fills the kernel arguments (kvm_stagein.hip): the rope
// table covers the largest window; *max_items = the most (slot, tile) items of
// a lane, *lds = the rows buffer for the largest lane.
int kvm_stage_prepare(kvm_state *st, const kvm_stagein_lane *lanes, uint32_t n_lanes,
                      const kvm_rope_params *rope, stage_lanes *sl, uint32_t *max_items, size_t *lds);
// Launches the stage-in kernel over prepared lanes (kvm_stagein.hip).
int kvm_stage_launch(kvm_state *st, const stage_lanes &sl, uint32_t n_lanes, uint32_t max_items, size_t lds,
                     uint32_t head_dim);
