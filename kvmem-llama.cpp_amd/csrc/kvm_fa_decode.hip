// kvm_fa_decode.hip -- flash attention over the tiled window for decode and
// MTP-verify widths (<= 32 query rows per kv head).
//
// Semantics follow ggml's flash_attn_ext for a q8_0 K / q4_0 V cache (as called
// by build_attn, patches/0002-attn-qk-capture-hook.patch:225,256): the query row
// is quantised to q8_0 per 32 dims exactly as ggml's vec_dot path does, the
// Q.K dot of each 32-dim block is an exact integer sum scaled by d_k * d_q in
// fp32, the softmax is online in fp32, and V is dequantised to fp16.  For an
// f16/f16 cache Q is rounded to fp16 and Q.K is an fp16 dot with fp32
// accumulation.
//
// Work split (gfx950, wave64, 4 waves per workgroup; one workgroup per
// (lane, kv head, key split)):
//   phase 1: wave w scores keys 16w..16w+15 of the 64-cell tile against all
//            rows with v_mfma_i32_16x16x32_i8 (one MFMA per 32-dim block and
//            16-row tile, then the per-block scale), masks by cell position
//            and reduces the row max; the four waves exchange maxima in LDS.
//   phase 2: wave w accumulates O[:, dims of quarter w] += P V with
//            v_mfma_f32_16x16x32_f16; the q4_0 block scale of V is folded
//            into P so V enters the MFMA as exact integers (nibble - 8).
// Partial (m, l, O) of each split go to a workspace and k_fa_combine merges them.
#include "kvm_internal.h"

#include <cmath>
#include <cstdlib>

#define KVM_MAX_LANES 8

struct fa_lane {
    const uint8_t *wk;
    const uint8_t *wv;
    const int32_t *cell_pos;
    const void *q;
    const int32_t *q_pos;
    float *out;
    uint32_t n_tiles;
    uint32_t n_tokens;
};

struct fa_args {
    fa_lane lanes[KVM_MAX_LANES];
    float *ws;              // partial O  [lane][H][split][RMAX][D]
    float *ws_ml;           // partial m,l [lane][H][split][RMAX][2]
    uint32_t H, G, n_head, n_splits;
    float scale_log2;       // kq_scale * log2(e)
    int q_bf16;
};

__device__ inline float load_q(const void *q, uint64_t i, int bf16) {
    return bf16 ? kvm_bf2f(((const uint16_t *)q)[i]) : ((const float *)q)[i];
}

// 8 q4_0 nibbles (keys j = 0..7, low nibble first) -> 8 fp16 values nibble - 8.
// (0x6400 | n) is the fp16 1024 + n; subtracting 1032 is exact.
__device__ inline kvm_f16x8 nib8_to_f16(uint32_t w) {
    const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
    uint32_t r[4];
    r[0] = __builtin_amdgcn_perm(hi, lo, 0x0c040c00u) | 0x64006400u;
    r[1] = __builtin_amdgcn_perm(hi, lo, 0x0c050c01u) | 0x64006400u;
    r[2] = __builtin_amdgcn_perm(hi, lo, 0x0c060c02u) | 0x64006400u;
    r[3] = __builtin_amdgcn_perm(hi, lo, 0x0c070c03u) | 0x64006400u;
    kvm_f16x8 v;
    __builtin_memcpy(&v, r, 16);
    const kvm_f16x8 off = {(_Float16)1032.0f, (_Float16)1032.0f, (_Float16)1032.0f, (_Float16)1032.0f,
                           (_Float16)1032.0f, (_Float16)1032.0f, (_Float16)1032.0f, (_Float16)1032.0f};
    return v - off;
}

template <int D, int NRT, bool QUANT>
__global__ void __launch_bounds__(256) k_fa_decode(fa_args a) {
    constexpr int NB = D / 32;          // 32-dim blocks per row
    constexpr int RMAX = 16 * NRT;      // padded query rows
    constexpr int DW = D / 4;           // output dims per wave
    constexpr int NT = DW / 16;         // 16-dim output tiles per wave
    constexpr uint32_t KTILE = QUANT ? 64u * D + 64u * NB * 2u : 64u * D * 2u;
    constexpr uint32_t VTILE = QUANT ? D * 32u + NB * 64u * 2u : 64u * D * 2u;
    constexpr int PSTR = 64 + 8;        // padded fp16 row stride of P in LDS

    const fa_lane ln = a.lanes[blockIdx.z];
    const uint32_t h = blockIdx.y, split = blockIdx.x;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 4, m = l & 15;
    const int R = (int)(ln.n_tokens * a.G);
    const uint32_t tps = (ln.n_tiles + a.n_splits - 1) / a.n_splits;
    const uint32_t t_begin = split * tps;
    const uint32_t t_end = t_begin + tps < ln.n_tiles ? t_begin + tps : ln.n_tiles;

    __shared__ __align__(16) int8_t s_qq[QUANT ? RMAX : 1][D];
    __shared__ __align__(16) _Float16 s_qh[QUANT ? 1 : RMAX][D];
    __shared__ float s_dq[RMAX][NB];
    __shared__ int32_t s_qpos[RMAX];
    __shared__ float s_max[4][RMAX];
    __shared__ float s_alpha[RMAX];
    __shared__ float s_l[4][RMAX];
    __shared__ __align__(16) _Float16 s_p[RMAX][PSTR];

    // ---- query rows of this kv head: row r = token r/G, query head h*G + r%G
    for (int idx = tid; idx < RMAX * NB; idx += 256) {
        const int r = idx / NB, b = idx % NB;
        float x[32];
        if (r < R) {
            const uint64_t base = ((uint64_t)(r / a.G) * a.n_head + h * a.G + r % a.G) * D + 32 * b;
#pragma unroll
            for (int j = 0; j < 32; ++j) x[j] = load_q(ln.q, base + j, a.q_bf16);
        } else {
#pragma unroll
            for (int j = 0; j < 32; ++j) x[j] = 0.0f;
        }
        if constexpr (QUANT) {
            uint16_t d16;
            kvm_quant_block_q8_0(x, &d16, &s_qq[r][32 * b]);
            s_dq[r][b] = kvm_h2f(d16);
        } else {
#pragma unroll
            for (int j = 0; j < 32; ++j) s_qh[r][32 * b + j] = (_Float16)x[j];
        }
    }
    if (tid < RMAX) s_qpos[tid] = tid < R ? ln.q_pos[tid / a.G] : -1;
    __syncthreads();

    // B operands (Q^T): lane (row m of row-tile rt, k-group g)
    long qop_i[QUANT ? NRT : 1][QUANT ? NB : 1];
    kvm_f16x8 qop_h[QUANT ? 1 : NRT][QUANT ? 1 : NB];
    float dqv[QUANT ? NRT : 1][QUANT ? NB : 1];
    int32_t qp[NRT];
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
        qp[rt] = s_qpos[16 * rt + m];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if constexpr (QUANT) {
                __builtin_memcpy(&qop_i[rt][b], &s_qq[16 * rt + m][32 * b + 8 * g], 8);
                dqv[rt][b] = s_dq[16 * rt + m][b];
            } else {
                __builtin_memcpy(&qop_h[rt][b], &s_qh[16 * rt + m][32 * b + 8 * g], 16);
            }
        }
    }

    kvm_f32x4 O[NRT][NT];
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) O[rt][nt] = {0.f, 0.f, 0.f, 0.f};
    float m_run[NRT], l_run[NRT];
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) { m_run[rt] = -INFINITY; l_run[rt] = 0.0f; }

    for (uint32_t T = t_begin; T < t_end; ++T) {
        const uint8_t *kt = ln.wk + ((uint64_t)h * ln.n_tiles + T) * KTILE;
        const uint8_t *vt = ln.wv + ((uint64_t)h * ln.n_tiles + T) * VTILE;
        // ---------------- phase 1: scores of keys 16w + 4g + i -----------------
        const int4 cp = *(const int4 *)(ln.cell_pos + (uint64_t)T * 64 + 16 * w + 4 * g);
        float s[NRT][4];
        if constexpr (QUANT) {
            uint4 ka[NB / 2];
#pragma unroll
            for (int p = 0; p < NB / 2; ++p)
                ka[p] = *(const uint4 *)(kt + (((w * (NB / 2) + p) * 64 + l) << 4));
            uint2 dkr[NB];
            const uint8_t *kd = kt + 64u * D + (((w * 4 + g) * NB) << 3);
#pragma unroll
            for (int b = 0; b < NB; ++b) dkr[b] = *(const uint2 *)(kd + 8 * b);
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
                for (int i = 0; i < 4; ++i) s[rt][i] = 0.0f;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                long av;
                const uint32_t *kw = (const uint32_t *)&ka[b >> 1];
                const uint64_t lo32 = kw[(b & 1) * 2], hi32 = kw[(b & 1) * 2 + 1];
                av = (long)(lo32 | (hi32 << 32));
                float dk[4];
                dk[0] = kvm_h2f((uint16_t)(dkr[b].x & 0xffffu));
                dk[1] = kvm_h2f((uint16_t)(dkr[b].x >> 16));
                dk[2] = kvm_h2f((uint16_t)(dkr[b].y & 0xffffu));
                dk[3] = kvm_h2f((uint16_t)(dkr[b].y >> 16));
#pragma unroll
                for (int rt = 0; rt < NRT; ++rt) {
                    const kvm_i32x4 c = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, qop_i[rt][b],
                                                                             kvm_i32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) s[rt][i] += (float)c[i] * (dk[i] * dqv[rt][b]);
                }
            }
        } else {
            kvm_f32x4 acc[NRT];
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt) acc[rt] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < NB; ++ks) {
                kvm_f16x8 av;
                __builtin_memcpy(&av, kt + (((w * NB + ks) * 64 + l) << 4), 16);
#pragma unroll
                for (int rt = 0; rt < NRT; ++rt)
                    acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, qop_h[rt][ks], acc[rt], 0, 0, 0);
            }
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
                for (int i = 0; i < 4; ++i) s[rt][i] = acc[rt][i];
        }
        const int32_t cpos[4] = {cp.x, cp.y, cp.z, cp.w};
        float mx[NRT];
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
            mx[rt] = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool vis = cpos[i] >= 0 && cpos[i] <= qp[rt];
                s[rt][i] = vis ? s[rt][i] * a.scale_log2 : -INFINITY;
                mx[rt] = fmaxf(mx[rt], s[rt][i]);
            }
            mx[rt] = fmaxf(mx[rt], __shfl_xor(mx[rt], 16, 64));
            mx[rt] = fmaxf(mx[rt], __shfl_xor(mx[rt], 32, 64));
            if (g == 0) s_max[w][16 * rt + m] = mx[rt];
        }
        __syncthreads();
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
            const int row = 16 * rt + m;
            const float tm = fmaxf(fmaxf(s_max[0][row], s_max[1][row]), fmaxf(s_max[2][row], s_max[3][row]));
            const float mn = fmaxf(m_run[rt], tm);
            const float alpha = mn == -INFINITY ? 1.0f : exp2f(m_run[rt] - mn);
            float psum = 0.0f;
            _Float16 ph[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p = mn == -INFINITY ? 0.0f : exp2f(s[rt][i] - mn);
                const _Float16 p16 = (_Float16)p;
                ph[i] = p16;
                psum += (float)p16;
            }
            l_run[rt] = l_run[rt] * alpha + psum;
            m_run[rt] = mn;
            __builtin_memcpy(&s_p[row][16 * w + 4 * g], ph, 8);
            if (w == 0 && g == 0) s_alpha[row] = alpha;
        }
        __syncthreads();
        // ---------------- phase 2: O[:, quarter w] += P V ----------------------
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
            float ar[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) ar[r] = s_alpha[16 * rt + 4 * g + r];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int r = 0; r < 4; ++r) O[rt][nt][r] *= ar[r];
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            kvm_f16x8 pa[NRT];
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt)
                __builtin_memcpy(&pa[rt], &s_p[16 * rt + m][32 * ks + 8 * g], 16);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int n = DW * w + 16 * nt + m;
                kvm_f16x8 vb;
                if constexpr (QUANT) {
                    const uint32_t nib = *(const uint32_t *)(vt + n * 32 + 4 * (2 * g + ks));
                    vb = nib8_to_f16(nib);
                    const int b = (DW * w + 16 * nt) / 32;
                    kvm_f16x8 dv;
                    __builtin_memcpy(&dv, vt + D * 32 + ((((b * 2 + ks) * 4 + g) * 8) << 1), 16);
#pragma unroll
                    for (int rt = 0; rt < NRT; ++rt) {
                        const kvm_f16x8 pp = pa[rt] * dv;
                        O[rt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pp, vb, O[rt][nt], 0, 0, 0);
                    }
                } else {
                    __builtin_memcpy(&vb, vt + ((n * 64 + 8 * (2 * g + ks)) << 1), 16);
#pragma unroll
                    for (int rt = 0; rt < NRT; ++rt)
                        O[rt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[rt], vb, O[rt][nt], 0, 0, 0);
                }
            }
        }
    }

    // ---- partial results of this split
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
        float lr = l_run[rt];
        lr += __shfl_xor(lr, 16, 64);
        lr += __shfl_xor(lr, 32, 64);
        if (g == 0) s_l[w][16 * rt + m] = lr;
    }
    __syncthreads();
    const uint64_t pidx = ((uint64_t)blockIdx.z * a.H + h) * a.n_splits + split;
    float *po = a.ws + pidx * RMAX * D;
    if (w == 0 && g == 0) {
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
            const int row = 16 * rt + m;
            if (row < R) {
                a.ws_ml[(pidx * RMAX + row) * 2 + 0] = m_run[rt];
                a.ws_ml[(pidx * RMAX + row) * 2 + 1] = s_l[0][row] + s_l[1][row] + s_l[2][row] + s_l[3][row];
            }
        }
    }
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 16 * rt + 4 * g + r;
                if (row < R) po[row * D + DW * w + 16 * nt + m] = O[rt][nt][r];
            }
}

// Merge the splits of one (lane, kv head, row): thread = output dim.  The split
// maxima / sums are reduced first; then every thread issues its loads of 32
// splits at once, so the merge streams the partials instead of paying one
// memory latency per split.
#define KVM_MAX_SPLITS 512
template <int D>
__global__ void __launch_bounds__(D) k_fa_combine(fa_args a, int rmax) {
    __shared__ float s_w[KVM_MAX_SPLITS];
    __shared__ float s_red[D / 64];
    const fa_lane ln = a.lanes[blockIdx.z];
    const uint32_t h = blockIdx.y, row = blockIdx.x;
    const uint32_t R = ln.n_tokens * a.G;
    if (row >= R) return;
    const uint32_t d = threadIdx.x, S = a.n_splits;
    const uint64_t p0 = ((uint64_t)blockIdx.z * a.H + h) * S;
    const float *ml = a.ws_ml + (p0 * rmax + row) * 2;
    const uint64_t mstride = (uint64_t)rmax * 2;
    float mloc = -INFINITY;
    for (uint32_t s = d; s < S; s += D) {
        const float m = ml[s * mstride];
        s_w[s] = m;
        mloc = fmaxf(mloc, m);
    }
    for (int o = 32; o > 0; o >>= 1) mloc = fmaxf(mloc, __shfl_xor(mloc, o, 64));
    if ((d & 63) == 0) s_red[d >> 6] = mloc;
    __syncthreads();
    float M = s_red[0];
#pragma unroll
    for (int w = 1; w < D / 64; ++w) M = fmaxf(M, s_red[w]);
    const uint32_t t = row / a.G, qh = h * a.G + row % a.G;
    float *out = ln.out + ((uint64_t)t * a.n_head + qh) * D + d;
    if (M == -INFINITY) {                     // no visible cell for this row
        *out = 0.0f;
        return;
    }
    float lloc = 0.0f;
    for (uint32_t s = d; s < S; s += D) {
        const float m = s_w[s];
        const float wgt = m == -INFINITY ? 0.0f : exp2f(m - M);
        s_w[s] = wgt;
        lloc += ml[s * mstride + 1] * wgt;
    }
    for (int o = 32; o > 0; o >>= 1) lloc += __shfl_xor(lloc, o, 64);
    __syncthreads();
    if ((d & 63) == 0) s_red[d >> 6] = lloc;
    __syncthreads();
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < D / 64; ++w) L += s_red[w];
    const float *po = a.ws + (p0 * rmax + row) * D + d;
    const uint64_t ostride = (uint64_t)rmax * D;
    float acc = 0.0f;
    for (uint32_t s0 = 0; s0 < S; s0 += 32) {
        float v[32];
#pragma unroll
        for (int j = 0; j < 32; ++j) v[j] = s0 + j < S ? po[(s0 + j) * ostride] : 0.0f;
#pragma unroll
        for (int j = 0; j < 32; ++j) acc += s0 + j < S ? v[j] * s_w[s0 + j] : 0.0f;
    }
    *out = L > 0.0f ? acc / L : 0.0f;
}

static uint32_t choose_splits(uint32_t n_lanes, uint32_t H, uint32_t n_tiles) {
    if (const char *e = getenv("KVM_FA_SPLITS")) {
        uint32_t v = (uint32_t)atoi(e);
        if (v > KVM_MAX_SPLITS) v = KVM_MAX_SPLITS;
        if (v > 0) return v < n_tiles ? v : n_tiles;
    }
    // about 2 workgroups per CU on a 256-CU device
    uint32_t s = (512 + n_lanes * H - 1) / (n_lanes * H);
    if (s < 1) s = 1;
    if (s > KVM_MAX_SPLITS) s = KVM_MAX_SPLITS;
    return s < n_tiles ? s : n_tiles;
}

template <int D, int NRT, bool QUANT>
static void launch_decode(const fa_args &a, uint32_t n_lanes, hipStream_t stream) {
    hipLaunchKernelGGL((k_fa_decode<D, NRT, QUANT>), dim3(a.n_splits, a.H, n_lanes), dim3(256), 0, stream, a);
}

static int fa_decode_impl(kvm_state *st, const kvm_lane *lanes, uint32_t n_lanes, int q_type,
                          uint32_t n_head, float scale) {
    if (!st || !lanes || n_lanes == 0) return kvm_fail(st, KVM_EINVAL, "fa_decode: no lanes");
    if (n_lanes > KVM_MAX_LANES) return kvm_fail(st, KVM_ERANGE, "fa_decode: %u lanes > %d", n_lanes, KVM_MAX_LANES);
    if (q_type != KVM_TYPE_F32 && q_type != KVM_TYPE_BF16) return kvm_fail(st, KVM_EUNSUPPORTED, "fa_decode: q type %d", q_type);
    const kvm_window *w0 = lanes[0].w;
    if (!w0) return kvm_fail(st, KVM_EINVAL, "fa_decode: null window");
    uint32_t max_rows = 0, max_tiles = 0;
    fa_args a{};
    for (uint32_t i = 0; i < n_lanes; ++i) {
        const kvm_lane &L = lanes[i];
        int rc = kvm_window_check(L.w);
        if (rc) return kvm_fail(st, rc, "fa_decode: lane %u: bad window", i);
        if (L.w->head_dim != w0->head_dim || L.w->n_head_kv != w0->n_head_kv || L.w->k_type != w0->k_type)
            return kvm_fail(st, KVM_EINVAL, "fa_decode: lanes differ in shape");
        if (!L.q || !L.q_pos || !L.out) return kvm_fail(st, KVM_EINVAL, "fa_decode: lane %u: null buffer", i);
        if (n_head % L.w->n_head_kv) return kvm_fail(st, KVM_EINVAL, "fa_decode: n_head %u not a multiple of n_head_kv %u", n_head, L.w->n_head_kv);
        const uint32_t rows = L.n_tokens * (n_head / L.w->n_head_kv);
        if (rows > 32) return kvm_fail(st, KVM_ERANGE, "fa_decode: %u rows per kv head > 32 (use kvm_fa_prefill)", rows);
        max_rows = rows > max_rows ? rows : max_rows;
        const uint32_t nt = L.w->n_cells / 64;
        max_tiles = nt > max_tiles ? nt : max_tiles;
        a.lanes[i] = fa_lane{(const uint8_t *)L.w->k, (const uint8_t *)L.w->v, L.w->cell_pos, L.q, L.q_pos, L.out, nt, L.n_tokens};
    }
    if (max_rows == 0) return KVM_OK;
    const uint32_t D = w0->head_dim, H = w0->n_head_kv;
    const int NRT = max_rows <= 16 ? 1 : 2;
    const uint32_t rmax = 16u * NRT;
    a.H = H;
    a.G = n_head / H;
    a.n_head = n_head;
    a.n_splits = choose_splits(n_lanes, H, max_tiles);
    a.scale_log2 = scale * 1.4426950408889634f;
    a.q_bf16 = q_type == KVM_TYPE_BF16;
    const size_t n_part = (size_t)n_lanes * H * a.n_splits * rmax;
    float *ws = (float *)kvm_workspace(st, n_part * (D + 2) * sizeof(float));
    if (!ws) return kvm_fail(st, KVM_ENOMEM, "fa_decode: workspace of %zu bytes", n_part * (D + 2) * 4);
    a.ws = ws;
    a.ws_ml = ws + n_part * D;
    KVM_HIP(st, hipSetDevice(st->device));
    const bool quant = w0->k_type == KVM_TYPE_Q8_0;
    if (D == 256) {
        if (quant) { if (NRT == 1) launch_decode<256, 1, true>(a, n_lanes, st->stream); else launch_decode<256, 2, true>(a, n_lanes, st->stream); }
        else       { if (NRT == 1) launch_decode<256, 1, false>(a, n_lanes, st->stream); else launch_decode<256, 2, false>(a, n_lanes, st->stream); }
    } else {
        if (quant) { if (NRT == 1) launch_decode<128, 1, true>(a, n_lanes, st->stream); else launch_decode<128, 2, true>(a, n_lanes, st->stream); }
        else       { if (NRT == 1) launch_decode<128, 1, false>(a, n_lanes, st->stream); else launch_decode<128, 2, false>(a, n_lanes, st->stream); }
    }
    KVM_LAUNCH_CHECK(st, "fa_decode");
    if (D == 256)
        hipLaunchKernelGGL(k_fa_combine<256>, dim3(rmax, H, n_lanes), dim3(256), 0, st->stream, a, (int)rmax);
    else
        hipLaunchKernelGGL(k_fa_combine<128>, dim3(rmax, H, n_lanes), dim3(128), 0, st->stream, a, (int)rmax);
    KVM_LAUNCH_CHECK(st, "fa_combine");
    return KVM_OK;
}

extern "C" int kvm_fa_decode(kvm_state *st, const kvm_window *w, const void *q, int q_type,
                             const int32_t *q_pos, uint32_t n_tokens, uint32_t n_head, float scale,
                             float *out) {
    kvm_lane lane{w, q, q_pos, out, n_tokens};
    return fa_decode_impl(st, &lane, 1, q_type, n_head, scale);
}

extern "C" int kvm_fa_decode_lanes(kvm_state *st, const kvm_lane *lanes, uint32_t n_lanes, int q_type,
                                   uint32_t n_head, float scale) {
    return fa_decode_impl(st, lanes, n_lanes, q_type, n_head, scale);
}

// Chunked prefill through the decode kernel: the query tokens are processed in
// groups whose rows per kv head fit the decode tile.  Correct for any width;
// the dense-tile MFMA kernel in kvm_fa_prefill.hip takes over for long chunks.
extern "C" int kvm_fa_prefill_chunked(kvm_state *st, const kvm_window *w, const void *q, int q_type,
                                      const int32_t *q_pos, uint32_t n_tokens, uint32_t n_head,
                                      float scale, float *out) {
    if (!st || !w || !q || !q_pos || !out) return kvm_fail(st, KVM_EINVAL, "fa_prefill: null argument");
    if (!w->n_head_kv || n_head % w->n_head_kv) return kvm_fail(st, KVM_EINVAL, "fa_prefill: head counts");
    const uint32_t G = n_head / w->n_head_kv;
    if (G > 32) return kvm_fail(st, KVM_ERANGE, "fa_prefill: %u query heads per kv head", G);
    const uint32_t per = 32 / G;
    const size_t qel = q_type == KVM_TYPE_BF16 ? 2 : 4;
    for (uint32_t t0 = 0; t0 < n_tokens; t0 += per) {
        const uint32_t nt = n_tokens - t0 < per ? n_tokens - t0 : per;
        const size_t off = (size_t)t0 * n_head * w->head_dim;
        kvm_lane lane{w, (const uint8_t *)q + off * qel, q_pos + t0, out + off, nt};
        const int rc = fa_decode_impl(st, &lane, 1, q_type, n_head, scale);
        if (rc) return rc;
    }
    return KVM_OK;
}
