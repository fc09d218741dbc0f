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
// One launch per call: one workgroup of 8 waves per (lane, kv head, key
// split); every wave loads its own operands of each 64-cell tile straight from
// HBM into registers, three buffers, two tiles in flight:
//   waves 0-3 score: wave kq takes keys 16kq..16kq+15 of the tile against all
//     padded query rows with v_mfma_i32_16x16x32_i8 (one MFMA per 32-dim block
//     and row tile; a last row tile of at most 8 rows takes two blocks per
//     v_mfma_i32_16x16x64_i8; the d_k*d_q products of four blocks come from one
//     v_mfma_f32_16x16x1_4b_f32 outer product), masks by cell position and
//     writes P (fp16) of its keys to LDS, keeping the online softmax state;
//   waves 4-7 accumulate: wave 4+dq takes O[:, dims D/4*dq ..] += P V with
//     v_mfma_f32_16x16x32_f16; the q4_0 block scale is folded into P and V
//     enters the MFMA as exact fp16 denormals (nibble * 2^-24).
// One barrier per tile: the scoring waves score tile t+1 while the P V waves
// multiply tile t.  The query is quantised by all 8 waves at the start.  Each
// split writes its partial (m, l, O) device-coherently and raises its flag
// with this launch's epoch; splits 0 .. NM-1 of a head then wait for the
// head's flags and each merges whole rows (or row chunks) of the head, so no
// combine launch follows.
//
// Two further forms of the same launch: the staged one first carries out the
// lanes' stage-in plans (its workgroups meet at in-launch barriers before any
// reads the window), and the selecting one adds a column of workgroups whose
// first runs the lane's top-k and layout while the others attend over the
// window as it is, then stage the plan and attend again only if it changed
// anything.  With the scoring grid before it, a decode step is two launches.
#include "kvm_stagein_dev.h"
#include "kvm_topk_dev.h"

#include <cmath>
#include <cstdlib>
#include <atomic>
#include <mutex>

#define KVM_FA_STAGE_IT 32        // tokens per stage-in item of a staged launch

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
    uint32_t *sync;         // [lane][64][512] by (lane, head, split): the epoch of the last launch that completed
                            // the split's partials; sync[KVM_FA_SYNC_STATUS]: KVM_WAIT_MERGE =
                            // a merge wait gave up, KVM_WAIT_PLAN = a wait for the plan gave up;
                            // sync[KVM_FA_SYNC_EPOCH + lane * 64 + h]: the (lane, head)'s
                            // epoch, one less than its next launch's; 64-bit words from
                            // KVM_FA_SYNC_PLAN, [lane * 64 + h]: the plan a selecting launch
                            // published to the head (epoch, entries to stage)
    uint32_t H, G, n_head, n_splits;
    uint32_t spin;          // polls of a wait before it gives up (0: at once, without a look)
    float scale_log2;       // kq_scale * log2(e)
    int q_bf16;
};

__device__ inline float load_q(const void *q, uint64_t i, int bf16) {
    return bf16 ? kvm_bf2f(((const uint16_t *)q)[i]) : ((const float *)q)[i];
}

// 8 q4_0 nibbles of one word (key j in byte j%4, high nibble for j >= 4) ->
// 8 fp16 denormals n * 2^-24 in key order (each v_perm puts a nibble byte
// under a zero high byte).  The matrix cores take fp16 denormals exactly; the
// "- 8" of q4_0 and the 2^24 are applied to the accumulated sums (see
// k_fa_decode), so no per-element subtraction is needed.
__device__ inline kvm_f16x8 nib8_to_f16den(uint32_t w) {
    const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
    uint32_t r[4];
    r[0] = __builtin_amdgcn_perm(0u, lo, 0x04010400u);
    r[1] = __builtin_amdgcn_perm(0u, lo, 0x04030402u);
    r[2] = __builtin_amdgcn_perm(0u, hi, 0x04010400u);
    r[3] = __builtin_amdgcn_perm(0u, hi, 0x04030402u);
    kvm_f16x8 v;
    __builtin_memcpy(&v, r, 16);
    return v;
}

// Running maximum of a row before any visible key: finite, so exp2(s - m)
// needs no guard (a visible key always moves it, see k_fa_decode).
#define KVM_M_NONE (-1.0e30f)

typedef float kvm_f32x16 __attribute__((ext_vector_type(16)));


// A row's running maximum moves only when a tile raises it by more than
// 2^KVM_LAZY_MAX (log2 domain), so most tiles skip rescaling O; probabilities
// stay below 2^KVM_LAZY_MAX, well inside fp16.
#define KVM_LAZY_MAX 8.0f

// Register buffers per wave for the tile operands: two tiles in flight (a
// third in flight measured no faster on the 24-row, 32K-cell workload).
#define KVM_FA_NBUF 3

// Operands of one 64-cell tile, loaded straight from HBM into registers in
// MFMA operand order (the window's tile layout is built for this).
// Scoring wave kq (keys 16kq..16kq+15): K quants of key 16kq+m (lane l = 16g+m
// holds dims 32b+8g..+7 of every block b), the fp16 scales of key 16kq+m for
// blocks 4gi+g (q8_0) and, for a packed row tile, for blocks 2g and 2g+1;
// positions of keys 16kq+4g..+3.
template <int D, bool QUANT, bool PK>
struct fa_k_regs {
    static constexpr int NB = D / 32;
    kvm_u32x4 k[QUANT ? NB / 2 : NB];     // q8_0: 2 blocks per 16 B; f16: one k-step
    uint32_t dk[QUANT ? NB / 4 : 1];      // fp16 scale (low half)
    uint32_t dkp[2];                      // packed row tile: scales of blocks 2g, 2g+1
    kvm_u32x4 cp;                          // 4 cell positions
};
// P V wave dq (dims D/4*dq ..): q4_0 nibble words of dims D/4*dq+16nt+m for
// keys 32ks+8g..+7 and the V scales of those keys per 32-dim block, or f16 V.
template <int D, bool QUANT, int NT, int NBW>
struct fa_v_regs {
    kvm_u32x2 vq[QUANT ? NT : 1];          // both ks nibble words
    kvm_u32x4 vs[QUANT ? NBW : 1][2];      // V scales [block][ks]
    kvm_u32x4 vh[QUANT ? 1 : NT][2];       // f16 V [ks]
};

// Split partials are written and read device-coherently (relaxed atomics at
// agent scope): the merging workgroup may run on another XCD, whose L2 holds no
// copy of them, and may hold a stale one from an earlier launch.
__device__ __forceinline__ void fa_store(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float fa_load(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A merging workgroup waits for the other splits' flags for at most a.spin
// polls (s_sleep rounds of ~128 cycles each; about 0.2 s by default): every
// split raises its flag without waiting on anything, so the wait ends unless
// workgroups cannot be scheduled; past the limit the status word says so
// (KVM_WAIT_MERGE) and the rows are left unmerged.
#define KVM_FA_POLL_WORDS 2048

// Merge units j, j + nm, ... of (lane blockIdx.z, head h): unit u is row
// u / dc, dims (u % dc) * D / dc .. + D / dc, over the S split partials:
// M = max_s m_s, w_s = exp2(m_s - M), out = sum_s w_s O_s / sum_s w_s l_s
// (zeros when no split saw a visible cell).  512 threads: thread t accumulates
// dim t % UD of the unit (UD = D / dc) over the splits s = t / UD (mod 512 /
// UD), whose partial outputs it loads in batches of NBAT before using any
// (NBAT: the smallest of 4, 8, 16, 32 that covers the thread's splits, so one
// batch, one memory round trip, serves the usual shapes).  Wave 0 loads (m, l) of splits t, t + 64, ... ahead of its first
// batch, reduces them within the wave and publishes the weights and
// 1 / sum_s w_s l_s while the other waves' partial outputs are still in flight
// (one memory round trip per unit, two barriers after it); the 512 / UD sums
// are then added in split-phase order.
struct fa_merge_lds {
    float w[KVM_MAX_SPLITS + 1];          // weights; [KVM_MAX_SPLITS] stays 0: splits past the last
    float acc[512];
    float inv;
    uint32_t ok;
};
template <int D, int RMAX, int NBAT>
__device__ __forceinline__ void fa_merge(const fa_args &a, const fa_lane &ln, uint32_t h, const uint32_t *flags,
                                         uint32_t n_flags, uint32_t epoch, uint32_t j, uint32_t nm, uint32_t dc,
                                         int R, fa_merge_lds &L_) {
    float *const s_w = L_.w, *const s_acc = L_.acc;
    float &s_inv = L_.inv;
    uint32_t &s_ok = L_.ok;
    const uint32_t tid = threadIdx.x, S = a.n_splits;
    // thread t < n_flags waits for flag t (the splits', and in a selecting
    // launch the selector column's at S; device-coherent polling, no cache
    // invalidation); the partials are then read device-coherently as well
    uint32_t ok = 1;
    if (tid < n_flags) {
        for (uint32_t it = 0;; ++it) {
            if (it >= a.spin) {
                __hip_atomic_fetch_or(a.sync + KVM_FA_SYNC_STATUS, (uint32_t)KVM_WAIT_MERGE, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
                ok = 0;
                break;
            }
            if (__hip_atomic_load(flags + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == epoch) break;
            __builtin_amdgcn_s_sleep(2);
        }
    }
    if (tid == 0) {
        s_ok = 1;
        s_w[KVM_MAX_SPLITS] = 0.0f;
    }
    __syncthreads();
    if (!ok) s_ok = 0;
    __syncthreads();
    // every workgroup of the head has read the head's epoch (each raised its
    // flag after reading it): the next launch may take the next one
    if (j == 0 && tid == 0)
        __hip_atomic_store(a.sync + KVM_FA_SYNC_EPOCH + blockIdx.z * KVM_FA_MAX_HEADS + h, epoch, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t p0 = ((uint64_t)blockIdx.z * a.H + h) * S;
    const uint32_t UD = D / dc, SP = 512 / UD;
    if (s_ok) {
        const uint32_t dd = tid % UD, sp = tid / UD;
        for (uint32_t u = j; u < (uint32_t)R * dc; u += nm) {
            const uint32_t row = u / dc, d = (u % dc) * UD + dd;
            const float *ml = a.ws_ml + (p0 * RMAX + row) * 2;
            // every load unconditional within its wave (a conditional load makes
            // the compiler wait for all loads in flight at the join): splits
            // past S re-read split S - 1 and get weight 0
            const float *po = a.ws + (p0 * RMAX + row) * D + d;
            auto ld = [&](uint32_t s) { return fa_load(po + (uint64_t)(s < S ? s : S - 1) * RMAX * D); };
            float m0 = 0.0f, l0 = 0.0f;
            if (tid < 64) {
                const uint32_t sc = tid < S ? tid : S - 1;
                m0 = fa_load(ml + (uint64_t)sc * RMAX * 2);
                l0 = fa_load(ml + (uint64_t)sc * RMAX * 2 + 1);
            }
            float v[NBAT];
#pragma unroll
            for (int i = 0; i < NBAT; ++i) v[i] = ld(sp + SP * i);
            if (tid < 64) {
                // the lane's splits tid, tid + 64, ...: running maximum and sum,
                // the maxima kept in s_w until the weights replace them
                float m_l = tid < S ? m0 : -INFINITY, l_l = tid < S ? l0 : 0.0f;
                s_w[tid] = m_l;
                for (uint32_t s = tid + 64; s < S; s += 64) {
                    const float ms = fa_load(ml + (uint64_t)s * RMAX * 2), ls = fa_load(ml + (uint64_t)s * RMAX * 2 + 1);
                    s_w[s] = ms;
                    const float mn = fmaxf(m_l, ms);
                    l_l = (m_l == -INFINITY ? 0.0f : l_l * __builtin_amdgcn_exp2f(m_l - mn)) +
                          (ms == -INFINITY ? 0.0f : ls * __builtin_amdgcn_exp2f(ms - mn));
                    m_l = mn;
                }
                const float M = kvm_wave_max_f32(m_l);
                const float L = kvm_wave_sum_f32(m_l == -INFINITY ? 0.0f : l_l * __builtin_amdgcn_exp2f(m_l - M));
                for (uint32_t s = tid; s < S; s += 64) {
                    const float ms = s_w[s];
                    s_w[s] = ms == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ms - M);
                }
                if (tid == 0) s_inv = M == -INFINITY || !(L > 0.0f) ? 0.0f : 1.0f / L;
            }
            __syncthreads();
            float acc = 0.0f;
            for (uint32_t s0 = sp;; ) {
#pragma unroll
                for (int i = 0; i < NBAT; ++i) {
                    const uint32_t si = s0 + SP * i;
                    acc += s_w[si < S ? si : KVM_MAX_SPLITS] * v[i];
                }
                s0 += SP * NBAT;
                if (s0 >= S) break;
#pragma unroll
                for (int i = 0; i < NBAT; ++i) v[i] = ld(s0 + SP * i);
            }
            s_acc[tid] = acc;
            __syncthreads();
            if (sp == 0) {
                float o = acc;
                for (uint32_t i = 1; i < SP; ++i) o += s_acc[i * UD + dd];
                const uint32_t t = row / a.G, qh = h * a.G + row % a.G;
                ln.out[((uint64_t)t * a.n_head + qh) * D + d] = o * s_inv;
            }
            if (u + nm < (uint32_t)R * dc) __syncthreads();   // s_w and s_acc are reused by the next unit
        }
    }
}

// The lane's stage-in plan, carried out by the attention's own workgroups
// before any of them reads the window: workgroup x = h * cols + column of the
// lane's G = H * cols stages its share of the items (after the gather of the
// blocks that move within the window, behind the plan's first barrier), then
// every workgroup waits at a second barrier for the whole plan.
// In a selecting launch (cols = n_splits + 1) the selector column stages too.
// FAST: the stage-in's device-coherent move staging, split gather and 16-lane
// K rows (stage_plan), which the selecting launch leaves out: with its
// attention state live around the staging they raise its registers to the
// limit and its steady-state time, though it never runs them there.
template <int D, bool FAST, int KQ = KVM_KQ_ANY>
__device__ __forceinline__ void fa_stage_lane(const fa_args &a, const stage_args &sg, uint32_t n_ent, uint32_t cols) {
    extern __shared__ __align__(16) uint8_t s_rows[];     // the staged launch's dynamic LDS
    __shared__ uint32_t s_e;
    if (threadIdx.x == 0) s_e = sync_load(sg.sync);
    __syncthreads();
    const uint32_t e = s_e, G = a.H * cols, x = blockIdx.y * cols + blockIdx.x;
    stage_plan<D, 512, KVM_FA_STAGE_IT, FAST, KQ>(sg, s_rows, n_ent, x, G, e + 1, false);
    if (!lane_barrier<512>(sg.sync, sg.status, sg.spin, e + 2, x, G, true, true) && threadIdx.x == 0)
        atomicOr(&sg.info[3], 16u);
}

// A selecting launch: workgroup (n_splits, 0) of each lane runs the lane's
// top-k and layout (kvm_topk_dev.h, 512 threads, at most KVM_SEL_MAXB blocks),
// while the lane's attention workgroups attend over the window as it is.
#define KVM_SEL_MAXB 4096
typedef topk_lds<512, KVM_SEL_MAXB, 1024> sel_lds;

// The selector publishes the plan to each of the lane's heads: one 64-bit
// word per (lane, head) = the head's epoch of this launch | the entries to
// stage << 32, after the selection's stores are written back (release).  It
// reads the epochs before the selection, and no split of a head raises its
// flag before it has seen the head's word, so the head's merger cannot have
// advanced the epoch yet.
__device__ __forceinline__ void fa_select_lane(const fa_args &a, const topk_args &t) {
    extern __shared__ __align__(16) uint8_t s_rows[];     // the launch's dynamic LDS
    __shared__ uint32_t s_ep[KVM_FA_MAX_HEADS];
    const uint32_t tid = threadIdx.x;
    const uint32_t *ep = a.sync + KVM_FA_SYNC_EPOCH + blockIdx.z * KVM_FA_MAX_HEADS;
    // (issued with the selection's loads: every lane loads, tid < H keeps it)
    const uint32_t my_ep = sync_load(ep + (tid < a.H ? tid : 0u));
    const uint32_t n_ent = topk_body(t, *reinterpret_cast<sel_lds *>(s_rows));
    if (tid < a.H) s_ep[tid] = my_ep;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
        __threadfence();
        uint64_t *plan = (uint64_t *)(a.sync + KVM_FA_SYNC_PLAN) + blockIdx.z * KVM_FA_MAX_HEADS;
        for (uint32_t h = 0; h < a.H; ++h)
            __hip_atomic_store(plan + h, (uint64_t)(s_ep[h] + 1u) | (uint64_t)n_ent << 32, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
}

// An attention workgroup's wait for its lane's plan (thread 0 polls the
// head's word for this launch's epoch): the entries to stage, 0 when the plan
// is empty or the wait gave up.  At most a.spin polls (s_sleep rounds of ~128
// cycles, about 0.2 s by default): the selector is resident with it (the grid
// never exceeds what the CUs hold at once) and waits on nothing; past the
// limit the status word says so (KVM_WAIT_PLAN) and the workgroup keeps its
// pass over the window as it was.
__device__ __forceinline__ uint32_t fa_await_plan(const fa_args &a, uint32_t h, uint32_t epoch) {
    __shared__ uint32_t s_n;
    if (threadIdx.x == 0) {
        const uint64_t *pw = (const uint64_t *)(a.sync + KVM_FA_SYNC_PLAN) + blockIdx.z * KVM_FA_MAX_HEADS + h;
        uint32_t n = 0;
        for (uint32_t it = 0;; ++it) {
            if (it >= a.spin) {
                __hip_atomic_fetch_or(a.sync + KVM_FA_SYNC_STATUS, (uint32_t)KVM_WAIT_PLAN, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            const uint64_t v = __hip_atomic_load(pw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((uint32_t)v == epoch) {
                n = (uint32_t)(v >> 32);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        s_n = n;
    }
    __syncthreads();
    return s_n;
}

// STAGE: the launch first carries out its lanes' stage-in plans.  SELECT
// (with STAGE): the plans come from the launch's selectors; the attention
// workgroups attend over the window as it is, then wait for the lane's plan,
// and only when it stages anything stage it and attend again.
template <int D, int NRT, bool QUANT, bool PK, bool STAGE, bool SELECT, int KQ = KVM_KQ_ANY>
__device__ __forceinline__ void fa_decode_body(const fa_args &a, const stage_args *stg, const topk_args *sel) {
    static_assert(!SELECT || STAGE, "a selecting launch stages its plans");
    constexpr int NB = D / 32;          // 32-dim blocks per row
    constexpr int NP = NB / 2;          // block pairs (packed row tile)
    constexpr int NG = QUANT ? NB / 4 : 1;   // 4-block scale groups
    constexpr int RMAX = 16 * NRT;      // padded query rows
    static_assert(!PK || QUANT, "only the q8_0 scores pack two blocks per MFMA");
    constexpr int DW = D / 4;           // output dims per P V wave
    constexpr int NT = DW / 16;         // 16-dim output tiles per P V wave
    constexpr int NBW = DW >= 32 ? DW / 32 : 1;   // V scale blocks per P V wave
    constexpr int NTB = NT / NBW;       // output tiles per V scale block
    constexpr uint32_t KTILE = QUANT ? 64u * D + 64u * NB * 2u : 64u * D * 2u;
    constexpr uint32_t VTILE = QUANT ? D * 32u + NB * 64u * 2u : 64u * D * 2u;
    constexpr int NITEM = RMAX * NB;    // query quantisation items (row, block)
    constexpr int QT = (NITEM + 127) / 128;   // items per lane group (8 waves x 16)
    constexpr int PSTR = 64 + 8;        // padded fp16 row stride of P in LDS
    static_assert(NT >= 1 && NT % NBW == 0, "P V dim split");
    // A packed row tile (PK: the last one, at most 8 rows) scores two 32-dim
    // blocks per v_mfma_i32_16x16x64_i8: column m < 8 is row 16rt+m against
    // the even block of the pair, column m >= 8 the same row against the odd
    // block (the query operand is zero in the other half), so half the MFMAs
    // and scale FMAs of a padded tile; the two halves are summed across lanes
    // m and m^8, which then both hold the row's scores.
    auto is_pk = [](int rt) { return PK && rt == NRT - 1; };
    using KRegs = fa_k_regs<D, QUANT, PK>;
    using VRegs = fa_v_regs<D, QUANT, NT, NBW>;

    const fa_lane ln = a.lanes[blockIdx.z];
    const uint32_t h = blockIdx.y, split = blockIdx.x;
    const int tid = threadIdx.x, l = tid & 63, g = l >> 4, m = l & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool scorer = w < 4;          // waves 0-3 score (key quarter w), 4-7 do P V (dim quarter w-4)
    const int R = (int)(ln.n_tokens * a.G);
    const uint32_t tps = (ln.n_tiles + a.n_splits - 1) / a.n_splits;
    const uint32_t t_begin = split * tps;
    const uint32_t t_end = t_begin + tps < ln.n_tiles ? t_begin + tps : ln.n_tiles;
    const uint32_t n_t = t_end > t_begin ? t_end - t_begin : 0;

    __shared__ __align__(16) int8_t s_qq[QUANT ? RMAX : 1][D];
    __shared__ __align__(16) _Float16 s_qh[QUANT ? 1 : RMAX][D];
    __shared__ float s_dq[RMAX][NB];
    __shared__ float s_max[4][4][RMAX];      // [key quarter][lane group][row]: max of 4 keys
    __shared__ float s_alpha[RMAX];
    __shared__ int32_t s_rescale[NRT];
    __shared__ __align__(4) uint8_t s_up[2][4];    // per scoring wave: a row's maximum moved (tile parity)
    __shared__ float s_l[4][RMAX];
    __shared__ __align__(16) _Float16 s_p[2][RMAX][PSTR];   // P of the tile (tile parity)

    if constexpr (SELECT) {
        if (split == a.n_splits) {           // the lane's selector column
            // the head's epoch, read before this workgroup raises its flag (the
            // head's merger waits for it, so the epoch cannot move before)
            const uint32_t ep_c = __hip_atomic_load(a.sync + KVM_FA_SYNC_EPOCH + blockIdx.z * KVM_FA_MAX_HEADS + h,
                                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (h == 0) {
                const topk_args t = sel[blockIdx.z];     // one copy out of the argument segment
                fa_select_lane(a, t);
            }
            // the column takes part in staging a plan that stages anything, so
            // that the items spread over every workgroup the CUs hold
            const uint32_t n = fa_await_plan(a, h, ep_c + 1);
            if (n) {
                __threadfence();             // acquire: the selection's stores
                fa_stage_lane<D, !SELECT, KQ>(a, stg[blockIdx.z], n, a.n_splits + 1);
            }
            __syncthreads();
            if (tid == 0)
                __hip_atomic_store(a.sync + ((uint64_t)blockIdx.z * KVM_FA_MAX_HEADS + h) * KVM_MAX_SPLITS + a.n_splits,
                                   ep_c + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
    }
    // lane without query rows: no partials (a selecting launch has none: its
    // workgroups could not tell this launch's plan from an earlier one)
    if (R == 0) {
        if constexpr (STAGE && !SELECT) {
            const uint32_t n_ent = stage_entries(stg[blockIdx.z]);
            if (n_ent) fa_stage_lane<D, !SELECT, KQ>(a, stg[blockIdx.z], n_ent, a.n_splits);
        }
        return;
    }

    // ---- query rows: item (row r = token r/G, query head h*G + r%G; block b),
    // four lanes per item, 8 dims each, quantised to q8_0 per 32 dims as
    // ggml's vec_dot path does, or rounded to fp16.  Every wave loads its items
    // first (unconditionally: items past the rows re-read row 0 and are zeroed;
    // a bf16 row loads its 16 bytes twice) and waits for them before any tile
    // load is issued: behind the whole grid's tile prologue the query would
    // arrive last.
    kvm_u32x4 qraw[QT][2];
    {
        const uint32_t esz = a.q_bf16 ? 2u : 4u;
#pragma unroll
        for (int t = 0; t < QT; ++t) {
            const int item = (t * 8 + w) * 16 + m, rr = item / NB, b = item % NB;
            const int r = item < NITEM && rr < R ? rr : 0;
            const uint64_t e0 = ((uint64_t)(r / a.G) * a.n_head + h * a.G + r % a.G) * D + 32 * b + 8 * g;
            const uint8_t *qb = (const uint8_t *)ln.q + e0 * esz;
            qraw[t][0] = *(const kvm_u32x4 *)qb;
            qraw[t][1] = *(const kvm_u32x4 *)(qb + (esz == 4u ? 16u : 0u));
        }
    }
    // positions of the rows a scoring lane holds (row 16rt + m; 16rt + m % 8 in
    // a packed row tile), with the query
    auto srow = [&](int rt) { return is_pk(rt) ? 16 * rt + (m & 7) : 16 * rt + m; };
    int32_t qpos_raw[NRT];
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
        const int row = srow(rt);
        qpos_raw[rt] = ln.q_pos[(row < R ? row : 0) / a.G];
    }
    // this launch's epoch for the (lane, head): one more than the stored one,
    // which the head's first merging split advances once every split has read it
    __shared__ uint32_t s_epoch;
    const uint32_t ep = __hip_atomic_load(a.sync + KVM_FA_SYNC_EPOCH + blockIdx.z * KVM_FA_MAX_HEADS + h,
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // a staged launch reads the lane's plan length with the query (an empty
    // plan, the decode loop's steady state, then costs no memory round trip)
    uint32_t n_ent = 0;
    if constexpr (STAGE && !SELECT) n_ent = stage_entries(stg[blockIdx.z]);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (tid == 0) s_epoch = ep + 1;
    if constexpr (STAGE && !SELECT) {
        if (n_ent) fa_stage_lane<D, !SELECT, KQ>(a, stg[blockIdx.z], n_ent, a.n_splits);
    }
    // SELECT, after the first pass over the window (both roles, at the same
    // barrier): true when the lane's plan staged anything, so the pass is redone
    auto restaged = [&](uint32_t pass) -> bool {
        if constexpr (!SELECT) {
            return false;
        } else {
            if (pass) return false;
            const uint32_t n = fa_await_plan(a, h, ep + 1);
            if (!n) return false;
            __threadfence();                 // acquire: the selection's stores
            fa_stage_lane<D, !SELECT, KQ>(a, stg[blockIdx.z], n, a.n_splits + 1);
            return true;
        }
    };
    // (the scoring waves call it behind their K prologue, the P V waves ahead
    // of their V prologue; it ends with the barrier)
    auto quantise_q = [&]() {
#pragma unroll
        for (int t = 0; t < QT; ++t) {
            const int item = (t * 8 + w) * 16 + m, r = item / NB, b = item % NB;
            if (item >= NITEM) continue;
            float qx[8];
            if (r >= R) {
#pragma unroll
                for (int j = 0; j < 8; ++j) qx[j] = 0.0f;
            } else if (a.q_bf16) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    qx[2 * j] = __uint_as_float(qraw[t][0][j] << 16);
                    qx[2 * j + 1] = __uint_as_float(qraw[t][0][j] & 0xffff0000u);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    qx[j] = __uint_as_float(qraw[t][0][j]);
                    qx[4 + j] = __uint_as_float(qraw[t][1][j]);
                }
            }
            if constexpr (QUANT) {
                float amax = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(qx[j]));
                amax = kvm_max_xor32(kvm_max_xor16(amax));
                const float d = kvm_div127(amax);
                const float id = kvm_recip_or0(d);
                uint32_t q01[2] = {0u, 0u};
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    q01[j >> 2] |= (uint32_t)(uint8_t)kvm_round_away(kvm_fmul(qx[j], id)) << (8 * (j & 3));
                *(kvm_u32x2 *)&s_qq[r][32 * b + 8 * g] = kvm_u32x2{q01[0], q01[1]};
                if (g == 0) s_dq[r][b] = kvm_h2f(kvm_f2h(d));
            } else {
                kvm_f16x8 hv;
#pragma unroll
                for (int j = 0; j < 8; ++j) hv[j] = (_Float16)qx[j];
                *(kvm_f16x8 *)&s_qh[r][32 * b + 8 * g] = hv;
            }
        }
        KVM_LDS_BARRIER();
    };

    // tile to load for step i: past the split's last tile the loads re-read it,
    // and an empty split reads tile 0 (every window has one), so every step
    // issues the same loads and the prologue needs no branch
    auto tile_index = [&](uint32_t i) { return n_t == 0 ? 0u : t_begin + (i < n_t ? i : n_t - 1); };
    // Both roles step through the same tiles with the same barriers: one per
    // tile, and a second one when a row's running maximum moves.  A ring of
    // KVM_FA_NBUF register buffers keeps KVM_FA_NBUF - 1 tiles in flight; the
    // loop body is straight line so the compiler's wait counts see the same
    // loads in flight on every trip; the last tiles are handled after the loop.
    auto run_tiles = [&](auto (&bf)[KVM_FA_NBUF], auto &&step) {
        uint32_t it = 0;
        for (; it + KVM_FA_NBUF <= n_t; it += KVM_FA_NBUF) {
#pragma unroll
            for (int j = 0; j < KVM_FA_NBUF; ++j) step(bf[j], bf[(j + KVM_FA_NBUF - 1) % KVM_FA_NBUF], it + j + KVM_FA_NBUF - 1);
        }
#pragma unroll
        for (int j = 0; j < KVM_FA_NBUF - 1; ++j)
            if (it + j < n_t) step(bf[j], bf[(j + KVM_FA_NBUF - 1) % KVM_FA_NBUF], it + j + KVM_FA_NBUF - 1);
    };
    const uint64_t pidx = ((uint64_t)blockIdx.z * a.H + h) * a.n_splits + split;

    if (scorer) {
        // ================= scoring waves: S = K Q^T, softmax, P to LDS =====
        const int kq = w;
        const uint8_t *kbase = ln.wk + (uint64_t)h * ln.n_tiles * KTILE;
        const uint32_t k_off = QUANT ? (uint32_t)((kq * (NB / 2) * 64 + l) << 4) : (uint32_t)((kq * NB * 64 + l) << 4);
        const uint32_t dk_off = 64u * D + (uint32_t)(((kq * NB + g) * 16 + m) << 1);
        // packed row tile: scales of blocks 2g, 2g+1 (lane groups past the pairs read block 0)
        const uint32_t dkp_off = 64u * D + (uint32_t)(((kq * NB + (g < NP ? 2 * g : 0)) * 16 + m) << 1);
        const uint32_t cp_off = (uint32_t)(16 * kq + 4 * g) * 4u;
        auto load_k = [&](KRegs &rg, uint32_t T) {
            const uint8_t *kt = kbase + (uint64_t)T * KTILE;
#pragma unroll
            for (int p = 0; p < (QUANT ? NB / 2 : NB); ++p) rg.k[p] = *(const kvm_u32x4 *)(kt + k_off + 1024u * p);
            if constexpr (QUANT && !(PK && NRT == 1)) {
#pragma unroll
                for (int gi = 0; gi < NG; ++gi) rg.dk[gi] = *(const uint16_t *)(kt + dk_off + 128u * gi);
            }
            if constexpr (PK) {
                rg.dkp[0] = *(const uint16_t *)(kt + dkp_off);
                rg.dkp[1] = *(const uint16_t *)(kt + dkp_off + 32u);
            }
            rg.cp = *(const kvm_u32x4 *)((const uint8_t *)(ln.cell_pos + (uint64_t)T * 64) + cp_off);
        };
        KRegs kb[KVM_FA_NBUF];
        auto prologue = [&]() {
#pragma unroll
            for (int j = 0; j < KVM_FA_NBUF - 1; ++j) load_k(kb[j], tile_index(j));
        };
        prologue();
        quantise_q();
        for (uint32_t pass = 0;; ++pass) {
            if (pass) prologue();

            // B operands (Q^T) of every row tile: lane (row 16rt+m, k-group g)
            long qop_i[QUANT ? NRT : 1][QUANT ? NB : 1];
            kvm_i32x4 qop_p[NP];                 // packed row tile: [even block | odd block] per pair
            kvm_f16x8 qop_h[QUANT ? 1 : NRT][QUANT ? 1 : NB];
            float dqo[NRT][NG];                  // scale MFMA B operand: dq * kq_scale * log2(e)
            float dqp[2];                        // packed row tile: even-block / odd-block columns
            uint32_t qlim[NRT];                  // cell visible iff (uint)cell_pos < qlim (= q_pos + 1; 0 for padding)
            float m_run[NRT], l_run[NRT];        // row 16rt + m (16rt + m % 8 packed) over this lane's keys
            // B operands from the workgroup's quantised query in LDS
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt) {
                const int row = srow(rt);
                if (is_pk(rt)) {
                    const bool odd = m >= 8;
#pragma unroll
                    for (int p = 0; p < NP; ++p) {
                        kvm_u32x2 v;
                        __builtin_memcpy(&v, &s_qq[row][32 * (2 * p + odd) + 8 * g], 8);
                        qop_p[p] = odd ? kvm_i32x4{0, 0, (int)v[0], (int)v[1]} : kvm_i32x4{(int)v[0], (int)v[1], 0, 0};
                    }
                    dqp[0] = !odd && g < NP ? s_dq[row][2 * g] * a.scale_log2 : 0.0f;
                    dqp[1] = odd && g < NP ? s_dq[row][2 * g + 1] * a.scale_log2 : 0.0f;
                } else {
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        if constexpr (QUANT) __builtin_memcpy(&qop_i[rt][b], &s_qq[row][32 * b + 8 * g], 8);
                        else qop_h[rt][b] = *(const kvm_f16x8 *)&s_qh[row][32 * b + 8 * g];
                    }
#pragma unroll
                    for (int gi = 0; gi < NG; ++gi) dqo[rt][gi] = QUANT ? s_dq[row][4 * gi + g] * a.scale_log2 : 0.0f;
                }
                qlim[rt] = row < R && qpos_raw[rt] >= 0 ? (uint32_t)qpos_raw[rt] + 1u : 0u;
                m_run[rt] = KVM_M_NONE;
                l_run[rt] = 0.0f;
            }
            // the smallest limit of a real row: keys below it are visible to
            // every row, and a tile whose keys all are needs no masking (the
            // padding rows then score unmasked keys, which only their own,
            // never stored, outputs see)
            uint32_t qmin = 0xffffffffu;
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt)
                if (srow(rt) < R) qmin = qlim[rt] < qmin ? qlim[rt] : qmin;
            qmin = kvm_wave_min_u32(qmin);
            int par = 0;                         // tile parity: P and flag buffers

            auto score = [&](const KRegs &rg, KRegs &nx, uint32_t inext) {
                load_k(nx, tile_index(inext));
                // ---- scores of keys 16kq + 4g + i, rows 16rt + m (log2 domain; q8_0:
                // kq_scale * log2(e) is folded into the query scales), masked
                float s[NRT][4];
#pragma unroll
                for (int rt = 0; rt < NRT; ++rt) {
                    if constexpr (QUANT) {
                        if (is_pk(rt)) {
                            // d_k * d_q of (key 4g+i, column m) for the four pairs: the
                            // even-block product in columns m < 8, the odd one in m >= 8
                            kvm_f32x16 dd = __builtin_amdgcn_mfma_f32_16x16x1f32(kvm_h2f((uint16_t)rg.dkp[0]), dqp[0],
                                                                                kvm_f32x16{}, 0, 0, 0);
                            dd = __builtin_amdgcn_mfma_f32_16x16x1f32(kvm_h2f((uint16_t)rg.dkp[1]), dqp[1], dd, 0, 0, 0);
#pragma unroll
                            for (int i = 0; i < 4; ++i) s[rt][i] = 0.0f;
#pragma unroll
                            for (int p = 0; p < NP; ++p) {
                                kvm_i32x4 kw;
                                __builtin_memcpy(&kw, &rg.k[p], 16);
                                const kvm_i32x4 c = __builtin_amdgcn_mfma_i32_16x16x64_i8(kw, qop_p[p], kvm_i32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                                for (int i = 0; i < 4; ++i) s[rt][i] = fmaf((float)c[i], dd[4 * p + i], s[rt][i]);
                            }
#pragma unroll
                            for (int i = 0; i < 4; ++i) s[rt][i] += kvm_ror8_f32(s[rt][i]);
                        } else {
                            // d_k * d_q of (key 4g+i, row m) for four blocks per MFMA
                            kvm_f32x16 dd[NG];
#pragma unroll
                            for (int gi = 0; gi < NG; ++gi)
                                dd[gi] = __builtin_amdgcn_mfma_f32_16x16x1f32(kvm_h2f((uint16_t)rg.dk[gi]), dqo[rt][gi],
                                                                               kvm_f32x16{}, 0, 0, 0);
#pragma unroll
                            for (int i = 0; i < 4; ++i) s[rt][i] = 0.0f;
#pragma unroll
                            for (int b = 0; b < NB; ++b) {
                                const kvm_u32x4 kw = rg.k[b >> 1];
                                const uint64_t lo32 = kw[(b & 1) * 2], hi32 = kw[(b & 1) * 2 + 1];
                                const long av = (long)(lo32 | (hi32 << 32));
                                const kvm_i32x4 c = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, qop_i[rt][b], kvm_i32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                                for (int i = 0; i < 4; ++i) s[rt][i] = fmaf((float)c[i], dd[b >> 2][4 * (b & 3) + i], s[rt][i]);
                            }
                        }
                    } else {
                        kvm_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int ks = 0; ks < NB; ++ks) {
                            kvm_f16x8 av;
                            __builtin_memcpy(&av, &rg.k[ks], 16);
                            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, qop_h[rt][ks], acc, 0, 0, 0);
                        }
#pragma unroll
                        for (int i = 0; i < 4; ++i) s[rt][i] = acc[i] * a.scale_log2;
                    }
                }
                // ---- mask; per lane maxima; P against the current maxima.  A wave
                // with a row whose maximum moves by more than 2^KVM_LAZY_MAX says so,
                // and then (rarely) the scoring waves take the row maxima from LDS
                // and redo P.  Before a row's first visible key m_run is KVM_M_NONE,
                // which every finite score moves.
                bool up_w = false;
                float psum[NRT];
                uint32_t cmax = rg.cp[0] > rg.cp[1] ? rg.cp[0] : rg.cp[1];
                cmax = cmax > rg.cp[2] ? cmax : rg.cp[2];
                cmax = cmax > rg.cp[3] ? cmax : rg.cp[3];
                if (__builtin_amdgcn_ballot_w64(!(cmax < qmin)) != 0) {
                    asm volatile("" ::: "memory");      // keep the masking a branch: most tiles skip it
#pragma unroll
                    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (!(rg.cp[i] < qlim[rt])) s[rt][i] = -INFINITY;    // empty (-1) or after the row
                }
                // (the sum of a lane's four fp16 probabilities in fp32 by two
                // v_dot2_f32_f16 against ones, from the pairs packed for LDS)
                auto make_p = [&](int rt, float mn) {
                    const kvm_f16x2 one2 = {(_Float16)1.0f, (_Float16)1.0f};
                    kvm_f16x2 ph[2];
#pragma unroll
                    for (int i = 0; i < 2; ++i)
                        ph[i] = kvm_f16x2{(_Float16)__builtin_amdgcn_exp2f(s[rt][2 * i] - mn),
                                          (_Float16)__builtin_amdgcn_exp2f(s[rt][2 * i + 1] - mn)};
                    psum[rt] = __builtin_amdgcn_fdot2(ph[1], one2, __builtin_amdgcn_fdot2(ph[0], one2, 0.0f, false), false);
                    __builtin_memcpy(&s_p[par][16 * rt + m][16 * kq + 4 * g], ph, 8);
                };
#pragma unroll
                for (int rt = 0; rt < NRT; ++rt) {
                    float mx = -INFINITY;
#pragma unroll
                    for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[rt][i]);
                    s_max[kq][g][16 * rt + m] = mx;
                    up_w = up_w || mx > m_run[rt] + KVM_LAZY_MAX;
                    make_p(rt, m_run[rt]);
                }
                const bool wave_up = __builtin_amdgcn_ballot_w64(up_w) != 0;
                if (l == 0) s_up[par][kq] = wave_up;
                KVM_LDS_BARRIER();
                if (*(const uint32_t *)&s_up[par][0] != 0) {
                    asm volatile("" ::: "memory");      // keep this (rare) path a branch
#pragma unroll
                    for (int rt = 0; rt < NRT; ++rt) {
                        const int row = 16 * rt + m;
                        float tm = s_max[0][0][row];
#pragma unroll
                        for (int j = 1; j < 16; ++j) tm = fmaxf(tm, s_max[j >> 2][j & 3][row]);
                        const bool up = tm > m_run[rt] + KVM_LAZY_MAX;
                        const float mn = up ? tm : m_run[rt];
                        const float alpha = up ? __builtin_amdgcn_exp2f(m_run[rt] - mn) : 1.0f;
                        make_p(rt, mn);
                        l_run[rt] = l_run[rt] * alpha + psum[rt];
                        m_run[rt] = mn;
                        if (kq == 0) {
                            if (g == 0) s_alpha[row] = alpha;
                            const bool any = __builtin_amdgcn_ballot_w64(up) != 0;
                            if (l == 0) s_rescale[rt] = any;
                        }
                    }
                    KVM_LDS_BARRIER();
                } else {
#pragma unroll
                    for (int rt = 0; rt < NRT; ++rt) l_run[rt] += psum[rt];
                }
                par ^= 1;
            };
            run_tiles(kb, score);
            if (restaged(pass)) continue;

            // ---- (m, l) of this split's rows (a packed row tile: the lanes m >= 8
            // repeat the rows of lanes m - 8 and are left out of the sum)
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt) {
                float lr = is_pk(rt) && m >= 8 ? 0.0f : l_run[rt];
                lr = kvm_add_xor32(kvm_add_xor16(lr));
                if (g == 0) s_l[kq][16 * rt + m] = lr;
            }
            __syncthreads();
            if (kq == 0 && g == 0) {
#pragma unroll
                for (int rt = 0; rt < NRT; ++rt) {
                    const int row = 16 * rt + m;
                    if (row < R) {
                        fa_store(&a.ws_ml[(pidx * RMAX + row) * 2 + 0], m_run[rt] == KVM_M_NONE ? -INFINITY : m_run[rt]);
                        fa_store(&a.ws_ml[(pidx * RMAX + row) * 2 + 1], s_l[0][row] + s_l[1][row] + s_l[2][row] + s_l[3][row]);
                    }
                }
            }
            break;
        }
    } else {
        // ================= P V waves: O[:, dims DW*dq ..] += P V ============
        const int dq = w - 4;
        const uint8_t *vbase = ln.wv + (uint64_t)h * ln.n_tiles * VTILE;
        const uint32_t vq_off = kvm_vq_word((uint32_t)(DW * dq + m), (uint32_t)g, 0);
        const uint32_t vs_off = D * 32u + (uint32_t)(((((DW * dq) / 32) * 2) * 4 + g) * 8 * 2);
        const uint32_t vh_off = kvm_vh_idx((uint32_t)(8 * g), (uint32_t)(DW * dq + m)) << 1;
        auto load_v = [&](VRegs &rg, uint32_t T) {
            const uint8_t *vt = vbase + (uint64_t)T * VTILE;
            if constexpr (QUANT) {
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) rg.vq[nt] = *(const kvm_u32x2 *)(vt + vq_off + 512u * nt);
#pragma unroll
                for (int bw = 0; bw < NBW; ++bw)
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) rg.vs[bw][ks] = *(const kvm_u32x4 *)(vt + vs_off + 128u * bw + 64u * ks);
            } else {
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) rg.vh[nt][ks] = *(const kvm_u32x4 *)(vt + vh_off + 2048u * nt + 16u * ks);
            }
        };
        quantise_q();                            // V is needed a tile later than K
        VRegs vbuf[KVM_FA_NBUF];
        for (uint32_t pass = 0;; ++pass) {
#pragma unroll
            for (int j = 0; j < KVM_FA_NBUF - 1; ++j) load_v(vbuf[j], tile_index(j));

            kvm_f32x4 O[NRT][NT];
            // q8_0/q4_0: O accumulates P * dv * n * 2^-24 (V as fp16 denormals) and
            // Oc P * dv * 8 * 2^-24 per row and 32-dim V block; (O - Oc) * 2^24 is P V
            kvm_f32x4 Oc[NRT][NBW];
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt) {
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) O[rt][nt] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int bw = 0; bw < NBW; ++bw) Oc[rt][bw] = {0.f, 0.f, 0.f, 0.f};
            }
            const kvm_f16x8 eight_den = {(_Float16)0x1p-21f, (_Float16)0x1p-21f, (_Float16)0x1p-21f, (_Float16)0x1p-21f,
                                         (_Float16)0x1p-21f, (_Float16)0x1p-21f, (_Float16)0x1p-21f, (_Float16)0x1p-21f};
            int par = 0;

            auto accumulate = [&](const VRegs &rg, VRegs &nx, uint32_t inext) {
                load_v(nx, tile_index(inext));
                KVM_LDS_BARRIER();                   // P of this tile is in LDS
                if (*(const uint32_t *)&s_up[par][0] != 0) {
                    asm volatile("" ::: "memory");
                    KVM_LDS_BARRIER();               // ... redone against the moved maxima
#pragma unroll
                    for (int rt = 0; rt < NRT; ++rt) {
                        if (s_rescale[rt]) {
                            float ar[4];
#pragma unroll
                            for (int r = 0; r < 4; ++r) ar[r] = s_alpha[16 * rt + 4 * g + r];
#pragma unroll
                            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                                for (int r = 0; r < 4; ++r) O[rt][nt][r] *= ar[r];
#pragma unroll
                            for (int bw = 0; bw < NBW; ++bw)
#pragma unroll
                                for (int r = 0; r < 4; ++r) Oc[rt][bw][r] *= ar[r];
                        }
                    }
                }
                kvm_f16x8 pa[2][NRT];
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                    for (int rt = 0; rt < NRT; ++rt) pa[ks][rt] = *(const kvm_f16x8 *)&s_p[par][16 * rt + m][32 * ks + 8 * g];
#pragma unroll
                for (int bw = 0; bw < NBW; ++bw) {
                    kvm_f16x8 pp[2][NRT];
                    if constexpr (QUANT) {
#pragma unroll
                        for (int ks = 0; ks < 2; ++ks) {
                            kvm_f16x8 dv;
                            __builtin_memcpy(&dv, &rg.vs[bw][ks], 16);
#pragma unroll
                            for (int rt = 0; rt < NRT; ++rt) {
                                pp[ks][rt] = pa[ks][rt] * dv;
                                Oc[rt][bw] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pp[ks][rt], eight_den, Oc[rt][bw], 0, 0, 0);
                            }
                        }
                    }
#pragma unroll
                    for (int ntb = 0; ntb < NTB; ++ntb) {
                        const int nt = bw * NTB + ntb;
#pragma unroll
                        for (int ks = 0; ks < 2; ++ks) {
                            kvm_f16x8 vb;
                            if constexpr (QUANT) vb = nib8_to_f16den(rg.vq[nt][ks]);
                            else __builtin_memcpy(&vb, &rg.vh[nt][ks], 16);
#pragma unroll
                            for (int rt = 0; rt < NRT; ++rt)
                                O[rt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(QUANT ? pp[ks][rt] : pa[ks][rt], vb, O[rt][nt], 0, 0, 0);
                        }
                    }
                }
                par ^= 1;
            };
            run_tiles(vbuf, accumulate);
            if (restaged(pass)) continue;

            __syncthreads();                          // pairs with the scoring waves' (m, l) exchange
            // a padding row (row >= R, so R < RMAX) is stored into row RMAX - 1,
            // itself padding and never read by the merge: the stores need no
            // guard (a guard puts each store behind a branch of its own in a
            // half-used row tile) and the padding lanes of a store share one
            // segment instead of writing their own
            float *po = a.ws + pidx * RMAX * D;
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int row = 16 * rt + 4 * g + r;
                        fa_store(&po[(row < R ? row : RMAX - 1) * D + DW * dq + 16 * nt + m],
                                 QUANT ? (O[rt][nt][r] - Oc[rt][nt / NTB][r]) * 0x1p24f : O[rt][nt][r]);
                    }
            break;
        }
    }

    // ---- arrival: the partials of this split are complete at device scope
    // (device-coherent stores, each wave waits for its own), then the split's
    // flag takes this launch's epoch.  Splits 0 .. NM-1 of the head then merge
    // units j = split, split + NM, ... once every flag of the head is up.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // flag slots are fixed per (lane, head, split), whatever the launch's head
    // and split counts, so a slot only ever holds its own head's epochs
    uint32_t *flags = a.sync + ((uint64_t)blockIdx.z * KVM_FA_MAX_HEADS + h) * KVM_MAX_SPLITS;
    const uint32_t epoch = s_epoch;
    if (tid == 0) __hip_atomic_store(flags + split, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // merge units: rows split into dc dim chunks (at least 64 dims) while at
    // most about half the splits merge and the head's mergers, each polling
    // every flag of the head, poll at most KVM_FA_POLL_WORDS flag words per
    // round (the head's flags share a few cache lines, and more pollers only
    // queue behind each other there)
    const uint32_t S = a.n_splits;
    uint32_t dc = 1;
    while (dc < D / 64 && (uint32_t)R * dc * 2 <= S && (uint32_t)R * dc * 2 * S <= KVM_FA_POLL_WORDS) dc *= 2;
    const uint32_t units = (uint32_t)R * dc, NM = units < S ? units : S;
    if (split >= NM) return;
    __shared__ fa_merge_lds s_mg;
    const uint32_t per = (S + 512 * dc / D - 1) / (512 * dc / D);     // splits per merging thread
    const uint32_t nf = SELECT ? S + 1 : S;
    if (per > 16) fa_merge<D, RMAX, 32>(a, ln, h, flags, nf, epoch, split, NM, dc, R, s_mg);
    else if (per > 8) fa_merge<D, RMAX, 16>(a, ln, h, flags, nf, epoch, split, NM, dc, R, s_mg);
    else if (per > 4) fa_merge<D, RMAX, 8>(a, ln, h, flags, nf, epoch, split, NM, dc, R, s_mg);
    else fa_merge<D, RMAX, 4>(a, ln, h, flags, nf, epoch, split, NM, dc, R, s_mg);
}

template <int D, int NRT, bool QUANT, bool PK>
__global__ void __launch_bounds__(512) k_fa_decode(fa_args a) {
    fa_decode_body<D, NRT, QUANT, PK, false, false>(a, nullptr, nullptr);
}

// Decode attention that first stages its lanes' plans (q8_0 windows only).
struct fa_staged_args {
    fa_args a;
    stage_args stage[KVM_MAX_LANES];
};
template <int D, int NRT, bool PK>
__global__ void __launch_bounds__(512) k_fa_decode_staged(fa_staged_args sa) {
    fa_decode_body<D, NRT, true, PK, true, false>(sa.a, sa.stage, nullptr);
}

// Decode attention whose launch also selects its lanes' plans (grid
// (n_splits + 1, H, lanes): column n_splits holds the selectors).
struct fa_select_args {
    fa_args a;
    stage_args stage[KVM_MAX_LANES];
    topk_args sel[KVM_MAX_LANES];
};
static_assert(sizeof(fa_select_args) <= 4096, "kernel argument segment");
// KQ: the windows' K type (KVM_KQ_Q8 or KVM_KQ_Q4), fixed so the staging
// code of the other type adds nothing to the registers.
template <int D, int NRT, bool PK, int KQ>
__global__ void __launch_bounds__(512) k_fa_decode_select(fa_select_args sa) {
    fa_decode_body<D, NRT, true, PK, true, true, KQ>(sa.a, sa.stage, sa.sel);
}

static uint32_t choose_splits(uint32_t n_cu, uint32_t n_lanes, uint32_t H, uint32_t n_tiles) {
    if (const char *e = getenv("KVM_FA_SPLITS")) {
        uint32_t v = (uint32_t)atoi(e);
        if (v > KVM_MAX_SPLITS) v = KVM_MAX_SPLITS;
        if (v > 0) return v < n_tiles ? v : n_tiles;
    }
    // about one workgroup per CU
    uint32_t s = (n_cu + n_lanes * H - 1) / (n_lanes * H);
    if (s < 1) s = 1;
    if (s > KVM_MAX_SPLITS) s = KVM_MAX_SPLITS;
    return s < n_tiles ? s : n_tiles;
}

template <int D, int NRT, bool QUANT, bool PK>
static void launch_decode(const fa_args &a, uint32_t n_lanes, hipStream_t stream) {
    hipLaunchKernelGGL((k_fa_decode<D, NRT, QUANT, PK>), dim3(a.n_splits, a.H, n_lanes), dim3(512), 0, stream, a);
}

// Row tiles of 16 query rows; with a q8_0 K a last tile of at most 8 rows is packed.
template <int D>
static void launch_decode_d(const fa_args &a, uint32_t n_lanes, uint32_t max_rows, bool quant, hipStream_t stream) {
    const int NRT = max_rows <= 16 ? 1 : 2;
    const bool pk = quant && max_rows - 16u * (NRT - 1) <= 8u;
    if (!quant) {
        if (NRT == 1) launch_decode<D, 1, false, false>(a, n_lanes, stream);
        else launch_decode<D, 2, false, false>(a, n_lanes, stream);
    } else if (NRT == 1) {
        if (pk) launch_decode<D, 1, true, true>(a, n_lanes, stream);
        else launch_decode<D, 1, true, false>(a, n_lanes, stream);
    } else {
        if (pk) launch_decode<D, 2, true, true>(a, n_lanes, stream);
        else launch_decode<D, 2, true, false>(a, n_lanes, stream);
    }
}

// Checks the lanes and fills the launch arguments.  scratch_cap == 0: the
// split partials go to the state's attention workspace
// (grown with hipMalloc when too small); otherwise to the caller's buffer
// `scratch` of scratch_cap bytes, with fewer key splits if the partials would
// not fit, and nothing is allocated.  *rows = 0: nothing to compute.
struct fa_plan {
    fa_args a;
    uint32_t n_lanes, rows, D;
    bool quant;
};
static int fa_prepare(kvm_state *st, const kvm_lane *lanes, uint32_t n_lanes, int q_type, uint32_t n_head,
                      float scale, void *scratch, size_t scratch_cap, fa_plan *fp, uint32_t max_wgs = 0,
                      uint32_t max_splits = KVM_MAX_SPLITS) {
    if (!st || !lanes || n_lanes == 0) return kvm_fail(st, KVM_EINVAL, "fa_decode: no lanes");
    if (n_lanes > KVM_MAX_LANES) return kvm_fail(st, KVM_ERANGE, "fa_decode: %u lanes > %d", n_lanes, KVM_MAX_LANES);
    if (q_type != KVM_TYPE_F32 && q_type != KVM_TYPE_BF16) return kvm_fail(st, KVM_EUNSUPPORTED, "fa_decode: q type %d", q_type);
    const kvm_window *w0 = lanes[0].w;
    if (!w0) return kvm_fail(st, KVM_EINVAL, "fa_decode: null window");
    uint32_t max_rows = 0, max_tiles = 0;
    fa_args &a = fp->a;
    a = fa_args{};
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
        a.lanes[i] = fa_lane{(const uint8_t *)L.w->k, (const uint8_t *)L.w->v, L.w->cell_pos, L.q, L.q_pos, L.out, nt,
                             L.n_tokens};
    }
    fp->n_lanes = n_lanes;
    fp->rows = max_rows;
    if (max_rows == 0) return KVM_OK;
    const uint32_t D = w0->head_dim, H = w0->n_head_kv;
    if (H > KVM_FA_MAX_HEADS) return kvm_fail(st, KVM_EUNSUPPORTED, "fa_decode: %u kv heads > %d", H, KVM_FA_MAX_HEADS);
    const int NRT = max_rows <= 16 ? 1 : 2;
    const uint32_t rmax = 16u * NRT;
    a.H = H;
    a.G = n_head / H;
    a.n_head = n_head;
    a.n_splits = choose_splits(st->n_cu, n_lanes, H, max_tiles);
    if (a.n_splits > max_splits) a.n_splits = max_splits;
    a.spin = st->wait_polls;
    // a grid whose workgroups must all be resident at once (a staged launch)
    if (max_wgs && a.n_splits * H * n_lanes > max_wgs) {
        a.n_splits = max_wgs / (H * n_lanes);
        if (a.n_splits == 0) return kvm_fail(st, KVM_ERANGE, "fa_decode: %u lanes x %u kv heads exceed the CUs", n_lanes, H);
    }
    a.scale_log2 = scale * 1.4426950408889634f;
    a.q_bf16 = q_type == KVM_TYPE_BF16;
    const bool quant = kvm_k_quant(w0->k_type);
    fp->D = D;
    fp->quant = quant;
    // workspace: the split partials, O then (m, l); with the caller's scratch,
    // the split flags first
    const size_t part_bytes = (size_t)n_lanes * H * rmax * (D + 2) * sizeof(float);   // per key split
    uint8_t *ws;
    if (scratch_cap) {
        const size_t sync_bytes = (KVM_FA_SYNC_WORDS * 4 + 255) & ~(size_t)255;
        const size_t avail = scratch_cap > sync_bytes ? scratch_cap - sync_bytes : 0;
        const size_t fit = avail / part_bytes;
        if (fit == 0)
            return kvm_fail(st, KVM_ERANGE, "fa_decode: the split flags and one key split's partials (%zu bytes) "
                            "exceed the %zu-byte scratch", sync_bytes + part_bytes, scratch_cap);
        if (a.n_splits > fit) a.n_splits = (uint32_t)fit;
        a.sync = (uint32_t *)scratch;
        ws = (uint8_t *)scratch + sync_bytes;
    } else {
        ws = (uint8_t *)kvm_fa_workspace(st, part_bytes * a.n_splits);
        if (!ws) return kvm_fail(st, KVM_ENOMEM, "fa_decode: workspace of %zu bytes", part_bytes * a.n_splits);
        a.sync = st->fa_sync;
    }
    const size_t n_part = (size_t)n_lanes * H * a.n_splits * rmax;
    a.ws = (float *)ws;
    a.ws_ml = a.ws + n_part * D;
    return KVM_OK;
}

// One launch on `stream`.  Every launch of a (lane, head) takes the next epoch
// from the device (a graph replay too): a split flag equals it only once this
// launch has completed that split (flags and epochs start at 0).
static int fa_launch(kvm_state *st, fa_plan &fp, hipStream_t stream) {
    KVM_HIP(st, hipSetDevice(st->device));
    if (fp.D == 256) launch_decode_d<256>(fp.a, fp.n_lanes, fp.rows, fp.quant, stream);
    else launch_decode_d<128>(fp.a, fp.n_lanes, fp.rows, fp.quant, stream);
    KVM_LAUNCH_CHECK(st, "fa_decode");
    return KVM_OK;
}

static int fa_decode_impl(kvm_state *st, const kvm_lane *lanes, uint32_t n_lanes, int q_type,
                          uint32_t n_head, float scale, void *scratch = nullptr, size_t scratch_cap = 0) {
    fa_plan fp;
    int rc = fa_prepare(st, lanes, n_lanes, q_type, n_head, scale, scratch, scratch_cap, &fp);
    if (rc || fp.rows == 0) return rc;
    return fa_launch(st, fp, st->stream);
}

size_t kvm_fa_sync_bytes() { return KVM_FA_SYNC_WORDS * sizeof(uint32_t); }

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

// ---------------------------------------------------------------------------
// Stage-in and decode attention in one launch
// ---------------------------------------------------------------------------
template <int D, int NRT, bool PK>
static const void *staged_kernel() { return (const void *)k_fa_decode_staged<D, NRT, PK>; }

static const void *staged_kernel_for(uint32_t D, uint32_t max_rows) {
    const int NRT = max_rows <= 16 ? 1 : 2;
    const bool pk = max_rows - 16u * (NRT - 1) <= 8u;
    if (D == 256) return NRT == 1 ? (pk ? staged_kernel<256, 1, true>() : staged_kernel<256, 1, false>())
                                  : (pk ? staged_kernel<256, 2, true>() : staged_kernel<256, 2, false>());
    return NRT == 1 ? (pk ? staged_kernel<128, 1, true>() : staged_kernel<128, 1, false>())
                    : (pk ? staged_kernel<128, 2, true>() : staged_kernel<128, 2, false>());
}

extern "C" int kvm_stagein_fa_decode_lanes(kvm_state *st, const kvm_stagein_lane *stage, const kvm_lane *lanes,
                                           uint32_t n_lanes, const kvm_rope_params *rope, int q_type,
                                           uint32_t n_head, float scale) {
    if (!st) return KVM_EINVAL;
    if (!stage || !lanes || n_lanes == 0) return kvm_fail(st, KVM_EINVAL, "stagein_fa_decode: no lanes");
    if (n_lanes > KVM_MAX_LANES) return kvm_fail(st, KVM_ERANGE, "stagein_fa_decode: %u lanes > %d", n_lanes, KVM_MAX_LANES);
    for (uint32_t i = 0; i < n_lanes; ++i) {
        if (!stage[i].w || !lanes[i].w) return kvm_fail(st, KVM_EINVAL, "stagein_fa_decode: lane %u: null window", i);
        if (stage[i].w->k != lanes[i].w->k || stage[i].w->v != lanes[i].w->v || stage[i].w->cell_pos != lanes[i].w->cell_pos)
            return kvm_fail(st, KVM_EINVAL, "stagein_fa_decode: lane %u stages another window than it attends", i);
    }
    fa_staged_args sa{};
    stage_lanes stl;
    uint32_t max_items = 0;
    size_t lds = 0;
    int rc = kvm_stage_prepare(st, stage, n_lanes, rope, &stl, &max_items, &lds);
    if (rc) return rc;
    lds = lds * KVM_FA_STAGE_IT / 64;                     // kvm_stage_prepare sizes 64-token items
    // every workgroup resident at once: the plan's barriers wait for all of a lane's
    uint32_t max_rows = 0;
    for (uint32_t i = 0; i < n_lanes; ++i)
        if (lanes[i].w->n_head_kv && n_head % lanes[i].w->n_head_kv == 0) {
            const uint32_t r = lanes[i].n_tokens * (n_head / lanes[i].w->n_head_kv);
            max_rows = r > max_rows ? r : max_rows;
        }
    const void *fn = staged_kernel_for(lanes[0].w->head_dim, max_rows ? max_rows : 1u);
    KVM_HIP(st, hipSetDevice(st->device));
    int occ = 0;
    rc = kvm_resident_blocks(st, fn, 512, lds, &occ);
    if (rc) return rc;
    // (and no lane with more workgroups than its barrier words count)
    uint64_t cap = (uint64_t)occ * st->n_cu;
    if (cap > (uint64_t)KVM_STAGE_MAX_WGS * n_lanes) cap = (uint64_t)KVM_STAGE_MAX_WGS * n_lanes;
    fa_plan fp;
    rc = fa_prepare(st, lanes, n_lanes, q_type, n_head, scale, nullptr, 0, &fp, (uint32_t)cap);
    if (rc) return rc;
    // no query rows at all: the plans alone
    if (fp.rows == 0) return kvm_stage_launch(st, stl, n_lanes, max_items, lds * 64 / KVM_FA_STAGE_IT, lanes[0].w->head_dim);
    if (!fp.quant) return kvm_fail(st, KVM_EUNSUPPORTED, "stagein_fa_decode: q8_0 windows only");
    sa.a = fp.a;
    for (uint32_t i = 0; i < n_lanes; ++i) sa.stage[i] = stl.lane[i];
    void *kargs[] = {&sa};
    KVM_HIP(st, hipLaunchKernel(fn, dim3(fp.a.n_splits, fp.a.H, n_lanes), dim3(512), kargs, lds, st->stream));
    return KVM_OK;
}

extern "C" int kvm_stagein_fa_decode(kvm_state *st, const kvm_history *h, const kvm_selection *sel,
                                     const kvm_rope_params *rope, const kvm_window *w, const void *q, int q_type,
                                     const int32_t *q_pos, uint32_t n_tokens, uint32_t n_head, float scale,
                                     float *out) {
    const kvm_stagein_lane sg{h, w, sel};
    const kvm_lane lane{w, q, q_pos, out, n_tokens};
    return kvm_stagein_fa_decode_lanes(st, &sg, &lane, 1, rope, q_type, n_head, scale);
}

// ---------------------------------------------------------------------------
// A whole decode step in two launches: the scoring grid, then one launch whose
// selector workgroups pick each lane's blocks while its attention workgroups
// attend over the window as it is; a lane whose plan stages anything is staged
// by its attention workgroups, which then attend again.
// ---------------------------------------------------------------------------
template <int D, int NRT, bool PK>
static const void *select_kernel(bool q4) {
    return q4 ? (const void *)k_fa_decode_select<D, NRT, PK, KVM_KQ_Q4>
              : (const void *)k_fa_decode_select<D, NRT, PK, KVM_KQ_Q8>;
}

static const void *select_kernel_for(uint32_t D, uint32_t max_rows, bool q4) {
    const int NRT = max_rows <= 16 ? 1 : 2;
    const bool pk = max_rows - 16u * (NRT - 1) <= 8u;
    if (D == 256) return NRT == 1 ? (pk ? select_kernel<256, 1, true>(q4) : select_kernel<256, 1, false>(q4))
                                  : (pk ? select_kernel<256, 2, true>(q4) : select_kernel<256, 2, false>(q4));
    return NRT == 1 ? (pk ? select_kernel<128, 1, true>(q4) : select_kernel<128, 1, false>(q4))
                    : (pk ? select_kernel<128, 2, true>(q4) : select_kernel<128, 2, false>(q4));
}

// The decode step's selecting launch over prepared top-k arguments (tl: from
// the scoring grid's layer contributions, or from caller scores); ret_score:
// the retrieval lanes to score first (a launch of the scoring grid ahead of
// it), or NULL when the scores are the caller's.  A step the selecting launch
// does not take runs as separate launches with the same results.
static int select_fa_launch(kvm_state *st, const kvm_retrieval_lane *ret_score, const topk_lanes &tl,
                            const kvm_window *const *wins, const kvm_selection *const *sels,
                            const uint32_t *n_blocks, const kvm_history *const *hist, const kvm_lane *lanes,
                            uint32_t n_lanes, const kvm_rope_params *rope, int q_type, uint32_t n_head, float scale,
                            const char *what) {
    kvm_stagein_lane sg[KVM_MAX_LANES];
    for (uint32_t i = 0; i < n_lanes; ++i) {
        const kvm_window *w = wins[i];
        if (!w || !lanes[i].w) return kvm_fail(st, KVM_EINVAL, "%s: lane %u: null window", what, i);
        if (w->k != lanes[i].w->k || w->v != lanes[i].w->v || w->cell_pos != lanes[i].w->cell_pos)
            return kvm_fail(st, KVM_EINVAL, "%s: lane %u selects for another window than it attends", what, i);
        sg[i] = kvm_stagein_lane{hist[i], w, sels[i]};
    }
    // every argument is checked before the first launch
    stage_lanes stl;
    uint32_t max_items = 0;
    size_t lds = 0;
    int rc = kvm_stage_prepare(st, sg, n_lanes, rope, &stl, &max_items, &lds);
    if (rc) return rc;
    // the selecting launch takes lanes that all have query rows, at most
    // KVM_SEL_MAXB blocks each and quantised (q8_0 or q4_0 K) windows; other
    // steps take the separate launches (scoring, top-k, stage-in + attention)
    bool fuse = kvm_k_quant(lanes[0].w->k_type);
    uint32_t max_rows = 0;
    for (uint32_t i = 0; i < n_lanes; ++i) {
        const kvm_window *w = lanes[i].w;
        const uint32_t r = w->n_head_kv && n_head % w->n_head_kv == 0 ? lanes[i].n_tokens * (n_head / w->n_head_kv) : 0u;
        fuse = fuse && r > 0 && n_blocks[i] <= KVM_SEL_MAXB && w->k_type == lanes[0].w->k_type;
        max_rows = r > max_rows ? r : max_rows;
    }
    size_t lds_sel = lds * KVM_FA_STAGE_IT / 64;           // kvm_stage_prepare sizes 64-token items
    if (lds_sel < sizeof(sel_lds)) lds_sel = sizeof(sel_lds);
    const void *fn = nullptr;
    fa_plan fp;
    if (fuse) {
        fn = select_kernel_for(lanes[0].w->head_dim, max_rows, lanes[0].w->k_type == KVM_TYPE_Q4_0);
        KVM_HIP(st, hipSetDevice(st->device));
        int occ = 0;
        rc = kvm_resident_blocks(st, fn, 512, lds_sel, &occ);
        if (rc) return rc;
        // every workgroup resident at once, the selector column included (and
        // no lane with more workgroups than its barrier words count: the
        // column stages too)
        const uint64_t cap = (uint64_t)occ * st->n_cu, sel_wgs = (uint64_t)lanes[0].w->n_head_kv * n_lanes;
        fuse = cap > 2 * sel_wgs;
        if (fuse) {
            uint64_t att = cap - sel_wgs;
            const uint64_t bar = (uint64_t)(KVM_STAGE_MAX_WGS - lanes[0].w->n_head_kv) * n_lanes;
            if (att > bar) att = bar;
            // (the selector column's flag takes slot n_splits of the head's
            // KVM_MAX_SPLITS, and the merge polls n_splits + 1 flags)
            rc = fa_prepare(st, lanes, n_lanes, q_type, n_head, scale, nullptr, 0, &fp, (uint32_t)att,
                            KVM_MAX_SPLITS - 1);
            if (rc) return rc;
        }
    }
    if (!fuse) {
        rc = fa_prepare(st, lanes, n_lanes, q_type, n_head, scale, nullptr, 0, &fp);
        if (rc) return rc;
        if (fp.rows && !fp.quant) return kvm_fail(st, KVM_EUNSUPPORTED, "%s: q8_0 or q4_0 K windows only", what);
        if (ret_score) {
            rc = kvm_retrieval_score(st, ret_score, n_lanes, tl);
            if (rc) return rc;
        }
        rc = kvm_topk_launch(st, tl, n_lanes);
        if (rc) return rc;
        return kvm_stagein_fa_decode_lanes(st, sg, lanes, n_lanes, rope, q_type, n_head, scale);
    }
    if (ret_score) {
        rc = kvm_retrieval_score(st, ret_score, n_lanes, tl);
        if (rc) return rc;
    }
    fa_select_args sa{};
    sa.a = fp.a;
    for (uint32_t i = 0; i < n_lanes; ++i) {
        sa.stage[i] = stl.lane[i];
        sa.sel[i] = tl.lane[i];
    }
    void *kargs[] = {&sa};
    KVM_HIP(st, hipLaunchKernel(fn, dim3(fp.a.n_splits + 1, fp.a.H, n_lanes), dim3(512), kargs, lds_sel, st->stream));
    return KVM_OK;
}

extern "C" int kvm_score_topk_stagein_fa_decode_lanes(kvm_state *st, const kvm_retrieval_lane *ret,
                                                      const kvm_history *const *hist, const kvm_lane *lanes,
                                                      uint32_t n_lanes, const kvm_rope_params *rope, int q_type,
                                                      uint32_t n_head, float scale) {
    if (!st) return KVM_EINVAL;
    if (!ret || !hist || !lanes || n_lanes == 0) return kvm_fail(st, KVM_EINVAL, "score_topk_stagein_fa_decode: no lanes");
    if (n_lanes > KVM_MAX_LANES)
        return kvm_fail(st, KVM_ERANGE, "score_topk_stagein_fa_decode: %u lanes > %d", n_lanes, KVM_MAX_LANES);
    const kvm_window *wins[KVM_MAX_LANES];
    const kvm_selection *sels[KVM_MAX_LANES];
    uint32_t nb[KVM_MAX_LANES];
    for (uint32_t i = 0; i < n_lanes; ++i) {
        wins[i] = ret[i].w;
        sels[i] = ret[i].out;
        nb[i] = ret[i].p ? ret[i].p->n_blocks : 0u;
    }
    topk_lanes tl;
    int rc = kvm_retrieval_prepare(st, ret, n_lanes, &tl);
    if (rc) return rc;
    return select_fa_launch(st, ret, tl, wins, sels, nb, hist, lanes, n_lanes, rope, q_type, n_head, scale,
                            "score_topk_stagein_fa_decode");
}

extern "C" int kvm_select_topk_stagein_fa_decode(kvm_state *st, const double *scores, const kvm_select_params *p,
                                                 const kvm_window *w, const kvm_selection *sel, const kvm_history *h,
                                                 const kvm_rope_params *rope, const void *q, int q_type,
                                                 const int32_t *q_pos, uint32_t n_tokens, uint32_t n_head,
                                                 float scale, float *out) {
    if (!st) return KVM_EINVAL;
    topk_lanes tl{};
    int rc = kvm_select_prepare(st, scores, p, w, sel, &tl.lane[0]);
    if (rc) return rc;
    const kvm_lane lane{w, q, q_pos, out, n_tokens};
    return select_fa_launch(st, nullptr, tl, &w, &sel, &p->n_blocks, &h, &lane, 1, rope, q_type, n_head, scale,
                            "select_topk_stagein_fa_decode");
}

extern "C" int kvm_score_topk_stagein_fa_decode(kvm_state *st, const kvm_meank_index *ix, const kvm_query_acc *qa,
                                                const kvm_select_params *p, const kvm_window *w,
                                                const kvm_selection *sel, const kvm_history *h,
                                                const kvm_rope_params *rope, const void *q, int q_type,
                                                const int32_t *q_pos, uint32_t n_tokens, uint32_t n_head,
                                                float scale, float *out) {
    const kvm_retrieval_lane ret{ix, qa, p, w, sel};
    const kvm_lane lane{w, q, q_pos, out, n_tokens};
    return kvm_score_topk_stagein_fa_decode_lanes(st, &ret, &h, &lane, 1, rope, q_type, n_head, scale);
}

// ---------------------------------------------------------------------------
// Allocation-free decode: the split partials live in a fixed device array
// instead of the state's workspace.  Each device holds its own copy of the
// array (KVM_NOALLOC_SCRATCH_BYTES, until the process ends); its address on a
// device is looked up once, with that device current, when the first state on
// the device is created, and only that address is handed to kernels.
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint8_t scratch[KVM_NOALLOC_SCRATCH_BYTES];

#define KVM_MAX_DEVICES 64
static void *g_scratch_ptr[KVM_MAX_DEVICES];
static std::mutex g_scratch_mu;

int kvm_noalloc_setup(kvm_state *st) {
    if (st->device < 0 || st->device >= KVM_MAX_DEVICES)
        return kvm_fail(st, KVM_ERANGE, "noalloc: device %d beyond %d", st->device, KVM_MAX_DEVICES);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[st->device]) {
        void *ptr = nullptr;
        KVM_HIP(st, hipSetDevice(st->device));
        KVM_HIP(st, hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (!ptr) return kvm_fail(st, KVM_EHIP, "noalloc: scratch has no address on device %d", st->device);
        g_scratch_ptr[st->device] = ptr;
    }
    st->scratch = g_scratch_ptr[st->device];
    return KVM_OK;
}

extern "C" int kvm_fa_decode_noalloc(kvm_state *st, const kvm_window *w, const void *q, int q_type,
                                     const int32_t *q_pos, uint32_t n_tokens, uint32_t n_head, float scale,
                                     float *out) {
    if (!st) return KVM_EINVAL;
    if (!st->scratch) return kvm_fail(st, KVM_EHIP, "fa_decode_noalloc: scratch not set up on device %d", st->device);
    kvm_lane lane{w, q, q_pos, out, n_tokens};
    st->used_scratch = true;
    return fa_decode_impl(st, &lane, 1, q_type, n_head, scale, st->scratch, KVM_NOALLOC_SCRATCH_BYTES);
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
