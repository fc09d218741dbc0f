// kvm_internal.h -- shared definitions of the gfx950 hot-path library:
// state object, error plumbing, the tiled window layout and small device helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "../../include/kvm_hotpath.h"

// ---------------------------------------------------------------------------
// Execution state (one per execution domain; replaces kvmem_gpu_state,
// src/adapter/llama-kvmem-stagein.cu:324-354).
// ---------------------------------------------------------------------------
struct kvm_stage_item {          // one queued enqueue_k / enqueue_v
    uint32_t kind;               // 0 = K (re-RoPE chain), 1 = V (byte move)
    uint32_t cell0;              // first window cell
    uint32_t nt;                 // tokens
    int32_t pos0;                // RoPE position of the first token (K)
    uint64_t off;                // byte offset of the packed rows in the slab
    kvm_window w;                // destination window
    uint32_t n_rot;              // RoPE dims (K)
    int32_t nrot;                // Hadamard width, 0 = off (K)
};

// Device sync words of the decode attention (kvm_state::fa_sync, or the head of
// the allocation-free entry point's scratch array), in 32-bit words:
//   [lane][head][split]          the epoch of the last launch that completed the split
//   KVM_FA_SYNC_STATUS           sticky status of the waits that gave up (KVM_WAIT_*)
//   KVM_FA_SYNC_EPOCH + lane*64+h  the (lane, head)'s epoch
//   KVM_FA_SYNC_PLAN, 64-bit [lane*64+h]  the plan a selecting launch published
#define KVM_MAX_LANES 8
#define KVM_LDS_PER_CU 163840u     // LDS bytes of one CU (gfx950)
#define KVM_FA_MAX_HEADS 64
#define KVM_MAX_SPLITS 512
#define KVM_FA_SYNC_STATUS (KVM_MAX_LANES * KVM_FA_MAX_HEADS * KVM_MAX_SPLITS)
#define KVM_FA_SYNC_EPOCH (KVM_FA_SYNC_STATUS + 64)
#define KVM_FA_SYNC_PLAN (KVM_FA_SYNC_EPOCH + KVM_MAX_LANES * KVM_FA_MAX_HEADS)
#define KVM_FA_SYNC_WORDS (KVM_FA_SYNC_PLAN + 2 * KVM_MAX_LANES * KVM_FA_MAX_HEADS)
static_assert(KVM_FA_SYNC_PLAN % 2 == 0, "64-bit plan words");

struct kvm_state {
    int device = 0;
    uint32_t n_cu = 256;         // compute units of the device (launch sizing)
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    std::string err;
    // growable device workspace (attention partials, top-k scratch, tables)
    void *ws = nullptr;
    size_t ws_bytes = 0;
    // RoPE cos/sin table: [n_pos][n_rot/2] float2, generated on the host
    float2 *rope_tab = nullptr;
    size_t rope_tab_bytes = 0;
    uint32_t rope_n_pos = 0, rope_n_half = 0;
    std::vector<float> rope_theta;  // theta_i the current table was built from
    // pinned slab for the enqueue/flush API (32 MiB like the reference's slab)
    uint8_t *slab = nullptr;
    size_t slab_bytes = 0, slab_used = 0;
    bool slab_busy = false;      // a flush's kernels may still read the slab
    std::vector<kvm_stage_item> items;
    std::vector<float> theta;    // theta of the queued K items
    // small device buffer for item descriptors / lane tables
    void *desc = nullptr;
    size_t desc_bytes = 0;
    hipEvent_t ev = nullptr;
    // device address of the fixed scratch array of the allocation-free entry
    // point on this state's device (kvm_noalloc_setup)
    void *scratch = nullptr;
    // per-split arrival flags of the decode attention's in-launch split merge
    // (each holds the epoch of the last launch that completed the split) and
    // its status word, kvm_fa_sync_bytes()
    uint32_t *fa_sync = nullptr;
    // attention workspace (split partials), apart from `ws`, whose retrieval
    // outputs a decode step's attention must not overwrite
    void *fa_ws = nullptr;
    size_t fa_ws_bytes = 0;
    // staging of the blocks a stage-in plan moves within the window (their
    // shadow K rows and V rows, gathered before any slot is written)
    void *mv_ws = nullptr;
    size_t mv_ws_bytes = 0;
    // the stage-in's per-lane barrier words (epoch, go, failure, arrivals),
    // KVM_STAGE_SYNC_BYTES, zero at creation
    uint32_t *stage_sync = nullptr;
    // polls of an in-launch wait before it gives up (kvm_state_set_wait_polls;
    // 0: every such wait gives up at once)
    uint32_t wait_polls = KVM_WAIT_POLLS_DEFAULT;
    // the allocation-free entry point ran on this state (its sync words and
    // status word live in the device's scratch array)
    bool used_scratch = false;
};

#define KVM_STAGE_MAX_WGS 1024                      // stage-in workgroups of one lane
#define KVM_STAGE_SYNC_LANE (64 + KVM_STAGE_MAX_WGS) // words per lane
#define KVM_STAGE_SYNC_BYTES (8 * KVM_STAGE_SYNC_LANE * 4)

// error helpers ----------------------------------------------------------------
int kvm_fail(kvm_state *st, int code, const char *fmt, ...);
#define KVM_HIP(st, expr)                                                          \
    do {                                                                           \
        hipError_t e__ = (expr);                                                   \
        if (e__ != hipSuccess)                                                     \
            return kvm_fail((st), KVM_EHIP, "%s: %s", #expr, hipGetErrorString(e__)); \
    } while (0)
#define KVM_LAUNCH_CHECK(st, what)                                                 \
    do {                                                                           \
        hipError_t e__ = hipGetLastError();                                        \
        if (e__ != hipSuccess)                                                     \
            return kvm_fail((st), KVM_EHIP, "%s launch: %s", (what), hipGetErrorString(e__)); \
    } while (0)

// Looks up (once per device) the address of the allocation-free entry point's
// scratch array on the state's device and records it in st->scratch.
int kvm_noalloc_setup(kvm_state *st);
// Bytes of the decode attention's counter block (kvm_state::fa_sync).
size_t kvm_fa_sync_bytes();
// Ensures the state's workspace holds at least `bytes`; returns it or nullptr.
void *kvm_workspace(kvm_state *st, size_t bytes);
// The same for the attention workspace (kvm_state::fa_ws).
void *kvm_fa_workspace(kvm_state *st, size_t bytes);
// The same for the stage-in move staging (kvm_state::mv_ws).
void *kvm_move_workspace(kvm_state *st, size_t bytes);
// Workgroups of `threads` threads and `lds` bytes of dynamic LDS of kernel fn
// that one CU holds at once (>= 1, or an error); also raises fn's dynamic LDS
// limit to lds.  Cached per (kernel, threads, lds).
int kvm_resident_blocks(kvm_state *st, const void *fn, int threads, size_t lds, int *blocks);
// Ensures a device copy of `bytes` of descriptor data; returns the device pointer.
void *kvm_upload_desc(kvm_state *st, const void *host, size_t bytes);
// theta_i = powf(base, -2i/n_rot) * scale for i < n_rot/2 (kvmem/src/host/rope.cpp:19-22)
std::vector<float> kvm_rope_theta(float freq_base, float freq_scale, uint32_t n_rot);
// Ensures the (cos, sin) table for `theta` covers positions [0, n_pos).
int kvm_rope_table(kvm_state *st, const float *theta, uint32_t n_half, uint32_t n_pos);

// ---------------------------------------------------------------------------
// Tiled window layout.  Per kv head, cells are grouped in tiles of 64; the K
// and V of one (head, tile) are contiguous and ordered as the attention
// kernel's matrix-core operands are loaded, so every wave load is a fully
// coalesced 16-byte-per-lane access.
//
// q8_0 K tile (head_dim D, NB = D/32 blocks):
//   quants  64*D bytes: [sub 4][pair NB/2][lane 64][16 B]; lane l = 16g + m
//           holds key 16*sub + m, dims 32*(2p)+8g..+7 then 32*(2p+1)+8g..+7
//   scales  64*NB fp16: [sub 4][block NB][m 16] = key 16*sub + m (a lane of
//           the 4-block scale MFMA reads 128 contiguous bytes per 4 blocks)
// q4_0 V tile:
//   nibbles D*32 bytes: for dim d, key c = 32ks + 8g + j: 4-byte word
//           ((d/16)*64 + 16g + d%16)*8 + 4ks holds keys j = 0..7 of (d, g, ks),
//           key j in byte j%4, low nibble for j < 4 and high nibble for
//           j >= 4 (so masking the low / shifted high nibbles gives keys 0..3 /
//           4..7 in byte order); a lane (dim d%16, key group g) reads both ks
//           words as one 8-byte access
//   scales  NB*64 fp16: [block NB][ks 2][g 4][j 8]
// f16 K tile: [sub 4][kstep D/32][lane 64][8 halves] = key 16*sub+m, dims 32ks+8g..+7
// f16 V tile: halves ((d/16)*64 + 16g + d%16)*16 + 8ks + j (same key order as q4_0)
// ---------------------------------------------------------------------------
// A quantised K window (q8_0, or q4_0 held as q8_0: the nibble minus 8 as an
// int8 quant under the block's fp16 scale, so the attention reads one tile
// format and computes ggml's q4_0 x q8_0 integer dot exactly).
__host__ __device__ inline bool kvm_k_quant(int ktype) { return ktype == KVM_TYPE_Q8_0 || ktype == KVM_TYPE_Q4_0; }
__host__ __device__ inline uint32_t kvm_ktile_bytes(int ktype, uint32_t D) {
    return kvm_k_quant(ktype) ? 64u * D + 64u * (D / 32u) * 2u : 64u * D * 2u;
}
__host__ __device__ inline uint32_t kvm_vtile_bytes(int vtype, uint32_t D) {
    return vtype == KVM_TYPE_Q4_0 ? D * 32u + (D / 32u) * 64u * 2u : 64u * D * 2u;
}
// byte offset, inside a q8_0 K tile, of quant (cell c in [0,64), dim d)
__host__ __device__ inline uint32_t kvm_kq_off(uint32_t D, uint32_t c, uint32_t d) {
    const uint32_t s = c >> 4, m = c & 15u, b = d >> 5, g = (d & 31u) >> 3, j = d & 7u;
    const uint32_t l = 16u * g + m;
    return (((s * (D / 64u) + (b >> 1)) * 64u + l) << 4) + (b & 1u) * 8u + j;
}
// byte offset of the fp16 scale of (cell c, block b) inside a q8_0 K tile
__host__ __device__ inline uint32_t kvm_kd_off(uint32_t D, uint32_t c, uint32_t b) {
    const uint32_t s = c >> 4, m = c & 15u;
    return 64u * D + (((s * (D / 32u) + b) * 16u + m) << 1);
}
// byte offset of the 4-byte nibble word holding keys 32ks+8g .. +7 of dim d
__host__ __device__ inline uint32_t kvm_vq_word(uint32_t d, uint32_t g, uint32_t ks) {
    return ((((d >> 4) * 64u + 16u * g + (d & 15u)) << 3) + (ks << 2));
}
// byte offset and nibble shift of (cell c, dim d) inside a q4_0 V tile
__host__ __device__ inline uint32_t kvm_vq_byte(uint32_t c, uint32_t d) {
    return kvm_vq_word(d, (c & 31u) >> 3, c >> 5) + (c & 3u);
}
__host__ __device__ inline uint32_t kvm_vq_shift(uint32_t c) { return c & 4u; }
// bit position of key j (0..7) inside its 4-byte nibble word
__host__ __device__ inline uint32_t kvm_vq_nib_shift(uint32_t j) { return ((j & 3u) << 3) | (j & 4u); }
__host__ __device__ inline uint32_t kvm_vd_off(uint32_t D, uint32_t c, uint32_t b) {
    const uint32_t ks = c >> 5, g = (c & 31u) >> 3, j = c & 7u;
    return D * 32u + ((((b * 2u + ks) * 4u + g) * 8u + j) << 1);
}
// f16 K tile: half index of (cell c, dim d)
__host__ __device__ inline uint32_t kvm_kh_idx(uint32_t D, uint32_t c, uint32_t d) {
    const uint32_t s = c >> 4, m = c & 15u, ks = d >> 5, g = (d & 31u) >> 3, j = d & 7u;
    return ((s * (D / 32u) + ks) * 64u + 16u * g + m) * 8u + j;
}
// f16 V tile: half index of (cell c, dim d)
__host__ __device__ inline uint32_t kvm_vh_idx(uint32_t c, uint32_t d) {
    const uint32_t ks = c >> 5, g = (c & 31u) >> 3, j = c & 7u;
    return ((((d >> 4) * 64u + 16u * g + (d & 15u)) * 2u + ks) << 3) + j;
}

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
typedef int32_t kvm_i32x4 __attribute__((ext_vector_type(4)));
typedef float kvm_f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 kvm_f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 kvm_f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 kvm_f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t kvm_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t kvm_u32x2 __attribute__((ext_vector_type(2)));

// Bulk data handed between workgroups of one launch, which may sit on
// different XCDs, each with its own L2: 16-byte stores written through past
// the writer's L2 and 16-byte loads that miss the reader's L2 (the agent-scope
// cache policy, sc1), so the flag that orders them needs no write-back or
// invalidation of whole caches (as the split partials' 4-byte agent-scope
// accesses).  Offsets from the base are below 2 GiB.
#define KVM_CPOL_SC1 16
__device__ __forceinline__ __amdgpu_buffer_rsrc_t kvm_rsrc(const void *base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ kvm_u32x4 kvm_ld16_dev(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, KVM_CPOL_SC1);
}
__device__ __forceinline__ void kvm_st16_dev(__amdgpu_buffer_rsrc_t r, uint32_t off, kvm_u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, 0, KVM_CPOL_SC1);
}

__device__ inline float kvm_h2f(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}
// Inclusive prefix sum over a wave64 with DPP: Kogge-Stone row shifts within
// each 16-lane row, then row broadcasts of lane 15 (to rows 1, 3) and lane 31
// (to rows 2, 3).
__device__ inline uint32_t kvm_wave_incl_scan(uint32_t x) {
    x += __builtin_amdgcn_update_dpp(0u, x, 0x111, 0xf, 0xf, true);   // row_shr:1
    x += __builtin_amdgcn_update_dpp(0u, x, 0x112, 0xf, 0xf, true);   // row_shr:2
    x += __builtin_amdgcn_update_dpp(0u, x, 0x114, 0xf, 0xf, true);   // row_shr:4
    x += __builtin_amdgcn_update_dpp(0u, x, 0x118, 0xf, 0xf, true);   // row_shr:8
    x += __builtin_amdgcn_update_dpp(0u, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
    x += __builtin_amdgcn_update_dpp(0u, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return x;
}
// Max / min / sum of a float over the wave (DPP row shifts and broadcasts as in
// kvm_wave_incl_scan; lanes without a source contribute the identity), read back
// from lane 63 to every lane.
// Workgroup barrier that orders LDS traffic only: it waits for this wave's LDS
// operations but not for its outstanding global loads or stores (a
// __syncthreads fence would drain a tile prefetch and serialise the pipeline).
#define KVM_LDS_BARRIER() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")

#define KVM_WAVE_REDUCE_F32(NAME, OP, IDENT)                                                          \
    __device__ inline float NAME(float x) {                                                          \
        const int id = __float_as_int(IDENT);                                                        \
        x = OP(x, __int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(x), 0x111, 0xf, 0xf, false))); \
        x = OP(x, __int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(x), 0x112, 0xf, 0xf, false))); \
        x = OP(x, __int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(x), 0x114, 0xf, 0xf, false))); \
        x = OP(x, __int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(x), 0x118, 0xf, 0xf, false))); \
        x = OP(x, __int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(x), 0x142, 0xa, 0xf, false))); \
        x = OP(x, __int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(x), 0x143, 0xc, 0xf, false))); \
        return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));                     \
    }
__device__ inline float kvm_add_f32(float a, float b) { return a + b; }
KVM_WAVE_REDUCE_F32(kvm_wave_max_f32, fmaxf, -INFINITY)
KVM_WAVE_REDUCE_F32(kvm_wave_min_f32, fminf, INFINITY)
KVM_WAVE_REDUCE_F32(kvm_wave_sum_f32, kvm_add_f32, 0.0f)
#undef KVM_WAVE_REDUCE_F32
// Unsigned minimum over the wave, the same way.
__device__ inline uint32_t kvm_wave_min_u32(uint32_t x) {
    const int id = -1;                    // 0xffffffff, the identity
    auto mn = [](uint32_t a, int b) { return a < (uint32_t)b ? a : (uint32_t)b; };
    x = mn(x, __builtin_amdgcn_update_dpp(id, (int)x, 0x111, 0xf, 0xf, false));
    x = mn(x, __builtin_amdgcn_update_dpp(id, (int)x, 0x112, 0xf, 0xf, false));
    x = mn(x, __builtin_amdgcn_update_dpp(id, (int)x, 0x114, 0xf, 0xf, false));
    x = mn(x, __builtin_amdgcn_update_dpp(id, (int)x, 0x118, 0xf, 0xf, false));
    x = mn(x, __builtin_amdgcn_update_dpp(id, (int)x, 0x142, 0xa, 0xf, false));
    x = mn(x, __builtin_amdgcn_update_dpp(id, (int)x, 0x143, 0xc, 0xf, false));
    return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}
// Max / sum with lane l ^ 16 or l ^ 32 without LDS: v_permlane16_swap /
// v_permlane32_swap with both operands x hand each lane the pair {x[l],
// x[l ^ 16 or 32]} (order unspecified; max and + do not care).
__device__ inline float kvm_max_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float kvm_max_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float kvm_add_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// x of lane l ^ 8 (DPP row_ror:8: a rotation by 8 within each row of 16 lanes)
__device__ inline float kvm_ror8_f32(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false));
}
__device__ inline float kvm_add_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// IEEE round-to-nearest-even fp32 -> fp16 (v_cvt_f16_f32 under the default mode).
// The empty asm keeps the conversion a separate instruction: fused with its
// producer (fptrunc(x * c) -> v_fma_mix(x, c, +0)) a -0.0 result turns into +0.0.
__device__ inline uint16_t kvm_f2h(float f) {
    asm volatile("" : "+v"(f));
    _Float16 v = (_Float16)f;
    uint16_t h;
    __builtin_memcpy(&h, &v, 2);
    return h;
}
__device__ inline float kvm_bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// IEEE binary32 operations, round to nearest even.  Hardware add/sub/mul round
// to nearest even; `/` and sqrtf are correctly rounded under
// -fhip-fp32-correctly-rounded-divide-sqrt.  Each one is its own rounding: no
// a*b+c built from them becomes an FMA, whatever the file's -ffp-contract
// (files whose results must equal host arithmetic bit for bit are also built
// with -ffp-contract=off).  (HIP's kvm_fsqrt is the approximate native sqrt.)
__device__ __forceinline__ float kvm_fadd(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}
__device__ __forceinline__ float kvm_fsub(float a, float b) {
#pragma clang fp contract(off)
    return a - b;
}
__device__ __forceinline__ float kvm_fmul(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}
__device__ __forceinline__ float kvm_fdiv(float a, float b) {
#pragma clang fp contract(off)
    return a / b;
}
__device__ __forceinline__ float kvm_fsqrt(float a) { return sqrtf(a); }

// a / 127 rounded as the IEEE quotient, without the division sequence: q =
// a * RN(1/127) is within an ulp, the residual a - 127 q is exact in one fma,
// and q + residual * RN(1/127) in a second fma rounds to the quotient.  Equal
// to IEEE a / 127.0f for every finite float a but -0, which gives +0 (an amax
// is never -0); checked exhaustively.
__device__ __forceinline__ float kvm_div127(float a) {
    constexpr float C = 1.0f / 127.0f;
    const float q = kvm_fmul(a, C);
    return __builtin_fmaf(__builtin_fmaf(-q, 127.0f, a), C, q);
}
// d != 0 ? 1 / d : 0 with IEEE rounding.  For 2^-126 <= |d| < 2^126 one
// Newton step from v_rcp_f32 (y + y (1 - |d| y), both fma) equals the IEEE
// quotient: checked on gfx950 against the division for every float in that
// range.  Subnormal and huge |d| take the division itself.
__device__ __forceinline__ float kvm_recip_or0(float d) {
    const float a = fabsf(d);
    if (__builtin_expect(a >= 0x1p-126f && a < 0x1p126f, 1)) {
        const float y = __builtin_amdgcn_rcpf(a);
        return copysignf(__builtin_fmaf(__builtin_fmaf(-a, y, 1.0f), y, y), d);
    }
    return d != 0.0f ? kvm_fdiv(1.0f, d) : 0.0f;
}
// (int)roundf(y) (halves away from zero) for |y| < 2^23: |y| + 0.5 is exact
// there, and truncating it rounds |y|, except for the largest float below one
// half, whose sum rounds up to 1.0.  Equal to roundf for every such y (checked
// exhaustively).
__device__ __forceinline__ int kvm_round_away(float y) {
    const float a = fabsf(y);
    const float t = a == 0x1.fffffep-2f ? 0.0f : kvm_fadd(a, 0.5f);
    return (int)copysignf(t, y);
}

// q8_0 / q4_0 block quantisers with the reference kernels' exact arithmetic
// (llama-kvmem-stagein.cu:181-234): fp32 amax, d = amax/127 (q8) or vmax/-8
// (q4), id = d ? 1/d : 0, fp16 d with RNE, roundf (ties away) / (int)(x*id+8.5).
// Division and reciprocal round as host IEEE division does (kvm_div127,
// kvm_recip_or0; vmax * -0.125 is vmax / -8 exactly).
__device__ __forceinline__ void kvm_quant_block_q8_0(const float (&x)[32], uint16_t *d_out, int8_t *q) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
    const float d = kvm_div127(amax);
    const float id = kvm_recip_or0(d);
    *d_out = kvm_f2h(d);
    uint32_t packed[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint32_t wv = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k)
            wv |= (uint32_t)(uint8_t)kvm_round_away(kvm_fmul(x[4 * j + k], id)) << (8 * k);
        packed[j] = wv;
    }
    __builtin_memcpy(q, packed, 32);
}
__device__ __forceinline__ void kvm_quant_block_q4_0(const float (&x)[32], uint16_t *d_out, uint8_t *q) {
    float amax = 0.0f, vmax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const float a = fabsf(x[j]);
        if (amax < a) { amax = a; vmax = x[j]; }
    }
    const float d = kvm_fmul(vmax, -0.125f);
    const float id = kvm_recip_or0(d);
    *d_out = kvm_f2h(d);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        int x0 = (int)kvm_fadd(kvm_fmul(x[j], id), 8.5f);
        int x1 = (int)kvm_fadd(kvm_fmul(x[j + 16], id), 8.5f);
        x0 = x0 > 15 ? 15 : x0;
        x1 = x1 > 15 ? 15 : x1;
        q[j] = (uint8_t)((x0 & 15) | ((x1 & 15) << 4));
    }
}

inline uint32_t kvm_cdiv(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

// ---------------------------------------------------------------------------
// Captured views (kvm_view): element (token t, head hh, dim d) at byte
// t*nb2 + hh*nb1 + d*nb0, an fp32, fp16 or bf16 value, read as fp32.
// ---------------------------------------------------------------------------
struct view_args {
    const uint8_t *data;
    int type;
    uint32_t ne0;                // dims per head; embedding e = hh * ne0 + d
    size_t nb0, nb1, nb2;
};

__device__ inline float view_load(const view_args &v, uint32_t t, uint32_t e) {
    const uint8_t *p = v.data + (size_t)t * v.nb2 + (size_t)(e / v.ne0) * v.nb1 + (size_t)(e % v.ne0) * v.nb0;
    if (v.type == KVM_TYPE_F16) return kvm_h2f(*(const uint16_t *)p);
    if (v.type == KVM_TYPE_BF16) return kvm_bf2f(*(const uint16_t *)p);
    return *(const float *)p;
}

inline int view_check(kvm_state *st, const kvm_view *v, uint32_t n_embd, const char *what) {
    if (!v || !v->data) return kvm_fail(st, KVM_EINVAL, "%s: null view", what);
    if (v->type != KVM_TYPE_F32 && v->type != KVM_TYPE_F16 && v->type != KVM_TYPE_BF16)
        return kvm_fail(st, KVM_EUNSUPPORTED, "%s: view type %d", what, v->type);
    if (v->ne0 <= 0 || v->ne1 <= 0 || v->ne2 < 0 || (uint64_t)v->ne0 * (uint64_t)v->ne1 != n_embd)
        return kvm_fail(st, KVM_EINVAL, "%s: view of %lld x %lld values per token, expected %u", what,
                        (long long)v->ne0, (long long)v->ne1, n_embd);
    return KVM_OK;
}

inline view_args view_of(const kvm_view *v) {
    return view_args{(const uint8_t *)v->data, v->type, (uint32_t)v->ne0, v->nb0, v->nb1, v->nb2};
}
