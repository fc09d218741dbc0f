// kvm_stagein.hip -- fused stage-in: pinned-host history -> tiled window.
//
// K: dequant q8_0 -> NeoX RoPE at the window position -> normalised
// Walsh-Hadamard -> q8_0, the order of llama-kvmem-stagein.cu:731-786, fused in
// one pass with the row held in registers (one wave per (token, head) row,
// lane L owning dims DPL*L .. DPL*L+DPL-1).  Every operation is an explicitly
// rounded IEEE op, so the output bytes equal the host restatement's.
// V: q4_0 bytes are moved unchanged into the tiled layout (stagein.cu:733-744).
#include "kvm_internal.h"

#include <cmath>
#include <cstring>

struct rope_ctx {
    const float2 *tab;     // [n_pos][n_half] (cos, sin)
    uint32_t n_half;       // n_rot / 2
    uint32_t n_pos;
    int32_t nrot;          // Hadamard width, 0 = off
    float hscale;          // 1 / sqrtf(nrot), computed on the host as the reference does
};

// One (token, head) row of D dims: src = NB q8_0 blocks (34 B each) readable by
// every lane; writes the requantised row into K tile `kt` at cell c (0..63).
template <int D>
__device__ inline void stage_k_row(const uint8_t *src, uint8_t *kt, uint32_t c, int32_t pos,
                                   const rope_ctx &rc) {
    constexpr int DPL = D / 64;
    const int L = threadIdx.x & 63;
    const int d0 = DPL * L;
    const int b = d0 >> 5, e = d0 & 31;
    const uint8_t *blk = src + b * 34;
    const float dsc = kvm_h2f((uint16_t)(blk[0] | (blk[1] << 8)));
    float x[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) x[i] = (float)(int8_t)blk[2 + e + i] * dsc;

    // NeoX RoPE: dims i and i + n_half rotate together for i < n_half.
    const int nh = (int)rc.n_half;
    if (nh > 0) {
        const int pl = nh / DPL;                       // lane distance of the partner
        const bool lo = d0 < nh, hi = d0 >= nh && d0 < 2 * nh;
        float y[DPL];
#pragma unroll
        for (int i = 0; i < DPL; ++i) {
            const float up = __shfl(x[i], (L + pl) & 63, 64);
            const float dn = __shfl(x[i], (L - pl) & 63, 64);
            y[i] = lo ? up : dn;
        }
        if (lo || hi) {
            const float2 *cs = rc.tab + (size_t)pos * rc.n_half + (lo ? d0 : d0 - nh);
#pragma unroll
            for (int i = 0; i < DPL; ++i) {
                const float2 t = cs[i];
                if (lo)   // x0' = x0 c - x1 s
                    x[i] = kvm_fsub(kvm_fmul(x[i], t.x), kvm_fmul(y[i], t.y));
                else      // x1' = x0 s + x1 c
                    x[i] = kvm_fadd(kvm_fmul(y[i], t.y), kvm_fmul(x[i], t.x));
            }
        }
    }

    // normalised Walsh-Hadamard over nrot-wide chunks: pre-scale, then
    // butterflies h = 1, 2, ..., nrot/2 (stagein.cu:105-131)
    if (rc.nrot > 0) {
#pragma unroll
        for (int i = 0; i < DPL; ++i) x[i] = kvm_fmul(x[i], rc.hscale);
#pragma unroll
        for (int h = 1; h < DPL; h <<= 1) {
#pragma unroll
            for (int i = 0; i < DPL; ++i) {
                if (!(i & h)) {
                    const float a = x[i], bb = x[i + h];
                    x[i] = kvm_fadd(a, bb);
                    x[i + h] = kvm_fsub(a, bb);
                }
            }
        }
        for (int h = DPL; h < rc.nrot; h <<= 1) {
            const int lx = h / DPL;
            const bool first = (L & lx) == 0;
#pragma unroll
            for (int i = 0; i < DPL; ++i) {
                const float o = __shfl_xor(x[i], lx, 64);
                x[i] = first ? kvm_fadd(x[i], o) : kvm_fsub(o, x[i]);
            }
        }
    }

    // q8_0 requantisation of each 32-dim block (32/DPL lanes per block)
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) amax = fmaxf(amax, fabsf(x[i]));
#pragma unroll
    for (int o = 1; o < 32 / DPL; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    const float d = kvm_fdiv(amax, 127.0f);
    const float id = d != 0.0f ? kvm_fdiv(1.0f, d) : 0.0f;
    uint8_t *qd = kt + kvm_kq_off(D, c, d0);
#pragma unroll
    for (int i = 0; i < DPL; ++i) qd[i] = (uint8_t)(int8_t)roundf(kvm_fmul(x[i], id));
    if (e == 0) {
        const uint16_t h16 = kvm_f2h(d);
        uint8_t *sd = kt + kvm_kd_off(D, c, b);
        sd[0] = (uint8_t)h16;
        sd[1] = (uint8_t)(h16 >> 8);
    }
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
};


#define KVM_STAGEIN_WGS 256       // one per CU of an MI355X (the rows buffer takes most of the LDS)

// One workgroup per CU walks the (plan entry, 64-token tile) items, so an
// empty plan (the steady state) costs one short launch; the plan length is
// only known on the device (info[2]).
template <int D>
__device__ __forceinline__ void stagein_item(const stage_args &a, uint8_t *s_rows, uint32_t si, uint32_t tt) {
    constexpr uint32_t NB = D / 32;
    const uint32_t slot = a.stage_slots[si];
    const uint32_t id = a.ids[slot];
    const int32_t base = a.to_base[slot];
    // history blocks are consecutive block_tokens-sized runs (register_append,
    // kvmem_store.cpp:179-205): block id covers [id*bt, min((id+1)*bt, h_tokens))
    const uint64_t first = (uint64_t)id * a.bt;
    const uint32_t tid = threadIdx.x;
    if (first >= a.h_tokens) {
        if (tid == 0) atomicOr(&a.info[3], 4u);     // block outside the history: skip it
        return;
    }
    const uint32_t nt = a.h_tokens - first < a.bt ? (uint32_t)(a.h_tokens - first) : a.bt;
    const uint32_t t0 = tt * 64;
    const uint32_t count = nt > t0 ? (nt - t0 < 64 ? nt - t0 : 64) : 0;
    const uint64_t htok0 = first + t0;
    const uint32_t rowK = a.H * NB * 34, rowV = a.H * NB * 18;
    uint8_t *lk = s_rows, *lv = s_rows + 64 * rowK;
    // bulk copy of `count` consecutive token rows of K and V (contiguous in host memory)
    const uint8_t *gk = a.hk + htok0 * rowK, *gv = a.hv + htok0 * rowV;
    const uint32_t nk = count * rowK, nv = count * rowV;
    const bool al16 = (((uintptr_t)gk | (uintptr_t)gv | rowK | rowV) & 15u) == 0;
    if (al16) {
#pragma unroll 4
        for (uint32_t i = tid; i < nk / 16; i += 256) ((uint4 *)lk)[i] = ((const uint4 *)gk)[i];
#pragma unroll 4
        for (uint32_t i = tid; i < nv / 16; i += 256) ((uint4 *)lv)[i] = ((const uint4 *)gv)[i];
    } else {
        for (uint32_t i = tid; i < nk; i += 256) lk[i] = gk[i];
        for (uint32_t i = tid; i < nv; i += 256) lv[i] = gv[i];
    }
    __syncthreads();

    const uint32_t tile = (slot * a.bt + t0) / 64;
    // K rows: wave w takes rows (cell j, head h) = r, r + 4, ...
    const uint32_t wave = tid >> 6;
    for (uint32_t r = wave; r < count * a.H; r += 4) {
        const uint32_t j = r / a.H, h = r % a.H;
        uint8_t *kt = a.wk + ((uint64_t)h * a.n_tiles + tile) * kvm_ktile_bytes(KVM_TYPE_Q8_0, D);
        stage_k_row<D>(lk + j * rowK + h * NB * 34, kt, j, base + (int32_t)(t0 + j), a.rc);
    }
    // V nibbles: destination-driven, one 32-bit word (8 keys of one dim) per step
    const uint32_t vtile = kvm_vtile_bytes(KVM_TYPE_Q4_0, D);
    for (uint32_t wi = tid; wi < a.H * D * 8; wi += 256) {
        const uint32_t h = wi / (D * 8), r = wi % (D * 8);
        const uint32_t X = r >> 1, ks = r & 1u;
        const uint32_t dd = (X >> 6) * 16 + (X & 15u), gg = (X & 63u) >> 4;
        const uint32_t b = dd / 32, e = dd % 32;
        uint32_t word = 0;
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) {
            const uint32_t cj = 32 * ks + 8 * gg + j;
            uint32_t nib = 0;
            if (cj < count) {
                const uint8_t *blk = lv + cj * rowV + h * NB * 18 + b * 18;
                nib = e < 16 ? (blk[2 + e] & 15u) : (uint32_t)(blk[2 + e - 16] >> 4);
            }
            word |= nib << kvm_vq_nib_shift(j);
        }
        *(uint32_t *)(a.wv + ((uint64_t)h * a.n_tiles + tile) * vtile + kvm_vq_word(dd, gg, ks)) = word;
    }
    for (uint32_t si2 = tid; si2 < a.H * 64 * NB; si2 += 256) {
        const uint32_t h = si2 / (64 * NB), cj = (si2 / NB) % 64, b = si2 % NB;
        uint8_t *sd = a.wv + ((uint64_t)h * a.n_tiles + tile) * vtile + kvm_vd_off(D, cj, b);
        if (cj < count) {
            const uint8_t *blk = lv + cj * rowV + h * NB * 18 + b * 18;
            sd[0] = blk[0];
            sd[1] = blk[1];
        } else {
            sd[0] = 0;
            sd[1] = 0;
        }
    }
    if (tid < 64) a.cell_pos[slot * a.bt + t0 + tid] = tid < count ? base + (int32_t)(t0 + tid) : -1;
    if (tt == 0 && tid == 0) {
        a.slot_block[slot] = id;
        a.slot_base[slot] = base;
    }
}

// Every lane's plan in one launch (blockIdx.y = lane): the lanes' windows,
// histories and plans are independent, so the workgroups of one lane never touch
// another lane's memory.
#define KVM_STAGEIN_LANES 8
struct stage_lanes {
    stage_args lane[KVM_STAGEIN_LANES];
};

template <int D>
__global__ void __launch_bounds__(256) k_stagein(stage_lanes sl) {
    extern __shared__ __align__(16) uint8_t s_rows[];
    const stage_args &a = sl.lane[blockIdx.y];
    const uint32_t tps = a.bt / 64;
    const uint32_t n_items = a.info[3] != 0 ? 0u : a.info[2] * tps;
    for (uint32_t item = blockIdx.x; item < n_items; item += gridDim.x) {
        stagein_item<D>(a, s_rows, item / tps, item % tps);
        __syncthreads();                 // LDS rows of this item read before the next overwrites them
    }
}


static int rope_ctx_for(kvm_state *st, const float *theta, uint32_t n_half, int32_t nrot,
                        uint32_t max_pos, rope_ctx *rc) {
    int r = kvm_rope_table(st, theta, n_half, max_pos);
    if (r) return r;
    rc->tab = st->rope_tab;
    rc->n_half = n_half;
    rc->n_pos = st->rope_n_pos;
    rc->nrot = nrot;
    // the reference computes this scale on the host (llama-kvmem-stagein.cu:594)
    rc->hscale = nrot > 0 ? 1.0f / sqrtf((float)nrot) : 1.0f;
    return KVM_OK;
}

static int hadamard_width(const kvm_window *w, int32_t req) {
    if (req >= 0) return req;
    if (w->k_type != KVM_TYPE_Q8_0 || w->head_dim < 64 || w->head_dim % 64) return 0;
    int nrot = 64;                               // kvmem_hadamard_nrot_k, llama-kvmem-quant.h:30-36
    do { nrot *= 2; } while (w->head_dim % nrot == 0);
    return nrot / 2;
}

static bool hadamard_ok(int nrot, uint32_t D) {
    return nrot == 0 || (nrot >= 64 && nrot <= (int)D && !(nrot & (nrot - 1)) && D % nrot == 0);
}

// Checks one lane and fills its kernel arguments (all but the RoPE context).
static int stage_lane_args(kvm_state *st, const kvm_history *h, const kvm_window *w,
                           const kvm_selection *sel, stage_args *a, uint32_t *max_items) {
    if (!h || !w || !sel) return kvm_fail(st, KVM_EINVAL, "stagein: null argument");
    int rc = kvm_window_check(w);
    if (rc) return kvm_fail(st, rc, "stagein: bad window");
    if (w->k_type != KVM_TYPE_Q8_0) return kvm_fail(st, KVM_EUNSUPPORTED, "stagein: re-RoPE stage-in needs q8_0 K");
    if (w->block_tokens % 64) return kvm_fail(st, KVM_EUNSUPPORTED, "stagein: block_tokens %u not a multiple of 64", w->block_tokens);
    if (!w->slot_block || !w->slot_base) return kvm_fail(st, KVM_EINVAL, "stagein: window without slot map");
    if (!h->k_raw || !h->v || !sel->ids || !sel->to_base || !sel->stage_slots || !sel->info)
        return kvm_fail(st, KVM_EINVAL, "stagein: null buffer");
    const uint32_t NB = w->head_dim / 32;
    const size_t lds = (size_t)64 * w->n_head_kv * NB * (34 + 18);
    if (lds > 150 * 1024) return kvm_fail(st, KVM_ERANGE, "stagein: %u kv heads x %u dims exceed the staging tile", w->n_head_kv, w->head_dim);
    a->hk = (const uint8_t *)h->k_raw;
    a->hv = (const uint8_t *)h->v;
    a->h_tokens = h->n_tokens;
    a->wk = (uint8_t *)w->k;
    a->wv = (uint8_t *)w->v;
    a->cell_pos = w->cell_pos;
    a->slot_block = w->slot_block;
    a->slot_base = w->slot_base;
    a->n_tiles = w->n_cells / 64;
    a->H = w->n_head_kv;
    a->bt = w->block_tokens;
    a->n_slots = w->n_cells / w->block_tokens;
    a->ids = sel->ids;
    a->to_base = sel->to_base;
    a->stage_slots = sel->stage_slots;
    a->info = sel->info;
    const uint32_t max_slots = sel->cap < a->n_slots ? sel->cap : a->n_slots;
    *max_items = max_slots * (w->block_tokens / 64);
    return KVM_OK;
}

extern "C" int kvm_stagein_selection_lanes(kvm_state *st, const kvm_stagein_lane *lanes, uint32_t n_lanes,
                                           const kvm_rope_params *rope) {
    if (!st || !lanes || !rope) return kvm_fail(st, KVM_EINVAL, "stagein: null argument");
    if (n_lanes == 0) return KVM_OK;
    if (n_lanes > KVM_STAGEIN_LANES) return kvm_fail(st, KVM_ERANGE, "stagein: %u lanes > %d", n_lanes, KVM_STAGEIN_LANES);
    stage_lanes sl;
    std::memset(&sl, 0, sizeof(sl));
    uint32_t max_items = 0, max_cells = 0, max_h = 0;
    for (uint32_t i = 0; i < n_lanes; ++i) {
        uint32_t items = 0;
        int rc = stage_lane_args(st, lanes[i].h, lanes[i].w, lanes[i].sel, &sl.lane[i], &items);
        if (rc) return rc;
        if (lanes[i].w->head_dim != lanes[0].w->head_dim)
            return kvm_fail(st, KVM_EUNSUPPORTED, "stagein: lanes with head_dim %u and %u", lanes[0].w->head_dim, lanes[i].w->head_dim);
        max_items = items > max_items ? items : max_items;
        max_cells = lanes[i].w->n_cells > max_cells ? lanes[i].w->n_cells : max_cells;
        max_h = lanes[i].w->n_head_kv > max_h ? lanes[i].w->n_head_kv : max_h;
    }
    const kvm_window *w0 = lanes[0].w;
    if (rope->n_rot < 8 || rope->n_rot > w0->head_dim || rope->n_rot % 8)
        return kvm_fail(st, KVM_EUNSUPPORTED, "stagein: n_rot %u (needs a multiple of 8 <= head_dim)", rope->n_rot);
    const int nrot = hadamard_width(w0, rope->hadamard_nrot);
    if (!hadamard_ok(nrot, w0->head_dim)) return kvm_fail(st, KVM_EUNSUPPORTED, "stagein: hadamard width %d", nrot);
    KVM_HIP(st, hipSetDevice(st->device));
    const std::vector<float> theta = kvm_rope_theta(rope->freq_base, rope->freq_scale, rope->n_rot);
    rope_ctx rc0;
    int rc = rope_ctx_for(st, theta.data(), rope->n_rot / 2, nrot, max_cells, &rc0);
    if (rc) return rc;
    for (uint32_t i = 0; i < n_lanes; ++i) sl.lane[i].rc = rc0;
    const size_t lds = (size_t)64 * max_h * (w0->head_dim / 32) * (34 + 18);
    // about one workgroup per CU in all: an empty plan (the steady state) is one short launch
    const uint32_t per_lane = (KVM_STAGEIN_WGS + n_lanes - 1) / n_lanes;
    const dim3 grid(max_items < per_lane ? max_items : per_lane, n_lanes);
    if (grid.x == 0) return KVM_OK;
    if (w0->head_dim == 256) {
        KVM_HIP(st, hipFuncSetAttribute((const void *)k_stagein<256>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        hipLaunchKernelGGL(k_stagein<256>, grid, dim3(256), lds, st->stream, sl);
    } else {
        KVM_HIP(st, hipFuncSetAttribute((const void *)k_stagein<128>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        hipLaunchKernelGGL(k_stagein<128>, grid, dim3(256), lds, st->stream, sl);
    }
    KVM_LAUNCH_CHECK(st, "stagein");
    return KVM_OK;
}

extern "C" int kvm_stagein_selection(kvm_state *st, const kvm_history *h, const kvm_window *w,
                                     const kvm_selection *sel, const kvm_rope_params *rope) {
    const kvm_stagein_lane one = {h, w, sel};
    return kvm_stagein_selection_lanes(st, &one, 1, rope);
}

// ---------------------------------------------------------------------------
// Item-at-a-time API (llama-kvmem-stagein.h:36-46): packed rows are copied
// into a 32 MiB pinned slab; flush launches one kernel over every queued K
// item (reading the slab over PCIe) and moves V items with the import kernels.
// ---------------------------------------------------------------------------
struct kitem_desc {
    const uint8_t *src;
    uint8_t *wk;
    int32_t *cell_pos;
    uint32_t n_tiles, H, cell0, nt;
    int32_t pos0;
    int32_t nrot;
};

template <int D>
__global__ void __launch_bounds__(256) k_stagein_items(const kitem_desc *items, rope_ctx rc0) {
    constexpr uint32_t NB = D / 32;
    const kitem_desc it = items[blockIdx.y];
    const uint32_t r = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t t = r / it.H, h = r % it.H;
    if (t >= it.nt) return;
    rope_ctx rc = rc0;
    rc.nrot = it.nrot;
    rc.hscale = it.nrot > 0 ? rc0.hscale : 1.0f;
    const uint32_t cell = it.cell0 + t;
    uint8_t *kt = it.wk + ((uint64_t)h * it.n_tiles + cell / 64) * kvm_ktile_bytes(KVM_TYPE_Q8_0, D);
    stage_k_row<D>(it.src + (uint64_t)t * it.H * NB * 34 + h * NB * 34, kt, cell % 64,
                   it.pos0 + (int32_t)t, rc);
    if ((threadIdx.x & 63) == 0 && h == 0) it.cell_pos[cell] = it.pos0 + (int32_t)t;
}

static int slab_ready(kvm_state *st) {
    if (!st->slab) {
        if (hipHostMalloc((void **)&st->slab, (size_t)32 << 20, hipHostMallocDefault) != hipSuccess) {
            st->slab = nullptr;
            return kvm_fail(st, KVM_ENOMEM, "stagein slab: pinned allocation failed");
        }
        st->slab_bytes = (size_t)32 << 20;
        st->slab_used = 0;
    }
    if (st->slab_busy) {                     // kernels of the last flush read the slab
        KVM_HIP(st, hipEventSynchronize(st->ev));
        st->slab_busy = false;
    }
    return KVM_OK;
}

static int slab_reserve(kvm_state *st, size_t nbytes) {
    int rc = slab_ready(st);
    if (rc) return rc;
    if (nbytes > st->slab_bytes) return kvm_fail(st, KVM_ERANGE, "stagein: item of %zu bytes exceeds the slab", nbytes);
    if (st->slab_used + nbytes > st->slab_bytes) {
        rc = kvm_stagein_flush(st);
        if (rc) return rc;
        rc = slab_ready(st);
        if (rc) return rc;
    }
    return KVM_OK;
}

extern "C" int kvm_stagein_enqueue_k(kvm_state *st, int type, const void *packed, size_t nbytes,
                                     const kvm_window *w, uint32_t cell0, int64_t nt, int64_t n_embd,
                                     int nrot, int n_head, int n_embd_head, int n_rot_rope, int32_t pos0,
                                     const float *theta, int n_theta) {
    if (!st || !packed || !w) return kvm_fail(st, KVM_EINVAL, "enqueue_k: null argument");
    int rc = kvm_window_check(w);
    if (rc) return kvm_fail(st, rc, "enqueue_k: bad window");
    if (type != KVM_TYPE_Q8_0 || w->k_type != KVM_TYPE_Q8_0) return kvm_fail(st, KVM_EUNSUPPORTED, "enqueue_k: q8_0 only");
    if ((int64_t)n_head * n_embd_head != n_embd || (uint32_t)n_head != w->n_head_kv || (uint32_t)n_embd_head != w->head_dim)
        return kvm_fail(st, KVM_EINVAL, "enqueue_k: n_embd %lld != %d x %d or window shape", (long long)n_embd, n_head, n_embd_head);
    if (nt <= 0 || (uint64_t)cell0 + (uint64_t)nt > w->n_cells) return kvm_fail(st, KVM_ERANGE, "enqueue_k: cells past window");
    if ((size_t)nt * (size_t)(n_embd / 32 * 34) != nbytes) return kvm_fail(st, KVM_EINVAL, "enqueue_k: nbytes %zu mismatch", nbytes);
    if (n_rot_rope < 8 || n_rot_rope % 8 || n_rot_rope > n_embd_head || n_theta != n_rot_rope / 2 || !theta)
        return kvm_fail(st, KVM_EUNSUPPORTED, "enqueue_k: n_rot %d / n_theta %d", n_rot_rope, n_theta);
    if (!hadamard_ok(nrot, w->head_dim)) return kvm_fail(st, KVM_EUNSUPPORTED, "enqueue_k: hadamard width %d", nrot);
    // one theta per flush: a different theta flushes what is queued first
    if (!st->items.empty() && !st->theta.empty() &&
        (st->theta.size() != (size_t)n_theta || std::memcmp(st->theta.data(), theta, n_theta * 4))) {
        rc = kvm_stagein_flush(st);
        if (rc) return rc;
    }
    rc = slab_reserve(st, nbytes);
    if (rc) return rc;
    st->theta.assign(theta, theta + n_theta);
    std::memcpy(st->slab + st->slab_used, packed, nbytes);
    kvm_stage_item it;
    it.kind = 0;
    it.cell0 = cell0;
    it.nt = (uint32_t)nt;
    it.pos0 = pos0;
    it.off = st->slab_used;
    it.w = *w;
    it.n_rot = (uint32_t)n_rot_rope;
    it.nrot = nrot;
    st->items.push_back(it);
    st->slab_used += (nbytes + 15) & ~(size_t)15;
    return KVM_OK;
}

extern "C" int kvm_stagein_enqueue_v(kvm_state *st, const void *packed, size_t nbytes,
                                     const kvm_window *w, uint32_t cell0, int64_t nt) {
    if (!st || !packed || !w || nbytes == 0) return kvm_fail(st, KVM_EINVAL, "enqueue_v: null argument");
    int rc = kvm_window_check(w);
    if (rc) return kvm_fail(st, rc, "enqueue_v: bad window");
    if (nt <= 0 || (uint64_t)cell0 + (uint64_t)nt > w->n_cells) return kvm_fail(st, KVM_ERANGE, "enqueue_v: cells past window");
    const size_t row = w->v_type == KVM_TYPE_Q4_0 ? (size_t)w->n_head_kv * w->head_dim / 32 * 18
                                                   : (size_t)w->n_head_kv * w->head_dim * 2;
    if (row * (size_t)nt != nbytes) return kvm_fail(st, KVM_EINVAL, "enqueue_v: nbytes %zu mismatch", nbytes);
    rc = slab_reserve(st, nbytes);
    if (rc) return rc;
    std::memcpy(st->slab + st->slab_used, packed, nbytes);
    kvm_stage_item it;
    it.kind = 1;
    it.cell0 = cell0;
    it.nt = (uint32_t)nt;
    it.pos0 = 0;
    it.off = st->slab_used;
    it.w = *w;
    it.n_rot = 0;
    it.nrot = 0;
    st->items.push_back(it);
    st->slab_used += (nbytes + 15) & ~(size_t)15;
    return KVM_OK;
}

extern "C" int kvm_stagein_flush(kvm_state *st) {
    if (!st) return KVM_EINVAL;
    if (st->items.empty()) return KVM_OK;
    KVM_HIP(st, hipSetDevice(st->device));
    std::vector<kvm_stage_item> items;
    items.swap(st->items);
    int rc = KVM_OK;
    // K items grouped by head_dim
    for (int D : {128, 256}) {
        std::vector<kitem_desc> ds;
        uint32_t max_rows = 0, max_pos = 0, n_half = 0;
        float hscale = 1.0f;
        for (const auto &it : items) {
            if (it.kind != 0 || it.w.head_dim != (uint32_t)D) continue;
            kitem_desc d;
            d.src = st->slab + it.off;
            d.wk = (uint8_t *)it.w.k;
            d.cell_pos = it.w.cell_pos;
            d.n_tiles = it.w.n_cells / 64;
            d.H = it.w.n_head_kv;
            d.cell0 = it.cell0;
            d.nt = it.nt;
            d.pos0 = it.pos0;
            d.nrot = it.nrot;
            ds.push_back(d);
            max_rows = std::max(max_rows, it.nt * it.w.n_head_kv);
            max_pos = std::max(max_pos, (uint32_t)std::max(0, it.pos0) + it.nt);
            n_half = it.n_rot / 2;
            if (it.nrot > 0) hscale = 1.0f / sqrtf((float)it.nrot);
            if (it.pos0 < 0) rc = kvm_fail(st, KVM_EINVAL, "flush: negative pos0");
        }
        if (ds.empty() || rc) continue;
        if (ds.size() > 65535) { rc = kvm_fail(st, KVM_ERANGE, "flush: too many items"); break; }
        rope_ctx rcx;
        rc = rope_ctx_for(st, st->theta.data(), n_half, 0, max_pos, &rcx);
        if (rc) break;
        rcx.hscale = hscale;
        void *dd = kvm_upload_desc(st, ds.data(), ds.size() * sizeof(kitem_desc));
        if (!dd) { rc = kvm_fail(st, KVM_ENOMEM, "flush: descriptor upload"); break; }
        const dim3 grid(kvm_cdiv(max_rows, 4), (uint32_t)ds.size());
        if (D == 256)
            hipLaunchKernelGGL(k_stagein_items<256>, grid, dim3(256), 0, st->stream, (const kitem_desc *)dd, rcx);
        else
            hipLaunchKernelGGL(k_stagein_items<128>, grid, dim3(256), 0, st->stream, (const kitem_desc *)dd, rcx);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) { rc = kvm_fail(st, KVM_EHIP, "flush launch: %s", hipGetErrorString(e)); break; }
        // the descriptor buffer is reused by the next upload
        e = hipStreamSynchronize(st->stream);
        if (e != hipSuccess) { rc = kvm_fail(st, KVM_EHIP, "flush sync: %s", hipGetErrorString(e)); break; }
    }
    if (!rc) {
        for (const auto &it : items) {
            if (it.kind != 1) continue;
            rc = kvm_window_import_rows(st, &it.w, it.cell0, it.nt, nullptr, st->slab + it.off, nullptr);
            if (rc) break;
        }
    }
    st->slab_used = 0;
    st->theta.clear();
    if (hipEventRecord(st->ev, st->stream) == hipSuccess) st->slab_busy = true;
    else (void)hipStreamSynchronize(st->stream);
    return rc;
}
