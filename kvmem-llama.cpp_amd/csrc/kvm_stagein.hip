// kvm_stagein.hip -- fused stage-in: pinned-host history -> tiled window.
// The kernels and the host entry points; the per-row and per-item device
// routines (dequant -> RoPE -> Walsh-Hadamard -> q8_0 for K, V moved
// unchanged) are in kvm_stagein_dev.h.
#include "kvm_stagein_dev.h"

#include <cmath>
#include <cstring>

#define KVM_STAGEIN_IT 32         // tokens per item: half a window tile
#define KVM_STAGEIN_WGS_PER_CU 2  // workgroups per CU (a 32-token rows buffer takes a third of the LDS)
static_assert(KVM_STAGE_SYNC_BYTES == KVM_STAGEIN_LANES * KVM_STAGE_SYNC_LANE * 4, "stage-in sync words");

// Up to two workgroups per CU walk the (plan entry, 32-token run) items, so
// an empty plan (the steady state) costs one short launch; the plan length is
// only known on the device (info[2]).  Every lane's plan in one launch
// (blockIdx.y = lane): the lanes' windows, histories and plans are independent.
template <int D>
__global__ void __launch_bounds__(256) k_stagein(stage_lanes sl) {
    extern __shared__ __align__(16) uint8_t s_rows[];
    const stage_args &a = sl.lane[blockIdx.y];
    const uint32_t n_ent = stage_entries(a);
    if (n_ent == 0) return;
    // one barrier at most (the gather's): it takes the epoch's next value
    __shared__ uint32_t s_e;
    if (threadIdx.x == 0) s_e = sync_load(a.sync);
    __syncthreads();
    stage_plan<D, 256, KVM_STAGEIN_IT>(a, s_rows, n_ent, blockIdx.x, gridDim.x, s_e + 1, true);
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
    if (!kvm_k_quant(w->k_type) || w->head_dim < 64 || w->head_dim % 64) return 0;   // attn_rot_on
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
    if (!kvm_k_quant(w->k_type)) return kvm_fail(st, KVM_EUNSUPPORTED, "stagein: re-RoPE stage-in needs q8_0 or q4_0 K");
    if (w->block_tokens % 64) return kvm_fail(st, KVM_EUNSUPPORTED, "stagein: block_tokens %u not a multiple of 64", w->block_tokens);
    if (!w->slot_block || !w->slot_base) return kvm_fail(st, KVM_EINVAL, "stagein: window without slot map");
    if (!h->k_raw || !h->v || !sel->ids || !sel->to_base || !sel->stage_slots || !sel->info)
        return kvm_fail(st, KVM_EINVAL, "stagein: null buffer");
    const uint32_t NB = w->head_dim / 32;
    // a 32-token item's rows in LDS (the RoPE rows come on top)
    const size_t lds = (size_t)32 * w->n_head_kv * NB * (34 + 18);
    if (lds > 120 * 1024) return kvm_fail(st, KVM_ERANGE, "stagein: %u kv heads x %u dims exceed the staging tile", w->n_head_kv, w->head_dim);
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
    // the shadow is kept whenever the window has one; blocks move within the
    // window when the plan also names their sources (moves: set by the caller)
    a->k_shadow = (uint8_t *)w->k_shadow;
    a->shadow_rows = w->shadow_rows;
    a->stage_src = w->k_shadow ? sel->stage_src : nullptr;
    a->moves = nullptr;
    a->sync = nullptr;
    a->k_q4 = w->k_type == KVM_TYPE_Q4_0 ? 1u : 0u;
    const uint32_t max_slots = sel->cap < a->n_slots ? sel->cap : a->n_slots;
    *max_items = max_slots * (w->block_tokens / 64);
    return KVM_OK;
}

// Bytes of a lane's move staging: every plan entry may move (bt K rows and the
// slot's V tiles each).
static uint64_t move_bytes(const kvm_window *w, const kvm_selection *sel) {
    if (!w->k_shadow || !sel->stage_src) return 0;
    const uint32_t n_slots = w->n_cells / w->block_tokens, max_slots = sel->cap < n_slots ? sel->cap : n_slots;
    const uint64_t NB = w->head_dim / 32;
    return (uint64_t)max_slots * w->block_tokens * w->n_head_kv * NB * (34 + 18);
}

int kvm_stage_prepare(kvm_state *st, const kvm_stagein_lane *lanes, uint32_t n_lanes,
                      const kvm_rope_params *rope, stage_lanes *sl, uint32_t *max_items, size_t *lds) {
    if (!st || !lanes || !rope || !sl) return kvm_fail(st, KVM_EINVAL, "stagein: null argument");
    if (n_lanes > KVM_STAGEIN_LANES) return kvm_fail(st, KVM_ERANGE, "stagein: %u lanes > %d", n_lanes, KVM_STAGEIN_LANES);
    std::memset(sl, 0, sizeof(*sl));
    *max_items = 0;
    *lds = 0;
    if (n_lanes == 0) return KVM_OK;
    uint32_t max_cells = 0, max_h = 0;
    for (uint32_t i = 0; i < n_lanes; ++i) {
        uint32_t items = 0;
        int rc = stage_lane_args(st, lanes[i].h, lanes[i].w, lanes[i].sel, &sl->lane[i], &items);
        if (rc) return rc;
        if (lanes[i].w->head_dim != lanes[0].w->head_dim)
            return kvm_fail(st, KVM_EUNSUPPORTED, "stagein: lanes with head_dim %u and %u", lanes[0].w->head_dim, lanes[i].w->head_dim);
        *max_items = items > *max_items ? items : *max_items;
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
    for (uint32_t i = 0; i < n_lanes; ++i) {
        sl->lane[i].rc = rc0;
        sl->lane[i].sync = st->stage_sync + (size_t)i * KVM_STAGE_SYNC_LANE;
        sl->lane[i].status = st->fa_sync + KVM_FA_SYNC_STATUS;
        sl->lane[i].spin = st->wait_polls;
    }
    // 64-token items: K and V rows, then the (cos, sin) rows of their positions
    *lds = (size_t)64 * (max_h * (w0->head_dim / 32) * (34 + 18) + (rope->n_rot / 2) * 8);
    // the lanes' move staging regions, one after the other (256-byte aligned)
    uint64_t mv_total = 0;
    for (uint32_t i = 0; i < n_lanes; ++i) mv_total += (move_bytes(lanes[i].w, lanes[i].sel) + 255) & ~255ull;
    if (mv_total) {
        uint8_t *mv = (uint8_t *)kvm_move_workspace(st, mv_total);
        if (!mv) return kvm_fail(st, KVM_ENOMEM, "stagein: move staging of %llu bytes", (unsigned long long)mv_total);
        for (uint32_t i = 0; i < n_lanes; ++i) {
            const uint64_t b = (move_bytes(lanes[i].w, lanes[i].sel) + 255) & ~255ull;
            if (b) sl->lane[i].moves = mv;
            mv += b;
        }
    }
    return KVM_OK;
}

int kvm_stage_launch(kvm_state *st, const stage_lanes &sl, uint32_t n_lanes, uint32_t max_items, size_t lds,
                     uint32_t head_dim) {
    if (n_lanes == 0) return KVM_OK;
    // kvm_stage_prepare sizes 64-token items; this kernel's are 32 tokens
    max_items *= 64 / KVM_STAGEIN_IT;
    lds = lds * KVM_STAGEIN_IT / 64;
    const void *fn = head_dim == 256 ? (const void *)k_stagein<256> : (const void *)k_stagein<128>;
    // every workgroup resident at once (the gather barrier waits for all of a
    // lane's): at most what the CUs hold, two per CU at most
    int occ = 0;
    int rc = kvm_resident_blocks(st, fn, 256, lds, &occ);
    if (rc) return rc;
    if (occ > KVM_STAGEIN_WGS_PER_CU) occ = KVM_STAGEIN_WGS_PER_CU;
    uint32_t per_lane = (uint32_t)occ * st->n_cu / n_lanes;
    if (per_lane > KVM_STAGE_MAX_WGS) per_lane = KVM_STAGE_MAX_WGS;
    if (per_lane == 0) return kvm_fail(st, KVM_ERANGE, "stagein: %u lanes exceed the CUs", n_lanes);
    const dim3 grid(max_items < per_lane ? max_items : per_lane, n_lanes);
    if (grid.x == 0) return KVM_OK;
    if (head_dim == 256) hipLaunchKernelGGL(k_stagein<256>, grid, dim3(256), lds, st->stream, sl);
    else hipLaunchKernelGGL(k_stagein<128>, grid, dim3(256), lds, st->stream, sl);
    KVM_LAUNCH_CHECK(st, "stagein");
    return KVM_OK;
}

extern "C" int kvm_stagein_selection_lanes(kvm_state *st, const kvm_stagein_lane *lanes, uint32_t n_lanes,
                                           const kvm_rope_params *rope) {
    if (!st) return KVM_EINVAL;
    stage_lanes sl;
    uint32_t max_items = 0;
    size_t lds = 0;
    int rc = kvm_stage_prepare(st, lanes, n_lanes, rope, &sl, &max_items, &lds);
    if (rc || n_lanes == 0) return rc;
    return kvm_stage_launch(st, sl, n_lanes, max_items, lds, lanes[0].w->head_dim);
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
    int32_t nrot;       // Hadamard width of this item, 0 = off
    float hscale;       // 1 / sqrtf(nrot), per item: items of different widths may share a flush
    uint32_t q4;        // the rows are q4_0 (a q4_0 K window), else q8_0
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
    rc.hscale = it.hscale;
    const uint32_t cell = it.cell0 + t;
    uint8_t *kt = it.wk + ((uint64_t)h * it.n_tiles + cell / 64) * kvm_ktile_bytes(KVM_TYPE_Q8_0, D);
    const uint32_t kb = it.q4 ? 18u : 34u;
    stage_k_row<D>(it.src + (uint64_t)t * it.H * NB * kb + h * NB * kb, kt, cell % 64,
                   rc.tab + (uint64_t)(it.pos0 + (int32_t)t) * rc.n_half, rc, it.q4 != 0);
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
    if (!kvm_k_quant(type) || type != w->k_type)
        return kvm_fail(st, KVM_EUNSUPPORTED, "enqueue_k: rows of type %d into a window of K type %d (q8_0 or q4_0)", type,
                        w->k_type);
    if ((int64_t)n_head * n_embd_head != n_embd || (uint32_t)n_head != w->n_head_kv || (uint32_t)n_embd_head != w->head_dim)
        return kvm_fail(st, KVM_EINVAL, "enqueue_k: n_embd %lld != %d x %d or window shape", (long long)n_embd, n_head, n_embd_head);
    if (nt <= 0 || (uint64_t)cell0 + (uint64_t)nt > w->n_cells) return kvm_fail(st, KVM_ERANGE, "enqueue_k: cells past window");
    const size_t kb = type == KVM_TYPE_Q4_0 ? 18u : 34u;
    if ((size_t)nt * (size_t)(n_embd / 32 * kb) != nbytes) return kvm_fail(st, KVM_EINVAL, "enqueue_k: nbytes %zu mismatch", nbytes);
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
            // the reference computes the scale on the host (llama-kvmem-stagein.cu:594)
            d.hscale = it.nrot > 0 ? 1.0f / sqrtf((float)it.nrot) : 1.0f;
            d.q4 = it.w.k_type == KVM_TYPE_Q4_0 ? 1u : 0u;
            ds.push_back(d);
            max_rows = std::max(max_rows, it.nt * it.w.n_head_kv);
            max_pos = std::max(max_pos, (uint32_t)std::max(0, it.pos0) + it.nt);
            n_half = it.n_rot / 2;
            if (it.pos0 < 0) rc = kvm_fail(st, KVM_EINVAL, "flush: negative pos0");
        }
        if (ds.empty() || rc) continue;
        if (ds.size() > 65535) { rc = kvm_fail(st, KVM_ERANGE, "flush: too many items"); break; }
        rope_ctx rcx;
        rc = rope_ctx_for(st, st->theta.data(), n_half, 0, max_pos, &rcx);
        if (rc) break;
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
