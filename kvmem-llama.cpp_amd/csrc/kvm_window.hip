// kvm_window.hip -- window geometry, ggml-row <-> tiled-window conversion,
// row codecs and batched device copies.
#include "kvm_internal.h"

#include <algorithm>

// ---------------------------------------------------------------------------
// geometry
// ---------------------------------------------------------------------------
extern "C" int kvm_window_check(const kvm_window *w) {
    if (!w) return KVM_EINVAL;
    if (w->n_cells == 0 || w->n_cells % KVM_TILE_CELLS) return KVM_EINVAL;
    if (w->head_dim != 128 && w->head_dim != 256) return KVM_EUNSUPPORTED;
    if (w->n_head_kv == 0 || w->block_tokens == 0 || w->n_cells % w->block_tokens) return KVM_EINVAL;
    const bool q = kvm_k_quant(w->k_type) && w->v_type == KVM_TYPE_Q4_0;
    const bool h = w->k_type == KVM_TYPE_F16 && w->v_type == KVM_TYPE_F16;
    if (!q && !h) return KVM_EUNSUPPORTED;
    if (!w->k || !w->v || !w->cell_pos) return KVM_EINVAL;
    // a shadow comes with its row counts and the slot map, and holds the
    // history's q8_0 or q4_0 K rows
    if (!w->k_shadow != !w->shadow_rows) return KVM_EINVAL;
    if (w->k_shadow && (!q || !w->slot_block || !w->slot_base)) return KVM_EINVAL;
    return KVM_OK;
}

extern "C" size_t kvm_window_shadow_bytes(const kvm_window *w) {
    if (!w || !kvm_k_quant(w->k_type)) return 0;
    return (size_t)w->n_cells * w->n_head_kv * (w->head_dim / 32) * (w->k_type == KVM_TYPE_Q4_0 ? 18u : 34u);
}

extern "C" size_t kvm_window_k_bytes(const kvm_window *w) {
    if (!w || w->n_cells % KVM_TILE_CELLS) return 0;
    return (size_t)w->n_head_kv * (w->n_cells / KVM_TILE_CELLS) * kvm_ktile_bytes(w->k_type, w->head_dim);
}

extern "C" size_t kvm_window_v_bytes(const kvm_window *w) {
    if (!w || w->n_cells % KVM_TILE_CELLS) return 0;
    return (size_t)w->n_head_kv * (w->n_cells / KVM_TILE_CELLS) * kvm_vtile_bytes(w->v_type, w->head_dim);
}

__global__ void k_fill_i32(int32_t *p, int32_t v, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

extern "C" int kvm_window_reset(kvm_state *st, const kvm_window *w) {
    if (!st) return KVM_EINVAL;
    int rc = kvm_window_check(w);
    if (rc) return kvm_fail(st, rc, "window_reset: bad window");
    KVM_HIP(st, hipSetDevice(st->device));
    hipLaunchKernelGGL(k_fill_i32, dim3(kvm_cdiv(w->n_cells, 256)), dim3(256), 0, st->stream,
                       w->cell_pos, -1, w->n_cells);
    const uint32_t n_slots = w->n_cells / w->block_tokens;
    if (w->slot_block)
        hipLaunchKernelGGL(k_fill_i32, dim3(kvm_cdiv(n_slots, 256)), dim3(256), 0, st->stream,
                           (int32_t *)w->slot_block, -1, n_slots);
    if (w->slot_base)
        hipLaunchKernelGGL(k_fill_i32, dim3(kvm_cdiv(n_slots, 256)), dim3(256), 0, st->stream,
                           w->slot_base, -1, n_slots);
    if (w->shadow_rows)
        hipLaunchKernelGGL(k_fill_i32, dim3(kvm_cdiv(n_slots, 256)), dim3(256), 0, st->stream,
                           (int32_t *)w->shadow_rows, 0, n_slots);
    if (w->pending_rows)
        hipLaunchKernelGGL(k_fill_i32, dim3(kvm_cdiv(n_slots, 256)), dim3(256), 0, st->stream,
                           (int32_t *)w->pending_rows, 0, n_slots);
    KVM_LAUNCH_CHECK(st, "window_reset");
    return KVM_OK;
}

// ---------------------------------------------------------------------------
// ggml rows -> tiled window
// ---------------------------------------------------------------------------
struct win_geo {
    uint8_t *k, *v;
    uint32_t H, D, n_tiles, ktile, vtile;
    uint32_t *shadow_rows;       // null, or the shadow row counts an import voids
    uint32_t bt, n_slots;
};

// An import into cell `cell` voids its slot's shadow (the shadow holds only
// what a stage-in wrote); called by the thread of the cell's first row block.
__device__ inline void void_shadow(const win_geo &g, uint32_t cell) {
    if (g.shadow_rows && cell / g.bt < g.n_slots) g.shadow_rows[cell / g.bt] = 0u;
}

static win_geo geo_of(const kvm_window *w) {
    win_geo g;
    g.k = (uint8_t *)w->k;
    g.v = (uint8_t *)w->v;
    g.H = w->n_head_kv;
    g.D = w->head_dim;
    g.n_tiles = w->n_cells / KVM_TILE_CELLS;
    g.ktile = kvm_ktile_bytes(w->k_type, w->head_dim);
    g.vtile = kvm_vtile_bytes(w->v_type, w->head_dim);
    g.shadow_rows = w->shadow_rows;
    g.bt = w->block_tokens;
    g.n_slots = w->n_cells / w->block_tokens;
    return g;
}

// one thread per (cell, head, 32-dim block) of q8_0 K rows
__global__ void k_import_k_q8(win_geo g, uint32_t cell0, uint32_t n, const uint8_t *rows) {
    const uint32_t NB = g.D / 32;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)n * g.H * NB) return;
    const uint32_t b = i % NB, h = (i / NB) % g.H, t = (uint32_t)(i / ((uint64_t)NB * g.H));
    const uint32_t cell = cell0 + t, tile = cell / 64, c = cell % 64;
    const uint8_t *src = rows + ((uint64_t)t * g.H + h) * NB * 34 + (uint64_t)b * 34;
    uint8_t *dst = g.k + ((uint64_t)h * g.n_tiles + tile) * g.ktile;
#pragma unroll
    for (uint32_t gg = 0; gg < 4; ++gg) {
        uint8_t *q = dst + kvm_kq_off(g.D, c, 32 * b + 8 * gg);
#pragma unroll
        for (int j = 0; j < 8; ++j) q[j] = src[2 + 8 * gg + j];
    }
    uint8_t *sd = dst + kvm_kd_off(g.D, c, b);
    sd[0] = src[0];
    sd[1] = src[1];
    if (b == 0 && h == 0) void_shadow(g, cell);
}

// q4_0 K rows into the q8_0 tile format: quant j = nibble - 8 (low nibbles
// are dims 0-15 of the block, high nibbles 16-31), the fp16 scale as it is
__global__ void k_import_k_q4(win_geo g, uint32_t cell0, uint32_t n, const uint8_t *rows) {
    const uint32_t NB = g.D / 32;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)n * g.H * NB) return;
    const uint32_t b = i % NB, h = (i / NB) % g.H, t = (uint32_t)(i / ((uint64_t)NB * g.H));
    const uint32_t cell = cell0 + t, tile = cell / 64, c = cell % 64;
    const uint8_t *src = rows + ((uint64_t)t * g.H + h) * NB * 18 + (uint64_t)b * 18;
    uint8_t *dst = g.k + ((uint64_t)h * g.n_tiles + tile) * g.ktile;
#pragma unroll
    for (uint32_t gg = 0; gg < 4; ++gg) {
        uint8_t *q = dst + kvm_kq_off(g.D, c, 32 * b + 8 * gg);
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) {
            const uint32_t e = 8 * gg + j, nib = e < 16 ? src[2 + e] & 15u : (uint32_t)src[2 + e - 16] >> 4;
            q[j] = (uint8_t)(int8_t)((int)nib - 8);
        }
    }
    uint8_t *sd = dst + kvm_kd_off(g.D, c, b);
    sd[0] = src[0];
    sd[1] = src[1];
    if (b == 0 && h == 0) void_shadow(g, cell);
}

// f16 K rows: one thread per (cell, head, dim)
__global__ void k_import_k_f16(win_geo g, uint32_t cell0, uint32_t n, const uint16_t *rows) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)n * g.H * g.D) return;
    const uint32_t d = i % g.D, h = (i / g.D) % g.H, t = (uint32_t)(i / ((uint64_t)g.D * g.H));
    const uint32_t cell = cell0 + t, tile = cell / 64, c = cell % 64;
    uint16_t *dst = (uint16_t *)(g.k + ((uint64_t)h * g.n_tiles + tile) * g.ktile);
    dst[kvm_kh_idx(g.D, c, d)] = rows[((uint64_t)t * g.H + h) * g.D + d];
}

// q4_0 V nibbles: one thread per destination 32-bit word (8 keys of one dim),
// so the cells sharing a byte are written by one thread; cells outside
// [cell0, cell0+n) keep their nibble.
__global__ void k_import_v_q4(win_geo g, uint32_t cell0, uint32_t n, const uint8_t *rows) {
    const uint32_t NB = g.D / 32;
    const uint32_t t0 = cell0 / 64, t1 = (cell0 + n + 63) / 64;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)(t1 - t0) * g.H * g.D * 8) return;
    const uint32_t wi = i % (g.D * 8), h = (i / (8ull * g.D)) % g.H;
    const uint32_t tile = t0 + (uint32_t)(i / (8ull * g.D * g.H));
    const uint32_t X = wi >> 1, ks = wi & 1u;
    const uint32_t d = (X >> 6) * 16 + (X & 15u), gg = (X & 63u) >> 4;
    uint32_t *dst = (uint32_t *)(g.v + ((uint64_t)h * g.n_tiles + tile) * g.vtile + kvm_vq_word(d, gg, ks));
    uint32_t word = *dst;
    const uint32_t b = d / 32, e = d % 32;
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) {
        const uint32_t cell = tile * 64 + 32 * ks + 8 * gg + j;
        if (cell < cell0 || cell >= cell0 + n) continue;
        const uint8_t *blk = rows + ((uint64_t)(cell - cell0) * g.H + h) * NB * 18 + (uint64_t)b * 18;
        const uint32_t nib = e < 16 ? (blk[2 + e] & 15u) : (uint32_t)(blk[2 + e - 16] >> 4);
        word = (word & ~(15u << kvm_vq_nib_shift(j))) | (nib << kvm_vq_nib_shift(j));
    }
    *dst = word;
}

__global__ void k_import_v_q4_scales(win_geo g, uint32_t cell0, uint32_t n, const uint8_t *rows) {
    const uint32_t NB = g.D / 32;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)n * g.H * NB) return;
    const uint32_t b = i % NB, h = (i / NB) % g.H, t = (uint32_t)(i / ((uint64_t)NB * g.H));
    const uint32_t cell = cell0 + t, tile = cell / 64, c = cell % 64;
    const uint8_t *blk = rows + ((uint64_t)t * g.H + h) * NB * 18 + (uint64_t)b * 18;
    uint8_t *dst = g.v + ((uint64_t)h * g.n_tiles + tile) * g.vtile + kvm_vd_off(g.D, c, b);
    dst[0] = blk[0];
    dst[1] = blk[1];
    if (b == 0 && h == 0) void_shadow(g, cell);
}

__global__ void k_import_v_f16(win_geo g, uint32_t cell0, uint32_t n, const uint16_t *rows) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)n * g.H * g.D) return;
    const uint32_t d = i % g.D, h = (i / g.D) % g.H, t = (uint32_t)(i / ((uint64_t)g.D * g.H));
    const uint32_t cell = cell0 + t, tile = cell / 64, c = cell % 64;
    uint16_t *dst = (uint16_t *)(g.v + ((uint64_t)h * g.n_tiles + tile) * g.vtile);
    dst[kvm_vh_idx(c, d)] = rows[((uint64_t)t * g.H + h) * g.D + d];
}

__global__ void k_copy_i32(int32_t *dst, const int32_t *src, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

// The unharvested-row count of every slot that cells [cell0, cell0 + n) touch:
// raised by the rows an import writes there (add), lowered by the rows a
// harvest takes into the host history (sub, not below zero).  One thread per
// slot.
// Per touched slot: the end (rows from the slot's first cell) of the rows
// imported since the last harvest that reached them.  An import raises it to
// the end of its rows in the slot (a re-import of the same cells, e.g. after
// rejected draft tokens, adds nothing); a harvest whose cells reach that end
// clears it; a copy of the slot from the host clears it.
enum pending_op { PENDING_IMPORT = 0, PENDING_HARVEST = 1, PENDING_CLEAR = 2 };
__global__ void k_pending_rows(uint32_t *pending, uint32_t bt, uint32_t n_slots, uint32_t cell0, uint32_t n,
                               int op) {
    const uint32_t slot = cell0 / bt + blockIdx.x * blockDim.x + threadIdx.x;
    if (slot >= n_slots || slot * bt >= cell0 + n) return;
    const uint32_t hi = (slot + 1) * bt < cell0 + n ? (slot + 1) * bt : cell0 + n;
    const uint32_t end = hi - slot * bt, cur = pending[slot];
    if (op == PENDING_IMPORT)
        pending[slot] = end > cur ? end : cur;
    else if (op == PENDING_CLEAR || end >= cur)
        pending[slot] = 0u;
}

static void pending_rows(kvm_state *st, const kvm_window *w, uint32_t cell0, uint32_t n, pending_op op) {
    const uint32_t bt = w->block_tokens, n_slots = w->n_cells / bt;
    const uint32_t touched = (cell0 + n - 1) / bt - cell0 / bt + 1;
    hipLaunchKernelGGL(k_pending_rows, dim3(kvm_cdiv(touched, 256)), dim3(256), 0, st->stream, w->pending_rows,
                       bt, n_slots, cell0, n, (int)op);
}

extern "C" int kvm_window_import_rows(kvm_state *st, const kvm_window *w, uint32_t cell0,
                                      uint32_t n, const void *k_rows, const void *v_rows,
                                      const int32_t *pos) {
    if (!st) return KVM_EINVAL;
    int rc = kvm_window_check(w);
    if (rc) return kvm_fail(st, rc, "import_rows: bad window");
    if ((uint64_t)cell0 + n > w->n_cells) return kvm_fail(st, KVM_ERANGE, "import_rows: cells past window");
    if (n == 0) return KVM_OK;
    KVM_HIP(st, hipSetDevice(st->device));
    const win_geo g = geo_of(w);
    const uint32_t NB = g.D / 32;
    if (k_rows) {
        if (w->k_type == KVM_TYPE_Q8_0) {
            const uint64_t nt = (uint64_t)n * g.H * NB;
            hipLaunchKernelGGL(k_import_k_q8, dim3(kvm_cdiv(nt, 256)), dim3(256), 0, st->stream, g, cell0, n,
                               (const uint8_t *)k_rows);
        } else if (w->k_type == KVM_TYPE_Q4_0) {
            const uint64_t nt = (uint64_t)n * g.H * NB;
            hipLaunchKernelGGL(k_import_k_q4, dim3(kvm_cdiv(nt, 256)), dim3(256), 0, st->stream, g, cell0, n,
                               (const uint8_t *)k_rows);
        } else {
            const uint64_t nt = (uint64_t)n * g.H * g.D;
            hipLaunchKernelGGL(k_import_k_f16, dim3(kvm_cdiv(nt, 256)), dim3(256), 0, st->stream, g, cell0, n,
                               (const uint16_t *)k_rows);
        }
    }
    if (v_rows) {
        if (w->v_type == KVM_TYPE_Q4_0) {
            const uint32_t t0 = cell0 / 64, t1 = (cell0 + n + 63) / 64;
            const uint64_t nb = (uint64_t)(t1 - t0) * g.H * g.D * 8;
            hipLaunchKernelGGL(k_import_v_q4, dim3(kvm_cdiv(nb, 256)), dim3(256), 0, st->stream, g, cell0, n,
                               (const uint8_t *)v_rows);
            const uint64_t ns = (uint64_t)n * g.H * NB;
            hipLaunchKernelGGL(k_import_v_q4_scales, dim3(kvm_cdiv(ns, 256)), dim3(256), 0, st->stream, g,
                               cell0, n, (const uint8_t *)v_rows);
        } else {
            const uint64_t nt = (uint64_t)n * g.H * g.D;
            hipLaunchKernelGGL(k_import_v_f16, dim3(kvm_cdiv(nt, 256)), dim3(256), 0, st->stream, g, cell0, n,
                               (const uint16_t *)v_rows);
        }
    }
    if (pos)
        hipLaunchKernelGGL(k_copy_i32, dim3(kvm_cdiv(n, 256)), dim3(256), 0, st->stream,
                           w->cell_pos + cell0, pos, n);
    if (w->pending_rows && (k_rows || v_rows)) pending_rows(st, w, cell0, n, PENDING_IMPORT);
    KVM_LAUNCH_CHECK(st, "import_rows");
    return KVM_OK;
}

// ---------------------------------------------------------------------------
// tiled window -> ggml rows
// ---------------------------------------------------------------------------
__global__ void k_export_k_q8(win_geo g, uint32_t cell0, uint32_t n, uint8_t *rows) {
    const uint32_t NB = g.D / 32;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)n * g.H * NB) return;
    const uint32_t b = i % NB, h = (i / NB) % g.H, t = (uint32_t)(i / ((uint64_t)NB * g.H));
    const uint32_t cell = cell0 + t, tile = cell / 64, c = cell % 64;
    uint8_t *dst = rows + ((uint64_t)t * g.H + h) * NB * 34 + (uint64_t)b * 34;
    const uint8_t *src = g.k + ((uint64_t)h * g.n_tiles + tile) * g.ktile;
    const uint8_t *sd = src + kvm_kd_off(g.D, c, b);
    dst[0] = sd[0];
    dst[1] = sd[1];
#pragma unroll
    for (uint32_t gg = 0; gg < 4; ++gg) {
        const uint8_t *q = src + kvm_kq_off(g.D, c, 32 * b + 8 * gg);
#pragma unroll
        for (int j = 0; j < 8; ++j) dst[2 + 8 * gg + j] = q[j];
    }
}

// the q8_0-format tile of a q4_0 K window back to q4_0 rows (quant + 8)
__global__ void k_export_k_q4(win_geo g, uint32_t cell0, uint32_t n, uint8_t *rows) {
    const uint32_t NB = g.D / 32;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)n * g.H * NB) return;
    const uint32_t b = i % NB, h = (i / NB) % g.H, t = (uint32_t)(i / ((uint64_t)NB * g.H));
    const uint32_t cell = cell0 + t, tile = cell / 64, c = cell % 64;
    uint8_t *dst = rows + ((uint64_t)t * g.H + h) * NB * 18 + (uint64_t)b * 18;
    const uint8_t *src = g.k + ((uint64_t)h * g.n_tiles + tile) * g.ktile;
    const uint8_t *sd = src + kvm_kd_off(g.D, c, b);
    dst[0] = sd[0];
    dst[1] = sd[1];
    const uint8_t *lo = src + kvm_kq_off(g.D, c, 32 * b), *lo2 = src + kvm_kq_off(g.D, c, 32 * b + 8);
    const uint8_t *hi = src + kvm_kq_off(g.D, c, 32 * b + 16), *hi2 = src + kvm_kq_off(g.D, c, 32 * b + 24);
#pragma unroll
    for (uint32_t e = 0; e < 16; ++e) {
        const uint32_t n0 = (uint32_t)((int)(int8_t)(e < 8 ? lo[e] : lo2[e - 8]) + 8) & 15u;
        const uint32_t n1 = (uint32_t)((int)(int8_t)(e < 8 ? hi[e] : hi2[e - 8]) + 8) & 15u;
        dst[2 + e] = (uint8_t)(n0 | (n1 << 4));
    }
}

__global__ void k_export_v_q4(win_geo g, uint32_t cell0, uint32_t n, uint8_t *rows) {
    const uint32_t NB = g.D / 32;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)n * g.H * NB) return;
    const uint32_t b = i % NB, h = (i / NB) % g.H, t = (uint32_t)(i / ((uint64_t)NB * g.H));
    const uint32_t cell = cell0 + t, tile = cell / 64, c = cell % 64;
    uint8_t *dst = rows + ((uint64_t)t * g.H + h) * NB * 18 + (uint64_t)b * 18;
    const uint8_t *src = g.v + ((uint64_t)h * g.n_tiles + tile) * g.vtile;
    const uint8_t *sd = src + kvm_vd_off(g.D, c, b);
    dst[0] = sd[0];
    dst[1] = sd[1];
    const uint32_t sh = kvm_vq_shift(c);
    for (uint32_t e = 0; e < 16; ++e) {
        const uint8_t n0 = (src[kvm_vq_byte(c, 32 * b + e)] >> sh) & 15;
        const uint8_t n1 = (src[kvm_vq_byte(c, 32 * b + e + 16)] >> sh) & 15;
        dst[2 + e] = (uint8_t)(n0 | (n1 << 4));
    }
}

__global__ void k_export_f16(win_geo g, uint32_t cell0, uint32_t n, uint16_t *krows, uint16_t *vrows) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)n * g.H * g.D) return;
    const uint32_t d = i % g.D, h = (i / g.D) % g.H, t = (uint32_t)(i / ((uint64_t)g.D * g.H));
    const uint32_t cell = cell0 + t, tile = cell / 64, c = cell % 64;
    if (krows) {
        const uint16_t *src = (const uint16_t *)(g.k + ((uint64_t)h * g.n_tiles + tile) * g.ktile);
        krows[((uint64_t)t * g.H + h) * g.D + d] = src[kvm_kh_idx(g.D, c, d)];
    }
    if (vrows) {
        const uint16_t *src = (const uint16_t *)(g.v + ((uint64_t)h * g.n_tiles + tile) * g.vtile);
        vrows[((uint64_t)t * g.H + h) * g.D + d] = src[kvm_vh_idx(c, d)];
    }
}

extern "C" int kvm_window_export_rows(kvm_state *st, const kvm_window *w, uint32_t cell0,
                                      uint32_t n, void *k_rows, void *v_rows) {
    if (!st) return KVM_EINVAL;
    int rc = kvm_window_check(w);
    if (rc) return kvm_fail(st, rc, "export_rows: bad window");
    if ((uint64_t)cell0 + n > w->n_cells) return kvm_fail(st, KVM_ERANGE, "export_rows: cells past window");
    if (n == 0) return KVM_OK;
    KVM_HIP(st, hipSetDevice(st->device));
    const win_geo g = geo_of(w);
    const uint32_t NB = g.D / 32;
    if (kvm_k_quant(w->k_type)) {
        const uint64_t nt = (uint64_t)n * g.H * NB;
        if (k_rows && w->k_type == KVM_TYPE_Q8_0)
            hipLaunchKernelGGL(k_export_k_q8, dim3(kvm_cdiv(nt, 256)), dim3(256), 0, st->stream, g, cell0, n,
                               (uint8_t *)k_rows);
        if (k_rows && w->k_type == KVM_TYPE_Q4_0)
            hipLaunchKernelGGL(k_export_k_q4, dim3(kvm_cdiv(nt, 256)), dim3(256), 0, st->stream, g, cell0, n,
                               (uint8_t *)k_rows);
        if (v_rows)
            hipLaunchKernelGGL(k_export_v_q4, dim3(kvm_cdiv(nt, 256)), dim3(256), 0, st->stream, g, cell0, n,
                               (uint8_t *)v_rows);
    } else {
        const uint64_t nt = (uint64_t)n * g.H * g.D;
        hipLaunchKernelGGL(k_export_f16, dim3(kvm_cdiv(nt, 256)), dim3(256), 0, st->stream, g, cell0, n,
                           (uint16_t *)k_rows, (uint16_t *)v_rows);
    }
    KVM_LAUNCH_CHECK(st, "export_rows");
    return KVM_OK;
}

// ---------------------------------------------------------------------------
// row codecs: one thread per 32-value block
// ---------------------------------------------------------------------------
__global__ void k_quant_q8(const float *x, uint8_t *y, uint64_t nblk) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk) return;
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = x[i * 32 + j];
    uint16_t d;
    int8_t q[32];
    kvm_quant_block_q8_0(v, &d, q);
    uint8_t *o = y + i * 34;
    o[0] = (uint8_t)d;
    o[1] = (uint8_t)(d >> 8);
#pragma unroll
    for (int j = 0; j < 32; ++j) o[2 + j] = (uint8_t)q[j];
}

__global__ void k_quant_q4(const float *x, uint8_t *y, uint64_t nblk) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk) return;
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = x[i * 32 + j];
    uint16_t d;
    uint8_t q[16];
    kvm_quant_block_q4_0(v, &d, q);
    uint8_t *o = y + i * 18;
    o[0] = (uint8_t)d;
    o[1] = (uint8_t)(d >> 8);
#pragma unroll
    for (int j = 0; j < 16; ++j) o[2 + j] = q[j];
}

__global__ void k_quant_f16(const float *x, uint16_t *y, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = kvm_f2h(x[i]);
}

__global__ void k_dequant_q8(const uint8_t *x, float *y, uint64_t nblk) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk) return;
    const uint8_t *b = x + i * 34;
    const float d = kvm_h2f((uint16_t)(b[0] | (b[1] << 8)));
#pragma unroll
    for (int j = 0; j < 32; ++j) y[i * 32 + j] = (float)(int8_t)b[2 + j] * d;
}

__global__ void k_dequant_q4(const uint8_t *x, float *y, uint64_t nblk) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk) return;
    const uint8_t *b = x + i * 18;
    const float d = kvm_h2f((uint16_t)(b[0] | (b[1] << 8)));
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        y[i * 32 + j] = (float)((b[2 + j] & 15) - 8) * d;
        y[i * 32 + j + 16] = (float)((b[2 + j] >> 4) - 8) * d;
    }
}

__global__ void k_dequant_f16(const uint16_t *x, float *y, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = kvm_h2f(x[i]);
}

extern "C" int kvm_quantize_rows(kvm_state *st, int type, const float *src, void *dst,
                                 int64_t n_rows, int64_t n_per_row) {
    if (!st || !src || !dst || n_rows < 0 || n_per_row <= 0) return kvm_fail(st, KVM_EINVAL, "quantize_rows: args");
    if (n_rows == 0) return KVM_OK;
    KVM_HIP(st, hipSetDevice(st->device));
    const uint64_t n = (uint64_t)n_rows * (uint64_t)n_per_row;
    if (type == KVM_TYPE_Q8_0 || type == KVM_TYPE_Q4_0) {
        if (n_per_row % 32) return kvm_fail(st, KVM_EINVAL, "quantize_rows: row not a multiple of 32");
        const uint64_t nb = n / 32;
        if (type == KVM_TYPE_Q8_0)
            hipLaunchKernelGGL(k_quant_q8, dim3(kvm_cdiv(nb, 256)), dim3(256), 0, st->stream, src, (uint8_t *)dst, nb);
        else
            hipLaunchKernelGGL(k_quant_q4, dim3(kvm_cdiv(nb, 256)), dim3(256), 0, st->stream, src, (uint8_t *)dst, nb);
    } else if (type == KVM_TYPE_F16) {
        hipLaunchKernelGGL(k_quant_f16, dim3(kvm_cdiv(n, 256)), dim3(256), 0, st->stream, src, (uint16_t *)dst, n);
    } else {
        return kvm_fail(st, KVM_EUNSUPPORTED, "quantize_rows: type %d", type);
    }
    KVM_LAUNCH_CHECK(st, "quantize_rows");
    return KVM_OK;
}

extern "C" int kvm_dequantize_rows(kvm_state *st, int type, const void *src, float *dst,
                                   int64_t n_rows, int64_t n_per_row) {
    if (!st || !src || !dst || n_rows < 0 || n_per_row <= 0) return kvm_fail(st, KVM_EINVAL, "dequantize_rows: args");
    if (n_rows == 0) return KVM_OK;
    KVM_HIP(st, hipSetDevice(st->device));
    const uint64_t n = (uint64_t)n_rows * (uint64_t)n_per_row;
    if (type == KVM_TYPE_Q8_0 || type == KVM_TYPE_Q4_0) {
        if (n_per_row % 32) return kvm_fail(st, KVM_EINVAL, "dequantize_rows: row not a multiple of 32");
        const uint64_t nb = n / 32;
        if (type == KVM_TYPE_Q8_0)
            hipLaunchKernelGGL(k_dequant_q8, dim3(kvm_cdiv(nb, 256)), dim3(256), 0, st->stream, (const uint8_t *)src, dst, nb);
        else
            hipLaunchKernelGGL(k_dequant_q4, dim3(kvm_cdiv(nb, 256)), dim3(256), 0, st->stream, (const uint8_t *)src, dst, nb);
    } else if (type == KVM_TYPE_F16) {
        hipLaunchKernelGGL(k_dequant_f16, dim3(kvm_cdiv(n, 256)), dim3(256), 0, st->stream, (const uint16_t *)src, dst, n);
    } else {
        return kvm_fail(st, KVM_EUNSUPPORTED, "dequantize_rows: type %d", type);
    }
    KVM_LAUNCH_CHECK(st, "dequantize_rows");
    return KVM_OK;
}

// ---------------------------------------------------------------------------
// batched device copies (kvmem_d2d_batched / copy_bytes, stagein.cu:236-261)
// ---------------------------------------------------------------------------
struct kvm_copy_op {
    const uint8_t *src;
    uint8_t *dst;
    uint64_t nbytes;
};

// The host cuts every op into chunks of at most KVM_COPY_CHUNK bytes at
// multiples of KVM_COPY_CHUNK from the op's start (so a chunk's source and
// destination keep the op's alignment to each other); one wave copies one
// chunk, four per workgroup.  Where source and destination agree modulo 16,
// the wave moves the bytes up to the destination's next 16-byte boundary one
// per lane, the body in 16-byte loads (four in flight per lane before their
// stores) and the last bytes one per lane; otherwise byte by byte.
#define KVM_COPY_CHUNK 16384u
__global__ void __launch_bounds__(256) k_copy_ops(const kvm_copy_op *ops, uint32_t n) {
    const uint32_t i = blockIdx.x * 4u + (threadIdx.x >> 6), l = threadIdx.x & 63u;
    if (i >= n) return;
    const kvm_copy_op op = ops[i];
    const uint8_t *s = op.src;
    uint8_t *d = op.dst;
    uint64_t nb = op.nbytes;
    if ((((uintptr_t)s ^ (uintptr_t)d) & 15u) != 0) {
        for (uint64_t j = l; j < nb; j += 64) d[j] = s[j];
        return;
    }
    const uint64_t head = (16u - ((uintptr_t)d & 15u)) & 15u;
    const uint64_t hn = head < nb ? head : nb;
    if (l < hn) d[l] = s[l];
    s += hn;
    d += hn;
    nb -= hn;
    const uint64_t nv = nb / 16;
    const uint4 *s4 = (const uint4 *)s;
    uint4 *d4 = (uint4 *)d;
    uint64_t j = l;
    for (; j + 192 < nv; j += 256) {
        const uint4 a = s4[j], b = s4[j + 64], c = s4[j + 128], e = s4[j + 192];
        d4[j] = a;
        d4[j + 64] = b;
        d4[j + 128] = c;
        d4[j + 192] = e;
    }
    for (; j < nv; j += 64) d4[j] = s4[j];
    const uint64_t t = nv * 16 + l;
    if (t < nb) d[t] = s[t];
}

extern "C" int kvm_d2d_batched(kvm_state *st, const void *const *src, void *const *dst,
                               const size_t *nbytes, int n) {
    if (!st || n < 0 || (n > 0 && (!src || !dst || !nbytes))) return kvm_fail(st, KVM_EINVAL, "d2d_batched: args");
    if (n == 0) return KVM_OK;
    if (n > 65535) return kvm_fail(st, KVM_ERANGE, "d2d_batched: %d ops > 65535", n);
    std::vector<kvm_copy_op> ops;
    for (int i = 0; i < n; ++i) {
        if (nbytes[i] && (!src[i] || !dst[i])) return kvm_fail(st, KVM_EINVAL, "d2d_batched: op %d: null pointer", i);
        for (uint64_t off = 0; off < nbytes[i]; off += KVM_COPY_CHUNK) {
            const uint64_t left = nbytes[i] - off;
            ops.push_back({(const uint8_t *)src[i] + off, (uint8_t *)dst[i] + off,
                           left < KVM_COPY_CHUNK ? left : (uint64_t)KVM_COPY_CHUNK});
        }
    }
    if (ops.empty()) return KVM_OK;
    if (ops.size() > (1u << 26)) return kvm_fail(st, KVM_ERANGE, "d2d_batched: %zu chunks", ops.size());
    KVM_HIP(st, hipSetDevice(st->device));
    void *d = kvm_upload_desc(st, ops.data(), ops.size() * sizeof(kvm_copy_op));
    if (!d) return kvm_fail(st, KVM_ENOMEM, "d2d_batched: descriptor upload");
    const uint32_t nc = (uint32_t)ops.size();
    hipLaunchKernelGGL(k_copy_ops, dim3(kvm_cdiv(nc, 4)), dim3(256), 0, st->stream, (const kvm_copy_op *)d, nc);
    KVM_LAUNCH_CHECK(st, "d2d_batched");
    return KVM_OK;
}

// ---------------------------------------------------------------------------
// The slot seam of the reference runtime (kvmem::KvMemBackend,
// kvmem/include/kvmem/kvmem_backend.hpp:11-27, as SlotBackend implements it,
// llama-memory-kvmem.h:220-232): a host free list of window slots and byte
// copies of one slot's rows, every layer's K rows then V rows.
// ---------------------------------------------------------------------------
extern "C" int kvm_slot_pool_reset(kvm_slot_pool *p) {
    if (!p || (p->n_slots && !p->free_slots)) return KVM_EINVAL;
    // reset_slots (llama-memory-kvmem.cpp:1018-1024): pushed n-1 .. 0, so the
    // first allocations return 0, 1, 2, ...
    for (uint32_t i = 0; i < p->n_slots; ++i) p->free_slots[i] = (int32_t)(p->n_slots - 1 - i);
    p->n_free = p->n_slots;
    return KVM_OK;
}

extern "C" int32_t kvm_slot_alloc(kvm_slot_pool *p) {
    if (!p || p->n_free == 0) return -1;                        // alloc_slot, 1720-1727
    return p->free_slots[--p->n_free];
}

extern "C" int kvm_slot_free(kvm_slot_pool *p, int32_t slot) {
    if (!p) return KVM_EINVAL;
    if (slot < 0) return KVM_OK;                                // free_slot, 1729-1734
    if ((uint32_t)slot >= p->n_slots || p->n_free >= p->n_slots) return KVM_ERANGE;
    p->free_slots[p->n_free++] = slot;
    return KVM_OK;
}

// Bytes per layer of one slot: block_tokens K rows, then block_tokens V rows.
static uint64_t slot_span(const kvm_window *w, uint64_t *kspan) {
    const uint64_t krow = (uint64_t)w->n_head_kv * (w->k_type == KVM_TYPE_Q8_0   ? w->head_dim / 32 * 34
                                                     : w->k_type == KVM_TYPE_Q4_0 ? w->head_dim / 32 * 18
                                                                                  : w->head_dim * 2);
    const uint64_t vrow = (uint64_t)w->n_head_kv * (w->v_type == KVM_TYPE_Q4_0 ? w->head_dim / 32 * 18 : w->head_dim * 2);
    *kspan = w->block_tokens * krow;
    return *kspan + w->block_tokens * vrow;
}

static int slot_copy_check(kvm_state *st, const kvm_window *const *layers, uint32_t n_layers, int32_t slot,
                           const void *host, uint64_t bytes, uint64_t *need, const char *what) {
    if (!st || !layers || !host) return kvm_fail(st, KVM_EINVAL, "%s: null argument", what);
    *need = 0;
    for (uint32_t il = 0; il < n_layers; ++il) {
        int rc = kvm_window_check(layers[il]);
        if (rc) return kvm_fail(st, rc, "%s: layer %u: bad window", what, il);
        if (slot < 0 || (uint64_t)(slot + 1) * layers[il]->block_tokens > layers[il]->n_cells)
            return kvm_fail(st, KVM_ERANGE, "%s: slot %d outside layer %u's window", what, slot, il);
        uint64_t kspan;
        *need += slot_span(layers[il], &kspan);
    }
    if (bytes < *need) return kvm_fail(st, KVM_ERANGE, "%s: %llu bytes < %llu", what, (unsigned long long)bytes,
                                       (unsigned long long)*need);
    return KVM_OK;
}

extern "C" int kvm_slot_copy_to_host(kvm_state *st, const kvm_window *const *layers, uint32_t n_layers,
                                     int32_t slot, void *host, uint64_t bytes) {
    uint64_t need;
    int rc = slot_copy_check(st, layers, n_layers, slot, host, bytes, &need, "slot_copy_to_host");
    if (rc || need == 0) return rc;
    uint8_t *stage = (uint8_t *)kvm_workspace(st, need);
    if (!stage) return kvm_fail(st, KVM_ENOMEM, "slot_copy_to_host: staging of %llu bytes", (unsigned long long)need);
    uint64_t off = 0;
    for (uint32_t il = 0; il < n_layers; ++il) {
        const kvm_window *w = layers[il];
        uint64_t kspan;
        const uint64_t span = slot_span(w, &kspan);
        rc = kvm_window_export_rows(st, w, (uint32_t)slot * w->block_tokens, w->block_tokens, stage + off, stage + off + kspan);
        if (rc) return rc;
        off += span;
    }
    KVM_HIP(st, hipMemcpyAsync(host, stage, need, hipMemcpyDeviceToHost, st->stream));
    KVM_HIP(st, hipStreamSynchronize(st->stream));
    return KVM_OK;
}

extern "C" int kvm_slot_copy_from_host(kvm_state *st, const kvm_window *const *layers, uint32_t n_layers,
                                       int32_t slot, const void *host, uint64_t bytes) {
    uint64_t need;
    int rc = slot_copy_check(st, layers, n_layers, slot, host, bytes, &need, "slot_copy_from_host");
    if (rc || need == 0) return rc;
    uint8_t *stage = (uint8_t *)kvm_workspace(st, need);
    if (!stage) return kvm_fail(st, KVM_ENOMEM, "slot_copy_from_host: staging of %llu bytes", (unsigned long long)need);
    KVM_HIP(st, hipMemcpyAsync(stage, host, need, hipMemcpyHostToDevice, st->stream));
    uint64_t off = 0;
    for (uint32_t il = 0; il < n_layers; ++il) {
        const kvm_window *w = layers[il];
        uint64_t kspan;
        const uint64_t span = slot_span(w, &kspan);
        rc = kvm_window_import_rows(st, w, (uint32_t)slot * w->block_tokens, w->block_tokens, stage + off,
                                    stage + off + kspan, nullptr);
        if (rc) return rc;
        if (w->pending_rows)   // the slot now equals its host copy: nothing to harvest
            pending_rows(st, w, (uint32_t)slot * w->block_tokens, w->block_tokens, PENDING_CLEAR);
        off += span;
    }
    KVM_HIP(st, hipStreamSynchronize(st->stream));
    return KVM_OK;
}

// ---------------------------------------------------------------------------
// Harvest of a block of generated tokens into the host history
// (harvest_gpu_v, llama-memory-kvmem.cpp:3583-3690, through the stage-out
// gather and one device-to-host copy, llama-kvmem-stagein.cu:879-969).  The
// history keeps unrotated K (the stage-in re-applies RoPE), so the block's K
// rows are the q8_0 rows of its captured pre-RoPE K, quantised here with the
// ggml q8_0 formula; its V rows are the window's cache rows, unchanged.
// ---------------------------------------------------------------------------
__global__ void k_quant_view_q8(view_args v, uint32_t tok0, uint32_t n, uint32_t n_embd, uint8_t *dst) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;     // 32-value block
    const uint32_t nb = n_embd / 32;
    if (i >= (uint64_t)n * nb) return;
    const uint32_t t = (uint32_t)(i / nb), b = (uint32_t)(i % nb);
    float x[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) x[j] = view_load(v, tok0 + t, 32 * b + j);
    uint16_t d;
    int8_t q[32];
    kvm_quant_block_q8_0(x, &d, q);
    uint8_t *o = dst + i * 34;
    o[0] = (uint8_t)d;
    o[1] = (uint8_t)(d >> 8);
#pragma unroll
    for (int j = 0; j < 32; ++j) o[2 + j] = (uint8_t)q[j];
}

// the same for a q4_0 K cache (quant_q4_0's arithmetic)
__global__ void k_quant_view_q4(view_args v, uint32_t tok0, uint32_t n, uint32_t n_embd, uint8_t *dst) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;     // 32-value block
    const uint32_t nb = n_embd / 32;
    if (i >= (uint64_t)n * nb) return;
    const uint32_t t = (uint32_t)(i / nb), b = (uint32_t)(i % nb);
    float x[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) x[j] = view_load(v, tok0 + t, 32 * b + j);
    uint16_t d;
    uint8_t q[16];
    kvm_quant_block_q4_0(x, &d, q);
    uint8_t *o = dst + i * 18;
    o[0] = (uint8_t)d;
    o[1] = (uint8_t)(d >> 8);
#pragma unroll
    for (int j = 0; j < 16; ++j) o[2 + j] = q[j];
}

extern "C" int kvm_harvest_block(kvm_state *st, const kvm_window *w, uint32_t cell0, uint32_t n,
                                 const kvm_view *k_prerope, uint32_t tok0, void *k_raw_rows, void *v_rows,
                                 const kvm_meank_index *ix, uint32_t il, uint32_t pos0) {
    if (!st) return KVM_EINVAL;
    int rc = kvm_window_check(w);
    if (rc) return kvm_fail(st, rc, "harvest: bad window");
    if (!kvm_k_quant(w->k_type)) return kvm_fail(st, KVM_EUNSUPPORTED, "harvest: q8_0 or q4_0 K history only");
    if ((uint64_t)cell0 + n > w->n_cells) return kvm_fail(st, KVM_ERANGE, "harvest: cells past the window");
    const uint32_t n_embd = w->n_head_kv * w->head_dim;
    rc = view_check(st, k_prerope, n_embd, "harvest");
    if (rc) return rc;
    if ((uint64_t)tok0 + n > (uint64_t)k_prerope->ne2) return kvm_fail(st, KVM_ERANGE, "harvest: tokens past the view");
    if (!k_raw_rows || !v_rows) return kvm_fail(st, KVM_EINVAL, "harvest: null history rows");
    if (n == 0) return KVM_OK;
    const bool q4 = w->k_type == KVM_TYPE_Q4_0;
    const uint64_t krow = (uint64_t)n_embd / 32 * (q4 ? 18 : 34);
    const uint64_t vrow = w->v_type == KVM_TYPE_Q4_0 ? (uint64_t)n_embd / 32 * 18 : (uint64_t)n_embd * 2;
    const uint64_t kb = n * krow, vb = n * vrow;
    uint8_t *stage = (uint8_t *)kvm_workspace(st, kb + vb);
    if (!stage) return kvm_fail(st, KVM_ENOMEM, "harvest: staging of %llu bytes", (unsigned long long)(kb + vb));
    KVM_HIP(st, hipSetDevice(st->device));
    // the gather: K rows quantised from the view, V rows out of the tiles
    const uint64_t nblk = (uint64_t)n * (n_embd / 32);
    if (q4)
        hipLaunchKernelGGL(k_quant_view_q4, dim3(kvm_cdiv(nblk, 256)), dim3(256), 0, st->stream, view_of(k_prerope),
                           tok0, n, n_embd, stage);
    else
        hipLaunchKernelGGL(k_quant_view_q8, dim3(kvm_cdiv(nblk, 256)), dim3(256), 0, st->stream, view_of(k_prerope),
                           tok0, n, n_embd, stage);
    KVM_LAUNCH_CHECK(st, "harvest");
    rc = kvm_window_export_rows(st, w, cell0, n, nullptr, stage + kb);
    if (rc) return rc;
    if (ix) {
        // the mean-K index from the same captured rows (write_layer_mean_k)
        kvm_view part = *k_prerope;
        part.data = (const uint8_t *)k_prerope->data + (size_t)tok0 * k_prerope->nb2;
        part.ne2 = n;
        rc = kvm_meank_add_view(st, ix, il, pos0, &part);
        if (rc) return rc;
    }
    KVM_HIP(st, hipMemcpyAsync(k_raw_rows, stage, kb, hipMemcpyDeviceToHost, st->stream));
    KVM_HIP(st, hipMemcpyAsync(v_rows, stage + kb, vb, hipMemcpyDeviceToHost, st->stream));
    // the rows are in the host history once the copies are done (stream
    // order): later plans on this stream may overwrite their slots
    if (w->pending_rows) {
        pending_rows(st, w, cell0, n, PENDING_HARVEST);
        KVM_LAUNCH_CHECK(st, "harvest");
    }
    return KVM_OK;
}

