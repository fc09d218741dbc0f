/*
 * kvm_hotpath.h -- C ABI of the MI355X (gfx950) KVMem retrieval + attention hot path.
 *
 * Plain C: pointers, sizes and status codes only.  Every entry point names the
 * reference interface it replaces (paths relative to the reference repository).
 * All device pointers are HIP device addresses on the state's device; "host"
 * pointers must be pinned (hipHostMalloc) so kernels can read them over PCIe.
 *
 * Return convention: KVM_OK (0) on success, a negative KVM_E* code otherwise;
 * the message is available from kvm_state_last_error().  This replaces the
 * reference's `bool` + stderr convention (src/adapter/llama-kvmem-stagein.cu:93-99):
 * a failed call leaves the window unchanged where the reference caller would
 * fall back (src/adapter/llama-memory-kvmem.cpp:4032-4038).
 *
 * Threading: a kvm_state is one execution domain (src/adapter/llama-kvmem-hooks.h:46-55);
 * it must not be used from two threads at once.  All GPU work of a state is
 * enqueued in order on its stream.
 */
#ifndef KVM_HOTPATH_H
#define KVM_HOTPATH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVM_ABI_VERSION 6

enum kvm_status {
    KVM_OK = 0,
    KVM_EINVAL = -1,       /* bad argument or shape */
    KVM_EHIP = -2,         /* HIP runtime error */
    KVM_ENOMEM = -3,       /* allocation failed */
    KVM_ERANGE = -4,       /* size beyond a documented maximum */
    KVM_EUNSUPPORTED = -5, /* type combination not implemented */
    KVM_ETIMEOUT = -6      /* an in-launch wait gave up (kvm_state_sync, kvm_state_status) */
};

/* Waits inside a launch that gave up, as kvm_state_status reports them. */
enum kvm_wait_status {
    KVM_WAIT_MERGE = 1,    /* the attention's split merge: some output rows were not written */
    KVM_WAIT_PLAN = 2,     /* a selecting launch's plan: the attention used the window as it was
                            * and the plan was not staged (the slot map is unchanged) */
    KVM_WAIT_STAGE = 4     /* a stage-in barrier: the plan's items were emptied (selection
                            * info[3] bit 16), so the next plan restages them */
};

/* ggml type ids (ggml.h enum ggml_type) for the types this path handles. */
enum kvm_type {
    KVM_TYPE_F32 = 0,
    KVM_TYPE_F16 = 1,
    KVM_TYPE_Q4_0 = 2,
    KVM_TYPE_Q8_0 = 8,
    KVM_TYPE_BF16 = 30
};

/* Cells per window tile: the window is stored in tiles of 64 cells per kv head. */
#define KVM_TILE_CELLS 64u
/* Largest block count one top-k selection handles (1 M tokens at 128-token blocks). */
#define KVM_MAX_TOPK_BLOCKS 8192u

/* ------------------------------------------------------------------------ */
/* Execution state                                                           */
/* ------------------------------------------------------------------------ */
typedef struct kvm_state kvm_state;

/* Replaces kvmem_gpu_state_create / kvmem_gpu_state_free
 * (src/adapter/llama-kvmem-stagein.h:12-15).  Creates a non-blocking stream of
 * default priority on `device`.  NULL on failure. */
kvm_state *kvm_state_create(int device);
void kvm_state_free(kvm_state *st);
/* Run subsequent work on `hip_stream` (a hipStream_t; NULL is the device's
 * default null stream, as in HIP).  A new state runs on its own non-blocking
 * stream.  Replaces the per-execution stream (llama-kvmem-stagein.cu:334-343). */
int kvm_state_set_stream(kvm_state *st, void *hip_stream);
void *kvm_state_stream(kvm_state *st);
/* Replaces kvmem_stagein_sync (src/adapter/llama-kvmem-stagein.h:31): waits
 * for the state's stream.  Returns KVM_ETIMEOUT when a wait inside one of the
 * state's launches gave up since the last kvm_state_sync / kvm_state_status
 * (the reference's stage-in returns false there and the caller falls back,
 * llama-kvmem-stagein.cu:93-99, llama-memory-kvmem.cpp:4032-4038); the message
 * names the waits.  Reporting clears the status and resets the state's
 * in-launch sync words, so the next launch starts clean: after KVM_ETIMEOUT
 * the results of the launches since the previous sync are not to be used. */
int kvm_state_sync(kvm_state *st);
/* kvm_state_sync that hands back the KVM_WAIT_* bits of the waits that gave up
 * (0 = none) in *status and returns KVM_OK for them. */
int kvm_state_status(kvm_state *st, uint32_t *status);
/* Polls of an in-launch wait (split merge, plan, stage-in barrier) before it
 * gives up; the default (about 0.1-0.2 s of waiting) is restored by
 * KVM_WAIT_POLLS_DEFAULT.  0 makes every such wait give up at once, without a
 * look at its flag: a host-side way to drive the failure paths, under which
 * every kernel still runs to its end.  No counterpart in the reference. */
#define KVM_WAIT_POLLS_DEFAULT (1u << 21)
int kvm_state_set_wait_polls(kvm_state *st, uint32_t polls);
const char *kvm_state_last_error(const kvm_state *st);
int kvm_abi_version(void);
/* Pinned, device-mapped host memory for histories and staging buffers
 * (hipHostMalloc); kernels read it directly over PCIe.  NULL on failure. */
void *kvm_host_alloc(size_t bytes);
void kvm_host_free(void *p);

/* ------------------------------------------------------------------------ */
/* Window: the bounded GPU slot pool of one attention layer                 */
/* (llama-memory-kvmem.cpp:611-779 sizing, 1720-1741 slots).                  */
/* Cell c belongs to slot c / block_tokens.  K and V are kept in a tiled      */
/* layout private to this library (64-cell tiles, per kv head, laid out in    */
/* the order the attention kernel's matrix-core operands consume them);      */
/* kvm_window_import_rows / kvm_window_export_rows convert from / to ggml    */
/* cache rows ([cell][n_head_kv * row(head_dim)]).                            */
/* ------------------------------------------------------------------------ */
typedef struct kvm_window {
    uint32_t n_cells;       /* multiple of KVM_TILE_CELLS and of block_tokens */
    uint32_t n_head_kv;
    uint32_t head_dim;      /* 128 or 256 */
    uint32_t block_tokens;  /* cells per slot (llama_kvmem_params.block_tokens) */
    int32_t k_type;         /* KVM_TYPE_Q8_0 or KVM_TYPE_Q4_0 (with v_type Q4_0), or KVM_TYPE_F16
                             * (with F16); a q4_0 K window holds its rows as q8_0 tile quants
                             * (the nibble minus 8), so its K bytes are q8_0's */
    int32_t v_type;
    void *k;                /* device, kvm_window_k_bytes() */
    void *v;                /* device, kvm_window_v_bytes() */
    int32_t *cell_pos;      /* device [n_cells]: position of the cell's token, -1 = empty */
    uint32_t *slot_block;   /* device [n_slots]: block id held by the slot, 0xffffffff = none */
    int32_t *slot_base;     /* device [n_slots]: position the slot's first cell is baked at */
    /* Optional HBM shadow of the staged blocks' raw K (both NULL = none).  A
     * stage-in writes every staged cell's unrotated K row (the history's q8_0
     * or q4_0 bytes) here and the slot's staged row count into shadow_rows; a later
     * plan that moves a full block to another slot or base re-rotates it from
     * the shadow and moves its V within HBM instead of reading the host
     * history again (the reference reloads such blocks from the host, or moves
     * them with kvmem_d2d_batched without re-rotation,
     * llama-memory-kvmem.cpp:1958-2285).  Importing rows into a slot's cells
     * and kvm_slot_copy_from_host void that slot's shadow (shadow_rows = 0). */
    void *k_shadow;         /* device [n_cells][n_head_kv * row(head_dim)] of the K type */
    uint32_t *shadow_rows;  /* device [n_slots]: rows of the slot the shadow holds */
    /* Optional (NULL = not tracked): per slot the end, in rows from the slot's
     * first cell, of the rows imported into its cells (generated tokens,
     * kvm_window_import_rows) that no kvm_harvest_block has taken into the
     * host history since; 0 = none.  An import raises it to the end of its
     * rows in the slot (importing the same cells again adds nothing), a
     * harvest whose cells reach it clears it, and so does
     * kvm_slot_copy_from_host.  A plan that would overwrite a slot with a
     * nonzero count is refused (kvm_selection info[3] bit 2): the reference harvests
     * the outgoing blocks' generated rows before it spills them and admits
     * the stage-in (apply_plan_to_kv, llama-memory-kvmem.cpp:1811-1857,
     * KvMemRuntime::spill_outgoing / admit_incoming, kvmem_runtime.cpp:225-249). */
    uint32_t *pending_rows; /* device [n_slots] */
} kvm_window;

size_t kvm_window_k_bytes(const kvm_window *w);
size_t kvm_window_v_bytes(const kvm_window *w);
/* Bytes of the optional K shadow (q8_0 and q4_0 K windows; 0 otherwise). */
size_t kvm_window_shadow_bytes(const kvm_window *w);
/* Checks geometry; KVM_OK when the window is usable. */
int kvm_window_check(const kvm_window *w);
/* Empties every cell and slot (reset_slots + seq_rm of the pool,
 * llama-memory-kvmem.cpp:1018-1024). */
int kvm_window_reset(kvm_state *st, const kvm_window *w);
/* Copies ggml cache rows for cells [cell0, cell0+n) into the tiled window and
 * sets their positions (pos: device int32[n], NULL = leave cell_pos alone).
 * k_rows / v_rows: device (or pinned host) rows of w->k_type / w->v_type.
 * This is the cpy of new K/V rows into cache cells (llama-kvmem-batch.cpp:42-50).
 * With w->pending_rows, every slot the cells touch records the end of the rows
 * written (see kvm_window.pending_rows). */
int kvm_window_import_rows(kvm_state *st, const kvm_window *w, uint32_t cell0, uint32_t n,
                           const void *k_rows, const void *v_rows, const int32_t *pos);
/* Inverse of import: ggml rows of cells [cell0, cell0+n).  Used by stage-out
 * (src/adapter/llama-kvmem-stagein.h:48-54) and by byte-exact checks. */
int kvm_window_export_rows(kvm_state *st, const kvm_window *w, uint32_t cell0, uint32_t n,
                           void *k_rows, void *v_rows);

/* ------------------------------------------------------------------------ */
/* The slot seam of the reference runtime (kvmem::KvMemBackend,              */
/* kvmem/include/kvmem/kvmem_backend.hpp:11-27, implemented by SlotBackend,  */
/* src/adapter/llama-memory-kvmem.h:220-232).                                  */
/* ------------------------------------------------------------------------ */
/* A host free list of window slots (free_slots_, llama-memory-kvmem.cpp:
 * 1018-1024, 1720-1741).  free_slots: caller memory of n_slots entries. */
typedef struct kvm_slot_pool {
    uint32_t n_slots;
    uint32_t n_free;
    int32_t *free_slots;
} kvm_slot_pool;
/* reset_slots: every slot free, pushed n_slots-1 .. 0 so that allocation
 * yields 0, 1, 2, ... */
int kvm_slot_pool_reset(kvm_slot_pool *p);
/* alloc_gpu_slot / alloc_slot: the last freed slot, -1 when none is free. */
int32_t kvm_slot_alloc(kvm_slot_pool *p);
/* free_gpu_slot / free_slot: a negative slot is ignored; KVM_ERANGE for a slot
 * outside the pool or a full list. */
int kvm_slot_free(kvm_slot_pool *p, int32_t slot);
/* copy_block_to_host / copy_block_from_host (copy_gpu_block_to_host /
 * _from_host, llama-memory-kvmem.cpp:4073-4147): one slot's cells of every
 * layer, in layer order: block_tokens ggml K rows, then block_tokens V rows.
 * host may be pageable; both return once the copy is complete.  The reference
 * stops silently when `bytes` runs out; here fewer bytes than the layers need
 * is KVM_ERANGE and nothing is copied. */
int kvm_slot_copy_to_host(kvm_state *st, const kvm_window *const *layers, uint32_t n_layers,
                          int32_t slot, void *host, uint64_t bytes);
int kvm_slot_copy_from_host(kvm_state *st, const kvm_window *const *layers, uint32_t n_layers,
                            int32_t slot, const void *host, uint64_t bytes);

/* ------------------------------------------------------------------------ */
/* Row codecs (src/adapter/llama-kvmem-stagein.cu:133-234, ggml quantizers)  */
/* ------------------------------------------------------------------------ */
/* n_rows x n_per_row fp32 (device) -> ggml rows of type (Q8_0, Q4_0 or F16). */
int kvm_quantize_rows(kvm_state *st, int type, const float *src, void *dst, int64_t n_rows,
                      int64_t n_per_row);
/* ggml rows -> fp32 (Q8_0, Q4_0, F16). */
int kvm_dequantize_rows(kvm_state *st, int type, const void *src, float *dst, int64_t n_rows,
                        int64_t n_per_row);

/* ------------------------------------------------------------------------ */
/* Capture-side index upkeep (the GPU half of the attn-qk-capture hook,      */
/* patches/0002-attn-qk-capture-hook.patch:33-60, harvest_pending             */
/* llama-memory-kvmem.cpp:3194).                                              */
/* ------------------------------------------------------------------------ */
/* Query accumulator q_sum_ / q_count_ (llama-memory-kvmem.cpp:3300-3315 reset,
 * 3417-3433 / 3470-3483 add). */
typedef struct kvm_query_acc {
    uint32_t n_layer;
    uint32_t n_head;        /* query heads */
    uint32_t head_dim;
    float *q_sum;           /* device [n_layer][n_head * head_dim] */
    uint32_t *q_count;      /* device [n_layer] */
    /* Optional: the query terms of score_retrieval, formed once per change of
     * the sums instead of once per block tile by the scorer.  With q_vec !=
     * NULL, for kv head h of n_head_kv (group g = n_head / n_head_kv):
     *   q_vec[il][h][d] = (q_sum rows h*g .. h*g+g-1 of layer il added in row
     *                      order) * (1 / (q_count[il] * g))
     *   q_norm[il][h]   = the sum over d, in dim order, of q_vec[il][h][d]^2
     * (fp32, each operation one IEEE rounding: the reference's qv and nq,
     * llama-memory-kvmem.cpp:4167-4185).  kvm_query_reset, _add and _add_view
     * keep them current; a caller that writes q_sum or q_count itself calls
     * kvm_query_refresh before the next scoring.  The scorers then read them
     * (n_head_kv must equal the mean-K index's); NULL: the scorer forms them
     * itself. */
    uint32_t n_head_kv;
    float *q_vec;           /* device [n_layer][n_head_kv * head_dim] or NULL */
    float *q_norm;          /* device [n_layer][n_head_kv] or NULL */
} kvm_query_acc;

/* A captured graph output as the attn-qk-capture hook sees it (patches/
 * 0002-attn-qk-capture-hook.patch:275-290): ne2 tokens of ne1 heads of ne0
 * values; element (token t, head h, dim d) at byte t*nb2 + h*nb1 + d*nb0 of
 * `data` (device), of type F32, F16 or BF16.  The values enter every sum
 * converted exactly to fp32, as the reference's token-major flattening does
 * (bytes_to_f32_token_major, llama-memory-kvmem.cpp:3317-3341). */
typedef struct kvm_view {
    const void *data;
    int type;
    int64_t ne0, ne1, ne2;
    size_t nb0, nb1, nb2;
} kvm_view;

int kvm_query_reset(kvm_state *st, const kvm_query_acc *acc);
/* q_sum[il] += each of the n_rows pre-RoPE query rows in order; q_count[il] += n_rows.
 * q_rows: device fp32 [n_rows][n_head * head_dim]. */
int kvm_query_add(kvm_state *st, const kvm_query_acc *acc, uint32_t il, const float *q_rows,
                  uint32_t n_rows);
/* The capture-format form (harvest_capture / harvest_from_host q-branch,
 * llama-memory-kvmem.cpp:3417-3433, 3470-3483): the pre-RoPE Q view's tokens
 * (ne0 * ne1 = n_head * head_dim) are added in token order, those with keep[t]
 * != 0 only (the rows query_contains admits; keep is host [ne2], NULL = all);
 * q_count[il] += the rows added. */
int kvm_query_add_view(kvm_state *st, const kvm_query_acc *acc, uint32_t il, const kvm_view *q,
                       const uint8_t *keep);
/* Forms q_vec / q_norm of every layer from q_sum / q_count (no counterpart in
 * the reference, which forms them inside score_retrieval): for callers that
 * write the sums directly.  KVM_OK without work when q_vec is NULL. */
int kvm_query_refresh(kvm_state *st, const kvm_query_acc *acc);

/* Mean-K index: per (layer, block) the ordered fp32 sum of pre-RoPE K rows and
 * its token count (RawKvStore k_sum / mean_tokens, raw_kv_store.cpp:215-234). */
typedef struct kvm_meank_index {
    uint32_t n_layer;
    uint32_t n_blocks;      /* capacity in blocks */
    uint32_t n_head_kv;
    uint32_t head_dim;
    uint32_t block_tokens;
    float *k_sum;           /* device [n_layer][ceil(n_blocks/8)][n_head_kv * head_dim][8]:
                             * 8-block tiles, embedding-major inside a tile, so one tile's
                             * sums for every head are one contiguous slab for the scorer;
                             * kvm_meank_k_sum_floats() gives the size */
    uint32_t *mean_tokens;  /* device [n_layer][n_blocks] */
    uint8_t *present;       /* device [n_blocks] (RawKvStore::has_block), or NULL = all */
    float *acc;             /* device [n_layer][n_head_kv * head_dim]: the decode running sum
                             * (kvmem_meank_*, llama-kvmem-stagein.h:58-66), or NULL */
    /* Optional: the block term of score_retrieval that no query changes, formed
     * once per change of a block's sum instead of once per scoring.  With
     * k_norm != NULL, k_norm[il][h][b] = the sum over d, in dim order, of
     * kh[d]^2 with kh = k_sum * (1 / mean_tokens) of kv head h (0 for a block
     * without tokens): the reference's nk (llama-memory-kvmem.cpp:4176-4183),
     * each operation one IEEE rounding.  kvm_meank_add(_view),
     * kvm_meank_acc_flush and kvm_harvest_block keep it current for the blocks
     * they change; a caller that writes k_sum or mean_tokens itself calls
     * kvm_meank_refresh before the next scoring.  The scorers then read it. */
    float *k_norm;          /* device [n_layer][n_head_kv][n_blocks] or NULL */
} kvm_meank_index;

/* Number of floats k_sum must hold for the index geometry in *ix. */
size_t kvm_meank_k_sum_floats(const kvm_meank_index *ix);
/* Forms k_norm of every layer and block from k_sum / mean_tokens (no
 * counterpart in the reference, which forms nk inside score_retrieval): for
 * callers that write the sums directly.  KVM_OK without work when k_norm is
 * NULL. */
int kvm_meank_refresh(kvm_state *st, const kvm_meank_index *ix);

/* RawKvStore::write_layer_mean_k (raw_kv_store.cpp:685-705): add n token rows of
 * layer il starting at original position pos0.  k_rows: device fp32
 * [n][n_head_kv * head_dim].  Also the decode running sum meank_add_f32
 * (llama-kvmem-stagein.cu:270-286). */
int kvm_meank_add(kvm_state *st, const kvm_meank_index *ix, uint32_t il, uint32_t pos0,
                  uint32_t n, const float *k_rows);
/* The same from a captured pre-RoPE K view (harvest_from_host k-branch,
 * llama-memory-kvmem.cpp:3403-3416): its ne2 tokens at positions pos0 ..,
 * ne0 * ne1 = n_head_kv * head_dim. */
int kvm_meank_add_view(kvm_state *st, const kvm_meank_index *ix, uint32_t il, uint32_t pos0,
                       const kvm_view *k);
/* The decode running sum of accepted tokens, ix->acc (kvmem_meank_zero /
 * kvmem_meank_add, llama-kvmem-stagein.cu:1066-1097): zero layer il; add view
 * tokens tok0 .. tok0+n_keep-1 in order; flush it into the block holding
 * positions pos0 .. pos0+n-1 as RawKvStore::write_layer_mean_sum does
 * (raw_kv_store.cpp:707-731, called by decode_mean_flush,
 * llama-memory-kvmem.cpp:3939-3993): the block's sum is zeroed when pos0
 * starts the block, then += acc; mean_tokens as there.  Flushing does not
 * zero the running sum (decode_mean_flush zeroes it next). */
int kvm_meank_acc_zero(kvm_state *st, const kvm_meank_index *ix, uint32_t il);
int kvm_meank_acc_add(kvm_state *st, const kvm_meank_index *ix, uint32_t il, const kvm_view *k,
                      uint32_t tok0, uint32_t n_keep);
int kvm_meank_acc_flush(kvm_state *st, const kvm_meank_index *ix, uint32_t il, uint32_t pos0,
                        uint32_t n);

/* Harvest of n generated tokens into the host history (harvest_gpu_v,
 * llama-memory-kvmem.cpp:3583-3690, through the stage-out gather and one
 * device-to-host copy, llama-kvmem-stagein.cu:879-969): the window cells
 * [cell0, cell0+n) give their V rows (cache format, unchanged) and the view
 * tokens tok0 .. tok0+n-1 of their captured pre-RoPE K give the history's
 * unrotated K rows, quantised to the window's K type (q8_0 or q4_0) with
 * ggml's formula (the rows the re-RoPE stage-in reads back); both are gathered
 * on the device and copied to k_raw_rows / v_rows (host: the history rows of
 * the tokens' positions).  When ix is given the same K rows are added to its
 * layer il at pos0 (write_layer_mean_k).  q8_0 or q4_0 K windows; the copies
 * are done when the state's stream reaches this point (kvm_state_sync).  With w->pending_rows, a slot
 * whose recorded end the cells reach is clear again. */
int kvm_harvest_block(kvm_state *st, const kvm_window *w, uint32_t cell0, uint32_t n,
                      const kvm_view *k_prerope, uint32_t tok0, void *k_raw_rows, void *v_rows,
                      const kvm_meank_index *ix, uint32_t il, uint32_t pos0);

/* ------------------------------------------------------------------------ */
/* Retrieval: scoring + top-k + chronological window layout                 */
/* ------------------------------------------------------------------------ */
typedef struct kvm_select_params {
    uint32_t n_blocks;          /* blocks in the store (<= index capacity) */
    uint32_t budget_blocks;     /* KvMemStore::budget_blocks() */
    uint32_t sink_blocks;       /* always-kept prefix */
    uint32_t recent_blocks;     /* always-kept suffix */
    const uint32_t *mandatory;  /* device [n_mandatory], caller order (newest last), or NULL */
    uint32_t n_mandatory;
    const uint32_t *n_tokens;   /* device [n_blocks] tokens per block */
} kvm_select_params;

/* Device outputs of one retrieval.  info[0] = selected blocks, info[1] = total
 * window tokens, info[2] = slots that need stage-in, info[3] = status (0 ok;
 * bit 0: more selected blocks than `cap`, bit 1: more than the window's slots,
 * bit 2: the plan would overwrite a slot with pending rows and was not staged,
 * bit 4: a stage-in barrier gave up and the plan's items were emptied),
 * info[4] = blocks in stage_out; info[5..7] are zero. */
typedef struct kvm_selection {
    uint32_t cap;               /* capacity of ids / to_base / stage_slots */
    double *scores;             /* device [n_blocks] (score_retrieval output) */
    uint32_t *ids;              /* device [cap], ascending block ids */
    int32_t *to_base;           /* device [cap], window position of each block */
    uint32_t *stage_slots;      /* device [cap], slots whose contents must be (re)staged */
    uint32_t *info;             /* device [8] */
    /* device [cap] or NULL: for stage_slots[i], the slot whose shadow and V
     * hold that block before the plan (a full block already in the window of a
     * window with a shadow), else -1 = stage from the host history */
    int32_t *stage_src;
    /* device [cap] or NULL: the blocks the window's slots hold before the plan
     * that the new selection does not keep, ascending (the plan's stage_out,
     * KvMemStore::set_selection, kvmem/src/host/kvmem_store.cpp:789-795);
     * a window with pending_rows needs them harvested before the plan stages */
    uint32_t *stage_out;
} kvm_selection;

/* A half-open range [begin, end) of original token positions (llama_kvmem_row_range,
 * src/adapter/llama-kvmem-hooks.h:206-209). */
typedef struct kvm_row_range {
    int32_t begin;
    int32_t end;
} kvm_row_range;

/* llama_memory_kvmem::retrieval_mandatory (llama-memory-kvmem.cpp:4306-4325): the
 * block ids a retrieval must keep, for kvm_select_params.mandatory.  The ranges
 * are the turn's explicit mandatory spans when spans is not NULL (the turn set
 * its spans, explicit_spans_; n_spans may be 0: then no range), else the query
 * span [query_begin, query_end > 0 ? query_end : store end) when
 * query_begin >= 0, else none; every block overlapping a range is listed once, in block order;
 * then the block containing force_pos (KvMemStore::block_id_containing,
 * kvmem/src/host/kvmem_store.cpp:158-177) is appended when force_pos >= 0 lies
 * inside the store, even if already listed (the top-k counts each id once).
 * n_tokens: host [n_blocks], block b covering original positions from
 * sum_{i<b} n_tokens[i].  ids: host, capacity cap (n_blocks + 1 always fits).
 * Host code only; st only receives the error message and may be NULL. */
int kvm_retrieval_mandatory(kvm_state *st, const uint32_t *n_tokens, uint32_t n_blocks,
                            const kvm_row_range *spans, uint32_t n_spans, int32_t query_begin,
                            int32_t query_end, int32_t force_pos, uint32_t *ids, uint32_t cap,
                            uint32_t *n_ids);

/* score_retrieval (llama-memory-kvmem.cpp:4149-4196) + pick_topk_blocks
 * (kvmem/src/host/kvmem_store.cpp:357-359, 482-623, TopK policy, no media ranges)
 * + the window remap of set_selection (kvmem_store.cpp:758-882) with the
 * chronological slot order of layout_gpu_slots_by_orig_pos
 * (llama-memory-kvmem.cpp:1958-1993): slot k holds the k-th selected block at
 * window position to_base[k].  When `w` is given, stage_slots lists the slots
 * whose current (block, base) differs from the new layout.  Scores are
 * bit-identical to the reference's host loop; ids are chosen by the strict
 * order (score desc, block id desc).  n_blocks <= KVM_MAX_TOPK_BLOCKS. */
int kvm_score_topk(kvm_state *st, const kvm_meank_index *ix, const kvm_query_acc *q,
                   const kvm_select_params *p, const kvm_window *w, const kvm_selection *out);

/* Several independent retrievals (conversation lanes, each with its own
 * index, query accumulator, parameters, window and outputs) in one launch
 * sequence: one scoring grid over every lane's blocks, then one top-k
 * workgroup per lane.  Each lane's results equal kvm_score_topk on that lane
 * alone.  The reference runs score_retrieval + pick_topk_blocks once per lane
 * from the host (docs/multi-lane-conversations.md:1-20,
 * llama-memory-kvmem.cpp:4149-4196).  n_lanes <= 8. */
typedef struct kvm_retrieval_lane {
    const kvm_meank_index *ix;
    const kvm_query_acc *q;
    const kvm_select_params *p;
    const kvm_window *w;
    const kvm_selection *out;
} kvm_retrieval_lane;
int kvm_score_topk_lanes(kvm_state *st, const kvm_retrieval_lane *lanes, uint32_t n_lanes);

/* Top-k + layout on caller-provided scores (KvMemStore::set_retrieval_scores,
 * kvmem_store.cpp:242-248, then pick_topk_blocks as above): `scores` is a device
 * double [p->n_blocks]; out->scores is not written. */
int kvm_select_topk(kvm_state *st, const double *scores, const kvm_select_params *p,
                    const kvm_window *w, const kvm_selection *out);

/* ------------------------------------------------------------------------ */
/* Stage-in: host history -> window, re-applying RoPE at the window position */
/* ------------------------------------------------------------------------ */
/* NeoX RoPE on the first n_rot dims, theta_i = freq_base^(-2i/n_rot) * freq_scale
 * (kvmem/src/host/rope.cpp:8-45); hadamard_nrot > 0 applies the normalised
 * Walsh-Hadamard transform in hadamard_nrot-wide chunks after RoPE
 * (llama-kvmem-quant.h:22-36; 0 = off, -1 = the attn_rot default for the K type). */
typedef struct kvm_rope_params {
    uint32_t n_rot;
    float freq_base;
    float freq_scale;
    int32_t hadamard_nrot;
} kvm_rope_params;

/* Host-resident (pinned) packed history of one layer: the raw (unrotated,
 * pre-RoPE) K rows and the V rows in cache format, as RawKvStore keeps them
 * (copy_k_gpu / copy_v_gpu, raw_kv_store.cpp:930-985). */
typedef struct kvm_history {
    const void *k_raw;          /* [n_tokens][n_head_kv * row(head_dim)] of window k_type */
    const void *v;              /* [n_tokens][n_head_kv * row(head_dim)] of window v_type */
    uint32_t n_tokens;
} kvm_history;

/* Stages every slot listed by kvm_score_topk's stage_slots: reads the block's
 * raw K and V rows straight from pinned host memory, dequantises K, applies
 * RoPE at to_base + t, the Walsh-Hadamard rotation and q8_0 requantisation
 * (llama-kvmem-stagein.cu:731-786 order) and writes the tiled window; V bytes
 * are moved unchanged (stagein.cu:733-744).  Updates cell_pos, slot_block and
 * slot_base.  Replaces write_block_to_gpu + kvmem_stagein_flush
 * (llama-memory-kvmem.cpp:4000-4071, stagein.cu:669-790) for one retrieval.
 * Entries with sel->stage_src[i] >= 0 (a window with a shadow) take their raw K
 * rows from the shadow of that slot and their V from that slot's tiles, all
 * gathered before any slot is written, so the window ends byte-equal to a
 * stage-in of the whole plan from the host.  A q4_0 K window has
 * q4_0 raw K rows in its history (and shadow), requantised to q4_0 (quant_q4_0,
 * llama-kvmem-stagein.cu:201-234). */
int kvm_stagein_selection(kvm_state *st, const kvm_history *h, const kvm_window *w,
                          const kvm_selection *sel, const kvm_rope_params *rope);

/* Several lanes' stage-in plans in one launch (multi-lane decode,
 * docs/multi-lane-conversations.md:1-20): the reference queues every lane's
 * write_block_to_gpu items and kvmem_stagein_flush runs them as one fused launch
 * (llama-kvmem-stagein.cu:669-790).  At most 8 lanes; all windows share head_dim;
 * each lane is staged exactly as kvm_stagein_selection would stage it. */
typedef struct kvm_stagein_lane {
    const kvm_history *h;
    const kvm_window *w;
    const kvm_selection *sel;
} kvm_stagein_lane;
int kvm_stagein_selection_lanes(kvm_state *st, const kvm_stagein_lane *lanes, uint32_t n_lanes,
                                const kvm_rope_params *rope);

/* Retrieval and stage-in in one call: kvm_score_topk (or its lanes form,
 * hist[i] being lane i's history) then kvm_stagein_selection of every lane's
 * plan, with every argument checked before the first launch.  The reference
 * retrieves (pick_topk_blocks, kvmem_store.cpp:357-623) and then flushes the
 * queued stage-in items (llama-kvmem-stagein.cu:669-790).  An empty plan (the
 * decode loop's steady state) costs the stage-in one short launch. */
int kvm_score_topk_stagein(kvm_state *st, const kvm_meank_index *ix, const kvm_query_acc *q,
                           const kvm_select_params *p, const kvm_window *w, const kvm_selection *out,
                           const kvm_history *h, const kvm_rope_params *rope);
int kvm_score_topk_stagein_lanes(kvm_state *st, const kvm_retrieval_lane *lanes,
                                 const kvm_history *const *hist, uint32_t n_lanes,
                                 const kvm_rope_params *rope);

/* Item-at-a-time form with the reference's arguments
 * (src/adapter/llama-kvmem-stagein.h:36-46).  `dst` is (window, first cell)
 * instead of a raw cache pointer; packed rows are copied into the state's
 * pinned slab, so the host buffer is free on return (stagein.h:23).  flush
 * runs one fused launch over all queued items.  `type` is the window's K type,
 * q8_0 or q4_0 (kvmem_stagein_quant_ok, llama-kvmem-stagein.cu:481-483); q4_0
 * rows are requantised with quant_q4_0's arithmetic (:201-234). */
int kvm_stagein_enqueue_k(kvm_state *st, int type, const void *packed, size_t nbytes,
                          const kvm_window *w, uint32_t cell0, int64_t nt, int64_t n_embd,
                          int nrot, int n_head, int n_embd_head, int n_rot_rope, int32_t pos0,
                          const float *theta, int n_theta);
int kvm_stagein_enqueue_v(kvm_state *st, const void *packed, size_t nbytes,
                          const kvm_window *w, uint32_t cell0, int64_t nt);
int kvm_stagein_flush(kvm_state *st);

/* ------------------------------------------------------------------------ */
/* Flash attention over the window (ggml_flash_attn_ext as called by          */
/* build_attn, patches/0002-attn-qk-capture-hook.patch:225,256)              */
/* ------------------------------------------------------------------------ */
/* q: device [n_tokens][n_head][head_dim] (KVM_TYPE_F32 or KVM_TYPE_BF16);
 * q_pos: device int32 [n_tokens]; out: device fp32 [n_tokens][n_head][head_dim].
 * Cell c is visible to token t iff 0 <= cell_pos[c] <= q_pos[t]
 * (patches/0003-kv-cache-skip-hole-purge.patch:78-90).  Query head h reads kv
 * head h / (n_head / n_head_kv).  A token with no visible cell outputs zeros.
 * Decode form: n_tokens * (n_head / n_head_kv) <= 32 (MTP verify widths). */
int kvm_fa_decode(kvm_state *st, const kvm_window *w, const void *q, int q_type,
                  const int32_t *q_pos, uint32_t n_tokens, uint32_t n_head, float scale,
                  float *out);

/* Several independent conversations in one launch sequence (multi-lane
 * decode, docs/multi-lane-conversations.md:1-20). */
typedef struct kvm_lane {
    const kvm_window *w;
    const void *q;
    const int32_t *q_pos;
    float *out;
    uint32_t n_tokens;
} kvm_lane;
int kvm_fa_decode_lanes(kvm_state *st, const kvm_lane *lanes, uint32_t n_lanes, int q_type,
                        uint32_t n_head, float scale);

/* A decode step's stage-in and attention in one launch: kvm_stagein_selection
 * of (h, sel) into w, then kvm_fa_decode over w, with the results of those two
 * calls.  The attention's workgroups stage the plan themselves and meet at an
 * in-launch barrier before reading the window; with an empty plan (the decode
 * loop's steady state) the step's stage-in launch disappears.  The reference
 * stages in the memory module (write_block_to_gpu + kvmem_stagein_flush,
 * llama-memory-kvmem.cpp:4000-4071) before the graph's flash attention runs
 * (ggml_cuda_flash_attn_ext, ggml-cuda/fattn.cu:457).  q8_0 or q4_0 K / q4_0 V windows;
 * in the lanes form stage[i].w must be lanes[i].w's window. */
int kvm_stagein_fa_decode(kvm_state *st, const kvm_history *h, const kvm_selection *sel,
                          const kvm_rope_params *rope, const kvm_window *w, const void *q, int q_type,
                          const int32_t *q_pos, uint32_t n_tokens, uint32_t n_head, float scale, float *out);
int kvm_stagein_fa_decode_lanes(kvm_state *st, const kvm_stagein_lane *stage, const kvm_lane *lanes,
                                uint32_t n_lanes, const kvm_rope_params *rope, int q_type, uint32_t n_head,
                                float scale);

/* A whole decode step: kvm_score_topk of (ix, qa, p) into sel for window w,
 * then kvm_stagein_fa_decode of (h, sel) and the query into w, with the
 * results of those calls.  Two launches: the scoring grid, then one launch in
 * which one workgroup per lane selects the blocks while the lane's attention
 * workgroups attend over w as it is; a lane whose plan stages anything is
 * staged by those workgroups, which then attend again.  The reference
 * selects (prepare_reselect -> pick_topk_blocks, kvmem_runtime.cpp:112-119,
 * kvmem_store.cpp:357-623),
 * stages the plan (llama-memory-kvmem.cpp:4000-4071, llama-kvmem-stagein.cu:669-790)
 * and then runs the graph's flash attention (ggml-cuda/fattn.cu:457), one
 * after the other.  Steps with more than 4,096 blocks in a lane or a lane
 * without query tokens run as three launches (kvm_score_topk, then
 * kvm_stagein_fa_decode) with the same results; a
 * window that is not q8_0 or q4_0 K / q4_0 V is refused (KVM_EUNSUPPORTED), as
 * kvm_stagein_fa_decode refuses it.  A step whose plan stages anything pays for
 * the attention's first pass: where a plan change is expected (the first
 * retrieval after a new query) the separate calls are faster, and for a plan
 * that moves most of the window kvm_score_topk_stagein then kvm_fa_decode is
 * the fastest (the stage-in kernel runs two workgroups per CU).  In the lanes form ret[i].w must be
 * lanes[i].w's window and hist[i] is lane i's history; every argument is
 * checked before the first launch. */
int kvm_score_topk_stagein_fa_decode(kvm_state *st, const kvm_meank_index *ix, const kvm_query_acc *qa,
                                     const kvm_select_params *p, const kvm_window *w, const kvm_selection *sel,
                                     const kvm_history *h, const kvm_rope_params *rope, const void *q, int q_type,
                                     const int32_t *q_pos, uint32_t n_tokens, uint32_t n_head, float scale,
                                     float *out);
int kvm_score_topk_stagein_fa_decode_lanes(kvm_state *st, const kvm_retrieval_lane *ret,
                                           const kvm_history *const *hist, const kvm_lane *lanes, uint32_t n_lanes,
                                           const kvm_rope_params *rope, int q_type, uint32_t n_head, float scale);
/* The same step from caller scores (set_retrieval_scores, kvmem_store.cpp:242-248,
 * then pick_topk_blocks as in kvm_select_topk): one launch, in which the
 * selector workgroup picks the blocks from scores[n_blocks] while the
 * attention workgroups attend, staging and attending again when the plan
 * stages anything; the results of kvm_select_topk then kvm_stagein_fa_decode.
 * Falls back to those two calls where the one launch does not fit, as
 * kvm_score_topk_stagein_fa_decode does. */
int kvm_select_topk_stagein_fa_decode(kvm_state *st, const double *scores, const kvm_select_params *p,
                                      const kvm_window *w, const kvm_selection *sel, const kvm_history *h,
                                      const kvm_rope_params *rope, const void *q, int q_type,
                                      const int32_t *q_pos, uint32_t n_tokens, uint32_t n_head, float scale,
                                      float *out);

/* kvm_fa_decode without any allocation, for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc.  It has no counterpart in the reference.  The split
 * partials go to a fixed device array of KVM_NOALLOC_SCRATCH_BYTES that the
 * library holds on each GPU until the process ends (looked up when the first
 * kvm_state on the device is created), instead of the state's workspace; the
 * key splits are reduced to fit it, and KVM_ERANGE is returned when even one
 * split's partials (n_head_kv * 32 * (head_dim + 2) * 4 bytes) do not.  Every
 * call on a GPU shares that GPU's array: calls that overlap on one GPU (two
 * streams, two states) race and must be serialised by the caller.  Same
 * arguments, rules and results as kvm_fa_decode. */
#define KVM_NOALLOC_SCRATCH_BYTES (16u << 20)
int kvm_fa_decode_noalloc(kvm_state *st, const kvm_window *w, const void *q, int q_type,
                          const int32_t *q_pos, uint32_t n_tokens, uint32_t n_head, float scale,
                          float *out);

/* Chunked prefill / long MTP verify: any n_tokens; same visibility rule. */
int kvm_fa_prefill(kvm_state *st, const kvm_window *w, const void *q, int q_type,
                   const int32_t *q_pos, uint32_t n_tokens, uint32_t n_head, float scale,
                   float *out);

/* ------------------------------------------------------------------------ */
/* Batched device copies (kvmem_d2d_batched, llama-kvmem-stagein.h:55-56).   */
/* src/dst/nbytes: host arrays of n entries.                                  */
/* ------------------------------------------------------------------------ */
int kvm_d2d_batched(kvm_state *st, const void *const *src, void *const *dst,
                    const size_t *nbytes, int n);

/* ------------------------------------------------------------------------ */
/* Host history from the reference's raw-store session snapshot: the format  */
/* RawKvStore::snapshot_write emits (kvmem/src/host/raw_kv_store.cpp:1225-1247) */
/* and snapshot_read checks (1249-1287).  Host-side parsing only, no GPU work; */
/* st only receives the error message and may be NULL.                        */
/* ------------------------------------------------------------------------ */
typedef struct kvm_snapshot_info {
    uint32_t n_layer, n_embd_k, n_embd_v, block_tokens;
    uint64_t k_row_bytes;      /* unrotated K row (0 in the file = fp16 rows: 2 * n_embd_k) */
    uint64_t k_gpu_row_bytes;  /* packed rotated K row, 0 = none */
    uint64_t v_gpu_row_bytes;  /* packed V row, 0 = none */
    uint64_t n_blocks;
} kvm_snapshot_info;
int kvm_snapshot_info_read(kvm_state *st, const void *snap, size_t bytes, kvm_snapshot_info *info);

/* One layer's history, in the layout kvm_history_* and the stage-in read:
 * K rows and packed V rows token-major, block b at row b * block_tokens (rows
 * a block does not hold are zero); the mean-K sum (n_embd_k fp32), its token
 * count and the block's token count per block.  NULL outputs are skipped.
 * Refusals follow the reference reader (raw_kv_store.cpp:1249-1287): a snapshot
 * of more than max_blocks + 1 blocks (max_blocks is the store's block count;
 * UINT64_MAX = no limit), and, when `expect` is given, one whose geometry
 * differs from it (its SnapshotReader::expect of each configured field).
 * Without `expect` the header is bounded instead: n_embd_k, n_embd_v <= 2^20,
 * block_tokens <= 2^16 and rows at most 4 bytes per value.  fp16-only V is
 * refused.  The per-block outputs hold n_blocks (<= max_blocks + 1) entries. */
typedef struct kvm_snapshot_layer {
    uint8_t *k_rows;
    size_t k_rows_bytes;       /* >= n_blocks * block_tokens * k_row_bytes */
    uint8_t *v_rows;
    size_t v_rows_bytes;       /* >= n_blocks * block_tokens * v_gpu_row_bytes */
    float *k_sum;              /* n_blocks * n_embd_k */
    uint32_t *mean_tokens;     /* n_blocks */
    uint32_t *n_tokens;        /* n_blocks */
    uint64_t max_blocks;
    const kvm_snapshot_info *expect;   /* the store's configuration, or NULL */
} kvm_snapshot_layer;
int kvm_snapshot_read_layer(kvm_state *st, const void *snap, size_t bytes, uint32_t layer,
                            const kvm_snapshot_layer *out);

#ifdef __cplusplus
}
#endif
#endif /* KVM_HOTPATH_H */
