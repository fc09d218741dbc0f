/* A C caller of the library through include/kvm_hotpath.h only (plain C99, no
 * C++ and no torch).  First: a q8_0/q4_0 window is filled from pinned host
 * rows, exported back, and attended by one decode launch; the output is
 * checked against the C oracle's ggml-semantics restatement, and an error path
 * is checked for its status code and message.  Second: a whole decode step on
 * a stream the caller created, with no synchronisation between the calls, as
 * a ggml-hip backend would issue them on its own stream: the mean-K index and
 * the query accumulator from device rows, the current tokens' K/V rows
 * imported from device memory into the window's generation cells, the
 * two-launch step (scoring, then top-k + stage-in + attention), and the
 * harvest of the current tokens into pinned history rows; one sync at the
 * end, then the selection, the staged bytes, the attention output and the
 * harvested rows are checked against the C oracle.  Device memory comes from
 * the HIP runtime, as a llama.cpp backend's tensors would.  Exit status 0 =
 * pass. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "kvm_hotpath.h"
#include "kvm_oracle.h"

#define H 4
#define G 6
#define D 256
#define NQ (H * G)
#define CELLS 512
#define BT 128
#define NTOK 4
#define KROW (H * D / 32 * 34)
#define VROW (H * D / 32 * 18)

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static float frand(void) {   /* uniform in [-1, 1), xorshift64* */
    rng_state ^= rng_state >> 12;
    rng_state ^= rng_state << 25;
    rng_state ^= rng_state >> 27;
    return (float)((rng_state * 2685821657736338717ull) >> 40) / (float)(1u << 23) - 1.0f;
}

#define CHECK_HIP(x)                                                          \
    do {                                                                      \
        if ((x) != hipSuccess) {                                              \
            fprintf(stderr, "%s:%d: %s failed\n", __FILE__, __LINE__, #x);    \
            return 2;                                                         \
        }                                                                     \
    } while (0)

#define CHECK_KVM(x)                                                                   \
    do {                                                                               \
        if ((x) != KVM_OK) {                                                           \
            fprintf(stderr, "%s:%d: %s: %s\n", __FILE__, __LINE__, #x, kvm_state_last_error(st)); \
            return 1;                                                                  \
        }                                                                              \
    } while (0)

/* the decode step on the caller's stream (see the file's comment) */
#define S_BLOCKS 12
#define S_HIST (S_BLOCKS * BT)
#define S_SLOTS 8
#define S_CELLS (S_SLOTS * BT)
#define S_BUDGET 6
#define S_GEN0 (S_BUDGET * BT) /* the current tokens' cells and positions */
#define EMBD (H * D)
#define QEMBD (NQ * D)
static int decode_step_on_caller_stream(void) {
    hipStream_t stream;
    CHECK_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
    kvm_state *st = kvm_state_create(0);
    if (!st || kvm_state_set_stream(st, stream) != KVM_OK) return 2;
    /* host data: the history (pinned, raw K q8_0 and V q4_0 rows), its fp32 K,
     * the query rows, the current tokens' rows and pre-RoPE K */
    float *kf = malloc(sizeof(float) * S_HIST * EMBD), *vf = malloc(sizeof(float) * S_HIST * EMBD);
    float *qrows = malloc(sizeof(float) * NTOK * QEMBD), *q = malloc(sizeof(float) * NTOK * QEMBD);
    float *cur_k = malloc(sizeof(float) * NTOK * EMBD), *cur_v = malloc(sizeof(float) * NTOK * EMBD);
    uint8_t *hk = kvm_host_alloc(S_HIST * KROW), *hv = kvm_host_alloc(S_HIST * VROW);
    uint8_t *cur_kq = malloc(NTOK * KROW), *cur_vq = malloc(NTOK * VROW);
    if (!kf || !vf || !qrows || !q || !cur_k || !cur_v || !hk || !hv || !cur_kq || !cur_vq) return 2;
    for (int i = 0; i < S_HIST * EMBD; ++i) {
        kf[i] = frand() * 1.7f;
        vf[i] = frand() * 1.7f;
    }
    oracle_quant_q8_0(kf, hk, (int64_t)S_HIST * EMBD);
    oracle_quant_q4_0(vf, hv, (int64_t)S_HIST * EMBD);
    for (int i = 0; i < NTOK * QEMBD; ++i) {
        qrows[i] = frand();
        q[i] = frand();
    }
    for (int i = 0; i < NTOK * EMBD; ++i) {
        cur_k[i] = frand() * 1.7f;
        cur_v[i] = frand() * 1.7f;
    }
    oracle_quant_q8_0(cur_k, cur_kq, (int64_t)NTOK * EMBD);   /* stands in for the rotated cache rows */
    oracle_quant_q4_0(cur_v, cur_vq, (int64_t)NTOK * EMBD);
    int32_t qpos[NTOK], cur_pos[NTOK];
    uint32_t ntok[S_BLOCKS];
    for (int t = 0; t < NTOK; ++t) qpos[t] = cur_pos[t] = S_GEN0 + t;
    for (int b = 0; b < S_BLOCKS; ++b) ntok[b] = BT;

    /* device buffers */
    float *d_kf, *d_qrows, *d_q, *d_out, *d_cur_kf;
    uint8_t *d_cur_kq, *d_cur_vq;
    int32_t *d_qpos, *d_cur_pos;
    uint32_t *d_ntok;
    CHECK_HIP(hipMalloc((void **)&d_kf, sizeof(float) * S_HIST * EMBD));
    CHECK_HIP(hipMalloc((void **)&d_qrows, sizeof(float) * NTOK * QEMBD));
    CHECK_HIP(hipMalloc((void **)&d_q, sizeof(float) * NTOK * QEMBD));
    CHECK_HIP(hipMalloc((void **)&d_out, sizeof(float) * NTOK * QEMBD));
    CHECK_HIP(hipMalloc((void **)&d_cur_kf, sizeof(float) * NTOK * EMBD));
    CHECK_HIP(hipMalloc((void **)&d_cur_kq, NTOK * KROW));
    CHECK_HIP(hipMalloc((void **)&d_cur_vq, NTOK * VROW));
    CHECK_HIP(hipMalloc((void **)&d_qpos, sizeof(qpos)));
    CHECK_HIP(hipMalloc((void **)&d_cur_pos, sizeof(cur_pos)));
    CHECK_HIP(hipMalloc((void **)&d_ntok, sizeof(ntok)));
    CHECK_HIP(hipMemcpyAsync(d_kf, kf, sizeof(float) * S_HIST * EMBD, hipMemcpyHostToDevice, stream));
    CHECK_HIP(hipMemcpyAsync(d_qrows, qrows, sizeof(float) * NTOK * QEMBD, hipMemcpyHostToDevice, stream));
    CHECK_HIP(hipMemcpyAsync(d_q, q, sizeof(float) * NTOK * QEMBD, hipMemcpyHostToDevice, stream));
    CHECK_HIP(hipMemcpyAsync(d_cur_kf, cur_k, sizeof(float) * NTOK * EMBD, hipMemcpyHostToDevice, stream));
    CHECK_HIP(hipMemcpyAsync(d_cur_kq, cur_kq, NTOK * KROW, hipMemcpyHostToDevice, stream));
    CHECK_HIP(hipMemcpyAsync(d_cur_vq, cur_vq, NTOK * VROW, hipMemcpyHostToDevice, stream));
    CHECK_HIP(hipMemcpyAsync(d_qpos, qpos, sizeof(qpos), hipMemcpyHostToDevice, stream));
    CHECK_HIP(hipMemcpyAsync(d_cur_pos, cur_pos, sizeof(cur_pos), hipMemcpyHostToDevice, stream));
    CHECK_HIP(hipMemcpyAsync(d_ntok, ntok, sizeof(ntok), hipMemcpyHostToDevice, stream));

    /* the mean-K index and the query accumulator */
    kvm_meank_index ix;
    memset(&ix, 0, sizeof(ix));
    ix.n_layer = 1;
    ix.n_blocks = S_BLOCKS;
    ix.n_head_kv = H;
    ix.head_dim = D;
    ix.block_tokens = BT;
    CHECK_HIP(hipMalloc((void **)&ix.k_sum, sizeof(float) * kvm_meank_k_sum_floats(&ix)));
    CHECK_HIP(hipMalloc((void **)&ix.mean_tokens, sizeof(uint32_t) * S_BLOCKS));
    CHECK_HIP(hipMemsetAsync(ix.k_sum, 0, sizeof(float) * kvm_meank_k_sum_floats(&ix), stream));
    CHECK_HIP(hipMemsetAsync(ix.mean_tokens, 0, sizeof(uint32_t) * S_BLOCKS, stream));
    /* the index carries the blocks' score terms, kept current by kvm_meank_add */
    CHECK_HIP(hipMalloc((void **)&ix.k_norm, sizeof(float) * H * S_BLOCKS));
    /* the accumulator carries the scorer's query terms (kept current by
       reset and add) */
    kvm_query_acc qa = {1, NQ, D, NULL, NULL, H, NULL, NULL};
    CHECK_HIP(hipMalloc((void **)&qa.q_sum, sizeof(float) * QEMBD));
    CHECK_HIP(hipMalloc((void **)&qa.q_count, sizeof(uint32_t)));
    CHECK_HIP(hipMalloc((void **)&qa.q_vec, sizeof(float) * EMBD));
    CHECK_HIP(hipMalloc((void **)&qa.q_norm, sizeof(float) * H));
    CHECK_KVM(kvm_meank_add(st, &ix, 0, 0, S_HIST, d_kf));
    CHECK_KVM(kvm_query_reset(st, &qa));
    CHECK_KVM(kvm_query_add(st, &qa, 0, d_qrows, NTOK));

    /* the window with its slot map, the selection and the history */
    kvm_window w;
    memset(&w, 0, sizeof(w));
    w.n_cells = S_CELLS;
    w.n_head_kv = H;
    w.head_dim = D;
    w.block_tokens = BT;
    w.k_type = KVM_TYPE_Q8_0;
    w.v_type = KVM_TYPE_Q4_0;
    CHECK_HIP(hipMalloc(&w.k, kvm_window_k_bytes(&w)));
    CHECK_HIP(hipMalloc(&w.v, kvm_window_v_bytes(&w)));
    CHECK_HIP(hipMalloc((void **)&w.cell_pos, sizeof(int32_t) * S_CELLS));
    CHECK_HIP(hipMalloc((void **)&w.slot_block, sizeof(uint32_t) * S_SLOTS));
    CHECK_HIP(hipMalloc((void **)&w.slot_base, sizeof(int32_t) * S_SLOTS));
    CHECK_KVM(kvm_window_reset(st, &w));
    kvm_selection sel;
    memset(&sel, 0, sizeof(sel));
    sel.cap = S_BUDGET;
    CHECK_HIP(hipMalloc((void **)&sel.scores, sizeof(double) * S_BLOCKS));
    CHECK_HIP(hipMalloc((void **)&sel.ids, sizeof(uint32_t) * S_BUDGET));
    CHECK_HIP(hipMalloc((void **)&sel.to_base, sizeof(int32_t) * S_BUDGET));
    CHECK_HIP(hipMalloc((void **)&sel.stage_slots, sizeof(uint32_t) * S_BUDGET));
    CHECK_HIP(hipMalloc((void **)&sel.info, sizeof(uint32_t) * 8));
    const kvm_select_params prm = {S_BLOCKS, S_BUDGET, 1, 0, NULL, 0, d_ntok};
    const kvm_history hist = {hk, hv, S_HIST};
    const kvm_rope_params rope = {64, 1e7f, 1.0f, -1};

    /* the current tokens' rows from device memory into the generation cells,
     * the step, and the harvest of those tokens: no sync in between */
    CHECK_KVM(kvm_window_import_rows(st, &w, S_GEN0, NTOK, d_cur_kq, d_cur_vq, d_cur_pos));
    const float scale = 1.0f / sqrtf((float)D);
    CHECK_KVM(kvm_score_topk_stagein_fa_decode(st, &ix, &qa, &prm, &w, &sel, &hist, &rope, d_q, KVM_TYPE_F32, d_qpos,
                                               NTOK, NQ, scale, d_out));
    uint8_t *harv_k = kvm_host_alloc(NTOK * KROW), *harv_v = kvm_host_alloc(NTOK * VROW);
    const kvm_view kview = {d_cur_kf, KVM_TYPE_F32, D, H, NTOK, 4, (size_t)D * 4, (size_t)EMBD * 4};
    CHECK_KVM(kvm_harvest_block(st, &w, S_GEN0, NTOK, &kview, 0, harv_k, harv_v, NULL, 0, 0));
    /* results to pinned host memory on the same stream */
    uint8_t *ek = kvm_host_alloc(S_CELLS * KROW), *ev = kvm_host_alloc(S_CELLS * VROW);
    float *out = kvm_host_alloc(sizeof(float) * NTOK * QEMBD);
    int32_t *cpos = kvm_host_alloc(sizeof(int32_t) * S_CELLS);
    uint32_t *ids = kvm_host_alloc(sizeof(uint32_t) * (S_BUDGET + 8));
    int32_t *to_base = kvm_host_alloc(sizeof(int32_t) * S_BUDGET);
    double *scores = kvm_host_alloc(sizeof(double) * S_BLOCKS);
    if (!harv_k || !harv_v || !ek || !ev || !out || !cpos || !ids || !to_base || !scores) return 2;
    CHECK_KVM(kvm_window_export_rows(st, &w, 0, S_CELLS, ek, ev));
    CHECK_HIP(hipMemcpyAsync(out, d_out, sizeof(float) * NTOK * QEMBD, hipMemcpyDeviceToHost, stream));
    CHECK_HIP(hipMemcpyAsync(cpos, w.cell_pos, sizeof(int32_t) * S_CELLS, hipMemcpyDeviceToHost, stream));
    CHECK_HIP(hipMemcpyAsync(ids, sel.ids, sizeof(uint32_t) * S_BUDGET, hipMemcpyDeviceToHost, stream));
    CHECK_HIP(hipMemcpyAsync(ids + S_BUDGET, sel.info, sizeof(uint32_t) * 8, hipMemcpyDeviceToHost, stream));
    CHECK_HIP(hipMemcpyAsync(to_base, sel.to_base, sizeof(int32_t) * S_BUDGET, hipMemcpyDeviceToHost, stream));
    CHECK_HIP(hipMemcpyAsync(scores, sel.scores, sizeof(double) * S_BLOCKS, hipMemcpyDeviceToHost, stream));
    CHECK_KVM(kvm_state_sync(st));

    /* the selection against the oracle's scores and top-k */
    float *q_sum = calloc(QEMBD, sizeof(float)), *k_sum = calloc((size_t)S_BLOCKS * EMBD, sizeof(float));
    uint32_t mt[S_BLOCKS] = {0}, want_ids[S_BLOCKS + 1];
    double want_scores[S_BLOCKS];
    if (!q_sum || !k_sum) return 2;
    for (int t = 0; t < NTOK; ++t)
        for (int e = 0; e < QEMBD; ++e) q_sum[e] += qrows[t * QEMBD + e];
    for (int b = 0; b < S_BLOCKS; ++b)
        oracle_meank_add(k_sum + (size_t)b * EMBD, &mt[b], kf + (size_t)b * BT * EMBD, 0, BT, EMBD);
    const uint32_t qc = NTOK;
    oracle_score_retrieval(S_BLOCKS, 1, NQ, H, D, q_sum, &qc, k_sum, mt, NULL, want_scores, 1);
    if (memcmp(scores, want_scores, sizeof(want_scores)) != 0) {
        fprintf(stderr, "step: scores differ from the oracle's\n");
        return 1;
    }
    const uint32_t n_sel = oracle_pick_topk(S_BLOCKS, want_scores, S_BUDGET, 1, 0, NULL, 0, want_ids);
    if (ids[S_BUDGET] != n_sel || ids[S_BUDGET + 3] != 0 || memcmp(ids, want_ids, sizeof(uint32_t) * n_sel) != 0) {
        fprintf(stderr, "step: selection differs (n %u vs %u, status %u)\n", ids[S_BUDGET], n_sel, ids[S_BUDGET + 3]);
        return 1;
    }
    /* a staged block's K bytes: RoPE re-applied at its window position */
    float theta[32];
    oracle_rope_theta(1e7f, 1.0f, 64, theta);
    uint8_t *want_k = malloc(BT * KROW);
    if (!want_k) return 2;
    oracle_stagein_k(hk + (size_t)ids[2] * BT * KROW, want_k, BT, H, D, 64, oracle_hadamard_nrot_k(D), to_base[2], theta);
    if (memcmp(ek + (size_t)2 * BT * KROW, want_k, BT * KROW) != 0 ||
        memcmp(ev + (size_t)2 * BT * VROW, hv + (size_t)ids[2] * BT * VROW, BT * VROW) != 0) {
        fprintf(stderr, "step: staged block differs from the oracle's stage-in\n");
        return 1;
    }
    /* the attention over the window the step left (current tokens included) */
    float *ref = malloc(sizeof(float) * NTOK * QEMBD);
    if (!ref) return 2;
    if (oracle_fa_ggml(KVM_TYPE_Q8_0, KVM_TYPE_Q4_0, q, ek, ev, cpos, qpos, NTOK, NQ, H, D, S_CELLS, scale, ref, 1) != 0)
        return 1;
    double err = 0.0, amax = 0.0;
    for (int i = 0; i < NTOK * QEMBD; ++i) {
        const double e = fabs((double)out[i] - (double)ref[i]);
        err = e > err ? e : err;
        amax = fabs(ref[i]) > amax ? fabs(ref[i]) : amax;
    }
    if (!(err <= 2e-3 && err <= 1e-3 * amax)) {
        fprintf(stderr, "step: attention max err %.3g (max |ref| %.3g)\n", err, amax);
        return 1;
    }
    for (int c = S_GEN0; c < S_GEN0 + NTOK; ++c)
        if (cpos[c] != c) {
            fprintf(stderr, "step: current token cell %d at position %d\n", c, cpos[c]);
            return 1;
        }
    /* the harvested rows: q8_0 of the captured pre-RoPE K, the cache's V rows */
    if (memcmp(harv_k, cur_kq, NTOK * KROW) != 0 || memcmp(harv_v, cur_vq, NTOK * VROW) != 0) {
        fprintf(stderr, "step: harvested rows differ\n");
        return 1;
    }
    printf("ok step on the caller's stream: ids");
    for (uint32_t i = 0; i < n_sel; ++i) printf(" %u", ids[i]);
    printf(", attention max err %.3g\n", err);
    kvm_state_free(st);
    CHECK_HIP(hipStreamDestroy(stream));
    return 0;
}

int main(void) {
    if (kvm_abi_version() != KVM_ABI_VERSION) {
        fprintf(stderr, "abi version %d, header %d\n", kvm_abi_version(), KVM_ABI_VERSION);
        return 1;
    }
    kvm_state *st = kvm_state_create(0);
    if (!st) {
        fprintf(stderr, "kvm_state_create failed\n");
        return 2;
    }
    /* host rows: K, V of N(0,1)-like values, quantised by the oracle */
    float *kf = malloc(sizeof(float) * CELLS * H * D), *vf = malloc(sizeof(float) * CELLS * H * D);
    uint8_t *krows = kvm_host_alloc(CELLS * KROW), *vrows = kvm_host_alloc(CELLS * VROW);
    int32_t *cpos = kvm_host_alloc(sizeof(int32_t) * CELLS);
    if (!kf || !vf || !krows || !vrows || !cpos) return 2;
    for (int i = 0; i < CELLS * H * D; ++i) {
        kf[i] = frand() * 1.7f;
        vf[i] = frand() * 1.7f;
    }
    oracle_quant_q8_0(kf, krows, (int64_t)CELLS * H * D);
    oracle_quant_q4_0(vf, vrows, (int64_t)CELLS * H * D);
    for (int c = 0; c < CELLS; ++c) cpos[c] = c % 7 == 3 ? -1 : c;     /* holes */

    /* the window in device memory */
    kvm_window w;
    memset(&w, 0, sizeof(w));
    w.n_cells = CELLS;
    w.n_head_kv = H;
    w.head_dim = D;
    w.block_tokens = BT;
    w.k_type = KVM_TYPE_Q8_0;
    w.v_type = KVM_TYPE_Q4_0;
    CHECK_HIP(hipMalloc(&w.k, kvm_window_k_bytes(&w)));
    CHECK_HIP(hipMalloc(&w.v, kvm_window_v_bytes(&w)));
    CHECK_HIP(hipMalloc((void **)&w.cell_pos, sizeof(int32_t) * CELLS));
    if (kvm_window_check(&w) != KVM_OK) return 1;
    int32_t *dpos;
    CHECK_HIP(hipMalloc((void **)&dpos, sizeof(int32_t) * CELLS));
    CHECK_HIP(hipMemcpy(dpos, cpos, sizeof(int32_t) * CELLS, hipMemcpyHostToDevice));
    if (kvm_window_import_rows(st, &w, 0, CELLS, krows, vrows, dpos) != KVM_OK) {
        fprintf(stderr, "import: %s\n", kvm_state_last_error(st));
        return 1;
    }
    /* export round trip: the same ggml row bytes */
    uint8_t *ek = kvm_host_alloc(CELLS * KROW), *ev = kvm_host_alloc(CELLS * VROW);
    if (kvm_window_export_rows(st, &w, 0, CELLS, ek, ev) != KVM_OK || kvm_state_sync(st) != KVM_OK) return 1;
    if (memcmp(ek, krows, CELLS * KROW) || memcmp(ev, vrows, CELLS * VROW)) {
        fprintf(stderr, "export differs from import\n");
        return 1;
    }

    /* one decode launch: NTOK fp32 query tokens at the last positions */
    float *q = malloc(sizeof(float) * NTOK * NQ * D), *ref = malloc(sizeof(float) * NTOK * NQ * D);
    float *out = malloc(sizeof(float) * NTOK * NQ * D);
    int32_t qpos[NTOK];
    for (int i = 0; i < NTOK * NQ * D; ++i) q[i] = frand();
    for (int t = 0; t < NTOK; ++t) qpos[t] = 300 + 50 * t;       /* later cells are masked */
    float *dq, *dout;
    int32_t *dqpos;
    CHECK_HIP(hipMalloc((void **)&dq, sizeof(float) * NTOK * NQ * D));
    CHECK_HIP(hipMalloc((void **)&dout, sizeof(float) * NTOK * NQ * D));
    CHECK_HIP(hipMalloc((void **)&dqpos, sizeof(qpos)));
    CHECK_HIP(hipMemcpy(dq, q, sizeof(float) * NTOK * NQ * D, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(dqpos, qpos, sizeof(qpos), hipMemcpyHostToDevice));
    const float scale = 1.0f / sqrtf((float)D);
    if (kvm_fa_decode(st, &w, dq, KVM_TYPE_F32, dqpos, NTOK, NQ, scale, dout) != KVM_OK) {
        fprintf(stderr, "fa_decode: %s\n", kvm_state_last_error(st));
        return 1;
    }
    if (kvm_state_sync(st) != KVM_OK) return 1;
    CHECK_HIP(hipMemcpy(out, dout, sizeof(float) * NTOK * NQ * D, hipMemcpyDeviceToHost));
    if (oracle_fa_ggml(KVM_TYPE_Q8_0, KVM_TYPE_Q4_0, q, krows, vrows, cpos, qpos, NTOK, NQ, H, D, CELLS, scale,
                       ref, 1) != 0) {
        fprintf(stderr, "oracle failed\n");
        return 1;
    }
    double err = 0.0, amax = 0.0;
    for (int i = 0; i < NTOK * NQ * D; ++i) {
        const double e = fabs((double)out[i] - (double)ref[i]);
        err = e > err ? e : err;
        amax = fabs(ref[i]) > amax ? fabs(ref[i]) : amax;
    }
    if (!(err <= 2e-3 && err <= 1e-3 * amax)) {
        fprintf(stderr, "attention max err %.3g (max |ref| %.3g)\n", err, amax);
        return 1;
    }

    /* an error path: query heads not a multiple of the kv heads */
    const int rc = kvm_fa_decode(st, &w, dq, KVM_TYPE_F32, dqpos, NTOK, NQ + 1, scale, dout);
    if (rc != KVM_EINVAL || strlen(kvm_state_last_error(st)) == 0) {
        fprintf(stderr, "bad head count: status %d, message '%s'\n", rc, kvm_state_last_error(st));
        return 1;
    }
    printf("ok attention max err %.3g of max |ref| %.3g\n", err, amax);
    hipFree(dq);
    hipFree(dout);
    hipFree(dqpos);
    hipFree(dpos);
    hipFree(w.k);
    hipFree(w.v);
    hipFree(w.cell_pos);
    kvm_host_free(krows);
    kvm_host_free(vrows);
    kvm_host_free(cpos);
    kvm_host_free(ek);
    kvm_host_free(ev);
    free(kf);
    free(vf);
    free(q);
    free(ref);
    free(out);
    kvm_state_free(st);
    return decode_step_on_caller_stream();
}
