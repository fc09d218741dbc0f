/* A C caller of the library through include/kvm_hotpath.h only (plain C99, no
 * C++ and no torch): a q8_0/q4_0 window is filled from pinned host rows,
 * exported back, and attended by one decode launch; the output is checked
 * against the C oracle's ggml-semantics restatement, and an error path is
 * checked for its status code and message.  Device memory comes from the HIP
 * runtime, as a llama.cpp backend's tensors would.  Exit status 0 = pass. */
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
    return 0;
}
