/*
 * kvm_oracle.h -- CPU restatement of the KVMem retrieval + attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links this code:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it,
 * and only to check results against (or as the timed CPU baseline), never as
 * the thing being measured or shipped.
 *
 * Every function restates one piece of the reference's algorithm in plain C and
 * cites the reference file:line it follows (paths relative to the reference
 * repository root).  Where the reference's arithmetic lives in ggml, which is an
 * un-vendored submodule (ggml-org/llama.cpp, pinned 7fe450e19305b828c199d602c23a8337aaa1f03b),
 * the published ggml-CPU semantics are restated and the call site is cited.
 *
 * Pinning status (see tests/test_oracle_*.py for the checks):
 *   f16 codec, q8_0/q4_0 codecs, NeoX RoPE, FWHT, mean-K, top-k, window layout:
 *       pinned (reference KATs, oracle/_ref built from the reference's own
 *       kvmem sources, closed forms and brute force).
 *   score_retrieval: pinned by closed-form / invariant checks only (the adapter
 *       source it restates cannot be compiled without llama.cpp internals).
 *   flash attention: pinned against an independent float64 textbook softmax,
 *       special cases (one live key, equal keys, fully masked) and brute force;
 *       ggml itself is absent, so bit-level ggml parity is "parity unpinned".
 */
#ifndef KVM_ORACLE_H
#define KVM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids used by the reference (ggml.h enum ggml_type). */
enum { ORACLE_T_F32 = 0, ORACLE_T_F16 = 1, ORACLE_T_Q4_0 = 2, ORACLE_T_Q8_0 = 8 };

/* ---- half precision: kvmem/src/host/raw_kv_store.cpp:33-95 (RNE, subnormals) */
uint16_t oracle_f32_to_f16(float f);
float    oracle_f16_to_f32(uint16_t h);

/* ---- ggml block codecs: src/adapter/llama-kvmem-stagein.cu:133-234 -------- */
/* n = number of values, a multiple of 32.  q8_0 block = fp16 d + 32 x int8 (34 B),
 * q4_0 block = fp16 d + 16 B of nibbles (18 B). */
void oracle_quant_q8_0(const float *x, uint8_t *y, int64_t n);
void oracle_dequant_q8_0(const uint8_t *x, float *y, int64_t n);
void oracle_quant_q4_0(const float *x, uint8_t *y, int64_t n);
void oracle_dequant_q4_0(const uint8_t *x, float *y, int64_t n);
/* bytes per row of n values for a ggml type (ggml_row_size). */
int64_t oracle_row_bytes(int type, int64_t n);

/* ---- NeoX RoPE: kvmem/src/host/rope.cpp:8-45, src/adapter/llama-kvmem-stagein.cu:160-179 */
void oracle_rope_theta(float freq_base, float freq_scale, int n_rot, float *theta);
/* cos/sin of the fp32 angle (float)pos * theta[i], correctly rounded from double. */
void oracle_rope_cs(const float *theta, int n_half, int32_t pos, float *c, float *s);
/* In place on x[n_tokens][n_head][head_dim] (token-major), positions pos0 + t. */
void oracle_rope_neox(float *x, int64_t n_tokens, int n_head, int head_dim, int n_rot,
                      int32_t pos0, const float *theta);

/* ---- Walsh-Hadamard: src/adapter/llama-kvmem-stagein.cu:105-131, 583-609 -- */
void oracle_fwht(float *x, int64_t n_rows, int n);
int  oracle_hadamard_nrot_k(int head_dim);            /* llama-kvmem-quant.h:30-36 */
int  oracle_attn_rot_on(int type, int head_dim);       /* llama-kvmem-quant.h:22-28 */

/* ---- stage-in of one K item: stagein.cu:731-786 (dequant -> rope -> fwht -> quant)
 * packed: q8_0 rows [nt][n_head*head_dim]; out: same format.  nrot == 0 skips FWHT. */
void oracle_stagein_k(const uint8_t *packed, uint8_t *out, int64_t nt, int n_head,
                      int head_dim, int n_rot, int nrot, int32_t pos0, const float *theta);
/* The same chain for a q4_0 K cache (k_type ORACLE_T_Q4_0): dequant_q4_0 ->
 * RoPE -> FWHT -> quant_q4_0 (llama-kvmem-stagein.cu:145-158, 201-234, 731-786). */
void oracle_stagein_k_type(int k_type, const uint8_t *packed, uint8_t *out, int64_t nt, int n_head,
                           int head_dim, int n_rot, int nrot, int32_t pos0, const float *theta);

/* ---- mean-K index: kvmem/src/host/raw_kv_store.cpp:215-234, 987-1006 ------ */
/* Ordered fp32 accumulation of `take` token rows starting at in-block offset off. */
void oracle_meank_add(float *k_sum, uint32_t *mean_tokens, const float *k, uint32_t off,
                      uint32_t take, int n_embd);
void oracle_meank_normalize(const float *k_sum, uint32_t mean_tokens, float *out, int n_embd);

/* ---- score_retrieval: src/adapter/llama-memory-kvmem.cpp:4149-4196 ------------
 * q_sum   [n_layer][n_head*head_dim] fp32, q_count [n_layer]
 * k_sum   [n_layer][n_blocks][n_head_kv*head_dim] fp32, mean_tokens [n_layer][n_blocks]
 * present [n_blocks] (raw_->has_block), scores [n_blocks] (double).
 * n_threads > 1 parallelises over blocks (same bits; baseline timing only). */
void oracle_score_retrieval(int n_blocks, int n_layer, int n_head, int n_head_kv, int head_dim,
                            const float *q_sum, const uint32_t *q_count, const float *k_sum,
                            const uint32_t *mean_tokens, const uint8_t *present,
                            double *scores, int n_threads);

/* ---- top-k: kvmem/src/host/kvmem_store.cpp:482-623 (TopK policy) -------------
 * Returns the number of selected ids written to out (ascending). */
uint32_t oracle_pick_topk(uint32_t n, const double *scores, uint32_t budget_blocks,
                          uint32_t sink_blocks, uint32_t recent_blocks,
                          const uint32_t *mandatory, uint32_t n_mandatory, uint32_t *out);

/* ---- window layout: kvmem_store.cpp:758-882 (to_base), llama-memory-kvmem.cpp:1958-1993
 * (slot k <- k-th selected block in chronological order).  n_tokens [n_blocks].
 * Writes to_base[n_sel] and cell_pos[n_slots*block_tokens] (-1 = empty cell);
 * returns total_window_tokens. */
uint32_t oracle_window_layout(const uint32_t *sel, uint32_t n_sel, const uint32_t *n_tokens,
                              uint32_t block_tokens, uint32_t n_slots, int32_t *to_base,
                              int32_t *cell_pos);

/* ---- mandatory block ids from row ranges and force_pos (retrieval_mandatory) ----
 * ranges: n_ranges pairs (begin, end), used when explicit_spans (the turn set its
 * spans; none is then no range), else the query span; out holds n_blocks + 1 ids;
 * returns the count. */
uint32_t oracle_retrieval_mandatory(const uint32_t *n_tokens, uint32_t n_blocks, const int32_t *ranges,
                                    uint32_t n_ranges, int explicit_spans, int32_t query_begin,
                                    int32_t query_end, int32_t force_pos, uint32_t *out);

/* ---- flash attention over a ggml-layout KV window ------------------------------
 * q        [n_tokens][n_head][head_dim] fp32
 * k, v     ggml rows [n_cells][n_head_kv * row(head_dim)] of k_type / v_type
 * cell_pos [n_cells] (-1 empty), q_pos [n_tokens]; visible iff 0 <= cell_pos <= q_pos
 *          (patches/0003-kv-cache-skip-hole-purge.patch:78-90)
 * out      [n_tokens][n_head][head_dim] fp32; a row with no visible key is all zeros.
 * GQA: query head h reads kv head h / (n_head / n_head_kv).
 * oracle_fa_ggml restates ggml-CPU ggml_compute_forward_flash_attn_ext_f16 (Q converted
 * to K's vec_dot type, online softmax with expf, fp32 V accumulation or fp16 for f16 V);
 * oracle_fa_f64 is the float64 textbook softmax over dequantised K/V and unquantised Q. */
int oracle_fa_ggml(int k_type, int v_type, const float *q, const void *k, const void *v,
                   const int32_t *cell_pos, const int32_t *q_pos, int n_tokens, int n_head,
                   int n_head_kv, int head_dim, int n_cells, float scale, float *out,
                   int n_threads);
int oracle_fa_f64(int k_type, int v_type, const float *q, const void *k, const void *v,
                  const int32_t *cell_pos, const int32_t *q_pos, int n_tokens, int n_head,
                  int n_head_kv, int head_dim, int n_cells, double scale, double *out,
                  int n_threads);

/* ---- q8_0 quantisation of a query row as ggml's vec_dot does (quantize_row_q8_0) */
void oracle_quant_q8_0_rows(const float *x, uint8_t *y, int64_t n_rows, int64_t n_per_row);

#ifdef __cplusplus
}
#endif
#endif
