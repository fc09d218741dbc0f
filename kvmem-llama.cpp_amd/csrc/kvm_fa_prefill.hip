// kvm_fa_prefill.hip -- flash attention for long query chunks (chunked prefill,
// long MTP verify).
#include "kvm_internal.h"

extern "C" int kvm_fa_prefill_chunked(kvm_state *st, const kvm_window *w, const void *q, int q_type,
                                      const int32_t *q_pos, uint32_t n_tokens, uint32_t n_head,
                                      float scale, float *out);

extern "C" int kvm_fa_prefill(kvm_state *st, const kvm_window *w, const void *q, int q_type,
                              const int32_t *q_pos, uint32_t n_tokens, uint32_t n_head, float scale,
                              float *out) {
    return kvm_fa_prefill_chunked(st, w, q, q_type, q_pos, n_tokens, n_head, scale, out);
}
