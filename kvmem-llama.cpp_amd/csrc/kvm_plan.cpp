// kvm_plan.cpp -- host-side planning of a retrieval: the mandatory block ids
// of the turn (row spans, the query span, force_pos).  Host code only.
#include "kvm_internal.h"

// llama_memory_kvmem::retrieval_mandatory (src/adapter/llama-memory-kvmem.cpp:
// 4306-4325) over a store whose block b holds n_tokens[b] consecutive original
// positions from sum_{i<b} n_tokens[i] (KvMemStore::register_append,
// kvmem/src/host/kvmem_store.cpp:179-205).  The block containing force_pos is
// found by KvMemStore::block_id_containing's rule (kvmem_store.cpp:158-177):
// none when force_pos lies at or past the store's end.
extern "C" int kvm_retrieval_mandatory(kvm_state *st, const uint32_t *n_tokens, uint32_t n_blocks,
                                       const kvm_row_range *spans, uint32_t n_spans, int32_t query_begin,
                                       int32_t query_end, int32_t force_pos, uint32_t *ids, uint32_t cap,
                                       uint32_t *n_ids) {
    if (!n_ids || (n_blocks && !n_tokens) || (n_spans && !spans) || (cap && !ids))
        return kvm_fail(st, KVM_EINVAL, "retrieval_mandatory: null argument");
    *n_ids = 0;
    int64_t total = 0;
    for (uint32_t b = 0; b < n_blocks; ++b) total += n_tokens[b];
    // the turn's explicit mandatory spans (spans != NULL, possibly none), else
    // the query span (the reference's explicit_spans_ test)
    kvm_row_range query{query_begin, query_end > 0 ? query_end : (int32_t)(total < INT32_MAX ? total : INT32_MAX)};
    const kvm_row_range *rg = spans;
    uint32_t nr = spans ? n_spans : 0u;
    if (!spans && query_begin >= 0) {
        rg = &query;
        nr = 1;
    }
    uint32_t n = 0;
    auto push = [&](uint32_t id) -> bool {
        if (n >= cap) return false;
        ids[n++] = id;
        return true;
    };
    int64_t start = 0;
    for (uint32_t b = 0; b < n_blocks; ++b) {
        const int64_t end = start + n_tokens[b];
        for (uint32_t r = 0; r < nr; ++r) {
            if (end > rg[r].begin && start < rg[r].end) {
                if (!push(b)) return kvm_fail(st, KVM_ERANGE, "retrieval_mandatory: more than %u ids", cap);
                break;
            }
        }
        start = end;
    }
    if (force_pos >= 0 && force_pos < total) {
        start = 0;
        for (uint32_t b = 0; b < n_blocks; ++b) {
            if (force_pos >= start && force_pos < start + n_tokens[b]) {
                if (!push(b)) return kvm_fail(st, KVM_ERANGE, "retrieval_mandatory: more than %u ids", cap);
                break;
            }
            start += n_tokens[b];
        }
    }
    *n_ids = n;
    return KVM_OK;
}
