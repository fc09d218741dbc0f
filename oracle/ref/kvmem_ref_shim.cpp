// kvmem_ref_shim.cpp -- C entry points over the reference's own kvmem host
// library (kvmem/src/host/{kvmem_store,raw_kv_store,rope}.cpp), compiled from the
// reference sources where they lie by oracle/ref/Makefile into oracle/_ref/.
//
// TEST INFRASTRUCTURE ONLY: the tests use these functions to check the C oracle
// (oracle/kvm_oracle.c) against the real reference code for top-k, selection /
// window remap, mean-K and host RoPE.  Nothing here is shipped or measured.
#include "kvmem/kvmem_store.hpp"
#include "kvmem/raw_kv_store.hpp"
#include "kvmem/rope.hpp"
#include "kvmem/snapshot.hpp"

#include <cstdint>
#include <cstring>
#include <exception>
#include <vector>

extern "C" {

// KvMemStore::pick_topk_blocks (kvmem_store.cpp:357-359) on a store holding
// total_tokens tokens in blocks of block_tokens, with scores installed through
// set_retrieval_scores (kvmem_store.cpp:242-248).  Returns #ids or -1.
int ref_pick_topk(uint32_t total_tokens, uint32_t block_tokens, uint32_t budget_tokens,
                  uint32_t sink_blocks, uint32_t recent_blocks, const double *scores,
                  uint32_t n_scores, const uint32_t *mandatory, uint32_t n_mandatory,
                  uint32_t *out, uint32_t out_cap) {
    try {
        kvmem::KvMemStoreConfig cfg;
        cfg.block_tokens = block_tokens;
        cfg.select_budget = budget_tokens;
        cfg.sink_blocks = sink_blocks;
        cfg.recent_blocks = recent_blocks;
        kvmem::KvMemStore s(cfg);
        s.register_append(total_tokens);
        s.set_retrieval_scores(std::vector<double>(scores, scores + n_scores));
        const auto sel = s.pick_topk_blocks(std::vector<uint32_t>(mandatory, mandatory + n_mandatory));
        if (sel.size() > out_cap) return -1;
        for (size_t i = 0; i < sel.size(); ++i) out[i] = sel[i];
        return static_cast<int>(sel.size());
    } catch (const std::exception &) {
        return -1;
    }
}

// Block bounds of a store filled by register_append in the given chunks
// (kvmem_store.cpp:179-205): orig_pos_start and n_tokens per block; and
// KvMemStore::block_id_containing (kvmem_store.cpp:158-177) of each position in
// `pos`.  Returns #blocks or -1.
int ref_block_layout(const uint32_t *appends, uint32_t n_appends, uint32_t block_tokens, uint32_t *start,
                     uint32_t *n_tokens, uint32_t cap, const int32_t *pos, uint32_t n_pos, int32_t *containing) {
    try {
        kvmem::KvMemStoreConfig cfg;
        cfg.block_tokens = block_tokens;
        kvmem::KvMemStore s(cfg);
        for (uint32_t i = 0; i < n_appends; ++i) s.register_append(appends[i]);
        const auto &blocks = s.blocks();
        if (blocks.size() > cap) return -1;
        for (size_t i = 0; i < blocks.size(); ++i) {
            start[i] = blocks[i].orig_pos_start;
            n_tokens[i] = blocks[i].n_tokens;
        }
        for (uint32_t i = 0; i < n_pos; ++i)
            containing[i] = pos[i] < 0 ? -1 : s.block_id_containing(static_cast<uint32_t>(pos[i]));
        return static_cast<int>(blocks.size());
    } catch (const std::exception &) {
        return -1;
    }
}

// One remap record as the executor sees it (kvmem_store.hpp:75-94).
struct ref_remap {
    uint32_t block_id, n_tokens;
    int32_t from_base, to_base;
    int32_t skip, raw_refresh, working_k_resident, pad;
};

// Runs a sequence of set_selection calls (kvmem_store.cpp:758-882) on one store.
// sel_flat holds n_steps selections back to back, lengths in sel_len.  After
// each step every stage_out block is moved to the CPU tier, as the runtime's
// spill does (kvmem_runtime.cpp:225-249).  The LAST step's plan is returned:
// remaps, stage_in, stage_out, total window tokens.
int ref_set_selection_seq(uint32_t total_tokens, uint32_t block_tokens,
                          const uint32_t *sel_flat, const uint32_t *sel_len, uint32_t n_steps,
                          ref_remap *remaps, uint32_t remap_cap, uint32_t *n_remaps,
                          uint32_t *stage_in, uint32_t *n_stage_in,
                          uint32_t *stage_out, uint32_t *n_stage_out, uint32_t cap,
                          uint32_t *total_window_tokens) {
    try {
        kvmem::KvMemStoreConfig cfg;
        cfg.block_tokens = block_tokens;
        kvmem::KvMemStore s(cfg);
        s.register_append(total_tokens);
        kvmem::KvMemPlan plan;
        size_t off = 0;
        for (uint32_t step = 0; step < n_steps; ++step) {
            std::vector<uint32_t> sel(sel_flat + off, sel_flat + off + sel_len[step]);
            off += sel_len[step];
            plan = s.set_selection(sel);
            for (uint32_t id : plan.stage_out)
                s.set_block_tier(id, kvmem::KvTier::CPU, static_cast<int32_t>(id), -1);
        }
        if (plan.remaps.size() > remap_cap || plan.stage_in.size() > cap || plan.stage_out.size() > cap)
            return -1;
        for (size_t i = 0; i < plan.remaps.size(); ++i) {
            const auto &r = plan.remaps[i];
            remaps[i] = ref_remap{r.block_id, r.n_tokens, r.from_base, r.to_base,
                                  r.skip ? 1 : 0, r.raw_refresh ? 1 : 0,
                                  r.working_k_resident ? 1 : 0, 0};
        }
        *n_remaps = static_cast<uint32_t>(plan.remaps.size());
        std::memcpy(stage_in, plan.stage_in.data(), plan.stage_in.size() * 4);
        *n_stage_in = static_cast<uint32_t>(plan.stage_in.size());
        std::memcpy(stage_out, plan.stage_out.data(), plan.stage_out.size() * 4);
        *n_stage_out = static_cast<uint32_t>(plan.stage_out.size());
        *total_window_tokens = plan.total_window_tokens;
        return 0;
    } catch (const std::exception &) {
        return -1;
    }
}

// RawKvStore::write_layer_mean_k + mean_k (raw_kv_store.cpp:685-705, 987-1054)
// for one layer of n_tokens fp32 token-major K rows written in chunks of
// `chunk` tokens; writes the mean of every block into means[n_blocks][n_embd].
int ref_mean_k(uint32_t n_embd, uint32_t block_tokens, uint32_t n_tokens, uint32_t chunk,
               const float *k, float *means) {
    try {
        kvmem::RawKvStoreConfig cfg;
        cfg.n_layer = 1;
        cfg.n_embd_k = n_embd;
        cfg.n_embd_v = n_embd;
        cfg.block_tokens = block_tokens;
        cfg.k_row_bytes = 1;  // quantized product path: mean-only K authority
        kvmem::RawKvStore raw(cfg);
        for (uint32_t pos = 0; pos < n_tokens;) {
            const uint32_t n = std::min(chunk, n_tokens - pos);
            raw.write_layer_mean_k(pos, n, 0, k + static_cast<size_t>(pos) * n_embd);
            pos += n;
        }
        const uint32_t nb = (n_tokens + block_tokens - 1) / block_tokens;
        for (uint32_t b = 0; b < nb; ++b) raw.mean_k(b, 0, means + static_cast<size_t>(b) * n_embd);
        return static_cast<int>(nb);
    } catch (const std::exception &) {
        return -1;
    }
}

// RawKvStore::write_layer_k_rows (raw_kv_store.cpp:560-598; the fp32 rows feed
// the block mean-K sums) and write_layer_v_gpu (600-646) for every layer in
// chunks of `chunk` tokens, then RawKvStore::snapshot_write (1225-1247) through
// a SnapshotWriter (snapshot.hpp:21-48).  k_rows [n_layer][n_tokens][k_row_bytes],
// k_f32 [n_layer][n_tokens][n_embd_k], v_rows [n_layer][n_tokens][v_gpu_row_bytes].
// Returns the snapshot's byte count (copied to out only if it fits in cap), or -1.
long long ref_raw_snapshot(uint32_t n_layer, uint32_t n_embd_k, uint32_t n_embd_v, uint32_t block_tokens,
                           uint64_t k_row_bytes, uint64_t v_gpu_row_bytes, uint32_t n_tokens, uint32_t chunk,
                           const uint8_t *k_rows, const float *k_f32, const uint8_t *v_rows, uint8_t *out,
                           uint64_t cap) {
    try {
        kvmem::RawKvStoreConfig cfg;
        cfg.n_layer = n_layer;
        cfg.n_embd_k = n_embd_k;
        cfg.n_embd_v = n_embd_v;
        cfg.block_tokens = block_tokens;
        cfg.k_row_bytes = k_row_bytes;
        cfg.v_gpu_row_bytes = v_gpu_row_bytes;
        kvmem::RawKvStore raw(cfg);
        for (uint32_t il = 0; il < n_layer; ++il)
            for (uint32_t pos = 0; pos < n_tokens;) {
                const uint32_t n = std::min(chunk, n_tokens - pos);
                const size_t t = static_cast<size_t>(il) * n_tokens + pos;
                raw.write_layer_k_rows(pos, n, il, k_rows + t * k_row_bytes, k_f32 + t * n_embd_k);
                raw.write_layer_v_gpu(pos, n, il, v_rows + t * v_gpu_row_bytes);
                pos += n;
            }
        std::vector<uint8_t> bytes;
        kvmem::SnapshotWriter w([&](const void *p, size_t n) {
            const uint8_t *b = static_cast<const uint8_t *>(p);
            bytes.insert(bytes.end(), b, b + n);
        });
        raw.snapshot_write(w);
        if (bytes.size() <= cap) std::memcpy(out, bytes.data(), bytes.size());
        return static_cast<long long>(bytes.size());
    } catch (const std::exception &) {
        return -1;
    }
}

// kvmem::rope_neox_apply (rope.cpp:8-45).
void ref_rope_neox(uint32_t n_rot, uint32_t head_dim, uint32_t n_head, float freq_base,
                   float freq_scale, const float *k, uint32_t n_tokens, int32_t pos0, float *out) {
    kvmem::RopeConfig rc;
    rc.n_rot = n_rot;
    rc.n_embd_head = head_dim;
    rc.n_head_kv = n_head;
    rc.freq_base = freq_base;
    rc.freq_scale = freq_scale;
    kvmem::rope_neox_apply(rc, k, n_tokens, pos0, out);
}

}  // extern "C"
