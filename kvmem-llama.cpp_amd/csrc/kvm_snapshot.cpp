// kvm_snapshot.cpp -- reader of the reference's raw-store session snapshot, the
// host history format the stage-in consumes (kvmem/src/host/raw_kv_store.cpp:
// 1225-1287, archive primitives kvmem/include/kvmem/snapshot.hpp:21-80).
//
// Layout (little endian, no padding): u32 magic 0x31564b52, u32 n_layer,
// n_embd_k, n_embd_v, block_tokens, u64 k_row_bytes, k_gpu_row_bytes,
// v_gpu_row_bytes, u64 n_blocks; then per block a u64 section length followed,
// per layer, by u32 n_tokens, k_gpu_tokens, v_gpu_tokens, mean_tokens, u8 k_gpu
// and v_gpu format flags, and five length-prefixed vectors (u64 element count,
// then the elements): k (u8, unrotated K rows), v (u16, fp16 V), k_gpu (u8),
// v_gpu (u8, packed V rows), k_sum (fp32 mean-K sum).  The reader applies the
// reference reader's checks (raw_kv_store.cpp:1251-1282) and hands out one
// layer at a time in the history layout the stage-in reads: rows token-major,
// block b at row b * block_tokens.
#include "kvm_internal.h"

#include <cstring>

// Bounds a reader without the store's configuration puts on header fields.
#define KVM_SNAPSHOT_MAX_EMBD (1u << 20)
#define KVM_SNAPSHOT_MAX_BLOCK_TOKENS (1u << 16)

namespace {

struct snap_cursor {
    const uint8_t *p;
    size_t left;
    bool ok = true;
    template <class T> T scalar() {
        T v{};
        if (left < sizeof(T)) { ok = false; return v; }
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        left -= sizeof(T);
        return v;
    }
    // a vector of at most max_count elements of `esz` bytes: its data pointer and count
    const uint8_t *vec(uint64_t max_count, size_t esz, uint64_t *count) {
        const uint64_t n = scalar<uint64_t>();
        if (!ok || n > max_count || n > left / esz) { ok = false; *count = 0; return nullptr; }
        const uint8_t *d = p;
        p += n * esz;
        left -= n * esz;
        *count = n;
        return d;
    }
};

int read_header(kvm_state *st, snap_cursor &c, kvm_snapshot_info *info) {
    const uint32_t magic = c.scalar<uint32_t>();
    if (!c.ok || magic != 0x31564b52u) return kvm_fail(st, KVM_EINVAL, "snapshot: not a raw-store snapshot");
    info->n_layer = c.scalar<uint32_t>();
    info->n_embd_k = c.scalar<uint32_t>();
    info->n_embd_v = c.scalar<uint32_t>();
    info->block_tokens = c.scalar<uint32_t>();
    info->k_row_bytes = c.scalar<uint64_t>();
    info->k_gpu_row_bytes = c.scalar<uint64_t>();
    info->v_gpu_row_bytes = c.scalar<uint64_t>();
    info->n_blocks = c.scalar<uint64_t>();
    if (!c.ok) return kvm_fail(st, KVM_EINVAL, "snapshot: truncated header");
    if (info->n_layer == 0 || info->block_tokens == 0 || info->n_blocks > c.left / 8)
        return kvm_fail(st, KVM_EINVAL, "snapshot: invalid header");
    // k_row_bytes 0 means fp16 K rows (raw_kv_store.hpp:32)
    if (info->k_row_bytes == 0) info->k_row_bytes = (uint64_t)info->n_embd_k * 2;
    // The reference reader compares every geometry field with its store's
    // configuration (raw_kv_store.cpp:1251-1254).  A reader without one still
    // bounds them: a row is at most fp32 wide, and a block holds at most
    // KVM_SNAPSHOT_MAX_BLOCK_TOKENS rows, so every size product below stays far
    // from 64-bit overflow.
    if (info->n_embd_k == 0 || info->n_embd_k > KVM_SNAPSHOT_MAX_EMBD || info->n_embd_v > KVM_SNAPSHOT_MAX_EMBD ||
        info->block_tokens > KVM_SNAPSHOT_MAX_BLOCK_TOKENS || info->k_row_bytes > 4ull * info->n_embd_k ||
        info->k_gpu_row_bytes > 4ull * info->n_embd_k || info->v_gpu_row_bytes > 4ull * info->n_embd_v)
        return kvm_fail(st, KVM_EINVAL, "snapshot: row geometry out of bounds");
    return KVM_OK;
}

// The reference's SnapshotReader::expect of each configured field
// (raw_kv_store.cpp:1251-1254); k_row_bytes 0 stands for fp16 rows on both sides.
int check_expected(kvm_state *st, const kvm_snapshot_info &in, const kvm_snapshot_info *ex) {
    if (!ex) return KVM_OK;
    const uint64_t ekr = ex->k_row_bytes ? ex->k_row_bytes : (uint64_t)ex->n_embd_k * 2;
    if (in.n_layer != ex->n_layer || in.n_embd_k != ex->n_embd_k || in.n_embd_v != ex->n_embd_v ||
        in.block_tokens != ex->block_tokens || in.k_row_bytes != ekr || in.k_gpu_row_bytes != ex->k_gpu_row_bytes ||
        in.v_gpu_row_bytes != ex->v_gpu_row_bytes)
        return kvm_fail(st, KVM_EINVAL, "snapshot: geometry differs from the store's configuration");
    return KVM_OK;
}

// a * b * c, false on 64-bit overflow
bool mul3(uint64_t a, uint64_t b, uint64_t c, uint64_t *r) {
    uint64_t t;
    return !__builtin_mul_overflow(a, b, &t) && !__builtin_mul_overflow(t, c, r);
}

}  // namespace

extern "C" int kvm_snapshot_info_read(kvm_state *st, const void *snap, size_t bytes, kvm_snapshot_info *info) {
    if (!snap || !info) return kvm_fail(st, KVM_EINVAL, "snapshot: null argument");
    snap_cursor c{(const uint8_t *)snap, bytes};
    return read_header(st, c, info);
}

extern "C" int kvm_snapshot_read_layer(kvm_state *st, const void *snap, size_t bytes, uint32_t layer,
                                       const kvm_snapshot_layer *out) {
    if (!snap || !out) return kvm_fail(st, KVM_EINVAL, "snapshot: null argument");
    snap_cursor c{(const uint8_t *)snap, bytes};
    kvm_snapshot_info in{};
    int rc = read_header(st, c, &in);
    if (rc) return rc;
    rc = check_expected(st, in, out->expect);
    if (rc) return rc;
    if (layer >= in.n_layer) return kvm_fail(st, KVM_ERANGE, "snapshot: layer %u of %u", layer, in.n_layer);
    const uint64_t bt = in.block_tokens, nb = in.n_blocks;
    // the reference reader's block-count rule: a store of max_blocks blocks may
    // hold one more, partly filled (raw_kv_store.cpp:1255-1257)
    if (out->max_blocks != UINT64_MAX && nb > out->max_blocks + 1)
        return kvm_fail(st, KVM_ERANGE, "snapshot: %llu blocks > %llu + 1", (unsigned long long)nb,
                        (unsigned long long)out->max_blocks);
    uint64_t k_need = 0, v_need = 0;
    if (!mul3(nb, bt, in.k_row_bytes, &k_need) || !mul3(nb, bt, in.v_gpu_row_bytes, &v_need))
        return kvm_fail(st, KVM_EINVAL, "snapshot: history size overflows");
    if (out->k_rows && out->k_rows_bytes < k_need)
        return kvm_fail(st, KVM_ERANGE, "snapshot: K rows buffer of %zu bytes < %llu", out->k_rows_bytes,
                        (unsigned long long)k_need);
    if (out->v_rows && out->v_rows_bytes < v_need)
        return kvm_fail(st, KVM_ERANGE, "snapshot: V rows buffer of %zu bytes < %llu", out->v_rows_bytes,
                        (unsigned long long)v_need);
    for (uint64_t b = 0; b < nb; ++b) {
        const uint64_t size = c.scalar<uint64_t>();
        if (!c.ok || size > c.left) return kvm_fail(st, KVM_EINVAL, "snapshot: truncated block %llu", (unsigned long long)b);
        const size_t before = c.left;
        for (uint32_t il = 0; il < in.n_layer; ++il) {
            const uint32_t n_tokens = c.scalar<uint32_t>(), k_gpu_tokens = c.scalar<uint32_t>();
            const uint32_t v_gpu_tokens = c.scalar<uint32_t>(), mean_tokens = c.scalar<uint32_t>();
            const uint8_t kfmt = c.scalar<uint8_t>(), vfmt = c.scalar<uint8_t>();
            uint64_t nk, nv, nkg, nvg, ns;
            const uint8_t *k = c.vec(bt * in.k_row_bytes, 1, &nk);
            c.vec(bt * in.n_embd_v, 2, &nv);
            c.vec(bt * in.k_gpu_row_bytes, 1, &nkg);
            const uint8_t *vg = c.vec(bt * in.v_gpu_row_bytes, 1, &nvg);
            const uint8_t *ks = c.vec(in.n_embd_k, 4, &ns);
            if (!c.ok) return kvm_fail(st, KVM_EINVAL, "snapshot: block %llu layer %u: bad vector", (unsigned long long)b, il);
            uint32_t mx = n_tokens > k_gpu_tokens ? n_tokens : k_gpu_tokens;
            mx = mx > v_gpu_tokens ? mx : v_gpu_tokens;
            mx = mx > mean_tokens ? mx : mean_tokens;
            if (mx > bt) return kvm_fail(st, KVM_EINVAL, "snapshot: block %llu: token count above the block", (unsigned long long)b);
            if (kfmt > 1 || vfmt > 1) return kvm_fail(st, KVM_EINVAL, "snapshot: block %llu: KV format flag", (unsigned long long)b);
            if (nkg < (uint64_t)k_gpu_tokens * in.k_gpu_row_bytes || nvg < (uint64_t)v_gpu_tokens * in.v_gpu_row_bytes ||
                (mean_tokens && ns != in.n_embd_k))
                return kvm_fail(st, KVM_EINVAL, "snapshot: block %llu: incomplete KV block", (unsigned long long)b);
            if (il != layer) continue;
            if (out->k_rows) {
                uint8_t *dst = out->k_rows + b * bt * in.k_row_bytes;
                if (nk) std::memcpy(dst, k, nk);
                std::memset(dst + nk, 0, bt * in.k_row_bytes - nk);
            }
            if (out->v_rows) {
                if (nv && !nvg)
                    return kvm_fail(st, KVM_EUNSUPPORTED, "snapshot: block %llu holds fp16 V, not packed V rows", (unsigned long long)b);
                uint8_t *dst = out->v_rows + b * bt * in.v_gpu_row_bytes;
                if (nvg) std::memcpy(dst, vg, nvg);
                std::memset(dst + nvg, 0, bt * in.v_gpu_row_bytes - nvg);
            }
            if (out->k_sum) {
                float *dst = out->k_sum + b * in.n_embd_k;
                if (ns) std::memcpy(dst, ks, ns * 4);
                else std::memset(dst, 0, (size_t)in.n_embd_k * 4);
            }
            if (out->mean_tokens) out->mean_tokens[b] = mean_tokens;
            if (out->n_tokens) out->n_tokens[b] = n_tokens;
        }
        if (before - c.left != size) return kvm_fail(st, KVM_EINVAL, "snapshot: block %llu: section length", (unsigned long long)b);
    }
    return KVM_OK;
}
