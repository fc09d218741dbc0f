// kvm_state.cpp -- execution state, error reporting, device workspace and the
// host-generated RoPE cos/sin table.
#include "kvm_internal.h"

#include <mutex>
#include <vector>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

int kvm_fail(kvm_state *st, int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (st) st->err = buf;
    return code;
}

extern "C" int kvm_abi_version(void) { return KVM_ABI_VERSION; }

extern "C" kvm_state *kvm_state_create(int device) {
    kvm_state *st = new (std::nothrow) kvm_state();
    if (!st) return nullptr;
    st->device = device;
    if (hipSetDevice(device) != hipSuccess ||
        hipStreamCreateWithFlags(&st->own_stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&st->ev, hipEventDisableTiming) != hipSuccess) {
        if (st->own_stream) (void)hipStreamDestroy(st->own_stream);
        delete st;
        return nullptr;
    }
    st->stream = st->own_stream;
    int n_cu = 0;
    if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && n_cu > 0)
        st->n_cu = (uint32_t)n_cu;
    if (kvm_noalloc_setup(st) != KVM_OK || hipMalloc((void **)&st->fa_sync, kvm_fa_sync_bytes()) != hipSuccess ||
        hipMemsetAsync(st->fa_sync, 0, kvm_fa_sync_bytes(), st->own_stream) != hipSuccess ||
        hipMalloc((void **)&st->stage_sync, KVM_STAGE_SYNC_BYTES) != hipSuccess ||
        hipMemsetAsync(st->stage_sync, 0, KVM_STAGE_SYNC_BYTES, st->own_stream) != hipSuccess ||
        hipStreamSynchronize(st->own_stream) != hipSuccess) {
        if (st->fa_sync) (void)hipFree(st->fa_sync);
        if (st->stage_sync) (void)hipFree(st->stage_sync);
        (void)hipEventDestroy(st->ev);
        (void)hipStreamDestroy(st->own_stream);
        delete st;
        return nullptr;
    }
    return st;
}

extern "C" void kvm_state_free(kvm_state *st) {
    if (!st) return;
    (void)hipSetDevice(st->device);
    if (st->stream) (void)hipStreamSynchronize(st->stream);
    if (st->ws) (void)hipFree(st->ws);
    if (st->rope_tab) (void)hipFree(st->rope_tab);
    if (st->desc) (void)hipFree(st->desc);
    if (st->fa_sync) (void)hipFree(st->fa_sync);
    if (st->fa_ws) (void)hipFree(st->fa_ws);
    if (st->mv_ws) (void)hipFree(st->mv_ws);
    if (st->stage_sync) (void)hipFree(st->stage_sync);
    if (st->slab) (void)hipHostFree(st->slab);
    if (st->ev) (void)hipEventDestroy(st->ev);
    if (st->own_stream) (void)hipStreamDestroy(st->own_stream);
    delete st;
}

extern "C" int kvm_state_set_stream(kvm_state *st, void *hip_stream) {
    if (!st) return KVM_EINVAL;
    st->stream = static_cast<hipStream_t>(hip_stream);
    return KVM_OK;
}

extern "C" void *kvm_state_stream(kvm_state *st) { return st ? (void *)st->stream : nullptr; }

// Waits for the stream, then reads and clears the sticky wait status of the
// state's sync words (and of the scratch array's, when the allocation-free
// entry point ran on the state).  A wait that gave up may have left flags,
// epochs or a plan word that a workgroup of that launch wrote after its
// head's or lane's epoch had moved on; with the stream idle, every sync word
// is zeroed, so the next launch's epochs start from a clean slate.
static int read_status(kvm_state *st, uint32_t *status) {
    *status = 0;
    KVM_HIP(st, hipSetDevice(st->device));
    KVM_HIP(st, hipStreamSynchronize(st->stream));
    uint32_t v[2] = {0u, 0u};
    KVM_HIP(st, hipMemcpy(&v[0], st->fa_sync + KVM_FA_SYNC_STATUS, 4, hipMemcpyDeviceToHost));
    if (st->used_scratch && st->scratch)
        KVM_HIP(st, hipMemcpy(&v[1], (uint32_t *)st->scratch + KVM_FA_SYNC_STATUS, 4, hipMemcpyDeviceToHost));
    *status = v[0] | v[1];
    if (*status) {
        KVM_HIP(st, hipMemsetAsync(st->fa_sync, 0, kvm_fa_sync_bytes(), st->stream));
        KVM_HIP(st, hipMemsetAsync(st->stage_sync, 0, KVM_STAGE_SYNC_BYTES, st->stream));
        if (st->used_scratch && st->scratch)
            KVM_HIP(st, hipMemsetAsync(st->scratch, 0, kvm_fa_sync_bytes(), st->stream));
        KVM_HIP(st, hipStreamSynchronize(st->stream));
    }
    return KVM_OK;
}

extern "C" int kvm_state_sync(kvm_state *st) {
    if (!st) return KVM_EINVAL;
    uint32_t status = 0;
    int rc = read_status(st, &status);
    if (rc) return rc;
    if (status)
        return kvm_fail(st, KVM_ETIMEOUT, "in-launch waits gave up:%s%s%s (status 0x%x)",
                        status & KVM_WAIT_MERGE ? " split merge (output rows not written)" : "",
                        status & KVM_WAIT_PLAN ? " selected plan (not staged, window unchanged)" : "",
                        status & KVM_WAIT_STAGE ? " stage-in barrier (plan items emptied)" : "", status);
    return KVM_OK;
}

extern "C" int kvm_state_status(kvm_state *st, uint32_t *status) {
    if (!st) return KVM_EINVAL;
    if (!status) return kvm_fail(st, KVM_EINVAL, "state_status: null output");
    return read_status(st, status);
}

extern "C" int kvm_state_set_wait_polls(kvm_state *st, uint32_t polls) {
    if (!st) return KVM_EINVAL;
    st->wait_polls = polls;
    return KVM_OK;
}

extern "C" const char *kvm_state_last_error(const kvm_state *st) {
    return st ? st->err.c_str() : "null state";
}

static void *grow(kvm_state *st, void **buf, size_t *have, size_t bytes) {
    if (bytes <= *have) return *buf;
    // The old buffer may still be read by queued kernels: wait before freeing.
    if (*buf) {
        if (hipStreamSynchronize(st->stream) != hipSuccess) return nullptr;
        (void)hipFree(*buf);
        *buf = nullptr;
        *have = 0;
    }
    size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
    if (hipMalloc(buf, want) != hipSuccess) {
        *buf = nullptr;
        return nullptr;
    }
    *have = want;
    return *buf;
}

void *kvm_workspace(kvm_state *st, size_t bytes) { return grow(st, &st->ws, &st->ws_bytes, bytes); }

void *kvm_fa_workspace(kvm_state *st, size_t bytes) { return grow(st, &st->fa_ws, &st->fa_ws_bytes, bytes); }

void *kvm_move_workspace(kvm_state *st, size_t bytes) { return grow(st, &st->mv_ws, &st->mv_ws_bytes, bytes); }

int kvm_resident_blocks(kvm_state *st, const void *fn, int threads, size_t lds, int *blocks) {
    struct entry {
        int device;
        const void *fn;
        int threads;
        size_t lds;
        int blocks;
    };
    static std::mutex mu;
    static std::vector<entry> cache;
    {
        std::lock_guard<std::mutex> lk(mu);
        for (const entry &e : cache)
            if (e.device == st->device && e.fn == fn && e.threads == threads && e.lds == lds) {
                *blocks = e.blocks;
                return KVM_OK;
            }
    }
    KVM_HIP(st, hipSetDevice(st->device));
    KVM_HIP(st, hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    int n = 0;
    KVM_HIP(st, hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, threads, lds));
    if (n < 1) return kvm_fail(st, KVM_ERANGE, "a workgroup of %d threads with %zu bytes of LDS does not fit a CU", threads, lds);
    std::lock_guard<std::mutex> lk(mu);
    cache.push_back(entry{st->device, fn, threads, lds, n});
    *blocks = n;
    return KVM_OK;
}


void *kvm_upload_desc(kvm_state *st, const void *host, size_t bytes) {
    if (bytes > st->desc_bytes) {
        if (st->desc) {
            if (hipStreamSynchronize(st->stream) != hipSuccess) return nullptr;
            (void)hipFree(st->desc);
            st->desc = nullptr;
        }
        size_t want = bytes < 65536 ? 65536 : bytes;
        if (hipMalloc(&st->desc, want) != hipSuccess) {
            st->desc = nullptr;
            st->desc_bytes = 0;
            return nullptr;
        }
        st->desc_bytes = want;
    }
    // The descriptor buffer is reused by the next call: make the copy ordered
    // on the stream and keep the host source alive until it has been consumed.
    if (hipMemcpyAsync(st->desc, host, bytes, hipMemcpyHostToDevice, st->stream) != hipSuccess)
        return nullptr;
    if (hipStreamSynchronize(st->stream) != hipSuccess) return nullptr;
    return st->desc;
}

std::vector<float> kvm_rope_theta(float freq_base, float freq_scale, uint32_t n_rot) {
    std::vector<float> theta(n_rot / 2);
    for (uint32_t i = 0; i < n_rot / 2; ++i)
        theta[i] = powf(freq_base, -2.0f * (float)i / (float)n_rot) * freq_scale;
    return theta;
}

// cos/sin of the fp32 angle (float)pos * theta_i, evaluated in double and
// rounded once to fp32.  The reference evaluates the same angle with libm
// (host, kvmem/src/host/rope.cpp:34-35) or the device sincosf
// (llama-kvmem-stagein.cu:171); a single host-built table makes every
// stage-in bit-reproducible across devices.
int kvm_rope_table(kvm_state *st, const float *theta, uint32_t n_half, uint32_t n_pos) {
    if (n_half == 0 || !theta) return kvm_fail(st, KVM_EINVAL, "rope table: empty theta");
    const bool same = st->rope_tab && st->rope_theta.size() == n_half &&
                      std::memcmp(st->rope_theta.data(), theta, n_half * sizeof(float)) == 0;
    if (same && st->rope_n_pos >= n_pos) return KVM_OK;
    uint32_t want_pos = 4096;
    while (want_pos < n_pos) want_pos *= 2;
    std::vector<float2> tab((size_t)want_pos * n_half);
    for (uint32_t p = 0; p < want_pos; ++p) {
        const float pf = (float)p;
        for (uint32_t i = 0; i < n_half; ++i) {
            const float ang = pf * theta[i];
            tab[(size_t)p * n_half + i] = make_float2((float)cos((double)ang), (float)sin((double)ang));
        }
    }
    const size_t bytes = tab.size() * sizeof(float2);
    if (st->rope_tab) {
        KVM_HIP(st, hipStreamSynchronize(st->stream));
        (void)hipFree(st->rope_tab);
        st->rope_tab = nullptr;
    }
    if (hipMalloc(&st->rope_tab, bytes) != hipSuccess) {
        st->rope_tab = nullptr;
        st->rope_tab_bytes = 0;
        st->rope_theta.clear();
        return kvm_fail(st, KVM_ENOMEM, "rope table: %zu bytes", bytes);
    }
    KVM_HIP(st, hipMemcpyAsync(st->rope_tab, tab.data(), bytes, hipMemcpyHostToDevice, st->stream));
    KVM_HIP(st, hipStreamSynchronize(st->stream));
    st->rope_tab_bytes = bytes;
    st->rope_n_pos = want_pos;
    st->rope_n_half = n_half;
    st->rope_theta.assign(theta, theta + n_half);
    return KVM_OK;
}

extern "C" void *kvm_host_alloc(size_t bytes) {
    void *p = nullptr;
    if (bytes == 0) bytes = 1;
    if (hipHostMalloc(&p, bytes, hipHostMallocMapped | hipHostMallocPortable) != hipSuccess) return nullptr;
    return p;
}

extern "C" void kvm_host_free(void *p) {
    if (p) (void)hipHostFree(p);
}
