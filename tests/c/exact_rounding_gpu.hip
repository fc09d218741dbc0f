// Exhaustive gfx950 check of the device quantisers' division-free helpers
// (kvm_internal.h) against the IEEE operations they replace, on the device
// itself: kvm_recip_or0(d) against d != 0 ? 1/d : 0 and kvm_div127(a) against
// a / 127 for every finite float of either sign (but a = -0, for which
// kvm_div127 gives +0: it divides an amax), kvm_round_away(y) against
// (int)roundf(y) for every |y| < 2^23.  Thread t checks the 1024 magnitudes
// t*1024 .. t*1024+1023 and writes its three mismatch counts to out[3t..3t+2].
// Prints "ok" and exits 0 when every count is zero.
#include "../../kvmem-llama.cpp_amd/csrc/kvm_internal.h"

#include <cstdio>
#include <vector>

#define NT (1u << 21)      // threads: NT * PER = 2^31 magnitudes
#define PER 1024u

__global__ void __launch_bounds__(256) k_check(uint32_t *out) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    uint32_t c_rcp = 0, c_div = 0, c_rnd = 0;
    for (uint32_t j = 0; j < PER; ++j) {
        const uint32_t u = t * PER + j;
        if (u >= 0x7f800000u) break;                 // inf and NaN are not inputs
        for (uint32_t s = 0; s < 2; ++s) {
            const float x = __uint_as_float(u | (s << 31));
            const float r = x != 0.0f ? kvm_fdiv(1.0f, x) : 0.0f;
            c_rcp += __float_as_uint(kvm_recip_or0(x)) != __float_as_uint(r);
            if (u != 0u || s == 0u)
                c_div += __float_as_uint(kvm_div127(x)) != __float_as_uint(kvm_fdiv(x, 127.0f));
            if (u < 0x4b000000u) c_rnd += kvm_round_away(x) != (int)roundf(x);
        }
    }
    out[3u * t + 0] = c_rcp;
    out[3u * t + 1] = c_div;
    out[3u * t + 2] = c_rnd;
}

int main() {
    uint32_t *d_out = nullptr;
    if (hipMalloc(&d_out, sizeof(uint32_t) * 3u * NT) != hipSuccess) { std::puts("hipMalloc failed"); return 2; }
    hipLaunchKernelGGL(k_check, dim3(NT / 256u), dim3(256), 0, 0, d_out);
    if (hipDeviceSynchronize() != hipSuccess) { std::puts("kernel failed"); return 3; }
    std::vector<uint32_t> h(3u * NT);
    if (hipMemcpy(h.data(), d_out, sizeof(uint32_t) * h.size(), hipMemcpyDeviceToHost) != hipSuccess) return 4;
    (void)hipFree(d_out);
    unsigned long long c[3] = {0, 0, 0};
    for (size_t t = 0; t < NT; ++t)
        for (int j = 0; j < 3; ++j) c[j] += h[3 * t + j];
    std::printf("%s recip_or0 %llu div127 %llu round_away %llu mismatches\n",
                c[0] || c[1] || c[2] ? "FAIL" : "ok", c[0], c[1], c[2]);
    return c[0] || c[1] || c[2] ? 1 : 0;
}
