/* Exhaustive CPU check of two IEEE-exact rewrites the device quantisers use
 * (kvm_internal.h): kvm_div127, a / 127 as a product and two fma, and
 * kvm_round_away, roundf as a biased truncation.  Host float arithmetic is
 * IEEE binary32 with round-to-nearest-even and a correctly rounded fmaf, as
 * gfx950's v_mul_f32 / v_add_f32 / v_fma_f32 are with denormals kept.
 * Prints the mismatch counts; exits non-zero on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float asf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t asu(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float div127(float a) {
    const float C = 1.0f / 127.0f;
    const float q = a * C;
    return fmaf(fmaf(-q, 127.0f, a), C, q);
}
static int round_away(float y) {
    const float a = fabsf(y);
    const float t = a == 0x1.fffffep-2f ? 0.0f : a + 0.5f;
    return (int)copysignf(t, y);
}

int main(void) {
    unsigned long long bad_div = 0, bad_round = 0;
    /* every finite a >= +0, the amax it divides (the steps are odd in a, but
     * -0 gives +0: the fma sums of zeros round to +0) */
#pragma omp parallel for reduction(+ : bad_div) schedule(static)
    for (int64_t u = 0; u < 0x7f800000LL; ++u) {
        const float a = asf((uint32_t)u);
        const volatile float ref = a / 127.0f;
        if (asu(div127(a)) != asu(ref)) ++bad_div;
    }
    /* every y with |y| < 2^23, both signs */
#pragma omp parallel for reduction(+ : bad_round) schedule(static)
    for (int64_t u = 0; u < 2 * 0x4b000000LL; ++u) {
        const float y = asf((uint32_t)(u >> 1) | ((uint32_t)(u & 1) << 31));
        if (round_away(y) != (int)roundf(y)) ++bad_round;
    }
    printf("div127 mismatches %llu, round_away mismatches %llu\n", bad_div, bad_round);
    return bad_div || bad_round;
}
