/* Exhaustive CPU check of the row quantisers' quotient (csrc/q38m_select.h
 * quant_scale / quantize8_with<true>).
 *
 * For every positive finite bf16 absmax a, s = RN(a/127) and r = RN(1/s);
 * where 2^-120 <= s <= FLT_MAX (the device's fast condition), and for every
 * bf16 x with 0 <= x <= a, the device forms q0 = RN(x r) and
 * q = RN(q0 + RN(x - q0 s) r) with two fmas.  The contract needs
 * rint(RN(x/s)); this program counts the pairs where rint(q) differs from
 * it (x < 0 mirrors x > 0: RN, fma and rint are sign-symmetric).  As a
 * control it also counts the pairs where rint(RN(x r)) alone differs, which
 * must be non-zero for the check to mean anything.
 *
 * Prints: "pairs <n> mismatches <m> uncorrected_mismatches <u>".
 * Build: cc -O2 -fopenmp -ffp-contract=off -o check quantize_division_check.c -lm
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float from_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

int main(void) {
    long long pairs = 0, mismatches = 0, uncorrected = 0;
    const float lo = ldexpf(1.0f, -120);
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : pairs, mismatches, uncorrected)
    for (int ah = 1; ah < 0x7f80; ++ah) {
        const float a = from_bits((uint32_t)ah << 16);
        const float s = a / 127.0f;
        if (!(s >= lo && s <= 0x1.fffffep+127f)) continue;
        const float r = 1.0f / s;
        for (int xh = 0; xh <= ah; ++xh) {
            const float x = from_bits((uint32_t)xh << 16);
            const float reference = rintf(x / s);
            const float q0 = x * r;
            const float q = fmaf(fmaf(-q0, s, x), r, q0);
            ++pairs;
            if (rintf(q) != reference) ++mismatches;
            if (rintf(q0) != reference) ++uncorrected;
        }
    }
    printf("pairs %lld mismatches %lld uncorrected_mismatches %lld\n", pairs, mismatches,
           uncorrected);
    return 0;
}
