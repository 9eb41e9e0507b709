/* Build-time generator of the SwiGLU gate table used by the chunk-path
 * gate/up kernels (csrc/q38m_wide.hip).
 *
 * The gate value enters SwiGLU already rounded to bf16
 * (cuda/q38_moe_prefill.cu:449-461: g = bf16(y_gate), silu = g/(1+exp(-g))),
 * so silu(g) is a function of the 16-bit pattern of g alone: 65,536 fp32
 * results.  This program evaluates them with the arithmetic contract's
 * exp (Cody-Waite reduction, degree-7 Taylor polynomial in Horner form
 * with explicit fma, exact 2^n scaling, flush below -87.3; the same
 * operation sequence as exp_q in csrc/q38m_device.h) and one IEEE fp32
 * division, and prints the result words as a C initializer list, entry h
 * holding silu(bits h << 16).  x86-64 evaluates float arithmetic in
 * binary32 (SSE), fmaf and rintf are correctly rounded, and the build
 * passes -ffp-contract=off, so every entry equals what the device computes
 * for the same g (the tests compare all 65,536 entries with the oracle,
 * NaN results as NaN).
 *
 * Usage: q38m_silu_gen > q38m_silu_table.inc
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

static uint32_t to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return u;
}

/* The contract's exp, operation for operation as the device evaluates it:
 * the body runs on x clamped into its domain and the special cases are
 * selected afterwards. */
static float exp_contract(float x) {
    const float xb = fminf(fmaxf(x, -87.3f), 88.72283935546875f);
    const float n = rintf(xb * 1.44269502162933349609375f);
    float r = fmaf(n, -0.693145751953125f, xb);
    r = fmaf(n, -1.42860682030941723212e-6f, r);
    float p = 1.98412698412698412698e-4f;
    p = fmaf(p, r, 1.38888888888888888889e-3f);
    p = fmaf(p, r, 8.33333333333333333333e-3f);
    p = fmaf(p, r, 4.16666666666666666667e-2f);
    p = fmaf(p, r, 1.66666666666666666667e-1f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int e = (int)n; /* -126 .. 128 */
    const float scaled = e > 127 ? (p * 2.0f) * from_bits(254u << 23)
                                 : p * from_bits((uint32_t)(e + 127) << 23);
    const float ranged = x > 88.72283935546875f ? INFINITY : (x < -87.3f ? 0.0f : scaled);
    return x != x ? x + x : ranged;
}

int main(void) {
    printf("/* silu(g) = g / (1 + exp(-g)) for every bf16 g (entry h: g = bits h << 16),\n"
           " * fp32 result words; written by q38m_silu_gen. */\n");
    for (uint32_t h = 0; h < 65536u; ++h) {
        const float g = from_bits(h << 16);
        const float den = 1.0f + exp_contract(-g);
        const float silu = g / den;
        printf("0x%08xu,%c", to_bits(silu), (h % 8u) == 7u ? '\n' : ' ');
    }
    return ferror(stdout) ? 1 : 0;
}
