/*
 * q38m self-check entry points -- not part of the MoE operator surface.
 *
 * libq38m_selftest.so, a library of their own next to libq38m.so (which
 * exports none of them), holds these for the test suite: each runs one
 * instruction-level building block of the kernels on the device so the
 * tests can pin it in isolation (the contract's exp against libm, the
 * int8 MFMA lane layouts against an integer matrix product).  A caller of
 * the MoE data plane never needs them; they allocate nothing and follow the
 * conventions of q38m.h (device pointers, opaque stream, status codes,
 * without a message: q38m_last_error belongs to libq38m.so).
 */
#ifndef Q38M_SELFTEST_H
#define Q38M_SELFTEST_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* out[i] = the contract's exp(x[i]) (Cody-Waite reduction + degree-7
 * polynomial), the function every sigmoid / SiLU of the path uses. */
int q38m_debug_expf(const float* x, uint32_t n, float* out, void* stream,
                    int device);
/* All 2^32 fp32 bit patterns through the hardware bf16 conversion and the
 * contract's integer round-to-nearest-even; result[4] (device memory, set by
 * the caller to {0, ~0, 0, ~0}) receives {mismatches, first mismatching
 * pattern, mismatches on non-NaN inputs, first such pattern}. */
int q38m_debug_bf16_sweep(uint32_t* result, void* stream, int device);
/* One int8 MFMA product d = a * b^T with a, b row-major (16x32 and 16x32,
 * or 32x32 and 32x32), through the lane layouts the grouped kernels use. */
int q38m_debug_mfma_16x16x32_i8(const int8_t* a, const int8_t* b, int32_t* d,
                                void* stream, int device);
int q38m_debug_mfma_32x32x32_i8(const int8_t* a, const int8_t* b, int32_t* d,
                                void* stream, int device);

#ifdef __cplusplus
}
#endif

#endif
