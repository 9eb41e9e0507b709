// Self-check kernels of the test suite (include/q38m_selftest.h), built
// into libq38m_selftest.so, a library of their own that the tests load
// beside libq38m.so: the product library exports none of them.  Each runs
// one instruction-level building block of the product kernels so the tests
// can pin it in isolation -- the contract's exp against libm, the hardware
// bf16 conversion against the contract's integer rounding, the int8 MFMA
// lane layouts against an integer matrix product.  The building blocks
// themselves come from q38m_device.h, the header the product kernels use.
#include "q38m_device.h"
#include "q38m_selftest.h"

namespace q38m {
namespace {

__global__ void debug_expf_kernel(const float* __restrict__ x, uint32_t n, float* __restrict__ out) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = exp_q(x[i]);
}

// Every fp32 bit pattern through the hardware bf16 conversion
// (v_cvt_pk_bf16_f32, what a cast to __bf16 compiles to on gfx950) and the
// integer round-to-nearest-even of f32_to_bf16_int; result = {mismatches, first
// mismatching pattern, mismatches on non-NaN inputs, first such pattern}.
__global__ __launch_bounds__(256) void debug_bf16_kernel(uint32_t* __restrict__ result) {
    uint32_t bad = 0u, first = 0xffffffffu, bad_num = 0u, first_num = 0xffffffffu;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * 256u;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x; i < (1ull << 32);
         i += stride) {
        const uint32_t bits = static_cast<uint32_t>(i);
        const float v = __uint_as_float(bits);
        const uint32_t hw = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
        if (hw != f32_to_bf16_int(v)) {
            ++bad;
            first = min(first, bits);
            if (v == v) {
                ++bad_num;
                first_num = min(first_num, bits);
            }
        }
    }
    if (bad != 0u) {
        atomicAdd(&result[0], bad);
        atomicMin(&result[1], first);
    }
    if (bad_num != 0u) {
        atomicAdd(&result[2], bad_num);
        atomicMin(&result[3], first_num);
    }
}

// One v_mfma_i32_16x16x32_i8 with A (16x32) and B (32x16) given row-major
// in memory, loaded in the operand layout the kernels assume; D (16x16) is
// written row-major from the assumed result layout.
__global__ void debug_mfma_kernel(const int8_t* __restrict__ a, const int8_t* __restrict__ b,
                                  int32_t* __restrict__ d) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t n = lane & 15u, q = lane >> 4;
    uint64_t av = 0, bv = 0;
    for (uint32_t i = 0; i < 8u; ++i) {
        av |= static_cast<uint64_t>(static_cast<uint8_t>(a[n * 32u + 8u * q + i])) << (8u * i);
        bv |= static_cast<uint64_t>(static_cast<uint8_t>(b[(8u * q + i) * 16u + n])) << (8u * i);
    }
    const v4i zero = {0, 0, 0, 0};
    const v4i r = mfma_i8_16x16x32(static_cast<long>(av), static_cast<long>(bv), zero);
    for (uint32_t i = 0; i < 4u; ++i) d[(4u * q + i) * 16u + n] = r[i];
}

// The same for v_mfma_i32_32x32x32_i8 (A 32x32, B 32x32, D 32x32).
__global__ void debug_mfma32_kernel(const int8_t* __restrict__ a, const int8_t* __restrict__ b,
                                    int32_t* __restrict__ d) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t c = lane & 31u, h = lane >> 5;
    uint32_t av[4] = {0u, 0u, 0u, 0u}, bv[4] = {0u, 0u, 0u, 0u};
    for (uint32_t i = 0; i < 16u; ++i) {
        av[i / 4u] |= static_cast<uint32_t>(static_cast<uint8_t>(a[c * 32u + 16u * h + i])) << (8u * (i % 4u));
        bv[i / 4u] |= static_cast<uint32_t>(static_cast<uint8_t>(b[(16u * h + i) * 32u + c])) << (8u * (i % 4u));
    }
    const v4i at = {static_cast<int>(av[0]), static_cast<int>(av[1]), static_cast<int>(av[2]),
                    static_cast<int>(av[3])};
    const v4i bt = {static_cast<int>(bv[0]), static_cast<int>(bv[1]), static_cast<int>(bv[2]),
                    static_cast<int>(bv[3])};
    v16i zero;
    for (int i = 0; i < 16; ++i) zero[i] = 0;
    const v16i r = mfma_i8_32x32x32(at, bt, zero);
    for (uint32_t i = 0; i < 16u; ++i) d[(8u * (i / 4u) + 4u * h + i % 4u) * 32u + c] = r[i];
}

}  // namespace
}  // namespace q38m

extern "C" {

int q38m_debug_expf(const float* x, uint32_t n, float* out, void* stream, int device) {
    if (!x || !out || n == 0) return Q38M_ERR_INVALID_ARGUMENT;
    if (device < 0 || hipSetDevice(device) != hipSuccess) return Q38M_ERR_DEVICE;
    q38m::debug_expf_kernel<<<(n + 255u) / 256u, 256, 0, static_cast<hipStream_t>(stream)>>>(
        x, n, out);
    return hipGetLastError() == hipSuccess ? Q38M_OK : Q38M_ERR_DEVICE;
}

int q38m_debug_bf16_sweep(uint32_t* result, void* stream, int device) {
    if (!result) return Q38M_ERR_INVALID_ARGUMENT;
    if (device < 0 || hipSetDevice(device) != hipSuccess) return Q38M_ERR_DEVICE;
    q38m::debug_bf16_kernel<<<4096, 256, 0, static_cast<hipStream_t>(stream)>>>(result);
    return hipGetLastError() == hipSuccess ? Q38M_OK : Q38M_ERR_DEVICE;
}

int q38m_debug_mfma_16x16x32_i8(const int8_t* a, const int8_t* b, int32_t* d, void* stream,
                                int device) {
    if (!a || !b || !d) return Q38M_ERR_INVALID_ARGUMENT;
    if (device < 0 || hipSetDevice(device) != hipSuccess) return Q38M_ERR_DEVICE;
    q38m::debug_mfma_kernel<<<1, 64, 0, static_cast<hipStream_t>(stream)>>>(a, b, d);
    return hipGetLastError() == hipSuccess ? Q38M_OK : Q38M_ERR_DEVICE;
}

int q38m_debug_mfma_32x32x32_i8(const int8_t* a, const int8_t* b, int32_t* d, void* stream,
                                int device) {
    if (!a || !b || !d) return Q38M_ERR_INVALID_ARGUMENT;
    if (device < 0 || hipSetDevice(device) != hipSuccess) return Q38M_ERR_DEVICE;
    q38m::debug_mfma32_kernel<<<1, 64, 0, static_cast<hipStream_t>(stream)>>>(a, b, d);
    return hipGetLastError() == hipSuccess ? Q38M_OK : Q38M_ERR_DEVICE;
}

}  // extern "C"
