// Per-row int8 activation quantisation and the bf16 hidden gather.
#include "q38m_device.h"
#include "q38m_internal.h"
#include "q38m_select.h"

namespace q38m {
namespace {

// One wave per row; lane l owns elements [8l + 512c, 8l + 512c + 8) so
// every load is a coalesced 16-byte vector.  s = absmax/127 (IEEE
// division), zero -> 1, q = clamp(rint(x/s), -127, 127): the convention of
// tools/q38_artifact_compiler.py:214-222 applied per token row (quotients
// through quant_scale / quantize8).
template <uint32_t kChunks>
__global__ __launch_bounds__(256) void quantize_rows_kernel(
    const uint16_t* __restrict__ x, uint32_t rows, int8_t* __restrict__ q,
    float* __restrict__ scales) {
    constexpr uint32_t kWidth = kChunks * 512u;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint4* src = reinterpret_cast<const uint4*>(x + static_cast<size_t>(row) * kWidth);
    uint4 v[kChunks];
#pragma unroll
    for (uint32_t c = 0; c < kChunks; ++c) v[c] = src[c * 64u + lane];
    float amax = 0.0f;
#pragma unroll
    for (uint32_t c = 0; c < kChunks; ++c) {
        const uint32_t w[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            amax = fmaxf(amax, fabsf(bf16_to_f32(w[i] & 0xffffu)));
            amax = fmaxf(amax, fabsf(bf16_to_f32(w[i] >> 16)));
        }
    }
    const QuantScale qs = quant_scale(wave_max_f32(amax));
    uint2* dst = reinterpret_cast<uint2*>(q + static_cast<size_t>(row) * kWidth);
#pragma unroll
    for (uint32_t c = 0; c < kChunks; ++c) {
        const uint32_t w[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
        dst[c * 64u + lane] = quantize8(w, qs);
    }
    if (lane == 0) scales[row] = qs.s;
}

// 512-wide rows (the mid rows), kRows rows per wave with all their loads
// issued together and non-temporal (each row is read once; 327,680 rows:
// 101 -> 94 us against one row per wave); the same per-row arithmetic as
// quantize_rows_kernel.
template <uint32_t kRows>
__global__ __launch_bounds__(256) void quantize_rows512_kernel(
    const uint16_t* __restrict__ x, uint32_t rows, int8_t* __restrict__ q,
    float* __restrict__ scales) {
    typedef unsigned int u4v __attribute__((ext_vector_type(4)));
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row0 = (blockIdx.x * 4u + (threadIdx.x >> 6)) * kRows;
    u4v v[kRows];
#pragma unroll
    for (uint32_t j = 0; j < kRows; ++j) {
        const uint32_t row = row0 + j < rows ? row0 + j : rows - 1u;
        v[j] = __builtin_nontemporal_load(
            reinterpret_cast<const u4v*>(x + static_cast<size_t>(row) * 512u) + lane);
    }
#pragma unroll
    for (uint32_t j = 0; j < kRows; ++j) {
        const uint32_t row = row0 + j;
        if (row >= rows) break;
        const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            amax = fmaxf(amax, fabsf(bf16_to_f32(w[i] & 0xffffu)));
            amax = fmaxf(amax, fabsf(bf16_to_f32(w[i] >> 16)));
        }
        const QuantScale qs = quant_scale(wave_max_f32(amax));
        reinterpret_cast<uint2*>(q + static_cast<size_t>(row) * 512u)[lane] = quantize8(w, qs);
        if (lane == 0) scales[row] = qs.s;
    }
}

// Gather hidden[token(packed)] -> packed order (q38_moe_prefill.cu:292-306).
__global__ __launch_bounds__(256) void pack_hidden_kernel(
    const uint16_t* __restrict__ hidden, const uint32_t* __restrict__ packed,
    uint32_t width, uint16_t* __restrict__ out) {
    const uint32_t p = blockIdx.x;
    const uint32_t token = checked(packed[p], Q38M_WIDE_MAX_TOKENS * kTopK, kCheckToken) / kTopK;
    const uint4* src = reinterpret_cast<const uint4*>(hidden + static_cast<size_t>(token) * width);
    uint4* dst = reinterpret_cast<uint4*>(out + static_cast<size_t>(p) * width);
    for (uint32_t i = threadIdx.x; i < width / 8u; i += blockDim.x) dst[i] = src[i];
}

// out = bf16(a + b) in fp32, 8 elements per thread; both inputs are read
// once, with non-temporal loads (32,768 x 2048: 71 -> 62 us).
__global__ __launch_bounds__(256) void residual_add_kernel(
    const uint4* __restrict__ a, const uint4* __restrict__ b, uint4* __restrict__ out,
    uint64_t vectors) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= vectors) return;
    typedef unsigned int u4v __attribute__((ext_vector_type(4)));
    const u4v na = __builtin_nontemporal_load(reinterpret_cast<const u4v*>(a) + i);
    const u4v nb = __builtin_nontemporal_load(reinterpret_cast<const u4v*>(b) + i);
    const uint4 va = make_uint4(na.x, na.y, na.z, na.w), vb = make_uint4(nb.x, nb.y, nb.z, nb.w);
    const uint32_t wa[4] = {va.x, va.y, va.z, va.w};
    const uint32_t wb[4] = {vb.x, vb.y, vb.z, vb.w};
    uint32_t r[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float lo = bf16_to_f32(wa[k] & 0xffffu) + bf16_to_f32(wb[k] & 0xffffu);
        const float hi = bf16_to_f32(wa[k] >> 16) + bf16_to_f32(wb[k] >> 16);
        r[k] = f32_to_bf16(lo) | (f32_to_bf16(hi) << 16);
    }
    out[i] = make_uint4(r[0], r[1], r[2], r[3]);
}

}  // namespace

hipError_t launch_residual_add(const uint16_t* a, const uint16_t* b, uint16_t* out,
                               uint64_t elements, hipStream_t stream) {
    const uint64_t vectors = elements / 8u;
    residual_add_kernel<<<static_cast<uint32_t>((vectors + 255u) / 256u), 256, 0, stream>>>(
        reinterpret_cast<const uint4*>(a), reinterpret_cast<const uint4*>(b),
        reinterpret_cast<uint4*>(out), vectors);
    return hipGetLastError();
}

hipError_t launch_quantize_rows(const uint16_t* x, uint32_t rows, uint32_t width,
                                int8_t* q, float* scales, hipStream_t stream) {
    const dim3 grid((rows + 3u) / 4u);
    switch (width / 512u) {
        case 1:
            quantize_rows512_kernel<4><<<(rows + 15u) / 16u, 256, 0, stream>>>(x, rows, q, scales);
            break;
        case 2: quantize_rows_kernel<2><<<grid, 256, 0, stream>>>(x, rows, q, scales); break;
        case 4: quantize_rows_kernel<4><<<grid, 256, 0, stream>>>(x, rows, q, scales); break;
        case 8: quantize_rows_kernel<8><<<grid, 256, 0, stream>>>(x, rows, q, scales); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_pack_hidden(const uint16_t* hidden, const uint32_t* packed,
                              uint32_t routes, uint32_t width, uint16_t* out,
                              hipStream_t stream) {
    pack_hidden_kernel<<<routes, 256, 0, stream>>>(hidden, packed, width, out);
    return hipGetLastError();
}

}  // namespace q38m
