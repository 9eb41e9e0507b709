// Device weight layout conversion (the load-time re-tiling of
// cuda/cuda_weights.cu:229-285, for this build's MFMA16 layout),
// deterministic synthetic data, and kernel-level self checks.
#include "q38m_device.h"
#include "q38m_internal.h"

namespace q38m {
namespace {

// Slot -> row tile of the quad-major W4 layouts: identity, or, paired, tile
// s/2 of the first half and tile s/2 of the second half alternating.
__device__ __forceinline__ uint32_t slot_tile(uint32_t slot, uint32_t row_tiles, bool paired) {
    return paired ? (slot >> 1) + (slot & 1u) * (row_tiles >> 1) : slot;
}

// W4 row-major [E][R][K/2] -> MFMA16 [E][K/128][slot][64][4 dwords].
// Output dword (e, kq, slot, lane=(q,n), j) covers row 16*tile(slot)+n,
// group g=4kq+j, k0 = 32g+8q: byte i = nib(k0+i) | nib(k0+4+i) << 4.  The
// source dword at k0/2 holds nibbles k0..k0+7 in order.
__global__ void repack_w4_kernel(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst,
                                 uint32_t rows, uint32_t cols, bool paired, uint64_t total) {
    const uint64_t o = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (o >= total) return;
    const uint32_t quads = cols / 128u;
    const uint32_t row_tiles = rows / 16u;
    const uint32_t j = static_cast<uint32_t>(o & 3u);
    const uint32_t lane = static_cast<uint32_t>((o >> 2) & 63u);
    const uint64_t unit = o >> 8;
    const uint32_t slot = static_cast<uint32_t>(unit % row_tiles);
    const uint64_t tmp = unit / row_tiles;
    const uint32_t kq = static_cast<uint32_t>(tmp % quads);
    const uint64_t e = tmp / quads;
    const uint32_t n = lane & 15u, q = lane >> 4;
    const uint32_t row = slot_tile(slot, row_tiles, paired) * 16u + n;
    const uint32_t g = kq * 4u + j;
    const uint32_t c = src[(e * rows + row) * (cols / 8u) + g * 4u + q];
    uint32_t out = 0;
#pragma unroll
    for (uint32_t i = 0; i < 4u; ++i) {
        out |= ((c >> (4u * i)) & 0xfu) << (8u * i);
        out |= ((c >> (16u + 4u * i)) & 0xfu) << (8u * i + 4u);
    }
    dst[o] = out;
}

// W4 scales [E][R][K/g] -> [E][K/128][slot][16][128/g] (g = 32, 64, 128:
// per_quad = 4, 2, 1 words per row and quad).
__global__ void repack_w4_scales_kernel(const uint16_t* __restrict__ src,
                                        uint16_t* __restrict__ dst, uint32_t rows,
                                        uint32_t cols, uint32_t per_quad, bool paired,
                                        uint64_t total) {
    const uint64_t o = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (o >= total) return;
    const uint32_t quads = cols / 128u;
    const uint32_t row_tiles = rows / 16u;
    const uint32_t j = static_cast<uint32_t>(o % per_quad);
    const uint32_t n = static_cast<uint32_t>((o / per_quad) & 15u);
    const uint64_t unit = o / (16u * per_quad);
    const uint32_t slot = static_cast<uint32_t>(unit % row_tiles);
    const uint64_t tmp = unit / row_tiles;
    const uint32_t kq = static_cast<uint32_t>(tmp % quads);
    const uint64_t e = tmp / quads;
    const uint32_t row = slot_tile(slot, row_tiles, paired) * 16u + n;
    dst[o] = src[(e * rows + row) * (quads * per_quad) + kq * per_quad + j];
}

// W8 row-major [E][R][K] -> MFMA16 [E][R/16][K/64][64][16 B]; lane (q,n)
// holds row 16rt+n, columns 64kb+16q .. +15.
__global__ void repack_w8_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                 uint32_t rows, uint32_t cols, uint64_t total) {
    const uint64_t o = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (o >= total) return;
    const uint32_t blocks = cols / 64u;
    const uint32_t row_tiles = rows / 16u;
    const uint32_t lane = static_cast<uint32_t>(o & 63u);
    const uint64_t block = o >> 6;
    const uint32_t kb = static_cast<uint32_t>(block % blocks);
    const uint64_t tmp = block / blocks;
    const uint32_t rt = static_cast<uint32_t>(tmp % row_tiles);
    const uint64_t e = tmp / row_tiles;
    const uint32_t n = lane & 15u, q = lane >> 4;
    dst[o] = src[((e * rows + rt * 16u + n) * cols + kb * 64u + q * 16u) / 16u];
}

// W8 gate/up row-major [E][R][K] -> paired K-block-major MFMA16
// [E][K/64][slot][64][16 B]: for block kb every slot (1 KiB) is adjacent,
// slot s holding row tile s/2 + (s%2)*R/32 (the gate tile of channel block
// p next to its up tile), lane (q,n) row 16t+n, columns 64kb+16q .. +15.
__global__ void repack_w8_paired_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                        uint32_t rows, uint32_t cols, uint64_t total) {
    const uint64_t o = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (o >= total) return;
    const uint32_t blocks = cols / 64u;
    const uint32_t row_tiles = rows / 16u;
    const uint32_t lane = static_cast<uint32_t>(o & 63u);
    const uint64_t unit = o >> 6;
    const uint32_t slot = static_cast<uint32_t>(unit % row_tiles);
    const uint64_t tmp = unit / row_tiles;
    const uint32_t kb = static_cast<uint32_t>(tmp % blocks);
    const uint64_t e = tmp / blocks;
    const uint32_t n = lane & 15u, q = lane >> 4;
    const uint32_t row = slot_tile(slot, row_tiles, true) * 16u + n;
    dst[o] = src[((e * rows + row) * cols + kb * 64u + q * 16u) / 16u];
}

// ---------------------------------------------------------------------------
// Weight quantiser (tools/q38_artifact_compiler.py:193-253, quantize_groupwise):
// per group s = max|w| / qmax (qmax 7 for W4, 127 for W8), s == 0 -> 1,
// q = clamp(rint(w / s), +-qmax); W4 packs column 2i in the low nibble.
// Scales are stored as fp16 (round to nearest even, subnormals kept) or,
// as the reference does (f32_to_bf16_rne, :232), as RNE bf16; q always
// comes from the fp32 s.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t f32_to_f16_bits(float v) {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(v)));
}

template <uint32_t kBits>
__device__ __forceinline__ uint32_t quant_weight(uint32_t bf16, float s) {
    constexpr float kMax = kBits == 4u ? 7.0f : 127.0f;
    float v = __builtin_rintf(bf16_to_f32(bf16) / s);
    v = fminf(fmaxf(v, -kMax), kMax);
    return static_cast<uint32_t>(static_cast<int32_t>(v)) & (kBits == 4u ? 0xfu : 0xffu);
}

// One thread per group of kGroup columns (groups are contiguous in memory).
template <uint32_t kBits, uint32_t kGroup>
__global__ __launch_bounds__(256) void quantize_weights_group_kernel(
    const uint4* __restrict__ src, uint64_t groups, uint8_t* __restrict__ data,
    uint16_t* __restrict__ scales, bool scale_bf16) {
    constexpr uint32_t kVec = kGroup / 8u;  // uint4 of 8 bf16
    constexpr float kMax = kBits == 4u ? 7.0f : 127.0f;
    const uint64_t g = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g >= groups) return;
    uint32_t w[kGroup / 2u];
#pragma unroll
    for (uint32_t i = 0; i < kVec; ++i) {
        const uint4 v = src[g * kVec + i];
        w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < kGroup / 2u; ++i) {
        amax = fmaxf(amax, fabsf(bf16_to_f32(w[i] & 0xffffu)));
        amax = fmaxf(amax, fabsf(bf16_to_f32(w[i] >> 16)));
    }
    float s = amax / kMax;
    if (s == 0.0f) s = 1.0f;
    scales[g] = static_cast<uint16_t>(scale_bf16 ? f32_to_bf16(s) : f32_to_f16_bits(s));
    if constexpr (kBits == 4u) {
        // two bf16 per word -> one byte (low nibble = even column)
        uint32_t packed[kGroup / 8u];
#pragma unroll
        for (uint32_t i = 0; i < kGroup / 8u; ++i) {
            uint32_t b = 0;
#pragma unroll
            for (uint32_t j = 0; j < 4u; ++j) {
                const uint32_t word = w[4 * i + j];
                const uint32_t byte = quant_weight<4>(word & 0xffffu, s) |
                                      (quant_weight<4>(word >> 16, s) << 4);
                b |= byte << (8 * j);
            }
            packed[i] = b;
        }
        uint4* out = reinterpret_cast<uint4*>(data + g * (kGroup / 2u));
#pragma unroll
        for (uint32_t i = 0; i < kGroup / 32u; ++i)
            out[i] = make_uint4(packed[4 * i], packed[4 * i + 1], packed[4 * i + 2], packed[4 * i + 3]);
    } else {
        uint32_t packed[kGroup / 4u];
#pragma unroll
        for (uint32_t i = 0; i < kGroup / 4u; ++i) {
            const uint32_t lo = w[2 * i], hi = w[2 * i + 1];
            packed[i] = quant_weight<8>(lo & 0xffffu, s) | (quant_weight<8>(lo >> 16, s) << 8) |
                        (quant_weight<8>(hi & 0xffffu, s) << 16) | (quant_weight<8>(hi >> 16, s) << 24);
        }
        uint4* out = reinterpret_cast<uint4*>(data + g * kGroup);
#pragma unroll
        for (uint32_t i = 0; i < kGroup / 16u; ++i)
            out[i] = make_uint4(packed[4 * i], packed[4 * i + 1], packed[4 * i + 2], packed[4 * i + 3]);
    }
}

// W8 per output channel: one wave per row (columns % 512 == 0), two passes.
__global__ __launch_bounds__(256) void quantize_weights_row_w8_kernel(
    const uint16_t* __restrict__ src, uint64_t rows, uint32_t cols, uint8_t* __restrict__ data,
    uint16_t* __restrict__ scales, bool scale_bf16) {
    const uint64_t row = static_cast<uint64_t>(blockIdx.x) * 4u + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint32_t lane = threadIdx.x & 63u;
    const uint4* r = reinterpret_cast<const uint4*>(src + row * cols);
    float amax = 0.0f;
    for (uint32_t c = lane; c < cols / 8u; c += 64u) {
        const uint4 v = r[c];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            amax = fmaxf(amax, fabsf(bf16_to_f32(w[i] & 0xffffu)));
            amax = fmaxf(amax, fabsf(bf16_to_f32(w[i] >> 16)));
        }
    }
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) amax = fmaxf(amax, __shfl_xor(amax, offset, 64));
    float s = amax / 127.0f;
    if (s == 0.0f) s = 1.0f;
    if (lane == 0)
        scales[row] = static_cast<uint16_t>(scale_bf16 ? f32_to_bf16(s) : f32_to_f16_bits(s));
    uint2* out = reinterpret_cast<uint2*>(data + row * cols);
    for (uint32_t c = lane; c < cols / 8u; c += 64u) {
        const uint4 v = r[c];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        uint32_t packed[2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
            packed[i] = quant_weight<8>(w[2 * i] & 0xffffu, s) |
                        (quant_weight<8>(w[2 * i] >> 16, s) << 8) |
                        (quant_weight<8>(w[2 * i + 1] & 0xffffu, s) << 16) |
                        (quant_weight<8>(w[2 * i + 1] >> 16, s) << 24);
        out[c] = make_uint2(packed[0], packed[1]);
    }
}

__global__ void copy_u16_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                uint64_t total) {
    const uint64_t o = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (o < total) dst[o] = src[o];
}

// Synthetic data, one element (or one packed W4 byte) per thread, grid-
// stride so any count fits the grid.
__global__ void synth_kernel(uint32_t kind, uint64_t base, uint64_t count, float sigma,
                             int32_t lo, int32_t hi, const float* __restrict__ bias,
                             uint32_t bias_len, void* __restrict__ out) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        switch (kind) {
            case Q38M_SYNTH_NORMAL_F32: {
                float v = normal_at(base, i) * sigma;
                if (bias) v = v + bias[i % bias_len];
                static_cast<float*>(out)[i] = v;
                break;
            }
            case Q38M_SYNTH_NORMAL_BF16:
                static_cast<uint16_t*>(out)[i] =
                    static_cast<uint16_t>(f32_to_bf16(normal_at(base, i) * sigma));
                break;
            case Q38M_SYNTH_ABS_NORMAL_F16:
                static_cast<uint16_t*>(out)[i] =
                    static_cast<uint16_t>(f32_to_f16(fabsf(normal_at(base, i) * sigma)));
                break;
            case Q38M_SYNTH_UNIFORM_W4: {
                const int low = uniform_at(base, 2u * i, lo, hi);
                const int high = uniform_at(base, 2u * i + 1u, lo, hi);
                static_cast<uint8_t*>(out)[i] = static_cast<uint8_t>(
                    (static_cast<uint32_t>(low) & 0xfu) | ((static_cast<uint32_t>(high) & 0xfu) << 4));
                break;
            }
            case Q38M_SYNTH_UNIFORM_I8:
                static_cast<int8_t*>(out)[i] = static_cast<int8_t>(uniform_at(base, i, lo, hi));
                break;
            default:
                break;
        }
    }
}

inline uint32_t blocks_for(uint64_t total, uint32_t threads) {
    return static_cast<uint32_t>((total + threads - 1u) / threads);
}

}  // namespace

hipError_t launch_repack(const q38m_expert_weights_v1& src,
                         const q38m_expert_weights_v1& dst, hipStream_t stream) {
    const uint64_t elements = static_cast<uint64_t>(src.experts) * src.rows * src.columns;
    if (src.format == Q38M_FORMAT_W4_SYM) {
        const bool paired = dst.layout == Q38M_LAYOUT_MFMA16_PAIRED;
        const uint64_t dwords = elements / 8u;
        repack_w4_kernel<<<blocks_for(dwords, 256), 256, 0, stream>>>(
            static_cast<const uint32_t*>(src.data), static_cast<uint32_t*>(const_cast<void*>(dst.data)),
            src.rows, src.columns, paired, dwords);
        const uint64_t scales = elements / src.group_size;
        repack_w4_scales_kernel<<<blocks_for(scales, 256), 256, 0, stream>>>(
            static_cast<const uint16_t*>(src.scales),
            static_cast<uint16_t*>(const_cast<void*>(dst.scales)), src.rows, src.columns,
            128u / src.group_size, paired, scales);
    } else {
        const uint64_t vectors = elements / 16u;
        if (dst.layout == Q38M_LAYOUT_MFMA16_PAIRED)
            repack_w8_paired_kernel<<<blocks_for(vectors, 256), 256, 0, stream>>>(
                static_cast<const uint4*>(src.data),
                static_cast<uint4*>(const_cast<void*>(dst.data)), src.rows, src.columns, vectors);
        else
            repack_w8_kernel<<<blocks_for(vectors, 256), 256, 0, stream>>>(
                static_cast<const uint4*>(src.data),
                static_cast<uint4*>(const_cast<void*>(dst.data)), src.rows, src.columns, vectors);
        // W8 scales keep the artifact order (per channel or [E][R][K/g])
        const uint64_t scales = src.group_size ? elements / src.group_size
                                               : static_cast<uint64_t>(src.experts) * src.rows;
        copy_u16_kernel<<<blocks_for(scales, 256), 256, 0, stream>>>(
            static_cast<const uint16_t*>(src.scales),
            static_cast<uint16_t*>(const_cast<void*>(dst.scales)), scales);
    }
    return hipGetLastError();
}

hipError_t launch_quantize_weights(const uint16_t* src, const q38m_expert_weights_v1& dst,
                                  hipStream_t stream) {
    const uint64_t rows = static_cast<uint64_t>(dst.experts) * dst.rows;
    uint8_t* data = static_cast<uint8_t*>(const_cast<void*>(dst.data));
    uint16_t* scales = static_cast<uint16_t*>(const_cast<void*>(dst.scales));
    const uint4* s4 = reinterpret_cast<const uint4*>(src);
    const uint32_t g = dst.group_size;
    const bool w4 = dst.format == Q38M_FORMAT_W4_SYM;
    const bool bf16 = dst.scale_dtype == Q38M_SCALE_BF16;
    if (g == 0u) {
        quantize_weights_row_w8_kernel<<<blocks_for(rows, 4), 256, 0, stream>>>(
            src, rows, dst.columns, data, scales, bf16);
        return hipGetLastError();
    }
    const uint64_t groups = rows * (dst.columns / g);
    const uint32_t grid = blocks_for(groups, 256);
#define Q38M_QUANT(BITS, G)                                                                  \
    quantize_weights_group_kernel<BITS, G><<<grid, 256, 0, stream>>>(s4, groups, data, scales, \
                                                                     bf16)
    if (w4 && g == 32u) Q38M_QUANT(4u, 32u);
    else if (w4 && g == 64u) Q38M_QUANT(4u, 64u);
    else if (w4) Q38M_QUANT(4u, 128u);
    else if (g == 32u) Q38M_QUANT(8u, 32u);
    else if (g == 64u) Q38M_QUANT(8u, 64u);
    else Q38M_QUANT(8u, 128u);
#undef Q38M_QUANT
    return hipGetLastError();
}

hipError_t launch_synth(uint32_t kind, uint64_t seed, uint64_t tag, uint64_t count,
                        float sigma, int32_t lo, int32_t hi, const float* bias,
                        uint32_t bias_len, void* out, hipStream_t stream) {
    const uint64_t items = kind == Q38M_SYNTH_UNIFORM_W4 ? count / 2u : count;
    const uint32_t blocks = static_cast<uint32_t>(
        items / 256u + 1u < 65536u ? items / 256u + 1u : 65536u);
    synth_kernel<<<blocks, 256, 0, stream>>>(kind, stream_base_host(seed, tag), items, sigma, lo,
                                             hi, bias, bias_len, out);
    return hipGetLastError();
}

}  // namespace q38m
