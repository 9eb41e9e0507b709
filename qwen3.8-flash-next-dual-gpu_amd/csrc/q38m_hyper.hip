// Hyper-connection prepare/finish around the MoE step: the producer of the
// MoE input ("mixed") and the consumer of its output ("block_output")
// (cuda_backend.cu:1219-1252, 1967-1971; kernels q38_hyper.cu:52-114).
// The hidden state is kept as 4 streams of H values per token.
//
//   prepare: normalized = group RMSNorm of each stream (eps 1e-6, weight
//              1 + w), low = silu(bf16(normalized * mix_down^T) / 4),
//              mix = sigmoid(bf16(low * mix_up^T)),
//              mixed[i] = bf16((sum_s normalized[s][i] * mix[s][i]) / 4),
//              injection = 2 * sigmoid(bf16(normalized * inject^T) / 4)
//   finish:  output[s][i] = bf16(original[s][i] + block[i] * injection[s])
//
// bf16 values in, bf16 values between the steps as in the reference, fp32
// arithmetic inside a step, this library's exp.  MI355X layout: one
// workgroup per token does the RMSNorm of all four streams and the four
// inject dot products (the token's 4H values stay in registers); the two
// low-rank projections are bf16 MFMA GEMMs with the SiLU / sigmoid applied
// in their epilogue; the stream mix and the inject are one pass each over
// 16-byte vectors.  Floating-point results: parity is a tolerance (the
// reference's rsqrtf/expf and summation order are not bit-specified).
#include "q38m_device.h"
#include "q38m_internal.h"

namespace q38m {
namespace {

constexpr uint32_t kStreams = Q38M_HYPER_STREAMS;
constexpr uint32_t kNormThreads = 256;

__device__ __forceinline__ void unpack8(uint4 v, float (&x)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[2 * i] = bf16_to_f32(w[i] & 0xffffu);
        x[2 * i + 1] = bf16_to_f32(w[i] >> 16);
    }
}

__device__ __forceinline__ uint4 pack8(const float (&x)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = f32_to_bf16(x[2 * i]) | (f32_to_bf16(x[2 * i + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
    return v;
}

// hyper[t][s*H + i] = embedding[t][i] (q38_hyper.cu:52-61), 8 values a thread
__global__ __launch_bounds__(256) void hyper_repeat_kernel(const uint4* __restrict__ embedding,
                                                           uint4* __restrict__ hyper,
                                                           uint32_t hidden8, uint64_t total8) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    if (i >= total8) return;
    const uint64_t token = i / (kStreams * hidden8);
    const uint32_t within = static_cast<uint32_t>(i % (kStreams * hidden8)) % hidden8;
    hyper[i] = embedding[token * hidden8 + within];
}

// One workgroup per token: the group RMSNorm of the four streams
// (q38_hyper.cu:63-85) and, when inject is given, the four inject dot
// products over the normalized row (the GEMV of cuda_backend.cu:1238-1242)
// followed by 2 * sigmoid(bf16(dot) / 4).  The token's 4H values are held
// in registers, 8 per 16-byte chunk, kChunks chunks per thread.
template <uint32_t kChunks>
__global__ __launch_bounds__(kNormThreads) void hyper_norm_kernel(
    const uint16_t* __restrict__ hyper, const uint16_t* __restrict__ weight,
    const uint16_t* __restrict__ inject, uint32_t hidden, uint16_t* __restrict__ normalized,
    uint16_t* __restrict__ injection) {
    __shared__ float partial[kNormThreads / 64u][kStreams];
    const uint32_t token = blockIdx.x;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t hidden8 = hidden / 8u;
    const uint32_t chunks = kStreams * hidden8;
    const uint4* row = reinterpret_cast<const uint4*>(hyper) + static_cast<size_t>(token) * chunks;
    uint4 v[kChunks];
#pragma unroll
    for (uint32_t u = 0; u < kChunks; ++u) {
        const uint32_t c = threadIdx.x + u * kNormThreads;
        v[u] = c < chunks ? row[c] : make_uint4(0u, 0u, 0u, 0u);
    }
    float squares[kStreams] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t u = 0; u < kChunks; ++u) {
        const uint32_t c = threadIdx.x + u * kNormThreads;
        if (c >= chunks) continue;
        float x[8];
        unpack8(v[u], x);
        float sq = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) sq = __builtin_fmaf(x[i], x[i], sq);
        const uint32_t s = c / hidden8;
#pragma unroll
        for (uint32_t k = 0; k < kStreams; ++k) squares[k] += k == s ? sq : 0.0f;
    }
#pragma unroll
    for (uint32_t k = 0; k < kStreams; ++k) {
        const float total = wave_sum(squares[k]);
        if (lane == 0u) partial[wave][k] = total;
    }
    __syncthreads();
    float inverse[kStreams];
#pragma unroll
    for (uint32_t k = 0; k < kStreams; ++k) {
        float sum = 0.0f;
#pragma unroll
        for (uint32_t w = 0; w < kNormThreads / 64u; ++w) sum += partial[w][k];
        inverse[k] = 1.0f / __builtin_sqrtf(sum / static_cast<float>(hidden) + 1.0e-6f);
    }
    __syncthreads();  // partial[] is reused below
    const uint4* wrow = reinterpret_cast<const uint4*>(weight);
    uint4* out = reinterpret_cast<uint4*>(normalized) + static_cast<size_t>(token) * chunks;
    float dots[kStreams] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t u = 0; u < kChunks; ++u) {
        const uint32_t c = threadIdx.x + u * kNormThreads;
        if (c >= chunks) continue;
        const uint32_t s = c / hidden8;
        float x[8], w[8];
        unpack8(v[u], x);
        unpack8(wrow[c], w);
        float inv = inverse[0];
#pragma unroll
        for (uint32_t k = 1; k < kStreams; ++k) inv = k == s ? inverse[k] : inv;
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = bf16_round((x[i] * inv) * (1.0f + w[i]));
        out[c] = pack8(x);
        if (inject != nullptr) {
#pragma unroll
            for (uint32_t j = 0; j < kStreams; ++j) {
                float g[8];
                unpack8(reinterpret_cast<const uint4*>(inject)[static_cast<size_t>(j) * chunks + c], g);
#pragma unroll
                for (int i = 0; i < 8; ++i) dots[j] = __builtin_fmaf(x[i], g[i], dots[j]);
            }
        }
    }
    if (inject == nullptr) return;
#pragma unroll
    for (uint32_t j = 0; j < kStreams; ++j) {
        const float total = wave_sum(dots[j]);
        if (lane == 0u) partial[wave][j] = total;
    }
    __syncthreads();
    if (threadIdx.x < kStreams) {
        float sum = 0.0f;
#pragma unroll
        for (uint32_t w = 0; w < kNormThreads / 64u; ++w) sum += partial[w][threadIdx.x];
        const float x = bf16_round(sum) / static_cast<float>(kStreams);
        const float sigmoid = 1.0f / (1.0f + exp_q(-x));
        injection[static_cast<size_t>(token) * kStreams + threadIdx.x] =
            static_cast<uint16_t>(f32_to_bf16(sigmoid * 2.0f));
    }
}

// out = bf16(f(bf16 in / divisor) * scale), f = silu or sigmoid
// (q38_hyper.cu:87-97), 8 values a thread.
__global__ __launch_bounds__(256) void hyper_elementwise_kernel(const uint4* __restrict__ in,
                                                                uint4* __restrict__ out,
                                                                uint64_t total8, float divisor,
                                                                float scale, int silu) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    if (i >= total8) return;
    float x[8];
    unpack8(in[i], x);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float value = x[k] / divisor;
        const float sigmoid = 1.0f / (1.0f + exp_q(-value));
        x[k] = (silu ? value * sigmoid : sigmoid) * scale;
    }
    out[i] = pack8(x);
}

// mixed[t][i] = bf16((sum over streams in order of n[s][i] * m[s][i]) / 4)
// (q38_hyper.cu:99-114), 8 values a thread.
__global__ __launch_bounds__(256) void hyper_mix_kernel(const uint4* __restrict__ normalized,
                                                        const uint4* __restrict__ mix,
                                                        uint4* __restrict__ mixed,
                                                        uint32_t hidden8, uint64_t total8) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    if (i >= total8) return;
    const uint64_t token = i / hidden8;
    const uint32_t within = static_cast<uint32_t>(i % hidden8);
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t s = 0; s < kStreams; ++s) {
        const uint64_t at = (token * kStreams + s) * hidden8 + within;
        float n[8], m[8];
        unpack8(normalized[at], n);
        unpack8(mix[at], m);
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] = __builtin_fmaf(n[k], m[k], acc[k]);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = acc[k] / static_cast<float>(kStreams);
    mixed[i] = pack8(acc);
}

// output[t][s][i] = bf16(original[t][s][i] + block[t][i] * injection[t][s])
// (q38_hyper.cu:116-135), 8 values a thread.
__global__ __launch_bounds__(256) void hyper_inject_kernel(const uint4* __restrict__ original,
                                                           const uint4* __restrict__ block,
                                                           const uint16_t* __restrict__ injection,
                                                           uint4* __restrict__ output,
                                                           uint32_t hidden8, uint64_t total8) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    if (i >= total8) return;
    const uint64_t token = i / (kStreams * hidden8);
    const uint32_t rest = static_cast<uint32_t>(i % (kStreams * hidden8));
    const uint32_t s = rest / hidden8, within = rest % hidden8;
    const float g = bf16_to_f32(injection[token * kStreams + s]);
    float o[8], b[8];
    unpack8(original[i], o);
    unpack8(block[token * hidden8 + within], b);
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = __builtin_fmaf(b[k], g, o[k]);
    output[i] = pack8(o);
}

inline uint32_t grid8(uint64_t total8) { return static_cast<uint32_t>((total8 + 255u) / 256u); }

}  // namespace

hipError_t launch_hyper_repeat(const uint16_t* embedding, uint16_t* hyper, uint32_t tokens,
                               uint32_t hidden, hipStream_t stream) {
    const uint64_t total8 = static_cast<uint64_t>(tokens) * kStreams * (hidden / 8u);
    hyper_repeat_kernel<<<grid8(total8), 256, 0, stream>>>(
        reinterpret_cast<const uint4*>(embedding), reinterpret_cast<uint4*>(hyper), hidden / 8u,
        total8);
    return hipGetLastError();
}

hipError_t launch_hyper_norm(const uint16_t* hyper, const uint16_t* weight,
                             const uint16_t* inject, uint32_t tokens, uint32_t hidden,
                             uint16_t* normalized, uint16_t* injection, hipStream_t stream) {
    const uint32_t chunks = kStreams * hidden / 8u;
    const uint32_t per_thread = (chunks + kNormThreads - 1u) / kNormThreads;
#define Q38M_NORM(n)                                                                          \
    hyper_norm_kernel<n><<<tokens, kNormThreads, 0, stream>>>(hyper, weight, inject, hidden, \
                                                               normalized, injection)
    if (per_thread <= 2u)
        Q38M_NORM(2);
    else if (per_thread <= 4u)
        Q38M_NORM(4);
    else if (per_thread <= 6u)
        Q38M_NORM(6);
    else if (per_thread <= 8u)
        Q38M_NORM(8);
    else
        Q38M_NORM(16);
#undef Q38M_NORM
    return hipGetLastError();
}

hipError_t launch_hyper_elementwise(const uint16_t* in, uint16_t* out, uint64_t elements,
                                    float divisor, float scale, bool silu, hipStream_t stream) {
    const uint64_t total8 = elements / 8u;
    hyper_elementwise_kernel<<<grid8(total8), 256, 0, stream>>>(
        reinterpret_cast<const uint4*>(in), reinterpret_cast<uint4*>(out), total8, divisor, scale,
        silu ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_hyper_mix(const uint16_t* normalized, const uint16_t* mix, uint16_t* mixed,
                            uint32_t tokens, uint32_t hidden, hipStream_t stream) {
    const uint64_t total8 = static_cast<uint64_t>(tokens) * (hidden / 8u);
    hyper_mix_kernel<<<grid8(total8), 256, 0, stream>>>(
        reinterpret_cast<const uint4*>(normalized), reinterpret_cast<const uint4*>(mix),
        reinterpret_cast<uint4*>(mixed), hidden / 8u, total8);
    return hipGetLastError();
}

hipError_t launch_hyper_inject(const uint16_t* original, const uint16_t* block,
                               const uint16_t* injection, uint16_t* output, uint32_t tokens,
                               uint32_t hidden, hipStream_t stream) {
    const uint64_t total8 = static_cast<uint64_t>(tokens) * kStreams * (hidden / 8u);
    hyper_inject_kernel<<<grid8(total8), 256, 0, stream>>>(
        reinterpret_cast<const uint4*>(original), reinterpret_cast<const uint4*>(block),
        injection, reinterpret_cast<uint4*>(output), hidden / 8u, total8);
    return hipGetLastError();
}

size_t hyper_prepare_scratch_bytes(uint32_t tokens, uint32_t hidden, uint32_t low_rank) {
    const size_t wide = static_cast<size_t>(tokens) * kStreams * hidden * sizeof(uint16_t);
    return 2u * wide + static_cast<size_t>(tokens) * low_rank * sizeof(uint16_t);
}

hipError_t launch_hyper_prepare(const uint16_t* hyper, const uint16_t* norm_weight,
                                const uint16_t* mix_down, const uint16_t* mix_up,
                                const uint16_t* inject, uint32_t tokens, uint32_t hidden,
                                uint32_t low_rank, void* scratch, uint16_t* mixed,
                                uint16_t* injection, hipStream_t stream) {
    const uint32_t width = kStreams * hidden;
    uint16_t* normalized = static_cast<uint16_t*>(scratch);
    uint16_t* mix = normalized + static_cast<size_t>(tokens) * width;
    uint16_t* low = mix + static_cast<size_t>(tokens) * width;
    hipError_t e = launch_hyper_norm(hyper, norm_weight, inject, tokens, hidden, normalized,
                                     injection, stream);
    if (e == hipSuccess)
        e = launch_dense_gemm_act(normalized, mix_down, tokens, low_rank, width, true,
                                  static_cast<float>(kStreams), 1.0f, low, stream);
    if (e == hipSuccess)
        e = launch_dense_gemm_act(low, mix_up, tokens, width, low_rank, false, 1.0f, 1.0f, mix,
                                  stream);
    if (e == hipSuccess) e = launch_hyper_mix(normalized, mix, mixed, tokens, hidden, stream);
    return e;
}

}  // namespace q38m
