// Batch-1 decode: streams only the top_k selected experts (the tokens == 1
// branch of cuda_moe_routed_bf16, cuda/q38_moe.cu:388-458).  The
// arithmetic is the prefill contract evaluated for one token -- int8 token
// quantisation, per-group int32 accumulators, the fp32 group chain in group
// order, the SwiGLU fold, per-route mid quantisation, down, and the rank-
// order sum -- so decode equals the grouped prefill with tokens == 1 bit
// for bit.  (The reference's decode applies the router weight after down
// and differs from its prefill by up to 0.075, cuda_kernel_tests.cu:370.)
//
// Two launches per layer:
//   gate/up  grid (I/16 tile pairs, top_k), 4 waves split K in quarters and
//            every wave issues all of its weight loads before any math, so
//            the whole 10-expert weight set is in flight at once; the int32
//            group accumulators meet in LDS for the ordered fp32 chain.
//   down     grid (H/16 tiles), one wave per route; quantises its route's
//            mid row, runs the down tile, and the block sums the routes in
//            rank order.
#include "q38m_device.h"
#include "q38m_internal.h"

namespace q38m {
namespace {

template <uint32_t H, uint32_t I>
__global__ __launch_bounds__(256) void decode_gate_up_kernel(
    const uint4* __restrict__ w, const uint2* __restrict__ s,
    const uint16_t* __restrict__ hidden, const int32_t* __restrict__ ids,
    const float* __restrict__ route_weights, uint16_t* __restrict__ mid) {
    constexpr uint32_t kQuads = H / 128u;
    constexpr uint32_t kGroups = H / 32u;
    constexpr uint32_t kTiles = 2u * I / 16u;
    constexpr uint32_t kQuadsPerWave = kQuads / 4u;
    static_assert(H == 256u * 8u, "one 8-element chunk of the token per thread");
    __shared__ float acc_lds[kGroups][32];
    __shared__ float scale_lds[kGroups][32];
    __shared__ uint2 xq_lds[H / 8u];
    __shared__ float wave_max[4];

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t n = lane & 15u;
    const uint32_t q = lane >> 4;
    const uint32_t gate_tile = blockIdx.x;  // = the gate/up pair index
    const uint32_t route = blockIdx.y;
    const int32_t id = ids[route];
    const bool valid = id >= 0 && id < static_cast<int32_t>(kExperts);
    const uint32_t e = valid ? static_cast<uint32_t>(id) : 0u;

    // weights first: every load of this wave's K quarter is issued now
    // (paired quad-major layout: gate tile of pair p in slot 2p, up in 2p+1)
    uint4 bg[kQuadsPerWave], bu[kQuadsPerWave];
    uint2 cg[kQuadsPerWave], cu[kQuadsPerWave];
    const uint4* wg = w + (static_cast<size_t>(e) * kQuads * kTiles + 2u * gate_tile) * 64u + lane;
    const uint4* wu = wg + 64u;
    const uint2* sg = s + (static_cast<size_t>(e) * kQuads * kTiles + 2u * gate_tile) * 16u + n;
    const uint2* su = sg + 16u;
#pragma unroll
    for (uint32_t i = 0; i < kQuadsPerWave; ++i) {
        const uint32_t kq = wave * kQuadsPerWave + i;
        bg[i] = wg[kq * kTiles * 64u];
        bu[i] = wu[kq * kTiles * 64u];
        cg[i] = sg[kq * kTiles * 16u];
        cu[i] = su[kq * kTiles * 16u];
    }

    // int8 quantisation of the token (same arithmetic as the row kernel)
    const uint4 hv = reinterpret_cast<const uint4*>(hidden)[threadIdx.x];
    const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        amax = fmaxf(amax, fabsf(bf16_to_f32(hw[i] & 0xffffu)));
        amax = fmaxf(amax, fabsf(bf16_to_f32(hw[i] >> 16)));
    }
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1)
        amax = fmaxf(amax, __shfl_xor(amax, offset, 64));
    if (lane == 0) wave_max[wave] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wave_max[0], wave_max[1]), fmaxf(wave_max[2], wave_max[3]));
    float xs = amax / 127.0f;
    if (xs == 0.0f) xs = 1.0f;
    {
        uint32_t packed[2] = {0u, 0u};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t h = (i & 1) ? (hw[i >> 1] >> 16) : (hw[i >> 1] & 0xffffu);
            float r = __builtin_rintf(bf16_to_f32(h) / xs);
            r = fminf(fmaxf(r, -127.0f), 127.0f);
            packed[i >> 2] |= (static_cast<uint32_t>(static_cast<int32_t>(r)) & 0xffu) << (8 * (i & 3));
        }
        xq_lds[threadIdx.x] = make_uint2(packed[0], packed[1]);
    }
    __syncthreads();

    const v4i zero = {0, 0, 0, 0};
#pragma unroll
    for (uint32_t i = 0; i < kQuadsPerWave; ++i) {
        const uint32_t kq = wave * kQuadsPerWave + i;
        const uint32_t wgw[4] = {bg[i].x, bg[i].y, bg[i].z, bg[i].w};
        const uint32_t wuw[4] = {bu[i].x, bu[i].y, bu[i].z, bu[i].w};
        const uint32_t sgw[2] = {cg[i].x, cg[i].y};
        const uint32_t suw[2] = {cu[i].x, cu[i].y};
#pragma unroll
        for (uint32_t j = 0; j < 4u; ++j) {
            const uint32_t g = 4u * kq + j;
            const long a = as_long(xq_lds[4u * g + q]);
            const v4i dg = mfma_i8_16x16x32(a, unpack_w4x16(wgw[j]), zero);
            const v4i du = mfma_i8_16x16x32(a, unpack_w4x16(wuw[j]), zero);
            if (q == 0u) {
                const uint32_t hg = (j & 1u) ? (sgw[j >> 1] >> 16) : (sgw[j >> 1] & 0xffffu);
                const uint32_t hu = (j & 1u) ? (suw[j >> 1] >> 16) : (suw[j >> 1] & 0xffffu);
                acc_lds[g][n] = static_cast<float>(dg[0]);
                acc_lds[g][16u + n] = static_cast<float>(du[0]);
                scale_lds[g][n] = f16_to_f32(hg) * 0.0625f;
                scale_lds[g][16u + n] = f16_to_f32(hu) * 0.0625f;
            }
        }
    }
    __syncthreads();

    if (wave == 0u && lane < 32u) {
        float y = 0.0f;
        for (uint32_t g = 0; g < kGroups; ++g)
            y = __builtin_fmaf(acc_lds[g][lane], scale_lds[g][lane], y);
        const float y_up = __shfl(y, static_cast<int>(lane + 16u), 64);
        if (lane < 16u) {
            const float y_gate = y * xs;
            const float y_u = y_up * xs;
            const uint32_t value = valid ? swiglu_fold(y_gate, y_u, route_weights[route]) : 0u;
            mid[static_cast<size_t>(route) * I + gate_tile * 16u + n] =
                static_cast<uint16_t>(value);
        }
    }
}

template <uint32_t H, uint32_t I, bool kW4>
__global__ __launch_bounds__(640) void decode_down_kernel(
    const uint4* __restrict__ w, const void* __restrict__ s,
    const uint16_t* __restrict__ mid, const int32_t* __restrict__ ids,
    uint32_t top_k, uint16_t* __restrict__ out) {
    constexpr uint32_t kTiles = H / 16u;
    constexpr uint32_t kBlocks = kW4 ? I / 128u : I / 64u;  // W4: quads, W8: 64-wide blocks
    static_assert(I == 64u * 8u, "one 8-element chunk of the mid row per lane");
    __shared__ uint2 mq_lds[kTopK][I / 8u];
    __shared__ float o_lds[kTopK][16];

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t route = threadIdx.x >> 6;
    const uint32_t n = lane & 15u;
    const uint32_t q = lane >> 4;
    const uint32_t tile = blockIdx.x;
    const int32_t id = ids[route];
    const bool valid = id >= 0 && id < static_cast<int32_t>(kExperts);
    const uint32_t e = valid ? static_cast<uint32_t>(id) : 0u;

    // W8: tile-major [e][tile][kb]; W4: quad-major [e][kq][tile]
    uint4 b[kBlocks];
    const uint4* wt = kW4 ? w + (static_cast<size_t>(e) * kBlocks * kTiles + tile) * 64u + lane
                          : w + static_cast<size_t>(e * kTiles + tile) * kBlocks * 64u + lane;
    const uint32_t block_stride = kW4 ? kTiles * 64u : 64u;
#pragma unroll
    for (uint32_t kb = 0; kb < kBlocks; ++kb) b[kb] = wt[kb * block_stride];
    uint2 c[kW4 ? kBlocks : 1];
    float ws = 0.0f;
    if constexpr (kW4) {
        const uint2* st = static_cast<const uint2*>(s) +
                          (static_cast<size_t>(e) * kBlocks * kTiles + tile) * 16u + n;
#pragma unroll
        for (uint32_t kb = 0; kb < kBlocks; ++kb) c[kb] = st[kb * kTiles * 16u];
    } else {
        ws = f16_to_f32(static_cast<const uint16_t*>(s)[static_cast<size_t>(e) * H + tile * 16u + n]);
    }

    // quantise this route's mid row (8 elements per lane)
    const uint4 mv = reinterpret_cast<const uint4*>(mid + static_cast<size_t>(route) * I)[lane];
    const uint32_t mw[4] = {mv.x, mv.y, mv.z, mv.w};
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        amax = fmaxf(amax, fabsf(bf16_to_f32(mw[i] & 0xffffu)));
        amax = fmaxf(amax, fabsf(bf16_to_f32(mw[i] >> 16)));
    }
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1)
        amax = fmaxf(amax, __shfl_xor(amax, offset, 64));
    float sm = amax / 127.0f;
    if (sm == 0.0f) sm = 1.0f;
    {
        uint32_t packed[2] = {0u, 0u};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t h = (i & 1) ? (mw[i >> 1] >> 16) : (mw[i >> 1] & 0xffffu);
            float r = __builtin_rintf(bf16_to_f32(h) / sm);
            r = fminf(fmaxf(r, -127.0f), 127.0f);
            packed[i >> 2] |= (static_cast<uint32_t>(static_cast<int32_t>(r)) & 0xffu) << (8 * (i & 3));
        }
        mq_lds[route][lane] = make_uint2(packed[0], packed[1]);
    }
    __syncthreads();

    float o = 0.0f;
    if constexpr (kW4) {
        const v4i zero = {0, 0, 0, 0};
        float y = 0.0f;
#pragma unroll
        for (uint32_t kq = 0; kq < kBlocks; ++kq) {
            const uint32_t bw[4] = {b[kq].x, b[kq].y, b[kq].z, b[kq].w};
            const uint32_t cw[2] = {c[kq].x, c[kq].y};
#pragma unroll
            for (uint32_t j = 0; j < 4u; ++j) {
                const uint32_t g = 4u * kq + j;
                const long a = as_long(mq_lds[route][4u * g + q]);
                const v4i d = mfma_i8_16x16x32(a, unpack_w4x16(bw[j]), zero);
                const uint32_t h = (j & 1u) ? (cw[j >> 1] >> 16) : (cw[j >> 1] & 0xffffu);
                y = __builtin_fmaf(static_cast<float>(d[0]), f16_to_f32(h) * 0.0625f, y);
            }
        }
        o = y * sm;
    } else {
        v4i acc = {0, 0, 0, 0};
#pragma unroll
        for (uint32_t kb = 0; kb < kBlocks; ++kb) {
            const uint2 lo = mq_lds[route][8u * kb + 2u * q];
            const uint2 hi = mq_lds[route][8u * kb + 2u * q + 1u];
            const uint4 a = make_uint4(lo.x, lo.y, hi.x, hi.y);
            acc = mfma_i8_16x16x64(as_v4i(a), as_v4i(b[kb]), acc);
        }
        o = (static_cast<float>(acc[0]) * ws) * sm;
    }
    if (q == 0u) o_lds[route][n] = valid ? o : 0.0f;
    __syncthreads();
    if (route == 0u && lane < 16u) {
        float total = 0.0f;
        for (uint32_t r = 0; r < top_k; ++r) total += o_lds[r][lane];
        out[tile * 16u + lane] = static_cast<uint16_t>(f32_to_bf16(total));
    }
}

}  // namespace

size_t decode_scratch_bytes() { return static_cast<size_t>(kTopK) * kInter * sizeof(uint16_t); }

hipError_t launch_decode(const q38m_expert_weights_v1& gate_up,
                         const q38m_expert_weights_v1& down,
                         const uint16_t* hidden, const int32_t* ids,
                         const float* weights, uint32_t top_k, void* scratch,
                         uint16_t* output, hipStream_t stream) {
    uint16_t* mid = static_cast<uint16_t*>(scratch);
    decode_gate_up_kernel<kHidden, kInter><<<dim3(kInter / 16u, top_k), 256, 0, stream>>>(
        static_cast<const uint4*>(gate_up.data), static_cast<const uint2*>(gate_up.scales),
        hidden, ids, weights, mid);
    if (down.format == Q38M_FORMAT_W8_SYM)
        decode_down_kernel<kHidden, kInter, false><<<kHidden / 16u, 64u * top_k, 0, stream>>>(
            static_cast<const uint4*>(down.data), down.scales, mid, ids, top_k, output);
    else
        decode_down_kernel<kHidden, kInter, true><<<kHidden / 16u, 64u * top_k, 0, stream>>>(
            static_cast<const uint4*>(down.data), down.scales, mid, ids, top_k, output);
    return hipGetLastError();
}

}  // namespace q38m
