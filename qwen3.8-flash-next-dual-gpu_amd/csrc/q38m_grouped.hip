// Expert-grouped prefill: gate/up (W4 g32) with fused SwiGLU and router
// weight, down (W8 per-channel or W4 g32), and the fixed-order combine.
//
// Work decomposition: one workgroup per (task, output slice), where a task
// is one M=16 tile of one expert from the V1 route plan.  Each wave owns a
// 16-channel tile (W4 gate/up: a gate or an up tile, the pair meeting in
// LDS for the SwiGLU; W8 gate/up: a gate tile and its matching up tile, so
// the SwiGLU pair sits in the same lane) and streams the expert's weights
// straight from HBM into VGPRs in the MFMA16 layout: every wave-wide
// 16-byte load is 1 KiB contiguous.  Tasks beyond the plan's task_count
// carry valid_rows == 0 and exit at once (q38_moe_prefill.cu:316-317).
#include "q38m_device.h"
#include "q38m_internal.h"
#include "q38m_select.h"

namespace q38m {
namespace {

// The down kernels' A operand: the int8 mid rows and their scales (the
// staged entry point), or -- kQuantize, the one-call step -- the bf16 mid
// rows, which the kernel quantises itself while its first weights stream:
// one wave per row, lane l holding elements [8l, 8l + 8), the arithmetic of
// quantize_rows_kernel<1> (row_absmax8, wave_max_f32, quant_scale,
// quantize8), so the int8 rows and scales are the same bit for bit.  The
// workgroups of output slice 0 also store them to q / s, where the caller's
// workspace keeps them.
struct MidRows {
    const int8_t* q;        // [routes][I] int8 (written by slice 0 when kQuantize)
    const float* s;         // [routes] scales (likewise)
    const uint16_t* bf16;   // kQuantize: [routes][I] bf16 rows
};

// Quantise one 512-wide bf16 row held as lane l's elements [8l, 8l + 8).
__device__ __forceinline__ uint2 quantize_mid_row(uint4 v, float& scale) {
    const uint32_t hw[4] = {v.x, v.y, v.z, v.w};
    const QuantScale qs = quant_scale(wave_max_f32(row_absmax8(hw)));
    scale = qs.s;
    return quantize8(hw, qs);
}

// Device-coherent (agent-scope) loads and stores: seen by every XCD
// without a cache writeback or invalidation around them.
template <typename T>
__device__ __forceinline__ T load_device(const T* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void store_device(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct TileWeights {
    uint4 w;   // one quad of the wave's tile
    uint2 s;   // its scale words (load_quad_scales)
};

// One quad (128 columns) of the chain for one 16-channel tile.  Per 32-wide
// sub-block one MFMA; the kSub sub-blocks of a group chain through the
// int32 accumulator input (the first from zero), giving the group's exact
// 16*acc; then the fp32 chain y16 = fma(16*acc, s_g, y16) (fp16 scales) or
// y = fma(16*acc, s_g/16, y) (bf16 scales).
template <uint32_t kSub, bool kBf16>
__device__ __forceinline__ void tile_quad(const uint2* __restrict__ a_quad, uint4 wt, uint2 sc,
                                          float (&y)[4]) {
    const v4i zero = {0, 0, 0, 0};
    const uint32_t ww[4] = {wt.x, wt.y, wt.z, wt.w};
    v4i c = zero;  // kSub > 1: the group's running int32 tile
#pragma unroll
    for (uint32_t j = 0; j < 4u; ++j) {
        const long a = as_long(a_quad[j * 64u]);
        const v4i d = mfma_i8_16x16x32(a, unpack_w4x16(ww[j]), j % kSub == 0u ? zero : c);
        if (j % kSub != kSub - 1u) {
            c = d;
            continue;
        }
        const uint32_t ws = quad_scale_word(sc, j / kSub);
        const float scale = kBf16 ? bf16_to_f32(ws) * 0.0625f : f16_to_f32(ws);
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] = __builtin_fmaf(static_cast<float>(d[i]), scale, y[i]);
    }
}

// ---------------------------------------------------------------------------
// Gate/up, W4 in groups of 32 (64, 128), MFMA16 layout.
//   acc[r][j][g] = sum_{k in g} xq[token(r)][k] * W[e][j][k]        (int32)
//   y[r][j]      = fmaf-chain over g = 0..H/32-1 of acc * s[e][j][g]  (fp32)
//   then y * xs[token(r)] and the SwiGLU fold of the reference epilogue.
// One v_mfma_i32_16x16x32_i8 per group gives that group's exact int32
// tile (zero accumulator), so the fp32 chain runs in group order in the
// same lanes that hold the accumulators.
//
// Work: a workgroup of kWaves waves covers kWaves/2 channel pairs of one
// task; wave w streams one tile -- the gate tile (w even) or the up tile (w
// odd) of pair blockIdx.x * kWaves/2 + w/2 -- two quads ahead through three
// register sets, and the up wave hands its chain to the gate wave through
// LDS for the SwiGLU epilogue.  One tile per wave (not a gate + up pair)
// halves a wave's stream (16 KiB of weights), so the slab's last
// workgroups drain in half the time, and at ~57 VGPRs and 36 KiB of LDS
// four workgroups (32 waves) fit per CU: config 2's step 0.2247 -> 0.2216
// ms against the pair-per-wave form (bit-identical; two or four quads
// ahead, or 4 / 16 waves per workgroup, measured slower).
// The task's 16 int8 token rows (32 KiB) are staged into LDS once in the
// MFMA A-operand order ([group][lane], 8 bytes per lane), so the waves read
// activations with conflict-free 512-byte ds_read_b64 instead of each
// re-reading them from L2.
//
// The MFMA gives 16*acc (nibbles in the high half of each byte).  fp16
// scales: the raw scale feeds the fma, so y16 = 16*y exactly at every step
// (power-of-two scaling commutes with rounding; all partial sums are
// multiples of 2^-24, far from the subnormal range), and y = y16 * 0.0625.
// bf16 scale words can sit near the subnormal range, so the fma takes s/16
// (exact in fp32, subnormals included; |16*acc| < 2^24): each product is
// acc*s exactly and the chain holds y itself.  Then y * s_t.
//
// gate_up_w4_item is one (task, channel slice) item of this plan, shared by
// gate_up_w4_kernel (one item per workgroup) and gate_up_down_kernel: a_lds
// holds H / 32 * 64 uint2, up_lds kWaves / 2 blocks of 4 x 64 floats,
// row_info the task's 16 (token scale, route weight) pairs, read while the
// rows stage so that the epilogue makes no global round trip.
// kPublish (the fused launch): the mid words are stored device-coherently
// and, once every wave's stores are complete, *flag is set to 1.
// ---------------------------------------------------------------------------
template <uint32_t H, uint32_t I, uint32_t kWaves, uint32_t kSub, bool kBf16, bool kPublish>
__device__ __forceinline__ void gate_up_w4_item(
    const uint4* __restrict__ w, const uint16_t* __restrict__ s,
    const int8_t* __restrict__ xq, const float* __restrict__ xs,
    const uint32_t* __restrict__ packed, const float* __restrict__ route_weights,
    const TaskRecord task, const uint32_t slice, uint16_t* __restrict__ mid, uint2* a_lds,
    float (*up_lds)[4][64], float2* row_info, uint32_t* flag) {
    constexpr uint32_t kQuads = H / 128u;
    constexpr uint32_t kTiles = 2u * I / 16u;
    constexpr uint32_t kThreads = kWaves * 64u;
    constexpr uint32_t kDepth = 2u, kSets = kDepth + 1u;
    static_assert(kWaves % 2u == 0u, "gate and up waves in pairs");

    const uint32_t rows = task.rows;
    if (rows == 0u) return;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n = lane & 15u;
    const uint32_t q = lane >> 4;
    const uint32_t pair = slice * (kWaves / 2u) + (wave >> 1);
    const uint32_t up = wave & 1u;
    const uint32_t e = task.expert;
    const uint32_t p0 = task.begin;

    // Paired quad-major layout: for quad kq the gate tile of pair p is slot
    // 2p and its up tile slot 2p+1 (1 KiB each, 256 B of scale words)
    constexpr uint32_t kQuadWords = kTiles * 64u;  // uint4 per quad of one expert
    constexpr uint32_t kRowScales = 4u / kSub;     // scale words per row and quad
    constexpr uint32_t kSlotScales = 16u * kRowScales;
    constexpr uint32_t kQuadScales = kTiles * kSlotScales;
    // uniform bases (scalar registers) plus 32-bit per-lane offsets
    const uint32_t slot = 2u * pair + up;
    const uint4* wbase = w + (static_cast<size_t>(e) * kQuads * kTiles + slot) * 64u;
    const uint16_t* sbase =
        s + (static_cast<size_t>(e) * kQuads * kTiles + slot) * kSlotScales;
    auto load = [&](uint32_t kq) {
        const uint32_t k = kq < kQuads ? kq : kQuads - 1u;  // past the end: re-read (L1 hit)
        return TileWeights{load_stream(wbase + k * kQuadWords + lane),
                           load_quad_scales<kSub>(sbase + k * kQuadScales + n * kRowScales)};
    };

    // Stage A: 16-byte chunk c of token row r holds group c/2 for lane groups
    // q = 2(c%2) and 2(c%2)+1.  Rows past valid_rows replicate row 0.  The
    // row indices are loaded first, then the first two quads of weights and
    // all row chunks, so A costs two round trips and the weights stay in
    // flight meanwhile.
    // Piece i is row i % 16, chunk i / 16: consecutive lanes take
    // consecutive rows, so a store instruction spreads over the banks (a
    // row's chunks all fall in its bank pair; row-major pieces put 32 lanes
    // on one), and every piece of a thread is in the same row (one index).
    constexpr uint32_t kChunks = 16u * (H / 16u) / kThreads;
    static_assert(16u * (H / 16u) % kThreads == 0u && kThreads % 16u == 0u,
                  "whole chunks per thread, one row per thread");
    const uint32_t srow = threadIdx.x % 16u;
    const uint32_t token = checked(packed[p0 + (srow < rows ? srow : 0u)],
                                   Q38M_PREFILL_SLAB_MAX_TOKENS * kTopK, kCheckToken);
    if (threadIdx.x < 16u) row_info[srow] = make_float2(xs[token / kTopK], route_weights[token]);
    TileWeights r[kSets];
#pragma unroll
    for (uint32_t i = 0; i < kDepth; ++i) r[i] = load(i);
    const uint4* arow = reinterpret_cast<const uint4*>(xq + static_cast<size_t>(token / kTopK) * H);
    uint4 v[kChunks];
#pragma unroll
    for (uint32_t c = 0; c < kChunks; ++c) v[c] = arow[(threadIdx.x + c * kThreads) / 16u];
#pragma unroll
    for (uint32_t c = 0; c < kChunks; ++c) {
        const uint32_t chunk = (threadIdx.x + c * kThreads) / 16u;
        const uint32_t base = (chunk >> 1) * 64u + (chunk & 1u) * 32u + srow;
        a_lds[base] = make_uint2(v[c].x, v[c].y);
        a_lds[base + 16u] = make_uint2(v[c].z, v[c].w);
    }
    __syncthreads();

    // kDepth quads ahead through kSets register sets in a fixed rotation:
    // each load lands in the set consumed one step earlier, so no register
    // with a load in flight is ever copied (a copy would wait for the
    // load).  Each step issues its load before any of its math (scheduling
    // barrier).
    float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const uint2* a_base = a_lds + lane;
    constexpr uint32_t kFull = kQuads / kSets * kSets;
#pragma unroll 1
    for (uint32_t kq = 0; kq < kFull; kq += kSets) {
#pragma unroll
        for (uint32_t i = 0; i < kSets; ++i) {
            r[(i + kDepth) % kSets] = load(kq + i + kDepth);
            __builtin_amdgcn_sched_barrier(0);
            tile_quad<kSub, kBf16>(a_base + 4u * (kq + i) * 64u, r[i].w, r[i].s, y);
        }
    }
#pragma unroll
    for (uint32_t i = 0; i < kQuads - kFull; ++i) {
        if (kFull + i + kDepth < kQuads) r[(i + kDepth) % kSets] = load(kFull + i + kDepth);
        __builtin_amdgcn_sched_barrier(0);
        tile_quad<kSub, kBf16>(a_base + 4u * (kFull + i) * 64u, r[i].w, r[i].s, y);
    }

    // the up wave's chain to its gate wave
    if (up) {
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) up_lds[wave >> 1][i][lane] = y[i];
    }
    __syncthreads();
    if constexpr (!kPublish) {
        if (up) return;
    }
    if (!up) {
        const uint32_t channel = pair * 16u + n;
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) {
            const uint32_t rr = 4u * q + i;
            if (rr >= rows) continue;
            const uint32_t p = p0 + rr;
            const float2 info = row_info[rr];  // (token scale, route weight)
            const float unscale = kBf16 ? 1.0f : 0.0625f;
            const float y_gate = (y[i] * unscale) * info.x;
            const float y_up = (up_lds[wave >> 1][i][lane] * unscale) * info.x;
            const uint16_t m = static_cast<uint16_t>(swiglu_fold(y_gate, y_up, info.y));
            if constexpr (kPublish)
                store_device(mid + static_cast<size_t>(p) * I + channel, m);
            else
                mid[static_cast<size_t>(p) * I + channel] = m;
        }
    }
    if constexpr (kPublish) {
        // every wave's mid words have reached the device coherence point
        // before the flag is set
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0u) store_device(flag, 1u);
    }
}

template <uint32_t H, uint32_t I, uint32_t kWaves, uint32_t kSub, bool kBf16>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(6, 8)))
void gate_up_w4_kernel(
    const uint4* __restrict__ w, const uint16_t* __restrict__ s,
    const int8_t* __restrict__ xq, const float* __restrict__ xs,
    const uint32_t* __restrict__ packed, const float* __restrict__ route_weights,
    const q38m_task_v1* __restrict__ tasks, uint16_t* __restrict__ mid) {
    __shared__ uint2 a_lds[H / 32u * 64u];
    __shared__ float up_lds[kWaves / 2u][4][64];
    __shared__ float2 row_info[16];
    gate_up_w4_item<H, I, kWaves, kSub, kBf16, false>(w, s, xq, xs, packed, route_weights,
                                                      read_task(tasks, blockIdx.y), blockIdx.x,
                                                      mid, a_lds, up_lds, row_info, nullptr);
}

// ---------------------------------------------------------------------------
// Gate/up, W8 (the reference's edge-layer format, tools/q38_quant_policy.py:
// 164-190), paired K-block-major MFMA16 layout: per 64-wide K block one
// v_mfma_i32_16x16x64_i8 per tile.  Groups of kBlocksPerGroup blocks (64 or
// 128 columns): the group's blocks chain through the accumulator input and
// at its last block y = fmaf((float)acc_g, s_g, y) in group order; per
// channel (kBlocksPerGroup == H/64): one int32 over K, y = (float)acc * s.
// Scales stay in the artifact order [E][rows][K/G] (gate rows 0..I-1, up
// rows I..2I-1).  Then y * s_t and the SwiGLU fold, as the W4 kernel.
// Same plan as the W4 kernel: the task's 16 token rows (32 KiB) staged once
// in LDS in the A-operand order ([block][lane], 16 bytes per lane); each
// wave streams ONE tile (the gate tile, w even, or the up tile, w odd, of
// pair blockIdx.x * kWaves/2 + w/2) two blocks ahead through three register
// sets, and the up wave hands its y to the gate wave through LDS for the
// SwiGLU (against a gate + up pair per wave: edge-format slab step 0.3162
// -> 0.3116 ms; 16 waves per workgroup 0.324 ms).
// ---------------------------------------------------------------------------

template <uint32_t H, uint32_t I, uint32_t kWaves, uint32_t kBlocksPerGroup, bool kBf16>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(6, 8)))
void gate_up_w8_kernel(
    const uint4* __restrict__ w, const uint16_t* __restrict__ s,
    const int8_t* __restrict__ xq, const float* __restrict__ xs,
    const uint32_t* __restrict__ packed, const float* __restrict__ route_weights,
    const q38m_task_v1* __restrict__ tasks, uint16_t* __restrict__ mid) {
    constexpr uint32_t kBlocks = H / 64u;
    constexpr uint32_t kTiles = 2u * I / 16u;
    constexpr uint32_t kThreads = kWaves * 64u;
    constexpr bool kPerChannel = kBlocksPerGroup == kBlocks;
    constexpr uint32_t kGroups = kBlocks / kBlocksPerGroup;
    __shared__ uint4 a_lds[kBlocks * 64u];
    __shared__ float up_lds[kWaves / 2u][4][64];

    const TaskRecord task = read_task(tasks, blockIdx.y);
    const uint32_t rows = task.rows;
    if (rows == 0u) return;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n = lane & 15u;
    const uint32_t q = lane >> 4;
    const uint32_t pair = blockIdx.x * (kWaves / 2u) + (wave >> 1);
    const uint32_t up = wave & 1u;
    const uint32_t e = task.expert;
    const uint32_t p0 = task.begin;

    constexpr uint32_t kBlockWords = kTiles * 64u;  // uint4 per K block of one expert
    const uint4* wbase = w + (static_cast<size_t>(e) * kBlocks * kTiles + 2u * pair + up) * 64u;
    // this lane's row: gate 16p+n or up I+16p+n
    const uint16_t* s_row =
        s + (static_cast<size_t>(e) * 2u * I + (up ? I : 0u) + pair * 16u + n) * kGroups;
    struct TileBlock {
        uint4 w;
        uint32_t s;
    };
    auto load = [&](uint32_t kb) {
        const uint32_t k = kb < kBlocks ? kb : kBlocks - 1u;  // past the end: re-read (L1 hit)
        const uint32_t wi = k * kBlockWords + lane;
        const uint32_t g = kPerChannel ? 0u : k / kBlocksPerGroup;
        return TileBlock{load_stream(wbase + wi), static_cast<uint32_t>(s_row[g])};
    };

    // Stage A: 16-byte chunk c of token row r is K block c/4, lane group c%4;
    // rows past valid_rows replicate row 0.
    constexpr uint32_t kChunks = 16u * (H / 16u) / kThreads;
    static_assert(16u * (H / 16u) % kThreads == 0u, "whole chunks per thread");
    uint32_t token[kChunks];
#pragma unroll
    for (uint32_t c = 0; c < kChunks; ++c) {
        const uint32_t r = (threadIdx.x + c * kThreads) / (H / 16u);
        token[c] = checked(packed[p0 + (r < rows ? r : 0u)], Q38M_PREFILL_SLAB_MAX_TOKENS * kTopK, kCheckToken);
    }
    TileBlock r0 = load(0), r1 = load(1), r2;
    uint4 v[kChunks];
#pragma unroll
    for (uint32_t c = 0; c < kChunks; ++c) {
        const uint32_t chunk = (threadIdx.x + c * kThreads) % (H / 16u);
        v[c] = reinterpret_cast<const uint4*>(xq + static_cast<size_t>(token[c] / kTopK) * H)[chunk];
    }
#pragma unroll
    for (uint32_t c = 0; c < kChunks; ++c) {
        const uint32_t i = threadIdx.x + c * kThreads;
        const uint32_t chunk = i % (H / 16u);
        a_lds[(chunk >> 2) * 64u + (chunk & 3u) * 16u + i / (H / 16u)] = v[c];
    }
    __syncthreads();

    const v4i zero = {0, 0, 0, 0};
    v4i c = zero;
    float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto block = [&](uint32_t kb, const TileBlock& b) {
        const v4i a = as_v4i(a_lds[kb * 64u + lane]);
        const bool first = kb % kBlocksPerGroup == 0u;
        c = mfma_i8_16x16x64(a, as_v4i(b.w), first ? zero : c);
        if constexpr (!kPerChannel) {
            if (kb % kBlocksPerGroup == kBlocksPerGroup - 1u) {
                const float scale = scale_to_f32(b.s, kBf16);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    y[i] = __builtin_fmaf(static_cast<float>(c[i]), scale, y[i]);
            }
        }
    };
    static_assert(kBlocks % 3u == 2u, "three-set rotation plus two peeled blocks");
#pragma unroll 1
    for (uint32_t kb = 0; kb + 2u < kBlocks; kb += 3u) {
        r2 = load(kb + 2u);
        __builtin_amdgcn_sched_barrier(0);
        block(kb, r0);
        r0 = load(kb + 3u);
        __builtin_amdgcn_sched_barrier(0);
        block(kb + 1u, r1);
        r1 = load(kb + 4u);
        __builtin_amdgcn_sched_barrier(0);
        block(kb + 2u, r2);
    }
    block(kBlocks - 2u, r0);
    block(kBlocks - 1u, r1);
    if constexpr (kPerChannel) {
        const float scale = scale_to_f32(r1.s, kBf16);
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] = static_cast<float>(c[i]) * scale;
    }

    // the up wave's y to its gate wave
    if (up) {
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) up_lds[wave >> 1][i][lane] = y[i];
    }
    __syncthreads();
    if (up) return;
    const uint32_t channel = pair * 16u + n;
#pragma unroll
    for (uint32_t i = 0; i < 4u; ++i) {
        const uint32_t r = 4u * q + i;
        if (r >= rows) continue;
        const uint32_t p = p0 + r;
        const uint32_t a = checked(packed[p], Q38M_PREFILL_SLAB_MAX_TOKENS * kTopK, kCheckToken);
        const float st = xs[a / kTopK];
        mid[static_cast<size_t>(p) * I + channel] =
            static_cast<uint16_t>(swiglu_fold(y[i] * st, up_lds[wave >> 1][i][lane] * st, route_weights[a]));
    }
}

// ---------------------------------------------------------------------------
// Down, W8, MFMA16 layout (16 int8 per lane per 64-wide K block), per output
// channel or in groups of kBlocksPerGroup K blocks (64 or 128 columns).
// Per channel (kBlocksPerGroup == I/64): acc = sum_k qm[r][k] * W[e][c][k]
// over all of K in one int32 (exact in fp32, |acc| < 2^24),
// o = ((float)acc * ws[e][c]) * sm[r].  Grouped: one int32 per group
// (its blocks chain through the MFMA accumulator input), the fp32 chain
// y = fmaf((float)acc_g, s[e][c][g], y) in group order from 0, o = y * sm[r].
// Group scales stay in the artifact order [E][rows][K/group].
//
// A workgroup of kWaves waves covers kWaves * kTilesPerWave 16-channel
// output tiles of one task.  The task's 16 int8 mid rows (8 KiB) are staged
// into LDS once in the MFMA A-operand order ([k block][lane], 16 bytes per
// lane).  Each wave streams its tiles in half-tile units (4 K blocks = 4 KiB
// per wave) with a pinned one-unit-ahead prefetch; the launch uses 16 waves
// of one tile each, and at ~51-71 VGPRs seven or eight waves per SIMD keep
// ~128 KB of weights in flight per CU.
//
// down_w8_item is one (task, output slice) item, shared by down_w8_kernel
// and gate_up_down_kernel: a_lds holds I / 64 * 64 uint4, scale_lds 16
// floats.  kAwait (the fused launch, kQuantize only): every wave requests
// its first weights, then wave 0 waits for the task's gate/up items
// (await_gate_up) and the workgroup reads the mid rows once they are
// complete; each item then counts itself in the task's counter, and the
// last of the task's eight down items clears the task's flags and counter
// at its end, so the flags are zero again when the launch ends.
// ---------------------------------------------------------------------------

// Poll budget of a down item waiting for its task's eight gate/up items:
// each poll is one device-coherent load (~1-5 us under load) and a short
// sleep.  Workgroups are dispatched in block order, so by the time a down
// item waits, every gate/up item is resident or done and the wait ends
// within a gate/up item's lifetime (~20 us); the budget only bounds it.
constexpr uint32_t kAwaitPolls = 1u << 14;

// Wave 0 of a down item: wait until the task's eight gate/up flags are set;
// if the budget runs out, record Q38M_PLAN_STEP_TIMEOUT in *status and tell
// the workgroup (expired_lds) to skip the item.
__device__ __forceinline__ void await_gate_up(const uint32_t* flags, uint32_t* status,
                                              uint32_t* expired_lds) {
    const uint32_t lane = threadIdx.x & 63u;
    bool expired = false;
    for (uint32_t polls = 1u;; ++polls) {
        const uint32_t v = lane < 8u ? load_device(flags + lane) : 1u;
        if (__all(v == 1u)) break;
        if (polls >= kAwaitPolls) {
            expired = true;
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    if (lane == 0u) {
        *expired_lds = expired ? 1u : 0u;
        if (expired)
            __hip_atomic_fetch_or(status, Q38M_PLAN_STEP_TIMEOUT, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <uint32_t H, uint32_t I, uint32_t kWaves, uint32_t kTilesPerWave,
          uint32_t kBlocksPerGroup, bool kBf16, bool kQuantize, bool kAwait>
__device__ __forceinline__ void down_w8_item(
    const uint4* __restrict__ w, const uint16_t* __restrict__ s, MidRows mid,
    const TaskRecord task, const uint32_t slice, float* __restrict__ out, uint4* a_lds,
    float* scale_lds, uint32_t* flags, uint32_t* counter, uint32_t* status,
    uint32_t* expired_lds) {
    constexpr uint32_t kBlocks = I / 64u;
    constexpr uint32_t kHalf = kBlocks / 2u;
    constexpr uint32_t kTiles = H / 16u;
    constexpr uint32_t kThreads = kWaves * 64u;
    constexpr bool kPerChannel = kBlocksPerGroup == kBlocks;
    constexpr uint32_t kGroups = kBlocks / kBlocksPerGroup;
    static_assert(kBlocks % 2u == 0u, "half-tile units");
    static_assert(kPerChannel || kHalf % kBlocksPerGroup == 0u, "groups within half tiles");
    static_assert(!kAwait || kQuantize, "the fused launch quantises the mid rows");

    const uint32_t rows = task.rows;
    if (rows == 0u) return;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n = lane & 15u;
    const uint32_t q = lane >> 4;
    const uint32_t e = task.expert;
    const uint32_t p0 = task.begin;
    const uint32_t tile0 = (slice * kWaves + wave) * kTilesPerWave;
    const uint4* wt = w + static_cast<size_t>(e * kTiles + tile0) * kBlocks * 64u + lane;

    // Stage A: 16-byte chunk c of mid row r is K block c/4, lane group c%4.
    // The row chunks are requested first, then the first half-tile of
    // weights, so the LDS stores wait for the rows only.
    constexpr uint32_t kStage = (16u * (I / 16u) + kThreads - 1u) / kThreads;
    constexpr uint32_t kRowsPerWave = 16u / kWaves;  // kQuantize: whole rows per wave
    static_assert(!kQuantize || (I == 512u && 16u % kWaves == 0u), "one wave per 512-wide row");
    float row_scale[4];
    uint4 b[kHalf];
    uint32_t ticket = 0u;  // kAwait, wave 0 lane 0: the items of the task counted before this one
    if constexpr (kQuantize) {
        uint4 mv[kRowsPerWave];
        auto load_rows = [&] {
#pragma unroll
            for (uint32_t j = 0; j < kRowsPerWave; ++j) {
                const uint32_t r = wave * kRowsPerWave + j;
                mv[j] = reinterpret_cast<const uint4*>(
                    mid.bf16 + static_cast<size_t>(p0 + (r < rows ? r : 0u)) * I)[lane];
            }
        };
        if constexpr (kAwait) {
            // the first weights stream while wave 0 waits; the rows are read
            // (ordinary loads) only once every line of them is final: the
            // fused launch started with no line of them in any L2, and the
            // gate/up items wrote each 128-byte line of a row whole, through
            // to the coherence point, before their flags
#pragma unroll
            for (uint32_t kb = 0; kb < kHalf; ++kb) b[kb] = load_stream(wt + kb * 64u);
            __builtin_amdgcn_sched_barrier(0);
            if (wave == 0u) await_gate_up(flags, status, expired_lds);
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (*expired_lds != 0u) return;
            // this item is past its wait: count it (the result is read at
            // the item's end)
            if (wave == 0u && lane == 0u)
                ticket = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
            load_rows();
        } else {
            load_rows();
#pragma unroll
            for (uint32_t kb = 0; kb < kHalf; ++kb) b[kb] = load_stream(wt + kb * 64u);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (uint32_t j = 0; j < kRowsPerWave; ++j) {
            const uint32_t r = wave * kRowsPerWave + j;
            float scale;
            const uint2 qv = quantize_mid_row(mv[j], scale);
            // lane l holds half of 16-byte chunk l/2
            const uint32_t chunk = lane >> 1;
            reinterpret_cast<uint2*>(a_lds)[2u * ((chunk >> 2) * 64u + (chunk & 3u) * 16u + r) +
                                            (lane & 1u)] = qv;
            if (lane == 0u) scale_lds[r] = scale;
            if (slice == 0u && r < rows) {
                reinterpret_cast<uint2*>(const_cast<int8_t*>(mid.q) +
                                         static_cast<size_t>(p0 + r) * I)[lane] = qv;
                if (lane == 0u) const_cast<float*>(mid.s)[p0 + r] = scale;
            }
        }
        __syncthreads();
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) row_scale[i] = scale_lds[4u * q + i];
    } else {
        // piece i: row i % 16, chunk i / 16 (consecutive lanes, consecutive
        // rows: the LDS stores fall in distinct banks)
        uint4 av[kStage];
#pragma unroll
        for (uint32_t u = 0; u < kStage; ++u) {
            const uint32_t i0 = threadIdx.x + u * kThreads;
            const uint32_t i = i0 < 16u * (I / 16u) ? i0 : 0u;
            const uint32_t r = i % 16u;
            av[u] = reinterpret_cast<const uint4*>(
                mid.q + static_cast<size_t>(p0 + (r < rows ? r : 0u)) * I)[i / 16u];
        }
#pragma unroll
        for (uint32_t kb = 0; kb < kHalf; ++kb) b[kb] = load_stream(wt + kb * 64u);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (uint32_t u = 0; u < kStage; ++u) {
            const uint32_t i = threadIdx.x + u * kThreads;
            if (i >= 16u * (I / 16u)) continue;
            const uint32_t chunk = i / 16u;
            a_lds[(chunk >> 2) * 64u + (chunk & 3u) * 16u + i % 16u] = av[u];
        }
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) {
            const uint32_t r = 4u * q + i;
            row_scale[i] = mid.s[p0 + (r < rows ? r : 0u)];
        }
        __syncthreads();
    }

    const v4i zero = {0, 0, 0, 0};
#pragma unroll
    for (uint32_t t = 0; t < kTilesPerWave; ++t) {
        const uint32_t tile = tile0 + t;
        const uint4* wtile = wt + static_cast<size_t>(t) * kBlocks * 64u;
        uint4 nb[kHalf];
#pragma unroll
        for (uint32_t kb = 0; kb < kHalf; ++kb) nb[kb] = load_stream(wtile + (kHalf + kb) * 64u);
        // the row's scale words, requested with the tile's weights and
        // widened where they are used: relaxed atomic loads stay here (a
        // plain load would be sunk to its use after the K loop, and its wait
        // would then also cover the next tile's weight requests)
        uint32_t gbits[kGroups];
#pragma unroll
        for (uint32_t g = 0; g < kGroups; ++g)
            gbits[g] = __hip_atomic_load(
                s + (static_cast<size_t>(e) * H + tile * 16u + n) * kGroups + g, __ATOMIC_RELAXED,
                __HIP_MEMORY_SCOPE_WORKGROUP);
        __builtin_amdgcn_sched_barrier(0);
        v4i acc = zero;
        float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        // K block kb of the tile: acc restarts at each group's first block
        // and, grouped, joins the chain at its last
        auto block = [&](uint32_t kb, uint4 bv) {
            acc = mfma_i8_16x16x64(as_v4i(a_lds[kb * 64u + lane]), as_v4i(bv),
                                   kb % kBlocksPerGroup == 0u ? zero : acc);
            if constexpr (!kPerChannel) {
                if (kb % kBlocksPerGroup == kBlocksPerGroup - 1u) {
                    const float gs = scale_to_f32(gbits[kb / kBlocksPerGroup], kBf16);
#pragma unroll
                    for (uint32_t i = 0; i < 4u; ++i)
                        y[i] = __builtin_fmaf(static_cast<float>(acc[i]), gs, y[i]);
                }
            }
        };
#pragma unroll
        for (uint32_t kb = 0; kb < kHalf; ++kb) block(kb, b[kb]);
        // next tile's first half (unrolled: the last tile issues none)
        if (t + 1u < kTilesPerWave) {
#pragma unroll
            for (uint32_t kb = 0; kb < kHalf; ++kb)
                b[kb] = load_stream(wtile + (kBlocks + kb) * 64u);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (uint32_t kb = 0; kb < kHalf; ++kb) block(kHalf + kb, nb[kb]);
        const float cs = scale_to_f32(gbits[0], kBf16);  // per channel: the one scale
        const uint32_t channel = tile * 16u + n;
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) {
            const uint32_t r = 4u * q + i;
            if (r >= rows) continue;
            const float o = kPerChannel ? (static_cast<float>(acc[i]) * cs) * row_scale[i]
                                        : y[i] * row_scale[i];
            out[static_cast<size_t>(p0 + r) * H + channel] = o;
        }
    }
    if constexpr (kAwait) {
        // the task's eighth down item: every item of the task is past its
        // wait, so nothing reads the flags any more
        if (wave == 0u && lane == 0u && ticket == 7u) {
#pragma unroll
            for (uint32_t i = 0; i < 8u; ++i) store_device(flags + i, 0u);
            store_device(counter, 0u);
        }
    }
}

template <uint32_t H, uint32_t I, uint32_t kWaves, uint32_t kTilesPerWave,
          uint32_t kBlocksPerGroup, bool kBf16, bool kQuantize>
__global__ __launch_bounds__(kWaves * 64) void down_w8_kernel(
    const uint4* __restrict__ w, const uint16_t* __restrict__ s, MidRows mid,
    const q38m_task_v1* __restrict__ tasks, float* __restrict__ out) {
    __shared__ uint4 a_lds[I / 64u * 64u];
    __shared__ float scale_lds[16];  // kQuantize: the rows' scales
    down_w8_item<H, I, kWaves, kTilesPerWave, kBlocksPerGroup, kBf16, kQuantize, false>(
        w, s, mid, read_task(tasks, blockIdx.y), blockIdx.x, out, a_lds, scale_lds, nullptr,
        nullptr, nullptr, nullptr);
}

// ---------------------------------------------------------------------------
// Gate/up (W4) and down (W8) of a slab in ONE launch of 8-wave workgroups,
// so that the down items start while the last gate/up items still stream
// instead of after the launch boundary (config-2 step 0.2199 -> 0.2163 ms,
// bit-identical).  Blocks [0, 8 * slots): gate/up items (task b / 8,
// channel slice b % 8; gate_up_w4_item with kPublish); blocks
// [8 * slots, 16 * slots): down items (task, 256 output channels;
// down_w8_item as 8 waves x 2 tiles, kQuantize and kAwait).  Block b runs
// on XCD b % 8, so both kinds keep their slice-to-XCD placement.
//
// The hand-off: a gate/up item stores its mid words device-coherently,
// waits for them, then sets flags[8 * task + slice]; a down item's wave 0
// polls the task's eight flags (device-coherent loads) while the first
// weights stream, and the item then reads the mid rows.  The flags and the
// per-task counters (flags[8 * slots + task]) are zero at the launch -- the
// step's plan kernel clears them, and every launch leaves them zero (the
// last down item of a task clears the task's words) -- unless a wait ran
// out.  Workgroups are dispatched in block order, so every gate/up item has
// been dispatched -- and, never waiting on anything, will finish -- before
// any down item polls.
// ---------------------------------------------------------------------------
struct GateUpDownArgs {
    const uint4* gate_up_w;
    const uint16_t* gate_up_s;
    const int8_t* xq;
    const float* xs;
    const uint32_t* packed;
    const float* route_weights;
    const q38m_task_v1* tasks;
    uint16_t* weighted_mid;
    const uint4* down_w;
    const uint16_t* down_s;
    int8_t* mid_q;
    float* mid_s;
    float* route_output;
    uint32_t* flags;   // [9 * slots]: 8 flags per task, then a counter per task
    uint32_t* status;  // Q38M_PLAN_STEP_TIMEOUT on a wait that ran out
    uint32_t slots;
};

template <uint32_t H, uint32_t I, uint32_t kSub, bool kGuBf16, uint32_t kDnBlocksPerGroup,
          bool kDnBf16>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(6, 8)))
void gate_up_down_kernel(GateUpDownArgs a) {
    constexpr uint32_t kWaves = 8u;
    constexpr uint32_t kGateUpLds = H / 32u * 64u * 8u + kWaves / 2u * 4u * 64u * 4u + 16u * 8u;
    constexpr uint32_t kDownLds = I / 64u * 64u * 16u + 16u * 4u + 4u;
    __shared__ __align__(16) uint8_t lds[kGateUpLds > kDownLds ? kGateUpLds : kDownLds];
    const uint32_t b = blockIdx.x;
    if (b < 8u * a.slots) {
        const uint32_t task = b >> 3, slice = b & 7u;
        gate_up_w4_item<H, I, kWaves, kSub, kGuBf16, true>(
            a.gate_up_w, a.gate_up_s, a.xq, a.xs, a.packed, a.route_weights,
            read_task(a.tasks, task), slice, a.weighted_mid, reinterpret_cast<uint2*>(lds),
            reinterpret_cast<float(*)[4][64]>(lds + H / 32u * 64u * 8u),
            reinterpret_cast<float2*>(lds + H / 32u * 64u * 8u + kWaves / 2u * 4u * 64u * 4u),
            a.flags + 8u * task + slice);
        return;
    }
    const uint32_t task = (b - 8u * a.slots) >> 3, slice = b & 7u;
    down_w8_item<H, I, kWaves, 2u, kDnBlocksPerGroup, kDnBf16, true, true>(
        a.down_w, a.down_s, MidRows{a.mid_q, a.mid_s, a.weighted_mid}, read_task(a.tasks, task),
        slice, a.route_output, reinterpret_cast<uint4*>(lds),
        reinterpret_cast<float*>(lds + I / 64u * 64u * 16u), a.flags + 8u * task,
        a.flags + 8u * a.slots + task, a.status,
        reinterpret_cast<uint32_t*>(lds + I / 64u * 64u * 16u + 16u * 4u));
}

__global__ __launch_bounds__(256) void clear_words_kernel(uint32_t* __restrict__ p,
                                                          uint32_t count) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < count) p[i] = 0u;
}

// ---------------------------------------------------------------------------
// Down, W4 in groups of 32, 64 or 128 columns (kSub sub-blocks of 32 per
// group; the all-W4 layer policy): the gate/up group chain over K = I, then
// * sm[r].  A workgroup covers 16 output tiles of one task: kWaves waves of
// kTilesPerWave tiles (8 x 2, or 16 x 1 for groups of 128, whose chain is
// light enough that more waves with one tile each stream faster); the
// task's 16 rows are staged once in LDS as int8 MFMA fragments (quantised
// there, kQuantize, 16 / kWaves rows per wave) and read from LDS by every
// MFMA, which keeps the waves small enough for 4-8 per SIMD.
// ---------------------------------------------------------------------------
template <uint32_t H, uint32_t I, uint32_t kTilesPerWave, uint32_t kSub, bool kBf16,
          bool kQuantize, uint32_t kWaves>
__global__ __launch_bounds__(kWaves * 64) void down_w4_kernel(
    const uint4* __restrict__ w, const uint16_t* __restrict__ s, MidRows mid,
    const q38m_task_v1* __restrict__ tasks, float* __restrict__ out) {
    constexpr uint32_t kQuads = I / 128u;
    constexpr uint32_t kTiles = H / 16u;
    constexpr uint32_t kRowScales = 4u / kSub;
    constexpr uint32_t kGroups = kQuads * 4u;  // 32-wide K groups
    static_assert(kWaves * kTilesPerWave == 16u && 16u % kWaves == 0u,
                  "16 tiles and 16 rows per workgroup");
    // the int8 rows in the MFMA A order, [group][lane] (lane n + 16q: row n,
    // columns 32g + 8q ..+7), and (kQuantize) the rows' scales
    __shared__ uint2 a_lds[kGroups * 64u];
    __shared__ float scale_lds[16];
    const TaskRecord task = read_task(tasks, blockIdx.y);
    const uint32_t rows = task.rows;
    if (rows == 0u) return;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t n = lane & 15u;
    const uint32_t q = lane >> 4;
    const uint32_t e = task.expert;
    const uint32_t p0 = task.begin;
    // quad-major layout: quad kq of tile t is unit (e*kQuads + kq)*kTiles + t;
    // a tile's four quads are requested together, one tile ahead, the first
    // tile's before the A rows are staged
    const uint32_t tile0 = (blockIdx.x * kWaves + wave) * kTilesPerWave;
    auto load_tile = [&](uint32_t t, uint4 (&b)[kQuads], uint2 (&c)[kQuads]) {
        const size_t unit = static_cast<size_t>(e) * kQuads * kTiles + tile0 + t;
#pragma unroll
        for (uint32_t kq = 0; kq < kQuads; ++kq) {
            b[kq] = load_stream(w + (unit + kq * kTiles) * 64u + lane);
            c[kq] = load_quad_scales<kSub>(s + ((unit + kq * kTiles) * 16u + n) * kRowScales);
        }
    };
    uint4 wb[kTilesPerWave][kQuads];
    uint2 wc[kTilesPerWave][kQuads];
    load_tile(0, wb[0], wc[0]);
    float row_scale[4];
    if constexpr (kQuantize) {
        static_assert(I == 512u, "one wave per 512-wide row");
        constexpr uint32_t kRowsPerWave = 16u / kWaves;
        uint4 mv[kRowsPerWave];
#pragma unroll
        for (uint32_t j = 0; j < kRowsPerWave; ++j) {
            const uint32_t r = wave * kRowsPerWave + j;
            mv[j] = reinterpret_cast<const uint4*>(
                mid.bf16 + static_cast<size_t>(p0 + (r < rows ? r : 0u)) * I)[lane];
        }
#pragma unroll
        for (uint32_t j = 0; j < kRowsPerWave; ++j) {
            const uint32_t r = wave * kRowsPerWave + j;
            float scale;
            const uint2 qv = quantize_mid_row(mv[j], scale);
            // lane l holds columns 8l..8l+7: group l/4, lane group l%4
            a_lds[(lane >> 2) * 64u + 16u * (lane & 3u) + r] = qv;
            if (lane == 0u) scale_lds[r] = scale;
            if (blockIdx.x == 0u && r < rows) {
                reinterpret_cast<uint2*>(const_cast<int8_t*>(mid.q) +
                                         static_cast<size_t>(p0 + r) * I)[lane] = qv;
                if (lane == 0u) const_cast<float*>(mid.s)[p0 + r] = scale;
            }
        }
        __syncthreads();
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) row_scale[i] = scale_lds[4u * q + i];
    } else {
        // row n, lane group q of every group, through LDS like the
        // quantising path
        if (wave == 0u) {
            const uint32_t a_row = n < rows ? n : 0u;
            const uint2* xa =
                reinterpret_cast<const uint2*>(mid.q + static_cast<size_t>(p0 + a_row) * I) + q;
#pragma unroll
            for (uint32_t g = 0; g < kGroups; ++g) a_lds[g * 64u + lane] = xa[g * 4u];
        }
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) {
            const uint32_t r = 4u * q + i;
            row_scale[i] = mid.s[p0 + (r < rows ? r : 0u)];
        }
        __syncthreads();
    }
    const v4i zero = {0, 0, 0, 0};
#pragma unroll
    for (uint32_t t = 0; t < kTilesPerWave; ++t) {
        if (t + 1u < kTilesPerWave) load_tile(t + 1u, wb[t + 1u], wc[t + 1u]);
        float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (uint32_t kq = 0; kq < kQuads; ++kq) {
            const uint32_t bw[4] = {wb[t][kq].x, wb[t][kq].y, wb[t][kq].z, wb[t][kq].w};
            v4i d = zero;
#pragma unroll
            for (uint32_t j = 0; j < 4u; ++j) {
                d = mfma_i8_16x16x32(as_long(a_lds[(kq * 4u + j) * 64u + lane]), unpack_w4x16(bw[j]), j % kSub == 0u ? zero : d);
                if (j % kSub != kSub - 1u) continue;
                const float scale =
                    scale_to_f32(quad_scale_word(wc[t][kq], j / kSub), kBf16) * 0.0625f;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    y[i] = __builtin_fmaf(static_cast<float>(d[i]), scale, y[i]);
            }
        }
        const uint32_t channel = (tile0 + t) * 16u + n;
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) {
            const uint32_t r = 4u * q + i;
            if (r >= rows) continue;
            out[static_cast<size_t>(p0 + r) * H + channel] = y[i] * row_scale[i];
        }
    }
}

// ---------------------------------------------------------------------------
// Fixed rank-order reduce from 0.0f plus the optional gated shared term
// (q38_moe_prefill.cu:601-631), added as fma(shared, multiplier, routed): the
// contraction nvcc's default -fmad applies to the reference expression.
// One workgroup per token; thread t sums columns 4t..4t+3 of each 1024-column
// half, so every load instruction reads 1 KB of whole 128-byte lines.
// kStream: the route outputs are read with non-temporal loads (for route
// outputs larger than the memory-side cache, read once from HBM).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float4 load_f4(const float* p, std::true_type) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    const f4v v = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 load_f4(const float* p, std::false_type) {
    return *reinterpret_cast<const float4*>(p);
}

template <uint32_t H, bool kStream>
__global__ __launch_bounds__(256) void combine_kernel(
    const float* __restrict__ route_output, const uint32_t* __restrict__ inverse,
    const uint16_t* __restrict__ shared_output, const uint16_t* __restrict__ shared_gate,
    uint16_t* __restrict__ output) {
    static_assert(H == 2u * 1024u, "two 1024-column halves, four columns per thread");
    const uint32_t token = blockIdx.x;
    const bool shared = shared_output != nullptr && shared_gate != nullptr;
    float multiplier = 0.0f;
    if (shared) {
        const float g = bf16_to_f32(shared_gate[token]);
        multiplier = 1.0f / (1.0f + exp_q(-g));
    }
    uint32_t rows[kTopK];
#pragma unroll
    for (uint32_t r = 0; r < kTopK; ++r)
        rows[r] = checked(inverse[token * kTopK + r], gridDim.x * kTopK, kCheckRoute);
    const uint32_t c = 4u * threadIdx.x;
    float acc[2][4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
    for (uint32_t r = 0; r < kTopK; ++r) {
        const float* row = route_output + static_cast<size_t>(rows[r]) * H + c;
#pragma unroll
        for (uint32_t h = 0; h < 2u; ++h) {
            const float4 v = load_f4(row + 1024u * h, std::integral_constant<bool, kStream>{});
            acc[h][0] += v.x; acc[h][1] += v.y; acc[h][2] += v.z; acc[h][3] += v.w;
        }
    }
#pragma unroll
    for (uint32_t h = 0; h < 2u; ++h) {
        const uint32_t col = c + 1024u * h;
        if (shared) {
            const uint2 sv = *reinterpret_cast<const uint2*>(
                shared_output + static_cast<size_t>(token) * H + col);
            const uint32_t sw[2] = {sv.x, sv.y};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t bits = (i & 1) ? (sw[i >> 1] >> 16) : (sw[i >> 1] & 0xffffu);
                acc[h][i] = __builtin_fmaf(bf16_to_f32(bits), multiplier, acc[h][i]);
            }
        }
        uint2 packed;
        packed.x = f32_to_bf16(acc[h][0]) | (f32_to_bf16(acc[h][1]) << 16);
        packed.y = f32_to_bf16(acc[h][2]) | (f32_to_bf16(acc[h][3]) << 16);
        *reinterpret_cast<uint2*>(output + static_cast<size_t>(token) * H + col) = packed;
    }
}

// Decode combine: routed + shared * sigmoid(gate) (q38_moe.cu:337-350), the
// sum contracted into one fma as nvcc builds the reference expression.
template <uint32_t H>
__global__ __launch_bounds__(256) void combine_shared_kernel(
    const uint16_t* __restrict__ routed, const uint16_t* __restrict__ shared,
    const uint16_t* __restrict__ gate, uint16_t* __restrict__ output, uint64_t elements) {
    const uint64_t index = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (index >= elements) return;
    const float g = bf16_to_f32(gate[index / H]);
    const float sigmoid = 1.0f / (1.0f + exp_q(-g));
    output[index] = static_cast<uint16_t>(
        f32_to_bf16(__builtin_fmaf(bf16_to_f32(shared[index]), sigmoid, bf16_to_f32(routed[index]))));
}

}  // namespace

namespace {

template <uint32_t kSub>
void launch_gate_up_sub(const q38m_expert_weights_v1& w, const int8_t* xq, const float* xs,
                        const uint32_t* packed, const float* route_weights,
                        const q38m_task_v1* tasks, uint32_t task_count, uint16_t* weighted_mid,
                        hipStream_t stream) {
    constexpr uint32_t kWaves = 8;
    const dim3 grid(kInter / 16u / (kWaves / 2u), task_count);
    const auto* data = static_cast<const uint4*>(w.data);
    const auto* scales = static_cast<const uint16_t*>(w.scales);
    if (w.scale_dtype == Q38M_SCALE_BF16)
        gate_up_w4_kernel<kHidden, kInter, kWaves, kSub, true><<<grid, kWaves * 64u, 0, stream>>>(
            data, scales, xq, xs, packed, route_weights, tasks, weighted_mid);
    else
        gate_up_w4_kernel<kHidden, kInter, kWaves, kSub, false><<<grid, kWaves * 64u, 0, stream>>>(
            data, scales, xq, xs, packed, route_weights, tasks, weighted_mid);
}

template <uint32_t kBlocksPerGroup>
void launch_gate_up_w8_groups(const q38m_expert_weights_v1& w, const int8_t* xq, const float* xs,
                              const uint32_t* packed, const float* route_weights,
                              const q38m_task_v1* tasks, uint32_t task_count,
                              uint16_t* weighted_mid, hipStream_t stream) {
    constexpr uint32_t kWaves = 8;
    const dim3 grid(kInter / 16u / (kWaves / 2u), task_count);
    const auto* data = static_cast<const uint4*>(w.data);
    const auto* scales = static_cast<const uint16_t*>(w.scales);
    if (w.scale_dtype == Q38M_SCALE_BF16)
        gate_up_w8_kernel<kHidden, kInter, kWaves, kBlocksPerGroup, true>
            <<<grid, kWaves * 64u, 0, stream>>>(data, scales, xq, xs, packed, route_weights, tasks,
                                                weighted_mid);
    else
        gate_up_w8_kernel<kHidden, kInter, kWaves, kBlocksPerGroup, false>
            <<<grid, kWaves * 64u, 0, stream>>>(data, scales, xq, xs, packed, route_weights, tasks,
                                                weighted_mid);
}

template <uint32_t kBlocksPerGroup, bool kQuantize>
void launch_down_w8_groups(const q38m_expert_weights_v1& w, const MidRows& mid,
                           const q38m_task_v1* tasks, uint32_t task_count,
                           float* route_output, hipStream_t stream) {
    // 16 waves of one tile each (8 waves x 2 tiles: config-2 step 0.2215
    // -> 0.2202 ms with this shape)
    constexpr uint32_t kWaves = 16, kTilesPerWave = 1;
    const dim3 grid(kHidden / 16u / (kWaves * kTilesPerWave), task_count);
    const auto* data = static_cast<const uint4*>(w.data);
    const auto* scales = static_cast<const uint16_t*>(w.scales);
    if (w.scale_dtype == Q38M_SCALE_BF16)
        down_w8_kernel<kHidden, kInter, kWaves, kTilesPerWave, kBlocksPerGroup, true, kQuantize>
            <<<grid, kWaves * 64u, 0, stream>>>(data, scales, mid, tasks, route_output);
    else
        down_w8_kernel<kHidden, kInter, kWaves, kTilesPerWave, kBlocksPerGroup, false, kQuantize>
            <<<grid, kWaves * 64u, 0, stream>>>(data, scales, mid, tasks, route_output);
}

template <uint32_t kSub, bool kQuantize>
void launch_down_w4_sub(const q38m_expert_weights_v1& w, const MidRows& mid,
                        const q38m_task_v1* tasks, uint32_t task_count,
                        float* route_output, hipStream_t stream) {
    // groups of 128: 16 waves x 1 tile (interior reference format, slab
    // step 0.1818 -> 0.1759 ms); 32 and 64: 8 waves x 2 tiles
    constexpr uint32_t kWaves = kSub == 4u ? 16u : 8u;
    constexpr uint32_t kTilesPerWave = 16u / kWaves;
    const dim3 grid(kHidden / 16u / 16u, task_count);
    const auto* data = static_cast<const uint4*>(w.data);
    const auto* scales = static_cast<const uint16_t*>(w.scales);
    if (w.scale_dtype == Q38M_SCALE_BF16)
        down_w4_kernel<kHidden, kInter, kTilesPerWave, kSub, true, kQuantize, kWaves>
            <<<grid, kWaves * 64u, 0, stream>>>(data, scales, mid, tasks, route_output);
    else
        down_w4_kernel<kHidden, kInter, kTilesPerWave, kSub, false, kQuantize, kWaves>
            <<<grid, kWaves * 64u, 0, stream>>>(data, scales, mid, tasks, route_output);
}

template <bool kQuantize>
hipError_t launch_down_rows(const q38m_expert_weights_v1& w, const MidRows& mid,
                            const q38m_task_v1* tasks, uint32_t task_count,
                            float* route_output, hipStream_t stream) {
    constexpr uint32_t kBlocks = kInter / 64u;
    if (w.format == Q38M_FORMAT_W8_SYM) {
        switch (w.group_size) {
            case 0u: launch_down_w8_groups<kBlocks, kQuantize>(w, mid, tasks, task_count,
                                                               route_output, stream); break;
            case 64u: launch_down_w8_groups<1, kQuantize>(w, mid, tasks, task_count,
                                                          route_output, stream); break;
            case 128u: launch_down_w8_groups<2, kQuantize>(w, mid, tasks, task_count,
                                                           route_output, stream); break;
            default: return hipErrorInvalidValue;
        }
    } else {
        switch (w.group_size) {
            case 32u: launch_down_w4_sub<1, kQuantize>(w, mid, tasks, task_count, route_output,
                                                       stream); break;
            case 64u: launch_down_w4_sub<2, kQuantize>(w, mid, tasks, task_count, route_output,
                                                       stream); break;
            case 128u: launch_down_w4_sub<4, kQuantize>(w, mid, tasks, task_count, route_output,
                                                        stream); break;
            default: return hipErrorInvalidValue;
        }
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gate_up(const q38m_expert_weights_v1& w, const int8_t* xq, const float* xs,
                          const uint32_t* packed, const float* route_weights,
                          const q38m_task_v1* tasks, uint32_t task_count, uint16_t* weighted_mid,
                          hipStream_t stream) {
    if (w.format == Q38M_FORMAT_W8_SYM) {
        constexpr uint32_t kBlocks = kHidden / 64u;
        switch (w.group_size) {
            case 0u: launch_gate_up_w8_groups<kBlocks>(w, xq, xs, packed, route_weights, tasks,
                                                       task_count, weighted_mid, stream); break;
            case 64u: launch_gate_up_w8_groups<1>(w, xq, xs, packed, route_weights, tasks,
                                                  task_count, weighted_mid, stream); break;
            case 128u: launch_gate_up_w8_groups<2>(w, xq, xs, packed, route_weights, tasks,
                                                   task_count, weighted_mid, stream); break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    switch (w.group_size) {
        case 32u: launch_gate_up_sub<1>(w, xq, xs, packed, route_weights, tasks, task_count,
                                        weighted_mid, stream); break;
        case 64u: launch_gate_up_sub<2>(w, xq, xs, packed, route_weights, tasks, task_count,
                                        weighted_mid, stream); break;
        case 128u: launch_gate_up_sub<4>(w, xq, xs, packed, route_weights, tasks, task_count,
                                         weighted_mid, stream); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// W4 gate/up with per-channel W8 down, one scale dtype: at <= 64 VGPRs the
// fused kernel keeps the gate/up kernel's four workgroups per CU (the
// grouped W8 down items take 69-80)
bool gate_up_down_fusable(const q38m_expert_weights_v1& gate_up,
                          const q38m_expert_weights_v1& down) {
    const bool gu = gate_up.format == Q38M_FORMAT_W4_SYM &&
                    (gate_up.group_size == 32u || gate_up.group_size == 64u ||
                     gate_up.group_size == 128u);
    const bool dn = down.format == Q38M_FORMAT_W8_SYM && down.group_size == 0u;
    return gu && dn && gate_up.scale_dtype == down.scale_dtype;
}

namespace {

template <uint32_t kSub, bool kGuBf16, uint32_t kDnBlocksPerGroup, bool kDnBf16>
void launch_gate_up_down_as(const GateUpDownArgs& a, hipStream_t stream) {
    gate_up_down_kernel<kHidden, kInter, kSub, kGuBf16, kDnBlocksPerGroup, kDnBf16>
        <<<16u * a.slots, 512, 0, stream>>>(a);
}

// one scale dtype for both projections, per-channel down (gate_up_down_fusable)
template <uint32_t kSub>
void launch_gate_up_down_gu(const q38m_expert_weights_v1& gate_up, const GateUpDownArgs& a,
                            hipStream_t stream) {
    constexpr uint32_t kBlocks = kInter / 64u;
    if (gate_up.scale_dtype == Q38M_SCALE_BF16)
        launch_gate_up_down_as<kSub, true, kBlocks, true>(a, stream);
    else
        launch_gate_up_down_as<kSub, false, kBlocks, false>(a, stream);
}

}  // namespace

hipError_t launch_gate_up_down(const q38m_expert_weights_v1& gate_up,
                               const q38m_expert_weights_v1& down, const int8_t* xq,
                               const float* xs, const uint32_t* packed,
                               const float* route_weights, const q38m_task_v1* tasks,
                               uint32_t task_count, uint16_t* weighted_mid, int8_t* mid_q,
                               float* mid_s, float* route_output, uint32_t* task_flags,
                               uint32_t* status, hipStream_t stream) {
    if (!gate_up_down_fusable(gate_up, down)) {
        hipError_t rc = launch_gate_up(gate_up, xq, xs, packed, route_weights, tasks, task_count,
                                       weighted_mid, stream);
        if (rc == hipSuccess)
            rc = launch_down_quantize(down, weighted_mid, mid_q, mid_s, tasks, task_count,
                                      route_output, stream);
        return rc;
    }
    const GateUpDownArgs a{static_cast<const uint4*>(gate_up.data),
                           static_cast<const uint16_t*>(gate_up.scales),
                           xq, xs, packed, route_weights, tasks, weighted_mid,
                           static_cast<const uint4*>(down.data),
                           static_cast<const uint16_t*>(down.scales),
                           mid_q, mid_s, route_output, task_flags, status, task_count};
    switch (gate_up.group_size) {
        case 32u: launch_gate_up_down_gu<1>(gate_up, a, stream); break;
        case 64u: launch_gate_up_down_gu<2>(gate_up, a, stream); break;
        default: launch_gate_up_down_gu<4>(gate_up, a, stream); break;
    }
    return hipGetLastError();
}

hipError_t launch_clear_words(uint32_t* words, uint32_t count, hipStream_t stream) {
    clear_words_kernel<<<(count + 255u) / 256u, 256, 0, stream>>>(words, count);
    return hipGetLastError();
}

hipError_t launch_down(const q38m_expert_weights_v1& w, const int8_t* mid_q, const float* mid_s,
                       const q38m_task_v1* tasks, uint32_t task_count, float* route_output,
                       hipStream_t stream) {
    return launch_down_rows<false>(w, MidRows{mid_q, mid_s, nullptr}, tasks, task_count,
                                   route_output, stream);
}

hipError_t launch_down_quantize(const q38m_expert_weights_v1& w, const uint16_t* weighted_mid,
                                int8_t* mid_q, float* mid_s, const q38m_task_v1* tasks,
                                uint32_t task_count, float* route_output, hipStream_t stream) {
    return launch_down_rows<true>(w, MidRows{mid_q, mid_s, weighted_mid}, tasks, task_count,
                                  route_output, stream);
}

hipError_t launch_combine(const float* route_output, const uint32_t* inverse,
                          const uint16_t* shared_output, const uint16_t* shared_gate,
                          uint32_t tokens, uint16_t* output, hipStream_t stream) {
    // route outputs beyond the 256 MB memory-side cache (a chunk's: 80 KB per
    // token) are read once from HBM, with non-temporal loads (config-5 layer:
    // 523 -> 480 us); a slab's were just written and are read through the caches
    constexpr size_t kCachedRouteBytes = size_t(256) << 20;
    const size_t bytes = static_cast<size_t>(tokens) * kTopK * kHidden * sizeof(float);
    if (bytes > kCachedRouteBytes)
        combine_kernel<kHidden, true><<<tokens, 256, 0, stream>>>(route_output, inverse,
                                                                  shared_output, shared_gate,
                                                                  output);
    else
        combine_kernel<kHidden, false><<<tokens, 256, 0, stream>>>(route_output, inverse,
                                                                   shared_output, shared_gate,
                                                                   output);
    return hipGetLastError();
}

hipError_t launch_combine_shared(const uint16_t* routed, const uint16_t* shared,
                                 const uint16_t* gate, uint16_t* output,
                                 uint32_t tokens, hipStream_t stream) {
    const uint64_t elements = static_cast<uint64_t>(tokens) * kHidden;
    combine_shared_kernel<kHidden><<<static_cast<uint32_t>((elements + 255u) / 256u), 256, 0,
                                     stream>>>(routed, shared, gate, output, elements);
    return hipGetLastError();
}

}  // namespace q38m
