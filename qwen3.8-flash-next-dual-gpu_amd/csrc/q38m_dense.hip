// Dense bf16 GEMMs of the MoE block on either side of the routed experts:
// the router (cuda_backend.cu:1518-1519, cuda_gemv_bf16 over the
// "preserved" bf16 router, tools/q38_quant_policy.py:205) and the shared
// expert (cuda_backend.cu:1573-1590: gate and up projections, SiLU
// multiply, down projection, the scalar output gate).
//
// C[M][N] = A[M][K] * B[N][K]^T: both operands keep K contiguous (the
// activation rows and the weight matrices' [out][in] rows), bf16 in, fp32
// accumulation on v_mfma_f32_16x16x32_bf16, fp32 or bf16 (round to nearest
// even) out.  These are floating-point results: their parity with a CPU
// restatement is a stated tolerance (the MFMA's internal summation order is
// not specified), unlike the integer expert GEMMs.  The order of the
// partial sums is fixed, so a launch's results are the same on every run.
#include "q38m_device.h"
#include "q38m_internal.h"
#include "q38m_select.h"

namespace q38m {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// u32x4 (q38m_select.h): 16 bytes as a native vector, so loads and stores
// of it stay plain vector moves (a HIP_vector_type copy is a memcpy the
// compiler may keep in scratch memory)

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

constexpr uint32_t kDenseWaves = 4;
// the 64 x 64 workgroup tile serves K up to this and grids of at least
// this many tiles
constexpr uint32_t kTile64MaxK = 1024;
constexpr uint32_t kTile64MinTiles = 192;

// Operands reach the MFMAs through a per-wave LDS slab.  A wave's panels
// (16 rows each: its A panels, then its B panels) are stacked into one list
// of rows; staging instruction i loads rows 8i .. 8i+7 of that list, lane l
// reading row 8i + l/8 at the 16-byte chunk l%8 of the current 64-wide K
// chunk, so each instruction reads eight whole 128-byte lines.  (Loading
// the MFMA layout straight from memory -- lane l at row l%16 -- reads
// sixteen half lines per instruction and runs at a third of the rate from
// L2.)  In LDS, row r keeps its chunk c in slot c ^ (r%8): both the row
// writes and the MFMA-layout reads (eight rows, one chunk) fall in distinct
// banks.

// Lane pointer of staging instruction `half` (0/1) of the 16-row panel at
// `row`: row row + 8 half + l/8 (clamped to the last row, never stored),
// column 8 (l%8).
__device__ __forceinline__ const u32x4* stage_ptr(const uint16_t* base, uint32_t row,
                                                  uint32_t rows, uint32_t k, uint32_t half,
                                                  uint32_t lane) {
    const uint32_t r = min(row + 8u * half + (lane >> 3), rows - 1u);
    return reinterpret_cast<const u32x4*>(base + static_cast<size_t>(r) * k + (lane & 7u) * 8u);
}

// One wave's partial products over 32-wide K steps [s0, s1) for kTM A
// panels against kNB x kTN B panels; ga[2p + half] are the panel p staging
// pointers (p < kTM: A panel p; then B panel (v, j) at kTM + v kTN + j).
// Steps go in pairs (one 64-wide chunk, a half chunk at an odd end); two
// chunks are in flight in registers while the wave multiplies the one in
// its slab.  The slab is private to the wave and a wave's LDS operations
// complete in program order, so no barrier is needed.  Each accumulator
// receives its K steps in increasing order, lane l contributing
// k = 32 s + 8 (l/16) .. +7 of step s.
//
// With kGate, the wave also multiplies its A panels by one extra B row
// (`gate`, the lane's pointer at k = 8 (l/16) of that row) into
// acc_gate[i]: the row rides in the MFMA B operand of lanes l%16 == 0 and
// the other fifteen columns are zero, so column 0 of acc_gate holds the dot
// products, summed exactly as in a 16-row panel.
template <uint32_t kTM, uint32_t kTN, uint32_t kNB, bool kGate = false>
__device__ __forceinline__ void wave_partial(const u32x4* const (&ga)[2 * (kTM + kNB * kTN)],
                                             u32x4* slab, uint32_t lane, uint32_t s0,
                                             uint32_t s1, f32x4 (&acc)[kNB][kTM][kTN],
                                             const u32x4* gate = nullptr,
                                             f32x4* acc_gate = nullptr) {
    constexpr uint32_t kL = 2u * (kTM + kNB * kTN);
    struct Chunk {
        u32x4 v[kL];
        u32x4 g[kGate ? 2 : 1];  // the gate row's two steps
    };
    const bool gate_lane = (lane & 15u) == 0u;
    const uint32_t write_at = 8u * (lane >> 3) + ((lane & 7u) ^ (lane >> 3));
    const uint32_t read_at = 8u * (lane & 15u);
    const uint32_t read_slot[2] = {(lane >> 4) ^ (lane & 7u), (4u + (lane >> 4)) ^ (lane & 7u)};
    const uint32_t chunks = (s1 - s0 + 1u) / 2u;
    // At a half chunk, lanes l%8 >= 4 load their row's first half again
    // instead of the next step (which may lie past the matrix): every lane
    // loads, so the loads stay outside divergent control flow, and the
    // duplicated slots are never read.
    // (ga[i] points at the lane's 16 bytes l%8 of its row, so stepping back
    // four vectors from step s stays within the row)
    const uint32_t back = (lane & 7u) < 4u ? 0u : 4u;
    auto load = [&](Chunk& x, uint32_t c) __attribute__((always_inline)) {
        const uint32_t s = s0 + 2u * c;
        const bool whole = s + 1u < s1;  // uniform: both steps lie in the range
        const size_t shift = whole ? 0u : back;
#pragma unroll
        for (uint32_t i = 0; i < kL; ++i) x.v[i] = *(ga[i] + 4u * s - shift);
        if constexpr (kGate) {
            x.g[0] = gate[4u * s];
            x.g[1] = gate[4u * (whole ? s + 1u : s)];
        }
    };
    u32x4 staged_gate[2];
    auto stage = [&](const Chunk& x) __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t i = 0; i < kL; ++i) slab[64u * i + write_at] = x.v[i];
        if constexpr (kGate) {
            const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
            for (uint32_t h = 0; h < 2u; ++h) staged_gate[h] = gate_lane ? x.g[h] : zero;
        }
    };
    // the MFMAs of the staged chunk over `steps` (1 or 2) K steps
    auto multiply = [&](uint32_t steps) __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t h = 0; h < 2u; ++h) {
            if (h >= steps) break;
            u32x4 a[kTM], b[kNB][kTN];
#pragma unroll
            for (uint32_t i = 0; i < kTM; ++i) a[i] = slab[128u * i + read_at + read_slot[h]];
#pragma unroll
            for (uint32_t v = 0; v < kNB; ++v)
#pragma unroll
                for (uint32_t j = 0; j < kTN; ++j)
                    b[v][j] = slab[128u * (kTM + v * kTN + j) + read_at + read_slot[h]];
#pragma unroll
            for (uint32_t v = 0; v < kNB; ++v)
#pragma unroll
                for (uint32_t i = 0; i < kTM; ++i)
#pragma unroll
                    for (uint32_t j = 0; j < kTN; ++j)
                        acc[v][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            as_bf16x8(a[i]), as_bf16x8(b[v][j]), acc[v][i][j], 0, 0, 0);
            if constexpr (kGate) {
#pragma unroll
                for (uint32_t i = 0; i < kTM; ++i)
                    acc_gate[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        as_bf16x8(a[i]), as_bf16x8(staged_gate[h]), acc_gate[i], 0, 0, 0);
            }
        }
    };
    if (chunks == 0u) return;
    const uint32_t last_steps = s1 - s0 - 2u * (chunks - 1u);  // 1 or 2
    Chunk x0, x1;
    load(x0, 0u);
    if (chunks == 1u) {
        stage(x0);
        multiply(last_steps);
        return;
    }
    load(x1, 1u);
    // steady state: every load in the loop is taken, so the wait for a
    // chunk leaves the next chunk's loads in flight
    uint32_t c = 0;
    for (; c + 3u < chunks; c += 2u) {
        stage(x0);
        load(x0, c + 2u);
        // keep the scheduler from sinking the loads below the next stage
        __builtin_amdgcn_sched_barrier(0);
        multiply(2u);
        stage(x1);
        load(x1, c + 3u);
        __builtin_amdgcn_sched_barrier(0);
        multiply(2u);
    }
    // two or three chunks left; only the last may be a half chunk
    if (chunks - c == 3u) {
        stage(x0);
        load(x0, c + 2u);
        __builtin_amdgcn_sched_barrier(0);
        multiply(2u);
        stage(x1);
        multiply(2u);
        stage(x0);
        multiply(last_steps);
    } else {
        stage(x0);
        multiply(2u);
        stage(x1);
        multiply(last_steps);
    }
}

// The four waves of a block split K; their partial tiles meet in LDS and
// are summed in wave order (((w0 + w1) + w2) + w3), the same for every
// launch.  acc holds kTiles tiles as kTiles / per_b groups of per_b (one
// group per B matrix); wave w finishes output tiles o = w, w + 4, ... of
// every group, calling finish(o, group, sum).
template <uint32_t kTiles, uint32_t kPerB, typename Finish>
__device__ __forceinline__ void reduce_waves(f32x4* lds, const f32x4* acc, uint32_t wave,
                                             uint32_t lane, Finish finish) {
#pragma unroll
    for (uint32_t t = 0; t < kTiles; ++t) lds[(wave * kTiles + t) * 64u + lane] = acc[t];
    __syncthreads();
#pragma unroll
    for (uint32_t o = 0; o < kPerB; ++o) {
        if (o % kDenseWaves != wave) continue;
#pragma unroll
        for (uint32_t v = 0; v < kTiles / kPerB; ++v) {
            const uint32_t t = v * kPerB + o;
            f32x4 sum = lds[t * 64u + lane];
#pragma unroll
            for (uint32_t w = 1; w < kDenseWaves; ++w) sum += lds[(w * kTiles + t) * 64u + lane];
            finish(o, v, sum);
        }
    }
}

// Output of the dense GEMM: fp32, bf16, or bf16 through the hyper-connection
// elementwise step applied to the bf16-rounded product v
// (q38_hyper.cu:87-97): bf16(silu(v / divisor) * scale) or
// bf16(sigmoid(v / divisor) * scale), sigmoid(x) = 1 / (1 + exp(-x)).
enum class DenseOut { kF32, kBf16, kBf16Silu, kBf16Sigmoid };

__device__ __forceinline__ uint32_t dense_epilogue(DenseOut mode, float acc, float divisor,
                                                   float scale) {
    if (mode == DenseOut::kBf16) return f32_to_bf16(acc);
    const float v = bf16_round(acc) / divisor;
    const float sigmoid = 1.0f / (1.0f + exp_q(-v));
    return f32_to_bf16((mode == DenseOut::kBf16Silu ? v * sigmoid : sigmoid) * scale);
}

// C[M][N] = A[M][K] * B[N][K]^T for a (16 kTM) x (16 kTN) tile of C per
// workgroup of four waves that split K.  The D layout of each 16 x 16 MFMA
// tile: lane l holds rows 4*(l/16) + e, e = 0..3, of column l%16.
template <uint32_t kTM, uint32_t kTN, DenseOut kOut>
__global__ __launch_bounds__(256) void dense_gemm_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, uint32_t m, uint32_t n,
    uint32_t k, float* __restrict__ c_f32, uint16_t* __restrict__ c_bf16, float divisor,
    float scale) {
    constexpr uint32_t kL = 2u * (kTM + kTN);
    __shared__ u32x4 slab[kDenseWaves * kL * 64];
    __shared__ f32x4 lds[kDenseWaves * kTM * kTN * 64];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t m0 = blockIdx.y * 16u * kTM;
    const uint32_t n0 = blockIdx.x * 16u * kTN;
    const u32x4* ga[kL];
#pragma unroll
    for (uint32_t h = 0; h < 2u; ++h) {
#pragma unroll
        for (uint32_t i = 0; i < kTM; ++i) ga[2u * i + h] = stage_ptr(a, m0 + 16u * i, m, k, h, lane);
#pragma unroll
        for (uint32_t j = 0; j < kTN; ++j)
            ga[2u * (kTM + j) + h] = stage_ptr(b, n0 + 16u * j, n, k, h, lane);
    }
    f32x4 acc[1][kTM][kTN];
#pragma unroll
    for (uint32_t i = 0; i < kTM; ++i)
#pragma unroll
        for (uint32_t j = 0; j < kTN; ++j) acc[0][i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t steps = k / 32u;
    wave_partial<kTM, kTN, 1>(ga, slab + wave * kL * 64u, lane, wave * steps / kDenseWaves,
                              (wave + 1u) * steps / kDenseWaves, acc);
    reduce_waves<kTM * kTN, kTM * kTN>(lds, &acc[0][0][0], wave, lane,
                                       [&](uint32_t o, uint32_t, f32x4 sum) {
        const uint32_t col = n0 + 16u * (o % kTN) + (lane & 15u);
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) {
            const uint32_t row = m0 + 16u * (o / kTN) + 4u * (lane >> 4) + e;
            if (row >= m || col >= n) continue;
            const size_t at = static_cast<size_t>(row) * n + col;
            if constexpr (kOut == DenseOut::kF32)
                c_f32[at] = sum[e];
            else
                c_bf16[at] = static_cast<uint16_t>(dense_epilogue(kOut, sum[e], divisor, scale));
        }
    });
}

// C[M][N] = A[M][K] * B[N][K]^T for a 64 x 64 tile of C per workgroup, for
// short K (the products whose grid of 64 x 64 tiles fills the GPU): the
// four waves share each 64-wide K chunk of the tile's 64 A rows and 64 B
// rows (16 KB, four whole-line loads per thread) in a double-buffered LDS
// stage, and wave w multiplies its 32 x 32 quarter (rows 32 (w/2), columns
// 32 (w%2)) over all of K, the K steps in increasing order.  Two chunks are
// in flight in registers; the barriers wait for LDS only.
template <DenseOut kOut>
__global__ __launch_bounds__(256) void dense_tile64_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, uint32_t m, uint32_t n,
    uint32_t k, float* __restrict__ c_f32, uint16_t* __restrict__ c_bf16, float divisor,
    float scale) {
    constexpr uint32_t kRows = 128;  // 64 A rows, then 64 B rows
    __shared__ u32x4 stage_lds[2][kRows * 8];
    const uint32_t t = threadIdx.x;
    const uint32_t lane = t & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t m0 = blockIdx.y * 64u, n0 = blockIdx.x * 64u;
    // staging instruction i: stacked row 32 i + t/8, 16-byte chunk t%8,
    // kept in slot (t%8) ^ (row%8)
    const u32x4* gp[4];
#pragma unroll
    for (uint32_t i = 0; i < 4u; ++i) {
        const uint32_t row = 32u * i + (t >> 3);
        const uint16_t* base = row < 64u ? a + static_cast<size_t>(min(m0 + row, m - 1u)) * k
                                         : b + static_cast<size_t>(min(n0 + row - 64u, n - 1u)) * k;
        gp[i] = reinterpret_cast<const u32x4*>(base + (t & 7u) * 8u);
    }
    const uint32_t write_at = 8u * (t >> 3) + ((t & 7u) ^ ((t >> 3) & 7u));
    const uint32_t read_at = 8u * (lane & 15u);
    const uint32_t read_slot[2] = {(lane >> 4) ^ (lane & 7u), (4u + (lane >> 4)) ^ (lane & 7u)};
    const uint32_t a_row = 32u * (wave >> 1), b_row = 64u + 32u * (wave & 1u);
    const uint32_t steps = k / 32u;
    const uint32_t chunks = (steps + 1u) / 2u;
    const uint32_t last_steps = steps - 2u * (chunks - 1u);
    const size_t back = (t & 7u) < 4u ? 0u : 4u;
    struct Chunk {
        u32x4 v[4];
    };
    auto load = [&](Chunk& x, uint32_t c) __attribute__((always_inline)) {
        const uint32_t s = 2u * c;
        const size_t shift = s + 1u < steps ? 0u : back;  // a half chunk re-reads its step
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) x.v[i] = *(gp[i] + 4u * s - shift);
    };
    auto stage = [&](const Chunk& x, uint32_t slot) __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) stage_lds[slot][256u * i + write_at] = x.v[i];
    };
    auto lds_barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
    f32x4 acc[2][2];
#pragma unroll
    for (uint32_t i = 0; i < 2u; ++i)
#pragma unroll
        for (uint32_t j = 0; j < 2u; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    auto multiply = [&](uint32_t slot, uint32_t count) __attribute__((always_inline)) {
        const u32x4* lds = stage_lds[slot];
#pragma unroll
        for (uint32_t h = 0; h < 2u; ++h) {
            if (h >= count) break;
            u32x4 av[2], bv[2];
#pragma unroll
            for (uint32_t i = 0; i < 2u; ++i) {
                av[i] = lds[8u * (a_row + 16u * i) + read_at + read_slot[h]];
                bv[i] = lds[8u * (b_row + 16u * i) + read_at + read_slot[h]];
            }
#pragma unroll
            for (uint32_t i = 0; i < 2u; ++i)
#pragma unroll
                for (uint32_t j = 0; j < 2u; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        as_bf16x8(av[i]), as_bf16x8(bv[j]), acc[i][j], 0, 0, 0);
        }
    };
    Chunk x0, x1;
    load(x0, 0u);
    if (chunks == 1u) {
        stage(x0, 0u);
        lds_barrier();
        multiply(0u, last_steps);
    } else {
        load(x1, 1u);
        stage(x0, 0u);
        lds_barrier();
        // at the top of each pass: chunk c in slot 0, chunk c + 1 in flight in x1
        uint32_t c = 0;
        for (; c + 3u < chunks; c += 2u) {
            load(x0, c + 2u);
            __builtin_amdgcn_sched_barrier(0);
            multiply(0u, 2u);
            stage(x1, 1u);
            lds_barrier();
            load(x1, c + 3u);
            __builtin_amdgcn_sched_barrier(0);
            multiply(1u, 2u);
            stage(x0, 0u);
            lds_barrier();
        }
        if (chunks - c == 3u) {
            load(x0, c + 2u);
            __builtin_amdgcn_sched_barrier(0);
            multiply(0u, 2u);
            stage(x1, 1u);
            lds_barrier();
            multiply(1u, 2u);
            stage(x0, 0u);
            lds_barrier();
            multiply(0u, last_steps);
        } else {
            multiply(0u, 2u);
            stage(x1, 1u);
            lds_barrier();
            multiply(1u, last_steps);
        }
    }
    // D layout: lane l holds rows 4 (l/16) + e of column l%16 of each tile
#pragma unroll
    for (uint32_t i = 0; i < 2u; ++i)
#pragma unroll
        for (uint32_t j = 0; j < 2u; ++j) {
            const uint32_t col = n0 + 32u * (wave & 1u) + 16u * j + (lane & 15u);
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e) {
                const uint32_t row = m0 + a_row + 16u * i + 4u * (lane >> 4) + e;
                if (row >= m || col >= n) continue;
                const size_t at = static_cast<size_t>(row) * n + col;
                if constexpr (kOut == DenseOut::kF32)
                    c_f32[at] = acc[i][j][e];
                else
                    c_bf16[at] =
                        static_cast<uint16_t>(dense_epilogue(kOut, acc[i][j][e], divisor, scale));
            }
        }
}

// Router logits with the first level of the top-10 selection in the
// epilogue (the router GEMM, cuda_backend.cu:1518-1519, fused with level 1
// of cuda_topk_router_bf16's selection, q38_kernels.cu:406-458): workgroup
// (b, y) computes tokens 16y .. 16y+15 against experts 64b .. 64b+63 with
// the four waves splitting K exactly as dense_gemm_kernel does, so every
// logit is the value q38m_moe_router_v1 writes, bit for bit; the 16 x 64
// logits then stay in LDS, and wave w selects the top 10 of tokens 4w ..
// 4w+3 over its block (wave_top10), writing ten keys per (token, block)
// and the block's largest order key.  The fp32 logits never leave the CU.
__global__ __launch_bounds__(256) void router_select_kernel(
    const uint16_t* __restrict__ hidden, const uint16_t* __restrict__ router, uint32_t m,
    uint64_t* __restrict__ cand, uint32_t* __restrict__ block_max) {
    constexpr uint32_t kTM = 1, kTN = 4;
    constexpr uint32_t kL = 2u * (kTM + kTN);
    constexpr uint32_t kBlocks = kExperts / 64u;
    __shared__ u32x4 slab[kDenseWaves * kL * 64];
    __shared__ f32x4 lds[kDenseWaves * kTM * kTN * 64];
    __shared__ float logit_lds[16][64];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t m0 = blockIdx.y * 16u;
    const uint32_t n0 = blockIdx.x * 64u;
    const u32x4* ga[kL];
#pragma unroll
    for (uint32_t h = 0; h < 2u; ++h) {
        ga[h] = stage_ptr(hidden, m0, m, kHidden, h, lane);
#pragma unroll
        for (uint32_t j = 0; j < kTN; ++j)
            ga[2u * (kTM + j) + h] = stage_ptr(router, n0 + 16u * j, kExperts, kHidden, h, lane);
    }
    f32x4 acc[1][kTM][kTN];
#pragma unroll
    for (uint32_t j = 0; j < kTN; ++j) acc[0][0][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    constexpr uint32_t steps = kHidden / 32u;
    wave_partial<kTM, kTN, 1>(ga, slab + wave * kL * 64u, lane, wave * steps / kDenseWaves,
                              (wave + 1u) * steps / kDenseWaves, acc);
    // tile o: tokens 4 (l/16) + e, experts 16 o + l%16
    reduce_waves<kTM * kTN, kTM * kTN>(lds, &acc[0][0][0], wave, lane,
                                       [&](uint32_t o, uint32_t, f32x4 sum) {
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) logit_lds[4u * (lane >> 4) + e][16u * o + (lane & 15u)] = sum[e];
    });
    __syncthreads();
    // wave w: tokens 4w .. 4w+3, their four selections interleaved (rows
    // past the last token select over their clamped copies and store nothing)
    uint32_t k32[4], kmax[4];
#pragma unroll
    for (uint32_t r = 0; r < 4u; ++r) k32[r] = order_key(logit_lds[4u * wave + r][lane]);
    const size_t slot0 = static_cast<size_t>(m0 + 4u * wave) * kBlocks + blockIdx.x;
    wave_top10_rows<4>(k32, n0 + lane, [&](uint32_t r, uint32_t at, uint64_t key) {
        if (m0 + 4u * wave + r < m) cand[(slot0 + r * kBlocks) * kTopK + at] = key;
    }, kmax);
    if (lane < 4u && m0 + 4u * wave + lane < m) {
        const uint32_t mine = lane == 0u ? kmax[0] : lane == 1u ? kmax[1] : lane == 2u ? kmax[2] : kmax[3];
        block_max[slot0 + lane * kBlocks] = mine;
    }
}

// Level 2 of the fused router selection, one workgroup per token: the
// eight blocks' candidate lists and maxima into LDS, rank_candidates, then
// the rank-order denominator over the first top_k ranks and the weights
// (q38_kernels.cu:460-479), as q38m_topk_router_f32 computes them.
__global__ __launch_bounds__(kSelectThreads) void router_merge_kernel(
    const uint64_t* __restrict__ cand, const uint32_t* __restrict__ block_max, uint32_t top_k,
    int32_t* __restrict__ ids, float* __restrict__ weights) {
    constexpr uint32_t kBlocks = kExperts / 64u;
    __shared__ SelectLds select_lds;
    __shared__ int32_t ids_lds[kTopK];
    __shared__ float num_lds[kTopK];
    const uint32_t token = blockIdx.x;
    const uint32_t t = threadIdx.x;
    if (t < kBlocks * kTopK) select_lds.cand[t] = cand[static_cast<size_t>(token) * kBlocks * kTopK + t];
    if (t < kBlocks) select_lds.wave_max[t] = block_max[static_cast<size_t>(token) * kBlocks + t];
    __syncthreads();
    rank_candidates<kBlocks>(select_lds, ids_lds, num_lds);
    __syncthreads();
    if (t < 64u) {
        float denominator = 0.0f;
        for (uint32_t r = 0; r < top_k; ++r) denominator += num_lds[r];
        if (t < top_k) {
            ids[static_cast<size_t>(token) * top_k + t] = ids_lds[t];
            weights[static_cast<size_t>(token) * top_k + t] = num_lds[t] / denominator;
        }
    }
}


// The shared expert's first half in one launch: block (x, y) computes the
// 32 x 32 tiles (y, x) of g = bf16(X Wg^T) and u = bf16(X Wu^T) and
// h = silu_multiply(g, u) from them; the blocks of column 0 also compute
// the scalar output gate bf16(X wo^T) of their 32 rows.
__global__ __launch_bounds__(256) void shared_gate_up_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w_gate,
    const uint16_t* __restrict__ w_up, const uint16_t* __restrict__ w_out_gate, uint32_t m,
    uint32_t inter, uint16_t* __restrict__ g_out, uint16_t* __restrict__ u_out,
    uint16_t* __restrict__ h_out, uint16_t* __restrict__ gate_out) {
    constexpr uint32_t kTM = 2, kTN = 2;
    constexpr uint32_t kL = 2u * (kTM + 2u * kTN);
    __shared__ u32x4 slab[kDenseWaves * kL * 64];
    __shared__ f32x4 lds[kDenseWaves * 2 * kTM * kTN * 64];
    __shared__ float gate_lds[kDenseWaves][16 * kTM];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t m0 = blockIdx.y * 16u * kTM;
    const uint32_t n0 = blockIdx.x * 16u * kTN;
    const uint32_t steps = kHidden / 32u;
    const uint32_t s0 = wave * steps / kDenseWaves, s1 = (wave + 1u) * steps / kDenseWaves;
    const u32x4* ga[kL];
#pragma unroll
    for (uint32_t h = 0; h < 2u; ++h) {
#pragma unroll
        for (uint32_t i = 0; i < kTM; ++i)
            ga[2u * i + h] = stage_ptr(x, m0 + 16u * i, m, kHidden, h, lane);
#pragma unroll
        for (uint32_t j = 0; j < kTN; ++j) {
            ga[2u * (kTM + j) + h] = stage_ptr(w_gate, n0 + 16u * j, inter, kHidden, h, lane);
            ga[2u * (kTM + kTN + j) + h] = stage_ptr(w_up, n0 + 16u * j, inter, kHidden, h, lane);
        }
    }
    f32x4 acc[2][kTM][kTN];
#pragma unroll
    for (uint32_t v = 0; v < 2u; ++v)
#pragma unroll
        for (uint32_t i = 0; i < kTM; ++i)
#pragma unroll
            for (uint32_t j = 0; j < kTN; ++j) acc[v][i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 acc_gate[kTM];
#pragma unroll
    for (uint32_t i = 0; i < kTM; ++i) acc_gate[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    u32x4* const wave_slab = slab + wave * kL * 64u;
    const bool with_gate = blockIdx.x == 0u;
    if (with_gate) {
        const u32x4* gate = reinterpret_cast<const u32x4*>(w_out_gate + 8u * (lane >> 4));
        wave_partial<kTM, kTN, 2, true>(ga, wave_slab, lane, s0, s1, acc, gate, acc_gate);
        // column 0 of the gate tiles: lane 16 q holds rows 4 q + e of panel i
        if ((lane & 15u) == 0u) {
#pragma unroll
            for (uint32_t i = 0; i < kTM; ++i)
#pragma unroll
                for (uint32_t e = 0; e < 4u; ++e)
                    gate_lds[wave][16u * i + 4u * (lane >> 4) + e] = acc_gate[i][e];
        }
    } else {
        wave_partial<kTM, kTN, 2>(ga, wave_slab, lane, s0, s1, acc);
    }
    uint32_t g_bits[4] = {0u, 0u, 0u, 0u};
    reduce_waves<2 * kTM * kTN, kTM * kTN>(lds, &acc[0][0][0], wave, lane,
                                           [&](uint32_t o, uint32_t v, f32x4 sum) {
        const uint32_t col = n0 + 16u * (o % kTN) + (lane & 15u);
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) {
            const uint32_t row = m0 + 16u * (o / kTN) + 4u * (lane >> 4) + e;
            const uint32_t bits = f32_to_bf16(sum[e]);
            if (v == 0u) {  // the g tile comes first, then the u tile
                g_bits[e] = bits;
                continue;
            }
            if (row >= m) continue;
            const size_t at = static_cast<size_t>(row) * inter + col;
            g_out[at] = static_cast<uint16_t>(g_bits[e]);
            u_out[at] = static_cast<uint16_t>(bits);
            h_out[at] = static_cast<uint16_t>(silu_multiply(g_bits[e], bits));
        }
    });
    // reduce_waves' barrier has made gate_lds visible; the gate's partials
    // are summed in wave order like every other tile
    if (with_gate && wave == 0u && lane < 16u * kTM) {
        float sum = gate_lds[0][lane];
#pragma unroll
        for (uint32_t w = 1; w < kDenseWaves; ++w) sum += gate_lds[w][lane];
        const uint32_t row = m0 + lane;
        if (row < m) gate_out[row] = static_cast<uint16_t>(f32_to_bf16(sum));
    }
}

// ---- one activation row (m = 1: the batch-1 decode step) --------------
// At m = 1 a GEMM is a GEMV: every weight byte is used once, so the bound is
// how fast the weight rows stream, and a 16 x 16 MFMA tile would waste 15 of
// its 16 rows.  One wave per output row (wave_dot_bf16, q38m_select.h: four
// 16-byte chunks in flight per lane, fixed summation order); the
// activation's chunks are L2 hits after the first wave.

// C[n] = a . B[n], four waves (rows) per workgroup.
template <DenseOut kOut>
__global__ __launch_bounds__(256) void gemv_kernel(const uint16_t* __restrict__ a,
                                                   const uint16_t* __restrict__ b, uint32_t n,
                                                   uint32_t k, float* __restrict__ c_f32,
                                                   uint16_t* __restrict__ c_bf16, float divisor,
                                                   float scale) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * 4u + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (row >= n) return;
    const float acc = wave_dot_bf16(a, b + static_cast<size_t>(row) * k, k, lane);
    if (lane != 0u) return;
    if constexpr (kOut == DenseOut::kF32)
        c_f32[row] = acc;
    else
        c_bf16[row] = static_cast<uint16_t>(dense_epilogue(kOut, acc, divisor, scale));
}

// The shared expert's first half for one token: wave c < inter computes
// channel c's g = bf16(x Wg[c]) and u = bf16(x Wu[c]) (both rows' loads in
// flight together) and h = silu_multiply(g, u); wave `inter` computes the
// scalar output gate bf16(x wo).  Two waves per workgroup.
__global__ __launch_bounds__(128) void shared_gate_up_gemv_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w_gate,
    const uint16_t* __restrict__ w_up, const uint16_t* __restrict__ w_out_gate, uint32_t inter,
    uint16_t* __restrict__ g_out, uint16_t* __restrict__ u_out, uint16_t* __restrict__ h_out,
    uint16_t* __restrict__ gate_out) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t c = blockIdx.x * 2u + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (c > inter) return;
    if (c == inter) {
        const float gate = wave_dot_bf16(x, w_out_gate, kHidden, lane);
        if (lane == 0u) gate_out[0] = static_cast<uint16_t>(f32_to_bf16(gate));
        return;
    }
    const float g = wave_dot_bf16(x, w_gate + static_cast<size_t>(c) * kHidden, kHidden, lane);
    const float u = wave_dot_bf16(x, w_up + static_cast<size_t>(c) * kHidden, kHidden, lane);
    if (lane != 0u) return;
    const uint32_t g_bits = f32_to_bf16(g), u_bits = f32_to_bf16(u);
    g_out[c] = static_cast<uint16_t>(g_bits);
    u_out[c] = static_cast<uint16_t>(u_bits);
    h_out[c] = static_cast<uint16_t>(silu_multiply(g_bits, u_bits));
}

}  // namespace

namespace {

// one activation row: the GEMV form (grids of up to 65535 workgroups)
constexpr uint32_t kGemvMaxRows = 65535u * 4u;

template <DenseOut kOut>
void launch_dense_tiles(const uint16_t* a, const uint16_t* b, uint32_t m, uint32_t n, uint32_t k,
                        float* c_f32, uint16_t* c_bf16, float divisor, float scale,
                        hipStream_t stream) {
    if (m == 1u && n <= kGemvMaxRows) {
        gemv_kernel<kOut><<<(n + 3u) / 4u, 256, 0, stream>>>(a, b, n, k, c_f32, c_bf16, divisor,
                                                             scale);
        return;
    }
    // short K with a 64 x 64 grid that fills the GPU: workgroup-shared
    // tiles read half the bytes per output of the K-split 32 x 32 tiles
    const uint32_t tiles64 = ((m + 63u) / 64u) * ((n + 63u) / 64u);
    if (k <= kTile64MaxK && tiles64 >= kTile64MinTiles) {
        const dim3 grid((n + 63u) / 64u, (m + 63u) / 64u);
        dense_tile64_kernel<kOut><<<grid, 256, 0, stream>>>(a, b, m, n, k, c_f32, c_bf16, divisor,
                                                            scale);
        return;
    }
    const uint32_t tm = m <= 16u ? 1u : 2u;
    const uint32_t tn = (m <= 16u || n <= 16u) ? 1u : 2u;
    const dim3 grid((n + 16u * tn - 1u) / (16u * tn), (m + 16u * tm - 1u) / (16u * tm));
    if (tm == 1u)
        dense_gemm_kernel<1, 1, kOut><<<grid, 256, 0, stream>>>(a, b, m, n, k, c_f32, c_bf16,
                                                               divisor, scale);
    else if (tn == 1u)
        dense_gemm_kernel<2, 1, kOut><<<grid, 256, 0, stream>>>(a, b, m, n, k, c_f32, c_bf16,
                                                               divisor, scale);
    else
        dense_gemm_kernel<2, 2, kOut><<<grid, 256, 0, stream>>>(a, b, m, n, k, c_f32, c_bf16,
                                                               divisor, scale);
}

}  // namespace

hipError_t launch_dense_gemm(const uint16_t* a, const uint16_t* b, uint32_t m, uint32_t n,
                             uint32_t k, float* c_f32, uint16_t* c_bf16, hipStream_t stream) {
    if (c_bf16 != nullptr)
        launch_dense_tiles<DenseOut::kBf16>(a, b, m, n, k, nullptr, c_bf16, 1.0f, 1.0f, stream);
    else
        launch_dense_tiles<DenseOut::kF32>(a, b, m, n, k, c_f32, nullptr, 1.0f, 1.0f, stream);
    return hipGetLastError();
}

hipError_t launch_dense_gemm_act(const uint16_t* a, const uint16_t* b, uint32_t m, uint32_t n,
                                 uint32_t k, bool silu, float divisor, float scale,
                                 uint16_t* c_bf16, hipStream_t stream) {
    if (silu)
        launch_dense_tiles<DenseOut::kBf16Silu>(a, b, m, n, k, nullptr, c_bf16, divisor, scale,
                                                stream);
    else
        launch_dense_tiles<DenseOut::kBf16Sigmoid>(a, b, m, n, k, nullptr, c_bf16, divisor,
                                                   scale, stream);
    return hipGetLastError();
}

size_t router_topk_workspace_bytes(uint32_t tokens) {
    constexpr uint32_t kBlocks = kExperts / 64u;
    // one token: the GEMV's fp32 logits
    if (tokens == 1u) return kExperts * sizeof(float);
    return static_cast<size_t>(tokens) * kBlocks * (kTopK * sizeof(uint64_t) + sizeof(uint32_t));
}

hipError_t launch_router_topk(const uint16_t* hidden, const uint16_t* router, uint32_t tokens,
                              uint32_t top_k, void* workspace, int32_t* ids, float* weights,
                              hipStream_t stream) {
    constexpr uint32_t kBlocks = kExperts / 64u;
    if (tokens == 1u) {
        // one token: a GEMM tile would waste 15 of its 16 rows, so the
        // logits come from the GEMV (the same words q38m_moe_router_v1
        // writes for one token) and the block top-k ranks them
        float* logits = static_cast<float*>(workspace);
        gemv_kernel<DenseOut::kF32><<<kExperts / 4u, 256, 0, stream>>>(
            hidden, router, kExperts, kHidden, logits, nullptr, 1.0f, 1.0f);
        hipError_t e = hipGetLastError();
        return e == hipSuccess ? launch_topk(logits, ids, weights, 1u, kExperts, top_k, true,
                                             stream)
                               : e;
    }
    uint64_t* cand = static_cast<uint64_t*>(workspace);
    uint32_t* block_max = reinterpret_cast<uint32_t*>(cand + static_cast<size_t>(tokens) * kBlocks * kTopK);
    router_select_kernel<<<dim3(kBlocks, (tokens + 15u) / 16u), 256, 0, stream>>>(
        hidden, router, tokens, cand, block_max);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess)
        router_merge_kernel<<<tokens, kSelectThreads, 0, stream>>>(cand, block_max, top_k, ids,
                                                                   weights);
    return e == hipSuccess ? hipGetLastError() : e;
}

size_t shared_expert_scratch_bytes(uint32_t tokens, uint32_t inter) {
    return 3u * static_cast<size_t>(tokens) * inter * sizeof(uint16_t);
}

hipError_t launch_shared_expert(const uint16_t* hidden, const uint16_t* w_gate,
                                const uint16_t* w_up, const uint16_t* w_down,
                                const uint16_t* w_out_gate, uint32_t tokens, uint32_t inter,
                                void* scratch, uint16_t* shared_output, uint16_t* shared_gate,
                                hipStream_t stream) {
    const size_t elements = static_cast<size_t>(tokens) * inter;
    uint16_t* g = static_cast<uint16_t*>(scratch);
    uint16_t* u = g + elements;
    uint16_t* h = u + elements;
    if (tokens == 1u) {
        shared_gate_up_gemv_kernel<<<(inter + 2u) / 2u, 128, 0, stream>>>(
            hidden, w_gate, w_up, w_out_gate, inter, g, u, h, shared_gate);
    } else {
        const dim3 grid(inter / 32u, (tokens + 31u) / 32u);
        shared_gate_up_kernel<<<grid, 256, 0, stream>>>(hidden, w_gate, w_up, w_out_gate, tokens,
                                                        inter, g, u, h, shared_gate);
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess)
        e = launch_dense_gemm(h, w_down, tokens, kHidden, inter, nullptr, shared_output, stream);
    return e;
}

}  // namespace q38m
