// Chunks above the 512-token slab: one MoE layer over up to 32,768 tokens
// in a single pass, so that every active expert's weights are streamed once
// per 128 routed rows instead of once per 16.  The reference prefills in
// slabs of at most 512 tokens (include/q38/cuda_moe_prefill.h:14, the V1
// plan); this path keeps the V1 plan's packed order (expert-major, stable
// in route index, q38_moe_prefill.cu:192-262) and per-route arithmetic, so
// every route's weighted_mid and route_output row and every token's output
// are bit-identical to the slab path's, and changes only the task height
// (128 rows) and how the plan is built (three launches instead of one
// workgroup).
//
// Plan: (1) per-chunk expert histograms, (2) one workgroup scans them into
// expert offsets, per-chunk bases and 128-row tasks, (3) one wave per chunk
// assigns stable positions with an LDS table of equal-id lane masks.
//
// Weights are read with ordinary (cached) loads, unlike the slab kernels'
// non-temporal streams: a hot expert's 128-row tasks run side by side and
// share its weights through L2.
//
// GEMMs: the slab kernels' decomposition (gate/up: a workgroup of 8 waves
// covers 8 gate/up tile pairs of one task; down: 16-channel output tiles)
// with up to 8 MFMA row tiles per weight fragment.  The gate/up chain costs
// a v_cvt and a v_fma per accumulator element and group, so at 128 rows the
// kernel is VALU-bound (~1/4 of int8 MFMA peak); down W8 is MFMA/HBM-bound.
#include "q38m_device.h"
#include "q38m_internal.h"
#include "q38m_select.h"

namespace q38m {
namespace {

constexpr uint32_t kWideRows = Q38M_WIDE_TASK_ROWS;
constexpr uint32_t kRowTiles = kWideRows / 16u;
constexpr uint32_t kCountSlots = kExperts + 1u;  // slot 512 counts invalid ids

// The contract's SwiGLU gate, silu(g) = g / (1 + exp(-g)), for every bf16 g:
// entry h holds the fp32 word of silu(bits h << 16).  The gate enters SwiGLU
// rounded to bf16 (q38_moe_prefill.cu:449-461), so silu depends on g's 16
// bits only; the table is written at build time by q38m_silu_gen.c (the
// contract's exp and one IEEE division, equal to swiglu_fold's evaluation
// for every g), and one gather replaces ~40 VALU instructions per element
// in the compute-bound gate/up epilogue.  256 KiB, read through L2.
__device__ const uint32_t kSiluTable[65536] = {
#include "q38m_silu_table.inc"
};

// ---- plan -------------------------------------------------------------------

__global__ __launch_bounds__(256) void wide_count_kernel(const int32_t* __restrict__ ids,
                                                         uint32_t routes,
                                                         uint32_t* __restrict__ chunk_counts) {
    __shared__ uint32_t hist[kCountSlots];
    for (uint32_t i = threadIdx.x; i < kCountSlots; i += 256u) hist[i] = 0u;
    __syncthreads();
    const uint32_t begin = blockIdx.x * kWideChunkRoutes;
    const uint32_t end = min(begin + kWideChunkRoutes, routes);
    for (uint32_t a = begin + threadIdx.x; a < end; a += 256u) {
        const int32_t id = ids[a];
        const bool valid = id >= 0 && id < static_cast<int32_t>(kExperts);
        atomicAdd(&hist[valid ? static_cast<uint32_t>(id) : kExperts], 1u);
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < kCountSlots; i += 256u)
        chunk_counts[static_cast<size_t>(blockIdx.x) * kCountSlots + i] = hist[i];
}

// One workgroup of 512 threads, thread e = expert e.  Turns the per-chunk
// counts into per-chunk bases within each expert's segment (in place) and
// writes the plan's counts, offsets, task offsets, tasks and header.
constexpr uint32_t kMaxChunks = (Q38M_WIDE_MAX_TOKENS * kTopK + kWideChunkRoutes - 1u) /
                                kWideChunkRoutes;

__global__ __launch_bounds__(512) void wide_scan_kernel(uint32_t* __restrict__ chunk_counts,
                                                        uint32_t chunks, uint32_t tokens,
                                                        q38m_route_plan_v1 plan,
                                                        uint32_t max_tasks) {
    __shared__ uint32_t wave_totals[2][8];
    __shared__ uint32_t wave_active[8];
    __shared__ uint32_t offsets[kExperts + 1u];
    __shared__ uint32_t task_offsets[kExperts + 1u];
    __shared__ uint32_t invalid;
    const uint32_t e = threadIdx.x;
    const uint32_t tid = e;
    const uint32_t lane = e & 63u;
    const uint32_t wave = e >> 6;
    const uint32_t routes = tokens * kTopK;

    // 1. running count of expert e over the chunks, in chunk order; each
    // chunk's slot becomes the expert's count in the chunks before it.
    // Batches of 32 chunks, the next batch's loads issued before this
    // batch's sums (two batches in flight), unconditionally (a chunk past
    // the last re-reads the last one and adds nothing), so no branch sits
    // between a load and the wait for it.  (One batch at a time: ~9.5 us at
    // 160 chunks, a round trip each.)
    constexpr uint32_t kBatch = 32;
    auto load_batch = [&](uint32_t c0, uint32_t (&v)[kBatch]) {
#pragma unroll
        for (uint32_t j = 0; j < kBatch; ++j)
            v[j] = chunk_counts[static_cast<size_t>(min(c0 + j, chunks - 1u)) * kCountSlots + e];
    };
    uint32_t count = 0;
    uint32_t va[kBatch], vb[kBatch];
    load_batch(0u, va);
    for (uint32_t c0 = 0; c0 < chunks; c0 += 2u * kBatch) {
        load_batch(c0 + kBatch, vb);
#pragma unroll
        for (uint32_t j = 0; j < kBatch; ++j) {
            const bool live = c0 + j < chunks;
            if (live) chunk_counts[static_cast<size_t>(c0 + j) * kCountSlots + e] = count;
            count += live ? va[j] : 0u;
        }
        if (c0 + kBatch >= chunks) break;  // uniform
        load_batch(c0 + 2u * kBatch, va);
#pragma unroll
        for (uint32_t j = 0; j < kBatch; ++j) {
            const bool live = c0 + kBatch + j < chunks;
            if (live) chunk_counts[static_cast<size_t>(c0 + kBatch + j) * kCountSlots + e] = count;
            count += live ? vb[j] : 0u;
        }
    }
    // invalid ids: wave 0 sums slot 512 of every chunk (at most 160, three
    // unconditional loads per lane, one round trip)
    static_assert(kMaxChunks <= 192u, "three invalid-slot loads per lane");
    if (wave == 0u) {
        uint32_t bad[3];
#pragma unroll
        for (uint32_t j = 0; j < 3u; ++j)
            bad[j] = chunk_counts[static_cast<size_t>(min(lane + 64u * j, chunks - 1u)) *
                                      kCountSlots + kExperts];
        uint32_t sum = 0;
#pragma unroll
        for (uint32_t j = 0; j < 3u; ++j) sum += lane + 64u * j < chunks ? bad[j] : 0u;
        sum = wave_inclusive_sum(sum);
        if (lane == 63u) invalid = sum;
    }
    const uint32_t tasks = (count + kWideRows - 1u) / kWideRows;

    // 2. exclusive scans of counts and task counts over experts
    {
        plan.expert_counts[e] = static_cast<uint16_t>(count);
        const uint32_t inc_count = wave_inclusive_sum(count);
        const uint32_t inc_tasks = wave_inclusive_sum(tasks);
        const uint64_t active = __ballot(count != 0u);
        if (lane == 63u) {
            wave_totals[0][wave] = inc_count;
            wave_totals[1][wave] = inc_tasks;
        }
        if (lane == 0u) wave_active[wave] = __popcll(active);
        // inclusive values kept for after the barrier
        offsets[e] = inc_count;
        task_offsets[e] = inc_tasks;
    }
    __syncthreads();
    {
        uint32_t prefix_count = 0, prefix_tasks = 0;
#pragma unroll
        for (uint32_t w = 0; w < 8u; ++w) {
            prefix_count += w < wave ? wave_totals[0][w] : 0u;
            prefix_tasks += w < wave ? wave_totals[1][w] : 0u;
        }
        const uint32_t offset = prefix_count + offsets[e] - count;
        const uint32_t task_offset = prefix_tasks + task_offsets[e] - tasks;
        plan.expert_offsets[e] = offset;
        plan.expert_task_offsets[e] = task_offset;
        if (e == kExperts - 1u) {
            plan.expert_offsets[kExperts] = prefix_count + offsets[e];
            plan.expert_task_offsets[kExperts] = prefix_tasks + task_offsets[e];
        }
        // every read of offsets[] above precedes the writes below (one
        // thread reads and writes only its own slot)
        offsets[e] = offset;
        task_offsets[e] = task_offset;
        if (e == kExperts - 1u) {
            offsets[kExperts] = offset + count;
            task_offsets[kExperts] = task_offset + tasks;
        }
    }
    __syncthreads();
    const uint32_t total = offsets[kExperts];
    const uint32_t task_total = task_offsets[kExperts];

    // 3. tasks: 128-row tiles of each expert's segment, zero past the count.
    // Spread over the threads (a Zipf-hot expert has hundreds of tasks, and
    // one thread per expert took ~12 us at 32,768 tokens): task t's expert
    // is the last e with task_offsets[e] <= t, by binary search in LDS.
    uint2* task_words = reinterpret_cast<uint2*>(plan.tasks);
    for (uint32_t t = tid; t < max_tasks; t += 512u) {
        uint2 word = make_uint2(0u, 0u);
        if (t < task_total) {
            uint32_t lo = 0u, hi = kExperts - 1u;  // task_offsets[lo] <= t < task_offsets[lo + 1]
            while (lo < hi) {
                const uint32_t mid = (lo + hi + 1u) >> 1;
                if (task_offsets[mid] <= t) lo = mid; else hi = mid - 1u;
            }
            const uint32_t tile = t - task_offsets[lo];
            const uint32_t remaining = (offsets[lo + 1u] - offsets[lo]) - tile * kWideRows;
            const uint32_t rows = remaining < kWideRows ? remaining : kWideRows;
            word = make_uint2(offsets[lo] + tile * kWideRows, lo | (rows << 16));
        }
        task_words[t] = word;
    }
    // packed positions no valid route fills hold their own index
    for (uint32_t p = total + tid; p < routes; p += 512u) plan.packed_assignment[p] = p;

    if (tid == 0u) {
        uint32_t active_experts = 0;
        for (uint32_t w = 0; w < 8u; ++w) active_experts += wave_active[w];
        uint32_t status = Q38M_PLAN_OK;
        if (invalid != 0u)
            status = Q38M_PLAN_INVALID_EXPERT;
        else if (total != routes || task_total > max_tasks)
            status = Q38M_PLAN_INVALID_SHAPE;
        q38m_route_plan_header_v1* h = plan.header;
        h->magic = Q38M_ROUTE_PLAN_MAGIC_V1;
        h->version = Q38M_ROUTE_PLAN_VERSION_WIDE;
        h->tokens = tokens;
        h->routes = routes;
        h->active_experts = active_experts;
        h->task_count = task_total;
        h->status = status;
        h->flags = 0u;
        h->route_hash = 0u;
        h->plan_hash = 0u;
        h->reserved0 = 0u;
        h->reserved1 = 0u;
    }
}

// One wave per chunk walks its routes 64 at a time in route order, from
// the expert offsets plus the chunk's bases within each segment.  Lanes
// with equal ids find each other through an LDS table of lane masks (each
// lane ORs its bit into its id's slot, reads the slot back, clears it; one
// wave's LDS operations execute in order); the stable position is the
// chunk's running base for the id plus the equal lanes below.
__global__ __launch_bounds__(64) void wide_scatter_kernel(const int32_t* __restrict__ ids,
                                                          uint32_t routes,
                                                          const uint32_t* __restrict__ bases,
                                                          q38m_route_plan_v1 plan) {
    __shared__ uint32_t running[kExperts];
    __shared__ unsigned long long table[kCountSlots];
    const uint32_t lane = threadIdx.x;
    const uint32_t* base = bases + static_cast<size_t>(blockIdx.x) * kCountSlots;
    const uint32_t begin = blockIdx.x * kWideChunkRoutes;
    const uint32_t end = min(begin + kWideChunkRoutes, routes);
    // every load of the chunk is issued before the first use: the segment
    // bases and the chunk's ids (clamped to its last route, unused past it)
    constexpr uint32_t kPerLane = kExperts / 64u, kSteps = kWideChunkRoutes / 64u;
    static_assert(kExperts % 64u == 0u && kWideChunkRoutes % 64u == 0u, "whole waves");
    uint32_t offset[kPerLane], chunk_base[kPerLane];
    int32_t idv[kSteps];
#pragma unroll
    for (uint32_t k = 0; k < kPerLane; ++k) {
        offset[k] = plan.expert_offsets[lane + 64u * k];
        chunk_base[k] = base[lane + 64u * k];
    }
#pragma unroll
    for (uint32_t j = 0; j < kSteps; ++j) idv[j] = ids[min(begin + 64u * j + lane, end - 1u)];
#pragma unroll
    for (uint32_t k = 0; k < kPerLane; ++k) running[lane + 64u * k] = offset[k] + chunk_base[k];
    for (uint32_t i = lane; i < kCountSlots; i += 64u) table[i] = 0ull;
    __syncthreads();
    const uint64_t below_mask = (1ull << lane) - 1ull;
#pragma unroll
    for (uint32_t j = 0; j < kSteps; ++j) {
        const uint32_t a = begin + 64u * j + lane;
        if (begin + 64u * j >= end) break;  // uniform
        const bool in = a < end;
        const int32_t id = in ? idv[j] : -1;
        const bool valid = in && id >= 0 && id < static_cast<int32_t>(kExperts);
        const uint32_t slot = valid ? static_cast<uint32_t>(id) : kExperts;
        atomicOr(&table[slot], 1ull << lane);
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        const unsigned long long equal = table[slot];
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        table[slot] = 0ull;
        const uint32_t below = __popcll(equal & below_mask);
        const uint32_t run = valid ? running[valid ? slot : 0u] : 0u;
        if (valid && below == 0u) running[slot] = run + __popcll(equal);
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (valid) {
            const uint32_t position = run + below;
            plan.packed_assignment[position] = a;
            plan.assignment_to_packed[a] = position;
        } else if (in) {
            plan.assignment_to_packed[a] = a;
        }
    }
}

// ---- workgroup placement -----------------------------------------------------

// The grouped GEMMs below run on (slice, task) grids: gridDim.x slices of
// the output channels times one row per task slot.  The dispatcher hands
// workgroups to the 8 XCDs round-robin by linear id, and each XCD has its
// own L2.  This maps the live pairs (task < the plan's task count) so that
// each XCD runs one contiguous range of them: a task's slices read the same
// rows, and an expert's consecutive tasks read the same weights, from one
// L2.  Workgroups past the live pairs return at once, spread evenly over
// the XCDs.
struct Placement {
    uint32_t task, slice;
};

__device__ inline bool place_on_xcds(const uint32_t* live_tasks, Placement& at) {
    constexpr uint32_t kXcds = 8;
    const uint32_t slices = gridDim.x;
    const uint32_t live = min(*live_tasks, gridDim.y) * slices;
    const uint32_t id = blockIdx.y * slices + blockIdx.x;
    if (id >= live) return false;
    const uint32_t per = live / kXcds, extra = live % kXcds;
    const uint32_t xcd = id % kXcds;
    const uint32_t j = xcd * per + min(xcd, extra) + id / kXcds;
    at.task = j / slices;
    at.slice = j % slices;
    return true;
}

// ---- gate/up ----------------------------------------------------------------

struct TileQuad {
    uint4 w;  // one 16-channel tile's data of one quad
    uint2 s;  // its scale words (4, 2 or 1 groups; load_quad_scales)
};

// Gate/up, W4, over a task of up to 128 rows.  A workgroup of 16 waves
// covers 8 gate/up channel pairs (16 channels each) of one task; wave w
// owns pair w % 8 for rows 64 (w / 8) .. +63 (up to 4 row tiles of 16) and
// runs both the pair's gate tile and its up tile, so each A fragment feeds
// two MFMAs and the SwiGLU epilogue stays in registers.
//
// Per quad (128 columns of K) the workgroup stages into LDS the task's 128
// int8 rows (16 KB), its 16 weight tiles (16 KB) and their scale words;
// every thread moves one 16-byte row piece, one 16-byte weight piece and
// one 4-byte scale piece.  Those loads are issued two quads ahead into two
// register sets and stored one quad ahead into a double-buffered image, and
// the barrier between quads waits only for LDS operations, so the global
// loads of later quads stay in flight across it (a full workgroup fence
// would wait for them).
//
// Arithmetic per scale group and tile: kSub v_mfma_i32_16x16x32_i8 chained
// through the accumulator, started from the bits of 1.5 * 2^23 so that the
// result read as a float is 12582912 + acc exactly (|acc| < 2^22); one
// v_add_f32 recovers (float)acc and one v_fma_f32 continues the group chain
// -- the contract's y = fmaf((float)acc_g, s_g, y) in group order.  The
// next tile's MFMAs are issued before this tile's fp32 step.  The W4
// nibbles sit in the high half of each int8 (16 * w); fp16 scales run the
// chain on 16 * y, bf16 scales take s / 16.  Per-row token scale and route
// weight are staged in LDS once for the epilogue.
template <uint32_t H, uint32_t I, uint32_t kSub, bool kBf16>
__global__ __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(4)))
void gate_up_w4_wide_kernel(const uint4* __restrict__ w, const uint16_t* __restrict__ s,
                            const int8_t* __restrict__ xq, const float* __restrict__ xs,
                            const uint32_t* __restrict__ packed,
                            const float* __restrict__ route_weights,
                            const q38m_task_v1* __restrict__ tasks, const uint32_t* __restrict__ live_tasks, uint16_t* __restrict__ mid) {
    constexpr uint32_t kQuads = H / 128u;
    constexpr uint32_t kTilesAll = 2u * I / 16u;
    constexpr uint32_t kRowScales = 4u / kSub;                           // words per row per quad
    constexpr uint32_t kGroups = 4u / kSub;                              // scale groups per quad
    constexpr uint32_t kScalePieces = 16u * 16u * kRowScales * 2u / 4u;  // 4-byte pieces per quad
    static_assert(kQuads % 2u == 0u, "two staging register sets");
    static_assert(kScalePieces <= 1024u, "one scale piece per thread");
    // per buffer: A [sub-block j][row tile][lane] 8-byte MFMA fragments, the
    // workgroup's 16 weight tiles [tile][lane] and their scale words
    __shared__ __align__(16) uint2 a_lds[2][4u * kRowTiles * 64u];
    __shared__ __align__(16) uint4 w_lds[2][16u * 64u];
    __shared__ __align__(16) uint32_t s_lds[2][kScalePieces];
    __shared__ float2 row_info[kWideRows];  // (token scale, route weight)

    Placement at;
    if (!place_on_xcds(live_tasks, at)) return;
    const TaskRecord task = read_task(tasks, at.task);
    const uint32_t rows = task.rows;
    if (rows == 0u) return;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t rh = wave >> 3;
    const uint32_t pr = wave & 7u;
    const uint32_t n = lane & 15u, qh = lane >> 4;
    const uint32_t e = task.expert;
    const uint32_t p0 = task.begin;
    const int here = static_cast<int>(rows) - static_cast<int>(64u * rh);
    const uint32_t nt = __builtin_amdgcn_readfirstlane(
        here <= 0 ? 0u : (here >= 64 ? 4u : (static_cast<uint32_t>(here) + 15u) / 16u));

    // staging: row piece (row tid/8, 16-byte chunk tid%8), weight piece
    // (slot tid/64 of the workgroup's 16, lane tid%64), scale piece tid
    const uint32_t sr = tid >> 3, sch = tid & 7u;
    const bool alive = sr < rows;
    const uint32_t assignment = alive ? checked(packed[p0 + sr], Q38M_WIDE_MAX_TOKENS * kTopK, kCheckToken) : 0u;
    if (sch == 0u && alive)
        row_info[sr] = make_float2(xs[assignment / kTopK], route_weights[assignment]);
    const uint4* a_src =
        reinterpret_cast<const uint4*>(xq + static_cast<size_t>(assignment / kTopK) * H) + sch;
    const uint32_t a_at = ((sch >> 1) * kRowTiles + (sr >> 4)) * 64u + (sch & 1u) * 32u + (sr & 15u);
    const size_t slot0 = static_cast<size_t>(e) * kQuads * kTilesAll + at.slice * 16u;
    const uint4* w_src = w + slot0 * 64u + tid;
    const uint32_t* s_src = reinterpret_cast<const uint32_t*>(s) + slot0 * 16u * kRowScales / 2u + tid;
    const bool s_thread = tid < kScalePieces;
    struct Stage {
        uint4 a, w;
        uint32_t s;
    };
    auto load_stage = [&](uint32_t kq) __attribute__((always_inline)) {
        Stage st;
        st.a = alive ? a_src[kq * 8u] : make_uint4(0u, 0u, 0u, 0u);
        st.w = w_src[static_cast<size_t>(kq) * kTilesAll * 64u];
        st.s = s_thread ? s_src[static_cast<size_t>(kq) * kTilesAll * 16u * kRowScales / 2u] : 0u;
        return st;
    };
    auto store_stage = [&](const Stage& st, uint32_t buffer) __attribute__((always_inline)) {
        a_lds[buffer][a_at] = make_uint2(st.a.x, st.a.y);
        a_lds[buffer][a_at + 16u] = make_uint2(st.a.z, st.a.w);
        w_lds[buffer][tid] = st.w;
        if (s_thread) s_lds[buffer][tid] = st.s;
    };

    float y[4][2][4];
#pragma unroll
    for (uint32_t t = 0; t < 4u; ++t)
#pragma unroll
        for (uint32_t u = 0; u < 2u; ++u)
#pragma unroll
            for (uint32_t i = 0; i < 4u; ++i) y[t][u][i] = 0.0f;
    v4i bias;
    bias.x = bias.y = bias.z = bias.w = 0x4B400000;
    float unbias;  // -12582912.0f in a scalar register (no literal per use)
    asm volatile("s_mov_b32 %0, 0xcb400000" : "=s"(unbias));

    // One quad for kNt row tiles.  Chain k = (scale group gg, row tile t,
    // gate/up u); the A fragments of (gg, t) are read one set ahead and a
    // group's B fragments are unpacked once for all row tiles.
    auto multiply = [&](auto tiles, uint32_t buffer) __attribute__((always_inline)) {
        constexpr uint32_t kNt = decltype(tiles)::value;
        constexpr uint32_t kSets = kGroups * kNt;
        constexpr uint32_t kChains = kSets * 2u;
        const uint2* abuf = a_lds[buffer] + lane;
        const uint4 gq = w_lds[buffer][(2u * pr) * 64u + lane];
        const uint4 uq = w_lds[buffer][(2u * pr + 1u) * 64u + lane];
        const uint16_t* sbase = reinterpret_cast<const uint16_t*>(s_lds[buffer]);
        const uint2 gs = load_quad_scales<kSub, false>(sbase + ((2u * pr) * 16u + n) * kRowScales);
        const uint2 us =
            load_quad_scales<kSub, false>(sbase + ((2u * pr + 1u) * 16u + n) * kRowScales);
        const uint32_t gw[4] = {gq.x, gq.y, gq.z, gq.w};
        const uint32_t uw[4] = {uq.x, uq.y, uq.z, uq.w};
        float sc[2][kGroups];
#pragma unroll
        for (uint32_t gg = 0; gg < kGroups; ++gg) {
#pragma unroll
            for (uint32_t u = 0; u < 2u; ++u) {
                const uint32_t word = quad_scale_word(u ? us : gs, gg);
                sc[u][gg] = kBf16 ? bf16_to_f32(word) * 0.0625f : f16_to_f32(word);
                asm volatile("" : "+v"(sc[u][gg]));  // a plain v_fma_f32, not v_fma_mix
            }
        }
        long fa[2][kSub];
        auto read_set = [&](uint32_t m) __attribute__((always_inline)) {
            const uint32_t gg = m / kNt, t = m % kNt;
#pragma unroll
            for (uint32_t sb = 0; sb < kSub; ++sb)
                fa[m & 1u][sb] = as_long(abuf[((gg * kSub + sb) * kRowTiles + 4u * rh + t) * 64u]);
        };
        long bf[2][kSub];
        v4i d[2];
        auto issue = [&](uint32_t k) __attribute__((always_inline)) {
            const uint32_t m = k / 2u, u = k & 1u;
            const uint32_t gg = m / kNt, t = m % kNt;
            if (u == 0u) {
                if (m + 1u < kSets) read_set(m + 1u);
                if (t == 0u) {
#pragma unroll
                    for (uint32_t sb = 0; sb < kSub; ++sb) {
                        bf[0][sb] = unpack_w4x16(gw[gg * kSub + sb]);
                        bf[1][sb] = unpack_w4x16(uw[gg * kSub + sb]);
                    }
                }
            }
            v4i acc = bias;
#pragma unroll
            for (uint32_t sb = 0; sb < kSub; ++sb)
                acc = mfma_i8_16x16x32(fa[m & 1u][sb], bf[u][sb], acc);
            d[k & 1u] = acc;
        };
        auto step = [&](uint32_t k) __attribute__((always_inline)) {
            const uint32_t m = k / 2u, u = k & 1u;
            const uint32_t gg = m / kNt, t = m % kNt;
            const float scale = sc[u][gg];
#pragma unroll
            for (uint32_t i = 0; i < 4u; ++i)
                y[t][u][i] =
                    __builtin_fmaf(__int_as_float(d[k & 1u][i]) + unbias, scale, y[t][u][i]);
            // keep the chain step here, between this tile's MFMAs and the next
            // ones (otherwise it can sink to the end of the loop body, and
            // every accumulator of the quad stays live until then)
            asm volatile("" : "+v"(y[t][u][0]), "+v"(y[t][u][1]), "+v"(y[t][u][2]),
                         "+v"(y[t][u][3]));
        };
        read_set(0);
#pragma unroll
        for (uint32_t k = 0; k <= kChains; ++k) {
            if (k < kChains) issue(k);
            __builtin_amdgcn_sched_barrier(0);
            if (k > 0u) step(k - 1u);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // barrier over LDS only: this wave's LDS operations are complete, its
    // global loads (the staging of later quads) stay in flight
    auto lds_barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

    // quad q: loaded at the start of quad q-2 into register set q%2, stored
    // at the end of quad q-1 into LDS buffer q%2, multiplied during quad q.
    // The loop is instantiated per row-tile count (three tiles run as four,
    // one as two; the extra rows are zero), so a wave's accumulators keep
    // one register assignment through it; every instance passes the same
    // barriers.
    Stage set0 = load_stage(0), set1 = load_stage(1);
    store_stage(set0, 0u);
    __syncthreads();
    auto k_loop = [&](auto tiles) __attribute__((always_inline)) {
        constexpr uint32_t kNt = decltype(tiles)::value;
#pragma unroll 1
        for (uint32_t kq = 0; kq < kQuads; kq += 2u) {
            if (kq + 2u < kQuads) set0 = load_stage(kq + 2u);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (kNt > 0u) multiply(tiles, 0u);
            store_stage(set1, 1u);
            lds_barrier();
            if (kq + 3u < kQuads) set1 = load_stage(kq + 3u);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (kNt > 0u) multiply(tiles, 1u);
            if (kq + 2u < kQuads) store_stage(set0, 0u);
            lds_barrier();
        }
    };
    if (nt > 2u)
        k_loop(std::integral_constant<uint32_t, 4>{});
    else if (nt > 0u)
        k_loop(std::integral_constant<uint32_t, 2>{});
    else
        k_loop(std::integral_constant<uint32_t, 0>{});

    // SwiGLU: D lane (qh, n) holds rows 4qh + i of each tile, channel n
    const uint32_t channel = (at.slice * 8u + pr) * 16u + n;
    const float unscale = kBf16 ? 1.0f : 0.0625f;
#pragma unroll
    for (uint32_t t = 0; t < 4u; ++t) {
        if (t >= nt) break;
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) {
            const uint32_t r = 64u * rh + 16u * t + 4u * qh + i;
            if (r >= rows) continue;
            const float2 info = row_info[r];
            const float yg = (y[t][0][i] * unscale) * info.x;
            const float yu = (y[t][1][i] * unscale) * info.x;
            mid[static_cast<size_t>(p0 + r) * I + channel] =
                static_cast<uint16_t>(swiglu_fold(yg, yu, info.y));
        }
    }
}

// ---- gate/up, W4 groups of 32, on fp16 MFMA --------------------------------
//
// The int8 values of both operands (activations in [-127, 127], W4 nibbles
// as 16 * w in [-128, 112]) are exact in fp16, their products (< 2^14) and
// every partial sum of a 32-wide group (< 2^19) exact in fp32, so
// v_mfma_f32_16x16x32_f16 returns (float)(16 * acc_g) itself -- the value
// the int8 MFMA path recovers with one extra VALU op per accumulator element
// and group.  The chain step is then a single v_fma_f32, and the MFMA runs
// at the same 16 cycles as v_mfma_i32_16x16x32_i8.
//
// fp16 images.  Weights (MFMA16 W4 word: byte i = k_i | k_{4+i} << 4): a
// nibble u' = w + 8 (offset binary: the nibble's top bit inverted) placed
// under the exponent bits of 1024 (0x6400) is the fp16 1024 + 16 u' (nibble
// in bits 4-7) or 1024 + u' (bits 0-3), exact; one v_pk_add_f16 of -1152 or
// -1032 leaves 16 w or w.  One v_bitop3_b32 forms two such values from a
// word (or the word shifted right by 8): per bit, field bits pass (sign bit
// inverted), exponent bits are set, the rest cleared.  A lane's eight K
// values come out as (4, 6) and (5, 7) times 16, (0, 2) and (1, 3) times 1;
// the activations are staged in the same K order with the (0, 2), (1, 3)
// pairs times 16 (one v_cvt_f16_i16 per sign-extended byte, one v_pk_mul_f16
// per pair), so every product is 16 a w, as on the int8 path.  A dot
// product does not depend on the order of its K terms, only on A and B
// agreeing; every value and product here is an integer below 2^14.
__device__ __forceinline__ uint32_t pk_add_f16(uint32_t v, float c) {
    typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
    const _Float16 h = static_cast<_Float16>(c);
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, v) + h2_t{h, h});
}
__device__ __forceinline__ uint32_t pk_times16_f16(uint32_t v) {
    typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
    const _Float16 h = static_cast<_Float16>(16.0f);
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, v) * h2_t{h, h});
}

// one MFMA16 W4 word -> fp16 K order (4, 6)x16, (5, 7)x16, (0, 2), (1, 3)
__device__ __forceinline__ uint4 w4_to_f16x16(uint32_t d) {
    // bitop3 truth table (index = S0*4 + S1*2 + S2): out = S0 where S1 & !S2,
    // !S0 where S1 & S2, 1 where !S1 & S2, 0 elsewhere
    constexpr uint32_t kTable = 0x6A;
    constexpr uint32_t kHiField = 0x00F000F0u, kHiConst = 0x64806480u;
    constexpr uint32_t kLoField = 0x000F000Fu, kLoConst = 0x64086408u;
    const uint32_t t = d >> 8;
    return make_uint4(
        pk_add_f16(__builtin_amdgcn_bitop3_b32(d, kHiField, kHiConst, kTable), -1152.0f),
        pk_add_f16(__builtin_amdgcn_bitop3_b32(t, kHiField, kHiConst, kTable), -1152.0f),
        pk_add_f16(__builtin_amdgcn_bitop3_b32(d, kLoField, kLoConst, kTable), -1032.0f),
        pk_add_f16(__builtin_amdgcn_bitop3_b32(t, kLoField, kLoConst, kTable), -1032.0f));
}

// bytes 0 and 2 (or 1 and 3) of v as signed integers -> two fp16 (exact):
// v_cvt_f16_i16 with a sign-extended byte source selected by SDWA, the
// second conversion writing the high half and keeping the low one
__device__ __forceinline__ uint32_t sbytes02_to_f16(uint32_t v) {
    uint32_t r;
    asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_2"
        : "=&v"(r)
        : "v"(v));
    return r;
}
__device__ __forceinline__ uint32_t sbytes13_to_f16(uint32_t v) {
    uint32_t r;
    asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
        "v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3"
        : "=&v"(r)
        : "v"(v));
    return r;
}

// eight int8 (k 0-3 in lo, 4-7 in hi) -> fp16 in the order and scaling of
// w4_to_f16x16's partners: (4, 6), (5, 7), 16 (0, 2), 16 (1, 3)
__device__ __forceinline__ uint4 i8_to_f16(uint32_t lo, uint32_t hi) {
    return make_uint4(sbytes02_to_f16(hi), sbytes13_to_f16(hi),
                      pk_times16_f16(sbytes02_to_f16(lo)), pk_times16_f16(sbytes13_to_f16(lo)));
}

// Staging swizzle of the fp16 A image: in fragment (group j, row tile t)
// the slot of row r (0..15) in 16-byte chunk c (0..3) is c*16 + (r ^ f(s)),
// s = (c >> 1) + 2j, f = {0, 6, 10, 12}.  A staging store instruction writes
// four rows x the four chunk pairs of a 64-column step: unswizzled, its
// eight- and sixteen-lane groups land on two and four bank groups (2- and
// 4-way conflicts); with f every group hits distinct banks, and the MFMA
// reads (one chunk, sixteen rows) stay conflict-free.
__device__ __forceinline__ uint32_t a_swizzle(uint32_t s) { return (0xCA60u >> (4u * s)) & 15u; }

__device__ __forceinline__ v4f mfma_f16_16x16x32(uint4 a, uint4 b, v4f c) {
    typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, a),
                                                  __builtin_bit_cast(h8_t, b), c, 0, 0, 0);
}

// A workgroup of 8 waves covers 8 gate/up channel pairs (128 + 128
// channels) of one task; wave p owns pair p for all of the task's row tiles
// (1, 2, 4 or 8 of 16 rows, a compile-time choice per task), so each weight
// fragment, converted once per wave, feeds up to 8 MFMAs.  The workgroup
// stages half a quad (64 columns of K, two scale groups) at a time into a
// double-buffered LDS image of 26 KB: the task's rows as fp16 MFMA
// fragments, its 16 weight tiles and their scale words; every thread loads
// one 16-byte row piece, two 8-byte weight pieces and (half of them) one
// scale word a step ahead and converts the row piece when it stores it.
// The barrier between steps waits for LDS operations only.  Two workgroups
// share a CU (8 waves each at 4 waves per SIMD), so one's barriers,
// prologue and epilogue overlap the other's MFMAs.  fp16 scales carry
// 16 * y, bf16 scales take s / 16, as in the int8 kernel above; the
// epilogue is the same.
template <uint32_t H, uint32_t I, bool kBf16>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4)))
void gate_up_w4g32_f16_kernel(const uint4* __restrict__ w, const uint16_t* __restrict__ s,
                              const int8_t* __restrict__ xq, const float* __restrict__ xs,
                              const uint32_t* __restrict__ packed,
                              const float* __restrict__ route_weights,
                              const q38m_task_v1* __restrict__ tasks,
                              const uint32_t* __restrict__ live_tasks, uint16_t* __restrict__ mid) {
    constexpr uint32_t kHalves = H / 64u;  // staging steps
    constexpr uint32_t kTilesAll = 2u * I / 16u;
    constexpr uint32_t kWgTiles = 16u;  // 8 pairs
    static_assert(kHalves % 2u == 0u, "steps run in pairs of LDS buffers");
    // per buffer: A [K step j][row tile][lane] fp16 fragments (16 B), the
    // workgroup's 16 weight tiles [tile][K step j][lane] (one word: eight
    // nibbles) and their scale words [tile][channel] (two groups)
    __shared__ __align__(16) uint4 a_lds[2][2u * kRowTiles * 64u];
    __shared__ __align__(16) uint32_t w_lds[2][kWgTiles * 2u * 64u];
    __shared__ __align__(16) uint32_t s_lds[2][kWgTiles * 16u];
    __shared__ float2 row_info[kWideRows];  // (token scale, route weight)

    Placement at;
    if (!place_on_xcds(live_tasks, at)) return;
    const TaskRecord task = read_task(tasks, at.task);
    const uint32_t rows = task.rows;
    if (rows == 0u) return;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t pr = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t n = lane & 15u, qh = lane >> 4;
    const uint32_t e = task.expert;
    const uint32_t p0 = task.begin;
    const uint32_t tiles = __builtin_amdgcn_readfirstlane((rows + 15u) / 16u);

    // staging: row piece (row tid/4, 16-byte chunk tid%4 of the step's 64
    // bytes), weight pieces (tiles tid/64 and 8 + tid/64, lane tid%64: the
    // step's two words of the quad's four), scale piece (tile, channel) =
    // tid for tid < 256 (the step's two group words of the quad's four)
    const uint32_t sr = tid >> 2, sch = tid & 3u;
    const bool alive = sr < rows;
    const uint32_t assignment = alive ? checked(packed[p0 + sr], Q38M_WIDE_MAX_TOKENS * kTopK, kCheckToken) : 0u;
    if (sch == 0u && alive)
        row_info[sr] = make_float2(xs[assignment / kTopK], route_weights[assignment]);
    const uint4* a_src =
        reinterpret_cast<const uint4*>(xq + static_cast<size_t>(assignment / kTopK) * H) + sch;
    const uint32_t a_at = ((sch >> 1) * kRowTiles + (sr >> 4)) * 64u + (sch & 1u) * 32u +
                          ((sr & 15u) ^ a_swizzle(sch));
    const size_t slot0 = static_cast<size_t>(e) * (H / 128u) * kTilesAll + at.slice * kWgTiles;
    const uint2* w_src = reinterpret_cast<const uint2*>(w + slot0 * 64u + tid);
    // threads past the scale piece re-read thread tid % 256's word and
    // store the same value to the same LDS word
    const uint32_t s_at = tid % (kWgTiles * 16u);
    const uint32_t* s_src =
        reinterpret_cast<const uint32_t*>(s) + slot0 * 32u + 2u * s_at;
    struct Stage {
        uint4 a;
        uint2 w0, w1;
        uint32_t s;
    };
    // step h: quad h/2, words 2(h%2), 2(h%2)+1 of each weight piece and
    // scale record.  Every thread issues the same loads unconditionally (a
    // row past the task reads token 0's row, whose products land in rows
    // that are never stored), so the wait before each LDS store covers
    // exactly that step's loads and nothing waits on a prefetch early.
    auto load_stage = [&](uint32_t h) __attribute__((always_inline)) {
        Stage st;
        st.a = a_src[h * 4u];
        const uint2* wq = w_src + (static_cast<size_t>(h >> 1) * kTilesAll * 64u) * 2u + (h & 1u);
        st.w0 = wq[0];
        st.w1 = wq[8u * 64u * 2u];
        st.s = s_src[static_cast<size_t>(h >> 1) * kTilesAll * 32u + (h & 1u)];
        return st;
    };
    auto store_stage = [&](const Stage& st, uint32_t buffer) __attribute__((always_inline)) {
        a_lds[buffer][a_at] = i8_to_f16(st.a.x, st.a.y);
        a_lds[buffer][a_at + 16u] = i8_to_f16(st.a.z, st.a.w);
        const uint32_t w_at = (tid >> 6) * 128u + lane;
        w_lds[buffer][w_at] = st.w0.x;
        w_lds[buffer][w_at + 64u] = st.w0.y;
        w_lds[buffer][w_at + 8u * 128u] = st.w1.x;
        w_lds[buffer][w_at + 8u * 128u + 64u] = st.w1.y;
        s_lds[buffer][s_at] = st.s;
    };

    float y[kRowTiles][2][4];
#pragma unroll
    for (uint32_t t = 0; t < kRowTiles; ++t)
#pragma unroll
        for (uint32_t u = 0; u < 2u; ++u)
#pragma unroll
            for (uint32_t i = 0; i < 4u; ++i) y[t][u][i] = 0.0f;
    const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};

    // One step for kNt row tiles: per K step (= scale group) the pair's two
    // weight fragments are converted once; chain k = (row tile, gate/up),
    // tile t+1's A fragment read one chain ahead, each chain's fma step
    // issued after the next chain's MFMA.
    auto multiply = [&](auto ntiles, uint32_t buffer) __attribute__((always_inline)) {
        constexpr uint32_t kNt = decltype(ntiles)::value;
        constexpr uint32_t kChains = 2u * kNt * 2u;
        // lane l reads row l%16 of chunk l/16, through the staging swizzle
        const uint4* abuf0 = a_lds[buffer] + ((lane & 48u) | ((lane & 15u) ^ a_swizzle(lane >> 5)));
        const uint4* abuf1 = a_lds[buffer] + ((lane & 48u) | ((lane & 15u) ^ a_swizzle((lane >> 5) + 2u)));
        const uint32_t* srow = s_lds[buffer] + (2u * pr) * 16u + n;  // up: + 16 words
        // the step's scale words (gate, up; two groups each), read before
        // the first MFMA instead of one LDS round trip per group
        const uint32_t sword[2] = {srow[0], srow[16u]};
        const uint32_t* wrow = w_lds[buffer] + (2u * pr) * 128u + lane;  // up: + 128
        uint4 fa[2];
        uint4 bf[2];
        float sc[2];
        v4f d[2];
        auto issue = [&](uint32_t k) __attribute__((always_inline)) {
            const uint32_t m = k / 2u, u = k & 1u;
            const uint32_t j = m / kNt, t = m % kNt;
            if (u == 0u) {
                if (t == 0u) {
                    bf[0] = w4_to_f16x16(wrow[j * 64u]);
                    bf[1] = w4_to_f16x16(wrow[128u + j * 64u]);
                }
                if (m + 1u < 2u * kNt) {
                    const uint32_t jn = (m + 1u) / kNt, tn = (m + 1u) % kNt;
                    fa[(m + 1u) & 1u] = (jn == 0u ? abuf0 : abuf1)[(jn * kRowTiles + tn) * 64u];
                }
            }
            d[k & 1u] = mfma_f16_16x16x32(fa[m & 1u], bf[u], zero);
        };
        auto step = [&](uint32_t k) __attribute__((always_inline)) {
            const uint32_t m = k / 2u, u = k & 1u;
            const uint32_t j = m / kNt, t = m % kNt;
            if (t == 0u) {
                const uint32_t word = (sword[u] >> (16u * j)) & 0xFFFFu;
                sc[u] = kBf16 ? bf16_to_f32(word) * 0.0625f : f16_to_f32(word);
                asm volatile("" : "+v"(sc[u]));  // a plain v_fma_f32, not v_fma_mix
            }
#pragma unroll
            for (uint32_t i = 0; i < 4u; ++i)
                y[t][u][i] = __builtin_fmaf(d[k & 1u][i], sc[u], y[t][u][i]);
            // keep the step between the MFMAs it follows and precedes
            asm volatile("" : "+v"(y[t][u][0]), "+v"(y[t][u][1]), "+v"(y[t][u][2]),
                         "+v"(y[t][u][3]));
        };
        fa[0] = abuf0[0];
#pragma unroll
        for (uint32_t k = 0; k <= kChains; ++k) {
            if (k < kChains) issue(k);
            __builtin_amdgcn_sched_barrier(0);
            if (k > 0u) step(k - 1u);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto lds_barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

    // step h: loaded at the start of step h-1, stored at its end into LDS
    // buffer h%2, multiplied during step h; the loop is instantiated per
    // row-tile count, every instance passing the same barriers
    {
        const Stage first = load_stage(0);
        store_stage(first, 0u);
    }
    __syncthreads();
    auto k_loop = [&](auto ntiles) __attribute__((always_inline)) {
#pragma unroll 1
        for (uint32_t h = 0; h < kHalves; h += 2u) {
            Stage next = load_stage(h + 1u);
            __builtin_amdgcn_sched_barrier(0);
            multiply(ntiles, 0u);
            store_stage(next, 1u);
            lds_barrier();
            // the last pair's second load repeats step h + 1 into buffer 0,
            // which nothing reads after it (unconditional, so the loads stay
            // ahead of the multiply instead of sinking into a branch)
            next = load_stage(h + 2u < kHalves ? h + 2u : h + 1u);
            __builtin_amdgcn_sched_barrier(0);
            multiply(ntiles, 1u);
            store_stage(next, 0u);
            lds_barrier();
        }
    };
    if (tiles > 4u)
        k_loop(std::integral_constant<uint32_t, 8>{});
    else if (tiles > 2u)
        k_loop(std::integral_constant<uint32_t, 4>{});
    else if (tiles > 1u)
        k_loop(std::integral_constant<uint32_t, 2>{});
    else
        k_loop(std::integral_constant<uint32_t, 1>{});

    // SwiGLU (swiglu_fold's rounding sequence with silu(g) from the table,
    // NaN written as 0x7fc0 like swiglu_fold):
    // D lane (qh, n) holds rows 4qh + i of each tile, channel n.  Four
    // tiles' gathers are in flight before their first store.
    const uint32_t channel = (at.slice * 8u + pr) * 16u + n;
    const float unscale = kBf16 ? 1.0f : 0.0625f;
    constexpr uint32_t kBatch = 4u;
#pragma unroll
    for (uint32_t t0 = 0; t0 < kRowTiles; t0 += kBatch) {
        if (16u * t0 >= rows) break;
        uint32_t silu_word[kBatch][4];
        float up_value[kBatch][4];
#pragma unroll
        for (uint32_t b = 0; b < kBatch; ++b)
#pragma unroll
            for (uint32_t i = 0; i < 4u; ++i) {
                const uint32_t r = 16u * (t0 + b) + 4u * qh + i;
                const float st = row_info[r < rows ? r : 0u].x;
                const float yg = (y[t0 + b][0][i] * unscale) * st;
                up_value[b][i] = bf16_round((y[t0 + b][1][i] * unscale) * st);
                silu_word[b][i] = kSiluTable[f32_to_bf16(yg)];
            }
#pragma unroll
        for (uint32_t b = 0; b < kBatch; ++b)
#pragma unroll
            for (uint32_t i = 0; i < 4u; ++i) {
                const uint32_t r = 16u * (t0 + b) + 4u * qh + i;
                if (r >= rows) continue;
                const float h = bf16_round(__uint_as_float(silu_word[b][i]) * up_value[b][i]);
                mid[static_cast<size_t>(p0 + r) * I + channel] = static_cast<uint16_t>(
                    bf16_canonical_nan(f32_to_bf16(h * row_info[r].y)));
            }
    }
}

// Gate/up, W8 (paired K-block-major layout; the reference's edge-layer
// format) over a task of up to 128 rows: the W4 kernel's plan with 64-wide
// K blocks -- 16 waves (8 gate tiles, 8 up tiles), one tile per wave for
// kTiles 16-row tiles, A staged one K block (8 KiB) at a time into a
// double-buffered LDS image [row tile][lane] of 16-byte fragments, weights
// two blocks ahead.  Groups of one block (64 columns): per tile one
// v_mfma_i32_16x16x64_i8 from zero, then y = fma((float)acc, s_g, y) with
// the MFMA/fma interleave pinned; groups of two blocks or per channel: each
// tile's int32 accumulator chains through the MFMA input (kTiles more
// registers) and joins the chain at the group's last block (per channel:
// y = (float)acc * s at the end).  Scales in the artifact order.
template <uint32_t H, uint32_t I, uint32_t kThreads, uint32_t kTiles, uint32_t kBlocksPerGroup,
          bool kBf16>
__device__ __forceinline__ void gate_up_w8_wide_rows(
    const uint4* __restrict__ wbase, const uint16_t* __restrict__ srow,
    const int8_t* __restrict__ xq, const float* __restrict__ xs,
    const uint32_t* __restrict__ packed, const float* __restrict__ route_weights,
    uint16_t* __restrict__ mid, uint4 (*a_lds)[kRowTiles * 64u], float* gate_lds,
    uint32_t rows, uint32_t p0, uint32_t pair, bool up) {
    constexpr uint32_t kBlocks = H / 64u;
    constexpr uint32_t kBlockWords = 2u * I / 16u * 64u;  // uint4 per K block of one expert
    constexpr bool kPerChannel = kBlocksPerGroup == kBlocks;
    constexpr uint32_t kPieces = kTiles * 16u * 4u;  // 16-byte row pieces per block
    constexpr uint32_t kPerThread = (kPieces + kThreads - 1u) / kThreads;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t n = lane & 15u;
    const uint32_t q = lane >> 4;
    const uint32_t wave_in_half = (threadIdx.x >> 6) & 7u;
    const v4i zero = {0, 0, 0, 0};

    struct Block {
        uint4 w;     // the tile's 16 bytes of one K block
        uint32_t s;  // the scale word of the block's group
    };
    auto load = [&](uint32_t kb) {
        const uint32_t k = kb < kBlocks ? kb : kBlocks - 1u;  // past the end: re-read (L1 hit)
        const uint32_t g = kPerChannel ? 0u : k / kBlocksPerGroup;
        return Block{wbase[k * kBlockWords + lane], static_cast<uint32_t>(srow[g])};
    };

    // Piece i: row r = i/4, 16-byte piece c = i%4 of the row's 64 bytes of
    // the block (lane group c).  Rows past valid_rows stage zeros.
    const uint4* row_src[kPerThread];
    uint32_t lds_at[kPerThread];
    bool alive[kPerThread], staged[kPerThread];
#pragma unroll
    for (uint32_t u = 0; u < kPerThread; ++u) {
        const uint32_t i = threadIdx.x + u * kThreads;
        const uint32_t r = i / 4u, c = i % 4u;
        staged[u] = i < kPieces;
        alive[u] = staged[u] && r < rows;
        const uint32_t token = alive[u] ? checked(packed[p0 + r], Q38M_WIDE_MAX_TOKENS * kTopK, kCheckToken) / kTopK : 0u;
        row_src[u] = reinterpret_cast<const uint4*>(xq + static_cast<size_t>(token) * H) + c;
        lds_at[u] = (r / 16u) * 64u + c * 16u + r % 16u;
    }
    uint4 pieces[kPerThread];
    auto load_a = [&](uint32_t kb) {
#pragma unroll
        for (uint32_t u = 0; u < kPerThread; ++u)
            pieces[u] = alive[u] ? row_src[u][kb * 4u] : make_uint4(0u, 0u, 0u, 0u);
    };
    auto store_a = [&](uint32_t buffer) {
#pragma unroll
        for (uint32_t u = 0; u < kPerThread; ++u)
            if (staged[u]) a_lds[buffer][lds_at[u]] = pieces[u];
    };

    float y[kTiles][4];
    v4i acc[kTiles];  // groups of two blocks / per channel: the running int32 tiles
#pragma unroll
    for (uint32_t t = 0; t < kTiles; ++t) {
        acc[t] = zero;
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) y[t][i] = 0.0f;
    }

    auto multiply = [&](uint32_t kb, const Block& b) {
        const uint4* abuf = a_lds[kb & 1u] + lane;
        const v4i bw = as_v4i(b.w);
        const float scale = kBf16 ? bf16_to_f32(b.s) : f16_to_f32(b.s);
        if constexpr (kBlocksPerGroup == 1u) {
            v4i d[2];
            d[0] = mfma_i8_16x16x64(as_v4i(abuf[0]), bw, zero);
#pragma unroll
            for (uint32_t t = 0; t < kTiles; ++t) {
                if (t + 1u < kTiles)
                    d[(t + 1u) & 1u] = mfma_i8_16x16x64(as_v4i(abuf[(t + 1u) * 64u]), bw, zero);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    y[t][i] = __builtin_fmaf(static_cast<float>(d[t & 1u][i]), scale, y[t][i]);
                asm volatile("" : "+v"(y[t][0]), "+v"(y[t][1]), "+v"(y[t][2]), "+v"(y[t][3]));
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            const bool first = kb % kBlocksPerGroup == 0u;
#pragma unroll
            for (uint32_t t = 0; t < kTiles; ++t)
                acc[t] = mfma_i8_16x16x64(as_v4i(abuf[t * 64u]), bw, first ? zero : acc[t]);
            if constexpr (!kPerChannel) {
                if (kb % kBlocksPerGroup == kBlocksPerGroup - 1u) {
#pragma unroll
                    for (uint32_t t = 0; t < kTiles; ++t)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            y[t][i] = __builtin_fmaf(static_cast<float>(acc[t][i]), scale, y[t][i]);
                }
            }
        }
    };
    // one block: weights two ahead into the set just consumed, A one ahead
    auto step = [&](uint32_t kb, const Block& cur, Block& refill) {
        refill = load(kb + 2u);
        if (kb + 1u < kBlocks) load_a(kb + 1u);
        __builtin_amdgcn_sched_barrier(0);
        multiply(kb, cur);
        if (kb + 1u < kBlocks) store_a((kb + 1u) & 1u);
        __syncthreads();
    };

    load_a(0);
    Block r0 = load(0), r1 = load(1), r2;
    store_a(0);
    __syncthreads();
    static_assert(kBlocks % 3u == 2u, "three-set rotation plus two peeled blocks");
#pragma unroll 1
    for (uint32_t kb = 0; kb + 2u < kBlocks; kb += 3u) {
        step(kb, r0, r2);
        step(kb + 1u, r1, r0);
        step(kb + 2u, r2, r1);
    }
    step(kBlocks - 2u, r0, r2);
    multiply(kBlocks - 1u, r1);
    if constexpr (kPerChannel) {
        const float scale = kBf16 ? bf16_to_f32(r1.s) : f16_to_f32(r1.s);
#pragma unroll
        for (uint32_t t = 0; t < kTiles; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) y[t][i] = static_cast<float>(acc[t][i]) * scale;
    }

    // gate waves hand y over: gate_lds[pair in workgroup][row][channel],
    // over the A image, once every wave has finished reading it
    float* handoff = gate_lds + wave_in_half * (kWideRows * 16u);
    __syncthreads();
    if (!up) {
#pragma unroll
        for (uint32_t t = 0; t < kTiles; ++t)
#pragma unroll
            for (uint32_t i = 0; i < 4u; ++i) handoff[(16u * t + 4u * q + i) * 16u + n] = y[t][i];
    }
    __syncthreads();
    if (!up) return;
    const uint32_t channel = pair * 16u + n;
#pragma unroll
    for (uint32_t t = 0; t < kTiles; ++t) {
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) {
            const uint32_t r = 16u * t + 4u * q + i;
            if (r >= rows) continue;
            const uint32_t p = p0 + r;
            const uint32_t a = checked(packed[p], Q38M_WIDE_MAX_TOKENS * kTopK, kCheckToken);
            const float st = xs[a / kTopK];
            mid[static_cast<size_t>(p) * I + channel] = static_cast<uint16_t>(
                swiglu_fold(handoff[r * 16u + n] * st, y[t][i] * st, route_weights[a]));
        }
    }
}

template <uint32_t H, uint32_t I, uint32_t kPairs, uint32_t kBlocksPerGroup, bool kBf16>
__global__ __launch_bounds__(kPairs * 128) __attribute__((amdgpu_waves_per_eu(4)))
void gate_up_w8_wide_kernel(
    const uint4* __restrict__ w, const uint16_t* __restrict__ s,
    const int8_t* __restrict__ xq, const float* __restrict__ xs,
    const uint32_t* __restrict__ packed, const float* __restrict__ route_weights,
    const q38m_task_v1* __restrict__ tasks, const uint32_t* __restrict__ live_tasks, uint16_t* __restrict__ mid) {
    constexpr uint32_t kBlocks = H / 64u;
    constexpr uint32_t kSlots = 2u * I / 16u;
    constexpr uint32_t kGroups = kBlocks / kBlocksPerGroup;
    constexpr uint32_t kThreads = kPairs * 128u;
    // the A image (two blocks) and, after the K loop, the gate hand-off
    constexpr uint32_t kABytes = 2u * kRowTiles * 64u * 16u;
    constexpr uint32_t kHandoffBytes = kPairs * kWideRows * 16u * 4u;
    __shared__ __align__(16) uint8_t lds[kABytes > kHandoffBytes ? kABytes : kHandoffBytes];
    auto a_lds = reinterpret_cast<uint4 (*)[kRowTiles * 64u]>(lds);
    float* gate_lds = reinterpret_cast<float*>(lds);

    Placement at;
    if (!place_on_xcds(live_tasks, at)) return;
    const TaskRecord task = read_task(tasks, at.task);
    const uint32_t rows = task.rows;
    if (rows == 0u) return;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool up = wave >= kPairs;
    const uint32_t pair = at.slice * kPairs + (wave % kPairs);
    const uint32_t e = task.expert;
    const uint32_t p0 = task.begin;
    const uint32_t n = threadIdx.x & 15u;
    // paired K-block-major layout: for block kb the gate tile of pair p is
    // slot 2p and its up tile slot 2p+1
    const uint32_t slot = 2u * pair + (up ? 1u : 0u);
    const uint4* wbase = w + (static_cast<size_t>(e) * kBlocks * kSlots + slot) * 64u;
    const uint16_t* srow =
        s + (static_cast<size_t>(e) * 2u * I + (up ? I : 0u) + pair * 16u + n) * kGroups;
    const uint32_t tiles = (rows + 15u) / 16u;  // uniform per workgroup
    auto run = [&](auto row_tiles) {
        gate_up_w8_wide_rows<H, I, kThreads, decltype(row_tiles)::value, kBlocksPerGroup, kBf16>(
            wbase, srow, xq, xs, packed, route_weights, mid, a_lds, gate_lds, rows, p0, pair, up);
    };
    if (tiles > 4u)
        run(std::integral_constant<uint32_t, 8>{});
    else if (tiles > 2u)
        run(std::integral_constant<uint32_t, 4>{});
    else if (tiles == 2u)
        run(std::integral_constant<uint32_t, 2>{});
    else
        run(std::integral_constant<uint32_t, 1>{});
}

// ---- down -------------------------------------------------------------------

// The route outputs of a chunk (fp32 [R][H], 2.68 GB for a config-5 layer)
// are written once here and read once by the combine, far more than the
// L2s hold: stored with ordinary stores they are allocated in L2 and evict
// the expert weights and mid rows that an expert's later tasks re-read
// (the W8 down kernel fetched 1.44x its unique bytes), so they are stored
// non-temporally.
__device__ __forceinline__ void store_route_output(float* p, float v) {
    __builtin_nontemporal_store(v, p);
}

// Down, W8 per output channel, over a task of up to 128 rows: the mid rows
// (contiguous in packed order) are staged once into LDS as [K block][row
// tile][lane] 16-byte MFMA fragments.  Each wave owns kTilesPerWave
// 16-channel output tiles and walks K in the outer loop: a K block's kRows
// A fragments are read from LDS once and multiplied into every owned tile
// (v_mfma_i32_16x16x64_i8), with the tiles' weight fragments two K blocks
// ahead.  One A fragment is live at a time (row by row): holding all kRows
// of them took the kernel to 256 VGPRs with spills (1.07 ms vs 1.00 ms on
// a config-5 layer).  kRows (8, 4, 2 or 1 row tiles) is picked per task from its row
// count.  Per channel (kBlocksPerGroup == I/64): o = ((float)acc * ws[e][c])
// * sm[r], as the slab kernel.  Groups of 64 or 128 columns (kBlocksPerGroup
// 1 or 2 K blocks): acc restarts at each group's first block and, at its
// last, joins the fp32 chain y = fma((float)acc, s[e][c][g], y) in group
// order; o = y * sm[r].
template <uint32_t H, uint32_t I, uint32_t kTilesPerWave, uint32_t kRows,
          uint32_t kBlocksPerGroup, bool kBf16>
__device__ __forceinline__ void down_w8_wide_rows(const uint4* __restrict__ wt,
                                                  const uint16_t* __restrict__ ws_expert,
                                                  const uint4* a_lds, const float* row_scale,
                                                  uint32_t rows, uint32_t p0, uint32_t tile0,
                                                  float* __restrict__ out) {
    constexpr uint32_t kBlocks = I / 64u;
    constexpr bool kPerChannel = kBlocksPerGroup == kBlocks;
    constexpr uint32_t kGroups = kBlocks / kBlocksPerGroup;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t n = lane & 15u;
    const uint32_t q = lane >> 4;
    const v4i zero = {0, 0, 0, 0};
    // the tiles' scales of channel 16*(tile0+t)+n, artifact order
    // [E][rows][groups]; per channel read after the K loop (fewer live VGPRs)
    float ws[kTilesPerWave][kGroups];
    auto load_scales = [&]() {
#pragma unroll
        for (uint32_t t = 0; t < kTilesPerWave; ++t)
#pragma unroll
            for (uint32_t g = 0; g < kGroups; ++g) {
                const uint32_t word = ws_expert[((tile0 + t) * 16u + n) * kGroups + g];
                ws[t][g] = kBf16 ? bf16_to_f32(word) : f16_to_f32(word);
            }
    };
    if constexpr (!kPerChannel) load_scales();
    v4i acc[kTilesPerWave][kRows];
    float y[kTilesPerWave][kRows][4];  // grouped: the fp32 chain
#pragma unroll
    for (uint32_t t = 0; t < kTilesPerWave; ++t)
#pragma unroll
        for (uint32_t r = 0; r < kRows; ++r) {
            acc[t][r] = zero;
#pragma unroll
            for (uint32_t i = 0; i < 4u; ++i) y[t][r][i] = 0.0f;
        }
    // tile t's K block kb: wt[(t * kBlocks + kb) * 64]
    uint4 wq[3][kTilesPerWave];
    auto load_w = [&](uint32_t kb, uint4 (&dst)[kTilesPerWave]) {
        const uint32_t k = kb < kBlocks ? kb : kBlocks - 1u;
#pragma unroll
        for (uint32_t t = 0; t < kTilesPerWave; ++t) dst[t] = wt[(t * kBlocks + k) * 64u];
    };
    load_w(0, wq[0]);
    load_w(1, wq[1]);
#pragma unroll
    for (uint32_t kb = 0; kb < kBlocks; ++kb) {
        load_w(kb + 2u, wq[(kb + 2u) % 3u]);
#pragma unroll
        for (uint32_t r = 0; r < kRows; ++r) {
            const v4i a = as_v4i(a_lds[(kb * kRowTiles + r) * 64u + lane]);
#pragma unroll
            for (uint32_t t = 0; t < kTilesPerWave; ++t)
                acc[t][r] = mfma_i8_16x16x64(a, as_v4i(wq[kb % 3u][t]),
                                             !kPerChannel && kb % kBlocksPerGroup == 0u
                                                 ? zero
                                                 : acc[t][r]);
        }
        if constexpr (!kPerChannel) {
            if (kb % kBlocksPerGroup == kBlocksPerGroup - 1u) {
#pragma unroll
                for (uint32_t t = 0; t < kTilesPerWave; ++t)
#pragma unroll
                    for (uint32_t r = 0; r < kRows; ++r)
#pragma unroll
                        for (uint32_t i = 0; i < 4u; ++i)
                            y[t][r][i] = __builtin_fmaf(static_cast<float>(acc[t][r][i]),
                                                        ws[t][kb / kBlocksPerGroup], y[t][r][i]);
            }
            // one K block's tiles live at a time (unpinned, the zero-started
            // blocks would all be issued at once)
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if constexpr (kPerChannel) load_scales();
    // a row's kTilesPerWave adjacent 16-channel pieces go out in consecutive
    // stores, so its 64*kTilesPerWave bytes meet in L2 as whole lines
#pragma unroll
    for (uint32_t r = 0; r < kRows; ++r)
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) {
            const uint32_t row = 16u * r + 4u * q + i;
            if (row >= rows) continue;
            const float sm = row_scale[row];
            float* dst = out + static_cast<size_t>(p0 + row) * H + tile0 * 16u + n;
#pragma unroll
            for (uint32_t t = 0; t < kTilesPerWave; ++t)
                store_route_output(dst + 16u * t,
                                   kPerChannel ? (static_cast<float>(acc[t][r][i]) * ws[t][0]) * sm
                                               : y[t][r][i] * sm);
        }
}

template <uint32_t H, uint32_t I, uint32_t kWaves, uint32_t kTilesPerWave,
          uint32_t kBlocksPerGroup, bool kBf16>
__global__ __launch_bounds__(kWaves * 64) void down_w8_wide_kernel(
    const uint4* __restrict__ w, const uint16_t* __restrict__ s,
    const int8_t* __restrict__ mq, const float* __restrict__ ms,
    const q38m_task_v1* __restrict__ tasks, const uint32_t* __restrict__ live_tasks, float* __restrict__ out) {
    constexpr uint32_t kBlocks = I / 64u;
    constexpr uint32_t kTiles = H / 16u;
    constexpr uint32_t kThreads = kWaves * 64u;
    constexpr uint32_t kPieces = kWideRows * (I / 16u);
    static_assert(kPieces % kThreads == 0u, "whole pieces per thread");
    __shared__ uint4 a_lds[kBlocks * kRowTiles * 64u];
    __shared__ float row_scale[kWideRows];

    Placement at;
    if (!place_on_xcds(live_tasks, at)) return;
    const TaskRecord task = read_task(tasks, at.task);
    const uint32_t rows = task.rows;
    if (rows == 0u) return;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t e = task.expert;
    const uint32_t p0 = task.begin;
    const uint32_t tile0 = (at.slice * kWaves + wave) * kTilesPerWave;
    const uint4* wt = w + static_cast<size_t>(e * kTiles + tile0) * kBlocks * 64u + lane;
    const uint32_t tiles = (rows + 15u) / 16u;  // uniform per workgroup

    // Piece i: row r = i / (I/16), 16-byte piece c: K block c/4, lane group
    // c%4.  Every load is issued before the first store (rows past the task
    // re-read its first row and stage zeros), so staging is one round trip.
    constexpr uint32_t kPer = kPieces / kThreads;
    uint4 v[kPer];
#pragma unroll
    for (uint32_t u = 0; u < kPer; ++u) {
        const uint32_t i = threadIdx.x + u * kThreads;
        const uint32_t r = i / (I / 16u), c = i % (I / 16u);
        v[u] = reinterpret_cast<const uint4*>(mq + static_cast<size_t>(p0 + (r < rows ? r : 0u)) *
                                                       I)[c];
    }
#pragma unroll
    for (uint32_t u = 0; u < kPer; ++u) {
        const uint32_t i = threadIdx.x + u * kThreads;
        const uint32_t r = i / (I / 16u), c = i % (I / 16u);
        if (r < 16u * tiles)
            a_lds[((c >> 2) * kRowTiles + r / 16u) * 64u + (c & 3u) * 16u + r % 16u] =
                r < rows ? v[u] : make_uint4(0u, 0u, 0u, 0u);
    }
    if (threadIdx.x < kWideRows)
        row_scale[threadIdx.x] = threadIdx.x < rows ? ms[p0 + threadIdx.x] : 0.0f;
    __syncthreads();

    const uint16_t* ws_expert = s + static_cast<size_t>(e) * H * (kBlocks / kBlocksPerGroup);
    auto run = [&](auto row_tiles) {
        down_w8_wide_rows<H, I, kTilesPerWave, decltype(row_tiles)::value, kBlocksPerGroup,
                          kBf16>(wt, ws_expert, a_lds, row_scale, rows, p0, tile0, out);
    };
    if (tiles > 4u)
        run(std::integral_constant<uint32_t, 8>{});
    else if (tiles > 2u)
        run(std::integral_constant<uint32_t, 4>{});
    else if (tiles == 2u)
        run(std::integral_constant<uint32_t, 2>{});
    else
        run(std::integral_constant<uint32_t, 1>{});
}

// Down, W4 group-32 (the all-W4 layer policy), over a task of up to 128
// rows: the gate/up chain over K = I.  The mid rows are staged once in LDS
// as [group][row tile][lane] 8-byte fragments; a workgroup of 16 waves
// covers 32 output tiles, two per wave, kStride tiles apart: the two
// 64-byte halves of an output line come from neighbouring waves at about
// the same time and meet in L2 (adjacent tiles in one wave were stored a
// whole tile's chain apart, and 9 % of the route-output bytes went to HBM
// twice).  A wave streams its tiles' weights
// one quad ahead and runs the chain group by group with the
// same pinned MFMA/v_cvt/v_fma interleave as the gate/up kernel, over kRows
// (8, 4, 2 or 1) row tiles picked per task; groups of 64 or 128 columns
// chain their sub-blocks' int32 tiles as the gate/up kernel does.
template <uint32_t H, uint32_t I, uint32_t kTilesPerWave, uint32_t kStride, uint32_t kRows,
          uint32_t kSub, bool kBf16>
__device__ __forceinline__ void down_w4_wide_rows(const uint4* __restrict__ wt,
                                                  const uint16_t* __restrict__ st,
                                                  const uint2* a_lds, const float* row_scale,
                                                  uint32_t rows, uint32_t p0, uint32_t tile0,
                                                  float* __restrict__ out) {
    constexpr uint32_t kQuads = I / 128u;
    constexpr uint32_t kTiles = H / 16u;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t n = lane & 15u;
    const uint32_t q = lane >> 4;
    const uint2* abuf = a_lds + lane;
    const v4i zero = {0, 0, 0, 0};
    // quad-major layout: quad kq of tile t is unit kq*kTiles + t of the
    // expert; weights stream one quad ahead, across tile boundaries too
    auto load = [&](uint32_t t, uint32_t kq) {
        const uint32_t tt = t < kTilesPerWave ? t : kTilesPerWave - 1u;
        return TileQuad{wt[(kq * kTiles + tt * kStride) * 64u],
                        load_quad_scales<kSub, false>(st + (kq * kTiles + tt * kStride) * 16u *
                                                               (4u / kSub))};
    };
    TileQuad cur = load(0, 0);
#pragma unroll 1
    for (uint32_t t = 0; t < kTilesPerWave; ++t) {
        float y[kRows][4];
#pragma unroll
        for (uint32_t r = 0; r < kRows; ++r)
#pragma unroll
            for (uint32_t i = 0; i < 4u; ++i) y[r][i] = 0.0f;
#pragma unroll 1
        for (uint32_t kq = 0; kq < kQuads; ++kq) {
          const TileQuad next = kq + 1u < kQuads ? load(t, kq + 1u) : load(t + 1u, 0);
          const uint32_t bw[4] = {cur.w.x, cur.w.y, cur.w.z, cur.w.w};
          v4i chain[kRows];  // kSub > 1: the group's running int32 tiles
#pragma unroll
          for (uint32_t j = 0; j < 4u; ++j) {
            const uint32_t g = kq * 4u + j;
            long a[kRows];
#pragma unroll
            for (uint32_t r = 0; r < kRows; ++r) a[r] = as_long(abuf[(g * kRowTiles + r) * 64u]);
            const long bj = unpack_w4x16(bw[j]);
            if (j % kSub != kSub - 1u) {
#pragma unroll
              for (uint32_t r = 0; r < kRows; ++r)
                chain[r] = mfma_i8_16x16x32(a[r], bj, j % kSub == 0u ? zero : chain[r]);
              continue;
            }
            const uint32_t word = quad_scale_word(cur.s, j / kSub);
            const float scale = (kBf16 ? bf16_to_f32(word) : f16_to_f32(word)) * 0.0625f;
            // the group's int32 tile r: d[r & 1] (kSub == 1) or chain[r] in place
            v4i d[2];
            auto issue = [&](uint32_t r) {
                if constexpr (kSub == 1u) d[r & 1u] = mfma_i8_16x16x32(a[r], bj, zero);
                else chain[r] = mfma_i8_16x16x32(a[r], bj, chain[r]);
            };
            auto tile = [&](uint32_t r) -> const v4i& {
                if constexpr (kSub == 1u) return d[r & 1u];
                else return chain[r];
            };
            issue(0);
#pragma unroll
            for (uint32_t r = 0; r < kRows; ++r) {
                if (r + 1u < kRows) issue(r + 1u);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    y[r][i] = __builtin_fmaf(static_cast<float>(tile(r)[i]), scale, y[r][i]);
                asm volatile("" : "+v"(y[r][0]), "+v"(y[r][1]), "+v"(y[r][2]), "+v"(y[r][3]));
                __builtin_amdgcn_sched_barrier(0);
            }
          }
          cur = next;
        }
        const uint32_t channel = (tile0 + t * kStride) * 16u + n;
        // re-derived in every tile, so the 32 output addresses are not
        // hoisted out of the tile loop into registers
        uint32_t lane_row = 4u * q;
        asm volatile("" : "+v"(lane_row));
#pragma unroll
        for (uint32_t r = 0; r < kRows; ++r)
#pragma unroll
            for (uint32_t i = 0; i < 4u; ++i) {
                const uint32_t row = 16u * r + lane_row + i;
                if (row >= rows) continue;
                store_route_output(out + static_cast<size_t>(p0 + row) * H + channel,
                                   y[r][i] * row_scale[row]);
            }
    }
}

template <uint32_t H, uint32_t I, uint32_t kWaves, uint32_t kTilesPerWave, uint32_t kSub,
          bool kBf16>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(4)))
void down_w4_wide_kernel(
    const uint4* __restrict__ w, const uint16_t* __restrict__ s,
    const int8_t* __restrict__ mq, const float* __restrict__ ms,
    const q38m_task_v1* __restrict__ tasks, const uint32_t* __restrict__ live_tasks, float* __restrict__ out) {
    constexpr uint32_t kQuads = I / 128u;
    constexpr uint32_t kGroups = I / 32u;
    constexpr uint32_t kTiles = H / 16u;
    constexpr uint32_t kThreads = kWaves * 64u;
    constexpr uint32_t kPieces = kWideRows * (I / 16u);
    static_assert(kPieces % kThreads == 0u, "whole pieces per thread");
    __shared__ uint2 a_lds[kGroups * kRowTiles * 64u];
    __shared__ float row_scale[kWideRows];

    Placement at;
    if (!place_on_xcds(live_tasks, at)) return;
    const TaskRecord task = read_task(tasks, at.task);
    const uint32_t rows = task.rows;
    if (rows == 0u) return;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n = lane & 15u;
    const uint32_t e = task.expert;
    const uint32_t p0 = task.begin;

    // Piece i: row r, 16-byte piece c = group c/2, lane groups 2(c%2),
    // 2(c%2)+1; all loads before the first store.
    constexpr uint32_t kPer = kPieces / kThreads;
    uint4 v[kPer];
#pragma unroll
    for (uint32_t u = 0; u < kPer; ++u) {
        const uint32_t i = threadIdx.x + u * kThreads;
        const uint32_t r = i / (I / 16u), c = i % (I / 16u);
        v[u] = reinterpret_cast<const uint4*>(mq + static_cast<size_t>(p0 + (r < rows ? r : 0u)) *
                                                       I)[c];
    }
#pragma unroll
    for (uint32_t u = 0; u < kPer; ++u) {
        const uint32_t i = threadIdx.x + u * kThreads;
        const uint32_t r = i / (I / 16u), c = i % (I / 16u);
        const uint4 x = r < rows ? v[u] : make_uint4(0u, 0u, 0u, 0u);
        const uint32_t at = ((c >> 1) * kRowTiles + r / 16u) * 64u + (c & 1u) * 32u + r % 16u;
        a_lds[at] = make_uint2(x.x, x.y);
        a_lds[at + 16u] = make_uint2(x.z, x.w);
    }
    if (threadIdx.x < kWideRows)
        row_scale[threadIdx.x] = threadIdx.x < rows ? ms[p0 + threadIdx.x] : 0.0f;
    __syncthreads();

    // wave w: tiles tile0 + t * kWaves
    const uint32_t tile0 = at.slice * kWaves * kTilesPerWave + wave;
    const uint4* wt = w + (static_cast<size_t>(e) * kQuads * kTiles + tile0) * 64u + lane;
    const uint16_t* st =
        s + ((static_cast<size_t>(e) * kQuads * kTiles + tile0) * 16u + n) * (4u / kSub);
    const uint32_t tiles = (rows + 15u) / 16u;  // uniform per workgroup
    auto run = [&](auto row_tiles) {
        down_w4_wide_rows<H, I, kTilesPerWave, kWaves, decltype(row_tiles)::value, kSub, kBf16>(
            wt, st, a_lds, row_scale, rows, p0, tile0, out);
    };
    if (tiles > 4u)
        run(std::integral_constant<uint32_t, 8>{});
    else if (tiles > 2u)
        run(std::integral_constant<uint32_t, 4>{});
    else if (tiles == 2u)
        run(std::integral_constant<uint32_t, 2>{});
    else
        run(std::integral_constant<uint32_t, 1>{});
}

// Down, W4 groups of 32, on fp16 MFMA (see the gate/up kernel above for
// why the products are exact): a workgroup of 8 waves covers 16 output
// tiles of one task, two adjacent tiles per wave over all of the task's row
// tiles, so a row's 128-byte output line leaves one wave in two
// consecutive stores.  The mid rows are staged 64 columns at a time as fp16
// fragments in a double-buffered LDS image (16 KB per buffer); each wave
// streams its two tiles' weights and scale words one step ahead from
// global memory and converts each weight fragment once for all row tiles.
// The chain is the int8 kernel's: y = fmaf((float)acc_g, s_g / 16, y) in
// group order, then y * s_row.
template <uint32_t H, uint32_t I, bool kBf16>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4)))
void down_w4g32_f16_kernel(const uint4* __restrict__ w, const uint16_t* __restrict__ s,
                           const int8_t* __restrict__ mq, const float* __restrict__ ms,
                           const q38m_task_v1* __restrict__ tasks,
                           const uint32_t* __restrict__ live_tasks, float* __restrict__ out) {
    constexpr uint32_t kSteps = I / 64u;
    constexpr uint32_t kTiles = H / 16u;
    static_assert(kSteps % 2u == 0u, "steps run in pairs of LDS buffers");
    __shared__ __align__(16) uint4 a_lds[2][2u * kRowTiles * 64u];
    __shared__ float row_scale[kWideRows];

    Placement at;
    if (!place_on_xcds(live_tasks, at)) return;
    const TaskRecord task = read_task(tasks, at.task);
    const uint32_t rows = task.rows;
    if (rows == 0u) return;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t n = lane & 15u, qh = lane >> 4;
    const uint32_t e = task.expert;
    const uint32_t p0 = task.begin;
    const uint32_t tiles = __builtin_amdgcn_readfirstlane((rows + 15u) / 16u);

    // staging: row piece (row tid/4, 16-byte chunk tid%4 of the step's 64
    // bytes); the task's mid rows are contiguous
    const uint32_t sr = tid >> 2, sch = tid & 3u;
    const bool alive = sr < rows;
    const uint4* a_src =
        reinterpret_cast<const uint4*>(mq + static_cast<size_t>(p0 + (alive ? sr : 0u)) * I) + sch;
    const uint32_t a_at = ((sch >> 1) * kRowTiles + (sr >> 4)) * 64u + (sch & 1u) * 32u + (sr & 15u);
    if (tid < kWideRows) row_scale[tid] = tid < rows ? ms[p0 + tid] : 0.0f;
    auto load_a = [&](uint32_t h) __attribute__((always_inline)) {
        return alive ? a_src[h * 4u] : make_uint4(0u, 0u, 0u, 0u);
    };
    auto store_a = [&](const uint4& v, uint32_t buffer) __attribute__((always_inline)) {
        a_lds[buffer][a_at] = i8_to_f16(v.x, v.y);
        a_lds[buffer][a_at + 16u] = i8_to_f16(v.z, v.w);
    };

    // this wave's tiles tile0, tile0 + 1; quad-major layout: quad kq of tile
    // t is unit kq * kTiles + t of the expert, four K steps (one word each)
    // per lane and four scale words per channel; step h takes words
    // 2(h%2), 2(h%2)+1 of quad h/2
    const uint32_t tile0 = (at.slice * 8u + wave) * 2u;
    const size_t unit0 = static_cast<size_t>(e) * (I / 128u) * kTiles + tile0;
    const uint2* wsrc = reinterpret_cast<const uint2*>(w + unit0 * 64u + lane);
    const uint32_t* ssrc = reinterpret_cast<const uint32_t*>(s + (unit0 * 16u + n) * 4u);
    struct Step {
        uint2 w0, w1;
        uint32_t s0, s1;
    };
    auto load_w = [&](uint32_t h) __attribute__((always_inline)) {
        const size_t unit = static_cast<size_t>(h >> 1) * kTiles;
        Step st;
        st.w0 = wsrc[unit * 128u + (h & 1u)];
        st.w1 = wsrc[(unit + 1u) * 128u + (h & 1u)];
        st.s0 = ssrc[unit * 32u + (h & 1u)];
        st.s1 = ssrc[(unit + 1u) * 32u + (h & 1u)];
        return st;
    };

    float y[kRowTiles][2][4];
#pragma unroll
    for (uint32_t t = 0; t < kRowTiles; ++t)
#pragma unroll
        for (uint32_t u = 0; u < 2u; ++u)
#pragma unroll
            for (uint32_t i = 0; i < 4u; ++i) y[t][u][i] = 0.0f;
    const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};

    // one step (two groups) for kNt row tiles; chain k = (group j, row tile
    // t, tile u) as in the gate/up kernel
    auto multiply = [&](auto ntiles, uint32_t buffer, const Step& ws)
                        __attribute__((always_inline)) {
        constexpr uint32_t kNt = decltype(ntiles)::value;
        constexpr uint32_t kChains = 2u * kNt * 2u;
        const uint4* abuf = a_lds[buffer] + lane;
        const uint32_t wj[2][2] = {{ws.w0.x, ws.w0.y}, {ws.w1.x, ws.w1.y}};
        const uint32_t sj[2] = {ws.s0, ws.s1};
        uint4 fa[2];
        uint4 bf[2];
        float sc[2];
        v4f d[2];
        auto issue = [&](uint32_t k) __attribute__((always_inline)) {
            const uint32_t m = k / 2u, u = k & 1u;
            const uint32_t j = m / kNt, t = m % kNt;
            if (u == 0u) {
                if (t == 0u) {
                    bf[0] = w4_to_f16x16(wj[0][j]);
                    bf[1] = w4_to_f16x16(wj[1][j]);
                }
                if (m + 1u < 2u * kNt) {
                    const uint32_t jn = (m + 1u) / kNt, tn = (m + 1u) % kNt;
                    fa[(m + 1u) & 1u] = abuf[(jn * kRowTiles + tn) * 64u];
                }
            }
            d[k & 1u] = mfma_f16_16x16x32(fa[m & 1u], bf[u], zero);
        };
        auto step = [&](uint32_t k) __attribute__((always_inline)) {
            const uint32_t m = k / 2u, u = k & 1u;
            const uint32_t j = m / kNt, t = m % kNt;
            if (t == 0u) {
                const uint32_t word = j ? sj[u] >> 16 : sj[u] & 0xffffu;
                sc[u] = (kBf16 ? bf16_to_f32(word) : f16_to_f32(word)) * 0.0625f;
                asm volatile("" : "+v"(sc[u]));
            }
#pragma unroll
            for (uint32_t i = 0; i < 4u; ++i)
                y[t][u][i] = __builtin_fmaf(d[k & 1u][i], sc[u], y[t][u][i]);
            asm volatile("" : "+v"(y[t][u][0]), "+v"(y[t][u][1]), "+v"(y[t][u][2]),
                         "+v"(y[t][u][3]));
        };
        fa[0] = abuf[0];
#pragma unroll
        for (uint32_t k = 0; k <= kChains; ++k) {
            if (k < kChains) issue(k);
            __builtin_amdgcn_sched_barrier(0);
            if (k > 0u) step(k - 1u);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto lds_barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

    store_a(load_a(0), 0u);
    Step cur = load_w(0);
    __syncthreads();
    auto k_loop = [&](auto ntiles) __attribute__((always_inline)) {
#pragma unroll 1
        for (uint32_t h = 0; h < kSteps; h += 2u) {
            uint4 a_next = load_a(h + 1u);
            Step nxt = load_w(h + 1u);
            __builtin_amdgcn_sched_barrier(0);
            multiply(ntiles, 0u, cur);
            store_a(a_next, 1u);
            lds_barrier();
            cur = nxt;
            if (h + 2u < kSteps) {
                a_next = load_a(h + 2u);
                nxt = load_w(h + 2u);
            }
            __builtin_amdgcn_sched_barrier(0);
            multiply(ntiles, 1u, cur);
            if (h + 2u < kSteps) store_a(a_next, 0u);
            lds_barrier();
            cur = nxt;
        }
    };
    if (tiles > 4u)
        k_loop(std::integral_constant<uint32_t, 8>{});
    else if (tiles > 2u)
        k_loop(std::integral_constant<uint32_t, 4>{});
    else if (tiles > 1u)
        k_loop(std::integral_constant<uint32_t, 2>{});
    else
        k_loop(std::integral_constant<uint32_t, 1>{});

    const uint32_t channel = tile0 * 16u + n;
#pragma unroll
    for (uint32_t t = 0; t < kRowTiles; ++t) {
        if (16u * t >= rows) break;
#pragma unroll
        for (uint32_t i = 0; i < 4u; ++i) {
            const uint32_t row = 16u * t + 4u * qh + i;
            if (row >= rows) continue;
            float* dst = out + static_cast<size_t>(p0 + row) * H + channel;
            store_route_output(dst, y[t][0][i] * row_scale[row]);
            store_route_output(dst + 16, y[t][1][i] * row_scale[row]);
        }
    }
}

}  // namespace

uint32_t wide_chunks(uint32_t tokens) {
    return (routes_v1(tokens) + kWideChunkRoutes - 1u) / kWideChunkRoutes;
}

hipError_t launch_build_wide_plan(const int32_t* ids, uint32_t tokens,
                                  const q38m_route_plan_v1& plan, uint32_t* chunk_counts,
                                  hipStream_t stream) {
    const uint32_t routes = routes_v1(tokens);
    const uint32_t chunks = wide_chunks(tokens);
    wide_count_kernel<<<chunks, 256, 0, stream>>>(ids, routes, chunk_counts);
    wide_scan_kernel<<<1, 512, 0, stream>>>(chunk_counts, chunks, tokens, plan,
                                            max_tasks_wide(tokens));
    wide_scatter_kernel<<<chunks, 64, 0, stream>>>(ids, routes, chunk_counts, plan);
    return hipGetLastError();
}

namespace {

// the task slots a launch covers: grid rows, and the device word with the
// number the plan filled
struct TaskSlots {
    const q38m_task_v1* tasks;
    const uint32_t* live;
    uint32_t count;
};

template <uint32_t kSub, bool kBf16>
void launch_gate_up_wide_sub(const q38m_expert_weights_v1& w, const int8_t* xq, const float* xs,
                             const uint32_t* packed, const float* route_weights,
                             const TaskSlots& t, uint16_t* weighted_mid, hipStream_t stream) {
    if constexpr (kSub == 1u) {
        // fp16 MFMA form: 8 channel pairs (256 rows of gate/up) per workgroup
        const dim3 grid(kInter / 16u / 8u, t.count);
        gate_up_w4g32_f16_kernel<kHidden, kInter, kBf16>
            <<<grid, 512, 0, stream>>>(static_cast<const uint4*>(w.data),
                                        static_cast<const uint16_t*>(w.scales), xq, xs, packed,
                                        route_weights, t.tasks, t.live, weighted_mid);
        return;
    }
    // 8 channel pairs (256 rows of gate/up) per workgroup
    const dim3 grid(kInter / 16u / 8u, t.count);
    gate_up_w4_wide_kernel<kHidden, kInter, kSub, kBf16>
        <<<grid, 1024, 0, stream>>>(static_cast<const uint4*>(w.data),
                                    static_cast<const uint16_t*>(w.scales), xq, xs, packed,
                                    route_weights, t.tasks, t.live, weighted_mid);
}

// Per channel: four tiles per wave (the tuned BASELINE shape).  Grouped:
// the fp32 chain doubles the live accumulator state, so one tile per wave.
template <uint32_t kBlocksPerGroup, bool kBf16>
void launch_down_w8_wide_groups(const q38m_expert_weights_v1& w, const int8_t* mid_q,
                                const float* mid_s, const TaskSlots& t, float* route_output,
                                hipStream_t stream) {
    constexpr uint32_t kWaves = 8;
    constexpr uint32_t kTilesPerWave = kBlocksPerGroup == kInter / 64u ? 4u : 1u;
    const dim3 grid(kHidden / 16u / (kWaves * kTilesPerWave), t.count);
    down_w8_wide_kernel<kHidden, kInter, kWaves, kTilesPerWave, kBlocksPerGroup, kBf16>
        <<<grid, kWaves * 64u, 0, stream>>>(static_cast<const uint4*>(w.data),
                                            static_cast<const uint16_t*>(w.scales), mid_q, mid_s,
                                            t.tasks, t.live, route_output);
}

template <uint32_t kSub, bool kBf16>
void launch_down_w4_wide_sub(const q38m_expert_weights_v1& w, const int8_t* mid_q,
                             const float* mid_s, const TaskSlots& t, float* route_output,
                             hipStream_t stream) {
    if constexpr (kSub == 1u) {
        // fp16 MFMA form: 16 output tiles per 8-wave workgroup
        const dim3 grid(kHidden / 16u / 16u, t.count);
        down_w4g32_f16_kernel<kHidden, kInter, kBf16>
            <<<grid, 512, 0, stream>>>(static_cast<const uint4*>(w.data),
                                       static_cast<const uint16_t*>(w.scales), mid_q, mid_s,
                                       t.tasks, t.live, route_output);
        return;
    }
    constexpr uint32_t kWaves = 16, kTilesPerWave = 2;
    const dim3 grid(kHidden / 16u / (kWaves * kTilesPerWave), t.count);
    down_w4_wide_kernel<kHidden, kInter, kWaves, kTilesPerWave, kSub, kBf16>
        <<<grid, kWaves * 64u, 0, stream>>>(static_cast<const uint4*>(w.data),
                                            static_cast<const uint16_t*>(w.scales), mid_q, mid_s,
                                            t.tasks, t.live, route_output);
}

template <uint32_t kBlocksPerGroup, bool kBf16>
void launch_gate_up_w8_wide_groups(const q38m_expert_weights_v1& w, const int8_t* xq,
                                   const float* xs, const uint32_t* packed,
                                   const float* route_weights, const TaskSlots& t,
                                   uint16_t* weighted_mid, hipStream_t stream) {
    constexpr uint32_t kPairs = 8;
    const dim3 grid(kInter / 16u / kPairs, t.count);
    gate_up_w8_wide_kernel<kHidden, kInter, kPairs, kBlocksPerGroup, kBf16>
        <<<grid, kPairs * 128u, 0, stream>>>(static_cast<const uint4*>(w.data),
                                             static_cast<const uint16_t*>(w.scales), xq, xs,
                                             packed, route_weights, t.tasks, t.live,
                                             weighted_mid);
}

template <bool kBf16>
hipError_t launch_gate_up_wide_dtype(const q38m_expert_weights_v1& w, const int8_t* xq,
                                     const float* xs, const uint32_t* packed,
                                     const float* route_weights, const TaskSlots& t,
                                     uint16_t* mid, hipStream_t stream) {
    if (w.format == Q38M_FORMAT_W8_SYM) {
        switch (w.group_size) {
            case 0u:
                launch_gate_up_w8_wide_groups<kHidden / 64u, kBf16>(w, xq, xs, packed,
                                                                    route_weights, t, mid, stream);
                break;
            case 64u:
                launch_gate_up_w8_wide_groups<1, kBf16>(w, xq, xs, packed, route_weights, t, mid,
                                                        stream);
                break;
            case 128u:
                launch_gate_up_w8_wide_groups<2, kBf16>(w, xq, xs, packed, route_weights, t, mid,
                                                        stream);
                break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    switch (w.group_size) {
        case 32u: launch_gate_up_wide_sub<1, kBf16>(w, xq, xs, packed, route_weights, t, mid, stream); break;
        case 64u: launch_gate_up_wide_sub<2, kBf16>(w, xq, xs, packed, route_weights, t, mid, stream); break;
        case 128u: launch_gate_up_wide_sub<4, kBf16>(w, xq, xs, packed, route_weights, t, mid, stream); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <bool kBf16>
hipError_t launch_down_wide_dtype(const q38m_expert_weights_v1& w, const int8_t* mid_q,
                                  const float* mid_s, const TaskSlots& t, float* out,
                                  hipStream_t stream) {
    constexpr uint32_t kBlocks = kInter / 64u;
    if (w.format == Q38M_FORMAT_W8_SYM) {
        switch (w.group_size) {
            case 0u: launch_down_w8_wide_groups<kBlocks, kBf16>(w, mid_q, mid_s, t, out, stream); break;
            case 64u: launch_down_w8_wide_groups<1, kBf16>(w, mid_q, mid_s, t, out, stream); break;
            case 128u: launch_down_w8_wide_groups<2, kBf16>(w, mid_q, mid_s, t, out, stream); break;
            default: return hipErrorInvalidValue;
        }
    } else {
        switch (w.group_size) {
            case 32u: launch_down_w4_wide_sub<1, kBf16>(w, mid_q, mid_s, t, out, stream); break;
            case 64u: launch_down_w4_wide_sub<2, kBf16>(w, mid_q, mid_s, t, out, stream); break;
            case 128u: launch_down_w4_wide_sub<4, kBf16>(w, mid_q, mid_s, t, out, stream); break;
            default: return hipErrorInvalidValue;
        }
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gate_up_wide(const q38m_expert_weights_v1& w, const int8_t* xq, const float* xs,
                               const uint32_t* packed, const float* route_weights,
                               const q38m_task_v1* tasks, const uint32_t* live_tasks,
                               uint32_t task_count, uint16_t* weighted_mid, hipStream_t stream) {
    const TaskSlots t{tasks, live_tasks, task_count};
    return w.scale_dtype == Q38M_SCALE_BF16
               ? launch_gate_up_wide_dtype<true>(w, xq, xs, packed, route_weights, t,
                                                 weighted_mid, stream)
               : launch_gate_up_wide_dtype<false>(w, xq, xs, packed, route_weights, t,
                                                  weighted_mid, stream);
}

hipError_t launch_down_wide(const q38m_expert_weights_v1& w, const int8_t* mid_q,
                            const float* mid_s, const q38m_task_v1* tasks,
                            const uint32_t* live_tasks, uint32_t task_count,
                            float* route_output, hipStream_t stream) {
    const TaskSlots t{tasks, live_tasks, task_count};
    return w.scale_dtype == Q38M_SCALE_BF16
               ? launch_down_wide_dtype<true>(w, mid_q, mid_s, t, route_output, stream)
               : launch_down_wide_dtype<false>(w, mid_q, mid_s, t, route_output, stream);
}

}  // namespace q38m
