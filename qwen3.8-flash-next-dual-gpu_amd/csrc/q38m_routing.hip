// Routing: top-k of the router logits and the deterministic expert-major
// route plan (V1 byte layout of include/q38/cuda_moe_prefill.h:11-93).
#include "q38m_device.h"
#include "q38m_internal.h"
#include "q38m_select.h"

namespace q38m {
namespace {

// ---------------------------------------------------------------------------
// Top-k: one wave per token.  Lane l holds experts l, l+64, ...  Each of the
// top_k rounds takes every lane's best unselected (value desc, id asc) and a
// six-step butterfly to the wave winner -- the order of the reference's
// bitonic sort (q38_kernels.cu:431-458).  Numerators exp(l_r - l_0) and the
// rank-order fp32 denominator follow q38_kernels.cu:460-479.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool better(float v, int id, float ov, int oid) {
    return v > ov || (v == ov && id < oid);
}

// Router logits are fp32 (the BASELINE router output) or bf16 words (the
// reference's router writes bf16 logits, cuda_topk_router_bf16); bf16 widens
// to fp32 exactly, so both run the same fp32 selection.
__device__ __forceinline__ float logit_at(const float* row, size_t i) { return row[i]; }
__device__ __forceinline__ float logit_at(const uint16_t* row, size_t i) {
    return bf16_to_f32(row[i]);
}

// The wave's top_k by (value desc, id asc) over v[j] = logit of expert
// lane + 64j: lane r < top_k receives the rank-r value and id; every lane
// receives the rank-0 value.
template <int kPerLane>
__device__ __forceinline__ void wave_topk(const float (&v)[kPerLane], uint32_t experts,
                                          uint32_t top_k, uint32_t lane, float& mine_v,
                                          int& mine_id, float& top_v) {
    uint32_t taken = 0;
    mine_v = 0.0f;
    mine_id = 0;
    top_v = 0.0f;
    for (uint32_t rank = 0; rank < top_k; ++rank) {
        float best_v = -__builtin_huge_valf();
        int best_id = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < kPerLane; ++j) {
            const int e = static_cast<int>(lane + 64u * j);
            if (((taken >> j) & 1u) == 0u && e < static_cast<int>(experts) &&
                better(v[j], e, best_v, best_id)) {
                best_v = v[j];
                best_id = e;
            }
        }
#pragma unroll
        for (int offset = 32; offset > 0; offset >>= 1) {
            const float ov = __shfl_xor(best_v, offset, 64);
            const int oid = __shfl_xor(best_id, offset, 64);
            if (better(ov, oid, best_v, best_id)) {
                best_v = ov;
                best_id = oid;
            }
        }
        if (static_cast<uint32_t>(best_id & 63) == lane)
            taken |= 1u << (best_id >> 6);
        if (lane == rank) {
            mine_v = best_v;
            mine_id = best_id;
        }
        if (rank == 0) top_v = best_v;
    }
}

template <int kPerLane, typename Logit>
__global__ __launch_bounds__(256) void topk_kernel(
    const Logit* __restrict__ logits, uint32_t tokens, uint32_t experts,
    uint32_t top_k, int normalize, int32_t* __restrict__ ids,
    float* __restrict__ weights) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t token = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (token >= tokens) return;
    const Logit* row = logits + static_cast<size_t>(token) * experts;
    float v[kPerLane];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
        const uint32_t e = lane + 64u * j;
        v[j] = e < experts ? logit_at(row, e) : -__builtin_huge_valf();
    }
    float mine_v, top_v;
    int mine_id;
    wave_topk<kPerLane>(v, experts, top_k, lane, mine_v, mine_id, top_v);
    const float numerator = lane < top_k ? exp_q(mine_v - top_v) : 0.0f;
    float denominator = 0.0f;
    if (normalize) {
        for (uint32_t rank = 0; rank < top_k; ++rank)
            denominator += __shfl(numerator, static_cast<int>(rank), 64);
    } else {
        for (int j = 0; j < kPerLane; ++j) {
            const float ex = (lane + 64u * j) < experts ? exp_q(v[j] - top_v) : 0.0f;
            for (uint32_t src = 0; src < 64u; ++src) {
                const float term = __shfl(ex, static_cast<int>(src), 64);
                if (src + 64u * j < experts) denominator += term;
            }
        }
    }
    if (lane < top_k) {
        ids[static_cast<size_t>(token) * top_k + lane] = mine_id;
        weights[static_cast<size_t>(token) * top_k + lane] = numerator / denominator;
    }
}

// ---------------------------------------------------------------------------
// Routing + activation quantisation for chunks, one wave per token (four per
// workgroup): the top 10 of the token's 512 logits by wave_top10_of_512 (a
// ballot radix search, the order of the reference's sort,
// cuda/q38_kernels.cu:431-458), exp(l_r - l_0) summed in rank order for
// the normalisation (cuda/q38_kernels.cu:460-479); then the int8 quantisation of its 2048-wide row, lane l owning elements
// 8l + 512c .. +7 (c = 0..3).  The logit and hidden loads go out together.
// Same ids, weights and int8 rows as route_quantize_kernel (block_topk512's
// keys and order) bit for bit; at tens of thousands of tokens it keeps 32
// tokens in flight per CU where the ten-wave workgroups of
// route_quantize_kernel keep three.  (Ten rounds of a wave-wide argmax, each
// six shuffle steps through the LDS crossbar, took 88 us per 32,768-token
// layer, VALU-bound.)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void route_quantize_wave_kernel(
    const float* __restrict__ logits, const uint16_t* __restrict__ hidden, uint32_t tokens,
    int32_t* __restrict__ ids, float* __restrict__ weights, int8_t* __restrict__ xq,
    float* __restrict__ xs) {
    constexpr uint32_t kChunks = kHidden / 512u;
    constexpr uint32_t kPerLane = kExperts / 64u;
    __shared__ uint64_t top_lds[4][kTopK];
    __shared__ float num_lds[4][kTopK];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t token = blockIdx.x * 4u + wave;
    if (token >= tokens) return;
    const float* row = logits + static_cast<size_t>(token) * kExperts;
    const uint4* src = reinterpret_cast<const uint4*>(hidden + static_cast<size_t>(token) * kHidden);
    float v[kPerLane];
#pragma unroll
    for (uint32_t j = 0; j < kPerLane; ++j) v[j] = row[lane + 64u * j];
    uint4 h[kChunks];
#pragma unroll
    for (uint32_t c = 0; c < kChunks; ++c) h[c] = src[c * 64u + lane];

    int32_t my_id = 0;
    uint32_t my_rank = 0u;
    float numerator = 0.0f;
    wave_top10_of_512(v, top_lds[wave], [&](uint32_t rank, int32_t id, float num) {
        my_rank = rank;
        my_id = id;
        numerator = num;
        num_lds[wave][rank] = num;
    });
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    float denominator = 0.0f;
#pragma unroll
    for (uint32_t r = 0; r < kTopK; ++r) denominator += num_lds[wave][r];
    if (lane < kTopK) {
        ids[static_cast<size_t>(token) * kTopK + my_rank] = my_id;
        weights[static_cast<size_t>(token) * kTopK + my_rank] = numerator / denominator;
    }

    float amax = 0.0f;
#pragma unroll
    for (uint32_t c = 0; c < kChunks; ++c) {
        const uint32_t w[4] = {h[c].x, h[c].y, h[c].z, h[c].w};
        amax = fmaxf(amax, row_absmax8(w));
    }
    const QuantScale qs = quant_scale(wave_max_f32(amax));
    uint2* dst = reinterpret_cast<uint2*>(xq + static_cast<size_t>(token) * kHidden);
#pragma unroll
    for (uint32_t c = 0; c < kChunks; ++c) {
        const uint32_t w[4] = {h[c].x, h[c].y, h[c].z, h[c].w};
        dst[c * 64u + lane] = quantize8(w, qs);
    }
    if (lane == 0) xs[token] = qs.s;
}

// ---------------------------------------------------------------------------
// Routing + activation quantisation, one ten-wave workgroup per token: the
// top-k of the token's 512 logits (block_topk512) with the rank-order
// normalisation, and -- when hidden is given -- the int8 quantisation of
// the token's 2048-wide row by waves 0-3 (the same arithmetic as
// quantize_rows_kernel).  Replaces a top-k launch and a quantisation launch.
// ---------------------------------------------------------------------------
template <typename Logit>
__global__ __launch_bounds__(kSelectThreads) void route_quantize_kernel(
    const Logit* __restrict__ logits, const uint16_t* __restrict__ hidden, uint32_t top_k,
    int32_t* __restrict__ ids, float* __restrict__ weights, int8_t* __restrict__ xq,
    float* __restrict__ xs) {
    __shared__ SelectLds select_lds;
    __shared__ int32_t ids_lds[kTopK];
    __shared__ float num_lds[kTopK];
    __shared__ float amax_lds[4];
    const uint32_t token = blockIdx.x;
    const uint32_t t = threadIdx.x;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const bool quantize = hidden != nullptr;
    float logit = 0.0f;
    if (wave < 8u) logit = logit_at(logits, static_cast<size_t>(token) * kExperts + t);
    uint4 hv = make_uint4(0u, 0u, 0u, 0u);
    if (quantize && wave < 4u)
        hv = reinterpret_cast<const uint4*>(hidden + static_cast<size_t>(token) * kHidden)[t];
    const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
    if (quantize && wave < 4u) row_absmax_partial(hw, amax_lds);
    block_topk512(logit, select_lds, ids_lds, num_lds);
    if (quantize && wave < 4u) {
        const QuantScale qs = row_scale(amax_lds);
        reinterpret_cast<uint2*>(xq + static_cast<size_t>(token) * kHidden)[t] = quantize8(hw, qs);
        if (t == 0) xs[token] = qs.s;
    }
    if (wave == kTopK - 1u) {
        const uint32_t lane = t & 63u;
        float denominator = 0.0f;
        for (uint32_t r = 0; r < top_k; ++r) denominator += num_lds[r];
        if (lane < top_k) {
            ids[static_cast<size_t>(token) * top_k + lane] = ids_lds[lane];
            weights[static_cast<size_t>(token) * top_k + lane] = num_lds[lane] / denominator;
        }
    }
}

// ---------------------------------------------------------------------------
// Route plan: one workgroup of 16 waves.  The reference runs one lane per
// expert over every route (O(routes * experts) LDS compares, then a serial
// prefix on lane 0; q38_moe_prefill.cu:198-233).  Here:
//   1. each wave owns a contiguous segment of assignments and, 64 at a time,
//      finds the lanes with equal expert ids through an LDS table of lane
//      masks (each lane ORs its bit into its id's slot, reads it back and
//      clears it); the stable rank inside the segment is the popcount of
//      equal lanes below plus the wave's running per-expert count in LDS;
//   2. a per-expert exclusive scan over the 16 wave histograms gives each
//      wave's base inside its expert;
//   3. a 512-wide scan (DPP wave prefix + wave totals) gives expert and task
//      offsets;
//   4. scatter: packed = offset[e] + wave_base[w][e] + local rank.
// The result is the stable counting sort of the reference, byte for byte.
// ---------------------------------------------------------------------------
constexpr uint32_t kPlanThreads = 1024;
constexpr uint32_t kPlanWaves = kPlanThreads / 64;
constexpr uint32_t kMaxRoutes = kSlabMaxTokens * kTopK;
static_assert(kMaxRoutes / kPlanWaves <= 512u && kPlanWaves <= 128u,
              "a local rank and its wave share 16 bits");

__global__ __launch_bounds__(kPlanThreads) void build_plan_kernel(
    const int32_t* __restrict__ expert_ids, uint32_t tokens,
    q38m_route_plan_v1 plan, uint32_t max_tasks, uint32_t* __restrict__ task_flags,
    uint32_t flag_words) {
    __shared__ uint16_t key[kMaxRoutes];
    __shared__ uint16_t local_rank[kMaxRoutes];
    __shared__ uint16_t hist[kPlanWaves][kExperts];
    __shared__ unsigned long long peers[kPlanWaves][kExperts + 1u];  // slot 512: invalid ids
    __shared__ uint32_t counts[kExperts];
    __shared__ uint32_t offsets[kExperts + 1];
    __shared__ uint32_t task_offsets[kExperts + 1];
    __shared__ uint32_t wave_totals[2][8];
    __shared__ uint32_t wave_active[8];
    __shared__ uint32_t invalid;

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    const uint32_t routes = tokens * kTopK;

    // every id load is issued first (one round trip), the LDS tables are
    // cleared while they are in flight
    constexpr uint32_t kPerThread = (kMaxRoutes + kPlanThreads - 1u) / kPlanThreads;
    int32_t loaded[kPerThread];
#pragma unroll
    for (uint32_t i = 0; i < kPerThread; ++i) {
        const uint32_t a = tid + i * kPlanThreads;
        loaded[i] = a < routes ? expert_ids[a] : 0;
    }
    // the one-launch gate/up + down that follows in the step waits on these
    // (q38m_grouped.hip, gate_up_down_kernel): cleared every call
    for (uint32_t i = tid; i < flag_words; i += kPlanThreads) task_flags[i] = 0u;
    if (tid == 0) invalid = 0u;
    static_assert(kPlanWaves * kExperts * 2u == kPlanThreads * 16u, "one 16-byte clear per thread");
    reinterpret_cast<uint4*>(&hist[0][0])[tid] = make_uint4(0u, 0u, 0u, 0u);
    for (uint32_t i = tid; i < kPlanWaves * (kExperts + 1u); i += kPlanThreads)
        (&peers[0][0])[i] = 0ull;
    // LDS only: the id loads stay in flight
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (uint32_t i = 0; i < kPerThread; ++i) {
        const uint32_t a = tid + i * kPlanThreads;
        if (a < routes) {
            const int32_t id = loaded[i];
            const bool valid = id >= 0 && id < static_cast<int32_t>(kExperts);
            key[a] = valid ? static_cast<uint16_t>(id) : static_cast<uint16_t>(0xffffu);
            if (!valid) invalid = 1u;
        }
    }
    __syncthreads();

    // 1. stable local ranks per wave segment
    const uint32_t segment = ((routes + kPlanWaves * 64u - 1u) / (kPlanWaves * 64u)) * 64u;
    const uint32_t begin = wave * segment;
    const uint32_t end = min(begin + segment, routes);
    const uint64_t below_mask = (1ull << lane) - 1ull;
    // Lanes of a 64-route chunk with equal ids: each lane ORs its bit into
    // its id's slot of the wave's table, reads the slot back and clears it
    // (one wave's LDS operations execute in order).  Then the stable rank
    // inside the wave's segment is the wave's running count for the id plus
    // the equal lanes below.
    constexpr uint32_t kChunks = (kMaxRoutes + kPlanThreads - 1u) / kPlanThreads;
    unsigned long long* table = peers[wave];
#pragma unroll
    for (uint32_t i = 0; i < kChunks; ++i) {
        const uint32_t a = begin + 64u * i + lane;
        const bool in = 64u * i < segment && a < end;
        const uint32_t raw = key[a < kMaxRoutes ? a : kMaxRoutes - 1u];
        const uint32_t k = in ? raw : 0xffffu;
        const bool valid = k != 0xffffu;
        const uint32_t slot = valid ? k : kExperts;
        atomicOr(&table[slot], 1ull << lane);
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        const unsigned long long equal = table[slot];
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        table[slot] = 0ull;
        const uint32_t below = __popcll(equal & below_mask);
        const uint32_t running = valid ? hist[wave][k] : 0u;
        // the rank inside the segment (< 512) and the wave above it
        if (valid) local_rank[a] = static_cast<uint16_t>((wave << 9) | (running + below));
        if (valid && below == 0u)
            hist[wave][k] = static_cast<uint16_t>(running + __popcll(equal));
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();

    // 2. per-expert base of every wave
    if (tid < kExperts) {
        uint32_t c[kPlanWaves];
#pragma unroll
        for (uint32_t w = 0; w < kPlanWaves; ++w) c[w] = hist[w][tid];
        uint32_t running = 0;
#pragma unroll
        for (uint32_t w = 0; w < kPlanWaves; ++w) {
            hist[w][tid] = static_cast<uint16_t>(running);
            running += c[w];
        }
        counts[tid] = running;
        plan.expert_counts[tid] = static_cast<uint16_t>(running);
    }
    __syncthreads();

    // 3. expert and task offsets
    uint32_t count = 0, tasks = 0, inc_count = 0, inc_tasks = 0;
    if (tid < kExperts) {
        count = counts[tid];
        tasks = (count + kMmqM - 1u) / kMmqM;
        inc_count = wave_inclusive_sum(count);
        inc_tasks = wave_inclusive_sum(tasks);
        const uint64_t active = __ballot(count != 0u);
        if (lane == 63u) {
            wave_totals[0][wave] = inc_count;
            wave_totals[1][wave] = inc_tasks;
        }
        if (lane == 0u) wave_active[wave] = __popcll(active);
    }
    __syncthreads();
    if (tid < kExperts) {
        uint32_t prefix_count = 0, prefix_tasks = 0;
#pragma unroll
        for (uint32_t w = 0; w < 8u; ++w) {
            const uint32_t c = wave_totals[0][w], t = wave_totals[1][w];
            prefix_count += w < wave ? c : 0u;
            prefix_tasks += w < wave ? t : 0u;
        }
        offsets[tid] = prefix_count + inc_count - count;
        task_offsets[tid] = prefix_tasks + inc_tasks - tasks;
        if (tid == kExperts - 1u) {
            offsets[kExperts] = prefix_count + inc_count;
            task_offsets[kExperts] = prefix_tasks + inc_tasks;
        }
    }
    __syncthreads();

    for (uint32_t i = tid; i <= kExperts; i += kPlanThreads) {
        plan.expert_offsets[i] = offsets[i];
        plan.expert_task_offsets[i] = task_offsets[i];
    }
    const uint32_t total = offsets[kExperts];
    const uint32_t task_total = task_offsets[kExperts];
    if (tid == 0) {
        uint32_t active = 0;
        for (uint32_t w = 0; w < 8u; ++w) active += wave_active[w];
        uint32_t status = Q38M_PLAN_OK;
        if (invalid)
            status = Q38M_PLAN_INVALID_EXPERT;
        else if (total != routes || task_total > max_tasks)
            status = Q38M_PLAN_INVALID_SHAPE;
        q38m_route_plan_header_v1* h = plan.header;
        h->magic = Q38M_ROUTE_PLAN_MAGIC_V1;
        h->version = Q38M_ROUTE_PLAN_VERSION_V1;
        h->tokens = tokens;
        h->routes = routes;
        h->active_experts = active;
        h->task_count = task_total;
        h->status = status;
        h->flags = 0u;
        h->route_hash = 0u;
        h->plan_hash = 0u;
        h->reserved0 = 0u;
        h->reserved1 = 0u;
    }

    // 4. scatter; identity for invalid assignments and unfilled positions
#pragma unroll
    for (uint32_t i = 0; i < kPerThread; ++i) {
        const uint32_t a = tid + i * kPlanThreads;
        if (a >= routes) continue;
        const uint32_t k = key[a];
        if (k == 0xffffu) {
            plan.assignment_to_packed[a] = a;
            continue;
        }
        const uint32_t lr = local_rank[a];
        const uint32_t position = offsets[k] + hist[lr >> 9][k] + (lr & 511u);
        plan.packed_assignment[position] = a;
        plan.assignment_to_packed[a] = position;
    }
    for (uint32_t p = total + tid; p < routes; p += kPlanThreads)
        plan.packed_assignment[p] = p;

    uint2* task_words = reinterpret_cast<uint2*>(plan.tasks);
    if (tid < kExperts) {
        const uint32_t c = counts[tid];
        const uint32_t first = task_offsets[tid];
        const uint32_t n = (c + kMmqM - 1u) / kMmqM;
        for (uint32_t tile = 0; tile < n; ++tile) {
            const uint32_t remaining = c - tile * kMmqM;
            const uint32_t rows = remaining < kMmqM ? remaining : kMmqM;
            task_words[first + tile] = make_uint2(offsets[tid] + tile * kMmqM,
                                                  tid | (rows << 16));
        }
    }
    for (uint32_t t = task_total + tid; t < max_tasks; t += kPlanThreads)
        task_words[t] = make_uint2(0u, 0u);
}

// FNV-1a over 64-bit words, the serial hash pass of
// cuda/q38_moe_prefill.cu:262-289.  Requested explicitly: it is a single
// dependent chain of ~2*routes+1026 multiplies and would dominate the step.
__global__ void plan_hash_kernel(const int32_t* __restrict__ expert_ids,
                                 q38m_route_plan_v1 plan) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    constexpr uint64_t kOffset = 1469598103934665603ull;
    constexpr uint64_t kPrime = 1099511628211ull;
    const uint32_t routes = plan.header->routes;
    uint64_t route_hash = kOffset;
    for (uint32_t a = 0; a < routes; ++a) {
        const int32_t id = expert_ids[a];
        const uint64_t k = (id >= 0 && id < static_cast<int32_t>(kExperts))
                               ? static_cast<uint64_t>(id)
                               : 0xffffull;
        route_hash = (route_hash ^ k) * kPrime;
    }
    uint64_t plan_hash = kOffset;
    for (uint32_t e = 0; e <= kExperts; ++e) {
        plan_hash = (plan_hash ^ plan.expert_offsets[e]) * kPrime;
        plan_hash = (plan_hash ^ plan.expert_task_offsets[e]) * kPrime;
    }
    for (uint32_t p = 0; p < routes; ++p)
        plan_hash = (plan_hash ^ plan.packed_assignment[p]) * kPrime;
    const uint32_t task_count = plan.header->task_count;
    for (uint32_t t = 0; t < task_count; ++t) {
        const q38m_task_v1 task = plan.tasks[t];
        const uint64_t low = static_cast<uint64_t>(task.packed_begin) |
                             (static_cast<uint64_t>(task.expert) << 32);
        const uint64_t high = static_cast<uint64_t>(task.valid_rows) |
                              (static_cast<uint64_t>(task.flags) << 8);
        plan_hash = (plan_hash ^ low) * kPrime;
        plan_hash = (plan_hash ^ high) * kPrime;
    }
    plan.header->route_hash = route_hash;
    plan.header->plan_hash = plan_hash;
}

}  // namespace

namespace {

template <typename Logit>
hipError_t launch_topk_any(const Logit* logits, int32_t* ids, float* weights, uint32_t tokens,
                           uint32_t experts, uint32_t top_k, int normalize,
                           hipStream_t stream) {
    const dim3 grid((tokens + 3u) / 4u);
    const uint32_t per_lane = (experts + 63u) / 64u;
    if (per_lane <= 8u)
        topk_kernel<8><<<grid, 256, 0, stream>>>(logits, tokens, experts, top_k,
                                                 normalize, ids, weights);
    else
        topk_kernel<16><<<grid, 256, 0, stream>>>(logits, tokens, experts, top_k,
                                                  normalize, ids, weights);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_topk(const float* logits, int32_t* ids, float* weights,
                       uint32_t tokens, uint32_t experts, uint32_t top_k,
                       int normalize, hipStream_t stream) {
    return launch_topk_any(logits, ids, weights, tokens, experts, top_k, normalize, stream);
}

hipError_t launch_topk(const uint16_t* logits, int32_t* ids, float* weights,
                       uint32_t tokens, uint32_t experts, uint32_t top_k,
                       int normalize, hipStream_t stream) {
    return launch_topk_any(logits, ids, weights, tokens, experts, top_k, normalize, stream);
}

hipError_t launch_route_quantize(const float* logits, const uint16_t* hidden, uint32_t tokens,
                                uint32_t top_k, int32_t* ids, float* weights, int8_t* xq,
                                float* xs, hipStream_t stream) {
    route_quantize_kernel<<<tokens, kSelectThreads, 0, stream>>>(logits, hidden, top_k, ids,
                                                                 weights, xq, xs);
    return hipGetLastError();
}

hipError_t launch_route_quantize_wave(const float* logits, const uint16_t* hidden,
                                     uint32_t tokens, int32_t* ids, float* weights, int8_t* xq,
                                     float* xs, hipStream_t stream) {
    route_quantize_wave_kernel<<<(tokens + 3u) / 4u, 256, 0, stream>>>(logits, hidden, tokens,
                                                                      ids, weights, xq, xs);
    return hipGetLastError();
}

hipError_t launch_route_bf16(const uint16_t* logits, uint32_t tokens, uint32_t top_k,
                             int32_t* ids, float* weights, hipStream_t stream) {
    route_quantize_kernel<<<tokens, kSelectThreads, 0, stream>>>(
        logits, static_cast<const uint16_t*>(nullptr), top_k, ids, weights,
        static_cast<int8_t*>(nullptr), static_cast<float*>(nullptr));
    return hipGetLastError();
}

hipError_t launch_build_plan(const int32_t* ids, uint32_t tokens,
                             const q38m_route_plan_v1& plan, bool hashes,
                             hipStream_t stream, uint32_t* task_flags, uint32_t flag_words) {
    build_plan_kernel<<<1, kPlanThreads, 0, stream>>>(ids, tokens, plan, max_tasks_v1(tokens),
                                                      task_flags, flag_words);
    if (hashes) plan_hash_kernel<<<1, 64, 0, stream>>>(ids, plan);
    return hipGetLastError();
}

}  // namespace q38m
