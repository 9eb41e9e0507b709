// Batch-1 decode: streams only the top_k selected experts (the tokens == 1
// branch of run_moe, cuda/cuda_backend.cu:1516-1605: cuda_topk_router_bf16,
// cuda_moe_routed_bf16 (cuda/q38_moe.cu:388-458), cuda_moe_combine_shared_bf16).
// The arithmetic is the prefill contract evaluated for one token -- int8
// token quantisation, per-group int32 accumulators, the fp32 group chain in
// group order, the SwiGLU fold, per-route mid quantisation, down, and the
// rank-order sum -- so decode equals the grouped prefill with tokens == 1
// bit for bit.  (The reference's decode applies the router weight after
// down and differs from its prefill by up to 0.075, cuda_kernel_tests.cu:370.)
//
// At one token the layer is a latency chain: on MI355X a dependent kernel
// boundary costs ~1.7 us in a graph and a device-scope grid barrier ~5 us,
// so the layer is two launches and every byte of each launch is requested
// as early as its address is known.
//
//   gate/up  256 workgroups x 12 waves (three route slots x four quarters
//            of K).  Waves 0-7 rank the 512 router logits (or wave 9 reads
//            the given ids) while waves 0-3 also load the token; then every
//            lane issues its weight loads at once (46 KB per workgroup, the
//            layer's 11.8 MB in flight together).  Workgroup b owns eight
//            channels (gate and up rows) of one pair tile for a group of 2-3
//            routes; the two halves of a pair tile's group sit on one XCD
//            (b % 8), so each scale line crosses HBM once.
//            Once its weights are in, each wave requests the lines the
//            down launch's workgroup b will read, so they are cached.
//   down     256 workgroups x 10 waves.  Each wave loads the ids and its
//            route's mid row together, quantises the row in registers, and
//            streams 8 output channels x 512 columns; int32 partials meet by
//            shuffles, routes are summed in rank order, then the optional
//            gated shared term and residual are applied.
#include "q38m_device.h"
#include "q38m_internal.h"
#include "q38m_select.h"

#ifdef Q38M_PHASE_TIMESTAMPS
#include <atomic>

#include "q38m_phase.h"
#endif

namespace q38m {
namespace {

// ---- phase timestamps (include/q38m_phase.h) ------------------------------
// PhaseStamps reads the constant 100 MHz clock at a kernel's phase
// boundaries in the timing build (-DQ38M_PHASE_TIMESTAMPS) and is empty in
// the product build, where every call on it compiles to nothing.  PhaseCall
// carries the host's call counter (always 0 in the product build).
struct PhaseCall {
    uint32_t index;
};

#ifdef Q38M_PHASE_TIMESTAMPS
__device__ q38m_phase_record_v1* g_phase_records;
__device__ uint32_t g_phase_calls_held;  // log capacity / 512
std::atomic<uint32_t> g_phase_calls{0};

struct PhaseStamps {
    static constexpr uint32_t kStamps = 16u;  // the first wave's phases
    static constexpr uint32_t kWaveStamps = 16u;  // one per wave: its weights arrived
    uint64_t t[kStamps];
    __device__ PhaseStamps() {
#pragma unroll
        for (uint32_t i = 1; i < kStamps; ++i) t[i] = 0u;
        t[0] = __builtin_amdgcn_s_memrealtime();
        // the start stays ahead of the kernel-argument loads and their wait
        __builtin_amdgcn_sched_barrier(0);
    }
    __device__ void mark(uint32_t i) { t[i] = __builtin_amdgcn_s_memrealtime(); }
    // after this wave's outstanding vector loads have arrived
    __device__ void mark_loaded(uint32_t i) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        mark(i);
    }
    // every wave: the time its own loads have all arrived, into wave_lds
    __device__ void mark_wave_loaded(uint64_t* wave_lds) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const uint64_t now = __builtin_amdgcn_s_memrealtime();
        if ((threadIdx.x & 63u) == 0u) wave_lds[threadIdx.x >> 6] = now;
    }
    // thread 0 writes the record (a vector store under a lane branch);
    // wave_lds (the per-wave stamps, visible after a barrier) may be null
    __device__ void finish(uint32_t kernel, PhaseCall call, const uint64_t* wave_lds = nullptr) {
        q38m_phase_record_v1* log = g_phase_records;
        const uint32_t held = g_phase_calls_held;
        if (threadIdx.x != 0u || log == nullptr || held == 0u) return;
        q38m_phase_record_v1& r = log[(call.index % held) * 512u + 256u * kernel + blockIdx.x];
#pragma unroll
        for (uint32_t i = 0; i < kStamps; ++i) r.stamp[i] = t[i];
        const uint32_t waves = blockDim.x / 64u;
        for (uint32_t i = 0; i < kWaveStamps; ++i)
            r.wave_stamp[i] = wave_lds != nullptr && i < waves ? wave_lds[i] : 0u;
        r.kernel = kernel;
        r.block = blockIdx.x;
        r.call = call.index;
        r.valid = 1u;
    }
};

PhaseCall next_phase_call() { return PhaseCall{g_phase_calls.fetch_add(1u)}; }
#else
struct PhaseStamps {
    __device__ void mark(uint32_t) {}
    __device__ void mark_loaded(uint32_t) {}
    __device__ void mark_wave_loaded(uint64_t*) {}
    __device__ void finish(uint32_t, PhaseCall, const uint64_t* = nullptr) {}
};

PhaseCall next_phase_call() { return PhaseCall{0u}; }
#endif

constexpr uint32_t kDecodeBlocks = 256;
constexpr uint32_t kDecodeThreads = kSelectThreads;

// The whole MoE block of a decode step (q38m_moe_decode_block_v1) adds the
// bf16 shared expert to the two routed launches: gate/up workgroup b also
// computes channels 2b and 2b + 1 of g = bf16(x Wg^T), u = bf16(x Wu^T)
// and h = silu_multiply(g, u) (workgroup 0 also the output gate
// bf16(x wo)), and down workgroup b computes its eight channels of
// bf16(h Wd^T) before the gated combine.  Every dot product is
// wave_dot_bf16's (one wave per row, the same summation order as the GEMV
// entry points), so the block equals q38m_moe_router_v1 +
// q38m_moe_shared_expert_v1 + q38m_moe_decode_v1 bit for bit.
struct SharedGateUp {
    const uint16_t* w_gate;
    const uint16_t* w_up;
    const uint16_t* w_out_gate;
    uint16_t* h;     // [I] bf16
    uint16_t* gate;  // the output gate word
};
struct SharedDown {
    const uint16_t* w_down;  // [H][I] bf16
    const uint16_t* h;       // [I] bf16, from the gate/up launch
    const uint16_t* gate;    // the output gate word
};

// The down launch's weight and scale lines, requested by the gate/up launch
// once its own weights have arrived: gate/up workgroup b touches every
// 64-byte piece that down workgroup b will read (both grids have 256
// workgroups, and workgroup b runs on XCD b % 8 in both), so the down
// launch finds its weights in a cache (that XCD's L2 or the memory-side
// Infinity Cache) instead of streaming them from HBM after its ids arrive.  The loaded words are only folded into a
// value the wave keeps live to its end; nothing is computed from them.
struct DownPrefetch {
    const uint8_t* w;       // the down weights
    const uint16_t* s;      // their scale words
    uint32_t w4;            // 1: W4 (MFMA16 quad-major), 0: W8 (K-block-major)
    uint32_t scale_words;   // W8: scale words per channel; W4: per row and quad
};

// wave `route` of gate/up workgroup b: the route's pieces of down workgroup
// b (decode_down_kernel's load addresses), one 4-byte load per 64 bytes
__device__ __forceinline__ uint32_t prefetch_down(const DownPrefetch& pf, uint32_t e,
                                                  uint32_t lane) {
    constexpr uint32_t kTiles = kHidden / 16u;
    const uint32_t slot8 = blockIdx.x >> 3;
    const uint32_t tile = 16u * (blockIdx.x & 7u) + (slot8 >> 1);
    const uint32_t n0 = 8u * (slot8 & 1u);
    size_t piece;  // 16-byte index into the weights
    size_t scale;  // scale word index
    if (pf.w4) {
        // lanes 0-31: (quad kq, half qh, chunk x, 64-byte half hs) of the
        // route's 16 lines; lanes 32-63: the scale words of (kq, channel)
        constexpr uint32_t kQuads = kInter / 128u;
        const uint32_t kq = (lane >> 3) & 3u;
        const size_t t = (static_cast<size_t>(e) * kQuads + kq) * kTiles + tile;
        piece = t * 64u + 32u * ((lane >> 2) & 1u) + 16u * ((lane >> 1) & 1u) + n0 +
                4u * (lane & 1u);
        scale = (t * 16u + n0 + (lane & 7u)) * pf.scale_words;
    } else {
        // (K block kb, chunk q, 64-byte half hs) of the route's 32 lines;
        // the channel's scale words
        constexpr uint32_t kBlocks = kInter / 64u;
        piece = ((static_cast<size_t>(e) * kTiles + tile) * kBlocks + (lane >> 3)) * 64u + n0 +
                16u * ((lane >> 1) & 3u) + 4u * (lane & 1u);
        scale = (static_cast<size_t>(e) * kHidden + 16u * tile + n0 + (lane & 7u)) *
                pf.scale_words;
    }
    const uint32_t word = *reinterpret_cast<const uint32_t*>(pf.w + 16u * piece);
    return word ^ static_cast<uint32_t>(pf.s[scale]);
}

// gate/up: 12 waves, three route slots x four quarters of K.
constexpr uint32_t kGateUpThreads = 768u;
constexpr uint32_t kRouteSlots = 3u;
static_assert(kGateUpThreads >= kSelectThreads, "the block top-k needs ten waves");
static_assert(kRouteSlots * 64u * 4u == kGateUpThreads, "wave = route slot x K quarter");

// Routes of workgroup group g (0..3): {0,1,2}, {3,4,5}, {6,7}, {8,9}.
__device__ __forceinline__ uint32_t route_group_first(uint32_t g) {
    return g < 2u ? 3u * g : 2u * g + 2u;
}
__device__ __forceinline__ uint32_t route_group_count(uint32_t g) { return g < 2u ? 3u : 2u; }

// W4 (kW8 false): kPer = 32-column sub-blocks per group (1, 2 or 4: groups
// of 32, 64, 128), the MFMA16 quad-major layout.  W8: kPer = 64-column K
// blocks per group (1, 2, or H/64 = per output channel), the paired
// K-block-major layout, scales in the artifact order.  A group's partial
// accumulators add exactly in int32 before the fp32 chain; bf16: scale
// words are bf16 (else fp16).
//
// Workgroup b owns channels 16p + 8h .. +7 (gate and up rows) of pair tile
// p for one group of routes; the two halves h of a (p, group) sit on one XCD
// (b % 8), so each 128-byte line of scale words crosses HBM once.  Load
// layout: wave = (route slot rs, K quarter), lane = n + 8u + 16kq' (row
// 8h + n of the tile's gate (u = 0) or up (u = 1) slot, quad 4 quarter +
// kq'): every load instruction reads 8 whole 128-byte lines, 8 consecutive
// lanes per line.  The int32 group sums and their scales then move through
// LDS into the chain layout: wave = route slot x two channels, lane =
// quad + 16 (2 n' + u), where the fp32 chain runs along each 16-lane row.
//
// kShared (the decode block): waves 8-11, which hold no logits, issue their
// shared-expert row (gate and up rows of channels 2b, 2b + 1) before the
// selection and finish the dot products while the routed weights stream.
template <uint32_t H, uint32_t I, bool kW8, uint32_t kPer, bool kShared = false>
__global__ __launch_bounds__(kGateUpThreads) void decode_gate_up_kernel(
    const uint4* __restrict__ w, const uint16_t* __restrict__ s, bool bf16,
    const uint16_t* __restrict__ hidden, const float* __restrict__ logits,
    const int32_t* __restrict__ ids_in, const float* __restrict__ weights_in, uint32_t top_k,
    int32_t* __restrict__ ids_out, uint16_t* __restrict__ mid, PhaseCall call,
    SharedGateUp shared, DownPrefetch prefetch) {
    PhaseStamps stamps;
    constexpr uint32_t kQuads = H / 128u;
    constexpr uint32_t kSlots = 2u * I / 16u;
    constexpr uint32_t kPairs = I / 16u;
    constexpr uint32_t kQuadPad = 9u;  // 144-byte rows: the 16 quads hit disjoint banks
    constexpr uint32_t kChains = kRouteSlots * 16u;  // (route slot, channel, gate/up)
    static_assert(H == 256u * 8u && kQuads == 16u, "16 quads, one 8-element token chunk per thread");
    static_assert(kPairs * 2u * 4u == kDecodeBlocks, "pair tile x half x route group");
    __shared__ int32_t ids_lds[kTopK];
    __shared__ float num_lds[kTopK];
    __shared__ float amax_lds[4];
    __shared__ uint4 x_lds[kQuads * kQuadPad];
    __shared__ SelectLds select_lds;
    // [chain][quad]: int32 group sums, then their fp32 scales
    __shared__ uint4 xch[kChains * kQuads][2];
    __shared__ float shared_dot[4];  // kShared: g, u of channel 2b; g, u of 2b + 1
#ifdef Q38M_PHASE_TIMESTAMPS
    __shared__ uint64_t wave_stamp_lds[kGateUpThreads / 64u];
#else
    uint64_t* const wave_stamp_lds = nullptr;
#endif

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t xcd = blockIdx.x & 7u, within = blockIdx.x >> 3;
    const uint32_t pg = 16u * xcd + (within >> 1);
    const uint32_t pair = pg % kPairs, group = pg / kPairs, half = within & 1u;
    const bool fused = logits != nullptr;

    uint4 hv = make_uint4(0u, 0u, 0u, 0u);
    if (wave < 4u) hv = reinterpret_cast<const uint4*>(hidden)[threadIdx.x];
    float logit = 0.0f;
    if (fused && wave < 8u) logit = logits[threadIdx.x];
    if (!fused && wave == kTopK - 1u && lane < top_k) {
        ids_lds[lane] = ids_in[lane];
        num_lds[lane] = weights_in[lane];
    }
    const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
    Bf16RowPass shared_row, gate_row;
    if constexpr (kShared) {
        if (wave >= 8u) {
            const uint32_t c = 2u * blockIdx.x + ((wave - 8u) >> 1);
            const uint16_t* rowp = ((wave & 1u) ? shared.w_up : shared.w_gate) +
                                   static_cast<size_t>(c) * H;
            shared_row = bf16_row_load(hidden, rowp, H / 8u, 0u, lane);
            if (blockIdx.x == 0u && wave == 8u)
                gate_row = bf16_row_load(hidden, shared.w_out_gate, H / 8u, 0u, lane);
        }
    }
    stamps.mark_loaded(1);
    // the selection first: the token row's absmax waits for its load, the
    // selection only for the logits
    if (fused) {
        block_topk512(logit, select_lds, ids_lds, num_lds,
                      [&](uint32_t level) { stamps.mark(10u + level); });
        if (blockIdx.x == 0 && threadIdx.x < top_k) ids_out[threadIdx.x] = ids_lds[threadIdx.x];
    } else {
        __syncthreads();
    }
    stamps.mark(2);

    // this wave's route (the same in the load and the chain layout)
    const uint32_t slot_rs = wave >> 2;
    const uint32_t route = route_group_first(group) + slot_rs;
    const bool active = slot_rs < route_group_count(group) && route < top_k;
    const int32_t id = active ? ids_lds[route] : -1;
    const bool valid = id >= 0 && id < static_cast<int32_t>(kExperts);
    const uint32_t e = valid ? static_cast<uint32_t>(id) : 0u;

    // load layout
    const uint32_t n = lane & 7u, u = (lane >> 3) & 1u;
    const uint32_t kq = 4u * (wave & 3u) + (lane >> 4);
    const uint32_t row = 8u * half + n;
    const uint32_t slot = 2u * pair + u;
    // W4: quad kq of the slot's tile, 16 bytes per row per 32-column group.
    // W8: blocks 2kq and 2kq+1 (the same 128 columns), 16 bytes per row and
    // lane group q: bq[4*block + q].  A wave without a route reads one
    // common kilobyte instead (an L2 hit), so every load stays unconditional.
    uint4 bq[kW8 ? 8 : 4];
    uint2 sc = make_uint2(0u, 0u);
    uint32_t sw = 0;
    if constexpr (!kW8) {
        const size_t tile = (static_cast<size_t>(e) * kQuads + kq) * kSlots + slot;
        const uint4* wp = active ? w + tile * 64u + row : w + lane;
        bq[0] = wp[0];
        bq[1] = wp[16];
        bq[2] = wp[32];
        bq[3] = wp[48];
        sc = load_quad_scales<kPer, false>(s + (active ? (tile * 16u + row) * (4u / kPer) : 0u));
    } else {
        constexpr uint32_t kBlocks = H / 64u;
#pragma unroll
        for (uint32_t b = 0; b < 2u; ++b) {
            const uint4* wp =
                active ? w + ((static_cast<size_t>(e) * kBlocks + 2u * kq + b) * kSlots + slot) *
                                 64u + row
                       : w + lane;
#pragma unroll
            for (uint32_t q = 0; q < 4u; ++q) bq[4u * b + q] = wp[16u * q];
        }
        const size_t srow = active ? static_cast<size_t>(e) * 2u * I + (u ? I : 0u) +
                                         16u * pair + row
                                   : 0u;
        if constexpr (kPer == kBlocks)
            sw = s[srow];
        else if constexpr (kPer == 1u)
            sw = *reinterpret_cast<const uint32_t*>(s + srow * kBlocks + 2u * kq);
        else
            sw = s[srow * (kBlocks / 2u) + kq];
    }

    stamps.mark(3);

    if constexpr (kShared) {
        // the shared rows' products, while the routed weights stream
        if (wave >= 8u) {
            const float dot = wave_sum_f32(bf16_row_accumulate(shared_row, 0.0f));
            if (lane == 0u) shared_dot[wave - 8u] = dot;
        }
        if (blockIdx.x == 0u && wave == 8u) {
            const float gate = wave_sum_f32(bf16_row_accumulate(gate_row, 0.0f));
            if (lane == 0u) shared.gate[0] = static_cast<uint16_t>(f32_to_bf16(gate));
        }
    }

    // the route's weight, while the weights stream: given, or
    // exp(l_r - l_0) over the rank-order sum (q38_kernels.cu:460-479)
    float wr = 0.0f;
    if (active) {
        wr = num_lds[route];
        if (fused) {
            float denominator = 0.0f;
            for (uint32_t r = 0; r < top_k; ++r) denominator += num_lds[r];
            wr = wr / denominator;
        }
    }

    // int8 token (same arithmetic as the row quantiser); the barrier waits
    // for LDS only, so the weight loads above stay in flight
    if (wave < 4u) row_absmax_partial(hw, amax_lds);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const QuantScale row_q = row_scale(amax_lds);
    const float xs = row_q.s;
    if (wave < 4u) {
        const uint32_t k = 8u * threadIdx.x;
        reinterpret_cast<uint2*>(x_lds)[(k >> 7) * (2u * kQuadPad) + ((k & 127u) >> 3)] =
            quantize8(hw, row_q);
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    stamps.mark(4);
    stamps.mark_loaded(5);
    stamps.mark_wave_loaded(wave_stamp_lds);


    // this lane's group sums (int32) and their scales (fp32 words)
    uint4 xa = make_uint4(0u, 0u, 0u, 0u), xf = make_uint4(0u, 0u, 0u, 0u);
    if constexpr (!kW8) {
        // group j of quad kq, chunk q: k = 32(4kq+j) + 8q + {0..3} (low
        // nibbles) and + {4..7} (high nibbles); nibbles sit in the high half
        // of each byte (16*w), so acc is 16x the group accumulator.
        uint32_t xw[32];
#pragma unroll
        for (uint32_t i = 0; i < 8u; ++i) {
            const uint4 xv = x_lds[kq * kQuadPad + i];
            xw[4 * i] = xv.x; xw[4 * i + 1] = xv.y; xw[4 * i + 2] = xv.z; xw[4 * i + 3] = xv.w;
        }
        int acc[4] = {0, 0, 0, 0};
#pragma unroll
        for (uint32_t q = 0; q < 4u; ++q) {
            const uint32_t wq[4] = {bq[q].x, bq[q].y, bq[q].z, bq[q].w};
#pragma unroll
            for (uint32_t j = 0; j < 4u; ++j) {
                const uint32_t lo = (wq[j] << 4) & 0xf0f0f0f0u;
                const uint32_t hi = wq[j] & 0xf0f0f0f0u;
                acc[j] = __builtin_amdgcn_sdot4(static_cast<int>(lo), static_cast<int>(xw[8u * j + 2u * q]), acc[j], false);
                acc[j] = __builtin_amdgcn_sdot4(static_cast<int>(hi), static_cast<int>(xw[8u * j + 2u * q + 1u]), acc[j], false);
            }
        }
        uint32_t ga[4] = {0u, 0u, 0u, 0u}, gf[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (uint32_t gi = 0; gi < 4u / kPer; ++gi) {
            gf[gi] = __float_as_uint(scale_to_f32(quad_scale_word(sc, gi), bf16) * 0.0625f);
            int sum = acc[gi * kPer];
#pragma unroll
            for (uint32_t j = 1; j < kPer; ++j) sum += acc[gi * kPer + j];
            ga[gi] = static_cast<uint32_t>(sum);
        }
        xa = make_uint4(ga[0], ga[1], ga[2], ga[3]);
        xf = make_uint4(gf[0], gf[1], gf[2], gf[3]);
    } else {
        // block b (= 2kq + b), lane group q: columns 64(2kq+b) + 16q .. +15
        int acc[2] = {0, 0};
#pragma unroll
        for (uint32_t b = 0; b < 2u; ++b)
#pragma unroll
            for (uint32_t q = 0; q < 4u; ++q) {
                const uint4 xv = x_lds[kq * kQuadPad + 4u * b + q];
                const uint4 wv = bq[4u * b + q];
                acc[b] = __builtin_amdgcn_sdot4(static_cast<int>(wv.x), static_cast<int>(xv.x), acc[b], false);
                acc[b] = __builtin_amdgcn_sdot4(static_cast<int>(wv.y), static_cast<int>(xv.y), acc[b], false);
                acc[b] = __builtin_amdgcn_sdot4(static_cast<int>(wv.z), static_cast<int>(xv.z), acc[b], false);
                acc[b] = __builtin_amdgcn_sdot4(static_cast<int>(wv.w), static_cast<int>(xv.w), acc[b], false);
            }
        if constexpr (kPer == 1u) {
            xa = make_uint4(static_cast<uint32_t>(acc[0]), static_cast<uint32_t>(acc[1]), 0u, 0u);
            xf = make_uint4(__float_as_uint(scale_to_f32(sw & 0xffffu, bf16)),
                            __float_as_uint(scale_to_f32(sw >> 16, bf16)), 0u, 0u);
        } else {
            // per channel: this lane's 128-column part of the row's one
            // int32; groups of 128: the group's sum
            xa.x = static_cast<uint32_t>(acc[0] + acc[1]);
            xf.x = __float_as_uint(scale_to_f32(sw, bf16));
        }
    }
    // This wave's weights and scales are consumed: now the down launch's
    // pieces of route `wave` (waves 10 and 11 repeat expert 0's), issued
    // while the waves wait for each other at the exchange.  Issued right
    // behind this launch's own weight requests they share HBM with the other
    // workgroups' gate/up weights and delay them more than they save; issued
    // before the group sums they hold those up.  Every barrier after this
    // point waits for LDS only, so the prefetch stays in flight until the
    // kernel's end.
    __builtin_amdgcn_sched_barrier(0);
    uint32_t prefetched;
    {
        const int32_t pid = wave < top_k ? ids_lds[wave] : -1;
        const uint32_t pe =
            pid >= 0 && pid < static_cast<int32_t>(kExperts) ? static_cast<uint32_t>(pid) : 0u;
        prefetched = prefetch_down(prefetch, pe, lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    stamps.mark(6);
    {
        const uint32_t chain = 16u * slot_rs + 2u * n + u;
        xch[chain * kQuads + kq][0] = xa;
        xch[chain * kQuads + kq][1] = xf;
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    stamps.mark(7);
    if constexpr (kShared) {
        // the exchange barrier made shared_dot visible
        if (threadIdx.x < 2u) {
            const uint32_t g_bits = f32_to_bf16(shared_dot[2u * threadIdx.x]);
            const uint32_t u_bits = f32_to_bf16(shared_dot[2u * threadIdx.x + 1u]);
            shared.h[2u * blockIdx.x + threadIdx.x] =
                static_cast<uint16_t>(silu_multiply(g_bits, u_bits));
        }
    }

    // chain layout: lane = quad + 16 c, chain 4 wave + c = (route slot,
    // channel 2 (wave % 4) + c / 2, gate/up c % 2)
    const uint32_t cq = lane & 15u;
    const uint4 ca = xch[(4u * wave + (lane >> 4)) * kQuads + cq][0];
    const uint4 cf = xch[(4u * wave + (lane >> 4)) * kQuads + cq][1];
    const int ga[4] = {static_cast<int>(ca.x), static_cast<int>(ca.y), static_cast<int>(ca.z),
                       static_cast<int>(ca.w)};
    const float gs[4] = {__uint_as_float(cf.x), __uint_as_float(cf.y), __uint_as_float(cf.z),
                         __uint_as_float(cf.w)};
    constexpr uint32_t kChainTerms = kW8 ? (kPer == 1u ? 2u : 1u) : 4u / kPer;
    float y = 0.0f;
    if constexpr (kW8 && kPer == H / 64u) {
        // per channel: one int32 over the row (16 lanes) by DPP rotations
        // (row_ror 8, 4, 2, 1), y = (float)acc * s
        int sum = ga[0];
        sum += __builtin_amdgcn_update_dpp(0, sum, 0x128, 0xf, 0xf, false);
        sum += __builtin_amdgcn_update_dpp(0, sum, 0x124, 0xf, 0xf, false);
        sum += __builtin_amdgcn_update_dpp(0, sum, 0x122, 0xf, 0xf, false);
        sum += __builtin_amdgcn_update_dpp(0, sum, 0x121, 0xf, 0xf, false);
        y = static_cast<float>(sum) * gs[0];
    } else {
        // fp32 chain in group order: lane cq continues lane cq-1's value
        // (row_shr:1 inside each 16-lane row); after 16 steps lane 15 of
        // the row holds the channel's y.
#pragma unroll
        for (uint32_t step = 0; step < kQuads; ++step) {
            float t = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(y), 0x111, 0xf, 0xf, true));
#pragma unroll
            for (uint32_t gi = 0; gi < kChainTerms; ++gi)
                t = __builtin_fmaf(static_cast<float>(ga[gi]), gs[gi], t);
            y = t;
        }
    }
    const float g0 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(y), 15));
    const float u0 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(y), 31));
    const float g1 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(y), 47));
    const float u1 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(y), 63));
    stamps.mark(8);
    // lane c computes channel 2 (wave % 4) + c (c = 0, 1)
    if (lane < 2u && active) {
        const float g = lane == 0u ? g0 : g1;
        const float up = lane == 0u ? u0 : u1;
        const uint32_t m = valid ? swiglu_fold(g * xs, up * xs, wr) : 0u;
        mid[static_cast<size_t>(route) * I + 16u * pair + 8u * half + 2u * (wave & 3u) + lane] =
            static_cast<uint16_t>(m);
    }
    stamps.mark(9);
    stamps.finish(0u, call, wave_stamp_lds);
    // the prefetch's words are consumed here, after everything else
    asm volatile("" ::"v"(prefetched));
}

// kPerGroup: W4, 32-column sub-blocks per group (1, 2, 4); W8, 64-column
// K blocks per group (1, 2; I/64 = per output channel).
// kShared (the decode block): two more waves compute the workgroup's
// eight channels of the shared down projection bf16(h Wd^T) and meet the
// route waves at their two barriers; the finisher takes those words and the
// output gate from the gate/up launch.
template <uint32_t H, uint32_t I, bool kW4, uint32_t kPerGroup, bool kShared = false>
__global__ __launch_bounds__(kShared ? kDecodeThreads + 128u : kDecodeThreads)
void decode_down_kernel(
    const uint4* __restrict__ w, const uint16_t* __restrict__ s, bool bf16,
    const uint16_t* __restrict__ mid,
    const int32_t* __restrict__ ids, uint32_t top_k, const uint16_t* __restrict__ shared_output,
    const uint16_t* __restrict__ shared_gate, const uint16_t* __restrict__ residual,
    uint16_t* __restrict__ out, PhaseCall call, SharedDown shared) {
    PhaseStamps stamps;
    constexpr uint32_t kTiles = H / 16u;
    static_assert(I == 64u * 8u, "one 8-element chunk of the mid row per lane");
    static_assert(kTiles * 2u == kDecodeBlocks, "eight output channels per workgroup");
    __shared__ uint4 mq_lds[kTopK][I / 16u];
    // route partials per output channel, ten routes padded to 12 floats
    __shared__ float4 o_lds[8][3];
    __shared__ uint32_t shared_lds[8];  // kShared: the eight shared-down words
#ifdef Q38M_PHASE_TIMESTAMPS
    __shared__ uint64_t wave_stamp_lds[kDecodeThreads / 64u + 2u];
#else
    uint64_t* const wave_stamp_lds = nullptr;
#endif

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t route = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t slot8 = blockIdx.x >> 3;
    const uint32_t tile = 16u * (blockIdx.x & 7u) + (slot8 >> 1);
    const uint32_t n0 = 8u * (slot8 & 1u);
    const bool active = route < top_k;

    if constexpr (kShared) {
        if (route >= kTopK) {
            // wave 10: channels n0 + 0..3 of the tile, wave 11: n0 + 4..7
            const uint32_t c0 = 4u * (route - kTopK);
            Bf16RowPass rows[4];
#pragma unroll
            for (uint32_t j = 0; j < 4u; ++j)
                rows[j] = bf16_row_load(shared.h,
                                        shared.w_down + static_cast<size_t>(16u * tile + n0 + c0 + j) * I,
                                        I / 8u, 0u, lane);
            stamps.mark_wave_loaded(wave_stamp_lds);
#pragma unroll
            for (uint32_t j = 0; j < 4u; ++j) {
                const float dot = wave_sum_f32(bf16_row_accumulate(rows[j], 0.0f));
                if (lane == 0u) shared_lds[c0 + j] = f32_to_bf16(dot);
            }
            __syncthreads();  // the route waves' mid-row barrier
            __syncthreads();  // their partials barrier (the finisher reads shared_lds after it)
            return;
        }
    }

    // the epilogue's operands, requested first: they depend on nothing.
    // Every thread loads them in straight-line code (an absent operand reads
    // the mid row's first word instead and is never used), so no branch
    // holds a wait for them ahead of the weight requests.
    const uint32_t channel = 16u * tile + n0 + (threadIdx.x & 7u);
    const bool finisher = threadIdx.x < 8u;
    const bool has_residual = residual != nullptr;
    const bool has_shared = kShared || (shared_output != nullptr && shared_gate != nullptr);
    const uint32_t residual_bits = (has_residual ? residual : mid)[has_residual ? channel : 0u];
    uint32_t shared_bits = 0u, gate_bits = 0u;
    if constexpr (kShared) {
        gate_bits = shared.gate[0];
    } else {
        shared_bits = (has_shared ? shared_output : mid)[has_shared ? channel : 0u];
        gate_bits = (has_shared ? shared_gate : mid)[0];
    }

    const int32_t id = active ? ids[route] : -1;
    // the scratch holds ten mid rows, so a route past top_k reads one too
    // (straight-line, no wait at a branch join); its partial is dropped
    const uint4 mv = reinterpret_cast<const uint4*>(mid + static_cast<size_t>(route) * I)[lane];
    const bool valid = id >= 0 && id < static_cast<int32_t>(kExperts);
    const uint32_t e = valid ? static_cast<uint32_t>(id) : 0u;

    const uint32_t c = lane & 7u;
    constexpr uint32_t kBlocks = I / 64u;  // W8
    constexpr uint32_t kW8Groups = kBlocks / kPerGroup;
    uint4 bq[4];
    uint2 sc = make_uint2(0u, 0u);
    uint32_t ws_bits = 0u;
    if constexpr (kW4) {
        // lane = c + 8*(kq + 4*qh): quad kq, chunks q = 2qh, 2qh+1
        constexpr uint32_t kQuads = I / 128u;
        const uint32_t kq = (lane >> 3) & 3u, qh = lane >> 5;
        const size_t t = (static_cast<size_t>(e) * kQuads + kq) * kTiles + tile;
        const uint4* wp = w + t * 64u + 32u * qh + n0 + c;
        bq[0] = wp[0];
        bq[1] = wp[16];
        sc = load_quad_scales<kPerGroup, false>(s + (t * 16u + n0 + c) * (4u / kPerGroup));
    } else {
        // lane = c + 8*kb: 64-column block kb, chunks q = 0..3
        const uint32_t kb = lane >> 3;
        const uint4* wp = w + ((static_cast<size_t>(e) * kTiles + tile) * kBlocks + kb) * 64u + n0 + c;
        bq[0] = wp[0];
        bq[1] = wp[16];
        bq[2] = wp[32];
        bq[3] = wp[48];
        // this lane's group (per channel: the one scale), artifact order; a
        // relaxed atomic load, which the compiler keeps here instead of
        // sinking it to its use after the barrier (a full round trip there)
        ws_bits = __hip_atomic_load(
            s + (static_cast<size_t>(e) * H + 16u * tile + n0 + c) * kW8Groups + kb / kPerGroup,
            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    // every request above is out before the quantisation below waits for
    // the mid row
    __builtin_amdgcn_sched_barrier(0);
    stamps.mark(1);

    // quantise this route's mid row (8 elements per lane)
    const uint32_t mw[4] = {mv.x, mv.y, mv.z, mv.w};
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        amax = fmaxf(amax, fabsf(bf16_to_f32(mw[i] & 0xffffu)));
        amax = fmaxf(amax, fabsf(bf16_to_f32(mw[i] >> 16)));
    }
    const QuantScale mid_q = quant_scale(wave_max_f32(amax));
    const float sm = mid_q.s;
    reinterpret_cast<uint2*>(mq_lds[route])[lane] = quantize8(mw, mid_q);
    __syncthreads();
    stamps.mark(2);
    stamps.mark_loaded(3);
    stamps.mark_wave_loaded(wave_stamp_lds);

    float o = 0.0f;
    if constexpr (kW4) {
        // chunk q of quad kq covers, for group j, k = 32(4kq+j) + 8q + {0..7}
        const uint32_t kq = (lane >> 3) & 3u, qh = lane >> 5;
        const uint32_t* mrow = reinterpret_cast<const uint32_t*>(mq_lds[route]);
        int acc[4] = {0, 0, 0, 0};
#pragma unroll
        for (uint32_t h = 0; h < 2u; ++h) {
            const uint32_t q = 2u * qh + h;
            const uint32_t wq[4] = {bq[h].x, bq[h].y, bq[h].z, bq[h].w};
#pragma unroll
            for (uint32_t j = 0; j < 4u; ++j) {
                const uint32_t d = (32u * (4u * kq + j) + 8u * q) >> 2;
                const uint2 xv = *reinterpret_cast<const uint2*>(mrow + d);
                acc[j] = __builtin_amdgcn_sdot4(static_cast<int>((wq[j] << 4) & 0xf0f0f0f0u), static_cast<int>(xv.x), acc[j], false);
                acc[j] = __builtin_amdgcn_sdot4(static_cast<int>(wq[j] & 0xf0f0f0f0u), static_cast<int>(xv.y), acc[j], false);
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < 4u; ++j) acc[j] += __shfl_xor(acc[j], 32, 64);
        float gs[4u / kPerGroup];
        int gacc[4u / kPerGroup];
#pragma unroll
        for (uint32_t gi = 0; gi < 4u / kPerGroup; ++gi) {
            gs[gi] = scale_to_f32(quad_scale_word(sc, gi), bf16) * 0.0625f;
            gacc[gi] = acc[gi * kPerGroup];
#pragma unroll
            for (uint32_t j = 1; j < kPerGroup; ++j) gacc[gi] += acc[gi * kPerGroup + j];
        }
        // chain over the four quads: lane c + 8kq continues lane c + 8(kq-1)
        float y = 0.0f;
#pragma unroll
        for (uint32_t step = 0; step < 4u; ++step) {
            float t = __shfl_up(y, 8, 64);
            if (kq == 0u) t = 0.0f;
#pragma unroll
            for (uint32_t gi = 0; gi < 4u / kPerGroup; ++gi)
                t = __builtin_fmaf(static_cast<float>(gacc[gi]), gs[gi], t);
            y = t;
        }
        o = __shfl(y, static_cast<int>(24u + c), 64) * sm;
    } else {
        const uint32_t kb = lane >> 3;
        const uint4* mrow = mq_lds[route] + 4u * kb;
        const float ws = scale_to_f32(ws_bits, bf16);
        int acc = 0;
#pragma unroll
        for (uint32_t q = 0; q < 4u; ++q) {
            const uint4 xv = mrow[q];
            acc = __builtin_amdgcn_sdot4(static_cast<int>(bq[q].x), static_cast<int>(xv.x), acc, false);
            acc = __builtin_amdgcn_sdot4(static_cast<int>(bq[q].y), static_cast<int>(xv.y), acc, false);
            acc = __builtin_amdgcn_sdot4(static_cast<int>(bq[q].z), static_cast<int>(xv.z), acc, false);
            acc = __builtin_amdgcn_sdot4(static_cast<int>(bq[q].w), static_cast<int>(xv.w), acc, false);
        }
        if constexpr (kPerGroup == kBlocks) {
            // lanes c + 8 kb, kb = 0..7: row_ror 8 within the row, then the
            // row pairs and the halves by the permlane swaps
            acc += __builtin_amdgcn_update_dpp(0, acc, 0x128, 0xf, 0xf, false);
            const auto rows = __builtin_amdgcn_permlane16_swap(acc, acc, false, false);
            acc = static_cast<int>(rows[0]) + static_cast<int>(rows[1]);
            const auto halves = __builtin_amdgcn_permlane32_swap(acc, acc, false, false);
            acc = static_cast<int>(halves[0]) + static_cast<int>(halves[1]);
            o = (static_cast<float>(acc) * ws) * sm;
        } else {
            // group g = kb / kPerGroup: its blocks' sum, then the chain over
            // groups (lane c + 8*kPerGroup*g continues the previous group)
            if constexpr (kPerGroup == 2u) acc += __shfl_xor(acc, 8, 64);
            const uint32_t g = kb / kPerGroup;
            float y = 0.0f;
#pragma unroll
            for (uint32_t step = 0; step < kW8Groups; ++step) {
                float t = __shfl_up(y, static_cast<int>(8u * kPerGroup), 64);
                if (g == 0u) t = 0.0f;
                y = __builtin_fmaf(static_cast<float>(acc), ws, t);
            }
            o = __shfl(y, static_cast<int>(8u * kPerGroup * (kW8Groups - 1u) + c), 64) * sm;
        }
    }
    stamps.mark(4);
    if (lane < 8u) reinterpret_cast<float*>(o_lds[lane])[route] = valid ? o : 0.0f;
    __syncthreads();
    stamps.mark(5);
    if (finisher) {
        // routes summed in rank order
        const float4 p0 = o_lds[threadIdx.x][0], p1 = o_lds[threadIdx.x][1];
        const float4 p2 = o_lds[threadIdx.x][2];
        const float part[12] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w,
                                p2.x, p2.y, p2.z, p2.w};
        float total = 0.0f;
#pragma unroll
        for (uint32_t r = 0; r < kTopK; ++r)
            if (r < top_k) total += part[r];
        if (has_shared) {
            if constexpr (kShared) shared_bits = shared_lds[threadIdx.x];
            const float g = bf16_to_f32(gate_bits);
            const float multiplier = 1.0f / (1.0f + exp_q(-g));
            total = __builtin_fmaf(bf16_to_f32(shared_bits), multiplier, total);
        }
        uint32_t result = f32_to_bf16(total);
        if (has_residual)
            result = f32_to_bf16(bf16_to_f32(residual_bits) + bf16_to_f32(result));
        out[channel] = static_cast<uint16_t>(result);
    }
    stamps.mark(6);
    stamps.finish(1u, call, wave_stamp_lds);
}

}  // namespace

size_t decode_scratch_bytes() {
    return 256u + static_cast<size_t>(kTopK) * kInter * sizeof(uint16_t);
}

// The decode block's scratch: the decode scratch (ids, mid rows), then the
// router's fp32 logits, the shared expert's h (bf16) and its output gate.
constexpr size_t kBlockLogits = 256u + static_cast<size_t>(kTopK) * kInter * sizeof(uint16_t);
constexpr size_t kBlockH = kBlockLogits + kExperts * sizeof(float);
constexpr size_t kBlockGate = kBlockH + kInter * sizeof(uint16_t);
size_t decode_block_scratch_bytes() { return kBlockGate + 256u; }

namespace {

template <bool kW4, uint32_t kPerGroup, bool kShared>
void launch_decode_down(const q38m_expert_weights_v1& down, const uint16_t* mid,
                        const int32_t* ids, uint32_t top_k, const uint16_t* shared_output,
                        const uint16_t* shared_gate, const uint16_t* residual, uint16_t* output,
                        PhaseCall call, SharedDown shared, hipStream_t stream) {
    decode_down_kernel<kHidden, kInter, kW4, kPerGroup, kShared>
        <<<kDecodeBlocks, kShared ? kDecodeThreads + 128u : kDecodeThreads, 0, stream>>>(
            static_cast<const uint4*>(down.data), static_cast<const uint16_t*>(down.scales),
            down.scale_dtype == Q38M_SCALE_BF16, mid, ids, top_k, shared_output, shared_gate,
            residual, output, call, shared);
}

// the two routed launches; kShared: with the shared expert (the decode block)
template <bool kShared>
hipError_t launch_decode_routed(const q38m_expert_weights_v1& gate_up,
                                const q38m_expert_weights_v1& down, const uint16_t* hidden,
                                const float* logits, const int32_t* ids, const float* weights,
                                uint32_t top_k, const uint16_t* shared_output,
                                const uint16_t* shared_gate, const uint16_t* residual,
                                void* scratch, uint16_t* output, SharedGateUp sgu,
                                SharedDown sdn, hipStream_t stream) {
    int32_t* scratch_ids = static_cast<int32_t*>(scratch);
    uint16_t* mid = reinterpret_cast<uint16_t*>(static_cast<char*>(scratch) + 256);
    const uint4* gw = static_cast<const uint4*>(gate_up.data);
    const uint16_t* gs = static_cast<const uint16_t*>(gate_up.scales);
    const bool gbf16 = gate_up.scale_dtype == Q38M_SCALE_BF16;
    int32_t* ids_out = logits != nullptr ? scratch_ids : nullptr;
    const PhaseCall call = next_phase_call();
    // the down weights' scale words per channel (W8) or per row and quad
    // (W4); the descriptor's format and group size were validated
    const bool down_w4 = down.format == Q38M_FORMAT_W4_SYM;
    const uint32_t down_scale_words =
        down_w4 ? 128u / down.group_size : (down.group_size == 0u ? 1u : kInter / down.group_size);
    const DownPrefetch prefetch{static_cast<const uint8_t*>(down.data),
                                static_cast<const uint16_t*>(down.scales), down_w4 ? 1u : 0u,
                                down_scale_words};
    auto gate_up_launch = [&](auto w8, auto per) {
        decode_gate_up_kernel<kHidden, kInter, decltype(w8)::value, decltype(per)::value, kShared>
            <<<kDecodeBlocks, kGateUpThreads, 0, stream>>>(gw, gs, gbf16, hidden, logits, ids,
                                                           weights, top_k, ids_out, mid, call,
                                                           sgu, prefetch);
    };
    using W4 = std::false_type;
    using W8 = std::true_type;
    if (gate_up.format == Q38M_FORMAT_W8_SYM) {
        switch (gate_up.group_size) {
            case 0u: gate_up_launch(W8{}, std::integral_constant<uint32_t, kHidden / 64u>{}); break;
            case 64u: gate_up_launch(W8{}, std::integral_constant<uint32_t, 1>{}); break;
            case 128u: gate_up_launch(W8{}, std::integral_constant<uint32_t, 2>{}); break;
            default: return hipErrorInvalidValue;
        }
    } else {
        switch (gate_up.group_size) {
            case 32u: gate_up_launch(W4{}, std::integral_constant<uint32_t, 1>{}); break;
            case 64u: gate_up_launch(W4{}, std::integral_constant<uint32_t, 2>{}); break;
            case 128u: gate_up_launch(W4{}, std::integral_constant<uint32_t, 4>{}); break;
            default: return hipErrorInvalidValue;
        }
    }
    const int32_t* down_ids = logits != nullptr ? scratch_ids : ids;
    constexpr uint32_t kBlocks = kInter / 64u;
    const bool w8 = down.format == Q38M_FORMAT_W8_SYM;
    auto down_launch = [&](auto w4, auto per) {
        launch_decode_down<decltype(w4)::value, decltype(per)::value, kShared>(
            down, mid, down_ids, top_k, shared_output, shared_gate, residual, output, call, sdn,
            stream);
    };
    switch (down.group_size) {
        case 0u:
            if (!w8) return hipErrorInvalidValue;
            down_launch(std::false_type{}, std::integral_constant<uint32_t, kBlocks>{});
            break;
        case 32u:
            if (w8) return hipErrorInvalidValue;
            down_launch(std::true_type{}, std::integral_constant<uint32_t, 1>{});
            break;
        case 64u:
            if (w8)
                down_launch(std::false_type{}, std::integral_constant<uint32_t, 1>{});
            else
                down_launch(std::true_type{}, std::integral_constant<uint32_t, 2>{});
            break;
        case 128u:
            if (w8)
                down_launch(std::false_type{}, std::integral_constant<uint32_t, 2>{});
            else
                down_launch(std::true_type{}, std::integral_constant<uint32_t, 4>{});
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_decode(const q38m_expert_weights_v1& gate_up,
                         const q38m_expert_weights_v1& down, const uint16_t* hidden,
                         const float* logits, const int32_t* ids, const float* weights,
                         uint32_t top_k, const uint16_t* shared_output,
                         const uint16_t* shared_gate, const uint16_t* residual, void* scratch,
                         uint16_t* output, hipStream_t stream) {
    return launch_decode_routed<false>(gate_up, down, hidden, logits, ids, weights, top_k,
                                       shared_output, shared_gate, residual, scratch, output,
                                       SharedGateUp{}, SharedDown{}, stream);
}

hipError_t launch_decode_block(const q38m_expert_weights_v1& gate_up,
                               const q38m_expert_weights_v1& down, const uint16_t* hidden,
                               const uint16_t* router, const uint16_t* w_gate,
                               const uint16_t* w_up, const uint16_t* w_down,
                               const uint16_t* w_out_gate, uint32_t top_k,
                               const uint16_t* residual, void* scratch, uint16_t* output,
                               hipStream_t stream) {
    char* base = static_cast<char*>(scratch);
    float* logits = reinterpret_cast<float*>(base + kBlockLogits);
    uint16_t* h = reinterpret_cast<uint16_t*>(base + kBlockH);
    uint16_t* gate = reinterpret_cast<uint16_t*>(base + kBlockGate);
    // the router GEMV (the same launch as q38m_moe_router_v1 at one token)
    hipError_t e = launch_dense_gemm(hidden, router, 1u, kExperts, kHidden, logits, nullptr, stream);
    if (e != hipSuccess) return e;
    return launch_decode_routed<true>(gate_up, down, hidden, logits, nullptr, nullptr, top_k,
                                      nullptr, nullptr, residual, scratch, output,
                                      SharedGateUp{w_gate, w_up, w_out_gate, h, gate},
                                      SharedDown{w_down, h, gate}, stream);
}

}  // namespace q38m

#ifdef Q38M_PHASE_TIMESTAMPS
extern "C" {

int q38m_phase_log_v1(q38m_phase_record_v1* records, uint32_t capacity, int device) {
    if (capacity % 512u != 0u || (records == nullptr) != (capacity == 0u) || device < 0)
        return Q38M_ERR_INVALID_ARGUMENT;
    if (hipSetDevice(device) != hipSuccess) return Q38M_ERR_DEVICE;
    const uint32_t held = capacity / 512u;
    if (hipMemcpyToSymbol(HIP_SYMBOL(q38m::g_phase_records), &records, sizeof(records)) !=
            hipSuccess ||
        hipMemcpyToSymbol(HIP_SYMBOL(q38m::g_phase_calls_held), &held, sizeof(held)) != hipSuccess)
        return Q38M_ERR_DEVICE;
    q38m::g_phase_calls.store(0u);
    return Q38M_OK;
}

uint32_t q38m_phase_calls_v1(void) { return q38m::g_phase_calls.load(); }

}  // extern "C"
#endif
