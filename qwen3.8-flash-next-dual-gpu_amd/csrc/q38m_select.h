// Block-wide top-k of one 512-logit router row, shared by the prefill
// routing kernel and the fused decode.
//
// Order: value descending, expert id ascending on ties (the order of the
// reference's sort, cuda/q38_kernels.cu:431-458), expressed as unique
// 64-bit keys (order key << 32 | 511 - id) so that "larger key" is "ranked
// first".  Two levels (wave_top10, rank_candidates; the fused router GEMM
// runs level 1 in its epilogue and level 2 in a second kernel):
//   1. each of waves 0-7 finds the 10th largest 32-bit order key of its 64
//      logits by a radix search on the wave's ballots (bit 31 down to 0:
//      keep the bit if at least ten keys reach the prefix with it set), then
//      takes every key above it and, among the keys equal to it, the lowest
//      lanes (lowest ids) up to ten: the wave's top 10, written unordered to
//      LDS -- 80 candidates in eight lists that contain the top 10, because
//      every key above a top-10 key is itself in its wave's top 10;
//   2. eight threads per candidate count the larger keys in one list each
//      and a DPP sum adds the eight counts: the global rank.
// The thread holding rank r writes id_r and exp(l_r - l_0); values come
// back from the keys (exactly, -0 as +0, which leaves every difference
// l_r - l_0 unchanged).  The caller forms the rank-order denominator
// (cuda/q38_kernels.cu:460-479).
#pragma once

#include "q38m_device.h"
#include "q38m_internal.h"

namespace q38m {

constexpr uint32_t kSelectThreads = 64u * kTopK;  // ten waves

struct alignas(16) SelectLds {
    uint64_t cand[8u * kTopK];
    uint32_t wave_max[8];  // each wave's largest order key
};

// Monotonic unsigned key of a float: larger key = larger value; -0 and +0
// share a key (equal under <), NaN maps below every number.
__device__ __forceinline__ uint32_t order_key(float v) {
    const uint32_t b = __float_as_uint(v + 0.0f);
    const uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return v == v ? k : 0u;
}

// Inverse of order_key for non-NaN keys (-0 comes back as +0).
__device__ __forceinline__ float key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Sum over each aligned group of eight lanes, valid in the group's last lane.
__device__ __forceinline__ uint32_t group8_sum(uint32_t x) {
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x111, 0xf, 0xf, true));
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x112, 0xf, 0xf, true));
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x114, 0xf, 0xf, true));
    return x;
}

// Inclusive prefix sum over the 64 lanes of a wave by DPP alone: row_shr
// 1, 2, 4, 8 within each 16-lane row (lanes shifted in from outside the
// row add 0), then row_bcast:15 (each row's last lane into the next row,
// rows 1 and 3) and row_bcast:31 (lane 31 into rows 2 and 3).
__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t x) {
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x111, 0xf, 0xf, false));
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x112, 0xf, 0xf, false));
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x114, 0xf, 0xf, false));
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x118, 0xf, 0xf, false));
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x142, 0xa, 0xf, false));
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x143, 0xc, 0xf, false));
    return x;
}

// Reductions over the 64 lanes of a wave without LDS round trips: the quad
// and row steps by DPP (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror,
// row_mirror), then row pairs and wave halves by the permlane swaps (with
// both operands x, permlane16_swap returns rows [0,0,2,2] and [1,1,3,3],
// permlane32_swap the halves [lo,lo] and [hi,hi]).  Every lane receives the
// result.  For max and integer sums the order of the steps does not matter.
template <typename Op>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t x, Op op) {
    x = op(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0xb1, 0xf, 0xf, false)));
    x = op(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x4e, 0xf, 0xf, false)));
    x = op(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x141, 0xf, 0xf, false)));
    x = op(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x140, 0xf, 0xf, false)));
    const auto rows = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    x = op(static_cast<uint32_t>(rows[0]), static_cast<uint32_t>(rows[1]));
    const auto halves = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return op(static_cast<uint32_t>(halves[0]), static_cast<uint32_t>(halves[1]));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
    return wave_reduce_u32(x, [](uint32_t a, uint32_t b) { return max(a, b); });
}

// ---- bf16 row dot products, one wave per row (the GEMV form) --------------
// fp32 dot product of a bf16 weight row with a bf16 activation row: lane l
// takes the 16-byte chunks l, l + 64, l + 128, l + 192 of each pass of 256
// chunks (every load instruction eight whole 128-byte lines), each chunk's
// eight products accumulated into its own fp32 partial in k order, the
// partials added to the running total in chunk order, then the lanes summed
// by wave_reduce_u32's fixed DPP / permlane tree.  Every addition is in a
// fixed order, so the result is the same on every run and in every kernel
// that uses these helpers (the dense GEMV, the decode block's shared
// expert).  A pass's loads (bf16_row_load) can be issued well before its
// products (bf16_row_accumulate).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct Bf16RowPass {
    u32x4 w[4], x[4];
};

// chunks [base, base + 256) of a row of `chunks` 16-byte chunks
__device__ __forceinline__ Bf16RowPass bf16_row_load(const uint16_t* __restrict__ a,
                                                     const uint16_t* __restrict__ row,
                                                     uint32_t chunks, uint32_t base,
                                                     uint32_t lane) {
    const u32x4* av = reinterpret_cast<const u32x4*>(a);
    const u32x4* bv = reinterpret_cast<const u32x4*>(row);
    Bf16RowPass p;
#pragma unroll
    for (uint32_t i = 0; i < 4u; ++i) {
        const uint32_t c = base + 64u * i + lane;
        const bool in = c < chunks;
        p.w[i] = in ? bv[c] : u32x4{0u, 0u, 0u, 0u};
        p.x[i] = in ? av[c] : u32x4{0u, 0u, 0u, 0u};
    }
    return p;
}

__device__ __forceinline__ float bf16_row_accumulate(const Bf16RowPass& p, float total) {
#pragma unroll
    for (uint32_t i = 0; i < 4u; ++i) {
        float part = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < 4u; ++j) {
            part = __builtin_fmaf(bf16_to_f32(p.x[i][j] & 0xffffu), bf16_to_f32(p.w[i][j] & 0xffffu), part);
            part = __builtin_fmaf(bf16_to_f32(p.x[i][j] >> 16), bf16_to_f32(p.w[i][j] >> 16), part);
        }
        total += part;
    }
    return total;
}

__device__ __forceinline__ float wave_sum_f32(float total) {
    return __uint_as_float(wave_reduce_u32(__float_as_uint(total), [](uint32_t x, uint32_t y) {
        return __float_as_uint(__uint_as_float(x) + __uint_as_float(y));
    }));
}

// the whole dot product over k (k % 8 == 0), the sum in every lane
__device__ __forceinline__ float wave_dot_bf16(const uint16_t* __restrict__ a,
                                               const uint16_t* __restrict__ row, uint32_t k,
                                               uint32_t lane) {
    const uint32_t chunks = k / 8u;
    float total = 0.0f;
    for (uint32_t base = 0; base < chunks; base += 256u)
        total = bf16_row_accumulate(bf16_row_load(a, row, chunks, base, lane), total);
    return wave_sum_f32(total);
}

__device__ __forceinline__ float wave_max_f32(float x) {
    return __uint_as_float(wave_reduce_u32(__float_as_uint(x), [](uint32_t a, uint32_t b) {
        return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
    }));
}

// Level 1 for one wave: the wave's top 10 of its 64 order keys (k32 of
// lane l, expert `expert`), found by a radix search on the wave's ballots
// (bit 31 down to 0: keep the bit if at least ten keys reach the prefix
// with it set), then every key above the threshold and, among the keys
// equal to it, the lowest lanes up to ten.  Lanes must hold ascending
// expert ids.  store(position, key64) receives the ten unique keys
// (k32 << 32 | 511 - expert) in positions 0..9, unordered; returns the
// wave's largest order key (in every lane).  Wave-uniform control flow.
template <typename Store>
__device__ __forceinline__ uint32_t wave_top10(uint32_t k32, uint32_t expert, Store store) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t prefix = 0u;
    // Unrolled, so the prefix stays in scalar registers (a rolled loop
    // carries it and the bit index in vector registers): per bit, scalar
    // count, compare, select, next candidate and exit test -- the waves share
    // the CU's scalar unit, and the compiler's own popcount of a 64-bit
    // ballot adds a 64-bit vector compare and an exec mask step.
#pragma unroll
    for (int b = 31; b >= 0; --b) {
        const uint32_t cand = prefix | (1u << b);
        const uint64_t reach = __builtin_amdgcn_ballot_w64(k32 >= cand);
        uint32_t count;
        asm("s_bcnt1_i32_b64 %0, %1" : "=s"(count) : "s"(reach));
        prefix = count >= kTopK ? cand : prefix;
        // exactly ten keys reach the prefix: they are the wave's top 10
        // (below, "above" and the ties at the prefix make up exactly that
        // set whether or not the prefix is itself a key), so the remaining
        // bits cannot change the selection.  Distinct logits usually get
        // here once the prefix separates the 10th key from the 11th, about
        // half way down.
        if (count == kTopK) break;
    }
    const uint64_t below = (1ull << lane) - 1ull;
    const uint64_t above = __ballot(k32 > prefix);
    const uint64_t equal = __ballot(k32 == prefix);
    const uint32_t need = kTopK - static_cast<uint32_t>(__popcll(above));
    const bool mine_eq = k32 == prefix && static_cast<uint32_t>(__popcll(equal & below)) < need;
    const uint64_t chosen = above | __ballot(mine_eq);
    if (k32 > prefix || mine_eq)
        store(static_cast<uint32_t>(__popcll(chosen & below)),
              (static_cast<uint64_t>(k32) << 32) | (kExperts - 1u - expert));
    return wave_max_u32(k32);
}

// wave_top10 over kRows independent rows at once (row r: k32[r] of lane
// l, expert `expert`): the rows' radix searches advance together, one bit
// per pass, so their scalar chains overlap.  store(row, position, key64);
// kmax[r] receives row r's largest order key.
template <uint32_t kRows, typename Store>
__device__ __forceinline__ void wave_top10_rows(const uint32_t (&k32)[kRows], uint32_t expert,
                                                Store store, uint32_t (&kmax)[kRows]) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t prefix[kRows];
#pragma unroll
    for (uint32_t r = 0; r < kRows; ++r) prefix[r] = 0u;
#pragma unroll
    for (int b = 31; b >= 0; --b) {
#pragma unroll
        for (uint32_t r = 0; r < kRows; ++r) {
            const uint32_t cand = prefix[r] | (1u << b);
            const uint64_t reach = __builtin_amdgcn_ballot_w64(k32[r] >= cand);
            uint32_t count;
            asm("s_bcnt1_i32_b64 %0, %1" : "=s"(count) : "s"(reach));
            prefix[r] = count >= kTopK ? cand : prefix[r];
        }
    }
    const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
    for (uint32_t r = 0; r < kRows; ++r) {
        const uint64_t above = __ballot(k32[r] > prefix[r]);
        const uint64_t equal = __ballot(k32[r] == prefix[r]);
        const uint32_t need = kTopK - static_cast<uint32_t>(__popcll(above));
        const bool mine_eq =
            k32[r] == prefix[r] && static_cast<uint32_t>(__popcll(equal & below)) < need;
        const uint64_t chosen = above | __ballot(mine_eq);
        if (k32[r] > prefix[r] || mine_eq)
            store(r, static_cast<uint32_t>(__popcll(chosen & below)),
                  (static_cast<uint64_t>(k32[r]) << 32) | (kExperts - 1u - expert));
        kmax[r] = wave_max_u32(k32[r]);
    }
}

// Level 2: lds.cand holds kLists lists of ten keys that contain the top 10
// (every key above a top-10 key is in its list's top 10), lds.wave_max the
// lists' largest order keys, visible to the block.  kLists threads per
// candidate (threads t < 10 kLists^2) count the larger keys in one list
// each and a DPP sum adds the counts: the global rank.  The thread holding
// rank r writes ids[r] and num[r] = exp(l_r - l_0); values come back from
// the keys (exactly, -0 as +0, which leaves every difference unchanged).
template <uint32_t kLists>
__device__ __forceinline__ void rank_candidates(const SelectLds& lds, int32_t* ids, float* num) {
    static_assert(kLists == 8u, "groups of eight lanes");
    const uint32_t t = threadIdx.x;
    if (t >= kTopK * kLists * kLists) return;
    const uint32_t c = t / kLists, list = t % kLists;
    const uint64_t mine = lds.cand[c];
    const uint64_t* other = lds.cand + kTopK * list;
    uint32_t larger = 0;
#pragma unroll
    for (uint32_t j = 0; j < kTopK; j += 2u) {
        const ulonglong2 pr = *reinterpret_cast<const ulonglong2*>(other + j);
        larger += pr.x > mine ? 1u : 0u;
        larger += pr.y > mine ? 1u : 0u;
    }
    // l_0's order key: the largest of the list maxima
    const uint4 m0 = *reinterpret_cast<const uint4*>(lds.wave_max);
    const uint4 m1 = *reinterpret_cast<const uint4*>(lds.wave_max + 4);
    const uint32_t top = max(max(max(m0.x, m0.y), max(m0.z, m0.w)),
                             max(max(m1.x, m1.y), max(m1.z, m1.w)));
    const uint32_t rank = group8_sum(larger);
    if (list == kLists - 1u && rank < kTopK) {
        ids[rank] = static_cast<int32_t>(kExperts - 1u - static_cast<uint32_t>(mine & 0xffffffffu));
        num[rank] = exp_q(key_value(static_cast<uint32_t>(mine >> 32)) - key_value(top));
    }
}

// popcount of a wave-uniform 64-bit mask, on the scalar unit
__device__ __forceinline__ uint32_t scalar_popcount(uint64_t mask) {
    uint32_t count;
    asm("s_bcnt1_i32_b64 %0, %1" : "=s"(count) : "s"(mask));
    return count;
}

// popcount of mask's bits below this lane
__device__ __forceinline__ uint32_t count_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

// Top-10 of one 512-logit row by ONE wave, lane l holding the logits of
// experts l + 64j (j = 0..7):
//   1. the 10th largest 32-bit order key of the 512 by a radix search on
//      the wave's ballots (bit 31 down: keep the bit if at least ten keys
//      reach the prefix with it set; stop once exactly ten do), eight
//      ballots and scalar popcounts per bit -- no cross-lane data movement;
//   2. every key above it and, among the keys equal to it, the lowest
//      expert ids up to ten: the top 10, written as unique 64-bit keys
//      (order key << 32 | 511 - id) to the wave's ten slots top_lds[0..9];
//   3. lanes 0-9 rank their slot's key among the ten (the count of larger
//      keys): the order (value desc, id asc) of block_topk512.
// emit(rank, id, exp(l_rank - l_0)) runs in lanes 0-9, each rank once; the
// values come back from the keys as in rank_candidates.  Wave-uniform
// control flow; top_lds is the calling wave's own.
template <typename Emit>
__device__ __forceinline__ void wave_top10_of_512(const float (&v)[kExperts / 64u],
                                                  uint64_t* top_lds, Emit emit) {
    constexpr uint32_t kPerLane = kExperts / 64u;
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t key[kPerLane];
#pragma unroll
    for (uint32_t j = 0; j < kPerLane; ++j) key[j] = order_key(v[j]);
    // 1. the threshold (unrolled, so the prefix stays in scalar registers)
    uint32_t prefix = 0u;
#pragma unroll
    for (int b = 31; b >= 0; --b) {
        const uint32_t cand = prefix | (1u << b);
        uint32_t count = 0u;
#pragma unroll
        for (uint32_t j = 0; j < kPerLane; ++j)
            count += scalar_popcount(__builtin_amdgcn_ballot_w64(key[j] >= cand));
        prefix = count >= kTopK ? cand : prefix;
        // exactly ten keys reach the prefix: they are the top 10
        if (count == kTopK) break;
    }
    // 2. the ten, in (j, lane) = expert id order among equal keys
    uint32_t above = 0u;
#pragma unroll
    for (uint32_t j = 0; j < kPerLane; ++j)
        above += scalar_popcount(__builtin_amdgcn_ballot_w64(key[j] > prefix));
    const uint32_t need = kTopK - above;
    uint32_t equal_before = 0u, taken = 0u;
#pragma unroll
    for (uint32_t j = 0; j < kPerLane; ++j) {
        const uint64_t equal = __builtin_amdgcn_ballot_w64(key[j] == prefix);
        const bool mine = key[j] > prefix ||
                          (key[j] == prefix && equal_before + count_below(equal) < need);
        const uint64_t chosen = __builtin_amdgcn_ballot_w64(mine);
        if (mine)
            top_lds[taken + count_below(chosen)] =
                (static_cast<uint64_t>(key[j]) << 32) | (kExperts - 1u - (lane + 64u * j));
        taken += scalar_popcount(chosen);
        equal_before += scalar_popcount(equal);
    }
    // the wave's own LDS writes are visible to its later reads
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    // 3. ranks and l_0
    uint64_t mine = 0u, top = 0u;
    uint32_t rank = 0u;
#pragma unroll
    for (uint32_t i = 0; i < kTopK; ++i) {
        const uint64_t other = top_lds[i];
        if (i == (lane < kTopK ? lane : 0u)) mine = other;
        top = other > top ? other : top;
    }
#pragma unroll
    for (uint32_t i = 0; i < kTopK; ++i) rank += top_lds[i] > mine ? 1u : 0u;
    if (lane < kTopK)
        emit(rank, static_cast<int32_t>(kExperts - 1u - static_cast<uint32_t>(mine & 0xffffffffu)),
             exp_q(key_value(static_cast<uint32_t>(mine >> 32)) -
                   key_value(static_cast<uint32_t>(top >> 32))));
}

// Block-wide top-k of one 512-logit row: called by all kSelectThreads
// threads of the block; `logit` is the row entry of threads 0..511.  LDS
// writes the caller made before the call are visible to the whole block on
// return.  On return ids[r] and num[r] (r < 10) hold the rank-r expert and
// exp(l_r - l_0).
// phase(i) is called after level 1 (i = 0), after the barrier that joins
// the lists (1) and after level 2 (2); the plain form passes a no-op.
template <typename Phase>
__device__ __forceinline__ void block_topk512(float logit, SelectLds& lds, int32_t* ids,
                                              float* num, Phase phase) {
    const uint32_t t = threadIdx.x;
    if (t < kExperts) {
        uint64_t* list = lds.cand + kTopK * (t >> 6);
        const uint32_t kmax = wave_top10(order_key(logit), t, [&](uint32_t at, uint64_t key) {
            list[at] = key;
        });
        if ((t & 63u) == 0u) lds.wave_max[t >> 6] = kmax;
    }
    phase(0u);
    __syncthreads();
    phase(1u);
    rank_candidates<8>(lds, ids, num);
    phase(2u);
    __syncthreads();
}

__device__ __forceinline__ void block_topk512(float logit, SelectLds& lds, int32_t* ids,
                                              float* num) {
    block_topk512(logit, lds, ids, num, [](uint32_t) {});
}

// max |x| over eight bf16 values (one 16-byte chunk)
__device__ __forceinline__ float row_absmax8(const uint32_t (&hw)[4]) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        amax = fmaxf(amax, fabsf(bf16_to_f32(hw[i] & 0xffffu)));
        amax = fmaxf(amax, fabsf(bf16_to_f32(hw[i] >> 16)));
    }
    return amax;
}

// int8 quantisation of one 2048-wide bf16 row held by threads 0..255 (eight
// elements each): s = absmax/127 (1 if zero), q = clamp(rint(x/s), +-127)
// (tools/q38_artifact_compiler.py:214-222).  Step 1 (before a barrier):
// the per-wave absmax of waves 0..3 into amax_lds.
__device__ __forceinline__ void row_absmax_partial(const uint32_t (&hw)[4], float* amax_lds) {
    const float amax = wave_max_f32(row_absmax8(hw));
    if ((threadIdx.x & 63u) == 0u) amax_lds[threadIdx.x >> 6] = amax;
}

// A row's quantisation scale s = absmax/127 (IEEE division, 1 if zero) and
// its reciprocal.  The contract rounds the quotient RN(x/s) to an integer.
// For bf16 x with |x| <= absmax and s in [2^-120, FLT_MAX], one Markstein
// correction step -- q0 = RN(x r), q = RN(q0 + RN(x - q0 s) r) with two
// fmas and r = RN(1/s) formed once per row -- rounds to the same integer as
// RN(x/s): checked over all 5.3e8 such (absmax, x) pairs of bf16 values
// (tests/quantize_division_check.c).  Other scales (tiny or infinite rows)
// take the IEEE division.  fast is uniform over the row's threads.
struct QuantScale {
    float s, r;
    bool fast;
};

__device__ __forceinline__ QuantScale quant_scale(float amax) {
    float s = amax / 127.0f;
    if (s == 0.0f) s = 1.0f;
    const bool fast = s >= 0x1p-120f && s <= 0x1.fffffep+127f;
    return QuantScale{s, 1.0f / s, __builtin_amdgcn_readfirstlane(fast ? 1 : 0) != 0};
}

// q = clamp(rint(x/s), -127, 127) of the contract for eight bf16 values (NaN
// quotients clamp to -127 through fmin(fmax()))
template <bool kFast>
__device__ __forceinline__ uint2 quantize8_with(const uint32_t (&hw)[4], float s, float r) {
    uint32_t packed[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t h = (i & 1) ? (hw[i >> 1] >> 16) : (hw[i >> 1] & 0xffffu);
        const float x = bf16_to_f32(h);
        float quotient;
        if constexpr (kFast) {
            const float q0 = x * r;
            quotient = __builtin_fmaf(__builtin_fmaf(-q0, s, x), r, q0);
        } else {
            quotient = x / s;
        }
        const float v = fminf(fmaxf(__builtin_rintf(quotient), -127.0f), 127.0f);
        packed[i >> 2] |= (static_cast<uint32_t>(static_cast<int32_t>(v)) & 0xffu) << (8 * (i & 3));
    }
    return make_uint2(packed[0], packed[1]);
}

__device__ __forceinline__ uint2 quantize8(const uint32_t (&hw)[4], const QuantScale& q) {
    return q.fast ? quantize8_with<true>(hw, q.s, q.r) : quantize8_with<false>(hw, q.s, q.r);
}

// Step 2 (after the barrier): the row scale of the four waves' maxima.
__device__ __forceinline__ QuantScale row_scale(const float* amax_lds) {
    const float amax = fmaxf(fmaxf(amax_lds[0], amax_lds[1]), fmaxf(amax_lds[2], amax_lds[3]));
    return quant_scale(amax);
}

}  // namespace q38m
