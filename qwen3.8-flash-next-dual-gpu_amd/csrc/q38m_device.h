// Device helpers shared by the q38m HIP kernels (gfx950 / CDNA4).
//
// The fp32 epilogue is part of the arithmetic contract: every kernel is
// compiled with -ffp-contract=off and every fused multiply-add is an
// explicit __builtin_fmaf, so the GPU performs exactly the operations of
// the CPU restatement in the same order.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "q38m.h"

namespace q38m {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

// ---- streaming loads -----------------------------------------------------

// Expert weights are read once per launch: non-temporal loads keep that
// stream from evicting the activations every workgroup re-reads from L2.
typedef unsigned int v4u_t __attribute__((ext_vector_type(4)));
typedef unsigned int v2u_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint4 load_stream(const uint4* p) {
    const v4u_t v = __builtin_nontemporal_load(reinterpret_cast<const v4u_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint2 load_stream(const uint2* p) {
    const v2u_t v = __builtin_nontemporal_load(reinterpret_cast<const v2u_t*>(p));
    return make_uint2(v.x, v.y);
}

// ---- checked build (-DQ38M_CHECKED: libq38m_checked.so) -------------------
// Index checks on values the kernels read from memory: the expert and row
// count of a task record, the plan's packed and inverse route indices.  In
// the checked build a value outside its range sets a bit of the status word
// of this translation unit (each unit has its own; q38m_checked_status_v1
// ORs them) and is replaced by 0, an in-range value, so the kernel completes
// without touching memory outside its buffers -- it never traps.  In the
// product build checked() is the value itself.
enum CheckBit : uint32_t {
    kCheckExpert = 1u,    // task expert >= 512
    kCheckTaskRows = 2u,  // task rows > the largest task (128)
    kCheckRoute = 4u,     // inverse (assignment -> packed) index >= routes
    kCheckToken = 8u,     // packed route index past the largest chunk
};

#ifdef Q38M_CHECKED
// Each unit registers a reader of its status word with the host
// (q38m_api.hip): a one-thread kernel that ORs the word into *out and, on
// reset, clears it (the word itself is internal to the unit, so no symbol
// lookup is involved).
bool register_checked_status(hipError_t (*read)(uint32_t* out, int reset, hipStream_t stream));
namespace {
__device__ uint32_t g_checked_status;
__global__ void checked_status_kernel(uint32_t* out, int reset) {
    if (threadIdx.x == 0u) {
        out[0] |= g_checked_status;
        if (reset) g_checked_status = 0u;
    }
}
hipError_t read_checked_status(uint32_t* out, int reset, hipStream_t stream) {
    checked_status_kernel<<<1, 64, 0, stream>>>(out, reset);
    return hipGetLastError();
}
[[maybe_unused]] const bool g_checked_registered = register_checked_status(&read_checked_status);
}  // namespace
#endif

__device__ __forceinline__ uint32_t checked(uint32_t v, uint32_t limit, CheckBit bit) {
#ifdef Q38M_CHECKED
    if (v >= limit) {
        atomicOr(&g_checked_status, static_cast<uint32_t>(bit));
        return 0u;
    }
#else
    (void)limit;
    (void)bit;
#endif
    return v;
}

// ---- plan tasks ------------------------------------------------------------
// A task record (q38m_task_v1: packed_begin, expert, valid_rows, flags) read
// as one 8-byte load of its two words: with a uniform index that is a single
// scalar load, where the struct's 16- and 8-bit fields would otherwise come
// from separate vector loads, a round trip each, before the first weight
// address of the task exists.
struct TaskRecord {
    uint32_t begin, expert, rows;
};
static_assert(sizeof(q38m_task_v1) == 8 && offsetof(q38m_task_v1, expert) == 4 &&
                  offsetof(q38m_task_v1, valid_rows) == 6,
              "read_task unpacks the record's second word as expert | valid_rows << 16");

__device__ __forceinline__ TaskRecord read_task(const q38m_task_v1* __restrict__ tasks,
                                                uint32_t index) {
    const uint2 w = reinterpret_cast<const uint2*>(tasks)[index];
    return TaskRecord{w.x, checked(w.y & 0xffffu, Q38M_ROUTE_EXPERTS, kCheckExpert),
                      checked((w.y >> 16) & 0xffu, Q38M_WIDE_TASK_ROWS + 1u, kCheckTaskRows)};
}

// ---- conversions ---------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint32_t h) {
    return __uint_as_float(h << 16);
}

// Round-to-nearest-even bf16 (tools/q38_artifact_compiler.py:61-66); a NaN
// keeps its sign and top payload bits with the quiet bit set.  This is the
// integer form the oracle restates; the kernels use bf16_hw below.
__device__ __forceinline__ uint32_t f32_to_bf16_int(float v) {
    const uint32_t b = __float_as_uint(v);
    const uint32_t rounded = (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
    const uint32_t quiet = (b >> 16) | 0x40u;
    return v != v ? quiet : rounded;
}

// The same rounding on the hardware conversion (v_cvt_pk_bf16_f32, what a
// cast to __bf16 compiles to on gfx950): equal to f32_to_bf16_int for all
// 2^32 inputs, NaNs included (q38m_debug_bf16_sweep checks every pattern
// on the device).
__device__ __forceinline__ uint32_t f32_to_bf16(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
}

// the same rounding, the result widened back to fp32
__device__ __forceinline__ float bf16_round(float v) {
    return bf16_to_f32(f32_to_bf16(v));
}

// Exact binary16 -> binary32 through the hardware conversion.
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// binary32 -> binary16, round-to-nearest-even, integer-only so the result
// does not depend on the conversion instruction's mode bits.
__device__ __forceinline__ uint32_t f32_to_f16(float v) {
    const uint32_t bits = __float_as_uint(v);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const uint32_t mag = bits & 0x7fffffffu;
    if (mag > 0x7f800000u) return sign | 0x7e00u;
    if (mag >= 0x477ff000u) return sign | 0x7c00u;
    if (mag >= 0x38800000u) {
        const uint32_t rounded = mag + 0x0fffu + ((mag >> 13) & 1u);
        return sign | ((rounded >> 13) - (112u << 10));
    }
    const uint32_t biased = mag >> 23;
    if (biased == 0u) return sign;
    const uint32_t shift = 126u - biased;
    if (shift > 24u) return sign;
    const uint32_t mant = (mag & 0x7fffffu) | 0x800000u;
    uint32_t result = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (result & 1u))) ++result;
    return sign | result;
}

// ---- the contract's exp ---------------------------------------------------
// Cody & Waite reduction x = n*ln2 + r (ln2 split so n*ln2_hi is exact),
// degree-7 Taylor polynomial of e^r in Horner form, exact 2^n scaling.
// Results below the smallest normal are flushed to 0 (x < -87.3).  The
// body runs on x clamped into its domain (equal to x wherever x is in it)
// and the special cases are selected afterwards, without branches.
__device__ __forceinline__ float exp_q(float x) {
    const float xb = __builtin_fminf(__builtin_fmaxf(x, -87.3f), 88.72283935546875f);
    const float n = __builtin_rintf(xb * 1.44269502162933349609375f);
    float r = __builtin_fmaf(n, -0.693145751953125f, xb);
    r = __builtin_fmaf(n, -1.42860682030941723212e-6f, r);
    float p = 1.98412698412698412698e-4f;
    p = __builtin_fmaf(p, r, 1.38888888888888888889e-3f);
    p = __builtin_fmaf(p, r, 8.33333333333333333333e-3f);
    p = __builtin_fmaf(p, r, 4.16666666666666666667e-2f);
    p = __builtin_fmaf(p, r, 1.66666666666666666667e-1f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int e = static_cast<int>(n);  // -126 .. 128
    const float scaled = e > 127 ? (p * 2.0f) * __uint_as_float(254u << 23)  // * 2^127
                                 : p * __uint_as_float(static_cast<uint32_t>(e + 127) << 23);
    const float ranged = x > 88.72283935546875f ? __builtin_huge_valf()
                                                : (x < -87.3f ? 0.0f : scaled);
    return x != x ? x + x : ranged;
}

// Every NaN bf16 word as the quiet NaN 0x7fc0.  A NaN's sign and payload
// follow the instruction set that produced it (the host table behind the
// chunk path's silu and the device's own exp and division differ), so the
// SwiGLU epilogues write NaN in this one form.
__device__ __forceinline__ uint32_t bf16_canonical_nan(uint32_t word) {
    return (word & 0x7fffu) > 0x7f80u ? 0x7fc0u : word;
}

// SwiGLU with the router-weight fold; rounding sequence of the reference
// gate/up epilogue (cuda/q38_moe_prefill.cu:449-461); NaN as 0x7fc0.
__device__ __forceinline__ uint32_t swiglu_fold(float y_gate, float y_up,
                                                float weight) {
    const float g = bf16_round(y_gate);
    const float u = bf16_round(y_up);
    const float e = exp_q(-g);
    const float den = 1.0f + e;
    const float silu = g / den;
    const float h = bf16_round(silu * u);
    return bf16_canonical_nan(f32_to_bf16(h * weight));
}

// The shared expert's h = bf16(g / (1 + exp(-g)) * u) on bf16 g and u
// (cuda_silu_multiply_bf16, q38_kernels.cu:286-296, with this library's exp).
__device__ __forceinline__ uint32_t silu_multiply(uint32_t g_bits, uint32_t u_bits) {
    const float g = bf16_to_f32(g_bits);
    return f32_to_bf16((g / (1.0f + exp_q(-g))) * bf16_to_f32(u_bits));
}

// ---- int8 MFMA -------------------------------------------------------------
// v_mfma_i32_16x16x32_i8: A 16x32 (lane l: row l%16, k 8*(l/16)..+7),
// B 32x16 (lane l: column l%16, same k), D lane l: rows 4*(l/16)+i,
// column l%16.  One instruction covers exactly one 32-wide scale group.
__device__ __forceinline__ v4i mfma_i8_16x16x32(long a, long b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}

// ---- group scales ----------------------------------------------------------
// Scale words are fp16 (Q38M_SCALE_F16) or bf16 (Q38M_SCALE_BF16); both
// widen to fp32 exactly.
__device__ __forceinline__ float scale_to_f32(uint32_t word, bool bf16) {
    return bf16 ? bf16_to_f32(word & 0xffffu) : f16_to_f32(word & 0xffffu);
}

// The scale words of one row for one W4 quad (128 columns) in the MFMA16
// layouts ([E][K/128][slot][16 rows][128/group] words): 4, 2 or 1 words for
// groups of 32, 64 or 128 columns, i.e. kSub = group/32 sub-blocks of 32
// per group.  Word gi of the quad is quad_scale_word(result, gi).  kStream:
// non-temporal loads (weights read once per call) or ordinary cached loads
// (weights re-read by several tasks of one expert).
template <uint32_t kSub, bool kStream = true>
__device__ __forceinline__ uint2 load_quad_scales(const uint16_t* row_words) {
    static_assert(kSub == 1u || kSub == 2u || kSub == 4u, "groups of 32, 64 or 128");
    if constexpr (!kStream) {
        if constexpr (kSub == 1u) return *reinterpret_cast<const uint2*>(row_words);
        else if constexpr (kSub == 2u)
            return make_uint2(*reinterpret_cast<const uint32_t*>(row_words), 0u);
        else return make_uint2(*row_words, 0u);
    } else if constexpr (kSub == 1u) {
        const v2u_t v = __builtin_nontemporal_load(reinterpret_cast<const v2u_t*>(row_words));
        return make_uint2(v.x, v.y);
    } else if constexpr (kSub == 2u) {
        return make_uint2(__builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(row_words)),
                          0u);
    } else {
        return make_uint2(__builtin_nontemporal_load(row_words), 0u);
    }
}
__device__ __forceinline__ uint32_t quad_scale_word(uint2 words, uint32_t gi) {
    const uint32_t d = gi < 2u ? words.x : words.y;
    return (gi & 1u) ? d >> 16 : d & 0xffffu;
}

// v_mfma_i32_16x16x64_i8 (gfx950): 16 int8 per lane per operand.
__device__ __forceinline__ v4i mfma_i8_16x16x64(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// v_mfma_i32_32x32x32_i8 (gfx950): A 32x32 (lane l: row l%32, k
// 16*(l/32)..+15), B 32x32 (lane l: column l%32, same k), D lane l:
// column l%32, rows 8*(i/4) + 4*(l/32) + i%4 for i = 0..15.  Like the
// 16x16x32 form it covers one 32-wide scale group, at twice its MAC rate.
typedef int v16i __attribute__((ext_vector_type(16)));
__device__ __forceinline__ v16i mfma_i8_32x32x32(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// Expands one MFMA16 W4 dword (byte i = k_i | k_{4+i} << 4) into the eight
// int8 B-operand bytes k_0..k_7, each multiplied by 16: the nibble lands
// in the high half of its byte, so the sign needs no extension.  The x16
// is exact and is removed by scaling the group scale by 1/16.
__device__ __forceinline__ long unpack_w4x16(uint32_t w) {
    const uint32_t lo = (w << 4) & 0xf0f0f0f0u;
    const uint32_t hi = w & 0xf0f0f0f0u;
    return static_cast<long>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ long as_long(uint2 v) {
    return static_cast<long>((static_cast<uint64_t>(v.y) << 32) | v.x);
}

__device__ __forceinline__ v4i as_v4i(uint4 v) {
    v4i r;
    r.x = static_cast<int>(v.x);
    r.y = static_cast<int>(v.y);
    r.z = static_cast<int>(v.z);
    r.w = static_cast<int>(v.w);
    return r;
}

// ---- counter-based SplitMix64 (Steele, Lea, Flood 2014) -------------------
constexpr uint64_t kGamma = 0x9e3779b97f4a7c15ull;

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z ^= z >> 30;
    z *= 0xbf58476d1ce4e5b9ull;
    z ^= z >> 27;
    z *= 0x94d049bb133111ebull;
    z ^= z >> 31;
    return z;
}

__host__ __device__ inline uint64_t stream_base_host(uint64_t seed, uint64_t tag) {
    uint64_t z = seed + kGamma * (tag + 1u);
    z ^= z >> 30;
    z *= 0xbf58476d1ce4e5b9ull;
    z ^= z >> 27;
    z *= 0x94d049bb133111ebull;
    z ^= z >> 31;
    return z;
}

__device__ __forceinline__ uint64_t stream_at(uint64_t base, uint64_t counter) {
    return mix64(base + kGamma * (counter + 1u));
}

// Natural log of a positive normal float (synthetic data only).
__device__ __forceinline__ float log_q(float x) {
    const uint32_t bits = __float_as_uint(x);
    int exponent = static_cast<int>(bits >> 23) - 127;
    float m = __uint_as_float((bits & 0x7fffffu) | 0x3f800000u);
    if (m > 1.41421353816986083984375f) {
        m = m * 0.5f;
        exponent += 1;
    }
    const float f = m - 1.0f;
    const float t = f / (2.0f + f);
    const float t2 = t * t;
    float p = 0.181818181818181818f;
    p = __builtin_fmaf(p, t2, 0.222222222222222222f);
    p = __builtin_fmaf(p, t2, 0.285714285714285714f);
    p = __builtin_fmaf(p, t2, 0.4f);
    p = __builtin_fmaf(p, t2, 0.666666666666666667f);
    p = __builtin_fmaf(p, t2, 2.0f);
    return __builtin_fmaf(static_cast<float>(exponent), 0.693147180559945309f, p * t);
}

// Marsaglia polar method; element i uses counters 32*i + attempt.
__device__ __forceinline__ float normal_at(uint64_t base, uint64_t index) {
    for (uint32_t attempt = 0; attempt < 32u; ++attempt) {
        const uint64_t r = stream_at(base, index * 32u + attempt);
        const int32_t ia = static_cast<int32_t>(2u * static_cast<uint32_t>(r >> 40)) - 16777215;
        const int32_t ib =
            static_cast<int32_t>(2u * static_cast<uint32_t>((r >> 16) & 0xffffffu)) - 16777215;
        const float a = static_cast<float>(ia) * 5.9604644775390625e-8f;
        const float b = static_cast<float>(ib) * 5.9604644775390625e-8f;
        const float s = a * a + b * b;
        if (s >= 1.0f) continue;
        float t = -2.0f * log_q(s);
        t = t / s;
        t = __builtin_sqrtf(t);
        return a * t;
    }
    return 0.0f;
}

__device__ __forceinline__ int uniform_at(uint64_t base, uint64_t index, int lo, int hi) {
    const uint64_t r = stream_at(base, index);
    const uint64_t span = static_cast<uint64_t>(static_cast<int64_t>(hi - lo + 1));
    return lo + static_cast<int>(((r >> 32) * span) >> 32);
}

}  // namespace q38m
