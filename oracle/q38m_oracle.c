/*
 * q38m CPU oracle -- TEST INFRASTRUCTURE ONLY (see q38m_oracle.h).
 *
 * Plain C restatement of the reference's grouped MoE step in the formats
 * the MI355X build computes in.  Every function cites the reference
 * lines it follows.  Build: oracle/Makefile (gcc -O3 -fopenmp
 * -ffp-contract=off -march=x86-64-v3).
 */
#include "q38m_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof(u));
    return u;
}

static inline float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof(f));
    return f;
}

/* ------------------------------------------------------------------ */
/* Scalar conversions                                                  */
/* ------------------------------------------------------------------ */

/* bf16 round-to-nearest-even: (bits + 0x7fff + lsb) >> 16, the rounding
 * of tools/q38_artifact_compiler.py:61-66 and src/mock_backend.cc:28-33;
 * NaN stays a quiet NaN. */
uint16_t q38o_f32_to_bf16(float value) {
    uint32_t bits = f2u(value);
    if ((bits & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)((bits >> 16) | 0x0040u);
    bits += 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)(bits >> 16);
}

float q38o_bf16_to_f32(uint16_t value) { return u2f((uint32_t)value << 16); }

/* IEEE binary16 -> binary32, exact (subnormals included). */
float q38o_f16_to_f32(uint16_t value) {
    const uint32_t sign = ((uint32_t)value & 0x8000u) << 16;
    const uint32_t exponent = ((uint32_t)value >> 10) & 0x1fu;
    const uint32_t mantissa = (uint32_t)value & 0x3ffu;
    if (exponent == 0u) {
        const float magnitude = (float)mantissa * 5.9604644775390625e-8f;
        return u2f(f2u(magnitude) | sign);
    }
    if (exponent == 31u) return u2f(sign | 0x7f800000u | (mantissa << 13));
    return u2f(sign | ((exponent + 112u) << 23) | (mantissa << 13));
}

/* binary32 -> binary16 round-to-nearest-even with subnormals and
 * overflow to infinity. */
uint16_t q38o_f32_to_f16(float value) {
    const uint32_t bits = f2u(value);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const uint32_t magnitude = bits & 0x7fffffffu;
    if (magnitude > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (magnitude >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (magnitude >= 0x38800000u) {
        const uint32_t rounded = magnitude + 0x0fffu + ((magnitude >> 13) & 1u);
        return (uint16_t)(sign | ((rounded >> 13) - (112u << 10)));
    }
    const uint32_t biased = magnitude >> 23;
    if (biased == 0u) return (uint16_t)sign;
    const uint32_t shift = 126u - biased;
    if (shift > 24u) return (uint16_t)sign;
    const uint32_t mantissa = (magnitude & 0x7fffffu) | 0x800000u;
    uint32_t result = mantissa >> shift;
    const uint32_t remainder = mantissa & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (remainder > half || (remainder == half && (result & 1u))) ++result;
    return (uint16_t)(sign | result);
}

/* The contract's exp.  Cody & Waite (1980) argument reduction
 * x = n*ln2 + r with a two-part ln2 (high part with 15 significant bits
 * so n*ln2_hi is exact), then the degree-7 Taylor polynomial of e^r in
 * Horner form (coefficients 1/k!), then exact scaling by 2^n.  Results
 * below the smallest normal float are flushed to 0 (x < -87.3), so CPU
 * and GPU never depend on subnormal handling.  The reference uses expf
 * at q38_moe_prefill.cu:454, :608 and q38_kernels.cu:461; this build
 * pins one shared implementation instead so CPU and GPU agree bitwise. */
float q38o_expf(float x) {
    if (x != x) return x + x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -87.3f) return 0.0f;
    const float n = rintf(x * 1.44269502162933349609375f);
    float r = fmaf(n, -0.693145751953125f, x);
    r = fmaf(n, -1.42860682030941723212e-6f, r);
    float p = 1.98412698412698412698e-4f;
    p = fmaf(p, r, 1.38888888888888888889e-3f);
    p = fmaf(p, r, 8.33333333333333333333e-3f);
    p = fmaf(p, r, 4.16666666666666666667e-2f);
    p = fmaf(p, r, 1.66666666666666666667e-1f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int exponent = (int)n;
    if (exponent > 127) return (p * 2.0f) * u2f(254u << 23); /* * 2^127 */
    return p * u2f((uint32_t)(exponent + 127) << 23);
}

void q38o_expf_array(const float* x, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = q38o_expf(x[i]);
}

void q38o_f32_to_bf16_array(const float* x, size_t n, uint16_t* out) {
    for (size_t i = 0; i < n; ++i) out[i] = q38o_f32_to_bf16(x[i]);
}

void q38o_f32_to_f16_array(const float* x, size_t n, uint16_t* out) {
    for (size_t i = 0; i < n; ++i) out[i] = q38o_f32_to_f16(x[i]);
}

void q38o_f16_to_f32_array(const uint16_t* x, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = q38o_f16_to_f32(x[i]);
}

/* Natural log for positive normal floats (synthetic data only):
 * x = m*2^e with m in [sqrt(1/2), sqrt(2)), log m = 2 atanh(f/(2+f)),
 * f = m-1, odd series to t^11. */
float q38o_logf(float x) {
    const uint32_t bits = f2u(x);
    int exponent = (int)(bits >> 23) - 127;
    float m = u2f((bits & 0x7fffffu) | 0x3f800000u);
    if (m > 1.41421353816986083984375f) {
        m = m * 0.5f;
        exponent += 1;
    }
    const float f = m - 1.0f;
    const float t = f / (2.0f + f);
    const float t2 = t * t;
    float p = 0.181818181818181818f;
    p = fmaf(p, t2, 0.222222222222222222f);
    p = fmaf(p, t2, 0.285714285714285714f);
    p = fmaf(p, t2, 0.4f);
    p = fmaf(p, t2, 0.666666666666666667f);
    p = fmaf(p, t2, 2.0f);
    return fmaf((float)exponent, 0.693147180559945309f, p * t);
}

/* ------------------------------------------------------------------ */
/* Counter-based synthetic data: SplitMix64 (Steele, Lea, Flood 2014)  */
/* ------------------------------------------------------------------ */

#define Q38O_GAMMA 0x9e3779b97f4a7c15ull

static inline uint64_t mix64(uint64_t z) {
    z ^= z >> 30;
    z *= 0xbf58476d1ce4e5b9ull;
    z ^= z >> 27;
    z *= 0x94d049bb133111ebull;
    z ^= z >> 31;
    return z;
}

static inline uint64_t stream_base(uint64_t seed, uint64_t tag) {
    return mix64(seed + Q38O_GAMMA * (tag + 1u));
}

static inline uint64_t stream_at(uint64_t base, uint64_t counter) {
    return mix64(base + Q38O_GAMMA * (counter + 1u));
}

uint64_t q38o_rand64(uint64_t seed, uint64_t tag, uint64_t counter) {
    return stream_at(stream_base(seed, tag), counter);
}

/* Marsaglia polar method; element i uses counters 32*i + attempt. */
static float normal_at(uint64_t base, uint64_t index) {
    for (uint32_t attempt = 0; attempt < 32u; ++attempt) {
        const uint64_t r = stream_at(base, index * 32u + attempt);
        const int32_t ia = (int32_t)(2u * (uint32_t)(r >> 40)) - 16777215;
        const int32_t ib =
            (int32_t)(2u * (uint32_t)((r >> 16) & 0xffffffu)) - 16777215;
        const float a = (float)ia * 5.9604644775390625e-8f;
        const float b = (float)ib * 5.9604644775390625e-8f;
        const float s = a * a + b * b;
        if (s >= 1.0f) continue;
        float t = -2.0f * q38o_logf(s);
        t = t / s;
        t = sqrtf(t);
        return a * t;
    }
    return 0.0f;
}

static inline int uniform_at(uint64_t base, uint64_t index, int lo, int hi) {
    const uint64_t r = stream_at(base, index);
    const uint64_t span = (uint64_t)(int64_t)(hi - lo + 1);
    return lo + (int)(((r >> 32) * span) >> 32);
}

void q38o_synth_normal_f32(uint64_t seed, uint64_t tag, float sigma,
                           int absolute, size_t n, float* out) {
    const uint64_t base = stream_base(seed, tag);
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) {
        const float v = normal_at(base, i) * sigma;
        out[i] = absolute ? fabsf(v) : v;
    }
}

void q38o_synth_normal_bf16(uint64_t seed, uint64_t tag, float sigma,
                            size_t n, uint16_t* out) {
    const uint64_t base = stream_base(seed, tag);
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i)
        out[i] = q38o_f32_to_bf16(normal_at(base, i) * sigma);
}

void q38o_synth_abs_normal_f16(uint64_t seed, uint64_t tag, float sigma,
                               size_t n, uint16_t* out) {
    const uint64_t base = stream_base(seed, tag);
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i)
        out[i] = q38o_f32_to_f16(fabsf(normal_at(base, i) * sigma));
}

void q38o_synth_logits(uint64_t seed, uint64_t tag, float sigma,
                       const float* bias, uint32_t tokens, uint32_t experts,
                       float* out) {
    const uint64_t base = stream_base(seed, tag);
    const size_t n = (size_t)tokens * experts;
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) {
        float v = normal_at(base, i) * sigma;
        if (bias) v = v + bias[i % experts];
        out[i] = v;
    }
}

void q38o_synth_uniform_w4(uint64_t seed, uint64_t tag, int lo, int hi,
                           size_t n, uint8_t* out) {
    const uint64_t base = stream_base(seed, tag);
#pragma omp parallel for schedule(static)
    for (size_t j = 0; j < n / 2; ++j) {
        const int low = uniform_at(base, 2 * j, lo, hi);
        const int high = uniform_at(base, 2 * j + 1, lo, hi);
        out[j] = (uint8_t)(((unsigned)low & 0xfu) | (((unsigned)high & 0xfu) << 4));
    }
}

void q38o_synth_uniform_i8(uint64_t seed, uint64_t tag, int lo, int hi,
                           size_t n, int8_t* out) {
    const uint64_t base = stream_base(seed, tag);
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) out[i] = (int8_t)uniform_at(base, i, lo, hi);
}

/* ------------------------------------------------------------------ */
/* Routing                                                             */
/* ------------------------------------------------------------------ */

/* Top-k by (logit desc, id asc) -- the order of the bitonic sort at
 * q38_kernels.cu:431-458 -- then numerators exp(l_r - l_0) and a rank-
 * order fp32 denominator (q38_kernels.cu:461-479).  normalize == 0 uses
 * the all-expert denominator in expert order (q38_kernels.cu:375-400). */
int q38o_topk(const float* logits, uint32_t tokens, uint32_t experts,
              uint32_t top_k, int normalize, int32_t* ids, float* weights) {
    if (!logits || !ids || !weights || tokens == 0 || experts == 0 ||
        experts > 4096u || top_k == 0 || top_k > experts || top_k > 32u)
        return 1;
#pragma omp parallel for schedule(static)
    for (uint32_t t = 0; t < tokens; ++t) {
        const float* row = logits + (size_t)t * experts;
        unsigned char chosen[4096];
        memset(chosen, 0, experts);
        float values[32];
        int32_t selected[32];
        for (uint32_t rank = 0; rank < top_k; ++rank) {
            int32_t best = -1;
            for (uint32_t e = 0; e < experts; ++e) {
                if (chosen[e]) continue;
                if (best < 0 || row[e] > row[best]) best = (int32_t)e;
            }
            chosen[best] = 1;
            selected[rank] = best;
            values[rank] = row[best];
        }
        float numerators[32];
        for (uint32_t rank = 0; rank < top_k; ++rank)
            numerators[rank] = q38o_expf(values[rank] - values[0]);
        float denominator = 0.0f;
        if (normalize) {
            for (uint32_t rank = 0; rank < top_k; ++rank)
                denominator += numerators[rank];
        } else {
            for (uint32_t e = 0; e < experts; ++e)
                denominator += q38o_expf(row[e] - values[0]);
        }
        for (uint32_t rank = 0; rank < top_k; ++rank) {
            ids[(size_t)t * top_k + rank] = selected[rank];
            weights[(size_t)t * top_k + rank] = numerators[rank] / denominator;
        }
    }
    return 0;
}

uint32_t q38o_routes(uint32_t tokens) { return tokens * Q38O_TOPK; }

/* include/q38/cuda_moe_prefill.h:77-83 */
uint32_t q38o_max_tasks(uint32_t tokens) {
    const uint32_t routes = q38o_routes(tokens);
    const uint32_t initially = routes < Q38O_EXPERTS ? routes : Q38O_EXPERTS;
    return initially + (routes - initially) / Q38O_MMQ_M;
}

/* include/q38/cuda_moe_prefill.h:85-93 */
size_t q38o_plan_bytes(uint32_t tokens) {
    const size_t routes = q38o_routes(tokens);
    return 64u + Q38O_EXPERTS * 2u + 2u * (Q38O_EXPERTS + 1u) * 4u +
           2u * routes * 4u + (size_t)q38o_max_tasks(tokens) * 8u;
}

static inline uint64_t fnv_word(uint64_t hash, uint64_t value) {
    hash ^= value;
    return hash * 1099511628211ull;
}

static void put_u32(uint8_t* p, uint32_t v) { memcpy(p, &v, 4); }
static void put_u64(uint8_t* p, uint64_t v) { memcpy(p, &v, 8); }

/* Stable expert-major counting sort with M=16 tasks, status and FNV-1a
 * hashes: cuda/q38_moe_prefill.cu:155-290.  Invalid ids keep the
 * reference's identity initialisation (:178-192): inverse[a] = a, and
 * packed positions beyond the valid total keep packed[p] = p. */
int q38o_build_plan(const int32_t* expert_ids, uint32_t tokens,
                    int with_hashes, uint8_t* plan) {
    if (!expert_ids || !plan || tokens == 0 || tokens > Q38O_SLAB_MAX_TOKENS)
        return 1;
    const uint32_t routes = q38o_routes(tokens);
    const uint32_t max_tasks = q38o_max_tasks(tokens);
    uint8_t* header = plan;
    uint8_t* counts_p = plan + 64;
    uint8_t* offsets_p = counts_p + Q38O_EXPERTS * 2u;
    uint8_t* task_offsets_p = offsets_p + (Q38O_EXPERTS + 1u) * 4u;
    uint8_t* packed_p = task_offsets_p + (Q38O_EXPERTS + 1u) * 4u;
    uint8_t* inverse_p = packed_p + (size_t)routes * 4u;
    uint8_t* tasks_p = inverse_p + (size_t)routes * 4u;

    uint16_t route_experts[Q38O_SLAB_MAX_TOKENS * Q38O_TOPK];
    uint32_t counts[Q38O_EXPERTS];
    uint32_t offsets[Q38O_EXPERTS + 1];
    uint32_t task_offsets[Q38O_EXPERTS + 1];
    uint32_t status = 0;
    memset(counts, 0, sizeof(counts));
    for (uint32_t a = 0; a < routes; ++a) {
        const int32_t id = expert_ids[a];
        const int valid = id >= 0 && id < (int32_t)Q38O_EXPERTS;
        route_experts[a] = valid ? (uint16_t)id : (uint16_t)0xffffu;
        if (valid)
            ++counts[id];
        else
            status = 1u;
    }
    uint32_t assignment_offset = 0, task_offset = 0, active = 0;
    for (uint32_t e = 0; e < Q38O_EXPERTS; ++e) {
        offsets[e] = assignment_offset;
        task_offsets[e] = task_offset;
        assignment_offset += counts[e];
        task_offset += (counts[e] + Q38O_MMQ_M - 1u) / Q38O_MMQ_M;
        active += counts[e] != 0u ? 1u : 0u;
    }
    offsets[Q38O_EXPERTS] = assignment_offset;
    task_offsets[Q38O_EXPERTS] = task_offset;
    if (status == 0u && (assignment_offset != routes || task_offset > max_tasks))
        status = 2u;

    uint32_t running[Q38O_EXPERTS];
    memset(running, 0, sizeof(running));
    uint32_t* packed = (uint32_t*)malloc((size_t)routes * 4u);
    uint32_t* inverse = (uint32_t*)malloc((size_t)routes * 4u);
    for (uint32_t p = 0; p < routes; ++p) packed[p] = p;
    for (uint32_t a = 0; a < routes; ++a) {
        const uint16_t e = route_experts[a];
        if (e == 0xffffu) {
            inverse[a] = a;
            continue;
        }
        const uint32_t position = offsets[e] + running[e]++;
        packed[position] = a;
        inverse[a] = position;
    }

    memset(tasks_p, 0, (size_t)max_tasks * 8u);
    for (uint32_t e = 0; e < Q38O_EXPERTS; ++e) {
        const uint32_t count = counts[e];
        const uint32_t n_tasks = (count + Q38O_MMQ_M - 1u) / Q38O_MMQ_M;
        for (uint32_t tile = 0; tile < n_tasks; ++tile) {
            const uint32_t remaining = count - tile * Q38O_MMQ_M;
            uint8_t* task = tasks_p + (size_t)(task_offsets[e] + tile) * 8u;
            const uint16_t expert = (uint16_t)e;
            put_u32(task, offsets[e] + tile * Q38O_MMQ_M);
            memcpy(task + 4, &expert, 2);
            task[6] = (uint8_t)(remaining < Q38O_MMQ_M ? remaining : Q38O_MMQ_M);
            task[7] = 0;
        }
    }

    for (uint32_t e = 0; e < Q38O_EXPERTS; ++e) {
        const uint16_t c = (uint16_t)counts[e];
        memcpy(counts_p + e * 2u, &c, 2);
    }
    memcpy(offsets_p, offsets, sizeof(offsets));
    memcpy(task_offsets_p, task_offsets, sizeof(task_offsets));
    memcpy(packed_p, packed, (size_t)routes * 4u);
    memcpy(inverse_p, inverse, (size_t)routes * 4u);

    uint64_t route_hash = 0, plan_hash = 0;
    if (with_hashes) {
        route_hash = 1469598103934665603ull;
        for (uint32_t a = 0; a < routes; ++a)
            route_hash = fnv_word(route_hash, route_experts[a]);
        plan_hash = 1469598103934665603ull;
        for (uint32_t e = 0; e <= Q38O_EXPERTS; ++e) {
            plan_hash = fnv_word(plan_hash, offsets[e]);
            plan_hash = fnv_word(plan_hash, task_offsets[e]);
        }
        for (uint32_t p = 0; p < routes; ++p)
            plan_hash = fnv_word(plan_hash, packed[p]);
        for (uint32_t t = 0; t < task_offset; ++t) {
            const uint8_t* task = tasks_p + (size_t)t * 8u;
            uint32_t begin;
            uint16_t expert;
            memcpy(&begin, task, 4);
            memcpy(&expert, task + 4, 2);
            const uint64_t low = (uint64_t)begin | ((uint64_t)expert << 32);
            const uint64_t high = (uint64_t)task[6] | ((uint64_t)task[7] << 8);
            plan_hash = fnv_word(plan_hash, low);
            plan_hash = fnv_word(plan_hash, high);
        }
    }
    free(packed);
    free(inverse);

    put_u32(header + 0, Q38O_PLAN_MAGIC);
    put_u32(header + 4, Q38O_PLAN_VERSION);
    put_u32(header + 8, tokens);
    put_u32(header + 12, routes);
    put_u32(header + 16, active);
    put_u32(header + 20, task_offset);
    put_u32(header + 24, status);
    put_u32(header + 28, 0u);
    put_u64(header + 32, route_hash);
    put_u64(header + 40, plan_hash);
    put_u64(header + 48, 0u);
    put_u64(header + 56, 0u);
    return 0;
}

/* ------------------------------------------------------------------ */
/* Quantisation (a6): s = absmax/127, 0 -> 1, q = clip(rint(x/s))      */
/* convention of tools/q38_artifact_compiler.py:214-222               */
/* ------------------------------------------------------------------ */

void q38o_quantize_rows(const uint16_t* x, uint32_t rows, uint32_t width,
                        int8_t* q, float* scales) {
#pragma omp parallel for schedule(static)
    for (uint32_t r = 0; r < rows; ++r) {
        const uint16_t* row = x + (size_t)r * width;
        float amax = 0.0f;
        for (uint32_t k = 0; k < width; ++k) {
            const float a = fabsf(q38o_bf16_to_f32(row[k]));
            if (a > amax) amax = a;
        }
        float s = amax / 127.0f;
        if (s == 0.0f) s = 1.0f;
        for (uint32_t k = 0; k < width; ++k) {
            /* fmaxf / fminf return the other operand for a NaN quotient
             * (an infinite element of a row whose absmax is infinite:
             * inf / inf), so it quantises to -127, defined, as the device
             * clamp does; a plain cast of NaN would be undefined */
            const float v = fminf(fmaxf(rintf(q38o_bf16_to_f32(row[k]) / s), -127.0f), 127.0f);
            q[(size_t)r * width + k] = (int8_t)v;
        }
        scales[r] = s;
    }
}

/* ------------------------------------------------------------------ */
/* Weight quantiser: tools/q38_artifact_compiler.py:193-253            */
/* ------------------------------------------------------------------ */

int q38o_quantize_weights(const uint16_t* src_bf16, uint64_t rows, uint32_t cols,
                          int bits, uint32_t group, uint8_t* data, uint16_t* scales,
                          int scale_bf16) {
    const uint32_t g = group ? group : cols;
    if (!src_bf16 || !data || !scales || rows == 0 || cols == 0 || (bits != 4 && bits != 8) ||
        cols % g != 0 || (bits == 4 && (g % 2 != 0 || cols % 2 != 0)))
        return 1;
    const float qmax = bits == 4 ? 7.0f : 127.0f;
    const uint32_t groups = cols / g;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; ++r) {
        const uint16_t* row = src_bf16 + (size_t)r * cols;
        for (uint32_t gi = 0; gi < groups; ++gi) {
            const uint16_t* w = row + (size_t)gi * g;
            float amax = 0.0f;
            for (uint32_t k = 0; k < g; ++k) {
                const float a = fabsf(q38o_bf16_to_f32(w[k]));
                if (a > amax) amax = a;
            }
            float s = amax / qmax;
            if (s == 0.0f) s = 1.0f;
            scales[(size_t)r * groups + gi] = scale_bf16 ? q38o_f32_to_bf16(s) : q38o_f32_to_f16(s);
            for (uint32_t k = 0; k < g; ++k) {
                /* NaN quotients clamp to -qmax (fmaxf returns the other
                 * operand), as the device quantiser does */
                const float v = fminf(fmaxf(rintf(q38o_bf16_to_f32(w[k]) / s), -qmax), qmax);
                const int q = (int)v;
                const size_t col = (size_t)gi * g + k;
                if (bits == 8) {
                    data[(size_t)r * cols + col] = (uint8_t)(int8_t)q;
                } else {
                    uint8_t* byte = data + (size_t)r * (cols / 2) + col / 2;
                    const uint8_t nib = (uint8_t)(q & 0xf);
                    *byte = (col & 1) ? (uint8_t)((*byte & 0x0f) | (nib << 4))
                                      : (uint8_t)((*byte & 0xf0) | nib);
                }
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Weights and the scaled row value                                    */
/* ------------------------------------------------------------------ */

/* Two's-complement nibble, even column in the low nibble
 * (cuda/q38_moe_prefill.cu:107-111, cuda/q38_moe.cu:112-114). */
static void unpack_row(const q38o_weights* w, uint32_t e, uint32_t row,
                       int8_t* out) {
    const size_t base = ((size_t)e * w->rows + row) * w->cols;
    if (w->bits == 8u) {
        memcpy(out, w->data + base, w->cols);
        return;
    }
    const uint8_t* bytes = w->data + base / 2u;
    for (uint32_t k = 0; k < w->cols; k += 2) {
        const uint8_t b = bytes[k / 2u];
        const int low = b & 0x0f;
        const int high = b >> 4;
        out[k] = (int8_t)(low >= 8 ? low - 16 : low);
        out[k + 1] = (int8_t)(high >= 8 ? high - 16 : high);
    }
}

static float scale_word(const q38o_weights* w, uint16_t word) {
    return w->scale_bf16 ? q38o_bf16_to_f32(word) : q38o_f16_to_f32(word);
}

static void row_scales(const q38o_weights* w, uint32_t e, uint32_t row,
                       float* out) {
    if (w->group == 0u) {
        out[0] = scale_word(w, w->scales[(size_t)e * w->rows + row]);
        return;
    }
    const uint32_t groups = w->cols / w->group;
    const uint16_t* s = w->scales + ((size_t)e * w->rows + row) * groups;
    for (uint32_t g = 0; g < groups; ++g) out[g] = scale_word(w, s[g]);
}

static float chain_row(const int8_t* wrow, const float* scales, uint32_t cols,
                       uint32_t group, const int8_t* x) {
    if (group == 0u) {
        int32_t acc = 0;
        for (uint32_t k = 0; k < cols; ++k)
            acc += (int32_t)x[k] * (int32_t)wrow[k];
        return (float)acc * scales[0];
    }
    float y = 0.0f;
    for (uint32_t g = 0; g < cols / group; ++g) {
        const int8_t* xg = x + (size_t)g * group;
        const int8_t* wg = wrow + (size_t)g * group;
        int32_t acc = 0;
        for (uint32_t k = 0; k < group; ++k)
            acc += (int32_t)xg[k] * (int32_t)wg[k];
        y = fmaf((float)acc, scales[g], y);
    }
    return y;
}

float q38o_row_value(const q38o_weights* w, uint32_t expert, uint32_t row,
                     const int8_t* x) {
    int8_t* unpacked = (int8_t*)malloc(w->cols);
    float* scales = (float*)malloc(sizeof(float) * (w->group ? w->cols / w->group : 1u));
    unpack_row(w, expert, row, unpacked);
    row_scales(w, expert, row, scales);
    const float y = chain_row(unpacked, scales, w->cols, w->group, x);
    free(scales);
    free(unpacked);
    return y;
}

void q38o_row_accumulators(const q38o_weights* w, uint32_t expert,
                           uint32_t row, const int8_t* x, int32_t* out) {
    int8_t* unpacked = (int8_t*)malloc(w->cols);
    unpack_row(w, expert, row, unpacked);
    const uint32_t group = w->group ? w->group : w->cols;
    for (uint32_t g = 0; g < w->cols / group; ++g) {
        int32_t acc = 0;
        for (uint32_t k = 0; k < group; ++k)
            acc += (int32_t)x[g * group + k] * (int32_t)unpacked[g * group + k];
        out[g] = acc;
    }
    free(unpacked);
}

/* ------------------------------------------------------------------ */
/* Grouped stages                                                      */
/* ------------------------------------------------------------------ */

typedef struct plan_view {
    uint32_t tokens, routes, task_count, status;
    const uint32_t* packed;
    const uint32_t* inverse;
    const uint8_t* tasks;
} plan_view;

static plan_view view_plan(const uint8_t* plan) {
    plan_view v;
    memcpy(&v.tokens, plan + 8, 4);
    memcpy(&v.routes, plan + 12, 4);
    memcpy(&v.task_count, plan + 20, 4);
    memcpy(&v.status, plan + 24, 4);
    const uint8_t* packed = plan + 64 + Q38O_EXPERTS * 2u + 2u * (Q38O_EXPERTS + 1u) * 4u;
    v.packed = (const uint32_t*)packed;
    v.inverse = (const uint32_t*)(packed + (size_t)v.routes * 4u);
    v.tasks = packed + (size_t)v.routes * 8u;
    return v;
}

static inline void task_fields(const uint8_t* task, uint32_t* begin,
                               uint32_t* expert, uint32_t* rows) {
    uint16_t e;
    memcpy(begin, task, 4);
    memcpy(&e, task + 4, 2);
    *expert = e;
    *rows = task[6];
}

static inline float bf16_round(float v) {
    return q38o_bf16_to_f32(q38o_f32_to_bf16(v));
}

/* SwiGLU and router-weight fold, the rounding sequence of
 * cuda/q38_moe_prefill.cu:449-461: g=bf16(y_g), u=bf16(y_u),
 * h=bf16(g/(1+exp(-g))*u), m=bf16(h*w).  A NaN m is written as the quiet
 * NaN 0x7fc0 (its sign and payload would otherwise follow the instruction
 * set; the GPU's epilogues write the same word). */
static inline uint16_t swiglu_fold(float y_gate, float y_up, float weight) {
    const float g = bf16_round(y_gate);
    const float u = bf16_round(y_up);
    const float e = q38o_expf(-g);
    const float den = 1.0f + e;
    const float silu = g / den;
    const float h = bf16_round(silu * u);
    const uint16_t m = q38o_f32_to_bf16(h * weight);
    return (m & 0x7fffu) > 0x7f80u ? (uint16_t)0x7fc0u : m;
}

/* Grouped gate/up over the plan's M=16 tasks (q38_moe_prefill.cu:308-464)
 * in int8 x W4/W8: y = chain(row) * s_t, then swiglu_fold. */
void q38o_gate_up(const q38o_weights* gate_up, uint32_t hidden,
                  uint32_t inter, const int8_t* xq, const float* xs,
                  const uint8_t* plan, const float* route_weights,
                  uint16_t* weighted_mid) {
    const plan_view v = view_plan(plan);
    const uint32_t groups = gate_up->group ? hidden / gate_up->group : 1u;
#pragma omp parallel
    {
        int8_t* wg = (int8_t*)malloc(hidden);
        int8_t* wu = (int8_t*)malloc(hidden);
        float* sg = (float*)malloc(sizeof(float) * groups);
        float* su = (float*)malloc(sizeof(float) * groups);
#pragma omp for schedule(dynamic, 1)
        for (uint32_t t = 0; t < v.task_count; ++t) {
            uint32_t begin, expert, rows;
            task_fields(v.tasks + (size_t)t * 8u, &begin, &expert, &rows);
            for (uint32_t j = 0; j < inter; ++j) {
                unpack_row(gate_up, expert, j, wg);
                unpack_row(gate_up, expert, inter + j, wu);
                row_scales(gate_up, expert, j, sg);
                row_scales(gate_up, expert, inter + j, su);
                for (uint32_t m = 0; m < rows; ++m) {
                    const uint32_t p = begin + m;
                    const uint32_t a = v.packed[p];
                    const uint32_t token = a / Q38O_TOPK;
                    const int8_t* x = xq + (size_t)token * hidden;
                    float y_gate = chain_row(wg, sg, hidden, gate_up->group, x);
                    float y_up = chain_row(wu, su, hidden, gate_up->group, x);
                    y_gate = y_gate * xs[token];
                    y_up = y_up * xs[token];
                    weighted_mid[(size_t)p * inter + j] =
                        swiglu_fold(y_gate, y_up, route_weights[a]);
                }
            }
        }
        free(su);
        free(sg);
        free(wu);
        free(wg);
    }
}

/* Grouped down (q38_moe_prefill.cu:466-599): one fp32 row per packed
 * assignment, o = chain(row) * s_m. */
void q38o_down(const q38o_weights* down, uint32_t hidden, uint32_t inter,
               const int8_t* mid_q, const float* mid_scales,
               const uint8_t* plan, float* route_output) {
    const plan_view v = view_plan(plan);
    const uint32_t groups = down->group ? inter / down->group : 1u;
#pragma omp parallel
    {
        int8_t* w = (int8_t*)malloc(inter);
        float* s = (float*)malloc(sizeof(float) * groups);
#pragma omp for schedule(dynamic, 1)
        for (uint32_t t = 0; t < v.task_count; ++t) {
            uint32_t begin, expert, rows;
            task_fields(v.tasks + (size_t)t * 8u, &begin, &expert, &rows);
            for (uint32_t c = 0; c < hidden; ++c) {
                unpack_row(down, expert, c, w);
                row_scales(down, expert, c, s);
                for (uint32_t m = 0; m < rows; ++m) {
                    const uint32_t p = begin + m;
                    float y = chain_row(w, s, inter, down->group,
                                        mid_q + (size_t)p * inter);
                    y = y * mid_scales[p];
                    route_output[(size_t)p * hidden + c] = y;
                }
            }
        }
        free(s);
        free(w);
    }
}

/* Fixed rank-order reduce from 0.0f plus the optional gated shared term
 * (cuda/q38_moe_prefill.cu:601-631).  The reference writes
 * `routed + shared * multiplier`, which nvcc's default -fmad=true contracts
 * into one fused multiply-add; the restatement uses that fma. */
void q38o_combine(const float* route_output, const uint32_t* inverse,
                  const uint16_t* shared_output, const uint16_t* shared_gate,
                  uint32_t tokens, uint32_t hidden, uint16_t* output) {
#pragma omp parallel for schedule(static)
    for (uint32_t t = 0; t < tokens; ++t) {
        float multiplier = 0.0f;
        const int shared = shared_output != NULL && shared_gate != NULL;
        if (shared) {
            const float g = q38o_bf16_to_f32(shared_gate[t]);
            multiplier = 1.0f / (1.0f + q38o_expf(-g));
        }
        for (uint32_t c = 0; c < hidden; ++c) {
            float routed = 0.0f;
            for (uint32_t r = 0; r < Q38O_TOPK; ++r)
                routed += route_output[(size_t)inverse[t * Q38O_TOPK + r] * hidden + c];
            if (shared)
                routed = fmaf(q38o_bf16_to_f32(shared_output[(size_t)t * hidden + c]),
                              multiplier, routed);
            output[(size_t)t * hidden + c] = q38o_f32_to_bf16(routed);
        }
    }
}

/* Decode combine of bf16 routed rows (cuda/q38_moe.cu:337-350):
 * out = bf16(routed + shared * (1 / (1 + exp(-gate[t])))), the sum
 * contracted into one fma as nvcc builds the reference expression. */
void q38o_combine_shared(const uint16_t* routed, const uint16_t* shared_output,
                         const uint16_t* shared_gate, uint32_t tokens, uint32_t hidden,
                         uint16_t* output) {
    for (uint32_t t = 0; t < tokens; ++t) {
        const float g = q38o_bf16_to_f32(shared_gate[t]);
        const float sigmoid = 1.0f / (1.0f + q38o_expf(-g));
        for (uint32_t c = 0; c < hidden; ++c) {
            const size_t i = (size_t)t * hidden + c;
            output[i] = q38o_f32_to_bf16(
                fmaf(q38o_bf16_to_f32(shared_output[i]), sigmoid, q38o_bf16_to_f32(routed[i])));
        }
    }
}

/* ------------------------------------------------------------------ */
/* Whole step                                                          */
/* ------------------------------------------------------------------ */

static void* take(void* given, size_t bytes, void** owned) {
    if (given) return given;
    *owned = malloc(bytes ? bytes : 1u);
    return *owned;
}

int q38o_moe_prefill(q38o_moe_io* io) {
    if (!io || !io->hidden_states || !io->ids || !io->weights || !io->gate_up ||
        !io->down || !io->output || io->tokens == 0 ||
        io->tokens > Q38O_SLAB_MAX_TOKENS)
        return 1;
    const uint32_t T = io->tokens, H = io->hidden, I = io->inter;
    const uint32_t R = q38o_routes(T);
    if (io->logits &&
        q38o_topk(io->logits, T, Q38O_EXPERTS, Q38O_TOPK, 1, io->ids, io->weights))
        return 1;
    void *o1 = NULL, *o2 = NULL, *o3 = NULL, *o4 = NULL, *o5 = NULL, *o6 = NULL, *o7 = NULL;
    uint8_t* plan = (uint8_t*)take(io->plan, q38o_plan_bytes(T), &o1);
    int8_t* xq = (int8_t*)take(io->xq, (size_t)T * H, &o2);
    float* xs = (float*)take(io->xs, (size_t)T * 4u, &o3);
    uint16_t* mid = (uint16_t*)take(io->weighted_mid, (size_t)R * I * 2u, &o4);
    int8_t* mq = (int8_t*)take(io->mid_q, (size_t)R * I, &o5);
    float* ms = (float*)take(io->mid_s, (size_t)R * 4u, &o6);
    float* ro = (float*)take(io->route_output, (size_t)R * H * 4u, &o7);
    int rc = q38o_build_plan(io->ids, T, 0, plan);
    uint32_t status = 1;
    if (rc == 0) memcpy(&status, plan + 24, 4);
    if (rc == 0 && status == 0) {
        q38o_quantize_rows(io->hidden_states, T, H, xq, xs);
        q38o_gate_up(io->gate_up, H, I, xq, xs, plan, io->weights, mid);
        q38o_quantize_rows(mid, R, I, mq, ms);
        q38o_down(io->down, H, I, mq, ms, plan, ro);
        const plan_view v = view_plan(plan);
        q38o_combine(ro, v.inverse, io->shared_output, io->shared_gate, T, H,
                     io->output);
    } else {
        rc = 2;
    }
    free(o7); free(o6); free(o5); free(o4); free(o3); free(o2); free(o1);
    return rc;
}

int q38o_moe_per_token(q38o_moe_io* io) {
    if (!io || !io->hidden_states || !io->ids || !io->weights || !io->gate_up ||
        !io->down || !io->output || io->tokens == 0)
        return 1;
    const uint32_t T = io->tokens, H = io->hidden, I = io->inter;
    if (io->logits &&
        q38o_topk(io->logits, T, Q38O_EXPERTS, Q38O_TOPK, 1, io->ids, io->weights))
        return 1;
    for (size_t a = 0; a < (size_t)T * Q38O_TOPK; ++a)
        if (io->ids[a] < 0 || io->ids[a] >= (int32_t)Q38O_EXPERTS) return 2;
    const uint32_t gu_groups = io->gate_up->group ? H / io->gate_up->group : 1u;
    const uint32_t dn_groups = io->down->group ? I / io->down->group : 1u;
#pragma omp parallel
    {
        int8_t* xq = (int8_t*)malloc(H);
        int8_t* wg = (int8_t*)malloc(H);
        int8_t* wu = (int8_t*)malloc(H);
        int8_t* wd = (int8_t*)malloc(I);
        float* sg = (float*)malloc(sizeof(float) * gu_groups);
        float* su = (float*)malloc(sizeof(float) * gu_groups);
        float* sd = (float*)malloc(sizeof(float) * dn_groups);
        uint16_t* mid = (uint16_t*)malloc((size_t)I * 2u);
        int8_t* mq = (int8_t*)malloc(I);
        float* routes = (float*)malloc(sizeof(float) * Q38O_TOPK * H);
#pragma omp for schedule(dynamic, 1)
        for (uint32_t t = 0; t < T; ++t) {
            float xs;
            q38o_quantize_rows(io->hidden_states + (size_t)t * H, 1, H, xq, &xs);
            for (uint32_t r = 0; r < Q38O_TOPK; ++r) {
                const uint32_t a = t * Q38O_TOPK + r;
                const uint32_t e = (uint32_t)io->ids[a];
                for (uint32_t j = 0; j < I; ++j) {
                    unpack_row(io->gate_up, e, j, wg);
                    unpack_row(io->gate_up, e, I + j, wu);
                    row_scales(io->gate_up, e, j, sg);
                    row_scales(io->gate_up, e, I + j, su);
                    float y_gate = chain_row(wg, sg, H, io->gate_up->group, xq);
                    float y_up = chain_row(wu, su, H, io->gate_up->group, xq);
                    y_gate = y_gate * xs;
                    y_up = y_up * xs;
                    mid[j] = swiglu_fold(y_gate, y_up, io->weights[a]);
                }
                float ms;
                q38o_quantize_rows(mid, 1, I, mq, &ms);
                for (uint32_t c = 0; c < H; ++c) {
                    unpack_row(io->down, e, c, wd);
                    row_scales(io->down, e, c, sd);
                    float y = chain_row(wd, sd, I, io->down->group, mq);
                    routes[(size_t)r * H + c] = y * ms;
                }
            }
            float multiplier = 0.0f;
            const int shared = io->shared_output != NULL && io->shared_gate != NULL;
            if (shared) {
                const float g = q38o_bf16_to_f32(io->shared_gate[t]);
                multiplier = 1.0f / (1.0f + q38o_expf(-g));
            }
            for (uint32_t c = 0; c < H; ++c) {
                float routed = 0.0f;
                for (uint32_t r = 0; r < Q38O_TOPK; ++r) routed += routes[(size_t)r * H + c];
                if (shared)
                    routed = fmaf(q38o_bf16_to_f32(io->shared_output[(size_t)t * H + c]),
                                  multiplier, routed);
                io->output[(size_t)t * H + c] = q38o_f32_to_bf16(routed);
            }
        }
        free(routes); free(mq); free(mid); free(sd); free(su); free(sg);
        free(wd); free(wu); free(wg); free(xq);
    }
    return 0;
}

int q38o_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void q38o_set_num_threads(int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
}
