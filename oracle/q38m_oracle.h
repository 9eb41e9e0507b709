/*
 * q38m CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference runtime's grouped MoE
 * step, written in the number formats the MI355X build computes in
 * (int8 per-token activations, W4 group-32 / W8 per-channel weights with
 * fp16 scales, int32 accumulators, fp32 epilogue, bf16 outputs).  It is
 * the checker for the HIP product library and the timed CPU baseline in
 * bench.py.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product never calls it.
 *
 * Reference algorithm followed (paths relative to the reference root):
 *   top-k order and rank-order denominator   cuda/q38_kernels.cu:406-480
 *   route plan (stable counting sort, tasks,  cuda/q38_moe_prefill.cu:155-290
 *     status, FNV-1a hashes)
 *   plan ABI and sizes                        include/q38/cuda_moe_prefill.h:11-93
 *   hidden gather                             cuda/q38_moe_prefill.cu:292-306
 *   gate/up epilogue rounding sequence        cuda/q38_moe_prefill.cu:441-462
 *   down projection per packed row            cuda/q38_moe_prefill.cu:589-598
 *   fixed-order top-10 reduce + shared term   cuda/q38_moe_prefill.cu:601-631
 *   decode shared combine                     cuda/q38_moe.cu:337-350
 *   int4 two's-complement nibble, low first   cuda/q38_moe.cu:112-114,
 *                                             tools/q38_artifact_compiler.py:240-243
 *   absmax/qmax scale, zero->1, rint, clip    tools/q38_artifact_compiler.py:214-222
 *   bf16 round-to-nearest-even               tools/q38_artifact_compiler.py:61-66
 *
 * Pins (tests/test_oracle_*.py): every function below is checked against
 * an independent computation -- the reference's own known-answer tests
 * restated (top-k ties, plan bounds 560/640/800 and 52,552 B, stable
 * packing, fail-closed invalid id, int4 packing [-7,-1,0,7]->[F9,70],
 * bf16 round trips, the one-hot grouped-MoE KAT), numpy/torch library
 * routines (stable argsort, int64 matmul for the int32 accumulators,
 * float16/bfloat16 casts, IEEE float32 division), a float64 restatement
 * of the whole layer within a stated tolerance, and libm exp within
 * 2 ulp.  See the header comment of each test file.  No function here is
 * "parity unpinned".
 *
 * Determinism contract: compiled with -ffp-contract=off; every fused
 * multiply-add is an explicit fmaf(); no reduction crosses an OpenMP
 * thread, so the OpenMP build is bit-identical to the serial one.
 */
#ifndef Q38M_ORACLE_H
#define Q38M_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q38O_EXPERTS 512u
#define Q38O_TOPK 10u
#define Q38O_MMQ_M 16u
#define Q38O_SLAB_MAX_TOKENS 512u
#define Q38O_PLAN_MAGIC 0x52383351u
#define Q38O_PLAN_VERSION 1u

/* ---- scalar conversions and the contract's exp ---------------------- */
uint16_t q38o_f32_to_bf16(float value);
float q38o_bf16_to_f32(uint16_t value);
uint16_t q38o_f32_to_f16(float value);
float q38o_f16_to_f32(uint16_t value);
float q38o_expf(float x);
float q38o_logf(float x);
void q38o_expf_array(const float* x, size_t n, float* out);
void q38o_f32_to_bf16_array(const float* x, size_t n, uint16_t* out);
void q38o_f32_to_f16_array(const float* x, size_t n, uint16_t* out);
void q38o_f16_to_f32_array(const uint16_t* x, size_t n, float* out);

/* ---- counter-based synthetic data (SplitMix64) ---------------------- */
uint64_t q38o_rand64(uint64_t seed, uint64_t tag, uint64_t counter);
void q38o_synth_normal_f32(uint64_t seed, uint64_t tag, float sigma,
                           int absolute, size_t n, float* out);
void q38o_synth_normal_bf16(uint64_t seed, uint64_t tag, float sigma,
                            size_t n, uint16_t* out);
void q38o_synth_abs_normal_f16(uint64_t seed, uint64_t tag, float sigma,
                               size_t n, uint16_t* out);
/* logits[t][e] = N(0,sigma) + bias[e]  (bias may be NULL) */
void q38o_synth_logits(uint64_t seed, uint64_t tag, float sigma,
                       const float* bias, uint32_t tokens, uint32_t experts,
                       float* out);
/* W4: n logical int4 values uniform in [lo,hi], packed two per byte,
 * even index in the low nibble.  n must be even. */
void q38o_synth_uniform_w4(uint64_t seed, uint64_t tag, int lo, int hi,
                           size_t n, uint8_t* out);
void q38o_synth_uniform_i8(uint64_t seed, uint64_t tag, int lo, int hi,
                           size_t n, int8_t* out);

/* ---- routing -------------------------------------------------------- */
/* Top-k by (logit desc, expert id asc); weights exp(l_r-l_0)/sum_rank,
 * denominator accumulated in rank order (normalize!=0), or over all
 * experts in expert order (normalize==0). */
int q38o_topk(const float* logits, uint32_t tokens, uint32_t experts,
              uint32_t top_k, int normalize, int32_t* ids, float* weights);

uint32_t q38o_routes(uint32_t tokens);
uint32_t q38o_max_tasks(uint32_t tokens);
size_t q38o_plan_bytes(uint32_t tokens);
/* Writes the complete V1 plan image (header, counts, offsets,
 * task_offsets, packed, inverse, tasks) into plan[0..plan_bytes).  The
 * FNV-1a route/plan hashes are written when with_hashes != 0, else 0. */
int q38o_build_plan(const int32_t* expert_ids, uint32_t tokens,
                    int with_hashes, uint8_t* plan);

/* ---- quantisation --------------------------------------------------- */
void q38o_quantize_rows(const uint16_t* x, uint32_t rows, uint32_t width,
                        int8_t* q, float* scales);

/* Weight quantiser (tools/q38_artifact_compiler.py:193-253,
 * quantize_groupwise) over `rows` bf16 rows of `cols` columns: per group
 * of `group` columns (0: the whole row) s = max|w| / qmax (fp32; qmax 7 for
 * bits 4, 127 for bits 8), s == 0 -> 1, q = clip(rint(w / s), +-qmax) from
 * the fp32 s.  W4 packs column 2i in the low and 2i+1 in the high nibble
 * (:240-243).  Scales are written as RNE fp16 (scale_bf16 == 0, the
 * BASELINE scale format) or RNE bf16 (scale_bf16 != 0, what the reference
 * writes, f32_to_bf16_rne at :232).  Returns 0, or 1 for an invalid shape. */
int q38o_quantize_weights(const uint16_t* src_bf16, uint64_t rows,
                          uint32_t cols, int bits, uint32_t group,
                          uint8_t* data, uint16_t* scales, int scale_bf16);

/* ---- decode combine (cuda/q38_moe.cu:337-350) ------------------------ */
/* out[t][c] = bf16(fmaf(shared[t][c], 1/(1+exp(-gate[t])), routed[t][c])) */
void q38o_combine_shared(const uint16_t* routed, const uint16_t* shared_output,
                         const uint16_t* shared_gate, uint32_t tokens, uint32_t hidden,
                         uint16_t* output);

/* ---- weights -------------------------------------------------------- */
typedef struct q38o_weights {
    const uint8_t* data;     /* canonical row-major: W4 [E][rows][cols/2]
                                (low nibble = even column); W8 [E][rows][cols] */
    const uint16_t* scales;  /* group g: [E][rows][cols/g];
                                per channel (group 0): [E][rows] */
    uint32_t bits;           /* 4 or 8 */
    uint32_t group;          /* 32, 64, 128 ... or 0 = per output channel */
    uint32_t experts, rows, cols;
    uint32_t scale_bf16;     /* scale words: 0 = fp16, 1 = bf16 (both
                                widen to fp32 exactly) */
} q38o_weights;

/* Scaled row value before the activation scale:
 *   group > 0: y = fmaf((float)acc_g, s_g, y) for g = 0..cols/group-1, y0 = 0
 *   group = 0: y = (float)acc * s                                        */
float q38o_row_value(const q38o_weights* w, uint32_t expert, uint32_t row,
                     const int8_t* x);
/* int32 accumulators of one row for debugging/pinning:
 * out[g] = sum_{k in group g} x[k]*w[k] (group 0 -> one value) */
void q38o_row_accumulators(const q38o_weights* w, uint32_t expert,
                           uint32_t row, const int8_t* x, int32_t* out);

/* ---- grouped stages (V1 plan image as produced by q38o_build_plan) -- */
void q38o_gate_up(const q38o_weights* gate_up, uint32_t hidden,
                  uint32_t inter, const int8_t* xq, const float* xs,
                  const uint8_t* plan, const float* route_weights,
                  uint16_t* weighted_mid);
void q38o_down(const q38o_weights* down, uint32_t hidden, uint32_t inter,
               const int8_t* mid_q, const float* mid_scales,
               const uint8_t* plan, float* route_output);
void q38o_combine(const float* route_output, const uint32_t* inverse,
                  const uint16_t* shared_output, const uint16_t* shared_gate,
                  uint32_t tokens, uint32_t hidden, uint16_t* output);

/* ---- whole step ----------------------------------------------------- */
typedef struct q38o_moe_io {
    uint32_t tokens, hidden, inter;
    const uint16_t* hidden_states;  /* bf16 [T][H] */
    const float* logits;            /* fp32 [T][E], or NULL: ids/weights given */
    int32_t* ids;                   /* [T][10] in (logits==NULL) or out */
    float* weights;                 /* [T][10] in or out */
    const q38o_weights* gate_up;    /* [E][2I][H] */
    const q38o_weights* down;       /* [E][H][I] */
    const uint16_t* shared_output;  /* optional bf16 [T][H] */
    const uint16_t* shared_gate;    /* optional bf16 [T] */
    uint16_t* output;               /* bf16 [T][H] */
    /* optional intermediates (NULL to skip; required internally) */
    uint8_t* plan;                  /* plan_bytes(T), T <= 512 */
    int8_t* xq; float* xs;          /* [T][H], [T] */
    uint16_t* weighted_mid;         /* [R][I] packed order */
    int8_t* mid_q; float* mid_s;    /* [R][I], [R] */
    float* route_output;            /* [R][H] packed order */
} q38o_moe_io;

/* Grouped expert-major step through a V1 plan (T <= 512). */
int q38o_moe_prefill(q38o_moe_io* io);
/* The same arithmetic evaluated token by token without a plan (any T).
 * Bit-identical to q38o_moe_prefill by construction of the contract. */
int q38o_moe_per_token(q38o_moe_io* io);

int q38o_num_threads(void);
void q38o_set_num_threads(int threads);

#ifdef __cplusplus
}
#endif

#endif
