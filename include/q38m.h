/*
 * q38m -- MI355X-native quantized MoE data plane, C ABI.
 *
 * Drop-in boundary for the executor's MoE step (reference caller:
 * run_moe, cuda/cuda_backend.cu:1516-1605).  Conventions follow the
 * reference headers: bf16 values travel as raw uint16_t words
 * (include/q38/cuda_kernels.h:11-12), the stream is an opaque void* and
 * the device an int so callers never include vendor headers
 * (include/q38/cuda_transport.h:25-26), every pointer is a device
 * pointer, the caller owns every buffer and no function allocates
 * (include/q38/cuda_moe_prefill.h:95-97).  All compute entry points are
 * asynchronous on the given stream and never read back to the host.
 *
 * Errors: every function returns Q38M_OK or an error code; the message
 * of the last failure on the calling thread is q38m_last_error().  The
 * C++ wrapper (q38m.hpp) rethrows invalid arguments as
 * std::invalid_argument and device errors as std::runtime_error, as the
 * reference does (cuda/q38_moe_prefill.cu:33-68).  Data errors found on
 * the device (invalid expert id) are reported in the plan header's
 * status word without a host sync (cuda/q38_moe_prefill.cu:163-191).
 *
 * Number formats (the arithmetic contract; bit-exact against the CPU
 * oracle): int8 per-token activations (s = absmax/127, q = rint(x/s)),
 * W4 symmetric group-32 or W8 symmetric per-output-channel weights with
 * fp16 scales, int32 accumulators per group, fp32 epilogue in a fixed
 * order, bf16 outputs.
 */
#ifndef Q38M_H
#define Q38M_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------- */
#define Q38M_OK 0
#define Q38M_ERR_INVALID_ARGUMENT 1
#define Q38M_ERR_DEVICE 2
#define Q38M_ERR_UNSUPPORTED 3

/* ---- routing constants: include/q38/cuda_moe_prefill.h:11-16 --------- */
#define Q38M_ROUTE_EXPERTS 512u
#define Q38M_ROUTE_TOPK 10u
#define Q38M_MMQ_M 16u
#define Q38M_PREFILL_SLAB_MAX_TOKENS 512u
#define Q38M_ROUTE_PLAN_MAGIC_V1 0x52383351u /* "Q38R" */
#define Q38M_ROUTE_PLAN_VERSION_V1 1u
/* Chunks above the slab (no reference counterpart: the reference prefills
 * in slabs of <= 512 tokens).  The chunk plan keeps the V1 layout, packed
 * order and status codes with tasks of up to 128 rows and version 2. */
#define Q38M_WIDE_MAX_TOKENS 32768u
#define Q38M_WIDE_TASK_ROWS 128u
#define Q38M_ROUTE_PLAN_VERSION_WIDE 2u
/* Hyper-connection streams per token (include/q38/cuda_hyper.h:9). */
#define Q38M_HYPER_STREAMS 4u
/* Model widths this build's kernels are instantiated for. */
#define Q38M_HIDDEN 2048u
#define Q38M_INTERMEDIATE 512u

/* Q38RoutePlanStatusV1, include/q38/cuda_moe_prefill.h:18-22 */
#define Q38M_PLAN_OK 0u
#define Q38M_PLAN_INVALID_EXPERT 1u
#define Q38M_PLAN_INVALID_SHAPE 2u
/* No reference counterpart: ORed into the plan status by the one-launch
 * gate/up + down (q38m_moe_prefill_v1, q38m_moe_grouped_gate_up_down_v1)
 * when a down workgroup's bounded wait for its task's gate/up workgroups
 * ran out; that step's outputs are then invalid.  Not expected to occur
 * (see q38m_moe_grouped_gate_up_down_v1). */
#define Q38M_PLAN_STEP_TIMEOUT 4u

/* Q38PrefillMoeModeV1, include/q38/cuda_moe_prefill.h:67-71.  The grouped
 * gate/up and down entry points take the mode argument of the reference and
 * accept the two grouped modes (identical kernels; "safe" is only the
 * validation label, cuda/q38_moe_prefill.cu:64-68); the legacy atomic
 * diagnostic is not built and is rejected as an invalid argument. */
#define Q38M_MOE_MODE_GROUPED_MMQ 1u
#define Q38M_MOE_MODE_GROUPED_MMQ_SAFE 2u
#define Q38M_MOE_MODE_LEGACY_ATOMIC_DIAGNOSTIC 3u

/* q38m_moe_build_route_plan_v1 flags */
#define Q38M_PLAN_FLAG_HASHES 1u /* also compute the FNV-1a route/plan hashes */

/* ---- plan ABI (byte-identical to the reference V1 layout) ------------ */
/* Q38ExpertMmqTaskV1, include/q38/cuda_moe_prefill.h:24-31 */
typedef struct __attribute__((aligned(8))) q38m_task_v1 {
    uint32_t packed_begin;
    uint16_t expert;
    uint8_t valid_rows;
    uint8_t flags;
} q38m_task_v1;

/* Q38RoutePlanHeaderV1, include/q38/cuda_moe_prefill.h:33-48 */
typedef struct __attribute__((aligned(16))) q38m_route_plan_header_v1 {
    uint32_t magic;
    uint32_t version;
    uint32_t tokens;
    uint32_t routes;
    uint32_t active_experts;
    uint32_t task_count;
    uint32_t status;
    uint32_t flags;
    uint64_t route_hash;
    uint64_t plan_hash;
    uint64_t reserved0;
    uint64_t reserved1;
} q38m_route_plan_header_v1;

/* Q38RoutePlanStorageV1, include/q38/cuda_moe_prefill.h:50-58 */
typedef struct q38m_route_plan_v1 {
    q38m_route_plan_header_v1* header;
    uint16_t* expert_counts;        /* [512] */
    uint32_t* expert_offsets;       /* [513] */
    uint32_t* expert_task_offsets;  /* [513] */
    uint32_t* packed_assignment;    /* [routes] expert-major, stable */
    uint32_t* assignment_to_packed; /* [routes] inverse */
    q38m_task_v1* tasks;            /* [max_tasks] M=16 tiles */
} q38m_route_plan_v1;

/* ---- expert weight descriptor ---------------------------------------- */
/* Generalises DeviceWeightFormatV1 (include/q38/device_artifact.h:12-18)
 * and CudaTensorViewV1/CudaWeightLayoutV1 (include/q38/cuda_weights.h:
 * 21-38) with the group size and scale dtype of this build's formats. */
#define Q38M_FORMAT_W4_SYM 2u /* int4 two's complement, even k in the low nibble */
#define Q38M_FORMAT_W8_SYM 3u /* int8 */
#define Q38M_SCALE_F16 1u  /* IEEE binary16 scale words (the BASELINE format) */
#define Q38M_SCALE_BF16 2u /* bfloat16 scale words (the reference artifact format,
                              tools/q38_artifact_compiler.py:232) */
#define Q38M_LAYOUT_ROW_MAJOR 0u   /* canonical artifact layout */
#define Q38M_LAYOUT_MFMA16 2u      /* device layout for the 16x16 int8 MFMA kernels */
#define Q38M_LAYOUT_MFMA16_PAIRED 3u /* MFMA16 with row tile t next to tile t+rows/32
                                        (the gate/up halves) */

typedef struct q38m_expert_weights_v1 {
    const void* data;
    const void* scales;
    uint32_t format;      /* Q38M_FORMAT_* */
    uint32_t group_size;  /* 32, 64, 128, or 0 = one scale per output channel */
    uint32_t scale_dtype; /* Q38M_SCALE_F16 or Q38M_SCALE_BF16 */
    uint32_t layout;      /* Q38M_LAYOUT_* */
    uint32_t experts;     /* 512 */
    uint32_t rows;        /* output channels: 2*I for gate/up, H for down */
    uint32_t columns;     /* K: H for gate/up, I for down */
} q38m_expert_weights_v1;

/* Formats the grouped kernels run (prefill, chunk and decode alike), for
 * gate/up (MFMA16_PAIRED) and down (MFMA16) alike: W4 in groups of 32, 64
 * or 128; W8 per channel or in groups of 64 or 128; fp16 or bf16 scale
 * words.  The reference model's routed
 * experts are W4 group-128 (interior layers) and W8 group-128 (edge layers,
 * gate/up too) with bf16 scales (tools/q38_quant_policy.py:164-190); the
 * BASELINE formats are W4 g32 / W8 per channel with fp16 scales.
 * Per group g: y = fmaf((float)acc_g, s_g, y) in group order from 0, acc_g
 * the group's exact int32 sum; per channel: y = (float)acc * s.
 * Row-major layouts (artifact): W4 data [E][rows][cols/2], W8 data
 * [E][rows][cols]; scales [E][rows][cols/group] or [E][rows] (per
 * channel).  MFMA16 layouts (produced by q38m_repack_expert_weights):
 *   W4 data  [E][cols/128][slot][64 lanes][16 B], quad-major: for one
 *     128-wide K block (quad kq) all row tiles are adjacent.  Slot s holds
 *     row tile s (MFMA16) or, paired, tile s/2 + (s%2)*rows/32.  Lane
 *     l = (q=l/16, n=l%16) holds for row 16t+n and groups 4kq+j (j=0..3) one
 *     dword each: byte i = nib(k0+i) | nib(k0+4+i)<<4, k0 = 32(4kq+j)+8q.
 *   W4 scales [E][cols/128][slot][16 rows][128/group] (same order: 4, 2
 *     or 1 words per row and quad for groups of 32, 64, 128).
 *   W8 data  [E][rows/16][cols/64][64 lanes][16 B]; lane l holds row 16t+n,
 *     columns 64kb+16q .. +15.   W8 scales stay in the artifact order.
 *   W8 paired (gate/up) [E][cols/64][slot][64 lanes][16 B], K-block-major:
 *     for one 64-wide K block every slot is adjacent; slot s holds row tile
 *     s/2 + (s%2)*rows/32, lanes as W8. */

/* ---- sizes: include/q38/cuda_moe_prefill.h:73-93 --------------------- */
uint32_t q38m_moe_prefill_routes_v1(uint32_t tokens);
uint32_t q38m_moe_prefill_max_tasks_v1(uint32_t tokens);
size_t q38m_moe_route_plan_bytes_v1(uint32_t tokens);

/* cuda_moe_route_plan_storage_v1, include/q38/cuda_moe_prefill.h:98-99
 * (cuda/q38_moe_prefill.cu:635-663).  Binds views; never touches memory. */
int q38m_moe_route_plan_storage_v1(void* allocation, size_t allocation_bytes,
                                   uint32_t tokens, q38m_route_plan_v1* out);

/* cuda_topk_router_bf16, include/q38/cuda_kernels.h:83-91, with fp32
 * logits (the BASELINE router output).  Experts must be a multiple of 64
 * and <= 1024; top_k <= 32. */
int q38m_topk_router_f32(const float* logits, int32_t* expert_ids,
                         float* expert_weights, uint32_t tokens,
                         uint32_t experts, uint32_t top_k, int normalize_top_k,
                         void* stream, int device);

/* cuda_topk_router_bf16, include/q38/cuda_kernels.h:83-91: the same
 * selection and weights as q38m_topk_router_f32 on bf16 logits (raw words),
 * the type the reference's router GEMM writes.  bf16 widens to fp32
 * exactly, so the result equals q38m_topk_router_f32 on the widened
 * logits.  Same limits as q38m_topk_router_f32. */
int q38m_topk_router_bf16(const uint16_t* logits, int32_t* expert_ids,
                          float* expert_weights, uint32_t tokens,
                          uint32_t experts, uint32_t top_k, int normalize_top_k,
                          void* stream, int device);

/* Top-10 routing and int8 activation quantisation in one launch (one
 * workgroup per token): cuda_topk_router_bf16 (include/q38/cuda_kernels.h:
 * 83-91; 512 experts, normalised) fused with the per-token quantisation
 * that feeds cuda_moe_grouped_gate_up_v1 (xq[T][2048] int8 + xs[T] fp32;
 * the reference gathers bf16 rows, cuda_moe_pack_hidden_v1).  Writes
 * expert_ids/expert_weights [T][10] as q38m_topk_router_f32 does.
 * logits and hidden 16-byte aligned, xq 8-byte aligned. */
int q38m_moe_route_quantize_v1(const float* logits, const uint16_t* hidden,
                               uint32_t tokens, int32_t* expert_ids,
                               float* expert_weights, int8_t* xq, float* xs,
                               void* stream, int device);

/* cuda_moe_build_route_plan_v1, include/q38/cuda_moe_prefill.h:101-104.
 * flags: Q38M_PLAN_FLAG_HASHES computes route_hash/plan_hash exactly as the
 * reference (a serial pass); without it both hashes are 0. */
int q38m_moe_build_route_plan_v1(const int32_t* expert_ids, uint32_t tokens,
                                 const q38m_route_plan_v1* plan, uint32_t flags,
                                 void* stream, int device);

/* cuda_moe_pack_hidden_v1, include/q38/cuda_moe_prefill.h:106-110.
 * Kept for callers of the bf16 gather; the int8 path gathers in-kernel. */
int q38m_moe_pack_hidden_v1(const uint16_t* hidden,
                            const uint32_t* packed_assignment, uint32_t routes,
                            uint32_t hidden_width, uint16_t* packed_hidden,
                            void* stream, int device);

/* Per-row int8 absmax quantisation of a bf16 matrix (no reference
 * counterpart; rounding convention of tools/q38_artifact_compiler.py:
 * 214-222).  width is 512, 1024, 2048 or 4096. */
int q38m_quantize_rows_i8(const uint16_t* x, uint32_t rows, uint32_t width,
                          int8_t* q, float* scales, void* stream, int device);

/* out = bf16(a + b), the residual add between stacked MoE layers (the
 * caller's side of the step; cf. the hyper-connection finish around
 * run_moe, cuda/cuda_backend.cu:1967-1971).  elements % 8 == 0. */
int q38m_residual_add_bf16(const uint16_t* a, const uint16_t* b, uint16_t* out,
                           uint64_t elements, void* stream, int device);

/* cuda_moe_grouped_gate_up_v1, include/q38/cuda_moe_prefill.h:112-118.
 * Reads int8 token rows xq[T][H] (scales xs[T]) through packed_assignment
 * instead of a packed bf16 copy; writes weighted_mid bf16 [routes][I] in
 * packed order: m = bf16(bf16(silu(g)*u) * w).  gate_up: MFMA16_PAIRED.
 * mode: Q38M_MOE_MODE_GROUPED_MMQ or _SAFE (validate_grouped_mode). */
int q38m_moe_grouped_gate_up_v1(const q38m_expert_weights_v1* gate_up,
                                const int8_t* xq, const float* xs,
                                const uint32_t* packed_assignment,
                                const float* token_rank_weights,
                                const q38m_task_v1* tasks, uint32_t task_count,
                                uint16_t* weighted_mid, uint32_t mode, void* stream,
                                int device);

/* cuda_moe_grouped_down_v1, include/q38/cuda_moe_prefill.h:120-125.
 * Input: the int8 quantised weighted_mid rows (q38m_quantize_rows_i8).
 * Output: route_output fp32 [routes][H] in packed order.  down: MFMA16.
 * mode as for gate/up. */
int q38m_moe_grouped_down_v1(const q38m_expert_weights_v1* down,
                             const int8_t* mid_q, const float* mid_scales,
                             const q38m_task_v1* tasks, uint32_t task_count,
                             float* route_output, uint32_t mode, void* stream, int device);

/* No reference counterpart: cuda_moe_grouped_gate_up_v1, the mid
 * quantisation (q38m_quantize_rows_i8) and cuda_moe_grouped_down_v1
 * (include/q38/cuda_moe_prefill.h:112-125) as one call, with their
 * results bit for bit (weighted_mid, mid_q/mid_scales, route_output).  W4
 * gate/up with per-channel W8 down of one scale dtype run as ONE launch
 * whose down workgroups start while the last gate/up workgroups still
 * stream; other format pairs run the three kernels.  task_flags:
 * 9 * task_count words (8 hand-off flags and a counter per task) that must
 * be ZERO on entry: clear them once with q38m_moe_clear_task_flags_v1
 * after allocating them; the call leaves them zero (the last down
 * workgroup of each task clears the task's words).  plan_status (normally
 * &plan.header->status): a down workgroup ORs Q38M_PLAN_STEP_TIMEOUT into
 * it if its bounded wait for its task's gate/up workgroups runs out --
 * that call's outputs are invalid and the flags must be cleared again.
 * Workgroups are dispatched in block order and every gate/up workgroup
 * precedes every down workgroup, so the wait always ends within a gate/up
 * workgroup's lifetime; the bound only caps a broken dispatch order.
 * mode as for gate/up. */
int q38m_moe_grouped_gate_up_down_v1(const q38m_expert_weights_v1* gate_up,
                                     const q38m_expert_weights_v1* down,
                                     const int8_t* xq, const float* xs,
                                     const uint32_t* packed_assignment,
                                     const float* token_rank_weights,
                                     const q38m_task_v1* tasks, uint32_t task_count,
                                     uint16_t* weighted_mid, int8_t* mid_q,
                                     float* mid_scales, uint32_t* task_flags,
                                     uint32_t* plan_status, float* route_output,
                                     uint32_t mode, void* stream, int device);

/* No reference counterpart: zeroes the 9 * task_count words of a
 * q38m_moe_grouped_gate_up_down_v1 task_flags buffer (a fill kernel). */
int q38m_moe_clear_task_flags_v1(uint32_t* task_flags, uint32_t task_count, void* stream,
                                 int device);

/* cuda_moe_reduce_top10_and_combine_shared_v1,
 * include/q38/cuda_moe_prefill.h:127-131.  shared_output/shared_gate may
 * both be NULL (no shared expert). */
int q38m_moe_reduce_top10_and_combine_shared_v1(
    const float* route_output, const uint32_t* assignment_to_packed,
    const uint16_t* shared_output, const uint16_t* shared_gate,
    uint32_t tokens, uint16_t* output, void* stream, int device);

/* cuda_moe_combine_shared_bf16, include/q38/cuda_moe.h:31-37. */
int q38m_moe_combine_shared_bf16(const uint16_t* routed_output,
                                 const uint16_t* shared_output,
                                 const uint16_t* shared_gate, uint16_t* output,
                                 uint32_t tokens, void* stream, int device);

/* ---- the whole step (the run_moe sequence, cuda_backend.cu:1523-1601) */
/* Workspace of the whole step, bound once for max_tokens (the reference's
 * MoE workspace, cuda/cuda_backend.cu:908-946); any slab of
 * tokens <= max_tokens reuses it. */
typedef struct q38m_prefill_workspace_v1 {
    uint32_t max_tokens;
    q38m_route_plan_v1 plan; /* bound for max_tokens */
    int32_t* expert_ids;     /* [T*10] */
    float* expert_weights;   /* [T*10] */
    int8_t* xq;              /* [T][H] */
    float* xs;               /* [T] */
    uint16_t* weighted_mid;  /* [T*10][I] */
    int8_t* mid_q;           /* [T*10][I] */
    float* mid_s;            /* [T*10] */
    float* route_output;     /* [T*10][H] */
    /* No reference counterpart: the gate/up -> down hand-off flags of the
     * one-launch gate/up + down (8 flags and a counter per task slot),
     * cleared by the step's plan kernel.  NULL: the step runs gate/up and
     * down as two launches. */
    uint32_t* task_flags;    /* [max_tasks(T)*9] */
} q38m_prefill_workspace_v1;

/* Bytes of one contiguous workspace for `tokens` (<= 512) and its binding
 * (allocation 256-byte aligned). */
size_t q38m_moe_prefill_workspace_bytes(uint32_t tokens);
int q38m_moe_prefill_workspace_bind(void* allocation, size_t bytes,
                                    uint32_t tokens,
                                    q38m_prefill_workspace_v1* out);

/* One MoE layer over a slab of <= 512 tokens: top-k (when logits is not
 * NULL; else expert_ids/expert_weights in the workspace are inputs),
 * route plan, int8 quantisation, grouped gate/up, mid quantisation,
 * grouped down, fixed-order combine.  With W4 gate/up and per-channel W8
 * down weights of one scale dtype (and ws->task_flags set), gate/up, the mid
 * quantisation and down run as one launch (q38m_moe_grouped_gate_up_down_v1);
 * the results are the same bit for bit. */
int q38m_moe_prefill_v1(const q38m_expert_weights_v1* gate_up,
                        const q38m_expert_weights_v1* down,
                        const uint16_t* hidden, const float* logits,
                        uint32_t tokens, const q38m_prefill_workspace_v1* ws,
                        const uint16_t* shared_output,
                        const uint16_t* shared_gate, uint16_t* output,
                        void* stream, int device);

/* ---- the same slab step without any allocation ----------------------
 * No counterpart in the reference.  For callers that cannot allocate or
 * pass a workspace: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  q38m_moe_prefill_v1 for a slab of at
 * most Q38M_NOALLOC_MAX_TOKENS (64) tokens with fp32 router logits (top-k
 * inside), bit-identical to it; its workspace is a device-resident array
 * of q38m_moe_prefill_noalloc_scratch_bytes() bytes (6.1 MiB) that each GPU
 * running the library holds until the process ends.  The function calls no
 * allocator: the caller still owns every input and output.  Every call on
 * one GPU shares that GPU's array, so calls that overlap on one GPU (other
 * streams, other threads) race; serialise them.  More than 64 tokens:
 * Q38M_ERR_INVALID_ARGUMENT. */
#define Q38M_NOALLOC_MAX_TOKENS 64u
size_t q38m_moe_prefill_noalloc_scratch_bytes(void);
int q38m_moe_prefill_noalloc_v1(const q38m_expert_weights_v1* gate_up,
                                const q38m_expert_weights_v1* down,
                                const uint16_t* hidden, const float* logits,
                                uint32_t tokens, const uint16_t* shared_output,
                                const uint16_t* shared_gate, uint16_t* output,
                                void* stream, int device);

/* ---- one layer over a chunk of up to 32,768 tokens ------------------
 * No reference counterpart: the reference runs run_moe per slab of <= 512
 * tokens (cuda/cuda_backend.cu:1529-1559).  Same inputs, outputs and
 * arithmetic as q38m_moe_prefill_v1 -- every token's output is
 * bit-identical to running its slab through that entry point -- with the
 * route plan built over the whole chunk, so each active expert's weights
 * are streamed once per 128 routed rows instead of once per 16.  The
 * plan's packed order is the V1 order (expert-major, stable in route
 * index); its tasks are 128-row tiles (header version 2). */
typedef struct q38m_wide_workspace_v1 {
    q38m_prefill_workspace_v1 step; /* bound for max_tokens <= 32768 */
    uint32_t* plan_scratch;         /* per-chunk expert counts */
} q38m_wide_workspace_v1;

/* Chunk plan alone: bytes of the plan views and of their build scratch. */
uint32_t q38m_moe_wide_max_tasks(uint32_t tokens);
size_t q38m_moe_wide_plan_bytes(uint32_t tokens);
size_t q38m_moe_wide_plan_scratch_bytes(uint32_t tokens);
int q38m_moe_wide_plan_storage(void* allocation, size_t allocation_bytes,
                               uint32_t tokens, q38m_route_plan_v1* out);
/* Builds the chunk plan of expert_ids [tokens][10] into a plan bound by
 * q38m_moe_wide_plan_storage for >= tokens; scratch holds
 * q38m_moe_wide_plan_scratch_bytes(tokens) bytes, 4-byte aligned. */
int q38m_moe_build_route_plan_wide(const int32_t* expert_ids, uint32_t tokens,
                                   const q38m_route_plan_v1* plan, uint32_t* scratch,
                                   void* stream, int device);

size_t q38m_moe_wide_workspace_bytes(uint32_t tokens);
int q38m_moe_wide_workspace_bind(void* allocation, size_t bytes, uint32_t tokens,
                                 q38m_wide_workspace_v1* out);
int q38m_moe_prefill_wide_v1(const q38m_expert_weights_v1* gate_up,
                             const q38m_expert_weights_v1* down,
                             const uint16_t* hidden, const float* logits,
                             uint32_t tokens, const q38m_wide_workspace_v1* ws,
                             const uint16_t* shared_output,
                             const uint16_t* shared_gate, uint16_t* output,
                             void* stream, int device);

/* ---- batch-1 decode: cuda_moe_routed_bf16 (include/q38/cuda_moe.h:
 * 17-29) tokens == 1 branch.  Streams only the top_k selected experts.
 * Bit-identical to q38m_moe_prefill_v1 with tokens == 1.  scratch:
 * q38m_moe_decode_scratch_bytes() bytes, 16-aligned. */
size_t q38m_moe_decode_scratch_bytes(void);
int q38m_moe_routed_decode_v1(const q38m_expert_weights_v1* gate_up,
                              const q38m_expert_weights_v1* down,
                              const uint16_t* hidden,
                              const int32_t* expert_ids,
                              const float* expert_weights, uint32_t top_k,
                              void* scratch, uint16_t* routed_output,
                              void* stream, int device);

/* Fused batch-1 decode from fp32 router logits: the whole tokens == 1
 * sequence of run_moe (cuda/cuda_backend.cu:1516-1605) after the router
 * GEMV -- cuda_topk_router_bf16 (include/q38/cuda_kernels.h:83-91, here on
 * 512 experts, normalised), cuda_moe_routed_bf16 (include/q38/cuda_moe.h:
 * 17-29) and cuda_moe_combine_shared_bf16 (include/q38/cuda_moe.h:31-37)
 * -- in two launches.  shared_output/shared_gate: both null (no shared
 * term) or both given.  residual: null, or output = bf16(residual + moe).
 * Bit-identical to q38m_moe_prefill_v1 with tokens == 1 (then
 * q38m_residual_add_bf16).  scratch as above; the chosen ids are left in
 * its first 40 bytes. */
int q38m_moe_decode_v1(const q38m_expert_weights_v1* gate_up,
                       const q38m_expert_weights_v1* down,
                       const uint16_t* hidden, const float* logits,
                       uint32_t top_k, const uint16_t* shared_output,
                       const uint16_t* shared_gate, const uint16_t* residual,
                       void* scratch, uint16_t* output, void* stream,
                       int device);

/* The whole MoE block of one decode step from the hidden row: the tokens
 * == 1 branch of run_moe (cuda/cuda_backend.cu:1516-1605) -- the router
 * GEMV over the bf16 router (:1518-1519), cuda_topk_router_bf16 (512
 * experts, normalised), cuda_moe_routed_bf16 (include/q38/cuda_moe.h:
 * 17-29), the bf16 shared expert (cuda_backend.cu:1573-1590) and
 * cuda_moe_combine_shared_bf16 (cuda_moe.h:31-37) -- in three launches
 * instead of five: the router GEMV; the routed gate/up with the top-k and
 * the shared gate/up; the routed down with the shared down, the gated
 * combine and the optional residual.  Bit-identical to
 * q38m_moe_router_v1 -> q38m_moe_shared_expert_v1 -> q38m_moe_decode_v1
 * on the same token.  router [512][2048], w_gate / w_up [shared_inter][2048],
 * w_down [2048][shared_inter], w_out_gate [2048], bf16, 16-byte aligned;
 * shared_inter must be Q38M_INTERMEDIATE (512).  residual: null, or
 * output = bf16(residual + moe).  scratch: 16-byte aligned,
 * q38m_moe_decode_block_scratch_bytes() bytes; the chosen ids are left in
 * its first 40 bytes. */
size_t q38m_moe_decode_block_scratch_bytes(void);
int q38m_moe_decode_block_v1(const q38m_expert_weights_v1* gate_up,
                             const q38m_expert_weights_v1* down,
                             const uint16_t* hidden, const uint16_t* router,
                             const uint16_t* w_gate, const uint16_t* w_up,
                             const uint16_t* w_down, const uint16_t* w_out_gate,
                             uint32_t shared_inter, uint32_t top_k,
                             const uint16_t* residual, void* scratch,
                             uint16_t* output, void* stream, int device);

/* ---- hyper-connection prepare/finish around the MoE step -------------
 * include/q38/cuda_hyper.h:15-58 (kernels cuda/q38_hyper.cu:52-114; call
 * sequence cuda_backend.cu:1219-1252).  The hidden state is
 * Q38M_HYPER_STREAMS streams of `hidden` bf16 values per token ([T][4][H]);
 * the reference fixes hidden = 2560 (cuda_hyper.h:9-12), here it is a
 * parameter (multiple of 8, <= 8192) so the prepare can feed this library's
 * H = 2048 MoE.  Floating-point results (fp32 inside a step, bf16 between
 * steps as the reference, this library's exp): parity is a tolerance.
 * Elementwise entry points need tokens * width to be a multiple of 8. */
int q38m_hyper_repeat_embedding_bf16(const uint16_t* embedding, uint16_t* hyper,
                                     uint32_t tokens, uint32_t hidden, void* stream,
                                     int device);
int q38m_hyper_group_rmsnorm_bf16(const uint16_t* hyper, const uint16_t* norm_weight,
                                  uint16_t* normalized, uint32_t tokens, uint32_t hidden,
                                  void* stream, int device);
int q38m_hyper_silu_scaled_bf16(const uint16_t* input, uint16_t* output, uint32_t tokens,
                                uint32_t width, float divisor, void* stream, int device);
int q38m_hyper_sigmoid_bf16(const uint16_t* input, uint16_t* output, uint32_t tokens,
                            uint32_t width, float input_divisor, float output_scale,
                            void* stream, int device);
int q38m_hyper_mix_bf16(const uint16_t* normalized_hyper, const uint16_t* mix_weights,
                        uint16_t* mixed, uint32_t tokens, uint32_t hidden, void* stream,
                        int device);
int q38m_hyper_inject_bf16(const uint16_t* original_hyper, const uint16_t* block_output,
                           const uint16_t* injection_weights, uint16_t* output_hyper,
                           uint32_t tokens, uint32_t hidden, void* stream, int device);
/* The whole prepare_hyper sequence (cuda_backend.cu:1219-1243) in four
 * launches: mix_down [low_rank][4H], mix_up [4H][low_rank], inject [4][4H]
 * or NULL (then injection is not written).  low_rank % 32 == 0.  Outputs
 * mixed [T][H] (the MoE input) and injection [T][4] (for the finish). */
size_t q38m_hyper_prepare_scratch_bytes(uint32_t tokens, uint32_t hidden, uint32_t low_rank);
int q38m_hyper_prepare_v1(const uint16_t* hyper, const uint16_t* norm_weight,
                          const uint16_t* mix_down, const uint16_t* mix_up,
                          const uint16_t* inject, uint32_t tokens, uint32_t hidden,
                          uint32_t low_rank, void* scratch, uint16_t* mixed,
                          uint16_t* injection, void* stream, int device);

/* ---- weight layout (cuda/cuda_weights.cu:229-285 re-tiles W4 at load) */
size_t q38m_expert_weights_bytes(const q38m_expert_weights_v1* w,
                                 size_t* scale_bytes);
/* Converts row-major weights into the MFMA16 device layout.  dst
 * describes the destination buffers (layout MFMA16, same shape/format). */
int q38m_repack_expert_weights(const q38m_expert_weights_v1* src,
                               const q38m_expert_weights_v1* dst,
                               void* stream, int device);

/* ---- dense bf16 GEMMs on either side of the routed experts ----------
 * C[m][n] = A[m][k] * B[n][k]^T (both K-contiguous: activation rows and
 * [out][in] weight rows), bf16 in, fp32 accumulation (MFMA), exactly one of
 * c_f32 / c_bf16 (round to nearest even) out.  k % 32 == 0; a, b 16-byte
 * aligned.  Floating-point parity: a tolerance, not bit-exact. */
int q38m_dense_gemm_bf16(const uint16_t* a, const uint16_t* b, uint32_t m,
                         uint32_t n, uint32_t k, float* c_f32,
                         uint16_t* c_bf16, void* stream, int device);

/* Router logits: hidden bf16 [T][hidden_width] times the bf16 router
 * [512][hidden_width] (the "preserved" router format,
 * tools/q38_quant_policy.py:205) -> fp32 logits [T][512], the input of
 * q38m_moe_route_quantize_v1 / q38m_moe_prefill_v1 / q38m_moe_decode_v1.
 * Replaces the router GEMV/GEMM of run_moe (cuda/cuda_backend.cu:1518-1519;
 * the reference rounds the logits to bf16).  hidden_width must be the
 * MoE's Q38M_HIDDEN (2048): any other width is rejected, so a caller
 * cannot feed it rows of another stride. */
int q38m_moe_router_v1(const uint16_t* hidden, const uint16_t* router,
                       uint32_t tokens, uint32_t hidden_width, float* logits,
                       void* stream, int device);

/* Router GEMM and top-k selection without the fp32 logits in memory: the
 * router step of run_moe (cuda/cuda_backend.cu:1518-1525: the router GEMM,
 * then cuda_topk_router_bf16 with 512 experts and normalize_top_k = true,
 * include/q38/cuda_kernels.h:83-91) in two launches.  The first computes
 * the logits exactly as q38m_moe_router_v1 does and keeps each 64-expert
 * block's top 10 per token (keys in the workspace); the second ranks the
 * 80 candidates per token.  expert_ids / expert_weights [T][top_k] equal
 * q38m_topk_router_f32 (512 experts, normalised) on q38m_moe_router_v1's
 * logits, bit for bit.  hidden_width must be Q38M_HIDDEN; 1 <= top_k <= 10;
 * workspace (16-byte aligned) of q38m_moe_router_topk_workspace_bytes(T).
 * No single reference function: the reference runs these as two calls. */
size_t q38m_moe_router_topk_workspace_bytes(uint32_t tokens);
int q38m_moe_router_topk_v1(const uint16_t* hidden, const uint16_t* router,
                            uint32_t tokens, uint32_t hidden_width,
                            uint32_t top_k, void* workspace,
                            size_t workspace_bytes, int32_t* expert_ids,
                            float* expert_weights, void* stream, int device);

/* Shared expert of the MoE block (cuda/cuda_backend.cu:1573-1590), bf16
 * weights: g = bf16(x Wg^T), u = bf16(x Wu^T) [T][inter],
 * h = bf16(g / (1 + exp(-g)) * u) (cuda_silu_multiply_bf16,
 * cuda/q38_kernels.cu:286-296), shared_output = bf16(h Wd^T) [T][2048],
 * shared_gate = bf16(x Wo^T) [T] -- the two inputs of the gated combine
 * (q38m_moe_prefill_v1 / q38m_moe_decode_v1 / combine entry points).
 * Wg, Wu [inter][2048]; Wd [2048][inter]; Wo [1][2048]; inter % 32 == 0.
 * hidden_width must be Q38M_HIDDEN (2048), as for the router.
 * scratch: q38m_moe_shared_expert_scratch_bytes(T, inter) bytes. */
size_t q38m_moe_shared_expert_scratch_bytes(uint32_t tokens, uint32_t inter);
int q38m_moe_shared_expert_v1(const uint16_t* hidden, const uint16_t* w_gate,
                              const uint16_t* w_up, const uint16_t* w_down,
                              const uint16_t* w_out_gate, uint32_t tokens,
                              uint32_t hidden_width, uint32_t inter, void* scratch,
                              uint16_t* shared_output, uint16_t* shared_gate,
                              void* stream, int device);

/* Weight quantiser of the artifact pipeline: quantize_groupwise
 * (tools/q38_artifact_compiler.py:193-253) on the device.  src: bf16
 * weights [experts*rows][columns]; dst: row-major layout, fp16 scales,
 * W4 (groups 32/64/128) or W8 (groups 32/64/128, or group 0 = per output
 * channel with columns % 512 == 0).  Per group s = max|w|/qmax (qmax 7 for
 * W4, 127 for W8), s == 0 -> 1, q = clamp(rint(w/s), +-qmax); W4 packs
 * column 2i in the low nibble.  The reference stores bf16 scales; here they
 * are fp16 (BASELINE's format).  Follow with q38m_repack_expert_weights. */
int q38m_quantize_expert_weights(const uint16_t* src_bf16,
                                 const q38m_expert_weights_v1* dst,
                                 void* stream, int device);

/* ---- deterministic synthetic data (counter-based SplitMix64) --------- */
#define Q38M_SYNTH_NORMAL_F32 1u     /* sigma*N(0,1) (+ bias[i % bias_len]) */
#define Q38M_SYNTH_NORMAL_BF16 2u    /* bf16(sigma*N(0,1)) */
#define Q38M_SYNTH_ABS_NORMAL_F16 3u /* f16(|sigma*N(0,1)|) */
#define Q38M_SYNTH_UNIFORM_W4 4u     /* int4 uniform in [lo,hi], packed pairs */
#define Q38M_SYNTH_UNIFORM_I8 5u     /* int8 uniform in [lo,hi] */
int q38m_synth_fill(uint32_t kind, uint64_t seed, uint64_t tag, uint64_t count,
                    float sigma, int32_t lo, int32_t hi, const float* bias,
                    uint32_t bias_len, void* out, void* stream, int device);

/* cuda_q38_moe_prefill_compiled / cuda_q38_moe_compiled */
int q38m_moe_compiled(void);
const char* q38m_last_error(void);

#ifdef __cplusplus
}
#endif

#endif
