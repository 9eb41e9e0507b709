// Internal launch interface between the C ABI layer (q38m_api.hip) and the
// kernel translation units.  Launchers assume validated arguments; each
// returns hipGetLastError() after its launches.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "q38m.h"

namespace q38m {

constexpr uint32_t kExperts = Q38M_ROUTE_EXPERTS;
constexpr uint32_t kTopK = Q38M_ROUTE_TOPK;
constexpr uint32_t kMmqM = Q38M_MMQ_M;
constexpr uint32_t kSlabMaxTokens = Q38M_PREFILL_SLAB_MAX_TOKENS;
constexpr uint32_t kHidden = Q38M_HIDDEN;
constexpr uint32_t kInter = Q38M_INTERMEDIATE;

constexpr uint32_t routes_v1(uint32_t tokens) { return tokens * kTopK; }
constexpr uint32_t max_tasks_v1(uint32_t tokens) {
    const uint32_t routes = routes_v1(tokens);
    const uint32_t initially = routes < kExperts ? routes : kExperts;
    return initially + (routes - initially) / kMmqM;
}

// Bytes of the V1 plan image and of the whole-step workspace
// (q38m_moe_route_plan_bytes_v1 / q38m_moe_prefill_workspace_bytes), as
// constants for a fixed slab size.
constexpr size_t align256(size_t v) { return (v + 255u) / 256u * 256u; }
constexpr size_t plan_bytes_v1(uint32_t tokens) {
    return 64u + kExperts * 2u + 2u * (kExperts + 1u) * 4u +
           2u * static_cast<size_t>(routes_v1(tokens)) * 4u +
           static_cast<size_t>(max_tasks_v1(tokens)) * 8u;
}
constexpr size_t prefill_workspace_bytes_v1(uint32_t tokens) {
    return align256(plan_bytes_v1(tokens)) + 2u * align256(routes_v1(tokens) * 4u) +
           align256(static_cast<size_t>(tokens) * kHidden) +
           align256(static_cast<size_t>(tokens) * 4u) +
           align256(static_cast<size_t>(routes_v1(tokens)) * kInter * 2u) +
           align256(static_cast<size_t>(routes_v1(tokens)) * kInter) +
           align256(routes_v1(tokens) * 4u) +
           align256(static_cast<size_t>(routes_v1(tokens)) * kHidden * 4u) +
           align256(static_cast<size_t>(max_tasks_v1(tokens)) * 9u * 4u);
}

// chunks above the slab (q38m_wide.hip): 128-row tasks, plans built from
// per-chunk expert histograms of kWideChunkRoutes routes each
constexpr uint32_t kWideChunkRoutes = 2048;
inline uint32_t max_tasks_wide(uint32_t tokens) {
    const uint32_t routes = routes_v1(tokens);
    const uint32_t initially = routes < kExperts ? routes : kExperts;
    return initially + (routes - initially) / Q38M_WIDE_TASK_ROWS;
}
uint32_t wide_chunks(uint32_t tokens);
// chunk_counts: wide_chunks(tokens) * 513 uint32 of scratch
hipError_t launch_build_wide_plan(const int32_t* ids, uint32_t tokens,
                                  const q38m_route_plan_v1& plan, uint32_t* chunk_counts,
                                  hipStream_t stream);
// the grouped GEMMs over 128-row tasks, for the formats launch_gate_up /
// launch_down take; task_count is the number of task slots (grid rows),
// live_tasks the device word holding how many of them the plan filled
hipError_t launch_gate_up_wide(const q38m_expert_weights_v1& w, const int8_t* xq, const float* xs,
                               const uint32_t* packed, const float* route_weights,
                               const q38m_task_v1* tasks, const uint32_t* live_tasks,
                               uint32_t task_count, uint16_t* weighted_mid, hipStream_t stream);
hipError_t launch_down_wide(const q38m_expert_weights_v1& w, const int8_t* mid_q,
                            const float* mid_s, const q38m_task_v1* tasks,
                            const uint32_t* live_tasks, uint32_t task_count,
                            float* route_output, hipStream_t stream);

// routing (q38m_routing.hip)
hipError_t launch_topk(const float* logits, int32_t* ids, float* weights,
                       uint32_t tokens, uint32_t experts, uint32_t top_k,
                       int normalize, hipStream_t stream);
// bf16 logits (uint16_t words)
hipError_t launch_topk(const uint16_t* logits, int32_t* ids, float* weights,
                       uint32_t tokens, uint32_t experts, uint32_t top_k,
                       int normalize, hipStream_t stream);
// 512 logits per token, top-10, normalised, plus the token's int8 row: one
// wave per token (the throughput form for chunks)
hipError_t launch_route_quantize_wave(const float* logits, const uint16_t* hidden,
                                     uint32_t tokens, int32_t* ids, float* weights, int8_t* xq,
                                     float* xs, hipStream_t stream);
// 512 bf16 logits per token, top_k <= 10, normalised (ranked-key kernel)
hipError_t launch_route_bf16(const uint16_t* logits, uint32_t tokens, uint32_t top_k,
                             int32_t* ids, float* weights, hipStream_t stream);
// 512 experts, top_k <= 10, normalised; hidden may be null (top-k only)
hipError_t launch_route_quantize(const float* logits, const uint16_t* hidden, uint32_t tokens,
                                uint32_t top_k, int32_t* ids, float* weights, int8_t* xq,
                                float* xs, hipStream_t stream);
// task_flags (may be null): flag_words words cleared while the ids load,
// the hand-off flags of the fused gate/up + down launch that follows
hipError_t launch_build_plan(const int32_t* ids, uint32_t tokens,
                             const q38m_route_plan_v1& plan, bool hashes,
                             hipStream_t stream, uint32_t* task_flags = nullptr,
                             uint32_t flag_words = 0);

// quantisation and gathers (q38m_quant.hip)
hipError_t launch_quantize_rows(const uint16_t* x, uint32_t rows, uint32_t width,
                                int8_t* q, float* scales, hipStream_t stream);
hipError_t launch_pack_hidden(const uint16_t* hidden, const uint32_t* packed,
                              uint32_t routes, uint32_t width, uint16_t* out,
                              hipStream_t stream);
hipError_t launch_residual_add(const uint16_t* a, const uint16_t* b, uint16_t* out,
                               uint64_t elements, hipStream_t stream);

// grouped GEMMs and combine (q38m_grouped.hip)
// weights validated by the API layer: gate/up W4 (groups 32/64/128,
// MFMA16_PAIRED); down W8 (per channel, groups 64/128) or W4 (groups
// 32/64/128); fp16 or bf16 scale words
hipError_t launch_gate_up(const q38m_expert_weights_v1& w, const int8_t* xq, const float* xs,
                          const uint32_t* packed, const float* route_weights,
                          const q38m_task_v1* tasks, uint32_t task_count, uint16_t* weighted_mid,
                          hipStream_t stream);
hipError_t launch_down(const q38m_expert_weights_v1& w, const int8_t* mid_q, const float* mid_s,
                       const q38m_task_v1* tasks, uint32_t task_count, float* route_output,
                       hipStream_t stream);
// down from the bf16 mid rows: each task's rows quantised inside the kernel
// (the same int8 rows and scales as launch_quantize_rows, also stored to
// mid_q / mid_s)
hipError_t launch_down_quantize(const q38m_expert_weights_v1& w, const uint16_t* weighted_mid,
                                int8_t* mid_q, float* mid_s, const q38m_task_v1* tasks,
                                uint32_t task_count, float* route_output, hipStream_t stream);
// gate/up and down (with the mid quantisation) in one launch when
// gate_up_down_fusable (W4 gate/up, per-channel W8 down, one scale dtype);
// otherwise launch_gate_up + launch_down_quantize.  task_flags:
// task_flag_words(task_count) words, zero at the launch and left zero
// (unless a wait ran out); status: where a down item whose wait ran out ORs
// Q38M_PLAN_STEP_TIMEOUT.
constexpr uint32_t task_flag_words(uint32_t task_count) { return 9u * task_count; }
bool gate_up_down_fusable(const q38m_expert_weights_v1& gate_up,
                          const q38m_expert_weights_v1& down);
hipError_t launch_gate_up_down(const q38m_expert_weights_v1& gate_up,
                               const q38m_expert_weights_v1& down, const int8_t* xq,
                               const float* xs, const uint32_t* packed,
                               const float* route_weights, const q38m_task_v1* tasks,
                               uint32_t task_count, uint16_t* weighted_mid, int8_t* mid_q,
                               float* mid_s, float* route_output, uint32_t* task_flags,
                               uint32_t* status, hipStream_t stream);
hipError_t launch_clear_words(uint32_t* words, uint32_t count, hipStream_t stream);
hipError_t launch_combine(const float* route_output, const uint32_t* inverse,
                          const uint16_t* shared_output, const uint16_t* shared_gate,
                          uint32_t tokens, uint16_t* output, hipStream_t stream);
hipError_t launch_combine_shared(const uint16_t* routed, const uint16_t* shared,
                                 const uint16_t* gate, uint16_t* output,
                                 uint32_t tokens, hipStream_t stream);

// decode (q38m_decode.hip)
size_t decode_scratch_bytes();
size_t decode_block_scratch_bytes();
// the whole MoE block of one decode step: router GEMV, routed experts and
// the bf16 shared expert (shared intermediate kInter) in three launches
hipError_t launch_decode_block(const q38m_expert_weights_v1& gate_up,
                               const q38m_expert_weights_v1& down, const uint16_t* hidden,
                               const uint16_t* router, const uint16_t* w_gate,
                               const uint16_t* w_up, const uint16_t* w_down,
                               const uint16_t* w_out_gate, uint32_t top_k,
                               const uint16_t* residual, void* scratch, uint16_t* output,
                               hipStream_t stream);
// logits != null: top-k inside the gate/up launch; else ids/weights given
hipError_t launch_decode(const q38m_expert_weights_v1& gate_up,
                         const q38m_expert_weights_v1& down, const uint16_t* hidden,
                         const float* logits, const int32_t* ids, const float* weights,
                         uint32_t top_k, const uint16_t* shared_output,
                         const uint16_t* shared_gate, const uint16_t* residual, void* scratch,
                         uint16_t* output, hipStream_t stream);

// dense bf16 GEMMs (q38m_dense.hip): C = A * B^T, K contiguous in both
hipError_t launch_dense_gemm(const uint16_t* a, const uint16_t* b, uint32_t m, uint32_t n,
                             uint32_t k, float* c_f32, uint16_t* c_bf16, hipStream_t stream);
// C = act(bf16(A * B^T)): silu or sigmoid of the bf16 product / divisor, * scale
hipError_t launch_dense_gemm_act(const uint16_t* a, const uint16_t* b, uint32_t m, uint32_t n,
                                 uint32_t k, bool silu, float divisor, float scale,
                                 uint16_t* c_bf16, hipStream_t stream);
// router logits with the top-10 selection: level 1 in the GEMM epilogue,
// level 2 in a second launch; the workspace holds the candidate keys
size_t router_topk_workspace_bytes(uint32_t tokens);
hipError_t launch_router_topk(const uint16_t* hidden, const uint16_t* router, uint32_t tokens,
                              uint32_t top_k, void* workspace, int32_t* ids, float* weights,
                              hipStream_t stream);
size_t shared_expert_scratch_bytes(uint32_t tokens, uint32_t inter);
hipError_t launch_shared_expert(const uint16_t* hidden, const uint16_t* w_gate,
                                const uint16_t* w_up, const uint16_t* w_down,
                                const uint16_t* w_out_gate, uint32_t tokens, uint32_t inter,
                                void* scratch, uint16_t* shared_output, uint16_t* shared_gate,
                                hipStream_t stream);

// hyper-connection prepare/finish (q38m_hyper.hip); hidden % 8 == 0
hipError_t launch_hyper_repeat(const uint16_t* embedding, uint16_t* hyper, uint32_t tokens,
                               uint32_t hidden, hipStream_t stream);
hipError_t launch_hyper_norm(const uint16_t* hyper, const uint16_t* weight,
                             const uint16_t* inject, uint32_t tokens, uint32_t hidden,
                             uint16_t* normalized, uint16_t* injection, hipStream_t stream);
hipError_t launch_hyper_elementwise(const uint16_t* in, uint16_t* out, uint64_t elements,
                                    float divisor, float scale, bool silu, hipStream_t stream);
hipError_t launch_hyper_mix(const uint16_t* normalized, const uint16_t* mix, uint16_t* mixed,
                            uint32_t tokens, uint32_t hidden, hipStream_t stream);
hipError_t launch_hyper_inject(const uint16_t* original, const uint16_t* block,
                               const uint16_t* injection, uint16_t* output, uint32_t tokens,
                               uint32_t hidden, hipStream_t stream);
size_t hyper_prepare_scratch_bytes(uint32_t tokens, uint32_t hidden, uint32_t low_rank);
hipError_t launch_hyper_prepare(const uint16_t* hyper, const uint16_t* norm_weight,
                                const uint16_t* mix_down, const uint16_t* mix_up,
                                const uint16_t* inject, uint32_t tokens, uint32_t hidden,
                                uint32_t low_rank, void* scratch, uint16_t* mixed,
                                uint16_t* injection, hipStream_t stream);

// layout and synthetic data (q38m_layout.hip)
hipError_t launch_repack(const q38m_expert_weights_v1& src,
                         const q38m_expert_weights_v1& dst, hipStream_t stream);
// bf16 [experts*rows][columns] -> dst (row-major, fp16 scales)
hipError_t launch_quantize_weights(const uint16_t* src, const q38m_expert_weights_v1& dst,
                                  hipStream_t stream);
hipError_t launch_synth(uint32_t kind, uint64_t seed, uint64_t tag, uint64_t count,
                        float sigma, int32_t lo, int32_t hi, const float* bias,
                        uint32_t bias_len, void* out, hipStream_t stream);

}  // namespace q38m
