// C++ wrapper over the q38m C ABI with the reference's function names,
// argument order and error behaviour (include/q38/cuda_moe_prefill.h:98-133,
// include/q38/cuda_moe.h:17-39, include/q38/cuda_kernels.h:83-91): invalid
// arguments throw std::invalid_argument, device failures throw
// std::runtime_error (cuda/q38_moe_prefill.cu:33-68).
//
// A caller of the reference switches by including this header and
// qualifying calls with q38m:: instead of q38::, with these differences
// (the activation format of this data plane is int8 per token, not bf16):
//  - cuda_moe_grouped_gate_up_v1 takes the int8 token rows xq[T][2048] and
//    their scales xs[T] (from q38m_moe_route_quantize_v1 or
//    quantize_rows_i8) instead of the packed bf16 rows of
//    cuda_moe_pack_hidden_v1; it gathers the rows through
//    packed_assignment itself, so the pack step is not needed;
//  - cuda_moe_grouped_down_v1 takes weighted_mid quantised to int8 rows
//    (one quantize_rows_i8 call between gate/up and down);
//  - expert tensors are q38m_expert_weights_v1 descriptors in the MFMA16
//    device layouts instead of CudaTensorViewV1;
//  - cuda_moe_routed_bf16 serves tokens == 1 only (the legacy route-wise
//    atomic path for tokens > 1 is not built);
//  - both grouped modes are accepted and the legacy atomic mode is
//    rejected, as validate_grouped_mode does.
#ifndef Q38M_HPP
#define Q38M_HPP

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "q38m.h"

namespace q38m {

using Q38ExpertMmqTaskV1 = q38m_task_v1;
using Q38RoutePlanHeaderV1 = q38m_route_plan_header_v1;
using Q38RoutePlanStorageV1 = q38m_route_plan_v1;
using ExpertWeightsV1 = q38m_expert_weights_v1;
using PrefillWorkspaceV1 = q38m_prefill_workspace_v1;

// Q38PrefillMoeModeV1, include/q38/cuda_moe_prefill.h:67-71
enum class Q38PrefillMoeModeV1 : std::uint32_t {
    kGroupedMmq = Q38M_MOE_MODE_GROUPED_MMQ,
    kGroupedMmqSafe = Q38M_MOE_MODE_GROUPED_MMQ_SAFE,
    kLegacyAtomicDiagnostic = Q38M_MOE_MODE_LEGACY_ATOMIC_DIAGNOSTIC,
};

static_assert(sizeof(Q38ExpertMmqTaskV1) == 8, "Q38ExpertMmqTaskV1 ABI changed");
static_assert(sizeof(Q38RoutePlanHeaderV1) == 64, "Q38RoutePlanHeaderV1 ABI changed");

inline void check(int status) {
    if (status == Q38M_OK) return;
    const std::string message = q38m_last_error();
    if (status == Q38M_ERR_INVALID_ARGUMENT || status == Q38M_ERR_UNSUPPORTED)
        throw std::invalid_argument(message);
    throw std::runtime_error(message);
}

constexpr std::uint32_t q38_moe_prefill_routes_v1(std::uint32_t tokens) {
    return tokens * Q38M_ROUTE_TOPK;
}

constexpr std::uint32_t q38_moe_prefill_max_tasks_v1(std::uint32_t tokens) {
    return (tokens * Q38M_ROUTE_TOPK < Q38M_ROUTE_EXPERTS ? tokens * Q38M_ROUTE_TOPK
                                                           : Q38M_ROUTE_EXPERTS) +
           (tokens * Q38M_ROUTE_TOPK -
            (tokens * Q38M_ROUTE_TOPK < Q38M_ROUTE_EXPERTS ? tokens * Q38M_ROUTE_TOPK
                                                            : Q38M_ROUTE_EXPERTS)) /
               Q38M_MMQ_M;
}

constexpr std::size_t q38_moe_route_plan_bytes_v1(std::uint32_t tokens) {
    return sizeof(Q38RoutePlanHeaderV1) + Q38M_ROUTE_EXPERTS * sizeof(std::uint16_t) +
           2 * (Q38M_ROUTE_EXPERTS + 1) * sizeof(std::uint32_t) +
           2 * static_cast<std::size_t>(q38_moe_prefill_routes_v1(tokens)) *
               sizeof(std::uint32_t) +
           q38_moe_prefill_max_tasks_v1(tokens) * sizeof(Q38ExpertMmqTaskV1);
}

inline Q38RoutePlanStorageV1 cuda_moe_route_plan_storage_v1(void* allocation,
                                                            std::size_t allocation_bytes,
                                                            std::uint32_t tokens) {
    Q38RoutePlanStorageV1 plan{};
    check(q38m_moe_route_plan_storage_v1(allocation, allocation_bytes, tokens, &plan));
    return plan;
}

// The reference always computes the FNV hashes; so does this wrapper.  The
// fast path (q38m_moe_prefill_v1) skips them.
inline void cuda_moe_build_route_plan_v1(const std::int32_t* expert_ids, std::uint32_t tokens,
                                         Q38RoutePlanStorageV1 plan, void* stream, int device) {
    check(q38m_moe_build_route_plan_v1(expert_ids, tokens, &plan, Q38M_PLAN_FLAG_HASHES, stream,
                                       device));
}

inline void cuda_moe_pack_hidden_v1(const std::uint16_t* hidden,
                                    const std::uint32_t* packed_assignment,
                                    std::uint32_t routes, std::uint16_t* packed_hidden,
                                    void* stream, int device) {
    check(q38m_moe_pack_hidden_v1(hidden, packed_assignment, routes, Q38M_HIDDEN, packed_hidden,
                                  stream, device));
}

inline void quantize_rows_i8(const std::uint16_t* x, std::uint32_t rows, std::uint32_t width,
                             std::int8_t* q, float* scales, void* stream, int device) {
    check(q38m_quantize_rows_i8(x, rows, width, q, scales, stream, device));
}

inline void cuda_moe_grouped_gate_up_v1(const ExpertWeightsV1& gate_up_experts,
                                        const std::int8_t* xq, const float* xs,
                                        const std::uint32_t* packed_assignment,
                                        const float* token_rank_weights,
                                        const Q38ExpertMmqTaskV1* tasks,
                                        std::uint32_t task_count, std::uint16_t* weighted_mid,
                                        Q38PrefillMoeModeV1 mode, void* stream, int device) {
    check(q38m_moe_grouped_gate_up_v1(&gate_up_experts, xq, xs, packed_assignment,
                                      token_rank_weights, tasks, task_count, weighted_mid,
                                      static_cast<std::uint32_t>(mode), stream, device));
}

inline void cuda_moe_grouped_down_v1(const ExpertWeightsV1& down_experts,
                                     const std::int8_t* mid_q, const float* mid_scales,
                                     const Q38ExpertMmqTaskV1* tasks, std::uint32_t task_count,
                                     float* route_output, Q38PrefillMoeModeV1 mode, void* stream,
                                     int device) {
    check(q38m_moe_grouped_down_v1(&down_experts, mid_q, mid_scales, tasks, task_count,
                                   route_output, static_cast<std::uint32_t>(mode), stream,
                                   device));
}

// No reference counterpart: the gate/up, mid quantisation and down calls
// above as one (one launch for W4 gate/up with per-channel W8 down), same
// results; task_flags (9 * task_count words) zero on entry, see q38m.h.
inline void moe_clear_task_flags_v1(std::uint32_t* task_flags, std::uint32_t task_count,
                                    void* stream, int device) {
    check(q38m_moe_clear_task_flags_v1(task_flags, task_count, stream, device));
}

inline void moe_grouped_gate_up_down_v1(const ExpertWeightsV1& gate_up_experts,
                                        const ExpertWeightsV1& down_experts,
                                        const std::int8_t* xq, const float* xs,
                                        const std::uint32_t* packed_assignment,
                                        const float* token_rank_weights,
                                        const Q38ExpertMmqTaskV1* tasks,
                                        std::uint32_t task_count, std::uint16_t* weighted_mid,
                                        std::int8_t* mid_q, float* mid_scales,
                                        std::uint32_t* task_flags, std::uint32_t* plan_status,
                                        float* route_output, Q38PrefillMoeModeV1 mode,
                                        void* stream, int device) {
    check(q38m_moe_grouped_gate_up_down_v1(&gate_up_experts, &down_experts, xq, xs,
                                           packed_assignment, token_rank_weights, tasks,
                                           task_count, weighted_mid, mid_q, mid_scales,
                                           task_flags, plan_status, route_output,
                                           static_cast<std::uint32_t>(mode), stream, device));
}

inline void cuda_moe_reduce_top10_and_combine_shared_v1(
    const float* route_output, const std::uint32_t* assignment_to_packed,
    const std::uint16_t* shared_output, const std::uint16_t* shared_gate, std::uint32_t tokens,
    std::uint16_t* output, void* stream, int device) {
    check(q38m_moe_reduce_top10_and_combine_shared_v1(route_output, assignment_to_packed,
                                                      shared_output, shared_gate, tokens,
                                                      output, stream, device));
}

// tokens == 1 branch of cuda_moe_routed_bf16; the scratch replaces the
// reference's gate_up/activated/accumulation scratch buffers.
inline void cuda_moe_routed_bf16(const ExpertWeightsV1& gate_up_experts,
                                 const ExpertWeightsV1& down_experts,
                                 const std::uint16_t* hidden, const std::int32_t* expert_ids,
                                 const float* expert_weights, std::uint32_t tokens,
                                 std::uint32_t top_k, void* scratch,
                                 std::uint16_t* routed_output, void* stream, int device) {
    if (tokens != 1)
        throw std::invalid_argument(
            "q38m routed MoE handles tokens == 1; use the grouped prefill path");
    check(q38m_moe_routed_decode_v1(&gate_up_experts, &down_experts, hidden, expert_ids,
                                    expert_weights, top_k, scratch, routed_output, stream,
                                    device));
}

// Fused tokens == 1 MoE step from fp32 router logits: top-k, routed experts
// and the optional gated shared term (and residual), in two launches.
inline void moe_decode(const q38m_expert_weights_v1& gate_up_experts,
                       const q38m_expert_weights_v1& down_experts, const std::uint16_t* hidden,
                       const float* logits, std::uint32_t top_k,
                       const std::uint16_t* shared_output, const std::uint16_t* shared_gate,
                       const std::uint16_t* residual, void* scratch, std::uint16_t* output,
                       void* stream, int device) {
    check(q38m_moe_decode_v1(&gate_up_experts, &down_experts, hidden, logits, top_k,
                             shared_output, shared_gate, residual, scratch, output, stream,
                             device));
}

inline void cuda_moe_combine_shared_bf16(const std::uint16_t* routed_output,
                                         const std::uint16_t* shared_output,
                                         const std::uint16_t* shared_gate,
                                         std::uint16_t* output, std::uint32_t tokens,
                                         void* stream, int device) {
    check(q38m_moe_combine_shared_bf16(routed_output, shared_output, shared_gate, output, tokens,
                                       stream, device));
}

// cuda_topk_router_bf16 (include/q38/cuda_kernels.h:83-91): same name and
// arguments as the reference.
inline void cuda_topk_router_bf16(const std::uint16_t* logits, std::int32_t* expert_ids,
                                  float* expert_weights, std::uint32_t tokens,
                                  std::uint32_t experts, std::uint32_t top_k,
                                  bool normalize_top_k, void* stream, int device) {
    check(q38m_topk_router_bf16(logits, expert_ids, expert_weights, tokens, experts, top_k,
                                normalize_top_k ? 1 : 0, stream, device));
}

// Router top-k over fp32 logits (the BASELINE router output).
inline void cuda_topk_router_f32(const float* logits, std::int32_t* expert_ids,
                                 float* expert_weights, std::uint32_t tokens,
                                 std::uint32_t experts, std::uint32_t top_k,
                                 bool normalize_top_k, void* stream, int device) {
    check(q38m_topk_router_f32(logits, expert_ids, expert_weights, tokens, experts, top_k,
                               normalize_top_k ? 1 : 0, stream, device));
}

// The whole run_moe step for one slab (cuda/cuda_backend.cu:1523-1601).
inline void run_moe_prefill(const ExpertWeightsV1& gate_up, const ExpertWeightsV1& down,
                            const std::uint16_t* hidden, const float* logits,
                            std::uint32_t tokens, const PrefillWorkspaceV1& workspace,
                            const std::uint16_t* shared_output,
                            const std::uint16_t* shared_gate, std::uint16_t* output,
                            void* stream, int device) {
    check(q38m_moe_prefill_v1(&gate_up, &down, hidden, logits, tokens, &workspace,
                              shared_output, shared_gate, output, stream, device));
}

// Router logits (cuda_backend.cu:1518-1519): fp32 [tokens][512] from
// hidden rows of hidden_width (must be 2048) values.
// The whole MoE block of one decode step (run_moe's tokens == 1 branch,
// cuda_backend.cu:1516-1605): router GEMV, routed experts, bf16 shared
// expert, gated combine and optional residual in three launches; equal to
// moe_router + moe_shared_expert + moe_decode bit for bit.
inline void moe_decode_block(const q38m_expert_weights_v1& gate_up_experts,
                             const q38m_expert_weights_v1& down_experts,
                             const std::uint16_t* hidden, const std::uint16_t* router,
                             const std::uint16_t* w_gate, const std::uint16_t* w_up,
                             const std::uint16_t* w_down, const std::uint16_t* w_out_gate,
                             std::uint32_t shared_inter, std::uint32_t top_k,
                             const std::uint16_t* residual, void* scratch,
                             std::uint16_t* output, void* stream, int device) {
    check(q38m_moe_decode_block_v1(&gate_up_experts, &down_experts, hidden, router, w_gate,
                                   w_up, w_down, w_out_gate, shared_inter, top_k, residual,
                                   scratch, output, stream, device));
}

inline void moe_router(const std::uint16_t* hidden, const std::uint16_t* router,
                       std::uint32_t tokens, std::uint32_t hidden_width, float* logits,
                       void* stream, int device) {
    check(q38m_moe_router_v1(hidden, router, tokens, hidden_width, logits, stream, device));
}

// Shared expert (cuda_backend.cu:1573-1590): shared_output bf16 [tokens][2048]
// and shared_gate bf16 [tokens] for the gated combine.
inline void moe_shared_expert(const std::uint16_t* hidden, const std::uint16_t* w_gate,
                              const std::uint16_t* w_up, const std::uint16_t* w_down,
                              const std::uint16_t* w_out_gate, std::uint32_t tokens,
                              std::uint32_t hidden_width, std::uint32_t inter, void* scratch,
                              std::uint16_t* shared_output, std::uint16_t* shared_gate,
                              void* stream, int device) {
    check(q38m_moe_shared_expert_v1(hidden, w_gate, w_up, w_down, w_out_gate, tokens,
                                    hidden_width, inter, scratch, shared_output, shared_gate,
                                    stream, device));
}

inline bool cuda_q38_moe_prefill_compiled() { return q38m_moe_compiled() == 1; }
inline bool cuda_q38_moe_compiled() { return q38m_moe_compiled() == 1; }

}  // namespace q38m

#endif
