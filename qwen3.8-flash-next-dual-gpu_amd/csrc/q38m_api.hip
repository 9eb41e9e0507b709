// C ABI of the q38m MoE data plane: argument validation, device selection,
// error reporting and launch sequencing.  Kernels live in the other
// translation units behind q38m_internal.h.
//
// Validation mirrors the reference host wrappers
// (cuda/q38_moe_prefill.cu:33-68, :635-866; cuda/q38_moe.cu:352-501):
// invalid arguments return Q38M_ERR_INVALID_ARGUMENT (the reference throws
// std::invalid_argument), launch failures Q38M_ERR_DEVICE (std::runtime_error).
#include <stdint.h>

#include <string>

#include "q38m_internal.h"

#include <atomic>
#include <initializer_list>
#include <mutex>

#ifdef Q38M_CHECKED
#include <vector>

#include "q38m_checked.h"

namespace q38m {
using CheckedReader = hipError_t (*)(uint32_t*, int, hipStream_t);
// every translation unit's status-word reader (q38m_device.h), registered
// at load
std::vector<CheckedReader>& checked_readers() {
    static std::vector<CheckedReader> readers;
    return readers;
}
bool register_checked_status(CheckedReader read) {
    checked_readers().push_back(read);
    return true;
}
}  // namespace q38m
#endif

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* message) {
    g_last_error = message;
    return code;
}

int device_fail(hipError_t status, const char* operation) {
    g_last_error = std::string(operation) + ": " + hipGetErrorString(status);
    return Q38M_ERR_DEVICE;
}

int select_device(int device) {
    if (device < 0) return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid q38m device");
    const hipError_t status = hipSetDevice(device);
    if (status != hipSuccess) return device_fail(status, "hipSetDevice(q38m)");
    return Q38M_OK;
}

int finish(hipError_t status, const char* operation) {
    if (status != hipSuccess) return device_fail(status, operation);
    g_last_error.clear();
    return Q38M_OK;
}

hipStream_t as_stream(void* stream) { return reinterpret_cast<hipStream_t>(stream); }

bool aligned(const void* p, uintptr_t alignment) {
    return (reinterpret_cast<uintptr_t>(p) % alignment) == 0u;
}

// every pointer non-null and 16-byte aligned
bool all16(std::initializer_list<const void*> ptrs) {
    for (const void* p : ptrs)
        if (!p || !aligned(p, 16)) return false;
    return true;
}

size_t align_up(size_t value, size_t alignment) {
    return (value + alignment - 1u) / alignment * alignment;
}

bool valid_plan(const q38m_route_plan_v1* plan) {
    return plan && plan->header && plan->expert_counts && plan->expert_offsets &&
           plan->expert_task_offsets && plan->packed_assignment &&
           plan->assignment_to_packed && plan->tasks;
}

// Shape/format checks of validate_expert_tensor (q38_moe_prefill.cu:51-62)
// for this build's formats.
bool valid_scale_dtype(uint32_t dtype) {
    return dtype == Q38M_SCALE_F16 || dtype == Q38M_SCALE_BF16;
}
bool w4_group(uint32_t g) { return g == 32u || g == 64u || g == 128u; }

bool w8_group(uint32_t g) { return g == 0u || g == 64u || g == 128u; }

bool valid_gate_up(const q38m_expert_weights_v1* w) {
    return w && w->data && w->scales && aligned(w->data, 16) && aligned(w->scales, 8) &&
           ((w->format == Q38M_FORMAT_W4_SYM && w4_group(w->group_size)) ||
            (w->format == Q38M_FORMAT_W8_SYM && w8_group(w->group_size))) &&
           valid_scale_dtype(w->scale_dtype) && w->layout == Q38M_LAYOUT_MFMA16_PAIRED &&
           w->experts == Q38M_ROUTE_EXPERTS && w->rows == 2u * Q38M_INTERMEDIATE &&
           w->columns == Q38M_HIDDEN;
}

bool valid_down(const q38m_expert_weights_v1* w) {
    if (!w || !w->data || !w->scales || !aligned(w->data, 16) || !aligned(w->scales, 8) ||
        !valid_scale_dtype(w->scale_dtype) || w->layout != Q38M_LAYOUT_MFMA16 ||
        w->experts != Q38M_ROUTE_EXPERTS || w->rows != Q38M_HIDDEN ||
        w->columns != Q38M_INTERMEDIATE)
        return false;
    return (w->format == Q38M_FORMAT_W8_SYM &&
            (w->group_size == 0u || w->group_size == 64u || w->group_size == 128u)) ||
           (w->format == Q38M_FORMAT_W4_SYM && w4_group(w->group_size));
}

// validate_grouped_mode (cuda/q38_moe_prefill.cu:64-68)
bool valid_grouped_mode(uint32_t mode) {
    return mode == Q38M_MOE_MODE_GROUPED_MMQ || mode == Q38M_MOE_MODE_GROUPED_MMQ_SAFE;
}

int check_weights(const q38m_expert_weights_v1* w, bool gate_up) {
    if (w && w->layout == Q38M_LAYOUT_ROW_MAJOR)
        return fail(Q38M_ERR_UNSUPPORTED,
                    "q38m kernels read the MFMA16 layouts (gate/up: MFMA16_PAIRED); convert with "
                    "q38m_repack_expert_weights");
    if (gate_up ? !valid_gate_up(w) : !valid_down(w))
        return fail(Q38M_ERR_INVALID_ARGUMENT,
                    gate_up ? "invalid grouped gate/up expert tensor"
                            : "invalid grouped down expert tensor");
    return Q38M_OK;
}

}  // namespace

extern "C" {

uint32_t q38m_moe_prefill_routes_v1(uint32_t tokens) { return q38m::routes_v1(tokens); }

uint32_t q38m_moe_prefill_max_tasks_v1(uint32_t tokens) { return q38m::max_tasks_v1(tokens); }

namespace {
// The V1 plan's views in one allocation (cuda/q38_moe_prefill.cu:635-663);
// the chunk plan uses the same order with its own task count after them.
void bind_plan_views(void* allocation, uint32_t tokens, q38m_route_plan_v1* out) {
    uint8_t* cursor = static_cast<uint8_t*>(allocation);
    const size_t routes = q38m::routes_v1(tokens);
    out->header = reinterpret_cast<q38m_route_plan_header_v1*>(cursor);
    cursor += sizeof(q38m_route_plan_header_v1);
    out->expert_counts = reinterpret_cast<uint16_t*>(cursor);
    cursor += Q38M_ROUTE_EXPERTS * sizeof(uint16_t);
    out->expert_offsets = reinterpret_cast<uint32_t*>(cursor);
    cursor += (Q38M_ROUTE_EXPERTS + 1u) * sizeof(uint32_t);
    out->expert_task_offsets = reinterpret_cast<uint32_t*>(cursor);
    cursor += (Q38M_ROUTE_EXPERTS + 1u) * sizeof(uint32_t);
    out->packed_assignment = reinterpret_cast<uint32_t*>(cursor);
    cursor += routes * sizeof(uint32_t);
    out->assignment_to_packed = reinterpret_cast<uint32_t*>(cursor);
    cursor += routes * sizeof(uint32_t);
    out->tasks = reinterpret_cast<q38m_task_v1*>(cursor);
}

}  // namespace

size_t q38m_moe_route_plan_bytes_v1(uint32_t tokens) {
    const size_t routes = q38m::routes_v1(tokens);
    return sizeof(q38m_route_plan_header_v1) + Q38M_ROUTE_EXPERTS * sizeof(uint16_t) +
           2u * (Q38M_ROUTE_EXPERTS + 1u) * sizeof(uint32_t) + 2u * routes * sizeof(uint32_t) +
           static_cast<size_t>(q38m::max_tasks_v1(tokens)) * sizeof(q38m_task_v1);
}

int q38m_moe_route_plan_storage_v1(void* allocation, size_t allocation_bytes, uint32_t tokens,
                                   q38m_route_plan_v1* out) {
    if (!out || !allocation || tokens == 0 || tokens > Q38M_PREFILL_SLAB_MAX_TOKENS)
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid prefill MoE route-plan allocation");
    if (allocation_bytes < q38m_moe_route_plan_bytes_v1(tokens))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "prefill MoE route-plan allocation is too small");
    if (!aligned(allocation, alignof(q38m_route_plan_header_v1)))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "prefill MoE route-plan allocation is unaligned");
    bind_plan_views(allocation, tokens, out);
    g_last_error.clear();
    return Q38M_OK;
}

int q38m_topk_router_f32(const float* logits, int32_t* expert_ids, float* expert_weights,
                         uint32_t tokens, uint32_t experts, uint32_t top_k,
                         int normalize_top_k, void* stream, int device) {
    if (!logits || !expert_ids || !expert_weights || tokens == 0 || experts == 0 ||
        experts % 64u != 0u || experts > 1024u || top_k == 0 || top_k > experts || top_k > 32u)
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid top-k router buffers");
    if (int rc = select_device(device)) return rc;
    if (experts == Q38M_ROUTE_EXPERTS && top_k <= Q38M_ROUTE_TOPK && normalize_top_k)
        return finish(q38m::launch_route_quantize(logits, nullptr, tokens, top_k, expert_ids,
                                                  expert_weights, nullptr, nullptr,
                                                  as_stream(stream)),
                      "route_quantize_kernel");
    return finish(q38m::launch_topk(logits, expert_ids, expert_weights, tokens, experts, top_k,
                                    normalize_top_k, as_stream(stream)),
                  "topk_kernel");
}

int q38m_topk_router_bf16(const uint16_t* logits, int32_t* expert_ids, float* expert_weights,
                          uint32_t tokens, uint32_t experts, uint32_t top_k,
                          int normalize_top_k, void* stream, int device) {
    if (!logits || !expert_ids || !expert_weights || tokens == 0 || experts == 0 ||
        experts % 64u != 0u || experts > 1024u || top_k == 0 || top_k > experts || top_k > 32u)
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid top-k router buffers");
    if (int rc = select_device(device)) return rc;
    if (experts == Q38M_ROUTE_EXPERTS && top_k <= Q38M_ROUTE_TOPK && normalize_top_k)
        return finish(q38m::launch_route_bf16(logits, tokens, top_k, expert_ids, expert_weights,
                                              as_stream(stream)),
                      "route_quantize_kernel");
    return finish(q38m::launch_topk(logits, expert_ids, expert_weights, tokens, experts, top_k,
                                    normalize_top_k, as_stream(stream)),
                  "topk_kernel");
}

int q38m_moe_route_quantize_v1(const float* logits, const uint16_t* hidden, uint32_t tokens,
                               int32_t* expert_ids, float* expert_weights, int8_t* xq, float* xs,
                               void* stream, int device) {
    if (!logits || !hidden || !expert_ids || !expert_weights || !xq || !xs || tokens == 0 ||
        !aligned(logits, 16) || !aligned(hidden, 16) || !aligned(xq, 8))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid route/quantise buffers");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_route_quantize(logits, hidden, tokens, Q38M_ROUTE_TOPK, expert_ids,
                                              expert_weights, xq, xs, as_stream(stream)),
                  "route_quantize_kernel");
}

int q38m_moe_build_route_plan_v1(const int32_t* expert_ids, uint32_t tokens,
                                 const q38m_route_plan_v1* plan, uint32_t flags, void* stream,
                                 int device) {
    if (!expert_ids || tokens == 0 || tokens > Q38M_PREFILL_SLAB_MAX_TOKENS ||
        (flags & ~Q38M_PLAN_FLAG_HASHES) != 0u)
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid prefill MoE route-plan input");
    if (!valid_plan(plan))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "incomplete prefill MoE route-plan storage");
    if (!aligned(plan->tasks, 8) || !aligned(plan->header, 16))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "unaligned prefill MoE route-plan storage");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_build_plan(expert_ids, tokens, *plan,
                                          (flags & Q38M_PLAN_FLAG_HASHES) != 0u,
                                          as_stream(stream)),
                  "build_plan_kernel");
}

int q38m_moe_pack_hidden_v1(const uint16_t* hidden, const uint32_t* packed_assignment,
                            uint32_t routes, uint32_t hidden_width, uint16_t* packed_hidden,
                            void* stream, int device) {
    if (!hidden || !packed_assignment || routes == 0 ||
        routes > Q38M_PREFILL_SLAB_MAX_TOKENS * Q38M_ROUTE_TOPK || routes % Q38M_ROUTE_TOPK != 0 ||
        hidden_width == 0 || hidden_width % 8u != 0u || !packed_hidden || !aligned(hidden, 16) ||
        !aligned(packed_hidden, 16))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid prefill MoE hidden-pack input");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_pack_hidden(hidden, packed_assignment, routes, hidden_width,
                                           packed_hidden, as_stream(stream)),
                  "pack_hidden_kernel");
}

int q38m_quantize_rows_i8(const uint16_t* x, uint32_t rows, uint32_t width, int8_t* q,
                          float* scales, void* stream, int device) {
    if (!x || !q || !scales || rows == 0 ||
        (width != 512u && width != 1024u && width != 2048u && width != 4096u) ||
        !aligned(x, 16) || !aligned(q, 8))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid int8 row quantisation input");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_quantize_rows(x, rows, width, q, scales, as_stream(stream)),
                  "quantize_rows_kernel");
}

int q38m_residual_add_bf16(const uint16_t* a, const uint16_t* b, uint16_t* out,
                           uint64_t elements, void* stream, int device) {
    if (!a || !b || !out || elements == 0 || elements % 8u != 0u || !aligned(a, 16) ||
        !aligned(b, 16) || !aligned(out, 16))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid residual add input");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_residual_add(a, b, out, elements, as_stream(stream)),
                  "residual_add_kernel");
}

int q38m_moe_grouped_gate_up_v1(const q38m_expert_weights_v1* gate_up, const int8_t* xq,
                                const float* xs, const uint32_t* packed_assignment,
                                const float* token_rank_weights, const q38m_task_v1* tasks,
                                uint32_t task_count, uint16_t* weighted_mid, uint32_t mode,
                                void* stream, int device) {
    if (!valid_grouped_mode(mode))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid grouped prefill MoE mode");
    if (int rc = check_weights(gate_up, true)) return rc;
    if (!xq || !xs || !packed_assignment || !token_rank_weights || !tasks || task_count == 0 ||
        task_count > q38m::max_tasks_v1(Q38M_PREFILL_SLAB_MAX_TOKENS) || !weighted_mid ||
        !aligned(xq, 8) || !aligned(tasks, 8))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid grouped prefill gate/up input");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_gate_up(*gate_up, xq, xs, packed_assignment, token_rank_weights,
                                       tasks, task_count, weighted_mid, as_stream(stream)),
                  "grouped gate/up kernel");
}

int q38m_moe_grouped_down_v1(const q38m_expert_weights_v1* down, const int8_t* mid_q,
                             const float* mid_scales, const q38m_task_v1* tasks,
                             uint32_t task_count, float* route_output, uint32_t mode,
                             void* stream, int device) {
    if (!valid_grouped_mode(mode))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid grouped prefill MoE mode");
    if (int rc = check_weights(down, false)) return rc;
    if (!mid_q || !mid_scales || !tasks || task_count == 0 ||
        task_count > q38m::max_tasks_v1(Q38M_PREFILL_SLAB_MAX_TOKENS) || !route_output ||
        !aligned(mid_q, 16) || !aligned(tasks, 8))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid grouped prefill down input");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_down(*down, mid_q, mid_scales, tasks, task_count, route_output,
                                    as_stream(stream)),
                  "grouped down kernel");
}

int q38m_moe_grouped_gate_up_down_v1(const q38m_expert_weights_v1* gate_up,
                                     const q38m_expert_weights_v1* down, const int8_t* xq,
                                     const float* xs, const uint32_t* packed_assignment,
                                     const float* token_rank_weights,
                                     const q38m_task_v1* tasks, uint32_t task_count,
                                     uint16_t* weighted_mid, int8_t* mid_q, float* mid_scales,
                                     uint32_t* task_flags, uint32_t* plan_status,
                                     float* route_output, uint32_t mode, void* stream,
                                     int device) {
    if (!valid_grouped_mode(mode))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid grouped prefill MoE mode");
    if (int rc = check_weights(gate_up, true)) return rc;
    if (int rc = check_weights(down, false)) return rc;
    if (!xq || !xs || !packed_assignment || !token_rank_weights || !tasks || task_count == 0 ||
        task_count > q38m::max_tasks_v1(Q38M_PREFILL_SLAB_MAX_TOKENS) || !weighted_mid ||
        !mid_q || !mid_scales || !task_flags || !plan_status || !route_output ||
        !aligned(xq, 8) || !aligned(tasks, 8) || !aligned(mid_q, 16) || !aligned(task_flags, 4) ||
        !aligned(plan_status, 4))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid grouped prefill gate/up + down input");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_gate_up_down(*gate_up, *down, xq, xs, packed_assignment,
                                            token_rank_weights, tasks, task_count, weighted_mid,
                                            mid_q, mid_scales, route_output, task_flags,
                                            plan_status, as_stream(stream)),
                  "grouped gate/up + down kernels");
}

int q38m_moe_clear_task_flags_v1(uint32_t* task_flags, uint32_t task_count, void* stream,
                                 int device) {
    if (!task_flags || task_count == 0 ||
        task_count > q38m::max_tasks_v1(Q38M_PREFILL_SLAB_MAX_TOKENS) || !aligned(task_flags, 4))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid task-flag clear input");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_clear_words(task_flags, q38m::task_flag_words(task_count),
                                           as_stream(stream)),
                  "clear_words_kernel");
}

int q38m_moe_reduce_top10_and_combine_shared_v1(const float* route_output,
                                                const uint32_t* assignment_to_packed,
                                                const uint16_t* shared_output,
                                                const uint16_t* shared_gate, uint32_t tokens,
                                                uint16_t* output, void* stream, int device) {
    if (!route_output || !assignment_to_packed || (shared_output == nullptr) != (shared_gate == nullptr) ||
        tokens == 0 || tokens > Q38M_PREFILL_SLAB_MAX_TOKENS || !output ||
        !aligned(route_output, 16) || !aligned(output, 16) ||
        (shared_output && !aligned(shared_output, 16)))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid grouped prefill reduction input");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_combine(route_output, assignment_to_packed, shared_output,
                                       shared_gate, tokens, output, as_stream(stream)),
                  "combine_kernel");
}

int q38m_moe_combine_shared_bf16(const uint16_t* routed_output, const uint16_t* shared_output,
                                 const uint16_t* shared_gate, uint16_t* output, uint32_t tokens,
                                 void* stream, int device) {
    if (!routed_output || !shared_output || !shared_gate || !output || tokens == 0)
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid shared MoE buffers");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_combine_shared(routed_output, shared_output, shared_gate, output,
                                              tokens, as_stream(stream)),
                  "combine_shared_kernel");
}

size_t q38m_moe_prefill_workspace_bytes(uint32_t tokens) {
    if (tokens == 0 || tokens > Q38M_PREFILL_SLAB_MAX_TOKENS) return 0;
    // plan, ids, weights, xq, xs, weighted_mid, mid_q, mid_s, route_output,
    // task_flags
    return q38m::prefill_workspace_bytes_v1(tokens);
}

int q38m_moe_prefill_workspace_bind(void* allocation, size_t bytes, uint32_t tokens,
                                    q38m_prefill_workspace_v1* out) {
    if (!allocation || !out || tokens == 0 || tokens > Q38M_PREFILL_SLAB_MAX_TOKENS ||
        bytes < q38m_moe_prefill_workspace_bytes(tokens) || !aligned(allocation, 256))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid prefill MoE workspace allocation");
    const size_t routes = q38m::routes_v1(tokens);
    uint8_t* cursor = static_cast<uint8_t*>(allocation);
    const size_t plan_bytes = q38m_moe_route_plan_bytes_v1(tokens);
    if (int rc = q38m_moe_route_plan_storage_v1(cursor, plan_bytes, tokens, &out->plan)) return rc;
    cursor += align_up(plan_bytes, 256);
    out->max_tokens = tokens;
    out->expert_ids = reinterpret_cast<int32_t*>(cursor);
    cursor += align_up(routes * 4u, 256);
    out->expert_weights = reinterpret_cast<float*>(cursor);
    cursor += align_up(routes * 4u, 256);
    out->xq = reinterpret_cast<int8_t*>(cursor);
    cursor += align_up(static_cast<size_t>(tokens) * Q38M_HIDDEN, 256);
    out->xs = reinterpret_cast<float*>(cursor);
    cursor += align_up(static_cast<size_t>(tokens) * 4u, 256);
    out->weighted_mid = reinterpret_cast<uint16_t*>(cursor);
    cursor += align_up(routes * Q38M_INTERMEDIATE * 2u, 256);
    out->mid_q = reinterpret_cast<int8_t*>(cursor);
    cursor += align_up(routes * Q38M_INTERMEDIATE, 256);
    out->mid_s = reinterpret_cast<float*>(cursor);
    cursor += align_up(routes * 4u, 256);
    out->route_output = reinterpret_cast<float*>(cursor);
    cursor += align_up(routes * Q38M_HIDDEN * 4u, 256);
    out->task_flags = reinterpret_cast<uint32_t*>(cursor);
    g_last_error.clear();
    return Q38M_OK;
}

}  // extern "C"

namespace {

// The run_moe sequence over one slab on a bound workspace (arguments
// validated by the caller): top-k + int8 rows (or int8 rows of given
// ids), plan, gate/up, down (quantising the mid rows as it stages them),
// combine; gate/up and down as one launch where the formats allow
// (launch_gate_up_down), its hand-off flags cleared by the plan kernel.
hipError_t launch_prefill_step(const q38m_expert_weights_v1& gate_up,
                               const q38m_expert_weights_v1& down, const uint16_t* hidden,
                               const float* logits, uint32_t tokens,
                               const q38m_prefill_workspace_v1& ws,
                               const uint16_t* shared_output, const uint16_t* shared_gate,
                               uint16_t* output, hipStream_t s) {
    const uint32_t tasks = q38m::max_tasks_v1(tokens);
    // one launch for gate/up and down: the plan kernel clears its flags
    const bool fused = ws.task_flags != nullptr && q38m::gate_up_down_fusable(gate_up, down);
    hipError_t status = hipSuccess;
    if (logits)
        status = q38m::launch_route_quantize(logits, hidden, tokens, Q38M_ROUTE_TOPK,
                                             ws.expert_ids, ws.expert_weights, ws.xq, ws.xs, s);
    else
        status = q38m::launch_quantize_rows(hidden, tokens, Q38M_HIDDEN, ws.xq, ws.xs, s);
    if (status == hipSuccess)
        status = q38m::launch_build_plan(ws.expert_ids, tokens, ws.plan, false, s,
                                         fused ? ws.task_flags : nullptr,
                                         fused ? q38m::task_flag_words(tasks) : 0u);
    if (status == hipSuccess && fused)
        status = q38m::launch_gate_up_down(gate_up, down, ws.xq, ws.xs,
                                           ws.plan.packed_assignment, ws.expert_weights,
                                           ws.plan.tasks, tasks, ws.weighted_mid, ws.mid_q,
                                           ws.mid_s, ws.route_output, ws.task_flags,
                                           &ws.plan.header->status, s);
    if (status == hipSuccess && !fused)
        status = q38m::launch_gate_up(gate_up, ws.xq, ws.xs, ws.plan.packed_assignment,
                                      ws.expert_weights, ws.plan.tasks, tasks, ws.weighted_mid, s);
    if (status == hipSuccess && !fused)
        status = q38m::launch_down_quantize(down, ws.weighted_mid, ws.mid_q, ws.mid_s,
                                            ws.plan.tasks, tasks, ws.route_output, s);
    if (status == hipSuccess)
        status = q38m::launch_combine(ws.route_output, ws.plan.assignment_to_packed,
                                      shared_output, shared_gate, tokens, output, s);
    return status;
}

}  // namespace

extern "C" {

int q38m_moe_prefill_v1(const q38m_expert_weights_v1* gate_up, const q38m_expert_weights_v1* down,
                        const uint16_t* hidden, const float* logits, uint32_t tokens,
                        const q38m_prefill_workspace_v1* ws, const uint16_t* shared_output,
                        const uint16_t* shared_gate, uint16_t* output, void* stream, int device) {
    if (int rc = check_weights(gate_up, true)) return rc;
    if (int rc = check_weights(down, false)) return rc;
    if (!hidden || !ws || !output || tokens == 0 || tokens > ws->max_tokens ||
        tokens > Q38M_PREFILL_SLAB_MAX_TOKENS || !valid_plan(&ws->plan) || !ws->expert_ids ||
        !ws->expert_weights || !ws->xq || !ws->xs ||
        !ws->weighted_mid || !ws->mid_q || !ws->mid_s || !ws->route_output ||
        (shared_output == nullptr) != (shared_gate == nullptr) || !aligned(hidden, 16) ||
        !aligned(output, 16))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid prefill MoE step input");
    if (int rc = select_device(device)) return rc;
    return finish(launch_prefill_step(*gate_up, *down, hidden, logits, tokens, *ws, shared_output,
                                      shared_gate, output, as_stream(stream)),
                  "prefill MoE step");
}

}  // extern "C"

// ---- the allocation-free slab step ---------------------------------------
// The whole-step workspace of a slab of up to Q38M_NOALLOC_MAX_TOKENS
// tokens, in a file-scope device array: each GPU the library runs on holds
// its own copy until the process ends.  In host code `scratch` names a
// host-side stand-in, so its device address is looked up once per device
// (with that device current) and only that address is used afterwards.
static __device__ __align__(256) uint8_t
    scratch[q38m::prefill_workspace_bytes_v1(Q38M_NOALLOC_MAX_TOKENS)];

namespace {

constexpr int kNoAllocDevices = 64;
// a successful lookup is kept per device; a failed one is not, so a later
// call (say, once the device's context exists) looks again
std::atomic<void*> g_scratch_address[kNoAllocDevices];
std::mutex g_scratch_mutex;

// Device address of `scratch` on `device`, which the caller made current.
int noalloc_scratch(int device, void** address) {
    if (device >= kNoAllocDevices)
        return fail(Q38M_ERR_INVALID_ARGUMENT, "allocation-free step: device index above 63");
    void* known = g_scratch_address[device].load(std::memory_order_acquire);
    if (known == nullptr) {
        std::lock_guard<std::mutex> lock(g_scratch_mutex);
        known = g_scratch_address[device].load(std::memory_order_relaxed);
        if (known == nullptr) {
            const hipError_t status = hipGetSymbolAddress(&known, HIP_SYMBOL(scratch));
            if (status != hipSuccess || known == nullptr)
                return device_fail(status != hipSuccess ? status : hipErrorInvalidSymbol,
                                   "hipGetSymbolAddress(scratch)");
            g_scratch_address[device].store(known, std::memory_order_release);
        }
    }
    *address = known;
    return Q38M_OK;
}

}  // namespace

extern "C" {

size_t q38m_moe_prefill_noalloc_scratch_bytes(void) {
    return q38m::prefill_workspace_bytes_v1(Q38M_NOALLOC_MAX_TOKENS);
}

int q38m_moe_prefill_noalloc_v1(const q38m_expert_weights_v1* gate_up,
                                const q38m_expert_weights_v1* down, const uint16_t* hidden,
                                const float* logits, uint32_t tokens,
                                const uint16_t* shared_output, const uint16_t* shared_gate,
                                uint16_t* output, void* stream, int device) {
    if (int rc = check_weights(gate_up, true)) return rc;
    if (int rc = check_weights(down, false)) return rc;
    if (tokens == 0 || tokens > Q38M_NOALLOC_MAX_TOKENS)
        return fail(Q38M_ERR_INVALID_ARGUMENT,
                    "q38m_moe_prefill_noalloc_v1 takes 1 to 64 tokens (its device-resident "
                    "workspace holds a 64-token slab); use q38m_moe_prefill_v1 with a "
                    "caller-owned workspace for more");
    if (!hidden || !logits || !output || (shared_output == nullptr) != (shared_gate == nullptr) ||
        !aligned(hidden, 16) || !aligned(logits, 16) || !aligned(output, 16) ||
        (shared_output && !aligned(shared_output, 16)))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid allocation-free prefill MoE step input");
    if (int rc = select_device(device)) return rc;
    void* base = nullptr;
    if (int rc = noalloc_scratch(device, &base)) return rc;
    // binding is pointer arithmetic on the device address; nothing is touched
    q38m_prefill_workspace_v1 ws;
    if (int rc = q38m_moe_prefill_workspace_bind(base, q38m_moe_prefill_noalloc_scratch_bytes(),
                                                 Q38M_NOALLOC_MAX_TOKENS, &ws))
        return rc;
    return finish(launch_prefill_step(*gate_up, *down, hidden, logits, tokens, ws, shared_output,
                                      shared_gate, output, as_stream(stream)),
                  "allocation-free prefill MoE step");
}

// ---- chunks above the slab ----------------------------------------------

uint32_t q38m_moe_wide_max_tasks(uint32_t tokens) {
    if (tokens == 0 || tokens > Q38M_WIDE_MAX_TOKENS) return 0;
    return q38m::max_tasks_wide(tokens);
}

// Task slots of a chunk plan bound for `tokens`: the chunk plan's own bound,
// or the V1 bound of a slab of up to 512 tokens if that is larger, so that a
// chunk workspace also serves q38m_moe_prefill_v1 for any slab it holds.
static size_t wide_task_slots(uint32_t tokens) {
    const uint32_t slab = tokens < Q38M_PREFILL_SLAB_MAX_TOKENS ? tokens
                                                                : Q38M_PREFILL_SLAB_MAX_TOKENS;
    const uint32_t wide = q38m::max_tasks_wide(tokens);
    const uint32_t v1 = q38m::max_tasks_v1(slab);
    return wide > v1 ? wide : v1;
}

size_t q38m_moe_wide_plan_bytes(uint32_t tokens) {
    if (tokens == 0 || tokens > Q38M_WIDE_MAX_TOKENS) return 0;
    const size_t routes = q38m::routes_v1(tokens);
    return sizeof(q38m_route_plan_header_v1) + Q38M_ROUTE_EXPERTS * sizeof(uint16_t) +
           2u * (Q38M_ROUTE_EXPERTS + 1u) * sizeof(uint32_t) + 2u * routes * sizeof(uint32_t) +
           wide_task_slots(tokens) * sizeof(q38m_task_v1);
}

size_t q38m_moe_wide_plan_scratch_bytes(uint32_t tokens) {
    if (tokens == 0 || tokens > Q38M_WIDE_MAX_TOKENS) return 0;
    return static_cast<size_t>(q38m::wide_chunks(tokens)) * (Q38M_ROUTE_EXPERTS + 1u) *
           sizeof(uint32_t);
}

int q38m_moe_wide_plan_storage(void* allocation, size_t allocation_bytes, uint32_t tokens,
                               q38m_route_plan_v1* out) {
    if (!out || !allocation || tokens == 0 || tokens > Q38M_WIDE_MAX_TOKENS)
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid chunk route-plan allocation");
    if (allocation_bytes < q38m_moe_wide_plan_bytes(tokens))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "chunk route-plan allocation is too small");
    if (!aligned(allocation, alignof(q38m_route_plan_header_v1)))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "chunk route-plan allocation is unaligned");
    bind_plan_views(allocation, tokens, out);
    g_last_error.clear();
    return Q38M_OK;
}

int q38m_moe_build_route_plan_wide(const int32_t* expert_ids, uint32_t tokens,
                                   const q38m_route_plan_v1* plan, uint32_t* scratch,
                                   void* stream, int device) {
    if (!expert_ids || !valid_plan(plan) || !scratch || tokens == 0 ||
        tokens > Q38M_WIDE_MAX_TOKENS || !aligned(scratch, 4))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid chunk route-plan input");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_build_wide_plan(expert_ids, tokens, *plan, scratch,
                                               as_stream(stream)),
                  "chunk route-plan kernels");
}

// hand-off flags for q38m_moe_prefill_v1 on a chunk workspace: the V1 task
// slots of the largest slab it holds
static uint32_t slab_flag_words(uint32_t tokens) {
    return q38m::task_flag_words(q38m::max_tasks_v1(
        tokens < Q38M_PREFILL_SLAB_MAX_TOKENS ? tokens : Q38M_PREFILL_SLAB_MAX_TOKENS));
}

size_t q38m_moe_wide_workspace_bytes(uint32_t tokens) {
    if (tokens == 0 || tokens > Q38M_WIDE_MAX_TOKENS) return 0;
    const size_t routes = q38m::routes_v1(tokens);
    size_t bytes = align_up(q38m_moe_wide_plan_bytes(tokens), 256);
    bytes += align_up(q38m_moe_wide_plan_scratch_bytes(tokens), 256);
    bytes += align_up(routes * 4u, 256) * 2u;                                // ids, weights
    bytes += align_up(static_cast<size_t>(tokens) * Q38M_HIDDEN, 256);      // xq
    bytes += align_up(static_cast<size_t>(tokens) * 4u, 256);               // xs
    bytes += align_up(routes * Q38M_INTERMEDIATE * 2u, 256);                // weighted_mid
    bytes += align_up(routes * Q38M_INTERMEDIATE, 256);                     // mid_q
    bytes += align_up(routes * 4u, 256);                                    // mid_s
    bytes += align_up(routes * Q38M_HIDDEN * 4u, 256);                      // route_output
    bytes += align_up(static_cast<size_t>(slab_flag_words(tokens)) * 4u, 256);  // task_flags
    return bytes;
}

int q38m_moe_wide_workspace_bind(void* allocation, size_t bytes, uint32_t tokens,
                                 q38m_wide_workspace_v1* out) {
    if (!allocation || !out || tokens == 0 || tokens > Q38M_WIDE_MAX_TOKENS ||
        bytes < q38m_moe_wide_workspace_bytes(tokens) || !aligned(allocation, 256))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid chunk workspace allocation");
    const size_t routes = q38m::routes_v1(tokens);
    uint8_t* cursor = static_cast<uint8_t*>(allocation);
    q38m_prefill_workspace_v1& w = out->step;
    bind_plan_views(cursor, tokens, &w.plan);
    cursor += align_up(q38m_moe_wide_plan_bytes(tokens), 256);
    out->plan_scratch = reinterpret_cast<uint32_t*>(cursor);
    cursor += align_up(q38m_moe_wide_plan_scratch_bytes(tokens), 256);
    w.max_tokens = tokens;
    w.expert_ids = reinterpret_cast<int32_t*>(cursor);
    cursor += align_up(routes * 4u, 256);
    w.expert_weights = reinterpret_cast<float*>(cursor);
    cursor += align_up(routes * 4u, 256);
    w.xq = reinterpret_cast<int8_t*>(cursor);
    cursor += align_up(static_cast<size_t>(tokens) * Q38M_HIDDEN, 256);
    w.xs = reinterpret_cast<float*>(cursor);
    cursor += align_up(static_cast<size_t>(tokens) * 4u, 256);
    w.weighted_mid = reinterpret_cast<uint16_t*>(cursor);
    cursor += align_up(routes * Q38M_INTERMEDIATE * 2u, 256);
    w.mid_q = reinterpret_cast<int8_t*>(cursor);
    cursor += align_up(routes * Q38M_INTERMEDIATE, 256);
    w.mid_s = reinterpret_cast<float*>(cursor);
    cursor += align_up(routes * 4u, 256);
    w.route_output = reinterpret_cast<float*>(cursor);
    cursor += align_up(routes * Q38M_HIDDEN * 4u, 256);
    w.task_flags = reinterpret_cast<uint32_t*>(cursor);
    g_last_error.clear();
    return Q38M_OK;
}

int q38m_moe_prefill_wide_v1(const q38m_expert_weights_v1* gate_up,
                             const q38m_expert_weights_v1* down, const uint16_t* hidden,
                             const float* logits, uint32_t tokens,
                             const q38m_wide_workspace_v1* wide,
                             const uint16_t* shared_output, const uint16_t* shared_gate,
                             uint16_t* output, void* stream, int device) {
    if (int rc = check_weights(gate_up, true)) return rc;
    if (int rc = check_weights(down, false)) return rc;
    if (!wide || !wide->plan_scratch)
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid chunk MoE workspace");
    const q38m_prefill_workspace_v1* ws = &wide->step;
    if (!hidden || !output || tokens == 0 || tokens > ws->max_tokens ||
        tokens > Q38M_WIDE_MAX_TOKENS || !valid_plan(&ws->plan) || !ws->expert_ids ||
        !ws->expert_weights || !ws->xq || !ws->xs || !ws->weighted_mid || !ws->mid_q ||
        !ws->mid_s || !ws->route_output ||
        (shared_output == nullptr) != (shared_gate == nullptr) || !aligned(hidden, 16) ||
        !aligned(output, 16) || (logits && !aligned(logits, 16)))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid chunk MoE step input");
    if (int rc = select_device(device)) return rc;
    const hipStream_t s = as_stream(stream);
    const uint32_t routes = q38m::routes_v1(tokens);
    const uint32_t tasks = q38m::max_tasks_wide(tokens);
    hipError_t status = hipSuccess;
    if (logits)
        status = q38m::launch_route_quantize_wave(logits, hidden, tokens, ws->expert_ids,
                                                  ws->expert_weights, ws->xq, ws->xs, s);
    else
        status = q38m::launch_quantize_rows(hidden, tokens, Q38M_HIDDEN, ws->xq, ws->xs, s);
    if (status == hipSuccess)
        status = q38m::launch_build_wide_plan(ws->expert_ids, tokens, ws->plan,
                                              wide->plan_scratch, s);
    if (status == hipSuccess)
        status = q38m::launch_gate_up_wide(*gate_up, ws->xq, ws->xs, ws->plan.packed_assignment,
                                           ws->expert_weights, ws->plan.tasks,
                                           &ws->plan.header->task_count, tasks,
                                           ws->weighted_mid, s);
    if (status == hipSuccess)
        status = q38m::launch_quantize_rows(ws->weighted_mid, routes, Q38M_INTERMEDIATE,
                                            ws->mid_q, ws->mid_s, s);
    if (status == hipSuccess)
        status = q38m::launch_down_wide(*down, ws->mid_q, ws->mid_s, ws->plan.tasks,
                                        &ws->plan.header->task_count, tasks,
                                        ws->route_output, s);
    if (status == hipSuccess)
        status = q38m::launch_combine(ws->route_output, ws->plan.assignment_to_packed,
                                      shared_output, shared_gate, tokens, output, s);
    return finish(status, "chunk MoE step");
}

size_t q38m_moe_decode_scratch_bytes(void) { return q38m::decode_scratch_bytes(); }

int q38m_moe_routed_decode_v1(const q38m_expert_weights_v1* gate_up,
                              const q38m_expert_weights_v1* down, const uint16_t* hidden,
                              const int32_t* expert_ids, const float* expert_weights,
                              uint32_t top_k, void* scratch, uint16_t* routed_output,
                              void* stream, int device) {
    if (int rc = check_weights(gate_up, true)) return rc;
    if (int rc = check_weights(down, false)) return rc;
    if (!hidden || !expert_ids || !expert_weights || top_k == 0 || top_k > Q38M_ROUTE_TOPK ||
        !scratch || !routed_output || !aligned(hidden, 16) || !aligned(scratch, 16))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid routed MoE buffers");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_decode(*gate_up, *down, hidden, nullptr, expert_ids,
                                      expert_weights, top_k, nullptr, nullptr, nullptr, scratch,
                                      routed_output, as_stream(stream)),
                  "decode routed MoE kernels");
}

int q38m_moe_decode_v1(const q38m_expert_weights_v1* gate_up, const q38m_expert_weights_v1* down,
                       const uint16_t* hidden, const float* logits, uint32_t top_k,
                       const uint16_t* shared_output, const uint16_t* shared_gate,
                       const uint16_t* residual, void* scratch, uint16_t* output, void* stream,
                       int device) {
    if (int rc = check_weights(gate_up, true)) return rc;
    if (int rc = check_weights(down, false)) return rc;
    if (!hidden || !logits || top_k == 0 || top_k > Q38M_ROUTE_TOPK || !scratch || !output ||
        !aligned(hidden, 16) || !aligned(logits, 16) || !aligned(scratch, 16) ||
        ((shared_output == nullptr) != (shared_gate == nullptr)))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid decode MoE buffers");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_decode(*gate_up, *down, hidden, logits, nullptr, nullptr, top_k,
                                      shared_output, shared_gate, residual, scratch, output,
                                      as_stream(stream)),
                  "decode MoE kernels");
}

size_t q38m_moe_decode_block_scratch_bytes(void) { return q38m::decode_block_scratch_bytes(); }

int q38m_moe_decode_block_v1(const q38m_expert_weights_v1* gate_up,
                             const q38m_expert_weights_v1* down, const uint16_t* hidden,
                             const uint16_t* router, const uint16_t* w_gate, const uint16_t* w_up,
                             const uint16_t* w_down, const uint16_t* w_out_gate,
                             uint32_t shared_inter, uint32_t top_k, const uint16_t* residual,
                             void* scratch, uint16_t* output, void* stream, int device) {
    if (int rc = check_weights(gate_up, true)) return rc;
    if (int rc = check_weights(down, false)) return rc;
    if (shared_inter != Q38M_INTERMEDIATE)
        return fail(Q38M_ERR_INVALID_ARGUMENT,
                    "decode block: the shared expert's intermediate size must be 512 (two "
                    "channels per gate/up workgroup)");
    if (!all16({hidden, router, w_gate, w_up, w_down, w_out_gate, scratch}) || !output ||
        top_k == 0 || top_k > Q38M_ROUTE_TOPK || (residual != nullptr && !aligned(residual, 2)) ||
        !aligned(output, 2))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid decode block buffers");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_decode_block(*gate_up, *down, hidden, router, w_gate, w_up, w_down,
                                            w_out_gate, top_k, residual, scratch, output,
                                            as_stream(stream)),
                  "decode block kernels");
}

size_t q38m_expert_weights_bytes(const q38m_expert_weights_v1* w, size_t* scale_bytes) {
    if (!w || (w->format != Q38M_FORMAT_W4_SYM && w->format != Q38M_FORMAT_W8_SYM)) {
        if (scale_bytes) *scale_bytes = 0;
        return 0;
    }
    const uint64_t elements = static_cast<uint64_t>(w->experts) * w->rows * w->columns;
    if (scale_bytes) {
        const uint64_t scales = w->group_size ? elements / w->group_size
                                              : static_cast<uint64_t>(w->experts) * w->rows;
        *scale_bytes = static_cast<size_t>(scales * 2u);
    }
    return static_cast<size_t>(w->format == Q38M_FORMAT_W4_SYM ? elements / 2u : elements);
}

int q38m_repack_expert_weights(const q38m_expert_weights_v1* src,
                               const q38m_expert_weights_v1* dst, void* stream, int device) {
    if (!src || !dst || !src->data || !src->scales || !dst->data || !dst->scales ||
        src->layout != Q38M_LAYOUT_ROW_MAJOR ||
        (dst->layout != Q38M_LAYOUT_MFMA16 && dst->layout != Q38M_LAYOUT_MFMA16_PAIRED) ||
        src->format != dst->format || src->group_size != dst->group_size ||
        !valid_scale_dtype(src->scale_dtype) || dst->scale_dtype != src->scale_dtype ||
        src->experts != dst->experts || src->rows != dst->rows || src->columns != dst->columns ||
        src->experts == 0 || src->rows % 16u != 0u || !aligned(src->data, 16) ||
        !aligned(dst->data, 16))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid expert weight repack");
    const bool w4 = src->format == Q38M_FORMAT_W4_SYM && w4_group(src->group_size) &&
                    src->columns % 128u == 0u &&
                    (dst->layout == Q38M_LAYOUT_MFMA16 || src->rows % 32u == 0u);
    const bool w8 = src->format == Q38M_FORMAT_W8_SYM &&
                    (src->group_size == 0u || src->group_size == 64u ||
                     src->group_size == 128u) &&
                    src->columns % 64u == 0u &&
                    (src->group_size == 0u || src->columns % src->group_size == 0u) &&
                    (dst->layout == Q38M_LAYOUT_MFMA16 || src->rows % 32u == 0u);
    if (!w4 && !w8)
        return fail(Q38M_ERR_UNSUPPORTED,
                    "repack supports W4 groups 32/64/128 and W8 per channel or groups 64/128 "
                    "(MFMA16 or MFMA16_PAIRED)");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_repack(*src, *dst, as_stream(stream)), "repack kernels");
}

// the GEMM grid's y dimension holds one 32-row tile per block and stays
// within 65535 blocks
constexpr uint32_t kDenseMaxRows = 65535u * 32u;

int q38m_dense_gemm_bf16(const uint16_t* a, const uint16_t* b, uint32_t m, uint32_t n,
                         uint32_t k, float* c_f32, uint16_t* c_bf16, void* stream, int device) {
    if (!a || !b || m == 0 || n == 0 || k == 0 || k % 32u != 0u || m > kDenseMaxRows ||
        (c_f32 == nullptr) == (c_bf16 == nullptr) || !aligned(a, 16) || !aligned(b, 16))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid dense GEMM buffers");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_dense_gemm(a, b, m, n, k, c_f32, c_bf16, as_stream(stream)),
                  "dense_gemm_kernel");
}

int q38m_moe_router_v1(const uint16_t* hidden, const uint16_t* router, uint32_t tokens,
                       uint32_t hidden_width, float* logits, void* stream, int device) {
    if (hidden_width != Q38M_HIDDEN)
        return fail(Q38M_ERR_INVALID_ARGUMENT, "router hidden width must be 2048");
    if (!hidden || !router || !logits || tokens == 0 || tokens > kDenseMaxRows ||
        !aligned(hidden, 16) || !aligned(router, 16))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid router buffers");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_dense_gemm(hidden, router, tokens, Q38M_ROUTE_EXPERTS,
                                          Q38M_HIDDEN, logits, nullptr, as_stream(stream)),
                  "router GEMM");
}

size_t q38m_moe_router_topk_workspace_bytes(uint32_t tokens) {
    return q38m::router_topk_workspace_bytes(tokens);
}

int q38m_moe_router_topk_v1(const uint16_t* hidden, const uint16_t* router, uint32_t tokens,
                            uint32_t hidden_width, uint32_t top_k, void* workspace,
                            size_t workspace_bytes, int32_t* expert_ids, float* expert_weights,
                            void* stream, int device) {
    if (hidden_width != Q38M_HIDDEN)
        return fail(Q38M_ERR_INVALID_ARGUMENT, "router hidden width must be 2048");
    // the selection grid's y dimension holds one 16-token block per workgroup
    if (!hidden || !router || !workspace || !expert_ids || !expert_weights || tokens == 0 ||
        tokens > 65535u * 16u || top_k == 0 || top_k > Q38M_ROUTE_TOPK ||
        !aligned(hidden, 16) || !aligned(router, 16) || !aligned(workspace, 16) ||
        workspace_bytes < q38m::router_topk_workspace_bytes(tokens))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid router top-k buffers");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_router_topk(hidden, router, tokens, top_k, workspace, expert_ids,
                                           expert_weights, as_stream(stream)),
                  "router top-k kernels");
}

size_t q38m_moe_shared_expert_scratch_bytes(uint32_t tokens, uint32_t inter) {
    return q38m::shared_expert_scratch_bytes(tokens, inter);
}

int q38m_moe_shared_expert_v1(const uint16_t* hidden, const uint16_t* w_gate,
                              const uint16_t* w_up, const uint16_t* w_down,
                              const uint16_t* w_out_gate, uint32_t tokens,
                              uint32_t hidden_width, uint32_t inter, void* scratch,
                              uint16_t* shared_output, uint16_t* shared_gate, void* stream,
                              int device) {
    if (hidden_width != Q38M_HIDDEN)
        return fail(Q38M_ERR_INVALID_ARGUMENT, "shared expert hidden width must be 2048");
    if (!hidden || !w_gate || !w_up || !w_down || !w_out_gate || !scratch || !shared_output ||
        !shared_gate || tokens == 0 || tokens > kDenseMaxRows || inter == 0 || inter % 32u != 0u ||
        !aligned(hidden, 16) || !aligned(w_gate, 16) || !aligned(w_up, 16) ||
        !aligned(w_down, 16) || !aligned(w_out_gate, 16) || !aligned(scratch, 16))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid shared expert buffers");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_shared_expert(hidden, w_gate, w_up, w_down, w_out_gate, tokens,
                                             inter, scratch, shared_output, shared_gate,
                                             as_stream(stream)),
                  "shared expert kernels");
}

int q38m_quantize_expert_weights(const uint16_t* src_bf16, const q38m_expert_weights_v1* dst,
                                 void* stream, int device) {
    if (!src_bf16 || !dst || !dst->data || !dst->scales || dst->layout != Q38M_LAYOUT_ROW_MAJOR ||
        !valid_scale_dtype(dst->scale_dtype) || dst->experts == 0 || dst->rows == 0 ||
        dst->columns == 0 || !aligned(src_bf16, 16) || !aligned(dst->data, 16) ||
        !aligned(dst->scales, 2))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid weight quantiser buffers");
    const uint32_t g = dst->group_size;
    const bool grouped = (g == 32u || g == 64u || g == 128u) && dst->columns % g == 0u;
    const bool w4 = dst->format == Q38M_FORMAT_W4_SYM && grouped;
    const bool w8 = dst->format == Q38M_FORMAT_W8_SYM &&
                    (grouped || (g == 0u && dst->columns % 512u == 0u));
    if (!w4 && !w8)
        return fail(Q38M_ERR_UNSUPPORTED,
                    "quantiser supports W4 groups 32/64/128 and W8 groups 32/64/128 or per "
                    "channel (columns a multiple of 512)");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_quantize_weights(src_bf16, *dst, as_stream(stream)),
                  "quantize_weights kernels");
}

int q38m_synth_fill(uint32_t kind, uint64_t seed, uint64_t tag, uint64_t count, float sigma,
                    int32_t lo, int32_t hi, const float* bias, uint32_t bias_len, void* out,
                    void* stream, int device) {
    if (!out || count == 0 || kind < Q38M_SYNTH_NORMAL_F32 || kind > Q38M_SYNTH_UNIFORM_I8 ||
        (kind == Q38M_SYNTH_UNIFORM_W4 && (count % 2u != 0u || lo < -8 || hi > 7 || lo > hi)) ||
        (kind == Q38M_SYNTH_UNIFORM_I8 && (lo < -128 || hi > 127 || lo > hi)) ||
        (bias && (bias_len == 0 || kind != Q38M_SYNTH_NORMAL_F32)))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid synthetic fill");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_synth(kind, seed, tag, count, sigma, lo, hi, bias, bias_len, out,
                                     as_stream(stream)),
                  "synth_kernel");
}

int q38m_moe_compiled(void) { return 1; }

const char* q38m_last_error(void) { return g_last_error.c_str(); }

// ---- hyper-connection prepare/finish ----------------------------------

namespace {
bool valid_hidden(uint32_t hidden) { return hidden != 0u && hidden % 8u == 0u && hidden <= 8192u; }
}  // namespace

int q38m_hyper_repeat_embedding_bf16(const uint16_t* embedding, uint16_t* hyper, uint32_t tokens,
                                     uint32_t hidden, void* stream, int device) {
    if (!all16({embedding, hyper}) || tokens == 0 || !valid_hidden(hidden))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid hyper repeat buffers");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_hyper_repeat(embedding, hyper, tokens, hidden, as_stream(stream)),
                  "hyper_repeat_kernel");
}

int q38m_hyper_group_rmsnorm_bf16(const uint16_t* hyper, const uint16_t* norm_weight,
                                  uint16_t* normalized, uint32_t tokens, uint32_t hidden,
                                  void* stream, int device) {
    if (!all16({hyper, norm_weight, normalized}) || tokens == 0 || !valid_hidden(hidden))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid hyper norm buffers");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_hyper_norm(hyper, norm_weight, nullptr, tokens, hidden, normalized,
                                          nullptr, as_stream(stream)),
                  "hyper_norm_kernel");
}

int q38m_hyper_silu_scaled_bf16(const uint16_t* input, uint16_t* output, uint32_t tokens,
                                uint32_t width, float divisor, void* stream, int device) {
    const uint64_t elements = static_cast<uint64_t>(tokens) * width;
    if (!all16({input, output}) || elements == 0 || elements % 8u != 0u || !(divisor > 0.0f))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid hyper elementwise buffers");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_hyper_elementwise(input, output, elements, divisor, 1.0f, true,
                                                 as_stream(stream)),
                  "hyper_elementwise_kernel");
}

int q38m_hyper_sigmoid_bf16(const uint16_t* input, uint16_t* output, uint32_t tokens,
                            uint32_t width, float input_divisor, float output_scale,
                            void* stream, int device) {
    const uint64_t elements = static_cast<uint64_t>(tokens) * width;
    if (!all16({input, output}) || elements == 0 || elements % 8u != 0u ||
        !(input_divisor > 0.0f))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid hyper elementwise buffers");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_hyper_elementwise(input, output, elements, input_divisor,
                                                 output_scale, false, as_stream(stream)),
                  "hyper_elementwise_kernel");
}

int q38m_hyper_mix_bf16(const uint16_t* normalized_hyper, const uint16_t* mix_weights,
                        uint16_t* mixed, uint32_t tokens, uint32_t hidden, void* stream,
                        int device) {
    if (!all16({normalized_hyper, mix_weights, mixed}) || tokens == 0 || !valid_hidden(hidden))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid hyper mix buffers");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_hyper_mix(normalized_hyper, mix_weights, mixed, tokens, hidden,
                                         as_stream(stream)),
                  "hyper_mix_kernel");
}

int q38m_hyper_inject_bf16(const uint16_t* original_hyper, const uint16_t* block_output,
                           const uint16_t* injection_weights, uint16_t* output_hyper,
                           uint32_t tokens, uint32_t hidden, void* stream, int device) {
    if (!all16({original_hyper, block_output, output_hyper}) || !injection_weights ||
        !aligned(injection_weights, 2) || tokens == 0 || !valid_hidden(hidden))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid hyper injection buffers");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_hyper_inject(original_hyper, block_output, injection_weights,
                                            output_hyper, tokens, hidden, as_stream(stream)),
                  "hyper_inject_kernel");
}

size_t q38m_hyper_prepare_scratch_bytes(uint32_t tokens, uint32_t hidden, uint32_t low_rank) {
    return q38m::hyper_prepare_scratch_bytes(tokens, hidden, low_rank);
}

int q38m_hyper_prepare_v1(const uint16_t* hyper, const uint16_t* norm_weight,
                          const uint16_t* mix_down, const uint16_t* mix_up,
                          const uint16_t* inject, uint32_t tokens, uint32_t hidden,
                          uint32_t low_rank, void* scratch, uint16_t* mixed,
                          uint16_t* injection, void* stream, int device) {
    if (!all16({hyper, norm_weight, mix_down, mix_up, scratch, mixed}) || tokens == 0 ||
        tokens > 65535u * 32u || !valid_hidden(hidden) || low_rank == 0u ||
        low_rank % 32u != 0u || (inject != nullptr && (!aligned(inject, 16) || !injection)) ||
        (injection != nullptr && !aligned(injection, 2)))
        return fail(Q38M_ERR_INVALID_ARGUMENT, "invalid hyper prepare input");
    if (int rc = select_device(device)) return rc;
    return finish(q38m::launch_hyper_prepare(hyper, norm_weight, mix_down, mix_up, inject, tokens,
                                             hidden, low_rank, scratch, mixed, injection,
                                             as_stream(stream)),
                  "hyper prepare kernels");
}

#ifdef Q38M_CHECKED
int q38m_checked_status_v1(uint32_t* status, int reset, int device) {
    if (!status) return fail(Q38M_ERR_INVALID_ARGUMENT, "null checked status");
    if (int rc = select_device(device)) return rc;
    // a diagnostic of the checked build: it allocates its own 4 bytes
    uint32_t* word = nullptr;
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMalloc(&word, sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(word, 0, sizeof(uint32_t));
    for (q38m::CheckedReader read : q38m::checked_readers())
        if (e == hipSuccess) e = read(word, reset, nullptr);
    uint32_t all = 0u;
    if (e == hipSuccess) e = hipMemcpy(&all, word, sizeof(all), hipMemcpyDeviceToHost);
    if (word != nullptr) {
        const hipError_t freed = hipFree(word);
        if (e == hipSuccess) e = freed;
    }
    if (e != hipSuccess) return device_fail(e, "checked status");
    *status = all;
    return finish(hipSuccess, "checked status");
}
#endif

}  // extern "C"
