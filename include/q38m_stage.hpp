// The MoE step of the reference's stage backend, written against the q38m C
// ABI: run_moe (cuda/cuda_backend.cu:1516-1605), the hyper-connection
// prepare/finish around it (:1219-1252) and the MoE half of run_prefill's
// slab x layer loop (:1905-2022, the moe_hyper / run_moe / finish_hyper
// steps at :1967-1971).  Host-only C++: every call goes through q38m.hpp,
// so this header needs no vendor headers and allocates nothing; the caller
// binds one device allocation as the workspace once, for the largest slab,
// as the reference sizes its MoE workspace at init (:908-946).
//
// One width runs end to end: the hyper state is Q38M_HYPER_STREAMS streams
// of Q38M_HIDDEN (2048) values per token, prepare writes `mixed` rows of
// 2048, and the router, shared expert and routed step take 2048-wide rows
// (the router and shared expert check the width they are given).
#ifndef Q38M_STAGE_HPP
#define Q38M_STAGE_HPP

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <utility>

#include "q38m.hpp"

namespace q38m {

// One layer's MoE weights as bind_moe (cuda/cuda_backend.cu:401-421) holds
// them: the routed experts in the MFMA16 device layouts and the dense bf16
// matrices ([out][in]) of the router and the shared expert.
struct MoeLayerWeights {
    ExpertWeightsV1 gate_up;
    ExpertWeightsV1 down;
    const std::uint16_t* router = nullptr;              // [512][2048]
    const std::uint16_t* shared_gate = nullptr;         // [shared_inter][2048]
    const std::uint16_t* shared_up = nullptr;           // [shared_inter][2048]
    const std::uint16_t* shared_down = nullptr;         // [2048][shared_inter]
    const std::uint16_t* shared_output_gate = nullptr;  // [1][2048]
    std::uint32_t shared_inter = Q38M_INTERMEDIATE;
};

// HyperWeights of the MoE block (prepare_hyper, cuda_backend.cu:1219-1243).
struct HyperWeights {
    const std::uint16_t* norm = nullptr;      // [4][2048]
    const std::uint16_t* mix_down = nullptr;  // [low_rank][4*2048]
    const std::uint16_t* mix_up = nullptr;    // [4*2048][low_rank]
    const std::uint16_t* inject = nullptr;    // [4][4*2048]
    std::uint32_t low_rank = 320;
};

struct StageLayer {
    HyperWeights moe_hyper;
    MoeLayerWeights moe;
};

// The MoE part of the stage workspace (cuda_backend.cu:908-946).
struct MoeStageWorkspace {
    std::uint32_t max_tokens = 0;
    PrefillWorkspaceV1 moe{};                 // plan + routed-step buffers
    float* logits = nullptr;                  // [T][512]
    std::uint16_t* mixed = nullptr;           // [T][2048], the MoE input
    std::uint16_t* injection = nullptr;       // [T][4]
    std::uint16_t* shared_output = nullptr;   // [T][2048]
    std::uint16_t* shared_gate = nullptr;     // [T]
    std::uint16_t* block_output = nullptr;    // [T][2048], the MoE output
    void* shared_scratch = nullptr;
    void* hyper_scratch = nullptr;
    void* decode_scratch = nullptr;
};

namespace detail {
inline std::size_t align256(std::size_t v) { return (v + 255u) / 256u * 256u; }

// Region sizes of the workspace in binding order.
inline void stage_regions(std::uint32_t t, std::uint32_t shared_inter, std::uint32_t low_rank,
                          std::size_t out[10]) {
    const std::size_t h = Q38M_HIDDEN;
    out[0] = q38m_moe_prefill_workspace_bytes(t);
    out[1] = static_cast<std::size_t>(t) * Q38M_ROUTE_EXPERTS * sizeof(float);
    out[2] = t * h * 2u;
    out[3] = static_cast<std::size_t>(t) * Q38M_HYPER_STREAMS * 2u;
    out[4] = t * h * 2u;
    out[5] = static_cast<std::size_t>(t) * 2u;
    out[6] = t * h * 2u;
    out[7] = q38m_moe_shared_expert_scratch_bytes(t, shared_inter);
    out[8] = q38m_hyper_prepare_scratch_bytes(t, Q38M_HIDDEN, low_rank);
    out[9] = q38m_moe_decode_block_scratch_bytes();  // covers the plain decode's too
}
}  // namespace detail

inline std::size_t moe_stage_workspace_bytes(std::uint32_t max_tokens,
                                             std::uint32_t shared_inter = Q38M_INTERMEDIATE,
                                             std::uint32_t low_rank = 320) {
    if (max_tokens == 0 || max_tokens > Q38M_PREFILL_SLAB_MAX_TOKENS) return 0;
    std::size_t regions[10];
    detail::stage_regions(max_tokens, shared_inter, low_rank, regions);
    std::size_t total = 0;
    for (std::size_t r : regions) total += detail::align256(r);
    return total;
}

// Binds a 256-byte aligned device allocation of moe_stage_workspace_bytes()
// bytes; never touches its contents.
inline MoeStageWorkspace bind_moe_stage_workspace(void* allocation, std::size_t bytes,
                                                  std::uint32_t max_tokens,
                                                  std::uint32_t shared_inter = Q38M_INTERMEDIATE,
                                                  std::uint32_t low_rank = 320) {
    const std::size_t need = moe_stage_workspace_bytes(max_tokens, shared_inter, low_rank);
    if (!allocation || need == 0 || bytes < need ||
        reinterpret_cast<std::uintptr_t>(allocation) % 256u != 0u)
        throw std::invalid_argument("invalid MoE stage workspace allocation");
    std::size_t regions[10];
    detail::stage_regions(max_tokens, shared_inter, low_rank, regions);
    auto* cursor = static_cast<unsigned char*>(allocation);
    void* at[10];
    for (int i = 0; i < 10; ++i) {
        at[i] = cursor;
        cursor += detail::align256(regions[i]);
    }
    MoeStageWorkspace ws;
    ws.max_tokens = max_tokens;
    check(q38m_moe_prefill_workspace_bind(at[0], regions[0], max_tokens, &ws.moe));
    ws.logits = static_cast<float*>(at[1]);
    ws.mixed = static_cast<std::uint16_t*>(at[2]);
    ws.injection = static_cast<std::uint16_t*>(at[3]);
    ws.shared_output = static_cast<std::uint16_t*>(at[4]);
    ws.shared_gate = static_cast<std::uint16_t*>(at[5]);
    ws.block_output = static_cast<std::uint16_t*>(at[6]);
    ws.shared_scratch = at[7];
    ws.hyper_scratch = at[8];
    ws.decode_scratch = at[9];
    return ws;
}

// run_moe (cuda/cuda_backend.cu:1516-1605): ws.mixed [tokens][2048] in,
// ws.block_output [tokens][2048] out, all on `stream`.
inline void run_moe(const MoeLayerWeights& m, std::uint32_t tokens, MoeStageWorkspace& ws,
                    void* stream, int device) {
    if (tokens == 0 || tokens > ws.max_tokens)
        throw std::invalid_argument("run_moe: tokens outside the bound workspace");
    if (tokens == 1 && m.shared_inter == Q38M_INTERMEDIATE) {
        // the decode step: router, top-k, routed experts, shared expert and
        // the gated combine (:1518-1601) in three launches
        moe_decode_block(m.gate_up, m.down, ws.mixed, m.router, m.shared_gate, m.shared_up,
                         m.shared_down, m.shared_output_gate, m.shared_inter, Q38M_ROUTE_TOPK,
                         /*residual=*/nullptr, ws.decode_scratch, ws.block_output, stream,
                         device);
        return;
    }
    // router logits (:1518) and the shared expert with its output gate
    // (:1573-1590), both reading the 2048-wide mixed rows
    moe_router(ws.mixed, m.router, tokens, Q38M_HIDDEN, ws.logits, stream, device);
    moe_shared_expert(ws.mixed, m.shared_gate, m.shared_up, m.shared_down,
                      m.shared_output_gate, tokens, Q38M_HIDDEN, m.shared_inter,
                      ws.shared_scratch, ws.shared_output, ws.shared_gate, stream, device);
    if (tokens > 1) {
        // top-k, route plan, int8 token rows, grouped gate/up + SwiGLU fold,
        // mid quantisation, grouped down, rank-order combine with the gated
        // shared term (:1523-1559, :1591-1596)
        run_moe_prefill(m.gate_up, m.down, ws.mixed, ws.logits, tokens, ws.moe,
                        ws.shared_output, ws.shared_gate, ws.block_output, stream, device);
    } else {
        // top-k, the routed experts and the gated shared combine (:1560-1568,
        // :1597-1601) in two launches
        moe_decode(m.gate_up, m.down, ws.mixed, ws.logits, Q38M_ROUTE_TOPK, ws.shared_output,
                   ws.shared_gate, /*residual=*/nullptr, ws.decode_scratch, ws.block_output,
                   stream, device);
    }
}

// prepare_hyper (cuda_backend.cu:1219-1243): state [tokens][4][2048] ->
// ws.mixed and ws.injection.
inline void prepare_hyper(const HyperWeights& h, const std::uint16_t* state,
                          std::uint32_t tokens, MoeStageWorkspace& ws, void* stream, int device) {
    check(q38m_hyper_prepare_v1(state, h.norm, h.mix_down, h.mix_up, h.inject, tokens,
                                Q38M_HIDDEN, h.low_rank, ws.hyper_scratch, ws.mixed, ws.injection,
                                stream, device));
}

// finish_hyper (cuda_backend.cu:1245-1252): destination = original +
// block_output x injection.
inline void finish_hyper(const std::uint16_t* original, std::uint16_t* destination,
                         std::uint32_t tokens, MoeStageWorkspace& ws, void* stream, int device) {
    check(q38m_hyper_inject_bf16(original, ws.block_output, ws.injection, destination, tokens,
                                 Q38M_HIDDEN, stream, device));
}

// The MoE half of run_prefill (cuda_backend.cu:1905-2022): slabs of at most
// ws.max_tokens tokens, each through every layer as prepare_hyper ->
// run_moe -> finish_hyper (:1967-1971), alternating between the two state
// buffers ([count][4][2048] each).  Every slab runs the same number of
// layers, so the result of all of them lies in `state` for an even layer
// count and in `alternate` for an odd one; that buffer is returned.
inline std::uint16_t* run_prefill_moe(const StageLayer* layers, std::size_t layer_count,
                                      std::uint16_t* state, std::uint16_t* alternate,
                                      std::uint32_t count, MoeStageWorkspace& ws, void* stream,
                                      int device) {
    const std::size_t row = static_cast<std::size_t>(Q38M_HYPER_STREAMS) * Q38M_HIDDEN;
    for (std::uint32_t first = 0; first < count; first += ws.max_tokens) {
        const std::uint32_t tokens = std::min(ws.max_tokens, count - first);
        std::uint16_t* current = state + first * row;
        std::uint16_t* other = alternate + first * row;
        for (std::size_t l = 0; l < layer_count; ++l) {
            prepare_hyper(layers[l].moe_hyper, current, tokens, ws, stream, device);
            run_moe(layers[l].moe, tokens, ws, stream, device);
            finish_hyper(current, other, tokens, ws, stream, device);
            std::swap(current, other);
        }
    }
    return layer_count % 2u == 0u ? state : alternate;
}

}  // namespace q38m

#endif
