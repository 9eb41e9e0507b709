// Drives the C++ MoE stage (include/q38m_stage.hpp) on one GPU the way the
// reference's stage worker drives run_prefill (cuda/cuda_backend.cu:
// 1905-2022): synthetic layers, a hyper state of `count` tokens, slabs of
// at most 512 tokens, every layer as prepare_hyper -> run_moe ->
// finish_hyper.  A token count that leaves a one-token tail slab takes
// run_moe's tokens == 1 branch (the decode entry point) for that slab.
//
// Two passes over the same initial state:
//   1. the slab x layer loop written out here, dumping each run_moe call's
//      inputs (mixed rows, router logits, shared output and gate) and its
//      block output, so the test can check every call against the CPU
//      oracle;
//   2. q38m::run_prefill_moe itself, whose final state must equal pass 1's.
//
// usage: run_moe_check <out_dir> <count> <layers> <seed>
// Expert weights use the synthetic streams of the config-2 layers (W4 g32
// fp16 gate/up, W8 per-channel fp16 down; tags 1000 + 10 l and +4), so the
// test regenerates them bit for bit.
#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "q38m_stage.hpp"

namespace {

void hip_check(hipError_t status, const char* what) {
    if (status != hipSuccess) {
        std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(status));
        std::exit(3);
    }
}

template <typename T>
T* device_alloc(std::size_t count) {
    void* p = nullptr;
    hip_check(hipMalloc(&p, count * sizeof(T)), "hipMalloc");
    return static_cast<T*>(p);
}

struct Context {
    std::uint64_t seed;
    void* stream;
    std::vector<void*> owned;

    template <typename T>
    T* alloc(std::size_t count) {
        T* p = device_alloc<T>(count);
        owned.push_back(p);
        return p;
    }

    // bf16(sigma * N(0,1)) words from stream `tag`
    std::uint16_t* normal_bf16(std::uint64_t tag, std::size_t count, float sigma) {
        auto* p = alloc<std::uint16_t>(count);
        q38m::check(q38m_synth_fill(Q38M_SYNTH_NORMAL_BF16, seed, tag, count, sigma, 0, 0,
                                    nullptr, 0, p, stream, 0));
        return p;
    }

    // Synthetic routed-expert weights (the streams of q38m_amd.synth_weights),
    // repacked into the MFMA16 device layout.
    q38m::ExpertWeightsV1 experts(std::uint64_t tag, std::uint32_t format, std::uint32_t group,
                                  std::uint32_t rows, std::uint32_t cols, float sigma,
                                  bool paired) {
        q38m_expert_weights_v1 rm{nullptr, nullptr, format, group, Q38M_SCALE_F16,
                                  Q38M_LAYOUT_ROW_MAJOR, Q38M_ROUTE_EXPERTS, rows, cols};
        std::size_t scale_bytes = 0;
        const std::size_t data_bytes = q38m_expert_weights_bytes(&rm, &scale_bytes);
        void* data = device_alloc<std::uint8_t>(data_bytes);
        void* scales = device_alloc<std::uint8_t>(scale_bytes);
        const std::uint64_t elements = std::uint64_t(Q38M_ROUTE_EXPERTS) * rows * cols;
        if (format == Q38M_FORMAT_W4_SYM)
            q38m::check(q38m_synth_fill(Q38M_SYNTH_UNIFORM_W4, seed, tag, elements, 1.0f, -8, 7,
                                        nullptr, 0, data, stream, 0));
        else
            q38m::check(q38m_synth_fill(Q38M_SYNTH_UNIFORM_I8, seed, tag, elements, 1.0f, -127,
                                        127, nullptr, 0, data, stream, 0));
        q38m::check(q38m_synth_fill(Q38M_SYNTH_ABS_NORMAL_F16, seed, tag + 1, scale_bytes / 2,
                                    sigma, 0, 0, nullptr, 0, scales, stream, 0));
        rm.data = data;
        rm.scales = scales;
        q38m_expert_weights_v1 dev = rm;
        dev.data = alloc<std::uint8_t>(data_bytes);
        dev.scales = alloc<std::uint8_t>(scale_bytes);
        dev.layout = paired ? Q38M_LAYOUT_MFMA16_PAIRED : Q38M_LAYOUT_MFMA16;
        q38m::check(q38m_repack_expert_weights(&rm, &dev, stream, 0));
        hip_check(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "repack");
        hip_check(hipFree(data), "hipFree");
        hip_check(hipFree(scales), "hipFree");
        return dev;
    }
};

void dump(const std::string& path, const void* device_ptr, std::size_t bytes, void* stream) {
    std::vector<unsigned char> host(bytes);
    hip_check(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "sync before dump");
    hip_check(hipMemcpy(host.data(), device_ptr, bytes, hipMemcpyDeviceToHost), "hipMemcpy");
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f || std::fwrite(host.data(), 1, bytes, f) != bytes) {
        std::fprintf(stderr, "cannot write %s\n", path.c_str());
        std::exit(4);
    }
    std::fclose(f);
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 5) {
        std::fprintf(stderr, "usage: %s <out_dir> <count> <layers> <seed>\n", argv[0]);
        return 2;
    }
    const std::string out = argv[1];
    const auto count = static_cast<std::uint32_t>(std::strtoul(argv[2], nullptr, 10));
    const auto layer_count = static_cast<std::uint32_t>(std::strtoul(argv[3], nullptr, 10));
    const std::uint64_t seed = std::strtoull(argv[4], nullptr, 10);
    if (count == 0 || layer_count == 0) return 2;
    hip_check(hipSetDevice(0), "hipSetDevice");
    hipStream_t hs = nullptr;
    hip_check(hipStreamCreate(&hs), "hipStreamCreate");
    Context ctx{seed, hs, {}};
    void* s = hs;

    try {
        const std::uint32_t H = Q38M_HIDDEN, I = Q38M_INTERMEDIATE, low_rank = 320;
        const std::size_t row = std::size_t(Q38M_HYPER_STREAMS) * H;
        std::vector<q38m::StageLayer> layers(layer_count);
        for (std::uint32_t l = 0; l < layer_count; ++l) {
            q38m::StageLayer& L = layers[l];
            const std::uint64_t tag = 1000 + 10 * l;  // workloads.layer_tags
            L.moe.gate_up = ctx.experts(tag, Q38M_FORMAT_W4_SYM, 32, 2 * I, H, 0.02f, true);
            L.moe.down = ctx.experts(tag + 4, Q38M_FORMAT_W8_SYM, 0, H, I, 0.002f, false);
            const std::uint64_t dense = 70000 + 100 * l;
            L.moe.router = ctx.normal_bf16(dense + 0, std::size_t(Q38M_ROUTE_EXPERTS) * H, 0.02f);
            L.moe.shared_gate = ctx.normal_bf16(dense + 1, std::size_t(I) * H, 0.02f);
            L.moe.shared_up = ctx.normal_bf16(dense + 2, std::size_t(I) * H, 0.02f);
            L.moe.shared_down = ctx.normal_bf16(dense + 3, std::size_t(H) * I, 0.02f);
            L.moe.shared_output_gate = ctx.normal_bf16(dense + 4, H, 0.02f);
            L.moe.shared_inter = I;
            L.moe_hyper.norm = ctx.normal_bf16(dense + 5, row, 0.1f);
            L.moe_hyper.mix_down = ctx.normal_bf16(dense + 6, std::size_t(low_rank) * row, 0.03f);
            L.moe_hyper.mix_up = ctx.normal_bf16(dense + 7, row * low_rank, 0.2f);
            L.moe_hyper.inject = ctx.normal_bf16(dense + 8, Q38M_HYPER_STREAMS * row, 0.03f);
            L.moe_hyper.low_rank = low_rank;
        }
        const std::size_t state_words = std::size_t(count) * row;
        std::uint16_t* initial = ctx.normal_bf16(90000, state_words, 1.0f);
        std::uint16_t* a = ctx.alloc<std::uint16_t>(state_words);
        std::uint16_t* b = ctx.alloc<std::uint16_t>(state_words);

        const std::uint32_t slab = count < Q38M_PREFILL_SLAB_MAX_TOKENS
                                       ? count
                                       : Q38M_PREFILL_SLAB_MAX_TOKENS;
        const std::size_t ws_bytes = q38m::moe_stage_workspace_bytes(slab);
        void* ws_mem = ctx.alloc<std::uint8_t>(ws_bytes);
        q38m::MoeStageWorkspace ws = q38m::bind_moe_stage_workspace(ws_mem, ws_bytes, slab);

        // pass 1: the slab x layer loop written out, with dumps
        hip_check(hipMemcpyAsync(a, initial, state_words * 2, hipMemcpyDeviceToDevice, hs),
                  "copy state");
        std::uint32_t slab_index = 0;
        for (std::uint32_t first = 0; first < count; first += slab, ++slab_index) {
            const std::uint32_t tokens = std::min(slab, count - first);
            std::uint16_t* current = a + first * row;
            std::uint16_t* other = b + first * row;
            for (std::uint32_t l = 0; l < layer_count; ++l) {
                const std::string stem =
                    out + "/s" + std::to_string(slab_index) + "_l" + std::to_string(l) + "_";
                q38m::prepare_hyper(layers[l].moe_hyper, current, tokens, ws, s, 0);
                dump(stem + "mixed.bin", ws.mixed, std::size_t(tokens) * H * 2, s);
                q38m::run_moe(layers[l].moe, tokens, ws, s, 0);
                if (tokens == 1) {
                    // the decode block keeps its logits and shared-expert
                    // words internal; the separate entry points (equal to
                    // them bit for bit) produce the oracle's inputs
                    const q38m::MoeLayerWeights& m = layers[l].moe;
                    q38m::moe_router(ws.mixed, m.router, 1, H, ws.logits, s, 0);
                    q38m::moe_shared_expert(ws.mixed, m.shared_gate, m.shared_up, m.shared_down,
                                            m.shared_output_gate, 1, H, m.shared_inter,
                                            ws.shared_scratch, ws.shared_output, ws.shared_gate,
                                            s, 0);
                }
                dump(stem + "logits.bin", ws.logits,
                     std::size_t(tokens) * Q38M_ROUTE_EXPERTS * 4, s);
                dump(stem + "shared_output.bin", ws.shared_output, std::size_t(tokens) * H * 2,
                     s);
                dump(stem + "shared_gate.bin", ws.shared_gate, std::size_t(tokens) * 2, s);
                dump(stem + "block_output.bin", ws.block_output, std::size_t(tokens) * H * 2, s);
                q38m::finish_hyper(current, other, tokens, ws, s, 0);
                std::swap(current, other);
            }
        }
        dump(out + "/final_explicit.bin", layer_count % 2 == 0 ? a : b, state_words * 2, s);

        // pass 2: the stage's own loop from the same initial state
        hip_check(hipMemcpyAsync(a, initial, state_words * 2, hipMemcpyDeviceToDevice, hs),
                  "copy state");
        const std::uint16_t* result =
            q38m::run_prefill_moe(layers.data(), layers.size(), a, b, count, ws, s, 0);
        dump(out + "/final_product.bin", result, state_words * 2, s);
        std::printf("run_moe_check: %u tokens, %u slabs, %u layers done\n", count, slab_index,
                    layer_count);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "run_moe_check: %s\n", e.what());
        return 1;
    }
    for (void* p : ctx.owned) hip_check(hipFree(p), "hipFree");
    hip_check(hipStreamDestroy(hs), "hipStreamDestroy");
    return 0;
}
