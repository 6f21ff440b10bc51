// Engine-level executors of the routed-expert path on the GPU, with the reference engine's names
// and semantics (tools/engine/gguf_experts.hpp:14-25, f32_experts.hpp:14-29,
// quantized_cuda.hpp:38-49), so an engine written against them switches by re-linking:
//   load_gguf_experts      one layer's selected experts from a GGUF file (or its shards): the
//                          packed ggml bytes of gate / up / down, their biases and fp32 copies
//   Mxfp4NativeHipDown     the down projection of GPU-resident MXFP4 experts for packed Q8_0
//                          activation rows (one per job), with bias; an ExpertRunner body
// ggml type ids are plain ints here (39 = MXFP4, 8 = Q8_0, 0 = F32), since no ggml header is
// involved. Errors follow the reference: std::invalid_argument for shapes, ids and residency,
// std::runtime_error for device failures and non-finite output.
#pragma once

#include "expert_dispatch.hpp"

#include <array>
#include <cstddef>
#include <cstdint>
#include <filesystem>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

namespace vrambridge::experimental {

enum class F32Activation { silu, openai_swiglu };
enum class F32Stage { gate, up, activation, down };

// Dequantized expert weights of one layer (f32_experts.hpp:17-29): gate / up [experts][intermediate
// rows][hidden], down [experts][hidden rows][intermediate]; biases empty or per expert.
struct F32ExpertWeights {
    std::size_t hidden;
    std::size_t intermediate;
    std::size_t experts;
    F32Activation activation;
    std::vector<float> gate;
    std::vector<float> up;
    std::vector<float> down;
    std::vector<float> gate_bias;
    std::vector<float> up_bias;
    std::vector<float> down_bias;

    void validate() const;
};

// f32_experts.hpp:29-33: observation hooks (only `observe` is honoured by the GPU executor).
struct F32Transforms {
    std::function<void(std::vector<float> &)> gate_up_input;
    std::function<void(std::vector<float> &)> down_input;
    std::function<void(const ExpertJob &, F32Stage, const std::vector<float> &)> observe;
};

// gguf_experts.hpp:14-20: packed_weights[i] holds the selected experts' ggml bytes of gate (0),
// up (1) and down (2) back to back in the order of `original_ids`.
struct LoadedExperts {
    F32ExpertWeights weights;
    std::vector<std::uint32_t> original_ids;
    std::vector<std::string> weight_types;
    std::array<int, 3> quant_types;
    std::array<std::vector<std::uint8_t>, 3> packed_weights;
};

// gguf_experts.cpp:44-140 semantics: 1..16 distinct ids, separate gate / up / down tensors,
// optional F32 biases; weights MXFP4 or Q8_0 (the types this build's banks hold).
LoadedExperts load_gguf_experts(const std::filesystem::path & first_shard, int layer,
                                const std::vector<std::uint32_t> & ids, F32Activation activation);

// quantized_cuda.hpp:38-49 / quantized_cuda.cu:373-453: the selected experts with resident[e] == 1
// are uploaded once into a device bank (slots in expert order) with their down biases; execute()
// takes one packed Q8_0 row of `intermediate` values per job and returns jobs x hidden floats in
// job order, bit-identical to the CPU vec_dot contract (the exact accumulation order).
class Mxfp4NativeHipDown {
public:
    Mxfp4NativeHipDown(const LoadedExperts & weights, const std::vector<std::uint8_t> & resident, int device = 0);
    ~Mxfp4NativeHipDown();
    Mxfp4NativeHipDown(const Mxfp4NativeHipDown &) = delete;
    Mxfp4NativeHipDown & operator=(const Mxfp4NativeHipDown &) = delete;

    std::vector<float> execute(const std::vector<std::uint8_t> & packed_q8, const std::vector<ExpertJob> & jobs);

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

// native_cpu.hpp:11-30 on the GPU: every loaded expert resident in three banks (gate, up,
// down; MXFP4 or Q8_0), the reference engine's CPU executor contract for one input row per job:
// Q8_0 quantization of the input, gate and up projections with biases, the activation, Q8_0
// requantization and the down projection with bias, all in the CPU vec_dot order (bit-identical
// dots). `activations` stops after the activation, `pack_down` quantizes activation rows to the
// ggml Q8_0 bytes `execute_down_packed` consumes. The constructor takes a device index where the
// reference's takes the CPU plugin path.
class NativeHipExperts {
public:
    explicit NativeHipExperts(const LoadedExperts & weights, int device = 0);
    ~NativeHipExperts();
    NativeHipExperts(const NativeHipExperts &) = delete;
    NativeHipExperts & operator=(const NativeHipExperts &) = delete;

    std::vector<float> execute(const std::vector<float> & input, const std::vector<ExpertJob> & jobs,
                               const F32Transforms & observations = {}) const;
    std::vector<float> activations(const std::vector<float> & input, const std::vector<ExpertJob> & jobs,
                                   const F32Transforms & observations = {}) const;
    std::vector<float> execute_down(const std::vector<float> & activations, const std::vector<ExpertJob> & jobs) const;
    std::vector<std::uint8_t> pack_down(const std::vector<float> & activations) const;
    std::vector<float> execute_down_packed(const std::vector<std::uint8_t> & packed, const std::vector<ExpertJob> & jobs) const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace vrambridge::experimental
