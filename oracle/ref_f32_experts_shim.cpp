// C-ABI shim over the reference's F32 expert executor (tools/engine/f32_experts.cpp, compiled from
// the reference sources in place into oracle/_ref/libref_f32_experts.so by oracle/build_oracle.py).
// TEST INFRASTRUCTURE ONLY: it exists so that tests can read the reference's own activation bits.
//
// ref_glu(activation, gate, up, out, n): runs execute_f32_cpu on one expert with hidden = 1,
// intermediate = n, gate weights gate[i], up weights up[i], no biases and the input row {1.0f}, so
// the gate and up sums are exactly 0 + gate[i] * 1 and 0 + up[i] * 1, and captures the activation
// stage (f32_experts.cpp:68-73) through the executor's observe hook. Returns 0, or -1 when the
// executor rejected the inputs (non-finite values, n out of range).
#include "f32_experts.hpp"

#include <cstdint>
#include <cstring>
#include <exception>

using vrambridge::experimental::ExpertJob;
using vrambridge::experimental::F32Activation;
using vrambridge::experimental::F32ExpertWeights;
using vrambridge::experimental::F32Stage;
using vrambridge::experimental::F32Transforms;

extern "C" int ref_glu(int activation, const float * gate, const float * up, float * out, int64_t n) {
    try {
        F32ExpertWeights w{};
        w.hidden = 1;
        w.intermediate = static_cast<std::size_t>(n);
        w.experts = 1;
        w.activation = activation == 1 ? F32Activation::openai_swiglu : F32Activation::silu;
        w.gate.assign(gate, gate + n);
        w.up.assign(up, up + n);
        w.down.assign(static_cast<std::size_t>(n), 0.0f);
        bool seen = false;
        F32Transforms t;
        t.observe = [&](const ExpertJob &, F32Stage stage, const std::vector<float> & values) {
            if (stage != F32Stage::activation) return;
            std::memcpy(out, values.data(), sizeof(float) * values.size());
            seen = true;
        };
        const std::vector<float> input{1.0f};
        const std::vector<ExpertJob> jobs{ExpertJob{0, 0, 0}};
        (void)vrambridge::experimental::execute_f32_cpu(w, input, jobs, t);
        return seen ? 0 : -1;
    } catch (const std::exception &) {
        return -1;
    }
}
