// Device helpers shared by the routing and GEMV kernels.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/vbmoe.h"

namespace vbm {

// exp() for the GLU and the softmax: rounded from double so it matches a correctly rounded expf
// (glibc expf) in practice.
__device__ __forceinline__ float expf_rn(float x) { return static_cast<float>(exp(static_cast<double>(x))); }

// SwiGLU-OAI (x = min(g, limit), y = clamp(u, -limit, limit), (x / (1 + exp(alpha * -x))) * (y + 1),
// tools/engine/native_cpu.cpp:155-158) or SiLU gate (g / (1 + exp(-g)) * u,
// tools/engine/f32_experts.cpp:253-254); min/clamp written as std::min / std::clamp evaluate.
__device__ __forceinline__ float glu(int activation, float g0, float u0, float alpha, float limit) {
    if (activation == VBM_ACT_SWIGLU_OAI) {
        const float g = limit < g0 ? limit : g0;
        const float u = u0 < -limit ? -limit : (limit < u0 ? limit : u0);
        return (g / (1.0f + expf_rn(alpha * (-g)))) * (u + 1.0f);
    }
    return g0 / (1.0f + expf_rn(-g0)) * u0;
}

// One wavefront: top-k of `logits[0..n)` in the total order (value desc, then lower index;
// tools/trace/topk-tie-probe.cpp:111-113), pick j being the best element strictly after pick j-1,
// then ggml soft_max over the k selected values (expf(v - max), sum in double, scale by
// (float)(1/sum)). Lane 0 writes ids[0..k) and weights[0..k). k <= 64.
__device__ __forceinline__ void wave_topk_softmax(const float * logits, int n, int k, int32_t * ids, float * weights) {
    const int lane = threadIdx.x & 63;
    float prev_v = INFINITY;
    int prev_i = -1;
    float sel_v = 0.0f;   // lane j keeps pick j
    int sel_i = -1;
    for (int j = 0; j < k; ++j) {
        float best = 0.0f;
        int best_i = -1;
        for (int i = lane; i < n; i += 64) {
            const float v = logits[i];
            const bool after_prev = v < prev_v || (v == prev_v && i > prev_i);
            if (after_prev && (best_i < 0 || v > best)) { best = v; best_i = i; }
        }
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(best, off);
            const int oi = __shfl_xor(best_i, off);
            const bool better = oi >= 0 && (best_i < 0 || ov > best || (ov == best && oi < best_i));
            if (better) { best = ov; best_i = oi; }
        }
        if (lane == j) { sel_v = best; sel_i = best_i; }
        prev_v = best;
        prev_i = best_i;
    }
    // softmax over the selected values, in pick order (lane j holds pick j)
    float max = -INFINITY;
    for (int j = 0; j < k; ++j) {
        const float v = __shfl(sel_v, j);
        max = v > max ? v : max;
    }
    const float e = lane < k ? expf_rn(sel_v - max) : 0.0f;
    double sum = 0.0;
    for (int j = 0; j < k; ++j) sum += static_cast<double>(__shfl(e, j));
    const float scale = static_cast<float>(1.0 / sum);
    if (lane < k) {
        ids[lane] = sel_i;
        weights[lane] = e * scale;
    }
}

}  // namespace vbm
