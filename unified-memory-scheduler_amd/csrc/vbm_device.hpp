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
// (float)(1/sum)). Lanes 0..k-1 write ids[0..k) and weights[0..k), and the ids to `ids_lds` too
// when it is given. k <= 64. NPL: logits per lane (n <= 64 * NPL, chosen by the launcher).
template <int NPL>
__device__ __forceinline__ void wave_topk_softmax(const float * logits, int n, int k, int32_t * ids, float * weights,
                                                  int32_t * ids_lds = nullptr) {
    const int lane = threadIdx.x & 63;
    float prev_v = INFINITY;
    int prev_i = -1;
    float sel_v = 0.0f;   // lane j keeps pick j
    int sel_i = -1;
    // The lane's logits stay in registers across the k rounds: one load each instead of one per
    // round.
    float lv[NPL];
#pragma unroll
    for (int c = 0; c < NPL; ++c) lv[c] = lane + 64 * c < n ? logits[lane + 64 * c] : 0.0f;
    for (int j = 0; j < k; ++j) {
        float best = 0.0f;
        int best_i = -1;
#pragma unroll
        for (int c = 0; c < NPL; ++c) {
            const int i = lane + 64 * c;
            const float v = lv[c];
            const bool after_prev = v < prev_v || (v == prev_v && i > prev_i);
            if (i < n && after_prev && (best_i < 0 || v > best)) { best = v; best_i = i; }
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
        if (ids_lds) ids_lds[lane] = sel_i;
    }
}

// Lane-crossing moves inside a row of 16 lanes (DPP): quad_perm [1,0,3,2] = 0xB1, quad_perm
// [2,3,0,1] = 0x4E, row_half_mirror = 0x141, row_mirror = 0x140.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// Maximum over each aligned group of four lanes (all four active).
__device__ __forceinline__ float quad_max(float v) {
    v = fmaxf(v, dpp_move<0xB1>(v));
    return fmaxf(v, dpp_move<0x4E>(v));
}

// Maximum over each half-wave (lanes 0..31, 32..63), all 32 lanes of the half active: quads,
// then mirrored halves of 8 and rows of 16 (DPP), then the two rows through a swizzle with
// xor mask 16.
__device__ __forceinline__ float half_wave_max(float v) {
    v = quad_max(v);
    v = fmaxf(v, dpp_move<0x141>(v));
    v = fmaxf(v, dpp_move<0x140>(v));
    return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F)));
}

constexpr int kMaxRouteExperts = 1024;

// Routing logit as staged for the rank count: NaN reads as -inf so the ranks stay a permutation.
__device__ __forceinline__ float route_key(float v) { return v != v ? -INFINITY : v; }

// Whole-workgroup top-k over n <= kMaxRouteExperts logits already staged in s_val (route_key) with
// s_rank zeroed, in the total order (value desc, then lower index;
// tools/trace/topk-tie-probe.cpp:111-113): the rank of every candidate is the number of elements
// that precede it, counted in 32-element chunks by independent threads and summed with LDS
// atomics, so there is no serial chain of k wave reductions. On return s_ids[j] is pick j
// (j < k). s_val must be 16-byte aligned. All NT threads of the workgroup must call it; it
// starts with a barrier.
template <int NT>
__device__ __forceinline__ void block_topk(int n, int k, const float * s_val, int * s_rank, int32_t * s_ids) {
    __syncthreads();
    const int nq = (n + 31) >> 5;
    for (int w = threadIdx.x; w < n * nq; w += NT) {
        const int q = w / n, c = w - q * n;
        const float vc = s_val[c];
        const int j0 = 32 * q;
        int cnt = 0;
        if (j0 + 32 <= n) {   // full chunk: eight 16-byte LDS reads, all issued before use
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = reinterpret_cast<const float4 *>(s_val + j0)[u];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int j = j0 + 4 * u;
                cnt += (v[u].x > vc || (v[u].x == vc && j < c)) ? 1 : 0;
                cnt += (v[u].y > vc || (v[u].y == vc && j + 1 < c)) ? 1 : 0;
                cnt += (v[u].z > vc || (v[u].z == vc && j + 2 < c)) ? 1 : 0;
                cnt += (v[u].w > vc || (v[u].w == vc && j + 3 < c)) ? 1 : 0;
            }
        } else {
            for (int j = j0; j < n; ++j) {
                const float vj = s_val[j];
                cnt += (vj > vc || (vj == vc && j < c)) ? 1 : 0;
            }
        }
        if (cnt) atomicAdd(&s_rank[c], cnt);
    }
    __syncthreads();
    for (int c = threadIdx.x; c < n; c += NT) {
        const int r = s_rank[c];
        if (r < k) s_ids[r] = c;
    }
    __syncthreads();
}

// ggml soft_max over the k selected logits, in pick order (expf(v - max), sum in double, scale by
// (float)(1/sum)); called by one full wave, returns the weight of pick `lane` (lane < k).
__device__ __forceinline__ float route_softmax(const float * s_val, const int32_t * s_ids, int k, int lane) {
    float max = -INFINITY;
    for (int j = 0; j < k; ++j) {
        const float v = s_val[s_ids[j]];
        max = v > max ? v : max;
    }
    const float e = lane < k ? expf_rn(s_val[s_ids[lane]] - max) : 0.0f;
    double sum = 0.0;
    for (int j = 0; j < k; ++j) sum += static_cast<double>(__shfl(e, j));
    return e * static_cast<float>(1.0 / sum);
}

// x86 quantize_row_q8_0 of one block by one 32-lane group: block bg (row bg / nb, block bg % nb)
// of the fp32 rows x, written into activation rows of the GEMV layout `Layout` (and optionally as
// a ggml Q8_0 block). Lane 0 of block 0 clears the row's -128 flag (this quantizer never produces
// -128). Every lane of the group must call it.
template <class Layout>
__device__ __forceinline__ void quantize_expand_block(const float * __restrict__ x, int64_t n_rows, int nb, int64_t x_stride,
                                                      const Layout & L, uint8_t * __restrict__ xrows,
                                                      uint8_t * __restrict__ q8, int64_t bg, int e) {
    const int64_t total = n_rows * nb;
    const bool live = bg < total;
    const int64_t row = live ? bg / nb : 0, b = live ? bg % nb : 0;
    const float v = live ? x[row * x_stride + b * 32 + e] : 0.0f;
    float amax = fabsf(v);
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
    if (!live) return;
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    float q = rintf(v * id);
    q = q > 127.0f ? 127.0f : (q < -128.0f ? -128.0f : q);
    const _Float16 dh = static_cast<_Float16>(d);
    uint8_t * out = xrows + row * L.stride();
    const int sk = e >> 2, pos = e & 3;
    if (L.weight_type == 39)
        reinterpret_cast<_Float16 *>(out + (static_cast<int64_t>(sk) * nb + b) * 8)[pos] = static_cast<_Float16>(q);
    else
        reinterpret_cast<signed char *>(out + (static_cast<int64_t>(sk) * nb + b) * 4)[pos] = static_cast<signed char>(q);
    if (e == 0) {
        reinterpret_cast<float *>(out + L.da_offset())[b] = static_cast<float>(dh);
        if (b == 0) *reinterpret_cast<int *>(out + L.flag_offset()) = 0;
    }
    if (q8) {
        uint8_t * blk = q8 + bg * 34;
        blk[2 + e] = static_cast<uint8_t>(static_cast<signed char>(q));
        if (e == 0) {
            const uint16_t h = __builtin_bit_cast(uint16_t, dh);
            blk[0] = static_cast<uint8_t>(h & 0xFF);
            blk[1] = static_cast<uint8_t>(h >> 8);
        }
    }
}


}  // namespace vbm
