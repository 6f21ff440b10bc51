// Expert GEMV for decode and ragged small batches: MXFP4 x Q8_0 and Q8_0 x Q8_0, bit-identical
// to the ggml x86 vec_dot contract.
//
// Work decomposition: one 256-thread workgroup per (32-row tile, active expert). Thread
// t = 32*k + r owns row r of the tile and lane slice k (elements 4k..4k+3 of every 32-block),
// which is exactly one of the eight 32-bit lanes of the CPU dot. It keeps the CPU's per-lane
// FMA chains (even/odd blocks for MXFP4, tools/trace/cpu_mxfp4_vnni.cpp:57-63; one chain for
// Q8_0), so the final tree over the eight slices (cpu_mxfp4_vnni.cpp:64-67) reproduces the CPU
// bits. Weights stream as one 16-byte load per lane per 8 (MXFP4) or 4 (Q8_0) blocks; the
// activation of every token routed to the expert sits in LDS (f16 for the MXFP4 dot2 path, int8
// for dot4). Up to MT tokens share one pass over the weights (GEMV -> small GEMM for ragged
// batches); more tokens loop over chunks.
//
// Integer part (MXFP4): v_cvt_scalef32_pk_f16_fp4 with scale 2 turns two e2m1 nibbles into the
// doubled-e2m1 integers {0,1,2,3,4,6,8,12,...} as f16; v_dot2 against f16 activation codes gives
// the lane's 4-product integer exactly (all partial sums are integers below 2^24). The VPSIGNB
// corner case (activation code -128 against a negative weight, cpu_mxfp4_vnni.cpp:43-44) is
// handled on a uniform slow path selected per token chunk.
#include "vbm_internal.hpp"

namespace vbm {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;

__device__ __forceinline__ half2_t as_half2(unsigned v) { return __builtin_bit_cast(half2_t, v); }

// exp() for the GLU: rounded from double so it matches a correctly rounded expf in practice.
__device__ __forceinline__ float expf_rn(float x) { return static_cast<float>(exp(static_cast<double>(x))); }

__device__ __forceinline__ float glu(int activation, float g0, float u0, float alpha, float limit) {
    if (activation == VBM_ACT_SWIGLU_OAI) {
        const float g = limit < g0 ? limit : g0;                       // std::min(gate, limit)
        const float u = u0 < -limit ? -limit : (limit < u0 ? limit : u0);  // std::clamp(up, -l, l)
        return (g / (1.0f + expf_rn(alpha * (-g)))) * (u + 1.0f);
    }
    return g0 / (1.0f + expf_rn(-g0)) * u0;
}

// Contract minus true product for one 4-element slice: +256*w for every element whose
// activation code is -128 and whose weight is negative (VPSIGNB keeps -128 when negating).
__device__ __forceinline__ float neg128_fix_half(half2_t w01, half2_t w23, half2_t a01, half2_t a23) {
    float fix = 0.0f;
    const float w[4] = {static_cast<float>(w01.x), static_cast<float>(w01.y), static_cast<float>(w23.x),
                        static_cast<float>(w23.y)};
    const float a[4] = {static_cast<float>(a01.x), static_cast<float>(a01.y), static_cast<float>(a23.x),
                        static_cast<float>(a23.y)};
    for (int i = 0; i < 4; ++i)
        if (a[i] == -128.0f && w[i] < 0.0f) fix += 256.0f * w[i];
    return fix;
}
__device__ __forceinline__ int neg128_fix_i8(unsigned w, unsigned a) {
    int fix = 0;
    for (int i = 0; i < 4; ++i) {
        const int wi = static_cast<signed char>(w >> (8 * i)), ai = static_cast<signed char>(a >> (8 * i));
        if (ai == -128 && wi < 0) fix += 256 * wi;
    }
    return fix;
}

struct Shape {
    int nb;             // blocks per row
    int rows;           // rows per expert (bank rows)
    int interleave;
    size_t slot_bytes;
    int64_t codes_bytes;
};

// LDS carve-up (bytes): act [MT][8][nb] x (8 B MXFP4 | 4 B Q8_0), da [MT][nb] f32,
// red [MT][8][32] f32, gu [MT][32] f32, misc ints.
template <int TYPE, int MT>
struct LdsPlan {
    static constexpr int act_entry = TYPE == 39 ? 8 : 4;
    __host__ __device__ static size_t act_bytes(int nb) { return static_cast<size_t>(MT) * 8 * nb * act_entry; }
    __host__ __device__ static size_t da_offset(int nb) { return act_bytes(nb); }
    __host__ __device__ static size_t red_offset(int nb) { return da_offset(nb) + static_cast<size_t>(MT) * nb * 4; }
    __host__ __device__ static size_t gu_offset(int nb) { return red_offset(nb) + static_cast<size_t>(MT) * 8 * 32 * 4; }
    __host__ __device__ static size_t total(int nb) { return gu_offset(nb) + static_cast<size_t>(MT) * 32 * 4; }
};

// Stage the activation of token slot m (Q8_0 blocks in global memory) into LDS.
template <int TYPE, int MT>
__device__ void stage_q8(uint8_t * lds, const uint8_t * __restrict__ src, int nb, int m, int & neg128) {
    const int t = threadIdx.x;
    float * da = reinterpret_cast<float *>(lds + LdsPlan<TYPE, MT>::da_offset(nb));
    for (int idx = t; idx < nb * 32; idx += kThreads) {
        const int b = idx >> 5, e = idx & 31;
        const signed char q = static_cast<signed char>(src[b * 34 + 2 + e]);
        const int k = e >> 2, p = e & 3;
        if (q == -128) neg128 = 1;
        if (TYPE == 39) {
            reinterpret_cast<_Float16 *>(lds)[((m * 8 + k) * nb + b) * 4 + p] = static_cast<_Float16>(q);
        } else {
            reinterpret_cast<signed char *>(lds)[((m * 8 + k) * nb + b) * 4 + p] = q;
        }
    }
    for (int b = t; b < nb; b += kThreads)
        da[m * nb + b] = half_bits_to_float(static_cast<uint16_t>(src[b * 34] | (src[b * 34 + 1] << 8)));
}

// Quantize an fp32 row to Q8_0 (x86 contract) straight into LDS: 8 blocks per round, 32 threads
// per block, amax by a 32-lane butterfly (exact in any order).
template <int TYPE, int MT>
__device__ void stage_f32(uint8_t * lds, const float * __restrict__ src, int nb, int m) {
    const int t = threadIdx.x;
    float * da = reinterpret_cast<float *>(lds + LdsPlan<TYPE, MT>::da_offset(nb));
    const int rounds = (nb + 7) / 8;
    for (int round = 0; round < rounds; ++round) {
        const int b = round * 8 + (t >> 5), e = t & 31;
        const bool live = b < nb;
        const float x = live ? src[b * 32 + e] : 0.0f;
        float amax = fabsf(x);
        for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
        if (live) {
            const float d = amax / 127.0f;
            const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
            float q = rintf(x * id);
            q = q > 127.0f ? 127.0f : (q < -128.0f ? -128.0f : q);
            const int k = e >> 2, p = e & 3;
            if (TYPE == 39) {
                reinterpret_cast<_Float16 *>(lds)[((m * 8 + k) * nb + b) * 4 + p] = static_cast<_Float16>(q);
            } else {
                reinterpret_cast<signed char *>(lds)[((m * 8 + k) * nb + b) * 4 + p] = static_cast<signed char>(q);
            }
            if (e == 0) da[m * nb + b] = static_cast<float>(static_cast<_Float16>(d));
        }
    }
}

// One MXFP4 block for one lane slice: bytes SEL and SEL+1 of `dw` hold the slice's 4 nibbles.
// v = the lane's exact contract integer; the FMA extends the block-parity chain PAR.
template <int MT, bool SLOW, int SEL, int PAR>
__device__ __forceinline__ void mx_block(unsigned dw, int e, int b, const uint8_t * lds, const float * da, int nb,
                                         int k, int mcount, float (&acc)[MT][2]) {
    const half2_t w01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, SEL);
    const half2_t w23 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, SEL + 1);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        if (m < mcount) {
            const uint2 a = *reinterpret_cast<const uint2 *>(lds + ((m * 8 + k) * nb + b) * 8);
            float v = __builtin_amdgcn_fdot2(w23, as_half2(a.y), 0.0f, false);
            v = __builtin_amdgcn_fdot2(w01, as_half2(a.x), v, false);
            if (SLOW) v += neg128_fix_half(w01, w23, as_half2(a.x), as_half2(a.y));
            const float s = __builtin_amdgcn_ldexpf(da[m * nb + b], e);
            acc[m][PAR] = __builtin_fmaf(s, v, acc[m][PAR]);
        }
    }
}

// Main loop, MXFP4 weights. acc[m][parity] are the lane's even/odd block chains.
template <int MT, bool SLOW>
__device__ __forceinline__ void mx_loop(const uint8_t * __restrict__ codes_tile, const uint8_t * __restrict__ exps_tile,
                                        const uint8_t * lds, int nb, int k, int r, int mcount, float (&acc)[MT][2]) {
    const int groups = nb >> 3, tail = nb & 7;
    const float * da = reinterpret_cast<const float *>(lds + LdsPlan<39, MT>::da_offset(nb));
    const uint8_t * cp = codes_tile + (k * 32 + r) * 16;
    const uint8_t * ep = exps_tile + r * 8;
    for (int g = 0; g < groups; ++g) {
        const u32x4 c = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(cp + g * 4096));
        const uint2 ex = *reinterpret_cast<const uint2 *>(ep + g * 256);
        const int b = g * 8;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const unsigned dw = q == 0 ? c.x : (q == 1 ? c.y : (q == 2 ? c.z : c.w));
            const unsigned ew = q < 2 ? ex.x : ex.y;
            const int e0 = static_cast<signed char>(ew >> ((2 * q & 3) * 8));
            const int e1 = static_cast<signed char>(ew >> (((2 * q + 1) & 3) * 8));
            mx_block<MT, SLOW, 0, 0>(dw, e0, b + 2 * q, lds, da, nb, k, mcount, acc);
            mx_block<MT, SLOW, 2, 1>(dw, e1, b + 2 * q + 1, lds, da, nb, k, mcount, acc);
        }
    }
    // Tail blocks (nb % 8, always even): pairs of blocks, even then odd.
    for (int bt = 0; bt < tail; bt += 2) {
        const int b = groups * 8 + bt;
        const unsigned dw = *reinterpret_cast<const unsigned *>(codes_tile + groups * 4096 + (k * 32 + r) * (tail * 2) + bt * 2);
        const uint8_t * et = exps_tile + groups * 256 + r * tail + bt;
        mx_block<MT, SLOW, 0, 0>(dw, static_cast<signed char>(et[0]), b, lds, da, nb, k, mcount, acc);
        mx_block<MT, SLOW, 2, 1>(dw, static_cast<signed char>(et[1]), b + 1, lds, da, nb, k, mcount, acc);
    }
}

// Main loop, Q8_0 weights: one FMA chain per lane (acc[m][0]).
template <int MT, bool SLOW>
__device__ __forceinline__ void q8_loop(const uint8_t * __restrict__ codes_tile, const uint8_t * __restrict__ scales_tile,
                                        const uint8_t * lds, int nb, int k, int r, int mcount, float (&acc)[MT][2]) {
    const int groups = nb >> 2, tail = nb & 3;
    const float * da = reinterpret_cast<const float *>(lds + LdsPlan<8, MT>::da_offset(nb));
    const uint8_t * cp = codes_tile + (k * 32 + r) * 16;
    const uint8_t * sp = scales_tile + r * 8;
    for (int g = 0; g < groups; ++g) {
        const u32x4 c = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(cp + g * 4096));
        const uint2 sc = *reinterpret_cast<const uint2 *>(sp + g * 256);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const unsigned w = j == 0 ? c.x : (j == 1 ? c.y : (j == 2 ? c.z : c.w));
            const float dw = half_bits_to_float(static_cast<uint16_t>((j < 2 ? sc.x : sc.y) >> ((j & 1) * 16)));
            const int b = g * 4 + j;
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                if (m < mcount) {
                    const unsigned a = *reinterpret_cast<const unsigned *>(lds + ((m * 8 + k) * nb + b) * 4);
                    int v = __builtin_amdgcn_sdot4(static_cast<int>(w), static_cast<int>(a), 0, false);
                    if (SLOW) v += neg128_fix_i8(w, a);
                    const float s = dw * da[m * nb + b];
                    acc[m][0] = __builtin_fmaf(s, static_cast<float>(v), acc[m][0]);
                }
            }
        }
    }
    for (int bt = 0; bt < tail; ++bt) {
        const int b = groups * 4 + bt;
        const unsigned w = *reinterpret_cast<const unsigned *>(codes_tile + groups * 4096 + (k * 32 + r) * (tail * 4) + bt * 4);
        const uint16_t bits = *reinterpret_cast<const uint16_t *>(scales_tile + groups * 256 + r * tail * 2 + bt * 2);
        const float dw = half_bits_to_float(bits);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m < mcount) {
                const unsigned a = *reinterpret_cast<const unsigned *>(lds + ((m * 8 + k) * nb + b) * 4);
                int v = __builtin_amdgcn_sdot4(static_cast<int>(w), static_cast<int>(a), 0, false);
                if (SLOW) v += neg128_fix_i8(w, a);
                const float s = dw * da[m * nb + b];
                acc[m][0] = __builtin_fmaf(s, static_cast<float>(v), acc[m][0]);
            }
        }
    }
}

struct KernelArgs {
    const uint8_t * bank;
    Shape shape;
    const int32_t * expert_to_slot;
    const uint8_t * act_q8;
    const float * act_f32;
    int64_t act_stride;
    int64_t n_ids, b_ne1;
    const int32_t * counts;
    const int32_t * offsets;
    const int32_t * rows_list;
    const int32_t * active;
    const int32_t * n_active;
    const float * bias;
    float * dst;
    int epilogue, activation;
    float alpha, limit;
};

template <int TYPE, int MT>
__global__ __launch_bounds__(kThreads) void expert_gemv_kernel(KernelArgs A) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    using P = LdsPlan<TYPE, MT>;
    const int a_index = blockIdx.y;
    if (a_index >= *A.n_active) return;
    const int expert = A.active[a_index];
    const int count = A.counts[expert];
    const int32_t * jobs = A.rows_list + A.offsets[expert];
    const int slot = A.expert_to_slot ? A.expert_to_slot[expert] : expert;
    if (slot < 0 || count <= 0) return;

    const Shape S = A.shape;
    const int nb = S.nb;
    const int t = threadIdx.x, k = t >> 5, r = t & 31;
    const int tile = blockIdx.x;
    const uint8_t * slot_base = A.bank + static_cast<size_t>(slot) * S.slot_bytes;
    const uint8_t * codes_tile = slot_base + static_cast<size_t>(tile) * 32 * nb * (TYPE == 39 ? 16 : 32);
    const uint8_t * meta_tile = slot_base + S.codes_bytes + static_cast<size_t>(tile) * 32 * nb * (TYPE == 39 ? 1 : 2);
    float * red = reinterpret_cast<float *>(lds + P::red_offset(nb));
    float * gu = reinterpret_cast<float *>(lds + P::gu_offset(nb));

    for (int c0 = 0; c0 < count; c0 += MT) {
        const int mcount = count - c0 < MT ? count - c0 : MT;
        int neg128 = 0;
        for (int m = 0; m < mcount; ++m) {
            const int64_t j = jobs[c0 + m];
            const int64_t row = A.b_ne1 == 1 ? j / A.n_ids : j;
            if (A.act_q8) stage_q8<TYPE, MT>(lds, A.act_q8 + row * A.act_stride, nb, m, neg128);
            else stage_f32<TYPE, MT>(lds, A.act_f32 + row * A.act_stride, nb, m);
        }
        const bool slow = __syncthreads_or(neg128) != 0;

        float acc[MT][2];
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m][0] = acc[m][1] = 0.0f;
        if (TYPE == 39) {
            if (slow) mx_loop<MT, true>(codes_tile, meta_tile, lds, nb, k, r, mcount, acc);
            else mx_loop<MT, false>(codes_tile, meta_tile, lds, nb, k, r, mcount, acc);
        } else {
            if (slow) q8_loop<MT, true>(codes_tile, meta_tile, lds, nb, k, r, mcount, acc);
            else q8_loop<MT, false>(codes_tile, meta_tile, lds, nb, k, r, mcount, acc);
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) red[(m * 8 + k) * 32 + r] = acc[m][0] + acc[m][1];
        __syncthreads();

        // Final tree over the eight lanes (cpu_mxfp4_vnni.cpp:64-67): ((l0+l4)+(l2+l6))+((l1+l5)+(l3+l7)).
        const int m = t >> 5;
        float v = 0.0f;
        int grow = 0;
        if (m < mcount) {
            const float * l = red + m * 8 * 32 + r;
            const float s0 = l[4 * 32] + l[0], s1 = l[5 * 32] + l[1 * 32];
            const float s2 = l[6 * 32] + l[2 * 32], s3 = l[7 * 32] + l[3 * 32];
            v = (s0 + s2) + (s1 + s3);
            grow = static_cast<int>(ggml_row(static_cast<int64_t>(tile) * 32 + r, S.rows, S.interleave));
            if (A.bias) v = v + A.bias[static_cast<size_t>(expert) * S.rows + grow];
        }
        if (A.epilogue == 0) {
            if (m < mcount) A.dst[static_cast<size_t>(jobs[c0 + m]) * S.rows + grow] = v;
        } else {
            if (m < mcount) gu[m * 32 + r] = v;
            __syncthreads();
            if (m < mcount && r < 16) {
                const int half = S.rows / 2;
                const float out = glu(A.activation, gu[m * 32 + r], gu[m * 32 + 16 + r], A.alpha, A.limit);
                A.dst[static_cast<size_t>(jobs[c0 + m]) * half + tile * 16 + r] = out;
            }
        }
        __syncthreads();
    }
}

template <int TYPE, int MT>
void launch_typed(const GemvArgs & g, const KernelArgs & ka, hipStream_t stream) {
    const size_t lds = LdsPlan<TYPE, MT>::total(ka.shape.nb);
    require(lds <= 160 * 1024, "expert GEMV activation tile exceeds LDS");
    const dim3 grid(static_cast<unsigned>(ka.shape.rows / 32), static_cast<unsigned>(g.max_active));
    hipLaunchKernelGGL((expert_gemv_kernel<TYPE, MT>), grid, dim3(kThreads), lds, stream, ka);
    check_hip(hipGetLastError(), "expert GEMV launch");
}

template <int TYPE>
void launch_mt(const GemvArgs & g, const KernelArgs & ka, hipStream_t stream) {
    if (g.max_per_expert <= 1) launch_typed<TYPE, 1>(g, ka, stream);
    else if (g.max_per_expert <= 2) launch_typed<TYPE, 2>(g, ka, stream);
    else if (g.max_per_expert <= 4) launch_typed<TYPE, 4>(g, ka, stream);
    else launch_typed<TYPE, 8>(g, ka, stream);
}

}  // namespace

void launch_gemv(const GemvArgs & g, hipStream_t stream) {
    const vbm_bank & bank = *g.bank;
    require(g.max_active >= 1 && g.max_active <= 65535, "active expert bound out of range");
    require(g.epilogue == 0 || (bank.interleave && g.dst), "GLU epilogue needs an interleaved gate|up bank");
    KernelArgs ka{};
    ka.bank = bank.base;
    ka.shape = Shape{static_cast<int>(bank.nb), static_cast<int>(bank.rows), bank.interleave, bank.slot_bytes,
                     bank.geometry().codes_bytes()};
    ka.expert_to_slot = g.expert_to_slot;
    ka.act_q8 = g.act_q8;
    ka.act_f32 = g.act_f32;
    ka.act_stride = g.act_stride;
    ka.n_ids = g.n_ids;
    ka.b_ne1 = g.b_ne1;
    ka.counts = g.group.counts;
    ka.offsets = g.group.offsets;
    ka.rows_list = g.group.rows;
    ka.active = g.group.active;
    ka.n_active = g.group.n_active;
    ka.bias = g.bias;
    ka.dst = g.dst;
    ka.epilogue = g.epilogue;
    ka.activation = g.activation;
    ka.alpha = g.alpha;
    ka.limit = g.limit;
    if (bank.type == VBM_TYPE_MXFP4) launch_mt<39>(g, ka, stream);
    else launch_mt<8>(g, ka, stream);
}

}  // namespace vbm
