// Expert GEMV for decode and ragged small batches: MXFP4 x Q8_0 and Q8_0 x Q8_0, bit-identical
// to the ggml x86 vec_dot contract.
//
// The CPU dot (tools/trace/cpu_mxfp4_vnni.cpp:49-68) splits every 32-element block into eight
// 4-element lanes and keeps per-lane FMA chains (even/odd blocks for MXFP4; one chain for Q8_0),
// then reduces the eight lanes with a fixed tree. Here one wavefront owns one lane slice k for 64
// rows: lane = row, wave = slice, so
//   - every lane keeps exactly the CPU's chains for its (row, slice) and the final tree over the
//     eight waves reproduces the CPU bits;
//   - the activation slice a wave needs is the same for all its lanes, so it comes through scalar
//     loads (SGPR operands of v_dot2 / v_dot4), costing no VGPRs and no LDS;
//   - each lane loads its whole row slice of weights (K=2880 MXFP4: 180 B codes + 90 B exponents)
//     into VGPRs up front: ~270 B in flight per lane saturates HBM even at batch 1, and the
//     weights are then reused from registers for every token routed to the expert.
// A 512-thread workgroup covers 64 rows (two 32-row bank tiles) of one active expert.
//
// Integer part (MXFP4): v_cvt_scalef32_pk_f16_fp4 with scale 2 turns two e2m1 nibbles into the
// doubled-e2m1 integers {0,1,2,3,4,6,8,12,...} as f16; v_dot2 against f16 activation codes gives
// the lane's 4-product integer exactly (all partial sums are integers below 2^24). The VPSIGNB
// corner case (activation code -128 against a negative weight, cpu_mxfp4_vnni.cpp:43-44) runs on
// a uniform slow path selected per activation row.
//
// Epilogue 1 (fused gate|up bank): the workgroup's 64 rows are gate rows 32p..32p+31 and up rows
// 32p..32p+31, i.e. exactly one 32-element Q8_0 block p of the GLU output; it applies the biases
// and the GLU, requantizes (x86 contract) and writes the down projection's activation row.
#include "vbm_internal.hpp"

namespace vbm {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef const __attribute__((address_space(4))) uint8_t * cptr;   // constant: uniform loads -> s_load

// Constant-address-space view of read-only global data: wave-uniform loads become s_load.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(4))) T * as_const(const void * p) {
    return (const __attribute__((address_space(4))) T *)(p);
}

// A wave-uniform address made explicit (both halves through readfirstlane) so that loads from
// it are selected as scalar loads.
template <class T>
__device__ __forceinline__ T * wave_uniform(T * p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    return reinterpret_cast<T *>((static_cast<uint64_t>(hi) << 32) | lo);
}

constexpr int kThreads = 512;
constexpr int kChunk = 4;        // tokens reduced per barrier

__device__ __forceinline__ half2_t as_half2(unsigned v) { return __builtin_bit_cast(half2_t, v); }

// exp() for the GLU: rounded from double so it matches a correctly rounded expf in practice.
__device__ __forceinline__ float expf_rn(float x) { return static_cast<float>(exp(static_cast<double>(x))); }

__device__ __forceinline__ float glu(int activation, float g0, float u0, float alpha, float limit) {
    if (activation == VBM_ACT_SWIGLU_OAI) {
        const float g = limit < g0 ? limit : g0;                           // std::min(gate, limit)
        const float u = u0 < -limit ? -limit : (limit < u0 ? limit : u0);  // std::clamp(up, -l, l)
        return (g / (1.0f + expf_rn(alpha * (-g)))) * (u + 1.0f);
    }
    return g0 / (1.0f + expf_rn(-g0)) * u0;
}

// Contract minus true product for one 4-element slice: +256*w for every element whose
// activation code is -128 and whose weight is negative (VPSIGNB keeps -128 when negating).
__device__ __forceinline__ float neg128_fix_half(half2_t w01, half2_t w23, unsigned a01, unsigned a23) {
    const half2_t x = as_half2(a01), y = as_half2(a23);
    const float w[4] = {static_cast<float>(w01.x), static_cast<float>(w01.y), static_cast<float>(w23.x),
                        static_cast<float>(w23.y)};
    const float a[4] = {static_cast<float>(x.x), static_cast<float>(x.y), static_cast<float>(y.x),
                        static_cast<float>(y.y)};
    float fix = 0.0f;
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
    int64_t n_slots;
};

struct KernelArgs {
    const uint8_t * bank;
    Shape shape;
    const int32_t * expert_to_slot;
    const uint8_t * xrows;
    XrowLayout lay;
    int64_t n_ids, b_ne1;
    const int32_t * counts;
    const int32_t * offsets;
    const int32_t * rows_list;
    const int32_t * active;
    const int32_t * n_active;
    const float * bias;
    float * dst;
    uint8_t * dst_xrows;
    XrowLayout dst_lay;
    int epilogue, activation;
    float alpha, limit;
};

// One lane's weights: G groups (8 MXFP4 / 4 Q8_0 blocks each: 16 B codes + 8 B exponents or
// scales) and up to 6 tail blocks.
template <int G>
struct LaneWeights {
    u32x4 c[G];
    uint2 m[G];
    unsigned tc[3];
    unsigned tm[2];
};

template <int TYPE, int G>
__device__ __forceinline__ void load_lane(LaneWeights<G> & w, const uint8_t * codes_tile, const uint8_t * meta_tile,
                                          int k, int r, int groups, int tail) {
    const uint8_t * cp = codes_tile + (k * 32 + r) * 16;
    const uint8_t * mp = meta_tile + r * 8;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        if (g < groups) {
            w.c[g] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(cp + g * 4096));
            const u32x2 mv = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(mp + g * 256));
            w.m[g] = make_uint2(mv.x, mv.y);
        }
    }
    constexpr int kCode = TYPE == 39 ? 2 : 4, kMeta = TYPE == 39 ? 1 : 2;
    const uint8_t * tcp = codes_tile + groups * 4096 + (k * 32 + r) * (tail * kCode);
    const uint8_t * tmp = meta_tile + groups * 256 + r * tail * kMeta;
#pragma unroll
    for (int i = 0; i < 3; ++i)
        if (4 * i < tail * kCode) w.tc[i] = *reinterpret_cast<const unsigned *>(tcp + 4 * i);
    unsigned m0 = 0, m1 = 0;
    for (int i = 0; i < tail * kMeta; ++i) {
        const unsigned byte = tmp[i];
        if (i < 4) m0 |= byte << (8 * i);
        else m1 |= byte << (8 * (i - 4));
    }
    w.tm[0] = m0;
    w.tm[1] = m1;
}

// One MXFP4 block of one lane: bytes SEL, SEL+1 of `dw` are the slice's 4 nibbles; the
// activation slice (4 f16 codes) and the block scale are wave-uniform.
template <bool SLOW, int SEL>
__device__ __forceinline__ void mx_block(unsigned dw, int e, u32x2 a, float d, float & acc) {
    const half2_t w01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, SEL);
    const half2_t w23 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, SEL + 1);
    float v = __builtin_amdgcn_fdot2(w23, as_half2(a.y), 0.0f, false);
    v = __builtin_amdgcn_fdot2(w01, as_half2(a.x), v, false);
    if (SLOW) v += neg128_fix_half(w01, w23, a.x, a.y);
    const float s = __builtin_amdgcn_ldexpf(d, e);
    acc = __builtin_fmaf(s, v, acc);
}

// All blocks of one token for one lane (MXFP4): returns even + odd chain.
template <bool SLOW, int G>
__device__ __forceinline__ float mx_token(const LaneWeights<G> & w, cptr act, const float * __restrict__ da_g,
                                          int groups, int tail) {
    const __attribute__((address_space(4))) u32x2 * a = (const __attribute__((address_space(4))) u32x2 *)(act);
    const __attribute__((address_space(4))) float * da = as_const<float>(da_g);
    float even = 0.0f, odd = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        if (g < groups) {
            u32x4 c = w.c[g];
            uint2 ex = w.m[g];
            // Decode inside the token loop: hoisting 180 decoded weights out of it would halve
            // occupancy for no gain at one token per expert.
            asm volatile("" : "+v"(c), "+v"(ex.x), "+v"(ex.y));
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const unsigned dw = q == 0 ? c.x : (q == 1 ? c.y : (q == 2 ? c.z : c.w));
                const unsigned ew = q < 2 ? ex.x : ex.y;
                const int b = g * 8 + 2 * q;
                mx_block<SLOW, 0>(dw, static_cast<signed char>(ew >> ((2 * q & 3) * 8)), a[b], da[b], even);
                mx_block<SLOW, 2>(dw, static_cast<signed char>(ew >> (((2 * q + 1) & 3) * 8)), a[b + 1], da[b + 1], odd);
            }
        }
    }
#pragma unroll
    for (int bt = 0; bt < 6; bt += 2) {
        if (bt < tail) {
            const int b = groups * 8 + bt;
            const unsigned ew = bt < 4 ? w.tm[0] : w.tm[1];
            const int sh = (bt & 3) * 8;
            mx_block<SLOW, 0>(w.tc[bt / 2], static_cast<signed char>(ew >> sh), a[b], da[b], even);
            mx_block<SLOW, 2>(w.tc[bt / 2], static_cast<signed char>(ew >> (sh + 8)), a[b + 1], da[b + 1], odd);
        }
    }
    return even + odd;
}

template <bool SLOW>
__device__ __forceinline__ void q8_block(unsigned w, unsigned short dbits, unsigned a, float d, float & acc) {
    int v = __builtin_amdgcn_sdot4(static_cast<int>(w), static_cast<int>(a), 0, false);
    if (SLOW) v += neg128_fix_i8(w, a);
    const float s = half_bits_to_float(dbits) * d;
    acc = __builtin_fmaf(s, static_cast<float>(v), acc);
}

// All blocks of one token for one lane (Q8_0 weights): one chain.
template <bool SLOW, int G>
__device__ __forceinline__ float q8_token(const LaneWeights<G> & w, cptr act, const float * __restrict__ da_g,
                                          int groups, int tail) {
    const __attribute__((address_space(4))) unsigned * a = (const __attribute__((address_space(4))) unsigned *)(act);
    const __attribute__((address_space(4))) float * da = as_const<float>(da_g);
    float acc = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        if (g < groups) {
            u32x4 c = w.c[g];
            uint2 sc = w.m[g];
            asm volatile("" : "+v"(c), "+v"(sc.x), "+v"(sc.y));
            const int b = g * 4;
            q8_block<SLOW>(c.x, static_cast<unsigned short>(sc.x), a[b], da[b], acc);
            q8_block<SLOW>(c.y, static_cast<unsigned short>(sc.x >> 16), a[b + 1], da[b + 1], acc);
            q8_block<SLOW>(c.z, static_cast<unsigned short>(sc.y), a[b + 2], da[b + 2], acc);
            q8_block<SLOW>(c.w, static_cast<unsigned short>(sc.y >> 16), a[b + 3], da[b + 3], acc);
        }
    }
#pragma unroll
    for (int bt = 0; bt < 3; ++bt) {
        if (bt < tail) {
            const unsigned mw = bt < 2 ? w.tm[0] : w.tm[1];
            q8_block<SLOW>(w.tc[bt], static_cast<unsigned short>(mw >> ((bt & 1) * 16)), a[groups * 4 + bt],
                           da[groups * 4 + bt], acc);
        }
    }
    return acc;
}

template <int TYPE, int G>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(G <= 12 ? 4 : 3))) void expert_gemv_kernel(KernelArgs A) {
    __shared__ float red[kChunk][8][64];
    __shared__ float vals[kChunk][64];
    // Per-expert metadata is read through the constant address space so it stays scalar (a
    // generic-pointer load would be treated as divergent and push the activation loads to VMEM).
    const int a_index = blockIdx.y;
    if (a_index >= *as_const<int32_t>(A.n_active)) return;
    const int expert = as_const<int32_t>(A.active)[a_index];
    const int count = as_const<int32_t>(A.counts)[expert];
    const __attribute__((address_space(4))) int32_t * jobs = as_const<int32_t>(A.rows_list) + as_const<int32_t>(A.offsets)[expert];
    const int slot = A.expert_to_slot ? as_const<int32_t>(A.expert_to_slot)[expert] : expert;
    if (slot < 0 || slot >= A.shape.n_slots || count <= 0) return;

    const Shape S = A.shape;
    const int nb = S.nb;
    const int k = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // lane slice, wave-uniform
    const int lane = threadIdx.x & 63;
    const int r = lane & 31;
    const int tile = blockIdx.x * 2 + (lane >> 5);
    const bool live = tile * 32 < S.rows;
    constexpr int kGroupBlocks = TYPE == 39 ? 8 : 4;
    const int groups = nb / kGroupBlocks, tail = nb % kGroupBlocks;

    LaneWeights<G> w = {};   // lanes past the last row keep zero weights and compute zeros
    if (live) {
        const uint8_t * slot_base = A.bank + static_cast<size_t>(slot) * S.slot_bytes;
        const uint8_t * codes_tile = slot_base + static_cast<size_t>(tile) * 32 * nb * (TYPE == 39 ? 16 : 32);
        const uint8_t * meta_tile = slot_base + S.codes_bytes + static_cast<size_t>(tile) * 32 * nb * (TYPE == 39 ? 1 : 2);
        load_lane<TYPE, G>(w, codes_tile, meta_tile, k, r, groups, tail);
    }
    const int64_t act_slice = static_cast<int64_t>(k) * nb * A.lay.code_entry();

    for (int c0 = 0; c0 < count; c0 += kChunk) {
        const int mcount = count - c0 < kChunk ? count - c0 : kChunk;
        for (int mi = 0; mi < mcount; ++mi) {
            const int64_t j = jobs[c0 + mi];
            const int64_t row = A.b_ne1 == 1 ? j / A.n_ids : j;
            const uint8_t * xr = A.xrows + row * A.lay.stride();
            cptr act = as_const<uint8_t>(wave_uniform(xr + act_slice));
            const float * da = wave_uniform(reinterpret_cast<const float *>(xr + A.lay.da_offset()));
            const int flag = *as_const<int>(wave_uniform(xr + A.lay.flag_offset()));
            // Uniform control flow here keeps the activation loads scalar.
            float v;
            if (TYPE == 39) v = flag ? mx_token<true, G>(w, act, da, groups, tail) : mx_token<false, G>(w, act, da, groups, tail);
            else v = flag ? q8_token<true, G>(w, act, da, groups, tail) : q8_token<false, G>(w, act, da, groups, tail);
            red[mi][k][lane] = v;
        }
        __syncthreads();
        // Final tree over the eight lanes (cpu_mxfp4_vnni.cpp:64-67): ((l0+l4)+(l2+l6))+((l1+l5)+(l3+l7)).
        const int mi = k;                       // wave mi reduces token mi of the chunk
        if (mi < mcount && live) {
            const float * l = &red[mi][0][lane];
            const float s0 = l[4 * 64] + l[0], s1 = l[5 * 64] + l[1 * 64];
            const float s2 = l[6 * 64] + l[2 * 64], s3 = l[7 * 64] + l[3 * 64];
            float v = (s0 + s2) + (s1 + s3);
            const int grow = static_cast<int>(ggml_row(static_cast<int64_t>(tile) * 32 + r, S.rows, S.interleave));
            if (A.bias) v = v + A.bias[static_cast<size_t>(expert) * S.rows + grow];
            if (A.epilogue == 0) A.dst[static_cast<size_t>(jobs[c0 + mi]) * S.rows + grow] = v;
            else vals[mi][lane] = v;
        }
        if (A.epilogue == 1) {
            __syncthreads();
            // Wave mi, lanes 0..31: GLU output element p*32 + lane, gate from local row
            // (lane/16)*32 + lane%16 and up from that row + 16; then Q8_0 (x86 contract).
            if (mi < mcount && lane < 32) {
                const int lr = (lane >> 4) * 32 + (lane & 15);
                const float act = glu(A.activation, vals[mi][lr], vals[mi][lr + 16], A.alpha, A.limit);
                float amax = fabsf(act);
                for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
                const float d = amax / 127.0f;
                const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
                float q = rintf(act * id);
                q = q > 127.0f ? 127.0f : (q < -128.0f ? -128.0f : q);
                const XrowLayout L = A.dst_lay;
                uint8_t * out = A.dst_xrows + static_cast<size_t>(jobs[c0 + mi]) * L.stride();
                const int p = blockIdx.x;                           // output block index
                const int sk = lane >> 2, pos = lane & 3;
                if (L.weight_type == 39)
                    reinterpret_cast<_Float16 *>(out + (static_cast<int64_t>(sk) * L.nb + p) * 8)[pos] = static_cast<_Float16>(q);
                else
                    reinterpret_cast<signed char *>(out + (static_cast<int64_t>(sk) * L.nb + p) * 4)[pos] = static_cast<signed char>(q);
                if (lane == 0) {
                    reinterpret_cast<float *>(out + L.da_offset())[p] = static_cast<float>(static_cast<_Float16>(d));
                    if (p == 0) *reinterpret_cast<int *>(out + L.flag_offset()) = 0;   // requantized codes are never -128
                }
            }
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------ activation rows
// One 32-lane group per (row, block): x86 quantize_row_q8_0, written as an xrow (and optionally
// as ggml Q8_0 blocks). Lane 0 of block 0 clears the row's -128 flag (this quantizer never
// produces -128).
__global__ __launch_bounds__(256) void quantize_expand_kernel(const float * __restrict__ x, int64_t n_rows, int nb,
                                                              int64_t x_stride, XrowLayout L, uint8_t * __restrict__ xrows,
                                                              uint8_t * __restrict__ q8) {
    const int64_t total = n_rows * nb;
    const int64_t bg = blockIdx.x * 8ll + (threadIdx.x >> 5);
    const int e = threadIdx.x & 31;
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

// One workgroup per row: ggml Q8_0 blocks -> xrow, with the row's -128 flag.
__global__ __launch_bounds__(256) void expand_q8_kernel(const uint8_t * __restrict__ q8, int nb, int64_t row_bytes,
                                                        XrowLayout L, uint8_t * __restrict__ xrows) {
    __shared__ int s_flag;
    const int64_t row = blockIdx.x;
    const uint8_t * src = q8 + row * row_bytes;
    uint8_t * out = xrows + row * L.stride();
    if (threadIdx.x == 0) s_flag = 0;
    __syncthreads();
    int neg = 0;
    for (int idx = threadIdx.x; idx < nb * 32; idx += 256) {
        const int b = idx >> 5, e = idx & 31, sk = e >> 2, pos = e & 3;
        const signed char q = static_cast<signed char>(src[b * 34 + 2 + e]);
        neg |= q == -128;
        if (L.weight_type == 39)
            reinterpret_cast<_Float16 *>(out + (static_cast<int64_t>(sk) * nb + b) * 8)[pos] = static_cast<_Float16>(q);
        else
            reinterpret_cast<signed char *>(out + (static_cast<int64_t>(sk) * nb + b) * 4)[pos] = q;
    }
    for (int b = threadIdx.x; b < nb; b += 256)
        reinterpret_cast<float *>(out + L.da_offset())[b] =
            half_bits_to_float(static_cast<uint16_t>(src[b * 34] | (src[b * 34 + 1] << 8)));
    if (neg) atomicOr(&s_flag, 1);
    __syncthreads();
    if (threadIdx.x == 0) *reinterpret_cast<int *>(out + L.flag_offset()) = s_flag;
}

template <int TYPE, int G>
void launch_typed(const GemvArgs & g, const KernelArgs & ka, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((ka.shape.rows + 63) / 64), static_cast<unsigned>(g.max_active));
    hipLaunchKernelGGL((expert_gemv_kernel<TYPE, G>), grid, dim3(kThreads), 0, stream, ka);
    check_hip(hipGetLastError(), "expert GEMV launch");
}

template <int TYPE>
void launch_g(const GemvArgs & g, const KernelArgs & ka, hipStream_t stream) {
    const int groups = ka.shape.nb / (TYPE == 39 ? 8 : 4);
    if (groups <= 4) launch_typed<TYPE, 4>(g, ka, stream);
    else if (groups <= 8) launch_typed<TYPE, 8>(g, ka, stream);
    else if (groups <= 12) launch_typed<TYPE, 12>(g, ka, stream);
    else launch_typed<TYPE, 16>(g, ka, stream);
}

}  // namespace

void launch_quantize_expand(const float * x, int64_t n_rows, int64_t k, int64_t x_stride, const XrowLayout & lay,
                            uint8_t * xrows, uint8_t * q8_blocks, hipStream_t stream) {
    require(k > 0 && k % 32 == 0 && n_rows > 0 && x_stride >= k && lay.nb == k / 32, "quantize shape mismatch");
    const int64_t blocks = n_rows * (k / 32);
    hipLaunchKernelGGL(quantize_expand_kernel, dim3(static_cast<unsigned>((blocks + 7) / 8)), dim3(256), 0, stream, x,
                       n_rows, static_cast<int>(k / 32), x_stride, lay, xrows, q8_blocks);
    check_hip(hipGetLastError(), "quantize launch");
}

void launch_expand_q8(const uint8_t * q8, int64_t n_rows, int64_t row_bytes, const XrowLayout & lay, uint8_t * xrows,
                      hipStream_t stream) {
    require(n_rows > 0 && n_rows < (1ll << 31) && row_bytes == lay.nb * 34, "expand shape mismatch");
    hipLaunchKernelGGL(expand_q8_kernel, dim3(static_cast<unsigned>(n_rows)), dim3(256), 0, stream, q8,
                       static_cast<int>(lay.nb), row_bytes, lay, xrows);
    check_hip(hipGetLastError(), "expand launch");
}

void launch_gemv(const GemvArgs & g, hipStream_t stream) {
    const vbm_bank & bank = *g.bank;
    require(g.max_active >= 1 && g.max_active <= 65535, "active expert bound out of range");
    require(bank.nb <= 128, "expert GEMV supports k <= 4096");
    require(g.epilogue == 0 || (bank.interleave && g.dst_xrows && bank.rows % 64 == 0 &&
                                g.dst_layout.nb == bank.rows / 64),
            "GLU epilogue needs an interleaved gate|up bank with rows % 64 == 0 and a matching down layout");
    require(g.epilogue == 1 || g.dst != nullptr, "missing GEMV output");
    KernelArgs ka{};
    ka.bank = bank.base;
    ka.shape = Shape{static_cast<int>(bank.nb), static_cast<int>(bank.rows), bank.interleave, bank.slot_bytes,
                     bank.geometry().codes_bytes(), bank.n_slots};
    ka.expert_to_slot = g.expert_to_slot;
    ka.xrows = g.xrows;
    ka.lay = XrowLayout{bank.nb, bank.type};
    ka.n_ids = g.n_ids;
    ka.b_ne1 = g.b_ne1;
    ka.counts = g.group.counts;
    ka.offsets = g.group.offsets;
    ka.rows_list = g.group.rows;
    ka.active = g.group.active;
    ka.n_active = g.group.n_active;
    ka.bias = g.bias;
    ka.dst = g.dst;
    ka.dst_xrows = g.dst_xrows;
    ka.dst_lay = g.dst_layout;
    ka.epilogue = g.epilogue;
    ka.activation = g.activation;
    ka.alpha = g.alpha;
    ka.limit = g.limit;
    if (bank.type == VBM_TYPE_MXFP4) launch_g<39>(g, ka, stream);
    else launch_g<8>(g, ka, stream);
}

}  // namespace vbm
