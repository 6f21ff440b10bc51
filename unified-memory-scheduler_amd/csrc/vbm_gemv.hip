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
#include "vbm_device.hpp"
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

constexpr int kDepth = 4;    // weight groups in flight per lane (ring buffer)

// One group of one lane: 16 B of codes (8 MXFP4 blocks x 2 B or 4 Q8_0 blocks x 4 B) and 8 B of
// exponents (MXFP4) or fp16 scales (Q8_0).
struct Group {
    u32x4 c;
    u32x2 m;
};

__device__ __forceinline__ Group load_group(const uint8_t * cp, const uint8_t * mp, int g) {
    Group r;
    r.c = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(cp + g * 4096));
    r.m = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(mp + g * 256));
    return r;
}

// One MXFP4 block of one lane for MT tokens: bytes SEL, SEL+1 of `dw` are the slice's 4 nibbles;
// the activation slice (4 f16 codes, 8 B per block) and the block scale of each token are read
// from LDS with wave-uniform addresses (broadcast).
template <int MT, bool SLOW, int SEL, int PAR>
__device__ __forceinline__ void mx_block(unsigned dw, int e, int b, const uint8_t * la, const float * lda,
                                         int tok_bytes, int mcount, float (&acc)[MT][2]) {
    const half2_t w01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, SEL);
    const half2_t w23 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, SEL + 1);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        if (m < mcount) {
            const u32x2 a = *reinterpret_cast<const u32x2 *>(la + m * tok_bytes + b * 8);
            const float d = *reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(lda) + m * tok_bytes + b * 4);
            float v = __builtin_amdgcn_fdot2(w23, as_half2(a.y), 0.0f, false);
            v = __builtin_amdgcn_fdot2(w01, as_half2(a.x), v, false);
            if (SLOW) v += neg128_fix_half(w01, w23, a.x, a.y);
            const float s = __builtin_amdgcn_ldexpf(d, e);
            acc[m][PAR] = __builtin_fmaf(s, v, acc[m][PAR]);
        }
    }
}

// Eight MXFP4 blocks (one group, starting at block b) for MT tokens.
template <int MT, bool SLOW>
__device__ __forceinline__ void mx_group(const Group & grp, int b, const uint8_t * la, const float * lda, int tok_bytes,
                                         int mcount, float (&acc)[MT][2]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const unsigned dw = q == 0 ? grp.c.x : (q == 1 ? grp.c.y : (q == 2 ? grp.c.z : grp.c.w));
        const unsigned ew = q < 2 ? grp.m.x : grp.m.y;
        mx_block<MT, SLOW, 0, 0>(dw, static_cast<signed char>(ew >> ((2 * q & 3) * 8)), b + 2 * q, la, lda, tok_bytes,
                                 mcount, acc);
        mx_block<MT, SLOW, 2, 1>(dw, static_cast<signed char>(ew >> (((2 * q + 1) & 3) * 8)), b + 2 * q + 1, la, lda,
                                 tok_bytes, mcount, acc);
    }
}

template <int MT, bool SLOW>
__device__ __forceinline__ void q8_block(unsigned w, unsigned short dbits, int b, const uint8_t * la, const float * lda,
                                         int tok_bytes, int mcount, float (&acc)[MT][2]) {
    const float dw = half_bits_to_float(dbits);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        if (m < mcount) {
            const unsigned a = *reinterpret_cast<const unsigned *>(la + m * tok_bytes + b * 4);
            const float d = *reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(lda) + m * tok_bytes + b * 4);
            int v = __builtin_amdgcn_sdot4(static_cast<int>(w), static_cast<int>(a), 0, false);
            if (SLOW) v += neg128_fix_i8(w, a);
            const float s = dw * d;
            acc[m][0] = __builtin_fmaf(s, static_cast<float>(v), acc[m][0]);
        }
    }
}

// Four Q8_0 blocks (one group, starting at block b) for MT tokens: one chain per lane.
template <int MT, bool SLOW>
__device__ __forceinline__ void q8_group(const Group & grp, int b, const uint8_t * la, const float * lda, int tok_bytes,
                                         int mcount, float (&acc)[MT][2]) {
    q8_block<MT, SLOW>(grp.c.x, static_cast<unsigned short>(grp.m.x), b, la, lda, tok_bytes, mcount, acc);
    q8_block<MT, SLOW>(grp.c.y, static_cast<unsigned short>(grp.m.x >> 16), b + 1, la, lda, tok_bytes, mcount, acc);
    q8_block<MT, SLOW>(grp.c.z, static_cast<unsigned short>(grp.m.y), b + 2, la, lda, tok_bytes, mcount, acc);
    q8_block<MT, SLOW>(grp.c.w, static_cast<unsigned short>(grp.m.y >> 16), b + 3, la, lda, tok_bytes, mcount, acc);
}

// Issues the first kDepth groups of one lane's row slice (before activation staging, so the
// weight stream is already in flight while the activation arrives).
__device__ __forceinline__ void preload_ring(Group (&ring)[kDepth], const uint8_t * cp, const uint8_t * mp, int groups,
                                             bool live) {
#pragma unroll
    for (int i = 0; i < kDepth; ++i) {
        ring[i] = Group{};
        if (live && i < groups) ring[i] = load_group(cp, mp, i);
    }
}

// Streams one lane's row slice once through the kDepth-deep register ring, applying every
// staged token to each group as it arrives.
template <int TYPE, int MT, bool SLOW>
__device__ __forceinline__ void stream_lane(Group (&ring)[kDepth], const uint8_t * codes_tile, const uint8_t * meta_tile,
                                            int k, int r, int nb, bool live, const uint8_t * la, const float * lda,
                                            int tok_bytes, int mcount, float (&acc)[MT][2]) {
    constexpr int kGroupBlocks = TYPE == 39 ? 8 : 4;
    const int groups = nb / kGroupBlocks, tail = nb % kGroupBlocks;
    const uint8_t * cp = codes_tile + (k * 32 + r) * 16;
    const uint8_t * mp = meta_tile + r * 8;
    for (int g0 = 0; g0 < groups; g0 += kDepth) {
#pragma unroll
        for (int i = 0; i < kDepth; ++i) {
            const int g = g0 + i;
            if (g < groups) {
                const Group cur = ring[i];
                if (live && g + kDepth < groups) ring[i] = load_group(cp, mp, g + kDepth);
                if (TYPE == 39) mx_group<MT, SLOW>(cur, g * 8, la, lda, tok_bytes, mcount, acc);
                else q8_group<MT, SLOW>(cur, g * 4, la, lda, tok_bytes, mcount, acc);
            }
        }
    }
    // Tail blocks past the last full group (MXFP4: nb % 8 in {0,2,4,6}; Q8_0: nb % 4).
    constexpr int kCode = TYPE == 39 ? 2 : 4, kMeta = TYPE == 39 ? 1 : 2;
    const uint8_t * tcp = codes_tile + groups * 4096 + (k * 32 + r) * (tail * kCode);
    const uint8_t * tmp = meta_tile + groups * 256 + r * tail * kMeta;
    for (int bt = 0; bt < tail; bt += (TYPE == 39 ? 2 : 1)) {
        const unsigned cw = live ? *reinterpret_cast<const unsigned *>(tcp + bt * kCode) : 0u;
        if (TYPE == 39) {
            const int e0 = live ? static_cast<signed char>(tmp[bt]) : 0;
            const int e1 = live ? static_cast<signed char>(tmp[bt + 1]) : 0;
            mx_block<MT, SLOW, 0, 0>(cw, e0, groups * 8 + bt, la, lda, tok_bytes, mcount, acc);
            mx_block<MT, SLOW, 2, 1>(cw, e1, groups * 8 + bt + 1, la, lda, tok_bytes, mcount, acc);
        } else {
            const unsigned short dbits = live ? *reinterpret_cast<const unsigned short *>(tmp + bt * 2) : 0;
            q8_block<MT, SLOW>(cw, dbits, groups * 4 + bt, la, lda, tok_bytes, mcount, acc);
        }
    }
}

// Final tree over the eight lane slices (cpu_mxfp4_vnni.cpp:64-67):
// ((l0+l4)+(l2+l6))+((l1+l5)+(l3+l7)); `l` points at slice 0 of one row, slices 64 floats apart.
__device__ __forceinline__ float lane_tree(const float * l) {
    const float s0 = l[4 * 64] + l[0], s1 = l[5 * 64] + l[1 * 64];
    const float s2 = l[6 * 64] + l[2 * 64], s3 = l[7 * 64] + l[3 * 64];
    return (s0 + s2) + (s1 + s3);
}

// GLU of one 32-element output block (wave lanes 0..31; gate from local row (lane/16)*32 +
// lane%16 of `vals`, up from that row + 16), then x86 Q8_0 quantization into activation row
// `out` at block p.
__device__ __forceinline__ void glu_requant_block(const float * vals, int lane, int p, uint8_t * out, const XrowLayout & L,
                                                  int activation, float alpha, float limit) {
    const int lr = (lane >> 4) * 32 + (lane & 15);
    const float act = glu(activation, vals[lr], vals[lr + 16], alpha, limit);
    float amax = fabsf(act);
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    float q = rintf(act * id);
    q = q > 127.0f ? 127.0f : (q < -128.0f ? -128.0f : q);
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

template <int TYPE, int MT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void expert_gemv_kernel(KernelArgs A) {
    __shared__ float red[MT][8][64];
    __shared__ float vals[MT][64];
    __shared__ int s_flag;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_tok[];   // MT activation rows
    // Per-expert metadata is read through the constant address space so it stays scalar.
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
    const bool live = tile * 32 < S.rows;                              // the last tile pair may be half
    const uint8_t * slot_base = A.bank + static_cast<size_t>(slot) * S.slot_bytes;
    const uint8_t * codes_tile = slot_base + static_cast<size_t>(live ? tile : 0) * 32 * nb * (TYPE == 39 ? 16 : 32);
    const uint8_t * meta_tile = slot_base + S.codes_bytes + static_cast<size_t>(live ? tile : 0) * 32 * nb * (TYPE == 39 ? 1 : 2);
    const int copy_bytes = static_cast<int>(A.lay.flag_offset());        // codes + scales of a row
    const int tok_bytes = (copy_bytes + 15) & ~15;
    const uint8_t * la = lds_tok + static_cast<int64_t>(k) * nb * A.lay.code_entry();
    const float * lda = reinterpret_cast<const float *>(lds_tok + A.lay.da_offset());

    constexpr int kGroupBlocks = TYPE == 39 ? 8 : 4;
    const int groups = nb / kGroupBlocks;
    const uint8_t * cp = codes_tile + (k * 32 + r) * 16;
    const uint8_t * mp = meta_tile + r * 8;

    for (int c0 = 0; c0 < count; c0 += MT) {
        const int mcount = count - c0 < MT ? count - c0 : MT;
        Group ring[kDepth];
        preload_ring(ring, cp, mp, groups, live);
        // Stage the chunk's activation rows (and their -128 flags) in LDS.
        if (threadIdx.x == 0) s_flag = 0;
        __syncthreads();
        int flag = 0;
        for (int mi = 0; mi < mcount; ++mi) {
            const int64_t j = jobs[c0 + mi];
            const int64_t row = A.b_ne1 == 1 ? j / A.n_ids : j;
            const uint8_t * xr = A.xrows + row * A.lay.stride();
            uint8_t * dst = lds_tok + mi * tok_bytes;
            for (int i = threadIdx.x; i * 16 < copy_bytes - 15; i += kThreads)
                *reinterpret_cast<u32x4 *>(dst + i * 16) = *reinterpret_cast<const u32x4 *>(xr + i * 16);
            for (int i = (copy_bytes & ~15) + threadIdx.x * 4; i < copy_bytes; i += kThreads * 4)
                *reinterpret_cast<unsigned *>(dst + i) = *reinterpret_cast<const unsigned *>(xr + i);
            if (threadIdx.x == 0) flag |= *reinterpret_cast<const int *>(xr + A.lay.flag_offset());
        }
        if (threadIdx.x == 0 && flag) s_flag = 1;
        __syncthreads();
        float acc[MT][2];
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m][0] = acc[m][1] = 0.0f;
        if (s_flag) stream_lane<TYPE, MT, true>(ring, codes_tile, meta_tile, k, r, nb, live, la, lda, tok_bytes, mcount, acc);
        else stream_lane<TYPE, MT, false>(ring, codes_tile, meta_tile, k, r, nb, live, la, lda, tok_bytes, mcount, acc);
#pragma unroll
        for (int m = 0; m < MT; ++m) red[m][k][lane] = acc[m][0] + acc[m][1];
        __syncthreads();
        for (int mi = k; mi < mcount; mi += 8) {                       // wave k reduces tokens k, k+8, ...
            if (live) {
                float v = lane_tree(&red[mi][0][lane]);
                const int grow = static_cast<int>(ggml_row(static_cast<int64_t>(tile) * 32 + r, S.rows, S.interleave));
                if (A.bias) v = v + A.bias[static_cast<size_t>(expert) * S.rows + grow];
                if (A.epilogue == 0) A.dst[static_cast<size_t>(jobs[c0 + mi]) * S.rows + grow] = v;
                else vals[mi][lane] = v;
            }
        }
        if (A.epilogue == 1) {
            __syncthreads();
            for (int mi = k; mi < mcount; mi += 8)
                if (lane < 32)
                    glu_requant_block(vals[mi], lane, blockIdx.x, A.dst_xrows + static_cast<size_t>(jobs[c0 + mi]) * A.dst_lay.stride(),
                                      A.dst_lay, A.activation, A.alpha, A.limit);
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------ fused decode
// Single-token decode, kernel A of a layer: the previous layer's weighted rank combine (or the
// layer input), x86 Q8_0 quantization, top-k + softmax over the given logits, and the gate_up
// GEMV of this workgroup's (tile pair, rank) with biases, GLU and requantization into the down
// projection's activation row. Wave 0 routes while waves 1..7 combine; every workgroup does both
// redundantly (a few KiB from L2), which removes four dependent launches per layer. Workgroup
// (0,0) publishes the routing and the down work list for kernel B (the generic expert GEMV).
struct DecodeArgs {
    const uint8_t * bank;
    Shape shape;
    const int32_t * expert_to_slot;
    XrowLayout lay;            // gate_up activation format (nb = hidden / 32)
    const float * logits;      // [n_expert] of this layer
    int n_expert, top_k;
    const float * x_in;        // [hidden] layer input, or null to combine the previous layer
    const float * prev_y;      // [top_k][hidden] previous layer's biased down outputs
    const float * prev_w;      // [top_k] previous layer's routing weights
    int hidden;
    const float * bias;        // gate_up bias [n_expert][rows] (ggml row order) or null
    uint8_t * act_rows;        // [top_k] down activation rows
    XrowLayout act_lay;
    int32_t * route_ids;       // [top_k] this layer's routing
    float * route_w;           // [top_k]
    GroupBuffers grp;          // this layer's down work list
    int activation;
    float alpha, limit;
};

template <int TYPE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void decode_gate_up_kernel(DecodeArgs A) {
    __shared__ float red[8][64];
    __shared__ float vals[64];
    __shared__ int32_t s_ids[64];
    __shared__ float s_w[64];
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_dyn[];
    const int H = A.hidden, nb = H / 32;
    float * xs = reinterpret_cast<float *>(lds_dyn);
    uint8_t * act = lds_dyn + ((H * 4 + 15) & ~15);
    const int k = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, r = lane & 31;
    const int rank = blockIdx.y;
    if (k == 0) {
        wave_topk_softmax(A.logits, A.n_expert, A.top_k, s_ids, s_w);
    } else {
        const int K = A.top_k;
        for (int i = threadIdx.x - 64; i < H; i += kThreads - 64) {
            float v;
            if (A.x_in) {
                v = A.x_in[i];
            } else {  // ggml MUL by the weight, then sequential ADD in rank order
                v = A.prev_y[i] * A.prev_w[0];
                for (int q = 1; q < K; ++q) {
                    const float term = A.prev_y[static_cast<int64_t>(q) * H + i] * A.prev_w[q];
                    v = v + term;
                }
            }
            xs[i] = v;
        }
    }
    __syncthreads();
    const int expert = s_ids[rank];
    const int slot = A.expert_to_slot ? A.expert_to_slot[expert] : expert;
    const bool slot_ok = slot >= 0 && slot < A.shape.n_slots;
    const Shape S = A.shape;
    const int tile = blockIdx.x * 2 + (lane >> 5);
    const bool live = slot_ok && tile * 32 < S.rows;
    const uint8_t * slot_base = A.bank + static_cast<size_t>(slot_ok ? slot : 0) * S.slot_bytes;
    const uint8_t * codes_tile = slot_base + static_cast<size_t>(live ? tile : 0) * 32 * nb * (TYPE == 39 ? 16 : 32);
    const uint8_t * meta_tile = slot_base + S.codes_bytes + static_cast<size_t>(live ? tile : 0) * 32 * nb * (TYPE == 39 ? 1 : 2);
    constexpr int kGroupBlocks = TYPE == 39 ? 8 : 4;
    Group ring[kDepth];
    preload_ring(ring, codes_tile + (k * 32 + r) * 16, meta_tile + r * 8, nb / kGroupBlocks, live);

    // x86 quantize_row_q8_0 of the layer input into the LDS activation row: one 32-lane group per
    // block, 16 blocks per round.
    const XrowLayout L = A.lay;
    for (int b = threadIdx.x >> 5; b < nb; b += kThreads / 32) {
        const int e = threadIdx.x & 31;
        const float x = xs[b * 32 + e];
        float amax = fabsf(x);
        for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
        const float d = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        float q = rintf(x * id);
        q = q > 127.0f ? 127.0f : (q < -128.0f ? -128.0f : q);
        const int sk = e >> 2, pos = e & 3;
        if (TYPE == 39) reinterpret_cast<_Float16 *>(act + (static_cast<int64_t>(sk) * nb + b) * 8)[pos] = static_cast<_Float16>(q);
        else reinterpret_cast<signed char *>(act + (static_cast<int64_t>(sk) * nb + b) * 4)[pos] = static_cast<signed char>(q);
        if (e == 0) reinterpret_cast<float *>(act + L.da_offset())[b] = static_cast<float>(static_cast<_Float16>(d));
    }
    __syncthreads();
    float acc[1][2] = {{0.0f, 0.0f}};
    stream_lane<TYPE, 1, false>(ring, codes_tile, meta_tile, k, r, nb, live,
                                act + static_cast<int64_t>(k) * nb * L.code_entry(),
                                reinterpret_cast<const float *>(act + L.da_offset()), 0, 1, acc);
    red[k][lane] = acc[0][0] + acc[0][1];
    __syncthreads();
    if (k == 0 && live) {
        float v = lane_tree(&red[0][lane]);
        const int grow = static_cast<int>(ggml_row(static_cast<int64_t>(tile) * 32 + r, S.rows, S.interleave));
        if (A.bias) v = v + A.bias[static_cast<size_t>(expert) * S.rows + grow];
        vals[lane] = v;
    }
    __syncthreads();
    if (k == 0 && lane < 32 && slot_ok)
        glu_requant_block(vals, lane, blockIdx.x, A.act_rows + static_cast<size_t>(rank) * A.act_lay.stride(), A.act_lay,
                          A.activation, A.alpha, A.limit);
    if (blockIdx.x == 0 && blockIdx.y == 0 && static_cast<int>(threadIdx.x) < A.top_k) {
        const int t = threadIdx.x;
        const int e = s_ids[t];
        A.route_ids[t] = e;
        A.route_w[t] = s_w[t];
        A.grp.active[t] = e;
        A.grp.counts[e] = 1;
        A.grp.offsets[e] = t;
        A.grp.rows[t] = t;
        if (t == 0) *A.grp.n_active = A.top_k;
    }
}

template <int TYPE>
void launch_decode_typed(const DecodeArgs & a, hipStream_t stream) {
    const size_t lds = ((static_cast<size_t>(a.hidden) * 4 + 15) & ~static_cast<size_t>(15)) +
                       static_cast<size_t>(a.lay.flag_offset());
    const dim3 grid(static_cast<unsigned>(a.shape.rows / 64), static_cast<unsigned>(a.top_k));
    hipLaunchKernelGGL((decode_gate_up_kernel<TYPE>), grid, dim3(kThreads), lds, stream, a);
    check_hip(hipGetLastError(), "decode gate_up launch");
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

template <int TYPE, int MT>
void launch_typed(const GemvArgs & g, const KernelArgs & ka, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((ka.shape.rows + 63) / 64), static_cast<unsigned>(g.max_active));
    const size_t tok_bytes = (static_cast<size_t>(ka.lay.flag_offset()) + 15) & ~static_cast<size_t>(15);
    hipLaunchKernelGGL((expert_gemv_kernel<TYPE, MT>), grid, dim3(kThreads), MT * tok_bytes, stream, ka);
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
    if (bank.type == VBM_TYPE_MXFP4) launch_mt<39>(g, ka, stream);
    else launch_mt<8>(g, ka, stream);
}

void launch_decode_gate_up(const DecodeGateUpArgs & d, hipStream_t stream) {
    const vbm_bank & bank = *d.bank;
    require(bank.interleave && bank.rows % 64 == 0, "decode gate_up needs an interleaved bank with rows % 64 == 0");
    require(d.top_k >= 1 && d.top_k <= 64 && d.n_expert >= d.top_k && d.n_expert <= 1024, "routing shape out of range");
    require(d.hidden == bank.k && d.hidden <= 4096, "hidden size mismatch");
    DecodeArgs a{};
    a.bank = bank.base;
    a.shape = Shape{static_cast<int>(bank.nb), static_cast<int>(bank.rows), bank.interleave, bank.slot_bytes,
                    bank.geometry().codes_bytes(), bank.n_slots};
    a.expert_to_slot = d.expert_to_slot;
    a.lay = XrowLayout{bank.nb, bank.type};
    a.logits = d.logits;
    a.n_expert = static_cast<int>(d.n_expert);
    a.top_k = static_cast<int>(d.top_k);
    a.x_in = d.x_in;
    a.prev_y = d.prev_y;
    a.prev_w = d.prev_w;
    a.hidden = static_cast<int>(d.hidden);
    a.bias = d.bias;
    a.act_rows = d.act_rows;
    a.act_lay = d.act_layout;
    a.route_ids = d.route_ids;
    a.route_w = d.route_w;
    a.grp = d.group;
    a.activation = d.activation;
    a.alpha = d.alpha;
    a.limit = d.limit;
    if (bank.type == VBM_TYPE_MXFP4) launch_decode_typed<39>(a, stream);
    else launch_decode_typed<8>(a, stream);
}

}  // namespace vbm
