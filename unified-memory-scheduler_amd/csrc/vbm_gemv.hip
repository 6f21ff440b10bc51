// Expert GEMV for decode and ragged small batches: MXFP4 x Q8_0 and Q8_0 x Q8_0, bit-identical
// to the ggml x86 vec_dot contract.
//
// The CPU dot (tools/trace/cpu_mxfp4_vnni.cpp:49-68) splits every 32-element block into eight
// 4-element lanes and keeps per-lane FMA chains (even/odd blocks for MXFP4; one chain for Q8_0),
// then reduces the eight lanes with a fixed tree. Here one wavefront owns one lane slice k of a
// tile pair's rows: lane = row, wave = slice, so
//   - every lane keeps exactly the CPU's chains for its (row, slice) and the final tree over the
//     eight slices (through LDS) reproduces the CPU bits;
//   - each lane streams its row slice of weights (16 B of codes per group of blocks) through a
//     register ring of coalesced 128-bit loads, and the weights are reused from registers for
//     every token routed to the expert;
//   - the activation rows are staged in LDS; a wave reads only its slice of them.
//
// Integer part (MXFP4): v_cvt_scalef32_pk_f16_fp4 with scale 2 turns the slice's four e2m1
// nibbles into the doubled-e2m1 integers {0,1,2,3,4,6,8,12,...} as f16, and the slice dot against
// the f16 activation codes is exact (integers below 2^24). The decode kernels and every batched
// chunk without the -128 correction take it from v_mfma_f32_4x4x4_16b_f16 (16 blocks of 4 x 4
// outputs with K = 4: exactly one slice); the correction path takes two v_dot2. Q8_0 uses
// v_dot4. The VPSIGNB corner case (activation code -128 against a negative weight,
// cpu_mxfp4_vnni.cpp:43-44) runs on a uniform slow path selected per activation row.
//
// Epilogue 1 (fused gate|up bank): the workgroup's 64 rows are gate rows 32p..32p+31 and up rows
// 32p..32p+31, i.e. exactly one 32-element Q8_0 block p of the GLU output; it applies the biases
// and the GLU, requantizes (x86 contract) and writes the down projection's activation row.
#include "vbm_device.hpp"
#include "vbm_internal.hpp"

namespace vbm {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
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
    const int32_t * chunk_expert;   // [n_chunks] expert of each chunk of up to MT jobs
    const int32_t * chunk_start;    // [n_chunks] its first job within the expert's jobs
    const int32_t * n_chunks;       // [1]
    int pairs;                      // 64-row tile pairs of the bank
    const float * bias;
    float * dst;
    uint8_t * dst_xrows;
    XrowLayout dst_lay;
    int epilogue, activation;
    float alpha, limit;
};

// One group of one lane: 16 B of codes (8 MXFP4 blocks x 2 B or 4 Q8_0 blocks x 4 B) and 8 B of
// exponents (MXFP4) or fp16 scales (Q8_0).
struct Group {
    u32x4 c;
    u32x2 m;
};

// MLDS: the workgroup staged its tiles' exponents / scales in LDS, so only the codes are loaded.
template <bool MLDS>
__device__ __forceinline__ Group load_group(const uint8_t * cp, const uint8_t * mp, int g) {
    Group r;
    r.c = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(cp + g * 4096));
    if (MLDS) r.m = u32x2{0u, 0u};
    else r.m = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(mp + g * 256));
    return r;
}

// One MXFP4 block of one lane for MT tokens: bytes SEL, SEL+1 of `dw` are the slice's 4 nibbles;
// the activation slice (4 f16 codes, 8 B per block) and the block scale of each token are read
// from LDS (broadcast). Called by every lane of the wave (uniform control flow): the one- and
// two-token form is a matrix-core instruction over the whole wave.
template <int MT, bool SLOW, int SEL, int PAR>
__device__ __forceinline__ void mx_block(unsigned dw, int e, int b, const uint8_t * la, const float * lda,
                                         int tok_bytes, int mcount, float (&acc)[MT][2]) {
    const half2_t w01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, SEL);
    const half2_t w23 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, SEL + 1);
    if constexpr (MT <= 2 && !SLOW) {
        // One v_mfma_f32_4x4x4_16b_f16 gives every token's slice dot: the row slice is B (lane =
        // row) and lane 4q + r holds token r's activation slice as A, so register m of lane l is
        // token m's dot with row l (exact: integers below 2^24), as in the single-token decode.
        const int am = (threadIdx.x & 3) < mcount ? (threadIdx.x & 3) : 0;
        const u32x2 a = *reinterpret_cast<const u32x2 *>(la + am * tok_bytes + b * 8);
        const f32x4_t v = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(half4_t, a), half4_t{w01.x, w01.y, w23.x, w23.y},
                                                             f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m < mcount) {
                const float d = *reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(lda) + m * tok_bytes + b * 4);
                acc[m][PAR] = __builtin_fmaf(__builtin_amdgcn_ldexpf(d, e), v[m], acc[m][PAR]);
            }
        }
        return;
    }
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
__device__ __forceinline__ void mx_group(const u32x4 & c, const u32x2 & m, int b, const uint8_t * la, const float * lda,
                                         int tok_bytes, int mcount, float (&acc)[MT][2]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const unsigned dw = q == 0 ? c.x : (q == 1 ? c.y : (q == 2 ? c.z : c.w));
        const unsigned ew = q < 2 ? m.x : m.y;
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
__device__ __forceinline__ void q8_group(const u32x4 & c, const u32x2 & m, int b, const uint8_t * la, const float * lda,
                                         int tok_bytes, int mcount, float (&acc)[MT][2]) {
    q8_block<MT, SLOW>(c.x, static_cast<unsigned short>(m.x), b, la, lda, tok_bytes, mcount, acc);
    q8_block<MT, SLOW>(c.y, static_cast<unsigned short>(m.x >> 16), b + 1, la, lda, tok_bytes, mcount, acc);
    q8_block<MT, SLOW>(c.z, static_cast<unsigned short>(m.y), b + 2, la, lda, tok_bytes, mcount, acc);
    q8_block<MT, SLOW>(c.w, static_cast<unsigned short>(m.y >> 16), b + 3, la, lda, tok_bytes, mcount, acc);
}

// Weight groups a lane keeps in flight. Both MXFP4 decode kernels stream through a 5-deep ring
// so compute overlaps the arrivals (120B-shape decode, A / B depth 6 / 12: 1511-1514 tok/s, 5 / 6:
// 1600-1618, 5 / 5: 1627-1638, 6 / 4: 1540-1561, 7 / 6: 1522-1531); the batched kernel's depth is
// set where it streams (gemv_chunk).
template <int TYPE>
constexpr int gate_up_depth() {
    return TYPE == 39 ? 5 : 4;
}
template <int TYPE>
constexpr int down_depth() {
    return TYPE == 39 ? 5 : 8;
}

// The blocks past the last full group of a lane's row slice (nb is even: MXFP4 tail in
// {0,2,4,6}, Q8_0 tail in {0,2}): MXFP4 keeps two blocks per code dword and two exponents per
// meta halfword, Q8_0 one block per code dword and one fp16 scale per meta halfword.
struct Tail {
    unsigned c[3];
    unsigned m[3];
};

template <int TYPE, bool MLDS>
__device__ __forceinline__ void preload_tail(Tail & t, const uint8_t * codes_tile, const uint8_t * meta_tile, int k,
                                             int r, int nb, bool live) {
    constexpr int kGroupBlocks = TYPE == 39 ? 8 : 4, kCode = TYPE == 39 ? 2 : 4, kMeta = TYPE == 39 ? 1 : 2;
    const int groups = nb / kGroupBlocks, tail = nb % kGroupBlocks;
    const int n = TYPE == 39 ? tail / 2 : tail;
    const uint8_t * tcp = codes_tile + groups * 4096 + (k * 32 + r) * (tail * kCode);
    const uint8_t * tmp = meta_tile + groups * 256 + r * tail * kMeta;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        t.c[i] = 0u;
        t.m[i] = 0u;
        if (live && i < n) {
            t.c[i] = __builtin_nontemporal_load(reinterpret_cast<const unsigned *>(tcp + 4 * i));
            if (!MLDS) t.m[i] = *reinterpret_cast<const unsigned short *>(tmp + 2 * i);
        }
    }
}

// Issues the first D groups of one lane's row slice (before activation staging, so the weight
// stream is in flight while the activation row arrives).
template <int TYPE, int D, bool MLDS>
__device__ __forceinline__ void preload_ring(Group (&ring)[D], const uint8_t * codes_tile, const uint8_t * meta_tile,
                                             int k, int r, int nb, bool live) {
    constexpr int kGroupBlocks = TYPE == 39 ? 8 : 4;
    const int groups = nb / kGroupBlocks;
    const uint8_t * cp = codes_tile + (k * 32 + r) * 16;
    const uint8_t * mp = meta_tile + r * 8;
#pragma unroll
    for (int i = 0; i < D; ++i) {
        ring[i] = Group{};
        if (live && i < groups) ring[i] = load_group<MLDS>(cp, mp, i);
    }
}

// The tail blocks of one lane's row slice (after its full groups: block order is chain order).
// With MLDS the exponents / scales come from the lane's tile meta staged in LDS (`meta_lds`).
template <int TYPE, int MT, bool SLOW, bool MLDS>
__device__ __forceinline__ void apply_tail(const Tail & tl, const uint8_t * meta_lds, int r, int nb, const uint8_t * la,
                                           const float * lda, int tok_bytes, int mcount, float (&acc)[MT][2]) {
    constexpr int kGroupBlocks = TYPE == 39 ? 8 : 4, kMeta = TYPE == 39 ? 1 : 2;
    const int groups = nb / kGroupBlocks, tail = nb % kGroupBlocks;
    const int n = TYPE == 39 ? tail / 2 : tail;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        if (i < n) {
            const unsigned m = MLDS ? *reinterpret_cast<const unsigned short *>(meta_lds + groups * 256 + r * tail * kMeta + 2 * i)
                                    : tl.m[i];
            if (TYPE == 39) {
                const int b = groups * 8 + 2 * i;
                mx_block<MT, SLOW, 0, 0>(tl.c[i], static_cast<signed char>(m & 0xFFu), b, la, lda, tok_bytes, mcount, acc);
                mx_block<MT, SLOW, 2, 1>(tl.c[i], static_cast<signed char>(m >> 8), b + 1, la, lda, tok_bytes, mcount, acc);
            } else {
                q8_block<MT, SLOW>(tl.c[i], static_cast<unsigned short>(m), groups * 4 + i, la, lda, tok_bytes, mcount, acc);
            }
        }
    }
}

// ------------------------------------------------------------------ buffer-descriptor weight stream
// The batched kernel reads one expert slot through a buffer descriptor (SGPRs) with one VGPR
// offset per lane and the group offsets as SGPR soffsets, so the ring costs no per-group address
// registers and no per-lane exec masking (lanes of a half-live tile pair read tile 0 and drop it).
// dword3 0x00020000 is the raw-buffer format word of the gfx9 family; aux 2 marks the loads
// non-temporal, as the pointer loads above.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t slot_rsrc(const uint8_t * base, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), static_cast<short>(0),
                                             static_cast<int>(bytes < 0x7fffffffu ? bytes : 0x7fffffffu), 0x00020000);
}

struct BufLane {
    __amdgpu_buffer_rsrc_t rsrc;
    int code_off;   // byte offset of the lane's first group of codes in the slot
    int meta_off;   // byte offset of the lane's first group of exponents / scales
    int tail_code;  // byte offset of the lane's tail codes
    int tail_meta;  // byte offset of the lane's tail exponents / scales
};

__device__ __forceinline__ Group load_group_buf(const BufLane & B, int g) {
    Group r;
    r.c = __builtin_amdgcn_raw_buffer_load_b128(B.rsrc, B.code_off, g * 4096, 2);
    r.m = __builtin_amdgcn_raw_buffer_load_b64(B.rsrc, B.meta_off, g * 256, 2);
    return r;
}

template <int TYPE>
__device__ __forceinline__ BufLane buf_lane(const uint8_t * slot_base, size_t slot_bytes, int64_t codes_bytes, int tile,
                                            int k, int r, int nb) {
    constexpr int kGroupBlocks = TYPE == 39 ? 8 : 4, kCode = TYPE == 39 ? 2 : 4, kMeta = TYPE == 39 ? 1 : 2;
    const int groups = nb / kGroupBlocks, tail = nb % kGroupBlocks;
    BufLane B;
    B.rsrc = slot_rsrc(slot_base, slot_bytes);
    const int codes_tile = tile * 32 * nb * (TYPE == 39 ? 16 : 32);
    const int meta_tile = static_cast<int>(codes_bytes) + tile * 32 * nb * kMeta;
    B.code_off = codes_tile + (k * 32 + r) * 16;
    B.meta_off = meta_tile + r * 8;
    B.tail_code = codes_tile + groups * 4096 + (k * 32 + r) * (tail * kCode);
    B.tail_meta = meta_tile + groups * 256 + r * tail * kMeta;
    return B;
}

template <int TYPE, int D>
__device__ __forceinline__ void preload_ring_buf(Group (&ring)[D], const BufLane & B, int nb) {
    constexpr int kGroupBlocks = TYPE == 39 ? 8 : 4;
    const int groups = nb / kGroupBlocks;
#pragma unroll
    for (int i = 0; i < D; ++i) {
        ring[i] = Group{};
        if (i < groups) ring[i] = load_group_buf(B, i);
    }
}

template <int TYPE>
__device__ __forceinline__ void preload_tail_buf(Tail & t, const BufLane & B, int nb) {
    constexpr int kGroupBlocks = TYPE == 39 ? 8 : 4;
    const int tail = nb % kGroupBlocks;
    const int n = TYPE == 39 ? tail / 2 : tail;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        t.c[i] = 0u;
        t.m[i] = 0u;
        if (i < n) {
            t.c[i] = __builtin_amdgcn_raw_buffer_load_b32(B.rsrc, B.tail_code, 4 * i, 2);
            t.m[i] = __builtin_amdgcn_raw_buffer_load_b16(B.rsrc, B.tail_meta, 2 * i, 0);
        }
    }
}

template <int TYPE, int MT, bool SLOW, int D>
__device__ __forceinline__ void stream_groups_buf(Group (&ring)[D], const BufLane & B, int nb, const uint8_t * la,
                                                  const float * lda, int tok_bytes, int mcount, float (&acc)[MT][2]) {
    constexpr int kGroupBlocks = TYPE == 39 ? 8 : 4;
    const int groups = nb / kGroupBlocks;
    for (int g0 = 0; g0 < groups; g0 += D) {
#pragma unroll
        for (int i = 0; i < D; ++i) {
            const int g = g0 + i;
            if (g < groups) {
                const Group cur = ring[i];
                if (g + D < groups) ring[i] = load_group_buf(B, g + D);
                if (TYPE == 39) mx_group<MT, SLOW>(cur.c, cur.m, g * 8, la, lda, tok_bytes, mcount, acc);
                else q8_group<MT, SLOW>(cur.c, cur.m, g * 4, la, lda, tok_bytes, mcount, acc);
            }
        }
    }
}

// ------------------------------------------------------ batched MXFP4 GEMV on the matrix cores
// Chunks of four or more tokens without the -128 correction take the lane slices' integer dots
// from v_mfma_f32_4x4x4_16b_f16, whose output register r of lane l is the dot over k of
// A(lane 4(l/4) + r, k) and B(lane l, k). A is the lane's own row slice (lane = row, as in the
// scalar path) and B the activation slice of token 4g + l % 4, so register r of lane l holds the
// slice dot of row 4(l/4) + r and token 4g + l % 4: one instruction gives the wave's 64 rows x 4
// tokens, each the value the two v_dot2 of the scalar path give (integers below 2^24 are exact
// in any order). Every (row, token, slice) keeps the CPU's chains: one FMA per block into the even
// or odd chain of the block.
//
// FOLD: when every exponent e of the tile pair's rows lies in [-14, 12], the conversion
// scales the e2m1 values by 2^(e+1) (exact normal f16), the dot comes out as 2^e * dot, and the
// chain's FMA takes d_act alone: d_act * (2^e * dot) is exactly the product ldexp(d_act, e) * dot
// (no overflow or underflow in that range), rounded once inside the same FMA. Otherwise each
// output takes ldexp(d_act, e) with e broadcast from its row's lane within the quad.
template <int MT>
using MmAcc = float[MT / 4][4][2];

// One block for the MT / 4 token groups: `a[g]` is token group g's activation slice (4 f16 codes)
// and `d[g]` its block scale, both for the lane's token 4g + l % 4.
template <int MT, int SEL, int PAR, bool FOLD>
__device__ __forceinline__ void mx_block_mm(unsigned dw, int e, const u32x2 (&a)[MT / 4], const float (&d)[MT / 4],
                                            MmAcc<MT> & acc) {
    constexpr int G = MT / 4;
    const float sc = FOLD ? __builtin_bit_cast(float, (e + 128) << 23) : 2.0f;
    const half2_t w01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, sc, SEL);
    const half2_t w23 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, sc, SEL + 1);
    const half4_t wv = half4_t{w01.x, w01.y, w23.x, w23.y};
    f32x4_t v[G];
#pragma unroll
    for (int g = 0; g < G; ++g)
        v[g] = __builtin_amdgcn_mfma_f32_4x4x4f16(wv, __builtin_bit_cast(half4_t, a[g]), f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
    if constexpr (FOLD) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[g][r][PAR] = __builtin_fmaf(d[g], v[g][r], acc[g][r][PAR]);
    } else {
        int eq[4];
        eq[0] = __builtin_amdgcn_mov_dpp(e, 0x00, 0xf, 0xf, false);   // quad_perm [r, r, r, r]
        eq[1] = __builtin_amdgcn_mov_dpp(e, 0x55, 0xf, 0xf, false);
        eq[2] = __builtin_amdgcn_mov_dpp(e, 0xAA, 0xf, 0xf, false);
        eq[3] = __builtin_amdgcn_mov_dpp(e, 0xFF, 0xf, 0xf, false);
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[g][r][PAR] = __builtin_fmaf(__builtin_amdgcn_ldexpf(d[g], eq[r]), v[g][r], acc[g][r][PAR]);
    }
}

// Two consecutive blocks b, b + 1 of one code dword (e0, e1 their exponents); `a2[g]` holds both
// blocks' activation slices of token group g, `d0[g]` / `d1[g]` their scales.
template <int MT, bool FOLD>
__device__ __forceinline__ void mx_pair_mm(unsigned dw, int e0, int e1, const u32x4 (&a2)[MT / 4], const float (&d0)[MT / 4],
                                           const float (&d1)[MT / 4], MmAcc<MT> & acc) {
    constexpr int G = MT / 4;
    u32x2 a0[G], a1[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        a0[g] = u32x2{a2[g].x, a2[g].y};
        a1[g] = u32x2{a2[g].z, a2[g].w};
    }
    mx_block_mm<MT, 0, 0, FOLD>(dw, e0, a0, d0, acc);
    mx_block_mm<MT, 2, 1, FOLD>(dw, e1, a1, d1, acc);
}

// One group of eight blocks starting at block b; each block reads its activation slices and
// scales itself, and the fence after it keeps the scheduler from hoisting every read of the group
// (register spills otherwise).
template <int MT, bool FOLD>
__device__ __forceinline__ void mx_group_mm(const u32x4 & c, const u32x2 & m, int b, const uint8_t * la_lane,
                                            const uint8_t * lda_lane, int tok_bytes, MmAcc<MT> & acc) {
    constexpr int G = MT / 4;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const unsigned dw = c[j >> 1];
        const int e = static_cast<signed char>((j < 4 ? m.x : m.y) >> (8 * (j & 3)));
        u32x2 a[G];
        float d[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            a[g] = *reinterpret_cast<const u32x2 *>(la_lane + 4 * g * tok_bytes + (b + j) * 8);
            d[g] = *reinterpret_cast<const float *>(lda_lane + 4 * g * tok_bytes + (b + j) * 4);
        }
        if (j & 1) mx_block_mm<MT, 2, 1, FOLD>(dw, e, a, d, acc);
        else mx_block_mm<MT, 0, 0, FOLD>(dw, e, a, d, acc);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Sixteen exponent bytes, each (signed) in [-14, 12].
__device__ __forceinline__ bool exps_foldable(const u32x4 & w) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int e = static_cast<signed char>(w[i >> 2] >> (8 * (i & 3)));
        ok = ok && e >= -14 && e <= 12;
    }
    return ok;
}

template <int MT, int D, bool FOLD>
__device__ __forceinline__ void stream_groups_mm(Group (&ring)[D], const BufLane & B, int nb, const uint8_t * la_lane,
                                                 const uint8_t * lda_lane, int tok_bytes, MmAcc<MT> & acc) {
    const int groups = nb / 8;
    for (int g0 = 0; g0 < groups; g0 += D) {
#pragma unroll
        for (int i = 0; i < D; ++i) {
            const int g = g0 + i;
            if (g < groups) {
                const Group cur = ring[i];
                if (g + D < groups) ring[i] = load_group_buf(B, g + D);
                mx_group_mm<MT, FOLD>(cur.c, cur.m, g * 8, la_lane, lda_lane, tok_bytes, acc);
            }
        }
    }
}

// The tail blocks (after the full groups, in chain order) with the unfolded scales.
template <int MT>
__device__ __forceinline__ void apply_tail_mm(const Tail & tl, int nb, const uint8_t * la_lane, const uint8_t * lda_lane,
                                              int tok_bytes, MmAcc<MT> & acc) {
    constexpr int G = MT / 4;
    const int groups = nb / 8, n = (nb % 8) / 2;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        if (i < n) {
            const int b = groups * 8 + 2 * i;
            u32x4 a2[G];
            float d0[G], d1[G];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                a2[g] = *reinterpret_cast<const u32x4 *>(la_lane + 4 * g * tok_bytes + b * 8);
                const float * dp = reinterpret_cast<const float *>(lda_lane + 4 * g * tok_bytes + b * 4);
                d0[g] = dp[0];
                d1[g] = dp[1];
            }
            mx_pair_mm<MT, false>(tl.c[i], static_cast<signed char>(tl.m[i] & 0xFFu), static_cast<signed char>(tl.m[i] >> 8),
                                  a2, d0, d1, acc);
        }
    }
}

// The matrix-core path serves MXFP4 chunks of four or more tokens in the kernels for rows this
// library quantized (never -128); the kernels for caller-quantized rows keep the scalar path.
template <int TYPE, int M, bool NEG>
constexpr bool use_mfma() {
    return TYPE == 39 && M >= 4 && !NEG;
}

// Stages the exponents / scales of a workgroup's (up to) two consecutive tiles: loads are issued
// into registers first (ahead of the code stream, so waiting for them never waits for codes),
// then written to LDS by store_meta.
template <int TYPE>
__device__ __forceinline__ int meta_tile_bytes(int nb) {
    return 32 * nb * (TYPE == 39 ? 1 : 2);
}
// Up to 2 * NT * 16 bytes (two tiles of K <= 4096 at NT = 512, one tile at NT = 256).
template <int NT>
__device__ __forceinline__ void load_meta(u32x4 (&st)[2], const uint8_t * meta, int bytes) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int off = (threadIdx.x + i * NT) * 16;
        st[i] = u32x4{0u, 0u, 0u, 0u};
        if (off < bytes) st[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(meta + off));
    }
}
// Copies one 32-row tile of a slot (its codes tile and its meta tile, the bytes the decode
// kernels read for it) from `src` to `dst`, both in the bank's slot layout, with NT threads:
// 16-byte units, four loads in flight per thread before their stores. The deferred host tier
// uses it to keep, in device memory, the copy of an expert that a kernel streams from pinned
// host memory. The caller's barrier (a workgroup-scope release: every store has reached L2)
// makes the copy readable by the workgroup's loads that follow; no other workgroup reads it.
template <int TYPE, int NT>
__device__ __forceinline__ void copy_slot_tile(const uint8_t * src, uint8_t * dst, int tile, int nb, int64_t codes_bytes) {
    const int64_t tile_codes = 32ll * nb * (TYPE == 39 ? 16 : 32);
    const int n_codes = static_cast<int>(tile_codes / 16), n = n_codes + meta_tile_bytes<TYPE>(nb) / 16;
    const int64_t codes0 = tile * tile_codes, meta0 = codes_bytes + static_cast<int64_t>(tile) * meta_tile_bytes<TYPE>(nb);
    for (int base = 0; base < n; base += 4 * NT) {
        u32x4 v[4];
        int64_t off[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = base + j * NT + static_cast<int>(threadIdx.x);
            off[j] = i < n_codes ? codes0 + static_cast<int64_t>(i) * 16 : meta0 + static_cast<int64_t>(i - n_codes) * 16;
            if (i < n) v[j] = *reinterpret_cast<const u32x4 *>(src + off[j]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (base + j * NT + static_cast<int>(threadIdx.x) < n) *reinterpret_cast<u32x4 *>(dst + off[j]) = v[j];
    }
}

template <int NT>
__device__ __forceinline__ void store_meta(const u32x4 (&st)[2], uint8_t * lds, int bytes) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int off = (threadIdx.x + i * NT) * 16;
        if (off < bytes) *reinterpret_cast<u32x4 *>(lds + off) = st[i];
    }
}

// ------------------------------------------------------------------------ decode block math
// In the single-token decode kernels every (row, block) scale is precomputed once per workgroup
// into an LDS table (MXFP4: ldexp(d_act, e - 128); Q8_0: fp16(d_w) * d_act, the same operations
// the batched path does per lane), laid out [tile][block / 4][row][block % 4] so one 16-byte read
// per lane brings four consecutive blocks without bank conflicts.

// One MXFP4 block of the lane's row slice against the wave's (uniform) activation slice `a`: the
// slice dot comes from v_mfma_f32_4x4x4_16b_f16 with the row slice as B (lane = row) and `a` as A
// in every lane, so register 0 of lane l is the dot of row l (exact: integers below 2^24), taken
// off the vector ALU where two v_dot2 did it (120B-shape decode step: 1627-1643 -> 1660-1678
// tok/s, kernel A 10.1 -> 9.6-9.9 us isolated).
template <int SEL, int PAR>
__device__ __forceinline__ void mx_block_s(unsigned dw, float s, u32x2 a, float (&acc)[2]) {
    const half2_t w01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, SEL);
    const half2_t w23 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, SEL + 1);
    const f32x4_t v = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(half4_t, a), half4_t{w01.x, w01.y, w23.x, w23.y},
                                                         f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
    acc[PAR] = __builtin_fmaf(s, v[0], acc[PAR]);
}

__device__ __forceinline__ void q8_block_s(unsigned w, float s, unsigned a, float (&acc)[2]) {
    const int v = __builtin_amdgcn_sdot4(static_cast<int>(w), static_cast<int>(a), 0, false);
    acc[0] = __builtin_fmaf(s, static_cast<float>(v), acc[0]);
}

// Streams one lane's row slice (full groups through the D-deep ring, then the tail) against one
// token: `la` is the wave's activation slice (8 B per block for MXFP4, 4 B for Q8_0), `ls` the
// lane's row in the scale table.
//
// With NB (blocks per row) a compile-time constant the group loop unrolls completely, every
// reload is unconditional straight-line code, and the compiler's wait counts stay exact: the
// consumer of group g waits for group g only, while the reloads issued after it stay in flight.
// With a run-time NB (NB = 0) the conditional reloads of the rolled loop leave the waits
// conservative (each group waits for every load issued before it, the latest reload included).
template <int TYPE, int D, int NB = 0>
__device__ __forceinline__ void decode_stream(Group (&ring)[D], const Tail & tl, const uint8_t * codes_tile, int k, int r,
                                              int nb_rt, bool live, const uint8_t * la, const float * ls,
                                              float (&acc)[2]) {
    constexpr int kGroupBlocks = TYPE == 39 ? 8 : 4;
    const int nb = NB > 0 ? NB : nb_rt;
    const int groups = nb / kGroupBlocks, tail = nb % kGroupBlocks;
    const uint8_t * cp = codes_tile + (k * 32 + r) * 16;
    auto group_step = [&](int g0, int i) {
            const int g = g0 + i;
            if (g < groups) {
                const u32x4 c = ring[i].c;
                if (live && g + D < groups) ring[i] = load_group<true>(cp, nullptr, g + D);
                if (TYPE == 39) {
                    const float4 s0 = *reinterpret_cast<const float4 *>(ls + (2 * g) * 128);
                    const float4 s1 = *reinterpret_cast<const float4 *>(ls + (2 * g + 1) * 128);
                    const u32x4 a0 = *reinterpret_cast<const u32x4 *>(la + (8 * g) * 8);
                    const u32x4 a1 = *reinterpret_cast<const u32x4 *>(la + (8 * g + 2) * 8);
                    const u32x4 a2 = *reinterpret_cast<const u32x4 *>(la + (8 * g + 4) * 8);
                    const u32x4 a3 = *reinterpret_cast<const u32x4 *>(la + (8 * g + 6) * 8);
                    mx_block_s<0, 0>(c.x, s0.x, a0.xy, acc);
                    mx_block_s<2, 1>(c.x, s0.y, a0.zw, acc);
                    mx_block_s<0, 0>(c.y, s0.z, a1.xy, acc);
                    mx_block_s<2, 1>(c.y, s0.w, a1.zw, acc);
                    mx_block_s<0, 0>(c.z, s1.x, a2.xy, acc);
                    mx_block_s<2, 1>(c.z, s1.y, a2.zw, acc);
                    mx_block_s<0, 0>(c.w, s1.z, a3.xy, acc);
                    mx_block_s<2, 1>(c.w, s1.w, a3.zw, acc);
                } else {
                    const float4 s0 = *reinterpret_cast<const float4 *>(ls + g * 128);
                    const u32x2 a01 = *reinterpret_cast<const u32x2 *>(la + (4 * g) * 4);
                    const u32x2 a23 = *reinterpret_cast<const u32x2 *>(la + (4 * g + 2) * 4);
                    q8_block_s(c.x, s0.x, a01.x, acc);
                    q8_block_s(c.y, s0.y, a01.y, acc);
                    q8_block_s(c.z, s0.z, a23.x, acc);
                    q8_block_s(c.w, s0.w, a23.y, acc);
                }
            }
    };
    if constexpr (NB > 0) {
#pragma unroll
        for (int g0 = 0; g0 < NB / kGroupBlocks; g0 += D) {
#pragma unroll
            for (int i = 0; i < D; ++i) group_step(g0, i);
        }
    } else {
        for (int g0 = 0; g0 < groups; g0 += D) {
#pragma unroll
            for (int i = 0; i < D; ++i) group_step(g0, i);
        }
    }
    const int n = TYPE == 39 ? tail / 2 : tail;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        if (i < n) {
            if (TYPE == 39) {
                const int b = groups * 8 + 2 * i;
                const u32x4 a = *reinterpret_cast<const u32x4 *>(la + b * 8);
                mx_block_s<0, 0>(tl.c[i], ls[(b >> 2) * 128 + (b & 3)], a.xy, acc);
                mx_block_s<2, 1>(tl.c[i], ls[((b + 1) >> 2) * 128 + ((b + 1) & 3)], a.zw, acc);
            } else {
                const int b = groups * 4 + i;
                q8_block_s(tl.c[i], ls[(b >> 2) * 128 + (b & 3)], *reinterpret_cast<const unsigned *>(la + b * 4), acc);
            }
        }
    }
}

// Builds the scale table of a workgroup's NTILES tiles from the staged tile meta (`lmeta`, bank
// layout) and the activation block scales `da`: one thread per (tile, group, row), lanes of a
// half-wave on consecutive rows of one group.
template <int TYPE, int NT, int NTILES>
__device__ __forceinline__ void build_scales(float * lscale, const uint8_t * lmeta, const float * da, int nb, int mbytes) {
    constexpr int kGroupBlocks = TYPE == 39 ? 8 : 4;
    const int groups = nb / kGroupBlocks, tail = nb % kGroupBlocks;
    const int g1 = groups + (tail ? 1 : 0);
    const int nb4 = (nb + 3) / 4;
    const int r = threadIdx.x & 31;
    for (int tg = threadIdx.x >> 5; tg < NTILES * g1; tg += NT / 32) {
        const int t = tg >= g1 ? 1 : 0, g = tg - t * g1;
        const uint8_t * m = lmeta + t * mbytes;
        float * out = lscale + (t * nb4 * 32 + r) * 4;
        const int b0 = g * kGroupBlocks;
        if (g < groups) {
            const u32x2 mv = *reinterpret_cast<const u32x2 *>(m + g * 256 + r * 8);
            if (TYPE == 39) {
                const float4 d0 = *reinterpret_cast<const float4 *>(da + b0);
                const float4 d1 = *reinterpret_cast<const float4 *>(da + b0 + 4);
                float4 s0, s1;
                s0.x = __builtin_amdgcn_ldexpf(d0.x, static_cast<signed char>(mv.x));
                s0.y = __builtin_amdgcn_ldexpf(d0.y, static_cast<signed char>(mv.x >> 8));
                s0.z = __builtin_amdgcn_ldexpf(d0.z, static_cast<signed char>(mv.x >> 16));
                s0.w = __builtin_amdgcn_ldexpf(d0.w, static_cast<signed char>(mv.x >> 24));
                s1.x = __builtin_amdgcn_ldexpf(d1.x, static_cast<signed char>(mv.y));
                s1.y = __builtin_amdgcn_ldexpf(d1.y, static_cast<signed char>(mv.y >> 8));
                s1.z = __builtin_amdgcn_ldexpf(d1.z, static_cast<signed char>(mv.y >> 16));
                s1.w = __builtin_amdgcn_ldexpf(d1.w, static_cast<signed char>(mv.y >> 24));
                *reinterpret_cast<float4 *>(out + (2 * g) * 128) = s0;
                *reinterpret_cast<float4 *>(out + (2 * g + 1) * 128) = s1;
            } else {
                const float4 d0 = *reinterpret_cast<const float4 *>(da + b0);
                float4 s0;
                s0.x = half_bits_to_float(static_cast<uint16_t>(mv.x)) * d0.x;
                s0.y = half_bits_to_float(static_cast<uint16_t>(mv.x >> 16)) * d0.y;
                s0.z = half_bits_to_float(static_cast<uint16_t>(mv.y)) * d0.z;
                s0.w = half_bits_to_float(static_cast<uint16_t>(mv.y >> 16)) * d0.w;
                *reinterpret_cast<float4 *>(out + g * 128) = s0;
            }
        } else {   // partial last group: the tail blocks, meta packed per row
            for (int j = 0; j < tail; ++j) {
                const int b = b0 + j;
                float sv;
                if (TYPE == 39) {
                    sv = __builtin_amdgcn_ldexpf(da[b], static_cast<signed char>(m[groups * 256 + r * tail + j]));
                } else {
                    const uint8_t * q = m + groups * 256 + (r * tail + j) * 2;
                    sv = half_bits_to_float(static_cast<uint16_t>(q[0] | (q[1] << 8))) * da[b];
                }
                out[(b >> 2) * 128 + (b & 3)] = sv;
            }
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
    const float amax = half_wave_max(fabsf(act));
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

// One chunk of mcount <= M tokens of the workgroup's tile pair: stage the activation rows in LDS,
// stream every lane's row slice once applying each token, reduce the eight slices per token and
// write the outputs (or the GLU block). M is the narrowest token width holding the chunk.
template <int TYPE, int M, bool NEG>
__device__ __forceinline__ void gemv_chunk(const KernelArgs & A, const BufLane & B, const __attribute__((address_space(4))) int32_t * jobs,
                                           int expert, int c0, int mcount, int pair, int k, int lane, int r, int tile,
                                           bool live, uint8_t * lds_tok, float * red, float * vals, int * s_flag) {
    const Shape S = A.shape;
    const int nb = S.nb;
    const int copy_bytes = static_cast<int>(A.lay.flag_offset());        // codes + scales of a row
    const int tok_bytes = (copy_bytes + 15) & ~15;
    const uint8_t * la = lds_tok + static_cast<int64_t>(k) * nb * A.lay.code_entry();
    const float * lda = reinterpret_cast<const float *>(lds_tok + A.lay.da_offset());
    // Two groups in flight: with many workgroups per CU the memory system stays busy and the VGPRs
    // a deeper ring would hold go to occupancy (batch 32 of the 120B shape: depth 8 / 6 (single-
    // token / wider) 2587-2620 tok/s, 5 / 4 2677-2721, 3 / 3 2755-2800, 2 / 2 2873-2911, 1 / 1
    // 2763-2782); the variant with the -128 slow path spilled with its former 6 / 4-deep rings.
    // With one chunk per workgroup and the matrix-core dots, depths 3 and 4 measured 3.0k against
    // 3.6k tok/s at batch 32 (config 1 shape at 64 tokens: 11.1k against 12.7k).
    constexpr int D = 2;
    Group ring[D];
    preload_ring_buf<TYPE, D>(ring, B, nb);
    // The matrix path folds the block exponents into the weight conversion when every exponent of
    // the tile pair's live rows lies in [-14, 12]: one 16-byte load per thread (K <= 4096: at most
    // 8 KiB of exponents), issued with the ring and checked at the staging barrier.
    u32x4 ex = u32x4{0u, 0u, 0u, 0u};
    if constexpr (use_mfma<TYPE, M, NEG>()) {
        const int pair_tiles = (2 * pair + 1) * 32 < S.rows ? 2 : 1;
        const int meta0 = static_cast<int>(S.codes_bytes) + 2 * pair * 32 * nb;
        if (static_cast<int>(threadIdx.x) * 16 < pair_tiles * 32 * nb)
            ex = __builtin_amdgcn_raw_buffer_load_b128(B.rsrc, meta0 + static_cast<int>(threadIdx.x) * 16, 0, 0);
    }
    // Stage the chunk's activation rows (and their -128 flags) in LDS.
    if (threadIdx.x == 0) *s_flag = 0;
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
    if (threadIdx.x == 0 && flag) *s_flag = 1;
    bool fold = false;
    if constexpr (use_mfma<TYPE, M, NEG>()) fold = __syncthreads_and(exps_foldable(ex) ? 1 : 0) != 0;
    else __syncthreads();
    Tail tl;
    if constexpr (use_mfma<TYPE, M, NEG>()) {
        MmAcc<M> acc;
#pragma unroll
        for (int g = 0; g < M / 4; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[g][i][0] = acc[g][i][1] = 0.0f;
        const uint8_t * la_lane = la + (lane & 3) * tok_bytes;   // token 4g + lane % 4
        const uint8_t * lda_lane = reinterpret_cast<const uint8_t *>(lda) + (lane & 3) * tok_bytes;
        if (fold) stream_groups_mm<M, D, true>(ring, B, nb, la_lane, lda_lane, tok_bytes, acc);
        else stream_groups_mm<M, D, false>(ring, B, nb, la_lane, lda_lane, tok_bytes, acc);
        preload_tail_buf<TYPE>(tl, B, nb);
        apply_tail_mm<M>(tl, nb, la_lane, lda_lane, tok_bytes, acc);
        __syncthreads();   // `red` reuses the staged activation rows the other waves may still read
        // register i of lane l: row 4(l / 4) + i (the red layout's lane index) of token 4g + l % 4
#pragma unroll
        for (int g = 0; g < M / 4; ++g)
            *reinterpret_cast<float4 *>(&red[((4 * g + (lane & 3)) * 8 + k) * 64 + 4 * (lane >> 2)]) =
                float4{acc[g][0][0] + acc[g][0][1], acc[g][1][0] + acc[g][1][1], acc[g][2][0] + acc[g][2][1],
                       acc[g][3][0] + acc[g][3][1]};
    } else {
        float acc[M][2];
#pragma unroll
        for (int m = 0; m < M; ++m) acc[m][0] = acc[m][1] = 0.0f;
        // widths 1 and 2 only ever carry full chunks: a constant count drops the per-token checks
        const int mc = M <= 2 ? M : mcount;
        if (NEG && *s_flag) {
            stream_groups_buf<TYPE, M, true, D>(ring, B, nb, la, lda, tok_bytes, mc, acc);
            preload_tail_buf<TYPE>(tl, B, nb);
            apply_tail<TYPE, M, true, false>(tl, nullptr, r, nb, la, lda, tok_bytes, mc, acc);
        } else {
            stream_groups_buf<TYPE, M, false, D>(ring, B, nb, la, lda, tok_bytes, mc, acc);
            preload_tail_buf<TYPE>(tl, B, nb);
            apply_tail<TYPE, M, false, false>(tl, nullptr, r, nb, la, lda, tok_bytes, mc, acc);
        }
        __syncthreads();   // `red` reuses the staged activation rows the other waves may still read
#pragma unroll
        for (int m = 0; m < M; ++m) red[(m * 8 + k) * 64 + lane] = acc[m][0] + acc[m][1];
    }
    __syncthreads();
    for (int mi = k; mi < mcount; mi += 8) {                           // wave k reduces tokens k, k+8, ...
        if (live) {
            float v = lane_tree(&red[mi * 8 * 64 + lane]);
            const int grow = static_cast<int>(ggml_row(static_cast<int64_t>(tile) * 32 + r, S.rows, S.interleave));
            if (A.bias) v = v + A.bias[static_cast<size_t>(expert) * S.rows + grow];
            if (A.epilogue == 0) A.dst[static_cast<size_t>(jobs[c0 + mi]) * S.rows + grow] = v;
            else vals[mi * 64 + lane] = v;
        }
    }
    if (A.epilogue == 1) {
        __syncthreads();
        for (int mi = k; mi < mcount; mi += 8)
            if (lane < 32)
                glu_requant_block(vals + mi * 64, lane, pair, A.dst_xrows + static_cast<size_t>(jobs[c0 + mi]) * A.dst_lay.stride(),
                                  A.dst_lay, A.activation, A.alpha, A.limit);
    }
    __syncthreads();
}

// Batched GEMV: one workgroup per (tile pair, chunk), a chunk being up to MT consecutive jobs of
// one active expert (the chunk list holds each chunk's expert and first job, built on the device
// from the grouping). Each XCD takes a contiguous range of (pair, chunk) items with the chunk
// fastest, so the chunks of one expert run side by side on one XCD and share the tile pair's
// weight stream through its L2, where a workgroup walking an expert's chunks in turn streamed the
// weights once per chunk (config 1 shape at 64 tokens: 40 % of the experts hold more than eight
// jobs). A chunk runs at the narrowest token width in {1, 2, 4, 8} that holds it (a uniform
// branch: most experts of a small decode batch see one or two tokens, and a narrow width keeps
// the per-block token loop short).
template <int TYPE, int MT, bool NEG>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void expert_gemv_kernel(KernelArgs A) {
    __shared__ float vals[MT * 64];
    __shared__ int s_flag;
    // MT activation rows; after the weight stream, the [MT][8 slices][64 rows] partial sums
    // (8 KiB less LDS per token of width than separate buffers: three workgroups per CU at MT = 8
    // with K = 2880)
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_tok[];
    float * red = reinterpret_cast<float *>(lds_tok);
    // Per-expert metadata is read through the constant address space so it stays scalar.
    const int n_items = *as_const<int32_t>(A.n_chunks);
    const int total = n_items * A.pairs;
    const int per_xcd = (total + 7) >> 3;
    const int slot8 = static_cast<int>(blockIdx.x >> 3);
    const int item_pair = static_cast<int>(blockIdx.x & 7) * per_xcd + slot8;
    if (slot8 >= per_xcd || item_pair >= total) return;
    const int pair = item_pair / n_items;
    const int item = item_pair - pair * n_items;
    const int expert = as_const<int32_t>(A.chunk_expert)[item];
    const int c0 = as_const<int32_t>(A.chunk_start)[item];
    const int count = as_const<int32_t>(A.counts)[expert];
    const __attribute__((address_space(4))) int32_t * jobs = as_const<int32_t>(A.rows_list) + as_const<int32_t>(A.offsets)[expert];
    const int slot = A.expert_to_slot ? as_const<int32_t>(A.expert_to_slot)[expert] : expert;
    const int mcount = count - c0 < MT ? count - c0 : MT;
    if (mcount <= 0) return;
    if (slot < 0 || slot >= A.shape.n_slots) {
        // Expert not resident in this bank: the chunk's outputs of this tile pair become NaN, as
        // in the decode kernels, so a bad expert->slot map can never leave stale workspace data in
        // a result. Epilogue 1 poisons the block scale of the GLU block this workgroup owns.
        const float nan = __builtin_nanf("");
        if (A.epilogue == 0) {
            for (int i = threadIdx.x; i < mcount * 64; i += kThreads) {
                const int64_t brow = static_cast<int64_t>(pair) * 64 + (i & 63);
                if (brow < A.shape.rows)
                    A.dst[static_cast<size_t>(jobs[c0 + (i >> 6)]) * A.shape.rows + ggml_row(brow, A.shape.rows, A.shape.interleave)] = nan;
            }
        } else {
            for (int j = threadIdx.x; j < mcount; j += kThreads)
                reinterpret_cast<float *>(A.dst_xrows + static_cast<size_t>(jobs[c0 + j]) * A.dst_lay.stride() +
                                          A.dst_lay.da_offset())[pair] = nan;
        }
        return;
    }

    const Shape S = A.shape;
    const int k = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // lane slice, wave-uniform
    const int lane = threadIdx.x & 63;
    const int r = lane & 31;
    const int tile = pair * 2 + (lane >> 5);
    const bool live = tile * 32 < S.rows;                              // the last tile pair may be half
    const uint8_t * slot_base = A.bank + static_cast<size_t>(slot) * S.slot_bytes;
    const BufLane B = buf_lane<TYPE>(slot_base, S.slot_bytes, S.codes_bytes, live ? tile : 0, k, r, S.nb);
    if (MT >= 8 && mcount > 4)
        gemv_chunk<TYPE, (MT >= 8 ? 8 : 1), NEG>(A, B, jobs, expert, c0, mcount, pair, k, lane, r, tile, live, lds_tok, red, vals, &s_flag);
    else if (MT >= 4 && mcount > 2)
        gemv_chunk<TYPE, (MT >= 4 ? 4 : 1), NEG>(A, B, jobs, expert, c0, mcount, pair, k, lane, r, tile, live, lds_tok, red, vals, &s_flag);
    else if (MT >= 2 && mcount > 1)
        gemv_chunk<TYPE, (MT >= 2 ? 2 : 1), NEG>(A, B, jobs, expert, c0, mcount, pair, k, lane, r, tile, live, lds_tok, red, vals, &s_flag);
    else
        gemv_chunk<TYPE, 1, NEG>(A, B, jobs, expert, c0, mcount, pair, k, lane, r, tile, live, lds_tok, red, vals, &s_flag);
}

// ------------------------------------------------------------------------------ fused decode
// Single-token decode runs two launches per layer.
// Kernel A (gate_up, 256 threads = 8 lane slices x 32 rows): every workgroup routes (top-k +
//   softmax over the layer's given logits; a few hundred bytes from L2) and, with the same
//   loads in flight, combines the previous layer (ggml MUL by the routing weight, then ADD in
//   rank order) or takes the input; it then issues its expert's weights, quantizes the input to
//   Q8_0, runs the gate_up GEMV of its tile pair with biases, GLU and requantization into one
//   32-element block of the rank's down activation row. Workgroup (0,0) publishes the routing.
// Kernel B (down, 256 threads = 8 lane slices x 32 rows, so its 360 workgroups spread over all
//   CUs): loads the activation row and the routed expert id together, streams the down weights
//   of one tile and writes y[rank] with the down bias.
// A single launch per layer with device-side readiness counters (down workgroups prefetching
// while gate_up runs) measured slower: producer-to-consumer signalling across XCDs took several
// microseconds under full HBM load, more than a kernel boundary.
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
    const float * bias;        // gate_up bias [n_expert][rows] (ggml row order) or null
    float * act_f;             // [top_k][intermediate] GLU outputs (fp32)
    int32_t * route_ids;       // [top_k] this layer's routing
    float * route_w;           // [top_k]
    int32_t * route_slots;     // [top_k] bank slot of each pick (expert_to_slot applied), or null
    int activation;
    float alpha, limit;
    const uint8_t * host_base; // pinned host copy of the layer's experts (slot layout), or null
    int64_t host_stride;
    uint8_t * stage;           // device copies of host-read picks: rank r at stage + r * stage_stride, or null
    int64_t stage_stride;
};

constexpr int kDownThreads = 256;


// x86 quantize_row_q8_0 of eight elements (part p of block b, thread t = 4b + p) of the layer input
// into the activation row `act` (codes + block scales); block maximum over the thread quad (DPP),
// so all four threads of a quad must call it together.
template <int TYPE>
__device__ __forceinline__ void quantize_x8(const float (&x)[8], int t, uint8_t * act, const XrowLayout & L, int nb) {
    const int b = t >> 2, part = t & 3;
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(x[i]));
    amax = quad_max(amax);
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    float q[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float v = rintf(x[i] * id);
        q[i] = v > 127.0f ? 127.0f : (v < -128.0f ? -128.0f : v);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int64_t sk = 2 * part + h;
        if (TYPE == 39) {
            half2_t p0, p1;
            p0.x = static_cast<_Float16>(q[4 * h]); p0.y = static_cast<_Float16>(q[4 * h + 1]);
            p1.x = static_cast<_Float16>(q[4 * h + 2]); p1.y = static_cast<_Float16>(q[4 * h + 3]);
            u32x2 v;
            v.x = __builtin_bit_cast(unsigned, p0);
            v.y = __builtin_bit_cast(unsigned, p1);
            *reinterpret_cast<u32x2 *>(act + (sk * nb + b) * 8) = v;
        } else {
            unsigned v = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                v |= static_cast<unsigned>(static_cast<uint8_t>(static_cast<signed char>(q[4 * h + i]))) << (8 * i);
            *reinterpret_cast<unsigned *>(act + (sk * nb + b) * 4) = v;
        }
    }
    if (part == 0) reinterpret_cast<float *>(act + L.da_offset())[b] = static_cast<float>(static_cast<_Float16>(d));
}

// One wavefront's top-k over n <= 64 NPL routing keys held in registers (lg[i]: expert lane + 64 i,
// already route_key'd, so never NaN), in the total order (value desc, then lower index;
// tools/trace/topk-tie-probe.cpp:111-113): pick j is the best element strictly after pick j - 1.
// Each round takes the wave maximum of the lanes' best remaining candidates (DPP and a swizzle,
// no LDS traffic), then the lowest expert index holding it with one ballot per register row.
// Lane j < k returns pick j in (sel_v, sel_i). No barrier: every wave can route for itself.
template <int NPL>
__device__ __forceinline__ void wave_topk_regs(const float (&lg)[NPL], int n, int k, float & sel_v, int & sel_i) {
    const int lane = threadIdx.x & 63;
    float prev_v = INFINITY;
    int prev_i = -1;
    sel_v = 0.0f;
    sel_i = -1;
    for (int j = 0; j < k; ++j) {
        float best = -INFINITY;
        int best_i = -1;
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            const int c = lane + 64 * i;
            const float v = lg[i];
            const bool after_prev = v < prev_v || (v == prev_v && c > prev_i);
            if (c < n && after_prev && (best_i < 0 || v > best)) { best = v; best_i = c; }
        }
        const float h = half_wave_max(best);
        const float m0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, h), 0));
        const float m1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, h), 32));
        const float top = m0 > m1 ? m0 : m1;
        int pick = -1;
#pragma unroll
        for (int i = NPL - 1; i >= 0; --i) {
            const uint64_t m = __ballot(best_i >= 0 && best == top && (best_i >> 6) == i);
            if (m) pick = 64 * i + __builtin_ctzll(m);
        }
        if (lane == j) { sel_v = top; sel_i = pick; }
        prev_v = top;
        prev_i = pick;
    }
}

// ggml soft_max over the k picks held by lanes 0..k-1 (expf(v - max), sum in double in pick order,
// scale by (float)(1/sum)); returns the weight of pick `lane` (lane < k).
__device__ __forceinline__ float wave_pick_softmax(float sel_v, int k) {
    const int lane = threadIdx.x & 63;
    float max = -INFINITY;
    for (int j = 0; j < k; ++j) {
        const float v = __shfl(sel_v, j);
        max = v > max ? v : max;
    }
    const float e = lane < k ? expf_rn(sel_v - max) : 0.0f;
    double sum = 0.0;
    for (int j = 0; j < k; ++j) sum += static_cast<double>(__shfl(e, j));
    return e * static_cast<float>(1.0 / sum);
}

// Dynamic LDS of kernels A and B: [meta of 1 tile][activation row][scale table of 1 tile].
template <int TYPE>
size_t decode_lds_bytes(int nb) {
    return 32 * static_cast<size_t>(nb) * (TYPE == 39 ? 1 : 2) +
           ((static_cast<size_t>(nb) * (TYPE == 39 ? 68 : 36) + 15) & ~static_cast<size_t>(15)) +
           static_cast<size_t>((nb + 3) / 4) * 512;
}

// Kernel A: one 32-row bank tile (16 gate + 16 up rows) of one rank per workgroup, wave w holding
// lane slices 2w (lanes 0..31) and 2w + 1 (lanes 32..63); 2 x hidden / 32 small workgroups spread
// evenly over the CUs. Prologue order is what sets its latency: the routing logits, this wave's
// share of the expert->slot map and the layer-input loads go out first; each wave routes on its
// own registers (no barrier), and the expert's weight stream is issued as soon as the logits are
// in, while the layer-input loads are still landing. Only then the input is combined (ggml MUL by
// the routing weight, then ADD in rank order) and quantized, thread t owning elements 8t..8t+7
// and 8(t + 256).., straight from registers into the activation row. The tile's 16 GLU outputs
// go out as fp32; kernel B quantizes each 32-element block of them (the pair of tiles).
// STAGE (launches with a staging area, the deferred host tier): a workgroup whose pick is read
// from the pinned host copy copies its tile into the staging area first and streams that copy.
// A separate instantiation, so the resident-only kernels carry none of that code.
template <int TYPE, int NPL, int NB, bool STAGE>
__global__ __launch_bounds__(kDownThreads) __attribute__((amdgpu_waves_per_eu(3))) void decode_gate_up_kernel(DecodeArgs A) {
    constexpr int D = gate_up_depth<TYPE>();
    constexpr int kChunks = 2;                     // 8-element input chunks per thread (hidden <= 4096)
    __shared__ float red[8][32];
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_dyn[];
    const Shape S = A.shape;
    const int nb = NB > 0 ? NB : S.nb;
    uint8_t * lmeta = lds_dyn;
    uint8_t * act = lmeta + meta_tile_bytes<TYPE>(nb);
    float * lscale = reinterpret_cast<float *>(act + ((A.lay.flag_offset() + 15) & ~15ll));
    const int lane = threadIdx.x & 63, r = lane & 31;
    const int k = (threadIdx.x >> 6) * 2 + (lane >> 5);
    const int tile = blockIdx.x, rank = blockIdx.y;
    const int n = A.n_expert;

    // 1. routing keys and slots of experts lane + 64 i; the first four ranks of the layer input.
    // Every load below is unconditional (clamped indices), so the compiler's in-order wait
    // counts stay exact: the top-k waits for the logits only, the slot for the map only, and the
    // input loads are still in flight when the weight stream goes out.
    float lg[NPL];
    int sl[NPL];
    const int32_t * map = A.expert_to_slot;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        const int c = lane + 64 * i;
        lg[i] = A.logits[c < n ? c : 0];
    }
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        const int c = lane + 64 * i;
        sl[i] = map ? map[c < n ? c : 0] : c;
    }
    const int k0 = A.x_in ? 1 : (A.top_k < 4 ? A.top_k : 4);
    float yv[kChunks][4][8];
#pragma unroll
    for (int h = 0; h < kChunks; ++h) {
        const int e0 = (threadIdx.x + h * kDownThreads) * 8;
        const int ec = e0 < nb * 32 ? e0 : 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int jj = j < k0 ? j : 0;
            const float * src = A.x_in ? A.x_in + ec : A.prev_y + static_cast<int64_t>(jj) * nb * 32 + ec;
            const float4 lo = *reinterpret_cast<const float4 *>(src);
            const float4 hi = *reinterpret_cast<const float4 *>(src + 4);
            yv[h][j][0] = lo.x; yv[h][j][1] = lo.y; yv[h][j][2] = lo.z; yv[h][j][3] = lo.w;
            yv[h][j][4] = hi.x; yv[h][j][5] = hi.y; yv[h][j][6] = hi.z; yv[h][j][7] = hi.w;
        }
    }

    // 2. this wave's routing; the slot of the pick at `rank`
#pragma unroll
    for (int i = 0; i < NPL; ++i) lg[i] = route_key(lg[i]);
    float sel_v;
    int sel_i;
    wave_topk_regs<NPL>(lg, n, A.top_k, sel_v, sel_i);
    const int expert = __builtin_amdgcn_readlane(sel_i, rank);
    int sv = sl[0];
#pragma unroll
    for (int i = 1; i < NPL; ++i)
        if ((expert >> 6) == i) sv = sl[i];
    const int slot = __builtin_amdgcn_readlane(sv, expert & 63);

    // 3. the weight stream: tile meta, the ring, the tail, the bias. A pick outside the bank
    // streams the pinned host copy when there is one (and is otherwise poisoned below).
    const bool in_bank = slot >= 0 && slot < S.n_slots;
    const bool slot_ok = in_bank || A.host_base != nullptr;
    const uint8_t * slot_base = in_bank ? A.bank + static_cast<size_t>(slot) * S.slot_bytes
                                        : (slot_ok ? A.host_base + static_cast<size_t>(expert) * A.host_stride : A.bank);
    if constexpr (STAGE) {
        if (!in_bank && slot_ok) {
            // a host-read pick: copy the tile into the staging area once, then stream the copy
            uint8_t * staged = A.stage + static_cast<size_t>(rank) * A.stage_stride;
            copy_slot_tile<TYPE, kDownThreads>(slot_base, staged, tile, nb, S.codes_bytes);
            __syncthreads();
            slot_base = staged;
        }
    }
    const uint8_t * codes_tile = slot_base + static_cast<size_t>(tile) * 32 * nb * (TYPE == 39 ? 16 : 32);
    const int mbytes = meta_tile_bytes<TYPE>(nb);
    u32x4 mst[2];
    load_meta<kDownThreads>(mst, slot_base + S.codes_bytes + static_cast<size_t>(tile) * mbytes, slot_ok ? mbytes : 0);
    Group ring[D];
    Tail tl;
    // unconditional loads (a pick with no valid slot reads the bank's first slot and is poisoned
    // below), so the stream's wait counts stay exact
    preload_ring<TYPE, D, true>(ring, codes_tile, nullptr, k, r, nb, true);
    preload_tail<TYPE, true>(tl, codes_tile, nullptr, k, r, nb, true);
    const int grow = static_cast<int>(ggml_row(static_cast<int64_t>(tile) * 32 + r, S.rows, S.interleave));
    float bias_v = 0.0f;
    if (k == 0 && slot_ok && A.bias) bias_v = A.bias[static_cast<size_t>(expert) * S.rows + grow];

    // 4. the layer input, combined in rank order, quantized into the activation row (the routing
    // weights are read only now: their scalar loads would otherwise hold up the routing's waits)
    float wv[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if (!A.x_in) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (j < k0) wv[j] = A.prev_w[j];
    }
#pragma unroll
    for (int h = 0; h < kChunks; ++h) {
        const int t = threadIdx.x + h * kDownThreads;
        const int e0 = t * 8;
        if (e0 < nb * 32) {
            float x[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = yv[h][0][i];
            if (!A.x_in) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (j < k0) {
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            const float term = yv[h][j][i] * wv[j];
                            x[i] = j == 0 ? term : x[i] + term;
                        }
                    }
                for (int j = 4; j < A.top_k; ++j) {
                    const float * src = A.prev_y + static_cast<int64_t>(j) * nb * 32 + e0;
                    const float w = A.prev_w[j];
                    const float4 lo = *reinterpret_cast<const float4 *>(src);
                    const float4 hi = *reinterpret_cast<const float4 *>(src + 4);
                    const float y[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
                    for (int i = 0; i < 8; ++i) x[i] = x[i] + y[i] * w;
                }
            }
            quantize_x8<TYPE>(x, t, act, A.lay, nb);
        }
    }
    store_meta<kDownThreads>(mst, lmeta, mbytes);
    __syncthreads();
    build_scales<TYPE, kDownThreads, 1>(lscale, lmeta, reinterpret_cast<const float *>(act + A.lay.da_offset()), nb, mbytes);
    __syncthreads();
    float acc[2] = {0.0f, 0.0f};
    decode_stream<TYPE, D, NB>(ring, tl, codes_tile, k, r, nb, true, act + static_cast<int64_t>(k) * nb * A.lay.code_entry(),
                               lscale + r * 4, acc);
    red[k][r] = acc[0] + acc[1];
    __syncthreads();
    if (threadIdx.x < 32) {
        const float * l = &red[0][r];
        const float s0 = l[4 * 32] + l[0], s1 = l[5 * 32] + l[1 * 32];
        const float s2 = l[6 * 32] + l[2 * 32], s3 = l[7 * 32] + l[3 * 32];
        float v = (s0 + s2) + (s1 + s3);           // lane_tree over slices 32 floats apart
        if (A.bias) v = v + bias_v;
        red[0][r] = v;                              // rows r: 0..15 gate, 16..31 up
    }
    __syncthreads();
    if (threadIdx.x < 16) {
        float g = glu(A.activation, red[0][threadIdx.x], red[0][threadIdx.x + 16], A.alpha, A.limit);
        if (!slot_ok) g = __builtin_nanf("");      // expert not resident in this bank: loud output
        A.act_f[static_cast<size_t>(rank) * (S.rows / 2) + tile * 16 + threadIdx.x] = g;
    }
    if (threadIdx.x < 64 && tile == 0 && rank == 0) {
        const float w = wave_pick_softmax(sel_v, A.top_k);
        int ps = 0;                               // lane j: slot of pick j
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            const int v = __shfl(sl[i], sel_i & 63);
            if ((sel_i >> 6) == i) ps = v;
        }
        if (lane < A.top_k) {
            A.route_ids[lane] = sel_i;
            A.route_w[lane] = w;
            if (A.route_slots) A.route_slots[lane] = ps;
        }
    }
}

struct DecodeDownArgs {
    const uint8_t * bank;
    Shape shape;
    const int32_t * expert_to_slot;
    XrowLayout lay;            // down activation format (nb = intermediate / 32)
    const float * act_f;       // [top_k][intermediate] GLU outputs written by kernel A
    const int32_t * route_ids; // [top_k]
    const int32_t * route_slots;  // [top_k] slots written by kernel A (same map), or null
    const float * bias;        // down bias [n_expert][rows] or null
    float * y;                 // [top_k][rows]
    const uint8_t * host_base; // pinned host copy of the layer's experts (slot layout), or null
    int64_t host_stride;
    uint8_t * stage;           // as in DecodeArgs (the down part of each rank's copy)
    int64_t stage_stride;
};

// Kernel B: one 32-row tile of one rank; wave w holds lane slices 2w (lanes 0..31) and 2w + 1
// (lanes 32..63) of the tile's rows. Its prologue requantizes the rank's GLU outputs (x86
// quantize_row_q8_0 per 32-element block, the arithmetic of the reference's activation
// quantization) into the LDS activation row while its weight stream is in flight.
template <int TYPE, int NB, bool STAGE>
__global__ __launch_bounds__(kDownThreads) void decode_down_kernel(DecodeDownArgs A) {
    constexpr int D = down_depth<TYPE>();
    __shared__ float red[8][32];
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_dyn[];
    const Shape S = A.shape;
    const int nb = NB > 0 ? NB : S.nb;
    uint8_t * lmeta = lds_dyn;
    uint8_t * act = lmeta + meta_tile_bytes<TYPE>(nb);
    float * lscale = reinterpret_cast<float *>(act + ((A.lay.flag_offset() + 15) & ~15ll));
    const int lane = threadIdx.x & 63, r = lane & 31;
    const int k = (threadIdx.x >> 6) * 2 + (lane >> 5);
    const int tile = blockIdx.x, rank = blockIdx.y;
    // The GLU outputs (independent of the routing) are loaded together with the expert id.
    constexpr int kChunks = 2;                     // 8-element chunks per thread (intermediate <= 4096)
    const float * xf = A.act_f + static_cast<size_t>(rank) * nb * 32;
    float xq[kChunks][8];
#pragma unroll
    for (int h = 0; h < kChunks; ++h) {
        const int e0 = (threadIdx.x + h * kDownThreads) * 8;
        const int ec = e0 < nb * 32 ? e0 : 0;
        const float4 lo = *reinterpret_cast<const float4 *>(xf + ec);
        const float4 hi = *reinterpret_cast<const float4 *>(xf + ec + 4);
        xq[h][0] = lo.x; xq[h][1] = lo.y; xq[h][2] = lo.z; xq[h][3] = lo.w;
        xq[h][4] = hi.x; xq[h][5] = hi.y; xq[h][6] = hi.z; xq[h][7] = hi.w;
    }
    const int expert = as_const<int32_t>(A.route_ids)[rank];
    const int slot = A.route_slots ? as_const<int32_t>(A.route_slots)[rank]
                                   : (A.expert_to_slot ? as_const<int32_t>(A.expert_to_slot)[expert] : expert);
    const bool in_bank = slot >= 0 && slot < S.n_slots;
    const bool slot_ok = in_bank || A.host_base != nullptr;
    const uint8_t * slot_base = in_bank ? A.bank + static_cast<size_t>(slot) * S.slot_bytes
                                        : (slot_ok ? A.host_base + static_cast<size_t>(expert) * A.host_stride : A.bank);
    if constexpr (STAGE) {                        // as in kernel A
        if (!in_bank && slot_ok) {
            uint8_t * staged = A.stage + static_cast<size_t>(rank) * A.stage_stride;
            copy_slot_tile<TYPE, kDownThreads>(slot_base, staged, tile, nb, S.codes_bytes);
            __syncthreads();
            slot_base = staged;
        }
    }
    const uint8_t * codes_tile = slot_base + static_cast<size_t>(tile) * 32 * nb * (TYPE == 39 ? 16 : 32);
    const int mbytes = meta_tile_bytes<TYPE>(nb);
    u32x4 mst[2];
    load_meta<kDownThreads>(mst, slot_base + S.codes_bytes + static_cast<size_t>(tile) * mbytes, slot_ok ? mbytes : 0);
    Group ring[D];
    Tail tl;
    preload_ring<TYPE, D, true>(ring, codes_tile, nullptr, k, r, nb, true);   // unconditional, as in kernel A
    preload_tail<TYPE, true>(tl, codes_tile, nullptr, k, r, nb, true);
    const int row = tile * 32 + r;
    float bias_v = 0.0f;
    if (k == 0 && slot_ok && A.bias) bias_v = A.bias[static_cast<size_t>(expert) * S.rows + row];
#pragma unroll
    for (int h = 0; h < kChunks; ++h) {
        const int t = threadIdx.x + h * kDownThreads;
        if (t * 8 < nb * 32) quantize_x8<TYPE>(xq[h], t, act, A.lay, nb);
    }
    store_meta<kDownThreads>(mst, lmeta, mbytes);
    __syncthreads();
    build_scales<TYPE, kDownThreads, 1>(lscale, lmeta, reinterpret_cast<const float *>(act + A.lay.da_offset()), nb,
                                        mbytes);
    __syncthreads();
    float acc[2] = {0.0f, 0.0f};
    decode_stream<TYPE, D, NB>(ring, tl, codes_tile, k, r, nb, true, act + static_cast<int64_t>(k) * nb * A.lay.code_entry(),
                               lscale + r * 4, acc);
    red[k][r] = acc[0] + acc[1];
    __syncthreads();
    if (threadIdx.x < 32) {
        const float * l = &red[0][r];
        const float s0 = l[4 * 32] + l[0], s1 = l[5 * 32] + l[1 * 32];
        const float s2 = l[6 * 32] + l[2 * 32], s3 = l[7 * 32] + l[3 * 32];
        float v = (s0 + s2) + (s1 + s3);           // lane_tree over slices 32 floats apart
        if (A.bias) v = v + bias_v;
        if (!slot_ok) v = __builtin_nanf("");      // expert not resident in this bank: loud output
        A.y[static_cast<size_t>(rank) * S.rows + row] = v;
    }
}

// ------------------------------------------------------------------------ linked decode layers
// One launch per layer boundary: launch j runs the down tiles of layer j - 1 (workgroups
// [0, n_down)) and the gate_up tiles of layer j (the rest), so the two weight streams overlap and
// a step takes L + 1 launches instead of 2L + 1. Every layer routes on its given logits, so a
// gate_up tile knows its expert at launch and issues its whole weight tile before its input
// exists. The input is published tile by tile by the down tiles of the same launch:
//   - a down tile writes its 32 rows of y[rank] with agent-coherent stores (sc1: written through
//     past the XCD's L2, read back the same way by any XCD), waits for them, then bumps the
//     tile's arrival counter (top_k arrivals per launch: no counter is contended);
//   - the last arriver of a tile combines the top_k ranks of its 32 rows in rank order (ggml MUL
//     by the routing weight, then ADD), quantizes that 32-element block of the next layer's input
//     (x86 quantize_row_q8_0) into the shared activation row, waits for those stores and sets the
//     tile's flag to the step's epoch, in kLinkCopies copies (one per group of pollers);
//   - in a gate_up workgroup a fifth wave, which issues no weight loads (vector loads retire in
//     order per wave, so a poll queued behind a weight stream would wait for all of it), polls
//     the flags with a bounded wait, copies the activation row into LDS and joins the scale-table
//     build while the four compute waves' weights are landing.
// No release/acquire fence is used: at agent scope those write back / invalidate a whole L2.
// Forward progress: down workgroups never wait and precede every gate_up workgroup in dispatch
// order. A gate_up wait that outlives kLinkPollRounds poll rounds sets the error word and leaves
// that workgroup's outputs unspecified instead of spinning, so every wave exits.
// The last launch (no gate_up part) combines into the step output and advances the epoch.
constexpr int kLinkThreads = 320;                  // 4 compute waves + 1 helper wave
constexpr int kLinkCopies = 8;
constexpr int kLinkCopyStride = 1152;              // u32 between flag copies (4.5 KiB)
// Poll rounds before a wait gives up: each round sleeps 4 x 64 cycles and waits for two loads, so
// this is more than 0.1 s. (No timer is read: s_memrealtime goes through the memory interface
// and waits behind the weight streams under full HBM load.)
constexpr uint32_t kLinkPollRounds = 1u << 20;

struct LinkArgs {
    int n_down, n_gate_up;      // workgroups of each role in this launch
    int n_expert, top_k;
    // down tiles of layer l - 1
    const uint8_t * dn_bank;
    Shape dn_shape;
    XrowLayout dn_lay;          // down activation row (nb = intermediate / 32)
    const float * dn_act_f;     // [top_k][intermediate] GLU outputs of layer l - 1
    const int32_t * dn_ids;     // [top_k]
    const int32_t * dn_slots;   // [top_k]
    const float * dn_w;         // [top_k]
    const float * dn_bias;      // [n_expert][hidden] or null
    float * y;                  // [top_k][hidden], agent-coherent accesses only
    uint32_t * counters;        // [hidden / 32] arrival counters of layer l - 1
    float * out;                // step output [hidden] (last launch), else null
    // the next-layer input row, published by the last arrivers and read by the gate_up tiles
    uint8_t * xq;               // gate_up activation layout, agent-coherent accesses only
    uint32_t * flags;           // [kLinkCopies][kLinkCopyStride] flags of layer l
    // gate_up tiles of layer l
    const uint8_t * gu_bank;
    Shape gu_shape;
    XrowLayout gu_lay;
    const int32_t * expert_to_slot;
    const float * logits;       // [n_expert]
    const float * x_in;         // layer input (first launch), else null
    const float * gu_bias;      // [n_expert][2 * intermediate] or null
    float * act_f;              // [top_k][intermediate] GLU outputs of layer l
    int32_t * route_ids;
    float * route_w;
    int32_t * route_slots;
    int activation;
    float alpha, limit;
    uint32_t * epoch;           // step counter: flags of this step hold its value
    int advance_epoch;          // last launch: workgroup 0 advances it
    uint32_t * error;           // set to 1 when a wait times out
};

// Groups of a lane's row slice held in flight from the start: the whole slice.
constexpr int link_ring_depth(int nb) { return nb / 8; }

template <class T>
__device__ __forceinline__ T coherent_load(const T * p) {
    return __hip_atomic_load(const_cast<T *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ void coherent_store(T * p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Every store this wave issued has been acknowledged (for agent-coherent stores: performed at the
// point where every XCD reads them); the "memory" clobber keeps the compiler from moving memory
// operations across it.
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Helper wave: x86 Q8_0 of a row of nb blocks (fp32, global) into the LDS activation row, eight
// elements per lane and round (thread t = 4b + part of quantize_x8), every load issued first.
template <int TYPE, int NB>
__device__ __forceinline__ void helper_quantize_row(const float * src, uint8_t * act, const XrowLayout & L) {
    constexpr int R = (NB * 4 + 63) / 64;
    const int lane = threadIdx.x & 63;
    float xv[R][8];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int t = lane + 64 * i;
        const int e0 = t < NB * 4 ? t * 8 : 0;
        const float4 lo = *reinterpret_cast<const float4 *>(src + e0);
        const float4 hi = *reinterpret_cast<const float4 *>(src + e0 + 4);
        xv[i][0] = lo.x; xv[i][1] = lo.y; xv[i][2] = lo.z; xv[i][3] = lo.w;
        xv[i][4] = hi.x; xv[i][5] = hi.y; xv[i][6] = hi.z; xv[i][7] = hi.w;
    }
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int t = lane + 64 * i;
        if (t < NB * 4) quantize_x8<TYPE>(xv[i], t, act, L, NB);   // quads of lanes stay whole: 4 | NB * 4
    }
}

// Helper wave: waits until the n tile flags of this copy hold `epoch` (bounded), then copies the
// published activation row (codes and block scales) into LDS.
template <int NB>
__device__ __forceinline__ void helper_fetch_row(const LinkArgs & A, uint32_t epoch, uint8_t * act) {
    const int lane = threadIdx.x & 63;
    const int n = NB;                                 // one flag per 32-element block
    const uint32_t * f = A.flags + (blockIdx.x % kLinkCopies) * kLinkCopyStride;
    const int i0 = lane < n ? lane : n - 1, i1 = lane + 64 < n ? lane + 64 : n - 1;
    for (uint32_t round = 0;; ++round) {
        const uint32_t v0 = coherent_load(f + i0), v1 = coherent_load(f + i1);
        if (__ballot(v0 != epoch || v1 != epoch) == 0) break;
        if (round == kLinkPollRounds) {
            if (lane == 0) coherent_store(A.error, 1u);
            break;
        }
        __builtin_amdgcn_s_sleep(4);
    }
    asm volatile("" ::: "memory");
    constexpr int kWords = NB * 68 / 8;               // NB x (64 B of f16 codes + 4 B scale)
    constexpr int W = (kWords + 127) / 128;           // two batches of W words per lane
    const uint64_t * src = reinterpret_cast<const uint64_t *>(A.xq);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        uint64_t v[W];
#pragma unroll
        for (int i = 0; i < W; ++i) {
            const int w = lane + 64 * (h * W + i);
            v[i] = coherent_load(src + (w < kWords ? w : 0));
        }
#pragma unroll
        for (int i = 0; i < W; ++i) {
            const int w = lane + 64 * (h * W + i);
            if (w < kWords) reinterpret_cast<uint64_t *>(act)[w] = v[i];
        }
    }
}

// Last arriver of down tile `blk`: lanes 0..31 of wave 0 hold the combined next-layer input of
// the tile's 32 rows, i.e. block blk. x86 Q8_0 of the block (the quantize_x8 arithmetic), the
// codes and scale stored into the shared row, then the flags.
__device__ __forceinline__ void publish_block(float x, int blk, const LinkArgs & A, uint32_t epoch) {
    const int lane = threadIdx.x & 63;
    const XrowLayout & L = A.gu_lay;
    const float amax = half_wave_max(lane < 32 ? fmaxf(0.0f, fabsf(x)) : 0.0f);
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    float q = rintf(x * id);
    q = q > 127.0f ? 127.0f : (q < -128.0f ? -128.0f : q);
    const unsigned h = __builtin_bit_cast(unsigned short, static_cast<_Float16>(q));
    const unsigned h1 = __shfl_down(h, 1), h2 = __shfl_down(h, 2), h3 = __shfl_down(h, 3);
    const uint64_t packed = static_cast<uint64_t>(h | (h1 << 16)) | (static_cast<uint64_t>(h2 | (h3 << 16)) << 32);
    if (lane < 32 && (lane & 3) == 0)
        coherent_store(reinterpret_cast<uint64_t *>(A.xq + (static_cast<int64_t>(lane >> 2) * L.nb + blk) * 8), packed);
    if (lane == 0)
        coherent_store(reinterpret_cast<float *>(A.xq + L.da_offset()) + blk, static_cast<float>(static_cast<_Float16>(d)));
    wait_stores();
    if (lane < kLinkCopies) coherent_store(A.flags + lane * kLinkCopyStride + blk, epoch);
}

// Down tile (rank, tile) of layer l - 1: as kernel B, with the whole tile preloaded, the GLU row
// quantized by the helper wave, and the y rows published for the last arriver.
template <int TYPE, int NB>
__device__ __forceinline__ void link_down(const LinkArgs & A, int wg, uint8_t * lds_dyn, float (&red)[8][32]) {
    constexpr int G = link_ring_depth(NB);
    const Shape S = A.dn_shape;
    const int tiles = S.rows / 32;
    const int rank = wg / tiles, tile = wg - rank * tiles;
    const int mbytes = meta_tile_bytes<TYPE>(NB);
    uint8_t * lmeta = lds_dyn;
    uint8_t * act = lmeta + mbytes;
    float * lscale = reinterpret_cast<float *>(act + ((A.dn_lay.flag_offset() + 15) & ~15ll));
    const int tid = threadIdx.x, lane = tid & 63, r = lane & 31;
    const bool compute = tid < kDownThreads;                // waves 0..3; wave 4 is the helper
    const int k = (tid >> 6) * 2 + (lane >> 5);
    const int row = tile * 32 + r;
    const int expert = as_const<int32_t>(A.dn_ids)[rank];
    const int slot = as_const<int32_t>(A.dn_slots)[rank];
    const bool slot_ok = slot >= 0 && slot < S.n_slots;
    const uint8_t * slot_base = A.dn_bank + (slot_ok ? static_cast<size_t>(slot) * S.slot_bytes : 0);
    const uint8_t * codes_tile = slot_base + static_cast<size_t>(tile) * 32 * NB * 16;
    Group ring[G];
    Tail tl;
    float bias_v = 0.0f;
    if (compute) {
        u32x4 mst[2];
        load_meta<kDownThreads>(mst, slot_base + S.codes_bytes + static_cast<size_t>(tile) * mbytes, mbytes);
        preload_ring<TYPE, G, true>(ring, codes_tile, nullptr, k, r, NB, true);
        preload_tail<TYPE, true>(tl, codes_tile, nullptr, k, r, NB, true);
        if (k == 0 && A.dn_bias) bias_v = A.dn_bias[static_cast<size_t>(expert) * S.rows + row];
        store_meta<kDownThreads>(mst, lmeta, mbytes);
    } else {
        helper_quantize_row<TYPE, NB>(A.dn_act_f + static_cast<size_t>(rank) * NB * 32, act, A.dn_lay);
    }
    __syncthreads();
    build_scales<TYPE, kLinkThreads, 1>(lscale, lmeta, reinterpret_cast<const float *>(act + A.dn_lay.da_offset()), NB, mbytes);
    __syncthreads();
    if (compute) {
        float acc[2] = {0.0f, 0.0f};
        decode_stream<TYPE, G, NB>(ring, tl, codes_tile, k, r, NB, false,
                                   act + static_cast<int64_t>(k) * NB * A.dn_lay.code_entry(), lscale + r * 4, acc);
        red[k][r] = acc[0] + acc[1];
    }
    __syncthreads();
    if (tid >= 64) return;
    // wave 0: this rank's rows, then the arrival count of the tile
    if (lane < 32) {
        const float * l = &red[0][r];
        const float s0 = l[4 * 32] + l[0], s1 = l[5 * 32] + l[1 * 32];
        const float s2 = l[6 * 32] + l[2 * 32], s3 = l[7 * 32] + l[3 * 32];
        float v = (s0 + s2) + (s1 + s3);
        if (A.dn_bias) v = v + bias_v;
        if (!slot_ok) v = __builtin_nanf("");      // expert not resident in this bank: loud output
        coherent_store(A.y + static_cast<size_t>(rank) * S.rows + row, v);
    }
    wait_stores();
    uint32_t old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(A.counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __shfl(old, 0);
    const uint32_t K = static_cast<uint32_t>(A.top_k);
    if (old % K != K - 1) return;
    // last arriver: every rank's rows of this tile are stored; combine in rank order
    constexpr int kBatch = 8;
    float x = 0.0f;
    for (int j0 = 0; j0 < A.top_k; j0 += kBatch) {
        float yv[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j)
            yv[j] = lane < 32 && j0 + j < A.top_k ? coherent_load(A.y + static_cast<size_t>(j0 + j) * S.rows + row) : 0.0f;
#pragma unroll
        for (int j = 0; j < kBatch; ++j)
            if (j0 + j < A.top_k) {
                const float term = yv[j] * A.dn_w[j0 + j];
                x = j0 + j == 0 ? term : x + term;
            }
    }
    if (A.out) {
        if (lane < 32) A.out[row] = x;
    } else {
        publish_block(x, tile, A, coherent_load(A.epoch));
    }
}

// Gate_up tile (rank, tile) of layer l: as kernel A, with the whole tile preloaded and the input
// taken from the published row (or quantized from x_in in the first launch) by the helper wave.
template <int TYPE, int NPL, int NB, bool FIRST>
__device__ __forceinline__ void link_gate_up(const LinkArgs & A, int wg, uint8_t * lds_dyn, float (&red)[8][32]) {
    constexpr int G = link_ring_depth(NB);
    const Shape S = A.gu_shape;
    const int tiles = S.rows / 32;
    const int rank = wg / tiles, tile = wg - rank * tiles;
    const int mbytes = meta_tile_bytes<TYPE>(NB);
    uint8_t * lmeta = lds_dyn;
    uint8_t * act = lmeta + mbytes;
    float * lscale = reinterpret_cast<float *>(act + ((A.gu_lay.flag_offset() + 15) & ~15ll));
    const int tid = threadIdx.x, lane = tid & 63, r = lane & 31;
    const bool compute = tid < kDownThreads;                // waves 0..3; wave 4 is the helper
    const int k = (tid >> 6) * 2 + (lane >> 5);
    const int n = A.n_expert;
    float sel_v = 0.0f;
    int sel_i = -1;
    bool slot_ok = false;
    float bias_v = 0.0f;
    Group ring[G];
    Tail tl;
    const uint8_t * codes_tile = A.gu_bank;
    if (compute) {
        // routing keys and slots of experts lane + 64 i (unconditional, clamped loads), this
        // wave's top-k, then the pick's whole weight tile
        float lg[NPL];
        int sl[NPL];
        const int32_t * map = A.expert_to_slot;
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            const int c = lane + 64 * i;
            lg[i] = A.logits[c < n ? c : 0];
        }
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            const int c = lane + 64 * i;
            sl[i] = map ? map[c < n ? c : 0] : c;
        }
#pragma unroll
        for (int i = 0; i < NPL; ++i) lg[i] = route_key(lg[i]);
        wave_topk_regs<NPL>(lg, n, A.top_k, sel_v, sel_i);
        const int expert = __builtin_amdgcn_readlane(sel_i, rank);
        int sv = sl[0];
#pragma unroll
        for (int i = 1; i < NPL; ++i)
            if ((expert >> 6) == i) sv = sl[i];
        const int slot = __builtin_amdgcn_readlane(sv, expert & 63);
        slot_ok = slot >= 0 && slot < S.n_slots;
        const uint8_t * slot_base = A.gu_bank + (slot_ok ? static_cast<size_t>(slot) * S.slot_bytes : 0);
        codes_tile = slot_base + static_cast<size_t>(tile) * 32 * NB * 16;
        u32x4 mst[2];
        load_meta<kDownThreads>(mst, slot_base + S.codes_bytes + static_cast<size_t>(tile) * mbytes, mbytes);
        preload_ring<TYPE, G, true>(ring, codes_tile, nullptr, k, r, NB, true);
        preload_tail<TYPE, true>(tl, codes_tile, nullptr, k, r, NB, true);
        const int grow = static_cast<int>(ggml_row(static_cast<int64_t>(tile) * 32 + r, S.rows, S.interleave));
        if (k == 0 && A.gu_bias) bias_v = A.gu_bias[static_cast<size_t>(expert) * S.rows + grow];
        store_meta<kDownThreads>(mst, lmeta, mbytes);
    } else {
        if (FIRST) helper_quantize_row<TYPE, NB>(A.x_in, act, A.gu_lay);
        else helper_fetch_row<NB>(A, coherent_load(A.epoch), act);
    }
    __syncthreads();
    build_scales<TYPE, kLinkThreads, 1>(lscale, lmeta, reinterpret_cast<const float *>(act + A.gu_lay.da_offset()), NB, mbytes);
    __syncthreads();
    if (compute) {
        float acc[2] = {0.0f, 0.0f};
        decode_stream<TYPE, G, NB>(ring, tl, codes_tile, k, r, NB, false,
                                   act + static_cast<int64_t>(k) * NB * A.gu_lay.code_entry(), lscale + r * 4, acc);
        red[k][r] = acc[0] + acc[1];
    }
    __syncthreads();
    if (tid < 32) {
        const float * l = &red[0][r];
        const float s0 = l[4 * 32] + l[0], s1 = l[5 * 32] + l[1 * 32];
        const float s2 = l[6 * 32] + l[2 * 32], s3 = l[7 * 32] + l[3 * 32];
        float v = (s0 + s2) + (s1 + s3);
        if (A.gu_bias) v = v + bias_v;
        red[0][r] = v;                              // rows r: 0..15 gate, 16..31 up
    }
    __syncthreads();
    if (tid < 16) {
        float g = glu(A.activation, red[0][tid], red[0][tid + 16], A.alpha, A.limit);
        if (!slot_ok) g = __builtin_nanf("");      // expert not resident in this bank: loud output
        A.act_f[static_cast<size_t>(rank) * (S.rows / 2) + tile * 16 + tid] = g;
    }
    if (tid < 64 && tile == 0 && rank == 0) {
        const float w = wave_pick_softmax(sel_v, A.top_k);
        if (lane < A.top_k) {
            A.route_ids[lane] = sel_i;
            A.route_w[lane] = w;
            A.route_slots[lane] = A.expert_to_slot ? A.expert_to_slot[sel_i] : sel_i;
        }
    }
}

template <int TYPE, int NPL, int NB, bool FIRST>
__global__ __launch_bounds__(kLinkThreads) void decode_link_kernel(LinkArgs A) {
    __shared__ float red[8][32];
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_dyn[];
    const int wg = blockIdx.x;
    if (!FIRST && wg < A.n_down) {
        link_down<TYPE, NB>(A, wg, lds_dyn, red);
        if (A.advance_epoch && wg == 0 && threadIdx.x == 0) *A.epoch = *A.epoch + 1u;
    } else {
        link_gate_up<TYPE, NPL, NB, FIRST>(A, FIRST ? wg : wg - A.n_down, lds_dyn, red);
    }
}

template <int TYPE, int NPL, int NB>
void launch_gate_up_npl(const DecodeArgs & a, dim3 grid, size_t lds, hipStream_t stream) {
    auto launch = [&](auto kernel) {
        if (lds > 65536)
            check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                          static_cast<int>(lds)), "decode gate_up LDS attribute");
        hipLaunchKernelGGL(kernel, grid, dim3(kDownThreads), lds, stream, a);
    };
    if (a.stage) launch(&decode_gate_up_kernel<TYPE, NPL, NB, true>);
    else launch(&decode_gate_up_kernel<TYPE, NPL, NB, false>);
}

// Row lengths (blocks) with a fully unrolled weight stream: hidden = intermediate = 2880 (MXFP4,
// 90 blocks) and the Q8_0 layer with hidden 2048 (64 blocks) and intermediate 768 (24 blocks).
template <int TYPE>
constexpr int fixed_gate_up_nb() {
    return TYPE == 39 ? 90 : 64;
}
template <int TYPE>
constexpr int fixed_down_nb() {
    return TYPE == 39 ? 90 : 24;
}

template <int TYPE>
void launch_decode_typed(const DecodeArgs & a, hipStream_t stream) {
    const size_t lds = decode_lds_bytes<TYPE>(a.shape.nb);
    const dim3 grid(static_cast<unsigned>(a.shape.rows / 32), static_cast<unsigned>(a.top_k));
    constexpr int kFixed = fixed_gate_up_nb<TYPE>();
    if (a.n_expert <= 128 && a.shape.nb == kFixed) launch_gate_up_npl<TYPE, 2, kFixed>(a, grid, lds, stream);
    else if (a.n_expert <= 128) launch_gate_up_npl<TYPE, 2, 0>(a, grid, lds, stream);
    else if (a.n_expert <= 256) launch_gate_up_npl<TYPE, 4, 0>(a, grid, lds, stream);
    else launch_gate_up_npl<TYPE, 16, 0>(a, grid, lds, stream);
    check_hip(hipGetLastError(), "decode gate_up launch");
}

template <int TYPE>
void launch_decode_down_typed(const DecodeDownArgs & a, int top_k, hipStream_t stream) {
    const size_t lds = decode_lds_bytes<TYPE>(a.shape.nb);
    const dim3 grid(static_cast<unsigned>(a.shape.rows / 32), static_cast<unsigned>(top_k));
    constexpr int kFixed = fixed_down_nb<TYPE>();
    const bool fixed = a.shape.nb == kFixed;
    if (a.stage) {
        if (fixed) hipLaunchKernelGGL((decode_down_kernel<TYPE, kFixed, true>), grid, dim3(kDownThreads), lds, stream, a);
        else hipLaunchKernelGGL((decode_down_kernel<TYPE, 0, true>), grid, dim3(kDownThreads), lds, stream, a);
    } else {
        if (fixed) hipLaunchKernelGGL((decode_down_kernel<TYPE, kFixed, false>), grid, dim3(kDownThreads), lds, stream, a);
        else hipLaunchKernelGGL((decode_down_kernel<TYPE, 0, false>), grid, dim3(kDownThreads), lds, stream, a);
    }
    check_hip(hipGetLastError(), "decode down launch");
}

// ------------------------------------------------------------------------------ activation rows
// One 32-lane group per (row, block): x86 quantize_row_q8_0 into xrows (quantize_expand_block).
__global__ __launch_bounds__(256) void quantize_expand_kernel(const float * __restrict__ x, int64_t n_rows, int nb,
                                                              int64_t x_stride, XrowLayout L, uint8_t * __restrict__ xrows,
                                                              uint8_t * __restrict__ q8) {
    quantize_expand_block(x, n_rows, nb, x_stride, L, xrows, q8, blockIdx.x * 8ll + (threadIdx.x >> 5),
                          static_cast<int>(threadIdx.x & 31));
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

template <int TYPE, int MT, bool NEG>
void launch_typed(const GemvArgs & g, KernelArgs ka, hipStream_t stream) {
    const int64_t max_items = gemv_max_chunks(g.max_active, g.n_entries, MT);
    require(max_items <= g.group.chunk_list_items, "chunk list exceeds its workspace");
    // the kernel hands each XCD ceil(items / 8) consecutive items: the grid is a multiple of 8
    const int64_t blocks = (static_cast<int64_t>(ka.pairs) * max_items + 7) / 8 * 8;
    require(blocks > 0 && blocks < (1ll << 31), "expert GEMV grid out of range");
    ka.chunk_expert = g.group.chunk_list;
    ka.chunk_start = g.group.chunk_list + max_items;
    ka.n_chunks = g.group.chunk_list + 2 * max_items;
    if (!g.chunks_built)
        launch_job_tiles(g.group, nullptr, MT, max_items, g.group.chunk_list, g.group.chunk_list + max_items,
                         g.group.chunk_list + 2 * max_items, stream);
    const size_t tok_bytes = (static_cast<size_t>(ka.lay.flag_offset()) + 15) & ~static_cast<size_t>(15);
    const size_t lds = std::max<size_t>(MT * tok_bytes, static_cast<size_t>(MT) * 8 * 64 * sizeof(float));
    hipLaunchKernelGGL((expert_gemv_kernel<TYPE, MT, NEG>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), lds, stream,
                       ka);
    check_hip(hipGetLastError(), "expert GEMV launch");
}

template <int TYPE, bool NEG>
void launch_mt(const GemvArgs & g, const KernelArgs & ka, hipStream_t stream) {
    switch (gemv_chunk_tokens(g.max_per_expert)) {
        case 1: launch_typed<TYPE, 1, NEG>(g, ka, stream); break;
        case 2: launch_typed<TYPE, 2, NEG>(g, ka, stream); break;
        case 4: launch_typed<TYPE, 4, NEG>(g, ka, stream); break;
        default: launch_typed<TYPE, 8, NEG>(g, ka, stream); break;
    }
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
    ka.pairs = static_cast<int>((bank.rows + 63) / 64);
    ka.bias = g.bias;
    ka.dst = g.dst;
    ka.dst_xrows = g.dst_xrows;
    ka.dst_lay = g.dst_layout;
    ka.epilogue = g.epilogue;
    ka.activation = g.activation;
    ka.alpha = g.alpha;
    ka.limit = g.limit;
    if (bank.type == VBM_TYPE_MXFP4) {
        if (g.may_have_neg128) launch_mt<39, true>(g, ka, stream);
        else launch_mt<39, false>(g, ka, stream);
    } else {
        if (g.may_have_neg128) launch_mt<8, true>(g, ka, stream);
        else launch_mt<8, false>(g, ka, stream);
    }
}

void launch_decode_gate_up(const DecodeGateUpArgs & d, hipStream_t stream) {
    const vbm_bank & bank = *d.bank;
    require(bank.interleave && bank.rows % 64 == 0, "decode gate_up needs an interleaved bank with rows % 64 == 0");
    require(d.top_k >= 1 && d.top_k <= 64 && d.n_expert >= d.top_k && d.n_expert <= kMaxRouteExperts,
            "routing shape out of range");
    require(d.hidden == bank.k && d.hidden <= 4096, "hidden size mismatch");
    require(d.x_in != nullptr || (d.prev_y != nullptr && d.prev_w != nullptr), "decode layer input missing");
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
    a.bias = d.bias;
    a.act_f = d.act_f;
    a.route_ids = d.route_ids;
    a.route_w = d.route_w;
    a.route_slots = d.route_slots;
    a.activation = d.activation;
    a.alpha = d.alpha;
    a.limit = d.limit;
    require(d.host_base == nullptr || d.host_stride >= static_cast<int64_t>(bank.slot_bytes), "host copy stride too small");
    a.host_base = d.host_base;
    a.host_stride = d.host_stride;
    require(d.stage == nullptr || (d.host_base != nullptr && d.stage_stride >= static_cast<int64_t>(bank.slot_bytes) &&
                                   reinterpret_cast<uintptr_t>(d.stage) % 16 == 0 && d.stage_stride % 16 == 0),
            "staging area needs a host copy, 16-byte alignment and a stride of at least a slot");
    a.stage = d.stage;
    a.stage_stride = d.stage_stride;
    if (bank.type == VBM_TYPE_MXFP4) launch_decode_typed<39>(a, stream);
    else launch_decode_typed<8>(a, stream);
}

bool decode_link_supported(const vbm_bank & gate_up, const vbm_bank & down, int64_t n_expert, int64_t top_k) {
    return gate_up.type == VBM_TYPE_MXFP4 && down.type == VBM_TYPE_MXFP4 && gate_up.nb == 90 && down.nb == 90 &&
           gate_up.interleave && gate_up.rows == 2 * 2880 && down.rows == 2880 && n_expert >= top_k &&
           n_expert <= 128 && top_k >= 1 && top_k <= 64;
}

void launch_decode_link(const DecodeLinkParams & d, hipStream_t stream) {
    static_assert(kLinkFlagWords == int64_t{kLinkCopies} * kLinkCopyStride, "flag region size");
    require(d.dn_bank != nullptr || d.gu_bank != nullptr, "linked decode launch without work");
    const vbm_bank * gu = d.gu_bank;
    const vbm_bank * dn = d.dn_bank;
    if (gu && dn) require(decode_link_supported(*gu, *dn, d.n_expert, d.top_k), "linked decode shape not supported");
    if (gu) require(gu->type == VBM_TYPE_MXFP4 && gu->nb == 90 && gu->interleave && gu->rows == 5760 && d.n_expert <= 128,
                    "linked decode gate_up shape not supported");
    if (dn) require(dn->type == VBM_TYPE_MXFP4 && dn->nb == 90 && dn->rows == 2880, "linked decode down shape not supported");
    require(d.top_k >= 1 && d.top_k <= 64 && d.n_expert >= d.top_k, "routing shape out of range");
    require(dn == nullptr || (d.out != nullptr) != (d.xq != nullptr && d.flags != nullptr),
            "a down part publishes either the next input row or the output");
    require(gu == nullptr || d.x_in != nullptr || (d.xq != nullptr && d.flags != nullptr), "gate_up input missing");
    require(!(gu && dn && d.x_in), "the first launch has no down part");
    require(d.epoch != nullptr && d.error != nullptr, "linked decode state missing");
    LinkArgs a{};
    a.n_expert = static_cast<int>(d.n_expert);
    a.top_k = static_cast<int>(d.top_k);
    if (dn) {
        a.n_down = static_cast<int>(d.top_k * (dn->rows / 32));
        a.dn_bank = dn->base;
        a.dn_shape = Shape{static_cast<int>(dn->nb), static_cast<int>(dn->rows), dn->interleave, dn->slot_bytes,
                           dn->geometry().codes_bytes(), dn->n_slots};
        a.dn_lay = XrowLayout{dn->nb, dn->type};
        a.dn_act_f = d.dn_act_f;
        a.dn_ids = d.dn_ids;
        a.dn_slots = d.dn_slots;
        a.dn_w = d.dn_w;
        a.dn_bias = d.dn_bias;
        a.y = d.y;
        a.counters = d.counters;
        a.out = d.out;
    }
    a.xq = d.xq;
    a.flags = d.flags;
    if (gu) {
        a.n_gate_up = static_cast<int>(d.top_k * (gu->rows / 32));
        a.gu_bank = gu->base;
        a.gu_shape = Shape{static_cast<int>(gu->nb), static_cast<int>(gu->rows), gu->interleave, gu->slot_bytes,
                           gu->geometry().codes_bytes(), gu->n_slots};
        a.gu_lay = XrowLayout{gu->nb, gu->type};
        a.expert_to_slot = d.expert_to_slot;
        a.logits = d.logits;
        a.x_in = d.x_in;
        a.gu_bias = d.gu_bias;
        a.act_f = d.act_f;
        a.route_ids = d.route_ids;
        a.route_w = d.route_w;
        a.route_slots = d.route_slots;
        a.activation = d.activation;
        a.alpha = d.alpha;
        a.limit = d.limit;
    } else {
        a.gu_lay = XrowLayout{dn->rows / 32, VBM_TYPE_MXFP4};
    }
    a.epoch = d.epoch;
    a.advance_epoch = d.advance_epoch ? 1 : 0;
    a.error = d.error;
    const size_t lds = decode_lds_bytes<39>(90);
    const dim3 grid(static_cast<unsigned>(a.n_down + a.n_gate_up));
    if (d.x_in) hipLaunchKernelGGL((decode_link_kernel<39, 2, 90, true>), grid, dim3(kLinkThreads), lds, stream, a);
    else hipLaunchKernelGGL((decode_link_kernel<39, 2, 90, false>), grid, dim3(kLinkThreads), lds, stream, a);
    check_hip(hipGetLastError(), "linked decode launch");
}

void launch_decode_down(const DecodeDownParams & d, hipStream_t stream) {
    const vbm_bank & bank = *d.bank;
    require(d.top_k >= 1 && d.top_k <= 64, "top_k out of range");
    require(bank.nb <= 128 && d.act_layout.nb == bank.nb && d.act_layout.weight_type == bank.type,
            "down activation layout does not match the down bank");
    DecodeDownArgs a{};
    a.bank = bank.base;
    a.shape = Shape{static_cast<int>(bank.nb), static_cast<int>(bank.rows), bank.interleave, bank.slot_bytes,
                    bank.geometry().codes_bytes(), bank.n_slots};
    a.expert_to_slot = d.expert_to_slot;
    a.lay = d.act_layout;
    a.act_f = d.act_f;
    a.route_ids = d.route_ids;
    a.route_slots = d.route_slots;
    a.bias = d.bias;
    a.y = d.y;
    require(d.host_base == nullptr || d.host_stride >= static_cast<int64_t>(bank.slot_bytes), "host copy stride too small");
    a.host_base = d.host_base;
    a.host_stride = d.host_stride;
    require(d.stage == nullptr || (d.host_base != nullptr && d.stage_stride >= static_cast<int64_t>(bank.slot_bytes) &&
                                   reinterpret_cast<uintptr_t>(d.stage) % 16 == 0 && d.stage_stride % 16 == 0),
            "staging area needs a host copy, 16-byte alignment and a stride of at least a slot");
    a.stage = d.stage;
    a.stage_stride = d.stage_stride;
    if (bank.type == VBM_TYPE_MXFP4) launch_decode_down_typed<39>(a, static_cast<int>(d.top_k), stream);
    else launch_decode_down_typed<8>(a, static_cast<int>(d.top_k), stream);
}

}  // namespace vbm
