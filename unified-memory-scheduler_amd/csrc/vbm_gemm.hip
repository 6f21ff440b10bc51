// Grouped expert GEMM on CDNA4 MFMA for prefill-sized token groups (the fast-order path).
//
// Each 32-element block's integer dot is computed exactly by the matrix cores:
//   - MXFP4 weights: v_cvt_scalef32_pk_f16_fp4 (scale 2) gives the doubled-e2m1 integers as f16,
//     activations are the int8 Q8_0 codes as f16, and v_mfma_f32_16x16x32_f16 sums the 32
//     products of one block; every partial sum is an integer below 2^24, so the block dot is
//     exact in fp32 whatever the order inside the matrix core.
//   - Q8_0 weights: v_mfma_i32_16x16x32_i8 on the int8 codes (exact int32).
// The block dot is then scaled (MXFP4: ldexp(d_act, e - 128); Q8_0: fp16(d_w) * d_act, the
// CPU's own products) and accumulated in fp32 block after block. That accumulation order is not
// the CPU's 8-lane chains, so outputs agree with the reference within fp32 rounding (the
// tolerance-checked order), while every integer block dot is bit-exact. The x86 VPSIGNB corner
// (activation code -128 against a negative weight) is applied as an exact correction on rows
// flagged by their quantizer.
//
// MFMA 16x16x32 lane layouts (checked on the device): A: lane l holds row l%16, k = 8(l/16)..+7;
// B: k = 8(l/16)..+7 of column l%16; D: rows 4(l/16)..+3 of column l%16. The bank's slice layout
// puts slices 2q and 2q+1 of a block (elements 8q..8q+7) in two 16-byte group entries, which is
// exactly lane group q's k range, so weights go from HBM to the matrix core without reshuffling.
//
// A workgroup (4 waves) computes 64 bank rows (a tile pair) x 64 jobs of one expert; wave w owns
// bank tile 2p + (w & 1) and jobs 32(w >> 1)..+31 as a 2x2 grid of 16x16 fragments.
#include "vbm_device.hpp"
#include "vbm_internal.hpp"

namespace vbm {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_g __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4g __attribute__((ext_vector_type(4)));
typedef unsigned u32x2g __attribute__((ext_vector_type(2)));

constexpr int kGemmThreads = 256;
constexpr int kJobTile = 64;

template <class T>
__device__ __forceinline__ const __attribute__((address_space(4))) T * cst(const void * p) {
    return (const __attribute__((address_space(4))) T *)(p);
}

struct GemmShape {
    int nb, rows, interleave;
    size_t slot_bytes;
    int64_t codes_bytes, n_slots;
};

struct GemmArgs {
    const uint8_t * bank;
    GemmShape shape;
    const int32_t * expert_to_slot;
    const uint8_t * rows_in;   // activation rows (GemmRowLayout lay)
    GemmRowLayout lay;
    int64_t n_ids, b_ne1;
    const int32_t * counts;
    const int32_t * offsets;
    const int32_t * jobs;      // grouped job list (token * n_ids + rank)
    const int32_t * tile_expert;
    const int32_t * tile_start;
    const int32_t * n_tiles;
    const float * bias;        // [n_expert][rows] in ggml row order, or null
    float * dst;               // epilogue 0: [job][rows]
    uint8_t * rows_out;        // epilogue 1: GLU output rows for the down projection (out_lay)
    GemmRowLayout out_lay;
    int activation;
    float alpha, limit;
};

__device__ __forceinline__ half2_g fp4x2(unsigned dw, int sel) {
    // sel is a compile-time constant at every call site after unrolling
    switch (sel) {
        case 0: return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, 0);
        case 1: return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, 1);
        case 2: return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, 2);
        default: return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, 2.0f, 3);
    }
}

// Weight operand of block b (index within its group, compile-time) from the two slice entries
// of the group: MXFP4 bytes 2b, 2b+1 of each 16-byte entry hold the slice's 4 nibbles.
template <int B>
__device__ __forceinline__ half8_t mx_a_operand(const u32x4g & s0, const u32x4g & s1) {
    const unsigned w0 = s0[B / 2], w1 = s1[B / 2];
    constexpr int sel = (B & 1) * 2;
    const half2_g p0 = fp4x2(w0, sel), p1 = fp4x2(w0, sel + 1), p2 = fp4x2(w1, sel), p3 = fp4x2(w1, sel + 1);
    return half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// Exact VPSIGNB correction of one fragment column: contract minus true product is 256 * w for
// every element whose activation code is -128 and whose weight is negative. Computed with the
// same MFMA on (min(w, 0), [a == -128]) operands; only for flagged rows.
__device__ __forceinline__ half8_t neg_part(half8_t w) {
    half8_t r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = w[i] < static_cast<_Float16>(0.0f) ? w[i] : static_cast<_Float16>(0.0f);
    return r;
}
__device__ __forceinline__ half8_t is_neg128(half8_t a) {
    half8_t r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = a[i] == static_cast<_Float16>(-128.0f) ? static_cast<_Float16>(1.0f) : static_cast<_Float16>(0.0f);
    return r;
}
__device__ __forceinline__ long neg_part_i8(long w) {
    long r = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const signed char v = static_cast<signed char>(w >> (8 * i));
        r |= static_cast<long>(static_cast<uint8_t>(v < 0 ? v : 0)) << (8 * i);
    }
    return r;
}
__device__ __forceinline__ long is_neg128_i8(long a) {
    long r = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        r |= static_cast<long>(static_cast<signed char>(a >> (8 * i)) == -128 ? 1 : 0) << (8 * i);
    return r;
}

template <int TYPE, int EPI>
__global__ __launch_bounds__(kGemmThreads) void grouped_gemm_kernel(GemmArgs A) {
    __shared__ float tile_vals[kJobTile][64 + 1];   // epilogue 1: [job][bank row of the pair]
    const int ti = blockIdx.y;
    if (ti >= *cst<int32_t>(A.n_tiles)) return;
    const int expert = cst<int32_t>(A.tile_expert)[ti];
    const int j0 = cst<int32_t>(A.tile_start)[ti];
    const int count = cst<int32_t>(A.counts)[expert];
    const int joff = cst<int32_t>(A.offsets)[expert];
    const int slot = A.expert_to_slot ? cst<int32_t>(A.expert_to_slot)[expert] : expert;
    const GemmShape S = A.shape;
    if (slot < 0 || slot >= S.n_slots) return;

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int lr = lane & 15, q = lane >> 4;
    const int pair = blockIdx.x;
    const int tile = pair * 2 + (wave & 1);
    const bool tile_live = tile * 32 < S.rows;
    const int nb = S.nb;
    constexpr int kGroupBlocks = TYPE == 39 ? 8 : 4;
    const int groups = nb / kGroupBlocks, tail = nb % kGroupBlocks;
    const uint8_t * slot_base = A.bank + static_cast<size_t>(slot) * S.slot_bytes;
    const uint8_t * codes = slot_base + static_cast<size_t>(tile_live ? tile : 0) * 32 * nb * (TYPE == 39 ? 16 : 32);
    const uint8_t * meta = slot_base + S.codes_bytes + static_cast<size_t>(tile_live ? tile : 0) * 32 * nb * (TYPE == 39 ? 1 : 2);

    // The two job columns of this lane (fragment column lr of job halves 0 and 1).
    const uint8_t * brow[2];
    bool jlive[2];
    int job[2];
    int flagged = 0;
#pragma unroll
    for (int jh = 0; jh < 2; ++jh) {
        const int jj = j0 + 32 * (wave >> 1) + 16 * jh + lr;
        jlive[jh] = jj < count;
        job[jh] = jlive[jh] ? A.jobs[joff + jj] : 0;
        const int64_t row_index = A.b_ne1 == 1 ? job[jh] / A.n_ids : job[jh];
        brow[jh] = A.rows_in + row_index * A.lay.stride();
        if (jlive[jh]) flagged |= *reinterpret_cast<const int *>(brow[jh] + A.lay.flag_offset());
    }
    const bool slow = __any(flagged != 0);   // wave-uniform: any flagged activation row in the wave

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jh = 0; jh < 2; ++jh) acc[i][jh] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Output rows of this lane's fragments: in-tile rows 16i + 4q + j.
    auto block_step = [&](int b, const auto & a_op, const u32x2g (&m)[2][4], int mb) {
        // b: block index; a_op[i]: weight operand of row half i; m[i][j]: meta word pair of output
        // row 16i + 4q + j; mb: position of block b inside the meta words.
#pragma unroll
        for (int jh = 0; jh < 2; ++jh) {
            float da = 0.0f;
            if constexpr (TYPE == 39) {
                half8_t bv = half8_t{};
                if (jlive[jh]) bv = *reinterpret_cast<const half8_t *>(brow[jh] + (static_cast<int64_t>(b) * 32 + 8 * q) * 2);
                if (jlive[jh]) da = reinterpret_cast<const float *>(brow[jh] + A.lay.da_offset())[b];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_op[i], bv, f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                    if (slow) {
                        const f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(neg_part(a_op[i]), is_neg128(bv),
                                                                               f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                        d = d + c * 256.0f;
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const unsigned w = m[i][j][mb >> 2];
                        const int e = static_cast<signed char>(w >> ((mb & 3) * 8));
                        const float s = __builtin_amdgcn_ldexpf(da, e);
                        acc[i][jh][j] = __builtin_fmaf(s, d[j], acc[i][jh][j]);
                    }
                }
            } else {
                long bv = 0;
                if (jlive[jh]) bv = *reinterpret_cast<const long *>(brow[jh] + static_cast<int64_t>(b) * 32 + 8 * q);
                if (jlive[jh]) da = reinterpret_cast<const float *>(brow[jh] + A.lay.da_offset())[b];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    i32x4 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_op[i], bv, i32x4{0, 0, 0, 0}, 0, 0, 0);
                    if (slow) {
                        const i32x4 c = __builtin_amdgcn_mfma_i32_16x16x32_i8(neg_part_i8(a_op[i]), is_neg128_i8(bv),
                                                                              i32x4{0, 0, 0, 0}, 0, 0, 0);
                        d = d + c * 256;
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const unsigned w = m[i][j][mb >> 1];
                        const float dw = half_bits_to_float(static_cast<uint16_t>(w >> ((mb & 1) * 16)));
                        const float s = dw * da;
                        acc[i][jh][j] = __builtin_fmaf(s, static_cast<float>(d[j]), acc[i][jh][j]);
                    }
                }
            }
        }
    };

    for (int g = 0; g < groups; ++g) {
        // weight entries of slices 2q, 2q+1 for in-tile rows lr and 16 + lr
        u32x4g s0[2], s1[2];
        u32x2g m[2][4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int r = 16 * i + lr;
            s0[i] = u32x4g{0u, 0u, 0u, 0u};
            s1[i] = u32x4g{0u, 0u, 0u, 0u};
            if (tile_live) {
                s0[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4g *>(codes + g * 4096 + ((2 * q) * 32 + r) * 16));
                s1[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4g *>(codes + g * 4096 + ((2 * q + 1) * 32 + r) * 16));
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int orow = 16 * i + 4 * q + j;
                m[i][j] = tile_live ? *reinterpret_cast<const u32x2g *>(meta + g * 256 + orow * 8) : u32x2g{0u, 0u};
            }
        }
        if constexpr (TYPE == 39) {
            half8_t a[2];
#define VBM_MX_STEP(BB)                                                       \
            a[0] = mx_a_operand<BB>(s0[0], s1[0]);                            \
            a[1] = mx_a_operand<BB>(s0[1], s1[1]);                            \
            block_step(g * 8 + BB, a, m, BB);
            VBM_MX_STEP(0) VBM_MX_STEP(1) VBM_MX_STEP(2) VBM_MX_STEP(3)
            VBM_MX_STEP(4) VBM_MX_STEP(5) VBM_MX_STEP(6) VBM_MX_STEP(7)
#undef VBM_MX_STEP
        } else {
            long a[2];
#pragma unroll
            for (int bb = 0; bb < 4; ++bb) {
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    a[i] = static_cast<long>(static_cast<uint64_t>(s0[i][bb]) | (static_cast<uint64_t>(s1[i][bb]) << 32));
                block_step(g * 4 + bb, a, m, bb);
            }
        }
    }
    // Tail blocks (nb even: MXFP4 tail in {0,2,4,6}, Q8_0 tail in {0,2}), per-row packed.
    for (int bt = 0; bt < tail; ++bt) {
        const int b = groups * kGroupBlocks + bt;
        u32x2g m[2][4];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int orow = 16 * i + 4 * q + j;
                unsigned w = 0;
                if (tile_live) {
                    if constexpr (TYPE == 39) w = meta[groups * 256 + orow * tail + bt];
                    else w = *reinterpret_cast<const uint16_t *>(meta + groups * 256 + (orow * tail + bt) * 2);
                }
                m[i][j] = u32x2g{w, 0u};
            }
        if constexpr (TYPE == 39) {
            half8_t a[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = 16 * i + lr;
                unsigned w0 = 0, w1 = 0;
                if (tile_live) {
                    w0 = *reinterpret_cast<const uint16_t *>(codes + groups * 4096 + ((2 * q) * 32 + r) * (tail * 2) + bt * 2);
                    w1 = *reinterpret_cast<const uint16_t *>(codes + groups * 4096 + ((2 * q + 1) * 32 + r) * (tail * 2) + bt * 2);
                }
                const half2_g p0 = fp4x2(w0, 0), p1 = fp4x2(w0, 1), p2 = fp4x2(w1, 0), p3 = fp4x2(w1, 1);
                a[i] = half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
            }
            block_step(b, a, m, 0);
        } else {
            long a[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = 16 * i + lr;
                uint64_t w0 = 0, w1 = 0;
                if (tile_live) {
                    w0 = *reinterpret_cast<const unsigned *>(codes + groups * 4096 + ((2 * q) * 32 + r) * (tail * 4) + bt * 4);
                    w1 = *reinterpret_cast<const unsigned *>(codes + groups * 4096 + ((2 * q + 1) * 32 + r) * (tail * 4) + bt * 4);
                }
                a[i] = static_cast<long>(w0 | (w1 << 32));
            }
            block_step(b, a, m, 0);
        }
    }

    // Epilogue: biases (ggml row order), then either fp32 rows or GLU + Q8_0 requantization.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int orow = 16 * i + 4 * q + j;
            const int grow = static_cast<int>(ggml_row(static_cast<int64_t>(tile) * 32 + orow, S.rows, S.interleave));
            const float bv = (A.bias && tile_live) ? A.bias[static_cast<size_t>(expert) * S.rows + grow] : 0.0f;
#pragma unroll
            for (int jh = 0; jh < 2; ++jh) {
                float v = acc[i][jh][j];
                if (A.bias) v = v + bv;
                if (EPI == 0) {
                    if (jlive[jh] && tile_live) A.dst[static_cast<size_t>(job[jh]) * S.rows + grow] = v;
                } else {
                    tile_vals[32 * (wave >> 1) + 16 * jh + lr][32 * (wave & 1) + orow] = v;
                }
            }
        }
    }
    if (EPI == 1) {
        __syncthreads();
        // one 32-element GLU block per job: four threads per job, eight elements each
        const int jl = threadIdx.x >> 2, part = threadIdx.x & 3;
        const int jj = j0 + jl;
        const bool live = jj < count;
        float x[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int e = part * 8 + t;                 // element of the block
            const int tl = e >> 4;                      // bank tile of the pair
            const float g = tile_vals[jl][32 * tl + (e & 15)];
            const float u = tile_vals[jl][32 * tl + 16 + (e & 15)];
            x[t] = glu(A.activation, g, u, A.alpha, A.limit);
        }
        float amax = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; ++t) amax = fmaxf(amax, fabsf(x[t]));
        amax = quad_max(amax);
        if (live) {
            const float d = amax / 127.0f;
            const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
            const int jb = A.jobs[joff + jj];
            uint8_t * out = A.rows_out + static_cast<int64_t>(jb) * A.out_lay.stride();
            const int64_t e0 = static_cast<int64_t>(pair) * 32 + part * 8;
            if (A.out_lay.weight_type == 39) {
                half8_t c;
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    float v = rintf(x[t] * id);
                    v = v > 127.0f ? 127.0f : (v < -128.0f ? -128.0f : v);
                    c[t] = static_cast<_Float16>(v);
                }
                *reinterpret_cast<half8_t *>(out + e0 * 2) = c;
            } else {
                uint64_t c = 0;
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    float v = rintf(x[t] * id);
                    v = v > 127.0f ? 127.0f : (v < -128.0f ? -128.0f : v);
                    c |= static_cast<uint64_t>(static_cast<uint8_t>(static_cast<signed char>(v))) << (8 * t);
                }
                *reinterpret_cast<uint64_t *>(out + e0) = c;
            }
            if (part == 0) {
                reinterpret_cast<float *>(out + A.out_lay.da_offset())[pair] = static_cast<float>(static_cast<_Float16>(d));
                if (pair == 0) *reinterpret_cast<int *>(out + A.out_lay.flag_offset()) = 0;   // never -128
            }
        }
    }
}

// Tiles of kJobTile jobs per active expert, in active order: one workgroup, wave scans plus a
// scan of the 16 wave totals.
__global__ __launch_bounds__(1024) void gemm_tiles_kernel(const int32_t * counts, const int32_t * active,
                                                          const int32_t * n_active, int max_tiles, int32_t * tile_expert,
                                                          int32_t * tile_start, int32_t * n_tiles, int32_t * error) {
    __shared__ int s_wave[16];
    const int na = *n_active;
    const int a = threadIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int e = a < na ? active[a] : 0;
    const int nt = a < na ? (counts[e] + kJobTile - 1) / kJobTile : 0;
    int incl = nt;
    for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_up(incl, off);
        if (lane >= off) incl += v;
    }
    if (lane == 63) s_wave[wave] = incl;
    __syncthreads();
    int before = 0;
    for (int w = 0; w < wave; ++w) before += s_wave[w];
    const int base = before + incl - nt;
    for (int t = 0; t < nt; ++t) {
        if (base + t < max_tiles) {
            tile_expert[base + t] = e;
            tile_start[base + t] = t * kJobTile;
        } else {
            *error = 1;
        }
    }
    if (threadIdx.x == 1023) {
        const int total = before + incl;
        *n_tiles = total < max_tiles ? total : max_tiles;
    }
}

// x86 quantize_row_q8_0 of fp32 rows into GEMM activation rows (row-major codes as f16 or int8,
// fp16-rounded fp32 block scales, and a 0 flag: this quantizer never produces -128).
__global__ __launch_bounds__(256) void gemm_rows_from_f32_kernel(const float * __restrict__ x, int64_t n_rows, int nb,
                                                                 int64_t x_stride, GemmRowLayout L, uint8_t * __restrict__ out) {
    const int64_t total = n_rows * nb * 4;
    const int64_t t = blockIdx.x * 256ll + threadIdx.x;
    const bool live = t < total;
    const int64_t quad = live ? t / 4 : 0;
    const int part = static_cast<int>(t & 3);
    const int64_t row = quad / nb, b = quad % nb;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = live ? x[row * x_stride + b * 32 + part * 8 + i] : 0.0f;
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = quad_max(amax);
    if (!live) return;
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    uint8_t * o = out + row * L.stride();
    const int64_t e0 = b * 32 + part * 8;
    if (L.weight_type == 39) {
        half8_t c;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float q = rintf(v[i] * id);
            q = q > 127.0f ? 127.0f : (q < -128.0f ? -128.0f : q);
            c[i] = static_cast<_Float16>(q);
        }
        *reinterpret_cast<half8_t *>(o + e0 * 2) = c;
    } else {
        uint64_t c = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float q = rintf(v[i] * id);
            q = q > 127.0f ? 127.0f : (q < -128.0f ? -128.0f : q);
            c |= static_cast<uint64_t>(static_cast<uint8_t>(static_cast<signed char>(q))) << (8 * i);
        }
        *reinterpret_cast<uint64_t *>(o + e0) = c;
    }
    if (part == 0) {
        reinterpret_cast<float *>(o + L.da_offset())[b] = static_cast<float>(static_cast<_Float16>(d));
        if (b == 0) *reinterpret_cast<int *>(o + L.flag_offset()) = 0;
    }
}

// ggml Q8_0 block rows -> GEMM activation rows, with each row's -128 flag.
__global__ __launch_bounds__(256) void gemm_rows_from_q8_kernel(const uint8_t * __restrict__ q8, int nb, int64_t row_bytes,
                                                                GemmRowLayout L, uint8_t * __restrict__ out) {
    __shared__ int s_flag;
    const int64_t row = blockIdx.x;
    const uint8_t * src = q8 + row * row_bytes;
    uint8_t * o = out + row * L.stride();
    if (threadIdx.x == 0) s_flag = 0;
    __syncthreads();
    int neg = 0;
    for (int idx = threadIdx.x; idx < nb * 32; idx += 256) {
        const int b = idx >> 5, e = idx & 31;
        const signed char q = static_cast<signed char>(src[b * 34 + 2 + e]);
        neg |= q == -128;
        if (L.weight_type == 39) reinterpret_cast<_Float16 *>(o)[idx] = static_cast<_Float16>(q);
        else o[idx] = static_cast<uint8_t>(q);
    }
    for (int b = threadIdx.x; b < nb; b += 256)
        reinterpret_cast<float *>(o + L.da_offset())[b] =
            half_bits_to_float(static_cast<uint16_t>(src[b * 34] | (src[b * 34 + 1] << 8)));
    if (neg) atomicOr(&s_flag, 1);
    __syncthreads();
    if (threadIdx.x == 0) *reinterpret_cast<int *>(o + L.flag_offset()) = s_flag;
}

template <int TYPE, int EPI>
void launch_gemm_typed(const GemmArgs & a, int row_pairs, int max_tiles, hipStream_t stream) {
    hipLaunchKernelGGL((grouped_gemm_kernel<TYPE, EPI>), dim3(static_cast<unsigned>(row_pairs), static_cast<unsigned>(max_tiles)),
                       dim3(kGemmThreads), 0, stream, a);
    check_hip(hipGetLastError(), "grouped GEMM launch");
}

}  // namespace

int64_t gemm_max_tiles(int64_t n_as, int64_t n_entries) {
    return (n_entries + kJobTile - 1) / kJobTile + (n_as < n_entries ? n_as : n_entries);
}

size_t gemm_tiles_bytes(int64_t n_as, int64_t n_entries) {
    return static_cast<size_t>((2 * gemm_max_tiles(n_as, n_entries) + 8) * sizeof(int32_t));
}

void launch_gemm_rows_from_f32(const float * x, int64_t n_rows, int64_t k, int64_t x_stride, const GemmRowLayout & lay,
                               uint8_t * rows, hipStream_t stream) {
    require(k > 0 && k % 32 == 0 && n_rows > 0 && x_stride >= k && lay.nb == k / 32, "GEMM quantize shape mismatch");
    const int64_t threads = n_rows * (k / 32) * 4;
    hipLaunchKernelGGL(gemm_rows_from_f32_kernel, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0, stream,
                       x, n_rows, static_cast<int>(k / 32), x_stride, lay, rows);
    check_hip(hipGetLastError(), "GEMM quantize launch");
}

void launch_gemm_rows_from_q8(const uint8_t * q8, int64_t n_rows, int64_t row_bytes, const GemmRowLayout & lay,
                              uint8_t * rows, hipStream_t stream) {
    require(n_rows > 0 && n_rows < (1ll << 31) && row_bytes == lay.nb * 34, "GEMM expand shape mismatch");
    hipLaunchKernelGGL(gemm_rows_from_q8_kernel, dim3(static_cast<unsigned>(n_rows)), dim3(256), 0, stream, q8,
                       static_cast<int>(lay.nb), row_bytes, lay, rows);
    check_hip(hipGetLastError(), "GEMM expand launch");
}

void launch_grouped_gemm(const GemmParams & p, hipStream_t stream) {
    const vbm_bank & bank = *p.bank;
    require(bank.nb <= 4096 / 32 && p.lay.nb == bank.nb && p.lay.weight_type == bank.type,
            "GEMM activation layout does not match the bank");
    require(p.epilogue == 0 || (bank.interleave && bank.rows % 64 == 0 && p.rows_out && p.out_layout.nb == bank.rows / 64),
            "GLU epilogue needs an interleaved gate|up bank with rows % 64 == 0 and a matching output layout");
    require(p.epilogue == 1 || p.dst != nullptr, "missing GEMM output");
    require(p.n_as >= 1 && p.n_as <= 1024 && p.n_entries >= 1, "GEMM group shape out of range");
    const int64_t max_tiles = gemm_max_tiles(p.n_as, p.n_entries);
    require(max_tiles <= 65535, "too many GEMM tiles for one launch");
    int32_t * tile_expert = static_cast<int32_t *>(p.tiles);
    int32_t * tile_start = tile_expert + max_tiles;
    int32_t * n_tiles = tile_start + max_tiles;
    hipLaunchKernelGGL(gemm_tiles_kernel, dim3(1), dim3(1024), 0, stream, p.group.counts, p.group.active,
                       p.group.n_active, static_cast<int>(max_tiles), tile_expert, tile_start, n_tiles, p.group.error);
    check_hip(hipGetLastError(), "GEMM tile list launch");
    GemmArgs a{};
    a.bank = bank.base;
    a.shape = GemmShape{static_cast<int>(bank.nb), static_cast<int>(bank.rows), bank.interleave, bank.slot_bytes,
                        bank.geometry().codes_bytes(), bank.n_slots};
    a.expert_to_slot = p.expert_to_slot;
    a.rows_in = p.rows_in;
    a.lay = p.lay;
    a.n_ids = p.n_ids;
    a.b_ne1 = p.b_ne1;
    a.counts = p.group.counts;
    a.offsets = p.group.offsets;
    a.jobs = p.group.rows;
    a.tile_expert = tile_expert;
    a.tile_start = tile_start;
    a.n_tiles = n_tiles;
    a.bias = p.bias;
    a.dst = p.dst;
    a.rows_out = p.rows_out;
    a.out_lay = p.out_layout;
    a.activation = p.activation;
    a.alpha = p.alpha;
    a.limit = p.limit;
    const int row_pairs = static_cast<int>((bank.rows + 63) / 64);
    if (bank.type == VBM_TYPE_MXFP4) {
        if (p.epilogue == 0) launch_gemm_typed<39, 0>(a, row_pairs, static_cast<int>(max_tiles), stream);
        else launch_gemm_typed<39, 1>(a, row_pairs, static_cast<int>(max_tiles), stream);
    } else {
        if (p.epilogue == 0) launch_gemm_typed<8, 0>(a, row_pairs, static_cast<int>(max_tiles), stream);
        else launch_gemm_typed<8, 1>(a, row_pairs, static_cast<int>(max_tiles), stream);
    }
}

}  // namespace vbm
