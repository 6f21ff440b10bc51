// Grouped expert GEMM on CDNA4 MFMA for prefill-sized token groups (the fast-order path).
//
// Each 32-element block's integer dot is computed exactly by the matrix cores:
//   - MXFP4 weights: v_cvt_scalef32_pk_f16_fp4 (scale 2) gives the doubled-e2m1 integers as f16,
//     activations are the int8 Q8_0 codes as f16, and v_mfma_f32_16x16x32_f16 sums the 32
//     products of one block; every partial sum is an integer below 2^24, so the block dot is
//     exact in fp32 whatever the order inside the matrix core.
//   - Q8_0 weights: v_mfma_i32_16x16x32_i8 on the int8 codes (exact int32).
// The block dot is then scaled (MXFP4: ldexp(d_act, e - 128); Q8_0: fp16(d_w) * d_act, the
// CPU's own products; in the Q8_0 loop those products come from a v_mfma_f32_16x16x16_f16 per
// fragment whose only nonzero terms are d_w and d_act, exact in fp32) and accumulated in fp32
// block after block. That accumulation order is not
// the CPU's 8-lane chains, so outputs agree with the reference within fp32 rounding (the
// tolerance-checked order), while every integer block dot is bit-exact. The x86 VPSIGNB corner
// (activation code -128 against a negative weight) is applied as an exact correction on rows
// flagged by their quantizer.
//
// MFMA 16x16x32 lane layouts (checked on the device): A: lane l holds row l%16, k = 8(l/16)..+7;
// B: k = 8(l/16)..+7 of column l%16; D: rows 4(l/16)..+3 of column l%16. The bank's slice layout
// puts slices 2q and 2q+1 of a block (elements 8q..8q+7) in two 16-byte group entries, which is
// exactly lane group q's k range, so a lane's A operand is two dwords of the bank as stored (the
// staging loads only place them in LDS).
//
// A workgroup (4 waves) computes 64 bank rows (a tile pair) x one job tile of one expert (192 jobs
// for Q8_0, 128 for MXFP4); wave w owns bank tile 2p + (w & 1) and half w >> 1 of the tile's live
// jobs (the halves split at a multiple of 16) as a 2 x (up to 6, resp. 4) grid of 16x16
// fragments. A 2048-token top-8 prefill over 128 experts gives every expert 96-158 jobs, one Q8_0
// tile, so each expert's weights are read once per row pair and every weight operand feeds up to
// five MFMAs per wave.
#include <type_traits>

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
typedef _Float16 half4_g __attribute__((ext_vector_type(4)));

constexpr int kGemmThreads = 256;
// Jobs per grouped-GEMM workgroup (gemm_job_tile) and 16-job fragment columns per wave: the two
// wave halves of a workgroup split its live jobs evenly.
template <int TYPE>
constexpr int job_tile() {
    return TYPE == 39 ? 128 : 192;
}
constexpr int kMxJobTile = 64;                             // the MXFP8 experiment's job tile

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
    const float * row_scale;   // epilogue 0: per-job factor applied after the bias (routing weights), or null
    float * dst;               // epilogue 0: [job][rows]
    int row_pairs;             // 64-row tile pairs of the bank
    uint8_t * rows_out;        // epilogue 1: GLU output rows for the down projection (out_lay)
    GemmRowLayout out_lay;
    int activation;
    float alpha, limit;
    int dst_vec4;              // epilogue 0: dst is 16-byte aligned (rows are multiples of 32)
};

__device__ __forceinline__ half2_g fp4x2(unsigned dw, int sel, float scale = 2.0f) {
    // sel is a compile-time constant at every call site after unrolling
    switch (sel) {
        case 0: return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, scale, 0);
        case 1: return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, scale, 1);
        case 2: return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, scale, 2);
        default: return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(dw, scale, 3);
    }
}

// Weight operand of one block from the dwords w0, w1 of slices 2q, 2q+1 that hold it: MXFP4
// bytes 2b, 2b+1 of a 16-byte slice entry carry the slice's 4 nibbles of block b, so block b is
// half (b & 1) of dword b / 2. The e2m1 values come out multiplied by `scale` (a power of two):
// 2 gives the doubled-table integers; 2^(e+1) folds the block exponent e in as well.
__device__ __forceinline__ half8_t mx_a_operand(unsigned w0, unsigned w1, int odd, float scale = 2.0f) {
    half2_g p0, p1, p2, p3;
    if (odd) {
        p0 = fp4x2(w0, 2, scale), p1 = fp4x2(w0, 3, scale), p2 = fp4x2(w1, 2, scale), p3 = fp4x2(w1, 3, scale);
    } else {
        p0 = fp4x2(w0, 0, scale), p1 = fp4x2(w0, 1, scale), p2 = fp4x2(w1, 0, scale), p3 = fp4x2(w1, 1, scale);
    }
    return half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// Exact VPSIGNB correction of one fragment column: contract minus true product is 256 * w for
// every element whose activation code is -128 and whose weight is negative. Computed by a second
// f16 MFMA on (min(w, 0), 256 [a == -128]) operands accumulating into the block dot (all partial
// sums stay integers below 2^24); only for waves holding flagged rows. Q8_0 takes the same route
// with its int8 codes widened to f16.
__device__ __forceinline__ half8_t neg_part(half8_t w) {
    half8_t r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = w[i] < static_cast<_Float16>(0.0f) ? w[i] : static_cast<_Float16>(0.0f);
    return r;
}
__device__ __forceinline__ half8_t is_neg128_x256(half8_t a) {
    half8_t r;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        r[i] = a[i] == static_cast<_Float16>(-128.0f) ? static_cast<_Float16>(256.0f) : static_cast<_Float16>(0.0f);
    return r;
}
__device__ __forceinline__ half8_t i8_to_f16(long v) {
    half8_t r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = static_cast<_Float16>(static_cast<signed char>(v >> (8 * i)));
    return r;
}
// Pipeline stages, filled by global-to-LDS DMA: a ring of S chunks of CB blocks, each stage
// holding the job tile's activation codes and block scales of its chunk and, for MXFP4, both tiles'
// weight dwords of those blocks ([slice][row] dwords, rows of odd slice pairs rotated by 16
// against bank conflicts) and their exponent dword per row. Q8_0 (GROUPED): a tile's weights of
// one 4-block bank group are 4 KB contiguous in the bank, so both tiles' group weights are staged
// once per group by 16-byte DMAs into a two-slot group ring beside the chunk ring ([tile][slice]
// [row] 16-byte units, the bank's own order), with the group's fp16 scales ([tile][row] 8 bytes)
// and the job tile's activation block scales of the group ([job][4 blocks], 16 bytes each):
// a third of the chunk's DMA instructions, whose issue (not their bytes) bounded the kernel
// (doubling the weight DMAs of the former per-chunk dword staging added 55 us to a 345 us
// gate_up launch, doubling the activation DMAs 30 us). The same group staging for MXFP4 (8-block
// groups over four chunks, 2 waves per SIMD) measured slower, 1215-1280 against 1110-1136 us for
// the MXFP4 gate_up of 2048 tokens top-4, so MXFP4 keeps per-chunk staging. Chunk c issues the loads of chunk c + 1
// (and of the next group at its last chunk); one wait and one barrier per chunk. Two stages: a
// third one, for every operand or for the weights alone, measured no faster (Q8_0 layer of 2048
// tokens). Q8_0 chunks of a whole group (4 blocks, one barrier per group) need 132 VGPRs, so 3
// instead of 4 workgroups per CU, and measured slower: 0.625 against 0.555 ms per layer.
template <int TYPE>
struct GemmStage {
    static constexpr int kJobTile = job_tile<TYPE>();
    static constexpr int EB = TYPE == 39 ? 2 : 1;                       // bytes per activation code
    static constexpr int GB = TYPE == 39 ? 8 : 4;                       // blocks per bank group
    static constexpr int CB = 2;                                        // blocks per chunk
    static constexpr int CPG = GB / CB;                                 // chunks per group
    static constexpr int S = 2;                                         // ring depth
    static constexpr int ROW = CB * 32 * EB;                            // bytes per job row and chunk
    static constexpr int ACT = kJobTile * ROW;
    static constexpr bool GROUPED = TYPE == 8;
    static constexpr int DA = GROUPED ? 0 : kJobTile * CB * 4;
    static constexpr int W = GROUPED ? 0 : 2 * 8 * 32 * 4;
    static constexpr int M = GROUPED ? 0 : 2 * 32 * 4;
    static constexpr int OFF_DA = ACT, OFF_W = OFF_DA + DA, OFF_M = OFF_W + W;
    static constexpr int STAGE = OFF_M + M;
    static constexpr int WG = GROUPED ? 2 * 8 * 32 * 16 : 0;   // group weight slot: [tile][slice][row] x 16 B
    static constexpr int MG = GROUPED ? 2 * 32 * 8 : 0;        // group scale slot: [tile][row] x 4 fp16
    static constexpr int DG = GROUPED ? kJobTile * GB * 4 : 0;   // group block-scale slot: [job][4 blocks] fp32
    static constexpr int OFF_WG = S * STAGE, OFF_MG = OFF_WG + 2 * WG, OFF_DG = OFF_MG + 2 * MG;
    static constexpr int BYTES = OFF_DG + 2 * DG;
    // DMA instructions per wave and chunk: activation rows (1 KiB each, ACT_JOBS job rows), block
    // scales, weights, meta. A wave skips the activation loads whose job rows are all past the
    // tile's live jobs, so its count per chunk varies; the wait before each chunk's barrier drains
    // every load of the wave, which the two-stage ring allows (the next chunk's loads are issued
    // after it).
    static constexpr int ACT_JOBS = 1024 / ROW;
    static constexpr int ACT_DMA = ACT / 1024 / 4;
    static constexpr int W_DMA = W / 256 / 4;
    static constexpr int WG_DMA = WG / 1024 / 4;   // 16-byte group weight loads per wave
    static_assert(S == 2, "the per-chunk wait is vmcnt(0)");
    static_assert(!GROUPED || (CPG == 2 && WG_DMA == 2), "Q8_0 group staging: two chunks per group, two loads per wave");
    static_assert(ACT % 4096 == 0 && (!GROUPED || kJobTile % 64 == 0), "whole activation and block-scale DMAs per wave");
};

// Global-to-LDS DMA (global_load_lds_*): lane l's bytes land at LDS address m0 + l * size. The
// loads are issued through inline assembly so that the compiler's wait-count pass, which would
// wait for every such load before any LDS read it cannot prove disjoint, leaves the multi-stage
// ring alone; the kernel waits for them explicitly (lds_dma_wait) before each barrier. The
// compiler's own waits stay correct: loads it does not know of only make its counts stricter.
// M0 is a register the compiler reserves; the kernels of this file use it for nothing else (no
// v_movrel, s_sendmsg or LDS-DMA builtin: their assembly holds no other M0 access), so the
// clobber it is told of costs nothing and -Winline-asm's caution about reserved registers does
// not apply.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma_x4(const void * src, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0) : "memory", "m0");
}
__device__ __forceinline__ void lds_dma_x1(const void * src, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(m0) : "memory", "m0");
}
__device__ __forceinline__ void lds_dma_x1_s(const void * base, uint32_t off, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(m0) : "memory", "m0");
}
__device__ __forceinline__ void lds_dma_x4_s(const void * base, uint32_t off, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m0) : "memory", "m0");
}
#pragma clang diagnostic pop
template <int N>
__device__ __forceinline__ void lds_dma_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// The GLU of the fast accumulation order's epilogue: the formulas of glu() (SwiGLU-OAI with its
// clamps, or SiLU), with the device library's fast exp (__expf) and a fast divide (__fdividef)
// instead of the correctly rounded exp and the IEEE division the exact order needs. The fast
// order is held to the tolerance of the fp32 layer outputs, not to bits.
__device__ __forceinline__ float glu_fast(int activation, float g0, float u0, float alpha, float limit) {
    if (activation == VBM_ACT_SWIGLU_OAI) {
        const float g = limit < g0 ? limit : g0;
        const float u = u0 < -limit ? -limit : (limit < u0 ? limit : u0);
        return __fdividef(g, 1.0f + __expf(alpha * (-g))) * (u + 1.0f);
    }
    return __fdividef(g0, 1.0f + __expf(-g0)) * u0;
}

// fp16 x fp32 product on one instruction: v_fma_mix_f32 with the half in the low (HI = 0) or high
// half of `h2` and -0 as the addend, i.e. exactly float(h) * x rounded once, signed zeros included.
template <int HI>
__device__ __forceinline__ float mul_half(unsigned h2, float x, float neg_zero) {
    float r;
    if constexpr (HI) asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(x), "s"(neg_zero));
    else asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(x), "s"(neg_zero));
    return r;
}

template <int TYPE, int EPI, bool FLAGGED>
__global__ __launch_bounds__(kGemmThreads, (TYPE == 8 && !FLAGGED) ? 3 : 1) void grouped_gemm_kernel(GemmArgs A) {
    using G = GemmStage<TYPE>;
    constexpr int CB = G::CB;
    constexpr int kJobTile = G::kJobTile;
    constexpr int kLdsBytes = G::BYTES > kJobTile * 68 * 4 ? G::BYTES : kJobTile * 68 * 4;   // stages / epilogue tile
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];
    float (*tile_vals)[68] = reinterpret_cast<float (*)[68]>(lds);    // epilogue tile [job][pair row], after the K loop

    // XCD-aware order: workgroup i runs on XCD i % 8, so hand each XCD a contiguous range of
    // (tile, pair) items; the pairs of one job tile then share its activation rows in one L2 and
    // consecutive tiles of an expert share its weights.
    const int n_items = *cst<int32_t>(A.n_tiles) * A.row_pairs;
    const int per_xcd = (n_items + 7) >> 3;
    const int slot8 = static_cast<int>(blockIdx.x >> 3);
    const int item = static_cast<int>(blockIdx.x & 7) * per_xcd + slot8;
    if (slot8 >= per_xcd || item >= n_items) return;
    const int ti = item / A.row_pairs;
    const int pair = item - ti * A.row_pairs;
    const int expert = cst<int32_t>(A.tile_expert)[ti];
    const int j0 = cst<int32_t>(A.tile_start)[ti];
    const int count = cst<int32_t>(A.counts)[expert];
    const int joff = cst<int32_t>(A.offsets)[expert];
    const int slot = A.expert_to_slot ? cst<int32_t>(A.expert_to_slot)[expert] : expert;
    const GemmShape S = A.shape;
    if (slot < 0 || slot >= S.n_slots) {
        // Expert not resident in this bank (a tile filter removes the experts a pass skips on
        // purpose, so this is a bad map): this workgroup's outputs become NaN, as in the decode
        // kernels, rather than leaving stale workspace data. Epilogue 1 poisons the block scale
        // of the GLU block of this tile pair.
        const float nan = __builtin_nanf("");
        const int live_jobs = count - j0 < kJobTile ? count - j0 : kJobTile;
        if (EPI == 0) {
            for (int i = threadIdx.x; i < live_jobs * 64; i += kGemmThreads) {
                const int64_t brow = static_cast<int64_t>(pair) * 64 + (i & 63);
                if (brow < S.rows)
                    A.dst[static_cast<size_t>(A.jobs[joff + j0 + (i >> 6)]) * S.rows + ggml_row(brow, S.rows, S.interleave)] = nan;
            }
        } else {
            for (int j = threadIdx.x; j < live_jobs; j += kGemmThreads)
                reinterpret_cast<float *>(A.rows_out + static_cast<int64_t>(A.jobs[joff + j0 + j]) * A.out_lay.stride() +
                                          A.out_lay.da_offset())[pair] = nan;
        }
        return;
    }

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int lr = lane & 15, q = lane >> 4;
    const int tile = pair * 2 + (wave & 1);
    const bool tile_live = tile * 32 < S.rows;
    const int nb = S.nb;
    const int groups = nb / G::GB, tail = nb % G::GB;
    constexpr int kCodeRow = TYPE == 39 ? 16 : 32;     // code bytes per row and block
    constexpr int kMetaRow = TYPE == 39 ? 1 : 2;       // exponent / scale bytes per row and block
    const uint8_t * slot_base = A.bank + static_cast<size_t>(slot) * S.slot_bytes;
    const uint8_t * codes = slot_base + static_cast<size_t>(tile_live ? tile : 0) * 32 * nb * kCodeRow;
    const uint8_t * meta = slot_base + S.codes_bytes + static_cast<size_t>(tile_live ? tile : 0) * 32 * nb * kMetaRow;
    auto row_of = [&](int jl) -> const uint8_t * {   // activation row of local job jl (must be live)
        const int jb = A.jobs[joff + j0 + jl];
        const int64_t row_index = A.b_ne1 == 1 ? jb / A.n_ids : jb;
        return A.rows_in + row_index * A.lay.stride();
    };

    // The two wave halves (waves 0-1, 2-3) split the tile's live jobs at a multiple of 16: jobs
    // [0, split) and [split, live), so a tile of n jobs costs each half about n / 2 of them (a
    // 64-job tile gives each half 32 instead of all 64 to the first). This lane's fragment columns
    // are jobs wj + 16jh + lr of its half; the -128 flags of the wave.
    // Rows converted from caller-quantized Q8_0 data (FLAGGED) may hold -128 codes.
    constexpr int JF = kJobTile / 32;
    const int wq = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 7));   // the wave's half
    const int live_jobs = count - j0 < kJobTile ? count - j0 : kJobTile;
    const int split = 16 * ((live_jobs + 31) / 32);
    const int wj = wq * split;                         // the wave's first job in the tile
    const int half_end = wq ? live_jobs : (split < live_jobs ? split : live_jobs);
    bool jlive[JF];
    int flagged = 0;
#pragma unroll
    for (int jh = 0; jh < JF; ++jh) {
        const int jl = wj + 16 * jh + lr;
        jlive[jh] = jl < half_end;
        if (FLAGGED && jlive[jh]) flagged |= *reinterpret_cast<const int *>(row_of(jl) + A.lay.flag_offset());
    }
    // Fragment columns of 16 jobs none of which is live (a half's live jobs are a prefix of it) cost
    // the wave no matrix or scale work. The K loop is instantiated per count of live columns (nf,
    // wave-uniform), so its body carries no per-column branch and the compiler can interleave the
    // columns' MFMAs and VALU work.
    static_assert(JF == 4 || JF == 6, "the K loop is instantiated for 0..6 live fragment columns");
    const int live_in_half = half_end - wj;
    const int nf = live_in_half <= 0 ? 0 : (live_in_half + 15) / 16;
    // Workgroup-uniform: every wave then runs the same K-loop instantiation, so each of its
    // barriers is reached from one control path (every thread gets here: the exits above are
    // uniform per workgroup).
    bool slow = false;
    if constexpr (FLAGGED) slow = __syncthreads_or(flagged != 0) != 0;

    // Stage loaders (global-to-LDS DMA). Lanes that have nothing to load are masked, and clamped
    // sources keep every address inside the operands.
    //   - activations: wave w's x4 loads j cover 16 (Q8_0) or 8 (MXFP4) job rows of the chunk;
    //     the 16-byte parts of row r sit at part p ^ s(r) (s(r) = (r >> 1) & 3, resp. r & 7) so
    //     the fragment reads of 16 consecutive rows spread over the banks; within a load that
    //     holds a live job, a row past the tile's jobs reads the first job's row, and a load
    //     whose rows are all past them is skipped (wave-uniform): those LDS rows keep stale
    //     bytes, which reach only the matrix columns of jobs that are never stored;
    //   - block scales: lane l of wave w loads job 32w + l / 2, block l % 2;
    //   - weights: dword loads; Q8_0 load I = 4w + i covers tile I >> 3, slice pair (I >> 1) & 3,
    //     rows 16 (I & 1) .. +15 (lane: row l >> 2, unit dword l & 3); MXFP4 load I = 2w + i covers
    //     tile I >> 2, slices 2 (I & 3) and 2 (I & 3) + 1 (lane: slice l >> 5, position l & 31);
    //     a tile past the bank's rows reads the pair's first tile (its rows are never stored);
    //   - meta: lanes 0..15 of wave w load the dword of rows 16 (w & 1) .. +15 of tile w >> 1.
    const int wu = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int live_rows = __builtin_amdgcn_readfirstlane(count - j0);   // the tile's live jobs
    // LDS address of the stage buffers: a generic pointer to LDS is the aperture base plus the
    // LDS address in its low 32 bits.
    const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
    const uint8_t * act_src[G::ACT_DMA];
#pragma unroll
    for (int j = 0; j < G::ACT_DMA; ++j) {
        const int jr = TYPE == 39 ? 8 * (wave * G::ACT_DMA + j) + (lane >> 3) : 16 * (wave * G::ACT_DMA + j) + (lane >> 2);
        const int part = TYPE == 39 ? (lane & 7) ^ (jr & 7) : (lane & 3) ^ ((jr >> 1) & 3);
        act_src[j] = row_of(j0 + jr < count ? jr : 0) + 16 * part;
    }
    // block scales: per chunk, lane l of wave w loads job 32w + l / 2, block l % 2; grouped (Q8_0),
    // per group, lane l of waves w < kJobTile / 64 loads the 16 bytes of job 64w + l
    static_assert(G::GROUPED || G::DA == kGemmThreads * 4, "one block-scale dword per thread and chunk");
    const int jd = G::GROUPED ? 64 * (wave < kJobTile / 64 ? wave : 0) + lane : 32 * wave + (lane >> 1);
    const uint8_t * da_src = row_of(j0 + jd < count ? jd : 0) + A.lay.da_offset() + (G::GROUPED ? 0 : 4 * (lane & 1));
    // weight dword of this lane within its load's group-relative source
    uint32_t woff;
    if constexpr (TYPE == 39) {
        const int k = lane >> 5, pos = lane & 31;            // slice within the pair of slices
        woff = static_cast<uint32_t>((k * 32 + pos) * 16);   // the rotation depends on the pair: added per load
    } else {
        woff = static_cast<uint32_t>(((lane & 1) * 32 + (lane >> 2)) * 16 + 4 * ((lane >> 1) & 1));
    }
    const uint32_t moff = static_cast<uint32_t>(lane) * 8;
    const size_t tile_bytes = static_cast<size_t>(32) * nb * kCodeRow, meta_tile_bytes = static_cast<size_t>(32) * nb * kMetaRow;
    auto tsel = [&](int t) -> size_t { return (pair * 2 + t) * 32 < S.rows ? pair * 2 + t : pair * 2; };
    // new_group: also stage chunk c's bank group (Q8_0), into group slot grp & 1; the slot of the
    // group before it is still being read, the one before that is free since the barrier that
    // ended its last chunk.
    auto dma_stage = [&](int c, int st, bool new_group) {
        const int grp = c / G::CPG, sub = c % G::CPG;
        const uint32_t sb = lds0 + st * G::STAGE;
#pragma unroll
        for (int j = 0; j < G::ACT_DMA; ++j)
            if (G::ACT_JOBS * (wu * G::ACT_DMA + j) < live_rows)
                lds_dma_x4(act_src[j] + static_cast<int64_t>(c) * G::ROW, sb + (wu * G::ACT_DMA + j) * 1024);
        if constexpr (!G::GROUPED) lds_dma_x1(da_src + static_cast<int64_t>(c) * CB * 4, sb + G::OFF_DA + wu * 256);
        if constexpr (G::GROUPED) {
            if (new_group) {
                // load I = 2w + i: tile I >> 2, the 1 KiB quarter I & 3 of its group (lane l: the
                // 16-byte unit 64 (I & 3) + l, i.e. slice 2 (I & 3) + l / 32, row l % 32)
                const uint32_t wslot = lds0 + G::OFF_WG + (grp & 1) * G::WG;
#pragma unroll
                for (int i = 0; i < G::WG_DMA; ++i) {
                    const int I = wu * G::WG_DMA + i, t = I >> 2, part = I & 3;
                    const uint8_t * base = slot_base + tsel(t) * tile_bytes + static_cast<size_t>(grp) * 4096 + part * 1024;
                    lds_dma_x4_s(base, static_cast<uint32_t>(lane) * 16, wslot + t * 4096 + part * 1024);
                }
                // the group's scales: lanes 0..31 of wave 0, 16 bytes (two rows) each, tile l / 16
                if (wu == 0 && lane < 32)
                    lds_dma_x4(slot_base + S.codes_bytes + tsel(lane >> 4) * meta_tile_bytes + static_cast<size_t>(grp) * 256 +
                                   (lane & 15) * 16,
                               lds0 + G::OFF_MG + (grp & 1) * G::MG);
                if (wu < kJobTile / 64)
                    lds_dma_x4(da_src + 16 * grp,
                               __builtin_amdgcn_readfirstlane(lds0 + G::OFF_DG + (grp & 1) * G::DG + wu * 1024));
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < G::W_DMA; ++i) {
            const int I = wu * G::W_DMA + i;
            if constexpr (TYPE == 39) {
                // slices 2 (I & 3) + (l >> 5): odd slice pairs hold row r at position r ^ 16
                const int t = I >> 2, kp = I & 3;
                const uint8_t * base = slot_base + tsel(t) * tile_bytes + static_cast<size_t>(grp) * 4096 + kp * 2 * 512 + 4 * sub;
                lds_dma_x1_s(base, (kp & 1) ? (woff ^ (16 * 16)) : woff, sb + G::OFF_W + (t * 8 + kp * 2) * 128);
            } else {
                const int t = I >> 3, qq = (I >> 1) & 3, rh = I & 1;
                const uint8_t * base =
                    slot_base + tsel(t) * tile_bytes + static_cast<size_t>(grp) * 4096 + (2 * qq * 32 + rh * 16) * 16 + 8 * sub;
                lds_dma_x1_s(base, woff, sb + G::OFF_W + t * 2048 + (qq * 32 + rh * 16) * 16);
            }
        }
        const uint8_t * mbase = slot_base + S.codes_bytes + tsel(wu >> 1) * meta_tile_bytes + static_cast<size_t>(grp) * 256 +
                                16 * (wu & 1) * 8 + (TYPE == 39 ? 4 * (sub >> 1) : 4 * sub);
        if (lane < 16) lds_dma_x1_s(mbase, moff, sb + G::OFF_M + wu * 64);
    };

    f32x4 acc[2][JF];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jh = 0; jh < JF; ++jh) acc[i][jh] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // One block: weight operands a_op[i] (row halves i), activation operand and scale of job half
    // jh from bsrc(jh) / dsrc(jh); factor(i, j, da) is the block's fp32 scale for output row
    // 16i + 4q + j: ldexp(da, e) for MXFP4 exponent e, fp16(d_w) * da for Q8_0. SLOW adds the
    // exact -128 correction, accumulated into the same MFMA result (its operands scaled by 256
    // are exact in fp16).
    const float neg_zero = -0.0f;
    auto block_step = [&](auto slow_c, auto nf_c, const auto & a_op, auto && factor, auto && bsrc, auto && dsrc) {
        constexpr bool SLOW = decltype(slow_c)::value;
        constexpr int NF = decltype(nf_c)::value;
#pragma unroll
        for (int jh = 0; jh < NF; ++jh) {
            const float da = dsrc(jh);
            const auto bv = bsrc(jh);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                f32x4 d;
                if constexpr (TYPE == 39) {
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_op[i], bv, f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                    if constexpr (SLOW) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(neg_part(a_op[i]), is_neg128_x256(bv), d, 0, 0, 0);
                } else if constexpr (!SLOW) {
                    const i32x4 di = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_op[i], bv, i32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                    for (int j = 0; j < 4; ++j) d[j] = static_cast<float>(di[j]);
                } else {
                    const half8_t a16 = i8_to_f16(a_op[i]), b16 = i8_to_f16(bv);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a16, b16, f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(neg_part(a16), is_neg128_x256(b16), d, 0, 0, 0);
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][jh][j] = __builtin_fmaf(factor(i, j, da), d[j], acc[i][jh][j]);
            }
        }
    };

    // The K loop, instantiated with and without the -128 correction (workgroup-uniform choice) and
    // per count of live fragment columns.
    const int n_chunks = groups * G::CPG;
    auto k_loop = [&](auto slow_c, auto nf_c) {
        constexpr int NF = decltype(nf_c)::value;
        // weight dwords of A rows lr + 16i, slices 2q / 2q + 1 (MXFP4: row r of an odd slice pair
        // at position r ^ 16), or their 16-byte unit (Q8_0)
        // (Q8_0: unit (2q, row) of the group slot; slice 2q + 1's unit is 512 bytes on)
        const uint8_t * w_lds[2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
            w_lds[i] = TYPE == 39 ? lds + G::OFF_W + ((wave & 1) * 256 + 2 * q * 32 + 16 * (i ^ (q & 1)) + lr) * 4
                                  : lds + G::OFF_WG + (wave & 1) * 4096 + (2 * q * 32 + 16 * i + lr) * 16;
        // exponent dword (MXFP4, per chunk stage) or the group's 8 scale bytes (Q8_0, group slot)
        // of output rows 4q + j (+16i) and of A rows lr (+16i)
        const uint8_t * m_lds = TYPE == 39 ? lds + G::OFF_M + ((wave & 1) * 32 + 4 * q) * 4
                                           : lds + G::OFF_MG + ((wave & 1) * 32 + 4 * q) * 8;
        const uint8_t * ma_lds = TYPE == 39 ? lds + G::OFF_M + ((wave & 1) * 32 + lr) * 4
                                            : lds + G::OFF_MG + ((wave & 1) * 32 + lr) * 8;
        const float * d_lds = G::GROUPED ? reinterpret_cast<const float *>(lds + G::OFF_DG) + (wj + lr) * G::GB
                                         : reinterpret_cast<const float *>(lds + G::OFF_DA) + (wj + lr) * CB;
        // fragment columns' activation codes: row rr = wj + 16jh + lr, block bb, codes 8q..8q+7
        uint32_t aoff[JF][2];
#pragma unroll
        for (int jh = 0; jh < JF; ++jh)
#pragma unroll
            for (int bb = 0; bb < 2; ++bb) {
                const int rr = wj + 16 * jh + lr;
                aoff[jh][bb] = TYPE == 39 ? rr * 128 + (((4 * bb + q) ^ (rr & 7)) << 4)
                                          : rr * 64 + (((2 * bb + (q >> 1)) ^ ((rr >> 1) & 3)) << 4) + 8 * (q & 1);
            }
#pragma clang loop unroll(disable)
        for (int c = 0; c < n_chunks; ++c) {
            const int sub = c % G::CPG, gs = (c / G::CPG) & 1;   // gs: this chunk's group slot
            // this chunk's loads: the stage of chunk c + 1, clamped to the last chunk (the stage
            // it fills is free either way), and chunk c + 1's bank group when it starts one
            dma_stage(c + 1 < n_chunks ? c + 1 : n_chunks - 1, (c + 1) % G::S, c + 1 < n_chunks && (c + 1) % G::CPG == 0);
            const int ab = c % G::S, wb = ab;
            const uint8_t * st = lds + ab * G::STAGE;     // this chunk's stage
            // This chunk's blocks 2sub, 2sub+1 in the group: weight dwords of slices 2q, 2q+1
            // (MXFP4: one dword holds both blocks; Q8_0: one dword each).
            unsigned w0[2][2], w1[2][2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                if constexpr (TYPE == 39) {
                    const uint8_t * w = w_lds[i] + wb * G::STAGE;
                    w0[i][0] = w0[i][1] = *reinterpret_cast<const unsigned *>(w);
                    w1[i][0] = w1[i][1] = *reinterpret_cast<const unsigned *>(w + 32 * 4);
                } else {
                    const uint8_t * w = w_lds[i] + gs * G::WG + 8 * sub;
                    const u32x2g a = *reinterpret_cast<const u32x2g *>(w), b = *reinterpret_cast<const u32x2g *>(w + 512);
                    w0[i][0] = a[0], w0[i][1] = a[1], w1[i][0] = b[0], w1[i][1] = b[1];
                }
            }
            // MXFP4 fast path: when every exponent e of the wave's A rows (16i + lr) lies in
            // [-14, 12], 2^(e+1) times the e2m1 values is an exact normal f16, so the exponent
            // rides in the A operand and the block result needs one FMA with d_act:
            // da * (2^e * dot) rounds the same product as ldexp(da, e) * dot.
            bool folded = false;
            float fsc[2][2];
            if constexpr (TYPE == 39 && !decltype(slow_c)::value) {
                bool ok = true;
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const unsigned ea = *reinterpret_cast<const uint16_t *>(ma_lds + wb * G::STAGE + i * 16 * 4 + (sub & 1) * 2);
#pragma unroll
                    for (int bb = 0; bb < 2; ++bb) {
                        const int e = static_cast<signed char>(ea >> (8 * bb));
                        ok = ok && e >= -14 && e <= 12;
                        fsc[i][bb] = __builtin_bit_cast(float, static_cast<unsigned>(e + 128) << 23);
                    }
                }
                folded = __all(ok);
            }
            if (folded) {
#pragma unroll
                for (int bb = 0; bb < CB; ++bb) {
                    half8_t a_op[2];
#pragma unroll
                    for (int i = 0; i < 2; ++i) a_op[i] = mx_a_operand(w0[i][bb], w1[i][bb], bb, fsc[i][bb]);
#pragma unroll
                    for (int jh = 0; jh < NF; ++jh) {
                        const float da = d_lds[ab * (G::STAGE / 4) + 16 * jh * CB + bb];
                        const half8_t bv = *reinterpret_cast<const half8_t *>(st + aoff[jh][bb]);
#pragma unroll
                        for (int i = 0; i < 2; ++i) {
                            const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_op[i], bv, f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                            for (int j = 0; j < 4; ++j) acc[i][jh][j] = __builtin_fmaf(da, d[j], acc[i][jh][j]);
                        }
                    }
                }
            } else if constexpr (TYPE == 8 && !decltype(slow_c)::value) {
                // Q8_0: the scale products fp16(d_w) * d_act of a 16 x 16 output fragment come
                // from one f16 MFMA per block: A holds d_w of the fragment's 16 rows at k = bb
                // (lanes 0..15, zero elsewhere), B the 16 jobs' d_act at k = bb. Each output is
                // the exact fp32 product of two fp16 values (11-bit significands) plus zeros:
                // the value the per-output VALU product gives, off the vector ALU.
                const unsigned sel[2] = {lane < 16 ? 0x0000FFFFu : 0u, lane < 16 ? 0xFFFF0000u : 0u};
                unsigned dw_row[2], da_pk[JF];
#pragma unroll
                for (int i = 0; i < 2; ++i) dw_row[i] = *reinterpret_cast<const unsigned *>(ma_lds + gs * G::MG + i * 16 * 8 + 4 * sub);
#pragma unroll
                for (int jh = 0; jh < NF; ++jh) {
                    // d_act holds fp16 values, so the packing conversion is exact
                    const float * dp = d_lds + gs * (G::DG / 4) + 16 * jh * G::GB + CB * sub;
                    da_pk[jh] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_pkrtz(dp[0], dp[1]));
                }
#pragma unroll
                for (int bb = 0; bb < CB; ++bb) {
                    long a_op[2];
                    half4_g as[2];
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        a_op[i] = static_cast<long>(static_cast<uint64_t>(w0[i][bb]) | (static_cast<uint64_t>(w1[i][bb]) << 32));
                        as[i] = __builtin_bit_cast(half4_g, u32x2g{dw_row[i] & sel[bb], 0u});
                    }
#pragma unroll
                    for (int jh = 0; jh < NF; ++jh) {
                        const long bv = *reinterpret_cast<const long *>(st + aoff[jh][bb]);
                        const half4_g bs = __builtin_bit_cast(half4_g, u32x2g{da_pk[jh] & sel[bb], 0u});
#pragma unroll
                        for (int i = 0; i < 2; ++i) {
                            const i32x4 di = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_op[i], bv, i32x4{0, 0, 0, 0}, 0, 0, 0);
                            const f32x4 sc = __builtin_amdgcn_mfma_f32_16x16x16f16(as[i], bs, f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                            for (int j = 0; j < 4; ++j)
                                acc[i][jh][j] = __builtin_fmaf(sc[j], static_cast<float>(di[j]), acc[i][jh][j]);
                        }
                    }
                }
            } else {
                // exponent / scale bytes of output rows 16i + 4q + j (MXFP4 one byte, Q8_0 two per block)
                // (Q8_0: both blocks' fp16 scales of a row in one dword)
                unsigned mw[2][4];
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if constexpr (TYPE == 39)
                            mw[i][j] = *reinterpret_cast<const uint16_t *>(m_lds + wb * G::STAGE + (16 * i + j) * 4 + (sub & 1) * 2);
                        else
                            mw[i][j] = *reinterpret_cast<const unsigned *>(m_lds + gs * G::MG + (16 * i + j) * 8 + 4 * sub);
                    }
                auto do_block = [&](int bb) {
                    auto bsrc = [&](int jh) {
                        const uint8_t * p = st + aoff[jh][bb];
                        if constexpr (TYPE == 39) return *reinterpret_cast<const half8_t *>(p);
                        else return *reinterpret_cast<const long *>(p);
                    };
                    auto dsrc = [&](int jh) {
                        if constexpr (G::GROUPED) return d_lds[gs * (G::DG / 4) + 16 * jh * G::GB + CB * sub + bb];
                        else return d_lds[ab * (G::STAGE / 4) + 16 * jh * CB + bb];
                    };
                    if constexpr (TYPE == 39) {
                        auto factor = [&](int i, int j, float da) {
                            return __builtin_amdgcn_ldexpf(da, static_cast<signed char>(mw[i][j] >> (8 * bb)));
                        };
                        half8_t a_op[2];
#pragma unroll
                        for (int i = 0; i < 2; ++i) a_op[i] = mx_a_operand(w0[i][bb], w1[i][bb], bb);
                        block_step(slow_c, nf_c, a_op, factor, bsrc, dsrc);
                    } else {
                        auto factor = [&](int i, int j, float da) {
                            return bb ? mul_half<1>(mw[i][j], da, neg_zero) : mul_half<0>(mw[i][j], da, neg_zero);
                        };
                        long a_op[2];
#pragma unroll
                        for (int i = 0; i < 2; ++i)
                            a_op[i] = static_cast<long>(static_cast<uint64_t>(w0[i][bb]) | (static_cast<uint64_t>(w1[i][bb]) << 32));
                        block_step(slow_c, nf_c, a_op, factor, bsrc, dsrc);
                    }
                };
                if constexpr (decltype(slow_c)::value) {
#pragma clang loop unroll(disable)
                    for (int bb = 0; bb < CB; ++bb) do_block(bb);
                } else {
#pragma unroll
                    for (int bb = 0; bb < CB; ++bb) do_block(bb);
                }
            }
            // the stage of chunk c + 1, issued at the top of this chunk
            lds_dma_wait<0>();
            __syncthreads();
        }

        // Tail blocks (nb even: MXFP4 tail in {0,2,4,6}, Q8_0 tail in {0,2}), per-row packed, read
        // straight from global memory.
        for (int bt = 0; bt < tail; ++bt) {
            const int b = groups * G::GB + bt;
            unsigned m[2][4];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int orow = 16 * i + 4 * q + j;
                    m[i][j] = 0;
                    if (tile_live) {
                        if constexpr (TYPE == 39) m[i][j] = meta[groups * 256 + orow * tail + bt];
                        else m[i][j] = *reinterpret_cast<const uint16_t *>(meta + groups * 256 + (orow * tail + bt) * 2);
                    }
                }
            auto factor = [&](int i, int j, float da) {
                if constexpr (TYPE == 39) return __builtin_amdgcn_ldexpf(da, static_cast<signed char>(m[i][j]));
                else return half_bits_to_float(static_cast<uint16_t>(m[i][j])) * da;
            };
            const uint8_t * brow[JF];
#pragma unroll
            for (int jh = 0; jh < JF; ++jh) brow[jh] = jlive[jh] ? row_of(wj + 16 * jh + lr) : nullptr;
            auto bsrc = [&](int jh) {
                if constexpr (TYPE == 39) {
                    half8_t v = half8_t{};
                    if (brow[jh]) v = *reinterpret_cast<const half8_t *>(brow[jh] + (static_cast<int64_t>(b) * 32 + 8 * q) * 2);
                    return v;
                } else {
                    long v = 0;
                    if (brow[jh]) v = *reinterpret_cast<const long *>(brow[jh] + static_cast<int64_t>(b) * 32 + 8 * q);
                    return v;
                }
            };
            auto dsrc = [&](int jh) { return brow[jh] ? reinterpret_cast<const float *>(brow[jh] + A.lay.da_offset())[b] : 0.0f; };
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
                block_step(slow_c, nf_c, a, factor, bsrc, dsrc);
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
                block_step(slow_c, nf_c, a, factor, bsrc, dsrc);
            }
        }
    };
    // Prologue: stages 0 .. S - 2 (clamped).
    if (groups > 0) {
        dma_stage(0, 0, true);
        lds_dma_wait<0>();
    }
    __syncthreads();
    // Waves of one workgroup may take different instantiations (their job halves hold different
    // numbers of live columns); every instantiation issues the same stage loads and reaches one
    // barrier per chunk.
    auto k_loop_nf = [&](auto slow_c) {
        switch (nf) {
            case 6: if constexpr (JF >= 6) k_loop(slow_c, std::integral_constant<int, 6>{}); break;
            case 5: if constexpr (JF >= 5) k_loop(slow_c, std::integral_constant<int, 5>{}); break;
            case 4: k_loop(slow_c, std::integral_constant<int, 4>{}); break;
            case 3: k_loop(slow_c, std::integral_constant<int, 3>{}); break;
            case 2: k_loop(slow_c, std::integral_constant<int, 2>{}); break;
            case 1: k_loop(slow_c, std::integral_constant<int, 1>{}); break;
            default: k_loop(slow_c, std::integral_constant<int, 0>{}); break;
        }
    };
    if constexpr (FLAGGED) {
        if (slow) k_loop_nf(std::true_type{});
        else k_loop_nf(std::false_type{});
    } else {
        k_loop_nf(std::false_type{});
    }
    // The clamped loads of the last chunks may still be landing in the stages the epilogue reuses.
    lds_dma_wait<0>();
    __syncthreads();

    // Epilogue: biases (ggml row order), then either fp32 rows (times the job's routing weight when
    // row_scale is given: ggml's ADD_ID, then MUL, hybrid-experts.patch:1636-1646) or GLU + Q8_0
    // requantization. The fp32 rows go through the LDS tile too when the output allows 16-byte
    // stores, so that each job's 64 rows leave as four full 64-byte segments instead of 4-byte
    // scatter.
    const bool via_lds = EPI == 1 || A.dst_vec4;
    // the fragment columns' jobs and routing weights, loaded only now (held through the K loop they
    // cost registers it needs)
    int job[JF];
    float rscale[JF];
#pragma unroll
    for (int jh = 0; jh < JF; ++jh) {
        job[jh] = jlive[jh] ? A.jobs[joff + j0 + wj + 16 * jh + lr] : 0;
        rscale[jh] = EPI == 0 && A.row_scale && jlive[jh] ? A.row_scale[job[jh]] : 1.0f;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int orow = 16 * i + 4 * q + j;
            const int grow = static_cast<int>(ggml_row(static_cast<int64_t>(tile) * 32 + orow, S.rows, S.interleave));
            const float bv = (A.bias && tile_live) ? A.bias[static_cast<size_t>(expert) * S.rows + grow] : 0.0f;
#pragma unroll
            for (int jh = 0; jh < JF; ++jh) {
                float v = acc[i][jh][j];
                if (A.bias) v = v + bv;
                if (EPI == 0 && A.row_scale) v = v * rscale[jh];
                if (!via_lds) {
                    if (jlive[jh] && tile_live) A.dst[static_cast<size_t>(job[jh]) * S.rows + grow] = v;
                } else if (jlive[jh]) {   // columns past the half's jobs belong to the other half
                    tile_vals[wj + 16 * jh + lr][32 * (wave & 1) + orow] = v;
                }
            }
        }
    }
    if (!via_lds) return;
    __syncthreads();
    for (int jl = threadIdx.x >> 2; jl < kJobTile; jl += kGemmThreads / 4) {   // four threads per job
        const int jj = j0 + jl;
        if (EPI == 0) {
            // 16 pair rows per thread; aligned runs of 4 device rows are 4 consecutive ggml rows
            // (also in interleaved gate|up banks)
            const int seg = threadIdx.x & 3;
            if (jj < count) {
                float * out = A.dst + static_cast<size_t>(A.jobs[joff + jj]) * S.rows;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int col = seg * 16 + 4 * k;
                    const int64_t brow = static_cast<int64_t>(pair) * 64 + col;
                    if (brow < S.rows)
                        *reinterpret_cast<float4 *>(out + ggml_row(brow, S.rows, S.interleave)) =
                            *reinterpret_cast<const float4 *>(&tile_vals[jl][col]);
                }
            }
        } else {
            // one 32-element GLU block per job, eight elements per thread
            const int part = threadIdx.x & 3;
            const bool live = jj < count;
            float x[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int e = part * 8 + t;                 // element of the block
                const int tl = e >> 4;                      // bank tile of the pair
                const float g = tile_vals[jl][32 * tl + (e & 15)];
                const float u = tile_vals[jl][32 * tl + 16 + (e & 15)];
                x[t] = glu_fast(A.activation, g, u, A.alpha, A.limit);
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
}

// Tiles of job_tile jobs per active expert, in active order: one workgroup, wave scans plus a
// scan of the 16 wave totals.
__global__ __launch_bounds__(1024) void gemm_tiles_kernel(const int32_t * counts, const int32_t * active,
                                                          const int32_t * n_active, const int32_t * filter, int job_tile,
                                                          int max_tiles,
                                                          int32_t * tile_expert, int32_t * tile_start, int32_t * n_tiles,
                                                          int32_t * error) {
    __shared__ int s_wave[16];
    const int na = *n_active;
    const int a = threadIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int e = a < na ? active[a] : 0;
    const bool kept = a < na && (filter == nullptr || filter[e] >= 0);   // filtered experts get no tiles
    const int nt = kept ? (counts[e] + job_tile - 1) / job_tile : 0;
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
            tile_start[base + t] = t * job_tile;
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
// Workgroup (row, 64-block segment seg) of it; four threads per block, eight elements each.
__device__ __forceinline__ void gemm_rows_segment(const float * __restrict__ x, int vec4, int nb, int64_t x_stride,
                                                  const GemmRowLayout & L, uint8_t * __restrict__ out, int64_t row,
                                                  int seg) {
    const int bq = seg * 64 + static_cast<int>(threadIdx.x >> 2);
    const bool live = bq < nb;
    const int b = live ? bq : 0;
    const int part = static_cast<int>(threadIdx.x & 3);
    float v[8];
    const float * src = x + row * x_stride + b * 32 + part * 8;
    if (vec4) {   // 16-byte aligned rows: two 16-byte loads per thread
        const float4 lo = live ? *reinterpret_cast<const float4 *>(src) : float4{0.0f, 0.0f, 0.0f, 0.0f};
        const float4 hi = live ? *reinterpret_cast<const float4 *>(src + 4) : float4{0.0f, 0.0f, 0.0f, 0.0f};
        v[0] = lo.x, v[1] = lo.y, v[2] = lo.z, v[3] = lo.w, v[4] = hi.x, v[5] = hi.y, v[6] = hi.z, v[7] = hi.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = live ? src[i] : 0.0f;
    }
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

__global__ __launch_bounds__(256) void gemm_rows_from_f32_kernel(const float * __restrict__ x, int vec4, int nb,
                                                                 int64_t x_stride, GemmRowLayout L, uint8_t * __restrict__ out) {
    gemm_rows_segment(x, vec4, nb, x_stride, L, out, blockIdx.x, static_cast<int>(blockIdx.y));
}

// The prefill's top-k + softmax (given logits; workgroups 0 .. ceil(T / 4) - 1, one wave per
// token) and its GEMM activation rows (the other workgroups, one per (row, 64-block segment)) in
// one launch: the two only share the launch.
template <int NPL>
__global__ __launch_bounds__(256) void topk_gemm_rows_kernel(const float * __restrict__ logits, int n_expert, int top_k,
                                                             int32_t * __restrict__ ids, float * __restrict__ weights,
                                                             int64_t n_tokens, int64_t topk_wgs, const float * __restrict__ x,
                                                             int vec4, int nb, int64_t x_stride, GemmRowLayout L,
                                                             int segments, uint8_t * __restrict__ out) {
    const int64_t b = blockIdx.x;
    if (b < topk_wgs) {
        const int64_t t = b * 4 + (threadIdx.x >> 6);
        if (t < n_tokens) wave_topk_softmax<NPL>(logits + t * n_expert, n_expert, top_k, ids + t * top_k, weights + t * top_k);
        return;
    }
    const int64_t r = b - topk_wgs;
    gemm_rows_segment(x, vec4, nb, x_stride, L, out, r / segments, static_cast<int>(r % segments));
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

template <int TYPE, int EPI, bool FLAGGED>
void launch_gemm_typed(const GemmArgs & a, int row_pairs, int max_tiles, hipStream_t stream) {
    GemmArgs b = a;
    b.row_pairs = row_pairs;
    const int64_t items = static_cast<int64_t>(row_pairs) * max_tiles;
    hipLaunchKernelGGL((grouped_gemm_kernel<TYPE, EPI, FLAGGED>), dim3(static_cast<unsigned>((items + 7) / 8 * 8)),
                       dim3(kGemmThreads), 0, stream, b);
    check_hip(hipGetLastError(), "grouped GEMM launch");
}

// ------------------------------------------------------------------ MXFP4 x MXFP8 experiment
// The CDNA4 block-scaled matrix core (v_mfma_scale_f32_16x16x128_f8f6f4) takes MXFP4 weights as
// they are stored (e2m1 codes, e8m0 exponents) and 8-bit activations with their own e8m0 block
// scales, applies both scales and accumulates four 32-element blocks per instruction: no
// per-block scale-accumulate work is left on the vector ALUs. Its activations must be an MX
// format, so this path quantizes them to MXFP8 (OCP MX e4m3, one e8m0 scale per 32 values)
// instead of the reference's Q8_0: a measured experiment beside the f16 MFMA path, outside the
// parity contract.
//
// Operand layout of one 128-element K step (blocks blk = 0..3), checked on the device:
//   A: lane row + 16 blk holds block blk of its row, element i at nibble i (low nibble first);
//      scale_a of that lane is the block's e8m0 exponent;
//   B: lane col + 16 g, byte j holds block g / 2 + 2 (j / 16), element 16 (g % 2) + j % 16;
//      scale_b of lane col + 16 blk is the block's e8m0 scale;
//   D: lane l holds column l % 16, rows 4 (l / 16) .. + 3.
// Products and block sums inside the instruction are not rounded as an fp32 chain would be (a
// random-data check puts the difference near 6e-5 of the sum of |products|).
typedef int mx_v8i __attribute__((ext_vector_type(8)));

// MXFP8 (e4m3) quantization of fp32 rows, one e8m0 scale X per 32 values: the smallest power of two
// with amax / X <= 448 (the e4m3 maximum), i.e. the OCP MX choice 2^(floor(log2 amax) - 8) raised
// by one when amax / 2^floor(log2 amax) > 1.75, so no value saturates; code = e4m3 of v / X
// rounded to nearest even; scale byte = 127 + log2 X. One thread per 4 values; the 8 threads of a
// block are adjacent lanes.
__device__ __forceinline__ uint32_t e4m3_rne(float v) {
    const uint32_t sign = __builtin_bit_cast(uint32_t, v) >> 31 << 7;
    float a = fabsf(v);
    a = a > 448.0f ? 448.0f : a;
    if (!(a >= 0.015625f)) {                                   // below 2^-6: subnormal steps of 2^-9
        const float m = rintf(a * 512.0f);                     // 0..8 (8 rounds up to the smallest normal)
        return sign | static_cast<uint32_t>(m);
    }
    const int e = static_cast<int>((__builtin_bit_cast(uint32_t, a) >> 23) & 0xFF) - 127;   // -6..8
    float m = rintf(__builtin_amdgcn_ldexpf(a, 3 - e));         // 8..16
    int ee = e;
    if (m >= 16.0f) { m = 8.0f; ++ee; }                        // carry into the next binade (<= 448 by the clamp)
    return sign | static_cast<uint32_t>((ee + 7) << 3) | (static_cast<uint32_t>(m) - 8u);
}

__global__ __launch_bounds__(256) void quantize_mxfp8_kernel(const float * __restrict__ x, int64_t n_rows, int nb,
                                                             int64_t x_stride, uint8_t * __restrict__ codes,
                                                             uint8_t * __restrict__ scales) {
    const int64_t t = blockIdx.x * 256ll + threadIdx.x;
    const bool live = t < n_rows * nb * 8;
    const int64_t blk = live ? t / 8 : 0;
    const int part = static_cast<int>(t & 7);
    const int64_t row = blk / nb, b = blk % nb;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = live ? x[row * x_stride + b * 32 + part * 4 + i] : 0.0f;
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const uint32_t ab = __builtin_bit_cast(uint32_t, amax);
    const int ea = ab >= 0x00800000u ? static_cast<int>(ab >> 23) - 127 : -127;   // subnormal or zero: X = 2^-127
    int sx = ea - 8 + (ab >= 0x00800000u && (ab & 0x7FFFFFu) > 0x600000u ? 1 : 0);
    sx = sx < -127 ? -127 : (sx > 127 ? 127 : sx);
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) packed |= e4m3_rne(__builtin_amdgcn_ldexpf(v[i], -sx)) << (8 * i);
    if (live) {
        reinterpret_cast<uint32_t *>(codes + row * nb * 32 + b * 32)[part] = packed;
        if (part == 0) scales[row * nb + b] = static_cast<uint8_t>(sx + 127);
    }
}

struct MxArgs {
    const uint8_t * bank;
    GemmShape shape;
    const int32_t * expert_to_slot;
    const uint8_t * codes;     // MXFP8 rows [n_rows][nb * 32]
    const uint8_t * scales;    // [n_rows][nb]
    int64_t n_ids, b_ne1;
    const int32_t * counts;
    const int32_t * offsets;
    const int32_t * jobs;
    const int32_t * tile_expert;
    const int32_t * tile_start;
    const int32_t * n_tiles;
    int row_pairs;
    float * dst;               // [job][rows]
};

// A workgroup (4 waves) computes 64 bank rows (a tile pair) x 64 jobs of one expert, like the f16
// path; wave w owns rows 32 (w & 1) .. + 31 and jobs 32 (w >> 1) .. + 31 as 2 x 2 fragments. Per
// bank group (8 blocks = two 128-element K steps) the tile pair's codes are restaged in LDS as
// [block][row][16 B], the operand order of the matrix core, and its exponents as [block][row]; the
// activation operands go from the MXFP8 rows straight into registers. The next group's loads
// (codes, exponents, activation operands) are in flight while the current group computes.
struct MxStage {
    uint32_t w[2][4];          // two (tile, slice, row) code entries: 8 blocks x 2 bytes each
    uint32_t m[2];             // threads 0..63: the row's 8 exponent bytes (stored as e - 128)
    u32x4g b[2][2][2];         // [K step][job half][low / high 16 bytes] activation operand
    int sb[2][2];              // [K step][job half] activation block scale
};

__global__ __launch_bounds__(256) void mx_gemm_kernel(MxArgs A) {
    __shared__ __attribute__((aligned(16))) uint8_t wl[8 * 64 * 16];
    __shared__ uint8_t el[8 * 64];
    const int n_items = *cst<int32_t>(A.n_tiles) * A.row_pairs;
    const int per_xcd = (n_items + 7) >> 3;
    const int slot8 = static_cast<int>(blockIdx.x >> 3);
    const int item = static_cast<int>(blockIdx.x & 7) * per_xcd + slot8;
    if (slot8 >= per_xcd || item >= n_items) return;
    const int ti = item / A.row_pairs;
    const int pair = item - ti * A.row_pairs;
    const int expert = cst<int32_t>(A.tile_expert)[ti];
    const int j0 = cst<int32_t>(A.tile_start)[ti];
    const int count = cst<int32_t>(A.counts)[expert];
    const int joff = cst<int32_t>(A.offsets)[expert];
    const int slot = A.expert_to_slot ? cst<int32_t>(A.expert_to_slot)[expert] : expert;
    const GemmShape S = A.shape;
    const int nb = S.nb, groups = nb / 8, tail = nb % 8;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
    const bool slot_ok = slot >= 0 && slot < S.n_slots;
    const uint8_t * slot_base = A.bank + static_cast<size_t>(slot_ok ? slot : 0) * S.slot_bytes;

    // this lane's two job columns
    const uint8_t * bcode[2];
    const uint8_t * bscale[2];
    int job[2];
    bool jlive[2];
#pragma unroll
    for (int jh = 0; jh < 2; ++jh) {
        const int jl = 32 * (wave >> 1) + 16 * jh + lr;
        jlive[jh] = j0 + jl < count;
        job[jh] = jlive[jh] ? A.jobs[joff + j0 + jl] : 0;
        const int64_t row_index = A.b_ne1 == 1 ? job[jh] / A.n_ids : job[jh];
        bcode[jh] = A.codes + row_index * nb * 32;
        bscale[jh] = A.scales + row_index * nb;
    }
    // this thread's two staging entries: e = t + 256 h -> tile tt, slice k, row r
    auto load = [&](int g, MxStage & R) {
        const bool is_tail = g == groups;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int e = threadIdx.x + 256 * h;
            const int tile = pair * 2 + (e >> 8), k = (e >> 5) & 7, r = e & 31;
#pragma unroll
            for (int d = 0; d < 4; ++d) R.w[h][d] = 0u;
            if (tile * 32 < S.rows) {
                const uint8_t * ct = slot_base + static_cast<size_t>(tile) * 32 * nb * 16;
                if (!is_tail) {
                    const u32x4g v = *reinterpret_cast<const u32x4g *>(ct + static_cast<size_t>(g) * 4096 + (k * 32 + r) * 16);
                    R.w[h][0] = v[0], R.w[h][1] = v[1], R.w[h][2] = v[2], R.w[h][3] = v[3];
                } else {
                    const uint8_t * tp = ct + static_cast<size_t>(groups) * 4096 + (k * 32 + r) * (tail * 2);
#pragma unroll
                    for (int b = 0; b < 8; ++b)       // constant indices keep the stage in registers
                        if (b < tail)
                            R.w[h][b >> 1] |= static_cast<uint32_t>(*reinterpret_cast<const uint16_t *>(tp + 2 * b)) << (16 * (b & 1));
                }
            }
        }
        R.m[0] = R.m[1] = 0x80808080u;                         // blocks past the tail: 2^0
        if (threadIdx.x < 64) {
            const int row = threadIdx.x, tile = pair * 2 + (row >> 5), r = row & 31;
            if (tile * 32 < S.rows) {
                const uint8_t * mt = slot_base + S.codes_bytes + static_cast<size_t>(tile) * 32 * nb;
                if (!is_tail) {
                    const u32x2g v = *reinterpret_cast<const u32x2g *>(mt + static_cast<size_t>(g) * 256 + r * 8);
                    R.m[0] = v[0], R.m[1] = v[1];
                } else {
#pragma unroll
                    for (int b = 0; b < 8; ++b) {
                        if (b < tail) {
                            const uint32_t byte = mt[groups * 256 + r * tail + b];
                            R.m[b >> 2] = (R.m[b >> 2] & ~(0xFFu << (8 * (b & 3)))) | (byte << (8 * (b & 3)));
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            const int b0 = 8 * g + 4 * st, blo = b0 + (q >> 1), bhi = b0 + 2 + (q >> 1);
#pragma unroll
            for (int jh = 0; jh < 2; ++jh) {
                R.b[st][jh][0] = R.b[st][jh][1] = u32x4g{0u, 0u, 0u, 0u};
                if (jlive[jh] && blo < nb) R.b[st][jh][0] = *reinterpret_cast<const u32x4g *>(bcode[jh] + blo * 32 + 16 * (q & 1));
                if (jlive[jh] && bhi < nb) R.b[st][jh][1] = *reinterpret_cast<const u32x4g *>(bcode[jh] + bhi * 32 + 16 * (q & 1));
                R.sb[st][jh] = jlive[jh] && b0 + q < nb ? bscale[jh][b0 + q] : 127;
            }
        }
    };
    auto stage = [&](const MxStage & R) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int e = threadIdx.x + 256 * h;
            const int row = 32 * (e >> 8) + (e & 31), k = (e >> 5) & 7;
#pragma unroll
            for (int b = 0; b < 8; ++b)
                *reinterpret_cast<uint16_t *>(wl + (b * 64 + row) * 16 + 2 * k) = static_cast<uint16_t>(R.w[h][b >> 1] >> (16 * (b & 1)));
        }
        if (threadIdx.x < 64) {
#pragma unroll
            for (int b = 0; b < 8; ++b) el[b * 64 + threadIdx.x] = static_cast<uint8_t>((R.m[b >> 2] >> (8 * (b & 3))) ^ 0x80u);
        }
    };
    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jh = 0; jh < 2; ++jh) acc[i][jh] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int n_groups = groups + (tail > 0 ? 1 : 0);
    MxStage cur, nxt;
    load(0, cur);
    stage(cur);
    __syncthreads();
    for (int g = 0; g < n_groups; ++g) {
        if (g + 1 < n_groups) load(g + 1, nxt);
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            if (8 * g + 4 * st >= nb) break;
            mx_v8i bop[2];
#pragma unroll
            for (int jh = 0; jh < 2; ++jh) {
                const u32x4g lo = cur.b[st][jh][0], hi = cur.b[st][jh][1];
                bop[jh] = mx_v8i{static_cast<int>(lo[0]), static_cast<int>(lo[1]), static_cast<int>(lo[2]), static_cast<int>(lo[3]),
                                 static_cast<int>(hi[0]), static_cast<int>(hi[1]), static_cast<int>(hi[2]), static_cast<int>(hi[3])};
            }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int row = 32 * (wave & 1) + 16 * i + lr;
                const u32x4g a = *reinterpret_cast<const u32x4g *>(wl + ((4 * st + q) * 64 + row) * 16);
                const mx_v8i aop = mx_v8i{static_cast<int>(a[0]), static_cast<int>(a[1]), static_cast<int>(a[2]), static_cast<int>(a[3]), 0, 0, 0, 0};
                const int sa = el[(4 * st + q) * 64 + row];
#pragma unroll
                for (int jh = 0; jh < 2; ++jh)
                    acc[i][jh] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(aop, bop[jh], acc[i][jh], 4, 0, 0, sa, 0, cur.sb[st][jh]);
            }
        }
        __syncthreads();
        if (g + 1 < n_groups) {
            stage(nxt);
            cur = nxt;
        }
        __syncthreads();
    }
    const float nan = __builtin_nanf("");
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jh = 0; jh < 2; ++jh) {
            if (!jlive[jh]) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t brow = static_cast<int64_t>(pair) * 64 + 32 * (wave & 1) + 16 * i + 4 * q + j;
                if (brow < S.rows)
                    A.dst[static_cast<size_t>(job[jh]) * S.rows + ggml_row(brow, S.rows, S.interleave)] = slot_ok ? acc[i][jh][j] : nan;
            }
        }
}

}  // namespace

void launch_job_tiles(const GroupBuffers & g, const int32_t * filter, int job_tile, int64_t max_tiles,
                      int32_t * tile_expert, int32_t * tile_start, int32_t * n_tiles, hipStream_t stream) {
    require(job_tile >= 1 && max_tiles >= 1 && max_tiles < (1ll << 31), "job tile list shape out of range");
    hipLaunchKernelGGL(gemm_tiles_kernel, dim3(1), dim3(1024), 0, stream, g.counts, g.active, g.n_active, filter, job_tile,
                       static_cast<int>(max_tiles), tile_expert, tile_start, n_tiles, g.error);
    check_hip(hipGetLastError(), "job tile list launch");
}

int64_t gemm_max_tiles(int64_t n_as, int64_t n_entries, int job_tile) {
    return (n_entries + job_tile - 1) / job_tile + (n_as < n_entries ? n_as : n_entries);
}

// sized for the smaller job tile of the two kernels that share it
size_t gemm_tiles_bytes(int64_t n_as, int64_t n_entries) {
    return static_cast<size_t>((2 * gemm_max_tiles(n_as, n_entries, kMxJobTile) + 8) * sizeof(int32_t));
}

void launch_gemm_rows_from_f32(const float * x, int64_t n_rows, int64_t k, int64_t x_stride, const GemmRowLayout & lay,
                               uint8_t * rows, hipStream_t stream) {
    require(k > 0 && k % 32 == 0 && n_rows > 0 && x_stride >= k && lay.nb == k / 32, "GEMM quantize shape mismatch");
    require(n_rows < (1ll << 31), "too many GEMM activation rows for one launch");
    const unsigned segments = static_cast<unsigned>((k / 32 + 63) / 64);
    const int vec4 = reinterpret_cast<uintptr_t>(x) % 16 == 0 && x_stride % 4 == 0;
    hipLaunchKernelGGL(gemm_rows_from_f32_kernel, dim3(static_cast<unsigned>(n_rows), segments), dim3(256), 0, stream,
                       x, vec4, static_cast<int>(k / 32), x_stride, lay, rows);
    check_hip(hipGetLastError(), "GEMM quantize launch");
}

void launch_topk_gemm_rows(const float * logits, int64_t n_expert, int64_t top_k, int32_t * ids, float * weights,
                           const float * x, int64_t n_rows, int64_t k, const GemmRowLayout & lay, uint8_t * rows,
                           hipStream_t stream) {
    require(k > 0 && k % 32 == 0 && n_rows > 0 && lay.nb == k / 32, "GEMM quantize shape mismatch");
    require(n_expert > 0 && n_expert <= 1024 && top_k > 0 && top_k <= n_expert && top_k <= 64,
            "router supports 1..1024 experts and top_k <= 64");
    const int segments = static_cast<int>((k / 32 + 63) / 64);
    const int64_t topk_wgs = (n_rows + 3) / 4, total = topk_wgs + n_rows * segments;
    require(total < (1ll << 31), "too many GEMM activation rows for one launch");
    const int vec4 = reinterpret_cast<uintptr_t>(x) % 16 == 0 && k % 4 == 0;
    const int ne = static_cast<int>(n_expert), tk = static_cast<int>(top_k), nb = static_cast<int>(k / 32);
    const dim3 grid(static_cast<unsigned>(total));
    if (n_expert <= 128)
        hipLaunchKernelGGL(topk_gemm_rows_kernel<2>, grid, dim3(256), 0, stream, logits, ne, tk, ids, weights, n_rows, topk_wgs,
                           x, vec4, nb, k, lay, segments, rows);
    else if (n_expert <= 256)
        hipLaunchKernelGGL(topk_gemm_rows_kernel<4>, grid, dim3(256), 0, stream, logits, ne, tk, ids, weights, n_rows, topk_wgs,
                           x, vec4, nb, k, lay, segments, rows);
    else
        hipLaunchKernelGGL(topk_gemm_rows_kernel<16>, grid, dim3(256), 0, stream, logits, ne, tk, ids, weights, n_rows,
                           topk_wgs, x, vec4, nb, k, lay, segments, rows);
    check_hip(hipGetLastError(), "top-k + GEMM rows launch");
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
    const int job_tile_n = gemm_job_tile(bank.type);
    const int64_t max_tiles = gemm_max_tiles(p.n_as, p.n_entries, job_tile_n);
    require(max_tiles <= 65535, "too many GEMM tiles for one launch");
    int32_t * tile_expert = static_cast<int32_t *>(p.tiles);
    int32_t * tile_start = tile_expert + max_tiles;
    int32_t * n_tiles = tile_start + max_tiles;
    if (!p.tiles_ready) {
        hipLaunchKernelGGL(gemm_tiles_kernel, dim3(1), dim3(1024), 0, stream, p.group.counts, p.group.active,
                           p.group.n_active, p.tile_filter, job_tile_n, static_cast<int>(max_tiles), tile_expert, tile_start,
                           n_tiles, p.group.error);
        check_hip(hipGetLastError(), "GEMM tile list launch");
    }
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
    a.row_scale = p.row_scale;
    a.dst = p.dst;
    a.dst_vec4 = p.dst != nullptr && reinterpret_cast<uintptr_t>(p.dst) % 16 == 0 && bank.rows % 4 == 0;
    a.rows_out = p.rows_out;
    a.out_lay = p.out_layout;
    a.activation = p.activation;
    a.alpha = p.alpha;
    a.limit = p.limit;
    const int row_pairs = static_cast<int>((bank.rows + 63) / 64);
    require(!p.flagged_rows || p.epilogue == 0, "flagged activation rows only with the plain epilogue");
    // the launch covers max_tiles tiles, or the caller's bound on this call's tiles (its tile filter
    // leaves only the experts whose tiles it counted)
    require(p.grid_tiles >= 0 && (p.grid_tiles == 0 || p.tile_filter != nullptr), "grid tile bound needs a tile filter");
    const int mt = static_cast<int>(p.grid_tiles > 0 ? std::min<int64_t>(p.grid_tiles, max_tiles) : max_tiles);
    if (bank.type == VBM_TYPE_MXFP4) {
        if (p.flagged_rows) launch_gemm_typed<39, 0, true>(a, row_pairs, mt, stream);
        else if (p.epilogue == 0) launch_gemm_typed<39, 0, false>(a, row_pairs, mt, stream);
        else launch_gemm_typed<39, 1, false>(a, row_pairs, mt, stream);
    } else {
        if (p.flagged_rows) launch_gemm_typed<8, 0, true>(a, row_pairs, mt, stream);
        else if (p.epilogue == 0) launch_gemm_typed<8, 0, false>(a, row_pairs, mt, stream);
        else launch_gemm_typed<8, 1, false>(a, row_pairs, mt, stream);
    }
}

void launch_quantize_mxfp8(const float * x, int64_t n_rows, int64_t k, int64_t x_stride, uint8_t * codes, uint8_t * scales,
                           hipStream_t stream) {
    require(k > 0 && k % 32 == 0 && n_rows > 0 && x_stride >= k, "MXFP8 quantize shape mismatch");
    const int64_t threads = n_rows * (k / 32) * 8;
    hipLaunchKernelGGL(quantize_mxfp8_kernel, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0, stream, x,
                       n_rows, static_cast<int>(k / 32), x_stride, codes, scales);
    check_hip(hipGetLastError(), "MXFP8 quantize launch");
}

void launch_mx_gemm(const vbm_bank & bank, const int32_t * expert_to_slot, const uint8_t * codes, const uint8_t * scales,
                    int64_t n_ids, int64_t b_ne1, int64_t n_as, int64_t n_entries, const GroupBuffers & group, void * tiles,
                    float * dst, hipStream_t stream) {
    require(bank.type == VBM_TYPE_MXFP4, "the MXFP8 experiment runs on MXFP4 banks");
    require(n_as >= 1 && n_as <= 1024 && n_entries >= 1, "GEMM group shape out of range");
    const int64_t max_tiles = gemm_max_tiles(n_as, n_entries, kMxJobTile);
    require(max_tiles <= 65535, "too many GEMM tiles for one launch");
    int32_t * tile_expert = static_cast<int32_t *>(tiles);
    int32_t * tile_start = tile_expert + max_tiles;
    int32_t * n_tiles = tile_start + max_tiles;
    hipLaunchKernelGGL(gemm_tiles_kernel, dim3(1), dim3(1024), 0, stream, group.counts, group.active, group.n_active,
                       nullptr, kMxJobTile, static_cast<int>(max_tiles), tile_expert, tile_start, n_tiles, group.error);
    check_hip(hipGetLastError(), "GEMM tile list launch");
    MxArgs a{};
    a.bank = bank.base;
    a.shape = GemmShape{static_cast<int>(bank.nb), static_cast<int>(bank.rows), bank.interleave, bank.slot_bytes,
                        bank.geometry().codes_bytes(), bank.n_slots};
    a.expert_to_slot = expert_to_slot;
    a.codes = codes;
    a.scales = scales;
    a.n_ids = n_ids;
    a.b_ne1 = b_ne1;
    a.counts = group.counts;
    a.offsets = group.offsets;
    a.jobs = group.rows;
    a.tile_expert = tile_expert;
    a.tile_start = tile_start;
    a.n_tiles = n_tiles;
    a.row_pairs = static_cast<int>((bank.rows + 63) / 64);
    a.dst = dst;
    const int64_t items = static_cast<int64_t>(a.row_pairs) * max_tiles;
    hipLaunchKernelGGL(mx_gemm_kernel, dim3(static_cast<unsigned>((items + 7) / 8 * 8)), dim3(256), 0, stream, a);
    check_hip(hipGetLastError(), "MXFP8 GEMM launch");
}

}  // namespace vbm
