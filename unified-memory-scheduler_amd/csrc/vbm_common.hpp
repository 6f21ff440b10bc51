// Shared host/device helpers: counter-based generator, fp16 conversion, bank tile layout.
// Everything here is plain integer / IEEE arithmetic so host and device agree bit for bit.
#pragma once

#include <cstddef>
#include <cstdint>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define VBM_HD __host__ __device__ __forceinline__
#else
#define VBM_HD inline
#endif

namespace vbm {

// ggml block sizes (ggml-common.h): block_mxfp4 {u8 e; u8 qs[16]}, block_q8_0 {f16 d; i8 qs[32]}.
constexpr int kBlock = 32;
constexpr int kMxfp4BlockBytes = 17;
constexpr int kQ8BlockBytes = 34;
constexpr int kTileRows = 32;          // rows per bank tile (one workgroup's output rows)
constexpr int kSlices = 8;             // 4-element lanes of the x86 vec_dot contract
constexpr int kMxGroup = 8;            // MXFP4 blocks per 16-byte lane load (8 x 2 bytes)
constexpr int kQ8Group = 4;            // Q8_0 blocks per 16-byte lane load (4 x 4 bytes)

// ---------------------------------------------------------------- counter-based generator
VBM_HD uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
VBM_HD uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return mix64(seed * 0x9E3779B97F4A7C15ULL ^ mix64(stream + 0x632BE59BD9B4E019ULL));
}
VBM_HD uint64_t hash_at(uint64_t key, uint64_t index) {
    return mix64(key + (index + 1) * 0xD1B54A32D192ED03ULL);
}

// One synthetic MXFP4 block (ggml layout) at global block index `j` of a tensor.
VBM_HD void synth_mxfp4_block(uint64_t key, uint64_t j, int exp_lo, int exp_hi, uint8_t out[17]) {
    const uint64_t h0 = hash_at(key, 3 * j), h1 = hash_at(key, 3 * j + 1), h2 = hash_at(key, 3 * j + 2);
    const uint64_t span = static_cast<uint64_t>(exp_hi - exp_lo + 1);
    out[0] = static_cast<uint8_t>(127 + exp_lo + static_cast<int>(h2 % span));
    for (int i = 0; i < 8; ++i) {
        out[1 + i] = static_cast<uint8_t>(h0 >> (8 * i));
        out[9 + i] = static_cast<uint8_t>(h1 >> (8 * i));
    }
}

// ---------------------------------------------------------------- fp16 (IEEE binary16)
VBM_HD float half_bits_to_float(uint16_t h) {
#if defined(__HIP_DEVICE_COMPILE__)
    return static_cast<float>(__builtin_bit_cast(_Float16, h));   // v_cvt_f32_f16, exact
#else
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    uint32_t exponent = (h >> 10) & 0x1Fu, mantissa = h & 0x3FFu, bits;
    if (exponent == 0x1F) {
        bits = sign | 0x7F800000u | (mantissa << 13);
    } else if (exponent != 0) {
        bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    } else if (mantissa == 0) {
        bits = sign;
    } else {  // subnormal: normalise
        int shift = 0;
        while ((mantissa & 0x400u) == 0) { mantissa <<= 1; ++shift; }
        bits = sign | ((113u - static_cast<uint32_t>(shift)) << 23) | ((mantissa & 0x3FFu) << 13);
    }
    float f;
    __builtin_memcpy(&f, &bits, 4);
    return f;
#endif
}

// Round-to-nearest-even float -> binary16 (the F16C _cvtss_sh(x, 0) result).
VBM_HD uint16_t float_to_half_bits(float f) {
    uint32_t x;
    __builtin_memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t abs = x & 0x7FFFFFFFu;
    if (abs >= 0x7F800000u) return static_cast<uint16_t>(sign | 0x7C00u | (abs > 0x7F800000u ? 0x200u : 0u));
    if (abs >= 0x477FF000u) return static_cast<uint16_t>(sign | 0x7C00u);  // rounds to >= 65520: inf
    if (abs < 0x38800000u) {                                               // result subnormal or zero
        if (abs < 0x33000000u) return static_cast<uint16_t>(sign);         // < 2^-25: rounds to 0
        const uint32_t exponent = abs >> 23;
        const uint32_t mantissa = (abs & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - exponent;                            // 14..24 for 2^-25..2^-14
        const uint32_t kept = mantissa >> shift;
        const uint32_t rest = mantissa & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        const uint32_t rounded = kept + ((rest > half || (rest == half && (kept & 1u))) ? 1u : 0u);
        return static_cast<uint16_t>(sign | rounded);
    }
    const uint32_t rounded = abs + 0xFFFu + ((abs >> 13) & 1u);
    return static_cast<uint16_t>(sign | ((rounded - 0x38000000u) >> 13));
}

// One synthetic Q8_0 block (ggml layout) at global block index `j`: codes uniform in
// [-127, 127], scale fp16_rn(lo + (hi - lo) * u) with u uniform in [0, 1).
VBM_HD void synth_q8_block(uint64_t key, uint64_t j, float lo, float hi, uint8_t out[34]) {
    for (int w = 0; w < 4; ++w) {
        const uint64_t h = hash_at(key, 5 * j + w);
        for (int b = 0; b < 8; ++b) {
            const uint32_t byte = static_cast<uint32_t>((h >> (8 * b)) & 0xFF);
            out[2 + 8 * w + b] = static_cast<uint8_t>(static_cast<int>((byte * 255u) >> 8) - 127);
        }
    }
    const double u = static_cast<double>(hash_at(key, 5 * j + 4) >> 11) * 0x1.0p-53;
    const uint16_t d = float_to_half_bits(static_cast<float>(static_cast<double>(lo) + (static_cast<double>(hi) - lo) * u));
    out[0] = static_cast<uint8_t>(d & 0xFF);
    out[1] = static_cast<uint8_t>(d >> 8);
}

// ---------------------------------------------------------------- bank tile layout
// A slot holds one expert matrix of `rows` x `nb` blocks. Rows are grouped in 32-row tiles.
// MXFP4: codes region (rows*nb*16 B) then exponent region (rows*nb B).
//   Lane slice k of a block = elements 4k..4k+3 packed in 2 bytes (element 4k+2i in the low
//   nibble of byte i, 4k+2i+1 in its high nibble). For a tile, blocks go in groups of 8; the
//   16 bytes of (group g, slice k, row r) are that lane's slices of the 8 blocks, so a
//   workgroup thread (k, r) issues one 16-byte load per group and the tile's 256 threads read
//   4 KiB contiguously. Blocks past the last full group (nb % 8) follow, 2 bytes per block.
//   Exponents: (group g, row r) -> 8 bytes, then the tail; stored as e ^ 0x80 (= e - 128).
// Q8_0: codes region (rows*nb*32 B) then scale region (rows*nb*2 B); slices of 4 bytes,
//   groups of 4 blocks; scales (group g, row r) -> 4 x fp16, then the tail.
struct SlotGeometry {
    int64_t rows, nb;
    int type;  // 39 = MXFP4, 8 = Q8_0
    VBM_HD int64_t codes_bytes() const { return rows * nb * (type == 39 ? 16 : 32); }
    VBM_HD int64_t slot_bytes() const { return rows * nb * (type == 39 ? 17 : 34); }
};

// Device row of ggml row `i` (interleave: gate rows [0, half) and up rows [half, 2*half) of a
// fused gate_up expert share tiles, 16 + 16 rows per tile).
VBM_HD int64_t device_row(int64_t i, int64_t rows, int interleave) {
    if (!interleave) return i;
    const int64_t half = rows / 2;
    const bool up = i >= half;
    const int64_t j = up ? i - half : i;
    return (j / 16) * kTileRows + (up ? 16 : 0) + (j % 16);
}
VBM_HD int64_t ggml_row(int64_t d, int64_t rows, int interleave) {
    if (!interleave) return d;
    const int64_t half = rows / 2;
    const int64_t tile = d / kTileRows, r = d % kTileRows;
    return (r >= 16 ? half : 0) + tile * 16 + (r % 16);
}

// Byte offset, within a slot, of slice `k` of block `b` of device row `d` (MXFP4: 2 bytes).
VBM_HD int64_t mx_code_offset(const SlotGeometry & g, int64_t d, int64_t b, int k) {
    const int64_t tile = d / kTileRows, r = d % kTileRows;
    const int64_t groups = g.nb / kMxGroup, tail = g.nb % kMxGroup;
    const int64_t base = tile * kTileRows * g.nb * 16;
    if (b < groups * kMxGroup)
        return base + (b / kMxGroup) * 4096 + (static_cast<int64_t>(k) * kTileRows + r) * 16 + (b % kMxGroup) * 2;
    return base + groups * 4096 + (static_cast<int64_t>(k) * kTileRows + r) * (tail * 2) + (b - groups * kMxGroup) * 2;
}
VBM_HD int64_t mx_exp_offset(const SlotGeometry & g, int64_t d, int64_t b) {
    const int64_t tile = d / kTileRows, r = d % kTileRows;
    const int64_t groups = g.nb / kMxGroup, tail = g.nb % kMxGroup;
    const int64_t base = g.codes_bytes() + tile * kTileRows * g.nb;
    if (b < groups * kMxGroup) return base + (b / kMxGroup) * 256 + r * 8 + (b % kMxGroup);
    return base + groups * 256 + r * tail + (b - groups * kMxGroup);
}
VBM_HD int64_t q8_code_offset(const SlotGeometry & g, int64_t d, int64_t b, int k) {
    const int64_t tile = d / kTileRows, r = d % kTileRows;
    const int64_t groups = g.nb / kQ8Group, tail = g.nb % kQ8Group;
    const int64_t base = tile * kTileRows * g.nb * 32;
    if (b < groups * kQ8Group)
        return base + (b / kQ8Group) * 4096 + (static_cast<int64_t>(k) * kTileRows + r) * 16 + (b % kQ8Group) * 4;
    return base + groups * 4096 + (static_cast<int64_t>(k) * kTileRows + r) * (tail * 4) + (b - groups * kQ8Group) * 4;
}
VBM_HD int64_t q8_scale_offset(const SlotGeometry & g, int64_t d, int64_t b) {
    const int64_t tile = d / kTileRows, r = d % kTileRows;
    const int64_t groups = g.nb / kQ8Group, tail = g.nb % kQ8Group;
    const int64_t base = g.codes_bytes() + tile * kTileRows * g.nb * 2;
    if (b < groups * kQ8Group) return base + (b / kQ8Group) * 256 + r * 8 + (b % kQ8Group) * 2;
    return base + groups * 256 + r * tail * 2 + (b - groups * kQ8Group) * 2;
}

// ggml MXFP4 element i of a block (i < 16: low nibble of qs[i]; else high nibble of qs[i-16]).
VBM_HD uint8_t mx_nibble(const uint8_t * qs, int i) {
    return i < 16 ? (qs[i] & 0x0F) : (qs[i - 16] >> 4);
}

// Scatter one ggml block (at ggml row i, block b) into its bank positions.
VBM_HD void mx_store_block(uint8_t * slot, const SlotGeometry & g, int64_t d, int64_t b, const uint8_t * blk) {
    const uint8_t * qs = blk + 1;
    for (int k = 0; k < kSlices; ++k) {
        const int64_t o = mx_code_offset(g, d, b, k);
        slot[o] = static_cast<uint8_t>(mx_nibble(qs, 4 * k) | (mx_nibble(qs, 4 * k + 1) << 4));
        slot[o + 1] = static_cast<uint8_t>(mx_nibble(qs, 4 * k + 2) | (mx_nibble(qs, 4 * k + 3) << 4));
    }
    slot[mx_exp_offset(g, d, b)] = static_cast<uint8_t>(blk[0] ^ 0x80);
}
VBM_HD void mx_load_block(const uint8_t * slot, const SlotGeometry & g, int64_t d, int64_t b, uint8_t * blk) {
    uint8_t e[32];
    for (int k = 0; k < kSlices; ++k) {
        const int64_t o = mx_code_offset(g, d, b, k);
        e[4 * k] = slot[o] & 0x0F; e[4 * k + 1] = slot[o] >> 4;
        e[4 * k + 2] = slot[o + 1] & 0x0F; e[4 * k + 3] = slot[o + 1] >> 4;
    }
    blk[0] = static_cast<uint8_t>(slot[mx_exp_offset(g, d, b)] ^ 0x80);
    for (int i = 0; i < 16; ++i) blk[1 + i] = static_cast<uint8_t>(e[i] | (e[i + 16] << 4));
}
VBM_HD void q8_store_block(uint8_t * slot, const SlotGeometry & g, int64_t d, int64_t b, const uint8_t * blk) {
    for (int k = 0; k < kSlices; ++k) {
        const int64_t o = q8_code_offset(g, d, b, k);
        for (int i = 0; i < 4; ++i) slot[o + i] = blk[2 + 4 * k + i];
    }
    const int64_t s = q8_scale_offset(g, d, b);
    slot[s] = blk[0]; slot[s + 1] = blk[1];
}
VBM_HD void q8_load_block(const uint8_t * slot, const SlotGeometry & g, int64_t d, int64_t b, uint8_t * blk) {
    for (int k = 0; k < kSlices; ++k) {
        const int64_t o = q8_code_offset(g, d, b, k);
        for (int i = 0; i < 4; ++i) blk[2 + 4 * k + i] = slot[o + i];
    }
    const int64_t s = q8_scale_offset(g, d, b);
    blk[0] = slot[s]; blk[1] = slot[s + 1];
}

}  // namespace vbm
