// Host check of the expert bank layout: for every supported geometry the per-block byte
// positions (codes + exponents/scales) cover [0, slot_bytes) exactly once, and scatter followed
// by gather returns the original ggml bytes. The device kernels use the same functions, so this
// bounds every device-side store before any kernel runs.
#include "vbm_common.hpp"

#include <cstdio>
#include <cstring>
#include <vector>

using namespace vbm;

static int check(int type, int64_t rows, int64_t k, int interleave) {
    const SlotGeometry g{rows, k / 32, type};
    const int64_t slot = g.slot_bytes();
    std::vector<int> hits(static_cast<size_t>(slot), 0);
    for (int64_t d = 0; d < rows; ++d)
        for (int64_t b = 0; b < g.nb; ++b) {
            if (type == 39) {
                for (int s = 0; s < kSlices; ++s) {
                    const int64_t o = mx_code_offset(g, d, b, s);
                    if (o < 0 || o + 2 > g.codes_bytes()) { std::printf("code offset out of range\n"); return 1; }
                    hits[o]++; hits[o + 1]++;
                }
                const int64_t e = mx_exp_offset(g, d, b);
                if (e < g.codes_bytes() || e >= slot) { std::printf("exp offset out of range\n"); return 1; }
                hits[e]++;
            } else {
                for (int s = 0; s < kSlices; ++s) {
                    const int64_t o = q8_code_offset(g, d, b, s);
                    if (o < 0 || o + 4 > g.codes_bytes()) { std::printf("q8 code offset out of range\n"); return 1; }
                    for (int i = 0; i < 4; ++i) hits[o + i]++;
                }
                const int64_t e = q8_scale_offset(g, d, b);
                if (e < g.codes_bytes() || e + 2 > slot) { std::printf("scale offset out of range\n"); return 1; }
                hits[e]++; hits[e + 1]++;
            }
        }
    for (int64_t i = 0; i < slot; ++i)
        if (hits[i] != 1) { std::printf("byte %lld hit %d times\n", (long long)i, hits[i]); return 1; }
    // device_row is a bijection on [0, rows)
    std::vector<int> rowhits(static_cast<size_t>(rows), 0);
    for (int64_t i = 0; i < rows; ++i) {
        const int64_t d = device_row(i, rows, interleave);
        if (d < 0 || d >= rows || ggml_row(d, rows, interleave) != i) { std::printf("row map broken\n"); return 1; }
        rowhits[d]++;
    }
    for (int h : rowhits) if (h != 1) { std::printf("row map not bijective\n"); return 1; }
    // scatter / gather round trip
    const int bb = type == 39 ? kMxfp4BlockBytes : kQ8BlockBytes;
    std::vector<uint8_t> src(static_cast<size_t>(slot)), bank(static_cast<size_t>(slot)), back(static_cast<size_t>(slot));
    uint64_t key = stream_key(7, static_cast<uint64_t>(type * 1000 + rows));
    for (int64_t i = 0; i < slot; ++i) src[i] = static_cast<uint8_t>(hash_at(key, i));
    for (int64_t i = 0; i < rows; ++i)
        for (int64_t b = 0; b < g.nb; ++b) {
            const uint8_t * blk = src.data() + (i * g.nb + b) * bb;
            const int64_t d = device_row(i, rows, interleave);
            if (type == 39) mx_store_block(bank.data(), g, d, b, blk); else q8_store_block(bank.data(), g, d, b, blk);
        }
    for (int64_t i = 0; i < rows; ++i)
        for (int64_t b = 0; b < g.nb; ++b) {
            uint8_t * blk = back.data() + (i * g.nb + b) * bb;
            const int64_t d = device_row(i, rows, interleave);
            if (type == 39) mx_load_block(bank.data(), g, d, b, blk); else q8_load_block(bank.data(), g, d, b, blk);
        }
    if (std::memcmp(src.data(), back.data(), static_cast<size_t>(slot)) != 0) { std::printf("round trip differs\n"); return 1; }
    return 0;
}

int main() {
    struct Case { int type; int64_t rows, k; int interleave; } cases[] = {
        {39, 32, 64, 0}, {39, 32, 128, 1}, {39, 64, 192, 0}, {39, 96, 320, 1}, {39, 64, 448, 0}, {39, 32, 256, 0},
        {39, 5760, 2880, 1}, {39, 2880, 2880, 0}, {8, 32, 64, 0}, {8, 64, 192, 0}, {8, 32, 96 * 2, 1},
        {8, 1536, 2048, 1}, {8, 2048, 768, 0}, {8, 768, 2048, 0}, {39, 128, 2048, 0}, {39, 2048, 768, 0},
    };
    for (const auto & c : cases) {
        if (check(c.type, c.rows, c.k, c.interleave)) {
            std::printf("FAILED type=%d rows=%lld k=%lld interleave=%d\n", c.type, (long long)c.rows, (long long)c.k, c.interleave);
            return 1;
        }
    }
    // fp16 conversion: exhaustive half -> float -> half round trip.
    for (uint32_t h = 0; h < 65536; ++h) {
        const float f = half_bits_to_float(static_cast<uint16_t>(h));
        const uint16_t back = float_to_half_bits(f);
        const bool nan = ((h >> 10) & 31) == 31 && (h & 1023);
        if (!nan && back != h) { std::printf("fp16 round trip failed at %u\n", h); return 1; }
    }
    std::printf("bank layout bijective and lossless for %zu geometries; fp16 round trip exact\n", sizeof(cases) / sizeof(cases[0]));
    return 0;
}
