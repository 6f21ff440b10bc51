/*
 * vbm_oracle.c — CPU oracle for the routed-expert MoE path. TEST INFRASTRUCTURE ONLY
 * (see vbm_oracle.h). Paths cited are relative to the reference repository root;
 * "HP:n" = third_party/patches/llama-b11669-hybrid-experts.patch line n,
 * "PARP:n" = third_party/patches/llama-b11669-mxfp4-q8-parity-experimental.patch line n.
 */
#include "vbm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#endif
#ifdef _OPENMP
#include <omp.h>
#endif

int orc_abi_version(void) { return 1; }

/* ------------------------------------------------------------------ fp16 / e8m0 */
float orc_fp16_to_fp32(uint16_t h) {
    const int sign = (h >> 15) & 1, exponent = (h >> 10) & 31, mantissa = h & 1023;
    float value;
    if (exponent == 0) value = ldexpf((float)mantissa, -24);
    else if (exponent == 31) value = mantissa ? NAN : INFINITY;
    else value = ldexpf((float)(mantissa | 1024), exponent - 25);
    return sign ? -value : value;
}

/* Round to nearest even, as F16C _cvtss_sh(x, 0) (GGML_CPU_FP32_TO_FP16 on x86). */
uint16_t orc_fp32_to_fp16(float f) {
    uint16_t sign = signbit(f) ? 0x8000 : 0;
    float a = fabsf(f);
    if (isnan(f)) return (uint16_t)(sign | 0x7E00);
    if (a >= 65520.0f) return (uint16_t)(sign | 0x7C00);
    int e;
    (void)frexpf(a, &e);                      /* a = m * 2^e, m in [0.5, 1) */
    int unit_exp = e - 11;                    /* ulp of an 11-bit significand */
    if (unit_exp < -24) unit_exp = -24;       /* subnormal ulp 2^-24 */
    const double scaled = ldexp((double)a, -unit_exp);   /* exact: a has 24 bits */
    double q = nearbyint(scaled);             /* default rounding mode: nearest even */
    const double total = ldexp(q, unit_exp);
    if (total == 0.0) return sign;
    int te;
    (void)frexp(total, &te);
    if (te - 1 < -14) return (uint16_t)(sign | (uint16_t)q);          /* subnormal */
    const int biased = te - 1 + 15;
    const uint32_t mant = (uint32_t)(ldexp(total, -(te - 1)) * 1024.0) - 1024u;
    return (uint16_t)(sign | (biased << 10) | mant);
}

/* GGML_E8M0_TO_FP32_HALF: tools/trace/cpu_mxfp4_vnni.cpp:22-24; tools/engine/quantized_cuda.cu:159-163. */
float orc_e8m0_half(uint8_t e) {
    uint32_t bits = e < 2 ? (0x00200000u << e) : ((uint32_t)(e - 1) << 23);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* ------------------------------------------------------------------ Q8_0 quantizer */
/* x86 quantize_row_q8_0 contract: PARP:41-44 (code = RNE(x * (127/amax)), 0 when amax == 0)
 * and PARP:95-96 (scale stored as fp16_rn(amax / 127)). Block layout {fp16 d; int8 qs[32]}
 * per tools/trace/cpu_mxfp4_vnni.cpp:15-18. */
void orc_quantize_row_q8_0(const float * x, void * vy, int64_t k) {
    uint8_t * y = (uint8_t *)vy;
    for (int64_t b = 0; b < k / 32; ++b) {
        const float * v = x + b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) {
            const float a = fabsf(v[i]);
            if (a > amax) amax = a;
        }
        const float d = amax / 127.0f;
        const uint16_t h = orc_fp32_to_fp16(d);
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        uint8_t * blk = y + b * 34;
        blk[0] = (uint8_t)(h & 0xFF);
        blk[1] = (uint8_t)(h >> 8);
        for (int i = 0; i < 32; ++i) {
            const float scaled = v[i] * id;
            float r = nearbyintf(scaled);         /* round half to even */
            if (r > 127.0f) r = 127.0f;
            if (r < -128.0f) r = -128.0f;
            blk[2 + i] = (uint8_t)(int8_t)(int)r;
        }
    }
}

/* ------------------------------------------------------------------ MXFP4 x Q8_0 */
static const int8_t kMxfp4Values[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

/* VPSIGNB(b, a): b if a > 0, 0 if a == 0, -b if a < 0 with -(-128) == -128. */
static inline int vpsign(int b, int a) {
    if (a == 0) return 0;
    if (a > 0) return b;
    return b == -128 ? -128 : -b;
}

/* Integer part of tools/trace/cpu_mxfp4_vnni.cpp:35-45 (dpbusd of VPSIGNB'd bytes; lane l covers
 * elements 4l..4l+3; element i < 16 is the low nibble of qs[i], i >= 16 the high nibble of
 * qs[i-16]); same per-lane map as tools/engine/quantized_cuda.cu:145-157. */
int32_t orc_mxfp4_block_lanes(const void * vx, const void * vy, int32_t lanes[8]) {
    const uint8_t * x = (const uint8_t *)vx;
    const int8_t * q = (const int8_t *)((const uint8_t *)vy + 2);
    int32_t total = 0;
    for (int lane = 0; lane < 8; ++lane) {
        int32_t sum = 0;
        for (int j = 0; j < 4; ++j) {
            const int i = 4 * lane + j;
            const int nibble = i < 16 ? (x[1 + i] & 15) : (x[1 + i - 16] >> 4);
            const int a = kMxfp4Values[nibble];
            sum += abs(a) * vpsign(q[i], a);
        }
        lanes[lane] = sum;
        total += sum;
    }
    return total;
}

/* hsum of eight lanes: ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)),
 * tools/trace/cpu_mxfp4_vnni.cpp:64-67 (extract-high add, movehl add, movehdup add). */
static inline float hsum8(const float l[8]) {
    const float s0 = l[4] + l[0], s1 = l[5] + l[1], s2 = l[6] + l[2], s3 = l[7] + l[3];
    return (s0 + s2) + (s1 + s3);
}

/* ggml_vec_dot_mxfp4_q8_0 as restated at tools/trace/cpu_mxfp4_vnni.cpp:49-68:
 * per block s = fp16(d_a) * E8M0_HALF(e) (one fp32 multiply); per lane even/odd block FMA
 * chains; lanes = even + odd; hsum8. Requires n % 64 == 0 (:51). */
float orc_vec_dot_mxfp4_q8_0(int n, const void * vx, const void * vy) {
    const uint8_t * x = (const uint8_t *)vx;
    const uint8_t * y = (const uint8_t *)vy;
    float even[8] = {0}, odd[8] = {0}, lanes[8];
    int32_t l0[8], l1[8];
    for (int block = 0; block < n / 32; block += 2) {
        const uint8_t * x0 = x + (size_t)block * 17, * y0 = y + (size_t)block * 34;
        const uint8_t * x1 = x0 + 17, * y1 = y0 + 34;
        const float d0 = orc_fp16_to_fp32((uint16_t)(y0[0] | (y0[1] << 8))) * orc_e8m0_half(x0[0]);
        const float d1 = orc_fp16_to_fp32((uint16_t)(y1[0] | (y1[1] << 8))) * orc_e8m0_half(x1[0]);
        orc_mxfp4_block_lanes(x0, y0, l0);
        orc_mxfp4_block_lanes(x1, y1, l1);
        for (int l = 0; l < 8; ++l) {
            even[l] = fmaf(d0, (float)l0[l], even[l]);
            odd[l] = fmaf(d1, (float)l1[l], odd[l]);
        }
    }
    for (int l = 0; l < 8; ++l) lanes[l] = even[l] + odd[l];
    return hsum8(lanes);
}

/* ------------------------------------------------------------------ repacked 8x8 contract (a8) */
/* block_mxfp4x8 {u8 e[8]; u8 qs[128]} for eight consecutive rows: e[r] is row r's exponent and
 * qs[(c*8 + r)*8 + j] is row r's qs[c*8 + j] (c = 0, 1). orc_unpack_mxfp4x8 restates the expert
 * export at HP:751-762; orc_pack_mxfp4x8 is its inverse. Rows must be a multiple of 8. */
void orc_unpack_mxfp4x8(const void * vpacked, int64_t rows, int64_t blocks, void * vraw) {
    const uint8_t * packed = (const uint8_t *)vpacked;
    uint8_t * raw = (uint8_t *)vraw;
    for (int64_t row = 0; row < rows; row += 8)
        for (int64_t block = 0; block < blocks; ++block) {
            const uint8_t * group = packed + ((row / 8) * blocks + block) * 136;
            for (int r = 0; r < 8; ++r) {
                uint8_t * result = raw + ((row + r) * blocks + block) * 17;
                result[0] = group[r];
                for (int chunk = 0; chunk < 2; ++chunk) memcpy(result + 1 + chunk * 8, group + 8 + (chunk * 8 + r) * 8, 8);
            }
        }
}

void orc_pack_mxfp4x8(const void * vraw, int64_t rows, int64_t blocks, void * vpacked) {
    const uint8_t * raw = (const uint8_t *)vraw;
    uint8_t * packed = (uint8_t *)vpacked;
    for (int64_t row = 0; row < rows; row += 8)
        for (int64_t block = 0; block < blocks; ++block) {
            uint8_t * group = packed + ((row / 8) * blocks + block) * 136;
            for (int r = 0; r < 8; ++r) {
                const uint8_t * src = raw + ((row + r) * blocks + block) * 17;
                group[r] = src[0];
                for (int chunk = 0; chunk < 2; ++chunk) memcpy(group + 8 + (chunk * 8 + r) * 8, src + 1 + chunk * 8, 8);
            }
        }
}

/* One dword lane of tools/trace/exact_packed_cpu.h:33-50 for row r: the four bytes j0..j0+3 of the
 * row's 8-byte chunk `c` (low or high nibbles) against activation codes act[a0..a0+3]: dpbusd of
 * |w| with the activation negated where w < 0 (byte wrap keeps -(-128) == -128, :34-39). */
static int32_t packed_lane(const uint8_t * group, int r, int chunk, int high, int j0, const int8_t * act) {
    int32_t sum = 0;
    for (int j = 0; j < 4; ++j) {
        const uint8_t byte = group[8 + (chunk * 8 + r) * 8 + j0 + j];
        const int w = kMxfp4Values[high ? byte >> 4 : byte & 15];
        int a = act[j];
        if (w < 0) a = a == -128 ? -128 : -a;
        sum += abs(w) * a;
    }
    return sum;
}

/* ggml_gemv_mxfp4_8x8_q8_0 as restated at tools/trace/exact_packed_cpu.h:52-88: one Q8_0
 * activation row against eight-row tiles. Vector v of a tile carries, per row r, two dword lanes
 * h = 0, 1 (activation codes 8v' + 4h.. with v' the activation octet of :56-57): v = 0 the low
 * nibbles of chunk 0 against codes 0..7, v = 1 chunk 1 low against 8..15, v = 2 chunk 0 high
 * against 16..23, v = 3 chunk 1 high against 24..31; per block s = fp16(d_a) * E8M0_HALF(e_r)
 * (:14-24); even/odd block FMA chains e_v / o_v (:58-70); a..d = e_v + o_v; pairs = (c + a) +
 * (d + b); output row r = pairs[2r] + pairs[2r + 1] (:71-76). n % 64 == 0, nc % 8 == 0 (:80). */
int orc_gemv_mxfp4x8_q8_0(int n, float * out, const void * vpacked, const void * vact, int nc) {
    if (n <= 0 || n % 64 || nc <= 0 || nc % 8) return -1;
    const uint8_t * packed = (const uint8_t *)vpacked;
    const uint8_t * act = (const uint8_t *)vact;
    const int blocks = n / 32;
    static const int kChunk[4] = {0, 1, 0, 1}, kHigh[4] = {0, 0, 1, 1}, kAct[4] = {0, 8, 16, 24};
    for (int column = 0; column < nc; column += 8) {
        float e[4][16], o[4][16];
        memset(e, 0, sizeof(e));
        memset(o, 0, sizeof(o));
        for (int block = 0; block < blocks; block += 2) {
            for (int par = 0; par < 2; ++par) {
                const uint8_t * group = packed + ((size_t)(column / 8) * blocks + block + par) * 136;
                const uint8_t * y = act + (size_t)(block + par) * 34;
                const float da = orc_fp16_to_fp32((uint16_t)(y[0] | (y[1] << 8)));
                const int8_t * q = (const int8_t *)(y + 2);
                for (int v = 0; v < 4; ++v)
                    for (int r = 0; r < 8; ++r) {
                        const float d = da * orc_e8m0_half(group[r]);
                        for (int h = 0; h < 2; ++h) {
                            const int32_t lane = packed_lane(group, r, kChunk[v], kHigh[v], 4 * h, q + kAct[v] + 4 * h);
                            float * acc = par ? &o[v][2 * r + h] : &e[v][2 * r + h];
                            *acc = fmaf(d, (float)lane, *acc);
                        }
                    }
            }
        }
        for (int r = 0; r < 8; ++r) {
            float pairs[2];
            for (int h = 0; h < 2; ++h) {
                const int i = 2 * r + h;
                const float a = e[0][i] + o[0][i], b = e[1][i] + o[1][i];
                const float c = e[2][i] + o[2][i], d = e[3][i] + o[3][i];
                pairs[h] = (c + a) + (d + b);
            }
            out[column + r] = pairs[0] + pairs[1];
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ Q8_0 x Q8_0 */
/* Integer part of ggml_vec_dot_q8_0_q8_0 on x86 (mul_sum_i8_pairs: |x| times VPSIGNB(y, x),
 * pairwise maddubs then madd, i.e. lane l = elements 4l..4l+3; no saturation is reachable since
 * |x| <= 128). The reference does not restate this function; its call sites are
 * tools/engine/native_cpu.cpp:100-102 (vec_dot through type_traits). Its fp32 order is pinned
 * against the reference's compiled MXFP4 restatement on inputs where both are the same
 * arithmetic (tests/test_oracle.py). */
int32_t orc_q8_block_lanes(const void * vx, const void * vy, int32_t lanes[8]) {
    const int8_t * x = (const int8_t *)((const uint8_t *)vx + 2);
    const int8_t * y = (const int8_t *)((const uint8_t *)vy + 2);
    int32_t total = 0;
    for (int lane = 0; lane < 8; ++lane) {
        int32_t sum = 0;
        for (int j = 0; j < 4; ++j) {
            const int i = 4 * lane + j;
            const int a = x[i];
            const int magnitude = a == -128 ? 128 : abs(a);
            sum += magnitude * vpsign(y[i], a);
        }
        lanes[lane] = sum;
        total += sum;
    }
    return total;
}

/* AVX2 ggml_vec_dot_q8_0_q8_0 (upstream ggml x86, not vendored): acc = fma(fp16(dx)*fp16(dy),
 * float(lanes), acc) per block, then the same hsum8 tree as the MXFP4 dot. */
float orc_vec_dot_q8_0_q8_0(int n, const void * vx, const void * vy) {
    const uint8_t * x = (const uint8_t *)vx;
    const uint8_t * y = (const uint8_t *)vy;
    float acc[8] = {0};
    int32_t lanes[8];
    for (int block = 0; block < n / 32; ++block) {
        const uint8_t * xb = x + (size_t)block * 34, * yb = y + (size_t)block * 34;
        const float d = orc_fp16_to_fp32((uint16_t)(xb[0] | (xb[1] << 8))) *
                        orc_fp16_to_fp32((uint16_t)(yb[0] | (yb[1] << 8)));
        orc_q8_block_lanes(xb, yb, lanes);
        for (int l = 0; l < 8; ++l) acc[l] = fmaf(d, (float)lanes[l], acc[l]);
    }
    return hsum8(acc);
}

/* ------------------------------------------------------------------ f32 dot */
/* ggml_vec_dot_f32 with GGML_SIMD on AVX2: four 8-wide accumulators over 32-element steps
 * (sum[j] = fma(x, y, sum[j])), reduce sum0+=sum2, sum1+=sum3, sum0+=sum1, then
 * (lo128 + hi128) and two horizontal adds; scalar tail (upstream ggml, not vendored; the router
 * logits of the reference are computed by upstream build_lora_mm, HP:1357-1385). Pinned by
 * hand-derived reduction-order probes for n % 32 == 0; the tail's accumulation width is not. */
float orc_vec_dot_f32(int n, const float * x, const float * y) {
    float sum[4][8];
    memset(sum, 0, sizeof(sum));
    const int np = n & ~31;
    for (int i = 0; i < np; i += 32)
        for (int j = 0; j < 4; ++j)
            for (int l = 0; l < 8; ++l)
                sum[j][l] = fmaf(x[i + 8 * j + l], y[i + 8 * j + l], sum[j][l]);
    for (int l = 0; l < 8; ++l) {
        sum[0][l] = sum[0][l] + sum[2][l];
        sum[1][l] = sum[1][l] + sum[3][l];
    }
    for (int l = 0; l < 8; ++l) sum[0][l] = sum[0][l] + sum[1][l];
    const float t0[4] = {sum[0][0] + sum[0][4], sum[0][1] + sum[0][5], sum[0][2] + sum[0][6], sum[0][3] + sum[0][7]};
    const float t1a = t0[0] + t0[1], t1b = t0[2] + t0[3];
    float result = t1a + t1b;
    for (int i = np; i < n; ++i) result += x[i] * y[i];
    return result;
}

/* ------------------------------------------------------------------ fast (SIMD) dots */
#if defined(__x86_64__)
__attribute__((target("avx2,fma,f16c")))
static float mxfp4_dot_avx2(int n, const uint8_t * x, const uint8_t * y) {
    const __m128i table = _mm_setr_epi8(0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12);
    const __m128i mask = _mm_set1_epi8(15);
    const __m256i ones = _mm256_set1_epi16(1);
    __m256 even = _mm256_setzero_ps(), odd = _mm256_setzero_ps();
    for (int block = 0; block < n / 32; block += 2) {
        for (int p = 0; p < 2; ++p) {
            const uint8_t * xb = x + (size_t)(block + p) * 17;
            const uint8_t * yb = y + (size_t)(block + p) * 34;
            const __m128i bits = _mm_loadu_si128((const __m128i *)(xb + 1));
            const __m128i lo = _mm_shuffle_epi8(table, _mm_and_si128(bits, mask));
            const __m128i hi = _mm_shuffle_epi8(table, _mm_and_si128(_mm_srli_epi16(bits, 4), mask));
            const __m256i a = _mm256_set_m128i(hi, lo);
            const __m256i b = _mm256_loadu_si256((const __m256i *)(yb + 2));
            const __m256i p16 = _mm256_maddubs_epi16(_mm256_sign_epi8(a, a), _mm256_sign_epi8(b, a));
            const __m256i p32 = _mm256_madd_epi16(p16, ones);
            uint16_t hbits = (uint16_t)(yb[0] | (yb[1] << 8));
            const float d = _cvtsh_ss(hbits) * orc_e8m0_half(xb[0]);
            if (p == 0) even = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(p32), even);
            else odd = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(p32), odd);
        }
    }
    const __m256 lanes = _mm256_add_ps(even, odd);
    __m128 sum = _mm_add_ps(_mm256_extractf128_ps(lanes, 1), _mm256_castps256_ps128(lanes));
    sum = _mm_add_ps(sum, _mm_movehl_ps(sum, sum));
    return _mm_cvtss_f32(_mm_add_ss(sum, _mm_movehdup_ps(sum)));
}

__attribute__((target("avx2,fma,f16c")))
static float q8_dot_avx2(int n, const uint8_t * x, const uint8_t * y) {
    const __m256i ones = _mm256_set1_epi16(1);
    __m256 acc = _mm256_setzero_ps();
    for (int block = 0; block < n / 32; ++block) {
        const uint8_t * xb = x + (size_t)block * 34, * yb = y + (size_t)block * 34;
        const __m256i qx = _mm256_loadu_si256((const __m256i *)(xb + 2));
        const __m256i qy = _mm256_loadu_si256((const __m256i *)(yb + 2));
        const __m256i p16 = _mm256_maddubs_epi16(_mm256_sign_epi8(qx, qx), _mm256_sign_epi8(qy, qx));
        const __m256i p32 = _mm256_madd_epi16(p16, ones);
        const float d = _cvtsh_ss((uint16_t)(xb[0] | (xb[1] << 8))) * _cvtsh_ss((uint16_t)(yb[0] | (yb[1] << 8)));
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(p32), acc);
    }
    __m128 sum = _mm_add_ps(_mm256_extractf128_ps(acc, 1), _mm256_castps256_ps128(acc));
    sum = _mm_add_ps(sum, _mm_movehl_ps(sum, sum));
    return _mm_cvtss_f32(_mm_add_ss(sum, _mm_movehdup_ps(sum)));
}

static int g_isa = -1;
int orc_fast_isa(void) {
    if (g_isa < 0) {
        __builtin_cpu_init();
        g_isa = (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) ? 2 : 0;
    }
    return g_isa;
}
#else
int orc_fast_isa(void) { return 0; }
#endif

static float row_dot(int type, int n, const uint8_t * w, const uint8_t * a, int fast) {
#if defined(__x86_64__)
    if (fast && orc_fast_isa() >= 2)
        return type == ORC_TYPE_MXFP4 ? mxfp4_dot_avx2(n, w, a) : q8_dot_avx2(n, w, a);
#endif
    (void)fast;
    return type == ORC_TYPE_MXFP4 ? orc_vec_dot_mxfp4_q8_0(n, w, a) : orc_vec_dot_q8_0_q8_0(n, w, a);
}

static size_t row_bytes(int type, int64_t k) {
    return (size_t)(k / 32) * (type == ORC_TYPE_MXFP4 ? 17 : 34);
}

/* Rows [0, rows) of one expert matrix times one Q8_0 activation row. threads > 0: SIMD dots on
 * that many OpenMP threads; threads < 0: SIMD dots on the calling thread; 0: scalar dots. */
static void gemv_rows(int type, const uint8_t * matrix, int64_t k, int64_t rows, const uint8_t * act,
                      const float * bias, float * out, int threads) {
    const size_t stride = row_bytes(type, k);
    if (threads < 0) {
        for (int64_t r = 0; r < rows; ++r) {
            const float v = row_dot(type, (int)k, matrix + r * stride, act, 1);
            out[r] = bias ? v + bias[r] : v;
        }
    } else if (threads > 0) {
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads) schedule(static)
#endif
        for (int64_t r = 0; r < rows; ++r) {
            const float v = row_dot(type, (int)k, matrix + r * stride, act, 1);
            out[r] = bias ? v + bias[r] : v;
        }
    } else {
        for (int64_t r = 0; r < rows; ++r) {
            const float v = row_dot(type, (int)k, matrix + r * stride, act, 0);
            out[r] = bias ? v + bias[r] : v;
        }
    }
}

/* ------------------------------------------------------------------ MUL_MAT_ID */
/* ggml_compute_forward_mul_mat_id (HP:559-640) with the hybrid mask: src1 rows are converted to
 * the vec_dot type once (HP:600-603), id == -1 zeroes the output row (HP:617-621), other ids
 * must lie in [0, n_as) (HP:622); the activation row is b[:, r mod ne11, t] (broadcast when
 * ne11 == 1, HP:1413). Bias = ADD_ID (HP:1464-1480). */
int orc_mul_mat_id(int type, const void * as, int64_t k, int64_t rows, int64_t n_as,
                   int b_type, const void * b, int64_t b_ne1,
                   const int32_t * ids, int64_t n_ids, int64_t n_tokens, int64_t ids_stride,
                   const float * bias, float * dst, int threads) {
    if ((type != ORC_TYPE_MXFP4 && type != ORC_TYPE_Q8_0) || k <= 0 || k % 64 || rows <= 0 || n_as <= 0 ||
        (b_ne1 != 1 && b_ne1 != n_ids) || (b_type != ORC_TYPE_F32 && b_type != ORC_TYPE_Q8_0))
        return -1;
    const size_t qrow = (size_t)(k / 32) * 34;
    const int64_t n_b = b_ne1 * n_tokens;
    uint8_t * q = NULL;
    if (b_type == ORC_TYPE_F32) {
        q = (uint8_t *)malloc(qrow * (size_t)n_b);
        if (!q) return -1;
        for (int64_t i = 0; i < n_b; ++i) orc_quantize_row_q8_0((const float *)b + i * k, q + i * qrow, k);
    }
    const uint8_t * qb = b_type == ORC_TYPE_F32 ? q : (const uint8_t *)b;
    const size_t expert_bytes = row_bytes(type, k) * (size_t)rows;
    int status = 0;
    for (int64_t t = 0; t < n_tokens && !status; ++t) {
        for (int64_t r = 0; r < n_ids; ++r) {
            const int32_t id = ids[t * ids_stride + r];
            float * out = dst + (t * n_ids + r) * rows;
            if (id == -1) { memset(out, 0, (size_t)rows * sizeof(float)); continue; }
            if (id < 0 || id >= n_as) { status = -1; break; }
            const uint8_t * act = qb + ((t * b_ne1) + (b_ne1 == 1 ? 0 : r)) * qrow;
            gemv_rows(type, (const uint8_t *)as + (size_t)id * expert_bytes, k, rows, act,
                      bias ? bias + (size_t)id * rows : NULL, out, threads);
        }
    }
    free(q);
    return status;
}

/* ------------------------------------------------------------------ grouping */
/* Row mapping of ggml_compute_forward_mul_mat_id (HP:606-631): for each token (outer) and rank
 * (inner), append (rank, token) to the list of its expert; -1 ids are skipped (HP:617-621).
 * Equivalent to a stable counting sort by expert of token*n_ids + rank. */
int orc_group_by_expert(const int32_t * ids, int64_t n_ids, int64_t n_tokens, int64_t ids_stride,
                        int64_t n_as, int32_t * counts, int32_t * offsets, int32_t * rows) {
    memset(counts, 0, (size_t)n_as * sizeof(int32_t));
    for (int64_t t = 0; t < n_tokens; ++t)
        for (int64_t r = 0; r < n_ids; ++r) {
            const int32_t id = ids[t * ids_stride + r];
            if (id == -1) continue;
            if (id < 0 || id >= n_as) return -1;
            counts[id] += 1;
        }
    offsets[0] = 0;
    for (int64_t e = 0; e < n_as; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t * fill = (int32_t *)calloc((size_t)n_as, sizeof(int32_t));
    if (!fill) return -1;
    for (int64_t t = 0; t < n_tokens; ++t)
        for (int64_t r = 0; r < n_ids; ++r) {
            const int32_t id = ids[t * ids_stride + r];
            if (id == -1) continue;
            rows[offsets[id] + fill[id]++] = (int32_t)(t * n_ids + r);
        }
    free(fill);
    return 0;
}

/* ------------------------------------------------------------------ router */
/* Canonical top-k: value descending, then lower index (tools/trace/topk-tie-probe.cpp:111-113). */
void orc_topk(const float * logits, int64_t n, int64_t k, int32_t * ids) {
    for (int64_t j = 0; j < k; ++j) {
        int64_t best = -1;
        for (int64_t i = 0; i < n; ++i) {
            int taken = 0;
            for (int64_t p = 0; p < j; ++p) taken |= ids[p] == i;
            if (taken) continue;
            if (best < 0 || logits[i] > logits[best]) best = i;   /* ties keep the lower index */
        }
        ids[j] = (int32_t)best;
    }
}

/* ggml soft_max over the selected weights (gpt-oss SOFTMAX_WEIGHT gating after top-k): max,
 * y = expf(x - max) summed in double (ggml_float), scale by (float)(1.0/sum). Parity unpinned
 * (upstream ggml soft_max, not vendored; scalar expf path for k < 8). */
void orc_softmax_selected(const float * values, int64_t k, float * out) {
    float max = -INFINITY;
    for (int64_t i = 0; i < k; ++i) if (values[i] > max) max = values[i];
    double sum = 0.0;
    for (int64_t i = 0; i < k; ++i) {
        const float v = expf(values[i] - max);
        out[i] = v;
        sum += (double)v;
    }
    const float scale = (float)(1.0 / sum);
    for (int64_t i = 0; i < k; ++i) out[i] *= scale;
}

void orc_router(const float * router_w, const float * router_b, const float * x, int64_t hidden,
                float * logits, int64_t n_expert, int64_t n_tokens, int64_t top_k,
                int32_t * ids, float * weights) {
    float * selected = (float *)malloc((size_t)top_k * sizeof(float));
    for (int64_t t = 0; t < n_tokens; ++t) {
        float * l = logits + t * n_expert;
        if (router_w)
            for (int64_t e = 0; e < n_expert; ++e) {
                const float v = orc_vec_dot_f32((int)hidden, router_w + e * hidden, x + t * hidden);
                l[e] = router_b ? v + router_b[e] : v;
            }
        orc_topk(l, n_expert, top_k, ids + t * top_k);
        for (int64_t j = 0; j < top_k; ++j) selected[j] = l[ids[t * top_k + j]];
        orc_softmax_selected(selected, top_k, weights + t * top_k);
    }
    free(selected);
}

/* ------------------------------------------------------------------ GLU, combine */
/* SwiGLU-OAI: tools/engine/native_cpu.cpp:155-158 (x = min(g, limit), y = clamp(u, -limit, limit),
 * (x / (1 + exp(alpha * -x))) * (y + 1)); SiLU gate: tools/engine/f32_experts.cpp:253-254. */
void orc_glu(int activation, const float * gate, const float * up, float * out, int64_t n,
             float alpha, float limit) {
    for (int64_t i = 0; i < n; ++i) {
        if (activation == ORC_ACT_SWIGLU_OAI) {
            const float g = fminf(gate[i], limit);
            const float u = fminf(fmaxf(up[i], -limit), limit);
            out[i] = (g / (1.0f + expf(alpha * (-g)))) * (u + 1.0f);
        } else {
            const float g = gate[i];
            out[i] = g / (1.0f + expf(-g)) * up[i];
        }
    }
}

/* ggml MUL by the routing weight then sequential ADD over ranks (HP:1620-1646, HP:1910-1916). */
void orc_weighted_combine(const float * y, const float * weights, int64_t rows, int64_t n_ids,
                          int64_t n_tokens, float * out) {
    for (int64_t t = 0; t < n_tokens; ++t)
        for (int64_t i = 0; i < rows; ++i) {
            float acc = y[(t * n_ids) * rows + i] * weights[t * n_ids];
            for (int64_t r = 1; r < n_ids; ++r) {
                const float term = y[(t * n_ids + r) * rows + i] * weights[t * n_ids + r];
                acc = acc + term;
            }
            out[t * rows + i] = acc;
        }
}

/* ------------------------------------------------------------------ layer */
/* expert_branch (HP:1394-1683) for the non-weight-before-ffn case, fused gate_up:
 * gate_up MUL_MAT_ID -> ADD_ID biases after the gate|up split (HP:1472-1480) -> GLU ->
 * MUL_MAT_ID down (activation requantized to Q8_0, tools/engine/native_cpu.cpp:190) -> ADD_ID ->
 * MUL weights -> sequential rank sum. */
/* One token of orc_moe_layer: quantize, then per rank gate_up -> GLU -> requantize -> down, then
 * the weighted rank combine. `inner` is gemv_rows' thread argument. */
static void moe_token(const orc_layer * L, const float * x, int64_t t, const int32_t * ids, const float * weights,
                      float * out, float * act_out, float * y_out, int inner) {
    const int64_t H = L->hidden, I = L->intermediate, K = L->top_k;
    const size_t qh = (size_t)(H / 32) * 34, qi = (size_t)(I / 32) * 34;
    const size_t gu_bytes = row_bytes(L->type, H) * (size_t)(2 * I);
    const size_t dn_bytes = row_bytes(L->type, I) * (size_t)H;
    uint8_t * xq = (uint8_t *)malloc(qh), * aq = (uint8_t *)malloc(qi);
    float * gu = (float *)malloc(sizeof(float) * (size_t)(2 * I));
    float * act = (float *)malloc(sizeof(float) * (size_t)I);
    float * y = (float *)malloc(sizeof(float) * (size_t)(K * H));
    orc_quantize_row_q8_0(x + t * H, xq, H);
    for (int64_t r = 0; r < K; ++r) {
        const int32_t e = ids[t * K + r];
        gemv_rows(L->type, (const uint8_t *)L->gate_up + (size_t)e * gu_bytes, H, 2 * I, xq,
                  L->gate_up_bias ? L->gate_up_bias + (size_t)e * 2 * I : NULL, gu, inner);
        orc_glu(L->activation, gu, gu + I, act, I, 1.702f, 7.0f);
        if (act_out) memcpy(act_out + (t * K + r) * I, act, sizeof(float) * (size_t)I);
        orc_quantize_row_q8_0(act, aq, I);
        gemv_rows(L->type, (const uint8_t *)L->down + (size_t)e * dn_bytes, I, H, aq,
                  L->down_bias ? L->down_bias + (size_t)e * H : NULL, y + r * H, inner);
    }
    if (y_out) memcpy(y_out + t * K * H, y, sizeof(float) * (size_t)(K * H));
    orc_weighted_combine(y, weights + t * K, H, K, 1, out + t * H);
    free(xq); free(aq); free(gu); free(act); free(y);
}

int orc_moe_layer(const orc_layer * L, const float * x, float * logits, int64_t n_tokens,
                  float * out, int32_t * ids, float * weights, float * act_out, float * y_out,
                  int threads) {
    const int64_t H = L->hidden, I = L->intermediate, K = L->top_k;
    if (H % 64 || I % 64 || K <= 0 || K > L->n_expert) return -1;
    orc_router(L->router_w, L->router_b, x, H, logits, L->n_expert, n_tokens, K, ids, weights);
    /* Tokens are independent: with many tokens each thread takes whole tokens (SIMD dots on the
     * thread), otherwise the rows of each projection are split over the threads (a top-level
     * parallel region per projection, never nested in another). Either way every output is the
     * same function of its token's inputs, so the bits do not depend on it. */
    if (threads > 0 && n_tokens >= 2 * threads) {
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
#endif
        for (int64_t t = 0; t < n_tokens; ++t) moe_token(L, x, t, ids, weights, out, act_out, y_out, -1);
    } else {
        for (int64_t t = 0; t < n_tokens; ++t) moe_token(L, x, t, ids, weights, out, act_out, y_out, threads);
    }
    return 0;
}
