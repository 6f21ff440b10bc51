// Routing-side kernels: token->expert grouping, Q8_0 activation quantizer, router
// (logits, top-k, softmax over the selected), weighted rank-ordered combine, ADD_ID, GLU.
#include "vbm_device.hpp"
#include "vbm_internal.hpp"

namespace vbm {
namespace {

constexpr int kGroupThreads = 1024;
constexpr int kMaxExperts = 1024;

// Token->expert grouping: a stable counting sort of entries i = token * n_ids + rank by expert
// (the (token outer, rank inner) append order of ggml's MMID row mapping). Entries with id -1
// are skipped; ids outside [-1, n_as) raise the error flag and are skipped. Three launches over
// chunks of 1024 entries:
//   count: per-chunk expert histograms (LDS atomics, order-free) and per-chunk error flags;
//   scan:  one workgroup turns the histograms into per-(chunk, expert) bases, then scans the
//          expert totals into counts / offsets and the active-expert list;
//   place: each wave finds, for every lane, the lanes holding the same expert with one ballot
//          per id bit, ranks its entry among them, and adds the counts of the same expert in
//          the chunk's earlier waves and the chunk base: positions follow i exactly.
constexpr int kGroupChunk = kGroupThreads;

__device__ __forceinline__ int group_id(const int32_t * __restrict__ ids, int64_t i, int n_ids, int64_t ids_stride,
                                        int n_as, bool & bad) {
    int id = ids[(i / n_ids) * ids_stride + i % n_ids];
    bad = id != -1 && (id < 0 || id >= n_as);
    return bad ? -2 : id;
}

__global__ __launch_bounds__(kGroupThreads) void group_count_kernel(const int32_t * __restrict__ ids, int n_ids,
                                                                     int64_t n, int64_t ids_stride, int n_as,
                                                                     int32_t * __restrict__ chunk_counts) {
    __shared__ int s_hist[kMaxExperts];
    __shared__ int s_bad;
    const int t = threadIdx.x;
    for (int e = t; e < n_as; e += kGroupThreads) s_hist[e] = 0;
    if (t == 0) s_bad = 0;
    __syncthreads();
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kGroupChunk + t;
    if (i < n) {
        bool bad;
        const int id = group_id(ids, i, n_ids, ids_stride, n_as, bad);
        if (bad) s_bad = 1;
        if (id >= 0) atomicAdd(&s_hist[id], 1);
    }
    __syncthreads();
    int32_t * row = chunk_counts + static_cast<int64_t>(blockIdx.x) * (n_as + 1);
    for (int e = t; e < n_as; e += kGroupThreads) row[e] = s_hist[e];
    if (t == 0) row[n_as] = s_bad;
}

// One workgroup, thread t = expert t: per-expert totals and chunk bases, offsets, the active
// list and, when job_tile > 0, the batched GEMV's job chunks (up to job_tile consecutive jobs of an
// active expert each, in active order: expert at [0, max_tiles), first job at [max_tiles,
// 2 max_tiles), their count at [2 max_tiles]).
__global__ __launch_bounds__(kGroupThreads) void group_scan_kernel(int n_chunks, int n_as, int32_t * chunk_counts,
                                                                    int32_t * counts, int32_t * offsets,
                                                                    int32_t * active, int32_t * n_active,
                                                                    int32_t * error, int job_tile, int max_tiles,
                                                                    int32_t * tiles) {
    __shared__ int s_wave_sum[3][kGroupThreads / 64];
    __shared__ int s_bad;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    if (t == 0) s_bad = 0;
    __syncthreads();
    // expert e = t: chunk bases (exclusive prefix over chunks) and the total; eight chunks' counts
    // are loaded before their bases are stored, so their loads are in flight together
    int c = 0;
    if (t < n_as) {
        for (int k0 = 0; k0 < n_chunks; k0 += 8) {
            int v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                v[j] = k0 + j < n_chunks ? chunk_counts[static_cast<int64_t>(k0 + j) * (n_as + 1) + t] : 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (k0 + j < n_chunks) chunk_counts[static_cast<int64_t>(k0 + j) * (n_as + 1) + t] = c;
                c += v[j];
            }
        }
    }
    for (int k = t; k < n_chunks; k += kGroupThreads)
        if (chunk_counts[static_cast<int64_t>(k) * (n_as + 1) + n_as]) s_bad = 1;
    // two-level exclusive scans of the totals, of (total > 0) and of the job chunks
    const int live = c > 0 ? 1 : 0;
    const int nk = job_tile > 0 ? (c + job_tile - 1) / job_tile : 0;
    int inc_c = c, inc_l = live, inc_k = nk;
    for (int off = 1; off < 64; off <<= 1) {
        const int oc = __shfl_up(inc_c, off), ol = __shfl_up(inc_l, off), ok = __shfl_up(inc_k, off);
        if (lane >= off) { inc_c += oc; inc_l += ol; inc_k += ok; }
    }
    if (lane == 63) { s_wave_sum[0][wave] = inc_c; s_wave_sum[1][wave] = inc_l; s_wave_sum[2][wave] = inc_k; }
    __syncthreads();
    int base_c = 0, base_l = 0, base_k = 0;
    for (int w = 0; w < wave; ++w) { base_c += s_wave_sum[0][w]; base_l += s_wave_sum[1][w]; base_k += s_wave_sum[2][w]; }
    const int ex_c = base_c + inc_c - c, ex_l = base_l + inc_l - live, ex_k = base_k + inc_k - nk;
    bool over = false;
    if (t < n_as) {
        counts[t] = c;
        offsets[t] = ex_c;
        if (live) active[ex_l] = t;
        for (int j = 0; j < nk; ++j) {
            if (ex_k + j < max_tiles) {
                tiles[ex_k + j] = t;
                tiles[max_tiles + ex_k + j] = j * job_tile;
            } else {
                over = true;
            }
        }
        if (t == n_as - 1) {
            offsets[n_as] = ex_c + c;
            *n_active = ex_l + live;
            if (job_tile > 0) tiles[2 * max_tiles] = ex_k + nk < max_tiles ? ex_k + nk : max_tiles;
        }
    }
    if (over) s_bad = 1;   // (cannot happen with the launch bound: flagged as a grouping error)
    __syncthreads();
    if (t == 0) *error = s_bad;
}

__global__ __launch_bounds__(kGroupThreads) void group_place_kernel(const int32_t * __restrict__ ids, int n_ids,
                                                                     int64_t n, int64_t ids_stride, int n_as, int id_bits,
                                                                     const int32_t * __restrict__ chunk_counts,
                                                                     const int32_t * __restrict__ offsets,
                                                                     int32_t * __restrict__ rows) {
    constexpr int kWaves = kGroupThreads / 64;
    __shared__ int16_t s_wave_count[kWaves][kMaxExperts];   // counts <= 64
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    for (int k = t; k < kWaves * n_as; k += kGroupThreads) s_wave_count[k / n_as][k % n_as] = 0;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kGroupChunk + t;
    int id = -2;
    if (i < n) {
        bool bad;
        id = group_id(ids, i, n_ids, ids_stride, n_as, bad);
    }
    const bool valid = id >= 0;
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < id_bits; ++b) {
        const bool bit = valid && ((id >> b) & 1);
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
    }
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    const int rank = __popcll(peers & below);
    __syncthreads();   // zeroed counts visible
    if (valid && rank == 0) s_wave_count[wave][id] = static_cast<int16_t>(__popcll(peers));
    __syncthreads();
    if (!valid) return;
    int pos = offsets[id] + chunk_counts[static_cast<int64_t>(blockIdx.x) * (n_as + 1) + id] + rank;
    for (int w = 0; w < wave; ++w) pos += s_wave_count[w][id];
    rows[pos] = static_cast<int32_t>(i);
}

// Small groupings (n <= 1024 entries, every decode batch here) in one launch instead of three:
// workgroup 0 counts in LDS, scans (thread t = expert t) and places, with the same arithmetic as
// group_count / group_scan / group_place over a single chunk, so the outputs are the same. With
// ROUTE it first routes every token itself (one wave per token, wave_topk_softmax, the ids kept in
// LDS for the grouping); the other workgroups, when there are any, quantize the layer input into
// its activation rows (one 32-lane group per block), so a batched decode layer's routing, grouping
// and input quantization take one launch.
struct SmallGroupArgs {
    const float * logits;     // ROUTE: [n / n_ids][n_expert]
    int n_expert;
    int32_t * ids_out;        // ROUTE: [n / n_ids][n_ids]
    float * weights;          // ROUTE: [n / n_ids][n_ids]
    const int32_t * ids;      // without ROUTE: ids[token * ids_stride + rank]
    int64_t ids_stride;
    int n_ids, n, n_as, id_bits;
    GroupBuffers g;
    int job_tile, max_tiles;
    int32_t * tiles;
    const float * x;          // workgroups 1..: fp32 rows -> activation rows
    int64_t q_rows, x_stride;
    int q_nb;
    XrowLayout lay;
    uint8_t * xrows;
};

template <int NPL, bool ROUTE>
__global__ __launch_bounds__(kGroupThreads) void group_small_kernel(SmallGroupArgs a) {
    if (blockIdx.x > 0) {
        quantize_expand_block(a.x, a.q_rows, a.q_nb, a.x_stride, a.lay, a.xrows, static_cast<uint8_t *>(nullptr),
                              (blockIdx.x - 1) * static_cast<int64_t>(kGroupThreads / 32) + (threadIdx.x >> 5),
                              static_cast<int>(threadIdx.x & 31));
        return;
    }
    constexpr int kWaves = kGroupThreads / 64;
    __shared__ int s_hist[kMaxExperts];
    __shared__ int s_off[kMaxExperts];
    __shared__ int16_t s_wave_count[kWaves][kMaxExperts];   // counts <= 64
    __shared__ int32_t s_ids[kGroupChunk];
    __shared__ int s_wave_sum[3][kWaves];
    __shared__ int s_bad;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n_as = a.n_as, n = a.n;
    for (int e = t; e < n_as; e += kGroupThreads) s_hist[e] = 0;
    for (int k = t; k < kWaves * n_as; k += kGroupThreads) s_wave_count[k / n_as][k % n_as] = 0;
    if (t == 0) s_bad = 0;
    if constexpr (ROUTE) {
        const int n_tok = n / a.n_ids;
        for (int tok = wave; tok < n_tok; tok += kWaves)
            wave_topk_softmax<NPL>(a.logits + static_cast<int64_t>(tok) * a.n_expert, a.n_expert, a.n_ids,
                                   a.ids_out + static_cast<int64_t>(tok) * a.n_ids,
                                   a.weights + static_cast<int64_t>(tok) * a.n_ids, s_ids + tok * a.n_ids);
    }
    __syncthreads();
    // count
    int id = -2;
    if (t < n) {
        if constexpr (ROUTE) {
            id = s_ids[t];
        } else {
            bool bad;
            id = group_id(a.ids, t, a.n_ids, a.ids_stride, n_as, bad);
            if (bad) s_bad = 1;
        }
    }
    if (id >= 0) atomicAdd(&s_hist[id], 1);
    __syncthreads();
    // scan: totals, offsets, the active list and the job chunks, two-level exclusive scans
    const int c = t < n_as ? s_hist[t] : 0;
    const int live = c > 0 ? 1 : 0;
    const int nk = a.job_tile > 0 ? (c + a.job_tile - 1) / a.job_tile : 0;
    int inc_c = c, inc_l = live, inc_k = nk;
    for (int off = 1; off < 64; off <<= 1) {
        const int oc = __shfl_up(inc_c, off), ol = __shfl_up(inc_l, off), ok = __shfl_up(inc_k, off);
        if (lane >= off) { inc_c += oc; inc_l += ol; inc_k += ok; }
    }
    if (lane == 63) { s_wave_sum[0][wave] = inc_c; s_wave_sum[1][wave] = inc_l; s_wave_sum[2][wave] = inc_k; }
    __syncthreads();
    int base_c = 0, base_l = 0, base_k = 0;
    for (int w = 0; w < wave; ++w) { base_c += s_wave_sum[0][w]; base_l += s_wave_sum[1][w]; base_k += s_wave_sum[2][w]; }
    const int ex_c = base_c + inc_c - c, ex_l = base_l + inc_l - live, ex_k = base_k + inc_k - nk;
    if (t < n_as) {
        a.g.counts[t] = c;
        a.g.offsets[t] = ex_c;
        s_off[t] = ex_c;
        if (live) a.g.active[ex_l] = t;
        bool over = false;
        for (int j = 0; j < nk; ++j) {
            if (ex_k + j < a.max_tiles) {
                a.tiles[ex_k + j] = t;
                a.tiles[a.max_tiles + ex_k + j] = j * a.job_tile;
            } else {
                over = true;
            }
        }
        if (over) s_bad = 1;   // (cannot happen with the launch bound: flagged as a grouping error)
        if (t == n_as - 1) {
            a.g.offsets[n_as] = ex_c + c;
            *a.g.n_active = ex_l + live;
            if (a.job_tile > 0) a.tiles[2 * a.max_tiles] = ex_k + nk < a.max_tiles ? ex_k + nk : a.max_tiles;
        }
    }
    // place: the entry's rank among the wave's lanes holding its expert (one ballot per id bit),
    // plus the counts of that expert in the earlier waves and the expert's offset
    const bool valid = id >= 0;
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < a.id_bits; ++b) {
        const bool bit = valid && ((id >> b) & 1);
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
    }
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    const int rank = __popcll(peers & below);
    if (valid && rank == 0) s_wave_count[wave][id] = static_cast<int16_t>(__popcll(peers));
    __syncthreads();
    if (t == 0) *a.g.error = s_bad;
    if (!valid) return;
    int pos = s_off[id] + rank;
    for (int w = 0; w < wave; ++w) pos += s_wave_count[w][id];
    a.g.rows[pos] = t;
}

// x86 quantize_row_q8_0: one 32-lane group per block.
__global__ __launch_bounds__(256) void quantize_kernel(const float * __restrict__ x, int64_t n_rows, int nb,
                                                       int64_t x_stride, uint8_t * __restrict__ dst) {
    const int64_t total = n_rows * nb;
    const int64_t b_global = blockIdx.x * 8ll + (threadIdx.x >> 5);
    const int e = threadIdx.x & 31;
    const bool live = b_global < total;
    const int64_t row = live ? b_global / nb : 0, b = live ? b_global % nb : 0;
    const float v = live ? x[row * x_stride + b * 32 + e] : 0.0f;
    float amax = fabsf(v);
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
    if (!live) return;
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    float q = rintf(v * id);
    q = q > 127.0f ? 127.0f : (q < -128.0f ? -128.0f : q);
    uint8_t * blk = dst + b_global * 34;
    blk[2 + e] = static_cast<uint8_t>(static_cast<signed char>(q));
    if (e == 0) {
        const uint16_t h = __builtin_bit_cast(uint16_t, static_cast<_Float16>(d));
        blk[0] = static_cast<uint8_t>(h & 0xFF);
        blk[1] = static_cast<uint8_t>(h >> 8);
    }
}

// Router logits in the x86 ggml_vec_dot_f32 order: 32 lanes = 4 accumulators x 8 floats, each a
// sequential FMA chain over 32-element steps, then the fixed reduction tree. One 32-lane group
// per (expert, token).
__global__ __launch_bounds__(256) void router_logits_kernel(const float * __restrict__ w, const float * __restrict__ bias,
                                                            const float * __restrict__ x, int hidden, int n_expert,
                                                            int n_tokens, float * __restrict__ logits) {
    const int group = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int lane = threadIdx.x & 31;
    const bool live = group < n_expert * n_tokens;
    const int e = live ? group % n_expert : 0, t = live ? group / n_expert : 0;
    const float * wr = w + static_cast<int64_t>(e) * hidden;
    const float * xr = x + static_cast<int64_t>(t) * hidden;
    const int np = hidden & ~31;
    float acc = 0.0f;
    if (live)
        for (int i = 0; i < np; i += 32) acc = __builtin_fmaf(wr[i + lane], xr[i + lane], acc);
    // lane = 8*j + l: sum[j][l]. sum0 += sum2, sum1 += sum3 (lanes +16), sum0 += sum1 (lanes +8).
    float v = acc + __shfl_down(acc, 16, 32);
    v = v + __shfl_down(v, 8, 32);
    // lanes 0..7 hold sum0[l]; t0[l] = s[l] + s[l+4]; then (t0[0]+t0[1]) + (t0[2]+t0[3]).
    const float t0 = v + __shfl_down(v, 4, 32);
    const float t1 = t0 + __shfl_down(t0, 1, 32);
    const float r = t1 + __shfl_down(t1, 2, 32);
    if (live && lane == 0) {
        float result = r;
        for (int i = np; i < hidden; ++i) result += w[static_cast<int64_t>(e) * hidden + i] * x[static_cast<int64_t>(t) * hidden + i];
        logits[static_cast<int64_t>(t) * n_expert + e] = bias ? result + bias[e] : result;
    }
}

// One wave per token: top-k + softmax over the selected (wave_topk_softmax), NPL logits per lane.
template <int NPL>
__global__ __launch_bounds__(64) void topk_softmax_kernel(const float * __restrict__ logits, int n_expert,
                                                          int top_k, int32_t * __restrict__ ids,
                                                          float * __restrict__ weights) {
    const int64_t t = blockIdx.x;
    wave_topk_softmax<NPL>(logits + t * n_expert, n_expert, top_k, ids + t * top_k, weights + t * top_k);
}

// out[t][i] = ((w0*y0 + w1*y1) + w2*y2) + ... : ggml MUL by the weight then sequential ADD, or the
// ADDs alone when the rows are already weighted (w null: the grouped GEMM's epilogue weighted them).
// Workgroup (token, 1024-row segment); each thread owns 4 consecutive rows and issues the 16-byte
// loads of up to 8 ranks before adding them in rank order (rows % 4 == 0, 16-byte aligned).
template <bool WEIGHTED>
__global__ __launch_bounds__(256) void combine4_kernel(const float * __restrict__ y, const float * __restrict__ w,
                                                       int64_t rows, int n_ids, float * __restrict__ out) {
    const int64_t t = blockIdx.x;
    const int64_t i = (blockIdx.y * 256ll + threadIdx.x) * 4;
    if (i >= rows) return;
    const float * yt = y + t * n_ids * rows + i;
    const float * wt = WEIGHTED ? w + t * n_ids : nullptr;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int r0 = 0; r0 < n_ids; r0 += 8) {
        float4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (r0 + j < n_ids) v[j] = *reinterpret_cast<const float4 *>(yt + static_cast<int64_t>(r0 + j) * rows);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int r = r0 + j;
            if (r < n_ids) {
                float4 term = v[j];
                if constexpr (WEIGHTED) {
                    const float wr = wt[r];
                    term = make_float4(term.x * wr, term.y * wr, term.z * wr, term.w * wr);
                }
                acc = r == 0 ? term : make_float4(acc.x + term.x, acc.y + term.y, acc.z + term.z, acc.w + term.w);
            }
        }
    }
    *reinterpret_cast<float4 *>(out + t * rows + i) = acc;
}

// The same sum one row per thread, for rows not a multiple of 4 or unaligned buffers.
// Workgroup (token, 256-row segment).
__global__ void combine_kernel(const float * __restrict__ y, const float * __restrict__ w, int64_t rows,
                               int n_ids, int64_t n_tokens, float * __restrict__ out) {
    const int64_t t = blockIdx.x;
    const int64_t i = blockIdx.y * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (i >= rows) return;
    const int64_t idx = t * rows + i;
    const float * yt = y + t * n_ids * rows + i;
    if (w == nullptr) {   // rows already weighted (the grouped GEMM's epilogue): the rank-ordered ADDs
        float acc = yt[0];
        for (int r = 1; r < n_ids; ++r) acc = acc + yt[r * rows];
        out[idx] = acc;
        return;
    }
    const float * wt = w + t * n_ids;
    float acc = yt[0] * wt[0];
    for (int r = 1; r < n_ids; ++r) {
        const float term = yt[r * rows] * wt[r];
        acc = acc + term;
    }
    out[idx] = acc;
}

__global__ void glu_kernel(int activation, const float * __restrict__ gate, const float * __restrict__ up,
                           float * __restrict__ out, int64_t n_rows, int64_t width, int64_t gs, int64_t us,
                           int64_t os, float alpha, float limit) {
    const int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (idx >= n_rows * width) return;
    const int64_t row = idx / width, i = idx % width;
    const float g0 = gate[row * gs + i], u0 = up[row * us + i];
    float v;
    if (activation == VBM_ACT_SWIGLU_OAI) {
        const float g = limit < g0 ? limit : g0;
        const float u = u0 < -limit ? -limit : (limit < u0 ? limit : u0);
        v = (g / (1.0f + expf_rn(alpha * (-g)))) * (u + 1.0f);
    } else {
        v = g0 / (1.0f + expf_rn(-g0)) * u0;
    }
    out[row * os + i] = v;
}

unsigned blocks_for(int64_t n, int threads) { return static_cast<unsigned>((n + threads - 1) / threads); }

// Top-k + softmax of n_tokens tokens (workgroups 0..n_tokens-1, wave 0 of each) and the input's
// activation rows (the other workgroups, one 32-lane group per block) in one launch.
template <int NPL>
__global__ __launch_bounds__(256) void topk_quantize_kernel(const float * __restrict__ logits, int n_expert, int top_k,
                                                            int32_t * __restrict__ ids, float * __restrict__ weights,
                                                            int64_t n_tokens, const float * __restrict__ x, int nb,
                                                            int64_t x_stride, XrowLayout lay, uint8_t * __restrict__ xrows) {
    const int64_t b = blockIdx.x;
    if (b < n_tokens) {
        if (threadIdx.x < 64)
            wave_topk_softmax<NPL>(logits + b * n_expert, n_expert, top_k, ids + b * top_k, weights + b * top_k);
        return;
    }
    quantize_expand_block(x, n_tokens, nb, x_stride, lay, xrows, static_cast<uint8_t *>(nullptr),
                          (b - n_tokens) * 8 + (threadIdx.x >> 5), static_cast<int>(threadIdx.x & 31));
}

}  // namespace

int64_t group_chunk_ints(int64_t n_as, int64_t n_entries) {
    return (n_entries + kGroupChunk - 1) / kGroupChunk * (n_as + 1);
}

size_t group_workspace_bytes(int64_t n_as, int64_t n_entries) {
    return static_cast<size_t>(n_as + (n_as + 1) + n_entries + n_as + 1 + 1 + group_chunk_ints(n_as, n_entries) +
                               2 * (n_as + n_entries) + 1 + 8) *
           sizeof(int32_t);
}

GroupBuffers carve_group(void * base, int64_t n_as, int64_t n_entries) {
    auto * p = static_cast<int32_t *>(base);
    GroupBuffers g{};
    g.counts = p; p += n_as;
    g.offsets = p; p += n_as + 1;
    g.rows = p; p += n_entries;
    g.active = p; p += n_as;
    g.n_active = p; p += 1;
    g.error = p; p += 1;
    g.chunk_counts = p; p += group_chunk_ints(n_as, n_entries);
    g.chunk_list = p;
    g.chunk_list_items = n_as + n_entries;
    return g;
}

void launch_group(const int32_t * ids, int64_t n_ids, int64_t n_tokens, int64_t ids_stride, int64_t n_as,
                  const GroupBuffers & g, hipStream_t stream, int job_tile, int32_t * tiles_out, int64_t tiles_max) {
    require(n_as > 0 && n_as <= kMaxExperts, "grouping supports 1..1024 experts");
    require(n_ids > 0 && n_tokens > 0 && n_ids * n_tokens <= (1ll << 24), "grouping entry count out of range");
    require(ids_stride >= n_ids, "ids token stride must be >= n_ids");
    require(g.chunk_counts != nullptr, "grouping needs its chunk-count scratch");
    const int64_t n = n_ids * n_tokens;
    const int n_chunks = static_cast<int>((n + kGroupChunk - 1) / kGroupChunk);
    int id_bits = 0;
    while ((1ll << id_bits) < n_as) ++id_bits;
    if (n > kGroupChunk)
        hipLaunchKernelGGL(group_count_kernel, dim3(n_chunks), dim3(kGroupThreads), 0, stream, ids, static_cast<int>(n_ids), n,
                           ids_stride, static_cast<int>(n_as), g.chunk_counts);
    check_hip(hipGetLastError(), "grouping count launch");
    int64_t max_tiles = 0;
    int32_t * tiles = g.chunk_list;
    if (job_tile > 0 && tiles_out) {
        // every active expert's tiles fit: at most entries / job_tile full ones plus one partial each
        require(tiles_max >= (n + job_tile - 1) / job_tile + std::min(n_as, n) && tiles_max < (1ll << 31),
                "job tile list bound too small");
        max_tiles = tiles_max;
        tiles = tiles_out;
    } else if (job_tile > 0) {
        max_tiles = gemv_max_chunks(std::min(n_as, n), n, job_tile);
        require(g.chunk_list != nullptr && max_tiles <= g.chunk_list_items, "job chunk list exceeds its workspace");
    }
    if (n <= kGroupChunk) {   // one workgroup, one launch
        SmallGroupArgs a{};
        a.ids = ids;
        a.ids_stride = ids_stride;
        a.n_ids = static_cast<int>(n_ids);
        a.n = static_cast<int>(n);
        a.n_as = static_cast<int>(n_as);
        a.id_bits = id_bits;
        a.g = g;
        a.job_tile = job_tile;
        a.max_tiles = static_cast<int>(max_tiles);
        a.tiles = tiles;
        hipLaunchKernelGGL((group_small_kernel<2, false>), dim3(1), dim3(kGroupThreads), 0, stream, a);
        check_hip(hipGetLastError(), "grouping launch");
        return;
    }
    hipLaunchKernelGGL(group_scan_kernel, dim3(1), dim3(kGroupThreads), 0, stream, n_chunks, static_cast<int>(n_as),
                       g.chunk_counts, g.counts, g.offsets, g.active, g.n_active, g.error, job_tile,
                       static_cast<int>(max_tiles), tiles);
    check_hip(hipGetLastError(), "grouping scan launch");
    hipLaunchKernelGGL(group_place_kernel, dim3(n_chunks), dim3(kGroupThreads), 0, stream, ids, static_cast<int>(n_ids), n,
                       ids_stride, static_cast<int>(n_as), id_bits, g.chunk_counts, g.offsets, g.rows);
    check_hip(hipGetLastError(), "grouping place launch");
}

void launch_route_group_quantize(const float * logits, int64_t n_expert, int64_t n_tokens, int64_t top_k, int32_t * ids,
                                 float * weights, const GroupBuffers & g, const float * x, int64_t hidden,
                                 const XrowLayout & lay, uint8_t * xrows, hipStream_t stream) {
    const int64_t n = n_tokens * top_k;
    require(route_group_fits(n_expert, n_tokens, top_k), "one-launch routing needs n_tokens * top_k <= 1024");
    require(top_k > 0 && top_k <= n_expert && top_k <= 64 && n_expert > 0 && n_expert <= kMaxExperts,
            "router supports 1..1024 experts and top_k <= 64");
    require(x != nullptr && hidden > 0 && hidden % 32 == 0 && lay.nb == hidden / 32, "quantize shape mismatch");
    int id_bits = 0;
    while ((1ll << id_bits) < n_expert) ++id_bits;
    const int job_tile = gemv_chunk_tokens(n_tokens);
    const int64_t max_tiles = gemv_max_chunks(std::min(n_expert, n), n, job_tile);
    require(g.chunk_list != nullptr && max_tiles <= g.chunk_list_items, "job chunk list exceeds its workspace");
    SmallGroupArgs a{};
    a.logits = logits;
    a.n_expert = static_cast<int>(n_expert);
    a.ids_out = ids;
    a.weights = weights;
    a.n_ids = static_cast<int>(top_k);
    a.n = static_cast<int>(n);
    a.n_as = static_cast<int>(n_expert);
    a.id_bits = id_bits;
    a.g = g;
    a.job_tile = job_tile;
    a.max_tiles = static_cast<int>(max_tiles);
    a.tiles = g.chunk_list;
    a.x = x;
    a.q_rows = n_tokens;
    a.x_stride = hidden;
    a.q_nb = static_cast<int>(hidden / 32);
    a.lay = lay;
    a.xrows = xrows;
    const int64_t q_groups = (n_tokens * (hidden / 32) + kGroupThreads / 32 - 1) / (kGroupThreads / 32);
    const dim3 grid(static_cast<unsigned>(1 + q_groups));
    if (n_expert <= 128) hipLaunchKernelGGL((group_small_kernel<2, true>), grid, dim3(kGroupThreads), 0, stream, a);
    else if (n_expert <= 256) hipLaunchKernelGGL((group_small_kernel<4, true>), grid, dim3(kGroupThreads), 0, stream, a);
    else hipLaunchKernelGGL((group_small_kernel<16, true>), grid, dim3(kGroupThreads), 0, stream, a);
    check_hip(hipGetLastError(), "routing + grouping + quantize launch");
}

// One token per wave of the routing workgroup: beyond 16 tokens its waves route several tokens in
// turn and the one-launch form measured slower (64 tokens top-4, 32 experts) than the parallel
// top-k launch.
bool route_group_fits(int64_t n_expert, int64_t n_tokens, int64_t top_k) {
    return n_expert <= kMaxExperts && n_tokens * top_k <= kGroupChunk && n_tokens <= kGroupThreads / 64;
}

void launch_topk_quantize(const float * logits, int64_t n_expert, int64_t n_tokens, int64_t top_k, int32_t * ids,
                          float * weights, const float * x, int64_t hidden, const XrowLayout & lay, uint8_t * xrows,
                          hipStream_t stream) {
    require(n_expert > 0 && n_expert <= 1024 && top_k > 0 && top_k <= n_expert && top_k <= 64 && n_tokens > 0,
            "router supports 1..1024 experts and top_k <= 64");
    require(x != nullptr && hidden > 0 && hidden % 32 == 0 && lay.nb == hidden / 32, "quantize shape mismatch");
    const int64_t q_wgs = (n_tokens * (hidden / 32) + 7) / 8;
    require(n_tokens + q_wgs < (1ll << 31), "too many rows for one launch");
    const dim3 grid(static_cast<unsigned>(n_tokens + q_wgs));
    const int ne = static_cast<int>(n_expert), tk = static_cast<int>(top_k), nb = static_cast<int>(hidden / 32);
    if (n_expert <= 128)
        hipLaunchKernelGGL(topk_quantize_kernel<2>, grid, dim3(256), 0, stream, logits, ne, tk, ids, weights, n_tokens, x, nb,
                           hidden, lay, xrows);
    else if (n_expert <= 256)
        hipLaunchKernelGGL(topk_quantize_kernel<4>, grid, dim3(256), 0, stream, logits, ne, tk, ids, weights, n_tokens, x, nb,
                           hidden, lay, xrows);
    else
        hipLaunchKernelGGL(topk_quantize_kernel<16>, grid, dim3(256), 0, stream, logits, ne, tk, ids, weights, n_tokens, x,
                           nb, hidden, lay, xrows);
    check_hip(hipGetLastError(), "top-k + quantize launch");
}

void launch_quantize_q8_0(const float * x, int64_t n_rows, int64_t k, int64_t x_stride, uint8_t * dst,
                          hipStream_t stream) {
    require(k > 0 && k % 32 == 0 && n_rows > 0 && x_stride >= k, "quantize needs k % 32 == 0 and stride >= k");
    const int64_t blocks = n_rows * (k / 32);
    hipLaunchKernelGGL(quantize_kernel, dim3(blocks_for(blocks, 8)), dim3(256), 0, stream, x, n_rows,
                       static_cast<int>(k / 32), x_stride, dst);
    check_hip(hipGetLastError(), "quantize launch");
}

void launch_router(const float * router_w, const float * router_b, const float * x, int64_t hidden, float * logits,
                   int64_t n_expert, int64_t n_tokens, int64_t top_k, int32_t * ids, float * weights,
                   hipStream_t stream, bool topk) {
    require(n_expert > 0 && n_expert <= 1024 && top_k > 0 && top_k <= n_expert && top_k <= 64 && n_tokens > 0,
            "router supports 1..1024 experts and top_k <= 64");
    if (router_w) {
        require(x != nullptr && logits != nullptr && hidden > 0, "router GEMV needs x, hidden and a logits buffer");
        hipLaunchKernelGGL(router_logits_kernel, dim3(blocks_for(n_expert * n_tokens, 8)), dim3(256), 0, stream,
                           router_w, router_b, x, static_cast<int>(hidden), static_cast<int>(n_expert),
                           static_cast<int>(n_tokens), logits);
        check_hip(hipGetLastError(), "router logits launch");
    }
    if (!topk) return;
    const dim3 grid(static_cast<unsigned>(n_tokens));
    const int ne = static_cast<int>(n_expert), tk = static_cast<int>(top_k);
    if (n_expert <= 128) hipLaunchKernelGGL(topk_softmax_kernel<2>, grid, dim3(64), 0, stream, logits, ne, tk, ids, weights);
    else if (n_expert <= 256) hipLaunchKernelGGL(topk_softmax_kernel<4>, grid, dim3(64), 0, stream, logits, ne, tk, ids, weights);
    else hipLaunchKernelGGL(topk_softmax_kernel<16>, grid, dim3(64), 0, stream, logits, ne, tk, ids, weights);
    check_hip(hipGetLastError(), "top-k launch");
}

void launch_combine(const float * y, const float * weights, int64_t rows, int64_t n_ids, int64_t n_tokens, float * out,
                    hipStream_t stream) {
    require(n_tokens > 0 && n_tokens < (1ll << 31) && rows > 0 && (rows + 255) / 256 <= 65535, "combine shape out of range");
    const bool vec = rows % 4 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0;
    if (vec) {
        const dim3 grid(static_cast<unsigned>(n_tokens), static_cast<unsigned>((rows + 1023) / 1024));
        if (weights) hipLaunchKernelGGL(combine4_kernel<true>, grid, dim3(256), 0, stream, y, weights, rows, static_cast<int>(n_ids), out);
        else hipLaunchKernelGGL(combine4_kernel<false>, grid, dim3(256), 0, stream, y, weights, rows, static_cast<int>(n_ids), out);
    } else {
        hipLaunchKernelGGL(combine_kernel, dim3(static_cast<unsigned>(n_tokens), static_cast<unsigned>((rows + 255) / 256)),
                           dim3(256), 0, stream, y, weights, rows, static_cast<int>(n_ids), n_tokens, out);
    }
    check_hip(hipGetLastError(), "combine launch");
}

void launch_glu(int activation, const float * gate, const float * up, float * out, int64_t n_rows, int64_t width,
                int64_t gate_stride, int64_t up_stride, int64_t out_stride, float alpha, float limit,
                hipStream_t stream) {
    hipLaunchKernelGGL(glu_kernel, dim3(blocks_for(n_rows * width, 256)), dim3(256), 0, stream, activation, gate, up, out,
                       n_rows, width, gate_stride, up_stride, out_stride, alpha, limit);
    check_hip(hipGetLastError(), "glu launch");
}

}  // namespace vbm
