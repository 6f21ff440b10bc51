// Internal declarations shared by the library's translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <new>
#include <stdexcept>
#include <string>

#include "../../include/vbmoe.h"
#include "vbm_common.hpp"

struct vbm_bank {
    int type = 0;              // VBM_TYPE_MXFP4 or VBM_TYPE_Q8_0
    int64_t rows = 0;          // rows per expert (ggml ne1)
    int64_t k = 0;             // weights per row (ggml ne0)
    int64_t nb = 0;            // blocks per row
    int64_t n_slots = 0;
    int interleave = 0;        // fused gate|up tile interleave
    size_t slot_bytes = 0;
    uint8_t * base = nullptr;  // device
    uint8_t * staging = nullptr;  // device scratch of slot_bytes for repack / export
    int device = 0;
    vbm::SlotGeometry geometry() const { return {rows, nb, type}; }
};

namespace vbm {

struct Error : std::runtime_error {
    vbm_status status;
    Error(vbm_status s, const std::string & message) : std::runtime_error(message), status(s) {}
};

[[noreturn]] inline void fail(vbm_status status, const std::string & message) { throw Error(status, message); }
inline void require(bool condition, const std::string & message) {
    if (!condition) fail(VBM_ERR_INVALID_ARGUMENT, message);
}
inline void check_hip(hipError_t e, const char * what) {
    if (e != hipSuccess) fail(e == hipErrorOutOfMemory ? VBM_ERR_OUT_OF_MEMORY : VBM_ERR_RUNTIME,
                              std::string(what) + ": " + hipGetErrorString(e));
}
inline hipStream_t as_stream(void * s) { return static_cast<hipStream_t>(s); }

inline bool stream_capturing(hipStream_t s) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    check_hip(hipStreamIsCapturing(s, &capture), "hipStreamIsCapturing");
    return capture == hipStreamCaptureStatusActive;
}
// hipEventRecord that, under stream capture, becomes an event-record node of the graph (an
// external record), so the event is recorded by every replay instead of only ordering the
// capture.
inline void record_event(hipEvent_t e, hipStream_t s, const char * what) {
    if (stream_capturing(s)) check_hip(hipEventRecordWithFlags(e, s, hipEventRecordExternal), what);
    else check_hip(hipEventRecord(e, s), what);
}

void set_last_error(const std::string & message);
void clear_last_error();

// Runs `body`, converting exceptions into a status plus the thread's last-error message.
template <class F>
vbm_status guarded(F && body) {
    try {
        clear_last_error();
        body();
        return VBM_OK;
    } catch (const Error & e) {
        set_last_error(e.what());
        return e.status;
    } catch (const std::bad_alloc &) {
        set_last_error("host allocation failed");
        return VBM_ERR_OUT_OF_MEMORY;
    } catch (const std::invalid_argument & e) {
        set_last_error(e.what());
        return VBM_ERR_INVALID_ARGUMENT;
    } catch (const std::exception & e) {
        set_last_error(e.what());
        return VBM_ERR_RUNTIME;
    }
}

// Launch helpers implemented in the .hip units (all enqueue on `stream`).
void launch_bank_scatter(const vbm_bank & bank, int64_t slot, const uint8_t * ggml_src, hipStream_t stream);
void launch_bank_gather(const vbm_bank & bank, int64_t slot, uint8_t * ggml_dst, hipStream_t stream);
void launch_bank_generate(const vbm_bank & bank, int64_t first_slot, int64_t count, uint64_t seed,
                          uint64_t stream_id, int64_t first_expert, float p0, float p1, hipStream_t stream);

struct GroupBuffers {
    int32_t * counts;    // [n_as]
    int32_t * offsets;   // [n_as + 1]
    int32_t * rows;      // [n_ids * n_tokens]
    int32_t * active;    // [n_as] experts with count > 0, ascending
    int32_t * n_active;  // [1]
    int32_t * error;     // [1]
    int32_t * chunk_counts;  // [group_chunk_ints]: per-chunk histograms, then chunk bases
    int32_t * chunk_list;    // [2 * chunk_list_items + 1]: the batched GEMV's job chunks
    int64_t chunk_list_items;
};
int64_t group_chunk_ints(int64_t n_as, int64_t n_entries);
size_t group_workspace_bytes(int64_t n_as, int64_t n_entries);
GroupBuffers carve_group(void * base, int64_t n_as, int64_t n_entries);
// job_tile > 0: also the job tiles of that many jobs per active expert, in active order: by
// default the batched GEMV's job chunks (gemv_chunk_tokens) into g.chunk_list, laid out for
// gemv_max_chunks entries; with tiles_out, the grouped GEMM's tile list (expert at [0, tiles_max),
// first job at [tiles_max, 2 tiles_max), count at [2 tiles_max]), as gemm_tiles_kernel writes it
// without a tile filter.
void launch_group(const int32_t * ids, int64_t n_ids, int64_t n_tokens, int64_t ids_stride, int64_t n_as,
                  const GroupBuffers & g, hipStream_t stream, int job_tile = 0, int32_t * tiles_out = nullptr,
                  int64_t tiles_max = 0);
// Token width of the batched GEMV's job chunks for a bound on jobs per expert, and the bound on
// the number of chunks: at most one partial chunk per active expert plus entries / width full ones.
inline int gemv_chunk_tokens(int64_t max_per_expert) {
    return max_per_expert <= 1 ? 1 : (max_per_expert <= 2 ? 2 : (max_per_expert <= 4 ? 4 : 8));
}
inline int64_t gemv_max_chunks(int64_t max_active, int64_t n_entries, int width) {
    return max_active + n_entries / width;
}

void launch_quantize_q8_0(const float * x, int64_t n_rows, int64_t k, int64_t x_stride, uint8_t * dst,
                          hipStream_t stream);
// Router logits (when router_w is given) and, unless topk is false, top-k + softmax per token.
void launch_router(const float * router_w, const float * router_b, const float * x, int64_t hidden,
                   float * logits, int64_t n_expert, int64_t n_tokens, int64_t top_k, int32_t * ids,
                   float * weights, hipStream_t stream, bool topk = true);
// out[t] = sum over ranks r in order of y[t][r] * weights[t][r] (ggml MUL then ADDs); weights
// NULL: the rows are already weighted, out[t] = sum of y[t][r] in rank order.
void launch_combine(const float * y, const float * weights, int64_t rows, int64_t n_ids, int64_t n_tokens,
                    float * out, hipStream_t stream);
void launch_glu(int activation, const float * gate, const float * up, float * out, int64_t n_rows,
                int64_t width, int64_t gate_stride, int64_t up_stride, int64_t out_stride, float alpha,
                float limit, hipStream_t stream);

// Activation rows ("xrows"): one Q8_0-quantized activation vector per token (or per token and
// rank), expanded for the GEMV's scalar loads. For a row of nb blocks:
//   codes  [8 slices][nb] x 8 B (4 x f16, MXFP4 consumer) or x 4 B (4 x int8, Q8_0 consumer);
//          slice k of block b holds elements 4k..4k+3 of the block's 32 codes;
//   da     [nb] f32 (the block's fp16 scale, widened);
//   flag   int32: 1 when any code is -128 (selects the VPSIGNB-exact slow path).
struct XrowLayout {
    int64_t nb;
    int weight_type;  // 39 (f16 codes) or 8 (int8 codes)
    VBM_HD int64_t code_entry() const { return weight_type == 39 ? 8 : 4; }
    VBM_HD int64_t da_offset() const { return 8 * nb * code_entry(); }
    VBM_HD int64_t flag_offset() const { return da_offset() + 4 * nb; }
    VBM_HD int64_t stride() const { return (flag_offset() + 4 + 63) / 64 * 64; }
};

// A batched decode layer's top-k + softmax (given logits), grouping (with the batched GEMV's job
// chunks) and input quantization into xrows, in one launch; for route_group_fits shapes.
bool route_group_fits(int64_t n_expert, int64_t n_tokens, int64_t top_k);
// Top-k + softmax (given logits) and the input quantization into xrows in one launch.
void launch_topk_quantize(const float * logits, int64_t n_expert, int64_t n_tokens, int64_t top_k, int32_t * ids,
                          float * weights, const float * x, int64_t hidden, const XrowLayout & lay, uint8_t * xrows,
                          hipStream_t stream);
void launch_route_group_quantize(const float * logits, int64_t n_expert, int64_t n_tokens, int64_t top_k, int32_t * ids,
                                 float * weights, const GroupBuffers & g, const float * x, int64_t hidden,
                                 const XrowLayout & lay, uint8_t * xrows, hipStream_t stream);
// fp32 rows -> Q8_0 (x86 contract) -> xrows (and optionally ggml Q8_0 blocks).
void launch_quantize_expand(const float * x, int64_t n_rows, int64_t k, int64_t x_stride, const XrowLayout & lay,
                            uint8_t * xrows, uint8_t * q8_blocks, hipStream_t stream);
// ggml Q8_0 block rows -> xrows.
void launch_expand_q8(const uint8_t * q8, int64_t n_rows, int64_t row_bytes, const XrowLayout & lay, uint8_t * xrows,
                      hipStream_t stream);

// Expert GEMV over grouped jobs, reading activation rows (xrows) with act_row(j) =
// b_ne1 == 1 ? j / n_ids : j. Epilogue 0 writes dst[j][rows] (+bias); epilogue 1 (fused gate|up
// bank) applies biases and the GLU, quantizes each 32-output block to Q8_0 and writes the down
// projection's activation row j into dst_xrows.
struct GemvArgs {
    const vbm_bank * bank;
    const int32_t * expert_to_slot;   // device or null
    const uint8_t * xrows;
    int64_t n_ids, b_ne1;
    GroupBuffers group;
    int64_t max_active;               // host bound on the number of active experts
    int64_t max_per_expert;           // host bound on jobs per expert (selects the token chunk)
    int64_t n_entries;                // routed (token, rank) entries of the grouping
    bool chunks_built = false;        // launch_group already wrote the job chunk list (job_tile =
                                      // gemv_chunk_tokens(max_per_expert))
    const float * bias;               // [n_as][rows] ggml row order, or null
    float * dst;                      // epilogue 0
    uint8_t * dst_xrows;              // epilogue 1
    XrowLayout dst_layout;            // epilogue 1 (the down bank's activation format)
    int epilogue;                     // 0 plain, 1 GLU + requantize
    int activation;
    float alpha, limit;
    // false when every activation row comes from this library's Q8_0 quantizer (fp32 inputs,
    // the GLU requantization), whose codes are never -128: the kernel then carries no VPSIGNB
    // slow path, which frees the registers for a deeper weight ring
    bool may_have_neg128 = true;
};
void launch_gemv(const GemvArgs & a, hipStream_t stream);

// Chunks of `job_tile` consecutive jobs per active expert (experts with filter[e] < 0 skipped),
// in active order: tile_expert / tile_start per chunk and their count, at most max_tiles.
void launch_job_tiles(const GroupBuffers & g, const int32_t * filter, int job_tile, int64_t max_tiles,
                      int32_t * tile_expert, int32_t * tile_start, int32_t * n_tiles, hipStream_t stream);

// Activation row of the MFMA grouped GEMM: row-major codes (f16 for MXFP4 weights, int8 for
// Q8_0), fp16-rounded fp32 block scales, and the row's -128 flag; 256-byte aligned stride.
struct GemmRowLayout {
    int64_t nb;
    int weight_type;
    VBM_HD int64_t code_bytes() const { return nb * 32 * (weight_type == 39 ? 2 : 1); }
    VBM_HD int64_t da_offset() const { return code_bytes(); }
    VBM_HD int64_t flag_offset() const { return da_offset() + 4 * nb; }
    VBM_HD int64_t stride() const { return (flag_offset() + 4 + 255) / 256 * 256; }
};
void launch_gemm_rows_from_f32(const float * x, int64_t n_rows, int64_t k, int64_t x_stride, const GemmRowLayout & lay,
                               uint8_t * rows, hipStream_t stream);
void launch_gemm_rows_from_q8(const uint8_t * q8, int64_t n_rows, int64_t row_bytes, const GemmRowLayout & lay,
                              uint8_t * rows, hipStream_t stream);
// Top-k + softmax of given logits and the GEMM activation rows of x (row stride k) in one launch.
void launch_topk_gemm_rows(const float * logits, int64_t n_expert, int64_t top_k, int32_t * ids, float * weights,
                           const float * x, int64_t n_rows, int64_t k, const GemmRowLayout & lay, uint8_t * rows,
                           hipStream_t stream);

// Grouped expert GEMM on MFMA (exact block dots, fp32 accumulation across blocks).
struct GemmParams {
    const vbm_bank * bank;
    const int32_t * expert_to_slot;
    const uint8_t * rows_in;          // activation rows, row index = job / n_ids (b_ne1 == 1) or job
    GemmRowLayout lay;
    int64_t n_ids, b_ne1, n_as, n_entries;
    GroupBuffers group;
    void * tiles;                     // gemm_tiles_bytes(n_as, n_entries) of scratch
    const float * bias;
    const float * row_scale;          // epilogue 0: per-job factor after the bias (routing weights), or null
    float * dst;                      // epilogue 0: [job][rows]
    uint8_t * rows_out;               // epilogue 1: GLU + Q8_0 rows per job (out_layout)
    GemmRowLayout out_layout;
    int epilogue, activation;
    float alpha, limit;
    bool flagged_rows;                // rows_in may hold -128 codes (converted from caller Q8_0)
    const int32_t * tile_filter;      // device [n_as]: experts with a negative entry get no tiles, or null
    int64_t grid_tiles;               // > 0: bound on the tiles left by tile_filter (launch size), else 0
    bool tiles_ready;                 // `tiles` already holds this group's list (same group and filter)
};
// Jobs per grouped-GEMM workgroup (one expert's job tile): 192 for Q8_0 banks, whose expert groups
// at 2048 tokens top-8 over 128 experts hold 96-158 jobs (one tile each instead of a nearly empty
// second tile for half of them), 128 for MXFP4.
inline int gemm_job_tile(int bank_type) { return bank_type == VBM_TYPE_MXFP4 ? 128 : 192; }
int64_t gemm_max_tiles(int64_t n_as, int64_t n_entries, int job_tile);
size_t gemm_tiles_bytes(int64_t n_as, int64_t n_entries);
void launch_grouped_gemm(const GemmParams & p, hipStream_t stream);
// MXFP4 x MXFP8 experiment on the block-scaled matrix cores: OCP MX quantization of fp32 rows
// (codes [n_rows][k], e8m0 scales [n_rows][k / 32]) and the grouped GEMM over them ([job][rows]).
void launch_quantize_mxfp8(const float * x, int64_t n_rows, int64_t k, int64_t x_stride, uint8_t * codes, uint8_t * scales,
                           hipStream_t stream);
void launch_mx_gemm(const vbm_bank & bank, const int32_t * expert_to_slot, const uint8_t * codes, const uint8_t * scales,
                    int64_t n_ids, int64_t b_ne1, int64_t n_as, int64_t n_entries, const GroupBuffers & group, void * tiles,
                    float * dst, hipStream_t stream);

// Device workspace of one fused layer forward (vbm_moe_layer_forward), carved from `base` (NULL:
// sizes only).
struct LayerWorkspace {
    int32_t * ids;
    float * weights;
    float * logits;
    uint8_t * xrows_x;     // [T] activation rows of the layer input (gate_up format)
    void * group;
    uint8_t * xrows_act;   // [T*K] requantized GLU outputs (down format)
    void * tiles;          // GEMM tile lists (fast order only)
    float * y;             // [T*K][H] down outputs per (token, rank)
    size_t total;
};
constexpr int64_t kGemmMinTokens = 16;
// Below 12 routed rows per expert on average the exact-order batched GEMV (matrix-core slice
// dots, one workgroup per job chunk) outruns the MFMA grouped GEMM: 6-layer stacks of the
// 2880 x 2880 MXFP4 shape, top-4, 32 / 128 experts, GEMV vs GEMM tok/s at 8 rows 47.6k vs 38.6k /
// 56.8k vs 44.6k, at 12 rows 54.8k vs 56.4k / 62.0k vs 64.7k, at 16 rows 60.4k vs 72.4k.
constexpr int64_t kGemmMinRowsPerExpert = 12;
bool use_gemm(const vbm_moe_layer_desc & d, int64_t n_tokens);
inline bool gemm_pays(int64_t n_tokens, int64_t top_k, int64_t n_expert) {
    return n_tokens >= kGemmMinTokens && n_tokens * top_k >= kGemmMinRowsPerExpert * n_expert;
}
LayerWorkspace plan_layer(const vbm_moe_layer_desc & d, int64_t max_tokens, uint8_t * base);
// Prefill through the grouped GEMM in steps: the input rows and the token->expert grouping once,
// then one or more passes over disjoint expert subsets (experts whose expert_to_slot entry is
// -1 are skipped: their workgroups exit without writing), each writing the down outputs y of its
// entries (times the entries' routing weights route_w when given: ggml's ADD_ID then MUL, so the
// combine is then the rank-ordered ADDs alone); the combine of y runs once all entries are
// written. events (optional) [4]: around the
// pass's gate_up and down GEMMs. grid_tiles > 0: the pass's expert->slot map also filters the tile
// list, and grid_tiles bounds its tiles (sum over its experts of ceil(count / gemm_job_tile)), so a pass over a
// few experts launches only their workgroups.
// gemm_tiles: prepare also writes the grouped GEMM's unfiltered tile list (then a pass with no
// grid_tiles may take tiles_ready = true and skip gemm_tiles_kernel).
// With logits (and weights), prepare also runs the top-k + softmax into ids / weights, in the
// launch that writes the activation rows.
void prefill_prepare(const vbm_moe_layer_desc & d, const float * x, const int32_t * ids, int64_t n_tokens,
                     const LayerWorkspace & w, hipStream_t s, bool gemm_tiles = false, const float * logits = nullptr,
                     float * weights = nullptr);
void prefill_pass(const vbm_moe_layer_desc & d, const int32_t * expert_to_slot, int64_t n_tokens,
                  const LayerWorkspace & w, const float * route_w, void * const * events, hipStream_t s,
                  int64_t grid_tiles = 0, bool tiles_ready = false);

// Kernel A of the fused single-token decode: routing, input combine + Q8_0, gate_up GEMV, GLU,
// requantization into the down activation rows.
struct DecodeGateUpArgs {
    const vbm_bank * bank;            // interleaved gate|up bank
    const int32_t * expert_to_slot;
    const float * logits;             // [n_expert]
    int64_t n_expert, top_k, hidden;
    const float * x_in;               // layer input (16-byte aligned), or null to combine prev_y with prev_w
    const float * prev_y;
    const float * prev_w;
    const float * bias;
    float * act_f;                    // [top_k][intermediate] GLU outputs for kernel B
    int32_t * route_ids;
    float * route_w;
    int32_t * route_slots;            // [top_k] slots of the picks for kernel B, or null
    int activation;
    float alpha, limit;
    // Optional: device-visible base of this layer's experts in pinned host memory, in the bank's
    // slot layout (expert e at host_base + e * host_stride). A pick whose map entry is -1 streams
    // its weights from there instead of being poisoned.
    const uint8_t * host_base = nullptr;
    int64_t host_stride = 0;
    // Optional with host_base: device staging area of the layer's picks (rank r's slot copy at
    // stage + r * stage_stride). A workgroup whose pick streams from the host copy first copies
    // its tile there and then reads that copy, so the whole expert is in device memory after the
    // launch.
    uint8_t * stage = nullptr;
    int64_t stage_stride = 0;
};
void launch_decode_gate_up(const DecodeGateUpArgs & d, hipStream_t stream);

// Kernel B of the fused single-token decode: down GEMV + bias of every routed rank into y.
struct DecodeDownParams {
    const vbm_bank * bank;
    const int32_t * expert_to_slot;
    const float * act_f;              // [top_k][intermediate] GLU outputs from kernel A
    XrowLayout act_layout;
    const int32_t * route_ids;        // [top_k]
    const int32_t * route_slots;      // [top_k] from kernel A with the same expert_to_slot, or null
    int64_t top_k;
    const float * bias;               // [n_expert][hidden] or null
    float * y;                        // [top_k][hidden]
    const uint8_t * host_base = nullptr;   // as in DecodeGateUpArgs (the down bank's slot layout)
    int64_t host_stride = 0;
    uint8_t * stage = nullptr;             // as in DecodeGateUpArgs
    int64_t stage_stride = 0;
};
void launch_decode_down(const DecodeDownParams & d, hipStream_t stream);

// One launch of the linked single-token decode: the down tiles of layer l - 1 (dn_bank non-null)
// and the gate_up tiles of layer l (gu_bank non-null) in one grid; the down tiles publish layer
// l's Q8_0 input row tile by tile (xq, flags) or, in the last launch, combine into `out`.
struct DecodeLinkParams {
    const vbm_bank * dn_bank = nullptr;
    const float * dn_act_f = nullptr;   // [top_k][intermediate] GLU outputs of layer l - 1
    const int32_t * dn_ids = nullptr;   // routing of layer l - 1 [top_k]
    const int32_t * dn_slots = nullptr;
    const float * dn_w = nullptr;
    const float * dn_bias = nullptr;
    float * y = nullptr;                // [top_k][hidden]
    uint32_t * counters = nullptr;      // [hidden / 32] arrival counters of layer l - 1
    float * out = nullptr;              // last launch: the step output [hidden]
    uint8_t * xq = nullptr;             // layer l's input row (gate_up activation layout)
    uint32_t * flags = nullptr;         // layer l's tile flags [kLinkFlagWords]
    const vbm_bank * gu_bank = nullptr;
    const int32_t * expert_to_slot = nullptr;
    const float * logits = nullptr;     // [n_expert] of layer l
    const float * x_in = nullptr;       // first launch: the layer input
    const float * gu_bias = nullptr;
    float * act_f = nullptr;            // [top_k][intermediate] GLU outputs of layer l
    int32_t * route_ids = nullptr;
    float * route_w = nullptr;
    int32_t * route_slots = nullptr;
    int64_t n_expert = 0, top_k = 0;
    int activation = 0;
    float alpha = 1.702f, limit = 7.0f;
    uint32_t * epoch = nullptr;         // device step counter
    bool advance_epoch = false;         // last launch
    uint32_t * error = nullptr;         // device word set to 1 by a timed-out wait
};
constexpr int64_t kLinkFlagWords = 8 * 1152;   // flag words per layer (8 copies)
// Shapes the linked decode is built for: MXFP4, hidden = intermediate = 2880 (90 blocks per row),
// at most 128 experts.
bool decode_link_supported(const vbm_bank & gate_up, const vbm_bank & down, int64_t n_expert, int64_t top_k);
void launch_decode_link(const DecodeLinkParams & d, hipStream_t stream);

// Ops-API device scratch reused per (device, stream); see vbm_ops.cpp.
void * stream_scratch(hipStream_t s, size_t bytes);
void release_stream_scratch(hipStream_t s);   // before the stream is destroyed

// GGML_OP_MUL_MAT_ID over a caller-provided scratch of mul_mat_id_scratch_bytes(). b_row_stride:
// floats between consecutive F32 rows of b (0 = contiguous rows of k floats); Q8_0 b is contiguous.
void check_mul_mat_id_shape(const vbm_bank & bank, int64_t n_as, int64_t b_ne1, int64_t n_ids, int64_t n_tokens,
                            int64_t ids_stride, int order);
size_t mul_mat_id_scratch_bytes(const vbm_bank & bank, int64_t n_as, int64_t b_ne1, int64_t n_ids, int64_t n_tokens,
                                int order);
void mul_mat_id(const vbm_bank * bank, const int32_t * expert_to_slot, const int32_t * expert_to_slot_host, int64_t n_as,
                int b_type, const void * b, int64_t b_ne1, const int32_t * ids, int64_t n_ids, int64_t n_tokens,
                int64_t ids_stride, const float * bias, float * dst, int order, uint8_t * scratch, size_t scratch_bytes,
                hipStream_t s, int64_t b_row_stride = 0);

}  // namespace vbm
