// C ABI: ggml-level operators and the fused routed-expert layer.
#include "vbm_internal.hpp"

#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <utility>
#include <vector>

using namespace vbm;

struct vbm_decode_plan {
    std::vector<vbm_moe_layer_desc> layers;
    int64_t L = 0, H = 0, I = 0, E = 0, K = 0;
    int device = 0;
    uint8_t * workspace = nullptr;
    int32_t * route_ids = nullptr;   // [L][K]
    float * route_w = nullptr;       // [L][K]
    int32_t * route_slots = nullptr; // [L][K] bank slots of the picks (kernel A -> kernel B)
    float * act_f = nullptr;         // [2][K][I] GLU outputs (kernel A -> kernel B; the linked step
                                     // alternates the halves by layer parity)
    XrowLayout act_layout{};
    float * y = nullptr;             // [K][H]
    // linked step (one launch per layer boundary)
    bool linked = false;             // the step runs the linked launches
    bool link_ok = false;            // the plan's shapes allow them
    uint8_t * xq = nullptr;          // next-layer input row (gate_up activation layout)
    uint32_t * flags = nullptr;      // [L][kLinkFlagWords]
    uint32_t * counters = nullptr;   // [L][H / 32]
    uint32_t * epoch = nullptr;      // step counter (starts at 1; flags start at 0)
    uint32_t * error = nullptr;      // timed-out waits
};

namespace {

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// MUL_MAT_ID output rows the expert kernels do not write: 0 for the rows of -1 ids
// (hybrid-experts.patch:617-621), NaN for ids outside [-1, n_as), which the grouping pass skips
// (the reference asserts on them, :622), so an invalid id is loud in the output even when no host
// copy of the ids was given for checking. Rows of routed ids are left to the expert kernels, which
// write every one of them (NaN where the expert has no slot).
// One workgroup per (token, rank) entry: a routed entry returns at once (its row is written by
// the expert kernels), a -1 entry gets a zero row and an invalid id a NaN row.
__global__ void init_dst_kernel(float * dst, const int32_t * ids, int64_t n_ids, int64_t ids_stride, int64_t n_as,
                                int64_t rows) {
    const int64_t entry = blockIdx.x, t = entry / n_ids, r = entry - t * n_ids;
    const int32_t id = ids[t * ids_stride + r];
    if (id >= 0 && id < n_as) return;
    const float v = id == -1 ? 0.0f : __builtin_nanf("");
    float * row = dst + entry * rows;
    for (int64_t i = threadIdx.x; i < rows; i += blockDim.x) row[i] = v;
}

void init_dst(float * dst, const int32_t * ids, int64_t n_ids, int64_t n_tokens, int64_t ids_stride, int64_t n_as,
              int64_t rows, hipStream_t stream) {
    const int64_t entries = n_ids * n_tokens;
    if (entries <= 0 || rows <= 0) return;
    require(entries < (int64_t{1} << 25), "too many MUL_MAT_ID entries for one launch");   // 128 x entries work-items
    hipLaunchKernelGGL(init_dst_kernel, dim3(static_cast<unsigned>(entries)), dim3(128), 0, stream, dst, ids, n_ids,
                       ids_stride, n_as, rows);
    check_hip(hipGetLastError(), "output init launch");
}

// Synchronous host-side validation of device ids against an expert->slot map (the reference's
// per-job residency check, tools/engine/quantized_cuda.cu:224-227).
void validate_ids_on_host(const int32_t * ids, int64_t n_ids, int64_t n_tokens, int64_t ids_stride, int64_t n_as,
                          const int32_t * expert_to_slot_host, hipStream_t stream) {
    std::vector<int32_t> host(static_cast<size_t>(ids_stride * (n_tokens - 1) + n_ids));
    check_hip(hipMemcpyAsync(host.data(), ids, host.size() * sizeof(int32_t), hipMemcpyDeviceToHost, stream), "ids copy");
    check_hip(hipStreamSynchronize(stream), "ids copy synchronize");
    for (int64_t t = 0; t < n_tokens; ++t)
        for (int64_t r = 0; r < n_ids; ++r) {
            const int32_t id = host[t * ids_stride + r];
            if (id == -1) continue;
            require(id >= 0 && id < n_as, "expert id out of range");
            require(expert_to_slot_host[id] >= 0, "expert is out of range or not resident");
        }
}

}  // namespace

namespace vbm {

// Layers of at least kGemmMinTokens tokens in the fast accumulation order may run the MFMA
// grouped GEMM: their workspace holds either path's layout. The forward takes the GEMM when it
// pays (gemm_pays: enough routed rows per expert), else the exact GEMV path, whose results
// satisfy either order.
bool use_gemm(const vbm_moe_layer_desc & d, int64_t n_tokens) {
    return d.order == VBM_ORDER_FAST && n_tokens >= kGemmMinTokens;
}

LayerWorkspace plan_layer(const vbm_moe_layer_desc & d, int64_t max_tokens, uint8_t * base) {
    LayerWorkspace w{};
    size_t off = 0;
    auto take = [&](size_t bytes) { uint8_t * p = base ? base + off : nullptr; off += align_up(bytes); return p; };
    const int64_t entries = max_tokens * d.top_k;
    w.ids = reinterpret_cast<int32_t *>(take(sizeof(int32_t) * entries));
    w.weights = reinterpret_cast<float *>(take(sizeof(float) * entries));
    w.logits = reinterpret_cast<float *>(take(sizeof(float) * max_tokens * d.n_expert));
    const int type = d.gate_up ? d.gate_up->type : VBM_TYPE_MXFP4;
    const XrowLayout lx{d.hidden / 32, type};
    const XrowLayout la{d.intermediate / 32, type};
    const GemmRowLayout gx{d.hidden / 32, type};
    const GemmRowLayout ga{d.intermediate / 32, type};
    const bool gemm = use_gemm(d, max_tokens);
    w.xrows_x = take(static_cast<size_t>(max_tokens * (gemm ? std::max(gx.stride(), lx.stride()) : lx.stride())));
    w.group = take(group_workspace_bytes(d.n_expert, entries));
    w.xrows_act = take(static_cast<size_t>(entries * (gemm ? std::max(ga.stride(), la.stride()) : la.stride())));
    w.tiles = gemm ? take(gemm_tiles_bytes(d.n_expert, entries)) : nullptr;
    w.y = reinterpret_cast<float *>(take(sizeof(float) * entries * d.hidden));
    w.total = off;
    return w;
}

void prefill_prepare(const vbm_moe_layer_desc & d, const float * x, const int32_t * ids, int64_t n_tokens,
                     const LayerWorkspace & w, hipStream_t s, bool gemm_tiles, const float * logits, float * weights) {
    const GemmRowLayout gx{d.hidden / 32, d.gate_up->type};
    if (logits)
        launch_topk_gemm_rows(logits, d.n_expert, d.top_k, const_cast<int32_t *>(ids), weights, x, n_tokens, d.hidden, gx,
                              w.xrows_x, s);
    else
        launch_gemm_rows_from_f32(x, n_tokens, d.hidden, d.hidden, gx, w.xrows_x, s);
    const int64_t entries = n_tokens * d.top_k;
    const GroupBuffers g = carve_group(w.group, d.n_expert, entries);
    if (gemm_tiles)   // the grouping scan also writes the GEMM's (unfiltered) job tile list
        launch_group(ids, d.top_k, n_tokens, d.top_k, d.n_expert, g, s, gemm_job_tile(d.gate_up->type),
                     static_cast<int32_t *>(w.tiles), gemm_max_tiles(d.n_expert, entries, gemm_job_tile(d.gate_up->type)));
    else
        launch_group(ids, d.top_k, n_tokens, d.top_k, d.n_expert, g, s);
}

void prefill_pass(const vbm_moe_layer_desc & d, const int32_t * expert_to_slot, int64_t n_tokens,
                  const LayerWorkspace & w, const float * route_w, void * const * events, hipStream_t s,
                  int64_t grid_tiles, bool tiles_ready) {
    const int64_t K = d.top_k;
    const GemmRowLayout gx{d.hidden / 32, d.gate_up->type}, ga{d.intermediate / 32, d.down->type};
    GemmParams p{};
    p.expert_to_slot = expert_to_slot;
    p.n_ids = K;
    p.n_as = d.n_expert;
    p.n_entries = n_tokens * K;
    p.group = carve_group(w.group, d.n_expert, n_tokens * K);
    p.tiles = w.tiles;
    p.activation = d.activation;
    p.alpha = 1.702f;
    p.limit = 7.0f;
    if (grid_tiles > 0) {
        p.tile_filter = expert_to_slot;
        p.grid_tiles = grid_tiles;
    }
    p.tiles_ready = tiles_ready;
    p.bank = d.gate_up;
    p.rows_in = w.xrows_x;
    p.lay = gx;
    p.b_ne1 = 1;
    p.bias = d.gate_up_bias;
    p.rows_out = w.xrows_act;
    p.out_layout = ga;
    p.epilogue = 1;
    if (events) check_hip(hipEventRecord(static_cast<hipEvent_t>(events[0]), s), "hipEventRecord");
    launch_grouped_gemm(p, s);
    if (events) check_hip(hipEventRecord(static_cast<hipEvent_t>(events[1]), s), "hipEventRecord");
    p.bank = d.down;
    p.tiles_ready = true;                 // same group and tile filter as the gate_up pass
    p.rows_in = w.xrows_act;
    p.lay = ga;
    p.b_ne1 = K;
    p.bias = d.down_bias;
    p.row_scale = route_w;
    p.dst = w.y;
    p.rows_out = nullptr;
    p.epilogue = 0;
    if (events) check_hip(hipEventRecord(static_cast<hipEvent_t>(events[2]), s), "hipEventRecord");
    launch_grouped_gemm(p, s);
    if (events) check_hip(hipEventRecord(static_cast<hipEvent_t>(events[3]), s), "hipEventRecord");
}

// Per-(device, stream) scratch reused by the ops API entry points that need device scratch
// (vbm_mul_mat_id, vbm_group_by_expert): it grows, stream-ordered, only when a call needs more
// than any earlier call on that stream, so steady-state calls allocate nothing. Calls on one
// stream are ordered, so they may share it; other streams get their own.
namespace {
struct ScratchCache {
    std::mutex mu;
    std::map<std::pair<int, hipStream_t>, std::pair<void *, size_t>> entries;   // (device, stream) -> (ptr, bytes)
};
ScratchCache & scratch_cache() {
    static ScratchCache cache;
    return cache;
}
}  // namespace

void * stream_scratch(hipStream_t s, size_t bytes) {
    int device = 0;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    ScratchCache & c = scratch_cache();
    std::lock_guard<std::mutex> lock(c.mu);
    auto & e = c.entries[{device, s}];
    if (e.second < bytes) {
        // Growing is stream-ordered allocation; under capture it would become a graph-owned
        // allocation that eager calls cannot use and relaunches cannot reuse.
        require(!stream_capturing(s),
                "this call needs more ops-API scratch than the capturing stream holds: run it once on the stream "
                "before capture, or use vbm_mul_mat_id_ws / vbm_mul_mat_id_noalloc");
        if (e.first) check_hip(hipFreeAsync(e.first, s), "scratch release");
        e = {nullptr, 0};
        const size_t cap = std::max<size_t>(bytes + (bytes >> 2), size_t(1) << 20);
        check_hip(hipMallocAsync(&e.first, cap, s), "scratch");
        e.second = cap;
    }
    return e.first;
}

void release_stream_scratch(hipStream_t s) {
    int device = 0;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    ScratchCache & c = scratch_cache();
    std::lock_guard<std::mutex> lock(c.mu);
    auto it = c.entries.find({device, s});
    if (it == c.entries.end()) return;
    if (it->second.first) check_hip(hipFreeAsync(it->second.first, s), "scratch release");
    c.entries.erase(it);
}

void check_mul_mat_id_shape(const vbm_bank & bank, int64_t n_as, int64_t b_ne1, int64_t n_ids, int64_t n_tokens,
                            int64_t ids_stride, int order) {
    require(order == VBM_ORDER_EXACT || order == VBM_ORDER_FAST, "unknown order");
    require(n_ids > 0 && n_tokens > 0 && (b_ne1 == 1 || b_ne1 == n_ids), "b_ne1 must be 1 or n_ids");
    require(ids_stride >= n_ids, "ids stride must be >= n_ids");
    require(n_as > 0 && n_as <= 1024, "n_as must be in 1..1024");
    (void)bank;
}

size_t mul_mat_id_scratch_bytes(const vbm_bank & bank, int64_t n_as, int64_t b_ne1, int64_t n_ids, int64_t n_tokens,
                                int order) {
    const int64_t entries = n_ids * n_tokens, n_b = b_ne1 * n_tokens;
    if (order == VBM_ORDER_FAST && gemm_pays(n_tokens, n_ids, n_as)) {
        const GemmRowLayout gl{bank.nb, bank.type};
        return align_up(static_cast<size_t>(n_b * gl.stride())) + align_up(group_workspace_bytes(n_as, entries)) +
               gemm_tiles_bytes(n_as, entries);
    }
    const XrowLayout lay{bank.nb, bank.type};
    return align_up(static_cast<size_t>(n_b * lay.stride())) + group_workspace_bytes(n_as, entries);
}

void mul_mat_id(const vbm_bank * bank, const int32_t * expert_to_slot, const int32_t * expert_to_slot_host, int64_t n_as,
                int b_type, const void * b, int64_t b_ne1, const int32_t * ids, int64_t n_ids, int64_t n_tokens,
                int64_t ids_stride, const float * bias, float * dst, int order, uint8_t * scratch, size_t scratch_bytes,
                hipStream_t s, int64_t b_row_stride) {
    require(bank && b && ids && dst && scratch, "null buffer");
    require(b_type == VBM_TYPE_F32 || b_type == VBM_TYPE_Q8_0, "b must be F32 or Q8_0");
    if (b_row_stride == 0) b_row_stride = bank->k;
    require(b_row_stride >= bank->k && (b_type == VBM_TYPE_F32 || b_row_stride == bank->k),
            "b rows must be at least k floats apart (Q8_0 b must be contiguous)");
    check_mul_mat_id_shape(*bank, n_as, b_ne1, n_ids, n_tokens, ids_stride, order);
    require(expert_to_slot != nullptr || n_as <= bank->n_slots, "identity map needs n_as <= bank slots");
    require(scratch_bytes >= mul_mat_id_scratch_bytes(*bank, n_as, b_ne1, n_ids, n_tokens, order), "workspace too small");
    if (expert_to_slot_host) validate_ids_on_host(ids, n_ids, n_tokens, ids_stride, n_as, expert_to_slot_host, s);
    const int64_t entries = n_ids * n_tokens;
    const int64_t n_b = b_ne1 * n_tokens;
    if (order == VBM_ORDER_FAST && gemm_pays(n_tokens, n_ids, n_as)) {
        const GemmRowLayout gl{bank->nb, bank->type};
        const size_t q_bytes = align_up(static_cast<size_t>(n_b * gl.stride()));
        const size_t g_bytes = align_up(group_workspace_bytes(n_as, entries));
        uint8_t * q = scratch;
        const GroupBuffers g = carve_group(q + q_bytes, n_as, entries);
        if (b_type == VBM_TYPE_F32)
            launch_gemm_rows_from_f32(static_cast<const float *>(b), n_b, bank->k, b_row_stride, gl, q, s);
        else
            launch_gemm_rows_from_q8(static_cast<const uint8_t *>(b), n_b, bank->nb * 34, gl, q, s);
        launch_group(ids, n_ids, n_tokens, ids_stride, n_as, g, s);
        init_dst(dst, ids, n_ids, n_tokens, ids_stride, n_as, bank->rows, s);
        GemmParams p{};
        p.bank = bank;
        p.expert_to_slot = expert_to_slot;
        p.rows_in = q;
        p.lay = gl;
        p.n_ids = n_ids;
        p.b_ne1 = b_ne1;
        p.n_as = n_as;
        p.n_entries = entries;
        p.group = g;
        p.tiles = q + q_bytes + g_bytes;
        p.bias = bias;
        p.dst = dst;
        p.epilogue = 0;
        p.flagged_rows = b_type != VBM_TYPE_F32;
        launch_grouped_gemm(p, s);
        return;
    }
    const XrowLayout lay{bank->nb, bank->type};
    const size_t q_bytes = align_up(static_cast<size_t>(n_b * lay.stride()));
    uint8_t * q = scratch;
    const GroupBuffers g = carve_group(q + q_bytes, n_as, entries);
    if (b_type == VBM_TYPE_F32)
        launch_quantize_expand(static_cast<const float *>(b), n_b, bank->k, b_row_stride, lay, q, nullptr, s);
    else
        launch_expand_q8(static_cast<const uint8_t *>(b), n_b, bank->nb * 34, lay, q, s);
    launch_group(ids, n_ids, n_tokens, ids_stride, n_as, g, s, gemv_chunk_tokens(entries));
    init_dst(dst, ids, n_ids, n_tokens, ids_stride, n_as, bank->rows, s);
    GemvArgs a{};
    a.bank = bank;
    a.expert_to_slot = expert_to_slot;
    a.xrows = q;
    a.n_ids = n_ids;
    a.b_ne1 = b_ne1;
    a.group = g;
    a.max_active = std::min<int64_t>(n_as, entries);
    a.max_per_expert = entries;
    a.n_entries = entries;
    a.chunks_built = true;
    a.bias = bias;
    a.dst = dst;
    a.epilogue = 0;
    a.may_have_neg128 = b_type != VBM_TYPE_F32;   // ggml Q8_0 rows may hold -128 codes
    launch_gemv(a, s);
}

}  // namespace vbm

namespace {

void validate_layer(const vbm_moe_layer_desc * d) {
    require(d != nullptr && d->gate_up != nullptr && d->down != nullptr, "layer needs gate_up and down banks");
    const vbm_bank & gu = *d->gate_up, & dn = *d->down;
    require(gu.interleave == 1, "gate_up bank must be created with interleave = 1");
    require(gu.type == dn.type, "gate_up and down banks must share a type");
    require(gu.rows == 2 * d->intermediate && gu.k == d->hidden, "gate_up bank shape must be [2*I rows, H]");
    require(dn.rows == d->hidden && dn.k == d->intermediate, "down bank shape must be [H rows, I]");
    require(d->hidden % 64 == 0 && d->intermediate % 64 == 0, "hidden and intermediate must be multiples of 64");
    require(d->n_expert > 0 && d->n_expert <= 1024 && d->top_k > 0 && d->top_k <= d->n_expert && d->top_k <= 64,
            "expert count / top_k out of range");
    require(d->expert_to_slot != nullptr || (gu.n_slots >= d->n_expert && dn.n_slots >= d->n_expert),
            "identity expert->slot map needs a slot per expert");
    require(d->activation == VBM_ACT_SILU || d->activation == VBM_ACT_SWIGLU_OAI, "unknown activation");
}


__global__ void copy_kernel(uint4 * __restrict__ dst, const uint4 * __restrict__ src, size_t n) {
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x)
        dst[i] = src[i];
}

// Under stream capture the record becomes an event-record node of the graph, so events bracketing
// kernels time every replay.
void record(void * const * events, int i, hipStream_t s) {
    if (events) record_event(static_cast<hipEvent_t>(events[i]), s, "hipEventRecord");
}

void layer_forward(const vbm_moe_layer_desc * d, const float * x, float * logits, int64_t n_tokens, float * out,
                   int32_t * ids, float * weights, void * workspace, size_t workspace_bytes, void * const * events,
                   hipStream_t s) {
    validate_layer(d);
    require(x && out && workspace && n_tokens > 0, "null buffer");
    require(d->router_w != nullptr || logits != nullptr, "logits input required when router_w is NULL");
    const LayerWorkspace w = plan_layer(*d, n_tokens, static_cast<uint8_t *>(workspace));
    require(workspace_bytes >= w.total, "workspace too small");
    const int64_t K = d->top_k, H = d->hidden, I = d->intermediate, entries = n_tokens * K;
    int32_t * ids_d = ids ? ids : w.ids;
    float * w_d = weights ? weights : w.weights;
    float * logits_d = logits ? logits : w.logits;
    const GroupBuffers g = carve_group(w.group, d->n_expert, entries);
    const bool gemm = use_gemm(*d, n_tokens) && gemm_pays(n_tokens, K, d->n_expert);
    const bool one_launch = !gemm && route_group_fits(d->n_expert, n_tokens, K);
    launch_router(d->router_w, d->router_b, x, H, logits_d, d->n_expert, n_tokens, K, ids_d, w_d, s, false);
    if (gemm) {
        // Prefill-sized groups: MFMA grouped GEMM (exact block dots, fp32 accumulation order); the
        // top-k runs in the launch that writes the activation rows.
        prefill_prepare(*d, x, ids_d, n_tokens, w, s, true, logits_d, w_d);
        prefill_pass(*d, d->expert_to_slot, n_tokens, w, w_d, events, s, 0, true);
        launch_combine(w.y, nullptr, H, K, n_tokens, out, s);   // rows weighted in the down epilogue
        return;
    }
    const XrowLayout lx{H / 32, d->gate_up->type}, la{I / 32, d->down->type};
    if (one_launch) {
        // top-k + softmax, grouping with the job chunks, and the input's activation rows
        launch_route_group_quantize(logits_d, d->n_expert, n_tokens, K, ids_d, w_d, g, x, H, lx, w.xrows_x, s);
    } else {
        launch_topk_quantize(logits_d, d->n_expert, n_tokens, K, ids_d, w_d, x, H, lx, w.xrows_x, s);
        launch_group(ids_d, K, n_tokens, K, d->n_expert, g, s, gemv_chunk_tokens(n_tokens));
    }

    GemvArgs a{};
    a.expert_to_slot = d->expert_to_slot;
    a.n_ids = K;
    a.group = g;
    a.max_active = std::min<int64_t>(d->n_expert, entries);
    a.max_per_expert = n_tokens;                 // top-k experts are distinct within a token
    a.n_entries = entries;
    a.chunks_built = true;                       // by launch_group, for both projections
    a.activation = d->activation;
    a.alpha = 1.702f;
    a.limit = 7.0f;
    // gate_up + biases + GLU + Q8_0 requantization -> down activation rows [entries]
    a.bank = d->gate_up;
    a.xrows = w.xrows_x;
    a.b_ne1 = 1;
    a.bias = d->gate_up_bias;
    a.dst_xrows = w.xrows_act;
    a.dst_layout = la;
    a.epilogue = 1;
    a.may_have_neg128 = false;               // fp32 input, and the GLU requantization feeds down
    record(events, 0, s);
    launch_gemv(a, s);
    record(events, 1, s);
    // down + bias -> y [entries][H]
    a.bank = d->down;
    a.xrows = w.xrows_act;
    a.b_ne1 = K;
    a.bias = d->down_bias;
    a.dst = w.y;
    a.epilogue = 0;
    record(events, 2, s);
    launch_gemv(a, s);
    record(events, 3, s);
    launch_combine(w.y, w_d, H, K, n_tokens, out, s);
}

}  // namespace

extern "C" {

vbm_status vbm_quantize_q8_0(const float * x, int64_t n_rows, int64_t k, int64_t x_stride, void * dst, void * stream) {
    return guarded([&] {
        require(x != nullptr && dst != nullptr, "null buffer");
        launch_quantize_q8_0(x, n_rows, k, x_stride, static_cast<uint8_t *>(dst), as_stream(stream));
    });
}

vbm_status vbm_group_by_expert(const int32_t * ids, int64_t n_ids, int64_t n_tokens, int64_t ids_stride, int64_t n_as,
                               int32_t * counts, int32_t * offsets, int32_t * rows, int32_t * error_flag, void * stream) {
    return guarded([&] {
        require(ids && counts && offsets && rows, "null buffer");
        require(n_as > 0 && n_ids > 0 && n_tokens > 0, "grouping sizes must be positive");
        const hipStream_t s = as_stream(stream);
        const int64_t chunk_ints = group_chunk_ints(n_as, n_ids * n_tokens);
        auto * scratch = static_cast<int32_t *>(stream_scratch(s, sizeof(int32_t) * (n_as + 2 + chunk_ints + 8)));
        GroupBuffers g{};
        g.counts = counts;
        g.offsets = offsets;
        g.rows = rows;
        g.active = scratch;
        g.n_active = g.active + n_as;
        g.chunk_counts = g.n_active + 2;
        g.error = error_flag ? error_flag : g.n_active + 1;
        launch_group(ids, n_ids, n_tokens, ids_stride, n_as, g, s);
    });
}

vbm_status vbm_mul_mat_id_workspace(const vbm_bank * bank, int64_t n_as, int64_t b_ne1, int64_t n_ids, int64_t n_tokens,
                                    int order, size_t * bytes) {
    return guarded([&] {
        require(bank != nullptr && bytes != nullptr, "null argument");
        check_mul_mat_id_shape(*bank, n_as, b_ne1, n_ids, n_tokens, n_ids, order);
        *bytes = mul_mat_id_scratch_bytes(*bank, n_as, b_ne1, n_ids, n_tokens, order);
    });
}

vbm_status vbm_mul_mat_id_ws(const vbm_bank * bank, const int32_t * expert_to_slot, const int32_t * expert_to_slot_host,
                             int64_t n_as, int b_type, const void * b, int64_t b_ne1, const int32_t * ids, int64_t n_ids,
                             int64_t n_tokens, int64_t ids_stride, const float * bias, float * dst, int order,
                             void * workspace, size_t workspace_bytes, void * stream) {
    return guarded([&] {
        require(workspace != nullptr, "null workspace");
        mul_mat_id(bank, expert_to_slot, expert_to_slot_host, n_as, b_type, b, b_ne1, ids, n_ids, n_tokens, ids_stride,
                   bias, dst, order, static_cast<uint8_t *>(workspace), workspace_bytes, as_stream(stream));
    });
}

vbm_status vbm_mul_mat_id(const vbm_bank * bank, const int32_t * expert_to_slot, const int32_t * expert_to_slot_host,
                          int64_t n_as, int b_type, const void * b, int64_t b_ne1, const int32_t * ids, int64_t n_ids,
                          int64_t n_tokens, int64_t ids_stride, const float * bias, float * dst, int order,
                          void * stream) {
    return guarded([&] {
        require(bank != nullptr, "null bank");
        check_mul_mat_id_shape(*bank, n_as, b_ne1, n_ids, n_tokens, ids_stride, order);
        const hipStream_t s = as_stream(stream);
        const size_t bytes = mul_mat_id_scratch_bytes(*bank, n_as, b_ne1, n_ids, n_tokens, order);
        mul_mat_id(bank, expert_to_slot, expert_to_slot_host, n_as, b_type, b, b_ne1, ids, n_ids, n_tokens, ids_stride,
                   bias, dst, order, static_cast<uint8_t *>(stream_scratch(s, bytes)), bytes, s);
    });
}

vbm_status vbm_mul_mat_id_mxfp8(const vbm_bank * bank, const int32_t * expert_to_slot, int64_t n_as, const float * b,
                                int64_t b_ne1, const int32_t * ids, int64_t n_ids, int64_t n_tokens,
                                int64_t ids_stride, float * dst, void * stream) {
    return guarded([&] {
        require(bank != nullptr && b != nullptr && ids != nullptr && dst != nullptr, "null buffer");
        require(bank->type == VBM_TYPE_MXFP4, "the MXFP8 path needs an MXFP4 bank");
        check_mul_mat_id_shape(*bank, n_as, b_ne1, n_ids, n_tokens, ids_stride, VBM_ORDER_FAST);
        require(expert_to_slot != nullptr || n_as <= bank->n_slots, "identity map needs n_as <= bank slots");
        const hipStream_t s = as_stream(stream);
        const int64_t entries = n_ids * n_tokens, n_b = b_ne1 * n_tokens;
        const size_t c_bytes = align_up(static_cast<size_t>(n_b * bank->k));
        const size_t s_bytes = align_up(static_cast<size_t>(n_b * bank->nb));
        const size_t g_bytes = align_up(group_workspace_bytes(n_as, entries));
        auto * base = static_cast<uint8_t *>(stream_scratch(s, c_bytes + s_bytes + g_bytes + gemm_tiles_bytes(n_as, entries)));
        const GroupBuffers g = carve_group(base + c_bytes + s_bytes, n_as, entries);
        launch_quantize_mxfp8(b, n_b, bank->k, bank->k, base, base + c_bytes, s);
        launch_group(ids, n_ids, n_tokens, ids_stride, n_as, g, s);
        init_dst(dst, ids, n_ids, n_tokens, ids_stride, n_as, bank->rows, s);
        launch_mx_gemm(*bank, expert_to_slot, base, base + c_bytes, n_ids, b_ne1, n_as, entries, g,
                       base + c_bytes + s_bytes + g_bytes, dst, s);
    });
}

vbm_status vbm_quantize_mxfp8(const float * x, int64_t n_rows, int64_t k, int64_t x_stride, void * codes, void * scales,
                              void * stream) {
    return guarded([&] {
        require(x && codes && scales, "null buffer");
        launch_quantize_mxfp8(x, n_rows, k, x_stride, static_cast<uint8_t *>(codes), static_cast<uint8_t *>(scales),
                              as_stream(stream));
    });
}

vbm_status vbm_glu(int activation, const float * gate, const float * up, float * out, int64_t n_rows, int64_t width,
                   int64_t gate_stride, int64_t up_stride, int64_t out_stride, float alpha, float limit, void * stream) {
    return guarded([&] {
        require(gate && up && out && n_rows > 0 && width > 0, "invalid glu");
        require(activation == VBM_ACT_SILU || activation == VBM_ACT_SWIGLU_OAI, "unknown activation");
        launch_glu(activation, gate, up, out, n_rows, width, gate_stride, up_stride, out_stride, alpha, limit,
                   as_stream(stream));
    });
}

vbm_status vbm_router_topk_softmax(const float * router_w, const float * router_b, const float * x, int64_t k_hidden,
                                   float * logits, int64_t n_expert, int64_t n_tokens, int64_t top_k, int32_t * ids,
                                   float * weights, void * stream) {
    return guarded([&] {
        require(ids && weights && logits, "router needs logits, ids and weights buffers");
        launch_router(router_w, router_b, x, k_hidden, logits, n_expert, n_tokens, top_k, ids, weights, as_stream(stream));
    });
}

vbm_status vbm_weighted_combine(const float * y, const float * weights, int64_t rows, int64_t n_ids, int64_t n_tokens,
                                float * out, void * stream) {
    return guarded([&] {
        require(y && weights && out && rows > 0 && n_ids > 0 && n_tokens > 0, "invalid combine");
        launch_combine(y, weights, rows, n_ids, n_tokens, out, as_stream(stream));
    });
}

vbm_status vbm_moe_layer_workspace(const vbm_moe_layer_desc * desc, int64_t max_tokens, size_t * bytes) {
    return guarded([&] {
        validate_layer(desc);
        require(bytes != nullptr && max_tokens > 0, "invalid workspace query");
        *bytes = plan_layer(*desc, max_tokens, nullptr).total;
    });
}

vbm_status vbm_moe_layer_forward(const vbm_moe_layer_desc * d, const float * x, float * logits, int64_t n_tokens,
                                 float * out, int32_t * ids, float * weights, void * workspace, size_t workspace_bytes,
                                 void * stream) {
    return guarded([&] { layer_forward(d, x, logits, n_tokens, out, ids, weights, workspace, workspace_bytes, nullptr,
                                       as_stream(stream)); });
}

vbm_status vbm_moe_layer_forward_profiled(const vbm_moe_layer_desc * d, const float * x, float * logits,
                                          int64_t n_tokens, float * out, int32_t * ids, float * weights,
                                          void * workspace, size_t workspace_bytes, void * const * events,
                                          void * stream) {
    return guarded([&] {
        require(events != nullptr && events[0] && events[1] && events[2] && events[3], "four events required");
        layer_forward(d, x, logits, n_tokens, out, ids, weights, workspace, workspace_bytes, events, as_stream(stream));
    });
}

vbm_status vbm_graph_begin_capture(void * stream) {
    return guarded([&] {
        require(stream != nullptr, "graph capture needs a non-default stream");
        check_hip(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    });
}

vbm_status vbm_graph_end_capture(void * stream, void ** graph_exec) {
    return guarded([&] {
        require(graph_exec != nullptr, "graph_exec is null");
        hipGraph_t graph = nullptr;
        check_hip(hipStreamEndCapture(as_stream(stream), &graph), "hipStreamEndCapture");
        hipGraphExec_t exec = nullptr;
        const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        check_hip(e, "hipGraphInstantiate");
        *graph_exec = exec;
    });
}

vbm_status vbm_graph_launch(void * graph_exec, void * stream) {
    return guarded([&] {
        require(graph_exec != nullptr, "graph_exec is null");
        check_hip(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), as_stream(stream)), "hipGraphLaunch");
    });
}

vbm_status vbm_graph_destroy(void * graph_exec) {
    return guarded([&] {
        if (graph_exec) check_hip(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)), "hipGraphExecDestroy");
    });
}

vbm_status vbm_copy_kernel(void * dst, const void * src, size_t bytes, void * stream) {
    return guarded([&] {
        require(dst && src && bytes % 16 == 0, "copy needs 16-byte multiples");
        const size_t n = bytes / 16;
        if (!n) return;
        const unsigned blocks = static_cast<unsigned>(std::min<size_t>((n + 255) / 256, 1u << 20));
        hipLaunchKernelGGL(copy_kernel, dim3(blocks), dim3(256), 0, as_stream(stream),
                           static_cast<uint4 *>(dst), static_cast<const uint4 *>(src), n);
        check_hip(hipGetLastError(), "copy launch");
    });
}

vbm_status vbm_decode_plan_create(const vbm_moe_layer_desc * layers, int64_t n_layers, vbm_decode_plan ** out) {
    return guarded([&] {
        require(out != nullptr && layers != nullptr && n_layers > 0, "invalid decode plan arguments");
        *out = nullptr;
        for (int64_t l = 0; l < n_layers; ++l) {
            validate_layer(&layers[l]);
            require(layers[l].router_w == nullptr, "fused decode needs given router logits (router_w == NULL)");
            require(layers[l].hidden == layers[0].hidden && layers[l].intermediate == layers[0].intermediate &&
                        layers[l].n_expert == layers[0].n_expert && layers[l].top_k == layers[0].top_k &&
                        layers[l].gate_up->type == layers[0].gate_up->type,
                    "all decode layers must share one shape and type");
            require(layers[l].gate_up->rows % 64 == 0, "fused decode needs 2*intermediate % 64 == 0");
        }
        auto plan = std::make_unique<vbm_decode_plan>();
        plan->layers.assign(layers, layers + n_layers);
        plan->L = n_layers;
        plan->H = layers[0].hidden;
        plan->I = layers[0].intermediate;
        plan->E = layers[0].n_expert;
        plan->K = layers[0].top_k;
        check_hip(hipGetDevice(&plan->device), "hipGetDevice");
        plan->act_layout = XrowLayout{plan->I / 32, layers[0].down->type};
        plan->link_ok = true;
        for (int64_t l = 0; l < n_layers; ++l)
            plan->link_ok = plan->link_ok && decode_link_supported(*layers[l].gate_up, *layers[l].down, plan->E, plan->K);
        plan->linked = false;   // opt-in: measured slower than two kernels per layer
        const XrowLayout xq_layout{plan->H / 32, layers[0].gate_up->type};
        const size_t route = align_up(sizeof(int32_t) * plan->L * plan->K);
        const size_t weights = align_up(sizeof(float) * plan->L * plan->K);
        const size_t act = align_up(sizeof(float) * 2 * plan->K * plan->I);
        const size_t y = align_up(sizeof(float) * plan->K * plan->H);
        const size_t xq = align_up(static_cast<size_t>(xq_layout.stride()));
        const size_t flags = align_up(sizeof(uint32_t) * plan->L * kLinkFlagWords);
        const size_t counters = align_up(sizeof(uint32_t) * plan->L * ((plan->H + 31) / 32));
        const size_t state = align_up(2 * sizeof(uint32_t));
        const size_t link = xq + flags + counters + state;
        check_hip(hipMalloc(reinterpret_cast<void **>(&plan->workspace), 2 * route + weights + act + y + link),
                  "decode plan workspace");
        uint8_t * p = plan->workspace;
        plan->route_ids = reinterpret_cast<int32_t *>(p); p += route;
        plan->route_slots = reinterpret_cast<int32_t *>(p); p += route;
        plan->route_w = reinterpret_cast<float *>(p); p += weights;
        plan->act_f = reinterpret_cast<float *>(p); p += act;
        plan->y = reinterpret_cast<float *>(p); p += y;
        uint8_t * link_base = p;
        plan->xq = p; p += xq;
        plan->flags = reinterpret_cast<uint32_t *>(p); p += flags;
        plan->counters = reinterpret_cast<uint32_t *>(p); p += counters;
        plan->epoch = reinterpret_cast<uint32_t *>(p);
        plan->error = plan->epoch + 1;
        check_hip(hipMemset(link_base, 0, link), "decode plan state");
        const uint32_t one = 1;
        check_hip(hipMemcpy(plan->epoch, &one, sizeof(one), hipMemcpyHostToDevice), "decode plan epoch");
        *out = plan.release();
    });
}

vbm_status vbm_decode_plan_destroy(vbm_decode_plan * plan) {
    return guarded([&] {
        if (!plan) return;
        (void)hipDeviceSynchronize();
        if (plan->workspace) (void)hipFree(plan->workspace);
        delete plan;
    });
}

}  // extern "C"

namespace {

void decode_launch_a(const vbm_decode_plan * plan, int64_t l, const float * x, const float * logits, hipStream_t s) {
    const vbm_moe_layer_desc & d = plan->layers[l];
    const int64_t K = plan->K;
    DecodeGateUpArgs a{};
    a.bank = d.gate_up;
    a.expert_to_slot = d.expert_to_slot;
    a.logits = logits + l * plan->E;
    a.n_expert = plan->E;
    a.top_k = K;
    a.hidden = plan->H;
    a.x_in = l == 0 ? x : nullptr;
    a.prev_y = plan->y;
    a.prev_w = l == 0 ? nullptr : plan->route_w + (l - 1) * K;
    a.bias = d.gate_up_bias;
    a.act_f = plan->act_f;
    a.route_ids = plan->route_ids + l * K;
    a.route_w = plan->route_w + l * K;
    a.route_slots = plan->route_slots + l * K;
    a.activation = d.activation;
    a.alpha = 1.702f;
    a.limit = 7.0f;
    launch_decode_gate_up(a, s);
}

void decode_launch_b(const vbm_decode_plan * plan, int64_t l, hipStream_t s) {
    const vbm_moe_layer_desc & d = plan->layers[l];
    DecodeDownParams b{};
    b.bank = d.down;
    b.expert_to_slot = d.expert_to_slot;
    b.act_f = plan->act_f;
    b.act_layout = plan->act_layout;
    b.route_ids = plan->route_ids + l * plan->K;
    b.route_slots = plan->route_slots + l * plan->K;
    b.top_k = plan->K;
    b.bias = d.down_bias;
    b.y = plan->y;
    launch_decode_down(b, s);
}

// Launch j of the linked step: the down tiles of layer j - 1 (j >= 1) and the gate_up tiles of
// layer j (j < L).
void decode_launch_link(const vbm_decode_plan * plan, int64_t j, const float * x, const float * logits, float * out,
                        hipStream_t s) {
    const int64_t K = plan->K, L = plan->L;
    DecodeLinkParams p{};
    p.n_expert = plan->E;
    p.top_k = K;
    p.epoch = plan->epoch;
    p.error = plan->error;
    if (j >= 1) {
        const vbm_moe_layer_desc & d = plan->layers[j - 1];
        p.dn_bank = d.down;
        p.dn_act_f = plan->act_f + ((j - 1) & 1) * K * plan->I;
        p.dn_ids = plan->route_ids + (j - 1) * K;
        p.dn_slots = plan->route_slots + (j - 1) * K;
        p.dn_w = plan->route_w + (j - 1) * K;
        p.dn_bias = d.down_bias;
        p.y = plan->y;
        p.counters = plan->counters + (j - 1) * ((plan->H + 31) / 32);
        if (j == L) {
            p.out = out;
            p.advance_epoch = true;
        }
    }
    if (j < L) {
        const vbm_moe_layer_desc & d = plan->layers[j];
        p.gu_bank = d.gate_up;
        p.expert_to_slot = d.expert_to_slot;
        p.logits = logits + j * plan->E;
        p.x_in = j == 0 ? x : nullptr;
        p.gu_bias = d.gate_up_bias;
        p.act_f = plan->act_f + (j & 1) * K * plan->I;
        p.route_ids = plan->route_ids + j * K;
        p.route_w = plan->route_w + j * K;
        p.route_slots = plan->route_slots + j * K;
        p.activation = d.activation;
        if (j >= 1) {
            p.xq = plan->xq;
            p.flags = plan->flags + j * kLinkFlagWords;
        }
    }
    launch_decode_link(p, s);
}

}  // namespace

extern "C" {

vbm_status vbm_decode_plan_set_linked(vbm_decode_plan * plan, int linked) {
    return guarded([&] {
        require(plan != nullptr, "null plan");
        require(!linked || plan->link_ok, "the linked decode step does not support this plan's shapes");
        plan->linked = linked != 0;
    });
}

vbm_status vbm_decode_plan_get_linked(const vbm_decode_plan * plan, int * linked) {
    return guarded([&] {
        require(plan != nullptr && linked != nullptr, "null argument");
        *linked = plan->linked ? 1 : 0;
    });
}

vbm_status vbm_decode_plan_check(vbm_decode_plan * plan, int64_t * timeouts) {
    return guarded([&] {
        require(plan != nullptr, "null plan");
        check_hip(hipDeviceSynchronize(), "decode plan check");
        uint32_t e = 0;
        check_hip(hipMemcpy(&e, plan->error, sizeof(e), hipMemcpyDeviceToHost), "decode plan error word");
        if (e) check_hip(hipMemset(plan->error, 0, sizeof(e)), "decode plan error reset");
        if (timeouts) *timeouts = e;
        if (e) fail(VBM_ERR_RUNTIME, "a linked decode wait timed out: that step's outputs are unspecified");
    });
}

vbm_status vbm_decode_step(vbm_decode_plan * plan, const float * x, const float * logits, float * out, int32_t * ids,
                           float * weights, void * const * events, void * stream) {
    return guarded([&] {
        require(plan != nullptr && x && logits && out, "null buffer");
        require(reinterpret_cast<uintptr_t>(x) % 16 == 0, "decode input must be 16-byte aligned");
        const hipStream_t s = as_stream(stream);
        const int64_t K = plan->K, H = plan->H;
        if (plan->linked) {
            for (int64_t j = 0; j <= plan->L; ++j) {
                record(events, 2 * j, s);
                decode_launch_link(plan, j, x, logits, out, s);
                record(events, 2 * j + 1, s);
            }
            if (ids) check_hip(hipMemcpyAsync(ids, plan->route_ids, sizeof(int32_t) * plan->L * K, hipMemcpyDeviceToDevice, s), "ids copy");
            if (weights) check_hip(hipMemcpyAsync(weights, plan->route_w, sizeof(float) * plan->L * K, hipMemcpyDeviceToDevice, s), "weights copy");
            return;
        }
        for (int64_t l = 0; l < plan->L; ++l) {
            void * const * ev = events ? events + 4 * l : nullptr;
            record(ev, 0, s);
            decode_launch_a(plan, l, x, logits, s);
            record(ev, 1, s);
            record(ev, 2, s);
            decode_launch_b(plan, l, s);
            record(ev, 3, s);
        }
        launch_combine(plan->y, plan->route_w + (plan->L - 1) * K, H, K, 1, out, s);
        if (ids) check_hip(hipMemcpyAsync(ids, plan->route_ids, sizeof(int32_t) * plan->L * K, hipMemcpyDeviceToDevice, s), "ids copy");
        if (weights) check_hip(hipMemcpyAsync(weights, plan->route_w, sizeof(float) * plan->L * K, hipMemcpyDeviceToDevice, s), "weights copy");
    });
}

vbm_status vbm_decode_kernel(vbm_decode_plan * plan, int64_t layer, int which, const float * x, const float * logits,
                             void * stream) {
    return guarded([&] {
        require(plan != nullptr && x && logits, "null buffer");
        require(layer >= 0 && layer < plan->L && (which == 0 || which == 1), "layer or kernel out of range");
        require(reinterpret_cast<uintptr_t>(x) % 16 == 0, "decode input must be 16-byte aligned");
        const hipStream_t s = as_stream(stream);
        if (which == 0) decode_launch_a(plan, layer, x, logits, s);
        else decode_launch_b(plan, layer, s);
    });
}

}  // extern "C"
