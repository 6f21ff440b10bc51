// Single-GPU host-RAM expert tier for single-token decode.
//
// Every expert of every layer lives in pinned host memory, already in the device bank layout, so
// staging one is a plain hipMemcpyAsync of its two slots (gate|up and down). A shared pool of
// n_slots device slots (one gate|up bank and one down bank serving all layers, like the reference's
// per-device slot group) holds the resident set under causal admission (vbm_admission_*); its
// first top_k slots, the admission's reserved zero slots, stage the current layer's remaining
// misses. Per layer:
//   1. the router kernel selects the layer's experts; their ids come back to the host (the
//      reference's dispatch op reads them on the host too, llama-b11669-hybrid-experts.patch:
//      3244-3298);
//   2. admission runs (llama-b11669-hybrid-experts.patch:3087-3242); admitted experts are copied
//      into their victim slots and the remaining misses into the staging slots, on a side stream;
//   3. the layer's expert->slot map is published and the decode kernels run only after the copy
//      stream's event (publish after event, llama-b11669-hybrid-experts.patch:2953-3005).
// Because step 1 waits for the layer's routing, every kernel that could read an overwritten slot
// has already finished, so eviction never races a reader.
//
// Deferred mode (vbm_tier_set_deferred) takes the host off the per-layer path, in the manner of the
// reference's hosted flush (llama-b11669-hybrid-experts.patch:2953-3005) and its event-protected ID
// hand-off (:3421-3453): the layers of a step run back to back on the device against per-layer
// expert->slot maps published at the step boundary; a routed expert that is not visible in the map
// is read from the pinned host copy inside the decode kernels (the device-side counterpart of the
// reference's CPU miss path, :1728-1847), each workgroup copying its tile into a device staging
// area ([layer][rank] expert copies) and computing from that copy. The step's routed ids come back
// asynchronously behind an event; the next step's flush runs admission on them and copies each
// admitted expert from the staging area into its victim slot (device to device, so an admitted
// expert crosses PCIe once), waits for those copies and publishes the admitted experts at once.
// The previous step has finished before the flush overwrites a victim or a staging copy.
#include "vbm_internal.hpp"

#include <algorithm>
#include <memory>
#include <vector>

using namespace vbm;

struct vbm_tier {
    vbm_tier_desc desc{};
    int device = 0;
    vbm_bank * gate_up = nullptr;     // n_slots slots; the first top_k stage misses
    vbm_bank * down = nullptr;
    vbm_admission * admission = nullptr;
    uint8_t * host_store = nullptr;   // pinned: [layer][expert] (gate_up slot bytes, down slot bytes)
    size_t gu_bytes = 0, dn_bytes = 0;
    hipStream_t copy_stream = nullptr;
    hipEvent_t copy_begin = nullptr, copy_end = nullptr;
    int32_t * host_ids = nullptr;     // pinned [top_k]
    int32_t * host_map = nullptr;     // pinned [n_expert]
    int32_t * dev_map = nullptr;      // [n_expert]
    uint8_t * workspace = nullptr;
    int32_t * route_ids = nullptr;    // [L][K]
    float * route_w = nullptr;        // [L][K]
    float * act_f = nullptr;          // [K][I] GLU outputs (kernel A -> kernel B)
    XrowLayout act_layout{};
    float * y = nullptr;
    std::vector<const float *> gu_bias, dn_bias;
    vbm_tier_stats stats{};
    hipEvent_t last_use = nullptr;    // end of the previous step / prefill on its stream
    bool used = false;
    // prefill (vbm_tier_prefill): layer workspace, per-pass expert->slot maps, ping-pong events
    uint8_t * pf_work = nullptr;
    size_t pf_work_bytes = 0;
    int32_t * pf_maps = nullptr;      // device [passes][n_expert]
    int32_t * pf_maps_host = nullptr; // pinned mirror
    int32_t * pf_ids_host = nullptr;  // pinned [max tokens][top_k]
    int64_t pf_tokens = 0;            // capacity of pf_work / pf_ids_host in tokens
    hipEvent_t pf_ready[2] = {nullptr, nullptr}, pf_done[2] = {nullptr, nullptr};
    vbm_trace * trace = nullptr;      // optional routing trace (caller-owned)
    std::vector<int64_t> trace_layer_ids;
    bool started = false;             // seeded or stepped: the pool's slots are live
    // deferred mode
    bool deferred = false;
    const uint8_t * host_dev = nullptr;   // device-visible address of host_store
    int32_t * dev_maps = nullptr;     // [L][E] published expert->slot maps (-1: the pinned host copy)
    int32_t * host_maps = nullptr;    // pinned mirror, rebuilt at each flush
    int32_t * step_ids_host = nullptr;   // pinned [L][K]: the last step's routed ids
    hipEvent_t step_done = nullptr;   // after that step's id hand-off
    bool step_pending = false;        // its ids still await admission
    bool awaiting = false;            // a step was begun; its device part (eager or a graph replay) follows
    bool enqueued = false;            // that step's device part was enqueued eagerly
    uint8_t * staged = nullptr;       // device [L][K] expert copies (gate_up | down) of host-read picks

    ~vbm_tier() {
        (void)hipSetDevice(device);
        (void)hipDeviceSynchronize();
        if (admission) vbm_admission_destroy(admission);
        if (gate_up) vbm_bank_destroy(gate_up);
        if (down) vbm_bank_destroy(down);
        if (host_store) (void)hipHostFree(host_store);
        if (host_ids) (void)hipHostFree(host_ids);
        if (host_map) (void)hipHostFree(host_map);
        if (dev_map) (void)hipFree(dev_map);
        if (workspace) (void)hipFree(workspace);
        if (copy_begin) (void)hipEventDestroy(copy_begin);
        if (copy_end) (void)hipEventDestroy(copy_end);
        if (copy_stream) (void)hipStreamDestroy(copy_stream);
        if (last_use) (void)hipEventDestroy(last_use);
        for (int i = 0; i < 2; ++i) {
            if (pf_ready[i]) (void)hipEventDestroy(pf_ready[i]);
            if (pf_done[i]) (void)hipEventDestroy(pf_done[i]);
        }
        if (pf_work) (void)hipFree(pf_work);
        if (pf_maps) (void)hipFree(pf_maps);
        if (pf_maps_host) (void)hipHostFree(pf_maps_host);
        if (pf_ids_host) (void)hipHostFree(pf_ids_host);
        if (dev_maps) (void)hipFree(dev_maps);
        if (host_maps) (void)hipHostFree(host_maps);
        if (step_ids_host) (void)hipHostFree(step_ids_host);
        if (step_done) (void)hipEventDestroy(step_done);
        if (staged) (void)hipFree(staged);
    }

    uint8_t * host_expert(int64_t layer, int64_t expert) const {
        return host_store + (static_cast<size_t>(layer) * desc.n_expert + expert) * (gu_bytes + dn_bytes);
    }
};

namespace {

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

void check_status(vbm_status st, const char * what) {
    if (st != VBM_OK) fail(st, std::string(what) + ": " + vbm_last_error());
}

// Copies the host copy of (layer, expert) into device slot `slot` of both banks (copy stream).
void stage(vbm_tier & t, int64_t layer, int64_t expert, int64_t slot) {
    const uint8_t * src = t.host_expert(layer, expert);
    check_hip(hipMemcpyAsync(t.gate_up->base + static_cast<size_t>(slot) * t.gu_bytes, src, t.gu_bytes,
                             hipMemcpyHostToDevice, t.copy_stream), "tier gate_up stage");
    check_hip(hipMemcpyAsync(t.down->base + static_cast<size_t>(slot) * t.dn_bytes, src + t.gu_bytes, t.dn_bytes,
                             hipMemcpyHostToDevice, t.copy_stream), "tier down stage");
    t.stats.uploaded_bytes += t.gu_bytes + t.dn_bytes;
}

// Copies `bytes` from one device range to another on the copy stream (device_copy_bytes).
void copy_device(vbm_tier & t, uint8_t * dst, const uint8_t * src, size_t bytes, const char * what) {
    check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, t.copy_stream), what);
    t.stats.device_copy_bytes += bytes;
}

// Deferred mode, at a step boundary: (1) wait for the last step; (2) run admission on its routed
// ids, layer by layer, as the synchronous mode does per layer; (3) copy each admitted expert into
// its slot from the device copy the step left: a pick that was not in the step's map was read from
// the host copy by the step's decode kernels, which left its copy in the staging area (rank r of
// layer l); a pick that was in a slot during the step but is admitted again (an earlier rank's
// admission of the same layer evicted it) is first saved from that slot into its own, unused,
// staging entry, before any slot is overwritten; then every admitted expert is copied from the
// staging area into its slot, all on the copy stream in that order (an upload from the host copy
// only for a pick outside the step's ids, which admission does not produce); (4) wait for the
// copies and rebuild the per-layer maps from the admission's slot maps, admitted experts
// included. The maps reach the device at the start of the next step.
void tier_flush(vbm_tier & t) {
    const vbm_tier_desc & d = t.desc;
    const int64_t L = d.n_layers, E = d.n_expert, K = d.top_k;
    if (t.step_pending) {
        check_hip(hipEventSynchronize(t.step_done), "tier step hand-off");
        std::vector<int32_t> hits(static_cast<size_t>(K)), slots(static_cast<size_t>(K)),
            experts(static_cast<size_t>(K)), evicted(static_cast<size_t>(K));
        std::vector<int32_t> map(static_cast<size_t>(E));
        struct Admitted { int64_t layer, rank, expert, slot, old_slot; };
        std::vector<Admitted> admitted;
        for (int64_t l = 0; l < L; ++l) {
            const int32_t * ids = t.step_ids_host + l * K;
            const int32_t * step_map = t.host_maps + l * E;     // the map the step ran with
            for (int64_t r = 0; r < K; ++r) t.stats.host_reads += step_map[ids[r]] < 0;
            int64_t n_admitted = 0;
            check_status(vbm_admission_admit(t.admission, l, ids, hits.data(), slots.data(), experts.data(),
                                             evicted.data(), &n_admitted), "tier admission");
            ++t.stats.dispatches;
            check_status(vbm_admission_slot_map(t.admission, l, map.data()), "tier slot map");
            for (int64_t r = 0; r < K; ++r) {
                t.stats.hits += hits[r];
                if (map[static_cast<size_t>(ids[r])] < 0) ++t.stats.staged;   // served from the host copy
            }
            t.stats.admissions += static_cast<uint64_t>(n_admitted);
            for (int64_t i = 0; i < n_admitted; ++i) {
                t.stats.evictions += evicted[i] >= 0;
                const int64_t rank = std::find(ids, ids + K, experts[i]) - ids;
                admitted.push_back({l, rank, experts[i], slots[i], rank < K ? step_map[experts[i]] : -1});
            }
        }
        t.step_pending = false;
        if (!admitted.empty()) {
            const size_t stride = t.gu_bytes + t.dn_bytes;
            auto staged_of = [&](const Admitted & a) { return t.staged + static_cast<size_t>(a.layer * K + a.rank) * stride; };
            check_hip(hipEventRecord(t.copy_begin, t.copy_stream), "tier copy event");
            for (const Admitted & a : admitted)
                if (a.rank < K && a.old_slot >= 0) {
                    copy_device(t, staged_of(a), t.gate_up->base + static_cast<size_t>(a.old_slot) * t.gu_bytes, t.gu_bytes,
                                "tier gate_up save");
                    copy_device(t, staged_of(a) + t.gu_bytes, t.down->base + static_cast<size_t>(a.old_slot) * t.dn_bytes,
                                t.dn_bytes, "tier down save");
                }
            for (const Admitted & a : admitted) {
                if (a.rank < K) {
                    copy_device(t, t.gate_up->base + static_cast<size_t>(a.slot) * t.gu_bytes, staged_of(a), t.gu_bytes,
                                "tier gate_up admission copy");
                    copy_device(t, t.down->base + static_cast<size_t>(a.slot) * t.dn_bytes, staged_of(a) + t.gu_bytes,
                                t.dn_bytes, "tier down admission copy");
                } else {
                    stage(t, a.layer, a.expert, a.slot);
                }
            }
            check_hip(hipEventRecord(t.copy_end, t.copy_stream), "tier copy event");
            check_hip(hipEventSynchronize(t.copy_end), "tier admission copies");
            float ms = 0.0f;
            check_hip(hipEventElapsedTime(&ms, t.copy_begin, t.copy_end), "tier copy timing");
            t.stats.copy_ms += ms;
        }
    }
    for (int64_t l = 0; l < L; ++l)
        check_status(vbm_admission_slot_map(t.admission, l, t.host_maps + l * E), "tier slot map");
}

// Completes the step in flight, its admissions and their copies (before a prefill, a seed, a
// mode change or teardown).
void tier_quiesce(vbm_tier & t) {
    if (!t.deferred) return;
    if (t.awaiting) t.step_pending = true;
    t.awaiting = false;
    tier_flush(t);
}

// The device part of a deferred step (no host waits): publish the maps, the layers back to back
// with misses from the pinned host copy, the combine, the id hand-off.
void tier_enqueue_step(vbm_tier & t, const float * x, const float * logits, float * out, int32_t * ids, hipStream_t s) {
    const vbm_tier_desc & d = t.desc;
    const int64_t L = d.n_layers, E = d.n_expert, K = d.top_k, H = d.hidden;
    const int64_t stride = static_cast<int64_t>(t.gu_bytes + t.dn_bytes);
    check_hip(hipMemcpyAsync(t.dev_maps, t.host_maps, sizeof(int32_t) * L * E, hipMemcpyHostToDevice, s), "tier maps");
    for (int64_t l = 0; l < L; ++l) {
        const uint8_t * layer_host = t.host_dev + static_cast<size_t>(l) * E * static_cast<size_t>(stride);
        DecodeGateUpArgs a{};
        a.bank = t.gate_up;
        a.expert_to_slot = t.dev_maps + l * E;
        a.logits = logits + l * E;
        a.n_expert = E;
        a.top_k = K;
        a.hidden = H;
        a.x_in = l == 0 ? x : nullptr;
        a.prev_y = t.y;
        a.prev_w = l == 0 ? nullptr : t.route_w + (l - 1) * K;
        a.bias = t.gu_bias[l];
        a.act_f = t.act_f;
        a.route_ids = t.route_ids + l * K;
        a.route_w = t.route_w + l * K;
        a.activation = d.activation;
        a.alpha = 1.702f;
        a.limit = 7.0f;
        a.host_base = layer_host;
        a.host_stride = stride;
        a.stage = t.staged + static_cast<size_t>(l * K) * static_cast<size_t>(stride);
        a.stage_stride = stride;
        launch_decode_gate_up(a, s);
        DecodeDownParams b{};
        b.bank = t.down;
        b.expert_to_slot = t.dev_maps + l * E;
        b.act_f = t.act_f;
        b.act_layout = t.act_layout;
        b.route_ids = t.route_ids + l * K;
        b.top_k = K;
        b.bias = t.dn_bias[l];
        b.y = t.y;
        b.host_base = layer_host + t.gu_bytes;
        b.host_stride = stride;
        b.stage = a.stage + t.gu_bytes;
        b.stage_stride = stride;
        launch_decode_down(b, s);
    }
    launch_combine(t.y, t.route_w + (L - 1) * K, H, K, 1, out, s);
    if (ids) check_hip(hipMemcpyAsync(ids, t.route_ids, sizeof(int32_t) * L * K, hipMemcpyDeviceToDevice, s), "ids copy");
    check_hip(hipMemcpyAsync(t.step_ids_host, t.route_ids, sizeof(int32_t) * L * K, hipMemcpyDeviceToHost, s),
              "tier id hand-off");
    // external records under capture: every replay records them, so the host waits on them
    // (the next flush, seed, reset or mode change) wait for that replay's hand-off and reads
    record_event(t.step_done, s, "tier step event");
    record_event(t.last_use, s, "tier last use");
    t.used = true;
}

// Host part of a deferred step: the step begun last time has run (eagerly or as a graph replay),
// so its ids are the next to admit.
void tier_begin_step(vbm_tier & t) {
    if (t.awaiting) t.step_pending = true;
    tier_flush(t);
    t.awaiting = true;
    t.enqueued = false;
    t.started = true;
}

}  // namespace

extern "C" {

vbm_status vbm_tier_create(const vbm_tier_desc * d, vbm_tier ** out) {
    return guarded([&] {
        require(d != nullptr && out != nullptr, "null argument");
        *out = nullptr;
        require(d->type == VBM_TYPE_MXFP4 || d->type == VBM_TYPE_Q8_0, "tier type must be MXFP4 or Q8_0");
        require(d->hidden > 0 && d->hidden % 64 == 0 && d->hidden <= 4096 && d->intermediate > 0 &&
                    d->intermediate % 64 == 0 && d->intermediate <= 4096, "tier shape out of range");
        require(d->n_layers > 0 && d->n_expert > 0 && d->n_expert <= 1024 && d->top_k > 0 && d->top_k <= 64 &&
                    d->top_k <= d->n_expert, "tier routing shape out of range");
        require(d->activation == VBM_ACT_SILU || d->activation == VBM_ACT_SWIGLU_OAI, "unknown activation");
        auto t = std::make_unique<vbm_tier>();
        t->desc = *d;
        check_hip(hipGetDevice(&t->device), "hipGetDevice");
        const int64_t L = d->n_layers, E = d->n_expert, K = d->top_k, H = d->hidden, I = d->intermediate;
        check_status(vbm_admission_create(L, E, K, d->n_slots, d->recent_window, d->margin, d->policy, &t->admission),
                     "tier admission");
        // device pool: slots [0, n_slots) resident (the first top_k are the admission's reserved
        // zero slots, used here as the staging slots of the current layer's misses)
        check_status(vbm_bank_create(d->type, 2 * I, H, d->n_slots, 1, &t->gate_up), "tier gate_up bank");
        check_status(vbm_bank_create(d->type, H, I, d->n_slots, 0, &t->down), "tier down bank");
        t->gu_bytes = t->gate_up->slot_bytes;
        t->dn_bytes = t->down->slot_bytes;
        const size_t store = static_cast<size_t>(L * E) * (t->gu_bytes + t->dn_bytes);
        check_hip(hipHostMalloc(reinterpret_cast<void **>(&t->host_store), store, hipHostMallocDefault),
                  "tier pinned host store");
        check_hip(hipHostMalloc(reinterpret_cast<void **>(&t->host_ids), sizeof(int32_t) * K, hipHostMallocDefault),
                  "tier pinned ids");
        check_hip(hipHostMalloc(reinterpret_cast<void **>(&t->host_map), sizeof(int32_t) * E, hipHostMallocDefault),
                  "tier pinned map");
        check_hip(hipMalloc(reinterpret_cast<void **>(&t->dev_map), sizeof(int32_t) * E), "tier map");
        check_hip(hipStreamCreateWithFlags(&t->copy_stream, hipStreamNonBlocking), "tier copy stream");
        check_hip(hipEventCreate(&t->copy_begin), "tier event");
        check_hip(hipEventCreate(&t->copy_end), "tier event");
        check_hip(hipEventCreateWithFlags(&t->last_use, hipEventDisableTiming), "tier event");
        for (int i = 0; i < 2; ++i) {
            check_hip(hipEventCreateWithFlags(&t->pf_ready[i], hipEventDisableTiming), "tier event");
            check_hip(hipEventCreateWithFlags(&t->pf_done[i], hipEventDisableTiming), "tier event");
        }
        check_hip(hipMalloc(reinterpret_cast<void **>(&t->pf_maps), sizeof(int32_t) * E * (E + 1)), "tier prefill maps");
        check_hip(hipHostMalloc(reinterpret_cast<void **>(&t->pf_maps_host), sizeof(int32_t) * E * (E + 1),
                                hipHostMallocDefault), "tier prefill maps");
        t->act_layout = XrowLayout{I / 32, d->type};
        const size_t route = align_up(sizeof(int32_t) * L * K), wts = align_up(sizeof(float) * L * K);
        const size_t act = align_up(sizeof(float) * K * I);
        const size_t y = align_up(sizeof(float) * K * H);
        check_hip(hipMalloc(reinterpret_cast<void **>(&t->workspace), route + wts + act + y), "tier workspace");
        uint8_t * p = t->workspace;
        t->route_ids = reinterpret_cast<int32_t *>(p); p += route;
        t->route_w = reinterpret_cast<float *>(p); p += wts;
        t->act_f = reinterpret_cast<float *>(p); p += act;
        t->y = reinterpret_cast<float *>(p);
        t->gu_bias.assign(static_cast<size_t>(L), nullptr);
        t->dn_bias.assign(static_cast<size_t>(L), nullptr);
        for (int64_t l = 0; l < L; ++l) {
            if (d->gate_up_bias) t->gu_bias[l] = d->gate_up_bias[l];
            if (d->down_bias) t->dn_bias[l] = d->down_bias[l];
        }
        *out = t.release();
    });
}

vbm_status vbm_tier_destroy(vbm_tier * t) {
    return guarded([&] { delete t; });
}

vbm_status vbm_tier_host_bytes(const vbm_tier * t, size_t * bytes) {
    return guarded([&] {
        require(t != nullptr && bytes != nullptr, "null argument");
        *bytes = static_cast<size_t>(t->desc.n_layers * t->desc.n_expert) * (t->gu_bytes + t->dn_bytes);
    });
}

vbm_status vbm_tier_set_expert(vbm_tier * t, int64_t layer, int64_t expert, const void * gate_up_ggml,
                               const void * down_ggml, void * stream) {
    return guarded([&] {
        require(t != nullptr && gate_up_ggml != nullptr && down_ggml != nullptr, "null argument");
        require(layer >= 0 && layer < t->desc.n_layers && expert >= 0 && expert < t->desc.n_expert,
                "expert out of range");
        require(!t->started, "experts must be stored before the tier is seeded or stepped");
        const hipStream_t s = as_stream(stream);
        // repack through staging slot 0 (a reserved slot) and keep the device layout bytes
        check_status(vbm_bank_upload(t->gate_up, 0, gate_up_ggml, 0, stream), "tier gate_up repack");
        check_status(vbm_bank_upload(t->down, 0, down_ggml, 0, stream), "tier down repack");
        uint8_t * dst = t->host_expert(layer, expert);
        check_hip(hipMemcpyAsync(dst, t->gate_up->base, t->gu_bytes, hipMemcpyDeviceToHost, s), "tier store");
        check_hip(hipMemcpyAsync(dst + t->gu_bytes, t->down->base, t->dn_bytes, hipMemcpyDeviceToHost, s), "tier store");
        check_hip(hipStreamSynchronize(s), "tier store synchronize");
    });
}

vbm_status vbm_tier_generate(vbm_tier * t, uint64_t seed, uint64_t layer_stride, uint64_t gate_up_stream,
                             uint64_t down_stream, float p0, float p1, void * stream) {
    return guarded([&] {
        require(t != nullptr, "null tier");
        require(!t->started, "experts must be stored before the tier is seeded or stepped");
        const hipStream_t s = as_stream(stream);
        const int64_t E = t->desc.n_expert;
        const int64_t chunk = std::max<int64_t>(1, std::min<int64_t>(t->gate_up->n_slots, E));
        for (int64_t l = 0; l < t->desc.n_layers; ++l)
            for (int64_t e0 = 0; e0 < E; e0 += chunk) {
                const int64_t n = std::min(chunk, E - e0);
                check_status(vbm_bank_generate(t->gate_up, 0, n, seed, layer_stride * l + gate_up_stream, e0, p0, p1, stream),
                             "tier generate");
                check_status(vbm_bank_generate(t->down, 0, n, seed, layer_stride * l + down_stream, e0, p0, p1, stream),
                             "tier generate");
                for (int64_t i = 0; i < n; ++i) {
                    uint8_t * dst = t->host_expert(l, e0 + i);
                    check_hip(hipMemcpyAsync(dst, t->gate_up->base + i * t->gu_bytes, t->gu_bytes, hipMemcpyDeviceToHost, s),
                              "tier store");
                    check_hip(hipMemcpyAsync(dst + t->gu_bytes, t->down->base + i * t->dn_bytes, t->dn_bytes,
                                             hipMemcpyDeviceToHost, s), "tier store");
                }
                check_hip(hipStreamSynchronize(s), "tier generate synchronize");
            }
    });
}

vbm_status vbm_tier_load_gguf(vbm_tier * t, const vbm_gguf * g, const int64_t * layer_ids, void * stream) {
    return guarded([&] {
        require(t != nullptr && g != nullptr && layer_ids != nullptr, "null argument");
        require(!t->started, "experts must be stored before the tier is seeded or stepped");
        const vbm_tier_desc & d = t->desc;
        std::vector<uint8_t> gu, dn;
        for (int64_t l = 0; l < d.n_layers; ++l) {
            vbm_gguf_expert_info info{};
            check_status(vbm_gguf_expert_layer_info(g, layer_ids[l], &info), "tier gguf layer");
            require(info.gate_up_type == d.type && info.down_type == d.type && info.hidden == d.hidden &&
                        info.intermediate == d.intermediate && info.n_expert == d.n_expert,
                    "GGUF layer " + std::to_string(layer_ids[l]) + " does not match the tier's shape and type");
            gu.resize(info.gate_up_bytes);
            dn.resize(info.down_bytes);
            for (int64_t e = 0; e < d.n_expert; ++e) {
                check_status(vbm_gguf_read_expert(g, layer_ids[l], e, gu.data(), dn.data(), nullptr, nullptr),
                             "tier gguf read");
                check_status(vbm_tier_set_expert(t, l, e, gu.data(), dn.data(), stream), "tier gguf store");
            }
        }
    });
}

vbm_status vbm_tier_seed(vbm_tier * t, int64_t layer, int64_t expert) {
    return guarded([&] {
        require(t != nullptr, "null tier");
        tier_quiesce(*t);
        if (t->used) check_hip(hipEventSynchronize(t->last_use), "tier seed");
        int32_t slot = -1;
        check_status(vbm_admission_seed(t->admission, layer, expert, &slot), "tier seed");
        t->started = true;
        stage(*t, layer, expert, slot);
        check_hip(hipStreamSynchronize(t->copy_stream), "tier seed synchronize");
        if (t->deferred)
            check_status(vbm_admission_slot_map(t->admission, layer, t->host_maps + layer * t->desc.n_expert), "tier slot map");
    });
}

vbm_status vbm_tier_step(vbm_tier * t, const float * x, const float * logits, float * out, int32_t * ids, void * stream) {
    return guarded([&] {
        require(t != nullptr && x && logits && out, "null buffer");
        require(reinterpret_cast<uintptr_t>(x) % 16 == 0, "decode input must be 16-byte aligned");
        const hipStream_t s = as_stream(stream);
        if (t->deferred) {
            tier_begin_step(*t);
            t->enqueued = true;
            tier_enqueue_step(*t, x, logits, out, ids, s);
            return;
        }
        const vbm_tier_desc & d = t->desc;
        const int64_t L = d.n_layers, E = d.n_expert, K = d.top_k, H = d.hidden;
        if (t->trace) {
            int64_t token = -1, next_layer = -1;
            check_status(vbm_trace_position(t->trace, nullptr, nullptr, &token, &next_layer), "tier trace");
            require(token >= 0 && next_layer == 0, "the attached trace has no open request at a token boundary");
        }
        t->started = true;
        std::vector<int32_t> hits(static_cast<size_t>(K)), slots(static_cast<size_t>(K)),
            experts(static_cast<size_t>(K)), evicted(static_cast<size_t>(K));
        for (int64_t l = 0; l < L; ++l) {
            // 1. routing of this layer, back to the host
            launch_router(nullptr, nullptr, nullptr, H, const_cast<float *>(logits + l * E), E, 1, K,
                          t->route_ids + l * K, t->route_w + l * K, s);
            check_hip(hipMemcpyAsync(t->host_ids, t->route_ids + l * K, sizeof(int32_t) * K, hipMemcpyDeviceToHost, s),
                      "tier ids");
            check_hip(hipStreamSynchronize(s), "tier ids synchronize");
            if (t->trace)
                check_status(vbm_trace_route(t->trace, t->trace_layer_ids[static_cast<size_t>(l)], t->host_ids, K),
                             "tier trace");
            // 2. admission, then copies of admitted experts and staged misses
            int64_t n_admitted = 0;
            check_status(vbm_admission_admit(t->admission, l, t->host_ids, hits.data(), slots.data(), experts.data(),
                                             evicted.data(), &n_admitted), "tier admission");
            ++t->stats.dispatches;
            if (l == 0 && t->used)   // slots the previous call's kernels read may be restaged now
                check_hip(hipStreamWaitEvent(t->copy_stream, t->last_use, 0), "tier reuse wait");
            check_hip(hipEventRecord(t->copy_begin, t->copy_stream), "tier copy event");
            const uint64_t before = t->stats.uploaded_bytes;
            for (int64_t i = 0; i < n_admitted; ++i) stage(*t, l, experts[i], slots[i]);
            check_status(vbm_admission_slot_map(t->admission, l, t->host_map), "tier slot map");
            for (int64_t r = 0; r < K; ++r) {
                t->stats.hits += hits[r];
                const int32_t e = t->host_ids[r];
                if (t->host_map[e] < 0) {         // miss without admission: reserved slot r
                    stage(*t, l, e, r);
                    t->host_map[e] = static_cast<int32_t>(r);
                    ++t->stats.staged;
                }
            }
            t->stats.admissions += static_cast<uint64_t>(n_admitted);
            for (int64_t i = 0; i < n_admitted; ++i) t->stats.evictions += evicted[i] >= 0;
            check_hip(hipMemcpyAsync(t->dev_map, t->host_map, sizeof(int32_t) * E, hipMemcpyHostToDevice, t->copy_stream),
                      "tier map upload");
            check_hip(hipEventRecord(t->copy_end, t->copy_stream), "tier copy event");
            // 3. publish after the copies: the layer's kernels wait for the copy stream
            check_hip(hipStreamWaitEvent(s, t->copy_end, 0), "tier publish");
            DecodeGateUpArgs a{};
            a.bank = t->gate_up;
            a.expert_to_slot = t->dev_map;
            a.logits = logits + l * E;
            a.n_expert = E;
            a.top_k = K;
            a.hidden = H;
            a.x_in = l == 0 ? x : nullptr;
            a.prev_y = t->y;
            a.prev_w = l == 0 ? nullptr : t->route_w + (l - 1) * K;
            a.bias = t->gu_bias[l];
            a.act_f = t->act_f;
            a.route_ids = t->route_ids + l * K;
            a.route_w = t->route_w + l * K;
            a.activation = d.activation;
            a.alpha = 1.702f;
            a.limit = 7.0f;
            launch_decode_gate_up(a, s);
            DecodeDownParams b{};
            b.bank = t->down;
            b.expert_to_slot = t->dev_map;
            b.act_f = t->act_f;
            b.act_layout = t->act_layout;
            b.route_ids = t->route_ids + l * K;
            b.top_k = K;
            b.bias = t->dn_bias[l];
            b.y = t->y;
            launch_decode_down(b, s);
            if (t->stats.uploaded_bytes != before) {
                check_hip(hipEventSynchronize(t->copy_end), "tier copy timing");
                float ms = 0.0f;
                check_hip(hipEventElapsedTime(&ms, t->copy_begin, t->copy_end), "tier copy timing");
                t->stats.copy_ms += ms;
            }
        }
        launch_combine(t->y, t->route_w + (L - 1) * K, H, K, 1, out, s);
        if (ids) check_hip(hipMemcpyAsync(ids, t->route_ids, sizeof(int32_t) * L * K, hipMemcpyDeviceToDevice, s), "ids copy");
        check_hip(hipEventRecord(t->last_use, s), "tier last use");
        t->used = true;
    });
}

vbm_status vbm_tier_prefill(vbm_tier * t, int64_t layer, const float * x, const float * logits, int64_t n_tokens,
                            float * out, int32_t * ids, float * weights, void * stream) {
    return guarded([&] {
        require(t != nullptr && x && logits && out, "null buffer");
        const vbm_tier_desc & d = t->desc;
        require(layer >= 0 && layer < d.n_layers, "layer out of range");
        require(n_tokens >= kGemmMinTokens && n_tokens <= 65536,
                "tier prefill takes 16..65536 tokens (single tokens: vbm_tier_step)");
        const hipStream_t s = as_stream(stream);
        tier_quiesce(*t);                 // deferred mode: admissions applied, uploads published
        const int64_t E = d.n_expert, K = d.top_k, H = d.hidden, T = n_tokens;
        vbm_moe_layer_desc desc{};
        desc.gate_up = t->gate_up;
        desc.down = t->down;
        desc.gate_up_bias = t->gu_bias[layer];
        desc.down_bias = t->dn_bias[layer];
        desc.hidden = H;
        desc.intermediate = d.intermediate;
        desc.n_expert = E;
        desc.top_k = K;
        desc.activation = d.activation;
        desc.order = VBM_ORDER_FAST;
        if (T > t->pf_tokens) {           // grow the workspace (rare: a larger batch than before)
            check_hip(hipStreamSynchronize(s), "tier prefill grow");
            if (t->used) check_hip(hipEventSynchronize(t->last_use), "tier prefill grow");
            if (t->pf_work) check_hip(hipFree(t->pf_work), "tier prefill grow");
            if (t->pf_ids_host) check_hip(hipHostFree(t->pf_ids_host), "tier prefill grow");
            t->pf_work = nullptr;
            t->pf_ids_host = nullptr;
            t->pf_tokens = 0;
            const size_t bytes = plan_layer(desc, T, nullptr).total;
            check_hip(hipMalloc(reinterpret_cast<void **>(&t->pf_work), bytes), "tier prefill workspace");
            check_hip(hipHostMalloc(reinterpret_cast<void **>(&t->pf_ids_host), sizeof(int32_t) * T * K,
                                    hipHostMallocDefault), "tier prefill ids");
            t->pf_work_bytes = bytes;
            t->pf_tokens = T;
        }
        const LayerWorkspace w = plan_layer(desc, T, t->pf_work);
        // 1. routing, input rows and grouping; the routed ids come to the host
        prefill_prepare(desc, x, w.ids, T, w, s, false, logits, w.weights);   // top-k in the rows launch
        check_hip(hipMemcpyAsync(t->pf_ids_host, w.ids, sizeof(int32_t) * T * K, hipMemcpyDeviceToHost, s), "prefill ids");
        check_hip(hipStreamSynchronize(s), "prefill ids synchronize");
        int prefill_summary = 0;
        if (t->trace) check_status(vbm_trace_prefill_enabled(t->trace, &prefill_summary), "tier trace");
        for (int64_t r = 0; prefill_summary && r < T; r += 32768)   // the summary's batches hold <= 32768 rows
            check_status(vbm_trace_prefill_route(t->trace, t->trace_layer_ids[static_cast<size_t>(layer)],
                                                 t->pf_ids_host + r * K, std::min<int64_t>(32768, T - r)),
                         "tier trace");
        if (t->used) check_hip(hipStreamWaitEvent(t->copy_stream, t->last_use, 0), "tier reuse wait");
        t->started = true;
        // 2. residency is frozen for multi-token batches: pass 0 covers the resident experts, then
        //    the remaining routed experts stream through the reserved slots in chunks
        int32_t * maps = t->pf_maps_host;
        check_status(vbm_admission_slot_map(t->admission, layer, maps), "prefill slot map");
        std::vector<int64_t> count(static_cast<size_t>(E), 0);
        for (int64_t i = 0; i < T * K; ++i) ++count[static_cast<size_t>(t->pf_ids_host[i])];
        const int64_t job_tile = gemm_job_tile(desc.gate_up->type);
        auto tiles_of = [&](int64_t e) { return (count[static_cast<size_t>(e)] + job_tile - 1) / job_tile; };   // GEMM job tiles
        std::vector<char> routed(static_cast<size_t>(E), 0);
        for (int64_t e = 0; e < E; ++e) routed[static_cast<size_t>(e)] = count[static_cast<size_t>(e)] > 0;
        std::vector<int32_t> cold;
        uint64_t resident_hits = 0;
        int64_t resident_tiles = 0;
        for (int64_t e = 0; e < E; ++e) {
            if (!routed[static_cast<size_t>(e)]) continue;
            if (maps[e] >= 0) {
                ++resident_hits;
                resident_tiles += tiles_of(e);
            } else {
                cold.push_back(static_cast<int32_t>(e));
            }
        }
        const int64_t chunk = std::max<int64_t>(1, K / 2);       // two halves of the reserved slots
        const int64_t n_chunks = (static_cast<int64_t>(cold.size()) + chunk - 1) / chunk;
        for (int64_t j = 0; j < n_chunks; ++j) {
            int32_t * m = maps + (j + 1) * E;
            std::fill(m, m + E, -1);
            const int64_t half = K >= 2 ? (j % 2) * chunk : 0;
            for (int64_t i = 0; i < chunk && j * chunk + i < static_cast<int64_t>(cold.size()); ++i)
                m[cold[static_cast<size_t>(j * chunk + i)]] = static_cast<int32_t>(half + i);
        }
        check_hip(hipMemcpyAsync(t->pf_maps, maps, sizeof(int32_t) * E * (n_chunks + 1), hipMemcpyHostToDevice, s),
                  "prefill maps");
        if (resident_hits) prefill_pass(desc, t->pf_maps, T, w, w.weights, nullptr, s, resident_tiles);
        for (int64_t j = 0; j < n_chunks; ++j) {
            const int b = K >= 2 ? static_cast<int>(j % 2) : 0;
            if (j >= (K >= 2 ? 2 : 1))    // the half's previous chunk must be consumed first
                check_hip(hipStreamWaitEvent(t->copy_stream, t->pf_done[b], 0), "prefill reuse wait");
            const int64_t half = K >= 2 ? (j % 2) * chunk : 0;
            int64_t chunk_tiles = 0;
            for (int64_t i = 0; i < chunk && j * chunk + i < static_cast<int64_t>(cold.size()); ++i) {
                stage(*t, layer, cold[static_cast<size_t>(j * chunk + i)], half + i);
                chunk_tiles += tiles_of(cold[static_cast<size_t>(j * chunk + i)]);
            }
            check_hip(hipEventRecord(t->pf_ready[b], t->copy_stream), "prefill ready");
            check_hip(hipStreamWaitEvent(s, t->pf_ready[b], 0), "prefill publish");
            prefill_pass(desc, t->pf_maps + (j + 1) * E, T, w, w.weights, nullptr, s, chunk_tiles);
            check_hip(hipEventRecord(t->pf_done[b], s), "prefill done");
        }
        // 3. rank-ordered weighted combine of every (token, rank) down output
        launch_combine(w.y, nullptr, H, K, T, out, s);   // rows weighted in the down epilogues
        if (ids) check_hip(hipMemcpyAsync(ids, w.ids, sizeof(int32_t) * T * K, hipMemcpyDeviceToDevice, s), "ids copy");
        if (weights) check_hip(hipMemcpyAsync(weights, w.weights, sizeof(float) * T * K, hipMemcpyDeviceToDevice, s),
                               "weights copy");
        check_hip(hipEventRecord(t->last_use, s), "tier last use");
        t->used = true;
        t->stats.prefill_tokens += static_cast<uint64_t>(T);
        t->stats.prefill_resident += resident_hits;
        t->stats.prefill_streamed += cold.size();
    });
}

vbm_status vbm_tier_set_deferred(vbm_tier * t, int enable) {
    return guarded([&] {
        require(t != nullptr, "null tier");
        require(!enable || t->trace == nullptr, "deferred mode records no routing trace; detach it first");
        if (static_cast<bool>(enable) == t->deferred) return;
        const vbm_tier_desc & d = t->desc;
        const int64_t L = d.n_layers, E = d.n_expert, K = d.top_k;
        if (enable) {
            if (!t->dev_maps) {
                check_hip(hipHostGetDevicePointer(reinterpret_cast<void **>(const_cast<uint8_t **>(&t->host_dev)),
                                                  t->host_store, 0), "tier host store device address");
                check_hip(hipMalloc(reinterpret_cast<void **>(&t->dev_maps), sizeof(int32_t) * L * E), "tier maps");
                check_hip(hipHostMalloc(reinterpret_cast<void **>(&t->host_maps), sizeof(int32_t) * L * E,
                                        hipHostMallocDefault), "tier maps");
                check_hip(hipHostMalloc(reinterpret_cast<void **>(&t->step_ids_host), sizeof(int32_t) * L * K,
                                        hipHostMallocDefault), "tier ids");
                check_hip(hipEventCreateWithFlags(&t->step_done, hipEventDisableTiming), "tier event");
                check_hip(hipMalloc(reinterpret_cast<void **>(&t->staged),
                                    static_cast<size_t>(L * K) * (t->gu_bytes + t->dn_bytes)), "tier staging area");
            }
            if (t->used) check_hip(hipEventSynchronize(t->last_use), "tier mode change");
            check_hip(hipStreamSynchronize(t->copy_stream), "tier mode change");
            for (int64_t l = 0; l < L; ++l)
                check_status(vbm_admission_slot_map(t->admission, l, t->host_maps + l * E), "tier slot map");
            t->deferred = true;
        } else {
            tier_quiesce(*t);
            t->deferred = false;
        }
    });
}

vbm_status vbm_tier_reset(vbm_tier * t, int policy, int64_t recent_window, int64_t margin) {
    return guarded([&] {
        require(t != nullptr, "null tier");
        tier_quiesce(*t);
        if (t->used) check_hip(hipEventSynchronize(t->last_use), "tier reset");
        check_hip(hipStreamSynchronize(t->copy_stream), "tier reset");
        const vbm_tier_desc & d = t->desc;
        vbm_admission * fresh = nullptr;
        check_status(vbm_admission_create(d.n_layers, d.n_expert, d.top_k, d.n_slots, recent_window, margin, policy,
                                          &fresh), "tier admission");
        vbm_admission_destroy(t->admission);
        t->admission = fresh;
        t->desc.policy = policy;
        t->desc.recent_window = recent_window;
        t->desc.margin = margin;
        t->stats = vbm_tier_stats{};
        t->step_pending = t->awaiting = t->enqueued = false;
        t->started = false;
        t->used = false;
        if (t->deferred)
            for (int64_t l = 0; l < d.n_layers; ++l)
                check_status(vbm_admission_slot_map(t->admission, l, t->host_maps + l * d.n_expert), "tier slot map");
    });
}

vbm_status vbm_tier_step_begin(vbm_tier * t) {
    return guarded([&] {
        require(t != nullptr && t->deferred, "vbm_tier_step_begin needs deferred mode");
        tier_begin_step(*t);
    });
}

vbm_status vbm_tier_step_enqueue(vbm_tier * t, const float * x, const float * logits, float * out, int32_t * ids,
                                 void * stream) {
    return guarded([&] {
        require(t != nullptr && t->deferred, "vbm_tier_step_enqueue needs deferred mode");
        require(x && logits && out, "null buffer");
        require(reinterpret_cast<uintptr_t>(x) % 16 == 0, "decode input must be 16-byte aligned");
        const hipStream_t s = as_stream(stream);
        // An eager enqueue belongs to the step begun last, once: a second one would overwrite that
        // step's id hand-off and lose its admissions. A captured enqueue is exempt (its replays,
        // one per begin, cannot be checked from here).
        if (!stream_capturing(s)) {
            require(t->awaiting && !t->enqueued, "vbm_tier_step_enqueue needs a vbm_tier_step_begin before it (one enqueue per begin)");
            t->enqueued = true;
        }
        tier_enqueue_step(*t, x, logits, out, ids, s);
    });
}

vbm_status vbm_tier_flush(vbm_tier * t) {
    return guarded([&] {
        require(t != nullptr, "null tier");
        tier_quiesce(*t);
    });
}

vbm_status vbm_tier_set_trace(vbm_tier * t, vbm_trace * trace) {
    return guarded([&] {
        require(t != nullptr, "null tier");
        require(trace == nullptr || !t->deferred, "deferred mode records no routing trace");
        std::vector<int64_t> ids;
        if (trace) {
            int64_t n = 0;
            check_status(vbm_trace_position(trace, &n, nullptr, nullptr, nullptr), "tier trace");
            require(n == t->desc.n_layers, "trace layer count does not match the tier");
            for (int64_t l = 0; l < n; ++l) {
                int64_t id = 0, experts = 0, active = 0;
                check_status(vbm_trace_layer_info(trace, l, &id, &experts, &active), "tier trace");
                require(experts == t->desc.n_expert && active == t->desc.top_k,
                        "trace layer expert counts do not match the tier");
                ids.push_back(id);
            }
        }
        t->trace = trace;
        t->trace_layer_ids = std::move(ids);
    });
}

vbm_status vbm_tier_get_stats(const vbm_tier * t, vbm_tier_stats * stats) {
    return guarded([&] {
        require(t != nullptr && stats != nullptr, "null argument");
        *stats = t->stats;
    });
}

}  // extern "C"
