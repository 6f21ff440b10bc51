// Decode routing traces in the reference's JSONL schema (host-side; no device calls).
//
// Record shapes, order and validity follow the reference's collector, tools/trace/routing_trace.cpp:
//   metadata       :701-728 (layers from inspect_experts :390-446, device bytes :704-707)
//   request_start  :501-503 (prompt plus decode must fit the context, :497-499)
//   route          :206-216 (one per routed layer and decoded token; ids checked :199-203)
//   request_end    :566-569 (per-token completeness, check_counts :448-461)
//   trace_end      :744, then the partial file ("<path>.part", opened exclusively) is hard-linked
//                  to the destination and removed (:632-634, :697-699, :745-749)
// and the consumer's reader, tools/benchmark/vrambridge-routing.py:79-188 (layers in ascending
// id order within a token, train requests before test requests is the caller's corpus order).
// Every record is one line of compact JSON with keys in ascending byte order and the reference
// serializer's string escapes, so a trace of the same routes is byte-identical to one written
// by the reference collector with the same metadata.
#include "vbm_internal.hpp"

#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <iterator>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

using namespace vbm;

namespace {

// Appends `s` as a JSON string: '"' and '\\' escaped, the five short control escapes, other
// bytes below 0x20 as \u00xx (lower-case hex), everything else (valid UTF-8) verbatim.
void append_json_string(std::string & out, const std::string & s) {
    // strict UTF-8 check: invalid sequences are rejected as the reference serializer rejects them
    for (size_t i = 0; i < s.size();) {
        const unsigned char c = static_cast<unsigned char>(s[i]);
        size_t n = c < 0x80 ? 1 : (c >> 5) == 0x6 ? 2 : (c >> 4) == 0xE ? 3 : (c >> 3) == 0x1E ? 4 : 0;
        require(n != 0 && i + n <= s.size(), "trace strings must be valid UTF-8");
        uint32_t cp = n == 1 ? c : n == 2 ? (c & 0x1F) : n == 3 ? (c & 0x0F) : (c & 0x07);
        for (size_t k = 1; k < n; ++k) {
            const unsigned char d = static_cast<unsigned char>(s[i + k]);
            require((d >> 6) == 0x2, "trace strings must be valid UTF-8");
            cp = (cp << 6) | (d & 0x3F);
        }
        const uint32_t min_cp[5] = {0, 0, 0x80, 0x800, 0x10000};
        require(cp >= min_cp[n] && cp <= 0x10FFFF && !(cp >= 0xD800 && cp <= 0xDFFF),
                "trace strings must be valid UTF-8");
        i += n;
    }
    out += '"';
    for (const char ch : s) {
        const unsigned char c = static_cast<unsigned char>(ch);
        switch (c) {
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            case '\b': out += "\\b"; break;
            case '\f': out += "\\f"; break;
            case '\n': out += "\\n"; break;
            case '\r': out += "\\r"; break;
            case '\t': out += "\\t"; break;
            default:
                if (c < 0x20) {
                    char buf[8];
                    std::snprintf(buf, sizeof(buf), "\\u%04x", c);
                    out += buf;
                } else {
                    out += ch;
                }
        }
    }
    out += '"';
}

// Minimal ordered writer for one JSON object; the caller supplies keys in ascending order.
struct Obj {
    std::string s = "{";
    bool first = true;
    Obj & key(const char * k) {
        if (!first) s += ',';
        first = false;
        append_json_string(s, k);
        s += ':';
        return *this;
    }
    Obj & str(const char * k, const std::string & v) { key(k); append_json_string(s, v); return *this; }
    Obj & num(const char * k, long long v) { key(k); s += std::to_string(v); return *this; }
    Obj & unum(const char * k, unsigned long long v) { key(k); s += std::to_string(v); return *this; }
    Obj & boolean(const char * k, bool v) { key(k); s += v ? "true" : "false"; return *this; }
    Obj & raw(const char * k, const std::string & v) { key(k); s += v; return *this; }
    std::string done() { return s + "}"; }
};

// A JSON value for the prefill summary, printed like the reference serializer's dump(2): keys in
// ascending order, two-space indentation, one element per line, "key": value, [] and {} when empty.
struct JVal {
    enum Kind { Null, Bool, Int, Str, Arr, Obj } kind = Null;
    bool b = false;
    long long i = 0;
    std::string s;
    std::vector<JVal> arr;
    std::map<std::string, JVal> obj;
    static JVal boolean(bool v) { JVal j; j.kind = Bool; j.b = v; return j; }
    static JVal integer(long long v) { JVal j; j.kind = Int; j.i = v; return j; }
    static JVal string(const std::string & v) { JVal j; j.kind = Str; j.s = v; return j; }
    static JVal array() { JVal j; j.kind = Arr; return j; }
    static JVal object() { JVal j; j.kind = Obj; return j; }
    JVal & set(const std::string & k, JVal v) { obj[k] = std::move(v); return *this; }
    void pretty(std::string & out, int depth) const {
        const std::string pad(static_cast<size_t>(2 * (depth + 1)), ' '), close(static_cast<size_t>(2 * depth), ' ');
        switch (kind) {
            case Null: out += "null"; break;
            case Bool: out += b ? "true" : "false"; break;
            case Int: out += std::to_string(i); break;
            case Str: append_json_string(out, s); break;
            case Arr:
                if (arr.empty()) { out += "[]"; break; }
                out += "[\n";
                for (size_t k = 0; k < arr.size(); ++k) {
                    out += pad;
                    arr[k].pretty(out, depth + 1);
                    out += k + 1 < arr.size() ? ",\n" : "\n";
                }
                out += close + "]";
                break;
            case Obj:
                if (obj.empty()) { out += "{}"; break; }
                out += "{\n";
                for (auto it = obj.begin(); it != obj.end(); ++it) {
                    out += pad;
                    append_json_string(out, it->first);
                    out += ": ";
                    it->second.pretty(out, depth + 1);
                    out += std::next(it) != obj.end() ? ",\n" : "\n";
                }
                out += close + "}";
                break;
        }
    }
};

struct TraceLayer {
    int64_t id = 0, experts = 0, active = 0;
    uint64_t bytes = 0, host_bytes = 0;
    std::vector<std::string> types;   // sorted, unique
};

}  // namespace

struct vbm_trace {
    std::string destination, partial;
    FILE * file = nullptr;
    int64_t context_tokens = 0;
    std::vector<TraceLayer> layers;   // ascending id
    std::set<std::string> request_ids;
    uint64_t requests = 0;
    // the open request
    bool in_request = false;
    std::string request;
    int64_t max_tokens = 0;
    int64_t token = 0;                // complete tokens of the open request
    size_t layer_index = 0;           // next layer expected within the current token
    // prefill summary (optional): observed expert rows per routed layer and prompt batch
    std::string architecture, backend_commit, model, collector_sha256;
    std::string prefill_path;         // empty: no summary
    int64_t batch_size = 0, microbatch_size = 0, cpu_threads = 0, batch_threads = 0;
    std::string layers_json;          // the metadata layers array (compact)
    JVal layers_val = JVal::array();
    JVal prefill_requests = JVal::array();
    JVal open_batches = JVal::array();
    std::map<int64_t, int64_t> open_rows;   // layer id -> observed rows of the open request
    std::string request_split, request_category;
    int64_t prompt_tokens = 0;

    void emit(const std::string & line) {
        const std::string text = line + '\n';
        if (std::fwrite(text.data(), 1, text.size(), file) != text.size())
            fail(VBM_ERR_RUNTIME, "Failed to write routing trace.");
    }
    size_t find_layer(int64_t id) const {
        for (size_t i = 0; i < layers.size(); ++i)
            if (layers[i].id == id) return i;
        fail(VBM_ERR_INVALID_ARGUMENT, "route layer " + std::to_string(id) + " is not a routed layer of the trace");
    }
    // With a prefill summary, every routed layer must have observed 1..prompt_tokens prompt rows
    // before decoding starts (routing_trace.cpp:510-519).
    void check_prefill_coverage() const {
        if (prefill_path.empty()) return;
        for (const TraceLayer & L : layers) {
            const auto it = open_rows.find(L.id);
            require(it != open_rows.end() && it->second > 0 && it->second <= prompt_tokens,
                    "Missing or duplicate prefill layer observations.");
        }
    }
    void route(int64_t layer_id, const int32_t * experts, int64_t n) {
        require(in_request, "route is outside a decode request");
        if (token == 0 && layer_index == 0) check_prefill_coverage();
        require(token < max_tokens, "route beyond the request's max_tokens");
        const size_t li = find_layer(layer_id);
        require(li == layer_index, "missing, duplicate, or out-of-order layer observation (expected layer " +
                                       std::to_string(layers[layer_index].id) + ")");
        const TraceLayer & L = layers[li];
        require(experts != nullptr && n == L.active, "route must hold exactly the layer's active experts");
        std::set<int32_t> unique;
        std::string list = "[";
        for (int64_t r = 0; r < n; ++r) {
            const int32_t e = experts[r];
            require(e >= 0 && e < L.experts && unique.insert(e).second, "Out-of-range or duplicate routed expert.");
            if (r) list += ',';
            list += std::to_string(e);
        }
        list += ']';
        emit(Obj().raw("experts", list).num("layer", layer_id).str("phase", "decode").str("request", request)
                 .num("token", token).str("type", "route").done());
        if (++layer_index == layers.size()) {
            layer_index = 0;
            ++token;
        }
    }
    ~vbm_trace() {
        if (file) {
            std::fclose(file);
            std::remove(partial.c_str());
        }
    }
};

extern "C" {

vbm_status vbm_trace_open(const char * path, const char * architecture, const char * backend_commit,
                          const char * model, int64_t context_tokens, const vbm_trace_layer * layers,
                          int64_t n_layers, const char * token_equivalence_check,
                          const char * collector_source_sha256, vbm_trace ** out) {
    return guarded([&] {
        require(path && *path && out, "null argument");
        require(architecture && *architecture, "architecture must be a nonempty string");
        require(backend_commit && *backend_commit, "backend_commit must be a nonempty string");
        require(context_tokens >= 1, "context_tokens must be >= 1");
        require(layers != nullptr && n_layers >= 1, "a trace needs at least one routed layer");
        *out = nullptr;
        if (collector_source_sha256 && *collector_source_sha256) {
            const std::string h = collector_source_sha256;
            require(h.size() == 64 && h.find_first_not_of("0123456789abcdef") == std::string::npos,
                    "collector_source_sha256 must be 64 lower-case hex digits");
        }
        auto t = std::make_unique<vbm_trace>();
        t->destination = path;
        t->architecture = architecture;
        t->backend_commit = backend_commit;
        t->model = model ? model : "";
        t->collector_sha256 = collector_source_sha256 ? collector_source_sha256 : "";
        t->partial = t->destination + ".part";
        t->context_tokens = context_tokens;
        uint64_t device_bytes = 0;
        for (int64_t i = 0; i < n_layers; ++i) {
            const vbm_trace_layer & d = layers[i];
            require(d.id >= 0 && d.experts >= 1 && d.active >= 1 && d.active <= d.experts,
                    "Invalid per-layer expert counts.");
            require(d.bytes_per_expert >= 1 && d.static_host_bytes_per_expert <= d.bytes_per_expert,
                    "invalid per-expert byte accounting");
            TraceLayer L;
            L.id = d.id;
            L.experts = d.experts;
            L.active = d.active;
            L.bytes = d.bytes_per_expert;
            L.host_bytes = d.static_host_bytes_per_expert;
            std::set<std::string> types;
            if (d.tensor_types) {
                std::string all = d.tensor_types, item;
                for (size_t p = 0; p <= all.size(); ++p) {
                    if (p == all.size() || all[p] == ',') {
                        if (!item.empty()) types.insert(item);
                        item.clear();
                    } else {
                        item += all[p];
                    }
                }
            }
            L.types.assign(types.begin(), types.end());
            for (const TraceLayer & other : t->layers) require(other.id != L.id, "duplicate layer id");
            t->layers.push_back(L);
            device_bytes += (L.bytes - L.host_bytes) * static_cast<uint64_t>(L.experts);
        }
        std::sort(t->layers.begin(), t->layers.end(), [](const TraceLayer & a, const TraceLayer & b) { return a.id < b.id; });
        require(access(t->destination.c_str(), F_OK) != 0 && access(t->partial.c_str(), F_OK) != 0,
                "Refusing to overwrite an existing trace or partial trace.");
        t->file = std::fopen(t->partial.c_str(), "wx");
        if (!t->file) fail(VBM_ERR_RUNTIME, "Cannot create partial trace: " + std::string(std::strerror(errno)));
        std::string list = "[";
        for (size_t i = 0; i < t->layers.size(); ++i) {
            const TraceLayer & L = t->layers[i];
            std::string types = "[";
            for (size_t k = 0; k < L.types.size(); ++k) {
                if (k) types += ',';
                append_json_string(types, L.types[k]);
            }
            types += ']';
            JVal lv = JVal::object(), tv = JVal::array();
            for (const auto & name : L.types) tv.arr.push_back(JVal::string(name));
            lv.set("active", JVal::integer(L.active)).set("bytes_per_expert", JVal::integer(static_cast<long long>(L.bytes)))
                .set("experts", JVal::integer(L.experts)).set("id", JVal::integer(L.id))
                .set("static_host_bytes_per_expert", JVal::integer(static_cast<long long>(L.host_bytes)))
                .set("tensor_types", tv);
            t->layers_val.arr.push_back(lv);
            if (i) list += ',';
            list += Obj().num("active", L.active).unum("bytes_per_expert", L.bytes).num("experts", L.experts)
                        .num("id", L.id).unum("static_host_bytes_per_expert", L.host_bytes)
                        .raw("tensor_types", types).done();
        }
        list += ']';
        Obj meta;
        t->layers_json = list;
        meta.str("architecture", architecture).str("backend_commit", backend_commit)
            .str("capture_scope", "decode_only");
        if (!t->collector_sha256.empty()) meta.str("collector_source_sha256", t->collector_sha256);
        meta.num("context_tokens", context_tokens).boolean("instrumented", true).raw("layers", list);
        if (model && *model) meta.str("model", model);
        meta.num("schema_version", 1).unum("static_device_expert_bytes", device_bytes);
        if (token_equivalence_check && *token_equivalence_check)
            meta.str("token_equivalence_check", token_equivalence_check);
        meta.str("type", "metadata");
        t->emit(meta.done());
        *out = t.release();
    });
}

vbm_status vbm_trace_request_start(vbm_trace * t, const char * id, const char * split, const char * category,
                                   int64_t prompt_tokens, int64_t max_tokens) {
    return guarded([&] {
        require(t != nullptr && t->file != nullptr, "closed or null trace");
        require(!t->in_request, "nested requests");
        require(id && *id, "request id must be a nonempty string");
        require(category && *category, "category must be a nonempty string");
        require(split && (std::strcmp(split, "train") == 0 || std::strcmp(split, "test") == 0),
                "split must be \"train\" or \"test\"");
        require(prompt_tokens >= 1 && max_tokens >= 1, "prompt_tokens and max_tokens must be >= 1");
        require(prompt_tokens + max_tokens <= t->context_tokens,
                "Prompt plus requested decode exceeds the actual context.");
        const std::string record = Obj().str("category", category).str("id", id).num("max_tokens", max_tokens)
                                       .num("prompt_tokens", prompt_tokens).str("split", split)
                                       .str("type", "request_start").done();   // validates the strings
        require(t->request_ids.insert(id).second, "duplicate request id");
        t->emit(record);
        t->in_request = true;
        t->request = id;
        t->max_tokens = max_tokens;
        t->token = 0;
        t->layer_index = 0;
        t->request_split = split;
        t->request_category = category;
        t->prompt_tokens = prompt_tokens;
        t->open_batches = JVal::array();
        t->open_rows.clear();
        ++t->requests;
    });
}

vbm_status vbm_trace_route(vbm_trace * t, int64_t layer_id, const int32_t * experts, int64_t n_active) {
    return guarded([&] {
        require(t != nullptr && t->file != nullptr, "closed or null trace");
        t->route(layer_id, experts, n_active);
    });
}

vbm_status vbm_trace_token(vbm_trace * t, const int32_t * ids, int64_t stride) {
    return guarded([&] {
        require(t != nullptr && t->file != nullptr, "closed or null trace");
        require(ids != nullptr, "null ids");
        require(t->layer_index == 0, "a token's routes must start at the first layer");
        for (size_t l = 0; l < t->layers.size(); ++l) {
            const int64_t s = stride > 0 ? stride : t->layers[l].active;
            t->route(t->layers[l].id, ids + static_cast<int64_t>(l) * s, t->layers[l].active);
        }
    });
}

vbm_status vbm_trace_request_end(vbm_trace * t, const char * stop_reason, int token_sequence_equivalent) {
    return guarded([&] {
        require(t != nullptr && t->file != nullptr, "closed or null trace");
        require(t->in_request, "no open request");
        require(t->layer_index == 0, "Missing or duplicate routing observations in layer " +
                                         std::to_string(t->layers[t->layer_index].id));
        require(stop_reason && (std::strcmp(stop_reason, "limit") == 0 || std::strcmp(stop_reason, "eos") == 0),
                "stop_reason must be \"limit\" or \"eos\"");
        const bool limit = std::strcmp(stop_reason, "limit") == 0;
        require(limit == (t->token == t->max_tokens), "stop reason does not match the decoded token count");
        Obj end;
        end.num("decode_tokens", t->token).str("id", t->request).str("stop_reason", stop_reason);
        if (token_sequence_equivalent) end.boolean("token_sequence_equivalent", true);
        end.str("type", "request_end");
        if (t->token == 0) t->check_prefill_coverage();
        t->emit(end.done());
        t->in_request = false;
        if (!t->prefill_path.empty()) {        // routing_trace.cpp:570-580
            JVal cov = JVal::array();
            for (const TraceLayer & L : t->layers) {
                const int64_t rows = t->open_rows[L.id];
                JVal c = JVal::object();
                c.set("covers_all_prompt_rows", JVal::boolean(rows == t->prompt_tokens))
                    .set("layer", JVal::integer(L.id)).set("observed_rows", JVal::integer(rows));
                cov.arr.push_back(c);
            }
            JVal r = JVal::object();
            r.set("batches", t->open_batches).set("category", JVal::string(t->request_category))
                .set("coverage", cov).set("id", JVal::string(t->request)).set("prompt_tokens", JVal::integer(t->prompt_tokens))
                .set("split", JVal::string(t->request_split)).set("token_sequence_equivalent", JVal::boolean(true));
            t->prefill_requests.arr.push_back(r);
        }
    });
}

vbm_status vbm_trace_close(vbm_trace * t) {
    return guarded([&] {
        require(t != nullptr, "null trace");
        std::unique_ptr<vbm_trace> owned(t);
        require(t->file != nullptr, "trace already closed");
        require(!t->in_request, "trace is incomplete: a request is still open");
        require(t->requests >= 1, "trace has no requests");
        t->emit(Obj().boolean("complete", true).unum("requests", t->requests).str("type", "trace_end").done());
        FILE * f = t->file;
        t->file = nullptr;
        if (std::fclose(f) != 0) {
            std::remove(t->partial.c_str());
            fail(VBM_ERR_RUNTIME, "Failed to close routing trace.");
        }
        if (link(t->partial.c_str(), t->destination.c_str()) != 0) {
            const std::string why = std::strerror(errno);
            std::remove(t->partial.c_str());
            fail(VBM_ERR_RUNTIME, "Cannot publish the routing trace: " + why);
        }
        std::remove(t->partial.c_str());
        if (!t->prefill_path.empty()) {        // routing_trace.cpp:750-769
            JVal doc = JVal::object();
            doc.set("schema_version", JVal::integer(1)).set("capture_scope", JVal::string("observed_prefill_expert_rows"))
                .set("instrumented", JVal::boolean(true)).set("performance_measurement", JVal::boolean(false))
                .set("full_model_acceleration_claim", JVal::boolean(false))
                .set("backend_commit", JVal::string(t->backend_commit)).set("architecture", JVal::string(t->architecture))
                .set("batch_size", JVal::integer(t->batch_size)).set("microbatch_size", JVal::integer(t->microbatch_size))
                .set("cpu_threads", JVal::integer(t->cpu_threads)).set("batch_threads", JVal::integer(t->batch_threads))
                .set("context_tokens", JVal::integer(t->context_tokens)).set("layers", t->layers_val)
                .set("coverage_note", JVal::string("Observed graph rows only; final-layer output pruning can omit prompt positions."))
                .set("requests", t->prefill_requests).set("complete", JVal::boolean(true));
            if (!t->model.empty()) doc.set("model", JVal::string(t->model));
            doc.set("collector_source_sha256", JVal::string(t->collector_sha256));
            std::string text;
            doc.pretty(text, 0);
            text += '\n';
            const std::string part = t->prefill_path + ".part";
            FILE * f = std::fopen(part.c_str(), "wx");
            if (!f) fail(VBM_ERR_RUNTIME, "Cannot exclusively create prefill summary.");
            const bool ok = std::fwrite(text.data(), 1, text.size(), f) == text.size();
            if (std::fclose(f) != 0 || !ok || link(part.c_str(), t->prefill_path.c_str()) != 0) {
                std::remove(part.c_str());
                fail(VBM_ERR_RUNTIME, "Failed to publish complete prefill summary.");
            }
            std::remove(part.c_str());
        }
    });
}

vbm_status vbm_trace_enable_prefill(vbm_trace * t, const char * summary_path, int64_t batch_size,
                                    int64_t microbatch_size, int64_t cpu_threads, int64_t batch_threads) {
    return guarded([&] {
        require(t != nullptr && t->file != nullptr, "closed or null trace");
        require(t->requests == 0, "the prefill summary must be enabled before the first request");
        require(t->prefill_path.empty(), "the prefill summary is already enabled");
        // the summary's reader matches it against the trace's collector hash (vrambridge-prefill-seed.py:37)
        require(!t->collector_sha256.empty(), "the prefill summary needs collector_source_sha256 in the trace");
        require(summary_path && *summary_path, "null summary path");
        const std::string path = summary_path;
        require(path != t->destination && path != t->partial && path + ".part" != t->destination &&
                    path + ".part" != t->partial,
                "Prefill output must not alias the trace or partial paths.");
        require(access(path.c_str(), F_OK) != 0 && access((path + ".part").c_str(), F_OK) != 0,
                "Refusing to overwrite an existing prefill summary or partial.");
        require(batch_size >= 1 && microbatch_size >= 1 && cpu_threads >= 0 && batch_threads >= 0,
                "batch sizes must be >= 1 and thread counts >= 0");
        t->prefill_path = path;
        t->batch_size = batch_size;
        t->microbatch_size = microbatch_size;
        t->cpu_threads = cpu_threads;
        t->batch_threads = batch_threads;
    });
}

vbm_status vbm_trace_prefill_enabled(const vbm_trace * t, int * enabled) {
    return guarded([&] {
        require(t != nullptr && enabled != nullptr, "null argument");
        *enabled = t->prefill_path.empty() ? 0 : 1;
    });
}

vbm_status vbm_trace_prefill_route(vbm_trace * t, int64_t layer_id, const int32_t * ids, int64_t rows) {
    return guarded([&] {
        require(t != nullptr && t->file != nullptr, "closed or null trace");
        require(!t->prefill_path.empty(), "no prefill summary enabled");
        require(t->in_request && t->token == 0 && t->layer_index == 0,
                "prefill batches precede the request's decode routes");
        require(rows >= 0 && rows <= 32768, "Unsupported routing tensor shape: prefill rows outside 0..32768");
        require(rows == 0 || ids != nullptr, "null ids");
        const TraceLayer & L = t->layers[t->find_layer(layer_id)];
        // routing_trace.cpp:188-223: each row's experts in range and distinct; rows per expert
        std::vector<int64_t> counts(static_cast<size_t>(L.experts), 0);
        std::vector<char> seen(static_cast<size_t>(L.experts), 0);
        for (int64_t r = 0; r < rows; ++r) {
            const int32_t * row = ids + r * L.active;
            for (int64_t k = 0; k < L.active; ++k) {
                const int32_t e = row[k];
                require(e >= 0 && e < L.experts && !seen[static_cast<size_t>(e)], "Out-of-range or duplicate routed expert.");
                seen[static_cast<size_t>(e)] = 1;
                ++counts[static_cast<size_t>(e)];
            }
            for (int64_t k = 0; k < L.active; ++k) seen[static_cast<size_t>(row[k])] = 0;
        }
        JVal hist = JVal::array();
        for (int64_t c : counts) hist.arr.push_back(JVal::integer(c));
        JVal b = JVal::object();
        b.set("active_experts_per_row", JVal::integer(L.active)).set("expert_row_counts", hist)
            .set("layer", JVal::integer(layer_id)).set("rows", JVal::integer(rows));
        t->open_batches.arr.push_back(b);
        t->open_rows[layer_id] += rows;
    });
}

vbm_status vbm_trace_abort(vbm_trace * t) {
    return guarded([&] { delete t; });
}

vbm_status vbm_trace_layer_info(const vbm_trace * t, int64_t index, int64_t * id, int64_t * experts,
                                int64_t * active) {
    return guarded([&] {
        require(t != nullptr, "null trace");
        require(index >= 0 && index < static_cast<int64_t>(t->layers.size()), "layer index out of range");
        const TraceLayer & L = t->layers[static_cast<size_t>(index)];
        if (id) *id = L.id;
        if (experts) *experts = L.experts;
        if (active) *active = L.active;
    });
}

vbm_status vbm_trace_position(const vbm_trace * t, int64_t * n_layers, int64_t * requests, int64_t * token,
                              int64_t * layer_index) {
    return guarded([&] {
        require(t != nullptr, "null trace");
        if (n_layers) *n_layers = static_cast<int64_t>(t->layers.size());
        if (requests) *requests = static_cast<int64_t>(t->requests);
        if (token) *token = t->in_request ? t->token : -1;
        if (layer_index) *layer_index = static_cast<int64_t>(t->layer_index);
    });
}

}  // extern "C"
