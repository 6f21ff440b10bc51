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
    void route(int64_t layer_id, const int32_t * experts, int64_t n) {
        require(in_request, "route is outside a decode request");
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
                          int64_t n_layers, const char * token_equivalence_check, vbm_trace ** out) {
    return guarded([&] {
        require(path && *path && out, "null argument");
        require(architecture && *architecture, "architecture must be a nonempty string");
        require(backend_commit && *backend_commit, "backend_commit must be a nonempty string");
        require(context_tokens >= 1, "context_tokens must be >= 1");
        require(layers != nullptr && n_layers >= 1, "a trace needs at least one routed layer");
        *out = nullptr;
        auto t = std::make_unique<vbm_trace>();
        t->destination = path;
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
            if (i) list += ',';
            list += Obj().num("active", L.active).unum("bytes_per_expert", L.bytes).num("experts", L.experts)
                        .num("id", L.id).unum("static_host_bytes_per_expert", L.host_bytes)
                        .raw("tensor_types", types).done();
        }
        list += ']';
        Obj meta;
        meta.str("architecture", architecture).str("backend_commit", backend_commit)
            .str("capture_scope", "decode_only").num("context_tokens", context_tokens).boolean("instrumented", true)
            .raw("layers", list);
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
        t->emit(end.done());
        t->in_request = false;
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
