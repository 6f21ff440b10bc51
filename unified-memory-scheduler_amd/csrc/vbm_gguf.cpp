// GGUF expert-tensor loader (host side): the routed-expert tensors of one or more shards of a
// GGUF file, read slice by slice (one expert at a time) into expert banks, bias arrays or the
// host-RAM tier's store.
//
// Follows the reference loader tools/engine/gguf_experts.cpp:
//   shard discovery "<stem>-00001-of-NNNNN.gguf" with 1..100 shards            :27-41
//   blk.L.ffn_{gate,up,down}_exps.{weight,bias}; a tensor in two shards is an error :53-63
//   shape checks (ne3 == 1, experts on ne2 for weights and ne1 for biases)       :64-71
//   uniform per-expert stride, offsets and sizes inside the shard                :75-86
//   projection compatibility (gate == up, down = transposed, same expert count) :114-126
// plus the fused blk.L.ffn_gate_up_exps.weight form that the reference's routing collector also
// accepts (tools/trace/routing_trace.cpp:392,415-419). The container is parsed from the GGUF
// specification (versions 2 and 3: little-endian, u64 counts and string lengths, key/value
// metadata, tensor infos, data section aligned to general.alignment, default 32); no ggml code
// is used.
#include "vbm_internal.hpp"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <memory>
#include <regex>
#include <string>
#include <vector>

using namespace vbm;

namespace {

struct TypeSize {
    int id;
    int block;   // elements per block
    int bytes;   // bytes per block
};
// ggml type ids with fixed block sizes (ggml.h enum ggml_type); others are indexed but unreadable.
constexpr TypeSize kTypes[] = {
    {0, 1, 4},     {1, 1, 2},     {2, 32, 18},   {3, 32, 20},   {6, 32, 22},   {7, 32, 24},
    {8, 32, 34},   {9, 32, 36},   {10, 256, 84}, {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
    {14, 256, 210}, {15, 256, 292}, {20, 32, 18}, {23, 256, 136}, {24, 1, 1},   {25, 1, 2},
    {26, 1, 4},    {27, 1, 8},    {28, 1, 8},    {30, 1, 2},    {39, 32, 17},
};

const TypeSize * type_size(int id) {
    for (const TypeSize & t : kTypes)
        if (t.id == id) return &t;
    return nullptr;
}

struct Tensor {
    int shard = 0;
    int type = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0;   // absolute file offset
    uint64_t nbytes = 0;   // 0 when the type's block size is not known
};

struct Value {
    int type = -1;         // GGUF value type; 9 = array
    uint64_t u = 0;        // integer / bool value
    bool is_signed_negative = false;
    std::string s;         // string value
};

// Bounded sequential reader over one shard.
struct Reader {
    int fd = -1;
    uint64_t size = 0, pos = 0;
    std::vector<uint8_t> buf;
    uint64_t buf_pos = 0;  // file offset of buf[0]

    void read(void * dst, uint64_t n) {
        if (n > size || pos > size - n) fail(VBM_ERR_INVALID_ARGUMENT, "GGUF header runs past the end of the file");
        uint8_t * out = static_cast<uint8_t *>(dst);
        while (n) {
            if (pos < buf_pos || pos >= buf_pos + buf.size()) {
                buf.resize(static_cast<size_t>(std::min<uint64_t>(1 << 20, size - pos)));
                buf_pos = pos;
                uint64_t got = 0;
                while (got < buf.size()) {
                    const ssize_t r = ::pread(fd, buf.data() + got, buf.size() - got, static_cast<off_t>(pos + got));
                    if (r <= 0) fail(VBM_ERR_RUNTIME, "GGUF shard could not be read");
                    got += static_cast<uint64_t>(r);
                }
            }
            const uint64_t off = pos - buf_pos;
            const uint64_t take = std::min<uint64_t>(n, buf.size() - off);
            std::memcpy(out, buf.data() + off, static_cast<size_t>(take));
            out += take;
            pos += take;
            n -= take;
        }
    }
    template <class T> T get() {
        T v;
        read(&v, sizeof(T));
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (n > (1u << 24)) fail(VBM_ERR_INVALID_ARGUMENT, "GGUF string longer than 16 MiB");
        std::string s(static_cast<size_t>(n), '\0');
        read(s.data(), n);
        return s;
    }
    void skip(uint64_t n) {
        if (n > size || pos > size - n) fail(VBM_ERR_INVALID_ARGUMENT, "GGUF header runs past the end of the file");
        pos += n;
    }
};

int scalar_bytes(uint32_t type) {
    switch (type) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
        default: return 0;
    }
}

Value read_value(Reader & r, uint32_t type, int depth) {
    Value v;
    v.type = static_cast<int>(type);
    if (type == 8) {
        v.s = r.str();
    } else if (type == 9) {
        if (depth > 0) fail(VBM_ERR_INVALID_ARGUMENT, "nested GGUF arrays are not supported");
        const uint32_t et = r.get<uint32_t>();
        const uint64_t n = r.get<uint64_t>();
        v.u = n;
        if (et == 8) {
            for (uint64_t i = 0; i < n; ++i) (void)r.str();
        } else if (const int b = scalar_bytes(et)) {
            if (n > r.size) fail(VBM_ERR_INVALID_ARGUMENT, "GGUF array runs past the end of the file");
            r.skip(n * static_cast<uint64_t>(b));
        } else {
            fail(VBM_ERR_INVALID_ARGUMENT, "unknown GGUF array element type " + std::to_string(et));
        }
    } else {
        const int b = scalar_bytes(type);
        if (!b) fail(VBM_ERR_INVALID_ARGUMENT, "unknown GGUF value type " + std::to_string(type));
        uint64_t raw = 0;
        r.read(&raw, static_cast<uint64_t>(b));
        const bool is_int = type != 6 && type != 12;
        const bool is_signed = type == 1 || type == 3 || type == 5 || type == 11;
        if (is_int) {
            if (is_signed) {
                const int shift = 64 - 8 * b;
                const int64_t sv = static_cast<int64_t>(raw << shift) >> shift;
                v.is_signed_negative = sv < 0;
                v.u = static_cast<uint64_t>(sv);
            } else {
                v.u = raw;
            }
        }
    }
    return v;
}

std::vector<std::string> shard_paths(const std::string & first) {
    std::vector<std::string> out{first};
    const size_t slash = first.find_last_of('/');
    const std::string dir = slash == std::string::npos ? "" : first.substr(0, slash + 1);
    const std::string name = slash == std::string::npos ? first : first.substr(slash + 1);
    std::smatch m;
    static const std::regex pattern(R"((.*)-00001-of-([0-9]{5})\.gguf)");
    if (std::regex_match(name, m, pattern)) {
        const int count = std::stoi(m[2].str());
        require(count >= 1 && count <= 100, "invalid GGUF shard count");
        for (int i = 2; i <= count; ++i) {
            char suffix[32];
            std::snprintf(suffix, sizeof(suffix), "-%05d-of-%05d.gguf", i, count);
            out.push_back(dir + m[1].str() + suffix);
        }
    }
    return out;
}

}  // namespace

struct vbm_gguf {
    std::vector<int> fds;
    std::vector<uint64_t> sizes;
    std::map<std::string, Value> kv;        // metadata of the first shard (and later ones, first wins)
    std::map<std::string, Tensor> tensors;

    ~vbm_gguf() {
        for (int fd : fds)
            if (fd >= 0) ::close(fd);
    }
    const Tensor * find(const std::string & name) const {
        const auto it = tensors.find(name);
        return it == tensors.end() ? nullptr : &it->second;
    }
    void read_at(const Tensor & t, uint64_t offset, void * dst, uint64_t n) const {
        uint8_t * out = static_cast<uint8_t *>(dst);
        uint64_t done = 0;
        while (done < n) {
            const ssize_t r = ::pread(fds[t.shard], out + done, static_cast<size_t>(std::min<uint64_t>(n - done, 1u << 30)),
                                      static_cast<off_t>(t.offset + offset + done));
            if (r <= 0) fail(VBM_ERR_RUNTIME, "GGUF expert slice could not be read");
            done += static_cast<uint64_t>(r);
        }
    }
};

namespace {

void parse_shard(vbm_gguf & g, int index, const std::string & path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    struct stat st{};
    if (fd < 0 || ::fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        if (fd >= 0) ::close(fd);
        fail(VBM_ERR_INVALID_ARGUMENT, "GGUF shard missing or not a file: " + path);
    }
    g.fds.push_back(fd);
    g.sizes.push_back(static_cast<uint64_t>(st.st_size));
    Reader r;
    r.fd = fd;
    r.size = static_cast<uint64_t>(st.st_size);
    const uint32_t magic = r.get<uint32_t>();
    require(magic == 0x46554747u, "not a GGUF file (bad magic): " + path);
    const uint32_t version = r.get<uint32_t>();
    require(version == 2 || version == 3, "unsupported GGUF version " + std::to_string(version));
    const uint64_t n_tensors = r.get<uint64_t>();
    const uint64_t n_kv = r.get<uint64_t>();
    require(n_tensors <= (1u << 24) && n_kv <= (1u << 24), "implausible GGUF header counts");
    uint64_t alignment = 32;
    for (uint64_t i = 0; i < n_kv; ++i) {
        const std::string key = r.str();
        const uint32_t type = r.get<uint32_t>();
        Value v = read_value(r, type, 0);
        if (key == "general.alignment") {
            require(type == 4 && v.u > 0 && (v.u & (v.u - 1)) == 0, "general.alignment must be a power-of-two u32");
            alignment = v.u;
        }
        g.kv.emplace(key, std::move(v));
    }
    struct Info {
        std::string name;
        Tensor t;
        uint64_t rel;
    };
    std::vector<Info> infos;
    infos.reserve(static_cast<size_t>(n_tensors));
    for (uint64_t i = 0; i < n_tensors; ++i) {
        Info info;
        info.name = r.str();
        const uint32_t n_dims = r.get<uint32_t>();
        require(n_dims >= 1 && n_dims <= 4, "invalid GGUF tensor rank for " + info.name);
        uint64_t elements = 1;
        for (uint32_t d = 0; d < n_dims; ++d) {
            const uint64_t ne = r.get<uint64_t>();
            require(ne >= 1 && ne < (1ull << 40), "invalid GGUF tensor shape for " + info.name);
            info.t.ne[d] = static_cast<int64_t>(ne);
            require(elements <= (1ull << 62) / ne, "GGUF tensor too large: " + info.name);
            elements *= ne;
        }
        info.t.type = static_cast<int>(r.get<uint32_t>());
        info.rel = r.get<uint64_t>();
        require(info.rel % alignment == 0, "misaligned GGUF tensor offset for " + info.name);
        info.t.shard = index;
        if (const TypeSize * ts = type_size(info.t.type)) {
            require(info.t.ne[0] % ts->block == 0, "GGUF tensor row is not a whole number of blocks: " + info.name);
            info.t.nbytes = elements / static_cast<uint64_t>(ts->block) * static_cast<uint64_t>(ts->bytes);
        }
        infos.push_back(std::move(info));
    }
    const uint64_t data = (r.pos + alignment - 1) / alignment * alignment;
    require(data <= r.size, "GGUF data section starts past the end of the file");
    for (Info & info : infos) {
        require(info.rel <= r.size - data, "GGUF tensor offset exceeds shard: " + info.name);
        info.t.offset = data + info.rel;
        require(info.t.nbytes <= r.size - info.t.offset, "GGUF tensor exceeds shard: " + info.name);
        require(g.tensors.emplace(info.name, info.t).second, "duplicate GGUF tensor across shards: " + info.name);
    }
}

struct ExpertLayer {
    const Tensor * w[3] = {nullptr, nullptr, nullptr};  // gate, up, down (gate == up when fused)
    const Tensor * b[3] = {nullptr, nullptr, nullptr};
    bool fused = false;
    int64_t hidden = 0, inter = 0, n_expert = 0;
    uint64_t stride[3] = {0, 0, 0};                      // per-expert weight bytes (fused: gate_up)
};

ExpertLayer expert_layer(const vbm_gguf & g, int64_t layer) {
    require(layer >= 0 && layer < 4096, "invalid layer");
    const std::string p = "blk." + std::to_string(layer) + ".ffn_";
    ExpertLayer L;
    const Tensor * fused = g.find(p + "gate_up_exps.weight");
    L.w[0] = g.find(p + "gate_exps.weight");
    L.w[1] = g.find(p + "up_exps.weight");
    L.w[2] = g.find(p + "down_exps.weight");
    require(L.w[2] != nullptr, "required expert tensors are missing in layer " + std::to_string(layer));
    if (fused) {
        require(!L.w[0] && !L.w[1], "both fused and separate gate/up expert tensors in layer " + std::to_string(layer));
        L.fused = true;
        L.w[0] = L.w[1] = fused;
    } else {
        require(L.w[0] && L.w[1], "required separate expert tensors are missing in layer " + std::to_string(layer));
    }
    for (int i = 0; i < 3; ++i) {
        const Tensor & t = *L.w[i];
        require(t.ne[3] == 1 && t.ne[2] >= 1 && t.ne[2] <= 65536, "invalid GGUF expert tensor shape");
        require(t.type == VBM_TYPE_MXFP4 || t.type == VBM_TYPE_Q8_0,
                "expert weights must be MXFP4 or Q8_0 (ggml type " + std::to_string(t.type) + ")");
        require(t.nbytes % static_cast<uint64_t>(t.ne[2]) == 0, "nonuniform GGUF expert tensor layout");
        L.stride[i] = t.nbytes / static_cast<uint64_t>(t.ne[2]);
    }
    const Tensor & gate = *L.w[0];
    const Tensor & down = *L.w[2];
    L.hidden = gate.ne[0];
    L.inter = L.fused ? gate.ne[1] / 2 : gate.ne[1];
    L.n_expert = gate.ne[2];
    require(!L.fused || gate.ne[1] % 2 == 0, "fused gate_up expert tensor has an odd row count");
    require(L.fused || (L.w[1]->ne[0] == gate.ne[0] && L.w[1]->ne[1] == gate.ne[1] && L.w[1]->ne[2] == gate.ne[2] &&
                        L.w[1]->type == gate.type),
            "incompatible expert projection shapes");
    require(down.ne[0] == L.inter && down.ne[1] == L.hidden && down.ne[2] == L.n_expert,
            "incompatible expert projection shapes");
    const char * parts[3] = {"gate", "up", "down"};
    for (int i = 0; i < 3; ++i) {
        const Tensor * b = g.find(p + parts[i] + "_exps.bias");
        if (!b) continue;
        require(b->type == VBM_TYPE_F32, "expert biases must be F32");
        require(b->ne[0] == (i == 2 ? L.hidden : L.inter) && b->ne[1] == L.n_expert && b->ne[2] == 1 && b->ne[3] == 1,
                "incompatible expert bias shape");
        L.b[i] = b;
    }
    if (L.fused) {
        const Tensor * b = g.find(p + "gate_up_exps.bias");
        if (b) {
            require(!L.b[0] && !L.b[1], "both fused and separate gate/up biases");
            require(b->type == VBM_TYPE_F32 && b->ne[0] == 2 * L.inter && b->ne[1] == L.n_expert && b->ne[2] == 1,
                    "incompatible expert bias shape");
            L.b[0] = L.b[1] = b;
        }
    }
    require((L.b[0] == nullptr) == (L.b[1] == nullptr), "gate and up biases must both be present or absent");
    return L;
}

// ggml bytes of expert e: gate rows then up rows (2I rows of H), and down rows (H rows of I).
void read_expert(const vbm_gguf & g, const ExpertLayer & L, int64_t e, uint8_t * gate_up, uint8_t * down) {
    require(e >= 0 && e < L.n_expert, "GGUF expert ID outside tensor");
    if (gate_up) {
        if (L.fused) {
            g.read_at(*L.w[0], static_cast<uint64_t>(e) * L.stride[0], gate_up, L.stride[0]);
        } else {
            g.read_at(*L.w[0], static_cast<uint64_t>(e) * L.stride[0], gate_up, L.stride[0]);
            g.read_at(*L.w[1], static_cast<uint64_t>(e) * L.stride[1], gate_up + L.stride[0], L.stride[1]);
        }
    }
    if (down) g.read_at(*L.w[2], static_cast<uint64_t>(e) * L.stride[2], down, L.stride[2]);
}

// fp32 biases of expert e: gate | up (2I) and down (H); zeros when the file has none.
void read_bias(const vbm_gguf & g, const ExpertLayer & L, int64_t e, float * gu, float * dn) {
    const uint64_t I = static_cast<uint64_t>(L.inter), H = static_cast<uint64_t>(L.hidden);
    if (gu) {
        if (!L.b[0]) {
            std::memset(gu, 0, 2 * I * sizeof(float));
        } else if (L.b[0] == L.b[1]) {
            g.read_at(*L.b[0], static_cast<uint64_t>(e) * 2 * I * 4, gu, 2 * I * 4);
        } else {
            g.read_at(*L.b[0], static_cast<uint64_t>(e) * I * 4, gu, I * 4);
            g.read_at(*L.b[1], static_cast<uint64_t>(e) * I * 4, gu + I, I * 4);
        }
    }
    if (dn) {
        if (!L.b[2]) std::memset(dn, 0, H * sizeof(float));
        else g.read_at(*L.b[2], static_cast<uint64_t>(e) * H * 4, dn, H * 4);
    }
}

// All experts' biases of a layer to device arrays indexed by expert id: gate | up [n_expert][2I]
// and down [n_expert][H] (zeros where the file has none). Synchronous on `stream`.
void upload_biases(const vbm_gguf & g, const ExpertLayer & L, float * gate_up_bias, float * down_bias, hipStream_t s) {
    if (!gate_up_bias && !down_bias) return;
    const size_t I2 = static_cast<size_t>(2 * L.inter), H = static_cast<size_t>(L.hidden);
    std::vector<float> bgu(gate_up_bias ? I2 * static_cast<size_t>(L.n_expert) : 0);
    std::vector<float> bdn(down_bias ? H * static_cast<size_t>(L.n_expert) : 0);
    for (int64_t e = 0; e < L.n_expert; ++e)
        read_bias(g, L, e, gate_up_bias ? bgu.data() + e * I2 : nullptr, down_bias ? bdn.data() + e * H : nullptr);
    if (gate_up_bias)
        check_hip(hipMemcpyAsync(gate_up_bias, bgu.data(), bgu.size() * 4, hipMemcpyHostToDevice, s), "bias upload");
    if (down_bias)
        check_hip(hipMemcpyAsync(down_bias, bdn.data(), bdn.size() * 4, hipMemcpyHostToDevice, s), "bias upload");
    check_hip(hipStreamSynchronize(s), "bias upload");
}

}  // namespace

extern "C" {

vbm_status vbm_gguf_open(const char * path, vbm_gguf ** out) {
    return guarded([&] {
        require(path && *path && out, "null argument");
        *out = nullptr;
        auto g = std::make_unique<vbm_gguf>();
        const std::vector<std::string> paths = shard_paths(path);
        for (size_t i = 0; i < paths.size(); ++i) parse_shard(*g, static_cast<int>(i), paths[i]);
        *out = g.release();
    });
}

vbm_status vbm_gguf_close(vbm_gguf * g) {
    return guarded([&] { delete g; });
}

vbm_status vbm_gguf_shards(const vbm_gguf * g, int64_t * shards, int64_t * tensors) {
    return guarded([&] {
        require(g != nullptr, "null gguf");
        if (shards) *shards = static_cast<int64_t>(g->fds.size());
        if (tensors) *tensors = static_cast<int64_t>(g->tensors.size());
    });
}

vbm_status vbm_gguf_get_u64(const vbm_gguf * g, const char * key, uint64_t * value, int * found) {
    return guarded([&] {
        require(g != nullptr && key != nullptr && value != nullptr, "null argument");
        const auto it = g->kv.find(key);
        const bool ok = it != g->kv.end() && it->second.type != 8 && it->second.type != 9 && it->second.type != 6 &&
                        it->second.type != 12 && !it->second.is_signed_negative;
        if (found) *found = ok ? 1 : 0;
        else require(ok, std::string("GGUF key missing or not a non-negative integer: ") + key);
        *value = ok ? it->second.u : 0;
    });
}

vbm_status vbm_gguf_get_string(const vbm_gguf * g, const char * key, char * dst, size_t capacity, int * found) {
    return guarded([&] {
        require(g != nullptr && key != nullptr && dst != nullptr && capacity > 0, "null argument");
        const auto it = g->kv.find(key);
        const bool ok = it != g->kv.end() && it->second.type == 8;
        if (found) *found = ok ? 1 : 0;
        else require(ok, std::string("GGUF key missing or not a string: ") + key);
        const std::string s = ok ? it->second.s : "";
        require(s.size() < capacity, "GGUF string value does not fit the buffer");
        std::memcpy(dst, s.c_str(), s.size() + 1);
    });
}

vbm_status vbm_gguf_tensor_info(const vbm_gguf * g, const char * name, int * type, int64_t * ne,
                                uint64_t * nbytes, int * found) {
    return guarded([&] {
        require(g != nullptr && name != nullptr, "null argument");
        const Tensor * t = g->find(name);
        if (found) *found = t ? 1 : 0;
        else require(t != nullptr, std::string("GGUF tensor not found: ") + name);
        if (type) *type = t ? t->type : -1;
        if (ne)
            for (int d = 0; d < 4; ++d) ne[d] = t ? t->ne[d] : 0;
        if (nbytes) *nbytes = t ? t->nbytes : 0;
    });
}

vbm_status vbm_gguf_expert_layer_info(const vbm_gguf * g, int64_t layer, vbm_gguf_expert_info * info) {
    return guarded([&] {
        require(g != nullptr && info != nullptr, "null argument");
        const ExpertLayer L = expert_layer(*g, layer);
        info->hidden = L.hidden;
        info->intermediate = L.inter;
        info->n_expert = L.n_expert;
        info->gate_up_type = L.w[0]->type;
        info->down_type = L.w[2]->type;
        info->fused_gate_up = L.fused ? 1 : 0;
        info->has_bias = L.b[0] != nullptr || L.b[2] != nullptr;
        info->gate_up_bytes = L.fused ? L.stride[0] : L.stride[0] + L.stride[1];
        info->down_bytes = L.stride[2];
    });
}

vbm_status vbm_gguf_read_expert(const vbm_gguf * g, int64_t layer, int64_t expert, void * gate_up, void * down,
                                float * gate_up_bias, float * down_bias) {
    return guarded([&] {
        require(g != nullptr, "null gguf");
        const ExpertLayer L = expert_layer(*g, layer);
        require(expert >= 0 && expert < L.n_expert, "GGUF expert ID outside tensor");
        read_expert(*g, L, expert, static_cast<uint8_t *>(gate_up), static_cast<uint8_t *>(down));
        read_bias(*g, L, expert, gate_up_bias, down_bias);
    });
}

vbm_status vbm_gguf_load_layer(const vbm_gguf * g, int64_t layer, const int32_t * experts, const int32_t * slots,
                               int64_t n, vbm_bank * gate_up, vbm_bank * down, float * gate_up_bias,
                               float * down_bias, void * stream) {
    return guarded([&] {
        require(g != nullptr && gate_up != nullptr && down != nullptr && experts != nullptr && n >= 1,
                "null argument");
        const ExpertLayer L = expert_layer(*g, layer);
        require(gate_up->type == L.w[0]->type && gate_up->rows == 2 * L.inter && gate_up->k == L.hidden &&
                    gate_up->interleave == 1,
                "gate_up bank does not match the GGUF layer (fused 2*I rows of H, interleaved, same type)");
        require(down->type == L.w[2]->type && down->rows == L.hidden && down->k == L.inter,
                "down bank does not match the GGUF layer (H rows of I, same type)");
        std::vector<uint8_t> gu(gate_up->slot_bytes), dn(down->slot_bytes);
        require(gu.size() == (L.fused ? L.stride[0] : L.stride[0] + L.stride[1]) && dn.size() == L.stride[2],
                "bank slot size does not match the GGUF expert stride");
        for (int64_t i = 0; i < n; ++i) {
            const int64_t e = experts[i];
            const int64_t slot = slots ? slots[i] : e;
            require(e >= 0 && e < L.n_expert, "GGUF expert ID outside tensor");
            require(slot >= 0 && slot < gate_up->n_slots && slot < down->n_slots, "bank slot out of range");
            read_expert(*g, L, e, gu.data(), dn.data());
            const vbm_status s1 = vbm_bank_upload(gate_up, slot, gu.data(), 0, stream);
            if (s1 != VBM_OK) fail(s1, std::string("gate_up upload: ") + vbm_last_error());
            const vbm_status s2 = vbm_bank_upload(down, slot, dn.data(), 0, stream);
            if (s2 != VBM_OK) fail(s2, std::string("down upload: ") + vbm_last_error());
        }
        upload_biases(*g, L, gate_up_bias, down_bias, as_stream(stream));
    });
}

vbm_status vbm_gguf_load_biases(const vbm_gguf * g, int64_t layer, float * gate_up_bias, float * down_bias,
                                void * stream) {
    return guarded([&] {
        require(g != nullptr, "null gguf");
        upload_biases(*g, expert_layer(*g, layer), gate_up_bias, down_bias, as_stream(stream));
    });
}

}  // extern "C"
