// Engine-level GPU executors over the C ABI of libvbmoe (see native_hip_down.hpp).
#include "native_hip_down.hpp"

#include "vbmoe.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <set>
#include <stdexcept>
#include <string>

namespace vrambridge::experimental {
namespace {

constexpr std::size_t kMaxFloats = 32 * 1024 * 1024;   // per-tensor bound of the reference engine

bool all_finite(const std::vector<float> & v) {
    return std::all_of(v.begin(), v.end(), [](float x) { return std::isfinite(x); });
}

// Library failures keep their class: argument errors stay std::invalid_argument.
void check(vbm_status st, const char * what) {
    if (st == VBM_OK) return;
    const std::string msg = std::string(what) + ": " + vbm_last_error();
    if (st == VBM_ERR_INVALID_ARGUMENT) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

// ggml dequantization of one row of `k` values: MXFP4 e2m1 x 2^(e - 127) (the doubled table
// scaled by 2^(e - 128)), Q8_0 q x fp16 d.
float half_to_float(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff, bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {                                  // subnormal: renormalize
            exp = 127 - 15 + 1;
            while (!(man & 0x400)) {
                man <<= 1;
                --exp;
            }
            bits = sign | (exp << 23) | ((man & 0x3ff) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, sizeof(f));
    return f;
}

void dequantize_row(int type, const uint8_t * src, float * dst, std::size_t k) {
    static const float kDoubledE2M1[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
    for (std::size_t b = 0; b < k / 32; ++b) {
        if (type == VBM_TYPE_MXFP4) {
            const uint8_t * blk = src + b * 17;
            const float scale = std::ldexp(1.0f, static_cast<int>(blk[0]) - 128);
            for (int i = 0; i < 16; ++i) {
                dst[b * 32 + i] = kDoubledE2M1[blk[1 + i] & 0xf] * scale;
                dst[b * 32 + 16 + i] = kDoubledE2M1[blk[1 + i] >> 4] * scale;
            }
        } else {
            const uint8_t * blk = src + b * 34;
            uint16_t d16;
            std::memcpy(&d16, blk, 2);
            const float d = half_to_float(d16);
            for (int i = 0; i < 32; ++i) dst[b * 32 + i] = static_cast<float>(static_cast<int8_t>(blk[2 + i])) * d;
        }
    }
}

const char * type_name(int type) { return type == VBM_TYPE_MXFP4 ? "mxfp4" : type == VBM_TYPE_Q8_0 ? "q8_0" : "f32"; }

}  // namespace

void F32ExpertWeights::validate() const {
    if (!hidden || !intermediate || !experts || hidden > 65536 || intermediate > 65536 || experts > 65536 ||
        hidden > kMaxFloats / intermediate || experts > kMaxFloats / (hidden * intermediate))
        throw std::invalid_argument("invalid or unbounded F32 expert dimensions");
    if (activation != F32Activation::silu && activation != F32Activation::openai_swiglu)
        throw std::invalid_argument("unsupported F32 expert activation");
    const std::size_t matrix = experts * hidden * intermediate;
    if (gate.size() != matrix || up.size() != matrix || down.size() != matrix ||
        (!gate_bias.empty() && gate_bias.size() != experts * intermediate) ||
        (!up_bias.empty() && up_bias.size() != experts * intermediate) ||
        (!down_bias.empty() && down_bias.size() != experts * hidden))
        throw std::invalid_argument("invalid F32 expert tensor shape");
    if (!all_finite(gate) || !all_finite(up) || !all_finite(down) || !all_finite(gate_bias) || !all_finite(up_bias) ||
        !all_finite(down_bias))
        throw std::invalid_argument("non-finite F32 expert weights");
}

LoadedExperts load_gguf_experts(const std::filesystem::path & first_shard, int layer,
                                const std::vector<std::uint32_t> & ids, F32Activation activation) {
    if (layer < 0 || layer >= 4096 || ids.empty() || ids.size() > 16 ||
        std::set<std::uint32_t>(ids.begin(), ids.end()).size() != ids.size())
        throw std::invalid_argument("invalid layer or selected expert IDs");
    vbm_gguf * g = nullptr;
    check(vbm_gguf_open(first_shard.c_str(), &g), "GGUF open");
    std::unique_ptr<vbm_gguf, vbm_status (*)(vbm_gguf *)> owner(g, vbm_gguf_close);
    vbm_gguf_expert_info info{};
    check(vbm_gguf_expert_layer_info(g, layer, &info), "GGUF expert layer");
    if (info.fused_gate_up) throw std::runtime_error("required separate expert tensors are missing");
    for (const auto id : ids)
        if (static_cast<int64_t>(id) >= info.n_expert) throw std::runtime_error("GGUF expert ID outside tensor");
    const std::size_t H = static_cast<std::size_t>(info.hidden), I = static_cast<std::size_t>(info.intermediate);
    const std::size_t n = ids.size();
    LoadedExperts out{};
    F32ExpertWeights & w = out.weights;
    w.hidden = H;
    w.intermediate = I;
    w.experts = n;
    w.activation = activation;
    out.original_ids = ids;
    out.quant_types = {info.gate_up_type, info.gate_up_type, info.down_type};
    out.weight_types = {type_name(info.gate_up_type), type_name(info.gate_up_type), type_name(info.down_type)};
    const std::size_t half = static_cast<std::size_t>(info.gate_up_bytes / 2);   // gate, then up rows
    std::vector<uint8_t> gu(static_cast<std::size_t>(info.gate_up_bytes)), dn(static_cast<std::size_t>(info.down_bytes));
    std::vector<float> bgu(2 * I), bdn(H);
    w.gate.resize(n * I * H);
    w.up.resize(n * I * H);
    w.down.resize(n * H * I);
    if (info.has_bias) {
        w.gate_bias.resize(n * I);
        w.up_bias.resize(n * I);
        w.down_bias.resize(n * H);
    }
    const std::size_t gate_row = half / I, down_row = dn.size() / H;   // bytes per row
    for (std::size_t j = 0; j < n; ++j) {
        check(vbm_gguf_read_expert(g, layer, ids[j], gu.data(), dn.data(), bgu.data(), bdn.data()), "GGUF expert read");
        out.packed_weights[0].insert(out.packed_weights[0].end(), gu.begin(), gu.begin() + static_cast<long>(half));
        out.packed_weights[1].insert(out.packed_weights[1].end(), gu.begin() + static_cast<long>(half), gu.end());
        out.packed_weights[2].insert(out.packed_weights[2].end(), dn.begin(), dn.end());
        for (std::size_t r = 0; r < I; ++r) {
            dequantize_row(info.gate_up_type, gu.data() + r * gate_row, w.gate.data() + (j * I + r) * H, H);
            dequantize_row(info.gate_up_type, gu.data() + half + r * gate_row, w.up.data() + (j * I + r) * H, H);
        }
        for (std::size_t r = 0; r < H; ++r)
            dequantize_row(info.down_type, dn.data() + r * down_row, w.down.data() + (j * H + r) * I, I);
        if (info.has_bias) {
            std::copy(bgu.begin(), bgu.begin() + static_cast<long>(I), w.gate_bias.begin() + static_cast<long>(j * I));
            std::copy(bgu.begin() + static_cast<long>(I), bgu.end(), w.up_bias.begin() + static_cast<long>(j * I));
            std::copy(bdn.begin(), bdn.end(), w.down_bias.begin() + static_cast<long>(j * H));
        }
    }
    w.validate();
    return out;
}

struct Mxfp4NativeHipDown::Impl {
    int device = 0;
    std::size_t hidden = 0, intermediate = 0, experts = 0;
    std::vector<int32_t> slots;          // local expert -> bank slot, -1 when not resident
    vbm_bank * bank = nullptr;
    void * map = nullptr;                // device copy of `slots`
    void * bias = nullptr;               // device [experts][hidden] or null
    void * stream = nullptr;
    std::mutex mutex;

    ~Impl() {
        (void)vbm_set_device(device);
        if (stream) {
            (void)vbm_stream_synchronize(stream);
            (void)vbm_stream_destroy(stream);
        }
        if (bias) (void)vbm_free(bias);
        if (map) (void)vbm_free(map);
        if (bank) (void)vbm_bank_destroy(bank);
    }
};

Mxfp4NativeHipDown::Mxfp4NativeHipDown(const LoadedExperts & loaded, const std::vector<std::uint8_t> & resident,
                                       int device)
    : impl_(std::make_unique<Impl>()) {
    loaded.weights.validate();
    Impl & m = *impl_;
    m.device = device;
    m.hidden = loaded.weights.hidden;
    m.intermediate = loaded.weights.intermediate;
    m.experts = loaded.weights.experts;
    if (device < 0 || resident.size() != m.experts || loaded.quant_types[2] != VBM_TYPE_MXFP4 || m.intermediate % 64 != 0 ||
        m.hidden % 32 != 0)
        throw std::invalid_argument("unsupported MXFP4 native GPU configuration");
    const std::size_t stride = m.hidden * (m.intermediate / 32) * 17;
    if (loaded.packed_weights[2].size() != stride * m.experts)
        throw std::invalid_argument("invalid MXFP4 native packed weights");
    m.slots.assign(m.experts, -1);
    int64_t n_resident = 0;
    for (std::size_t e = 0; e < m.experts; ++e) {
        if (resident[e] > 1) throw std::invalid_argument("invalid GPU residency value");
        if (resident[e]) m.slots[e] = static_cast<int32_t>(n_resident++);
    }
    if (!n_resident) throw std::invalid_argument("no GPU-resident experts");
    check(vbm_set_device(device), "GPU device selection");
    check(vbm_stream_create(&m.stream), "GPU stream creation");
    check(vbm_bank_create(VBM_TYPE_MXFP4, static_cast<int64_t>(m.hidden), static_cast<int64_t>(m.intermediate), n_resident,
                          0, &m.bank), "MXFP4 bank");
    for (std::size_t e = 0; e < m.experts; ++e)
        if (m.slots[e] >= 0)
            check(vbm_bank_upload(m.bank, m.slots[e], loaded.packed_weights[2].data() + e * stride, 0, m.stream),
                  "MXFP4 expert upload");
    check(vbm_malloc(&m.map, sizeof(int32_t) * m.experts), "slot map");
    check(vbm_memcpy_h2d(m.map, m.slots.data(), sizeof(int32_t) * m.experts, m.stream), "slot map upload");
    if (!loaded.weights.down_bias.empty()) {
        check(vbm_malloc(&m.bias, sizeof(float) * m.experts * m.hidden), "down bias");
        check(vbm_memcpy_h2d(m.bias, loaded.weights.down_bias.data(), sizeof(float) * m.experts * m.hidden, m.stream),
              "down bias upload");
    }
    check(vbm_stream_synchronize(m.stream), "MXFP4 upload");
}

Mxfp4NativeHipDown::~Mxfp4NativeHipDown() = default;

std::vector<float> Mxfp4NativeHipDown::execute(const std::vector<std::uint8_t> & packed_q8,
                                               const std::vector<ExpertJob> & jobs) {
    Impl & m = *impl_;
    std::lock_guard<std::mutex> lock(m.mutex);
    const std::size_t row_bytes = m.intermediate / 32 * 34;
    if (jobs.size() > kMaxFloats / m.hidden || jobs.size() > kMaxFloats / m.intermediate ||
        packed_q8.size() != jobs.size() * row_bytes)
        throw std::invalid_argument("invalid packed Q8 input shape");
    if (jobs.empty()) return {};
    std::vector<int32_t> ids;
    ids.reserve(jobs.size());
    for (const auto & job : jobs) {
        if (job.expert >= m.experts || m.slots[job.expert] < 0)
            throw std::invalid_argument("MXFP4 GPU expert is out of range or not resident");
        ids.push_back(static_cast<int32_t>(job.expert));
    }
    check(vbm_set_device(m.device), "GPU device selection");
    const int64_t n = static_cast<int64_t>(jobs.size());
    void *d_b = nullptr, *d_ids = nullptr, *d_out = nullptr;
    auto release = [&] {
        if (d_b) (void)vbm_free(d_b);
        if (d_ids) (void)vbm_free(d_ids);
        if (d_out) (void)vbm_free(d_out);
    };
    std::vector<float> output(static_cast<std::size_t>(n) * m.hidden);
    try {
        check(vbm_malloc(&d_b, packed_q8.size()), "packed Q8 buffer");
        check(vbm_malloc(&d_ids, sizeof(int32_t) * ids.size()), "route buffer");
        check(vbm_malloc(&d_out, sizeof(float) * output.size()), "output buffer");
        check(vbm_memcpy_h2d(d_b, packed_q8.data(), packed_q8.size(), m.stream), "packed Q8 upload");
        check(vbm_memcpy_h2d(d_ids, ids.data(), sizeof(int32_t) * ids.size(), m.stream), "route upload");
        // each job is one token with one routed expert and its own activation row
        // residency was checked above, so no host-side id validation (and its synchronization) here
        check(vbm_mul_mat_id(m.bank, static_cast<const int32_t *>(m.map), nullptr, static_cast<int64_t>(m.experts),
                             VBM_TYPE_Q8_0, d_b, 1, static_cast<const int32_t *>(d_ids), 1, n, 1,
                             static_cast<const float *>(m.bias), static_cast<float *>(d_out), VBM_ORDER_EXACT, m.stream),
              "MXFP4 down");
        check(vbm_memcpy_d2h(output.data(), d_out, sizeof(float) * output.size(), m.stream), "output download");
        check(vbm_stream_synchronize(m.stream), "MXFP4 down execution");
    } catch (...) {
        (void)vbm_stream_synchronize(m.stream);
        release();
        throw;
    }
    release();
    if (!all_finite(output)) throw std::runtime_error("MXFP4 GPU produced non-finite output");
    return output;
}

// ---------------------------------------------------------------------------------------------
// NativeHipExperts

namespace {

// One device allocation per call, released on every path.
struct DeviceBuffers {
    std::vector<void *> ptrs;
    void * get(std::size_t bytes, const char * what) {
        void * p = nullptr;
        check(vbm_malloc(&p, bytes ? bytes : 4), what);
        ptrs.push_back(p);
        return p;
    }
    ~DeviceBuffers() {
        for (void * p : ptrs) (void)vbm_free(p);
    }
};

}  // namespace

struct NativeHipExperts::Impl {
    int device = 0;
    std::size_t hidden = 0, intermediate = 0, experts = 0;
    F32Activation activation = F32Activation::openai_swiglu;
    vbm_bank * banks[3] = {nullptr, nullptr, nullptr};   // gate, up, down (slot = local expert)
    void * bias[3] = {nullptr, nullptr, nullptr};        // device [experts][rows] or null
    void * stream = nullptr;
    mutable std::mutex mutex;

    ~Impl() {
        (void)vbm_set_device(device);
        if (stream) {
            (void)vbm_stream_synchronize(stream);
            (void)vbm_stream_destroy(stream);
        }
        for (int i = 0; i < 3; ++i) {
            if (bias[i]) (void)vbm_free(bias[i]);
            if (banks[i]) (void)vbm_bank_destroy(banks[i]);
        }
    }

    void validate_jobs(const std::vector<float> & input, const std::vector<ExpertJob> & jobs) const {
        if (input.empty() || input.size() % hidden || jobs.size() > kMaxFloats / hidden ||
            jobs.size() > kMaxFloats / intermediate || !all_finite(input))
            throw std::invalid_argument("invalid native expert input");
        for (const auto & job : jobs)
            if (job.row >= input.size() / hidden || job.expert >= experts)
                throw std::invalid_argument("invalid native expert route");
    }

    std::vector<int32_t> route_ids(const std::vector<ExpertJob> & jobs) const {
        std::vector<int32_t> ids;
        ids.reserve(jobs.size());
        for (const auto & job : jobs) {
            if (job.expert >= experts) throw std::invalid_argument("invalid native expert route");
            ids.push_back(static_cast<int32_t>(job.expert));
        }
        return ids;
    }

    // gate / up (part 0 / 1) or down (2) of one activation row per job: b [n][k] of b_type
    void project(int part, int b_type, const void * d_b, const void * d_ids, int64_t n, float * d_out) const {
        check(vbm_mul_mat_id(banks[part], nullptr, nullptr, static_cast<int64_t>(experts), b_type, d_b, 1,
                             static_cast<const int32_t *>(d_ids), 1, n, 1, static_cast<const float *>(bias[part]), d_out,
                             VBM_ORDER_EXACT, stream),
              part == 2 ? "native down" : "native gate / up");
    }

    // activation rows [n][intermediate] on the device from the jobs' input rows
    void activate(const std::vector<float> & input, const std::vector<ExpertJob> & jobs, const F32Transforms & obs,
                  DeviceBuffers & mem, const void * d_ids, float * d_act) const {
        const int64_t n = static_cast<int64_t>(jobs.size());
        std::vector<float> rows(jobs.size() * hidden);
        for (std::size_t j = 0; j < jobs.size(); ++j)
            std::copy_n(input.data() + jobs[j].row * hidden, hidden, rows.data() + j * hidden);
        float * d_x = static_cast<float *>(mem.get(sizeof(float) * rows.size(), "native input"));
        float * d_g = static_cast<float *>(mem.get(sizeof(float) * jobs.size() * intermediate, "native gate"));
        float * d_u = static_cast<float *>(mem.get(sizeof(float) * jobs.size() * intermediate, "native up"));
        check(vbm_memcpy_h2d(d_x, rows.data(), sizeof(float) * rows.size(), stream), "native input upload");
        project(0, VBM_TYPE_F32, d_x, d_ids, n, d_g);
        project(1, VBM_TYPE_F32, d_x, d_ids, n, d_u);
        const int64_t I = static_cast<int64_t>(intermediate);
        check(vbm_glu(activation == F32Activation::silu ? VBM_ACT_SILU : VBM_ACT_SWIGLU_OAI, d_g, d_u, d_act, n, I, I, I, I,
                      1.702f, 7.0f, stream),
              "native activation");
        if (obs.observe) {                       // the observed stages come back to the host
            std::vector<float> g(jobs.size() * intermediate), u(g.size()), a(g.size());
            check(vbm_memcpy_d2h(g.data(), d_g, sizeof(float) * g.size(), stream), "gate download");
            check(vbm_memcpy_d2h(u.data(), d_u, sizeof(float) * u.size(), stream), "up download");
            check(vbm_memcpy_d2h(a.data(), d_act, sizeof(float) * a.size(), stream), "activation download");
            check(vbm_stream_synchronize(stream), "native activation");
            for (std::size_t j = 0; j < jobs.size(); ++j) {
                std::vector<float> gj(g.begin() + j * intermediate, g.begin() + (j + 1) * intermediate);
                std::vector<float> uj(u.begin() + j * intermediate, u.begin() + (j + 1) * intermediate);
                std::vector<float> aj(a.begin() + j * intermediate, a.begin() + (j + 1) * intermediate);
                obs.observe(jobs[j], F32Stage::gate, gj);
                obs.observe(jobs[j], F32Stage::up, uj);
                obs.observe(jobs[j], F32Stage::activation, aj);
            }
        }
    }

    std::vector<float> download(const float * d, std::size_t count, const char * what) const {
        std::vector<float> out(count);
        check(vbm_memcpy_d2h(out.data(), d, sizeof(float) * count, stream), what);
        check(vbm_stream_synchronize(stream), what);
        if (!all_finite(out)) throw std::runtime_error(std::string(what) + ": non-finite output");
        return out;
    }
};

NativeHipExperts::NativeHipExperts(const LoadedExperts & loaded, int device) : impl_(std::make_unique<Impl>()) {
    loaded.weights.validate();
    Impl & m = *impl_;
    m.device = device;
    m.hidden = loaded.weights.hidden;
    m.intermediate = loaded.weights.intermediate;
    m.experts = loaded.weights.experts;
    m.activation = loaded.weights.activation;
    if (device < 0 || m.hidden % 32 || m.intermediate % 32) throw std::invalid_argument("unsupported native GPU expert shape");
    check(vbm_set_device(device), "GPU device selection");
    check(vbm_stream_create(&m.stream), "GPU stream creation");
    const std::vector<float> * biases[3] = {&loaded.weights.gate_bias, &loaded.weights.up_bias, &loaded.weights.down_bias};
    for (int part = 0; part < 3; ++part) {
        const int type = loaded.quant_types[part];
        if (type != VBM_TYPE_MXFP4 && type != VBM_TYPE_Q8_0) throw std::invalid_argument("unsupported native dot format");
        const std::size_t rows = part == 2 ? m.hidden : m.intermediate, k = part == 2 ? m.intermediate : m.hidden;
        const std::size_t row_bytes = k / 32 * (type == VBM_TYPE_MXFP4 ? 17 : 34), stride = rows * row_bytes;
        if (loaded.packed_weights[part].size() != stride * m.experts)
            throw std::runtime_error("invalid native packed expert shape");
        check(vbm_bank_create(type, static_cast<int64_t>(rows), static_cast<int64_t>(k), static_cast<int64_t>(m.experts), 0,
                              &m.banks[part]), "native bank");
        for (std::size_t e = 0; e < m.experts; ++e)
            check(vbm_bank_upload(m.banks[part], static_cast<int64_t>(e), loaded.packed_weights[part].data() + e * stride, 0,
                                  m.stream), "native expert upload");
        if (!biases[part]->empty()) {
            check(vbm_malloc(&m.bias[part], sizeof(float) * biases[part]->size()), "native bias");
            check(vbm_memcpy_h2d(m.bias[part], biases[part]->data(), sizeof(float) * biases[part]->size(), m.stream),
                  "native bias upload");
        }
    }
    check(vbm_stream_synchronize(m.stream), "native expert upload");
}

NativeHipExperts::~NativeHipExperts() = default;

std::vector<float> NativeHipExperts::activations(const std::vector<float> & input, const std::vector<ExpertJob> & jobs,
                                                 const F32Transforms & observations) const {
    const Impl & m = *impl_;
    std::lock_guard<std::mutex> lock(m.mutex);
    m.validate_jobs(input, jobs);
    if (jobs.empty()) return {};
    check(vbm_set_device(m.device), "GPU device selection");
    DeviceBuffers mem;
    const auto ids = m.route_ids(jobs);
    void * d_ids = mem.get(sizeof(int32_t) * ids.size(), "route buffer");
    float * d_act = static_cast<float *>(mem.get(sizeof(float) * jobs.size() * m.intermediate, "activations"));
    try {
        check(vbm_memcpy_h2d(d_ids, ids.data(), sizeof(int32_t) * ids.size(), m.stream), "route upload");
        m.activate(input, jobs, observations, mem, d_ids, d_act);
        return m.download(d_act, jobs.size() * m.intermediate, "native activations");
    } catch (...) {
        (void)vbm_stream_synchronize(m.stream);
        throw;
    }
}

std::vector<float> NativeHipExperts::execute(const std::vector<float> & input, const std::vector<ExpertJob> & jobs,
                                             const F32Transforms & observations) const {
    const Impl & m = *impl_;
    std::lock_guard<std::mutex> lock(m.mutex);
    m.validate_jobs(input, jobs);
    if (jobs.empty()) return {};
    check(vbm_set_device(m.device), "GPU device selection");
    DeviceBuffers mem;
    const auto ids = m.route_ids(jobs);
    const int64_t n = static_cast<int64_t>(jobs.size());
    void * d_ids = mem.get(sizeof(int32_t) * ids.size(), "route buffer");
    float * d_act = static_cast<float *>(mem.get(sizeof(float) * jobs.size() * m.intermediate, "activations"));
    void * d_q = mem.get(jobs.size() * (m.intermediate / 32) * 34, "packed activations");
    float * d_out = static_cast<float *>(mem.get(sizeof(float) * jobs.size() * m.hidden, "output"));
    try {
        check(vbm_memcpy_h2d(d_ids, ids.data(), sizeof(int32_t) * ids.size(), m.stream), "route upload");
        m.activate(input, jobs, observations, mem, d_ids, d_act);
        const int64_t I = static_cast<int64_t>(m.intermediate);
        check(vbm_quantize_q8_0(d_act, n, I, I, d_q, m.stream), "down input quantization");
        m.project(2, VBM_TYPE_Q8_0, d_q, d_ids, n, d_out);
        auto out = m.download(d_out, jobs.size() * m.hidden, "native experts");
        if (observations.observe)
            for (std::size_t j = 0; j < jobs.size(); ++j) {
                std::vector<float> dj(out.begin() + j * m.hidden, out.begin() + (j + 1) * m.hidden);
                observations.observe(jobs[j], F32Stage::down, dj);
            }
        return out;
    } catch (...) {
        (void)vbm_stream_synchronize(m.stream);
        throw;
    }
}

std::vector<std::uint8_t> NativeHipExperts::pack_down(const std::vector<float> & activations) const {
    const Impl & m = *impl_;
    std::lock_guard<std::mutex> lock(m.mutex);
    if (activations.empty() || activations.size() % m.intermediate || activations.size() > kMaxFloats ||
        !all_finite(activations))
        throw std::invalid_argument("invalid native down activations");
    const int64_t n = static_cast<int64_t>(activations.size() / m.intermediate), I = static_cast<int64_t>(m.intermediate);
    check(vbm_set_device(m.device), "GPU device selection");
    DeviceBuffers mem;
    std::vector<std::uint8_t> packed(static_cast<std::size_t>(n) * (m.intermediate / 32) * 34);
    void * d_a = mem.get(sizeof(float) * activations.size(), "activations");
    void * d_q = mem.get(packed.size(), "packed activations");
    check(vbm_memcpy_h2d(d_a, activations.data(), sizeof(float) * activations.size(), m.stream), "activation upload");
    check(vbm_quantize_q8_0(static_cast<const float *>(d_a), n, I, I, d_q, m.stream), "down input quantization");
    check(vbm_memcpy_d2h(packed.data(), d_q, packed.size(), m.stream), "packed download");
    check(vbm_stream_synchronize(m.stream), "pack_down");
    return packed;
}

std::vector<float> NativeHipExperts::execute_down_packed(const std::vector<std::uint8_t> & packed,
                                                         const std::vector<ExpertJob> & jobs) const {
    const Impl & m = *impl_;
    std::lock_guard<std::mutex> lock(m.mutex);
    const std::size_t row_bytes = m.intermediate / 32 * 34;
    if (jobs.size() > kMaxFloats / m.hidden || packed.size() != jobs.size() * row_bytes)
        throw std::invalid_argument("invalid packed native down input");
    if (jobs.empty()) return {};
    const auto ids = m.route_ids(jobs);
    check(vbm_set_device(m.device), "GPU device selection");
    DeviceBuffers mem;
    void * d_ids = mem.get(sizeof(int32_t) * ids.size(), "route buffer");
    void * d_q = mem.get(packed.size(), "packed activations");
    float * d_out = static_cast<float *>(mem.get(sizeof(float) * jobs.size() * m.hidden, "output"));
    try {
        check(vbm_memcpy_h2d(d_ids, ids.data(), sizeof(int32_t) * ids.size(), m.stream), "route upload");
        check(vbm_memcpy_h2d(d_q, packed.data(), packed.size(), m.stream), "packed upload");
        m.project(2, VBM_TYPE_Q8_0, d_q, d_ids, static_cast<int64_t>(jobs.size()), d_out);
        return m.download(d_out, jobs.size() * m.hidden, "native down");
    } catch (...) {
        (void)vbm_stream_synchronize(m.stream);
        throw;
    }
}

std::vector<float> NativeHipExperts::execute_down(const std::vector<float> & activations,
                                                  const std::vector<ExpertJob> & jobs) const {
    if (activations.size() != jobs.size() * impl_->intermediate) throw std::invalid_argument("invalid native down activations");
    return execute_down_packed(pack_down(activations), jobs);
}

}  // namespace vrambridge::experimental
