// Driver for the engine-level mirror (unified-memory-scheduler_amd/host/native_hip_down.hpp),
// run by tests/test_native_hip_down.py. Modes:
//   load <gguf> <layer> <out> <ids...>
//       load_gguf_experts(..., openai_swiglu) and dump, in order: hidden, intermediate, experts,
//       quant_types[3] (int64 each), then packed gate / up / down bytes, then the fp32 gate, up,
//       down weights and gate / up / down biases (each preceded by its int64 length).
//   down <gguf> <layer> <in> <out> <ids...>
//       Mxfp4NativeHipDown over the loaded experts; <in> holds int64 n_jobs, the residency
//       bytes (experts of them), the jobs (int64 row, rank, expert each) and the packed Q8_0
//       rows; <out> receives the jobs x hidden floats. Then checks that a job on a non-resident
//       expert and a short input are rejected with std::invalid_argument.
//   experts <gguf> <layer> <in> <out> <ids...>
//       NativeHipExperts over the loaded experts; <in> holds int64 n_rows, int64 n_jobs, the fp32
//       input rows and the jobs; <out> receives execute() (jobs x hidden), activations() (jobs x
//       intermediate), pack_down(activations) bytes and execute_down(activations) (jobs x
//       hidden). Prints the number of observed stages and checks two rejections.
#include "native_hip_down.hpp"

#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <stdexcept>
#include <string>
#include <vector>

using namespace vrambridge::experimental;

namespace {

template <class T>
void put_vec(std::ofstream & f, const std::vector<T> & v) {
    const int64_t n = static_cast<int64_t>(v.size());
    f.write(reinterpret_cast<const char *>(&n), sizeof(n));
    f.write(reinterpret_cast<const char *>(v.data()), static_cast<std::streamsize>(v.size() * sizeof(T)));
}

void put(std::ofstream & f, int64_t v) { f.write(reinterpret_cast<const char *>(&v), sizeof(v)); }

int64_t get(std::ifstream & f) {
    int64_t v = 0;
    f.read(reinterpret_cast<char *>(&v), sizeof(v));
    if (!f) throw std::runtime_error("short input file");
    return v;
}

}  // namespace

int main(int argc, char ** argv) {
    try {
        if (argc < 5) {
            std::cerr << "usage: load <gguf> <layer> <out> <ids...> | down <gguf> <layer> <in> <out> <ids...>\n";
            return 2;
        }
        const std::string mode = argv[1];
        const int layer = std::atoi(argv[3]);
        const int first_id = mode == "load" ? 5 : 6;
        std::vector<std::uint32_t> ids;
        for (int i = first_id; i < argc; ++i) ids.push_back(static_cast<std::uint32_t>(std::atoi(argv[i])));
        const LoadedExperts loaded = load_gguf_experts(argv[2], layer, ids, F32Activation::openai_swiglu);
        if (mode == "experts") {
            std::ifstream in(argv[4], std::ios::binary);
            const int64_t n_rows = get(in), n_jobs = get(in);
            std::vector<float> input(static_cast<std::size_t>(n_rows) * loaded.weights.hidden);
            in.read(reinterpret_cast<char *>(input.data()), static_cast<std::streamsize>(input.size() * sizeof(float)));
            std::vector<ExpertJob> jobs(static_cast<std::size_t>(n_jobs));
            for (auto & j : jobs) {
                j.row = static_cast<std::size_t>(get(in));
                j.rank = static_cast<std::size_t>(get(in));
                j.expert = static_cast<std::uint32_t>(get(in));
            }
            NativeHipExperts gpu(loaded);
            std::size_t observed = 0;
            F32Transforms obs;
            obs.observe = [&](const ExpertJob &, F32Stage, const std::vector<float> &) { ++observed; };
            const auto out = gpu.execute(input, jobs, obs);
            const auto act = gpu.activations(input, jobs);
            const auto packed = gpu.pack_down(act);
            const auto down = gpu.execute_down(act, jobs);
            std::ofstream f(argv[5], std::ios::binary);
            f.write(reinterpret_cast<const char *>(out.data()), static_cast<std::streamsize>(out.size() * sizeof(float)));
            f.write(reinterpret_cast<const char *>(act.data()), static_cast<std::streamsize>(act.size() * sizeof(float)));
            f.write(reinterpret_cast<const char *>(packed.data()), static_cast<std::streamsize>(packed.size()));
            f.write(reinterpret_cast<const char *>(down.data()), static_cast<std::streamsize>(down.size() * sizeof(float)));
            int rejected = 0;
            try {
                (void)gpu.execute(input, {ExpertJob{static_cast<std::size_t>(n_rows), 0, 0}});
            } catch (const std::invalid_argument &) {
                ++rejected;
            }
            try {
                (void)gpu.execute_down_packed(std::vector<std::uint8_t>(packed.size() - 1), jobs);
            } catch (const std::invalid_argument &) {
                ++rejected;
            }
            std::cout << "observed " << observed << " stages; rejected " << rejected << "\n";
            return 0;
        }
        if (mode == "load") {
            std::ofstream f(argv[4], std::ios::binary);
            put(f, static_cast<int64_t>(loaded.weights.hidden));
            put(f, static_cast<int64_t>(loaded.weights.intermediate));
            put(f, static_cast<int64_t>(loaded.weights.experts));
            for (int t : loaded.quant_types) put(f, t);
            for (const auto & p : loaded.packed_weights) put_vec(f, p);
            for (const auto * v : {&loaded.weights.gate, &loaded.weights.up, &loaded.weights.down, &loaded.weights.gate_bias,
                                   &loaded.weights.up_bias, &loaded.weights.down_bias})
                put_vec(f, *v);
            std::cout << "loaded " << loaded.weights.experts << " experts (" << loaded.weight_types[2] << ")\n";
            return 0;
        }
        std::ifstream in(argv[4], std::ios::binary);
        const int64_t n_jobs = get(in);
        std::vector<std::uint8_t> resident(loaded.weights.experts);
        in.read(reinterpret_cast<char *>(resident.data()), static_cast<std::streamsize>(resident.size()));
        std::vector<ExpertJob> jobs(static_cast<std::size_t>(n_jobs));
        for (auto & j : jobs) {
            j.row = static_cast<std::size_t>(get(in));
            j.rank = static_cast<std::size_t>(get(in));
            j.expert = static_cast<std::uint32_t>(get(in));
        }
        const std::size_t row_bytes = loaded.weights.intermediate / 32 * 34;
        std::vector<std::uint8_t> packed(static_cast<std::size_t>(n_jobs) * row_bytes);
        in.read(reinterpret_cast<char *>(packed.data()), static_cast<std::streamsize>(packed.size()));
        if (!in) throw std::runtime_error("short input file");
        Mxfp4NativeHipDown down(loaded, resident);
        const std::vector<float> out = down.execute(packed, jobs);
        std::ofstream f(argv[5], std::ios::binary);
        f.write(reinterpret_cast<const char *>(out.data()), static_cast<std::streamsize>(out.size() * sizeof(float)));
        int rejected = 0;
        for (std::size_t e = 0; e < resident.size(); ++e)
            if (!resident[e]) {
                try {
                    (void)down.execute(std::vector<std::uint8_t>(row_bytes), {ExpertJob{0, 0, static_cast<std::uint32_t>(e)}});
                } catch (const std::invalid_argument &) {
                    ++rejected;
                }
                break;
            }
        try {
            (void)down.execute(std::vector<std::uint8_t>(row_bytes - 1), {ExpertJob{0, 0, 0}});
        } catch (const std::invalid_argument &) {
            ++rejected;
        }
        std::cout << "executed " << n_jobs << " jobs; rejected " << rejected << "\n";
        return 0;
    } catch (const std::invalid_argument & e) {
        std::cerr << "invalid_argument: " << e.what() << "\n";
        return 3;
    } catch (const std::exception & e) {
        std::cerr << "error: " << e.what() << "\n";
        return 4;
    }
}
