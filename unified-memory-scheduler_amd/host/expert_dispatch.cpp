// ExpertPlan: routes split into CPU and GPU job lists by residency, both runners executed (the GPU
// one on its own thread), and the weighted sum in rank order. The observable contract is the
// reference's (tools/engine/expert_dispatch.hpp:10-48; its tests/test_expert_dispatch.cpp passes
// against this file): invalid plans and missing runners are std::invalid_argument before any work
// starts; runner failures propagate CPU-first, only after both runners have returned; runner
// outputs of the wrong size or with non-finite values, and a non-finite weighted sum, are
// std::runtime_error; out[row] = ((0 + w0 * v0) + w1 * v1) + ... in route order.
#include "expert_dispatch.hpp"

#include <algorithm>
#include <cmath>
#include <exception>
#include <stdexcept>
#include <thread>

namespace vrambridge::experimental {
namespace {

// Sanity bounds of a plan: a width is one hidden or intermediate size, and the reduced output is
// kept under 1 GiB of fp32.
constexpr std::size_t kMaxWidth = std::size_t{1} << 20;
constexpr std::size_t kMaxOutputFloats = std::size_t{1} << 28;
constexpr std::size_t kMaxExperts = std::size_t{1} << 20;

[[noreturn]] void invalid(const char * why) { throw std::invalid_argument(std::string("expert plan: ") + why); }

void require_output(const std::vector<float> & out, std::size_t jobs, std::size_t width, const char * device) {
    if (out.size() != jobs * width)
        throw std::runtime_error(std::string("expert plan: the ") + device + " runner returned " +
                                 std::to_string(out.size()) + " values for " + std::to_string(jobs) + " jobs of width " +
                                 std::to_string(width));
    if (std::any_of(out.begin(), out.end(), [](float v) { return !std::isfinite(v); }))
        throw std::runtime_error(std::string("expert plan: the ") + device + " runner returned a non-finite value");
}

}  // namespace

ExpertPlan::ExpertPlan(std::size_t width, const std::vector<std::vector<Route>> & routes,
                       const std::vector<std::uint8_t> & gpu_resident)
    : width_(width), rows_(routes.size()) {
    if (width == 0 || width > kMaxWidth) invalid("width must be in 1..2^20");
    if (routes.empty()) invalid("a plan needs at least one row");
    if (gpu_resident.empty() || gpu_resident.size() > kMaxExperts) invalid("residency must list 1..2^20 experts");
    if (std::any_of(gpu_resident.begin(), gpu_resident.end(), [](std::uint8_t f) { return f > 1; }))
        invalid("residency entries must be 0 (CPU) or 1 (GPU)");
    const std::size_t n_experts = gpu_resident.size();
    row_begin_.reserve(rows_ + 1);
    row_begin_.push_back(0);
    std::vector<std::uint32_t> picked;
    for (std::size_t row = 0; row < rows_; ++row) {
        const std::vector<Route> & selection = routes[row];
        if (selection.empty() || selection.size() > n_experts) invalid("each row routes to 1..n_experts experts");
        picked.clear();
        for (const Route & r : selection) {
            if (r.expert >= n_experts) invalid("a route names an expert beyond the residency list");
            if (!std::isfinite(r.weight)) invalid("a route weight is not finite");
            picked.push_back(r.expert);
        }
        std::sort(picked.begin(), picked.end());
        if (std::adjacent_find(picked.begin(), picked.end()) != picked.end()) invalid("a row routes one expert twice");
        for (std::size_t rank = 0; rank < selection.size(); ++rank) {
            const Route & r = selection[rank];
            std::vector<ExpertJob> & list = gpu_resident[r.expert] ? gpu_jobs_ : cpu_jobs_;
            source_.push_back(2 * list.size() + gpu_resident[r.expert]);
            weight_.push_back(r.weight);
            list.push_back(ExpertJob{row, rank, r.expert});
        }
        row_begin_.push_back(source_.size());
        if (rows_ > kMaxOutputFloats / width_ || source_.size() > kMaxOutputFloats / width_)
            invalid("the plan's outputs exceed 2^28 floats");
    }
}

std::vector<float> ExpertPlan::execute(const ExpertRunner & cpu, const ExpertRunner & gpu) const {
    if (!cpu_jobs_.empty() && !cpu) invalid("CPU jobs but no CPU runner");
    if (!gpu_jobs_.empty() && !gpu) invalid("GPU jobs but no GPU runner");

    std::vector<float> gpu_out, cpu_out;
    std::exception_ptr gpu_error, cpu_error;
    std::thread gpu_thread;
    if (!gpu_jobs_.empty()) {
        gpu_thread = std::thread([&] {
            try {
                gpu_out = gpu(gpu_jobs_);
            } catch (...) {
                gpu_error = std::current_exception();
            }
        });
    }
    if (!cpu_jobs_.empty()) {
        try {
            cpu_out = cpu(cpu_jobs_);
        } catch (...) {
            cpu_error = std::current_exception();
        }
    }
    if (gpu_thread.joinable()) gpu_thread.join();   // the GPU runner never outlives this call
    if (cpu_error) std::rethrow_exception(cpu_error);
    if (gpu_error) std::rethrow_exception(gpu_error);
    require_output(cpu_out, cpu_jobs_.size(), width_, "CPU");
    require_output(gpu_out, gpu_jobs_.size(), width_, "GPU");

    std::vector<float> out(rows_ * width_, 0.0f);
    for (std::size_t row = 0; row < rows_; ++row) {
        float * dst = out.data() + row * width_;
        for (std::size_t i = row_begin_[row]; i < row_begin_[row + 1]; ++i) {
            const std::vector<float> & from = (source_[i] & 1) ? gpu_out : cpu_out;
            const float * src = from.data() + (source_[i] >> 1) * width_;
            const float w = weight_[i];
            for (std::size_t c = 0; c < width_; ++c) dst[c] = dst[c] + w * src[c];
        }
    }
    // A partial sum that became infinite or NaN can never turn finite again, so checking the
    // finished rows is the same as checking every step.
    if (std::any_of(out.begin(), out.end(), [](float v) { return !std::isfinite(v); }))
        throw std::runtime_error("expert plan: the weighted sum is not finite");
    return out;
}

}  // namespace vrambridge::experimental
