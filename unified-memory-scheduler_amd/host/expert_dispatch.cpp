// ExpertPlan: partition of routes into CPU/GPU jobs and the ordered weighted reduction.
// Semantics follow tools/engine/expert_dispatch.cpp:22-89 of the reference (validation rules,
// bounded sizes, CPU-before-GPU error precedence with both runners joined, per-contribution
// finiteness check, route-order accumulation starting from +0).
#include "expert_dispatch.hpp"

#include <cmath>
#include <exception>
#include <future>
#include <stdexcept>
#include <thread>

namespace vrambridge::experimental {
namespace {

constexpr std::size_t kMaxFloats = std::size_t{32} << 20;   // bound on any produced buffer
constexpr std::size_t kMaxWidth = 65536;
constexpr std::size_t kMaxRows = 4096;
constexpr std::size_t kMaxExperts = 65536;

bool all_finite(const std::vector<float> & values) {
    for (float v : values)
        if (!std::isfinite(v)) return false;
    return true;
}

void check_output(const std::vector<float> & values, std::size_t jobs, std::size_t width) {
    if (values.size() != jobs * width) throw std::runtime_error("expert runner returned a wrong-sized output");
    if (!all_finite(values)) throw std::runtime_error("expert runner returned a non-finite value");
}

}  // namespace

ExpertPlan::ExpertPlan(std::size_t width, const std::vector<std::vector<Route>> & routes,
                       const std::vector<std::uint8_t> & gpu_resident)
    : width_(width), rows_(routes.size()) {
    if (width == 0 || width > kMaxWidth || routes.empty() || routes.size() > kMaxRows || gpu_resident.empty() ||
        gpu_resident.size() > kMaxExperts || routes.size() > kMaxFloats / width)
        throw std::invalid_argument("expert plan dimensions out of range");
    for (std::uint8_t flag : gpu_resident)
        if (flag > 1) throw std::invalid_argument("residency flags must be 0 or 1");
    // last_row[e] = 1 + the last row that selected expert e (duplicate detection per row).
    std::vector<std::size_t> last_row(gpu_resident.size(), 0);
    for (std::size_t row = 0; row < routes.size(); ++row) {
        const auto & selection = routes[row];
        if (selection.empty() || selection.size() > gpu_resident.size())
            throw std::invalid_argument("each row needs between 1 and n_experts routes");
        for (std::size_t rank = 0; rank < selection.size(); ++rank) {
            const Route & route = selection[rank];
            if (route.expert >= gpu_resident.size()) throw std::invalid_argument("route expert out of range");
            if (!std::isfinite(route.weight)) throw std::invalid_argument("route weight is not finite");
            if (last_row[route.expert] == row + 1) throw std::invalid_argument("expert routed twice in one row");
            last_row[route.expert] = row + 1;
            if (order_.size() >= kMaxFloats / width) throw std::invalid_argument("plan output exceeds its bound");
            const bool on_gpu = gpu_resident[route.expert] == 1;
            std::vector<ExpertJob> & jobs = on_gpu ? gpu_jobs_ : cpu_jobs_;
            order_.push_back({row, jobs.size(), route.weight, on_gpu});
            jobs.push_back({row, rank, route.expert});
        }
    }
}

std::vector<float> ExpertPlan::execute(const ExpertRunner & cpu, const ExpertRunner & gpu) const {
    const bool need_cpu = !cpu_jobs_.empty(), need_gpu = !gpu_jobs_.empty();
    if ((need_cpu && !cpu) || (need_gpu && !gpu)) throw std::invalid_argument("a required expert runner is missing");

    std::future<std::vector<float>> gpu_future;
    if (need_gpu) gpu_future = std::async(std::launch::async, [this, &gpu] { return gpu(gpu_jobs_); });

    std::vector<float> cpu_out, gpu_out;
    std::exception_ptr cpu_failure, gpu_failure;
    if (need_cpu) {
        try { cpu_out = cpu(cpu_jobs_); } catch (...) { cpu_failure = std::current_exception(); }
    }
    if (gpu_future.valid()) {
        try { gpu_out = gpu_future.get(); } catch (...) { gpu_failure = std::current_exception(); }
    }
    if (cpu_failure) std::rethrow_exception(cpu_failure);
    if (gpu_failure) std::rethrow_exception(gpu_failure);
    check_output(cpu_out, cpu_jobs_.size(), width_);
    check_output(gpu_out, gpu_jobs_.size(), width_);

    std::vector<float> result(rows_ * width_, 0.0f);
    for (const Contribution & c : order_) {
        const float * source = (c.on_gpu ? gpu_out : cpu_out).data() + c.job_index * width_;
        float * target = result.data() + c.row * width_;
        for (std::size_t i = 0; i < width_; ++i) {
            const float term = c.weight * source[i];
            target[i] = target[i] + term;
            if (!std::isfinite(target[i])) throw std::runtime_error("weighted reduction overflowed");
        }
    }
    return result;
}

}  // namespace vrambridge::experimental
