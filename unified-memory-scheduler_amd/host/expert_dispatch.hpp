// Expert dispatch boundary (C++ host side). Same public interface and semantics as the
// reference's tools/engine/expert_dispatch.hpp:10-48 so callers and the reference's own tests
// (tests/test_expert_dispatch.cpp) compile unchanged: routes (row, rank, expert, weight) are split into CPU and GPU job lists by
// a 0/1 residency vector; the GPU runner runs asynchronously while the CPU runner runs on the
// caller; outputs are checked for shape and finiteness and summed weight*value in route order.
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <vector>

namespace vrambridge::experimental {

struct Route {
    std::uint32_t expert;
    float weight;
};

struct ExpertJob {
    std::size_t row;
    std::size_t rank;
    std::uint32_t expert;
};

// Returns jobs.size() x width floats in job order.
using ExpertRunner = std::function<std::vector<float>(const std::vector<ExpertJob> &)>;

class ExpertPlan {
public:
    // Throws std::invalid_argument for zero/oversized dimensions, residency entries other than
    // 0/1, empty or oversized route lists, out-of-range experts, non-finite weights and duplicate
    // experts within a row.
    ExpertPlan(std::size_t width, const std::vector<std::vector<Route>> & routes,
               const std::vector<std::uint8_t> & gpu_resident);

    std::size_t width() const noexcept { return width_; }
    std::size_t rows() const noexcept { return rows_; }
    const std::vector<ExpertJob> & cpu_jobs() const noexcept { return cpu_jobs_; }
    const std::vector<ExpertJob> & gpu_jobs() const noexcept { return gpu_jobs_; }

    // Runs both runners (GPU one on a separate thread), joins both before rethrowing the first
    // failure (CPU first), validates shapes/finiteness (std::runtime_error) and reduces in route
    // order: out[row] = ((w0*v0) + w1*v1) + ...
    std::vector<float> execute(const ExpertRunner & cpu, const ExpertRunner & gpu) const;

private:
    std::size_t width_;
    std::size_t rows_;
    std::vector<ExpertJob> cpu_jobs_;
    std::vector<ExpertJob> gpu_jobs_;
    // Routes in row-major, rank-minor order: row r owns [row_begin_[r], row_begin_[r + 1]).
    // source_[i] = 2 * (index of the route's job in its list) + (1 if that list is the GPU's).
    std::vector<std::size_t> row_begin_;
    std::vector<std::size_t> source_;
    std::vector<float> weight_;
};

}  // namespace vrambridge::experimental
