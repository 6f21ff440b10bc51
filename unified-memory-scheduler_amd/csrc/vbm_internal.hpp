// Internal declarations shared by the library's translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <new>
#include <stdexcept>
#include <string>

#include "../../include/vbmoe.h"
#include "vbm_common.hpp"

struct vbm_bank {
    int type = 0;              // VBM_TYPE_MXFP4 or VBM_TYPE_Q8_0
    int64_t rows = 0;          // rows per expert (ggml ne1)
    int64_t k = 0;             // weights per row (ggml ne0)
    int64_t nb = 0;            // blocks per row
    int64_t n_slots = 0;
    int interleave = 0;        // fused gate|up tile interleave
    size_t slot_bytes = 0;
    uint8_t * base = nullptr;  // device
    uint8_t * staging = nullptr;  // device scratch of slot_bytes for repack / export
    int device = 0;
    vbm::SlotGeometry geometry() const { return {rows, nb, type}; }
};

namespace vbm {

struct Error : std::runtime_error {
    vbm_status status;
    Error(vbm_status s, const std::string & message) : std::runtime_error(message), status(s) {}
};

[[noreturn]] inline void fail(vbm_status status, const std::string & message) { throw Error(status, message); }
inline void require(bool condition, const std::string & message) {
    if (!condition) fail(VBM_ERR_INVALID_ARGUMENT, message);
}
inline void check_hip(hipError_t e, const char * what) {
    if (e != hipSuccess) fail(e == hipErrorOutOfMemory ? VBM_ERR_OUT_OF_MEMORY : VBM_ERR_RUNTIME,
                              std::string(what) + ": " + hipGetErrorString(e));
}
inline hipStream_t as_stream(void * s) { return static_cast<hipStream_t>(s); }

void set_last_error(const std::string & message);
void clear_last_error();

// Runs `body`, converting exceptions into a status plus the thread's last-error message.
template <class F>
vbm_status guarded(F && body) {
    try {
        clear_last_error();
        body();
        return VBM_OK;
    } catch (const Error & e) {
        set_last_error(e.what());
        return e.status;
    } catch (const std::bad_alloc &) {
        set_last_error("host allocation failed");
        return VBM_ERR_OUT_OF_MEMORY;
    } catch (const std::invalid_argument & e) {
        set_last_error(e.what());
        return VBM_ERR_INVALID_ARGUMENT;
    } catch (const std::exception & e) {
        set_last_error(e.what());
        return VBM_ERR_RUNTIME;
    }
}

// Launch helpers implemented in the .hip units (all enqueue on `stream`).
void launch_bank_scatter(const vbm_bank & bank, int64_t slot, const uint8_t * ggml_src, hipStream_t stream);
void launch_bank_gather(const vbm_bank & bank, int64_t slot, uint8_t * ggml_dst, hipStream_t stream);
void launch_bank_generate(const vbm_bank & bank, int64_t first_slot, int64_t count, uint64_t seed,
                          uint64_t stream_id, int64_t first_expert, float p0, float p1, hipStream_t stream);

struct GroupBuffers {
    int32_t * counts;    // [n_as]
    int32_t * offsets;   // [n_as + 1]
    int32_t * rows;      // [n_ids * n_tokens]
    int32_t * active;    // [n_as] experts with count > 0, ascending
    int32_t * n_active;  // [1]
    int32_t * error;     // [1]
};
size_t group_workspace_bytes(int64_t n_as, int64_t n_entries);
GroupBuffers carve_group(void * base, int64_t n_as, int64_t n_entries);
void launch_group(const int32_t * ids, int64_t n_ids, int64_t n_tokens, int64_t ids_stride, int64_t n_as,
                  const GroupBuffers & g, hipStream_t stream);

void launch_quantize_q8_0(const float * x, int64_t n_rows, int64_t k, int64_t x_stride, uint8_t * dst,
                          hipStream_t stream);
void launch_router(const float * router_w, const float * router_b, const float * x, int64_t hidden,
                   float * logits, int64_t n_expert, int64_t n_tokens, int64_t top_k, int32_t * ids,
                   float * weights, hipStream_t stream);
void launch_combine(const float * y, const float * weights, int64_t rows, int64_t n_ids, int64_t n_tokens,
                    float * out, hipStream_t stream);
void launch_add_id(float * y, const float * bias, const int32_t * ids, int64_t rows, int64_t n_ids,
                   int64_t n_tokens, int64_t ids_stride, hipStream_t stream);
void launch_glu(int activation, const float * gate, const float * up, float * out, int64_t n_rows,
                int64_t width, int64_t gate_stride, int64_t up_stride, int64_t out_stride, float alpha,
                float limit, hipStream_t stream);

// Expert GEMV over grouped jobs. Activation input is Q8_0 blocks (act_q8, row stride in bytes)
// or fp32 rows (act_f32, row stride in floats) quantized inside the kernel. act_row(j) =
// b_ne1 == 1 ? j / n_ids : j. Epilogue 0 writes dst[j][rows] (+bias), epilogue 1 (fused
// gate|up bank) writes the GLU output dst[j][rows/2].
struct GemvArgs {
    const vbm_bank * bank;
    const int32_t * expert_to_slot;   // device or null
    const uint8_t * act_q8;
    const float * act_f32;
    int64_t act_stride;               // bytes for q8, floats for f32
    int64_t n_ids, b_ne1;
    GroupBuffers group;
    int64_t max_active;               // host bound on the number of active experts
    int64_t max_per_expert;           // host bound on jobs per expert
    const float * bias;               // [n_as][rows] ggml row order, or null
    float * dst;
    int epilogue;                     // 0 plain, 1 GLU
    int activation;
    float alpha, limit;
};
void launch_gemv(const GemvArgs & a, hipStream_t stream);

}  // namespace vbm
