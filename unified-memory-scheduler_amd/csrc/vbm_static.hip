// vbm_mul_mat_id_noalloc: GGML_OP_MUL_MAT_ID for callers that cannot allocate device memory (code
// under HIP graph capture, serving loops, harnesses that forbid it). Same kernels as
// vbm_mul_mat_id; its device scratch (the activation rows, the grouping buffers and the GEMM tile
// list) is a fixed file-scope device array instead of memory the library allocates.
//
// The array's name is only a host-side stand-in: the device address used everywhere (kernel
// arguments) is the one hipGetSymbolAddress returns, fetched once per device with that device
// current and kept per device (each GPU holds its own copy of the array). Nothing in it has to
// start at zero: every call's kernels write each scratch word (activation rows, grouping counts,
// offsets and lists, the tile list, the error flag) before reading it, so the previous call's
// contents are never observed.
#include "vbm_internal.hpp"

#include <mutex>
#include <string>

using namespace vbm;

namespace {

constexpr size_t kScratchBytes = VBM_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

__device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_mu;
uint8_t * g_scratch[kMaxDevices] = {};

// The scratch array's address on the current device (looked up on the device's first call).
uint8_t * scratch_on_current_device() {
    int device = 0;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    require(device >= 0 && device < kMaxDevices, "device index out of range for the fixed scratch table");
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch[device]) {
        void * p = nullptr;
        check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        require(p != nullptr, "hipGetSymbolAddress returned no address for the fixed scratch");
        g_scratch[device] = static_cast<uint8_t *>(p);
    }
    return g_scratch[device];
}

}  // namespace

extern "C" {

vbm_status vbm_mul_mat_id_noalloc(const vbm_bank * bank, const int32_t * expert_to_slot, int64_t n_as, int b_type,
                                  const void * b, int64_t b_ne1, const int32_t * ids, int64_t n_ids, int64_t n_tokens,
                                  int64_t ids_stride, const float * bias, float * dst, int order, void * stream) {
    return guarded([&] {
        require(bank != nullptr, "null bank");
        check_mul_mat_id_shape(*bank, n_as, b_ne1, n_ids, n_tokens, ids_stride, order);
        const size_t need = mul_mat_id_scratch_bytes(*bank, n_as, b_ne1, n_ids, n_tokens, order);
        require(need <= kScratchBytes, "vbm_mul_mat_id_noalloc: this call needs " + std::to_string(need) +
                                           " bytes of device scratch, above its fixed " +
                                           std::to_string(kScratchBytes) + "; use vbm_mul_mat_id_ws");
        mul_mat_id(bank, expert_to_slot, nullptr, n_as, b_type, b, b_ne1, ids, n_ids, n_tokens, ids_stride, bias, dst,
                   order, scratch_on_current_device(), kScratchBytes, as_stream(stream));
    });
}

}  // extern "C"
