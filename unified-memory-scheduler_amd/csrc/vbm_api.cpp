// C ABI: HIP runtime plumbing, synthetic generators and expert bank management.
#include "vbm_internal.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

namespace vbm {
namespace {
thread_local std::string g_last_error;
}
void set_last_error(const std::string & message) { g_last_error = message; }
void clear_last_error() { g_last_error.clear(); }
}  // namespace vbm

using namespace vbm;

extern "C" {

const char * vbm_last_error(void) { return g_last_error.c_str(); }
int vbm_abi_version(void) { return 1; }

// ------------------------------------------------------------------------------------ plumbing
vbm_status vbm_device_count(int * count) {
    return guarded([&] {
        require(count != nullptr, "count is null");
        check_hip(hipGetDeviceCount(count), "hipGetDeviceCount");
    });
}
vbm_status vbm_set_device(int device) {
    return guarded([&] { check_hip(hipSetDevice(device), "hipSetDevice"); });
}
vbm_status vbm_device_name(int device, char * name, size_t capacity) {
    return guarded([&] {
        require(name != nullptr && capacity > 0, "name buffer is empty");
        hipDeviceProp_t prop;
        check_hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
        std::snprintf(name, capacity, "%s (%s, %d CUs)", prop.name, prop.gcnArchName, prop.multiProcessorCount);
    });
}
vbm_status vbm_mem_info(size_t * free_bytes, size_t * total_bytes) {
    return guarded([&] { check_hip(hipMemGetInfo(free_bytes, total_bytes), "hipMemGetInfo"); });
}
vbm_status vbm_malloc(void ** ptr, size_t bytes) {
    return guarded([&] {
        require(ptr != nullptr, "ptr is null");
        *ptr = nullptr;
        if (bytes) check_hip(hipMalloc(ptr, bytes), "hipMalloc");
    });
}
vbm_status vbm_free(void * ptr) {
    return guarded([&] { if (ptr) check_hip(hipFree(ptr), "hipFree"); });
}
vbm_status vbm_host_alloc(void ** ptr, size_t bytes) {
    return guarded([&] {
        require(ptr != nullptr, "ptr is null");
        *ptr = nullptr;
        if (bytes) check_hip(hipHostMalloc(ptr, bytes, hipHostMallocDefault), "hipHostMalloc");
    });
}
vbm_status vbm_host_free(void * ptr) {
    return guarded([&] { if (ptr) check_hip(hipHostFree(ptr), "hipHostFree"); });
}
vbm_status vbm_memcpy_h2d(void * dst, const void * src, size_t bytes, void * stream) {
    return guarded([&] {
        if (bytes) check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)), "H2D copy");
    });
}
vbm_status vbm_memcpy_d2h(void * dst, const void * src, size_t bytes, void * stream) {
    return guarded([&] {
        if (bytes) {
            check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)), "D2H copy");
            check_hip(hipStreamSynchronize(as_stream(stream)), "D2H synchronize");
        }
    });
}
vbm_status vbm_memcpy_d2d(void * dst, const void * src, size_t bytes, void * stream) {
    return guarded([&] {
        if (bytes) check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)), "D2D copy");
    });
}
vbm_status vbm_memset(void * dst, int value, size_t bytes, void * stream) {
    return guarded([&] {
        if (bytes) check_hip(hipMemsetAsync(dst, value, bytes, as_stream(stream)), "hipMemsetAsync");
    });
}
vbm_status vbm_stream_create(void ** stream) {
    return guarded([&] {
        hipStream_t s = nullptr;
        check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
        *stream = s;
    });
}
vbm_status vbm_stream_destroy(void * stream) {
    return guarded([&] {
        if (!stream) return;
        check_hip(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
        release_stream_scratch(as_stream(stream));
        check_hip(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
        check_hip(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy");
    });
}
vbm_status vbm_stream_synchronize(void * stream) {
    return guarded([&] { check_hip(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize"); });
}
vbm_status vbm_device_synchronize(void) {
    return guarded([&] { check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize"); });
}
vbm_status vbm_event_create(void ** event) {
    return guarded([&] {
        hipEvent_t e = nullptr;
        check_hip(hipEventCreate(&e), "hipEventCreate");
        *event = e;
    });
}
vbm_status vbm_event_destroy(void * event) {
    return guarded([&] { if (event) check_hip(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy"); });
}
vbm_status vbm_event_record(void * event, void * stream) {
    return guarded([&] { check_hip(hipEventRecord(static_cast<hipEvent_t>(event), as_stream(stream)), "hipEventRecord"); });
}
vbm_status vbm_event_synchronize(void * event) {
    return guarded([&] { check_hip(hipEventSynchronize(static_cast<hipEvent_t>(event)), "hipEventSynchronize"); });
}
vbm_status vbm_event_query(void * event, int * done) {
    return guarded([&] {
        const hipError_t e = hipEventQuery(static_cast<hipEvent_t>(event));
        if (e == hipErrorNotReady) { *done = 0; return; }
        check_hip(e, "hipEventQuery");
        *done = 1;
    });
}
vbm_status vbm_event_elapsed_ms(void * start, void * stop, float * ms) {
    return guarded([&] {
        check_hip(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)),
                  "hipEventElapsedTime");
    });
}

// ------------------------------------------------------------------------------------ synthetic
vbm_status vbm_synth_mxfp4_host(uint64_t seed, uint64_t stream, uint64_t first_block, uint64_t n_blocks,
                                int exp_lo, int exp_hi, void * dst) {
    return guarded([&] {
        require(dst != nullptr && exp_lo <= exp_hi && exp_lo >= -127 && exp_hi <= 128, "invalid MXFP4 synth arguments");
        const uint64_t key = stream_key(seed, stream);
        auto * out = static_cast<uint8_t *>(dst);
        const unsigned threads = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
        std::vector<std::thread> pool;
        for (unsigned w = 0; w < threads; ++w)
            pool.emplace_back([&, w] {
                for (uint64_t i = w; i < n_blocks; i += threads)
                    synth_mxfp4_block(key, first_block + i, exp_lo, exp_hi, out + i * kMxfp4BlockBytes);
            });
        for (auto & t : pool) t.join();
    });
}

vbm_status vbm_synth_q8_0_host(uint64_t seed, uint64_t stream, uint64_t first_block, uint64_t n_blocks,
                               float scale_lo, float scale_hi, void * dst) {
    return guarded([&] {
        require(dst != nullptr && scale_lo <= scale_hi, "invalid Q8_0 synth arguments");
        const uint64_t key = stream_key(seed, stream);
        auto * out = static_cast<uint8_t *>(dst);
        for (uint64_t i = 0; i < n_blocks; ++i)
            synth_q8_block(key, first_block + i, scale_lo, scale_hi, out + i * kQ8BlockBytes);
    });
}

vbm_status vbm_synth_normal_host(uint64_t seed, uint64_t stream, uint64_t first, uint64_t n, float mean,
                                 float std_dev, float * dst) {
    return guarded([&] {
        require(dst != nullptr || n == 0, "dst is null");
        const uint64_t key = stream_key(seed, stream);
        const unsigned threads = n > 65536 ? std::max(1u, std::min(16u, std::thread::hardware_concurrency())) : 1u;
        std::vector<std::thread> pool;
        for (unsigned w = 0; w < threads; ++w)
            pool.emplace_back([&, w] {
                for (uint64_t i = w; i < n; i += threads) {
                    const uint64_t j = first + i;
                    const double u1 = (static_cast<double>(hash_at(key, 2 * j) >> 11) + 1.0) * 0x1.0p-53;
                    const double u2 = static_cast<double>(hash_at(key, 2 * j + 1) >> 11) * 0x1.0p-53;
                    const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
                    dst[i] = static_cast<float>(mean + std_dev * z);
                }
            });
        for (auto & t : pool) t.join();
    });
}

// ------------------------------------------------------------------------------------ banks
vbm_status vbm_bank_create(int type, int64_t rows, int64_t k, int64_t n_slots, int interleave, vbm_bank ** out) {
    return guarded([&] {
        require(out != nullptr, "bank output is null");
        *out = nullptr;
        require(type == VBM_TYPE_MXFP4 || type == VBM_TYPE_Q8_0, "bank type must be MXFP4 (39) or Q8_0 (8)");
        require(rows > 0 && rows % kTileRows == 0, "bank rows must be a positive multiple of 32");
        require(k > 0 && k % 64 == 0, "bank k must be a positive multiple of 64 (paired 32-blocks)");
        require(n_slots > 0, "bank needs at least one slot");
        require(!interleave || rows % 32 == 0, "interleaved gate|up banks need rows % 32 == 0");
        auto bank = new vbm_bank();
        bank->type = type;
        bank->rows = rows;
        bank->k = k;
        bank->nb = k / 32;
        bank->n_slots = n_slots;
        bank->interleave = interleave ? 1 : 0;
        bank->slot_bytes = static_cast<size_t>(bank->geometry().slot_bytes());
        check_hip(hipGetDevice(&bank->device), "hipGetDevice");
        const hipError_t e = hipMalloc(reinterpret_cast<void **>(&bank->base), bank->slot_bytes * static_cast<size_t>(n_slots));
        if (e != hipSuccess) {
            delete bank;
            check_hip(e, "expert bank allocation");
        }
        *out = bank;
    });
}

vbm_status vbm_bank_destroy(vbm_bank * bank) {
    return guarded([&] {
        if (!bank) return;
        int current = 0;
        (void)hipGetDevice(&current);
        (void)hipSetDevice(bank->device);
        (void)hipDeviceSynchronize();
        if (bank->staging) (void)hipFree(bank->staging);
        if (bank->base) (void)hipFree(bank->base);
        (void)hipSetDevice(current);
        delete bank;
    });
}

vbm_status vbm_bank_info(const vbm_bank * bank, int * type, int64_t * rows, int64_t * k, int64_t * n_slots,
                         size_t * slot_bytes, void ** device_base) {
    return guarded([&] {
        require(bank != nullptr, "bank is null");
        if (type) *type = bank->type;
        if (rows) *rows = bank->rows;
        if (k) *k = bank->k;
        if (n_slots) *n_slots = bank->n_slots;
        if (slot_bytes) *slot_bytes = bank->slot_bytes;
        if (device_base) *device_base = bank->base;
    });
}

static void ensure_staging(vbm_bank * bank) {
    if (!bank->staging) check_hip(hipMalloc(reinterpret_cast<void **>(&bank->staging), bank->slot_bytes), "bank staging");
}

vbm_status vbm_bank_upload(vbm_bank * bank, int64_t slot, const void * src, int src_on_device, void * stream) {
    return guarded([&] {
        require(bank != nullptr && src != nullptr, "bank or source is null");
        require(slot >= 0 && slot < bank->n_slots, "slot out of range");
        const uint8_t * device_src = static_cast<const uint8_t *>(src);
        if (!src_on_device) {
            ensure_staging(bank);
            check_hip(hipMemcpyAsync(bank->staging, src, bank->slot_bytes, hipMemcpyHostToDevice, as_stream(stream)),
                      "expert upload");
            device_src = bank->staging;
        }
        launch_bank_scatter(*bank, slot, device_src, as_stream(stream));
        if (!src_on_device) check_hip(hipStreamSynchronize(as_stream(stream)), "expert upload synchronize");
    });
}

vbm_status vbm_bank_export(const vbm_bank * cbank, int64_t slot, void * dst_host, size_t capacity, void * stream) {
    return guarded([&] {
        auto * bank = const_cast<vbm_bank *>(cbank);
        require(bank != nullptr && dst_host != nullptr, "bank or destination is null");
        require(slot >= 0 && slot < bank->n_slots, "slot out of range");
        require(capacity == bank->slot_bytes, "export destination must be exactly one expert's ggml bytes");
        ensure_staging(bank);
        launch_bank_gather(*bank, slot, bank->staging, as_stream(stream));
        check_hip(hipMemcpyAsync(dst_host, bank->staging, bank->slot_bytes, hipMemcpyDeviceToHost, as_stream(stream)),
                  "expert export");
        check_hip(hipStreamSynchronize(as_stream(stream)), "expert export synchronize");
    });
}

vbm_status vbm_bank_generate(vbm_bank * bank, int64_t first_slot, int64_t count, uint64_t seed, uint64_t stream_id,
                             int64_t first_expert, float p0, float p1, void * stream) {
    return guarded([&] {
        require(bank != nullptr, "bank is null");
        require(first_slot >= 0 && count >= 0 && first_slot + count <= bank->n_slots && first_expert >= 0,
                "slot range out of bounds");
        if (count) launch_bank_generate(*bank, first_slot, count, seed, stream_id, first_expert, p0, p1, as_stream(stream));
    });
}

}  // extern "C"
