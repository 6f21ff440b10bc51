// Expert bank kernels: ggml layout -> tiled bank layout (scatter), the lossless inverse (gather),
// and the on-device synthetic generator writing bank layout directly.
#include "vbm_internal.hpp"

namespace vbm {
namespace {

// One thread per (device row, block). Grid-stride over rows * nb.
__global__ void bank_scatter_kernel(uint8_t * __restrict__ slot, const uint8_t * __restrict__ src,
                                    SlotGeometry g, int interleave) {
    const int64_t total = g.rows * g.nb;
    const int block_bytes = g.type == 39 ? kMxfp4BlockBytes : kQ8BlockBytes;
    for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
         idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t i = idx / g.nb, b = idx % g.nb;              // ggml row, block
        const int64_t d = device_row(i, g.rows, interleave);
        uint8_t blk[34];
        const uint8_t * in = src + idx * block_bytes;
        for (int j = 0; j < block_bytes; ++j) blk[j] = in[j];
        if (g.type == 39) mx_store_block(slot, g, d, b, blk);
        else q8_store_block(slot, g, d, b, blk);
    }
}

__global__ void bank_gather_kernel(const uint8_t * __restrict__ slot, uint8_t * __restrict__ dst,
                                   SlotGeometry g, int interleave) {
    const int64_t total = g.rows * g.nb;
    const int block_bytes = g.type == 39 ? kMxfp4BlockBytes : kQ8BlockBytes;
    for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
         idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t i = idx / g.nb, b = idx % g.nb;
        const int64_t d = device_row(i, g.rows, interleave);
        uint8_t blk[34];
        if (g.type == 39) mx_load_block(slot, g, d, b, blk);
        else q8_load_block(slot, g, d, b, blk);
        uint8_t * out = dst + idx * block_bytes;
        for (int j = 0; j < block_bytes; ++j) out[j] = blk[j];
    }
}

// Slot s (of `count`) holds synthetic expert (first_expert + s): its ggml block (i, b) is global
// block (expert * rows + i) * nb + b of the tensor.
__global__ void bank_generate_kernel(uint8_t * __restrict__ base, size_t slot_bytes, SlotGeometry g,
                                     int interleave, int64_t count, uint64_t key, int64_t first_expert,
                                     float p0, float p1) {
    const int64_t per_slot = g.rows * g.nb;
    const int64_t total = per_slot * count;
    for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
         idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t s = idx / per_slot, within = idx % per_slot;
        const int64_t i = within / g.nb, b = within % g.nb;
        const uint64_t global = static_cast<uint64_t>((first_expert + s) * per_slot + within);
        uint8_t blk[34];
        uint8_t * slot = base + static_cast<size_t>(s) * slot_bytes;
        const int64_t d = device_row(i, g.rows, interleave);
        if (g.type == 39) {
            synth_mxfp4_block(key, global, static_cast<int>(p0), static_cast<int>(p1), blk);
            mx_store_block(slot, g, d, b, blk);
        } else {
            synth_q8_block(key, global, p0, p1, blk);
            q8_store_block(slot, g, d, b, blk);
        }
    }
}

unsigned grid_for(int64_t work, int threads) {
    const int64_t blocks = (work + threads - 1) / threads;
    return static_cast<unsigned>(blocks < 65536 ? blocks : 65536);
}

}  // namespace

void launch_bank_scatter(const vbm_bank & bank, int64_t slot, const uint8_t * src, hipStream_t stream) {
    const SlotGeometry g = bank.geometry();
    hipLaunchKernelGGL(bank_scatter_kernel, dim3(grid_for(g.rows * g.nb, 256)), dim3(256), 0, stream,
                       bank.base + static_cast<size_t>(slot) * bank.slot_bytes, src, g, bank.interleave);
    check_hip(hipGetLastError(), "bank scatter launch");
}

void launch_bank_gather(const vbm_bank & bank, int64_t slot, uint8_t * dst, hipStream_t stream) {
    const SlotGeometry g = bank.geometry();
    hipLaunchKernelGGL(bank_gather_kernel, dim3(grid_for(g.rows * g.nb, 256)), dim3(256), 0, stream,
                       bank.base + static_cast<size_t>(slot) * bank.slot_bytes, dst, g, bank.interleave);
    check_hip(hipGetLastError(), "bank gather launch");
}

void launch_bank_generate(const vbm_bank & bank, int64_t first_slot, int64_t count, uint64_t seed,
                          uint64_t stream_id, int64_t first_expert, float p0, float p1, hipStream_t stream) {
    const SlotGeometry g = bank.geometry();
    hipLaunchKernelGGL(bank_generate_kernel, dim3(grid_for(g.rows * g.nb * count, 256)), dim3(256), 0, stream,
                       bank.base + static_cast<size_t>(first_slot) * bank.slot_bytes, bank.slot_bytes, g,
                       bank.interleave, count, stream_key(seed, stream_id), first_expert, p0, p1);
    check_hip(hipGetLastError(), "bank generate launch");
}

}  // namespace vbm
