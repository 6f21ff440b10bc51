// Stream-ordered host calls: the HIP side of the reference's GGML_OP_CUSTOM host-call nodes
// (struct ggml_host_call, third_party/patches/llama-b11669-hybrid-experts.patch:82-101; the CUDA
// backend's implementation :800-1054). A call copies its device inputs into the call's host
// buffers, runs fn(ctx) on a host thread and copies the host result into the device output, all
// ordered on a side stream forked from the caller's stream, so device work enqueued after the
// call overlaps the host function until a join waits for it; every step is a graph node, so a
// captured graph replays the call.
//
// Two ways to run fn:
//   VBM_HOST_CALL_FUNC     hipLaunchHostFunc on the side stream.
//   VBM_HOST_CALL_MAILBOX  a one-workgroup kernel posts the call into a ring in mapped, coherent
//                          host memory served by a persistent host worker thread per device and
//                          waits for the worker's completion mark, with a bounded number of polls
//                          (on expiry the call counts as timed out and its output is zero-filled).
//                          The sequence counter lives in device memory so graph replays continue
//                          it. Calls whose miss ids hold no zero are posted for bookkeeping only,
//                          not waited for, and their output is zero-filled (ggml_host_call
//                          miss_src semantics).
// Inputs and outputs move by stream-ordered DMA copies (device to host before the post, host to
// device after it), so only the ring itself needs coherent host memory.
#include "vbm_internal.hpp"

#include <atomic>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <thread>

using namespace vbm;

namespace {

constexpr int kMaxDevices = 16;
constexpr uint64_t kRing = 1024;

struct Mailbox {
    uint64_t posted;          // newest request (written by the device)
    uint64_t done;            // newest finished request (written by the host worker)
    uint64_t call[kRing];     // host address of the vbm_host_call of each request
};

__device__ uint64_t g_seq[kMaxDevices];       // requests posted per device
__device__ uint32_t g_timeouts[kMaxDevices];  // posts whose wait expired

struct Worker {
    Mailbox * box = nullptr;  // host view (mapped, coherent)
    Mailbox * box_dev = nullptr;
    std::thread thread;
    std::atomic<bool> stop{false};
};

Worker * g_workers[kMaxDevices] = {};
std::mutex g_workers_mutex;
hipStream_t g_side[kMaxDevices] = {};
std::atomic<uint32_t> g_spin_limit{1u << 21};   // polls of ~1 us each before a waited call expires

struct CallState {
    int device = 0;
    hipEvent_t ready = nullptr, done = nullptr;
    int32_t * skipped = nullptr;   // device flag: output is zero-filled
    uint64_t * seq_host = nullptr; // mapped host word: the ring sequence of this call's last post (0: none)
    uint64_t * seq_dev = nullptr;  // its device address
};

void worker_loop(Worker * w) {
    Mailbox * box = w->box;
    uint64_t seen = 0;
    auto idle_since = std::chrono::steady_clock::now();
    while (!w->stop.load(std::memory_order_relaxed)) {
        const uint64_t posted = __atomic_load_n(&box->posted, __ATOMIC_ACQUIRE);
        if (posted == seen) {
            if (std::chrono::steady_clock::now() - idle_since > std::chrono::milliseconds(2))
                std::this_thread::sleep_for(std::chrono::microseconds(50));
            else
                __builtin_ia32_pause();
            continue;
        }
        while (seen < posted) {
            ++seen;
            auto * call = reinterpret_cast<vbm_host_call *>(__atomic_load_n(&box->call[seen % kRing], __ATOMIC_ACQUIRE));
            if (call && call->fn) call->fn(call->ctx);
            __atomic_store_n(&box->done, seen, __ATOMIC_SEQ_CST);
        }
        idle_since = std::chrono::steady_clock::now();
    }
}

// Stops and joins the workers at exit, before the runtime (initialized earlier, so torn down
// later) releases the mapped ring they poll.
void stop_workers() {
    for (Worker * w : g_workers) {
        if (!w) continue;
        w->stop.store(true);
        if (w->thread.joinable()) w->thread.join();
    }
}

Worker * worker(int device) {
    std::lock_guard<std::mutex> lock(g_workers_mutex);
    if (!g_workers[device]) {
        static const bool registered = std::atexit(stop_workers) == 0;
        (void)registered;
        auto * w = new Worker;
        check_hip(hipHostMalloc(reinterpret_cast<void **>(&w->box), sizeof(Mailbox),
                                hipHostMallocMapped | hipHostMallocCoherent | hipHostMallocPortable),
                  "host-call mailbox");
        std::memset(static_cast<void *>(w->box), 0, sizeof(Mailbox));
        check_hip(hipHostGetDevicePointer(reinterpret_cast<void **>(&w->box_dev), w->box, 0), "host-call mailbox");
        // g_seq[device] starts at zero with the module and only this worker's requests advance it
        w->thread = std::thread(worker_loop, w);
        g_workers[device] = w;
    }
    return g_workers[device];
}

hipStream_t side_stream(int device) {
    std::lock_guard<std::mutex> lock(g_workers_mutex);
    if (!g_side[device]) check_hip(hipStreamCreateWithFlags(&g_side[device], hipStreamNonBlocking), "host-call stream");
    return g_side[device];
}

struct PostArgs {
    const int32_t * miss;   // nullptr: always wait
    int64_t n_miss;
    uint64_t call;          // host address of the call descriptor
    Mailbox * box;          // device view of the ring
    int device;
    int32_t * skipped;
    uint64_t * seq_out;     // the call's last-post word (mapped host memory)
    uint32_t spin_limit;
};

__global__ void __launch_bounds__(256) host_call_post_kernel(PostArgs a) {
    int need = a.miss == nullptr;
    for (int64_t i = threadIdx.x; a.miss && i < a.n_miss; i += blockDim.x) need |= a.miss[i] == 0;
    need = __syncthreads_or(need);
    if (threadIdx.x != 0) return;
    const uint64_t seq = g_seq[a.device] + 1;
    g_seq[a.device] = seq;
    // keep at most kRing requests outstanding (bounded like the completion wait below)
    for (uint32_t i = 0; i < a.spin_limit; ++i) {
        if (__hip_atomic_load(&a.box->done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) + kRing > seq) break;
        __builtin_amdgcn_s_sleep(32);
    }
    __hip_atomic_store(&a.box->call[seq % kRing], a.call, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(a.seq_out, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(&a.box->posted, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    int skipped = !need;
    if (need) {
        bool finished = false;
        for (uint32_t i = 0; i < a.spin_limit && !finished; ++i) {
            finished = __hip_atomic_load(&a.box->done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) >= seq;
            if (!finished) __builtin_amdgcn_s_sleep(32);
        }
        if (!finished) {
            atomicAdd(&g_timeouts[a.device], 1u);
            skipped = 1;
        }
    }
    *a.skipped = skipped;
}

// Before a call's inputs are overwritten: its previous post (possibly one that was not waited for)
// must have been handled by the host worker, whose fn may still read them. Bounded like the post's
// own wait; an expiry counts as a timeout.
__global__ void wait_handled_kernel(const Mailbox * box, const uint64_t * seq_slot, int device, uint32_t spin_limit) {
    if (threadIdx.x != 0) return;
    const uint64_t seq = __hip_atomic_load(seq_slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    for (uint32_t i = 0; i < spin_limit; ++i) {
        if (__hip_atomic_load(&box->done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) >= seq) return;
        __builtin_amdgcn_s_sleep(32);
    }
    atomicAdd(&g_timeouts[device], 1u);
}

__global__ void zero_if_skipped_kernel(uint8_t * dst, int64_t n, const int32_t * skipped) {
    if (!*skipped) return;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        dst[i] = 0;
}

__global__ void join_add_kernel(const float * a, const float * b, float * dst, int64_t n) {
    const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (i < n) dst[i] = a[i] + b[i];
}

void trampoline(void * data) {
    auto * call = static_cast<vbm_host_call *>(data);
    call->fn(call->ctx);
}

CallState & state_of(vbm_host_call * call, int device) {
    auto * st = static_cast<CallState *>(call->backend_state);
    if (!st) {
        st = new CallState;
        st->device = device;
        check_hip(hipEventCreateWithFlags(&st->ready, hipEventDisableTiming), "host-call event");
        check_hip(hipEventCreateWithFlags(&st->done, hipEventDisableTiming), "host-call event");
        check_hip(hipMalloc(reinterpret_cast<void **>(&st->skipped), sizeof(int32_t)), "host-call flag");
        check_hip(hipHostMalloc(reinterpret_cast<void **>(&st->seq_host), sizeof(uint64_t),
                                hipHostMallocMapped | hipHostMallocCoherent | hipHostMallocPortable),
                  "host-call sequence word");
        *st->seq_host = 0;
        check_hip(hipHostGetDevicePointer(reinterpret_cast<void **>(&st->seq_dev), st->seq_host, 0),
                  "host-call sequence word");
        call->backend_state = st;
    }
    require(st->device == device, "a host call is bound to the device it first ran on");
    return *st;
}

}  // namespace

extern "C" {

vbm_status vbm_host_call_prepare(vbm_host_call * call, int mode) {
    return guarded([&] {
        require(call != nullptr && call->magic == VBM_HOST_CALL_MAGIC, "not a host-call descriptor");
        require(mode == VBM_HOST_CALL_FUNC || mode == VBM_HOST_CALL_MAILBOX, "unknown host-call mode");
        int device = 0;
        check_hip(hipGetDevice(&device), "hipGetDevice");
        require(device >= 0 && device < kMaxDevices, "device index out of range");
        (void)state_of(call, device);
        (void)side_stream(device);
        if (mode == VBM_HOST_CALL_MAILBOX) (void)worker(device);
    });
}

vbm_status vbm_host_call_enqueue(vbm_host_call * call, const void * const * srcs, const size_t * src_bytes, int n_src,
                                 void * dst, size_t dst_bytes, const int32_t * miss, int64_t n_miss, int mode,
                                 void * stream) {
    return guarded([&] {
        require(call != nullptr && call->magic == VBM_HOST_CALL_MAGIC, "not a host-call descriptor");
        require(call->fn != nullptr && call->dst_host != nullptr && dst != nullptr && dst_bytes > 0,
                "host call needs fn, dst_host and a device output");
        require(n_src >= 0 && n_src <= VBM_HOST_MAX_SRC && (n_src == 0 || (srcs && src_bytes)), "bad host-call inputs");
        for (int i = 0; i < n_src; ++i)
            require(srcs[i] != nullptr && call->src_host[i] != nullptr, "host-call input without a host buffer");
        require(mode == VBM_HOST_CALL_FUNC || mode == VBM_HOST_CALL_MAILBOX, "unknown host-call mode");
        require(miss == nullptr || (n_miss > 0 && mode == VBM_HOST_CALL_MAILBOX),
                "miss ids need the mailbox mode and a positive count");
        int device = 0;
        check_hip(hipGetDevice(&device), "hipGetDevice");
        require(device >= 0 && device < kMaxDevices, "device index out of range");
        CallState & st = state_of(call, device);
        const hipStream_t main = as_stream(stream), side = side_stream(device);
        check_hip(hipEventRecord(st.ready, main), "host-call fork");
        check_hip(hipStreamWaitEvent(side, st.ready, 0), "host-call fork");
        if (g_workers[device]) {   // a mailbox post of this call may still be queued or running
            hipLaunchKernelGGL(wait_handled_kernel, dim3(1), dim3(64), 0, side, g_workers[device]->box_dev, st.seq_dev,
                               device, g_spin_limit.load());
            check_hip(hipGetLastError(), "host-call handled-wait launch");
        }
        for (int i = 0; i < n_src; ++i)
            check_hip(hipMemcpyAsync(call->src_host[i], srcs[i], src_bytes[i], hipMemcpyDeviceToHost, side),
                      "host-call input copy");
        if (mode == VBM_HOST_CALL_FUNC) {
            check_hip(hipLaunchHostFunc(side, trampoline, call), "hipLaunchHostFunc");
            check_hip(hipMemcpyAsync(dst, call->dst_host, dst_bytes, hipMemcpyHostToDevice, side), "host-call output copy");
        } else {
            Worker * w = worker(device);
            PostArgs a{};
            a.miss = miss;
            a.n_miss = n_miss;
            a.call = reinterpret_cast<uint64_t>(call);
            a.box = w->box_dev;
            a.device = device;
            a.skipped = st.skipped;
            a.seq_out = st.seq_dev;
            a.spin_limit = g_spin_limit.load();
            hipLaunchKernelGGL(host_call_post_kernel, dim3(1), dim3(256), 0, side, a);
            check_hip(hipGetLastError(), "host-call post launch");
            check_hip(hipMemcpyAsync(dst, call->dst_host, dst_bytes, hipMemcpyHostToDevice, side), "host-call output copy");
            const int64_t n = static_cast<int64_t>(dst_bytes);
            hipLaunchKernelGGL(zero_if_skipped_kernel, dim3(static_cast<unsigned>(std::min<int64_t>(64, (n + 255) / 256))),
                               dim3(256), 0, side, static_cast<uint8_t *>(dst), n, st.skipped);
            check_hip(hipGetLastError(), "host-call zero launch");
        }
        check_hip(hipEventRecord(st.done, side), "host-call done");
    });
}

vbm_status vbm_host_join(vbm_host_call * call, const float * a, const float * b, float * dst, int64_t n, void * stream) {
    return guarded([&] {
        require(call != nullptr && call->magic == VBM_HOST_CALL_MAGIC && call->backend_state != nullptr,
                "join of a host call that was never enqueued");
        require(a && b && dst && n > 0, "bad join operands");
        auto * st = static_cast<CallState *>(call->backend_state);
        const hipStream_t s = as_stream(stream);
        check_hip(hipStreamWaitEvent(s, st->done, 0), "host-call join");
        hipLaunchKernelGGL(join_add_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, a, b, dst, n);
        check_hip(hipGetLastError(), "host-call join launch");
    });
}

vbm_status vbm_host_call_wait(vbm_host_call * call, void * stream) {
    return guarded([&] {
        require(call != nullptr && call->magic == VBM_HOST_CALL_MAGIC && call->backend_state != nullptr,
                "wait for a host call that was never enqueued");
        auto * st = static_cast<CallState *>(call->backend_state);
        check_hip(hipStreamWaitEvent(as_stream(stream), st->done, 0), "host-call wait");
    });
}

vbm_status vbm_host_call_release(vbm_host_call * call) {
    return guarded([&] {
        require(call != nullptr, "null host call");
        auto * st = static_cast<CallState *>(call->backend_state);
        if (!st) return;
        check_hip(hipEventSynchronize(st->done), "host-call release");
        // a post that was not waited for (or whose wait expired) may still be queued at the worker,
        // which holds the descriptor's address: wait for it, bounded, before anything is freed
        const uint64_t seq = __atomic_load_n(st->seq_host, __ATOMIC_ACQUIRE);
        Worker * w = g_workers[st->device];
        if (w && seq) {
            const auto start = std::chrono::steady_clock::now();
            const double limit_s = 1e-6 * static_cast<double>(g_spin_limit.load()) + 1.0;
            while (__atomic_load_n(&w->box->done, __ATOMIC_ACQUIRE) < seq) {
                if (std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count() > limit_s)
                    fail(VBM_ERR_RUNTIME, "host call release: its function is still queued or running at the worker");
                std::this_thread::sleep_for(std::chrono::microseconds(20));
            }
        }
        (void)hipEventDestroy(st->ready);
        (void)hipEventDestroy(st->done);
        (void)hipFree(st->skipped);
        (void)hipHostFree(st->seq_host);
        delete st;
        call->backend_state = nullptr;
    });
}

vbm_status vbm_host_mailbox_drain(int device, double timeout_s) {
    return guarded([&] {
        require(device >= 0 && device < kMaxDevices, "device index out of range");
        Worker * w = g_workers[device];
        if (!w) return;
        const uint64_t posted = __atomic_load_n(&w->box->posted, __ATOMIC_ACQUIRE);
        const auto start = std::chrono::steady_clock::now();
        while (__atomic_load_n(&w->box->done, __ATOMIC_ACQUIRE) < posted) {
            if (std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count() > timeout_s)
                fail(VBM_ERR_RUNTIME, "host-call mailbox did not drain in time");
            __builtin_ia32_pause();
        }
    });
}

vbm_status vbm_host_mailbox_stats(int device, uint64_t * posted, uint64_t * done, uint32_t * timeouts) {
    return guarded([&] {
        require(device >= 0 && device < kMaxDevices, "device index out of range");
        Worker * w = g_workers[device];
        if (posted) *posted = w ? __atomic_load_n(&w->box->posted, __ATOMIC_ACQUIRE) : 0;
        if (done) *done = w ? __atomic_load_n(&w->box->done, __ATOMIC_ACQUIRE) : 0;
        if (timeouts) {
            uint32_t t = 0;
            check_hip(hipMemcpyFromSymbol(&t, HIP_SYMBOL(g_timeouts), sizeof(t), sizeof(uint32_t) * device,
                                          hipMemcpyDeviceToHost), "host-call timeouts");
            *timeouts = t;
        }
    });
}

vbm_status vbm_host_mailbox_set_spin_limit(uint32_t polls) {
    return guarded([&] {
        require(polls >= 1, "spin limit must be positive");
        g_spin_limit.store(polls);
    });
}

}  // extern "C"
