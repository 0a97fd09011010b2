// Device-side status of the kernels' bounded waits.
//
// Kernels whose waves hand data to each other through LDS wait for each
// hand-over with a bounded number of polls, so every wave exits.  A wait
// that runs out of polls must not pass silently: the kernel poisons every
// output of its (batch, head) with NaN and adds one to this device's failure
// counter, which rwkv7m_device_status() (include/rwkv7m_wkv.h) reports and
// clears.  The counter is a file-scope device variable; its address on each
// device is looked up once per device, with that device current.

#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "wkv7_launch.h"

namespace rwkv7m {
namespace {

__device__ unsigned int g_wait_failures;
// the count taken by the last status call (read back by the host)
__device__ unsigned int g_wait_taken;

constexpr int kMaxDevices = 64;
std::mutex g_mu;
unsigned int* g_counter[kMaxDevices];
unsigned int* g_taken[kMaxDevices];
std::atomic<int64_t> g_limit{0};

// Takes the count and clears it in one atomic exchange, so that a failure a
// kernel on another stream adds meanwhile is kept for the next call.
__global__ void take_failures_kernel(unsigned int* counter,
                                     unsigned int* out) {
    *out = __hip_atomic_exchange(counter, 0u, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

hipError_t wait_config(WaitCfg* out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        if (g_counter[dev] == nullptr) {
            void* p = nullptr;
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_wait_failures));
            if (e != hipSuccess) return e;
            void* t = nullptr;
            e = hipGetSymbolAddress(&t, HIP_SYMBOL(g_wait_taken));
            if (e != hipSuccess) return e;
            g_taken[dev] = static_cast<unsigned int*>(t);
            g_counter[dev] = static_cast<unsigned int*>(p);
        }
        out->failures = g_counter[dev];
    }
    const int64_t lim = g_limit.load(std::memory_order_relaxed);
    out->limit = lim > 0 ? int(lim < (int64_t(1) << 30) ? lim : (1 << 30))
                         : kDefaultWaitPolls;
    return hipSuccess;
}

void set_wait_limit(int64_t polls) {
    g_limit.store(polls > 0 ? polls : 0, std::memory_order_relaxed);
}

hipError_t take_wait_failures(hipStream_t stream, unsigned int* count) {
    WaitCfg cfg;
    hipError_t e = wait_config(&cfg);
    if (e != hipSuccess) return e;
    int dev = 0;
    e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    unsigned int* taken = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        taken = g_taken[dev];
    }
    // after the stream's earlier work: exchange the count for zero, then
    // read what was taken
    hipLaunchKernelGGL(take_failures_kernel, dim3(1), dim3(1), 0, stream,
                       cfg.failures, taken);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return e;
    unsigned int n = 0;
    e = hipMemcpy(&n, taken, sizeof(n), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return e;
    *count = n;
    return hipSuccess;
}

}  // namespace rwkv7m
