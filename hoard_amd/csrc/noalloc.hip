// The fixed scratch of the batched stage's allocation-free entry point
// (hoard_moe_forward_batched_noalloc): one file-scope device array per GPU,
// held until the process ends, so that a call allocates nothing.
//
// In host code the array's name is a host-side stand-in, not a device address:
// each device's copy is looked up once with hipGetSymbolAddress, with that
// device current, and only the looked-up address is used afterwards (as kernel
// arguments).  Calls that overlap on one GPU share its array and race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "kernels.h"

namespace hoard {

constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

static_assert(kNoAllocCounterBytes % 256 == 0 && kNoAllocCounterBytes >= sizeof(unsigned) * kBatchedCounters,
              "the counters lead the array");

constexpr int kMaxDevices = 64;
std::mutex g_mu;
uint8_t *g_ptr[kMaxDevices] = {};

__global__ void zero_words_kernel(unsigned *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

}  // namespace

size_t noalloc_scratch_bytes() { return kScratchBytes; }

// Looks up the current device's copy of the array once per device and zeroes
// the route counters at its head (the kernels leave them zero after every
// launch).  Called by hoard_moe_create with the handle's device current.
hipError_t noalloc_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_ptr[device]) return hipSuccess;
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    const int n = (int)(kNoAllocCounterBytes / sizeof(unsigned));
    hipLaunchKernelGGL(zero_words_kernel, dim3((n + 255) / 256), dim3(256), 0, nullptr, static_cast<unsigned *>(p), n);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) return e;
    g_ptr[device] = static_cast<uint8_t *>(p);
    return hipSuccess;
}

uint8_t *noalloc_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_mu);
    return g_ptr[device];
}

}  // namespace hoard
