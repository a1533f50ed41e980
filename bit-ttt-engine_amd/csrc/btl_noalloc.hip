// btl_noalloc.hip -- the fixed scratch array behind btl_linear_noalloc.
//
// A caller that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc) gets the same
// contraction as btl_linear with its scratch (quantised activations, split-K
// partial sums) in this file-scope array instead of a workspace.  Each device
// that loads the library holds its own copy until the process ends.  In host
// code `scratch` names a host-side stand-in, never device memory: the device
// address is taken once per device with hipGetSymbolAddress and only that
// pointer is handed to kernels.
#include <hip/hip_runtime.h>

#include <mutex>

#include "btl_internal.hpp"

namespace btl {

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];
}  // namespace

// The device address of `scratch` on `dev`, looked up once per device with
// `dev` current (the caller's current device is restored).
hipError_t scratch_address(int dev, void** out)
{
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e != hipSuccess) return e;
        if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) {
            const hipError_t e2 = hipSetDevice(cur);
            if (e == hipSuccess) e = e2;
        }
        if (e != hipSuccess) return e;
        if (!p || ((uintptr_t)p & 255u)) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

}  // namespace btl
