// btl_probe.hip -- measurement kernels for the ceilings of the decode chain
// (bench.py --probe ceilings): a plain streaming read of a projection's packed
// bytes, and an empty kernel for the cost of a dependent launch.  They compute
// nothing of BitLinear; the library (libbitlinear_hip.so) does not contain them.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kThreads = 256;
constexpr int kLoads = 8;  // 16-byte loads per thread, all issued before the first use

// Streaming read of n16 16-byte words from p: thread t of workgroup b reads
// words b * 2048 + u * 256 + t, u < 8 (one 32 KiB span per workgroup, every load
// in flight at once, non-temporal as the weight loads of the decode kernels)
// and folds them with XOR.  The fold decides a store that never happens for the
// buffers bench.py reads (a word of the span equal to kNever), so every load is
// live and the workgroup ends as soon as its loads have landed.  (Swept on
// MI355X over 64..1024 threads and 4..16 loads per thread: within 0.1 us of
// the best form at 14.7 and 29.4 MB.)
constexpr uint32_t kNever = 0x9E3779B9u;
__global__ __launch_bounds__(kThreads) void k_stream_read(const uint4* p, int64_t n16, uint32_t* out)
{
    const int64_t base = (int64_t)blockIdx.x * kLoads * kThreads;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint4*>(p + base), (short)0, (int)(min<int64_t>(n16 - base, kLoads * kThreads) * 16), 0x00020000);
    uint4 v[kLoads];
#pragma unroll
    for (int u = 0; u < kLoads; ++u)
        v[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (u * kThreads + threadIdx.x) * 16,
                                                                              0, 2));
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < kLoads; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (acc == kNever) out[blockIdx.x] = acc;
}

__global__ __launch_bounds__(64) void k_empty() {}

}  // namespace

extern "C" {

// One streaming read of `bytes` (a multiple of 16) at p (16-byte aligned); out
// has room for probe_stream_read_words(bytes) words (one per 32 KiB span, written
// only when a span folds to kNever).  0 or the HIP error.
int probe_stream_read(const void* p, int64_t bytes, uint32_t* out, void* stream)
{
    const int64_t n16 = bytes / 16;
    const int64_t wgs = (n16 + kLoads * kThreads - 1) / (kLoads * kThreads);
    if (bytes <= 0 || bytes % 16 || wgs > (1 << 30)) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_stream_read, dim3((unsigned)wgs), dim3(kThreads), 0, (hipStream_t)stream, (const uint4*)p,
                       n16, out);
    return (int)hipGetLastError();
}

int64_t probe_stream_read_words(int64_t bytes) { return (bytes / 16 + kLoads * kThreads - 1) / (kLoads * kThreads); }

// An empty kernel of `wgs` workgroups of 64 threads.
int probe_empty(int wgs, void* stream)
{
    if (wgs < 1) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_empty, dim3((unsigned)wgs), dim3(64), 0, (hipStream_t)stream);
    return (int)hipGetLastError();
}

}  // extern "C"
