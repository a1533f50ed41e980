// btl_probe.hip -- measurement kernels for the ceilings the bench compares with
// (bench.py --probe ceilings): a plain streaming read of a projection's packed
// bytes and an empty kernel (the decode chain's read and launch floors), and an
// MFMA loop (the int8 matrix-core throughput the prefill GEMM can reach).  They
// compute nothing of BitLinear; the library (libbitlinear_hip.so) does not
// contain them.
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

typedef int v4i __attribute__((ext_vector_type(4)));

// MFMA throughput: every wave runs `iters` rounds of 8 independent
// v_mfma_i32_16x16x64_i8 (8 accumulators, so the matrix pipe never waits for a
// result), its operands four A and four B registers loaded once from `src`
// (each lane its own 16 bytes: random int8 bytes for the random-data figure,
// one repeated byte for the constant one).  Writes the accumulators' sum per
// lane, so no MFMA is dead.
__global__ __launch_bounds__(256) void k_mfma_loop(const v4i* src, int iters, int* out)
{
    const int g = blockIdx.x * 256 + threadIdx.x;
    const v4i a0 = src[(8 * g) & 0xFFFF], a1 = src[(8 * g + 1) & 0xFFFF], a2 = src[(8 * g + 2) & 0xFFFF],
              a3 = src[(8 * g + 3) & 0xFFFF];
    const v4i b0 = src[(8 * g + 4) & 0xFFFF], b1 = src[(8 * g + 5) & 0xFFFF], b2 = src[(8 * g + 6) & 0xFFFF],
              b3 = src[(8 * g + 7) & 0xFFFF];
    v4i c0 = v4i{0, 0, 0, 0}, c1 = c0, c2 = c0, c3 = c0, c4 = c0, c5 = c0, c6 = c0, c7 = c0;
    // written as assembly so the accumulators stay in their VGPRs (the compiler's
    // allocation copied accumulator registers between the MFMAs of a round)
    for (int it = 0; it < iters; ++it) {
        asm volatile(
            "v_mfma_i32_16x16x64_i8 %0, %8, %12, %0\n\t"
            "v_mfma_i32_16x16x64_i8 %1, %9, %12, %1\n\t"
            "v_mfma_i32_16x16x64_i8 %2, %10, %13, %2\n\t"
            "v_mfma_i32_16x16x64_i8 %3, %11, %13, %3\n\t"
            "v_mfma_i32_16x16x64_i8 %4, %8, %14, %4\n\t"
            "v_mfma_i32_16x16x64_i8 %5, %9, %14, %5\n\t"
            "v_mfma_i32_16x16x64_i8 %6, %10, %15, %6\n\t"
            "v_mfma_i32_16x16x64_i8 %7, %11, %15, %7"
            : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3), "+v"(c4), "+v"(c5), "+v"(c6), "+v"(c7)
            : "v"(a0), "v"(a1), "v"(a2), "v"(a3), "v"(b0), "v"(b1), "v"(b2), "v"(b3));
    }
    const v4i t = ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7));
    out[g] = t.x + t.y + t.z + t.w;
}

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

// `wgs` workgroups of 256 threads, each wave 8 x iters MFMAs of 16x16x64 int8
// (2 * 16 * 16 * 64 ops each); src: 65536 int4 (1 MiB), out: wgs * 256 ints.
int probe_mfma_loop(const void* src, int iters, int wgs, int* out, void* stream)
{
    if (wgs < 1 || iters < 1) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_mfma_loop, dim3((unsigned)wgs), dim3(256), 0, (hipStream_t)stream, (const v4i*)src, iters, out);
    return (int)hipGetLastError();
}

// An empty kernel of `wgs` workgroups of 64 threads.
int probe_empty(int wgs, void* stream)
{
    if (wgs < 1) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_empty, dim3((unsigned)wgs), dim3(64), 0, (hipStream_t)stream);
    return (int)hipGetLastError();
}

}  // extern "C"
