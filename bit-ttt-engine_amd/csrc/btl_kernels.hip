// btl_kernels.hip -- gfx950 (CDNA4) kernels of the BitLinear engine.
//
// Reference path (imonoonoko/Bit-TTT-Engine, crates/rust_engine):
//   packed layout / codes ........ src/kernels/packing.rs:6-21, 74-92
//   fp32 contraction order ....... src/kernels/cpu.rs:77-123, 172-238
//   absmax convention ............ src/layers/kv_cache.rs:95-119
//
// Kernels:
//   k_gemv<XK,YK>     decode / small-M contraction on the int8 MFMA
//                     (v_mfma_i32_16x16x64_i8), weights unpacked in registers,
//                     activations quantised (or copied) into LDS, split-K with
//                     exact int32 atomics and a self-cleaning last-block epilogue.
//   k_quant_act<XK>   per-token absmax int8 quantisation, natural layout.
//   k_ref_f32<XK,YK>  reference-semantics fp32 path: bit-identical to the
//                     8-lane FMA order of cpu.rs.
//   k_generic_i8<YK>  any k % 4 == 0 / any alignment, int8 activations.
//   k_unpack          dense f32 weights (PackedTensor::unpack on the device).
//   k_fill_zero       workspace clearing (a kernel, so it is graph-capture safe).
//
// Compiled with -ffp-contract=off: every fp32 operation below is rounded as
// written (the oracle restates the same operations in C).
#include <hip/hip_runtime.h>

#include "btl_internal.hpp"

namespace btl {

typedef int v4i __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// scalar helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Round-to-nearest-even f32 -> bf16; NaN becomes 0x7FC0.
__device__ __forceinline__ uint16_t f32_to_bf16(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

template <int YK>
__device__ __forceinline__ void store_y(void* y, int64_t idx, float v)
{
    if (YK == YK_F32) ((float*)y)[idx] = v;
    else ((uint16_t*)y)[idx] = f32_to_bf16(v);
}

// Quantisation parameters of one token row from max(|x|) as an IEEE bit
// pattern (sign cleared; NaN patterns compare above +inf).
//   non-finite row -> s = NaN, q = 0;  a < 2^-100 -> s = 0, q = 0;
//   else r = 127/a, s = a/127 (both correctly rounded divisions).
struct QParams {
    float r;
    float s;
    int ok;
};

__device__ __forceinline__ QParams qparams(uint32_t amax)
{
    QParams q;
    if (amax >= 0x7F800000u) {
        q.r = 0.0f; q.s = __uint_as_float(0x7FC00000u); q.ok = 0;
    } else if (amax < 0x0D800000u) {
        q.r = 0.0f; q.s = 0.0f; q.ok = 0;
    } else {
        float a = __uint_as_float(amax);
        q.r = __fdiv_rn(127.0f, a);
        q.s = __fdiv_rn(a, 127.0f);
        q.ok = 1;
    }
    return q;
}

// round_half_away(x * r) clamped to [-127, 127].  trunc(y + copysign(0.5 - 2^-25, y))
// equals roundf(y) for |y| < 2^23 (y + 0.49999997 never rounds up to the next
// integer unless y's fraction is >= 0.5); |y| <= 127.00002 here.
__device__ __forceinline__ int quant1(float x, float r, int ok)
{
    float y = __fmul_rn(x, r);
    float t = __fadd_rn(y, __builtin_copysignf(0.49999997f, y));
    int v = (int)t;
    v = v > 127 ? 127 : (v < -127 ? -127 : v);
    return ok ? v : 0;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        uint32_t o = (uint32_t)__shfl_xor((int)v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}

__device__ __forceinline__ int wave_sum_i32(int v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// ---------------------------------------------------------------------------
// 2-bit -> int8 unpack for the MFMA operand
// ---------------------------------------------------------------------------
// One 32-bit word holds 16 weights, weight i at bits 2i..2i+1 (packing.rs:89).
// Masks pick one code per byte: c_s = code of weight 4b+s in byte b.  The code
// becomes a v_perm_b32 selector into a constant byte table:
//   s = 0, 2: selector c in {0,1,2,3} -> table bytes {00, 01, FF, 00}
//   s = 1, 3: selector 4c in {0,4,8,12} -> byte0 = 00, byte4 = 01,
//             8 = sign of byte1 (0x80 -> FF), 12 = constant 00
// Result register s, byte b = t(weight 4b+s) in {-1,0,+1}: the 16 int8 of the
// operand are in k order [0,4,8,12, 1,5,9,13, 2,6,10,14, 3,7,11,15], and the
// activation operand is stored in the same order.
__device__ __forceinline__ v4i unpack16(uint32_t w)
{
    const uint32_t c0 = w & 0x03030303u;
    const uint32_t c1 = w & 0x0C0C0C0Cu;
    const uint32_t w4 = w >> 4;
    const uint32_t c2 = w4 & 0x03030303u;
    const uint32_t c3 = w4 & 0x0C0C0C0Cu;
    v4i r;
    r.x = (int)__builtin_amdgcn_perm(0u, 0x00FF0100u, c0);
    r.y = (int)__builtin_amdgcn_perm(0x00000001u, 0x00008000u, c1);
    r.z = (int)__builtin_amdgcn_perm(0u, 0x00FF0100u, c2);
    r.w = (int)__builtin_amdgcn_perm(0x00000001u, 0x00008000u, c3);
    return r;
}

// 16 int8 values q[0..15] (natural k order) -> the transposed operand order.
__device__ __forceinline__ uint4 pack_transposed(const int* q)
{
    uint4 o;
    uint32_t* ow = (uint32_t*)&o;
#pragma unroll
    for (int v = 0; v < 4; ++v)
        ow[v] = ((uint32_t)(q[v] & 0xFF)) | ((uint32_t)(q[4 + v] & 0xFF) << 8) |
                ((uint32_t)(q[8 + v] & 0xFF) << 16) | ((uint32_t)(q[12 + v] & 0xFF) << 24);
    return o;
}

// 16 int8 bytes in natural order (4 words, word b = k 4b..4b+3) -> transposed.
__device__ __forceinline__ uint4 transpose16(uint4 a)
{
    // out word v byte b = in word b byte v
    uint32_t lo01 = __builtin_amdgcn_perm(a.y, a.x, 0x05010400u); // x0 y0 x1 y1
    uint32_t lo23 = __builtin_amdgcn_perm(a.w, a.z, 0x05010400u); // z0 w0 z1 w1
    uint32_t hi01 = __builtin_amdgcn_perm(a.y, a.x, 0x07030602u); // x2 y2 x3 y3
    uint32_t hi23 = __builtin_amdgcn_perm(a.w, a.z, 0x07030602u); // z2 w2 z3 w3
    uint4 o;
    o.x = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u); // x0 y0 z0 w0
    o.y = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u); // x1 y1 z1 w1
    o.z = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u); // x2 y2 z2 w2
    o.w = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u); // x3 y3 z3 w3
    return o;
}

// ---------------------------------------------------------------------------
// k_gemv: small-M ternary contraction on the int8 MFMA
// ---------------------------------------------------------------------------
// Grid: x = rb_total * splits (row-block major, slice minor), y = M tiles of 16.
// Workgroup: 4 waves; wave w owns rows [64*rb + 16*w, +16) of its layer and the
// K slice [slice*s, +slice).  Per wave-load, lane (r = lane&15, kq = lane>>4)
// reads 16 bytes (64 weights) of row r at byte 64*j + 16*kq of the slice, i.e.
// each row contributes 64 contiguous bytes and a wave-load covers 16 x 256
// weights.  Each 4-byte word becomes one A operand (16 rows x 64 k) of
// v_mfma_i32_16x16x64_i8; the B operand is 16 token rows x 64 k from LDS.
// D lane l, element v = row 4*(l>>4)+v, token l&15.
constexpr int kPF = 4;  // wave-loads kept in flight per lane

template <int XK>
__device__ __forceinline__ void gemv_prologue(const GemvArgs& a, uint8_t* sq, int lp, int m0,
                                              int mt, int k0, int len, float* s_sx,
                                              uint32_t (*s_amax)[kGemvMaxM], float* s_r,
                                              int* s_ok)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = a.k;
    const int groups = len >> 4;  // len % 64 == 0
    if (XK == XK_I8) {
        const int8_t* xq = (const int8_t*)a.x;
        if (tid < mt) s_sx[tid] = a.xs[m0 + tid];
        for (int g = tid; g < mt * groups; g += 256) {
            const int m = g / groups, gi = g - m * groups;
            uint4 v = *(const uint4*)(xq + (int64_t)(m0 + m) * K + k0 + gi * 16);
            *(uint4*)(sq + m * lp + gi * 16) = transpose16(v);
        }
        return;
    }
    // 1. absmax of each token row over the full K
    for (int m = 0; m < mt; ++m) {
        uint32_t amax = 0;
        if (XK == XK_BF16) {
            const uint4* xr = (const uint4*)((const uint16_t*)a.x + (int64_t)(m0 + m) * K);
            for (int i = tid; i < (K >> 3); i += 256) {
                uint4 v = xr[i];
                const uint32_t* u = (const uint32_t*)&v;
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    uint32_t lo = (u[h] << 16) & 0x7FFF0000u, hi = u[h] & 0x7FFF0000u;
                    amax = lo > amax ? lo : amax;
                    amax = hi > amax ? hi : amax;
                }
            }
        } else {
            const uint4* xr = (const uint4*)((const float*)a.x + (int64_t)(m0 + m) * K);
            for (int i = tid; i < (K >> 2); i += 256) {
                uint4 v = xr[i];
                const uint32_t* u = (const uint32_t*)&v;
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    uint32_t b = u[h] & 0x7FFFFFFFu;
                    amax = b > amax ? b : amax;
                }
            }
        }
        amax = wave_max_u32(amax);
        if (lane == 0) s_amax[wave][m] = amax;
    }
    __syncthreads();
    if (tid < mt) {
        uint32_t am = s_amax[0][tid];
#pragma unroll
        for (int w = 1; w < 4; ++w) am = s_amax[w][tid] > am ? s_amax[w][tid] : am;
        QParams qp = qparams(am);
        s_r[tid] = qp.r;
        s_sx[tid] = qp.s;
        s_ok[tid] = qp.ok;
    }
    __syncthreads();
    // 2. quantise this K slice into LDS in operand order
    for (int g = tid; g < mt * groups; g += 256) {
        const int m = g / groups, gi = g - m * groups;
        const float r = s_r[m];
        const int ok = s_ok[m];
        int q[16];
        if (XK == XK_BF16) {
            const uint4* src =
                (const uint4*)((const uint16_t*)a.x + (int64_t)(m0 + m) * K + k0 + gi * 16);
            uint4 v0 = src[0], v1 = src[1];
            const uint32_t* u0 = (const uint32_t*)&v0;
            const uint32_t* u1 = (const uint32_t*)&v1;
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                q[2 * h] = quant1(bf16_to_f32(u0[h] & 0xFFFFu), r, ok);
                q[2 * h + 1] = quant1(bf16_to_f32(u0[h] >> 16), r, ok);
                q[8 + 2 * h] = quant1(bf16_to_f32(u1[h] & 0xFFFFu), r, ok);
                q[8 + 2 * h + 1] = quant1(bf16_to_f32(u1[h] >> 16), r, ok);
            }
        } else {
            const float4* src =
                (const float4*)((const float*)a.x + (int64_t)(m0 + m) * K + k0 + gi * 16);
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                float4 v = src[h];
                q[4 * h] = quant1(v.x, r, ok);
                q[4 * h + 1] = quant1(v.y, r, ok);
                q[4 * h + 2] = quant1(v.z, r, ok);
                q[4 * h + 3] = quant1(v.w, r, ok);
            }
        }
        *(uint4*)(sq + m * lp + gi * 16) = pack_transposed(q);
    }
}

template <int XK, int YK>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a)
{
    extern __shared__ __align__(16) uint8_t sq[];  // [mt][lp] int8 activation tile
    __shared__ uint32_t s_amax[4][kGemvMaxM];
    __shared__ float s_r[kGemvMaxM], s_sx[kGemvMaxM];
    __shared__ int s_ok[kGemvMaxM];
    __shared__ int s_last;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int S = a.splits;
    const int rbg = blockIdx.x / S;
    const int sidx = blockIdx.x - rbg * S;
    const int mtile = blockIdx.y;
    const int m0 = mtile * kGemvMaxM;
    const int mt = min(kGemvMaxM, a.m - m0);

    // layer of this row-block (uniform; explicit selects keep the kernel
    // arguments in scalar registers)
    const uint8_t* W = a.p[0].w;
    void* Y = a.p[0].y;
    int32_t* ACC = a.p[0].acc_out;
    int32_t* PART = a.p[0].partial;
    float SW = a.p[0].sw;
    int N = a.p[0].n;
    int RB0 = a.p[0].rb_begin;
#pragma unroll
    for (int i = 1; i < kMaxGroup; ++i) {
        if (i < a.nprob && rbg >= a.p[i].rb_begin) {
            W = a.p[i].w; Y = a.p[i].y; ACC = a.p[i].acc_out; PART = a.p[i].partial;
            SW = a.p[i].sw; N = a.p[i].n; RB0 = a.p[i].rb_begin;
        }
    }
    const int rb = rbg - RB0;
    const int K = a.k;
    const int k0 = sidx * a.slice;
    const int len = min(a.slice, K - k0);
    const int steps = (len + kStepWeights - 1) / kStepWeights;
    const int lp = a.slice + 16;

    // 1. put the first weight loads in flight before the activation prologue
    const int r = lane & 15, kq = lane >> 4;
    const int nrow = rb * kGemvRows + wave * 16 + r;
    const bool row_ok = nrow < N;
    const uint8_t* wp = W + (int64_t)(row_ok ? nrow : 0) * (K >> 2) + (k0 >> 2) + kq * 16;
    auto ld = [&](int j) -> uint4 {
        uint4 v = {0u, 0u, 0u, 0u};
        if (row_ok && j * kStepWeights + kq * 64 < len) v = *(const uint4*)(wp + j * 64);
        return v;
    };
    uint4 buf[kPF];
#pragma unroll
    for (int i = 0; i < kPF; ++i) buf[i] = ld(i);

    // 2. activation tile
    gemv_prologue<XK>(a, sq, lp, m0, mt, k0, len, s_sx, s_amax, s_r, s_ok);
    __syncthreads();

    // 3. main loop
    const int mcol = lane & 15;
    const bool m_ok = mcol < mt;
    const uint8_t* bq = sq + mcol * lp + kq * 64;
    v4i acc0 = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};
    const v4i zero = {0, 0, 0, 0};
    for (int j0 = 0; j0 < steps; j0 += kPF) {
#pragma unroll
        for (int i = 0; i < kPF; ++i) {
            const int j = j0 + i;
            if (j < steps) {
                const uint4 cur = buf[i];
                buf[i] = ld(j + kPF);
                const uint8_t* bj = bq + j * kStepWeights;
                v4i b0 = m_ok ? *(const v4i*)(bj + 0) : zero;
                v4i b1 = m_ok ? *(const v4i*)(bj + 16) : zero;
                v4i b2 = m_ok ? *(const v4i*)(bj + 32) : zero;
                v4i b3 = m_ok ? *(const v4i*)(bj + 48) : zero;
                acc0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack16(cur.x), b0, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack16(cur.y), b1, acc1, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack16(cur.z), b2, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack16(cur.w), b3, acc1, 0, 0, 0);
            }
        }
    }
    const v4i acc = acc0 + acc1;

    // 4. epilogue
    const int gm = m0 + mcol;
    const int nb = rb * kGemvRows + wave * 16 + 4 * (lane >> 4);
    if (S == 1) {
        if (m_ok) {
            const float c = __fmul_rn(s_sx[mcol], SW);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int n = nb + v;
                if (n < N) {
                    const int64_t o = (int64_t)gm * N + n;
                    store_y<YK>(Y, o, __fmul_rn((float)acc[v], c));
                    if (ACC) ACC[o] = acc[v];
                }
            }
        }
        return;
    }
    if (m_ok) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int n = nb + v;
            if (n < N) atomicAdd(&PART[(int64_t)gm * N + n], acc[v]);
        }
    }
    __threadfence();
    __syncthreads();
    uint32_t* cnt = a.counter + (int64_t)mtile * a.rb_total + rbg;
    if (tid == 0) s_last = (atomicAdd(cnt, 1u) == (uint32_t)(S - 1));
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    if (m_ok) {
        const float c = __fmul_rn(s_sx[mcol], SW);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int n = nb + v;
            if (n < N) {
                const int64_t o = (int64_t)gm * N + n;
                const int tot = atomicExch(&PART[o], 0);
                store_y<YK>(Y, o, __fmul_rn((float)tot, c));
                if (ACC) ACC[o] = tot;
            }
        }
    }
    if (tid == 0) atomicExch(cnt, 0u);
}

hipError_t launch_gemv(const GemvArgs& a, int xkind, int ykind, int mtiles, hipStream_t s)
{
    dim3 grid((unsigned)(a.rb_total * a.splits), (unsigned)mtiles);
    const int mt = a.m < kGemvMaxM ? a.m : kGemvMaxM;
    const size_t lds = (size_t)mt * (size_t)(a.slice + 16);
#define BTL_GEMV_CASE(XKV, YKV)                                              \
    if (xkind == XKV && ykind == YKV) {                                      \
        hipLaunchKernelGGL((k_gemv<XKV, YKV>), grid, dim3(256), lds, s, a);  \
        return hipGetLastError();                                            \
    }
    BTL_GEMV_CASE(XK_F32, YK_F32)
    BTL_GEMV_CASE(XK_F32, YK_BF16)
    BTL_GEMV_CASE(XK_BF16, YK_F32)
    BTL_GEMV_CASE(XK_BF16, YK_BF16)
    BTL_GEMV_CASE(XK_I8, YK_F32)
    BTL_GEMV_CASE(XK_I8, YK_BF16)
#undef BTL_GEMV_CASE
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// k_quant_act: one workgroup per token row, natural layout
// ---------------------------------------------------------------------------
template <int XK>
__device__ __forceinline__ float load_x(const void* x, int64_t i)
{
    if (XK == XK_BF16) return bf16_to_f32(((const uint16_t*)x)[i]);
    return ((const float*)x)[i];
}

template <int XK>
__global__ __launch_bounds__(256) void k_quant_act(const void* x, int64_t k, int8_t* q, float* s)
{
    __shared__ uint32_t s_w[4];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t base = row * k;
    uint32_t amax = 0;
    for (int64_t i = tid; i < k; i += 256) {
        uint32_t b = __float_as_uint(load_x<XK>(x, base + i)) & 0x7FFFFFFFu;
        amax = b > amax ? b : amax;
    }
    amax = wave_max_u32(amax);
    if ((tid & 63) == 0) s_w[tid >> 6] = amax;
    __syncthreads();
    amax = s_w[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) amax = s_w[w] > amax ? s_w[w] : amax;
    const QParams qp = qparams(amax);
    if (tid == 0) s[row] = qp.s;
    for (int64_t i = tid; i < k; i += 256) q[base + i] = (int8_t)quant1(load_x<XK>(x, base + i), qp.r, qp.ok);
}

hipError_t launch_quant_act(const void* x, int xkind, int64_t m, int64_t k, int8_t* q, float* s,
                            hipStream_t st)
{
    if (m <= 0) return hipSuccess;
    if (xkind == XK_BF16) hipLaunchKernelGGL(k_quant_act<XK_BF16>, dim3((unsigned)m), dim3(256), 0, st, x, k, q, s);
    else hipLaunchKernelGGL(k_quant_act<XK_F32>, dim3((unsigned)m), dim3(256), 0, st, x, k, q, s);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// k_ref_f32: reference-semantics fp32 contraction (cpu.rs:77-123)
// ---------------------------------------------------------------------------
// Eight lanes per output.  Lane b accumulates, in increasing k, every input
// k = 32c + 8g + b of the first 32*floor(K/32) inputs with fma(x, coeff, acc)
// -- exactly the b-th float lane of the reference's _mm256_fmadd_ps
// accumulator (cpu.rs:192-221).  Lane 0 then sums the eight lanes in order
// (cpu.rs:236-238), adds the scalar tail in order (cpu.rs:105-122) and scales
// (cpu.rs:123).
template <int XK, int YK>
__global__ __launch_bounds__(256) void k_ref_f32(const void* x, int64_t m, int64_t k,
                                                 const uint8_t* w, int64_t n, float scale, void* y)
{
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t out = gid >> 3;
    const int b = (int)(gid & 7);
    const bool active = out < m * n;
    const int64_t row = active ? out / n : 0;
    const int64_t col = active ? out - row * n : 0;
    const int64_t stride = k >> 2;  // k % 4 == 0
    const uint8_t* wr = w + col * stride;
    const int64_t xb = row * k;
    const int64_t nchunks = k >> 5;
    float acc = 0.0f;
    if (active) {
        for (int64_t c = 0; c < nchunks; ++c) {
            const uint8_t* p = wr + c * 8;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t wv = (uint32_t)p[2 * g] | ((uint32_t)p[2 * g + 1] << 8);
                const int code = (wv >> (2 * b)) & 3;
                const float coeff = (float)((code & 1) - (code >> 1));
                acc = __builtin_fmaf(load_x<XK>(x, xb + c * 32 + g * 8 + b), coeff, acc);
            }
        }
    }
    // lanes of one output are 8 consecutive lanes of the wave
    float lanes[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) lanes[i] = __shfl(acc, i, 8);
    if (!active || b != 0) return;
    float r = -0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) r = __fadd_rn(r, lanes[i]);
    float sum = __fadd_rn(0.0f, r);
    for (int64_t l = nchunks * 32; l < k; ++l) {
        const int code = (wr[l >> 2] >> ((l & 3) * 2)) & 3;
        const float coeff = code == 1 ? 1.0f : (code == 2 ? -1.0f : 0.0f);
        sum = __fadd_rn(sum, __fmul_rn(load_x<XK>(x, xb + l), coeff));
    }
    store_y<YK>(y, out, __fmul_rn(sum, scale));
}

hipError_t launch_ref_f32(const void* x, int xkind, int64_t m, int64_t k, const uint8_t* w,
                          int64_t n, float scale, void* y, int ykind, hipStream_t st)
{
    const int64_t threads = m * n * 8;
    if (threads <= 0) return hipSuccess;
    dim3 grid((unsigned)((threads + 255) / 256));
#define BTL_REF_CASE(XKV, YKV)                                                                  \
    if (xkind == XKV && ykind == YKV) {                                                         \
        hipLaunchKernelGGL((k_ref_f32<XKV, YKV>), grid, dim3(256), 0, st, x, m, k, w, n, scale, y); \
        return hipGetLastError();                                                               \
    }
    BTL_REF_CASE(XK_F32, YK_F32)
    BTL_REF_CASE(XK_F32, YK_BF16)
    BTL_REF_CASE(XK_BF16, YK_F32)
    BTL_REF_CASE(XK_BF16, YK_BF16)
#undef BTL_REF_CASE
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// k_generic_i8: one wave per output, any k % 4 == 0, any alignment
// ---------------------------------------------------------------------------
template <int YK>
__global__ __launch_bounds__(256) void k_generic_i8(const int8_t* q, const float* xs, int64_t m,
                                                    int64_t k, const uint8_t* w, int64_t n,
                                                    float sw, void* y, int32_t* acc_out)
{
    const int64_t out = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (out >= m * n) return;  // uniform per wave
    const int64_t row = out / n, col = out - row * n;
    const uint8_t* wr = w + col * (k >> 2);
    const int8_t* qr = q + row * k;
    int acc = 0;
    for (int64_t byte = lane; byte < (k >> 2); byte += 64) {
        const uint32_t bv = wr[byte];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int code = (bv >> (2 * i)) & 3;
            acc += (int)qr[4 * byte + i] * ((code & 1) - (code >> 1));
        }
    }
    acc = wave_sum_i32(acc);
    if (lane == 0) {
        store_y<YK>(y, out, __fmul_rn((float)acc, __fmul_rn(xs[row], sw)));
        if (acc_out) acc_out[out] = acc;
    }
}

hipError_t launch_generic_i8(const int8_t* q, const float* xs, int64_t m, int64_t k,
                             const uint8_t* w, int64_t n, float sw, void* y, int ykind,
                             int32_t* acc_out, hipStream_t st)
{
    const int64_t outs = m * n;
    if (outs <= 0) return hipSuccess;
    dim3 grid((unsigned)((outs + 3) / 4));
    if (ykind == YK_BF16)
        hipLaunchKernelGGL(k_generic_i8<YK_BF16>, grid, dim3(256), 0, st, q, xs, m, k, w, n, sw, y, acc_out);
    else
        hipLaunchKernelGGL(k_generic_i8<YK_F32>, grid, dim3(256), 0, st, q, xs, m, k, w, n, sw, y, acc_out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// k_unpack: PackedTensor::unpack on the device (packing.rs:113-132)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_unpack(const uint8_t* w, int64_t numel, float scale,
                                                float* out)
{
    const int64_t byte = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (byte * 4 >= numel) return;
    const uint32_t bv = w[byte];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t e = byte * 4 + i;
        if (e < numel) {
            const int code = (bv >> (2 * i)) & 3;
            const float v = code == 1 ? 1.0f : (code == 2 ? -1.0f : 0.0f);
            out[e] = __fmul_rn(v, scale);
        }
    }
}

hipError_t launch_unpack(const uint8_t* w, int64_t numel, float scale, float* out, hipStream_t st)
{
    const int64_t bytes = (numel + 3) / 4;
    if (bytes <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_unpack, dim3((unsigned)((bytes + 255) / 256)), dim3(256), 0, st, w, numel, scale, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// k_fill_zero
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_fill_zero(uint8_t* p, size_t bytes)
{
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 16;
    if (i + 16 <= bytes) {
        *(uint4*)(p + i) = uint4{0u, 0u, 0u, 0u};
    } else {
        for (size_t j = i; j < bytes; ++j) p[j] = 0;
    }
}

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t st)
{
    if (bytes == 0) return hipSuccess;
    const size_t chunks = (bytes + 15) / 16;
    hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, st, (uint8_t*)p, bytes);
    return hipGetLastError();
}

}  // namespace btl
