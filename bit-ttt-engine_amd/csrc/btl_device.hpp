// btl_device.hpp -- device helpers shared by the gfx950 kernel sources
// (btl_kernels.hip, btl_model.hip).  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "btl_internal.hpp"

namespace btl {

// Raw buffer loads: a per-workgroup resource descriptor bounds every access,
// and an out-of-range offset reads zeros without a branch, so the compiler can
// count the loads in flight exactly (s_waitcnt vmcnt(N) per step).
constexpr int kOOB = 0x7FFFFFF0;  // offset outside every descriptor range
// cache policy of a load read once (weights): the non-temporal bit (nt) of
// the gfx950 buffer instructions
constexpr int kCachePolicyNT = 2;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint4 bload(__amdgpu_buffer_rsrc_t r, int off)
{
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Max of a u32 over the wave, via DPP (quad perms, row rotations, row
// broadcasts); the result is read from lane 63.  The DPP source reads 0 (the
// identity of the max) where a lane is masked, which lets the compiler fold
// each step into one v_max_u32_dpp.
__device__ __forceinline__ uint32_t wave_max_dpp(uint32_t v)
{
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, true));   // quad [1,0,3,2]
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, true));   // quad [2,3,0,1]
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xF, 0xF, true));  // row_ror:4
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, true));  // row_ror:8
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, true));  // row_bcast:15
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, true));  // row_bcast:31
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// exp(x) in f32: Cody-Waite reduction x = n ln2 + r (ln2 = hi + lo, hi with 15
// significant bits so n*hi is exact), e^r by its Taylor polynomial to r^7/7!
// in Horner form, scaled by 2^n through exponent bits (two exact steps outside
// the normal range).  Every step is one rounded f32 operation, so the CPU
// oracle's restatement gives the same bits.
__device__ __forceinline__ float btl_expf(float x)
{
    if (x != x) return x;
    if (x > 88.72283935546875f) return __uint_as_float(0x7F800000u);
    if (x < -103.97208404541016f) return 0.0f;
    const float n = __builtin_rintf(__fmul_rn(x, 1.44269502162933349609375f));
    const float r = __fsub_rn(__fsub_rn(x, __fmul_rn(n, 0.693145751953125f)),
                              __fmul_rn(n, 1.428606765330187045037746429443359375e-6f));
    float p = 1.98412701138295233249664306640625e-4f;
    p = __fadd_rn(__fmul_rn(p, r), 1.3888889225199818611145019531250e-3f);
    p = __fadd_rn(__fmul_rn(p, r), 8.3333337679505348205566406250e-3f);
    p = __fadd_rn(__fmul_rn(p, r), 4.1666667908430099487304687500e-2f);
    p = __fadd_rn(__fmul_rn(p, r), 0.16666667163372039794921875f);
    p = __fadd_rn(__fmul_rn(p, r), 0.5f);
    p = __fadd_rn(__fmul_rn(p, r), 1.0f);
    p = __fadd_rn(__fmul_rn(p, r), 1.0f);
    const int ni = (int)n;
    if (ni > 127) return __fmul_rn(__fmul_rn(p, __uint_as_float(254u << 23)), __uint_as_float((uint32_t)(ni + 127 - 127) << 23));
    if (ni < -126) return __fmul_rn(__fmul_rn(p, __uint_as_float((uint32_t)(ni + 64 + 127) << 23)), __uint_as_float(63u << 23));
    return __fmul_rn(p, __uint_as_float((uint32_t)(ni + 127) << 23));
}

// Pairwise sum over the lanes of a wave (xor butterfly: at level j lane i adds
// lane i ^ 2^j, which is the pairwise tree over lanes in index order -- float
// addition commutes).  Every lane ends with the wave's sum.
__device__ __forceinline__ float wave_pairwise_sum(float v)
{
#pragma unroll
    for (int j = 1; j < 64; j <<= 1) v = __fadd_rn(v, __shfl_xor(v, j, 64));
    return v;
}

// Correctly rounded sqrt of an f32 (the hardware v_sqrt_f32 is not): for a
// positive finite x = M * 2^(2h) with M an integer in [2^46, 2^48), r =
// isqrt(M) is found from an f32 estimate corrected with exact 64-bit squares,
// rounded up when M - r^2 > r (the midpoint (r + 1/2)^2 = r^2 + r + 1/4 is
// never an integer), and r * 2^h is exact.  Zero, negative, inf and NaN
// inputs take the hardware sqrt, which is exact for them.
__device__ __forceinline__ float sqrt_rn(float x)
{
    const uint32_t b = __float_as_uint(x);
    if (!(x > 0.0f) || b >= 0x7F800000u) return __builtin_sqrtf(x);
    int e = (int)(b >> 23);
    uint32_t mant = b & 0x7FFFFFu;
    if (e == 0) {  // subnormal: normalise
        const int sh = __clz(mant) - 8;
        mant <<= sh;
        e = 1 - sh;
    } else {
        mant |= 0x800000u;
    }
    int ex = e - 150;                   // x = mant * 2^ex, mant in [2^23, 2^24)
    const int sft = (ex & 1) ? 23 : 24;  // ex - sft even
    const uint64_t M = (uint64_t)mant << sft;
    const int h = (ex - sft) / 2;
    uint64_t r = (uint64_t)__builtin_sqrtf((float)M);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        if (r * r > M) r -= 1;
        if ((r + 1) * (r + 1) <= M) r += 1;
    }
    if (M - r * r > r) r += 1;
    return __fmul_rn((float)r, __uint_as_float((uint32_t)(h + 127) << 23));
}

template <int XK>
__device__ __forceinline__ void widen16(const uint4* v, float* f)
{
    if (XK == XK_BF16) {
        const uint32_t u[8] = {v[0].x, v[0].y, v[0].z, v[0].w, v[1].x, v[1].y, v[1].z, v[1].w};
#pragma unroll
        for (int h = 0; h < 8; ++h) {
            f[2 * h] = __uint_as_float(u[h] << 16);
            f[2 * h + 1] = __uint_as_float(u[h] & 0xFFFF0000u);
        }
    } else {
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            f[4 * h] = __uint_as_float(v[h].x); f[4 * h + 1] = __uint_as_float(v[h].y);
            f[4 * h + 2] = __uint_as_float(v[h].z); f[4 * h + 3] = __uint_as_float(v[h].w);
        }
    }
}

}  // namespace btl
