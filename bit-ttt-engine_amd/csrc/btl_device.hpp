// btl_device.hpp -- device helpers shared by the gfx950 kernel sources
// (btl_kernels.hip, btl_model.hip).  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace btl {

// Raw buffer loads: a per-workgroup resource descriptor bounds every access,
// and an out-of-range offset reads zeros without a branch, so the compiler can
// count the loads in flight exactly (s_waitcnt vmcnt(N) per step).
constexpr int kOOB = 0x7FFFFFF0;  // offset outside every descriptor range

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint4 bload(__amdgpu_buffer_rsrc_t r, int off)
{
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Max of a u32 over the wave, via DPP (quad perms, row rotations, row
// broadcasts); the result is read from lane 63.
__device__ __forceinline__ uint32_t wave_max_dpp(uint32_t v)
{
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xB1, 0xF, 0xF, false));   // quad [1,0,3,2]
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xF, 0xF, false));   // quad [2,3,0,1]
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x124, 0xF, 0xF, false));  // row_ror:4
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x128, 0xF, 0xF, false));  // row_ror:8
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x142, 0xA, 0xF, false));  // row_bcast:15
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x143, 0xC, 0xF, false));  // row_bcast:31
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

}  // namespace btl
