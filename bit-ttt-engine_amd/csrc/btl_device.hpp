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

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 16 bytes per lane, global (descriptor r, byte offset voff) -> LDS lds + 16 * lane.
// Offsets outside the descriptor range read as zero.
__device__ __forceinline__ void copy_to_lds(__amdgpu_buffer_rsrc_t r, uint8_t* lds, int voff)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 16, voff, 0, 0, 0);
}

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 layout: vmcnt bits
// 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
constexpr int vmcnt_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

// s_waitcnt vmcnt(0): every global load (and LDS copy) of this wave has landed.
__device__ __forceinline__ void wait_loads() { __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); }

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

// round_half_away(x*r) as an int, for a finite row (see quant1)
__device__ __forceinline__ int quant_fast(float x, float r)
{
    const float y = __fmul_rn(x, r);
    return (int)__fadd_rn(y, __builtin_copysignf(0.49999997f, y));
}

// bytes {q[v], q[4+v], q[8+v], q[12+v]} of four ints -> one word
__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d)
{
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0C0C0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x04000C0Cu);
    return lo | hi;
}

typedef unsigned short us2 __attribute__((ext_vector_type(2)));

template <int XK>
struct DecX {
    static constexpr int kVec = XK == XK_F32 ? 4 : (XK == XK_BF16 ? 2 : 1);  // uint4 per group
    static constexpr bool kPreq = XK == XK_I8 || XK == XK_I8O;              // quantised by the caller
};

template <int XK>
__device__ __forceinline__ uint32_t group_absmax(const uint4* v)
{
    if (XK == XK_BF16) {
        us2 mx = __builtin_bit_cast(us2, v[0].x & 0x7FFF7FFFu);
        mx = __builtin_elementwise_max(mx, __builtin_bit_cast(us2, v[0].y & 0x7FFF7FFFu));
        mx = __builtin_elementwise_max(mx, __builtin_bit_cast(us2, v[0].z & 0x7FFF7FFFu));
        mx = __builtin_elementwise_max(mx, __builtin_bit_cast(us2, v[0].w & 0x7FFF7FFFu));
        mx = __builtin_elementwise_max(mx, __builtin_bit_cast(us2, v[1].x & 0x7FFF7FFFu));
        mx = __builtin_elementwise_max(mx, __builtin_bit_cast(us2, v[1].y & 0x7FFF7FFFu));
        mx = __builtin_elementwise_max(mx, __builtin_bit_cast(us2, v[1].z & 0x7FFF7FFFu));
        mx = __builtin_elementwise_max(mx, __builtin_bit_cast(us2, v[1].w & 0x7FFF7FFFu));
        return (uint32_t)(mx.x > mx.y ? mx.x : mx.y) << 16;
    }
    uint32_t m = 0;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        m = max(m, max(max(v[h].x & 0x7FFFFFFFu, v[h].y & 0x7FFFFFFFu),
                       max(v[h].z & 0x7FFFFFFFu, v[h].w & 0x7FFFFFFFu)));
    }
    return m;
}

// 16 f32 values -> operand-order int8 word quadruple (finite row, r = 127/a)
__device__ __forceinline__ uint4 group_quant_f(const float* f, float r)
{
    // one output word at a time (fewer live registers)
    uint4 o;
    o.x = pack4(quant_fast(f[0], r), quant_fast(f[4], r), quant_fast(f[8], r), quant_fast(f[12], r));
    o.y = pack4(quant_fast(f[1], r), quant_fast(f[5], r), quant_fast(f[9], r), quant_fast(f[13], r));
    o.z = pack4(quant_fast(f[2], r), quant_fast(f[6], r), quant_fast(f[10], r), quant_fast(f[14], r));
    o.w = pack4(quant_fast(f[3], r), quant_fast(f[7], r), quant_fast(f[11], r), quant_fast(f[15], r));
    return o;
}

// 16 activations of one group -> operand-order int8 word quadruple
template <int XK>
__device__ __forceinline__ uint4 group_quant(const uint4* v, float r)
{
    if (XK == XK_I8) return transpose16(v[0]);
    if (XK == XK_I8O) return v[0];
    float f[16];
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
    return group_quant_f(f, r);
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
