// btl_kernels.hip -- gfx950 (CDNA4) kernels of the BitLinear engine.
//
// Reference path (imonoonoko/Bit-TTT-Engine, crates/rust_engine):
//   packed layout / codes ........ src/kernels/packing.rs:6-21, 74-92
//   fp32 contraction order ....... src/kernels/cpu.rs:77-123, 172-238
//   absmax convention ............ src/layers/kv_cache.rs:95-119
//
// Kernels:
//   k_gemv_dec<XK,YK,WV>  the decode case (1..4 token rows): one 16-row tile
//                     per workgroup, WV waves split K, activations quantised
//                     per wave from registers loaded ahead of the weights.
//   k_gemm_i8         prefill GEMM (many token rows): int8 MFMA on 128x128 or 128x256
//                     tiles fed by direct global->LDS copies, the packed
//                     weight tile unpacked per wave; k_quant_op quantises the
//                     tokens ahead of it in operand order (k_op_order
//                     reorders pre-quantised ones).
//   k_quant_act<XK>   per-token absmax int8 quantisation, natural layout.
//   k_ref_f32<XK,YK>  reference-semantics fp32 path: bit-identical to the
//                     8-lane FMA order of cpu.rs; k_ref_f32_st is its form for
//                     k % 64 == 0 (weights streamed through LDS, f16 coefficient
//                     lookup by byte permute, v_fma_mix_f32).
//   k_generic_i8<YK>  any k % 4 == 0 / any alignment, int8 activations.
//   k_unpack          dense f32 weights (PackedTensor::unpack on the device).
//   k_fill_zero       workspace clearing (a kernel, so it is graph-capture safe).
//
// Compiled with -ffp-contract=off: every fp32 operation below is rounded as
// written (the oracle restates the same operations in C).
#include <hip/hip_runtime.h>

#include <utility>

#include <atomic>
#include <mutex>
#include <type_traits>
#include <stdlib.h>

#include "btl_device.hpp"
#include "btl_internal.hpp"

namespace btl {

// ---------------------------------------------------------------------------
// k_gemv_dec: decode (1..4 token rows)
// ---------------------------------------------------------------------------
// A workgroup owns RB row blocks of 16 weight rows and splits K into WV parts
// (both runtime, WV * RB <= 16): wave w works on row block w / WV, K part
// w % WV (kpart weights, at most ST loads of 256 weights per lane).  The workgroup first loads the token rows (every
// thread a few 16-element groups, issued before the weights), then each wave
// puts all of its weight loads in flight; the absmax of each row is reduced
// over the workgroup (DPP + LDS), and every thread quantises its groups into
// one shared LDS copy of the rows in operand order -- once per workgroup, so
// RB > 1 amortises this prologue over more weights.  The K parts of a row
// block are summed exactly through LDS; the part-0 wave applies the epilogue.
// Group slots per thread in the prologue: kDecGroups; a fused transform holds
// its row in fewer (the host checks k / 16 <= DG * threads) and launches at
// most 512 threads, leaving 256 registers per lane.
template <int XF>
struct DecXf {
    static constexpr int kGroups = XF == XF_NONE ? kDecGroups : (XF == XF_SWIGLU ? 2 : 1);
};

// Threads per workgroup a decode instantiation is compiled for: up to 16
// waves (128 registers per lane); 8 with a fused transform or 16 loads per
// wave in flight (256 registers per lane).
constexpr int dec_threads(int st, int xf, int ni)
{
    return xf != XF_NONE ? 512 : (ni > 0 && st > 8 ? 512 : 1024);
}

template <int XK, int ST, int MT, int XF, bool PAIR, int NI = 0>
__global__ __launch_bounds__(dec_threads(ST, XF, NI)) void k_gemv_dec(GemvArgs a)
{
    // NI > 0: the row-contiguous form (one token row, k <= NI * 4096).  Wave
    // `part` of a row block owns RPW = ST / NI whole rows, part + WV * rho
    // (rows interleaved over the waves, measured faster than consecutive
    // rows); its load t reads 1 KB of its row t / NI (chunk t % NI, lane l:
    // bytes 16l..16l+15), so one
    // load instruction covers 8 full 128-byte lines.  The activation operand
    // of MFMA word h is the 16 quantised values at k = 4096c + 64l + 16h, the
    // same for every row: the 16x16 product's diagonal D[i][i] sums lanes i,
    // i+16, i+32, i+48 of the row, and the row's dot product is the trace.
    // No K parts, so no cross-wave reduction.
    static_assert(NI == 0 || (MT == 1 && ST % NI == 0), "row-contiguous form: one token row");
    constexpr int RPW = NI > 0 ? ST / NI : 1;
    const int WV = NI > 0 ? 16 / RPW : a.parts, RB = a.tiles;  // NW = WV * RB <= 16 waves
    const int NW = WV * RB, NT = NW * 64;
    extern __shared__ __align__(16) uint8_t sq[];  // [mt][k + 16], operand order
    __shared__ uint32_t s_amax[16][MT];
    __shared__ v4i s_red[NI > 0 ? 1 : 16][64];  // K-part sums; the row-contiguous form stages gate outputs only
    __shared__ float s_ss[16];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rbi = wave / WV, part = wave - rbi * WV;
    // PAIR (SwiGLU epilogue): rbi 0 is gate's row block w, rbi 1 up's.  A
    // template parameter, so the plain launch's first weight address needs no
    // extra kernel-argument load.
    constexpr bool paired = PAIR;
    const int rbg = paired ? (rbi == 0 ? 0 : a.p[1].rb_begin) + (int)blockIdx.x
                           : (int)blockIdx.x * RB + rbi;  // past rb_total: no rows (zero loads, no stores)
    const int mt = MT == 1 ? 1 : min(MT, a.m);

    const uint8_t* W = a.p[0].w;
    void* Y = a.p[0].y;
    int32_t* ACC = a.p[0].acc_out;
    float SW = a.p[0].sw;
    int N = a.p[0].n;
    int RB0 = a.p[0].rb_begin;
#pragma unroll
    for (int i = 1; i < kMaxGroup; ++i) {
        if (i < a.nprob && rbg >= a.p[i].rb_begin) {
            W = a.p[i].w; Y = a.p[i].y; ACC = a.p[i].acc_out;
            SW = a.p[i].sw; N = a.p[i].n; RB0 = a.p[i].rb_begin;
        }
    }
    const int K = a.k;
    const int kp = a.kpart;
    const int kb = part * kp;
    const int len = max(0, min(kp, K - kb));
    const int lp = K + 16;

    // 1. the token rows -> registers, kDecGroups 16-element groups per thread at
    //    most (issued before the weight loads)
    constexpr int NV = DecX<XK>::kVec;
    constexpr int ES = XK == XK_F32 ? 4 : (XK == XK_BF16 ? 2 : 1);  // bytes per element
    constexpr bool PREQ = DecX<XK>::kPreq;
    const int gpr = K >> 4;  // groups per token row
    const int ng = mt * gpr;
    // the row-contiguous form launches at least 256 threads: NI groups per
    // thread cover k <= NI * 4096
    constexpr int DG = NI > 0 && XF == XF_NONE ? NI : DecXf<XF>::kGroups;
    int gm_[DG], gc_[DG];
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)(mt * K * ES));
    uint4 xv[DG][NV];
#pragma unroll
    for (int gi = 0; gi < DG; ++gi) {
        const int g = tid + NT * gi;
        const int m = MT == 1 ? 0 : g / max(gpr, 1);
        gm_[gi] = m;
        gc_[gi] = g - m * gpr;
        const int off = g < ng ? (m * K + 16 * gc_[gi]) * ES : kOOB;
#pragma unroll
        for (int h = 0; h < NV; ++h) xv[gi][h] = gi == 0 || NT * gi < ng ? bload(xr, off + 16 * h) : uint4{0u, 0u, 0u, 0u};
    }
    // fused transform input (one token row, f32): delta / up
    uint4 x2v[DG][4];
    if (XF == XF_ADD_RMSNORM || XF == XF_SWIGLU) {
        const __amdgpu_buffer_rsrc_t x2r = make_rsrc(a.x2, (uint32_t)(K * 4));
#pragma unroll
        for (int gi = 0; gi < DG; ++gi) {
            const int off = tid + NT * gi < ng ? 64 * (tid + NT * gi) : kOOB;
#pragma unroll
            for (int h = 0; h < 4; ++h)
                x2v[gi][h] = gi == 0 || NT * gi < ng ? bload(x2r, off + 16 * h) : uint4{0u, 0u, 0u, 0u};
        }
    }

    // 2. every weight load of this wave in flight.  K-part form: non-temporal
    //    pairs as in k_gemv_bat (load 2p + h: lane l reads row 8 h + (l & 7),
    //    bytes [128 p + 16 (l >> 3), +16) of the part; 8 rows x 128 bytes per
    //    instruction)
    const int kq = lane >> 4;
    const int row0 = (rbg - RB0) * 16;
    const int rows = __builtin_amdgcn_readfirstlane(max(0, min(16, N - row0)));
    const int rb_bytes = K >> 2;
    uint4 buf[ST];
    if (NI > 0) {
        // rows row0 + part * RPW + [0, RPW) of this row block, chunks past the row read zeros
        const __amdgpu_buffer_rsrc_t wr = make_rsrc(W + (int64_t)row0 * rb_bytes, (uint32_t)(rows * rb_bytes));
#pragma unroll
        for (int j = 0; j < ST; ++j) {
            const int rho = j / (NI > 0 ? NI : 1), c = j - rho * (NI > 0 ? NI : 1);
            buf[j] = bload(wr, c * 1024 + 16 * lane < rb_bytes ? (part + WV * rho) * rb_bytes + c * 1024 + 16 * lane : kOOB);
        }
    } else {
        static_assert(NI > 0 || ST % 2 == 0, "loads come in pairs");
        const __amdgpu_buffer_rsrc_t wr = make_rsrc(W + (int64_t)row0 * rb_bytes, (uint32_t)(rows * rb_bytes));
#pragma unroll
        for (int j = 0; j < ST; ++j) {
            const int kw = (j >> 1) * 512 + (lane >> 3) * 64;  // first weight of the lane's 16 bytes
            const int off = (8 * (j & 1) + (lane & 7)) * rb_bytes + (kb >> 2) + (kw >> 2);
            buf[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, kw < len ? off : kOOB, 0,
                                                                                     kCachePolicyNT));
        }
    }

    // 3. absmax of each token row over the workgroup; lane m then holds the
    //    quantisation parameters of token row m
    float r_l = 0.0f, s_l = 0.0f;
    float fv[XF != XF_NONE ? DG : 1][16];
    if (XF != XF_NONE) {
        // the transform of k_xform_quant, per workgroup on its own copy of the row
#pragma unroll
        for (int gi = 0; gi < DG; ++gi) {
            if (gi == 0 || NT * gi < ng) {
                widen16<XK_F32>(xv[gi], fv[gi]);
                if (XF == XF_ADD_RMSNORM || XF == XF_SWIGLU) {
                    float u[16];
                    widen16<XK_F32>(x2v[gi], u);
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const float v = fv[gi][e];
                        fv[gi][e] = XF == XF_SWIGLU ? __fmul_rn(__fdiv_rn(v, __fadd_rn(1.0f, btl_expf(-v))), u[e])
                                                    : __fadd_rn(v, u[e]);
                    }
                    if (XF == XF_ADD_RMSNORM && a.hout && blockIdx.x == 0 && tid + NT * gi < ng) {
                        float4* hp = (float4*)(a.hout + 16 * (tid + NT * gi));
#pragma unroll
                        for (int h = 0; h < 4; ++h)
                            hp[h] = make_float4(fv[gi][4 * h], fv[gi][4 * h + 1], fv[gi][4 * h + 2], fv[gi][4 * h + 3]);
                    }
                }
            }
        }
        if (XF == XF_RMSNORM || XF == XF_ADD_RMSNORM) {
            // sum of squares in the pairwise order of k_xform_quant: the host
            // launches this only when k / 16 <= NT, so thread t holds elements
            // [16t, 16t + 16) (zeros past k)
            float t[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) t[e] = __fmul_rn(fv[0][e], fv[0][e]);
#pragma unroll
            for (int len = 16; len > 1; len >>= 1)
#pragma unroll
                for (int i = 0; i < len / 2; ++i) t[i] = __fadd_rn(t[2 * i], t[2 * i + 1]);
            const float ws = wave_pairwise_sum(t[0]);
            if (lane == 0) s_ss[wave] = ws;
            uint4 gv[4];  // the norm weight, loaded only now (fewer live registers while loads fly)
            {
                const __amdgpu_buffer_rsrc_t gr = make_rsrc(a.g, (uint32_t)(K * 4));
                const int off = tid < ng ? 64 * tid : kOOB;
#pragma unroll
                for (int h = 0; h < 4; ++h) gv[h] = bload(gr, off + 16 * h);
            }
            __syncthreads();
            float p[16];
#pragma unroll
            for (int w = 0; w < 16; ++w) p[w] = w < NW ? s_ss[w] : 0.0f;
#pragma unroll
            for (int len = 16; len > 1; len >>= 1)
#pragma unroll
                for (int i = 0; i < len / 2; ++i) p[i] = __fadd_rn(p[2 * i], p[2 * i + 1]);
            const float inv_k = (float)(1.0 / (double)K);
            const float d = sqrt_rn(__fadd_rn(__fmul_rn(p[0], inv_k), a.eps));
            float gf[16];
            widen16<XK_F32>(gv, gf);
#pragma unroll
            for (int e = 0; e < 16; ++e) fv[0][e] = __fmul_rn(__fdiv_rn(fv[0][e], d), gf[e]);
        }
        uint32_t am = 0;
#pragma unroll
        for (int gi = 0; gi < DG; ++gi)
            if (tid + NT * gi < ng)
#pragma unroll
                for (int e = 0; e < 16; ++e) am = max(am, __float_as_uint(fv[gi][e]) & 0x7FFFFFFFu);
        const uint32_t v = wave_max_dpp(am);
        if (lane == 0) s_amax[wave][0] = v;
        __syncthreads();
        uint32_t vm = 0;
        for (int w = 0; w < NW; ++w) vm = max(vm, s_amax[w][0]);
        const QParams qp = qparams(vm);
        r_l = qp.ok ? qp.r : 0.0f;
        s_l = qp.s;
    } else if (!PREQ) {
        uint32_t am[MT];
#pragma unroll
        for (int mm = 0; mm < MT; ++mm) am[mm] = 0u;
#pragma unroll
        for (int gi = 0; gi < DG; ++gi) {
            if (gi == 0 || NT * gi < ng) {
                const uint32_t v = tid + NT * gi < ng ? group_absmax<XK>(xv[gi]) : 0u;
#pragma unroll
                for (int mm = 0; mm < MT; ++mm) am[mm] = (MT == 1 || mm == gm_[gi]) ? max(am[mm], v) : am[mm];
            }
        }
#pragma unroll
        for (int mm = 0; mm < MT; ++mm) {
            if (mm < mt) {
                const uint32_t v = wave_max_dpp(am[mm]);
                if (lane == 0) s_amax[wave][mm] = v;
            }
        }
        __syncthreads();
        const int lm = MT == 1 ? 0 : min(lane, mt - 1);
        uint32_t v = 0;
        for (int w = 0; w < NW; ++w) v = max(v, s_amax[w][lm]);
        const QParams qp = qparams(v);
        r_l = qp.ok ? qp.r : 0.0f;
        s_l = qp.s;
    } else {
        s_l = a.xs[MT == 1 ? 0 : min(lane, mt - 1)];
    }

    // 4. quantise this thread's groups into the shared rows
#pragma unroll
    for (int gi = 0; gi < DG; ++gi) {
        if (gi == 0 || NT * gi < ng) {
            const int g = tid + NT * gi;
            float rm = r_l;
            if (MT > 1) rm = __shfl(r_l, gm_[gi], 64);
            uint4 q = XF != XF_NONE ? (rm != 0.0f ? group_quant_f(fv[XF != XF_NONE ? gi : 0], rm) : uint4{0u, 0u, 0u, 0u})
                                    : group_quant<XK>(xv[gi], rm);
            if (!PREQ && rm == 0.0f) q = uint4{0u, 0u, 0u, 0u};  // zero or non-finite row
            if (g < ng) *(uint4*)(sq + gm_[gi] * lp + 16 * gc_[gi]) = q;
        }
    }
    __syncthreads();

    if constexpr (NI > 0) {
        // 5. row-contiguous contraction, row by row (one accumulator, the
        //    rows interleave in the schedule); 6. the trace of each
        //    row's product: lane l holds D[4(l/16) + v][l % 16], so D[i][i] is
        //    register l % 4 of lane l when (l / 4) % 4 == l / 16 (lanes 0-3,
        //    20-23, 40-43, 60-63); exact int32 sums.  Lanes past the row's end
        //    read the activation at k = 0 (their weights are zero).
        const bool diag = ((lane >> 2) & 3) == (lane >> 4);
        int sv = 0;
#pragma unroll
        for (int rho = 0; rho < RPW; ++rho) {
            v4i acc = v4i{0, 0, 0, 0};
#pragma unroll
            for (int c = 0; c < NI; ++c) {
                const int ko = c * 4096 + 64 * lane;
                const uint8_t* bj = sq + (ko < K ? ko : 0);
                const v4i b0 = *(const v4i*)(bj + 0);
                const v4i b1 = *(const v4i*)(bj + 16);
                const v4i b2 = *(const v4i*)(bj + 32);
                const v4i b3 = *(const v4i*)(bj + 48);
                const uint4 cur = buf[rho * NI + c];
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack16(cur.x), b0, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack16(cur.y), b1, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack16(cur.z), b2, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack16(cur.w), b3, acc, 0, 0, 0);
            }
            const v4i t = acc;
            int d = (lane & 2) ? ((lane & 1) ? t.w : t.z) : ((lane & 1) ? t.y : t.x);
            d = diag ? d : 0;
            d += __builtin_amdgcn_update_dpp(0, d, 0xB1, 0xF, 0xF, true);  // quad [1,0,3,2], one v_add_u32_dpp
            d += __builtin_amdgcn_update_dpp(0, d, 0x4E, 0xF, 0xF, true);  // quad [2,3,0,1]
            const int s = __builtin_amdgcn_readlane(d, 0) + __builtin_amdgcn_readlane(d, 20) +
                          __builtin_amdgcn_readlane(d, 40) + __builtin_amdgcn_readlane(d, 60);
            sv = lane == rho ? s : sv;
        }
        // lane rho stores row row0 + part + WV * rho
        const int n = row0 + part + WV * lane;
        const bool own = lane < RPW && n < N;
        const float yv = __fmul_rn((float)sv, __fmul_rn(s_l, SW));
        if (paired) {
            // gate's wave hands its outputs to the up wave of the same rows
            float* s_gate = (float*)s_red;
            if (rbi == 0 && own) s_gate[part + WV * lane] = yv;
            __syncthreads();
            if (!own) return;
            if (Y) {
                if (a.ykind == YK_BF16) ((uint16_t*)Y)[n] = f32_to_bf16(yv);
                else ((float*)Y)[n] = yv;
            }
            if (ACC) ACC[n] = sv;
            if (rbi == 1) {
                const float gv = s_gate[part + WV * lane];
                a.swiglu_out[n] = __fmul_rn(__fdiv_rn(gv, __fadd_rn(1.0f, btl_expf(-gv))), yv);
            }
            return;
        }
        if (!own) return;
        if (a.ykind == YK_BF16) ((uint16_t*)Y)[n] = f32_to_bf16(yv);
        else ((float*)Y)[n] = yv;
        if (ACC) ACC[n] = sv;
        return;
    }

    // 5. contraction: lane l holds row l & 15 after the pair exchange of
    //    k_gemv_bat (chunk 2 kq + b from load 2p + b, chunk 2 kq + 1 - b from
    //    lane l ^ 8 of the other load, b = bit 3 of l); word w of the 32 bytes
    //    takes the 16 activations at k = kb + 512 p + 128 kq + 16 w.  B lanes of
    //    token columns >= mt read row 0: those columns of D are never stored.
    const int mcol = lane & 15;
    const bool m_ok = mcol < mt;
    const bool hi = (lane & 8) != 0;
    const uint8_t* bq = sq + (m_ok ? mcol : 0) * lp + kb + kq * 128;
    v4i acc[2];
    acc[0] = acc[1] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int p = 0; p < ST / 2; ++p) {
        const uint8_t* bj = bq + p * 512;
        const uint32_t X[4] = {buf[2 * p].x, buf[2 * p].y, buf[2 * p].z, buf[2 * p].w};
        const uint32_t Y[4] = {buf[2 * p + 1].x, buf[2 * p + 1].y, buf[2 * p + 1].z, buf[2 * p + 1].w};
        uint32_t wd[8];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t own = hi ? Y[w] : X[w];
            const uint32_t give = hi ? X[w] : Y[w];
            const uint32_t got = (uint32_t)__builtin_amdgcn_mov_dpp((int)give, 0x128, 0xF, 0xF, false);  // row_ror:8
            wd[w] = hi ? got : own;
            wd[4 + w] = hi ? own : got;
        }
#pragma unroll
        for (int w = 0; w < 8; ++w)
            acc[w & 1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack16(wd[w]), *(const v4i*)(bj + 16 * w), acc[w & 1],
                                                              0, 0, 0);
    }
    v4i res = acc[0] + acc[1];

    // 6. sum the K parts of each row block (exact), epilogue by its part-0 wave
    if (WV > 1) {
        if (part > 0) s_red[wave][lane] = res;
        __syncthreads();
        if (part > 0 && !paired) return;
        if (part == 0)
            for (int p = 1; p < WV; ++p) res += s_red[wave + p][lane];
    }
    const float sx = MT == 1 ? s_l : __shfl(s_l, mcol < mt ? mcol : 0, 64);
    const float c = __fmul_rn(sx, SW);
    const bool ybf = a.ykind == YK_BF16;
    const int nb = row0 + 4 * (lane >> 4);
    if (paired) {
        // gate's part-0 wave hands its outputs to up's through LDS (every wave
        // reaches the barrier), which writes silu(gate) * up
        float* s_gate = (float*)s_red;  // [16 rows][4 token columns], free after the K-part sum
        __syncthreads();
        if (part == 0 && rbi == 0 && m_ok) {
#pragma unroll
            for (int v = 0; v < 4; ++v) s_gate[(nb - row0 + v) * 4 + mcol] = __fmul_rn((float)res[v], c);
        }
        __syncthreads();
        if (part != 0 || !m_ok) return;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int n = nb + v;
            if (n < N) {
                const int64_t o = (int64_t)mcol * N + n;
                const float yv = __fmul_rn((float)res[v], c);
                if (Y) {
                    if (ybf) ((uint16_t*)Y)[o] = f32_to_bf16(yv);
                    else ((float*)Y)[o] = yv;
                }
                if (ACC) ACC[o] = res[v];
                if (rbi == 1) {
                    const float gv = s_gate[(nb - row0 + v) * 4 + mcol];
                    a.swiglu_out[o] = __fmul_rn(__fdiv_rn(gv, __fadd_rn(1.0f, btl_expf(-gv))), yv);
                }
            }
        }
        return;
    }
    if (!m_ok) return;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int n = nb + v;
        if (n < N) {
            const int64_t o = (int64_t)mcol * N + n;
            const float yv = __fmul_rn((float)res[v], c);
            if (ybf) ((uint16_t*)Y)[o] = f32_to_bf16(yv);
            else ((float*)Y)[o] = yv;
            if (ACC) ACC[o] = res[v];
        }
    }
}

hipError_t launch_gemv_dec(const GemvArgs& a, int xkind, int xform, hipStream_t s)
{
    const int wv = a.parts, rb = a.tiles;
    const int st_need = (a.kpart + kStepWeights - 1) / kStepWeights;
    if (wv < 1 || rb < 1 || wv * rb > 16 || (a.rowc == 0 && (st_need > 8 || (int64_t)wv * a.kpart < a.k)) ||
        a.m < 1 || a.m > 4 || (int64_t)a.m * (a.k >> 4) > (int64_t)kDecGroups * wv * rb * 64)
        return hipErrorInvalidValue;
    if (a.swiglu_out && (a.nprob != 2 || a.p[0].n != a.p[1].n || rb != 2 || a.p[1].rb_begin != (a.p[0].n + 15) / 16 ||
                         a.rb_total != 2 * a.p[1].rb_begin))
        return hipErrorInvalidValue;
    if (xform != XF_NONE &&
        (xkind != XK_F32 || a.m != 1 || wv * rb > 8 || !a.x2 == (xform == XF_ADD_RMSNORM || xform == XF_SWIGLU) ||
         ((xform == XF_RMSNORM || xform == XF_ADD_RMSNORM) && (!a.g || (a.k >> 4) > wv * rb * 64)) ||
         (xform == XF_SWIGLU && (a.k >> 4) > 2 * wv * rb * 64) || (a.hout && (const void*)a.hout == a.x)))
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)((a.rb_total + rb - 1) / rb)), block((unsigned)(wv * rb * 64));
    // the token rows, plus what the last K part reads past the last row (its
    // weights there are zero) when the parts overrun k
    const size_t lds = (size_t)a.m * (size_t)(a.k + 16) +
                       (a.rowc == 0 && (int64_t)wv * a.kpart > a.k ? (size_t)((int64_t)wv * a.kpart - a.k) : 0);
    const bool pr = a.swiglu_out != nullptr;
    if (a.rowc != 0) {
        // (chunks, waves per row block) -> loads per wave ST = chunks * 16 / waves
        const int ni = a.rowc;
        const int st = wv > 0 ? ni * 16 / wv : 0;
        if ((ni != 1 && ni != 2 && ni != 4) || a.m != 1 || a.k % 64 != 0 || a.k > ni * 4096 || 16 % wv != 0 ||
            (st != 4 && st != 8 && st != 16) || wv * rb * 64 > dec_threads(st, xform, ni) || wv * rb < 4 ||
            (xform != XF_NONE && st != dec_row_st(ni)))
            return hipErrorInvalidValue;
#define BTL_ROW_ST(XKV, XFV, PRV, NIV)                                                                     \
    if (st == 4) hipLaunchKernelGGL((k_gemv_dec<XKV, 4, 1, XFV, PRV, NIV>), grid, block, lds, s, a);       \
    else if (st == 8) hipLaunchKernelGGL((k_gemv_dec<XKV, 8, 1, XFV, PRV, NIV>), grid, block, lds, s, a);  \
    else hipLaunchKernelGGL((k_gemv_dec<XKV, 16, 1, XFV, PRV, NIV>), grid, block, lds, s, a);
#define BTL_ROW_NI(XKV, XFV, PRV)             \
    if (ni == 1) { BTL_ROW_ST(XKV, XFV, PRV, 1) } \
    else if (ni == 2) { BTL_ROW_ST(XKV, XFV, PRV, 2) } \
    else { BTL_ROW_ST(XKV, XFV, PRV, 4) }
        if (xform != XF_NONE) {  // the default rows per wave only
#define BTL_ROW_XF(XFV)                                                                                      \
    if (ni == 1) hipLaunchKernelGGL((k_gemv_dec<XK_F32, 4, 1, XFV, false, 1>), grid, block, lds, s, a);      \
    else if (ni == 2) hipLaunchKernelGGL((k_gemv_dec<XK_F32, 8, 1, XFV, false, 2>), grid, block, lds, s, a); \
    else hipLaunchKernelGGL((k_gemv_dec<XK_F32, 8, 1, XFV, false, 4>), grid, block, lds, s, a);
            if (pr) return hipErrorInvalidValue;
            if (xform == XF_RMSNORM) { BTL_ROW_XF(XF_RMSNORM) }
            else if (xform == XF_ADD_RMSNORM) { BTL_ROW_XF(XF_ADD_RMSNORM) }
            else { BTL_ROW_XF(XF_SWIGLU) }
#undef BTL_ROW_XF
            return hipGetLastError();
        }
        if (pr) {
            if (xkind == XK_F32) { BTL_ROW_NI(XK_F32, XF_NONE, true) return hipGetLastError(); }
            if (xkind == XK_I8O) { BTL_ROW_NI(XK_I8O, XF_NONE, true) return hipGetLastError(); }
            return hipErrorInvalidValue;
        }
        if (xkind == XK_BF16) { BTL_ROW_NI(XK_BF16, XF_NONE, false) return hipGetLastError(); }
        if (xkind == XK_F32) { BTL_ROW_NI(XK_F32, XF_NONE, false) return hipGetLastError(); }
        if (xkind == XK_I8) { BTL_ROW_NI(XK_I8, XF_NONE, false) return hipGetLastError(); }
        if (xkind == XK_I8O) { BTL_ROW_NI(XK_I8O, XF_NONE, false) return hipGetLastError(); }
#undef BTL_ROW_NI
#undef BTL_ROW_ST
        return hipErrorInvalidValue;
    }
    const bool st4 = st_need <= 4;
    const bool mt1 = a.m == 1;
#define BTL_DEC_XF(XFV)                                                                                     \
    if (xform == XFV) {                                                                                     \
        if (pr) {                                                                                           \
            if (st4) hipLaunchKernelGGL((k_gemv_dec<XK_F32, 4, 1, XFV, true>), grid, block, lds, s, a);     \
            else hipLaunchKernelGGL((k_gemv_dec<XK_F32, 8, 1, XFV, true>), grid, block, lds, s, a);         \
        } else {                                                                                            \
            if (st4) hipLaunchKernelGGL((k_gemv_dec<XK_F32, 4, 1, XFV, false>), grid, block, lds, s, a);    \
            else hipLaunchKernelGGL((k_gemv_dec<XK_F32, 8, 1, XFV, false>), grid, block, lds, s, a);        \
        }                                                                                                   \
        return hipGetLastError();                                                                           \
    }
    BTL_DEC_XF(XF_RMSNORM) BTL_DEC_XF(XF_ADD_RMSNORM) BTL_DEC_XF(XF_SWIGLU)
#undef BTL_DEC_XF
#define BTL_DEC_MT(XKV, PRV)                                                                                    \
    if (st4 && mt1) hipLaunchKernelGGL((k_gemv_dec<XKV, 4, 1, XF_NONE, PRV>), grid, block, lds, s, a);          \
    else if (st4) hipLaunchKernelGGL((k_gemv_dec<XKV, 4, 4, XF_NONE, PRV>), grid, block, lds, s, a);            \
    else if (mt1) hipLaunchKernelGGL((k_gemv_dec<XKV, 8, 1, XF_NONE, PRV>), grid, block, lds, s, a);            \
    else hipLaunchKernelGGL((k_gemv_dec<XKV, 8, 4, XF_NONE, PRV>), grid, block, lds, s, a);
    if (pr) {  // the SwiGLU epilogue's inputs: f32 tokens or the operand-order int8 of a separate transform
        if (xkind == XK_F32) { BTL_DEC_MT(XK_F32, true) return hipGetLastError(); }
        if (xkind == XK_I8O) { BTL_DEC_MT(XK_I8O, true) return hipGetLastError(); }
        return hipErrorInvalidValue;
    }
#define BTL_DEC_CASE(XKV)                     \
    if (xkind == XKV) {                       \
        BTL_DEC_MT(XKV, false)                \
        return hipGetLastError();             \
    }
    BTL_DEC_CASE(XK_BF16) BTL_DEC_CASE(XK_F32) BTL_DEC_CASE(XK_I8) BTL_DEC_CASE(XK_I8O)
#undef BTL_DEC_CASE
#undef BTL_DEC_MT
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// k_gemv_rq: one-token decode, row-group form
// ---------------------------------------------------------------------------
// A workgroup is nqw quantising waves followed by wpc compute waves.
//
// Compute wave c owns R consecutive weight rows (R = 4, or 2 for k > 4096).
// Its load t, lane l = 16 g + i, reads 16 bytes of row i / (16 / R) at byte
// t * (1024 / R) + 16 s, slice s = (16 / R) g + i % (16 / R): one load
// instruction covers R rows x 1024 / R contiguous bytes (eight whole 128-byte
// lines), non-temporal (the weights are read once).  MFMA word h of the lane
// takes the 16 quantised activations at k = 4 (t * 1024 / R + 16 s) + 16 h as
// B.  In the 16x16 product D[i][j] = sum_g A[i][g] B[g][j] (lane 16 g + i
// holds A row i and B column i of k block g), D[i][i] pairs every lane's
// weights with its own activations; the 16 / R diagonal entries of row rho sit
// in register v of lanes 20 rho + v (R = 4), or of lanes 40 rho + v and
// 40 rho + 20 + v (R = 2), so one accumulator over all loads and three DPP
// adds give every row's exact int32 dot product.
//
// The quantising waves (two 16-element groups of the token per thread) load
// the token, exchange the absmax through an LDS atomic max and quantise into
// the shared LDS row in operand order; the compute waves issue their weight
// loads at once and wait for the quantised row on an LDS counter, not on a
// barrier, so no wave waits for another wave's loads to issue (the memory
// queue of a CU back-pressures the issue of later loads for microseconds).
// Every wait is bounded by a.spin polls (BTL_WAIT_SPIN, 2^22 by default, ~0.1 s);
// a wait that gives up sets kFaultRqWait in the device fault word.

template <int R>
struct RqShape {
    static constexpr int kSub = 16 / R;      // lanes of one row in a 16-lane group
    static constexpr int kBytes = 1024 / R;  // bytes of a row per load instruction
};

// The quantised token row in LDS: operand-order byte b at rq_pad(b), 16 bytes
// of padding after every 64.  A compute wave's lanes read 16 bytes each at a
// stride of 64 bytes (one slice per lane); unpadded, those reads fell on 4 of
// the 16 four-bank groups (4-way conflicts with 4 rows per wave, 8-way with 2).
// Rows of several tokens are rq_row_bytes(k) apart (k % 64 == 0).
__host__ __device__ constexpr int rq_pad(int b) { return b + ((b >> 6) << 4); }
__host__ __device__ constexpr int rq_row_bytes(int k) { return k + (k >> 2) + 16; }

// Fault bits of this source's kernels (kFault*), read and cleared by the host.
__device__ uint32_t g_faults;

__device__ __forceinline__ void rq_wait(const uint32_t* c, uint32_t target, int spin)
{
    int it = 0;
    for (; it < spin; ++it) {
        if (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) break;
        __builtin_amdgcn_s_sleep(1);
    }
    // gave up: the row in LDS is incomplete and this launch's outputs are not valid
    if (it >= spin) __hip_atomic_fetch_or(&g_faults, kFaultRqWait, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// The quantising waves of k_gemv_rq, f32 / bf16 / int8 tokens: thread t
// holds groups t + nq gi of the MT x gpr groups of the token rows (row g /
// gpr).  The absmax of every row over the quantising waves (LDS atomic max per
// row, arrivals counted in s_sync[1]), then the groups in operand order into
// sq (rows rq_row_bytes(k) apart, bytes at rq_pad); pre-quantised rows are only copied.  Ends with this
// wave's last arrival.
template <int XK, int DG, int MT>
__device__ __forceinline__ void rq_quantise(const uint4 (*xv)[DecX<XK>::kVec], int K, int gpr, int mt, int nqw,
                                            int nq, int tid, int lane, uint8_t* sq, uint32_t* s_sync,
                                            uint32_t* s_amax, float* s_scale, int spin)
{
    constexpr bool PREQ = DecX<XK>::kPreq;
    const int ng = mt * gpr;
    float rm[DG];
#pragma unroll
    for (int gi = 0; gi < DG; ++gi) rm[gi] = 0.0f;
    if (!PREQ) {
        uint32_t am[MT];
#pragma unroll
        for (int mm = 0; mm < MT; ++mm) am[mm] = 0u;
#pragma unroll
        for (int gi = 0; gi < DG; ++gi) {
            const int g = tid + nq * gi;
            const uint32_t v = g < ng ? group_absmax<XK>(xv[gi]) : 0u;
            const int row = MT == 1 ? 0 : g / gpr;
#pragma unroll
            for (int mm = 0; mm < MT; ++mm) am[mm] = (MT == 1 || mm == row) ? max(am[mm], v) : am[mm];
        }
#pragma unroll
        for (int mm = 0; mm < MT; ++mm) {
            if (mm < mt) {
                const uint32_t v = wave_max_dpp(am[mm]);
                if (lane == 0) __hip_atomic_fetch_max(&s_amax[mm], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        }
        if (lane == 0) __hip_atomic_fetch_add(&s_sync[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        rq_wait(&s_sync[1], (uint32_t)nqw, spin);
        // lane mm holds row mm's parameters
        const QParams qp = qparams(
            __hip_atomic_load(&s_amax[MT == 1 ? 0 : min(lane, mt - 1)], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        const float rl = qp.ok ? qp.r : 0.0f;
        if (tid < mt) s_scale[tid] = qp.s;
#pragma unroll
        for (int gi = 0; gi < DG; ++gi) {
            const int g = tid + nq * gi;
            rm[gi] = MT == 1 ? rl : __shfl(rl, min(g / gpr, mt - 1), 64);
        }
    }
#pragma unroll
    for (int gi = 0; gi < DG; ++gi) {
        const int g = tid + nq * gi;
        uint4 qv = group_quant<XK>(xv[gi], rm[gi]);
        if (!PREQ && rm[gi] == 0.0f) qv = uint4{0u, 0u, 0u, 0u};  // zero or non-finite row
        const int row = MT == 1 ? 0 : g / gpr;
        if (g < ng) *(uint4*)(sq + row * rq_row_bytes(K) + rq_pad(16 * (g - row * gpr))) = qv;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane == 0) __hip_atomic_fetch_add(&s_sync[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// The quantising waves of k_gemv_rq with a transform (f32 tokens, DG groups
// per thread: thread t holds groups t + nq gi): the transform of k_xform_quant
// on this workgroup's copy of the row.  Wave w's groups of slot gi are the 64
// consecutive groups of 1024-element block gi nqw + w (zeros past k), so the
// sum of squares is the pairwise tree in index order: in-thread, the lanes'
// xor butterfly, then the blocks zero-padded to 16 (per-block sums exchanged in
// LDS).  XF_ADD_RMSNORM's summed row goes to a.hout from workgroup 0.  Then the
// absmax and the quantisation as in rq_quantise.  PH arrivals per wave in
// s_sync[1].
template <int XF, int DG>
__device__ __forceinline__ void rq_transform(const GemvArgs& a, const uint4 (*xv)[4], const uint4 (*x2v)[4],
                                             const uint4 (*gv)[4], int K, int gpr, int nqw, int nq, uint32_t PH,
                                             int tid, int lane, int wave, uint8_t* sq, uint32_t* s_sync,
                                             uint32_t* s_amax, float* s_scale, float* s_ss)
{
    constexpr bool XN = XF == XF_RMSNORM || XF == XF_ADD_RMSNORM;
    constexpr bool X2 = XF == XF_ADD_RMSNORM || XF == XF_SWIGLU;
    // Two groups per thread (RMSNorm only, the SwiGLU pairing): the token row
    // and the norm weight would need all 64 registers at once, so the norm
    // weight was copied into LDS (sg, after the operand row) by the kernel's
    // first instructions, ahead of every weight load of the workgroup, and is
    // read from there group by group.
    constexpr bool GL = XN && DG == 2;
    const uint4* const sg = (const uint4*)(sq + rq_row_bytes(K));
    float fv[DG][16];
#pragma unroll
    for (int gi = 0; gi < DG; ++gi) {
        const int g = tid + nq * gi;
        widen16<XK_F32>(xv[gi], fv[gi]);
        if (X2) {
            float u[16];
            widen16<XK_F32>(x2v[gi], u);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float v = fv[gi][e];
                fv[gi][e] = XF == XF_SWIGLU ? __fmul_rn(__fdiv_rn(v, __fadd_rn(1.0f, btl_expf(-v))), u[e])
                                            : __fadd_rn(v, u[e]);
            }
            if (XF == XF_ADD_RMSNORM && a.hout && blockIdx.x == 0 && g < gpr) {
                float4* hp = (float4*)(a.hout + 16 * g);
#pragma unroll
                for (int h = 0; h < 4; ++h)
                    hp[h] = make_float4(fv[gi][4 * h], fv[gi][4 * h + 1], fv[gi][4 * h + 2], fv[gi][4 * h + 3]);
            }
        }
    }
    if (XN) {
#pragma unroll
        for (int gi = 0; gi < DG; ++gi) {
            float t[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) t[e] = __fmul_rn(fv[gi][e], fv[gi][e]);
#pragma unroll
            for (int len = 16; len > 1; len >>= 1)
#pragma unroll
                for (int i = 0; i < len / 2; ++i) t[i] = __fadd_rn(t[2 * i], t[2 * i + 1]);
            const float ws = wave_pairwise_sum(t[0]);
            if (lane == 0) s_ss[gi * nqw + wave] = ws;
        }
        // GL: this wave's copies of the norm weight are in LDS (its only
        // outstanding vector-memory operations); every quantising wave's are
        // once the arrivals below are complete
        if constexpr (GL) wait_loads();
        if (lane == 0) {
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the sums are in LDS
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __hip_atomic_fetch_add(&s_sync[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        rq_wait(&s_sync[1], (uint32_t)nqw, a.spin);
        const int nblk = DG * nqw;
        float p[16];
#pragma unroll
        for (int w = 0; w < 16; ++w) p[w] = w < nblk ? s_ss[w] : 0.0f;
#pragma unroll
        for (int len = 16; len > 1; len >>= 1)
#pragma unroll
            for (int i = 0; i < len / 2; ++i) p[i] = __fadd_rn(p[2 * i], p[2 * i + 1]);
        const float inv_k = (float)(1.0 / (double)K);
        const float d = sqrt_rn(__fadd_rn(__fmul_rn(p[0], inv_k), a.eps));
#pragma unroll
        for (int gi = 0; gi < DG; ++gi) {
            float gf[16];
            if constexpr (GL) {
                const int g = min(tid + nq * gi, gpr - 1);  // past k: any group (never stored)
                uint4 gl[4];
#pragma unroll
                for (int h = 0; h < 4; ++h) gl[h] = sg[4 * g + h];
                widen16<XK_F32>(gl, gf);
            } else {
                widen16<XK_F32>(gv[gi], gf);
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) fv[gi][e] = __fmul_rn(__fdiv_rn(fv[gi][e], d), gf[e]);
        }
    }
    uint32_t am = 0;
#pragma unroll
    for (int gi = 0; gi < DG; ++gi)
        if (tid + nq * gi < gpr)
#pragma unroll
            for (int e = 0; e < 16; ++e) am = max(am, __float_as_uint(fv[gi][e]) & 0x7FFFFFFFu);
    const uint32_t v = wave_max_dpp(am);
    if (lane == 0) {
        __hip_atomic_fetch_max(&s_amax[0], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        __hip_atomic_fetch_add(&s_sync[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    rq_wait(&s_sync[1], (PH - 1u) * (uint32_t)nqw, a.spin);
    const QParams qp = qparams(__hip_atomic_load(&s_amax[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
    const float rm = qp.ok ? qp.r : 0.0f;
    if (tid == 0) s_scale[0] = qp.s;
#pragma unroll
    for (int gi = 0; gi < DG; ++gi) {
        const int g = tid + nq * gi;
        const uint4 qv = rm != 0.0f ? group_quant_f(fv[gi], rm) : uint4{0u, 0u, 0u, 0u};
        if (g < gpr) *(uint4*)(sq + rq_pad(16 * g)) = qv;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane == 0) __hip_atomic_fetch_add(&s_sync[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

template <int XK, int R, int ST, bool PAIR = false, int XF = XF_NONE, int DG = 2, int MT = 1>
__global__ __launch_bounds__(1024)
__attribute__((amdgpu_waves_per_eu(R == 4 && (XF == XF_NONE || PAIR) && !(DG == 4 && XK == XK_F32) ? 8 : 4))) void k_gemv_rq(GemvArgs a)
{
    static_assert(XF == XF_NONE || (XK == XK_F32 && R == 4 && MT == 1 && (PAIR ? XF == XF_RMSNORM && DG == 2 : DG == 1)),
                  "transforms: one f32 token row, k <= 4096; with the SwiGLU pairing RMSNorm only");
    static_assert(DG == 1 || DG == 2 || (DG == 4 && MT == 2), "one, two or (two token rows) four token groups per thread");
    static_assert(MT == 1 || (MT == 2 && !PAIR && XF == XF_NONE), "two token rows: no transform, no SwiGLU epilogue");
    constexpr bool XN = XF == XF_RMSNORM || XF == XF_ADD_RMSNORM;   // a norm over the row
    constexpr bool X2 = XF == XF_ADD_RMSNORM || XF == XF_SWIGLU;    // a second input row
    constexpr int SUB = RqShape<R>::kSub, RB = RqShape<R>::kBytes;
    constexpr int NV = DecX<XK>::kVec;
    constexpr int ES = XK == XK_F32 ? 4 : (XK == XK_BF16 ? 2 : 1);
    constexpr bool PREQ = DecX<XK>::kPreq;
    extern __shared__ __align__(16) uint8_t sq[];  // [MT][rq_row_bytes(k)], operand order, padded
    __shared__ uint32_t s_sync[3];                 // (unused), quantiser arrivals, gate arrivals
    __shared__ uint32_t s_amax[MT];                // absmax bits of each token row
    __shared__ float s_scale[MT];
    __shared__ float s_gate[PAIR ? 8 * R : 1];     // PAIR: gate outputs of the workgroup's rows
    __shared__ float s_ss[XN ? 16 : 1];            // the norm's per-wave sums of squares

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = a.k;
    const int gpr = K >> 4;                               // 16-element groups of a token row
    const int mt = MT == 1 ? 1 : a.m;
    const int nqw = rq_quant_waves(K, DG, mt);
    const int nq = nqw * 64;
    // arrivals per quantising wave: the norm's sum (XN), the absmax (unless
    // pre-quantised), the quantised row
    constexpr uint32_t PH = PREQ ? 1u : (XN ? 3u : 2u);
    const uint32_t done = PH * (uint32_t)nqw;

    // The quantising waves and the compute waves take separate paths; each
    // meets the one barrier (after which the counters are set) once.
    if (wave < nqw) {
        // the quantising waves go first in their SIMDs' issue (the compute waves
        // only poll until the row is ready; measured on MI355X, Llama-3-8B: the
        // cfg2 step 0.656 -> 0.647 ms, the decoder 1.209 -> 1.187 ms/token)
        __builtin_amdgcn_s_setprio(3);
        // 1. the token groups (and the transform's second row), issued first
        uint4 xv[DG][NV];
        uint4 x2v[X2 ? DG : 1][4];
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)(mt * K * ES));
#pragma unroll
        for (int gi = 0; gi < DG; ++gi) {
            const int g = tid + nq * gi;
#pragma unroll
            for (int h = 0; h < NV; ++h) xv[gi][h] = bload(xr, g < mt * gpr ? 16 * g * ES + 16 * h : kOOB);
        }
        uint4 gv[XN ? DG : 1][4];  // the norm weight (two groups per thread: copied into LDS)
        if constexpr (XN && DG == 2) {
            // 1 KB copies of the norm weight into LDS after the operand row,
            // spread over the quantising waves (zeros past k)
            const __amdgpu_buffer_rsrc_t gr = make_rsrc(a.g, (uint32_t)(K * 4));
            for (int c = wave; c < (K * 4 + 1023) / 1024; c += nqw)
                copy_to_lds(gr, sq + rq_row_bytes(K) + c * 1024, c * 1024 + 16 * lane);
        }
#pragma unroll
        for (int gi = 0; gi < (XF != XF_NONE && !(XN && DG == 2) ? DG : 0); ++gi) {
            const int g = tid + nq * gi;
            if (X2) {
                const __amdgpu_buffer_rsrc_t x2r = make_rsrc(a.x2, (uint32_t)(K * 4));
#pragma unroll
                for (int h = 0; h < 4; ++h) x2v[X2 ? gi : 0][h] = bload(x2r, g < gpr ? 64 * g + 16 * h : kOOB);
            }
            if (XN) {
                const __amdgpu_buffer_rsrc_t gr = make_rsrc(a.g, (uint32_t)(K * 4));
#pragma unroll
                for (int h = 0; h < 4; ++h) gv[XN ? gi : 0][h] = bload(gr, g < gpr ? 64 * g + 16 * h : kOOB);
            }
        }
        if (tid < 3) s_sync[tid] = 0u;
        if (tid < MT) s_amax[tid] = 0u;
        // the counters' initialisation is in LDS; no wait for this wave's loads
        // and copies (__syncthreads' release would wait for the norm weight's
        // LDS copies, vmcnt(0), and hold the compute waves' weight loads behind
        // them); the empty asm statements keep LDS accesses on their side, the
        // scheduling barriers the arithmetic on the loaded token after it
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        __asm__ volatile("" ::: "memory");
        if constexpr (XF != XF_NONE)
            rq_transform<XF, DG>(a, xv, x2v, gv, K, gpr, nqw, nq, PH, tid, lane, wave, sq, s_sync, s_amax, s_scale,
                                 s_ss);
        else
            rq_quantise<XK, DG, MT>(xv, K, gpr, mt, nqw, nq, tid, lane, sq, s_sync, s_amax, s_scale, a.spin);
        return;
    }
    __syncthreads();

    // 3. this compute wave's rows.  Plain: R-row group q of the launch, in
    //    16-row block q / SUB of its layer.  PAIR: the first half of the
    //    compute waves take gate's row groups cw of the workgroup's span, the
    //    second half the same rows of up.
    const int cw = wave - nqw;
    const uint8_t* W = a.p[0].w;
    void* Y = a.p[0].y;
    int32_t* ACC = a.p[0].acc_out;
    float SW = a.p[0].sw;
    int N = a.p[0].n;
    int row0, rows;
    const int half = a.parts >> 1;
    const bool isup = PAIR && cw >= half;
    const int cp = isup ? cw - half : cw;  // PAIR: row group of the workgroup's span
    if (PAIR) {
        if (isup) {
            W = a.p[1].w; Y = a.p[1].y; ACC = a.p[1].acc_out; SW = a.p[1].sw;
        }
        row0 = ((int)blockIdx.x * half + cp) * R;
        rows = __builtin_amdgcn_readfirstlane(max(0, min(R, N - row0)));
    } else {
        const int q = (int)blockIdx.x * a.parts + cw;
        const int rbg = q / SUB;
        int RB0 = a.p[0].rb_begin;
#pragma unroll
        for (int i = 1; i < kMaxGroup; ++i) {
            if (i < a.nprob && rbg >= a.p[i].rb_begin) {
                W = a.p[i].w; Y = a.p[i].y; ACC = a.p[i].acc_out;
                SW = a.p[i].sw; N = a.p[i].n; RB0 = a.p[i].rb_begin;
            }
        }
        row0 = (rbg - RB0) * 16 + (q - rbg * SUB) * R;  // past rb_total: no rows
        rows = __builtin_amdgcn_readfirstlane(rbg < a.rb_total ? max(0, min(R, N - row0)) : 0);
    }
    const int rowb = K >> 2;
    const int gq = lane >> 4, il = lane & 15;
    const int rho = il / SUB, sl = SUB * gq + (il - rho * SUB);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(W + (int64_t)max(row0, 0) * rowb, (uint32_t)(rows * rowb));
    uint4 buf[ST];
#pragma unroll
    for (int t = 0; t < ST; ++t) {
        const int b = t * RB + 16 * sl;
        buf[t] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                               wr, b < rowb ? rho * rowb + b : kOOB, 0, kCachePolicyNT));
    }
    const int r = R == 4 ? lane / 20 : lane / 40;
    const bool own = lane - (R == 4 ? 20 : 40) * r == 0;
    float rres[MT];
#pragma unroll
    for (int mm = 0; mm < MT; ++mm)
        rres[mm] = a.resid && own && r < rows && mm < mt ? a.resid[(int64_t)mm * N + row0 + r] : 0.0f;
    rq_wait(&s_sync[1], done, a.spin);

    // 4. one accumulator per token row over every load; slices past the row
    //    read the activations at k = 0 (their weights are zero), token rows
    //    past m read row 0 (never stored)
    v4i acc[MT];
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) acc[mm] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < ST; ++t) {
        const int ko = 4 * (t * RB + 16 * sl);
        const uint4 cur = buf[t];
        const uint32_t wv[4] = {cur.x, cur.y, cur.z, cur.w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const v4i aw = unpack16(wv[h]);
#pragma unroll
            for (int mm = 0; mm < MT; ++mm) {
                const uint8_t* bj = sq + (mm < mt ? mm : 0) * rq_row_bytes(K) + rq_pad(ko < K ? ko : 0);
                acc[mm] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aw, *(const v4i*)(bj + 16 * h), acc[mm], 0, 0, 0);
            }
        }
    }

    // 5. quad position 0 gathers register v of quad lane v (quad_perm
    //    broadcasts of lanes 1, 2, 3): lanes 20 rho (R = 4) hold row rho; for
    //    R = 2 lanes 40 rho add their half from lane 40 rho + 20
    int dm[MT];
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) {
        int d = acc[mm][0] + __builtin_amdgcn_update_dpp(0, acc[mm][1], 0x55, 0xF, 0xF, true);
        d += __builtin_amdgcn_update_dpp(0, acc[mm][2], 0xAA, 0xF, 0xF, true);
        d += __builtin_amdgcn_update_dpp(0, acc[mm][3], 0xFF, 0xF, 0xF, true);
        if (R == 2) d += __shfl_down(d, 20, 64);
        dm[mm] = d;
    }
    if (MT > 1) {
        if (!own || r >= rows) return;
        const int n = row0 + r;
#pragma unroll
        for (int mm = 0; mm < MT; ++mm) {
            if (mm < mt) {
                const float s_x = PREQ ? a.xs[mm] : s_scale[mm];
                const float yv = __fmul_rn((float)dm[mm], __fmul_rn(s_x, SW));
                const int64_t o = (int64_t)mm * N + n;
                if (a.ykind == YK_BF16) ((uint16_t*)Y)[o] = f32_to_bf16(yv);
                else ((float*)Y)[o] = a.resid ? __fadd_rn(rres[mm], yv) : yv;
                if (ACC) ACC[o] = dm[mm];
            }
        }
        return;
    }
    const int d = dm[0];
    const float s_l = PREQ ? a.xs[0] : s_scale[0];
    const int n = row0 + r;
    const float yv = __fmul_rn((float)d, __fmul_rn(s_l, SW));
    if (PAIR) {
        // 6. gate's waves leave their outputs in LDS; up's waves wait for every
        //    gate wave of the workgroup and write silu(gate) * up
        if (!isup) {
            if (own && r < rows) s_gate[cp * R + r] = yv;
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the LDS writes are done
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            if (lane == 0) __hip_atomic_fetch_add(&s_sync[2], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        } else {
            rq_wait(&s_sync[2], (uint32_t)half, a.spin);
        }
        if (!own || r >= rows) return;
        if (Y) {
            if (a.ykind == YK_BF16) ((uint16_t*)Y)[n] = f32_to_bf16(yv);
            else ((float*)Y)[n] = yv;
        }
        if (ACC) ACC[n] = d;
        if (isup) {
            const float gv = s_gate[cp * R + r];
            a.swiglu_out[n] = __fmul_rn(__fdiv_rn(gv, __fadd_rn(1.0f, btl_expf(-gv))), yv);
        }
        return;
    }
    if (!own || r >= rows) return;
    if (a.ykind == YK_BF16) ((uint16_t*)Y)[n] = f32_to_bf16(yv);
    else ((float*)Y)[n] = a.resid ? __fadd_rn(rres[0], yv) : yv;  // the residual add of block.rs:119,131
    if (ACC) ACC[n] = d;
}

// Loads per compute wave: ceil(k * R / 4096); R = 4 for k <= 4096 (ST 1..4),
// R = 2 above (ST 3..8, k <= 16384).  Workgroup: rq_quant_waves(k) + a.parts
// waves, at most 16.  Two token rows: two or four groups per quantising
// thread for k <= 4096, four above (the quantising waves of one row's two groups).
hipError_t launch_gemv_rq(const GemvArgs& a, int xkind, int xform, hipStream_t s)
{
    const int R = a.k <= 4096 ? 4 : 2;
    const int st = (int)(((int64_t)a.k * R + 4095) / 4096);
    const int dg = a.tiles;
    const int nqw = rq_quant_waves(a.k, dg, a.m);
    const bool pair = a.swiglu_out != nullptr;
    if ((dg != 1 && dg != 2 && dg != 4) || (dg == 1 && (R != 4 || pair)) || (dg == 4 && a.m != 2) ||
        (xform != XF_NONE && dg != (pair ? 2 : 1)))
        return hipErrorInvalidValue;
    if (a.m < 1 || a.m > 2 || (a.m > 1 && (pair || xform != XF_NONE || (dg != 4 && (R != 4 || dg != 2)))) || a.k % 64 != 0 ||
        a.k < 64 || a.k > 16384 || a.parts < 1 || nqw + a.parts > 16 || a.rb_total < 1 ||
        (xkind != XK_F32 && xkind != XK_BF16 && xkind != XK_I8 && xkind != XK_I8O))
        return hipErrorInvalidValue;
    if (a.resid && (a.ykind != YK_F32 || pair || a.nprob != 1)) return hipErrorInvalidValue;
    if (xform != XF_NONE) {
        // a transform in the quantising waves: f32 tokens, k <= 4096, the inputs
        // it reads; the summed residual (XF_ADD_RMSNORM) goes to another buffer;
        // with the SwiGLU pairing RMSNorm only, two groups per thread
        if (xkind != XK_F32 || R != 4 || (pair && (xform != XF_RMSNORM || dg != 2)) || (!pair && dg != 1) ||
            !a.x2 == (xform == XF_ADD_RMSNORM || xform == XF_SWIGLU) ||
            ((xform == XF_RMSNORM || xform == XF_ADD_RMSNORM) && !a.g) || (a.hout && (const void*)a.hout == a.x))
            return hipErrorInvalidValue;
        const int64_t groups = pair ? ((int64_t)a.p[0].n + 3) / 4 : (int64_t)a.rb_total * 4;
        const int64_t per = pair ? a.parts / 2 : a.parts;
        const dim3 grid((unsigned)((groups + per - 1) / per)), block((unsigned)((nqw + a.parts) * 64));
        // the operand row; with the pairing also the norm weight (f32, whole 1 KB copies)
        const size_t lds = (size_t)rq_row_bytes(a.k) + (pair ? ((size_t)a.k * 4 + 1023) / 1024 * 1024 : 0);
#define BTL_RQ_XF(STV)                                                                                        \
    if (pair) hipLaunchKernelGGL((k_gemv_rq<XK_F32, 4, STV, true, XF_RMSNORM, 2>), grid, block, lds, s, a);       \
    else if (xform == XF_RMSNORM) hipLaunchKernelGGL((k_gemv_rq<XK_F32, 4, STV, false, XF_RMSNORM, 1>), grid, block, lds, s, a); \
    else if (xform == XF_ADD_RMSNORM)                                                                           \
        hipLaunchKernelGGL((k_gemv_rq<XK_F32, 4, STV, false, XF_ADD_RMSNORM, 1>), grid, block, lds, s, a);      \
    else hipLaunchKernelGGL((k_gemv_rq<XK_F32, 4, STV, false, XF_SWIGLU, 1>), grid, block, lds, s, a);
        switch (st) {
        case 1: { BTL_RQ_XF(1) break; }
        case 2: { BTL_RQ_XF(2) break; }
        case 3: { BTL_RQ_XF(3) break; }
        default: { BTL_RQ_XF(4) break; }
        }
#undef BTL_RQ_XF
        return hipGetLastError();
    }
    // SwiGLU pairing: gate and up of equal n, an even number of compute waves,
    // operand-order int8 tokens (a transform ran ahead of the launch)
    if (pair && (a.nprob != 2 || a.p[0].n != a.p[1].n || (a.parts & 1) || xkind != XK_I8O))
        return hipErrorInvalidValue;
    const int64_t groups = pair ? ((int64_t)a.p[0].n + R - 1) / R : (int64_t)a.rb_total * (16 / R);
    const int64_t per = pair ? a.parts / 2 : a.parts;
    const dim3 grid((unsigned)((groups + per - 1) / per)), block((unsigned)((nqw + a.parts) * 64));
    const int mt = a.m;
    const size_t lds = (size_t)mt * rq_row_bytes(a.k);
#define BTL_RQ_DG(XKV, RV, STV)                                                                                    \
    if (RV == 4 && mt == 2 && dg == 2) hipLaunchKernelGGL((k_gemv_rq<XKV, 4, STV, false, XF_NONE, 2, 2>), grid, block, lds, s, a); \
    else if (mt == 2) hipLaunchKernelGGL((k_gemv_rq<XKV, RV, STV, false, XF_NONE, 4, 2>), grid, block, lds, s, a); \
    else if (RV == 4 && dg == 1) hipLaunchKernelGGL((k_gemv_rq<XKV, RV, STV, false, XF_NONE, 1>), grid, block, lds, s, a); \
    else hipLaunchKernelGGL((k_gemv_rq<XKV, RV, STV>), grid, block, lds, s, a);
#define BTL_RQ_XK(RV, STV)                                                                                       \
    if (pair) hipLaunchKernelGGL((k_gemv_rq<XK_I8O, RV, STV, true>), grid, block, lds, s, a);                   \
    else if (xkind == XK_BF16) { BTL_RQ_DG(XK_BF16, RV, STV) }                                                  \
    else if (xkind == XK_F32) { BTL_RQ_DG(XK_F32, RV, STV) }                                                    \
    else if (xkind == XK_I8) { BTL_RQ_DG(XK_I8, RV, STV) }                                                      \
    else { BTL_RQ_DG(XK_I8O, RV, STV) }
    if (R == 4) {
        switch (st) {
        case 1: { BTL_RQ_XK(4, 1) break; }
        case 2: { BTL_RQ_XK(4, 2) break; }
        case 3: { BTL_RQ_XK(4, 3) break; }
        default: { BTL_RQ_XK(4, 4) break; }
        }
    } else {
        switch (st) {
        case 3: { BTL_RQ_XK(2, 3) break; }
        case 4: { BTL_RQ_XK(2, 4) break; }
        case 5: { BTL_RQ_XK(2, 5) break; }
        case 6: { BTL_RQ_XK(2, 6) break; }
        case 7: { BTL_RQ_XK(2, 7) break; }
        default: { BTL_RQ_XK(2, 8) break; }
        }
    }
#undef BTL_RQ_XK
#undef BTL_RQ_DG
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// k_quant_op: per-token quantisation into MFMA operand order (prefill)
// ---------------------------------------------------------------------------
// One workgroup per token row; the arithmetic of k_quant_act, but every group
// of 16 consecutive k is stored in the operand k order [0,4,8,12, 1,5,9,13,
// ...] that unpack16 gives the weights, so the GEMM copies it to LDS as is.
template <int XK>
__global__ __launch_bounds__(256) void k_quant_op(const void* x, int k, int8_t* q, float* s)
{
    __shared__ uint32_t s_w[4];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const int groups = k >> 4;  // k % 16 == 0
    constexpr int NV = XK == XK_F32 ? 4 : 2;
    const uint4* xr = XK == XK_F32 ? (const uint4*)((const float*)x + row * k)
                                   : (const uint4*)((const uint16_t*)x + row * k);
    uint32_t amax = 0;
    for (int g = tid; g < groups; g += 256) {
        uint4 v[NV];
#pragma unroll
        for (int h = 0; h < NV; ++h) v[h] = xr[g * NV + h];
        if (XK == XK_BF16) amax = max(amax, group_absmax<XK_BF16>(v));
        else amax = max(amax, group_absmax<XK_F32>(v));
    }
    amax = wave_max_dpp(amax);
    if ((tid & 63) == 0) s_w[tid >> 6] = amax;
    __syncthreads();
    amax = max(max(s_w[0], s_w[1]), max(s_w[2], s_w[3]));
    const QParams qp = qparams(amax);
    if (tid == 0) s[row] = qp.s;
    uint4* qr = (uint4*)(q + row * k);
    for (int g = tid; g < groups; g += 256) {
        uint4 o = {0u, 0u, 0u, 0u};
        if (qp.ok) {
            uint4 v[NV];
#pragma unroll
            for (int h = 0; h < NV; ++h) v[h] = xr[g * NV + h];
            o = XK == XK_BF16 ? group_quant<XK_BF16>(v, qp.r) : group_quant<XK_F32>(v, qp.r);
        }
        qr[g] = o;
    }
}

// Single pass: one workgroup per token row (64 * ceil(k / 1024) threads, at
// most 1024) holds G 16-element groups per thread in registers (k <= 16384 G),
// so x is read once.  TR: group g of the row goes to tr_offset(row, g, tr_mtb)
// (the token-register layout of k_gemv_tr) instead of row * k + 16 g.
template <int XK, int G, bool TR = false>
__global__ __launch_bounds__(1024) void k_quant_op1(const void* x, int k, int8_t* q, float* s, int tr_mtb)
{
    __shared__ uint32_t s_w[16];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x, nt = blockDim.x;
    const int groups = k >> 4;  // k % 16 == 0
    constexpr int NV = XK == XK_F32 ? 4 : 2;
    constexpr int ES = XK == XK_F32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc((const uint8_t*)x + row * k * ES, (uint32_t)(k * ES));
    uint4 v[G][NV];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int gi = tid + nt * g;
        const int off = gi < groups ? gi * 16 * ES : kOOB;
#pragma unroll
        for (int h = 0; h < NV; ++h) v[g][h] = bload(xr, off + 16 * h);
    }
    uint32_t amax = 0;
#pragma unroll
    for (int g = 0; g < G; ++g) amax = max(amax, group_absmax<XK>(v[g]));  // zeros past k
    amax = wave_max_dpp(amax);
    if ((tid & 63) == 0) s_w[tid >> 6] = amax;
    __syncthreads();
    amax = s_w[0];
    for (int w = 1; w < (nt >> 6); ++w) amax = max(amax, s_w[w]);
    const QParams qp = qparams(amax);
    if (tid == 0) s[row] = qp.s;
    uint4* qr = (uint4*)(q + row * k);
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int gi = tid + nt * g;
        if (gi < groups) {
            const uint4 o = qp.ok ? group_quant<XK>(v[g], qp.r) : uint4{0u, 0u, 0u, 0u};
            if (TR) *(uint4*)(q + tr_offset(row, gi, tr_mtb)) = o;
            else qr[gi] = o;
        }
    }
}

hipError_t launch_quant_op(const void* x, int xkind, int64_t m, int64_t k, int8_t* q, float* s,
                           hipStream_t st, int tr_mtb)
{
    if (m <= 0) return hipSuccess;
    const int64_t groups = k >> 4;
    const dim3 grid((unsigned)m);
    const int nt = groups <= 1024 ? (int)((groups + 63) / 64 * 64) : 1024;
    if (tr_mtb) {
        // the token-register layout: single pass only (k <= 65536)
        if (m > 16 * tr_mtb || groups > 4096 || (xkind != XK_BF16 && xkind != XK_F32)) return hipErrorInvalidValue;
#define BTL_QTR(XKV, GV)                                                                                 \
    if (groups <= 1024 * GV) {                                                                           \
        hipLaunchKernelGGL((k_quant_op1<XKV, GV, true>), grid, dim3(nt), 0, st, x, (int)k, q, s, tr_mtb); \
        return hipGetLastError();                                                                        \
    }
        if (xkind == XK_BF16) {
            BTL_QTR(XK_BF16, 1) BTL_QTR(XK_BF16, 2) BTL_QTR(XK_BF16, 4)
        } else {
            BTL_QTR(XK_F32, 1) BTL_QTR(XK_F32, 2) BTL_QTR(XK_F32, 4)
        }
#undef BTL_QTR
        return hipErrorInvalidValue;
    }
#define BTL_QOP1(XKV, GV)                                                                   \
    if (groups <= 1024 * GV) {                                                              \
        hipLaunchKernelGGL((k_quant_op1<XKV, GV>), grid, dim3(nt), 0, st, x, (int)k, q, s, 0); \
        return hipGetLastError();                                                           \
    }
    if (xkind == XK_BF16) {
        BTL_QOP1(XK_BF16, 1) BTL_QOP1(XK_BF16, 2) BTL_QOP1(XK_BF16, 4)
        hipLaunchKernelGGL(k_quant_op<XK_BF16>, grid, dim3(256), 0, st, x, (int)k, q, s);
    } else {
        BTL_QOP1(XK_F32, 1) BTL_QOP1(XK_F32, 2) BTL_QOP1(XK_F32, 4)
        hipLaunchKernelGGL(k_quant_op<XK_F32>, grid, dim3(256), 0, st, x, (int)k, q, s);
    }
#undef BTL_QOP1
    return hipGetLastError();
}





// k_xform_quant: transform + operand-order quantisation of one token row per
// workgroup.  Thread t holds the G consecutive 16-element groups [tG, tG+G) in
// registers, so the sum of squares can follow the pairwise tree in index order:
// in-thread pairwise over its 16G elements, xor butterfly over the 64 lanes,
// then pairwise over the waves (zero-padded to a power of two) -- the tree the
// oracle computes over the row zero-padded to any power of two.
template <int XK, int XF, int G>
__global__ __launch_bounds__(1024) void k_xform_quant(const void* x, const void* x2, const float* g, float eps,
                                                       int k, int8_t* q, float* s, float* hout)
{
    __shared__ float s_part[16];
    __shared__ uint32_t s_w[16];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwv = blockDim.x >> 6;
    const int groups = k >> 4;
    constexpr int NV = XK == XK_F32 ? 4 : 2;
    constexpr int ES = XK == XK_F32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc((const uint8_t*)x + row * k * ES, (uint32_t)(k * ES));
    // G <= 2 (k <= 32768): every input's loads in flight at once (x, the
    // residual delta, the norm weight); G = 4 loads the latter two where they
    // are used (the registers of all three would spill)
    constexpr bool XN = XF == XF_RMSNORM || XF == XF_ADD_RMSNORM;
    constexpr bool PRE = G <= 2;
    const __amdgpu_buffer_rsrc_t dr = make_rsrc((const uint8_t*)x2 + row * k * 4, (uint32_t)(k * 4));
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(g, (uint32_t)(k * 4));
    uint4 dv[PRE && XF == XF_ADD_RMSNORM ? G : 1][4];
    uint4 gw[PRE && XN ? G : 1][4];
    auto load_row4 = [&](__amdgpu_buffer_rsrc_t r, uint4* out, int gi) {
        const int gg = tid * G + gi;
#pragma unroll
        for (int h = 0; h < 4; ++h) out[h] = bload(r, (gg < groups ? gg * 64 : kOOB) + 16 * h);
    };
    float f[G][16];
    {
        uint4 v[G][NV];
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            const int gg = tid * G + gi;
            const int off = gg < groups ? gg * 16 * ES : kOOB;
#pragma unroll
            for (int h = 0; h < NV; ++h) v[gi][h] = bload(xr, off + 16 * h);
        }
        if (PRE) {
#pragma unroll
            for (int gi = 0; gi < G; ++gi) {
                if (XF == XF_ADD_RMSNORM) load_row4(dr, dv[gi], gi);
                if (XN) load_row4(gr, gw[gi], gi);
            }
        }
#pragma unroll
        for (int gi = 0; gi < G; ++gi) widen16<XK>(v[gi], f[gi]);
    }
    if (XF == XF_SWIGLU) {
        const __amdgpu_buffer_rsrc_t ur = make_rsrc((const uint8_t*)x2 + row * k * ES, (uint32_t)(k * ES));
        uint4 v[G][NV];
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            const int gg = tid * G + gi;
            const int off = gg < groups ? gg * 16 * ES : kOOB;
#pragma unroll
            for (int h = 0; h < NV; ++h) v[gi][h] = bload(ur, off + 16 * h);
        }
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            float u[16];
            widen16<XK>(v[gi], u);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float vv = f[gi][e];
                const float si = __fdiv_rn(vv, __fadd_rn(1.0f, btl_expf(-vv)));  // silu (candle: v / (1 + exp(-v)))
                f[gi][e] = __fmul_rn(si, u[e]);
            }
        }
    }
    if (XF == XF_ADD_RMSNORM) {
        // residual connection (block.rs:119,131: residual + mixed_out), f32 + f32
        float* hr = hout ? hout + row * k : nullptr;
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            const int gg = tid * G + gi;
            float u[16];
            if constexpr (PRE) {
                widen16<XK_F32>(dv[gi], u);
            } else {
                uint4 dl[4];
                load_row4(dr, dl, gi);
                widen16<XK_F32>(dl, u);
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) f[gi][e] = __fadd_rn(f[gi][e], u[e]);
            if (hr && gg < groups) {
#pragma unroll
                for (int h = 0; h < 4; ++h)
                    *(float4*)(hr + gg * 16 + 4 * h) =
                        make_float4(f[gi][4 * h], f[gi][4 * h + 1], f[gi][4 * h + 2], f[gi][4 * h + 3]);
            }
        }
    }
    if (XF == XF_RMSNORM || XF == XF_ADD_RMSNORM) {
        // pairwise sum of squares: 16G leaves per thread (zeros past k), lanes, waves
        float t[16 * G];
#pragma unroll
        for (int gi = 0; gi < G; ++gi)
#pragma unroll
            for (int e = 0; e < 16; ++e) t[gi * 16 + e] = __fmul_rn(f[gi][e], f[gi][e]);
#pragma unroll
        for (int len = 16 * G; len > 1; len >>= 1)
#pragma unroll
            for (int i = 0; i < len / 2; ++i) t[i] = __fadd_rn(t[2 * i], t[2 * i + 1]);
        const float ws = wave_pairwise_sum(t[0]);
        if (lane == 0) s_part[wave] = ws;
        __syncthreads();
        float p[16];
#pragma unroll
        for (int w = 0; w < 16; ++w) p[w] = w < nwv ? s_part[w] : 0.0f;
#pragma unroll
        for (int len = 16; len > 1; len >>= 1)
#pragma unroll
            for (int i = 0; i < len / 2; ++i) p[i] = __fadd_rn(p[2 * i], p[2 * i + 1]);
        // rms_norm.rs:39-42 with candle's scalar ops: ss * (f32)(1/k), + eps, sqrt, x / d, * g
        const float inv_k = (float)(1.0 / (double)k);
        const float d = sqrt_rn(__fadd_rn(__fmul_rn(p[0], inv_k), eps));
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            const int gg = tid * G + gi;
            if (gg < groups) {
                float gf[16];
                if constexpr (PRE) {
                    widen16<XK_F32>(gw[gi], gf);
                } else {
                    const float4* gp = (const float4*)(g + gg * 16);
#pragma unroll
                    for (int h = 0; h < 4; ++h) {
                        const float4 gq = gp[h];
                        gf[4 * h] = gq.x; gf[4 * h + 1] = gq.y; gf[4 * h + 2] = gq.z; gf[4 * h + 3] = gq.w;
                    }
                }
#pragma unroll
                for (int e = 0; e < 16; ++e) f[gi][e] = __fmul_rn(__fdiv_rn(f[gi][e], d), gf[e]);
            }
        }
    }
    // absmax of the transformed row (bit patterns, sign cleared; zeros past k)
    uint32_t amax = 0;
#pragma unroll
    for (int gi = 0; gi < G; ++gi)
        if (tid * G + gi < groups)
#pragma unroll
            for (int e = 0; e < 16; ++e) amax = max(amax, __float_as_uint(f[gi][e]) & 0x7FFFFFFFu);
    amax = wave_max_dpp(amax);
    if (lane == 0) s_w[wave] = amax;
    __syncthreads();
    amax = s_w[0];
    for (int w = 1; w < nwv; ++w) amax = max(amax, s_w[w]);
    const QParams qp = qparams(amax);
    if (tid == 0) s[row] = qp.s;
    uint4* qr = (uint4*)(q + row * k);
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
        const int gg = tid * G + gi;
        if (gg < groups) {
            uint4 o = {0u, 0u, 0u, 0u};
            if (qp.ok) {
                int qi[16];
#pragma unroll
                for (int e = 0; e < 16; ++e) qi[e] = quant_fast(f[gi][e], qp.r);
                o.x = pack4(qi[0], qi[4], qi[8], qi[12]);
                o.y = pack4(qi[1], qi[5], qi[9], qi[13]);
                o.z = pack4(qi[2], qi[6], qi[10], qi[14]);
                o.w = pack4(qi[3], qi[7], qi[11], qi[15]);
            }
            qr[gg] = o;
        }
    }
}

hipError_t launch_xform_quant(const void* x, const void* x2, int xkind, int xform, const float* g,
                              float eps, int64_t m, int64_t k, int8_t* q, float* s, hipStream_t st, float* hout)
{
    if (xform == XF_ADD_RMSNORM && (xkind != XK_F32 || !x2)) return hipErrorInvalidValue;
    if (m <= 0) return hipSuccess;
    const int64_t groups = k >> 4;
    if (k % 64 != 0 || groups > (xform == XF_SWIGLU ? 2048 : 4096) || (xkind != XK_F32 && xkind != XK_BF16))
        return hipErrorInvalidValue;
    const int G = groups <= 1024 ? 1 : groups <= 2048 ? 2 : 4;  // groups per thread (a power of two)
    const int threads = (int)((groups / G + 63) / 64 * 64);
    const dim3 grid((unsigned)m), block((unsigned)threads);
#define BTL_XQ(XKV, XFV, GV)                                                                            \
    if (xkind == XKV && xform == XFV && G == GV) {                                                      \
        hipLaunchKernelGGL((k_xform_quant<XKV, XFV, GV>), grid, block, 0, st, x, x2, g, eps, (int)k, q, s, hout); \
        return hipGetLastError();                                                                       \
    }
#define BTL_XQ_G(XKV, XFV) BTL_XQ(XKV, XFV, 1) BTL_XQ(XKV, XFV, 2) BTL_XQ(XKV, XFV, 4)
    BTL_XQ_G(XK_BF16, XF_RMSNORM) BTL_XQ_G(XK_F32, XF_RMSNORM) BTL_XQ_G(XK_F32, XF_ADD_RMSNORM)
    BTL_XQ(XK_BF16, XF_SWIGLU, 1) BTL_XQ(XK_BF16, XF_SWIGLU, 2) BTL_XQ(XK_F32, XF_SWIGLU, 1) BTL_XQ(XK_F32, XF_SWIGLU, 2)
#undef BTL_XQ_G
#undef BTL_XQ
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// k_op_order: natural-order int8 activations -> operand order (prefill)
// ---------------------------------------------------------------------------
// Pre-quantised activations (btl_linear_i8) arrive with k in natural order;
// the GEMM's LDS tile expects every 16-k group in unpack16's order.
__global__ __launch_bounds__(256) void k_op_order(const uint4* q, uint4* out, int64_t groups)
{
    for (int64_t g = blockIdx.x * 256ll + threadIdx.x; g < groups; g += (int64_t)gridDim.x * 256)
        out[g] = transpose16(q[g]);
}

hipError_t launch_op_order(const int8_t* q, int64_t m, int64_t k, int8_t* out, hipStream_t st)
{
    const int64_t groups = m * (k >> 4);  // k % 16 == 0
    if (groups <= 0) return hipSuccess;
    const int64_t blocks = groups / 256 + 1;
    hipLaunchKernelGGL(k_op_order, dim3((unsigned)(blocks < 8192 ? blocks : 8192)), dim3(256), 0, st,
                       (const uint4*)q, (uint4*)out, groups);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// k_gemm_i8: prefill GEMM, int8 activations x packed ternary weights
// ---------------------------------------------------------------------------
// Workgroup tile 128 (tokens) x TN (output rows, 128 or 256), K steps of 128;
// 4 waves, each a 64 x 64 (TN = 128: 2 x 2 waves) or 128 x 64 (TN = 256: 1 x 4
// waves) block of v_mfma_i32_16x16x64_i8 with the activations as A and the
// weights as B (D[m][n]).  The wider tile halves the unpack VALU per MFMA (a
// wave's 4 unpacked weight words feed 8 token blocks instead of 4; the VALU
// issue, 4 cycles per wave instruction, otherwise rivals the 16 cycles of an
// MFMA) and the activation re-reads from L2 (one per 256 output rows).  A 2 x 2
// layout of 64 x 128 wave tiles (less LDS traffic, same VALU as 64 x 64) and a
// third LDS stage (occupancy 2 instead of 3-4) measured slower.
//
// Global memory is copied straight into LDS by buffer_load_dwordx4 ... lds
// (each lane's 16 bytes land at M0 + 16 * lane), so no register staging sits
// between HBM/L2 and the matrix cores.  Two LDS stages (20 or 24 KB): the
// copies of step s+1 are issued right after the barrier that opens step s and
// have the whole of step s to land.  One barrier per step.
//
// Stage layout (the lane -> global mapping of the copies produces it):
//   A [half j (k 64j..64j+63)][row 0..127][64 B]: 16-byte slot s of row r
//     holds k group s ^ ((r >> 1) & 3), so the MFMA-operand reads (16 rows x
//     4 slots per instruction) hit every bank once;
//   B [half j][column 0..TN-1][16 B]: the packed word kq of a column at byte
//     4 kq, so a read of 16 columns x 4 words covers the 64 banks once.
// Each wave unpacks the 4 weight words of its 64 columns per half step.
constexpr int kGemmBM = 128, kGemmBK = 128;  // token rows of the prefill tile, K step

template <int TN, int WGN, int NW = 4, int TM = 128, int NS = 2>
__global__ __launch_bounds__(NW * 64, 2) void k_gemm_i8(GemmArgs a)
{
    static_assert(TM == 128 || TM == 64, "token tile of 128 or 64 rows");
    static_assert(NS >= 2 && NS <= 8, "2 to 8 LDS stages");
    constexpr int ABytes = TM * kGemmBK;
    static_assert(TN == 128 || TN == 256, "tile of 128 or 256 output rows");
    static_assert(NW == 4 && (WGN == 2 || WGN == 4), "2 x 2 or 1 x 4 waves");
    constexpr int WGM = NW / WGN;              // waves along the tokens
    constexpr int TMB = TM / 16 / WGM;         // 16-token blocks per wave
    constexpr int TNB = TN / 16 / WGN;         // 16-row weight blocks per wave
    constexpr int BBytes = TN * kGemmBK / 4;
    constexpr int Stage = ABytes + BBytes;
    constexpr int ACh = ABytes / 1024 / NW;  // A copies (1 KB) per wave per step
    constexpr int BCh = BBytes / 1024 / NW;       // B copies (1 KB) per wave per step
    __shared__ __align__(1024) uint8_t lds[NS * Stage];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    // consecutive workgroups go to consecutive XCDs: with tm = bid % tiles_m
    // each XCD keeps re-reading the same activation row tiles from its L2
    const int tiles_m = (a.m + TM - 1) / TM;
    const int tm = blockIdx.x % tiles_m;
    int tn = blockIdx.x / tiles_m;
    // the layers of a group share the activations: output tiles are numbered
    // across them (layer l owns tiles tile0[l] .. tile0[l+1]-1)
    GemmLayer Lw = a.L[0];
#pragma unroll
    for (int i = 1; i < kMaxGroup; ++i)
        if (i < a.nl && tn >= a.L[i].tile0) Lw = a.L[i];
    tn -= Lw.tile0;
    const int m0 = tm * TM, n0 = tn * TN;
    const int K = a.k, N = Lw.n;
    const int rows_a = min(TM, a.m - m0), rows_b = min(TN, N - n0);
    const int split = blockIdx.y;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(a.q + (int64_t)m0 * K, (uint32_t)(rows_a * K));
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(Lw.w + (int64_t)n0 * (K >> 2), (uint32_t)(rows_b * (K >> 2)));
    const int st_begin = split * a.split_steps;
    const int st_end = min((K + kGemmBK - 1) / kGemmBK, st_begin + a.split_steps);

    // source offsets (relative to the step's first k) of this wave's copies:
    // A chunk c = 16 rows x 64 B of half j; lane -> (row, slot) as laid out above
    int aoff[ACh];
#pragma unroll
    for (int i = 0; i < ACh; ++i) {
        const int c = wave * ACh + i;
        const int j = c / (TM / 16), row = (c % (TM / 16)) * 16 + (lane >> 2);
        const int grp = (lane & 3) ^ ((row >> 1) & 3);
        aoff[i] = row * K + j * 64 + grp * 16;
    }
    // B chunk c = 64 columns x 16 B of half j: columns 64 (c % (TN / 64)) + lane
    int boff[BCh];
#pragma unroll
    for (int i = 0; i < BCh; ++i) {
        const int c = wave * BCh + i;
        boff[i] = ((c % (TN / 64)) * 64 + lane) * (K >> 2) + (c / (TN / 64)) * 16;
    }

    auto issue = [&](int st, int stage) {
        const int ko = st * kGemmBK;
        uint8_t* base = lds + stage * Stage;
#pragma unroll
        for (int i = 0; i < ACh; ++i) copy_to_lds(ra, base + (wave * ACh + i) * 1024, aoff[i] + ko);
#pragma unroll
        for (int i = 0; i < BCh; ++i) copy_to_lds(rb, base + ABytes + (wave * BCh + i) * 1024, boff[i] + (ko >> 2));
    };

    v4i acc[TMB][TNB];
#pragma unroll
    for (int b = 0; b < TMB; ++b)
#pragma unroll
        for (int c = 0; c < TNB; ++c) acc[b][c] = v4i{0, 0, 0, 0};

    const int r16 = lane & 15, kq = lane >> 4;
    // row = wm TMB 16 + 16 b + r16, so (row >> 1) & 3 == (r16 >> 1) & 3
    const int aread = (wm * TMB * 16 + r16) * 64 + ((kq ^ ((r16 >> 1) & 3)) * 16);
    const int bread = ABytes + (wn * TNB * 16 + r16) * 16 + kq * 4;
    auto compute_half = [&](const uint8_t* base, int j) {
        v4i bop[TNB];
#pragma unroll
        for (int c = 0; c < TNB; ++c) bop[c] = unpack16(*(const uint32_t*)(base + bread + j * (TN * 16) + c * 256));
        const uint8_t* ab = base + j * (TM * 64) + aread;
#pragma unroll
        for (int b = 0; b < TMB; ++b) {
            const v4i aop = *(const v4i*)(ab + b * 1024);
#pragma unroll
            for (int c = 0; c < TNB; ++c)
                acc[b][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(aop, bop[c], acc[b][c], 0, 0, 0);
        }
    };

    // every step but the last has both halves, and the loop body no branch
    // (one basic block: the scheduler can overlap a half's unpack with the
    // other half's MFMAs)
    if constexpr (NS == 2) {
        if (st_begin < st_end) issue(st_begin, 0);
        int st = st_begin;
        for (; st + 1 < st_end; ++st) {
            const int stage = (st - st_begin) & 1;
            wait_loads();     // this wave's copies of step st are in LDS
            __syncthreads();  // ... every wave's; and the other stage is no longer read
            issue(st + 1, stage ^ 1);
            const uint8_t* base = lds + stage * Stage;
            compute_half(base, 0);
            compute_half(base, 1);
        }
        if (st < st_end) {
            wait_loads();
            __syncthreads();
            const uint8_t* base = lds + ((st - st_begin) & 1) * Stage;
            compute_half(base, 0);
            if (st * kGemmBK + 64 < K) compute_half(base, 1);  // k % 128 == 64: the last step is half
        }
    } else {
        // NS stages (few workgroups per CU: more of the copies' latency to hide):
        // the copies of NS - 1 steps in flight; at step st those of st + 1 ..
        // st + NS - 2 may still be outstanding, (NS - 2) (ACh + BCh) per wave
        constexpr int CPS = ACh + BCh;
        for (int i = 0; i < NS - 1; ++i)
            if (st_begin + i < st_end) issue(st_begin + i, i);
        int st = st_begin;
        // NS steps per iteration, so every stage index is a constant (the
        // compiler then sees which copies each LDS read depends on)
        for (; st + 2 * NS - 2 < st_end; st += NS) {
#pragma unroll
            for (int i = 0; i < NS; ++i) {
                // a barrier without the workgroup fence of __syncthreads (whose
                // release waits for every outstanding copy, vmcnt(0)); the empty
                // asm statements keep the compiler from moving LDS accesses
                // across it
                __builtin_amdgcn_s_waitcnt(vmcnt_imm((NS - 2) * CPS));
                __asm__ volatile("" ::: "memory");
                __builtin_amdgcn_s_barrier();  // every wave's copies of step st + i; stage i - 1 is no longer read
                __asm__ volatile("" ::: "memory");
                issue(st + i + NS - 1, (i + NS - 1) % NS);
                const uint8_t* base = lds + i * Stage;
                compute_half(base, 0);
                compute_half(base, 1);
            }
        }
        for (; st < st_end; ++st) {  // the last steps
            const int rel = st - st_begin;
            wait_loads();
            __syncthreads();
            if (st + NS - 1 < st_end) issue(st + NS - 1, (rel + NS - 1) % NS);
            const uint8_t* base = lds + (rel % NS) * Stage;
            compute_half(base, 0);
            if (st + 1 < st_end || st * kGemmBK + 64 < K) compute_half(base, 1);
        }
    }

    if (a.splits > 1) {
        // exact int32 partial sums; k_gemm_reduce adds the splits
        const int ncols = a.L[a.nl - 1].col0 + a.L[a.nl - 1].n;
#pragma unroll
        for (int b = 0; b < TMB; ++b)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int m = m0 + wm * TMB * 16 + b * 16 + 4 * kq + v;
                if (m < a.m) {
                    int32_t* prow = a.part + ((int64_t)split * a.m + m) * ncols + Lw.col0;
#pragma unroll
                    for (int c = 0; c < TNB; ++c) {
                        const int n = n0 + wn * TNB * 16 + c * 16 + r16;
                        if (n < N) prow[n] = acc[b][c][v];
                    }
                }
            }
        return;
    }

    // epilogue: y = (float)acc * (s_x[m] * s_w).  A whole tile (the common
    // case) takes the short path: one row address per token row, no bounds
    // checks, the output kind tested once.
    const bool ybf = a.ykind == YK_BF16;
    if (m0 + TM <= a.m && n0 + TN <= N) {
        const int nb = n0 + wn * TNB * 16 + r16;
        float cmv[TMB][4];  // every token scale load in flight before the first use
#pragma unroll
        for (int b = 0; b < TMB; ++b)
#pragma unroll
            for (int v = 0; v < 4; ++v) cmv[b][v] = a.sx[m0 + wm * TMB * 16 + b * 16 + 4 * kq + v];
        const int64_t rb0 = (int64_t)(m0 + wm * TMB * 16 + 4 * kq) * N + nb;
        if (ybf) {
#pragma unroll
            for (int b = 0; b < TMB; ++b)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float cm = __fmul_rn(cmv[b][v], Lw.sw);
                    uint16_t* yr = (uint16_t*)Lw.y + rb0 + (int64_t)(b * 16 + v) * N;
#pragma unroll
                    for (int c = 0; c < TNB; ++c) yr[c * 16] = f32_to_bf16(__fmul_rn((float)acc[b][c][v], cm));
                }
        } else {
#pragma unroll
            for (int b = 0; b < TMB; ++b)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float cm = __fmul_rn(cmv[b][v], Lw.sw);
                    float* yr = (float*)Lw.y + rb0 + (int64_t)(b * 16 + v) * N;
#pragma unroll
                    for (int c = 0; c < TNB; ++c) yr[c * 16] = __fmul_rn((float)acc[b][c][v], cm);
                }
        }
        if (Lw.acc_out) {
#pragma unroll
            for (int b = 0; b < TMB; ++b)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    int32_t* ar = Lw.acc_out + rb0 + (int64_t)(b * 16 + v) * N;
#pragma unroll
                    for (int c = 0; c < TNB; ++c) ar[c * 16] = acc[b][c][v];
                }
        }
        return;
    }
#pragma unroll
    for (int b = 0; b < TMB; ++b) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int m = m0 + wm * TMB * 16 + b * 16 + 4 * kq + v;
            if (m < a.m) {
                const float cm = __fmul_rn(a.sx[m], Lw.sw);
#pragma unroll
                for (int c = 0; c < TNB; ++c) {
                    const int n = n0 + wn * TNB * 16 + c * 16 + r16;
                    if (n < N) {
                        const int64_t o = (int64_t)m * N + n;
                        const float yv = __fmul_rn((float)acc[b][c][v], cm);
                        if (ybf) ((uint16_t*)Lw.y)[o] = f32_to_bf16(yv);
                        else ((float*)Lw.y)[o] = yv;
                        if (Lw.acc_out) Lw.acc_out[o] = acc[b][c][v];
                    }
                }
            }
        }
    }
}

// k_gemm_reduce: sum the split-K partials of every output, then the epilogue
// y = (float)acc * (s_x[m] * s_w) of its layer.  One thread per output, the
// splits' loads issued 8 at a time.
__global__ __launch_bounds__(256) void k_gemm_reduce(GemmArgs a, int ncols)
{
    const int64_t total = (int64_t)a.m * ncols;
    const bool ybf = a.ykind == YK_BF16;
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int m = (int)(i / ncols), col = (int)(i - (int64_t)m * ncols);
        int32_t acc = 0;
        int sp = 0;
        for (; sp + 8 <= a.splits; sp += 8) {
            int32_t v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = a.part[(sp + u) * total + i];
#pragma unroll
            for (int u = 0; u < 8; ++u) acc += v[u];
        }
        for (; sp < a.splits; ++sp) acc += a.part[sp * total + i];
        GemmLayer Lw = a.L[0];
#pragma unroll
        for (int l = 1; l < kMaxGroup; ++l)
            if (l < a.nl && col >= a.L[l].col0) Lw = a.L[l];
        const int n = col - Lw.col0;
        const int64_t o = (int64_t)m * Lw.n + n;
        const float yv = __fmul_rn((float)acc, __fmul_rn(a.sx[m], Lw.sw));
        if (ybf) ((uint16_t*)Lw.y)[o] = f32_to_bf16(yv);
        else ((float*)Lw.y)[o] = yv;
        if (Lw.acc_out) Lw.acc_out[o] = acc;
    }
}

int gemm_splits(int64_t m, int64_t tiles_n, int64_t k, int* split_steps)
{
    const int64_t steps = (k + kGemmBK - 1) / kGemmBK;
    if (m <= 64 && tiles_n >= kGemmSmallMUnsplit && knob(KN_GEMM_TM64) != 0) {
        // 64-token tiles that already cover most CUs: no split, no partials
        if (split_steps) *split_steps = (int)steps;
        return 1;
    }
    const int64_t tiles = (m + kGemmBM - 1) / kGemmBM * tiles_n;
    int64_t s = tiles >= kGemmSplitTarget || tiles <= 0 ? 1 : (kGemmSplitTarget + tiles - 1) / tiles;
    // Above 64 token rows a split pays only for long K on few tiles: its partial
    // sums and reduce launch cost more than the idle CUs of an unsplit launch
    // (measured on MI355X, Llama-3-8B calls with their quantiser, us split /
    // unsplit: q|k|v at m = 128 29.8 / 22.4, at 512 41.7 / 25.4; gate|up at 65
    // 37.0 / 28.5; o at 65 24.0 / 25.5, at 128 29.0 / 22.0; down (k = 14336, 32
    // tiles per 128 rows) at 65 28.8 / 60.0, at 512 56.0 / 60.5, at 1024 (256
    // tiles) 85.2 / 69.1)
    if (m > 64 && (k < kGemmSplitMinK || tiles > kGemmSplitMaxTiles)) s = 1;
    const int cap = knob(KN_GEMM_MAX_SPLITS);  // tuning / tests: 1 turns split-K off
    if (cap >= 1 && s > cap) s = cap;
    if (s > steps / 2) s = steps / 2;  // at least two K steps per split
    if (s < 1) s = 1;
    const int64_t per = (steps + s - 1) / s;
    if (split_steps) *split_steps = (int)per;
    return (int)((steps + per - 1) / per);  // no empty split
}

namespace {
thread_local const char* t_gemm_form = "";
}

const char* last_gemm_form() { return t_gemm_form; }

hipError_t launch_gemm_i8(const GemmArgs& a, hipStream_t s)
{
    // Tiles of 256 output rows when there is no K split and they still give
    // every CU two workgroups at once (measured on MI355X, Llama-3-8B prefill
    // shapes); else 128.  tile0 / col0 of every layer are filled in here.
    GemmArgs g = a;
    const int64_t tiles_m = (g.m + kGemmBM - 1) / kGemmBM;
    int64_t tn256 = 0;
    for (int l = 0; l < g.nl; ++l) tn256 += (g.L[l].n + 255) / 256;
    const int64_t wide_min = knob(KN_GEMM_WIDE_MIN_TILES);
    int TN = g.splits <= 1 && tiles_m * tn256 >= wide_min ? 256 : 128;
    // BTL_GEMM_TILE forces the tile (tuning): 1 = 128 rows (2 x 2 waves), 2 =
    // 256 rows (1 x 4 waves), 3 = 128 rows (1 x 4 waves).  (A 256-row tile of 2 x 4 waves, each 64 x 64,
    // measured slower for every Llama-3-8B prefill shape: gate|up 227 against
    // 195 us.)
    const int ftile = knob(KN_GEMM_TILE);
    if (ftile == 1 || ftile == 2 || ftile == 3) TN = ftile == 2 ? 256 : 128;
    // 3: 128 rows as 1 x 4 waves of 128 tokens x 32 rows (each unpacked weight
    // word feeds 8 token blocks, as in the 256-row tile)
    const bool w14f = ftile == 3;
    // up to 64 token rows: tiles of 64 tokens (a 128-row tile would be half
    // zero-filled, its MFMAs and LDS reads half wasted), 256 rows wide when
    // split (measured on MI355X, Llama-3-8B down at m = 24..64); BTL_GEMM_TM64
    // = 0 keeps 128
    const bool tm64 = g.m <= 64 && knob(KN_GEMM_TM64) != 0;
    if (tm64 && g.splits > 1 && ftile != 1) TN = 256;
    int64_t tn = 0, cols = 0;
    for (int l = 0; l < g.nl; ++l) {
        g.L[l].tile0 = (int)tn;
        g.L[l].col0 = (int)cols;
        tn += (g.L[l].n + TN - 1) / TN;
        cols += g.L[l].n;
    }
    const int64_t tiles = tiles_m * tn;
    if (tiles <= 0) return hipSuccess;
    if (tiles > INT32_MAX || g.nl < 1 || g.nl > kMaxGroup || cols > INT32_MAX) return hipErrorInvalidValue;
    if (g.splits < 1) g.splits = 1;
    if (g.splits == 1) g.split_steps = (g.k + kGemmBK - 1) / kGemmBK;
    if (g.splits > 1 && (!g.part || g.split_steps < 1 || (int64_t)g.splits * g.m * cols > INT32_MAX))
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)tiles, (unsigned)g.splits);
    // 64-token tiles: unsplit, 4 LDS stages (one workgroup per CU has the
    // copies' latency to hide); split, 2 (a split's few K steps would run
    // mostly in the stages' tail); BTL_GEMM_TM64_STAGES = 2 or 4 forces it
    const int fns = knob(KN_GEMM_TM64_STAGES);
    const int ns = fns == 2 || fns == 4 ? fns : (g.splits > 1 ? 2 : 4);
    // 128-token tiles: 3 LDS stages when every workgroup is resident at two per
    // CU (3 stages fit two, 2 stages three): measured on MI355X, Llama-3-8B
    // M = 2048, o 37.5 -> 36.5 and down 116.2 -> 111.5 us with 3 (512
    // workgroups); q|k|v (768) 48.9 -> 51.6 and gate|up (1792) 194.6 -> 200.2 keep 2
    // The 256-row tile has no 3-stage form: its 32 accumulator blocks and a third
    // stage's addressing do not fit the 256 registers of two waves per SIMD
    // (the compiler spilled to scratch), so it takes 2 stages where the rule
    // says 3, and a forced 3 means 4.
    const int fps = knob(KN_GEMM_STAGES);
    const int64_t wgs = tiles * g.splits;
    int pns = fps == 2 || fps == 3 || (fps == 4 && TN == 256) ? fps : (g.cus > 0 && wgs <= 2 * g.cus ? 3 : 2);
    if (TN == 256 && pns == 3) pns = fps == 3 ? 4 : 2;
    // unsplit 128-row tiles resident at two per CU (3 stages) take 1 x 4 waves of
    // 128 tokens x 32 rows: each unpacked weight word feeds 8 token blocks instead
    // of 4 (measured on MI355X, Llama-3-8B M = 2048, four alternating rounds: o
    // 34.3-35.8 -> 33.5-34.2 us against 2 x 2 waves; down 102.6-109.4 -> 98.7-101.7
    // against its earlier 256-row tiles with 4 stages; q|k|v, whose 768
    // workgroups take 2 stages, measured equal and keeps 2 x 2 waves)
    const bool w14rule = ftile == 0 && TN == 128 && !tm64 && g.splits <= 1 && pns == 3;
    const bool w14 = w14f || w14rule;
    const char* form;
    if (w14 && !tm64 && pns == 3) {
        form = "k_gemm_i8<128,4,4,128,3>";
        hipLaunchKernelGGL((k_gemm_i8<128, 4, 4, 128, 3>), grid, dim3(256), 0, s, g);
    } else if (w14 && !tm64) {
        form = "k_gemm_i8<128,4,4,128,2>";
        hipLaunchKernelGGL((k_gemm_i8<128, 4>), grid, dim3(256), 0, s, g);
    } else if (TN == 256 && tm64 && ns == 4) {
        form = "k_gemm_i8<256,4,4,64,4>";
        hipLaunchKernelGGL((k_gemm_i8<256, 4, 4, 64, 4>), grid, dim3(256), 0, s, g);
    } else if (TN == 256 && tm64) {
        form = "k_gemm_i8<256,4,4,64,2>";
        hipLaunchKernelGGL((k_gemm_i8<256, 4, 4, 64>), grid, dim3(256), 0, s, g);
    } else if (TN == 256 && pns == 4) {
        form = "k_gemm_i8<256,4,4,128,4>";
        hipLaunchKernelGGL((k_gemm_i8<256, 4, 4, 128, 4>), grid, dim3(256), 0, s, g);
    } else if (TN == 256) {
        form = "k_gemm_i8<256,4,4,128,2>";
        hipLaunchKernelGGL((k_gemm_i8<256, 4>), grid, dim3(256), 0, s, g);
    } else if (tm64 && ns == 4) {
        form = "k_gemm_i8<128,2,4,64,4>";
        hipLaunchKernelGGL((k_gemm_i8<128, 2, 4, 64, 4>), grid, dim3(256), 0, s, g);
    } else if (!tm64 && pns == 3) {
        form = "k_gemm_i8<128,2,4,128,3>";
        hipLaunchKernelGGL((k_gemm_i8<128, 2, 4, 128, 3>), grid, dim3(256), 0, s, g);
    } else if (tm64) {
        form = "k_gemm_i8<128,2,4,64,2>";
        hipLaunchKernelGGL((k_gemm_i8<128, 2, 4, 64>), grid, dim3(256), 0, s, g);
    } else {
        form = "k_gemm_i8<128,2,4,128,2>";
        hipLaunchKernelGGL((k_gemm_i8<128, 2>), grid, dim3(256), 0, s, g);
    }
    t_gemm_form = form;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || g.splits == 1) return e;
    const int64_t outs = (int64_t)g.m * cols;
    const int64_t blocks = (outs + 255) / 256;
    hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)(blocks < 8192 ? blocks : 8192)), dim3(256), 0, s, g, (int)cols);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// k_gemv_bat: batched decode (5..64 token rows, or 2..4 where k_gemv_dec's
// register budget does not hold the part)
// ---------------------------------------------------------------------------
// Weight-stationary like k_gemv_dec, with the tokens pre-quantised in operand
// order (k_quant_op).  Workgroup: NW waves x one 16-row weight tile = 16 NW
// rows (a row block), over one K range of 256 ST weights (grid.y = K splits):
// the token bytes a workgroup copies per weight byte fall as 4 m / (16 NW).
// Each wave first
// copies its share of the token rows of that range into LDS (direct
// global->LDS copies), then puts all ST of its weight loads in flight, so the
// copies wait only for themselves.  The tokens are the B operand: MTB blocks of
// 16 token columns per unpacked weight word.  LDS row t holds the range's
// ks bytes of token t with 16-byte slot s stored at slot s ^ (t & 15): the 16
// lanes of a quarter-wave read 16 different token rows at one k without bank
// conflicts.  One split: the epilogue stores y; several: exact int32 partial
// sums, added by k_gemm_reduce -- or, with a.ctr (one counter per row block,
// left at zero by every launch), stored coherently (sc1) and added by the last
// split of the row block to arrive, which applies the epilogue: no second
// launch.
constexpr int kSc1 = 16;  // buffer / global cache policy: coherent at agent scope

__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int ST, int MTB, int NW>
__global__ __launch_bounds__(NW ? NW * 64 : 1024) void k_gemv_bat(GemmArgs a)
{
    const int nw = NW ? NW : a.bat_nw;  // NW = 0: the waves of a.bat_nw
    const int RBW = 16 * nw;            // rows of a row block
    extern __shared__ __align__(1024) uint8_t sx_lds[];  // [16 MTB][ks], swizzled slots
    constexpr int KS = ST * kStepWeights;                 // weights of the K range
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int split = blockIdx.y;
    int rb = blockIdx.x;
    GemmLayer Lw = a.L[0];
#pragma unroll
    for (int i = 1; i < kMaxGroup; ++i)
        if (i < a.nl && rb >= a.L[i].tile0) Lw = a.L[i];
    rb -= Lw.tile0;
    const int K = a.k, M = a.m, N = Lw.n;
    const int kb = split * KS;
    const int len = min(KS, K - kb);

    // 1. token rows [0, M) x k in [kb, kb + KS) -> LDS, 1 KB (64 slots) per copy;
    //    slots past k read zeros or the next row: their weights are zero
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.q, (uint32_t)(M * K));
    constexpr int CPR = KS / 1024;  // copies per token row
    for (int c = wave; c < M * CPR; c += nw) {
        const int t = c / CPR, slot = (c - t * CPR) * 64 + lane;
        const int src = slot ^ (t & 15);
        copy_to_lds(xr, sx_lds + c * 1024, t * K + kb + src * 16);
    }
    __asm__ volatile("" ::: "memory");  // the copies stay ahead of the weight loads

    // 2. every weight load of this wave in flight, non-temporal, in pairs: load
    //    2p + h gives lane l row 8 h + (l & 7), bytes [128 p + 16 (l >> 3), +16)
    //    of the K range -- 8 rows x 128 contiguous bytes per instruction (16
    //    rows x 64 bytes would split every 128-byte line over two instructions;
    //    measured on MI355X, a 29 MB tile stream: 6.1 against 7.1 us)
    const int kq = lane >> 4;
    const int row0 = rb * RBW + wave * 16;
    // (uniform; readfirstlane keeps the clamp, and so the descriptor, scalar)
    const int rows = __builtin_amdgcn_readfirstlane(max(0, min(16, N - row0)));
    const int rbytes = K >> 2;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(Lw.w + (int64_t)row0 * rbytes, (uint32_t)(rows * rbytes));
    static_assert(ST % 2 == 0, "loads come in pairs");
    uint4 buf[ST];
#pragma unroll
    for (int j = 0; j < ST; ++j) {
        const int kw = (j >> 1) * 512 + (lane >> 3) * 64;  // first weight of the lane's 16 bytes
        const int off = (8 * (j & 1) + (lane & 7)) * rbytes + (kb >> 2) + (kw >> 2);
        buf[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, kw < len ? off : kOOB, 0,
                                                                                 kCachePolicyNT));
    }
    __builtin_amdgcn_sched_barrier(0);  // all ST loads issue before any of them is consumed

    // 3. the copies (issued first) have landed once at most ST loads are outstanding
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(ST));
    __syncthreads();

    // 4. contraction: A = 16 weight rows (lane l: row l & 15), B = 16 token
    //    columns per block.  Pair p: lane l (b = bit 3 of l) holds its own row
    //    in load 2p + b, 16-byte chunk 2 kq + b of the 128 bytes; the chunk
    //    2 kq + 1 - b of that row sits in the other load at lane l ^ 8 (a DPP
    //    row rotation by 8).  Word w of chunk c is token slot 32 p + 4 c + w.
    v4i acc[MTB];
#pragma unroll
    for (int tb = 0; tb < MTB; ++tb) acc[tb] = v4i{0, 0, 0, 0};
    const int tsw = lane & 15;  // (t & 15) of this lane's token row
    const bool hi = (lane & 8) != 0;
    const uint8_t* brow = sx_lds + (lane & 15) * KS;
#pragma unroll
    for (int p = 0; p < ST / 2; ++p) {
        const uint32_t X[4] = {buf[2 * p].x, buf[2 * p].y, buf[2 * p].z, buf[2 * p].w};
        const uint32_t Y[4] = {buf[2 * p + 1].x, buf[2 * p + 1].y, buf[2 * p + 1].z, buf[2 * p + 1].w};
        uint32_t wd[8];  // chunk 2 kq (words 0..3), chunk 2 kq + 1 (words 4..7)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t own = hi ? Y[w] : X[w];
            const uint32_t give = hi ? X[w] : Y[w];
            const uint32_t got = (uint32_t)__builtin_amdgcn_mov_dpp((int)give, 0x128, 0xF, 0xF, false);  // row_ror:8
            wd[w] = hi ? got : own;
            wd[4 + w] = hi ? own : got;
        }
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const v4i av = unpack16(wd[w]);
            const int slot = (32 * p + 8 * kq + w) ^ tsw;
#pragma unroll
            for (int tb = 0; tb < MTB; ++tb) {
                const v4i bv = *(const v4i*)(brow + tb * 16 * KS + slot * 16);
                acc[tb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, acc[tb], 0, 0, 0);
            }
        }
    }

    // 5. D lane l element v: weight row 4 (l >> 4) + v, token column l & 15
    const int nb = row0 + 4 * kq;
    const bool ybf = a.ykind == YK_BF16;
    if (a.splits > 1) {
        const int ncols = a.L[a.nl - 1].col0 + a.L[a.nl - 1].n;
        const bool merge = a.ctr != nullptr;
#pragma unroll
        for (int tb = 0; tb < MTB; ++tb) {
            const int t = tb * 16 + (lane & 15);
            if (t < M) {
                int32_t* prow = a.part + ((int64_t)split * M + t) * ncols + Lw.col0;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    if (nb + v < N) {
                        if (merge) st_agent((uint32_t*)prow + nb + v, (uint32_t)acc[tb][v]);
                        else prow[nb + v] = acc[tb][v];
                    }
                }
            }
        }
        if (!merge) return;  // k_gemm_reduce adds them
        // the last split of this row block adds every split's partials (exact
        // int32: any order) and applies the epilogue; its counter goes back to zero
        __shared__ uint32_t s_last;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partials are stored
        __syncthreads();
        const int rbg = (int)blockIdx.x;
        if (tid == 0) {
            const uint32_t old = __hip_atomic_fetch_add(a.ctr + rbg, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const bool last = old + 1u == (uint32_t)a.splits;
            if (last) __hip_atomic_fetch_sub(a.ctr + rbg, (uint32_t)a.splits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = last ? 1u : 0u;
        }
        __syncthreads();
        if (!s_last) return;
        const int rbase = rb * RBW;
        const int64_t sstride = (int64_t)M * ncols;
        // four outputs per thread at a time, every split's load in flight
        for (int o0 = tid; o0 < M * RBW; o0 += 4 * nw * 64) {
            uint32_t pv[4][kMergeMaxSplits];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int o = o0 + nw * 64 * u;
                const int t = min(o / RBW, M - 1), n = rbase + o % RBW;
                const bool ok = o < M * RBW && n < N;
                const uint32_t* p = (const uint32_t*)a.part + (int64_t)t * ncols + Lw.col0 + (ok ? n : 0);
#pragma unroll
                for (int sp = 0; sp < kMergeMaxSplits; ++sp)
                    pv[u][sp] = ok && sp < a.splits ? ld_agent(p + sp * sstride) : 0u;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int o = o0 + nw * 64 * u;
                const int t = o / RBW, n = rbase + o % RBW;
                if (o >= M * RBW || n >= N) continue;
                int32_t sum = 0;
#pragma unroll
                for (int sp = 0; sp < kMergeMaxSplits; ++sp) sum += (int32_t)pv[u][sp];
                const float yv = __fmul_rn((float)sum, __fmul_rn(a.sx[t], Lw.sw));
                const int64_t oi = (int64_t)t * N + n;
                if (ybf) ((uint16_t*)Lw.y)[oi] = f32_to_bf16(yv);
                else ((float*)Lw.y)[oi] = yv;
                if (Lw.acc_out) Lw.acc_out[oi] = sum;
            }
        }
        return;
    }
#pragma unroll
    for (int tb = 0; tb < MTB; ++tb) {
        const int t = tb * 16 + (lane & 15);
        if (t < M) {
            const float c = __fmul_rn(a.sx[t], Lw.sw);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int n = nb + v;
                if (n < N) {
                    const int64_t o = (int64_t)t * N + n;
                    const float yv = __fmul_rn((float)acc[tb][v], c);
                    if (ybf) ((uint16_t*)Lw.y)[o] = f32_to_bf16(yv);
                    else ((float*)Lw.y)[o] = yv;
                    if (Lw.acc_out) Lw.acc_out[o] = acc[tb][v];
                }
            }
        }
    }
}

BatPlan gemv_bat_plan(int64_t m, int64_t rows, int64_t k)
{
    // LDS holds the token rows of whole 16-row blocks (16, 32 or 64 rows) x ks
    // bytes (<= 64 KB); ks shrinks from 4096 until the launch has ~448
    // workgroups.  4 waves per workgroup; above 16 token rows 8 when that keeps
    // the K range (measured on MI355X, Llama-3-8B MLP at m = 32: gate|up 23.9
    // against 25.9 us; down keeps 4 waves, with 8 its K range would halve).
    // BTL_GEMV_BAT_NW / BTL_GEMV_BAT_KS force the waves per workgroup (1..16)
    // and the K range (1024, 2048, 4096; tuning).
    const int64_t mr = m <= 16 ? 16 : m <= 32 ? 32 : 64;
    auto range = [&](int nw) {
        const int64_t blocks = (rows + 16 * nw - 1) / (16 * nw);
        int64_t ks = 4096;
        while (ks > 1024 && (mr * ks > 65536 || blocks * ((k + ks - 1) / ks) < 448)) ks >>= 1;
        return ks;
    };
    BatPlan p;
    p.nw = 4;
    int64_t ks = range(4);
    if (m > 16 && range(8) == ks) p.nw = 8;
    const int fnw = knob(KN_GEMV_BAT_NW);
    if (fnw >= 1 && fnw <= 16) {
        p.nw = fnw;
        ks = range(fnw);
    }
    const int fks = knob(KN_GEMV_BAT_KS);
    if ((fks == 1024 || fks == 2048 || fks == 4096) && mr * fks <= 65536) ks = fks;
    p.steps = (int)(ks / kStepWeights);
    p.splits = (int)((k + ks - 1) / ks);
    return p;
}

hipError_t launch_gemv_bat(const GemmArgs& a, hipStream_t s)
{
    GemmArgs g = a;
    const int nw = g.bat_nw, rbw = 16 * nw;
    int64_t rbs = 0, cols = 0;
    for (int l = 0; l < g.nl; ++l) {
        g.L[l].tile0 = (int)rbs;
        g.L[l].col0 = (int)cols;
        rbs += (g.L[l].n + rbw - 1) / rbw;
        cols += g.L[l].n;
    }
    if (rbs <= 0 || g.m <= 0) return hipSuccess;
    const int mtb = (g.m + 15) / 16;
    const int mr = mtb == 3 ? 64 : 16 * mtb;  // token rows the LDS tile spans (MTB = 1, 2, 4)
    const int st = g.split_steps;
    if (g.m > 64 || g.nl < 1 || g.nl > kMaxGroup || (st != 4 && st != 8 && st != 16) ||
        nw < 1 || nw > 16 || (int64_t)mr * st * kStepWeights > 65536 || rbs > INT32_MAX ||
        (g.ctr && (rbs > kSplitCounters || g.splits > kMergeMaxSplits)) ||
        g.splits != (g.k + st * kStepWeights - 1) / (st * kStepWeights) || (g.splits > 1 && !g.part))
        return hipErrorInvalidValue;
    const size_t lds = (size_t)mr * st * kStepWeights;
    const dim3 grid((unsigned)rbs, (unsigned)g.splits);
#define BTL_BAT(STV, MTV, NWV)                                                                   \
    if (st == STV && (NWV == 0 || nw == NWV) && (mtb == MTV || (MTV == 4 && mtb == 3))) {        \
        hipLaunchKernelGGL((k_gemv_bat<STV, MTV, NWV>), grid, dim3(nw * 64), lds, s, g);         \
    } else
#define BTL_BAT_NW(NWV) \
    BTL_BAT(4, 1, NWV) BTL_BAT(4, 2, NWV) BTL_BAT(4, 4, NWV) BTL_BAT(8, 1, NWV) BTL_BAT(8, 2, NWV) \
    BTL_BAT(8, 4, NWV) BTL_BAT(16, 1, NWV) BTL_BAT(16, 2, NWV) BTL_BAT(16, 4, NWV)
    BTL_BAT_NW(4) BTL_BAT_NW(8) BTL_BAT_NW(16) BTL_BAT_NW(0) return hipErrorInvalidValue;
#undef BTL_BAT_NW
#undef BTL_BAT
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || g.splits == 1 || g.ctr) return e;
    const int64_t outs = (int64_t)g.m * cols;
    const int64_t blocks = (outs + 255) / 256;
    hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)(blocks < 8192 ? blocks : 8192)), dim3(256), 0, s, g, (int)cols);
    return hipGetLastError();
}

static __device__ uint32_t g_split_ctr[kSplitSlots * kSplitCounters];

hipError_t split_counters(int dev, const void* ws_key, uint32_t** out)
{
    static KeySlots<kSplitSlots> slots[64];
    static std::atomic<uint32_t*> base[64];
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    uint32_t* b = base[dev].load(std::memory_order_acquire);
    if (!b) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_split_ctr));
        if (e != hipSuccess) return e;
        b = (uint32_t*)p;
        base[dev].store(b, std::memory_order_release);
    }
    const int i = slots[dev].find(ws_key);
    *out = i < 0 ? nullptr : b + (size_t)i * kSplitCounters;
    return hipSuccess;
}

// ---------------------------------------------------------------------------
// k_gemv_tr: batched decode with the token rows resident in registers
// ---------------------------------------------------------------------------
// From a few token rows on, the operand that every workgroup re-reads is the
// token block, not the weights.  Wave w of a workgroup owns one K segment of
// 512 weights and loads that segment of all 16 MTB token rows into registers
// once (8 MFMA operands per 16-token block, 32 VGPRs; the quantiser writes the
// tokens in exactly this register order, so every token load instruction reads
// 1 KB contiguously).  The weights then stream through the wave once: per
// 16-row block two non-temporal loads per lane, each 8 rows x 128 contiguous
// bytes (whole cache lines), regrouped by one DPP exchange so that lane
// 16 kq + r holds dwords 8 kq .. 8 kq + 7 of row r; each dword is unpacked once
// and feeds MTB MFMAs (v_mfma_i32_16x16x64_i8, tokens as A, weights as B, so
// that an output's 16 lanes hold 16 consecutive rows of one token).  The
// loads of row block i + PD go out while row block i computes.  The NW segment
// sums of a row block meet in LDS; one barrier per group of row blocks (all of
// them, or 4 with 64 token columns) lets the waves add them and apply the
// epilogue, so the weights never pass through LDS, the tokens are read once
// per workgroup and the waves do not wait for each other between row blocks.
// With K splits (grid.y) each split stores its exact int32 sums coherently and
// the last split of the row group to arrive adds them (a.ctr, left at zero).
//
// MFMA w of a row block contracts the 16-weight groups {8 kq + w : kq = 0..3}
// of the wave's segment: lane 16 kq + j holds token 16 tb + j's group 8 kq + w
// (A, register tok[tb][w]) and lane 16 kq + r row r's dword 8 kq + w (B).
// f(std::integral_constant<int, 0>{}) ... f(std::integral_constant<int, N - 1>{}),
// in order: a loop whose index is a constant expression in the body
template <typename F, int... Is>
__device__ __forceinline__ void static_for(F&& f, std::integer_sequence<int, Is...>)
{
    (f(std::integral_constant<int, Is>{}), ...);
}

// The fields of the layer that workgroup wg works on (GemmLayer::tile0: the
// layer's first workgroup), picked field by field with selects once per
// workgroup: an indexed or conditionally copied GemmLayer made the compiler
// copy the kernel arguments to scratch.
struct TrLayer {
    const uint8_t* w;
    void* y;
    int32_t* acc;
    float sw;
    int n, tile0, col0;
};
__device__ __forceinline__ TrLayer tr_layer(const GemmArgs& a, int wg)
{
    TrLayer r{a.L[0].w, a.L[0].y, a.L[0].acc_out, a.L[0].sw, a.L[0].n, a.L[0].tile0, a.L[0].col0};
#pragma unroll
    for (int l = 1; l < kMaxGroup; ++l) {
        const bool in = l < a.nl && wg >= a.L[l].tile0;
        r.w = in ? a.L[l].w : r.w;
        r.y = in ? a.L[l].y : r.y;
        r.acc = in ? a.L[l].acc_out : r.acc;
        r.sw = in ? a.L[l].sw : r.sw;
        r.n = in ? a.L[l].n : r.n;
        r.tile0 = in ? a.L[l].tile0 : r.tile0;
        r.col0 = in ? a.L[l].col0 : r.col0;
    }
    return r;
}

template <int MTB, int RBW, int PD>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(MTB == 1 ? 4 : 2)))
void k_gemv_tr(GemmArgs a)
{
    static_assert(MTB == 1 || MTB == 2 || MTB == 4, "16, 32 or 64 token columns");
    static_assert(PD >= 1 && PD <= RBW && RBW <= 8, "prefetch depth within the row blocks");
    extern __shared__ __align__(16) uint8_t tr_lds[];  // [nw][G][MTB][64 lanes] x 16 B
    v4i* red = (v4i*)tr_lds;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nw = blockDim.x >> 6;
    const int K = a.k, M = a.m;
    const int split = blockIdx.y;
    const int seg = split * nw + wave;  // this wave's K segment
    const int kb = seg * kTrSeg;
    const bool kact = kb < K;  // uniform; past k the wave adds zeros
    const int rbytes = K >> 2;
    // this workgroup's layer and its row blocks rb0 .. rb0 + nrb - 1 of it
    const TrLayer Lw = tr_layer(a, (int)blockIdx.x);
    const int N = Lw.n;
    const int rb0 = ((int)blockIdx.x - Lw.tile0) * a.tr_rbpw;
    const int nrb = min(a.tr_rbpw, (N + 15) / 16 - rb0);  // uniform, >= 1
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(Lw.w + (int64_t)rb0 * 16 * rbytes,
                                                kact ? (uint32_t)(min(16 * nrb, N - 16 * rb0) * rbytes) : 0u);
    // load h of row block i: lane l reads row 8 h + (l & 7) of the block, bytes
    // [16 (l >> 3), +16) of the segment's 128 bytes of that row (past k: zeros)
    const int byte = (kb >> 2) + 16 * (lane >> 3);
    const int woff = byte < rbytes ? (lane & 7) * rbytes + byte : kOOB;
    auto issue = [&](int i, uint4 (&b)[2]) __attribute__((always_inline)) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
            b[h] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 wr, woff == kOOB ? kOOB : woff + (16 * i + 8 * h) * rbytes, 0,
                                                 kCachePolicyNT));
    };

    // 1. row block 0's weights (HBM first), the token segment and scales, row
    //    blocks 1 .. PD-1
    uint4 buf[PD][2];
    issue(0, buf[0]);
    // (scheduling barriers keep the issue order: row block 0's weights first,
    // row blocks 1 .. PD-1 after the tokens and scales, so that the first row
    // block waits for neither of those)
    __builtin_amdgcn_sched_barrier(0);
    v4i tok[MTB][8];
    {
        const __amdgpu_buffer_rsrc_t tr =
            make_rsrc(a.q + (int64_t)seg * MTB * 8192, kact ? (uint32_t)(MTB * 8192) : 0u);
#pragma unroll
        for (int tb = 0; tb < MTB; ++tb)
#pragma unroll
            for (int w = 0; w < 8; ++w)
                tok[tb][w] = __builtin_bit_cast(
                    v4i, bload(tr, tb * 16 + (lane & 15) < M ? ((tb * 8 + w) * 64 + lane) * 16 : kOOB));
    }
    // the token scales of this lane's epilogue tokens (loaded once, ahead of
    // the row blocks)
    float sxv[MTB][4];
#pragma unroll
    for (int tb = 0; tb < MTB; ++tb)
#pragma unroll
        for (int v = 0; v < 4; ++v) sxv[tb][v] = a.sx[min(16 * tb + 4 * (lane >> 4) + v, M - 1)];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 1; i < PD; ++i) issue(i, buf[i]);
    __builtin_amdgcn_sched_barrier(0);

    // 2. the row blocks.  Each wave's segment sums of a row block go to LDS
    //    slot i % G right away; after every G row blocks (and the last) one
    //    barrier (without the workgroup fence, whose release would wait for
    //    every load in flight), then task (row block i, token block tb) of the
    //    group goes to wave (task % nw), which adds the nw sums and applies the
    //    epilogue.  No barrier between the row blocks of a group: each wave
    //    streams them at its own pace.
    constexpr int G = MTB == 4 ? (RBW < 4 ? RBW : 4) : RBW;  // row blocks per LDS round
    const int ncols = a.tr_cols;
    const bool hi = (lane & 8) != 0;
    const float csw = Lw.sw;
    // (every lambda inlined: with RBW = 8 the inliner otherwise kept the row
    // block body out of line, and the register arrays it captures in scratch)
    static_for([&](auto ic) __attribute__((always_inline)) {
        constexpr int i = decltype(ic)::value;
        if (i >= nrb) return;  // uniform (and so for every later row block)
        // (the compiler's waits before the first use of buf[i % PD] count every
        // vector memory operation issued since)
        const uint4 X = buf[i % PD][0], Y = buf[i % PD][1];
        const uint32_t xw[4] = {X.x, X.y, X.z, X.w}, yw[4] = {Y.x, Y.y, Y.z, Y.w};
        uint32_t wd[8];  // row (lane & 15), dwords 8 kq .. 8 kq + 7 of the segment
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t own = hi ? yw[w] : xw[w];
            const uint32_t give = hi ? xw[w] : yw[w];
            const uint32_t got = (uint32_t)__builtin_amdgcn_mov_dpp((int)give, 0x128, 0xF, 0xF, false);  // row_ror:8
            wd[w] = hi ? got : own;
            wd[4 + w] = hi ? own : got;
        }
        if (i + PD < RBW) issue(i + PD, buf[i % PD]);
        v4i acc[MTB];
#pragma unroll
        for (int tb = 0; tb < MTB; ++tb) acc[tb] = v4i{0, 0, 0, 0};
        if (kact) {
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                const v4i bv = unpack16(wd[w]);
#pragma unroll
                for (int tb = 0; tb < MTB; ++tb)
                    acc[tb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(tok[tb][w], bv, acc[tb], 0, 0, 0);
            }
        }
#pragma unroll
        for (int tb = 0; tb < MTB; ++tb) red[((wave * G + i % G) * MTB + tb) * 64 + lane] = acc[tb];
        if (i % G != G - 1 && i != nrb - 1) return;  // uniform: the group goes on
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        __asm__ volatile("" ::: "memory");
        constexpr int i0 = i - i % G;
#pragma unroll
        for (int tb = 0; tb < MTB; ++tb)
        for (int ib = 0; ib <= i - i0; ++ib) {  // row block i0 + ib
            if ((ib * MTB + tb) % nw != wave) continue;  // uniform
            // D lane l element v: token 16 tb + 4 (l >> 4) + v, row l & 15, so
            // the 16 lanes of a quarter-wave store 16 consecutive outputs
            v4i sm = red[(ib * MTB + tb) * 64 + lane];
            for (int w = 1; w < nw; ++w) sm += red[((w * G + ib) * MTB + tb) * 64 + lane];
            const int n = (rb0 + i0 + ib) * 16 + (lane & 15);
            if (n >= N) continue;
            const int t0 = 16 * tb + 4 * (lane >> 4);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int t = t0 + v;
                if (t >= M) continue;
                if (a.splits > 1) {
                    st_agent((uint32_t*)a.part + ((int64_t)split * M + t) * ncols + Lw.col0 + n, (uint32_t)sm[v]);
                } else {
                    const float yv = __fmul_rn((float)sm[v], __fmul_rn(sxv[tb][v], csw));
                    const int64_t o = (int64_t)t * N + n;
                    if (a.ykind == YK_BF16) ((uint16_t*)Lw.y)[o] = f32_to_bf16(yv);
                    else ((float*)Lw.y)[o] = yv;
                    if (Lw.acc) Lw.acc[o] = sm[v];
                }
            }
        }
        if (i + 1 < nrb) {  // uniform: the next group writes these slots again
            __builtin_amdgcn_s_waitcnt(0xC07F);
            __asm__ volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            __asm__ volatile("" ::: "memory");
        }
    }, std::make_integer_sequence<int, RBW>{});
    if (a.splits <= 1) return;

    // 3. K splits: the last split of this row group to arrive adds every
    //    split's sums (exact int32, any order) and applies the epilogue; its
    //    counter goes back to zero
    __shared__ uint32_t s_last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial sums are stored
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(a.ctr + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = old + 1u == (uint32_t)a.splits;
        if (last) __hip_atomic_fetch_sub(a.ctr + blockIdx.x, (uint32_t)a.splits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = last ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
    const int64_t sstride = (int64_t)M * ncols;
    const int per = 16 * M;  // outputs of one row block
    for (int o = tid; o < nrb * per; o += blockDim.x) {
        const int i = o / per, rem = o - i * per;
        const int t = rem >> 4;
        const int n = (rb0 + i) * 16 + (rem & 15);
        if (n >= N) continue;
        const uint32_t* p = (const uint32_t*)a.part + (int64_t)t * ncols + Lw.col0 + n;
        uint32_t pv[kMergeMaxSplits];
#pragma unroll
        for (int sp = 0; sp < kMergeMaxSplits; ++sp) pv[sp] = sp < a.splits ? ld_agent(p + sp * sstride) : 0u;
        int32_t sum = 0;
#pragma unroll
        for (int sp = 0; sp < kMergeMaxSplits; ++sp) sum += (int32_t)pv[sp];
        const float yv = __fmul_rn((float)sum, __fmul_rn(a.sx[t], csw));
        const int64_t oi = (int64_t)t * N + n;
        if (a.ykind == YK_BF16) ((uint16_t*)Lw.y)[oi] = f32_to_bf16(yv);
        else ((float*)Lw.y)[oi] = yv;
        if (Lw.acc) Lw.acc[oi] = sum;
    }
}

TrPlan gemv_tr_plan(int64_t m, int64_t row_blocks, int64_t k, int cus)
{
    // waves per CU the kernel's registers allow (MTB 2 and 4: up to 256 VGPRs,
    // two waves per SIMD; 1: at most 128, four); the row blocks spread so that
    // every CU holds as many workgroups as that allows, at most 8 row blocks each
    TrPlan p;
    p.mtb = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
    const int64_t nseg = (k + kTrSeg - 1) / kTrSeg;
    p.splits = (int)((nseg + 7) / 8);
    p.nw = (int)((nseg + p.splits - 1) / p.splits);
    const int wpc = p.mtb == 1 ? 16 : 8;
    const int64_t per_cu = wpc / p.nw > 1 ? wpc / p.nw : 1;
    const int64_t target = (int64_t)(cus > 0 ? cus : 256) * per_cu;
    int64_t rbpw = (row_blocks * p.splits + target - 1) / target;
    rbpw = rbpw < 1 ? 1 : (rbpw > 8 ? 8 : rbpw);
    const int f = knob(KN_GEMV_TR_RBPW);
    if (f >= 1 && f <= 8) rbpw = f;
    p.rbpw = (int)rbpw;
    return p;
}

hipError_t launch_gemv_tr(const GemmArgs& a, const TrPlan& p, hipStream_t s)
{
    // workgroups never cross a layer: layer l owns workgroups tile0 ..
    // tile0 + ceil(ceil(n / 16) / rbpw) - 1
    GemmArgs g = a;
    int64_t groups = 0, cols = 0, rbs = 0;
    if (p.rbpw < 1) return hipErrorInvalidValue;
    for (int l = 0; l < g.nl; ++l) {
        g.L[l].tile0 = (int)groups;
        g.L[l].col0 = (int)cols;
        const int64_t rb = (g.L[l].n + 15) / 16;
        rbs += rb;
        groups += (rb + p.rbpw - 1) / p.rbpw;
        cols += g.L[l].n;
    }
    if (rbs <= 0 || g.m <= 0) return hipSuccess;
    const int64_t nseg = ((int64_t)g.k + kTrSeg - 1) / kTrSeg;
    if (g.m > 16 * p.mtb || (p.mtb != 1 && p.mtb != 2 && p.mtb != 4) || g.nl < 1 || g.nl > kMaxGroup ||
        g.k % 64 != 0 || g.k > 65536 || p.nw < 1 || p.nw > 8 || p.rbpw < 1 || p.rbpw > 8 || p.splits < 1 ||
        p.splits > kMergeMaxSplits || (int64_t)p.splits * p.nw < nseg || (int64_t)(p.splits - 1) * p.nw >= nseg ||
        rbs > INT32_MAX || cols > INT32_MAX ||
        (p.splits > 1 && (!g.ctr || !g.part || groups > kSplitCounters)))
        return hipErrorInvalidValue;
    g.splits = p.splits;
    g.tr_rbpw = p.rbpw;
    g.tr_cols = (int)cols;
    const dim3 grid((unsigned)groups, (unsigned)p.splits), block((unsigned)(p.nw * 64));
    const int rbw = p.rbpw <= 2 ? 2 : (p.rbpw <= 4 ? 4 : 8);
    const int grp = p.mtb == 4 && rbw > 4 ? 4 : rbw;  // the kernel's G
    const size_t lds = (size_t)p.nw * grp * p.mtb * 1024;
#define BTL_TR(MTV, RBV)                                                                                     \
    if (p.mtb == MTV && rbw == RBV) {                                                                         \
        hipLaunchKernelGGL((k_gemv_tr<MTV, RBV, (MTV == 1 ? 4 : 3) < RBV ? (MTV == 1 ? 4 : 3) : RBV>), grid, \
                           block, lds, s, g);                                                                 \
        return hipGetLastError();                                                                             \
    }
    BTL_TR(1, 2) BTL_TR(1, 4) BTL_TR(1, 8) BTL_TR(2, 2) BTL_TR(2, 4) BTL_TR(2, 8) BTL_TR(4, 2) BTL_TR(4, 4)
    BTL_TR(4, 8)
#undef BTL_TR
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

// x[i .. i + 3] (i % 4 == 0; 16-byte aligned f32 or 8-byte aligned bf16 rows),
// loaded as stored (x4_raw) and widened later (x4_f32), so that a caller can
// issue several loads before it waits for any
template <int XK>
struct X4 {
    using T = typename std::conditional<XK == XK_BF16, uint2, float4>::type;
};
template <int XK>
__device__ __forceinline__ typename X4<XK>::T x4_raw(const void* x, int64_t i)
{
    if constexpr (XK == XK_BF16) return *(const uint2*)((const uint16_t*)x + i);
    else return *(const float4*)((const float*)x + i);
}
template <int XK>
__device__ __forceinline__ float4 x4_f32(typename X4<XK>::T v)
{
    if constexpr (XK == XK_BF16)
        return float4{bf16_to_f32((uint16_t)v.x), bf16_to_f32((uint16_t)(v.x >> 16)), bf16_to_f32((uint16_t)v.y),
                      bf16_to_f32((uint16_t)(v.y >> 16))};
    else return v;
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

// The same contraction for k % 64 == 0, k <= 16384 and 16-byte aligned rows:
// grid (ceil(n / 32), m), 32 outputs of one token row per workgroup, 8 lanes
// each.  The row is staged once in LDS lane-major (sx[b][j] = x[8 j + b], rows
// padded by 4 floats: the lanes' 16-byte reads hit distinct banks), so lane b
// reads its inputs 8 at a time.  The 32 weight rows stream in stages of 256
// bytes per row (1024 weights): every lane loads its own 16 bytes of a stage
// (one load of a wave = 4 rows x 256 bytes) DEPTH stages ahead into
// registers, then writes them to one of two LDS buffers, rows 272 bytes
// apart (the 8 rows a wave reads at once hit distinct banks).  Lane b's code of weight 8 j' + b, j' = 8 q + e, sits at
// bit 16 (e % 2) + 2 b of word e / 2 of the q-th 16 bytes: a rotation brings
// the pair of codes of one word to bits 8 and 24, a byte permute looks both
// up as f16 coefficients (0x3C00 = 1, 0xBC00 = -1, 0 for codes 0 and 3: the
// reference's (code & 1) - (code >> 1)), and v_fma_mix_f32 runs
// fma(x, coeff, acc) on them with the f16 coefficient widened exactly.  The
// FMA order per lane (increasing j') and the lane sum are those of k_ref_f32
// (no tail: 32 divides k).
//
// Grouped (several layers reading the same x, btl_linear_group_mode): the
// workgroups of layer i are [g.wg_begin[i], g.wg_begin[i + 1]) of the grid's x.
constexpr int kRefRows = 32;                        // outputs (weight rows) per workgroup
constexpr int kRefMaxBlocks = 4;                    // 4096-element blocks of a staged row (k <= 16384)
constexpr int kRefStageBytes = 256;                 // bytes of each row per stage
constexpr int kRefRowStride = kRefStageBytes + 16;  // LDS bytes per row
constexpr int kRefDepth = 4;                        // stages loaded ahead

// the f16 coefficients of the codes at bits rot + 8 and rot + 24 (mod 32) of wd,
// in the low and high halves
__device__ __forceinline__ uint32_t ref_coeffs(uint32_t wd, uint32_t rot)
{
    const uint32_t sel = __builtin_amdgcn_alignbit(wd, wd, rot) & 0x03000300u;
    return __builtin_amdgcn_perm(0u, 0x00BC3C00u, sel);
}
// acc = fma(xa, c.lo, acc); acc = fma(xb, c.hi, acc) (v_fma_mix_f32: about 7
// clocks a wave back to back against 4 for v_fma_f32, still cheaper than
// widening each coefficient with v_cvt_f32_f16 first)
__device__ __forceinline__ float ref_apply2(float acc, float xa, float xb, uint32_t c)
{
    acc = __builtin_fmaf(xa, (float)__builtin_bit_cast(_Float16, (uint16_t)c), acc);
    return __builtin_fmaf(xb, (float)__builtin_bit_cast(_Float16, (uint16_t)(c >> 16)), acc);
}

// 4 waves, 32 weight rows per workgroup (measured against 2 waves, and
// against two outputs per group of 8 lanes sharing x's reads: neither is
// faster).  TR token rows per workgroup (grid.y = ceil(m / TR)): every lane
// runs its chain for each of them, so a weight chunk's read and coefficient
// lookup serve TR rows.  KX: the largest k of the instantiation (x's LDS rows
// are KX / 8 + 4 floats, TR of them per lane row).
//
// XF: the transform that makes x in the staging (f32 inputs, the same bits as
// the separate launch it replaces): 0 none; 1 the residual add and RMSNorm of
// k_rmsnorm_f32 (s = h (+ delta), the sum of s*s in its pairwise tree, d =
// sqrt(sum * (f32)(1/k) + eps), x = (s / d) * g; the workgroups of grid.x 0
// store s to h_out).  Thread t then holds the 16 consecutive elements
// 16 (256 b + t) .. of every 4096-element block b, as k_rmsnorm_f32's threads
// do.  (SwiGLU's activation staged by the down projection's workgroups measured
// slower than its own launch: every workgroup recomputes the whole row's exp.)
template <int XK, int YK, int DEPTH, int KX, int TR, int XF = 0>
__global__ __launch_bounds__(256) void k_ref_f32_st(const void* x, int64_t m, int64_t k, RefGroup g, RefXf xf)
{
    static_assert(DEPTH % 2 == 0, "the LDS buffer of a stage is a constant of the unrolled loop");
    constexpr int NW = 4;
    constexpr int S = KX / 8 + 4;
    constexpr int ROWS = kRefRows;
    constexpr int STAGE = ROWS * kRefRowStride;
    constexpr int LOADS = 2;  // 16-byte loads per lane per stage (4 rows x 256 bytes each)
    static_assert(LOADS * NW * 4 == ROWS && NW * 8 == ROWS, "the loads of a stage cover its rows");
    __shared__ __align__(1024) uint8_t sw[2 * STAGE];
    __shared__ __align__(16) float sx[TR * 8 * S];
    const int K = (int)k;
    const int64_t row0 = (int64_t)blockIdx.y * TR;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    int li = 0;
#pragma unroll
    for (int i = 1; i < kMaxGroup; ++i)
        if (i < g.count && (int)blockIdx.x >= g.wg_begin[i]) li = i;
    const uint8_t* w = g.w[li];
    const int64_t n = g.n[li];
    const float scale = g.scale[li];
    void* y = g.y[li];
    const int64_t col0 = (int64_t)((int)blockIdx.x - g.wg_begin[li]) * ROWS;
    const int rb = K >> 2;  // bytes per weight row
    const int nrows = (int)min((int64_t)ROWS, n - col0);
    // rows past n read as zero (outside the descriptor) and are not stored
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(w + col0 * rb, (uint32_t)(nrows * rb));
    const int nst = (rb + kRefStageBytes - 1) / kRefStageBytes;

    // this lane's loads: rows 4 grp .. 4 grp + 3, grp = LOADS wave + i
    int loff[LOADS], lds_off[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int r = 4 * (LOADS * wave + i) + (lane >> 4);
        loff[i] = r * rb + (lane & 15) * 16;
        lds_off[i] = r * kRefRowStride + (lane & 15) * 16;
    }
    uint4 R[DEPTH][LOADS];
    // stages past the row's end load from outside the descriptor: nothing is
    // read, zeros are written and never used
    auto load = [&](int st, uint4 (&r)[LOADS]) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i)
            r[i] = bload(rs, st < nst ? loff[i] + st * kRefStageBytes : INT32_MIN);
    };
    auto put = [&](const uint4 (&r)[LOADS], int buf) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) *(uint4*)(sw + buf * STAGE + lds_off[i]) = r[i];
    };
    // x's loads first (4 elements per load), then the weights' first stages,
    // then x's LDS writes: they wait for x's loads only.  The stages then
    // stand as at the top of every later iteration: R[1 .. DEPTH - 1] hold
    // stages 1 .. DEPTH - 1, R[0] stage DEPTH, LDS buffer 0 stage 0.
    // (a token row past m is not loaded: its lanes' sums are not stored)
    if constexpr (XF == 0) {
        constexpr int XL = KX / (4 * NW * 64);  // x loads per thread and token row
        typename X4<XK>::T xv[TR][XL];
        const int kv = K >> 2;
#pragma unroll
        for (int r = 0; r < TR; ++r)
#pragma unroll
            for (int j = 0; j < XL; ++j) {
                const int t = tid + NW * 64 * j;
                if (t < kv && row0 + r < m) xv[r][j] = x4_raw<XK>(x, (row0 + r) * k + 4 * t);
            }
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) load(d, R[d]);
#pragma unroll
        for (int r = 0; r < TR; ++r)
#pragma unroll
            for (int j = 0; j < XL; ++j) {
                const int t = tid + NW * 64 * j;
                if (t < kv && row0 + r < m) {
                    // elements 4 t .. 4 t + 3: lane rows (4 t) & 7 .. + 3, column t / 2
                    float* d = sx + (r * 8 + ((4 * t) & 7)) * S + (t >> 1);
                    const float4 v = x4_f32<XK>(xv[r][j]);
                    d[0] = v.x;
                    d[S] = v.y;
                    d[2 * S] = v.z;
                    d[3 * S] = v.w;
                }
            }
    } else {
        constexpr int NB = KX / 4096;  // 4096-element blocks
        static_assert(NB * 4096 == KX && NB <= kRefMaxBlocks, "KX is a multiple of 4096");
        float v[TR][NB][16];
#pragma unroll
        for (int r = 0; r < TR; ++r)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int e0 = 16 * (256 * b + tid);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    if (row0 + r < m && e0 + 4 * q < K) {
                        const int64_t e = (row0 + r) * k + e0 + 4 * q;
                        a = *(const float4*)(xf.a + e);
                        if (xf.b) {
                            const float4 c = *(const float4*)(xf.b + e);
                            a = make_float4(__fadd_rn(a.x, c.x), __fadd_rn(a.y, c.y), __fadd_rn(a.z, c.z),
                                            __fadd_rn(a.w, c.w));
                        }
                    }
                    v[r][b][4 * q] = a.x;
                    v[r][b][4 * q + 1] = a.y;
                    v[r][b][4 * q + 2] = a.z;
                    v[r][b][4 * q + 3] = a.w;
                }
            }
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) load(d, R[d]);
        {
            __shared__ float s_w[TR][4];
            __shared__ float s_blk[TR][kRefMaxBlocks];
            __shared__ float s_d[TR];
            const int nblk = (K + 4095) >> 12;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (b < nblk) {  // uniform
#pragma unroll
                    for (int r = 0; r < TR; ++r) {
                        float sq[16];
#pragma unroll
                        for (int e = 0; e < 16; ++e) sq[e] = __fmul_rn(v[r][b][e], v[r][b][e]);
#pragma unroll
                        for (int len = 16; len > 1; len >>= 1)
#pragma unroll
                            for (int i = 0; i < len / 2; ++i) sq[i] = __fadd_rn(sq[2 * i], sq[2 * i + 1]);
                        const float ws = wave_pairwise_sum(sq[0]);
                        if (lane == 0) s_w[r][wave] = ws;
                    }
                    __syncthreads();
                    if (tid < TR)
                        s_blk[tid][b] = __fadd_rn(__fadd_rn(s_w[tid][0], s_w[tid][1]), __fadd_rn(s_w[tid][2], s_w[tid][3]));
                    __syncthreads();
                }
            }
            if (tid < TR) {
                float p[kRefMaxBlocks];
#pragma unroll
                for (int b = 0; b < kRefMaxBlocks; ++b) p[b] = b < nblk ? s_blk[tid][b] : 0.0f;
#pragma unroll
                for (int len = kRefMaxBlocks; len > 1; len >>= 1)
#pragma unroll
                    for (int i = 0; i < len / 2; ++i) p[i] = __fadd_rn(p[2 * i], p[2 * i + 1]);
                const float inv_k = (float)(1.0 / (double)K);
                s_d[tid] = sqrt_rn(__fadd_rn(__fmul_rn(p[0], inv_k), xf.eps));
            }
            __syncthreads();
#pragma unroll
            for (int r = 0; r < TR; ++r) {
                const float dr = s_d[r];
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const int e0 = 16 * (256 * b + tid);
                    if (row0 + r < m && e0 < K) {
                        const int64_t e = (row0 + r) * k + e0;
                        if (xf.h_out && blockIdx.x == 0) {
#pragma unroll
                            for (int q = 0; q < 4; ++q)
                                *(float4*)(xf.h_out + e + 4 * q) = make_float4(
                                    v[r][b][4 * q], v[r][b][4 * q + 1], v[r][b][4 * q + 2], v[r][b][4 * q + 3]);
                        }
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const float4 gv = *(const float4*)(xf.g + e0 + 4 * q);
                            v[r][b][4 * q] = __fmul_rn(__fdiv_rn(v[r][b][4 * q], dr), gv.x);
                            v[r][b][4 * q + 1] = __fmul_rn(__fdiv_rn(v[r][b][4 * q + 1], dr), gv.y);
                            v[r][b][4 * q + 2] = __fmul_rn(__fdiv_rn(v[r][b][4 * q + 2], dr), gv.z);
                            v[r][b][4 * q + 3] = __fmul_rn(__fdiv_rn(v[r][b][4 * q + 3], dr), gv.w);
                        }
                    }
                }
            }
        }
        // x into LDS lane-major: element e at lane row e & 7, column e / 8
#pragma unroll
        for (int r = 0; r < TR; ++r)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int e0 = 16 * (256 * b + tid);
                if (row0 + r < m && e0 < K) {
                    float* d = sx + r * 8 * S + (e0 >> 3);
#pragma unroll
                    for (int e = 0; e < 16; ++e) d[(e & 7) * S + (e >> 3)] = v[r][b][e];
                }
            }
    }
    put(R[0], 0);
    load(DEPTH, R[0]);
    __syncthreads();  // x and stage 0 staged

    // output o, chain b
    const int o = wave * 8 + (lane >> 3), b = lane & 7;
    const uint32_t rot = (uint32_t)(2 * b + 24) & 31u;
    const float* xb = sx + b * S;
    const int wrd = o * kRefRowStride;
    float acc[TR];
#pragma unroll
    for (int r = 0; r < TR; ++r) acc[r] = 0.0f;
    // one 16-byte chunk of row o (64 weights) and the 8 inputs of chain b it
    // multiplies in each token row
    struct Chunk {
        uint4 w;
        float4 x0[TR], x1[TR];
    };
    auto rd = [&](const uint8_t* wq, const float* xq) {
        Chunk c;
        c.w = *(const uint4*)wq;
#pragma unroll
        for (int r = 0; r < TR; ++r) {
            c.x0[r] = *(const float4*)(xq + r * 8 * S);
            c.x1[r] = *(const float4*)(xq + r * 8 * S + 4);
        }
        return c;
    };
    auto fma8 = [&](const Chunk& c) {
        const uint32_t c0 = ref_coeffs(c.w.x, rot), c1 = ref_coeffs(c.w.y, rot);
        const uint32_t c2 = ref_coeffs(c.w.z, rot), c3 = ref_coeffs(c.w.w, rot);
#pragma unroll
        for (int r = 0; r < TR; ++r) {
            acc[r] = ref_apply2(acc[r], c.x0[r].x, c.x0[r].y, c0);
            acc[r] = ref_apply2(acc[r], c.x0[r].z, c.x0[r].w, c1);
            acc[r] = ref_apply2(acc[r], c.x1[r].x, c.x1[r].y, c2);
            acc[r] = ref_apply2(acc[r], c.x1[r].z, c.x1[r].w, c3);
        }
    };
    auto compute = [&](const uint8_t* stage, int st) {
        const int nq = min(16, (rb - st * kRefStageBytes) >> 4);
        const uint8_t* wq = stage + wrd;
        const float* xs = xb + st * 128;
        if (nq == 16) {  // uniform
            // the LDS reads of chunk q + 2 are issued before chunk q's FMAs
            // (one wave per SIMD is common here: nothing else hides their latency)
            Chunk cb[3];
            cb[0] = rd(wq, xs);
            cb[1] = rd(wq + 16, xs + 8);
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                if (q + 2 < 16) cb[(q + 2) % 3] = rd(wq + 16 * (q + 2), xs + 8 * (q + 2));
                __builtin_amdgcn_sched_barrier(0);
                fma8(cb[q % 3]);
            }
        } else {
            for (int q = 0; q < nq; ++q) fma8(rd(wq + 16 * q, xs + 8 * q));
        }
    };
    // DEPTH stages per iteration: every register set and LDS buffer index is
    // a constant.  Stage s sits in R[s % DEPTH] until it is written to LDS
    // buffer s % 2, one stage ahead of the compute.  The stages past nst of
    // the last iteration compute nothing (nq <= 0); they are not skipped by a
    // branch out of the loop, whose paths would make the compiler wait for
    // every outstanding load at the top of the loop.
    for (int st0 = 0; st0 < nst; st0 += DEPTH) {
#pragma unroll
        for (int i = 0; i < DEPTH; ++i) {
            const int st = st0 + i;
            if (st > 0) __syncthreads();  // stage st written; stage st - 1 no longer read
            put(R[(i + 1) % DEPTH], (i + 1) & 1);
            load(st + 1 + DEPTH, R[(i + 1) % DEPTH]);
            compute(sw + (i & 1) * STAGE, st);
        }
    }
#pragma unroll
    for (int t = 0; t < TR; ++t) {
        float lanes[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) lanes[i] = __shfl(acc[t], i, 8);
        if (o < nrows && b == 0 && row0 + t < m) {
            float r = -0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) r = __fadd_rn(r, lanes[i]);
            const float sum = __fadd_rn(0.0f, r);
            store_y<YK>(y, (row0 + t) * n + col0 + o, __fmul_rn(sum, scale));
        }
    }
}

// the staged kernel's launch; the transform (xf 1) exists for f32 inputs only
template <int XK, int YK, int KX, int TR>
static void launch_ref_st(dim3 grid, hipStream_t st, const void* x, int64_t m, int64_t k, const RefGroup& g,
                          const RefXf& tx, int xf)
{
    if constexpr (XK == XK_F32) {
        if (xf == 1) {
            hipLaunchKernelGGL((k_ref_f32_st<XK, YK, kRefDepth, KX, TR, 1>), grid, dim3(256), 0, st, x, m, k, g, tx);
            return;
        }
    }
    hipLaunchKernelGGL((k_ref_f32_st<XK, YK, kRefDepth, KX, TR>), grid, dim3(256), 0, st, x, m, k, g, tx);
}

hipError_t launch_ref_f32_group(const void* x, int xkind, int64_t m, int64_t k, const uint8_t* const* w,
                                const int64_t* n, const float* scale, void* const* y, int count, int ykind,
                                hipStream_t st, int xf, const RefXf* t)
{
    if (count < 1 || count > kMaxGroup) return hipErrorInvalidValue;
    // a transform runs only in the staged form, on f32 rows the caller checked
    // (k % 64 == 0, k <= 16384, 16-byte aligned)
    if (xf != 0 && (!t || xkind != XK_F32 || k % 64 != 0 || k > 16384 || m > 65535)) return hipErrorInvalidValue;
    bool lds_ok = k % 64 == 0 && k <= 16384 && m <= 65535 && (xf != 0 || ((uintptr_t)x & 15u) == 0);
    int64_t n_total = 0;
    for (int i = 0; i < count; ++i) {
        lds_ok = lds_ok && ((uintptr_t)w[i] & 15u) == 0;
        n_total += n[i];
    }
    if (m <= 0 || n_total == 0) return hipSuccess;
    const int rows = kRefRows;
    if (xf != 0 && (!lds_ok || n_total / rows + count > INT32_MAX)) return hipErrorInvalidValue;
    if (!lds_ok || n_total / rows + count > INT32_MAX) {
        for (int i = 0; i < count; ++i) {
            const hipError_t e = launch_ref_f32(x, xkind, m, k, w[i], n[i], scale[i], y[i], ykind, st);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    RefGroup g{};
    g.count = count;
    int b = 0;
    for (int i = 0; i < count; ++i) {
        g.w[i] = w[i];
        g.y[i] = y[i];
        g.scale[i] = scale[i];
        g.n[i] = n[i];
        g.wg_begin[i] = b;
        b += (int)((n[i] + rows - 1) / rows);
    }
    g.wg_begin[count] = b;
    // two token rows per workgroup from m = 2 on (the weight chunk's read and
    // coefficient lookup shared; x of both rows in LDS: at most 2 x 64 KB)
    const int tr = m >= 2 ? 2 : 1;
    const dim3 grid((unsigned)b, (unsigned)((m + tr - 1) / tr));
    const RefXf tx = t ? *t : RefXf{};
#define BTL_REF_ST(XKV, YKV, KXV)                                                          \
    if (tr == 2) launch_ref_st<XKV, YKV, KXV, 2>(grid, st, x, m, k, g, tx, xf);              \
    else launch_ref_st<XKV, YKV, KXV, 1>(grid, st, x, m, k, g, tx, xf);                      \
    return hipGetLastError();
#define BTL_REF_LDS(XKV, YKV)                              \
    if (xkind == XKV && ykind == YKV) {                    \
        if (k <= 4096) { BTL_REF_ST(XKV, YKV, 4096) }      \
        if (k <= 8192) { BTL_REF_ST(XKV, YKV, 8192) }      \
        BTL_REF_ST(XKV, YKV, 16384)                        \
    }
    BTL_REF_LDS(XK_F32, YK_F32)
    BTL_REF_LDS(XK_F32, YK_BF16)
    BTL_REF_LDS(XK_BF16, YK_F32)
    BTL_REF_LDS(XK_BF16, YK_BF16)
#undef BTL_REF_LDS
#undef BTL_REF_ST
    return hipErrorInvalidValue;
}

hipError_t launch_ref_f32(const void* x, int xkind, int64_t m, int64_t k, const uint8_t* w,
                          int64_t n, float scale, void* y, int ykind, hipStream_t st)
{
    const int64_t threads = m * n * 8;
    if (threads <= 0) return hipSuccess;
    if (k % 64 == 0 && k <= 16384 && ((uintptr_t)w & 15u) == 0 && ((uintptr_t)x & 15u) == 0 && m <= 65535 &&
        (n + 31) / 32 <= INT32_MAX)
        return launch_ref_f32_group(x, xkind, m, k, &w, &n, &scale, &y, 1, ykind, st);
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
// k_ref_seq: the reference's contraction on a host without AVX2/FMA
// ---------------------------------------------------------------------------
// cpu.rs:62-66 leaves the vector loop out, so the scalar loop of
// cpu.rs:105-122 covers every input: sum = +0.0f, then sum = sum + x[l] *
// coeff(l) in increasing l, the product and the sum each rounded to f32, and
// y = sum * scale (cpu.rs:123).  coeff is 0, 1 or -1, so the product is exact
// (x, -x, a signed zero, or NaN for an infinite or NaN x) and fma(x, coeff,
// sum) rounds once to the same value as the two operations (sum is never -0:
// it starts at +0 and a round-to-nearest add only gives -0 from two -0s).
// The chain cannot be split without changing the bits, so one thread owns one
// output: grid (ceil(n / 256), min(m, 65535)), a thread per weight row of one
// token row (rows past grid.y by a loop).  VEC (k % 64 == 0, w and x 16-byte
// aligned, the row's x under 2 GiB): each thread streams its weight row, 64
// weights per 16-byte load, and the token's 64 inputs of a block through a
// buffer descriptor (the same address in every lane, in-order vector loads),
// both one block ahead; the coefficients of a word's codes j and j + 8 are
// looked up together as f16 (ref_coeffs) and applied by v_fma_mix_f32.  Else
// one byte per 4 weights and plain loads.
template <int XK>
struct SeqX {
    static constexpr int ES = XK == XK_BF16 ? 2 : 4;  // bytes per input
    static constexpr int L = 4 * ES;                  // 16-byte loads per 64 inputs
};

// input j (a constant after unrolling) of a block held as loaded
template <int XK>
__device__ __forceinline__ float seq_elem(const uint4 (&r)[SeqX<XK>::L], int j)
{
    if (XK == XK_BF16) {
        const uint4 v = r[j >> 3];
        const int h = (j & 7) >> 1;
        const uint32_t wd = h == 0 ? v.x : (h == 1 ? v.y : (h == 2 ? v.z : v.w));
        return __uint_as_float((j & 1) ? (wd & 0xFFFF0000u) : (wd << 16));
    }
    const uint4 v = r[j >> 2];
    const int h = j & 3;
    return __uint_as_float(h == 0 ? v.x : (h == 1 ? v.y : (h == 2 ? v.z : v.w)));
}

template <int XK, int YK, bool VEC>
__global__ __launch_bounds__(256) void k_ref_seq(const void* __restrict__ x, int64_t m, int64_t k,
                                                 const uint8_t* __restrict__ w, int64_t n, float scale,
                                                 void* __restrict__ y)
{
    constexpr int ES = SeqX<XK>::ES, XL = SeqX<XK>::L;
    const int64_t col = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool active = col < n;
    const uint8_t* wr = w + (active ? col : 0) * (k >> 2);
    for (int64_t row = blockIdx.y; row < m; row += gridDim.y) {
        const int64_t xb = row * k;
        float sum = 0.0f;
        if (VEC) {
            // offsets past the row read as zero (the last block's look-ahead)
            const __amdgpu_buffer_rsrc_t xr = make_rsrc((const uint8_t*)x + xb * ES, (uint32_t)(k * ES));
            // one block: the chain over its 64 inputs (xc, weights qc) while the
            // next block's loads (xn, qn) are in flight
            auto block = [&](int64_t l, const uint4(&xc)[XL], uint4(&xn)[XL], const uint4& qc, uint4& qn) {
                if (l + 64 < k) qn = *(const uint4*)(wr + ((l + 64) >> 2));
#pragma unroll
                for (int i = 0; i < XL; ++i) xn[i] = bload(xr, (int)((l + 64) * ES) + 16 * i);
#pragma unroll
                for (int wi = 0; wi < 4; ++wi) {
                    const uint32_t wd = wi == 0 ? qc.x : (wi == 1 ? qc.y : (wi == 2 ? qc.z : qc.w));
                    uint32_t c[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) c[j] = ref_coeffs(wd, (uint32_t)((2 * j + 24) & 31));
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        const uint16_t h = j < 8 ? (uint16_t)c[j] : (uint16_t)(c[j - 8] >> 16);
                        sum = __builtin_fmaf(seq_elem<XK>(xc, 16 * wi + j), (float)__builtin_bit_cast(_Float16, h),
                                             sum);
                    }
                }
            };
            uint4 qa = make_uint4(0, 0, 0, 0), qb = qa, xa[XL], xbuf[XL];
            if (k > 0) qa = *(const uint4*)wr;
#pragma unroll
            for (int i = 0; i < XL; ++i) xa[i] = bload(xr, 16 * i);
            for (int64_t l = 0; l < k; l += 128) {  // two blocks, buffers alternating
                block(l, xa, xbuf, qa, qb);
                if (l + 64 < k) block(l + 64, xbuf, xa, qb, qa);
            }
        } else {
            for (int64_t l = 0; l < k; l += 4) {
                const uint32_t b = wr[l >> 2];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int code = (int)((b >> (2 * j)) & 3u);
                    const float coeff = (float)((code & 1) - (code >> 1));
                    sum = __fadd_rn(sum, __fmul_rn(load_x<XK>(x, xb + l + j), coeff));
                }
            }
        }
        if (active) store_y<YK>(y, row * n + col, __fmul_rn(sum, scale));
    }
}

hipError_t launch_ref_seq(const void* x, int xkind, int64_t m, int64_t k, const uint8_t* w, int64_t n,
                          float scale, void* y, int ykind, hipStream_t st)
{
    if (m <= 0 || n <= 0) return hipSuccess;
    if ((n + 255) / 256 > INT32_MAX) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((n + 255) / 256), (unsigned)(m < 65535 ? m : 65535));
    const bool vec = k % 64 == 0 && ((uintptr_t)w & 15u) == 0 && ((uintptr_t)x & 15u) == 0 && k * 4 <= INT32_MAX - 1024;
#define BTL_SEQ_CASE(XKV, YKV)                                                                             \
    if (xkind == XKV && ykind == YKV) {                                                                    \
        if (vec) hipLaunchKernelGGL((k_ref_seq<XKV, YKV, true>), grid, dim3(256), 0, st, x, m, k, w, n, scale, y); \
        else hipLaunchKernelGGL((k_ref_seq<XKV, YKV, false>), grid, dim3(256), 0, st, x, m, k, w, n, scale, y);   \
        return hipGetLastError();                                                                          \
    }
    BTL_SEQ_CASE(XK_F32, YK_F32)
    BTL_SEQ_CASE(XK_F32, YK_BF16)
    BTL_SEQ_CASE(XK_BF16, YK_F32)
    BTL_SEQ_CASE(XK_BF16, YK_BF16)
#undef BTL_SEQ_CASE
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
// k_abs_sum / k_pack_codes: PackedTensor::pack on the device
// ---------------------------------------------------------------------------
// The mean of |w| is the pairwise tree in double over the elements in index
// order (zero-padded to a power of two) -- the order btl_pack_host and the CPU
// oracle use, so the scale is bit-identical.  A workgroup sums an aligned block
// of 4096 elements: wave w the 1024 at 1024w, its load j the 256 at 1024w+256j,
// lane l the 4 at 4l of those (one coalesced 16-byte load).  The lane's 4 are
// an aligned subtree; the xor butterfly over the 64 lanes is the pairwise tree
// of the 256; then (j0+j1)+(j2+j3) per wave and (w0+w1)+(w2+w3) per block.
// Level 0 reads |w| (f32), later levels the block sums of the level below
// (doubles), 4096 at a time until one is left -- each block an aligned subtree.
template <int LEVEL0>
__global__ __launch_bounds__(256) void k_abs_sum(const void* in, int64_t n, double* out)
{
    __shared__ double s_part[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t base = blockIdx.x * 4096ll + wave * 1024 + lane * 4;
    double s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t idx = base + 256 * j;
        double v0 = 0.0, v1 = 0.0, v2 = 0.0, v3 = 0.0;
        if (LEVEL0) {
            const float* f = (const float*)in;
            if (idx + 4 <= n) {
                const float4 q = *(const float4*)(f + idx);  // f 16-byte aligned, idx % 4 == 0
                v0 = fabs((double)q.x); v1 = fabs((double)q.y); v2 = fabs((double)q.z); v3 = fabs((double)q.w);
            } else {
                if (idx < n) v0 = fabs((double)f[idx]);
                if (idx + 1 < n) v1 = fabs((double)f[idx + 1]);
                if (idx + 2 < n) v2 = fabs((double)f[idx + 2]);
            }
        } else {
            const double* d = (const double*)in;
            if (idx < n) v0 = d[idx];
            if (idx + 1 < n) v1 = d[idx + 1];
            if (idx + 2 < n) v2 = d[idx + 2];
            if (idx + 3 < n) v3 = d[idx + 3];
        }
        s[j] = __dadd_rn(__dadd_rn(v0, v1), __dadd_rn(v2, v3));
    }
#pragma unroll
    for (int sh = 1; sh < 64; sh <<= 1)
#pragma unroll
        for (int j = 0; j < 4; ++j) s[j] = __dadd_rn(s[j], __shfl_xor(s[j], sh, 64));
    if (lane == 0) s_part[wave] = __dadd_rn(__dadd_rn(s[0], s[1]), __dadd_rn(s[2], s[3]));
    __syncthreads();
    if (tid == 0) out[blockIdx.x] = __dadd_rn(__dadd_rn(s_part[0], s_part[1]), __dadd_rn(s_part[2], s_part[3]));
}

// scale = (f32)(sum / numel) + 1e-6, y = w * (f32)(1 / (double)scale); code 1 if
// round_half_away(y) clamped to [-1, 1] is 1 (y >= 0.5), 2 if it is -1
// (y <= -0.5), else 0 (packing.rs:56-92).  One packed byte = 4 elements = one
// 16-byte load; a workgroup covers 1024 bytes per pass (4 per thread, lanes
// on consecutive bytes), grid-stride over the tensor.
__device__ __forceinline__ uint32_t pack_code(float x, float inv)
{
    const float y = __fmul_rn(x, inv);
    return y >= 0.5f ? 1u : (y <= -0.5f ? 2u : 0u);
}

__global__ __launch_bounds__(256) void k_pack_codes(const float* w, int64_t numel, const double* total,
                                                     uint8_t* out, float* scale_out)
{
    const double acc = *total;
    const float mean = numel ? (float)(acc / (double)numel) : 0.0f;
    const float sc = __fadd_rn(mean, 1e-6f);
    const float inv = (float)(1.0 / (double)sc);
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = sc;
    const int64_t nbytes = (numel + 3) / 4;
    for (int64_t b0 = blockIdx.x * 1024ll; b0 < nbytes; b0 += (int64_t)gridDim.x * 1024) {
        float4 v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t b = b0 + 256 * j + threadIdx.x, e = 4 * b;
            v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (e + 4 <= numel) {
                v[j] = *(const float4*)(w + e);  // w 16-byte aligned
            } else if (e < numel) {
                v[j].x = w[e];
                if (e + 1 < numel) v[j].y = w[e + 1];
                if (e + 2 < numel) v[j].z = w[e + 2];
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t b = b0 + 256 * j + threadIdx.x;
            if (b < nbytes)
                out[b] = (uint8_t)(pack_code(v[j].x, inv) | pack_code(v[j].y, inv) << 2 |
                                   pack_code(v[j].z, inv) << 4 | pack_code(v[j].w, inv) << 6);
        }
    }
}

int64_t pack_partials(int64_t numel)
{
    int64_t total = 0;
    for (int64_t n = numel; ; ) {
        const int64_t p = (n + 4095) / 4096;
        total += p;
        if (p <= 1) break;
        n = p;
    }
    return total;
}

hipError_t launch_pack(const float* w, int64_t numel, uint8_t* out, float* scale_out, double* partials,
                       hipStream_t st)
{
    if (numel <= 0) return hipErrorInvalidValue;
    const void* in = w;
    int64_t n = numel;
    double* dst = partials;
    bool level0 = true;
    for (;;) {
        const int64_t p = (n + 4095) / 4096;
        if (p > INT32_MAX) return hipErrorInvalidValue;
        if (level0) hipLaunchKernelGGL((k_abs_sum<1>), dim3((unsigned)p), dim3(256), 0, st, in, n, dst);
        else hipLaunchKernelGGL((k_abs_sum<0>), dim3((unsigned)p), dim3(256), 0, st, in, n, dst);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        if (p == 1) break;
        in = dst;
        dst += p;
        n = p;
        level0 = false;
    }
    const int64_t blocks = ((numel + 3) / 4 + 1023) / 1024;
    hipLaunchKernelGGL(k_pack_codes, dim3((unsigned)(blocks < 8192 ? blocks : 8192)), dim3(256), 0, st, w, numel,
                       dst, out, scale_out);
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

hipError_t read_clear_faults_kernels(uint32_t* bits, hipStream_t st)
{
    hipError_t e = hipMemcpyFromSymbolAsync(bits, HIP_SYMBOL(g_faults), sizeof(uint32_t), 0, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess || !*bits) return e;
    static const uint32_t zero = 0;
    e = hipMemcpyToSymbolAsync(HIP_SYMBOL(g_faults), &zero, sizeof(uint32_t), 0, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return e;
}

hipError_t read_clear_faults(uint32_t* bits, hipStream_t st)
{
    uint32_t k = 0, s = 0;
    hipError_t e = read_clear_faults_kernels(&k, st);
    if (e == hipSuccess) e = stream_faults(&s, st);
    *bits = k | s;
    return e;
}

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t st)
{
    if (bytes == 0) return hipSuccess;
    const size_t chunks = (bytes + 15) / 16;
    hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, st, (uint8_t*)p, bytes);
    return hipGetLastError();
}

}  // namespace btl
