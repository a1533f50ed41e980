// btl_model.hip -- gfx950 kernels of the decoder ops around the BitLinear path.
//
// Reference (imonoonoko/Bit-TTT-Engine, crates/rust_engine):
//   rotary embedding ........ src/layers/attention.rs:15-87
//   Q8 KV cache ............. src/layers/kv_cache.rs:49-128
//   attention ............... src/layers/attention.rs:149-239
//   embedding / greedy pick . src/model/llama.rs:201-271, 509-515
//
// Kernels:
//   k_rope_kv_q8     RoPE on the new q and k rows, then QuantizedKVCache::append
//                    of k and v (per token-head absmax, zero point 128) into the
//                    cache rows at their positions.  One wave per (token, head).
//   k_attn_part      attention of a block of queries against one 64-key chunk of
//                    one KV head: the chunk is dequantised once into LDS, each
//                    wave takes one (query, head of the GQA group) pair at a
//                    time.  Writes the chunk's (max, sum, weighted values) per
//                    query and head.
//   k_attn_combine   merges the chunk partials of each (query, head).
//   k_embed          token ids -> f32 rows of the embedding table.
//   k_rmsnorm_f32    RMSNorm of f32 rows (+ a residual) into f32 rows.
//   k_dense_gemv     a dense f32 / bf16 linear (the reference's lm_head), f32 sums.
//   k_greedy         argmax over the logits (last maximum wins; workgroups fold
//                    into one device word), next id and
//                    position bookkeeping for a device-resident decode loop.
//
// Compiled with -ffp-contract=off: every f32 operation is rounded as written and
// the CPU oracle (oracle/bitllama_oracle.c) restates the same operations.
#include <hip/hip_runtime.h>

#include <atomic>

#include <algorithm>

#include "btl_device.hpp"
#include "btl_internal.hpp"

namespace btl {

// f32 max over the wave via DPP; every value finite or -inf.  Result from lane 63.
__device__ __forceinline__ float wave_max_f32(float v)
{
#define BTL_FMAX_DPP(CTRL, RM)                                                                                 \
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, RM, 0xF, false)))
    BTL_FMAX_DPP(0xB1, 0xF);
    BTL_FMAX_DPP(0x4E, 0xF);
    BTL_FMAX_DPP(0x124, 0xF);
    BTL_FMAX_DPP(0x128, 0xF);
    BTL_FMAX_DPP(0x142, 0xA);
    BTL_FMAX_DPP(0x143, 0xC);
#undef BTL_FMAX_DPP
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Rust `f32 as u8`: saturating, NaN -> 0 (kv_cache.rs:114 to_dtype(U8))
__device__ __forceinline__ uint32_t sat_u8(float r)
{
    if (!(r > 0.0f)) return 0u;
    if (r >= 255.0f) return 255u;
    return (uint32_t)r;
}

// kv_cache.rs:101 `max_val / 127.0`: candle's Tensor / f64 is affine(1/127, 0), a multiply
// by the f32-rounded reciprocal plus zero, not a division
__device__ __forceinline__ float q8_scale(float amax)
{
    return __fadd_rn(__fmul_rn(amax, (float)(1.0 / 127.0)), 0.0f);
}

// ---------------------------------------------------------------------------
// k_rope_kv_q8
// ---------------------------------------------------------------------------
// grid (m, nh + 2 nkv), block 64.  Slot s < nh: q head s (RoPE, f32 out);
// nh <= s < nh + nkv: k head (RoPE, then Q8 into the cache); else v head (Q8).
// Lane i < hd/2 holds the pair (i, i + hd/2) that RotaryEmbedding::apply
// rotates together (attention.rs:67-83).
__global__ __launch_bounds__(64) void k_rope_kv_q8(KvArgs a)
{
    const int t = blockIdx.x, slot = blockIdx.y, lane = threadIdx.x;
    const int pos = (a.d_pos ? *a.d_pos : a.pos) + t;
    if (pos < 0 || pos >= a.max_seq) return;  // uniform per workgroup
    const int hd = a.hd, half = hd >> 1;
    const bool act = lane < half;
    int kind, head;
    const float* src;
    if (slot < a.nh) {
        kind = 0; head = slot;
        src = a.q + ((int64_t)t * a.nh + head) * hd;
    } else if (slot < a.nh + a.nkv) {
        kind = 1; head = slot - a.nh;
        src = a.k + ((int64_t)t * a.nkv + head) * hd;
    } else {
        kind = 2; head = slot - a.nh - a.nkv;
        src = a.v + ((int64_t)t * a.nkv + head) * hd;
    }
    float x1 = act ? src[lane] : 0.0f, x2 = act ? src[lane + half] : 0.0f;
    if (kind < 2 && act) {
        const float c = a.cos_t[(int64_t)pos * half + lane], s = a.sin_t[(int64_t)pos * half + lane];
        const float o1 = __fsub_rn(__fmul_rn(x1, c), __fmul_rn(x2, s));
        const float o2 = __fadd_rn(__fmul_rn(x1, s), __fmul_rn(x2, c));
        x1 = o1;
        x2 = o2;
    }
    if (kind == 0) {
        if (act) {
            float* dst = a.q_out + ((int64_t)t * a.nh + head) * hd;
            dst[lane] = x1;
            dst[lane + half] = x2;
        }
        return;
    }
    // quantize_q8 (kv_cache.rs:95-119): s = max|x| * (f32)(1/127), code = u8(round(x / s) + 128)
    const uint32_t am = wave_max_dpp(max(__float_as_uint(x1) & 0x7FFFFFFFu, __float_as_uint(x2) & 0x7FFFFFFFu));
    const float s = q8_scale(__uint_as_float(am));
    const int64_t row = (int64_t)head * a.max_seq + pos;
    uint8_t* cache = (kind == 1 ? a.kc : a.vc) + row * hd;
    if (act) {
        cache[lane] = (uint8_t)sat_u8(__fadd_rn(__builtin_roundf(__fdiv_rn(x1, s)), 128.0f));
        cache[lane + half] = (uint8_t)sat_u8(__fadd_rn(__builtin_roundf(__fdiv_rn(x2, s)), 128.0f));
    }
    if (lane == 0) (kind == 1 ? a.ksc : a.vsc)[row] = s;
}

hipError_t launch_rope_kv_q8(const KvArgs& a, hipStream_t st)
{
    if (a.m <= 0) return hipSuccess;
    if (a.hd < 2 || a.hd > 128 || (a.hd & 1) || a.nh < 1 || a.nkv < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_rope_kv_q8, dim3((unsigned)a.m, (unsigned)(a.nh + 2 * a.nkv)), dim3(64), 0, st, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// k_attn_part: one 64-key chunk of one KV head against a block of queries
// ---------------------------------------------------------------------------
// grid (nkv, cmax, ceil(m / qb)), block 64 * rep * qw (rep = nh / nkv query
// heads share the KV head, repeat_kv attention.rs:227-239; qw queries of the
// block at a time, rep * qw <= 16 waves).  Query i sits at position pos0 + i
// and sees keys [0, pos0 + i] (the causal mask of attention.rs:245-270; a
// single decode query sees the whole cache).  Wave w takes query head w % rep
// of query w / rep of each pass; every (query, head) is one wave's pass over
// the chunk, so the bits do not depend on qw.
//   chunk keys dequantised once: kd = ((f32)code - 128) * s (kv_cache.rs:122-128)
//   s_j   = (fma chain over d of q[d] * kd[j][d]) * scal            (lane j)
//   m_c   = max_j s_j;  p_j = exp(s_j - m_c);  l_c = pairwise sum over the lanes
//   o_c[d] = fma chain over j of p_j * vd[j][d]                     (lane: d)
constexpr int kAttnChunk = 64;
constexpr int kAttnMaxHd = 128;
constexpr int kAttnMaxRep = 16;
constexpr int kAttnKs = kAttnMaxHd + 4;  // LDS key row stride (floats): 16-byte rows, conflict-free b128 reads

// One query of one head against the staged chunk (nj valid keys):
//   s_j   = (fma chain over d of q[d] * kd[j][d]) * scal            (lane j)
//   m_c   = max_j s_j;  p_j = exp(s_j - m_c);  l_c = pairwise sum over the lanes
//   o_c[d] = fma chain over j of p_j * vd[j][d]                     (lanes: d, d + 64)
// (an fma chain: acc = fma(a_i, b_i, acc) in index order from 0, one rounding
// per term, half the dependent instructions of a multiply and an add)
// and (m_c, l_c, o_c) to part.  Called by every thread of the workgroup (it
// holds a barrier); sq / sp are this wave's rows of s_q / s_p.
// a partial-sum store: plain, or coherent at agent scope (sc1, written through
// to memory) when another workgroup merges it in the same launch
template <bool SC1>
__device__ __forceinline__ void put_part(float* p, float v)
{
    if (SC1) __hip_atomic_store((uint32_t*)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *p = v;
}

template <int HD, bool SC1 = false>
__device__ __forceinline__ void attn_chunk_query(const float (*s_k)[kAttnKs], const float (*s_v)[kAttnMaxHd],
                                                 const float* sq, float* sp, int nj, int hd_rt, float scal, int lane,
                                                 float* part, bool store = true)
{
    const int hd = HD ? HD : hd_rt;  // HD > 0: the loops unroll and the LDS reads batch
    float sc = -__builtin_inff();
    if (lane < nj) {
        float acc = 0.0f;
        if ((hd & 3) == 0) {
#pragma unroll
            for (int d = 0; d < hd; d += 4) {
                const float4 q4 = *(const float4*)&sq[d];
                const float4 k4 = *(const float4*)&s_k[lane][d];
                acc = __fmaf_rn(q4.x, k4.x, acc);
                acc = __fmaf_rn(q4.y, k4.y, acc);
                acc = __fmaf_rn(q4.z, k4.z, acc);
                acc = __fmaf_rn(q4.w, k4.w, acc);
            }
        } else {
            for (int d = 0; d < hd; ++d) acc = __fmaf_rn(sq[d], s_k[lane][d], acc);
        }
        sc = __fadd_rn(__fmul_rn(acc, scal), 0.0f);  // candle affine(scal, 0)
    }
    const float mc = wave_max_f32(sc);
    const float p = lane < nj ? btl_expf(__fsub_rn(sc, mc)) : 0.0f;
    const float lc = wave_pairwise_sum(p);
    sp[lane] = p;
    __syncthreads();
    const int d0 = lane, d1 = lane + 64;
    float o0 = 0.0f, o1 = 0.0f;
    const bool h0 = d0 < hd, h1 = d1 < hd;
    const int c0 = h0 ? d0 : 0, c1 = h1 ? d1 : 0;  // clamped columns (values unused when out of range)
    int j = 0;
    auto four = [&](int jj) {
        const float4 p4 = *(const float4*)&sp[jj];
        const float a0 = s_v[jj][c0], a1 = s_v[jj + 1][c0], a2 = s_v[jj + 2][c0], a3 = s_v[jj + 3][c0];
        const float b0 = s_v[jj][c1], b1 = s_v[jj + 1][c1], b2 = s_v[jj + 2][c1], b3 = s_v[jj + 3][c1];
        o0 = __fmaf_rn(p4.x, a0, o0);
        o0 = __fmaf_rn(p4.y, a1, o0);
        o0 = __fmaf_rn(p4.z, a2, o0);
        o0 = __fmaf_rn(p4.w, a3, o0);
        o1 = __fmaf_rn(p4.x, b0, o1);
        o1 = __fmaf_rn(p4.y, b1, o1);
        o1 = __fmaf_rn(p4.z, b2, o1);
        o1 = __fmaf_rn(p4.w, b3, o1);
    };
    if (HD != 0 && nj == kAttnChunk) {
        // a full chunk: unrolled, so the LDS reads of later keys issue ahead of
        // the sums (the runtime loop waited for each group's reads in turn)
#pragma unroll
        for (int jj = 0; jj < kAttnChunk; jj += 4) four(jj);
        j = kAttnChunk;
    } else {
        for (; j + 4 <= nj; j += 4) four(j);
    }
    for (; j < nj; ++j) {
        const float pj = sp[j];
        o0 = __fmaf_rn(pj, s_v[j][c0], o0);
        o1 = __fmaf_rn(pj, s_v[j][c1], o1);
    }
    if (!store) return;  // a wave without a query this pass (it still met the barrier)
    if (h0) put_part<SC1>(&part[2 + d0], o0);
    if (h1) put_part<SC1>(&part[2 + d1], o1);
    if (lane == 0) {
        put_part<SC1>(&part[0], mc);
        put_part<SC1>(&part[1], lc);
    }
}

// Dequantise rows [j0, j0 + nstage) of KV head g's cache into LDS (every
// thread of the workgroup takes part): kd = ((f32)code - 128) * s
// (kv_cache.rs:122-128).
template <int HD>
__device__ __forceinline__ void attn_stage_chunk(const AttnArgs& a, int g, int j0, int nstage, int hd,
                                                 float (*s_k)[kAttnKs], float (*s_v)[kAttnMaxHd], int tid, int nthr)
{
    const int64_t base = (int64_t)g * a.max_seq + j0;
    if ((hd & 15) == 0) {
        // 16-byte loads, all in flight before the first conversion
        const int vpr = hd >> 4, nvec = nstage * vpr;
        uint4 kv[8], vv[8];
        float ks[8], vs[8];
        // a uniform bound and every lane loading (a lane past the chunk
        // reloads its last vector), as in k_attn_dec1
#pragma unroll
        for (int it = 0; it < 8; ++it) {
            if (it * nthr < nvec) {  // uniform
                const int idx = min(tid + it * nthr, nvec - 1);
                const int j = idx / vpr;
                kv[it] = ((const uint4*)(a.kc + (base + j) * hd))[idx - j * vpr];
                vv[it] = ((const uint4*)(a.vc + (base + j) * hd))[idx - j * vpr];
                ks[it] = a.ksc[base + j];
                vs[it] = a.vsc[base + j];
            }
        }
#pragma unroll
        for (int it = 0; it < 8; ++it) {
            const int idx = tid + it * nthr;
            if (idx < nvec) {
                const int j = idx / vpr, e0 = (idx - j * vpr) * 16;
                const uint32_t kw[4] = {kv[it].x, kv[it].y, kv[it].z, kv[it].w};
                const uint32_t vw[4] = {vv[it].x, vv[it].y, vv[it].z, vv[it].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float4 kf, vf;
                    kf.x = __fmul_rn(__fsub_rn((float)(kw[q] & 255u), 128.0f), ks[it]);
                    kf.y = __fmul_rn(__fsub_rn((float)((kw[q] >> 8) & 255u), 128.0f), ks[it]);
                    kf.z = __fmul_rn(__fsub_rn((float)((kw[q] >> 16) & 255u), 128.0f), ks[it]);
                    kf.w = __fmul_rn(__fsub_rn((float)(kw[q] >> 24), 128.0f), ks[it]);
                    vf.x = __fmul_rn(__fsub_rn((float)(vw[q] & 255u), 128.0f), vs[it]);
                    vf.y = __fmul_rn(__fsub_rn((float)((vw[q] >> 8) & 255u), 128.0f), vs[it]);
                    vf.z = __fmul_rn(__fsub_rn((float)((vw[q] >> 16) & 255u), 128.0f), vs[it]);
                    vf.w = __fmul_rn(__fsub_rn((float)(vw[q] >> 24), 128.0f), vs[it]);
                    *(float4*)&s_k[j][e0 + 4 * q] = kf;
                    *(float4*)&s_v[j][e0 + 4 * q] = vf;
                }
            }
        }
    } else {
        for (int idx = tid; idx < nstage * hd; idx += nthr) {
            const int j = idx / hd, d = idx - j * hd;
            const int64_t r = base + j;
            s_k[j][d] = __fmul_rn(__fsub_rn((float)a.kc[r * hd + d], 128.0f), a.ksc[r]);
            s_v[j][d] = __fmul_rn(__fsub_rn((float)a.vc[r * hd + d], 128.0f), a.vsc[r]);
        }
    }

}

template <int HD>
__global__ __launch_bounds__(1024) void k_attn_part(AttnArgs a)
{
    __shared__ __align__(16) float s_k[kAttnChunk][kAttnKs];
    __shared__ __align__(16) float s_v[kAttnChunk][kAttnMaxHd];
    __shared__ __align__(16) float s_q[kAttnMaxRep][kAttnMaxHd];
    __shared__ __align__(16) float s_p[kAttnMaxRep][kAttnChunk];
    const int g = blockIdx.x, c = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nthr = blockDim.x;
    const int hd = HD ? HD : a.hd, rep = a.nh / a.nkv;  // HD > 0: launched for a.hd == HD
    const int qw = nthr / (64 * rep);                   // queries per pass
    const int hw = wave % rep, qs = wave / rep;         // this wave's head and query slot
    const int h = g * rep + hw;
    const int pos0 = a.d_pos ? *a.d_pos : a.pos;
    const int i_begin = blockIdx.z * a.qb;
    const int i_end = min(a.m, i_begin + a.qb);
    const int j0 = c * kAttnChunk;
    const int t_last = min(pos0 + i_end, a.max_seq);  // keys any query of the block sees
    if (j0 >= t_last) return;                           // uniform
    const int nstage = min(kAttnChunk, t_last - j0);

    attn_stage_chunk<HD>(a, g, j0, nstage, hd, s_k, s_v, tid, nthr);

    for (int i0 = i_begin; i0 < i_end; i0 += qw) {
        // the last query of the pass sees the most keys (uniform)
        if (j0 >= min(pos0 + min(i0 + qw, i_end), a.max_seq)) continue;
        const int i = i0 + qs;
        const int T = i < i_end ? min(pos0 + i + 1, a.max_seq) : 0;
        const bool act = j0 < T;  // uniform per wave; an idle wave still meets the barriers
        const int nj = act ? min(kAttnChunk, T - j0) : 0;
        if (act) {
            const float* qg = a.q + ((int64_t)i * a.nh + h) * hd;
            for (int d = lane; d < hd; d += 64) s_q[wave][d] = qg[d];
        }
        __syncthreads();
        float* part = a.part + (((int64_t)(act ? i : 0) * a.nh + h) * a.cmax + c) * (hd + 2);
        attn_chunk_query<HD>(s_k, s_v, s_q[wave], s_p[wave], nj, hd, a.scal, lane, part, act);
        __syncthreads();  // s_q / s_p are rewritten by the next pass
    }
}

// k_attn_part with the G = rep query heads of a KV head in one wave: wave w
// takes query w of each pass and every head of the group, so each dequantised
// key and value element is read from LDS once per group instead of once per
// head (the partials of a long prompt were bound by those reads).  Per
// (query, head) the arithmetic is attn_chunk_query's, in the same order.
// The queries' elements come from global memory by scalar loads (qg: the G
// heads' rows of this wave's query, consecutive, the same for every lane; read
// only in this launch), an SGPR operand of each fma, instead of LDS broadcast
// reads, which cost the LDS as much as the key reads (measured on MI355X,
// Llama-3-8B shapes, a 512-token prompt through the decoder: 9.71-9.79 ->
// 9.41-9.44 ms; the p row by readlane instead of LDS as well: 9.65-9.67).
typedef const __attribute__((address_space(4))) float* attn_qptr;

template <int HD, int G>
__device__ __forceinline__ void attn_chunk_query_g(const float (*s_k)[kAttnKs], const float (*s_v)[kAttnMaxHd],
                                                   const float* qg, float (*sp)[kAttnChunk], int nj,
                                                   float scal, int lane, float* part, int64_t hstride, bool store)
{
    static_assert(HD == 64 || HD == 128, "head size 64 or 128");
    const attn_qptr qs = (attn_qptr)qg;
    float sc[G];
#pragma unroll
    for (int gg = 0; gg < G; ++gg) sc[gg] = -__builtin_inff();
    if (lane < nj) {
        float acc[G];
#pragma unroll
        for (int gg = 0; gg < G; ++gg) acc[gg] = 0.0f;
#pragma unroll
        for (int d = 0; d < HD; d += 4) {
            const float4 k4 = *(const float4*)&s_k[lane][d];
#pragma unroll
            for (int gg = 0; gg < G; ++gg) {
                const float4 q4 = make_float4(qs[gg * HD + d], qs[gg * HD + d + 1], qs[gg * HD + d + 2],
                                              qs[gg * HD + d + 3]);
                acc[gg] = __fmaf_rn(q4.x, k4.x, acc[gg]);
                acc[gg] = __fmaf_rn(q4.y, k4.y, acc[gg]);
                acc[gg] = __fmaf_rn(q4.z, k4.z, acc[gg]);
                acc[gg] = __fmaf_rn(q4.w, k4.w, acc[gg]);
            }
        }
#pragma unroll
        for (int gg = 0; gg < G; ++gg) sc[gg] = __fadd_rn(__fmul_rn(acc[gg], scal), 0.0f);  // candle affine(scal, 0)
    }
    float mc[G], lc[G];
#pragma unroll
    for (int gg = 0; gg < G; ++gg) {
        mc[gg] = wave_max_f32(sc[gg]);
        const float p = lane < nj ? btl_expf(__fsub_rn(sc[gg], mc[gg])) : 0.0f;
        lc[gg] = wave_pairwise_sum(p);
        sp[gg][lane] = p;
    }
    __syncthreads();
    const int d0 = lane, d1 = lane + 64;
    const bool h1 = d1 < HD;
    const int c1 = h1 ? d1 : 0;  // clamped column (values unused when out of range)
    float o0[G], o1[G];
#pragma unroll
    for (int gg = 0; gg < G; ++gg) o0[gg] = o1[gg] = 0.0f;
    auto four = [&](int jj) {
        const float a0 = s_v[jj][d0], a1 = s_v[jj + 1][d0], a2 = s_v[jj + 2][d0], a3 = s_v[jj + 3][d0];
        const float b0 = s_v[jj][c1], b1 = s_v[jj + 1][c1], b2 = s_v[jj + 2][c1], b3 = s_v[jj + 3][c1];
#pragma unroll
        for (int gg = 0; gg < G; ++gg) {
            const float4 p4 = *(const float4*)&sp[gg][jj];
            o0[gg] = __fmaf_rn(p4.x, a0, o0[gg]);
            o0[gg] = __fmaf_rn(p4.y, a1, o0[gg]);
            o0[gg] = __fmaf_rn(p4.z, a2, o0[gg]);
            o0[gg] = __fmaf_rn(p4.w, a3, o0[gg]);
            o1[gg] = __fmaf_rn(p4.x, b0, o1[gg]);
            o1[gg] = __fmaf_rn(p4.y, b1, o1[gg]);
            o1[gg] = __fmaf_rn(p4.z, b2, o1[gg]);
            o1[gg] = __fmaf_rn(p4.w, b3, o1[gg]);
        }
    };
    int j = 0;
    if (nj == kAttnChunk) {
#pragma unroll
        for (int jj = 0; jj < kAttnChunk; jj += 4) four(jj);
        j = kAttnChunk;
    } else {
        for (; j + 4 <= nj; j += 4) four(j);
    }
    for (; j < nj; ++j) {
        const float a0 = s_v[j][d0], b0 = s_v[j][c1];
#pragma unroll
        for (int gg = 0; gg < G; ++gg) {
            const float pj = sp[gg][j];
            o0[gg] = __fmaf_rn(pj, a0, o0[gg]);
            o1[gg] = __fmaf_rn(pj, b0, o1[gg]);
        }
    }
    if (!store) return;  // a wave without a query this pass (it still met the barrier)
#pragma unroll
    for (int gg = 0; gg < G; ++gg) {
        float* pg = part + gg * hstride;
        pg[2 + d0] = o0[gg];
        if (h1) pg[2 + d1] = o1[gg];
        if (lane == 0) {
            pg[0] = mc[gg];
            pg[1] = lc[gg];
        }
    }
}

// grid (nkv, cmax, ceil(m / qb)), block 64 * qw (rep = G query heads per KV
// head, qw queries of the block at a time); otherwise as k_attn_part.
template <int HD, int G>
__global__ __launch_bounds__(1024) void k_attn_part_g(AttnArgs a)
{
    __shared__ __align__(16) float s_k[kAttnChunk][kAttnKs];
    __shared__ __align__(16) float s_v[kAttnChunk][kAttnMaxHd];
    __shared__ __align__(16) float s_p[kAttnMaxRep * G][kAttnChunk];
    const int g = blockIdx.x, c = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the query rows' scalar loads
    const int nthr = blockDim.x;
    const int qw = nthr >> 6;  // queries per pass: one per wave
    const int pos0 = a.d_pos ? *a.d_pos : a.pos;
    const int i_begin = blockIdx.z * a.qb;
    const int i_end = min(a.m, i_begin + a.qb);
    const int j0 = c * kAttnChunk;
    const int t_last = min(pos0 + i_end, a.max_seq);  // keys any query of the block sees
    if (j0 >= t_last) return;                           // uniform
    const int nstage = min(kAttnChunk, t_last - j0);
    attn_stage_chunk<HD>(a, g, j0, nstage, HD, s_k, s_v, tid, nthr);
    __syncthreads();  // the staged chunk

    const int64_t hstride = (int64_t)a.cmax * (HD + 2);  // consecutive heads' partial slots
    for (int i0 = i_begin; i0 < i_end; i0 += qw) {
        // the last query of the pass sees the most keys (uniform)
        if (j0 >= min(pos0 + min(i0 + qw, i_end), a.max_seq)) continue;
        const int i = i0 + wave;
        const int T = i < i_end ? min(pos0 + i + 1, a.max_seq) : 0;
        const bool act = j0 < T;  // uniform per wave; an idle wave still meets the barriers
        const int nj = act ? min(kAttnChunk, T - j0) : 0;
        // the group's G heads of query i, consecutive (an idle wave: query i_begin's, unused)
        const float* qg = a.q + ((int64_t)(act ? i : i_begin) * a.nh + g * G) * HD;
        float* part = a.part + (((int64_t)(act ? i : 0) * a.nh + g * G) * a.cmax + c) * (HD + 2);
        attn_chunk_query_g<HD, G>(s_k, s_v, qg, &s_p[wave * G], nj, a.scal, lane, part, hstride, act);
        __syncthreads();  // s_p is rewritten by the next pass
    }
}

// a partial-sum load: plain, or coherent at agent scope (sc1) when other
// workgroups of the same launch wrote it
template <bool SC1>
__device__ __forceinline__ float ld_part(const float* p)
{
    if (SC1) return __uint_as_float(__hip_atomic_load((const uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    return *p;
}

// The chunk merge of one (query, head) by one wave, k_attn_combine's
// arithmetic: y[d] = (sum_c w_c o_c[d]) / (sum_c w_c l_c), w_c = exp(m_c -
// max_c m_c), both sums sequential over the chunks.  part: the head's chunk
// slots of st = hd + 2 floats.  Before the chunk count is known (cfun(): C,
// or <= 0 for no result -> NaN), the (m, l) of the first 64 slots below cpre
// and the values of the first 16 are loaded, all in flight together.  SC1: the
// slots were written by other workgroups of this launch (coherent loads).
template <bool SC1, typename CF>
__device__ __forceinline__ void attn_merge_head(const float* part, int st, int cpre, int hd, int lane, float* y,
                                                CF cfun)
{
    const int d0 = lane, d1 = lane + 64;
    const bool h0 = d0 < hd, h1 = d1 < hd;
    constexpr int kPre = 16;
    // every load unconditional, slots past cpre clamped to slot cpre - 1 (their
    // values are never used): a per-lane or per-slot condition here made the
    // compiler wait for the earlier loads before issuing the (m, l) loads
    const int clast = max(cpre, 1) - 1;
    const int cl = min(lane, clast);
    const float m_pre = ld_part<SC1>(&part[cl * st]);
    const float l_pre = ld_part<SC1>(&part[cl * st + 1]);
    float p0[kPre], p1[kPre];
#pragma unroll
    for (int c = 0; c < kPre; ++c) {
        const int cc = min(c, clast);
        p0[c] = h0 ? ld_part<SC1>(&part[cc * st + 2 + d0]) : 0.0f;
        p1[c] = h1 ? ld_part<SC1>(&part[cc * st + 2 + d1]) : 0.0f;
    }
    __builtin_amdgcn_sched_barrier(0);  // all of them issue before the first use
    const int C = cfun();
    if (C <= 0) {
        if (h0) y[d0] = __builtin_nanf("");
        if (h1) y[d1] = __builtin_nanf("");
        return;
    }
    float M = -__builtin_inff();
    for (int c0 = 0; c0 < C; c0 += 64) {
        const int cc = c0 + lane;
        const float mv = c0 == 0 ? m_pre : (cc < C ? ld_part<SC1>(&part[cc * st]) : 0.0f);
        M = fmaxf(M, wave_max_f32(cc < C ? mv : -__builtin_inff()));
    }
    float L = 0.0f, O0 = 0.0f, O1 = 0.0f;
    for (int c0 = 0; c0 < C; c0 += 64) {
        const int cc = c0 + lane;
        const float mv = c0 == 0 ? m_pre : (cc < C ? ld_part<SC1>(&part[cc * st]) : 0.0f);
        const float lv = c0 == 0 ? l_pre : (cc < C ? ld_part<SC1>(&part[cc * st + 1]) : 0.0f);
        const float w = cc < C ? btl_expf(__fsub_rn(mv, M)) : 0.0f;
        const float l = cc < C ? lv : 0.0f;
        const int n = min(64, C - c0);
        int u = 0;
        if (c0 == 0) {
#pragma unroll
            for (int q = 0; q < kPre; ++q) {
                if (q < n) {
                    const float wu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), q));
                    const float lu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(l), q));
                    L = __fadd_rn(L, __fmul_rn(wu, lu));
                    O0 = __fadd_rn(O0, __fmul_rn(wu, p0[q]));
                    O1 = __fadd_rn(O1, __fmul_rn(wu, p1[q]));
                }
            }
            u = min(n, kPre);
        }
        for (; u < n; ++u) {
            const int c = c0 + u;
            const float wu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), u));
            const float lu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(l), u));
            L = __fadd_rn(L, __fmul_rn(wu, lu));
            const float v0 = h0 ? ld_part<SC1>(&part[c * st + 2 + d0]) : 0.0f;
            const float v1 = h1 ? ld_part<SC1>(&part[c * st + 2 + d1]) : 0.0f;
            O0 = __fadd_rn(O0, __fmul_rn(wu, v0));
            O1 = __fadd_rn(O1, __fmul_rn(wu, v1));
        }
    }
    if (h0) y[d0] = __fdiv_rn(O0, L);
    if (h1) y[d1] = __fdiv_rn(O1, L);
}

// ---------------------------------------------------------------------------
// k_attn_dec1: one decode token -- RoPE, the Q8 append and the chunk partials
// ---------------------------------------------------------------------------
// grid (nkv, cmax), block 64 * rep.  The work of k_rope_kv_q8 + k_attn_part for
// m = 1 in one launch: every workgroup rotates its query heads itself; the
// workgroup whose chunk holds the position rotates and quantises the new k and
// v row, writes it to the cache and patches its LDS copy of the chunk with the
// dequantised row (the reference attends over the dequantised cache, new row
// included: kv_cache.rs:82-86).  Loads that do not depend on the position (the
// raw q / k / v rows and the chunk's cache rows) are issued before it arrives.
// MERGE: the chunk partials go out with coherent stores, the workgroups of a
// KV head count themselves on an agent-scope counter, and the last one merges
// every query head of the KV head (the counter is left at zero for the next
// launch): no second launch.
template <int HD, bool MERGE = false>
__global__ __launch_bounds__(1024) void k_attn_dec1(AttnArgs a, DecKv kv)
{
    __shared__ __align__(16) float s_k[kAttnChunk][kAttnKs];
    __shared__ __align__(16) float s_v[kAttnChunk][kAttnMaxHd];
    __shared__ __align__(16) float s_q[kAttnMaxRep][kAttnMaxHd];
    __shared__ __align__(16) float s_p[kAttnMaxRep][kAttnChunk];
    const int g = blockIdx.x, c = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nthr = blockDim.x;
    // HD > 0 (the host launches it for a.hd == HD): the head size is a
    // constant, so the rows' lane predicates fold and their loads issue
    // back to back instead of in one branch each
    const int hd = HD ? HD : a.hd, half = hd >> 1, rep = a.nh / a.nkv;
    const int h = g * rep + wave;
    const int j0 = c * kAttnChunk;
    if (j0 >= a.max_seq) return;  // uniform
    const bool act = lane < half;

    // position-independent loads: raw q of this wave's head, raw k / v of the KV head, the chunk rows
    float q1 = act ? kv.q[h * hd + lane] : 0.0f, q2 = act ? kv.q[h * hd + lane + half] : 0.0f;
    float k1 = act ? kv.k[g * hd + lane] : 0.0f, k2 = act ? kv.k[g * hd + lane + half] : 0.0f;
    float v1 = act ? kv.v[g * hd + lane] : 0.0f, v2 = act ? kv.v[g * hd + lane + half] : 0.0f;
    const int nrows = min(kAttnChunk, a.max_seq - j0);
    const int64_t base = (int64_t)g * a.max_seq + j0;
    const int vpr = hd >> 4, nvec = nrows * vpr;  // hd % 16 == 0 (host)
    uint4 kvv[8], vvv[8];
    float ks[8], vs[8];
    // a uniform bound and every lane loading (a lane past the chunk reloads its
    // last vector): a per-lane condition here made the compiler copy a loaded
    // scale between registers, waiting for it before the next loads issued
#pragma unroll
    for (int it = 0; it < 8; ++it) {
        if (it * nthr < nvec) {  // uniform
            const int idx = min(tid + it * nthr, nvec - 1);
            const int j = idx / vpr;
            kvv[it] = ((const uint4*)(a.kc + (base + j) * hd))[idx - j * vpr];
            vvv[it] = ((const uint4*)(a.vc + (base + j) * hd))[idx - j * vpr];
            ks[it] = a.ksc[base + j];
            vs[it] = a.vsc[base + j];
        }
    }
    const int pos = a.d_pos ? *a.d_pos : a.pos;
    if (pos < 0 || pos >= a.max_seq) {  // uniform: nothing to append or attend, no result
        if (MERGE && c == 0) {
            float* y = a.out + (int64_t)h * hd;
            if (lane < hd) y[lane] = __builtin_nanf("");
            if (lane + 64 < hd) y[lane + 64] = __builtin_nanf("");
        }
        return;
    }
    const int T = pos + 1;
    if (j0 >= T) return;  // uniform
    const int nj = min(kAttnChunk, T - j0);
    float cs = 1.0f, sn = 0.0f;
    if (act) {
        cs = kv.cos_t[(int64_t)pos * half + lane];
        sn = kv.sin_t[(int64_t)pos * half + lane];
    }
#pragma unroll
    for (int it = 0; it < 8; ++it) {
        const int idx = tid + it * nthr;
        if (idx < nvec) {
            const int j = idx / vpr, e0 = (idx - j * vpr) * 16;
            const uint32_t kw[4] = {kvv[it].x, kvv[it].y, kvv[it].z, kvv[it].w};
            const uint32_t vw[4] = {vvv[it].x, vvv[it].y, vvv[it].z, vvv[it].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float4 kf, vf;
                kf.x = __fmul_rn(__fsub_rn((float)(kw[q] & 255u), 128.0f), ks[it]);
                kf.y = __fmul_rn(__fsub_rn((float)((kw[q] >> 8) & 255u), 128.0f), ks[it]);
                kf.z = __fmul_rn(__fsub_rn((float)((kw[q] >> 16) & 255u), 128.0f), ks[it]);
                kf.w = __fmul_rn(__fsub_rn((float)(kw[q] >> 24), 128.0f), ks[it]);
                vf.x = __fmul_rn(__fsub_rn((float)(vw[q] & 255u), 128.0f), vs[it]);
                vf.y = __fmul_rn(__fsub_rn((float)((vw[q] >> 8) & 255u), 128.0f), vs[it]);
                vf.z = __fmul_rn(__fsub_rn((float)((vw[q] >> 16) & 255u), 128.0f), vs[it]);
                vf.w = __fmul_rn(__fsub_rn((float)(vw[q] >> 24), 128.0f), vs[it]);
                *(float4*)&s_k[j][e0 + 4 * q] = kf;
                *(float4*)&s_v[j][e0 + 4 * q] = vf;
            }
        }
    }
    // RoPE of this wave's query head (attention.rs:67-83)
    if (act) {
        s_q[wave][lane] = __fsub_rn(__fmul_rn(q1, cs), __fmul_rn(q2, sn));
        s_q[wave][lane + half] = __fadd_rn(__fmul_rn(q1, sn), __fmul_rn(q2, cs));
    }
    const bool owner = pos - j0 < kAttnChunk;  // uniform: this chunk holds the new row
    __syncthreads();
    if (owner && wave < 2) {
        // wave 0: RoPE + Q8 of k;  wave 1 (or wave 0 again when rep == 1): Q8 of v
        for (int which = wave; which < 2; which += (rep == 1 ? 1 : 2)) {
            float x1 = which == 0 ? k1 : v1, x2 = which == 0 ? k2 : v2;
            if (which == 0 && act) {
                const float o1 = __fsub_rn(__fmul_rn(x1, cs), __fmul_rn(x2, sn));
                const float o2 = __fadd_rn(__fmul_rn(x1, sn), __fmul_rn(x2, cs));
                x1 = o1;
                x2 = o2;
            }
            const uint32_t am =
                wave_max_dpp(max(__float_as_uint(x1) & 0x7FFFFFFFu, __float_as_uint(x2) & 0x7FFFFFFFu));
            const float sc = q8_scale(__uint_as_float(am));
            const int64_t row = (int64_t)g * a.max_seq + pos;
            uint8_t* cache = (which == 0 ? kv.kc_w : kv.vc_w) + row * hd;
            float* srow = which == 0 ? &s_k[pos - j0][0] : &s_v[pos - j0][0];
            if (act) {
                const uint32_t c1 = sat_u8(__fadd_rn(__builtin_roundf(__fdiv_rn(x1, sc)), 128.0f));
                const uint32_t c2 = sat_u8(__fadd_rn(__builtin_roundf(__fdiv_rn(x2, sc)), 128.0f));
                cache[lane] = (uint8_t)c1;
                cache[lane + half] = (uint8_t)c2;
                srow[lane] = __fmul_rn(__fsub_rn((float)c1, 128.0f), sc);
                srow[lane + half] = __fmul_rn(__fsub_rn((float)c2, 128.0f), sc);
            }
            if (lane == 0) (which == 0 ? kv.ksc_w : kv.vsc_w)[row] = sc;
        }
    }
    __syncthreads();
    float* part = a.part + ((int64_t)h * a.cmax + c) * (hd + 2);
    attn_chunk_query<HD, MERGE>(s_k, s_v, s_q[wave], s_p[wave], nj, hd, a.scal, lane, part);
    if (MERGE) {
        __shared__ uint32_t s_last;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partials are stored
        __syncthreads();
        if (tid == 0) {
            const int C = (T + kAttnChunk - 1) / kAttnChunk;  // workgroups of this KV head with keys
            const uint32_t old = __hip_atomic_fetch_add(a.ctr + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const bool last = old + 1u == (uint32_t)C;
            if (last) __hip_atomic_store(a.ctr + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = last ? 1u : 0u;
        }
        __syncthreads();
        if (!s_last) return;
        const int C = (T + kAttnChunk - 1) / kAttnChunk;
        attn_merge_head<true>(a.part + (int64_t)h * a.cmax * (hd + 2), hd + 2, C, hd, lane, a.out + (int64_t)h * hd,
                              [C]() { return C; });
    }
}

// grid (m, nh), block 64: y[d] = (sum_c w_c o_c[d]) / (sum_c w_c l_c),
// w_c = exp(m_c - max_c m_c), both sums sequential over the chunks.  Lane c
// holds chunk c's (m_c, l_c); the value loads of up to 16 chunks are all in
// flight before the sums.
__global__ __launch_bounds__(64) void k_attn_combine(AttnArgs a)
{
    const int i = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int hd = a.hd, st = hd + 2;
    const float* part = a.part + ((int64_t)i * a.nh + h) * a.cmax * st;
    float* y = a.out + ((int64_t)i * a.nh + h) * hd;
    attn_merge_head<false>(part, st, a.cmax, hd, lane, y, [&]() {
        const int T = (a.d_pos ? *a.d_pos : a.pos) + i + 1;
        // a device position outside the cache: no result
        return T <= 0 || T > a.max_seq ? 0 : (T + kAttnChunk - 1) / kAttnChunk;
    });
}

hipError_t launch_attention_dec1(const AttnArgs& a, const DecKv& kv, hipStream_t st)
{
    const int rep = a.nh / a.nkv;
    if (a.m != 1 || a.hd < 16 || a.hd > kAttnMaxHd || (a.hd & 15) || a.nkv < 1 || a.nh % a.nkv != 0 ||
        rep > kAttnMaxRep || a.cmax < 1)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)a.nkv, (unsigned)a.cmax), block((unsigned)(64 * rep));
    if (a.ctr) {
        if (a.nkv > kAttnMaxCtr) return hipErrorInvalidValue;
        if (a.hd == 128) hipLaunchKernelGGL((k_attn_dec1<128, true>), grid, block, 0, st, a, kv);
        else if (a.hd == 64) hipLaunchKernelGGL((k_attn_dec1<64, true>), grid, block, 0, st, a, kv);
        else hipLaunchKernelGGL((k_attn_dec1<0, true>), grid, block, 0, st, a, kv);
        return hipGetLastError();
    }
    if (a.hd == 128) hipLaunchKernelGGL(k_attn_dec1<128>, grid, block, 0, st, a, kv);
    else if (a.hd == 64) hipLaunchKernelGGL(k_attn_dec1<64>, grid, block, 0, st, a, kv);
    else hipLaunchKernelGGL(k_attn_dec1<0>, grid, block, 0, st, a, kv);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_attn_combine, dim3(1u, (unsigned)a.nh), dim3(64), 0, st, a);
    return hipGetLastError();
}

// The merge counters of the one-launch decode attention: kAttnMaxCtr words per
// workspace slot (KeySlots), zero at load and left at zero by every launch (the
// last workgroup of a KV head resets its word).  Launches that share a
// workspace share counters; they are ordered by their caller anyway (they also
// write the same chunk partials).
static __device__ uint32_t g_attn_ctr[kAttnSlots * kAttnMaxCtr];

hipError_t attn_counters(int dev, const void* ws_key, uint32_t** out)
{
    static KeySlots<kAttnSlots> slots[64];
    static std::atomic<uint32_t*> ptr[64];
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    uint32_t* p = ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        void* q = nullptr;
        hipError_t e = hipGetSymbolAddress(&q, HIP_SYMBOL(g_attn_ctr));
        if (e != hipSuccess) return e;
        p = (uint32_t*)q;
        ptr[dev].store(p, std::memory_order_release);
    }
    const int i = slots[dev].find(ws_key);
    *out = i < 0 ? nullptr : p + (size_t)i * kAttnMaxCtr;
    return hipSuccess;
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t st)
{
    if (a.m <= 0) return hipSuccess;
    const int rep = a.nh / a.nkv;
    if (a.hd < 1 || a.hd > kAttnMaxHd || a.nkv < 1 || a.nh % a.nkv != 0 || rep > kAttnMaxRep || a.qb < 1 ||
        a.cmax < 1)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)a.nkv, (unsigned)a.cmax, (unsigned)((a.m + a.qb - 1) / a.qb));
    if ((rep == 2 || rep == 4) && (a.hd == 128 || a.hd == 64) && a.qb > 1) {
        // the query heads of a KV head in one wave, up to 16 queries at a time
        // (measured on MI355X, Llama-3-8B prefill of 512 tokens, us per layer:
        // 153 with one wave per head walking the block's queries one by one,
        // 130 with a wave per (query, head))
        const dim3 block((unsigned)(64 * std::min(kAttnMaxRep, a.qb)));
#define BTL_ATTN_G(HDV, GV) \
    if (a.hd == HDV && rep == GV) hipLaunchKernelGGL((k_attn_part_g<HDV, GV>), grid, block, 0, st, a);
        BTL_ATTN_G(128, 4) else BTL_ATTN_G(128, 2) else BTL_ATTN_G(64, 4) else BTL_ATTN_G(64, 2)
#undef BTL_ATTN_G
    } else {
        // a wave per (query, head), qw queries of the block at a time
        const int qw = std::max(1, std::min(kAttnMaxRep / rep, a.qb));
        const dim3 block((unsigned)(64 * rep * qw));
        if (a.hd == 128) hipLaunchKernelGGL(k_attn_part<128>, grid, block, 0, st, a);
        else if (a.hd == 64) hipLaunchKernelGGL(k_attn_part<64>, grid, block, 0, st, a);
        else hipLaunchKernelGGL(k_attn_part<0>, grid, block, 0, st, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_attn_combine, dim3((unsigned)a.m, (unsigned)a.nh), dim3(64), 0, st, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// k_add_f32: y += r elementwise (the residual add after a contraction of many
// token rows; IEEE addition commutes, so the bits are those of r + y)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_add_f32(float* y, const float* r, int64_t n)
{
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) y[i] = __fadd_rn(y[i], r[i]);
}

hipError_t launch_add_f32(float* y, const float* r, int64_t n, hipStream_t st)
{
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(k_add_f32, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, st, y, r, n);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// k_swiglu_f32: silu(g) * u elementwise (swiglu.rs:29-35), candle's silu
// v / (1 + exp(-v)) with btl_expf; the route for many token rows
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_swiglu_f32(const float* g, const float* u, int64_t n, float* out)
{
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const float v = g[i];
        out[i] = __fmul_rn(__fdiv_rn(v, __fadd_rn(1.0f, btl_expf(-v))), u[i]);
    }
}

hipError_t launch_swiglu_f32(const float* g, const float* u, int64_t n, float* out, hipStream_t st)
{
    if (n <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(k_swiglu_f32, dim3((unsigned)blocks), dim3(256), 0, st, g, u, n, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Multi-base adaptive format (AdaptiveBitLinear, adaptive_linear.rs:51-160)
// ---------------------------------------------------------------------------
// The reference's weight_packed [n, k/4, nb] interleaves the bases per column
// pack (byte (r, cp, b) at (r * k/4 + cp) * nb + b, convert_llama_v2.py:111-151).
// k_adaptive_split copies base b's bytes into a PackedTensor array [n, k/4]
// (same 2-bit codes and bit positions), so every base runs through the
// BitLinear kernels; one thread per 4 column packs of one row.
__global__ __launch_bounds__(256) void k_adaptive_split(const uint8_t* packed, int64_t total, int nb,
                                                        AdaptiveOut out)
{
    // byte f of base b is packed[f * nb + b] over the flattened [n * k/4] index;
    // unit u = 4 consecutive f (one 32-bit store per base), the last < 4 by bytes
    const int64_t units = total >> 2;
    for (int64_t u = blockIdx.x * 256ll + threadIdx.x; u <= units; u += (int64_t)gridDim.x * 256) {
        const uint8_t* src = packed + u * 4 * nb;
        if (u < units) {
            for (int b = 0; b < nb; ++b) {
                const uint32_t v = (uint32_t)src[b] | ((uint32_t)src[nb + b] << 8) |
                                   ((uint32_t)src[2 * nb + b] << 16) | ((uint32_t)src[3 * nb + b] << 24);
                ((uint32_t*)out.p[b])[u] = v;
            }
        } else {
            for (int64_t f = 4 * u; f < total; ++f)
                for (int b = 0; b < nb; ++b) out.p[b][f] = packed[f * nb + b];
        }
    }
}

hipError_t launch_adaptive_split(const uint8_t* packed, int64_t n, int64_t k, int nb, const AdaptiveOut& out,
                                 hipStream_t st)
{
    const int64_t total = n * (k / 4);
    if (total <= 0) return hipSuccess;
    if (nb < 1 || nb > kMaxBases) return hipErrorInvalidValue;
    const int64_t blocks = std::min<int64_t>(((total >> 2) + 256) / 256, 8192);
    hipLaunchKernelGGL(k_adaptive_split, dim3((unsigned)blocks), dim3(256), 0, st, packed, total, nb, out);
    return hipGetLastError();
}

// AdaptiveBitLinear::load's dense reconstruction (adaptive_linear.rs:86-117):
// w[r][4cp + j] = ((0 + t_0 s_0) + t_1 s_1) + ..., bases in order, f32.
__global__ __launch_bounds__(256) void k_adaptive_reconstruct(const uint8_t* packed, int64_t cps, int nb,
                                                              AdaptiveScales sc, float* out)
{
    for (int64_t u = blockIdx.x * 256ll + threadIdx.x; u < cps; u += (int64_t)gridDim.x * 256) {
        float w[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int b = 0; b < nb; ++b) {
            const uint32_t byte = packed[u * nb + b];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t c = (byte >> (2 * j)) & 3u;
                const float v = c == 1u ? 1.0f : (c == 2u ? -1.0f : 0.0f);
                w[j] = __fadd_rn(w[j], __fmul_rn(v, sc.s[b]));
            }
        }
        ((float4*)out)[u] = make_float4(w[0], w[1], w[2], w[3]);
    }
}

hipError_t launch_adaptive_reconstruct(const uint8_t* packed, int64_t n, int64_t k, int nb, const AdaptiveScales& sc,
                                       float* out, hipStream_t st)
{
    const int64_t cps = n * (k / 4);
    if (cps <= 0) return hipSuccess;
    if (nb < 1 || nb > kMaxBases) return hipErrorInvalidValue;
    const int64_t blocks = std::min<int64_t>((cps + 255) / 256, 8192);
    hipLaunchKernelGGL(k_adaptive_reconstruct, dim3((unsigned)blocks), dim3(256), 0, st, packed, cps, nb, sc, out);
    return hipGetLastError();
}

// y = ys[0] + ys[1] + ... (f32, in base order), stored f32 or bf16
__device__ __forceinline__ uint16_t bf16_rne(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__global__ __launch_bounds__(256) void k_base_sum(AdaptiveSum a)
{
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < a.count; i += (int64_t)gridDim.x * 256) {
        float v = a.ys[0][i];
        for (int b = 1; b < a.nb; ++b) v = __fadd_rn(v, a.ys[b][i]);
        if (a.ykind == YK_BF16) ((uint16_t*)a.y)[i] = bf16_rne(v);
        else ((float*)a.y)[i] = v;
    }
}

hipError_t launch_base_sum(const AdaptiveSum& a, hipStream_t st)
{
    if (a.count <= 0) return hipSuccess;
    if (a.nb < 1 || a.nb > kMaxBases) return hipErrorInvalidValue;
    const int64_t blocks = std::min<int64_t>((a.count + 255) / 256, 4096);
    hipLaunchKernelGGL(k_base_sum, dim3((unsigned)blocks), dim3(256), 0, st, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// k_embed: candle_nn::Embedding::forward (llama.rs:208) -> f32 rows
// ---------------------------------------------------------------------------
// grid (m, ceil(dim / 1024)), block 256: workgroup (t, b) copies elements
// [1024 b, 1024 b + 1024) of row t, four per thread (vec: one 16-byte load of
// an f32 row or one 8-byte load of a bf16 row and one 16-byte store -- dim % 4
// == 0 and the pointers aligned for it; else four element loads, all in flight
// before the stores).  An id outside [0, vocab)
// gives a zero row (the reference's index_select would fail; ids from the
// greedy pick are always in range).
template <int XK>
__global__ __launch_bounds__(256) void k_embed(const void* table, int64_t vocab, int dim, const int32_t* ids,
                                               float* out, bool vec)
{
    const int t = blockIdx.x;
    const int d = blockIdx.y * 1024 + 4 * threadIdx.x;
    if (d >= dim) return;
    const int64_t id = ids[t];
    const bool ok = id >= 0 && id < vocab;
    float* y = out + (int64_t)t * dim;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (vec) {
        if (ok) {
            if (XK == XK_BF16) {
                const uint2 u = *(const uint2*)((const uint16_t*)table + id * dim + d);
                v[0] = __uint_as_float(u.x << 16);
                v[1] = __uint_as_float(u.x & 0xFFFF0000u);
                v[2] = __uint_as_float(u.y << 16);
                v[3] = __uint_as_float(u.y & 0xFFFF0000u);
            } else {
                const float4 f = *(const float4*)((const float*)table + id * dim + d);
                v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
            }
        }
        *(float4*)(y + d) = make_float4(v[0], v[1], v[2], v[3]);
        return;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        if (ok && d + u < dim) {
            if (XK == XK_BF16) v[u] = __uint_as_float((uint32_t)((const uint16_t*)table)[id * dim + d + u] << 16);
            else v[u] = ((const float*)table)[id * dim + d + u];
        }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
    for (int u = 0; u < 4; ++u)
        if (d + u < dim) y[d + u] = v[u];
}

hipError_t launch_embed(const void* table, int xkind, int64_t vocab, int64_t dim, const int32_t* ids, int64_t m,
                        float* out, hipStream_t st)
{
    if (m <= 0) return hipSuccess;
    if (m > INT32_MAX || dim < 1 || dim > INT32_MAX - 1024) return hipErrorInvalidValue;
    const uintptr_t ta = xkind == XK_BF16 ? 7u : 15u;
    const bool vec = dim % 4 == 0 && ((uintptr_t)table & ta) == 0 && ((uintptr_t)out & 15u) == 0;
    const dim3 grid((unsigned)m, (unsigned)((dim + 1023) / 1024));
    if (xkind == XK_BF16)
        hipLaunchKernelGGL(k_embed<XK_BF16>, grid, dim3(256), 0, st, table, vocab, (int)dim, ids, out, vec);
    else hipLaunchKernelGGL(k_embed<XK_F32>, grid, dim3(256), 0, st, table, vocab, (int)dim, ids, out, vec);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// k_greedy: the greedy pick of stream_completion (llama.rs:509-515)
// ---------------------------------------------------------------------------
// Each value maps to a key that orders floats totally (-0 taken as +0; NaN
// above +inf: the reference's partial_cmp would panic there); (key, index)
// pairs compare lexicographically as one 64-bit word, so equal maxima resolve
// to the largest index, as Iterator::max_by does.  The maximum of a set of
// words does not depend on the order they are visited in, so the workgroups
// fold their maxima into one device word with an atomic max; the last
// workgroup to arrive (device counter) takes the word, writes the id -- with
// d_pos also log[*d_pos + 1] (the sequence position the token will take) --
// advances *d_pos, and leaves the word and the counter at zero for the next
// launch.
__device__ __forceinline__ uint64_t greedy_key(float f, uint32_t idx)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) == 0u) u = 0u;
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | idx;
}

struct GreedyState {
    uint64_t best;   // the running maximum word of the launch
    uint32_t count;  // workgroups done
};
// one state per output word next_id (KeySlots): launches that write the same
// next_id are ordered by their caller, others never share a state
constexpr int kGreedySlots = 64;
static __device__ GreedyState g_greedy[kGreedySlots];

constexpr int kGreedyU = 4;       // float4 loads in flight per thread
constexpr int kGreedyMaxWg = 256;

// grid G, block 256: workgroup b reads the float4s b * 256 + tid + G * 256 * u
__global__ __launch_bounds__(256) void k_greedy(const float* x, int n, int32_t* next_id, int32_t* d_pos,
                                                int32_t* log, int log_len, GreedyState* gs)
{
    __shared__ uint64_t s_best[4];
    const int tid = threadIdx.x;
    const int G = gridDim.x;
    const int n4 = n >> 2;
    uint64_t best = 0;
    for (int i0 = blockIdx.x * 256 + tid; i0 < n4; i0 += G * 256 * kGreedyU) {
        float4 v[kGreedyU];
#pragma unroll
        for (int u = 0; u < kGreedyU; ++u) {
            const int i = i0 + G * 256 * u;
            v[u] = i < n4 ? ((const float4*)x)[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int u = 0; u < kGreedyU; ++u) {
            const int i = i0 + G * 256 * u;
            if (i < n4) {
                best = max(best, greedy_key(v[u].x, 4 * i));
                best = max(best, greedy_key(v[u].y, 4 * i + 1));
                best = max(best, greedy_key(v[u].z, 4 * i + 2));
                best = max(best, greedy_key(v[u].w, 4 * i + 3));
            }
        }
    }
    if (blockIdx.x == 0)
        for (int i = 4 * n4 + tid; i < n; i += 256) best = max(best, greedy_key(x[i], i));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)best, off, 64);
        const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(best >> 32), off, 64);
        best = max(best, ((uint64_t)hi << 32) | lo);
    }
    if ((tid & 63) == 0) s_best[tid >> 6] = best;
    __syncthreads();
    if (tid != 0) return;
    for (int w = 1; w < 4; ++w) best = max(best, s_best[w]);
    uint64_t win = best;  // one workgroup (gs == NULL): its maximum is the answer
    if (gs) {
        __hip_atomic_fetch_max(&gs->best, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the maximum is folded in before the arrival counts
        const uint32_t old = __hip_atomic_fetch_add(&gs->count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old + 1u != (uint32_t)G) return;
        win = __hip_atomic_exchange(&gs->best, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&gs->count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const int32_t id = (int32_t)(uint32_t)win;
    next_id[0] = id;
    if (d_pos) {
        const int32_t p = *d_pos;
        if (log && p + 1 >= 0 && p + 1 < log_len) log[p + 1] = id;
        *d_pos = p + 1;
    }
}

hipError_t launch_greedy(const float* x, int64_t n, int32_t* next_id, int32_t* d_pos, int32_t* log, int64_t log_len,
                         hipStream_t st)
{
    static std::atomic<GreedyState*> ptr[64];
    static KeySlots<kGreedySlots> slots[64];
    if (n <= 0 || n > INT32_MAX) return hipErrorInvalidValue;
    int dev;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    GreedyState* base = ptr[dev].load(std::memory_order_acquire);
    if (!base) {
        void* q = nullptr;
        if ((e = hipGetSymbolAddress(&q, HIP_SYMBOL(g_greedy))) != hipSuccess) return e;
        base = (GreedyState*)q;
        ptr[dev].store(base, std::memory_order_release);
    }
    const int slot = slots[dev].find(next_id);
    // no state of its own left for this output: one workgroup, no shared state
    GreedyState* gs = slot < 0 ? nullptr : base + slot;
    const int64_t n4 = n >> 2;
    const int G = gs ? (int)std::min<int64_t>(kGreedyMaxWg, std::max<int64_t>(1, (n4 + 256 * kGreedyU - 1) / (256 * kGreedyU)))
                     : 1;
    hipLaunchKernelGGL(k_greedy, dim3((unsigned)G), dim3(256), 0, st, x, (int)n, next_id, d_pos, log,
                       (int)(log_len > INT32_MAX ? INT32_MAX : log_len), gs);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// k_rmsnorm_f32: RMSNorm::forward (rms_norm.rs:33-56) into f32 rows
// ---------------------------------------------------------------------------
// grid (m), block 256.  s = h (+ delta); the sum of s*s is the pairwise tree
// over the row in index order (zero-padded): thread t folds the 16 elements of
// group b * 256 + t (pairwise), the lanes' xor butterfly the 64 groups of a
// wave, then ((w0 + w1) + (w2 + w3)) the 256 groups of block b, and thread 0
// the blocks pairwise.  d = sqrt(sum * (f32)(1/k) + eps); y = (s / d) * g;
// h_out = s (written in the second pass, so h_out may be h).  k % 64 == 0.
__device__ __forceinline__ void rms_load16(const float* h, const float* delta, int k, int64_t e0, float* v)
{
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (e0 + 4 * q < k) {
            a = *(const float4*)(h + e0 + 4 * q);
            if (delta) {
                const float4 b = *(const float4*)(delta + e0 + 4 * q);
                a = make_float4(__fadd_rn(a.x, b.x), __fadd_rn(a.y, b.y), __fadd_rn(a.z, b.z), __fadd_rn(a.w, b.w));
            }
        }
        v[4 * q] = a.x; v[4 * q + 1] = a.y; v[4 * q + 2] = a.z; v[4 * q + 3] = a.w;
    }
}

constexpr int kRmsMaxBlocks = 16;  // k <= 16 * 4096

__global__ __launch_bounds__(256) void k_rmsnorm_f32(const float* h, const float* delta, float* h_out, const float* g,
                                                     float eps, int k, float* y)
{
    __shared__ float s_w[4];
    __shared__ float s_blk[kRmsMaxBlocks];
    __shared__ float s_d;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t row = (int64_t)blockIdx.x * k;
    h += row;
    if (delta) delta += row;
    y += row;
    if (h_out) h_out += row;
    const int nblk = (k + 4095) / 4096;
    for (int b = 0; b < nblk; ++b) {
        float v[16];
        rms_load16(h, delta, k, (int64_t)(b * 256 + tid) * 16, v);
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = __fmul_rn(v[e], v[e]);
#pragma unroll
        for (int len = 16; len > 1; len >>= 1)
#pragma unroll
            for (int i = 0; i < len / 2; ++i) v[i] = __fadd_rn(v[2 * i], v[2 * i + 1]);
        const float ws = wave_pairwise_sum(v[0]);
        if (lane == 0) s_w[wave] = ws;
        __syncthreads();
        if (tid == 0) s_blk[b] = __fadd_rn(__fadd_rn(s_w[0], s_w[1]), __fadd_rn(s_w[2], s_w[3]));
        __syncthreads();
    }
    if (tid == 0) {
        float p[kRmsMaxBlocks];
#pragma unroll
        for (int b = 0; b < kRmsMaxBlocks; ++b) p[b] = b < nblk ? s_blk[b] : 0.0f;
#pragma unroll
        for (int len = kRmsMaxBlocks; len > 1; len >>= 1)
#pragma unroll
            for (int i = 0; i < len / 2; ++i) p[i] = __fadd_rn(p[2 * i], p[2 * i + 1]);
        const float inv_k = (float)(1.0 / (double)k);
        s_d = sqrt_rn(__fadd_rn(__fmul_rn(p[0], inv_k), eps));
    }
    __syncthreads();
    const float d = s_d;
    for (int b = 0; b < nblk; ++b) {
        const int64_t e0 = (int64_t)(b * 256 + tid) * 16;
        if (e0 >= k) break;
        float v[16];
        rms_load16(h, delta, k, e0, v);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 gv = *(const float4*)(g + e0 + 4 * q);
            if (h_out) *(float4*)(h_out + e0 + 4 * q) = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
            *(float4*)(y + e0 + 4 * q) =
                make_float4(__fmul_rn(__fdiv_rn(v[4 * q], d), gv.x), __fmul_rn(__fdiv_rn(v[4 * q + 1], d), gv.y),
                            __fmul_rn(__fdiv_rn(v[4 * q + 2], d), gv.z), __fmul_rn(__fdiv_rn(v[4 * q + 3], d), gv.w));
        }
    }
}

hipError_t launch_rmsnorm_f32(const float* h, const float* delta, float* h_out, const float* g, float eps, int64_t m,
                              int64_t k, float* y, hipStream_t st)
{
    if (m < 1 || m > INT32_MAX || k < 64 || k % 64 || k > 4096 * kRmsMaxBlocks) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_rmsnorm_f32, dim3((unsigned)m), dim3(256), 0, st, h, delta, h_out, g, eps, (int)k, y);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// k_dense_gemv: candle_nn::Linear::forward without a bias (the dense lm_head,
// llama.rs:129-141), f32 sums in a fixed order
// ---------------------------------------------------------------------------
// grid (G, m), block 256: wave gw = 4 blockIdx.x + wave computes rows j = gw,
// gw + 4G, ... of token row blockIdx.y.  Lane l takes the 4-element chunks
// c = l, l + 64, ... of the row and folds each chunk's elements in order into
// acc = fma(x, w, acc); six butterfly steps (xor 32 .. 1) add the lanes.  KX >
// 0: k == 256 KX and the lane's x chunks stay in registers (one weight load per
// chunk, all KX in flight); KX == 0: any k % 4 == 0, eight chunks of w and x
// in flight at a time.  Weights are read once: non-temporal loads.
typedef uint32_t dense_u2 __attribute__((ext_vector_type(2)));
typedef float dense_f4 __attribute__((ext_vector_type(4)));

template <int WK>
__device__ __forceinline__ float4 dense_w4(const void* w, int64_t off)
{
    if (WK == XK_BF16) {
        const dense_u2 u = __builtin_nontemporal_load((const dense_u2*)((const uint16_t*)w + off));
        return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xFFFF0000u), __uint_as_float(u.y << 16),
                           __uint_as_float(u.y & 0xFFFF0000u));
    }
    const dense_f4 f = __builtin_nontemporal_load((const dense_f4*)((const float*)w + off));
    return make_float4(f.x, f.y, f.z, f.w);
}

__device__ __forceinline__ float fma4(float4 x, float4 w, float acc)
{
    acc = __fmaf_rn(x.x, w.x, acc);
    acc = __fmaf_rn(x.y, w.y, acc);
    acc = __fmaf_rn(x.z, w.z, acc);
    return __fmaf_rn(x.w, w.w, acc);
}

template <int WK, int KX>
__global__ __launch_bounds__(256) void k_dense_gemv(const void* w, int64_t n, int k, const float* x, float* y)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float4* xr = (const float4*)(x + (int64_t)blockIdx.y * k);
    float* yr = y + (int64_t)blockIdx.y * n;
    const int nc = k >> 2;
    const int64_t stride = (int64_t)gridDim.x * 4;
    float4 xv[KX > 0 ? KX : 1];
#pragma unroll
    for (int u = 0; u < KX; ++u) xv[u] = xr[lane + 64 * u];
    for (int64_t j = (int64_t)blockIdx.x * 4 + wave; j < n; j += stride) {
        const int64_t base = j * k;
        float acc = 0.0f;
        if (KX > 0) {
            float4 wv[KX > 0 ? KX : 1];
#pragma unroll
            for (int u = 0; u < KX; ++u) wv[u] = dense_w4<WK>(w, base + 4 * (lane + 64 * u));
#pragma unroll
            for (int u = 0; u < KX; ++u) acc = fma4(xv[u], wv[u], acc);
        } else {
            constexpr int kU = 8;
            for (int c0 = lane; c0 < nc; c0 += 64 * kU) {
                float4 wv[kU], xq[kU];
#pragma unroll
                for (int u = 0; u < kU; ++u) {
                    const int c = c0 + 64 * u;
                    wv[u] = c < nc ? dense_w4<WK>(w, base + 4 * c) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    xq[u] = c < nc ? xr[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                }
#pragma unroll
                for (int u = 0; u < kU; ++u)
                    if (c0 + 64 * u < nc) acc = fma4(xq[u], wv[u], acc);
            }
        }
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) acc = __fadd_rn(acc, __shfl_xor(acc, s, 64));
        if (lane == 0) yr[j] = acc;
    }
}

hipError_t launch_dense_gemv(const void* w, int wkind, int64_t n, int64_t k, const float* x, int64_t m, float* y,
                             hipStream_t st)
{
    if (n < 1 || m < 1 || m > 65535 || k < 4 || k % 4 || k > INT32_MAX / 2) return hipErrorInvalidValue;
    const unsigned G = (unsigned)std::min<int64_t>((n + 3) / 4, 1024);
    const dim3 grid(G, (unsigned)m), block(256);
    const bool xr = k == 4096;
#define BTL_DENSE(WKV)                                                                                   \
    if (xr) hipLaunchKernelGGL((k_dense_gemv<WKV, 16>), grid, block, 0, st, w, n, (int)k, x, y);        \
    else hipLaunchKernelGGL((k_dense_gemv<WKV, 0>), grid, block, 0, st, w, n, (int)k, x, y);
    if (wkind == XK_BF16) {
        BTL_DENSE(XK_BF16)
    } else {
        BTL_DENSE(XK_F32)
    }
#undef BTL_DENSE
    return hipGetLastError();
}

}  // namespace btl
