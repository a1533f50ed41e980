/*
 * bitlinear_oracle.c -- CPU restatement of the reference BitLinear hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or, for bench.py, as the timed CPU baseline).  The product library
 * (libbitlinear_hip.so) never links, loads or calls anything in oracle/.
 *
 * What is restated, and from where (paths are inside the reference repo
 * imonoonoko/Bit-TTT-Engine, crate crates/rust_engine):
 *
 *   orc_pack             src/kernels/packing.rs:50-105   (PackedTensor::pack)
 *   orc_unpack           src/kernels/packing.rs:108-133  (PackedTensor::unpack)
 *   orc_forward_f32      src/kernels/cpu.rs:17-127 + 132-239
 *                        (BitLinearCpu::forward + compute_row_avx2): the exact
 *                        fp32 summation order, emulated lane by lane in scalar C
 *   orc_forward_f32_avx2 the same algorithm written with AVX2/FMA intrinsics and
 *                        a thread pool over the M*N outputs (cpu.rs:73-76 uses
 *                        rayon) -- used as the timed CPU baseline; a test checks
 *                        it is bit-identical to orc_forward_f32
 *   orc_quantize_act     per-token absmax int8 activation quantisation.  The
 *                        reference has none on this path; the convention is the
 *                        BitNet b1.58 one (q = round(x * 127/absmax)) with the
 *                        absmax/127 scale of src/layers/kv_cache.rs:95-119.
 *   orc_contract_i8      exact int32 ternary contraction acc = sum_k q*t
 *   orc_epilogue         y = (float)acc * (s_x * s_w), fixed op order
 *   orc_bf16_*           bf16 <-> f32 (round-to-nearest-even)
 *   orc_pairwise_sum     the fixed reduction order of the fused RMSNorm: a
 *                        pairwise tree over the elements in index order,
 *                        zero-padded to a power of two
 *   orc_rmsnorm          src/layers/rms_norm.rs:33-56 (RMSNorm::forward) with
 *                        candle 0.8's scalar ops (Tensor / f64 and + f64 are
 *                        affine(1/d, 0) and affine(1, eps) in f32): x / sqrt(
 *                        sum(x*x) * (f32)(1/k) + (f32)eps) * g; the sum in the
 *                        pairwise order above (candle's own reduction order is
 *                        not vendored: its last ulp is parity unpinned)
 *   orc_expf             exp in f32 by Cody-Waite reduction and a degree-7
 *                        Taylor polynomial (textbook method), every step a
 *                        separately rounded f32 operation; the GPU kernels run
 *                        the same sequence, so the two agree bit for bit
 *   orc_swiglu           src/layers/swiglu.rs:29-35: silu(g) * u with candle's
 *                        silu v / (1 + exp(-v)), exp from orc_expf (Rust's
 *                        f32::exp is libm's: ulp-level parity unpinned)
 *
 * Parity status of each function, and what pins it, is listed in the header
 * of tests/test_oracle.py; the short version: the packing layout, codes and the
 * fp32 contraction order are pinned by the reference's own unit tests
 * (packing.rs:155-261), closed forms and brute force; the last ulp of the
 * weight scale (candle's mean_all reduction order) is parity unpinned.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef __AVX2__
#include <immintrin.h>
#endif

#define ORC_OK 0
#define ORC_ERR_SHAPE 1
#define ORC_ERR_ARG 6

/* ------------------------------------------------------------------ */
/* bf16 helpers                                                         */
/* ------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_bf16_to_f32(uint16_t h) { return u2f(((uint32_t)h) << 16); }

/* Round-to-nearest-even f32 -> bf16; NaN becomes the quiet NaN 0x7FC0. */
uint16_t orc_f32_to_bf16(float f)
{
    uint32_t u = f2u(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void orc_bf16_to_f32_array(const uint16_t* h, int64_t n, float* out)
{
    for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_to_f32(h[i]);
}

void orc_f32_to_bf16_array(const float* f, int64_t n, uint16_t* out)
{
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(f[i]);
}

/* ------------------------------------------------------------------ */
/* A2: PackedTensor::pack  (packing.rs:50-105)                          */
/* ------------------------------------------------------------------ */
/*
 * scale = mean(|W|) + 1e-6   (packing.rs:4,56-57)
 * t     = clamp(round(W / scale), -1, 1)  (packing.rs:61-65)
 *         candle implements `tensor / f64` as an affine map x * (1/rhs); the
 *         restatement therefore multiplies by (float)(1.0 / (double)scale).
 *         round() is f32::round, i.e. half away from zero (C roundf).
 * code  = 1 if t > 0.5, 2 if t < -0.5, else 0  (packing.rs:82-88)
 * byte e/4 holds element e at bits 2*(e%4), little end first (packing.rs:74-92);
 * the last byte's unused fields stay 00.
 *
 * The mean is accumulated in double as the pairwise tree over |w| in index
 * order (zero-padded to a power of two: any thread count reproduces it) and
 * rounded once to f32.  candle's mean_all accumulates in f32 in an order set by
 * its CPU reduction kernel, which is not vendored with the reference, so the
 * last ulp of the scale is parity unpinned (pinned to 1e-3 by
 * packing.rs:166,184 and by closed forms).
 */
static double orc_abs_pairwise(const float* w, int64_t numel, int64_t a, int64_t len)
{
    if (len == 1) return a < numel ? fabs((double)w[a]) : 0.0;
    const int64_t h = len / 2;
    const double lo = orc_abs_pairwise(w, numel, a, h);
    const double hi = a + h < numel ? orc_abs_pairwise(w, numel, a + h, h) : 0.0;
    return lo + hi;
}

int orc_pack(const float* w, int64_t numel, uint8_t* out, float* scale_out)
{
    if (numel < 0 || (!w && numel) || !scale_out) return ORC_ERR_ARG;
    int64_t len = 1;
    while (len < numel) len *= 2;
    const double acc = numel ? orc_abs_pairwise(w, numel, 0, len) : 0.0;
    float mean = numel ? (float)(acc / (double)numel) : 0.0f;
    float scale = mean + 1e-6f;
    float inv = (float)(1.0 / (double)scale);
    int64_t nbytes = (numel + 3) / 4;
    memset(out, 0, (size_t)nbytes);
    for (int64_t e = 0; e < numel; ++e) {
        float v = roundf(w[e] * inv);
        if (v > 1.0f) v = 1.0f;
        if (v < -1.0f) v = -1.0f;
        uint8_t code = v > 0.5f ? 1 : (v < -0.5f ? 2 : 0);
        out[e >> 2] |= (uint8_t)(code << (2 * (e & 3)));
    }
    *scale_out = scale;
    return ORC_OK;
}

/* A4: PackedTensor::unpack (packing.rs:108-133): 1 -> +1, 2 -> -1, else 0, times scale. */
void orc_unpack(const uint8_t* data, int64_t numel, float scale, float* out)
{
    for (int64_t e = 0; e < numel; ++e) {
        uint8_t code = (data[e >> 2] >> (2 * (e & 3))) & 3u;
        float v = code == 1 ? 1.0f : (code == 2 ? -1.0f : 0.0f);
        out[e] = v * scale;
    }
}

/* Ternary value of element e of the flat packed buffer. */
static inline int orc_tern(const uint8_t* data, int64_t e)
{
    int code = (data[e >> 2] >> (2 * (e & 3))) & 3;
    return (code & 1) - (code >> 1); /* cpu.rs:161-166: (c&1) - (c>>1) */
}

/* ------------------------------------------------------------------ */
/* A6/A7: BitLinearCpu::forward, exact fp32 order  (cpu.rs:17-239)      */
/* ------------------------------------------------------------------ */
/*
 * Per output (i, j), cpu.rs:77-123:
 *   row start in the packed bytes = j * ceil(K/4)                 (cpu.rs:81)
 *   AVX2 part over the first 32*floor(K/32) inputs                (cpu.rs:86-102)
 *     one 8-lane accumulator; for each 32-weight chunk, 4 groups of 8:
 *     load u16 (2 bytes, 8 codes), coeff_b = (c&1)-(c>>1) for code b,
 *     lane b = fma(x[8g+b], coeff_b, lane b)                      (cpu.rs:192-221)
 *     result = sequential sum of lanes 0..7                       (cpu.rs:236-238)
 *   scalar tail over the remaining inputs, LUT [0,1,-1,0], stops if the byte
 *   index runs past the buffer                                    (cpu.rs:105-122)
 *   y = sum * scale                                               (cpu.rs:123)
 * Every product is x*{-1,0,1}, which is exact, so fma(x,c,s) == s + x*c and the
 * lane emulation below is bit-identical to the intrinsics.  avx2_order = 0
 * restates the non-AVX2 branch (pure sequential scalar loop).
 */
static float orc_row_f32(const float* xr, const uint8_t* w, int64_t wbytes, int64_t row_start,
                         int64_t k, float scale, int avx2_order)
{
    static const float LUT[4] = {0.0f, 1.0f, -1.0f, 0.0f};
    float sum = 0.0f;
    int64_t processed = 0;
    if (avx2_order) {
        int64_t nchunks = k / 32;
        float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        const uint8_t* wp = w + row_start;
        const float* xp = xr;
        for (int64_t c = 0; c < nchunks; ++c) {
            for (int g = 0; g < 4; ++g) {
                uint16_t wv = (uint16_t)(wp[0] | ((uint16_t)wp[1] << 8));
                wp += 2;
                for (int b = 0; b < 8; ++b) {
                    int code = (wv >> (2 * b)) & 3;
                    float coeff = (float)((code & 1) - (code >> 1));
                    lane[b] = fmaf(xp[b], coeff, lane[b]);
                }
                xp += 8;
            }
        }
        float r = -0.0f; /* Iterator::sum over the 8 stored lanes */
        for (int b = 0; b < 8; ++b) r += lane[b];
        sum += r;
        processed = nchunks * 32;
    }
    for (int64_t l = processed; l < k; ++l) {
        float xv = xr[l];
        int64_t byte_idx = l / 4;
        if (row_start + byte_idx >= wbytes) break;
        uint8_t byte = w[row_start + byte_idx];
        int code = (byte >> ((l % 4) * 2)) & 3;
        sum += xv * LUT[code];
    }
    return sum * scale;
}

/*
 * x [m,k] f32, w = packed bytes (wbytes long, normally ceil(n*k/4)), y [m,n].
 * The AVX2 branch reads 2*4*floor(k/32) bytes from each row start; if that
 * would run past wbytes (possible only for k % 4 != 0, where the reference's
 * row stride ceil(k/4) disagrees with the flat packing) the reference reads out
 * of bounds, so the restatement refuses with ORC_ERR_SHAPE instead.
 */
int orc_forward_f32(const float* x, int64_t m, int64_t k, const uint8_t* w, int64_t n,
                    int64_t wbytes, float scale, float* y, int avx2_order)
{
    if (m < 0 || n < 0 || k < 0) return ORC_ERR_ARG;
    int64_t stride = (k + 3) / 4;
    if (avx2_order && m > 0 && n > 0) {
        int64_t last = (n - 1) * stride + 8 * (k / 32);
        if (last > wbytes) return ORC_ERR_SHAPE;
    }
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j)
            y[i * n + j] = orc_row_f32(x + i * k, w, wbytes, j * stride, k, scale, avx2_order);
    return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* Timed CPU baseline: the same algorithm with AVX2/FMA intrinsics and  */
/* a pthread pool over M*N outputs (rayon par_iter_mut in cpu.rs:73).   */
/* ------------------------------------------------------------------ */
typedef struct {
    const float* x; const uint8_t* w; float* y;
    int64_t m, n, k, wbytes; float scale;
    int64_t begin, end;
} orc_job_t;

#ifdef __AVX2__
__attribute__((target("avx2,fma")))
static float orc_row_avx2(const float* xr, const uint8_t* wp, int64_t nchunks)
{
    __m256 sum_vec = _mm256_setzero_ps();
    for (int64_t c = 0; c < nchunks; ++c) {
        for (int g = 0; g < 4; ++g) {
            uint16_t wv;
            memcpy(&wv, wp, 2);
            wp += 2;
            float coeffs[8];
            for (int b = 0; b < 8; ++b) {
                int code = (wv >> (2 * b)) & 3;
                coeffs[b] = (float)((code & 1) - (code >> 1));
            }
            __m256 w_vec = _mm256_loadu_ps(coeffs);
            __m256 x_vec = _mm256_loadu_ps(xr);
            xr += 8;
            sum_vec = _mm256_fmadd_ps(x_vec, w_vec, sum_vec);
        }
    }
    float temp[8];
    _mm256_storeu_ps(temp, sum_vec);
    float r = -0.0f;
    for (int b = 0; b < 8; ++b) r += temp[b];
    return r;
}
#endif

static void* orc_worker(void* arg)
{
    static const float LUT[4] = {0.0f, 1.0f, -1.0f, 0.0f};
    orc_job_t* jb = (orc_job_t*)arg;
    int64_t stride = (jb->k + 3) / 4;
    for (int64_t g = jb->begin; g < jb->end; ++g) {
        int64_t i = g / jb->n, j = g % jb->n;
        const float* xr = jb->x + i * jb->k;
        int64_t row_start = j * stride;
        float sum = 0.0f;
        int64_t processed = 0;
#ifdef __AVX2__
        int64_t nchunks = jb->k / 32;
        sum += orc_row_avx2(xr, jb->w + row_start, nchunks);
        processed = nchunks * 32;
#endif
        for (int64_t l = processed; l < jb->k; ++l) {
            int64_t byte_idx = l / 4;
            if (row_start + byte_idx >= jb->wbytes) break;
            int code = (jb->w[row_start + byte_idx] >> ((l % 4) * 2)) & 3;
            sum += xr[l] * LUT[code];
        }
        jb->y[g] = sum * jb->scale;
    }
    return NULL;
}

/* Returns 1 when the library was built with the AVX2 path, 0 otherwise. */
int orc_has_avx2(void)
{
#ifdef __AVX2__
    return 1;
#else
    return 0;
#endif
}

int orc_forward_f32_avx2(const float* x, int64_t m, int64_t k, const uint8_t* w, int64_t n,
                         int64_t wbytes, float scale, float* y, int threads)
{
    if (m < 0 || n < 0 || k < 0) return ORC_ERR_ARG;
    int64_t stride = (k + 3) / 4;
    if (m > 0 && n > 0 && (n - 1) * stride + 8 * (k / 32) > wbytes) return ORC_ERR_SHAPE;
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    int64_t total = m * n;
    if (total == 0) return ORC_OK;
    if ((int64_t)threads > total) threads = (int)total;
    pthread_t tid[256];
    int joined[256];
    orc_job_t jobs[256];
    int64_t per = (total + threads - 1) / threads;
    for (int t = 0; t < threads; ++t) {
        orc_job_t jb = {x, w, y, m, n, k, wbytes, scale, t * per, (t + 1) * per};
        if (jb.end > total) jb.end = total;
        if (jb.begin > total) jb.begin = total;
        jobs[t] = jb;
        joined[t] = 0;
        if (t == 0 || jb.begin >= jb.end) continue; /* slice 0 runs on the caller */
        if (pthread_create(&tid[t], NULL, orc_worker, &jobs[t]) == 0) joined[t] = 1;
        else orc_worker(&jobs[t]);
    }
    orc_worker(&jobs[0]);
    for (int t = 1; t < threads; ++t)
        if (joined[t]) pthread_join(tid[t], NULL);
    return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* A8: per-token absmax int8 activation quantisation (build-defined)   */
/* ------------------------------------------------------------------ */
/*
 * For each row m:
 *   a  = max_k |x[m,k]|, taken as the max of the IEEE bit patterns with the
 *        sign cleared, so a NaN anywhere makes the row non-finite
 *   a non-finite        -> s = NaN,  q = 0      (outputs of the row become NaN)
 *   a <  2^-100         -> s = 0,    q = 0      (zero / negligible row)
 *   else r = 127.0f / a, s = a / 127.0f, q = clamp(round_half_away(x*r), -127, 127)
 * round_half_away is Rust's f32::round (kv_cache.rs:104-108 rounds x/s with it).
 * The 2^-100 floor keeps r finite and makes the result independent of how a
 * device treats fp32 subnormals (|x*r| < 2^-19 for any subnormal x).
 */
#define ORC_QMIN_BITS 0x0D800000u /* 2^-100 */

void orc_row_qparams(const float* xr, int64_t k, float* r_out, float* s_out, int* mode_out)
{
    uint32_t amax = 0;
    for (int64_t i = 0; i < k; ++i) {
        uint32_t b = f2u(xr[i]) & 0x7FFFFFFFu;
        if (b > amax) amax = b;
    }
    if (amax >= 0x7F800000u) { *r_out = 0.0f; *s_out = u2f(0x7FC00000u); *mode_out = 2; return; }
    if (amax < ORC_QMIN_BITS) { *r_out = 0.0f; *s_out = 0.0f; *mode_out = 0; return; }
    float a = u2f(amax);
    *r_out = 127.0f / a;
    *s_out = a / 127.0f;
    *mode_out = 1;
}

void orc_quantize_act(const float* x, int64_t m, int64_t k, int8_t* q, float* s)
{
    for (int64_t i = 0; i < m; ++i) {
        const float* xr = x + i * k;
        float r, sc; int mode;
        orc_row_qparams(xr, k, &r, &sc, &mode);
        s[i] = sc;
        for (int64_t j = 0; j < k; ++j) {
            int v = 0;
            if (mode == 1) {
                float t = roundf(xr[j] * r);
                if (t > 127.0f) t = 127.0f;
                if (t < -127.0f) t = -127.0f;
                v = (int)t;
            }
            q[i * k + j] = (int8_t)v;
        }
    }
}

/* ------------------------------------------------------------------ */
/* A9: exact integer contraction, A10: epilogue                        */
/* ------------------------------------------------------------------ */
/* acc[i,j] = sum_k q[i,k] * t[j,k], element e = j*k + kk of the flat packing. */
void orc_contract_i8(const int8_t* q, int64_t m, int64_t k, const uint8_t* w, int64_t n,
                     int32_t* acc)
{
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            int64_t a = 0;
            for (int64_t kk = 0; kk < k; ++kk) a += (int64_t)q[i * k + kk] * orc_tern(w, j * k + kk);
            acc[i * n + j] = (int32_t)a;
        }
}

/* y[i,j] = (float)acc[i,j] * (s_x[i] * s_w): the scale product is rounded first. */
void orc_epilogue(const int32_t* acc, const float* sx, float sw, int64_t m, int64_t n, float* y)
{
    for (int64_t i = 0; i < m; ++i) {
        float c = sx[i] * sw;
        for (int64_t j = 0; j < n; ++j) y[i * n + j] = (float)acc[i * n + j] * c;
    }
}

/* ------------------------------------------------------------------ */
/* Fused activation transforms (RMSNorm, SwiGLU) ahead of quantisation */
/* ------------------------------------------------------------------ */
/* sum of v[0..n) as the pairwise tree over `len` (a power of two >= n) leaves,
 * leaves past n being +0: sum(v[a, a+2h)) = sum(v[a, a+h)) + sum(v[a+h, a+2h)). */
static float orc_pairwise(const float* v, int64_t n, int64_t len)
{
    if (len == 1) return n > 0 ? v[0] : 0.0f;
    const int64_t h = len / 2;
    const float a = orc_pairwise(v, n < h ? n : h, h);
    const float b = n > h ? orc_pairwise(v + h, n - h, h) : 0.0f;
    return a + b;
}

float orc_pairwise_sum(const float* v, int64_t n)
{
    int64_t len = 1;
    while (len < n) len *= 2;
    return orc_pairwise(v, n, len);
}

/* rms_norm.rs:33-56: out = x / sqrt(ss * (f32)(1/k) + (f32)eps) * g per row,
 * ss = pairwise sum of x*x (products rounded to f32 first). */
void orc_rmsnorm(const float* x, int64_t m, int64_t k, const float* g, float eps, float* out)
{
    float* sq = (float*)malloc(sizeof(float) * (size_t)(k > 0 ? k : 1));
    const float inv_k = (float)(1.0 / (double)k);
    for (int64_t i = 0; i < m; ++i) {
        const float* xr = x + i * k;
        for (int64_t j = 0; j < k; ++j) sq[j] = xr[j] * xr[j];
        const float ms = orc_pairwise_sum(sq, k) * inv_k;
        const float d = sqrtf(ms + eps);
        for (int64_t j = 0; j < k; ++j) out[i * k + j] = (xr[j] / d) * g[j];
    }
    free(sq);
}

/* exp(x), Cody-Waite: x = n ln2 + r with ln2 = hi + lo (hi has 15 significant
 * bits, so n*hi is exact for |n| < 512), |r| <= ln2/2; e^r by the Taylor
 * polynomial to r^7/7! (truncation < 2^-27) in Horner form; the result scaled
 * by 2^n through exponent bits (two exact steps below 2^-126 or above 2^127). */
float orc_expf(float x)
{
    if (x != x) return x;
    if (x > 88.72283935546875f) return u2f(0x7F800000u);
    if (x < -103.97208404541016f) return 0.0f;
    const float n = rintf(x * 1.44269502162933349609375f);
    const float r = (x - n * 0.693145751953125f) - n * 1.428606765330187045037746429443359375e-6f;
    float p = 1.98412701138295233249664306640625e-4f;  /* 1/5040 */
    p = p * r + 1.3888889225199818611145019531250e-3f; /* 1/720 */
    p = p * r + 8.3333337679505348205566406250e-3f;    /* 1/120 */
    p = p * r + 4.1666667908430099487304687500e-2f;    /* 1/24 */
    p = p * r + 0.16666667163372039794921875f;         /* 1/6 */
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    const int ni = (int)n;
    if (ni > 127) return (p * u2f((uint32_t)(127 + 127) << 23)) * u2f((uint32_t)(ni - 127 + 127) << 23);
    if (ni < -126) return (p * u2f((uint32_t)(ni + 64 + 127) << 23)) * u2f((uint32_t)(-64 + 127) << 23);
    return p * u2f((uint32_t)(ni + 127) << 23);
}

/* swiglu.rs:29-35 (candle silu = v / (1 + exp(-v))): out = silu(g) * u. */
void orc_swiglu(const float* g, const float* u, int64_t n, float* out)
{
    for (int64_t i = 0; i < n; ++i) {
        const float v = g[i];
        const float si = v / (1.0f + orc_expf(-v));
        out[i] = si * u[i];
    }
}

/* Full W1.58-A8 forward: quantise, contract, scale.  q/sx/acc may be NULL. */
int orc_forward_i8(const float* x, int64_t m, int64_t k, const uint8_t* w, int64_t n,
                   float sw, float* y, int8_t* q_out, float* sx_out, int32_t* acc_out)
{
    if (m < 0 || n < 0 || k < 0) return ORC_ERR_ARG;
    int8_t* q = q_out ? q_out : (int8_t*)malloc((size_t)(m * k) + 1);
    float* sx = sx_out ? sx_out : (float*)malloc(sizeof(float) * (size_t)m + 4);
    int32_t* acc = acc_out ? acc_out : (int32_t*)malloc(sizeof(int32_t) * (size_t)(m * n) + 4);
    if (!q || !sx || !acc) return ORC_ERR_ARG;
    orc_quantize_act(x, m, k, q, sx);
    orc_contract_i8(q, m, k, w, n, acc);
    orc_epilogue(acc, sx, sw, m, n, y);
    if (!q_out) free(q);
    if (!sx_out) free(sx);
    if (!acc_out) free(acc);
    return ORC_OK;
}
