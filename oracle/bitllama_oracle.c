/*
 * bitllama_oracle.c -- CPU restatement of the reference's decoder ops around
 * the BitLinear path (rotary embedding, the Q8 KV cache, attention, greedy
 * argmax).
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker.
 * The product library (libbitlinear_hip.so) never links, loads or calls it.
 *
 * Restated from (paths inside imonoonoko/Bit-TTT-Engine, crate crates/rust_engine):
 *
 *   orc_rope_table   src/layers/attention.rs:15-42 (RotaryEmbedding::new):
 *                    inv_freq = 1.0f / (f32)theta^(2i/hd) (the f64 power rounded
 *                    to f32, then an f32 division: `as` binds before `/` at :19),
 *                    freq = (f32)p * inv_freq,
 *                    cos / sin in f32 (cosf / sinf, the libm Rust's f32::cos
 *                    calls on Linux)
 *   orc_rope_apply   src/layers/attention.rs:46-87 (RotaryEmbedding::apply):
 *                    [x1*cos - x2*sin, x1*sin + x2*cos], every op rounded
 *   orc_q8_quant     src/layers/kv_cache.rs:95-119 (quantize_q8): s = max|x| *
 *                    (f32)(1/127) + 0 (candle's Tensor / f64 is an affine multiply),
 *                    code = u8(round(x / s) + 128) with Rust's saturating
 *                    `as u8` (NaN -> 0)
 *   orc_q8_dequant   src/layers/kv_cache.rs:122-128 (dequantize_q8):
 *                    ((f32)code - 128) * s
 *   orc_attn_decode  src/layers/attention.rs:149-224 (BitAttention::forward at
 *                    one query position): softmax(q.k * (1/sqrt(hd))) . v over
 *                    the dequantised cache, GQA head h -> kv head h / (nh/nkv)
 *                    (repeat_kv, :227-239).  The reference's sums run in candle's
 *                    gemm order (not vendored); this restatement fixes the order
 *                    the GPU kernels use, so the two agree bit for bit:
 *                      dot(q, k_j) = orc_attn_dot: one fused multiply-add per
 *                      term, sequential over d (acc = fma(q[d], k_j[d], acc)),
 *                      scaled by (f32)(1/sqrt(hd));
 *                      keys in chunks of 64: m_c = max, p_j = exp(s_j - m_c),
 *                      l_c = pairwise tree over the 64 lanes (zero-padded),
 *                      o_c[d] = the same fma chain over j of p_j * v_j[d];
 *                      M = max_c m_c, w_c = exp(m_c - M), L = sum_c w_c * l_c,
 *                      O[d] = sum_c w_c * o_c[d] (sequential over c), y = O / L.
 *                    exp is orc_expf (bitlinear_oracle.c).  tests/test_model_oracle.py
 *                    pins the result against a float64 softmax-attention.
 *   orc_dense_linear candle_nn::Linear::forward without a bias (the dense lm_head of
 *                    llama.rs:129-141) in f32 with the GPU kernel's fixed order
 *                    (64 lane partial sums of fmas, then a butterfly; see below)
 *   orc_argmax       the greedy pick of Llama::stream_completion (llama.rs:509-515):
 *                    Iterator::max_by(partial_cmp) returns the LAST maximum
 *   orc_adaptive_reconstruct  AdaptiveBitLinear::load (adaptive_linear.rs:86-117): the
 *                    dense f32 weights of the multi-base format, bases added in order
 *   orc_adaptive_split        the interleaved [n, k/4, nb] bytes -> nb PackedTensor arrays
 *   orc_adaptive_forward_i8   W1.58-A8 over the bases (build-defined; the reference runs
 *                    a dense f32 matmul of the reconstruction, adaptive_linear.rs:131-160)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

float orc_expf(float x);
float orc_pairwise_sum(const float* v, int64_t n);

void orc_rope_table(double theta, int64_t hd, int64_t max_seq, float* cos_t, float* sin_t)
{
    const int64_t half = hd / 2;
    float* inv = (float*)malloc(sizeof(float) * (size_t)(half > 0 ? half : 1));
    /* attention.rs:19: `1.0 / (theta.powf(..)) as f32` rounds the power to f32 first,
     * then divides in f32 */
    for (int64_t i = 0; i < half; ++i) {
        const float pw = (float)pow(theta, (double)(2 * i) / (double)hd);
        inv[i] = 1.0f / pw;
    }
    for (int64_t p = 0; p < max_seq; ++p)
        for (int64_t i = 0; i < half; ++i) {
            const float f = (float)p * inv[i];
            cos_t[p * half + i] = cosf(f);
            sin_t[p * half + i] = sinf(f);
        }
    free(inv);
}

void orc_rope_apply(const float* x, int64_t hd, const float* c, const float* s, float* out)
{
    const int64_t half = hd / 2;
    for (int64_t i = 0; i < half; ++i) {
        const float x1 = x[i], x2 = x[i + half];
        const float a = x1 * c[i], b = x2 * s[i];
        const float e = x1 * s[i], f = x2 * c[i];
        out[i] = a - b;
        out[i + half] = e + f;
    }
}

static uint8_t sat_u8(float r)
{
    if (r != r || r <= 0.0f) return 0;
    if (r >= 255.0f) return 255;
    return (uint8_t)r;
}

void orc_q8_quant(const float* x, int64_t hd, uint8_t* q, float* s_out)
{
    float amax = fabsf(x[0]);
    for (int64_t d = 1; d < hd; ++d) {
        const float a = fabsf(x[d]);
        if (a > amax) amax = a;
    }
    /* kv_cache.rs:101 `max_val / 127.0` is candle's Tensor / f64 = affine(1/127, 0):
     * x * (f32)(1/127) + 0 -- a multiply by the rounded reciprocal, not a division */
    const float s = amax * (float)(1.0 / 127.0) + 0.0f;
    for (int64_t d = 0; d < hd; ++d) q[d] = sat_u8(roundf(x[d] / s) + 128.0f);
    *s_out = s;
}

void orc_q8_dequant(const uint8_t* q, int64_t hd, float s, float* out)
{
    for (int64_t d = 0; d < hd; ++d) out[d] = ((float)q[d] - 128.0f) * s;
}

#define ORC_CHUNK 64

/* The dot product of the attention scores and value sums: one fused
 * multiply-add per term (a single rounding), sequential over the terms. */
float orc_attn_dot(const float* a, const float* b, int64_t n, int64_t stride_b)
{
    float acc = 0.0f;
    for (int64_t i = 0; i < n; ++i) acc = fmaf(a[i], b[i * stride_b], acc);
    return acc;
}

/* q: [nh * hd] (rotated); cache arrays of ONE layer: kq/vq [nkv][max_seq][hd],
 * ks/vs [nkv][max_seq]; keys [0, T).  out: [nh * hd]. */
void orc_attn_decode(const float* q, const uint8_t* kq, const float* ks, const uint8_t* vq, const float* vs,
                     int64_t nh, int64_t nkv, int64_t hd, int64_t max_seq, int64_t T, float* out)
{
    const int64_t rep = nh / nkv;
    const float scal = (float)(1.0 / sqrt((double)hd));
    const int64_t C = (T + ORC_CHUNK - 1) / ORC_CHUNK;
    float* mc = (float*)malloc(sizeof(float) * (size_t)(C + 1));
    float* lc = (float*)malloc(sizeof(float) * (size_t)(C + 1));
    float* oc = (float*)malloc(sizeof(float) * (size_t)((C + 1) * hd));
    float* kd = (float*)malloc(sizeof(float) * (size_t)hd);
    float* vdq = (float*)malloc(sizeof(float) * (size_t)(ORC_CHUNK * hd));
    float sc[ORC_CHUNK], p[ORC_CHUNK];
    for (int64_t h = 0; h < nh; ++h) {
        const int64_t g = h / rep;
        const float* qh = q + h * hd;
        for (int64_t c = 0; c < C; ++c) {
            const int64_t j0 = c * ORC_CHUNK;
            const int64_t nj = T - j0 < ORC_CHUNK ? T - j0 : ORC_CHUNK;
            float m = -INFINITY;
            for (int64_t j = 0; j < nj; ++j) {
                const int64_t row = g * max_seq + j0 + j;
                orc_q8_dequant(kq + row * hd, hd, ks[row], kd);
                const float acc = orc_attn_dot(qh, kd, hd, 1);
                sc[j] = acc * scal + 0.0f; /* candle affine(mul, add): v * mul + add */
                if (sc[j] > m) m = sc[j];
            }
            for (int64_t j = 0; j < ORC_CHUNK; ++j) p[j] = j < nj ? orc_expf(sc[j] - m) : 0.0f;
            mc[c] = m;
            lc[c] = orc_pairwise_sum(p, ORC_CHUNK);
            for (int64_t j = 0; j < nj; ++j) {
                const int64_t row = g * max_seq + j0 + j;
                orc_q8_dequant(vq + row * hd, hd, vs[row], vdq + j * hd);
            }
            for (int64_t d = 0; d < hd; ++d) oc[c * hd + d] = orc_attn_dot(p, vdq + d, nj, hd);
        }
        float M = -INFINITY;
        for (int64_t c = 0; c < C; ++c)
            if (mc[c] > M) M = mc[c];
        float L = 0.0f;
        for (int64_t c = 0; c < C; ++c) L = L + orc_expf(mc[c] - M) * lc[c];
        for (int64_t d = 0; d < hd; ++d) {
            float O = 0.0f;
            for (int64_t c = 0; c < C; ++c) O = O + orc_expf(mc[c] - M) * oc[c * hd + d];
            out[h * hd + d] = O / L;
        }
    }
    free(mc);
    free(lc);
    free(oc);
    free(kd);
    free(vdq);
}

int64_t orc_argmax(const float* x, int64_t n)
{
    int64_t best = 0;
    for (int64_t i = 1; i < n; ++i)
        if (!(x[i] < x[best])) best = i;  /* max_by keeps the later of equal elements */
    return best;
}

/* ------------------------------------------------------------------ */
/* Multi-base adaptive format (AdaptiveBitLinear, adaptive_linear.rs)  */
/* ------------------------------------------------------------------ */
/* weight_packed [n, k/4, nb] u8 (adaptive_linear.rs:60, producer
 * convert_llama_v2.py:111-151): byte (row, cp, b) holds the 2-bit codes of
 * base b for columns 4cp..4cp+3 at bits 2j; scales [nb] f32. */

static float orc_lut(int code) { return code == 1 ? 1.0f : (code == 2 ? -1.0f : 0.0f); }

/* AdaptiveBitLinear::load's dense reconstruction (adaptive_linear.rs:86-117):
 * per row, bases in order, row_w[4cp + j] += LUT[byte][j] * scale[b]. */
void orc_adaptive_reconstruct(const uint8_t* packed, const float* scales, int64_t nb, int64_t n, int64_t k, float* out)
{
    const int64_t kp = k / 4;
    for (int64_t r = 0; r < n; ++r) {
        float* w = out + r * k;
        for (int64_t c = 0; c < k; ++c) w[c] = 0.0f;
        for (int64_t b = 0; b < nb; ++b) {
            const float s = scales[b];
            for (int64_t cp = 0; cp < kp; ++cp) {
                const uint8_t byte = packed[r * kp * nb + cp * nb + b];
                for (int j = 0; j < 4; ++j) w[cp * 4 + j] += orc_lut((byte >> (2 * j)) & 3) * s;
            }
        }
    }
}

/* The interleaved bytes -> nb standard PackedTensor byte arrays [n, k/4] each. */
void orc_adaptive_split(const uint8_t* packed, int64_t nb, int64_t n, int64_t k, uint8_t* out)
{
    const int64_t kp = k / 4;
    for (int64_t b = 0; b < nb; ++b)
        for (int64_t r = 0; r < n; ++r)
            for (int64_t cp = 0; cp < kp; ++cp) out[b * n * kp + r * kp + cp] = packed[r * kp * nb + cp * nb + b];
}

void orc_quantize_act(const float* x, int64_t m, int64_t k, int8_t* q, float* s);
void orc_contract_i8(const int8_t* q, int64_t m, int64_t k, const uint8_t* w, int64_t n, int32_t* acc);

/* W1.58-A8 multi-base forward (build-defined): the activations quantised as
 * for BitLinear, acc_b = sum_k q * t_b exact per base, and
 * y = (float)acc_0 * (s_x * s_0) + (float)acc_1 * (s_x * s_1) + ... in base order. */
int orc_adaptive_forward_i8(const float* x, int64_t m, int64_t k, const uint8_t* packed, const float* scales,
                            int64_t nb, int64_t n, float* y)
{
    const int64_t kp = k / 4;
    int8_t* q = (int8_t*)malloc((size_t)(m * k) + 1);
    float* sx = (float*)malloc(sizeof(float) * (size_t)(m + 1));
    int32_t* acc = (int32_t*)malloc(sizeof(int32_t) * (size_t)(m * n + 1));
    uint8_t* split = (uint8_t*)malloc((size_t)(nb * n * kp) + 1);
    if (!q || !sx || !acc || !split) return 1;
    orc_quantize_act(x, m, k, q, sx);
    orc_adaptive_split(packed, nb, n, k, split);
    for (int64_t b = 0; b < nb; ++b) {
        orc_contract_i8(q, m, k, split + b * n * kp, n, acc);
        for (int64_t i = 0; i < m; ++i) {
            const float c = sx[i] * scales[b];
            for (int64_t j = 0; j < n; ++j) {
                const float v = (float)acc[i * n + j] * c;
                y[i * n + j] = b == 0 ? v : y[i * n + j] + v;
            }
        }
    }
    free(q);
    free(sx);
    free(acc);
    free(split);
    return 0;
}

/* candle_nn::Linear::forward without a bias (the lm_head, llama.rs:129-141):
 * y[i][j] = sum_t x[i][t] * w[j][t] in f32, w f32 or bf16 (widened exactly).
 * The reference's sum runs in candle's gemm order (not vendored); this fixes
 * the order of the GPU kernel so the two agree bit for bit: 64 lanes, lane l
 * takes the 4-element chunks c = l, l + 64, l + 128, ... (c < k / 4) and folds
 * each chunk's elements in order into acc = fma(x, w, acc); then six butterfly
 * steps acc_l = acc_l + acc_(l xor s), s = 32, 16, 8, 4, 2, 1 (every lane ends
 * with the same value).  k % 4 == 0. */
void orc_dense_linear(const float* x, int64_t m, int64_t k, const void* w, int wbf16, int64_t n, float* y)
{
    const int64_t nc = k / 4;
    for (int64_t i = 0; i < m; ++i) {
        const float* xr = x + i * k;
        for (int64_t j = 0; j < n; ++j) {
            float acc[64], nxt[64];
            for (int l = 0; l < 64; ++l) {
                float a = 0.0f;
                for (int64_t c = l; c < nc; c += 64) {
                    for (int e = 0; e < 4; ++e) {
                        const int64_t t = 4 * c + e;
                        float wv;
                        if (wbf16) {
                            const uint32_t u = (uint32_t)((const uint16_t*)w)[j * k + t] << 16;
                            memcpy(&wv, &u, 4);
                        } else {
                            wv = ((const float*)w)[j * k + t];
                        }
                        a = fmaf(xr[t], wv, a);
                    }
                }
                acc[l] = a;
            }
            for (int s = 32; s >= 1; s >>= 1) {
                for (int l = 0; l < 64; ++l) nxt[l] = acc[l] + acc[l ^ s];
                memcpy(acc, nxt, sizeof(acc));
            }
            y[i * n + j] = acc[0];
        }
    }
}
