// btl_model_api.cpp -- C ABI of the decoder ops (include/bitllama.h): validation
// and dispatch to the kernels of btl_model.hip.
//
// Host-side counterparts of the reference's RotaryEmbedding, QuantizedKVCache,
// BitAttention::forward, Embedding and greedy pick (crates/rust_engine:
// src/layers/attention.rs:15-239, src/layers/kv_cache.rs:49-128,
// src/model/llama.rs:208, 509-515).
#include "bitllama.h"

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdio>
#include <vector>

#include "btl_host.hpp"
#include "btl_internal.hpp"

namespace {

using btl::host::fail_msg;
using btl::host::hip_error;

template <typename... A>
int failf(int code, const char* fmt, A... args)
{
    char buf[512];
    snprintf(buf, sizeof(buf), fmt, args...);
    return fail_msg(code, buf);
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

constexpr int64_t kChunk = 64;  // keys per attention chunk (k_attn_part)

int check_cache(const btl_kv_q8_t* c, int64_t n_heads)
{
    if (!c) return fail_msg(BTL_ERR_ARG, "null KV cache");
    if (!c->k || !c->v || !c->k_scale || !c->v_scale) return fail_msg(BTL_ERR_LAYOUT, "null KV cache buffer");
    if (c->n_kv_heads < 1 || c->max_seq < 1 || c->head_dim < 2 || c->head_dim > 128 || (c->head_dim & 1))
        return failf(BTL_ERR_SHAPE, "KV cache needs n_kv_heads >= 1, max_seq >= 1 and an even head_dim in 2..128 "
                                    "(got %lld, %lld, %lld)",
                     (long long)c->n_kv_heads, (long long)c->max_seq, (long long)c->head_dim);
    if (n_heads < 1 || n_heads % c->n_kv_heads != 0 || n_heads / c->n_kv_heads > 16)
        return failf(BTL_ERR_SHAPE, "n_heads %lld must be a multiple of n_kv_heads %lld, at most 16 times it",
                     (long long)n_heads, (long long)c->n_kv_heads);
    if (c->max_seq > (1 << 24) || c->n_kv_heads * c->max_seq * c->head_dim > ((int64_t)1 << 40))
        return fail_msg(BTL_ERR_SHAPE, "KV cache too large");
    return BTL_OK;
}

int check_pos(int64_t pos, int64_t m, const int32_t* d_pos, const btl_kv_q8_t* c)
{
    if (d_pos) return BTL_OK;  // read on the device; rows past max_seq are skipped there
    if (pos < 0 || pos + m > c->max_seq)
        return failf(BTL_ERR_SHAPE, "positions %lld..%lld outside the cache of %lld rows", (long long)pos,
                     (long long)(pos + m - 1), (long long)c->max_seq);
    return BTL_OK;
}

// queries per workgroup of k_attn_part: enough to reuse each dequantised chunk,
// few enough that the grid still covers the chip
int attn_qb(int64_t m) { return m <= 1 ? 1 : (m <= 64 ? 4 : 16); }

// workspace: [rotated q, m * n_heads * head_dim f32 (btl_rope_append_attention
// with m > 1)] [chunk partials, m * n_heads * cmax * (head_dim + 2) f32]
size_t qrot_bytes(int64_t m, int64_t n_heads, const btl_kv_q8_t* cache)
{
    return (size_t)((m * n_heads * cache->head_dim * 4 + 255) / 256 * 256);
}

}  // namespace

extern "C" {

int btl_rope_table(double theta, int64_t head_dim, int64_t max_seq, float* cos_out, float* sin_out)
{
    if (head_dim < 2 || (head_dim & 1) || max_seq < 0) return fail_msg(BTL_ERR_SHAPE, "head_dim must be even, max_seq >= 0");
    if (!(theta > 0.0)) return fail_msg(BTL_ERR_ARG, "theta must be positive");
    if (max_seq && (!cos_out || !sin_out)) return fail_msg(BTL_ERR_ARG, "null output");
    const int64_t half = head_dim / 2;
    std::vector<float> inv((size_t)half);
    // attention.rs:19 `1.0 / (theta.powf(2i / hd)) as f32`: the cast binds first, so the
    // f64 power is rounded to f32 and the reciprocal is an f32 division
    for (int64_t i = 0; i < half; ++i) {
        const float pw = (float)std::pow(theta, (double)(2 * i) / (double)head_dim);
        inv[(size_t)i] = 1.0f / pw;
    }
    for (int64_t p = 0; p < max_seq; ++p)
        for (int64_t i = 0; i < half; ++i) {
            const float f = (float)p * inv[(size_t)i];
            cos_out[p * half + i] = cosf(f);
            sin_out[p * half + i] = sinf(f);
        }
    return BTL_OK;
}

int btl_rope_kv_append(const float* q, const float* k, const float* v, int64_t m, int64_t n_heads,
                       const btl_kv_q8_t* cache, int64_t pos, const int32_t* d_pos, const float* rope_cos,
                       const float* rope_sin, float* q_out, void* stream)
{
    int rc;
    if ((rc = check_cache(cache, n_heads))) return rc;
    if (m < 0 || m > (1 << 24)) return fail_msg(BTL_ERR_SHAPE, "token count out of range");
    if ((rc = check_pos(pos, m, d_pos, cache))) return rc;
    if (m == 0) return BTL_OK;
    if (!q || !k || !v || !q_out || !rope_cos || !rope_sin) return fail_msg(BTL_ERR_LAYOUT, "null pointer");
    int dev;
    if ((rc = btl::host::device(&dev))) return rc;
    btl::KvArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.q_out = q_out;
    a.kc = cache->k;
    a.vc = cache->v;
    a.ksc = cache->k_scale;
    a.vsc = cache->v_scale;
    a.cos_t = rope_cos;
    a.sin_t = rope_sin;
    a.d_pos = d_pos;
    a.pos = (int)pos;
    a.m = (int)m;
    a.nh = (int)n_heads;
    a.nkv = (int)cache->n_kv_heads;
    a.hd = (int)cache->head_dim;
    a.max_seq = (int)cache->max_seq;
    hipError_t e = btl::launch_rope_kv_q8(a, (hipStream_t)stream);
    if (e != hipSuccess) return hip_error(e, "rope / kv append kernel launch");
    return BTL_OK;
}

size_t btl_attention_workspace_bytes(int64_t m, int64_t n_heads, const btl_kv_q8_t* cache)
{
    if (!cache || m < 0 || n_heads < 0 || cache->max_seq < 1) return 0;
    const int64_t cmax = (cache->max_seq + kChunk - 1) / kChunk;
    return qrot_bytes(m, n_heads, cache) + (size_t)(m * n_heads * cmax * (cache->head_dim + 2) * 4);
}

int btl_attention(const float* q, int64_t m, int64_t n_heads, const btl_kv_q8_t* cache, int64_t pos,
                  const int32_t* d_pos, float* out, void* ws, size_t ws_bytes, void* stream)
{
    int rc;
    if ((rc = check_cache(cache, n_heads))) return rc;
    if (m < 0 || m > (1 << 20)) return fail_msg(BTL_ERR_SHAPE, "query count out of range");
    if ((rc = check_pos(pos, m, d_pos, cache))) return rc;
    if (m == 0) return BTL_OK;
    if (!q || !out) return fail_msg(BTL_ERR_LAYOUT, "null pointer");
    int dev;
    if ((rc = btl::host::device(&dev))) return rc;
    void* wsp = nullptr;
    if ((rc = btl::host::workspace(dev, ws, ws_bytes, btl_attention_workspace_bytes(m, n_heads, cache), &wsp,
                                   (hipStream_t)stream)))
        return rc;
    void* part = (uint8_t*)wsp + qrot_bytes(m, n_heads, cache);
    btl::AttnArgs a{};
    a.q = q;
    a.kc = cache->k;
    a.vc = cache->v;
    a.ksc = cache->k_scale;
    a.vsc = cache->v_scale;
    a.d_pos = d_pos;
    a.pos = (int)pos;
    a.m = (int)m;
    a.nh = (int)n_heads;
    a.nkv = (int)cache->n_kv_heads;
    a.hd = (int)cache->head_dim;
    a.max_seq = (int)cache->max_seq;
    a.cmax = (int)((cache->max_seq + kChunk - 1) / kChunk);
    a.qb = attn_qb(m);
    a.scal = (float)(1.0 / std::sqrt((double)cache->head_dim));  // attention.rs:133, as candle's affine f32
    a.part = (float*)part;
    a.out = out;
    hipError_t e = btl::launch_attention(a, (hipStream_t)stream);
    if (e != hipSuccess) return hip_error(e, "attention kernel launch");
    return BTL_OK;
}

int btl_rope_append_attention(const float* q, const float* k, const float* v, int64_t m, int64_t n_heads,
                              const btl_kv_q8_t* cache, int64_t pos, const int32_t* d_pos, const float* rope_cos,
                              const float* rope_sin, float* out, void* ws, size_t ws_bytes, void* stream)
{
    int rc;
    if ((rc = check_cache(cache, n_heads))) return rc;
    if (m < 0 || m > (1 << 20)) return fail_msg(BTL_ERR_SHAPE, "token count out of range");
    if ((rc = check_pos(pos, m, d_pos, cache))) return rc;
    if (m == 0) return BTL_OK;
    if (!q || !k || !v || !out || !rope_cos || !rope_sin) return fail_msg(BTL_ERR_LAYOUT, "null pointer");
    int dev;
    if ((rc = btl::host::device(&dev))) return rc;
    void* wsp = nullptr;
    if ((rc = btl::host::workspace(dev, ws, ws_bytes, btl_attention_workspace_bytes(m, n_heads, cache), &wsp,
                                   (hipStream_t)stream)))
        return rc;
    float* qrot = (float*)wsp;
    btl::AttnArgs a{};
    a.kc = cache->k;
    a.vc = cache->v;
    a.ksc = cache->k_scale;
    a.vsc = cache->v_scale;
    a.d_pos = d_pos;
    a.pos = (int)pos;
    a.m = (int)m;
    a.nh = (int)n_heads;
    a.nkv = (int)cache->n_kv_heads;
    a.hd = (int)cache->head_dim;
    a.max_seq = (int)cache->max_seq;
    a.cmax = (int)((cache->max_seq + kChunk - 1) / kChunk);
    a.qb = attn_qb(m);
    a.scal = (float)(1.0 / std::sqrt((double)cache->head_dim));
    a.part = (float*)((uint8_t*)wsp + qrot_bytes(m, n_heads, cache));
    a.out = out;
    hipError_t e;
    if (m == 1 && cache->head_dim % 16 == 0) {
        // one decode token: RoPE, append and attention in one kernel, then the merge
        btl::DecKv kv{q, k, v, rope_cos, rope_sin, cache->k, cache->v, cache->k_scale, cache->v_scale};
        a.q = q;
        if (a.nkv <= btl::kAttnMaxCtr && btl::knob(btl::KN_ATTN_MERGE)) {
            // the merge in the same launch (per-KV-head counters of this workspace;
            // NULL when every counter slot has another workspace: a second launch)
            if ((e = btl::attn_counters(dev, wsp, &a.ctr)) != hipSuccess) return hip_error(e, "attention merge counters");
        }
        e = btl::launch_attention_dec1(a, kv, (hipStream_t)stream);
        if (e != hipSuccess) return hip_error(e, "decode attention kernel launch");
        return BTL_OK;
    }
    btl::KvArgs r{};
    r.q = q;
    r.k = k;
    r.v = v;
    r.q_out = qrot;
    r.kc = cache->k;
    r.vc = cache->v;
    r.ksc = cache->k_scale;
    r.vsc = cache->v_scale;
    r.cos_t = rope_cos;
    r.sin_t = rope_sin;
    r.d_pos = d_pos;
    r.pos = (int)pos;
    r.m = (int)m;
    r.nh = (int)n_heads;
    r.nkv = (int)cache->n_kv_heads;
    r.hd = (int)cache->head_dim;
    r.max_seq = (int)cache->max_seq;
    e = btl::launch_rope_kv_q8(r, (hipStream_t)stream);
    if (e != hipSuccess) return hip_error(e, "rope / kv append kernel launch");
    a.q = qrot;
    e = btl::launch_attention(a, (hipStream_t)stream);
    if (e != hipSuccess) return hip_error(e, "attention kernel launch");
    return BTL_OK;
}

int btl_embedding(const void* table, int dtype, int64_t vocab, int64_t dim, const int32_t* ids, int64_t m,
                  float* out, void* stream)
{
    if (dtype != BTL_F32 && dtype != BTL_BF16) return failf(BTL_ERR_DTYPE, "table dtype %d is not BTL_F32/BTL_BF16", dtype);
    if (vocab < 0 || dim < 0 || m < 0 || dim > (1 << 24) || m > (1 << 24)) return fail_msg(BTL_ERR_SHAPE, "size out of range");
    if (m == 0 || dim == 0) return BTL_OK;
    if (!table || !ids || !out) return fail_msg(BTL_ERR_LAYOUT, "null pointer");
    int dev;
    int rc = btl::host::device(&dev);
    if (rc) return rc;
    hipError_t e = btl::launch_embed(table, dtype == BTL_BF16 ? btl::XK_BF16 : btl::XK_F32, vocab, dim, ids, m, out,
                                     (hipStream_t)stream);
    if (e != hipSuccess) return hip_error(e, "embedding kernel launch");
    return BTL_OK;
}

int btl_greedy_next(const float* logits, int64_t n, int32_t* next_id, int32_t* d_pos, int32_t* log,
                    int64_t log_len, void* stream)
{
    if (n < 1 || n > INT32_MAX) return fail_msg(BTL_ERR_SHAPE, "logit count out of range");
    if (!logits || !next_id) return fail_msg(BTL_ERR_LAYOUT, "null pointer");
    if (!aligned16(logits)) return fail_msg(BTL_ERR_LAYOUT, "logits must be 16-byte aligned");
    if (log && log_len < 0) return fail_msg(BTL_ERR_ARG, "negative log length");
    int dev;
    int rc = btl::host::device(&dev);
    if (rc) return rc;
    hipError_t e = btl::launch_greedy(logits, n, next_id, d_pos, log, log ? log_len : 0, (hipStream_t)stream);
    if (e != hipSuccess) return hip_error(e, "greedy kernel launch");
    return BTL_OK;
}

int btl_add_rmsnorm(const float* h, const float* delta, float* h_out, const float* g, float eps, int64_t m, int64_t k,
                    float* y, void* stream)
{
    if (m < 0 || m > INT32_MAX) return fail_msg(BTL_ERR_SHAPE, "row count out of range");
    if (k < 64 || k % 64 || k > 65536) return failf(BTL_ERR_SHAPE, "k = %lld: need a multiple of 64 in [64, 65536]", (long long)k);
    if (m == 0) return BTL_OK;
    if (!h || !g || !y) return fail_msg(BTL_ERR_LAYOUT, "null pointer");
    if (!aligned16(h) || !aligned16(g) || !aligned16(y) || (delta && !aligned16(delta)) || (h_out && !aligned16(h_out)))
        return fail_msg(BTL_ERR_LAYOUT, "h, delta, h_out, g and y must be 16-byte aligned");
    const size_t rows = (size_t)m * (size_t)k * 4, row = (size_t)k * 4;
    auto overlap = [](const void* a, size_t na, const void* b, size_t nb) {
        return a && b && (const uint8_t*)a < (const uint8_t*)b + nb && (const uint8_t*)b < (const uint8_t*)a + na;
    };
    if (overlap(y, rows, h, rows) || overlap(y, rows, delta, rows) || overlap(y, rows, h_out, rows) ||
        overlap(y, rows, g, row))
        return fail_msg(BTL_ERR_LAYOUT, "y overlaps an input or h_out");
    if (h_out && h_out != h && (overlap(h_out, rows, h, rows) || overlap(h_out, rows, delta, rows) ||
                                overlap(h_out, rows, g, row)))
        return fail_msg(BTL_ERR_LAYOUT, "h_out must be h itself or not overlap h, delta and g");
    int dev;
    int rc = btl::host::device(&dev);
    if (rc) return rc;
    hipError_t e = btl::launch_rmsnorm_f32(h, delta, h_out, g, eps, m, k, y, (hipStream_t)stream);
    if (e != hipSuccess) return hip_error(e, "rmsnorm kernel launch");
    return BTL_OK;
}

int btl_swiglu(const float* gate, const float* up, int64_t count, float* out, void* stream)
{
    if (count < 0) return fail_msg(BTL_ERR_SHAPE, "negative count");
    if (count == 0) return BTL_OK;
    if (!gate || !up || !out) return fail_msg(BTL_ERR_LAYOUT, "null pointer");
    int dev;
    int rc = btl::host::device(&dev);
    if (rc) return rc;
    hipError_t e = btl::launch_swiglu_f32(gate, up, count, out, (hipStream_t)stream);
    if (e != hipSuccess) return hip_error(e, "swiglu kernel launch");
    return BTL_OK;
}

int btl_dense_linear(const void* w, int wdtype, int64_t n, int64_t k, const float* x, int64_t m, float* y,
                     void* stream)
{
    if (wdtype != BTL_F32 && wdtype != BTL_BF16) return failf(BTL_ERR_DTYPE, "weight dtype %d is not BTL_F32/BTL_BF16", wdtype);
    if (n < 0 || m < 0 || m > 65535 || n > ((int64_t)1 << 40)) return fail_msg(BTL_ERR_SHAPE, "size out of range");
    if (k < 4 || k % 4 || k > (1 << 28)) return failf(BTL_ERR_SHAPE, "k = %lld: need a positive multiple of 4", (long long)k);
    if (m == 0 || n == 0) return BTL_OK;
    if (!w || !x || !y) return fail_msg(BTL_ERR_LAYOUT, "null pointer");
    if (!aligned16(x) || ((uintptr_t)w & (wdtype == BTL_F32 ? 15u : 7u)))
        return fail_msg(BTL_ERR_LAYOUT, "x must be 16-byte aligned, w 16-byte (f32) or 8-byte (bf16) aligned");
    int dev;
    int rc = btl::host::device(&dev);
    if (rc) return rc;
    hipError_t e = btl::launch_dense_gemv(w, wdtype == BTL_BF16 ? btl::XK_BF16 : btl::XK_F32, n, k, x, m, y,
                                          (hipStream_t)stream);
    if (e != hipSuccess) return hip_error(e, "dense linear kernel launch");
    return BTL_OK;
}

}  // extern "C"
