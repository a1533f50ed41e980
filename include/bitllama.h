/*
 * bitllama.h -- C ABI of the decoder ops around the BitLinear path
 * (MI355X / gfx950), the neighbours that a Llama-shaped decoder built on
 * bitlinear.h needs to run end to end on the device.
 *
 * Reference seams (imonoonoko/Bit-TTT-Engine, crate crates/rust_engine; Rust,
 * not a C ABI):
 *
 *   RotaryEmbedding::{new, apply}            src/layers/attention.rs:15-87
 *   QuantizedKVCache::{append, quantize_q8, dequantize_q8}
 *                                            src/layers/kv_cache.rs:49-128
 *   BitAttention::forward (after q/k/v, before o_proj)
 *                                            src/layers/attention.rs:149-224
 *   BitLlamaBlock::forward residual + norm2  src/model/block.rs:122-137
 *   BitLlama::forward_one embedding          src/model/llama.rs:208
 *   RMSNorm::forward (final norm)            src/layers/rms_norm.rs:33-56
 *   lm_head (dense candle_nn::Linear)        src/model/llama.rs:129-141, 255-265
 *   Llama::stream_completion greedy pick     src/model/llama.rs:509-515
 *
 * Conventions are those of bitlinear.h: int status (BTL_OK / BTL_ERR_*),
 * btl_last_error(), device pointers, `stream` a hipStream_t as void*, nothing
 * allocated or freed on the caller's behalf except the library workspace when
 * ws == NULL.
 *
 * Positions.  Functions that place tokens in the sequence take `pos` (host) and
 * `d_pos` (a device int32, or NULL).  With d_pos != NULL the kernels read the
 * position from the device, so a captured HIP graph of one decode step can be
 * replayed as the position advances (btl_greedy_next advances it).
 */
#ifndef BITLLAMA_H
#define BITLLAMA_H

#include <stddef.h>
#include <stdint.h>

#include "bitlinear.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * The Q8 KV cache of one layer (QuantizedKVCache, kv_cache.rs:14-22): codes
 * u8 = round(x / s) + 128, s = max|x| / 127 per (token, KV head).
 * k, v:       device [n_kv_heads, max_seq, head_dim] u8
 * k_scale, v_scale: device [n_kv_heads, max_seq] f32
 * The reference grows its cache with Tensor::cat on every append
 * (kv_cache.rs:57-77); here the caller allocates max_seq rows once and the
 * append writes rows in place.
 */
typedef struct btl_kv_q8 {
    uint8_t* k;
    uint8_t* v;
    float* k_scale;
    float* v_scale;
    int64_t n_kv_heads;
    int64_t max_seq;
    int64_t head_dim;
} btl_kv_q8_t;

/*
 * RotaryEmbedding::new (attention.rs:15-42), host pointers:
 * inv_freq[i] = (f32)(1 / theta^(2i / head_dim)) in double, freq = (f32)p * inv_freq[i],
 * cos_out / sin_out [max_seq, head_dim / 2] = cosf / sinf of freq.
 */
int btl_rope_table(double theta, int64_t head_dim, int64_t max_seq, float* cos_out, float* sin_out);

/*
 * RoPE of m new tokens at positions p .. p + m - 1 (p = d_pos ? *d_pos : pos)
 * on q [m, n_heads * head_dim] -> q_out (may alias q) and on
 * k [m, n_kv * head_dim], then QuantizedKVCache::append of k and v
 * [m, n_kv * head_dim] (quantize_q8, kv_cache.rs:95-119) into the cache rows
 * of those positions.  RoPE per head pairs (i, i + head_dim/2):
 * [x1*cos - x2*sin, x1*sin + x2*cos] (attention.rs:67-83), every product and
 * sum an f32 rounding.  rope_cos / rope_sin: device copies of btl_rope_table.
 * head_dim even, 2..128.  Rows at positions >= max_seq are not written.
 */
int btl_rope_kv_append(const float* q, const float* k, const float* v, int64_t m, int64_t n_heads,
                       const btl_kv_q8_t* cache, int64_t pos, const int32_t* d_pos, const float* rope_cos,
                       const float* rope_sin, float* q_out, void* stream);

/*
 * Attention of m queries (rotated, [m, n_heads * head_dim] f32) at positions
 * p .. p + m - 1 over the Q8 cache, query i seeing keys [0, p + i] (the causal
 * mask of attention.rs:245-270; one decode query sees the whole cache):
 * softmax(q . k_deq * (f32)(1/sqrt(head_dim))) . v_deq, GQA head h reading KV
 * head h / (n_heads / n_kv) (repeat_kv, attention.rs:227-239).
 * out: [m, n_heads * head_dim] f32, heads in order (the reshape of
 * attention.rs:219).  Summation order (fixed, so results are reproducible bit
 * for bit): dot products sequential over head_dim; keys in chunks of 64, each
 * chunk's (max m_c, sum l_c of exp(s - m_c), values o_c) merged with weights
 * exp(m_c - max_c m_c) in chunk order; o = O / L.  n_heads % n_kv == 0,
 * n_heads / n_kv <= 16, head_dim <= 128.  ws: btl_attention_workspace_bytes.
 */
size_t btl_attention_workspace_bytes(int64_t m, int64_t n_heads, const btl_kv_q8_t* cache);
int btl_attention(const float* q, int64_t m, int64_t n_heads, const btl_kv_q8_t* cache, int64_t pos,
                  const int32_t* d_pos, float* out, void* ws, size_t ws_bytes, void* stream);

/*
 * The attention core of BitAttention::forward between the q/k/v projections and
 * o_proj (attention.rs:165-219): RoPE of q and k, QuantizedKVCache::append of
 * k and v, attention -- btl_rope_kv_append then btl_attention, same results
 * bit for bit.  q [m, n_heads * head_dim], k, v [m, n_kv * head_dim] raw
 * projection outputs (not modified), out [m, n_heads * head_dim].  For one
 * token (m == 1, head_dim % 16 == 0) the RoPE, the append, the attention and
 * the merge of its key chunks run in one launch (n_kv <= 64; the last
 * workgroup of a KV head merges, counted on per-device counters that every
 * launch leaves at zero, so such calls on one device must not overlap in
 * time -- order them on one stream, as the workspace already asks).
 * ws: btl_attention_workspace_bytes (it covers the rotated queries too).  A
 * device position outside the cache gives NaN outputs and no append.
 */
int btl_rope_append_attention(const float* q, const float* k, const float* v, int64_t m, int64_t n_heads,
                              const btl_kv_q8_t* cache, int64_t pos, const int32_t* d_pos, const float* rope_cos,
                              const float* rope_sin, float* out, void* ws, size_t ws_bytes, void* stream);

/*
 * Embedding::forward (llama.rs:208): out[t] = (f32) table[ids[t]] for
 * t < m.  table [vocab, dim] of dtype (BTL_F32 / BTL_BF16), ids device int32.
 * An id outside [0, vocab) gives a zero row.
 */
int btl_embedding(const void* table, int dtype, int64_t vocab, int64_t dim, const int32_t* ids, int64_t m,
                  float* out, void* stream);

/*
 * Greedy pick (llama.rs:509-515): next_id[0] = argmax(logits[0..n)), the last
 * index among equal maxima (Iterator::max_by).  With d_pos != NULL, also
 * log[*d_pos + 1] = id when it is inside log[0..log_len), then *d_pos += 1:
 * one decode step's bookkeeping on the device.  logits 16-byte aligned.  The
 * workgroups of the launch meet in a per-device word that every launch leaves
 * at zero: calls on one device must not overlap in time (order them on one
 * stream).
 */
int btl_greedy_next(const float* logits, int64_t n, int32_t* next_id, int32_t* d_pos, int32_t* log,
                    int64_t log_len, void* stream);

/*
 * RMSNorm::forward (rms_norm.rs:33-56) into f32 rows: s = h + delta (delta may
 * be NULL), y = s / sqrt(sum(s * s) * (f32)(1/k) + eps) * g, the sum a pairwise
 * tree over the row in index order; h_out = s when h_out != NULL (h_out may be
 * h itself).  h, delta, h_out, y [m, k] f32, g [k] f32, all 16-byte aligned;
 * k % 64 == 0, 64 <= k <= 65536; y overlaps none of the others.  The input of a
 * dense lm_head (btl_dense_linear).
 */
int btl_add_rmsnorm(const float* h, const float* delta, float* h_out, const float* g, float eps, int64_t m, int64_t k,
                    float* y, void* stream);

/*
 * SwiGLU's activation (swiglu.rs:29-35): out[i] = silu(gate[i]) * up[i], silu
 * as candle's v / (1 + exp(-v)), every operation rounded to f32 (exp by a
 * Cody-Waite reduction and a degree-7 Taylor polynomial, each step rounded;
 * oracle/bitlinear_oracle.c restates it).
 * count elements of f32; out may be gate or up.
 */
int btl_swiglu(const float* gate, const float* up, int64_t count, float* out, void* stream);

/*
 * candle_nn::Linear::forward without a bias -- the reference's lm_head, a dense
 * linear (llama.rs:129-141): y[m, n] = x[m, k] . w[n, k]^T in f32, w of dtype
 * BTL_F32 (the reference's) or BTL_BF16 (widened exactly).  Fixed order: lane l
 * of 64 folds the 4-element chunks l, l + 64, ... of a row into fma partial
 * sums, then a butterfly over the lanes (oracle/bitllama_oracle.c restates it).
 * k % 4 == 0; x 16-byte aligned, w 16-byte (f32) or 8-byte (bf16) aligned;
 * m <= 65535.
 */
int btl_dense_linear(const void* w, int wdtype, int64_t n, int64_t k, const float* x, int64_t m, float* y,
                     void* stream);

/*
 * Residual connection fused ahead of RMSNorm and a BitLinear group
 * (block.rs:122-123,137 then the next norm): s = h + delta (f32), stored to
 * h_out when h_out != NULL (h_out may be h itself, or a buffer that does not
 * overlap it), then btl_rmsnorm_linear_group on s.  delta == NULL: plain
 * RMSNorm of h, h_out not written.  h, delta, h_out [m, k] f32, g [k] f32.
 * k % 64 == 0, 64 <= k <= 65536; h, delta, h_out and g 16-byte aligned.
 * For one token row (decode) with h_out not aliasing h, the add and the norm
 * run inside the contraction kernel's prologue (one launch).
 */
int btl_add_rmsnorm_linear_group(const btl_packed_t* const* w, void* const* y, int count, const float* h,
                                 const float* delta, float* h_out, const float* g, float eps, int64_t m, int64_t k,
                                 int ydtype, void* ws, size_t ws_bytes, void* stream);

/*
 * The same in the reference's arithmetic (the BitLinears as BitLinearCpu::forward,
 * kernels/cpu.rs:17-127), in one launch: the same bits as
 * btl_add_rmsnorm(h, delta, h_out, g, eps, m, k, xn) followed by
 * btl_linear_group_mode(w, y, count, xn, BTL_F32, m, k, BTL_F32, BTL_ACT_F32_REF, ...).
 * Every workgroup forms the normalised rows it needs while staging them; the
 * first output tile's workgroups store s = h (+ delta) to h_out (when not NULL).
 * h, delta (or NULL), h_out (or NULL) [m, k] f32, g [k] f32, y[i] [m, n_i] f32;
 * k % 64 == 0, 64 <= k <= 16384, m <= 65535; h, delta, h_out, g and the packed
 * rows 16-byte aligned; h_out overlaps none of h, delta, g and y, and y no input.
 * No reference function of its own: the norm ahead of a block's projections
 * (block.rs:122-123,137) fused with them.
 */
int btl_add_rmsnorm_linear_group_ref(const btl_packed_t* const* w, void* const* y, int count, const float* h,
                                     const float* delta, float* h_out, const float* g, float eps, int64_t m,
                                     int64_t k, void* stream);

/*
 * A BitLinear with the residual connection after it (block.rs:119,131:
 * residual + mixed_out): y = resid + x W^T, the W1.58-A8 product as
 * btl_linear's then one f32 add per element.  x [m, k] f32 or bf16 (xdtype),
 * resid and y [m, n] f32; y must overlap neither resid nor x.  On the decode
 * kernel of whole weight rows (one token row with k % 64 == 0 and
 * 1024 <= k <= 16384, one or two token rows) the add runs in its epilogue (one
 * launch), otherwise in an elementwise launch after the product.  It lets the
 * decoder drop the add from the next residual + RMSNorm:
 * btl_add_rmsnorm_linear_group / btl_add_rmsnorm_swiglu on y with delta = NULL
 * give the same bits.  ws: as btl_linear (or NULL).
 * No reference function of its own: the residual add of BitLlamaBlock::forward.
 */
int btl_linear_residual(const btl_packed_t* w, const void* x, int xdtype, int64_t m, int64_t k, const float* resid,
                        float* y, void* ws, size_t ws_bytes, void* stream);

/*
 * The gate/up half of SwiGLU::forward (swiglu.rs:29-35) after the residual add
 * and RMSNorm of btl_add_rmsnorm_linear_group: out = silu(xn W1^T) * (xn W3^T),
 * xn = RMSNorm(h + delta) * g, silu(v) = v / (1 + exp(-v)), out [m, n] f32 --
 * the input of the down projection.  w_gate, w_up: [n, k] packed, equal n.
 * Same bits as btl_add_rmsnorm_linear_group into two f32 outputs followed by
 * the elementwise SwiGLU; for up to 4 rows the decode kernel computes the pair
 * and writes silu(gate) * up from its epilogue (no gate / up tensors).
 * ws: btl_add_rmsnorm_swiglu_workspace_bytes (or NULL: the library's).
 */
int btl_add_rmsnorm_swiglu(const btl_packed_t* w_gate, const btl_packed_t* w_up, const float* h,
                           const float* delta, float* h_out, const float* g, float eps, int64_t m, int64_t k,
                           float* out, void* ws, size_t ws_bytes, void* stream);
size_t btl_add_rmsnorm_swiglu_workspace_bytes(int64_t m, int64_t n, int64_t k);

/*
 * The decode stream: the one-token projections of every layer of a Llama block
 * stack in ONE persistent launch.  No single reference counterpart: it replaces
 * the sequence of BitLinear::forward calls (layers/bit_linear.rs:52-119) that
 * one decoder step issues per layer in dependency order -- q|k|v
 * (attention.rs:159-162), o_proj, w1|w3 and w2 (swiglu.rs:29-35) from
 * BitLlamaBlock::forward (model/block.rs:90-138) -- with the launch boundaries
 * between them replaced by a device-side handoff.  Per layer l:
 *   [q|k|v] = W1.58-A8(q, k, v; x_l);  o = W1.58-A8(o; q);
 *   h = silu(W1.58-A8(gate; o)) * W1.58-A8(up; o);  x_{l+1} = W1.58-A8(down; h)
 * every output rounded to bf16; each contraction bit-identical to btl_linear
 * on the bf16 input, silu as btl_add_rmsnorm_swiglu.  (Attention, norms and
 * residual adds are not part of this chain: it is the decoder's projection
 * chain, what a one-token step streams from HBM.)
 *
 * btl_stream_create: checks the shapes (q: [H, H], k/v: [nk/nv, H], o: [H, H],
 *   gate/up: [I, H], down: [H, I]; H a multiple of 64 up to 4096, I a multiple
 *   of 64 up to 14336, every layer alike, packed data 16-byte aligned; at most
 *   6 / 4 / 14 / 8 row groups of q|k|v / o / gate|up / down per CU) and
 *   allocates the plan's device buffers (layer table, handoff words, flags).
 * btl_stream_run: x bf16 [H] (device, 16-byte aligned) -> y bf16 [H]; stage_out
 *   NULL, or a bf16 buffer of btl_stream_stage_words(plan) elements that
 *   receives every stage's output (per layer: [q|k|v], o, h, down).  The launch
 *   takes every CU (one workgroup each, all resident): its occupancy is checked
 *   first (BTL_ERR_HIP, hipErrorCooperativeLaunchTooLarge, when the workgroups
 *   cannot all be resident), and outside a stream capture it is a cooperative
 *   launch, so the runtime runs every workgroup at once or fails the launch.
 *   Under a capture it is a plain launch: nothing else may then run on the
 *   device meanwhile.  Its waits are bounded in time (BTL_WAIT_SPIN); a wait
 *   that gives up is reported by btl_check_faults.  Runs on one plan must be
 *   ordered on one stream.
 * btl_stream_destroy: synchronises the device and frees the plan.
 */
typedef struct btl_stream_layer {
    btl_packed_t q, k, v, o, gate, up, down;
} btl_stream_layer_t;

int btl_stream_create(const btl_stream_layer_t* layers, int n_layers, void** plan);
size_t btl_stream_stage_words(const void* plan);
int btl_stream_run(void* plan, const void* x, void* y, void* stage_out, void* stream);
int btl_stream_destroy(void* plan);

#ifdef __cplusplus
}
#endif

#endif /* BITLLAMA_H */
