/*
 * bitlinear.h -- C ABI of the MI355X (gfx950) BitLinear engine.
 *
 * Drop-in boundary for the packed-ternary linear layer of
 * imonoonoko/Bit-TTT-Engine (crate crates/rust_engine).  The reference's seam is
 * Rust, not a C ABI:
 *
 *   BitLinear::forward(&self, x) -> Result<Tensor>        src/layers/bit_linear.rs:52-119
 *     -> BitLinearCpu::forward(input, &PackedTensor)       src/kernels/cpu.rs:17-127
 *     -> BitLinearCuda::forward(input, &PackedTensor)      src/kernels/cuda.rs:21-47
 *     -> bail!("... Custom Kernel not implemented ...")    src/layers/bit_linear.rs:76-84
 *
 * A Rust FFI crate calls the functions below from a new `Device::Hip` arm of
 * BitLinear::forward; rank flattening and reshaping stay in Rust
 * (bit_linear.rs:54-62, 88-95).
 *
 * Conventions (all functions):
 *  - Return 0 (BTL_OK) on success, a BTL_ERR_* code otherwise; the message of
 *    the last failure on the calling thread is returned by btl_last_error().
 *    This mirrors the reference's int-status C ABI precedent
 *    (dist/binaries/README.md:49-58: nonzero return means error) and carries
 *    the reference's error texts (e.g. cpu.rs:22-30 "Shape mismatch: ...").
 *  - Tensors are dense and row-major.  "Device pointer" means memory on the
 *    current HIP device (hipMalloc / torch.cuda); "host pointer" means CPU memory.
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream); every
 *    device function is asynchronous with respect to the host and stream ordered.
 *  - Nothing here allocates or frees caller memory.  Functions that take a
 *    workspace accept ws == NULL, in which case the library uses a per-device
 *    workspace it owns (allocated with hipMalloc and grown by at least
 *    doubling; a replaced workspace is kept until the process ends, so HIP
 *    graphs captured earlier stay valid; it cannot grow while the call's
 *    stream is being captured -- BTL_ERR_WORKSPACE -- so make the largest call
 *    once before capturing, or pass a workspace).  Calls that share the
 *    library's workspace must be ordered on one stream.
 *  - Functions are reentrant: no per-call global state besides that workspace
 *    and the per-thread error message.
 */
#ifndef BITLINEAR_H
#define BITLINEAR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BTL_VERSION 1

/* Status codes. */
#define BTL_OK 0
#define BTL_ERR_SHAPE 1     /* k != w.k ("Shape mismatch"), k % 4 != 0, negative sizes */
#define BTL_ERR_DTYPE 2     /* unsupported dtype / mode enum */
#define BTL_ERR_LAYOUT 3    /* null or misaligned pointer where one is required */
#define BTL_ERR_DEVICE 4    /* no usable gfx950 device / pointer not on the device */
#define BTL_ERR_HIP 5       /* a HIP runtime call failed */
#define BTL_ERR_ARG 6       /* any other invalid argument */
#define BTL_ERR_WORKSPACE 7 /* caller workspace smaller than btl_workspace_bytes(), or the
                               library's cannot grow during stream capture */
#define BTL_ERR_FAULT 8     /* btl_check_faults: a kernel's bounded wait gave up */

/* Element types of activations and outputs. */
#define BTL_F32 0
#define BTL_BF16 1

/* Arithmetic modes of btl_linear. */
#define BTL_ACT_F32_REF 0 /* reference semantics: fp32 x, y = scale * sum_k x*t in
                             the exact summation order of cpu.rs:86-123 */
#define BTL_ACT_I8 1      /* W1.58-A8: per-token absmax int8 x, exact int32 sum,
                             y = (float)acc * (s_x * s_w) */
#define BTL_ACT_F32_SEQ 2 /* reference semantics in the order of a host without
                             AVX2/FMA (cpu.rs:62-66,105-123): sum = sum + x*t over
                             k in increasing order, from +0.0f */

/*
 * Packed ternary weights: the reference's PackedTensor (kernels/packing.rs:14-21).
 * data: device pointer to ceil(n*k/4) bytes.  Element e = row*k + col of the
 *       row-major [n, k] matrix sits in byte e/4 at bits 2*(e%4); codes
 *       00 = 0, 01 = +1, 10 = -1, 11 = 0 (packing.rs:6-13, 74-92, cpu.rs:59).
 * n, k: the reference's `shape` [out_dim, in_dim].
 * scale: the per-tensor absmean scale mean|W| + 1e-6 (packing.rs:56-57).
 */
typedef struct btl_packed {
    const uint8_t* data;
    int64_t n;
    int64_t k;
    float scale;
} btl_packed_t;

/* Library version (BTL_VERSION). */
int btl_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* btl_last_error(void);

/* Short name of a status code. */
const char* btl_status_string(int status);

/*
 * Check that `device` is a usable gfx950 GPU and cache its properties.
 * Idempotent and thread-safe; every device function also initialises lazily.
 */
int btl_init(int device);

/*
 * Routing and tuning knobs (no reference counterpart: the reference has one
 * kernel per device).  Each knob starts from the environment variable of its
 * name when set -- read once, at the first library call -- else from a
 * measured default; afterwards only btl_set_tuning changes it, so the
 * environment of a running process cannot re-route calls.  Names are
 * "BTL_GEMV_DEC_PARTS", "BTL_DEC_RQ_WPC", "BTL_GEMV_DEC_MAX_M", "BTL_GEMV_DEC",
 * "BTL_DEC_ROW_MIN_K", "BTL_DEC_ROW", "BTL_DEC_ROW_RPW", "BTL_DEC_ROW_RB",
 * "BTL_GEMV_BAT_MAX_M", "BTL_GEMV_BAT", "BTL_FUSE_MAX_WG", "BTL_FUSE_DEC",
 * "BTL_DEC_RQ_MIN_K", "BTL_DEC_RQ", "BTL_DEC_RQ_DG", "BTL_GEMM_MAX_SPLITS",
 * "BTL_GEMM_WIDE_MIN_TILES", "BTL_WAIT_SPIN", "BTL_ATTN_MERGE", "BTL_SPLIT_MERGE",
 * "BTL_SPLIT_MERGE_MAX_M", "BTL_GEMV_BAT_NW", "BTL_GEMV_BAT_KS", "BTL_GEMM_TILE",
 * "BTL_GEMM_TM64", "BTL_GEMM_TM64_STAGES", "BTL_GEMM_STAGES", "BTL_DEC_RQ2_MAX_K",
 * "BTL_GEMV_TR", "BTL_GEMV_TR_MIN_M", "BTL_GEMV_TR_MAX_M", "BTL_GEMV_TR_RBPW",
 * "BTL_GEMV_TR_K16" (the "BTL_" prefix may be left out).  Every route gives the same bits; knobs only choose among kernels and
 * launch shapes -- except BTL_WAIT_SPIN, the number of polls after which a
 * kernel's internal wait gives up (2^22 by default; lowering it to force that
 * path is for tests: btl_check_faults then reports it).
 * Unknown names: BTL_ERR_ARG.  Process-wide; not ordered with calls already
 * issued on other threads.
 */
int btl_set_tuning(const char* name, int value);
int btl_get_tuning(const char* name, int* value);

/*
 * Synchronise `stream`, then read and clear the current device's fault word:
 * bits set by kernels whose bounded internal waits gave up (a wave of the
 * one-token decode kernel waiting for its workgroup's quantised token row, a
 * stage of the decode stream waiting for its input).  Such a launch has
 * finished but its outputs are not valid.  Returns BTL_ERR_FAULT with a
 * message naming the waits when any bit was set, else BTL_OK.  No reference
 * counterpart (the reference's kernels do not wait on each other).
 */
int btl_check_faults(void* stream);

/*
 * The instantiation ("k_gemm_i8<TN,WGN,NW,TM,NS>": output rows and waves
 * along them per tile, waves, token rows, LDS stages) of the last prefill
 * GEMM this thread launched, "" before the first.  A diagnostic for tests and
 * tuning, no reference counterpart.
 */
const char* btl_last_gemm_form(void);

/* Number of packed bytes for an [n, k] weight: ceil(n*k/4) (packing.rs:36,71). */
int64_t btl_packed_bytes(int64_t n, int64_t k);

/*
 * Host-side packing, PackedTensor::pack (packing.rs:50-105): host pointers.
 * w: [n, k] f32; out: btl_packed_bytes(n, k) bytes; *scale = mean|w| + 1e-6,
 * the mean summed in double as the pairwise tree over |w| in index order.
 * t = clamp(round(w * (1/scale)), -1, 1), round half away from zero.
 */
int btl_pack_host(const float* w, int64_t n, int64_t k, uint8_t* out, float* scale);

/* Host-side PackedTensor::unpack (packing.rs:108-133): out[n*k] = t * scale. */
int btl_unpack_host(const uint8_t* data, int64_t n, int64_t k, float scale, float* out);

/*
 * PackedTensor::pack (packing.rs:50-105) on the device, for load-time packing of
 * weights already on the GPU.  w: [n, k] f32 device (16-byte aligned); out:
 * btl_packed_bytes(n, k) device bytes (4-byte aligned); *scale: a device f32
 * that receives mean|w| + 1e-6.  Bit-identical to btl_pack_host: the mean is
 * the pairwise tree in double over |w| in index order (zero-padded to a power
 * of two), rounded once to f32.  ws / ws_bytes: optional workspace of
 * btl_pack_workspace_bytes(n, k) bytes for the partial sums.
 */
int btl_pack_device(const float* w, int64_t n, int64_t k, uint8_t* out, float* scale, void* ws, size_t ws_bytes,
                    void* stream);
size_t btl_pack_workspace_bytes(int64_t n, int64_t k);

/*
 * Device-side unpack to dense f32 [n, k] (what BitLinearCuda::forward builds
 * on the host on every call, cuda.rs:40 -> packing.rs:108-133).
 */
int btl_unpack_device(const btl_packed_t* w, float* out, void* stream);

/*
 * Per-token absmax int8 quantisation (no reference counterpart on the BitLinear
 * path; convention of kv_cache.rs:95-119 / BitNet b1.58).  Device pointers.
 * x: [m, k] of xdtype; xq: [m, k] int8; xscale: [m] f32.
 *   a = max|x[row]|;  a non-finite -> s = NaN, q = 0;  a < 2^-100 -> s = 0, q = 0;
 *   else q = clamp(round_half_away(x * (127/a)), -127, 127), s = a / 127.
 */
int btl_quantize_act(const void* x, int xdtype, int64_t m, int64_t k, int8_t* xq, float* xscale,
                     void* stream);

/*
 * BitLinear forward, y = x @ W^T: the replacement of BitLinearCpu::forward /
 * BitLinearCuda::forward (cpu.rs:17, cuda.rs:21).  Device pointers.
 * w:   packed weights; w->k must equal k (else BTL_ERR_SHAPE with the
 *      reference's "Shape mismatch: Input [m, k] vs Weight [n, k_w]").
 * x:   [m, k] of xdtype;  y: [m, w->n] of ydtype.
 * mode BTL_ACT_F32_REF: reference semantics (bf16 x is widened exactly first).
 * mode BTL_ACT_F32_SEQ: the same in the reference's non-AVX2 order (one
 *                       sequential chain of k adds per output: latency-bound).
 * mode BTL_ACT_I8:      W1.58-A8 (quantisation as btl_quantize_act).
 * acc_out: optional [m, n] int32 accumulators (BTL_ACT_I8 only; else NULL).
 * ws / ws_bytes: optional workspace, see btl_workspace_bytes.
 * k must be a multiple of 4 (the reference's CPU row stride ceil(k/4), cpu.rs:81,
 * only agrees with its flat packing, packing.rs:74, when k % 4 == 0).
 */
int btl_linear(const btl_packed_t* w, const void* x, int xdtype, int64_t m, int64_t k, void* y,
               int ydtype, int mode, int32_t* acc_out, void* ws, size_t ws_bytes, void* stream);

/*
 * btl_linear without a workspace and without any allocation: no counterpart in
 * the reference.  For callers that cannot allocate device memory -- code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.  The
 * scratch of BTL_ACT_I8 (quantised activations, split-K partial sums) lives in a
 * static device array of 32 MiB per device (held until the process ends; its
 * address is taken in btl_init or at the first call on a device); a shape whose
 * btl_workspace_bytes(m, n, k, BTL_ACT_I8) exceeds it fails with
 * BTL_ERR_WORKSPACE before any device work.  Results are those of btl_linear,
 * bit for bit.  Every call on one device shares that array and the kernels do
 * not need it cleared; calls that overlap on one device (different streams or
 * threads) race on it and must be ordered by the caller.
 */
int btl_linear_noalloc(const btl_packed_t* w, const void* x, int xdtype, int64_t m, int64_t k, void* y,
                       int ydtype, int mode, int32_t* acc_out, void* stream);

/*
 * Same contraction for pre-quantised activations (as produced by
 * btl_quantize_act, or fused into a producer kernel): xq [m, k] int8,
 * xscale [m] f32.  y = (float)acc * (xscale[row] * w->scale).
 */
int btl_linear_i8(const btl_packed_t* w, const int8_t* xq, const float* xscale, int64_t m,
                  int64_t k, void* y, int ydtype, int32_t* acc_out, void* ws, size_t ws_bytes,
                  void* stream);

/*
 * Several BitLinear layers that read the same input in one launch (the q/k/v
 * projections of BitAttention, attention.rs:159-162; the w1/w3 projections of
 * SwiGLU, swiglu.rs:29-35).  BTL_ACT_I8 semantics; each layer keeps its own
 * scale.  y[i] is a [m, w[i]->n] output of ydtype.  count in 1..4.
 */
int btl_linear_group(const btl_packed_t* const* w, void* const* y, int count, const void* x,
                     int xdtype, int64_t m, int64_t k, int ydtype, void* ws, size_t ws_bytes,
                     void* stream);

/*
 * btl_linear_group in either arithmetic mode: BTL_ACT_I8 is btl_linear_group;
 * BTL_ACT_F32_REF runs every layer in the reference's own fp32 semantics and
 * summation order (BitLinearCpu::forward, cpu.rs:17-127; the results of
 * btl_linear with that mode, bit for bit), all layers in one launch when k % 64
 * == 0, k <= 16384 and the weights are 16-byte aligned; BTL_ACT_F32_SEQ the
 * reference's non-AVX2 order, one launch per layer.  ws is unused in those
 * modes.  count in 1..4.
 */
int btl_linear_group_mode(const btl_packed_t* const* w, void* const* y, int count, const void* x, int xdtype,
                          int64_t m, int64_t k, int ydtype, int mode, void* ws, size_t ws_bytes, void* stream);

/*
 * Operand-order activations for prefill (many token rows).  No reference
 * counterpart: the reference quantises nothing on this path.  The prefill GEMM
 * reads every 16-element group of k in the order its unpacked weights take,
 * k = 16g + [0,4,8,12, 1,5,9,13, 2,6,10,14, 3,7,11,15]; producing that layout
 * once lets several contractions (or a producer kernel that fuses the
 * quantisation) skip the reordering.  Values and scales are exactly those of
 * btl_quantize_act; only the byte order within each 16-group differs.
 * k % 64 == 0, k < 2^24; x and xq 16-byte aligned.
 */
int btl_quantize_act_op(const void* x, int xdtype, int64_t m, int64_t k, int8_t* xq, float* xscale,
                        void* stream);

/*
 * The prefill GEMM alone on operand-order activations (btl_quantize_act_op):
 * `count` (1..4) layers that share xq in one launch, y[i] = [m, w[i]->n] of
 * ydtype, acc_out NULL or an array of count optional int32 [m, w[i]->n]
 * outputs.  Results are those of btl_linear_i8 on the natural-order data.
 * k % 64 == 0, k < 2^24; xq and every w[i]->data 16-byte aligned.  Needs no
 * workspace.
 */
int btl_linear_i8_op(const btl_packed_t* const* w, void* const* y, int32_t* const* acc_out, int count,
                     const int8_t* xq, const float* xscale, int64_t m, int64_t k, int ydtype,
                     void* stream);

/*
 * RMSNorm fused ahead of a BitLinear group: the activations the reference's
 * BitLlamaBlock feeds q/k/v and w1/w3 (block.rs:98,121 -> rms_norm.rs:33-56,
 * then attention.rs:159-162 / swiglu.rs:29-35), without the normalised tensor
 * in between.  Per token row:
 *   xn = x / sqrt(ss * (f32)(1/k) + eps) * g,  ss = sum of x*x (products
 *        rounded to f32) summed as the pairwise tree over the row in index
 *        order, zero-padded to a power of two;
 * every operation a separately rounded f32 operation (candle 0.8's scalar ops:
 * Tensor / f64 and + f64 are affine(1/d, 0) and affine(1, eps)); then
 * W1.58-A8 with each layer as btl_linear_group.  g: [k] f32 (device).
 * k % 64 == 0, 64 <= k <= 65536; x, g and the packed weights 16-byte aligned.
 */
int btl_rmsnorm_linear_group(const btl_packed_t* const* w, void* const* y, int count, const void* x,
                             int xdtype, const float* g, float eps, int64_t m, int64_t k, int ydtype,
                             void* ws, size_t ws_bytes, void* stream);

/*
 * SwiGLU fused ahead of a BitLinear group (swiglu.rs:29-35: w2(silu(w1 x) * w3 x)):
 * h = silu(gate) * up with silu(v) = v / (1 + exp(-v)), then W1.58-A8 with each
 * layer.  exp is this library's f32 exp (Cody-Waite reduction, Taylor polynomial
 * to degree 7; within 2 ulp of the exact value).  gate, up: [m, k] of xdtype.
 * k % 64 == 0, 64 <= k <= 32768; gate, up and the packed weights 16-byte aligned.
 */
int btl_swiglu_linear_group(const btl_packed_t* const* w, void* const* y, int count, const void* gate,
                            const void* up, int xdtype, int64_t m, int64_t k, int ydtype, void* ws,
                            size_t ws_bytes, void* stream);

/*
 * Multi-base adaptive format: AdaptiveBitLinear (layers/adaptive_linear.rs:51-160).
 * The reference stores weight_packed [n, k/4, nb] u8 -- byte (r, c, b) holds the
 * codes of base b for columns 4c..4c+3, bits and codes as PackedTensor
 * (tools/conversion/convert_llama_v2.py:111-151) -- and scales [nb] f32, and
 * reconstructs dense f32 weights at load time (adaptive_linear.rs:86-117).
 * nb in 1..8 (the loader's range, adaptive_linear.rs:56); k % 4 == 0.
 *
 * btl_adaptive_split: load-time repack of the interleaved bytes (device) into
 *   nb PackedTensor byte arrays out[b] [n, k/4] (device, 4-byte aligned), so each
 *   base is an ordinary btl_packed_t {out[b], n, k, scales[b]}.  For nb == 1 the
 *   bytes are unchanged.
 * btl_adaptive_reconstruct: the reference's dense weights on the device,
 *   out[r][4c + j] = ((0 + t_0 s_0) + t_1 s_1) + ... (f32, bases in order), for
 *   callers that want its fp32 matmul semantics.  scales: host array [nb].
 * btl_adaptive_linear: W1.58-A8 over the split bases (build-defined; no
 *   reference counterpart): the activations quantised once per launch as
 *   btl_linear, acc_b exact per base, y = (float)acc_0 (s_x s_0) + (float)acc_1
 *   (s_x s_1) + ... in base order.  bases: nb btl_packed_t of equal shape.
 *   ws: btl_adaptive_workspace_bytes (or NULL: the library's).
 */
int btl_adaptive_split(const uint8_t* packed, int64_t n, int64_t k, int nb, uint8_t* const* out, void* stream);
int btl_adaptive_reconstruct(const uint8_t* packed, const float* scales, int nb, int64_t n, int64_t k, float* out,
                             void* stream);
int btl_adaptive_linear(const btl_packed_t* const* bases, int nb, const void* x, int xdtype, int64_t m, int64_t k,
                        void* y, int ydtype, void* ws, size_t ws_bytes, void* stream);
size_t btl_adaptive_workspace_bytes(int64_t m, int64_t n, int64_t k, int nb);

/*
 * Workspace bytes needed by btl_linear / btl_linear_i8 / btl_linear_group (and
 * the fused RMSNorm / SwiGLU groups) for this shape and mode (for btl_linear_group pass n = sum of the layers' n):
 * scratch for the quantised activations.  Its contents between calls do not
 * matter (every call writes the scratch it reads), so one workspace serves
 * calls of any shapes that fit in it; calls that share one must be ordered on
 * one stream.
 */
size_t btl_workspace_bytes(int64_t m, int64_t n, int64_t k, int mode);

/* Zero a caller-provided workspace (a fill kernel on `stream`).  Optional. */
int btl_workspace_clear(void* ws, size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BITLINEAR_H */
