// btl_internal.hpp -- shared declarations between the C-ABI layer (btl_api.cpp)
// and the gfx950 kernels (btl_kernels.hip).  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#include <mutex>

namespace btl {

// Keys (a workspace or an output address) -> slots of a device counter array,
// one table per device.  A key keeps its slot for the life of the process and a
// slot never passes to another key, so two launches share counters only when
// they share the key -- and calls that share a workspace or an output are
// already ordered by their caller.  When every slot has a key, find() returns
// -1 and the caller takes a route that needs no counters.
template <int Slots>
struct KeySlots {
    std::mutex mu;
    const void* key[Slots] = {};
    int used = 0;
    int find(const void* k)
    {
        std::lock_guard<std::mutex> lk(mu);
        for (int i = 0; i < used; ++i)
            if (key[i] == k) return i;
        if (used == Slots) return -1;
        key[used] = k;
        return used++;
    }
};

// Routing and tuning knobs.  Each starts from the environment variable of its
// name ("BTL_" + the enumerator's suffix) when set, read once at the first
// library call, else from its built-in default; afterwards only
// btl_set_tuning changes it, so the process environment cannot re-route calls.
enum Knob {
    KN_GEMV_DEC_PARTS,       // force the K parts of the decode kernel (1..16; 0 = measured rule)
    KN_DEC_RQ_WPC,           // force the compute waves of the row-group decode form (0 = rule)
    KN_GEMV_DEC_MAX_M,       // plain launches of up to this many rows take the decode kernel (2)
    KN_GEMV_DEC,             // 0 turns the decode kernel off (1)
    KN_DEC_ROW_MIN_K,        // row-contiguous decode form from this k on (4096)
    KN_DEC_ROW,              // 0 turns the row-contiguous form off (1)
    KN_DEC_ROW_RPW,          // force rows per wave of the row-contiguous form (0 = rule)
    KN_DEC_ROW_RB,           // force row blocks per workgroup of the row-contiguous form (0 = rule)
    KN_GEMV_BAT_MAX_M,       // batched decode up to this many rows (32)
    KN_GEMV_BAT,             // 0 turns the batched decode kernel off (1)
    KN_FUSE_MAX_WG,          // fuse transforms into decode launches of at most this many workgroups (512)
    KN_FUSE_DEC,             // 0 turns transform fusion into the decode kernels off (1)
    KN_DEC_RQ_MIN_K,         // row-group decode form from this k on (1024)
    KN_DEC_RQ,               // 0 turns the row-group decode form off (1)
    KN_DEC_RQ_DG,            // 2 forces two token groups per quantising thread, 4 four for two token rows (0 = rule)
    KN_GEMM_MAX_SPLITS,      // cap on the K splits of the GEMM (0 = none; 1 turns split-K off)
    KN_GEMM_WIDE_MIN_TILES,  // 256-row GEMM tiles from this many workgroups on (512)
    KN_WAIT_SPIN,            // polls before a kernel's internal wait gives up (2^22; the only
                             // knob that can change results: a wait that gives up leaves
                             // invalid outputs and sets the device fault word)
    KN_ATTN_MERGE,           // 0: one-token attention merges its chunks in a second launch (1)
    KN_SPLIT_MERGE,          // 0: the batched decode adds its K splits in a reduce launch (1: in the launch)
    KN_SPLIT_MERGE_MAX_M,    // ... up to this many token rows (16)
    KN_GEMV_BAT_NW,          // force the waves per workgroup of the batched decode kernel (1..16; 0 = rule)
    KN_GEMV_BAT_KS,          // force its K range (1024, 2048, 4096 weights; 0 = rule)
    KN_GEMM_TILE,            // force the prefill GEMM tile (1: 128 rows 2x2 waves, 2: 256 rows, 3: 128 rows 1x4; 0 = rule)
    KN_GEMM_TM64,            // 0: the GEMM keeps 128-token tiles for m <= 64 (1: 64-token tiles)
    KN_GEMM_TM64_STAGES,     // force the LDS stages of the 64-token tiles (2 or 4; 0 = rule)
    KN_GEMM_STAGES,          // force the LDS stages of the 128-token tiles (2 or 3; 0 = rule)
    KN_DEC_RQ2_MAX_K,        // two token rows take the row-group decode form up to this k (16384)
    KN_GEMV_TR,              // 0 turns the token-register batched decode kernel off (1)
    KN_GEMV_TR_MIN_M,        // ... it takes launches from this many token rows (3)
    KN_GEMV_TR_MAX_M,        // ... up to this many (32; at most 64)
    KN_GEMV_TR_RBPW,         // force its 16-row blocks per workgroup (1..8; 0 = rule)
    KN_GEMV_TR_K16,          // ... and launches of at most 16 rows only from this k on (8192)
    KN_COUNT
};
int knob(Knob k);

// Device fault word: bits set by a kernel whose bounded wait gave up (the
// outputs of that launch are then not valid); btl_check_faults reads and
// clears it.
constexpr uint32_t kFaultRqWait = 1u;  // k_gemv_rq: a compute wave's wait for the token row
constexpr uint32_t kFaultStream = 2u;  // the decode stream: a stage's wait for its input
// the fault bits of every kernel source, read after the stream's work, then cleared
hipError_t read_clear_faults(uint32_t* bits, hipStream_t st);

// btl_linear_noalloc: its scratch is a static device array of this many bytes
// (btl_noalloc.hip); scratch_address gives its device address on `dev`, taken
// once per device with hipGetSymbolAddress.
constexpr size_t kScratchBytes = (size_t)32 << 20;
hipError_t scratch_address(int dev, void** out);

constexpr int kMaxGroup = 4;       // layers per grouped launch (q|k|v, w1|w3)
constexpr int kStepWeights = 256;  // weights of one row consumed per wave-load (64 B)

// token input kinds: f32 / bf16 (quantised in the kernel), int8 + scales in
// natural k order (XK_I8) or already in operand order (XK_I8O)
enum XKind { XK_F32 = 0, XK_BF16 = 1, XK_I8 = 2, XK_I8O = 3 };
// activation transforms fused ahead of the quantisation
// XF_ADD_RMSNORM: h = x + x2 (f32 residual + f32 delta, stored to hout), then RMSNorm of h
enum XForm { XF_NONE = 0, XF_RMSNORM = 1, XF_SWIGLU = 2, XF_ADD_RMSNORM = 3 };
enum YKind { YK_F32 = 0, YK_BF16 = 1 };

// One layer of a (possibly grouped) decode launch.
struct GemvProblem {
    const uint8_t* w;  // packed rows, row stride k/4 bytes, 16-byte aligned base
    void* y;           // [m, n] output
    int32_t* acc_out;  // optional [m, n] int32 accumulators
    float sw;          // per-tensor weight scale
    int n;             // output rows of this layer
    int rb_begin;      // first global row-block of this layer
};

struct GemvArgs {
    GemvProblem p[kMaxGroup];
    int nprob;
    const void* x;    // [m, k]: f32 / bf16 (fused quantisation) or int8 (XK_I8)
    const float* xs;  // XK_I8 only: per-row activation scales [m]
    int m, k;
    int rb_total;     // 16-row blocks over all layers
    int tiles;        // RB: row blocks per workgroup
    int parts;        // WV: waves per row block, each one K part (WV * RB <= 16)
    int kpart;        // weights per K part (multiple of 256, at most 2048)
    int ykind;        // YK_F32 / YK_BF16
    // transform fused into the prologue (m == 1, f32 x; XF_RMSNORM and
    // XF_ADD_RMSNORM need k / 16 <= threads): the second input (delta or up),
    // the norm weight, eps, and the summed residual written by workgroup 0
    // (XF_ADD_RMSNORM; must not alias x)
    const float* x2;
    const float* g;
    float eps;
    float* hout;
    // SwiGLU epilogue (swiglu.rs:29-35): layers 0 (gate) and 1 (up) of equal n,
    // tiles == 2; workgroup w computes row block w of both and writes
    // silu(gate) * up to swiglu_out [m, n] f32 (the layers' y may be NULL)
    float* swiglu_out;
    // residual stream added to the f32 output (the row-group form, one layer):
    // y = resid + (float)acc * (s_x * s_w); y may be resid
    const float* resid;
    // bound (polls) of the row-group form's LDS waits; one that gives up sets
    // kFaultRqWait
    int spin;
    // row-contiguous form (m == 1, k % 64 == 0): 0 = K parts; 1, 2, 4 = whole
    // rows of up to that many 4096-weight chunks, 16 / parts rows per wave
    // (parts in {1, 2, 4, 8}, chunks * 16 / parts loads of 1 KB per wave in
    // {4, 8, 16}; kpart unused)
    int rowc;
};

// Loads per wave of the row-contiguous form by default: 4 rows of 1 KB (one
// chunk), 4 rows of 2 KB (two), 2 rows of up to 4 KB (four).
constexpr int dec_row_st(int rowc) { return rowc == 1 ? 4 : 8; }

// Decode (k_gemv_dec): parts * tiles <= 16, parts * kpart >= k, kpart <= 2048,
// a.m <= 4, a.m * k / 16 <= kDecGroups * 64 * parts * tiles.
constexpr int kDecGroups = 4;  // 16-element token groups per thread in the prologue
hipError_t launch_gemv_dec(const GemvArgs& a, int xkind, int xform, hipStream_t s);

// Decode, row-group form (k_gemv_rq): m == 1, k % 64 == 0, k <= 16384, or m == 2
// token rows (no transform, no SwiGLU epilogue; dg = 2 for k <= 4096, else 4).
// R = 4 rows per compute wave for k <= 4096, else 2.  A workgroup is
// rq_quant_waves(k, dg) quantising waves, dg = a.tiles 16-element token groups
// per thread (1 for k <= 4096 only, else 2; 4 for two rows of k > 4096, or
// of any k), and a.parts compute waves, at most
// 16 in all; a.kpart unused.  The SwiGLU epilogue (a.swiglu_out) takes
// operand-order int8 tokens, dg = 2 and an even a.parts; a transform (xform,
// the fields of the decode kernel's) takes f32 tokens, k <= 4096 and dg = 1.
constexpr int rq_quant_waves(int k, int dg, int m = 1) { return ((m * (k / 16) + dg - 1) / dg + 63) / 64; }
hipError_t launch_gemv_rq(const GemvArgs& a, int xkind, int xform, hipStream_t s);

// Prefill GEMM (k_gemm_i8): q is [m, k] int8 in operand order (k_quant_op or
// k_op_order), k % 64 == 0, k < 2^24, 16-byte aligned q and w.  Up to
// kMaxGroup layers that share q run in one launch.
struct GemmLayer {
    const uint8_t* w;  // packed [n, k/4]
    float sw;
    int n;
    void* y;           // [m, n]
    int32_t* acc_out;  // optional [m, n]
    int tile0;         // first output tile of this layer (set by launch_gemm_i8)
    int col0;          // first column of this layer in the partial-sum rows (set by launch_gemm_i8)
};
struct GemmArgs {
    const int8_t* q;   // [m, k] quantised activations, operand order
    const float* sx;   // [m] activation scales
    GemmLayer L[kMaxGroup];
    int nl;
    int m, k;
    int ykind;
    // split-K: splits > 1 runs `splits` workgroups per output tile, each over
    // split_steps K steps of 128, writing exact int32 partial sums to
    // part[split][m][ncols] (ncols = sum of the layers' n); a reduce kernel
    // adds them and applies the epilogue.  splits == 1: part unused.
    int splits, split_steps;
    int32_t* part;
    uint32_t* ctr;     // k_gemv_bat: merge counters (split_counters) -- splits merged in the launch; NULL: reduce launch
    int bat_nw;        // k_gemv_bat: waves per workgroup (4, 8, 16), a row block of 16 bat_nw rows
    int cus;           // compute units of the device (0: unknown), for the GEMM's stage count
    int tr_rbpw;       // k_gemv_tr: 16-row blocks per workgroup (of one layer),
    int tr_cols;       // output columns over the layers (set by launch_gemv_tr)
};

constexpr int kGemmSplitTarget = 512;  // workgroups a split-K launch aims for
// above 64 token rows, K is split only from this k on, for at most this many
// 128 x 128 output tiles
constexpr int kGemmSplitMinK = 8192;
constexpr int kGemmSplitMaxTiles = 128;
// up to 64 token rows, a GEMM of at least this many 128-row tiles runs unsplit
// (64-token tiles, 4 LDS stages; measured on MI355X, Llama-3-8B gate|up at
// m = 24..64: 19-21 us against 31 split three ways)
constexpr int kGemmSmallMUnsplit = 192;
constexpr int kGemmWideMinTiles = 512;  // 256-row GEMM tiles from this many workgroups on
// K splits for an (m, ncols, k) GEMM: enough workgroups to cover the chip when
// the output has few tiles (small m); 1 when it already has kGemmSplitTarget.
int gemm_splits(int64_t m, int64_t tiles_n, int64_t k, int* split_steps);
hipError_t launch_gemm_i8(const GemmArgs& a, hipStream_t s);
// "k_gemm_i8<TN,WGN,NW,TM,NS>" of the calling thread's last launch_gemm_i8
// ("" before the first)
const char* last_gemm_form();

// Batched decode (k_gemv_bat): the GemmArgs of a GEMM with m <= 64, k % 64
// == 0; bat_nw, split_steps (4, 8 or 16 steps of 256 weights per K split)
// and splits = ceil(k / (256 split_steps)) from gemv_bat_plan (rows = the
// output rows of the launch's layers).
struct BatPlan {
    int nw, steps, splits;
};
BatPlan gemv_bat_plan(int64_t m, int64_t rows, int64_t k);
hipError_t launch_gemv_bat(const GemmArgs& a, hipStream_t s);

// The split-K merge of k_gemv_bat inside the launch: a slot of kSplitCounters
// per workspace (KeySlots), one counter per row block; *out = NULL when every
// slot belongs to another workspace (the caller then adds the splits in a
// reduce launch).  The current device must be `dev`.
constexpr int kSplitCounters = 2048;
constexpr int kSplitSlots = 128;
constexpr int kMergeMaxSplits = 16;  // K ranges of >= 1024 weights, k <= 16384
hipError_t split_counters(int dev, const void* ws_key, uint32_t** out);

// Batched decode with the tokens resident in registers (k_gemv_tr), m <= 64,
// k % 64 == 0, k <= 65536.  The tokens are quantised into the token-register
// layout by launch_quant_op(..., tr_mtb = plan.mtb): group g (16 weights) of
// token t at byte tr_offset(t, g, mtb) of a buffer of tr_bytes(k, mtb).  Wave
// w of a workgroup owns K segment (split * nw + w) of 512 weights; a launch
// has `splits` K splits (merged in the launch through a.ctr, which must then
// be non-null: one counter per row group, kSplitCounters at most).
constexpr int kTrSeg = 512;  // weights of one wave's K segment
constexpr int64_t tr_offset(int64_t t, int64_t g, int mtb)
{
    return (((((g >> 5) * mtb + (t >> 4)) * 8 + (g & 7)) * 64) + 16 * ((g >> 3) & 3) + (t & 15)) * 16;
}
constexpr int64_t tr_bytes(int64_t k, int mtb) { return (k + kTrSeg - 1) / kTrSeg * kTrSeg * 16 * mtb; }
struct TrPlan {
    int mtb;     // 16-token blocks held per wave (1, 2 or 4)
    int nw;      // waves (K segments) per workgroup, 1..8
    int splits;  // K splits
    int rbpw;    // 16-row blocks per workgroup, 1..8
};
TrPlan gemv_tr_plan(int64_t m, int64_t row_blocks, int64_t k, int cus);
hipError_t launch_gemv_tr(const GemmArgs& a, const TrPlan& p, hipStream_t s);
// natural-order int8 rows -> operand order (k % 16 == 0, 16-byte aligned)
hipError_t launch_op_order(const int8_t* q, int64_t m, int64_t k, int8_t* out, hipStream_t st);
hipError_t launch_quant_op(const void* x, int xkind, int64_t m, int64_t k, int8_t* q, float* s,
                           hipStream_t st, int tr_mtb = 0);
// fused transform + operand-order quantisation, one workgroup per token row:
// XF_RMSNORM: x / sqrt(pairwise_sum(x*x) * (f32)(1/k) + eps) * g (g: [k] f32);
// XF_SWIGLU:  silu(x) * x2;  XF_ADD_RMSNORM: hout = x + x2 (f32 both; hout may alias
// x), then XF_RMSNORM of it.  k % 64 == 0, k <= 65536; x (and x2) 16-byte aligned.
hipError_t launch_xform_quant(const void* x, const void* x2, int xkind, int xform, const float* g,
                              float eps, int64_t m, int64_t k, int8_t* q, float* s, hipStream_t st,
                              float* hout = nullptr);

hipError_t launch_quant_act(const void* x, int xkind, int64_t m, int64_t k, int8_t* q,
                            float* s, hipStream_t st);

hipError_t launch_ref_f32(const void* x, int xkind, int64_t m, int64_t k, const uint8_t* w,
                          int64_t n, float scale, void* y, int ykind, hipStream_t st);
// the reference's order without AVX2/FMA (one sequential chain per output)
hipError_t launch_ref_seq(const void* x, int xkind, int64_t m, int64_t k, const uint8_t* w,
                          int64_t n, float scale, void* y, int ykind, hipStream_t st);
// several layers over the same x (count <= kMaxGroup): one launch when the
// LDS form applies, else one launch per layer
struct RefGroup {
    const uint8_t* w[kMaxGroup];
    void* y[kMaxGroup];
    float scale[kMaxGroup];
    int64_t n[kMaxGroup];
    int wg_begin[kMaxGroup + 1];  // 32-output workgroups of each layer
    int count;
};
// the transform ahead of a reference-order launch (xf 1: residual add +
// RMSNorm; f32 rows of k, 16-byte aligned)
struct RefXf {
    const float* a;  // h
    const float* b;  // delta (or null)
    float* h_out;    // h (+ delta), stored by the first output tile's workgroups (or null)
    const float* g;  // the norm weight
    float eps;
};
hipError_t launch_ref_f32_group(const void* x, int xkind, int64_t m, int64_t k, const uint8_t* const* w,
                                const int64_t* n, const float* scale, void* const* y, int count, int ykind,
                                hipStream_t st, int xf = 0, const RefXf* t = nullptr);

hipError_t launch_generic_i8(const int8_t* q, const float* xs, int64_t m, int64_t k,
                             const uint8_t* w, int64_t n, float sw, void* y, int ykind,
                             int32_t* acc_out, hipStream_t st);

// PackedTensor::pack on the device: `partials` holds pack_partials(numel) doubles.
int64_t pack_partials(int64_t numel);
hipError_t launch_pack(const float* w, int64_t numel, uint8_t* out, float* scale_out, double* partials,
                       hipStream_t st);
hipError_t launch_unpack(const uint8_t* w, int64_t numel, float scale, float* out,
                         hipStream_t st);

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t st);

// ---------------------------------------------------------------------------
// decoder ops around the BitLinear path (btl_model.hip)
// ---------------------------------------------------------------------------
// RoPE on q / k rows of m new tokens, then the Q8 append of k and v into the
// cache of one layer ([nkv][max_seq][hd] u8 codes, [nkv][max_seq] f32 scales).
struct KvArgs {
    const float* q;        // [m, nh * hd]
    const float* k;        // [m, nkv * hd]
    const float* v;        // [m, nkv * hd]
    float* q_out;          // [m, nh * hd] rotated q (may alias q)
    uint8_t* kc;
    uint8_t* vc;
    float* ksc;
    float* vsc;
    const float* cos_t;    // [max_seq, hd / 2]
    const float* sin_t;
    const int32_t* d_pos;  // position of token 0 on the device, or NULL: `pos`
    int pos;
    int m, nh, nkv, hd, max_seq;
};
hipError_t launch_rope_kv_q8(const KvArgs& a, hipStream_t st);

// Attention of m queries (positions pos0 .. pos0 + m - 1, causal) over the Q8
// cache of one layer: chunk partials into `part` ([m][nh][cmax][hd + 2] f32),
// then their merge into out [m, nh * hd].
struct AttnArgs {
    const float* q;        // [m, nh * hd] rotated queries
    const uint8_t* kc;
    const uint8_t* vc;
    const float* ksc;
    const float* vsc;
    const int32_t* d_pos;  // position of query 0 on the device, or NULL: `pos`
    int pos;
    int m, nh, nkv, hd, max_seq;
    int cmax;              // chunk slots per (query, head): ceil(max_seq / 64)
    int qb;                // queries per workgroup
    float scal;            // (f32)(1 / sqrt(hd))
    float* part;
    float* out;
    uint32_t* ctr;         // one-token attention: the per-KV-head merge counters (attn_counters), or NULL
};
constexpr int kAttnMaxCtr = 64;  // KV heads the one-launch decode attention counts
constexpr int kAttnSlots = 64;   // workspaces with counters of their own, per device
// the merge counters of the workspace `ws_key` (KeySlots), or *out = NULL when
// every slot belongs to another workspace: the merge then runs in a second
// launch.  The current device must be `dev`.
hipError_t attn_counters(int dev, const void* ws_key, uint32_t** out);
hipError_t launch_attention(const AttnArgs& a, hipStream_t st);
// One decode token: RoPE of q and of the new k, the Q8 append of k / v and the
// attention chunk partials in one kernel, then the merge (m == 1, hd % 16 == 0).
struct DecKv {
    const float* q;      // [nh * hd] raw (before RoPE)
    const float* k;      // [nkv * hd] raw
    const float* v;      // [nkv * hd]
    const float* cos_t;  // [max_seq, hd / 2]
    const float* sin_t;
    uint8_t* kc_w;       // the cache, written at the position (same buffers as AttnArgs)
    uint8_t* vc_w;
    float* ksc_w;
    float* vsc_w;
};
hipError_t launch_attention_dec1(const AttnArgs& a, const DecKv& kv, hipStream_t st);

// out[i] = silu(g[i]) * u[i], silu(v) = v / (1 + exp(-v)) (swiglu.rs:29-35), f32
hipError_t launch_swiglu_f32(const float* g, const float* u, int64_t n, float* out, hipStream_t st);
// y[i] = fadd(y[i], r[i]) for i < n (the residual add after a contraction)
hipError_t launch_add_f32(float* y, const float* r, int64_t n, hipStream_t st);

// Multi-base adaptive format (adaptive_linear.rs): at most kMaxBases bases (the
// reference's loader tries 1..=8, adaptive_linear.rs:56).
constexpr int kMaxBases = 8;
struct AdaptiveOut {
    uint8_t* p[kMaxBases];  // base b's PackedTensor bytes [n, k/4]
};
struct AdaptiveScales {
    float s[kMaxBases];
};
struct AdaptiveSum {
    const float* ys[kMaxBases];  // per-base outputs [count] f32
    int nb;
    int64_t count;
    void* y;
    int ykind;
};
hipError_t launch_adaptive_split(const uint8_t* packed, int64_t n, int64_t k, int nb, const AdaptiveOut& out,
                                 hipStream_t st);
hipError_t launch_adaptive_reconstruct(const uint8_t* packed, int64_t n, int64_t k, int nb, const AdaptiveScales& sc,
                                       float* out, hipStream_t st);
hipError_t launch_base_sum(const AdaptiveSum& a, hipStream_t st);

// The decode stream (btl_stream.hip): the one-token projections of nl layers
// (q|k|v, o, gate|up with SwiGLU, down) in one persistent launch of nwg
// workgroups (one per CU, all resident), bf16 between the stages.
struct StreamLayer {
    const uint8_t* w[7];  // packed q, k, v, o, gate, up, down
    float sw[7];
};
struct StreamArgs {
    const StreamLayer* layers;  // [nl], device
    int nl, H, I, nq, nk, nv;   // nq == H; every n a multiple of 4
    int nwg, kmax;              // workgroups; max(H, I)
    const uint16_t* x0;         // bf16 [H] input of layer 0
    uint16_t* y;                // bf16 [H] output of the last layer
    uint32_t* tbuf;             // tagged transport words, nl * (nq + nk + nv + 2 H + I)
    uint64_t* flags;            // [8][nwg] stage flags (sequence | absmax << 32)
    uint32_t* epoch;            // launch epoch (device; starts at 1)
    uint16_t* dbg;              // optional plain bf16 copies of every stage output (tbuf layout)
    int64_t budget_ticks;       // time budget of the waits (s_memrealtime ticks, 100 MHz)
};
size_t stream_lds_bytes(int kmax);
hipError_t launch_dec_stream(const StreamArgs& a, hipStream_t s);
// kFaultStream bits of the stream kernel, read then cleared
hipError_t stream_faults(uint32_t* bits, hipStream_t st);

hipError_t launch_embed(const void* table, int xkind, int64_t vocab, int64_t dim, const int32_t* ids, int64_t m,
                        float* out, hipStream_t st);
hipError_t launch_greedy(const float* x, int64_t n, int32_t* next_id, int32_t* d_pos, int32_t* log,
                         int64_t log_len, hipStream_t st);
hipError_t launch_rmsnorm_f32(const float* h, const float* delta, float* h_out, const float* g, float eps, int64_t m,
                              int64_t k, float* y, hipStream_t st);
hipError_t launch_dense_gemv(const void* w, int wkind, int64_t n, int64_t k, const float* x, int64_t m, float* y,
                             hipStream_t st);

}  // namespace btl
