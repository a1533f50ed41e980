// btl_api.cpp -- the C ABI (include/bitlinear.h): validation, error reporting,
// workspace management, host-side packing and kernel dispatch.
//
// Host-side counterpart of the reference's BitLinearCpu/BitLinearCuda::forward
// (crates/rust_engine/src/kernels/cpu.rs:17-127, cuda.rs:21-47) and
// PackedTensor::{pack, unpack} (kernels/packing.rs:50-133).
#include "bitlinear.h"
#include "bitllama.h"

#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "btl_host.hpp"
#include "btl_internal.hpp"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what)
{
    return fail(BTL_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

constexpr int kMaxDevices = 64;

struct DeviceState {
    bool probed = false;
    bool ok = false;
    int cus = 0;
    std::string arch;
    void* ws = nullptr;  // library-owned workspace
    size_t ws_bytes = 0;
    // workspaces replaced by a larger one; never freed, because a HIP graph
    // captured while one was current still reads and writes it on replay
    std::vector<void*> retired;
};

std::mutex g_mu;
DeviceState g_dev[kMaxDevices];

int probe_device(int dev)
{
    if (dev < 0 || dev >= kMaxDevices) return fail(BTL_ERR_DEVICE, "device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceState& d = g_dev[dev];
    if (!d.probed) {
        d.probed = true;
        hipDeviceProp_t prop;
        hipError_t e = hipGetDeviceProperties(&prop, dev);
        if (e != hipSuccess) {
            d.ok = false;
            return hip_fail(e, "hipGetDeviceProperties");
        }
        d.arch = prop.gcnArchName;
        d.cus = prop.multiProcessorCount;
        d.ok = d.arch.compare(0, 6, "gfx950") == 0;
    }
    if (!d.ok)
        return fail(BTL_ERR_DEVICE, "device %d is '%s'; this library is built for gfx950 only", dev,
                    d.arch.c_str());
    return BTL_OK;
}

int current_device(int* dev)
{
    hipError_t e = hipGetDevice(dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    return probe_device(*dev);
}

// The knobs of btl::Knob: names, built-in defaults, current values.
struct KnobDef {
    const char* name;
    int dflt;
};
constexpr KnobDef kKnobs[btl::KN_COUNT] = {
    {"BTL_GEMV_DEC_PARTS", 0}, {"BTL_DEC_RQ_WPC", 0},     {"BTL_GEMV_DEC_MAX_M", 2},
    {"BTL_GEMV_DEC", 1},       {"BTL_DEC_ROW_MIN_K", 4096}, {"BTL_DEC_ROW", 1},
    {"BTL_DEC_ROW_RPW", 0},    {"BTL_DEC_ROW_RB", 0},     {"BTL_GEMV_BAT_MAX_M", 32},
    {"BTL_GEMV_BAT", 1},       {"BTL_FUSE_MAX_WG", 512},  {"BTL_FUSE_DEC", 1},
    {"BTL_DEC_RQ_MIN_K", 1024}, {"BTL_DEC_RQ", 1},        {"BTL_DEC_RQ_DG", 0},
    {"BTL_GEMM_MAX_SPLITS", 0}, {"BTL_GEMM_WIDE_MIN_TILES", btl::kGemmWideMinTiles},
    {"BTL_WAIT_SPIN", 1 << 22}, {"BTL_ATTN_MERGE", 1}, {"BTL_SPLIT_MERGE", 1},
    {"BTL_SPLIT_MERGE_MAX_M", 16}, {"BTL_GEMV_BAT_NW", 0}, {"BTL_GEMV_BAT_KS", 0},
    {"BTL_GEMM_TILE", 0}, {"BTL_GEMM_TM64", 1}, {"BTL_GEMM_TM64_STAGES", 0}, {"BTL_GEMM_STAGES", 0},
    {"BTL_DEC_RQ2_MAX_K", 16384}, {"BTL_GEMV_TR", 1}, {"BTL_GEMV_TR_MIN_M", 3}, {"BTL_GEMV_TR_MAX_M", 32},
    {"BTL_GEMV_TR_RBPW", 0}, {"BTL_GEMV_TR_K16", 8192},
};
std::atomic<int> g_knob[btl::KN_COUNT];
std::once_flag g_knob_once;

// the environment, read once per process
void knobs_init()
{
    std::call_once(g_knob_once, [] {
        for (int i = 0; i < btl::KN_COUNT; ++i) {
            const char* v = getenv(kKnobs[i].name);
            g_knob[i].store(v && *v ? atoi(v) : kKnobs[i].dflt, std::memory_order_relaxed);
        }
    });
}

int knob_index(const char* name)
{
    if (!name) return -1;
    for (int i = 0; i < btl::KN_COUNT; ++i)
        if (!strcmp(name, kKnobs[i].name) || !strcmp(name, kKnobs[i].name + 4)) return i;
    return -1;
}

inline int env_int(btl::Knob k) { return btl::knob(k); }

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Workspace: scratch for the int8 activations + scales when a call quantises
// once for several token tiles (GEMM, multi-tile GEMV, generic path).  Every
// kernel writes the scratch it reads in the same call, so its contents between
// calls do not matter and one workspace serves calls of any shapes.
struct WsLayout {
    size_t q_off, s_off, p_off, total;
};

// q [m, k] int8 (or q_bytes, when larger: the token-register layout), s [m]
// f32, then `part_bytes` of split-K partial sums
WsLayout ws_layout(int64_t m, int64_t k, size_t part_bytes, size_t q_bytes = 0)
{
    WsLayout l;
    l.q_off = 0;
    l.s_off = align_up((size_t)(m * k) > q_bytes ? (size_t)(m * k) : q_bytes, 256);
    l.p_off = l.s_off + align_up((size_t)(4 * m), 256);
    l.total = l.p_off + align_up(part_bytes, 256);
    return l;
}

// Library-owned per-device workspace, grown on demand (at least doubling).  A
// replaced workspace is retired, not freed: graphs captured while it was current
// keep valid memory (the retired total stays below the current size).  It
// cannot grow while `st` is being captured (the new buffer would not be the one
// the graph's later calls expect, and allocation during capture is not
// ordered with the captured work): the call fails with BTL_ERR_WORKSPACE.
int library_ws(int dev, size_t need, void** out, hipStream_t st)
{
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceState& d = g_dev[dev];
    if (d.ws_bytes < need) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        hipError_t e = hipStreamIsCapturing(st, &cs);
        if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
        if (cs != hipStreamCaptureStatusNone)
            return fail(BTL_ERR_WORKSPACE,
                        "the library workspace of device %d holds %zu bytes and this call needs %zu: it cannot "
                        "grow while the stream is being captured (make the largest call once before capture, "
                        "or pass a workspace of btl_workspace_bytes)",
                        dev, d.ws_bytes, need);
        size_t bytes = align_up(need, (size_t)1 << 20);
        if (bytes < 2 * d.ws_bytes) bytes = 2 * d.ws_bytes;
        void* p = nullptr;
        e = hipMalloc(&p, bytes);
        if (e != hipSuccess) return hip_fail(e, "hipMalloc (workspace)");
        if (d.ws) d.retired.push_back(d.ws);
        d.ws = p;
        d.ws_bytes = bytes;
    }
    *out = d.ws;
    return BTL_OK;
}

int get_ws(int dev, void* ws, size_t ws_bytes, size_t need, void** out, hipStream_t st)
{
    if (!ws) return library_ws(dev, need, out, st);
    if (ws_bytes < need)
        return fail(BTL_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu needed", ws_bytes,
                    need);
    if (((uintptr_t)ws & 255u) != 0) return fail(BTL_ERR_LAYOUT, "workspace must be 256-byte aligned");
    *out = ws;
    return BTL_OK;
}

int check_dtype(int dt, const char* what)
{
    if (dt != BTL_F32 && dt != BTL_BF16) return fail(BTL_ERR_DTYPE, "%s dtype %d is not BTL_F32/BTL_BF16", what, dt);
    return BTL_OK;
}

int check_packed(const btl_packed_t* w, int64_t m, int64_t k)
{
    if (!w) return fail(BTL_ERR_ARG, "null weights");
    if (w->n < 0 || w->k < 0 || m < 0 || k < 0) return fail(BTL_ERR_SHAPE, "negative size");
    if (k != w->k)  // cpu.rs:22-30, cuda.rs:27-35
        return fail(BTL_ERR_SHAPE, "Shape mismatch: Input [%lld, %lld] vs Weight [%lld, %lld]",
                    (long long)m, (long long)k, (long long)w->n, (long long)w->k);
    if (k % 4 != 0)
        return fail(BTL_ERR_SHAPE,
                    "in_features %lld is not a multiple of 4: the packed rows are not byte aligned",
                    (long long)k);
    if (w->n > INT32_MAX || k > INT32_MAX || m > INT32_MAX)
        return fail(BTL_ERR_SHAPE, "dimension exceeds 2^31-1");
    if (!w->data && w->n * k > 0) return fail(BTL_ERR_LAYOUT, "null weight data");
    return BTL_OK;
}

struct Layer {
    const btl_packed_t* w;
    void* y;
    int32_t* acc;
};

// One k_gemm_i8 (or, bat, k_gemv_bat) launch over the layers of a group
// (operand-order q); with splits > 1, the partial sums go to `part` and a
// reduce kernel follows -- or, k_gemv_bat with merge counters `ctr`, the last
// split of each row block adds them in the same launch.
hipError_t launch_gemm(const Layer* layers, int count, const int8_t* q, const float* sx, int64_t m,
                       int64_t k, int ykind, int splits, int split_steps, int32_t* part, bool bat,
                       hipStream_t st, uint32_t* ctr, int bat_nw = 4)
{
    btl::GemmArgs g;
    memset(&g, 0, sizeof(g));
    g.q = q;
    g.sx = sx;
    g.m = (int)m;
    g.k = (int)k;
    g.ykind = ykind;
    g.splits = splits;
    g.split_steps = split_steps;
    g.part = part;
    g.ctr = ctr;
    g.bat_nw = bat_nw;
    int dev = 0;
    if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices) g.cus = g_dev[dev].cus;
    for (int i = 0; i < count; ++i) {
        if (layers[i].w->n == 0) continue;
        btl::GemmLayer& L = g.L[g.nl++];
        L.w = layers[i].w->data;
        L.sw = layers[i].w->scale;
        L.n = (int)layers[i].w->n;
        L.y = layers[i].y;
        L.acc_out = layers[i].acc;
    }
    if (!g.nl) return hipSuccess;
    return bat ? btl::launch_gemv_bat(g, st) : btl::launch_gemm_i8(g, st);
}

int64_t gemm_tiles_n(const Layer* layers, int count)
{
    int64_t t = 0;
    for (int i = 0; i < count; ++i) t += ceil_div(layers[i].w->n, 128);
    return t;
}

int64_t rows_of(const Layer* layers, int count)
{
    int64_t t = 0;
    for (int i = 0; i < count; ++i) t += layers[i].w->n;
    return t;
}

// row blocks of 16 nw rows over the layers of a batched-decode launch
int64_t gemv_row_blocks(const Layer* layers, int count, int nw)
{
    int64_t t = 0;
    for (int i = 0; i < count; ++i) t += ceil_div(layers[i].w->n, 16 * nw);
    return t;
}

// Decode kernel geometry for m <= 4 token rows (measured on MI355X with the
// Llama-3-8B shapes): K parts of 1024 weights, or of 2048 where that would
// take more than 8 waves (k > 8192); RB = 4 / WV row blocks per workgroup
// when WV divides 4, else 1.  BTL_GEMV_DEC_PARTS forces WV (1..16).  0 when
// the tokens do not fit the prologue or the parts exceed 2048 weights.
int dec_waves(int64_t m, int64_t k, int* rb_out)
{
    if (m < 1 || m > 4 || k <= 0) return 0;
    int w = (int)ceil_div(k, 1024);
    if (w > 8) w = (int)ceil_div(k, 2048);
    const int forced = env_int(btl::KN_GEMV_DEC_PARTS);
    if (forced >= 1 && forced <= 16) w = forced;
    const int rb = (w == 1 || w == 2 || w == 4) ? 4 / w : 1;
    const int64_t kp = ceil_div(ceil_div(k, w), btl::kStepWeights) * btl::kStepWeights;
    if (w > 16 || w * rb > 16 || kp > 8 * btl::kStepWeights || m * (k / 16) > (int64_t)btl::kDecGroups * 64 * w * rb)
        return 0;
    *rb_out = rb;
    return w;
}

// Compute waves per workgroup of the row-group decode form: the count in
// [1, 16 - quantising waves] that minimises the compute waves of the busiest CU
// when the workgroups spread evenly over the CUs (ties: the larger workgroup,
// which quantises the token fewer times).  Llama-3-8B on 256 CUs: gate|up 14
// (two workgroups per CU), q|k|v 6, o 4, down 8 (one each).  With the SwiGLU
// pairing (pair_n = the rows of gate and of up) the count is even: half the
// waves take gate's rows, half the same rows of up.  BTL_DEC_RQ_WPC overrides
// it (tuning).
int rq_waves_per_group(int64_t rb_total, int64_t k, int cus, int64_t pair_n, int dg, int m)
{
    const int rows = k <= 4096 ? 4 : 2;
    const int64_t waves = pair_n ? 2 * ceil_div(pair_n, rows) : rb_total * (16 / rows);
    const int hi = 16 - btl::rq_quant_waves((int)k, dg, m);
    const int step = pair_n ? 2 : 1;
    const int forced = env_int(btl::KN_DEC_RQ_WPC);
    if (forced >= step && forced <= hi && forced % step == 0) return forced;
    if (cus < 1) cus = 1;
    int best = step;
    int64_t best_cost = -1;
    for (int w = step; w <= hi; w += step) {
        const int64_t cost = ceil_div(ceil_div(waves, w), cus) * w;
        if (best_cost < 0 || cost <= best_cost) {
            best = w;
            best_cost = cost;
        }
    }
    return best;
}

// Activation transform fused ahead of the quantisation (btl_rmsnorm_linear_group,
// btl_swiglu_linear_group).
struct Xform {
    int kind;        // btl::XF_*
    const void* x2;  // XF_SWIGLU: the up projection's output; XF_ADD_RMSNORM: the delta
    const float* g;  // XF_RMSNORM / XF_ADD_RMSNORM: the norm weight [k]
    float eps;
    float* hout;     // XF_ADD_RMSNORM: the summed residual stream (may alias x)
};

// y += resid for a launch whose kernel did not add it (f32, one layer, y and
// resid not overlapping: checked by the entry point)
int add_resid(const Layer& l, const float* resid, int64_t m, hipStream_t st)
{
    hipError_t e = btl::launch_add_f32((float*)l.y, resid, m * l.w->n, st);
    if (e != hipSuccess) return hip_fail(e, "residual add kernel launch");
    return BTL_OK;
}

// W1.58-A8 contraction of `count` layers sharing one input.
//   any k % 4 == 0 / any alignment .... quantise into scratch, k_generic_i8
//   m <= 4 (decode) ................... k_gemv_dec, quantisation fused
//   otherwise (batched decode, prefill)  quantise in operand order into the
//                                        workspace, one (split-K) launch of
//                                        k_gemv_bat (m <= 32) or k_gemm_i8
// With a transform (xf), the transform + quantisation runs first into the
// workspace on every route (k % 64 == 0 and aligned inputs are checked by the
// caller) and the decode kernel reads the operand-order rows.
// swiglu_out (decode route only; the caller checks it): two layers of equal n,
// silu(y0) * y1 written by the decode kernel's epilogue, y[i] may be NULL.
int run_i8(const Layer* layers, int count, const void* x, int xkind, const float* xs, int64_t m,
           int64_t k, int ykind, void* ws_user, size_t ws_bytes, hipStream_t st, const Xform* xf = nullptr,
           float* swiglu_out = nullptr, const float* resid = nullptr)
{
    int dev;
    int rc = current_device(&dev);
    if (rc) return rc;
    int64_t nsum = 0;
    bool fast = k >= 64 && k % 64 == 0 && k < (1 << 24) && aligned16(x);
    for (int i = 0; i < count; ++i) {
        nsum += layers[i].w->n;
        fast = fast && aligned16(layers[i].w->data);
    }
    if (m == 0 || nsum == 0) return BTL_OK;
    if (!x) return fail(BTL_ERR_LAYOUT, "null input");
    if (xf && !fast) return fail(BTL_ERR_LAYOUT, "fused transform needs k %% 64 == 0 and 16-byte aligned tensors");
    hipError_t e;

    if (!fast) {
        // any k % 4 == 0 / any alignment: quantise once into scratch, one wave per output
        const bool scratch = xkind != btl::XK_I8;
        const WsLayout L = ws_layout(m, k, 0);
        void* ws = nullptr;
        if (scratch && (rc = get_ws(dev, ws_user, ws_bytes, L.total, &ws, st))) return rc;
        const int8_t* q = (const int8_t*)x;
        const float* s = xs;
        if (scratch) {
            q = (const int8_t*)ws + L.q_off;
            s = (const float*)((uint8_t*)ws + L.s_off);
            e = btl::launch_quant_act(x, xkind, m, k, (int8_t*)q, (float*)s, st);
            if (e != hipSuccess) return hip_fail(e, "quantize kernel launch");
        }
        for (int i = 0; i < count; ++i) {
            if (layers[i].w->n == 0) continue;
            e = btl::launch_generic_i8(q, s, m, k, layers[i].w->data, layers[i].w->n, layers[i].w->scale,
                                       layers[i].y, ykind, layers[i].acc, st);
            if (e != hipSuccess) return hip_fail(e, "generic int8 kernel launch");
        }
        return resid ? add_resid(layers[0], resid, m, st) : BTL_OK;
    }

    // Route.  Decode (1..4 token rows): RB row blocks of 16 rows per
    // workgroup, WV waves per row block splitting K.  Batched decode (m <= 32;
    // measured on MI355X: the GEMM is faster from m = 64, Llama-3-8B MLP
    // shapes) and GEMM: K split over workgroups when the output has few tiles.
    int rbw = 1;
    // Plain launches of 3..4 token rows take the batched route (measured on
    // MI355X, Llama-3-8B MLP at m = 4: 24.8 against 29.2 us per layer through
    // the decode kernel); a transform or the SwiGLU epilogue keeps the decode
    // kernel.  BTL_GEMV_DEC_MAX_M overrides the limit (tuning, tests).
    const int dec_max_m = xf || swiglu_out ? 4 : env_int(btl::KN_GEMV_DEC_MAX_M);
    int wv = env_int(btl::KN_GEMV_DEC) != 0 && m <= dec_max_m ? dec_waves(m, k, &rbw) : 0;
    const bool dec = wv > 0;
    // One token row, k a multiple of 64 up to 16384: the row-contiguous form
    // (whole weight rows per wave, 1 KB per load instruction, no K parts).
    // Measured on MI355X for k >= 4096 (Llama-3-8B decode shapes).
    const int rowc = dec && m == 1 && k % 64 == 0 && k >= env_int(btl::KN_DEC_ROW_MIN_K) && k <= 16384 &&
                             env_int(btl::KN_DEC_ROW) != 0
                         ? (k <= 4096 ? 1 : (k <= 8192 ? 2 : 4))
                         : 0;
    if (rowc) {
        // rows per wave: 4 (2 for k > 8192), so 4 KB (8 KB) of loads per wave
        // in workgroups of one row block (measured on MI355X against 8 and 16
        // rows per wave and 2..7 row blocks per workgroup); BTL_DEC_ROW_RPW /
        // BTL_DEC_ROW_RB override them (tuning; launches with a fused
        // transform keep the default)
        int rpw = btl::dec_row_st(rowc) / rowc;
        rbw = 1;
        const int rpw_env = env_int(btl::KN_DEC_ROW_RPW), rb_env = env_int(btl::KN_DEC_ROW_RB);
        if (!xf && (rpw_env == 1 || rpw_env == 2 || rpw_env == 4 || rpw_env == 8 || rpw_env == 16)) {
            rpw = rpw_env;
            while (rowc * rpw > 16) rpw >>= 1;
            while (rowc * rpw < 4) rpw <<= 1;
            rbw = 16 / rpw >= 4 ? 1 : rpw / 4;
        }
        wv = 16 / rpw;
        if (!xf && rb_env >= 1 && rb_env * wv <= 16 && rb_env * wv >= 4) rbw = rb_env;
    }
    if (swiglu_out) {
        if (!dec || wv > 8) return fail(BTL_ERR_ARG, "SwiGLU epilogue needs the decode route");
        rbw = 2;  // workgroup w: row block w of gate and of up
    }
    // Batched decode of KN_GEMV_TR_MIN_M .. KN_GEMV_TR_MAX_M token rows (up to
    // 16 rows only from k = KN_GEMV_TR_K16 on): the token-register kernel
    // (bf16 / f32 input, no transform), tokens quantised straight into its
    // register layout; its K splits (k > 4096) are added in the launch, so it
    // needs this workspace's merge counters (else the routes below).  Measured
    // on MI355X, Llama-3-8B MLP, us per call with the quantiser launch:
    // gate|up (k = 4096) at m = 17..32 15.7-16.1 against 19.5-21.0 through
    // k_gemv_bat / the 64-token GEMM, at m = 3..16 12.5-13.8 against 11.8-12.9;
    // down (k = 14336) at m = 3..32 11.5-16.2 against 12.0-17.5; at m = 40
    // (64 token columns per wave) gate|up 21.0 against 21.2, down 19.3 against 18.0.
    if (!dec && !xf && !swiglu_out && (xkind == btl::XK_F32 || xkind == btl::XK_BF16) && k <= 65536 &&
        m >= env_int(btl::KN_GEMV_TR_MIN_M) && m <= env_int(btl::KN_GEMV_TR_MAX_M) && m <= 64 &&
        (m > 16 || k >= env_int(btl::KN_GEMV_TR_K16)) && env_int(btl::KN_GEMV_TR) != 0) {
        int64_t rbs = 0;
        for (int i = 0; i < count; ++i) rbs += ceil_div(layers[i].w->n, 16);
        const btl::TrPlan tp = btl::gemv_tr_plan(m, rbs, k, g_dev[dev].cus);
        const WsLayout L = ws_layout(m, k, tp.splits > 1 ? (size_t)tp.splits * m * nsum * 4 : 0,
                                     (size_t)btl::tr_bytes(k, tp.mtb));
        void* ws = nullptr;
        if ((rc = get_ws(dev, ws_user, ws_bytes, L.total, &ws, st))) return rc;
        uint32_t* ctr = nullptr;
        if (tp.splits > 1 && ceil_div(rbs, tp.rbpw) <= btl::kSplitCounters &&
            (e = btl::split_counters(dev, ws, &ctr)) != hipSuccess)
            return hip_fail(e, "split-K merge counters");
        if (tp.splits == 1 || ctr) {
            int8_t* q = (int8_t*)ws + L.q_off;
            float* sxp = (float*)((uint8_t*)ws + L.s_off);
            e = btl::launch_quant_op(x, xkind, m, k, q, sxp, st, tp.mtb);
            if (e != hipSuccess) return hip_fail(e, "quantize kernel launch");
            btl::GemmArgs g;
            memset(&g, 0, sizeof(g));
            g.q = q;
            g.sx = sxp;
            g.m = (int)m;
            g.k = (int)k;
            g.ykind = ykind;
            g.part = tp.splits > 1 ? (int32_t*)((uint8_t*)ws + L.p_off) : nullptr;
            g.ctr = ctr;
            for (int i = 0; i < count; ++i) {
                if (layers[i].w->n == 0) continue;
                btl::GemmLayer& gl = g.L[g.nl++];
                gl.w = layers[i].w->data;
                gl.sw = layers[i].w->scale;
                gl.n = (int)layers[i].w->n;
                gl.y = layers[i].y;
                gl.acc_out = layers[i].acc;
            }
            e = btl::launch_gemv_tr(g, tp, st);
            if (e != hipSuccess) return hip_fail(e, "token-register batched gemv kernel launch");
            return resid ? add_resid(layers[0], resid, m, st) : BTL_OK;
        }
    }
    // Batched decode up to KN_GEMV_BAT_MAX_M rows -- but from 21 rows on, a
    // layer group wide enough for the unsplit 64-token GEMM takes that
    // (measured on MI355X, Llama-3-8B gate|up: m = 20 19.6 against 20.8 us, m =
    // 24 21.3 against 20.8, m = 32 23.3 against 21.0)
    const bool gemm_wide = m > 20 && m <= 64 && gemm_tiles_n(layers, count) >= btl::kGemmSmallMUnsplit &&
                           env_int(btl::KN_GEMM_TM64) != 0;
    const bool bat = !dec && !gemm_wide && m <= env_int(btl::KN_GEMV_BAT_MAX_M) && m <= 64 &&
                     env_int(btl::KN_GEMV_BAT) != 0;
    int split_steps = 0, splits = 1;
    btl::BatPlan bp{4, 0, 1};
    if (bat) {
        bp = btl::gemv_bat_plan(m, rows_of(layers, count), k);
        splits = bp.splits;
        split_steps = bp.steps;
    } else if (!dec) {
        splits = btl::gemm_splits(m, gemm_tiles_n(layers, count), k, &split_steps);
    }

    // One-token decode with a transform: the decode kernel applies it in its own
    // prologue (every workgroup on its copy of the row), no separate launch --
    // for f32 input, when the row fits the workgroup for the norm's pairwise
    // sum, and (residual add) when the summed stream goes to another buffer.
    // Every workgroup repeats the transform, so it pays only for launches of
    // at most KN_FUSE_MAX_WG workgroups (measured on MI355X, Llama-3-8B shapes:
    // q|k|v with 384 and down with 256 gain ~2 us; gate|up with 1792 and the
    // 128256-row head lose 2-20 us against the separate one-workgroup
    // transform kernel).
    int64_t dec_rb = 0;
    for (int i = 0; i < count; ++i) dec_rb += ceil_div(layers[i].w->n, 16);
    const int64_t fuse_max_wg = env_int(btl::KN_FUSE_MAX_WG);
    const bool xf_ok = xf && m == 1 && xkind == btl::XK_F32 && env_int(btl::KN_FUSE_DEC) != 0 &&
                       !(xf->kind == btl::XF_ADD_RMSNORM && (const void*)xf->hout == x);

    // One or two token rows (measured on MI355X, Llama-3-8B MLP: down at m = 2
    // 8.1 against 9.1 us through the K-part form; from three rows on the
    // batched kernel is faster, with four rows the row-group form takes four
    // MFMAs per packed word): the row-group form (R whole rows per
    // wave, one accumulator per token row, workgroups of up to 16 waves of
    // which only the first few quantise the tokens).  Its quantising waves also apply a transform (k <=
    // 4096, no SwiGLU epilogue, at most KN_FUSE_MAX_WG workgroups: each repeats
    // it); the SwiGLU pairing takes tokens transformed by a launch of their own.
    const bool rq_on = dec && k % 64 == 0 && k >= env_int(btl::KN_DEC_RQ_MIN_K) && env_int(btl::KN_DEC_RQ) != 0 &&
                       ((m == 1 && k <= 16384) ||
                        (m == 2 && k <= 16384 && k <= env_int(btl::KN_DEC_RQ2_MAX_K) && !xf && !swiglu_out));
    bool rqx = false;
    int rqx_wpc = 0;
    if (rq_on && xf_ok && k <= 4096 && (!swiglu_out || xf->kind == btl::XF_RMSNORM)) {
        // with the SwiGLU pairing (RMSNorm only): two groups per quantising thread
        const int64_t pn = swiglu_out ? layers[0].w->n : 0;
        rqx_wpc = rq_waves_per_group(dec_rb, k, g_dev[dev].cus, pn, swiglu_out ? 2 : 1, 1);
        rqx = (swiglu_out ? ceil_div(ceil_div(pn, 4), rqx_wpc / 2) : ceil_div(dec_rb * 4, rqx_wpc)) <= fuse_max_wg;
    }
    // Otherwise the K-part / row-contiguous decode kernel applies a transform in
    // its own prologue for launches of at most KN_FUSE_MAX_WG workgroups.
    const bool fuse = !rqx && dec && xf_ok && ceil_div(dec_rb, rbw) <= fuse_max_wg && wv * rbw <= 8 &&
                      k / 16 <= (int64_t)(xf->kind == btl::XF_SWIGLU ? 2 : 1) * wv * rbw * 64;
    const bool rq = rq_on && !fuse && (!swiglu_out || xf);

    // operand-order quantisation into the workspace (all routes but plain decode)
    const bool pre = (xf && !fuse && !rqx) || !dec;
    const int8_t* q = nullptr;
    const float* sxp = xs;
    void* ws = nullptr;
    WsLayout L = ws_layout(m, k, splits > 1 ? (size_t)splits * m * nsum * 4 : 0);
    if (pre) {
        if ((rc = get_ws(dev, ws_user, ws_bytes, L.total, &ws, st))) return rc;
        q = (const int8_t*)ws + L.q_off;
        if (xf) {
            sxp = (const float*)((uint8_t*)ws + L.s_off);
            e = btl::launch_xform_quant(x, xf->x2, xkind, xf->kind, xf->g, xf->eps, m, k, (int8_t*)q, (float*)sxp, st,
                                        xf->hout);
        } else if (xkind == btl::XK_I8) {
            e = btl::launch_op_order((const int8_t*)x, m, k, (int8_t*)q, st);
        } else {
            sxp = (const float*)((uint8_t*)ws + L.s_off);
            e = btl::launch_quant_op(x, xkind, m, k, (int8_t*)q, (float*)sxp, st);
        }
        if (e != hipSuccess) return hip_fail(e, "quantize kernel launch");
    }

    if (dec) {
        const int64_t kpart = ceil_div(ceil_div(k, wv), btl::kStepWeights) * btl::kStepWeights;
        btl::GemvArgs a;
        memset(&a, 0, sizeof(a));
        int rb = 0, np = 0;
        for (int i = 0; i < count; ++i) {
            const int64_t n = layers[i].w->n;
            if (n == 0) continue;
            btl::GemvProblem& p = a.p[np++];
            p.w = layers[i].w->data;
            p.y = layers[i].y;
            p.acc_out = layers[i].acc;
            p.sw = layers[i].w->scale;
            p.n = (int)n;
            p.rb_begin = rb;
            rb += (int)ceil_div(n, 16);
        }
        a.nprob = np;
        a.x = pre ? (const void*)q : x;
        a.xs = sxp;
        a.m = (int)m;
        a.k = (int)k;
        a.rb_total = rb;
        a.tiles = rbw;
        a.parts = wv;
        a.kpart = (int)kpart;
        a.ykind = ykind;
        int xform = btl::XF_NONE;
        if (fuse || rqx) {
            xform = xf->kind;
            a.x2 = (const float*)xf->x2;
            a.g = xf->g;
            a.eps = xf->eps;
            a.hout = xf->hout;
        }
        a.swiglu_out = swiglu_out;
        a.rowc = rowc;
        a.spin = env_int(btl::KN_WAIT_SPIN);
        if (rq) {
            // two token rows of k > 4096: four token groups per quantising
            // thread (two would take 14 quantising waves of the 16)
            const int dg2 = m == 2 && (k > 4096 || env_int(btl::KN_DEC_RQ_DG) == 4) ? 4 : 2;
            a.parts = rqx ? rqx_wpc
                          : rq_waves_per_group(rb, k, g_dev[dev].cus, swiglu_out ? a.p[0].n : 0, dg2, (int)m);
            // one token group per quantising thread when the workgroup has room
            // for the quantising waves that takes (one token row, k <= 4096): a
            // shorter prologue for the launches of few compute waves
            a.tiles = (rqx && !swiglu_out) ||
                              (!rqx && m == 1 && k <= 4096 && !swiglu_out &&
                               btl::rq_quant_waves((int)k, 1) + a.parts <= 16 && env_int(btl::KN_DEC_RQ_DG) != 2)
                          ? 1
                          : dg2;
            a.resid = count == 1 ? resid : nullptr;
            e = btl::launch_gemv_rq(a, pre ? (int)btl::XK_I8O : xkind, rqx ? xform : (int)btl::XF_NONE, st);
            if (e != hipSuccess) return hip_fail(e, "decode gemv kernel launch");
            if (resid && !a.resid) return add_resid(layers[0], resid, m, st);
            return BTL_OK;
        }
        e = btl::launch_gemv_dec(a, pre ? (int)btl::XK_I8O : xkind, xform, st);
        if (e != hipSuccess) return hip_fail(e, "decode gemv kernel launch");
        return resid ? add_resid(layers[0], resid, m, st) : BTL_OK;
    }
    // batched decode: the K splits merged in the launch (counters of this
    // workspace) up to 16 token rows -- measured on MI355X, Llama-3-8B MLP: 1-2 us
    // per layer faster at m = 4..16, 4 us slower at m = 32, where one workgroup
    // per row block adds 2048 outputs' partials and gate|up splits too
    uint32_t* ctr = nullptr;
    if (bat && splits > 1 && m <= env_int(btl::KN_SPLIT_MERGE_MAX_M) && env_int(btl::KN_SPLIT_MERGE) != 0 &&
        splits <= btl::kMergeMaxSplits && gemv_row_blocks(layers, count, bp.nw) <= btl::kSplitCounters) {
        if ((e = btl::split_counters(dev, ws, &ctr)) != hipSuccess) return hip_fail(e, "split-K merge counters");
    }
    e = launch_gemm(layers, count, q, sxp, m, k, ykind, splits, split_steps,
                    splits > 1 ? (int32_t*)((uint8_t*)ws + L.p_off) : nullptr, bat, st, ctr, bp.nw);
    if (e != hipSuccess) return hip_fail(e, bat ? "batched gemv kernel launch" : "gemm kernel launch");
    return resid ? add_resid(layers[0], resid, m, st) : BTL_OK;
}

// Shared validation of the fused entry points; fills `ls`.
int check_group(const btl_packed_t* const* w, void* const* y, int count, int64_t m, int64_t k,
                int ydtype, Layer* ls)
{
    if (count < 1 || count > btl::kMaxGroup) return fail(BTL_ERR_ARG, "count %d not in 1..%d", count, btl::kMaxGroup);
    if (!w || !y) return fail(BTL_ERR_ARG, "null layer array");
    int rc;
    if ((rc = check_dtype(ydtype, "output"))) return rc;
    for (int i = 0; i < count; ++i) {
        if ((rc = check_packed(w[i], m, k))) return rc;
        if (!y[i] && m > 0 && w[i]->n > 0) return fail(BTL_ERR_LAYOUT, "null output %d", i);
        ls[i] = Layer{w[i], y[i], nullptr};
    }
    return BTL_OK;
}

int check_fused_shape(int64_t k, int64_t kmax, const char* what)
{
    if (k % 64 != 0 || k < 64 || k > kmax)
        return fail(BTL_ERR_SHAPE, "%s needs k %% 64 == 0 and 64 <= k <= %lld, got k = %lld", what,
                    (long long)kmax, (long long)k);
    return BTL_OK;
}

// sum of |w| in double as the pairwise tree over the elements in index order,
// zero-padded to a power of two (the order btl_pack_device reproduces)
double abs_pairwise_rec(const float* w, int64_t numel, int64_t a, int64_t len)
{
    if (len == 1) return a < numel ? std::fabs((double)w[a]) : 0.0;
    const int64_t h = len / 2;
    const double lo = abs_pairwise_rec(w, numel, a, h);
    const double hi = a + h < numel ? abs_pairwise_rec(w, numel, a + h, h) : 0.0;
    return lo + hi;
}

double abs_pairwise(const float* w, int64_t numel)
{
    if (numel <= 0) return 0.0;
    int64_t len = 1;
    while (len < numel) len *= 2;
    return abs_pairwise_rec(w, numel, 0, len);
}

}  // namespace

extern "C" {

int btl_version(void) { return BTL_VERSION; }

const char* btl_last_error(void) { return g_err.c_str(); }

const char* btl_status_string(int status)
{
    switch (status) {
    case BTL_OK: return "BTL_OK";
    case BTL_ERR_SHAPE: return "BTL_ERR_SHAPE";
    case BTL_ERR_DTYPE: return "BTL_ERR_DTYPE";
    case BTL_ERR_LAYOUT: return "BTL_ERR_LAYOUT";
    case BTL_ERR_DEVICE: return "BTL_ERR_DEVICE";
    case BTL_ERR_HIP: return "BTL_ERR_HIP";
    case BTL_ERR_ARG: return "BTL_ERR_ARG";
    case BTL_ERR_WORKSPACE: return "BTL_ERR_WORKSPACE";
    case BTL_ERR_FAULT: return "BTL_ERR_FAULT";
    default: return "BTL_ERR_UNKNOWN";
    }
}

int btl_set_tuning(const char* name, int value)
{
    knobs_init();
    const int i = knob_index(name);
    if (i < 0) return fail(BTL_ERR_ARG, "unknown tuning knob '%s'", name ? name : "(null)");
    g_knob[i].store(value, std::memory_order_relaxed);
    return BTL_OK;
}

int btl_get_tuning(const char* name, int* value)
{
    knobs_init();
    const int i = knob_index(name);
    if (i < 0) return fail(BTL_ERR_ARG, "unknown tuning knob '%s'", name ? name : "(null)");
    if (!value) return fail(BTL_ERR_ARG, "null pointer");
    *value = g_knob[i].load(std::memory_order_relaxed);
    return BTL_OK;
}

const char* btl_last_gemm_form(void) { return btl::last_gemm_form(); }

int btl_check_faults(void* stream)
{
    int dev;
    int rc = current_device(&dev);
    if (rc) return rc;
    uint32_t bits = 0;
    hipError_t e = btl::read_clear_faults(&bits, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "reading the device fault word");
    if (bits)
        return fail(BTL_ERR_FAULT,
                    "a bounded wait inside a kernel gave up on device %d (fault bits 0x%x: %s%s); the outputs of "
                    "the calls since the last check are not valid",
                    dev, bits, (bits & btl::kFaultRqWait) ? "decode workgroup token row" : "",
                    (bits & btl::kFaultStream) ? " decode stream stage" : "");
    return BTL_OK;
}

int btl_init(int device)
{
    knobs_init();
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    if (device < 0 || device >= count) return fail(BTL_ERR_DEVICE, "device %d not present (%d devices)", device, count);
    int rc = probe_device(device);
    if (rc) return rc;
    // the device address of btl_linear_noalloc's scratch array, taken once per device
    void* scratch = nullptr;
    e = btl::scratch_address(device, &scratch);
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress (scratch)");
    return BTL_OK;
}

int64_t btl_packed_bytes(int64_t n, int64_t k)
{
    if (n < 0 || k < 0) return -1;
    return (n * k + 3) / 4;
}

// PackedTensor::pack (packing.rs:50-105).  The mean of |w| is accumulated in
// double and rounded once; 1/scale is taken in double and rounded to f32, as
// candle's `tensor / f64` multiplies by the reciprocal (packing.rs:61).
int btl_pack_host(const float* w, int64_t n, int64_t k, uint8_t* out, float* scale)
{
    if (n < 0 || k < 0) return fail(BTL_ERR_SHAPE, "negative size");
    const int64_t numel = n * k;
    if ((numel && (!w || !out)) || !scale) return fail(BTL_ERR_ARG, "null pointer");
    const double acc = abs_pairwise(w, numel);
    const float mean = numel ? (float)(acc / (double)numel) : 0.0f;
    const float s = mean + 1e-6f;  // EPSILON, packing.rs:4
    const float inv = (float)(1.0 / (double)s);
    const int64_t nbytes = (numel + 3) / 4;
    for (int64_t b = 0; b < nbytes; ++b) {
        uint8_t byte = 0;
        for (int i = 0; i < 4; ++i) {
            const int64_t e = 4 * b + i;
            if (e >= numel) break;
            float v = std::round(w[e] * inv);  // f32::round: half away from zero
            v = v > 1.0f ? 1.0f : (v < -1.0f ? -1.0f : v);
            const uint8_t code = v > 0.5f ? 1 : (v < -0.5f ? 2 : 0);
            byte |= (uint8_t)(code << (2 * i));
        }
        out[b] = byte;
    }
    *scale = s;
    return BTL_OK;
}

int btl_unpack_host(const uint8_t* data, int64_t n, int64_t k, float scale, float* out)
{
    if (n < 0 || k < 0) return fail(BTL_ERR_SHAPE, "negative size");
    const int64_t numel = n * k;
    if (numel && (!data || !out)) return fail(BTL_ERR_ARG, "null pointer");
    for (int64_t e = 0; e < numel; ++e) {
        const int code = (data[e >> 2] >> (2 * (e & 3))) & 3;
        const float v = code == 1 ? 1.0f : (code == 2 ? -1.0f : 0.0f);
        out[e] = v * scale;
    }
    return BTL_OK;
}

size_t btl_pack_workspace_bytes(int64_t n, int64_t k)
{
    if (n < 0 || k < 0 || n * k == 0) return 0;
    return (size_t)btl::pack_partials(n * k) * sizeof(double);
}

int btl_pack_device(const float* w, int64_t n, int64_t k, uint8_t* out, float* scale, void* ws, size_t ws_bytes,
                    void* stream)
{
    if (n < 0 || k < 0) return fail(BTL_ERR_SHAPE, "negative size");
    const int64_t numel = n * k;
    if (!scale || (numel && (!w || !out))) return fail(BTL_ERR_ARG, "null pointer");
    if (!aligned16(w) || ((uintptr_t)out & 3u)) return fail(BTL_ERR_LAYOUT, "w must be 16-byte and out 4-byte aligned");
    int dev;
    int rc = current_device(&dev);
    if (rc) return rc;
    hipError_t e;
    if (numel == 0) {  // mean of nothing: 0, scale = 1e-6
        const float s = 1e-6f;
        e = hipMemcpyAsync(scale, &s, sizeof(float), hipMemcpyHostToDevice, (hipStream_t)stream);
        if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
        return e == hipSuccess ? BTL_OK : hip_fail(e, "scale copy");
    }
    void* wsp = nullptr;
    if ((rc = get_ws(dev, ws, ws_bytes, btl_pack_workspace_bytes(n, k), &wsp, (hipStream_t)stream))) return rc;
    e = btl::launch_pack(w, numel, out, scale, (double*)wsp, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "pack kernel launch");
    return BTL_OK;
}

int btl_unpack_device(const btl_packed_t* w, float* out, void* stream)
{
    if (!w) return fail(BTL_ERR_ARG, "null weights");
    if (w->n < 0 || w->k < 0) return fail(BTL_ERR_SHAPE, "negative size");
    const int64_t numel = w->n * w->k;
    if (numel == 0) return BTL_OK;
    if (!w->data || !out) return fail(BTL_ERR_LAYOUT, "null pointer");
    int dev;
    int rc = current_device(&dev);
    if (rc) return rc;
    hipError_t e = btl::launch_unpack(w->data, numel, w->scale, out, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "unpack kernel launch");
    return BTL_OK;
}

int btl_quantize_act(const void* x, int xdtype, int64_t m, int64_t k, int8_t* xq, float* xscale,
                     void* stream)
{
    int rc = check_dtype(xdtype, "input");
    if (rc) return rc;
    if (m < 0 || k < 0) return fail(BTL_ERR_SHAPE, "negative size");
    if (m == 0) return BTL_OK;
    if (!xscale || (k > 0 && (!x || !xq))) return fail(BTL_ERR_LAYOUT, "null pointer");
    int dev;
    rc = current_device(&dev);
    if (rc) return rc;
    hipError_t e = btl::launch_quant_act(x, xdtype == BTL_BF16 ? btl::XK_BF16 : btl::XK_F32, m, k, xq, xscale,
                                         (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "quantize kernel launch");
    return BTL_OK;
}

int btl_linear(const btl_packed_t* w, const void* x, int xdtype, int64_t m, int64_t k, void* y,
               int ydtype, int mode, int32_t* acc_out, void* ws, size_t ws_bytes, void* stream)
{
    int rc = check_packed(w, m, k);
    if (rc) return rc;
    if ((rc = check_dtype(xdtype, "input")) || (rc = check_dtype(ydtype, "output"))) return rc;
    if (mode != BTL_ACT_F32_REF && mode != BTL_ACT_I8 && mode != BTL_ACT_F32_SEQ)
        return fail(BTL_ERR_DTYPE, "unknown mode %d", mode);
    if (mode != BTL_ACT_I8 && acc_out) return fail(BTL_ERR_ARG, "acc_out is only defined for BTL_ACT_I8");
    if (m == 0 || w->n == 0) return BTL_OK;
    if (!y || (k > 0 && !x)) return fail(BTL_ERR_LAYOUT, "null input or output");
    const hipStream_t st = (hipStream_t)stream;
    const int xk = xdtype == BTL_BF16 ? btl::XK_BF16 : btl::XK_F32;
    const int yk = ydtype == BTL_BF16 ? btl::YK_BF16 : btl::YK_F32;
    if (mode == BTL_ACT_F32_REF) {
        int dev;
        rc = current_device(&dev);
        if (rc) return rc;
        hipError_t e = btl::launch_ref_f32(x, xk, m, k, w->data, w->n, w->scale, y, yk, st);
        if (e != hipSuccess) return hip_fail(e, "reference-order kernel launch");
        return BTL_OK;
    }
    if (mode == BTL_ACT_F32_SEQ) {
        int dev;
        rc = current_device(&dev);
        if (rc) return rc;
        hipError_t e = btl::launch_ref_seq(x, xk, m, k, w->data, w->n, w->scale, y, yk, st);
        if (e != hipSuccess) return hip_fail(e, "sequential reference-order kernel launch");
        return BTL_OK;
    }
    Layer l = {w, y, acc_out};
    return run_i8(&l, 1, x, xk, nullptr, m, k, yk, ws, ws_bytes, st);
}

int btl_linear_noalloc(const btl_packed_t* w, const void* x, int xdtype, int64_t m, int64_t k, void* y,
                       int ydtype, int mode, int32_t* acc_out, void* stream)
{
    int rc = check_packed(w, m, k);
    if (rc) return rc;
    if ((rc = check_dtype(xdtype, "input")) || (rc = check_dtype(ydtype, "output"))) return rc;
    if (mode == BTL_ACT_I8 && m > 0 && w->n > 0) {
        const size_t need = btl_workspace_bytes(m, w->n, k, BTL_ACT_I8);
        if (need > btl::kScratchBytes)
            return fail(BTL_ERR_WORKSPACE,
                        "btl_linear_noalloc: [%lld, %lld] x [%lld, %lld] needs %zu bytes of scratch; its fixed "
                        "device array holds %zu (use btl_linear with a workspace)",
                        (long long)m, (long long)k, (long long)w->n, (long long)k, need, btl::kScratchBytes);
        int dev;
        if ((rc = current_device(&dev))) return rc;
        void* scratch = nullptr;
        const hipError_t e = btl::scratch_address(dev, &scratch);
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress (scratch)");
        return btl_linear(w, x, xdtype, m, k, y, ydtype, mode, acc_out, scratch, btl::kScratchBytes, stream);
    }
    // the reference-order modes and empty calls use no scratch
    return btl_linear(w, x, xdtype, m, k, y, ydtype, mode, acc_out, nullptr, 0, stream);
}

int btl_linear_i8(const btl_packed_t* w, const int8_t* xq, const float* xscale, int64_t m, int64_t k,
                  void* y, int ydtype, int32_t* acc_out, void* ws, size_t ws_bytes, void* stream)
{
    int rc = check_packed(w, m, k);
    if (rc) return rc;
    if ((rc = check_dtype(ydtype, "output"))) return rc;
    if (m == 0 || w->n == 0) return BTL_OK;
    if (!y || !xscale || (k > 0 && !xq)) return fail(BTL_ERR_LAYOUT, "null input or output");
    Layer l = {w, y, acc_out};
    return run_i8(&l, 1, xq, btl::XK_I8, xscale, m, k, ydtype == BTL_BF16 ? btl::YK_BF16 : btl::YK_F32, ws,
                  ws_bytes, (hipStream_t)stream);
}

int btl_linear_group(const btl_packed_t* const* w, void* const* y, int count, const void* x,
                     int xdtype, int64_t m, int64_t k, int ydtype, void* ws, size_t ws_bytes,
                     void* stream)
{
    if (count < 1 || count > btl::kMaxGroup) return fail(BTL_ERR_ARG, "count %d not in 1..%d", count, btl::kMaxGroup);
    if (!w || !y) return fail(BTL_ERR_ARG, "null layer array");
    int rc;
    if ((rc = check_dtype(xdtype, "input")) || (rc = check_dtype(ydtype, "output"))) return rc;
    Layer ls[btl::kMaxGroup];
    for (int i = 0; i < count; ++i) {
        if ((rc = check_packed(w[i], m, k))) return rc;
        if (!y[i] && m > 0 && w[i]->n > 0) return fail(BTL_ERR_LAYOUT, "null output %d", i);
        ls[i] = Layer{w[i], y[i], nullptr};
    }
    return run_i8(ls, count, x, xdtype == BTL_BF16 ? btl::XK_BF16 : btl::XK_F32, nullptr, m, k,
                  ydtype == BTL_BF16 ? btl::YK_BF16 : btl::YK_F32, ws, ws_bytes, (hipStream_t)stream);
}

int btl_linear_group_mode(const btl_packed_t* const* w, void* const* y, int count, const void* x, int xdtype,
                          int64_t m, int64_t k, int ydtype, int mode, void* ws, size_t ws_bytes, void* stream)
{
    if (mode == BTL_ACT_I8) return btl_linear_group(w, y, count, x, xdtype, m, k, ydtype, ws, ws_bytes, stream);
    if (mode != BTL_ACT_F32_REF && mode != BTL_ACT_F32_SEQ) return fail(BTL_ERR_DTYPE, "unknown mode %d", mode);
    if (count < 1 || count > btl::kMaxGroup) return fail(BTL_ERR_ARG, "count %d not in 1..%d", count, btl::kMaxGroup);
    if (!w || !y) return fail(BTL_ERR_ARG, "null layer array");
    int rc;
    if ((rc = check_dtype(xdtype, "input")) || (rc = check_dtype(ydtype, "output"))) return rc;
    const uint8_t* wd[btl::kMaxGroup];
    int64_t n[btl::kMaxGroup];
    float sc[btl::kMaxGroup];
    void* yy[btl::kMaxGroup];
    int64_t nsum = 0;
    for (int i = 0; i < count; ++i) {
        if ((rc = check_packed(w[i], m, k))) return rc;
        if (!y[i] && m > 0 && w[i]->n > 0) return fail(BTL_ERR_LAYOUT, "null output %d", i);
        wd[i] = w[i]->data;
        n[i] = w[i]->n;
        sc[i] = w[i]->scale;
        yy[i] = y[i];
        nsum += w[i]->n;
    }
    if (m == 0 || nsum == 0) return BTL_OK;
    if (k > 0 && !x) return fail(BTL_ERR_LAYOUT, "null input");
    int dev;
    if ((rc = current_device(&dev))) return rc;
    const int xk = xdtype == BTL_BF16 ? btl::XK_BF16 : btl::XK_F32;
    const int yk = ydtype == BTL_BF16 ? btl::YK_BF16 : btl::YK_F32;
    if (mode == BTL_ACT_F32_SEQ) {  // one launch per layer
        for (int i = 0; i < count; ++i) {
            const hipError_t e = btl::launch_ref_seq(x, xk, m, k, wd[i], n[i], sc[i], yy[i], yk, (hipStream_t)stream);
            if (e != hipSuccess) return hip_fail(e, "sequential reference-order kernel launch");
        }
        return BTL_OK;
    }
    const hipError_t e = btl::launch_ref_f32_group(x, xk, m, k, wd, n, sc, yy, count, yk, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "reference-order kernel launch");
    return BTL_OK;
}

int btl_quantize_act_op(const void* x, int xdtype, int64_t m, int64_t k, int8_t* xq, float* xscale,
                        void* stream)
{
    int rc = check_dtype(xdtype, "input");
    if (rc) return rc;
    if (m < 0 || k < 0) return fail(BTL_ERR_SHAPE, "negative size");
    if (k % 64 != 0 || k >= (1 << 24))
        return fail(BTL_ERR_SHAPE, "operand-order layout needs k %% 64 == 0 and k < 2^24, got k = %lld",
                    (long long)k);
    if (m > INT32_MAX) return fail(BTL_ERR_SHAPE, "dimension exceeds 2^31-1");
    if (m == 0 || k == 0) return BTL_OK;
    if (!x || !xq || !xscale) return fail(BTL_ERR_LAYOUT, "null pointer");
    if (!aligned16(x) || !aligned16(xq)) return fail(BTL_ERR_LAYOUT, "x and xq must be 16-byte aligned");
    int dev;
    if ((rc = current_device(&dev))) return rc;
    hipError_t e = btl::launch_quant_op(x, xdtype == BTL_BF16 ? btl::XK_BF16 : btl::XK_F32, m, k, xq, xscale,
                                        (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "quantize kernel launch");
    return BTL_OK;
}

int btl_linear_i8_op(const btl_packed_t* const* w, void* const* y, int32_t* const* acc_out, int count,
                     const int8_t* xq, const float* xscale, int64_t m, int64_t k, int ydtype, void* stream)
{
    if (count < 1 || count > btl::kMaxGroup) return fail(BTL_ERR_ARG, "count %d not in 1..%d", count, btl::kMaxGroup);
    if (!w || !y) return fail(BTL_ERR_ARG, "null layer array");
    int rc;
    if ((rc = check_dtype(ydtype, "output"))) return rc;
    Layer ls[btl::kMaxGroup];
    int64_t nsum = 0;
    for (int i = 0; i < count; ++i) {
        if ((rc = check_packed(w[i], m, k))) return rc;
        if (!y[i] && m > 0 && w[i]->n > 0) return fail(BTL_ERR_LAYOUT, "null output %d", i);
        if (w[i]->n > 0 && k > 0 && !aligned16(w[i]->data))
            return fail(BTL_ERR_LAYOUT, "packed weights %d must be 16-byte aligned", i);
        ls[i] = Layer{w[i], y[i], acc_out ? acc_out[i] : nullptr};
        nsum += w[i]->n;
    }
    if (k % 64 != 0 || k >= (1 << 24))
        return fail(BTL_ERR_SHAPE, "operand-order layout needs k %% 64 == 0 and k < 2^24, got k = %lld",
                    (long long)k);
    if (m == 0 || nsum == 0) return BTL_OK;
    if (k > 0 && (!xq || !xscale)) return fail(BTL_ERR_LAYOUT, "null input");
    if (!aligned16(xq)) return fail(BTL_ERR_LAYOUT, "xq must be 16-byte aligned");
    int dev;
    if ((rc = current_device(&dev))) return rc;
    hipError_t e = launch_gemm(ls, count, xq, xscale, m, k, ydtype == BTL_BF16 ? btl::YK_BF16 : btl::YK_F32,
                               1, 0, nullptr, false, (hipStream_t)stream, nullptr);
    if (e != hipSuccess) return hip_fail(e, "gemm kernel launch");
    return BTL_OK;
}

int btl_rmsnorm_linear_group(const btl_packed_t* const* w, void* const* y, int count, const void* x,
                             int xdtype, const float* g, float eps, int64_t m, int64_t k, int ydtype,
                             void* ws, size_t ws_bytes, void* stream)
{
    Layer ls[btl::kMaxGroup];
    int rc;
    if ((rc = check_dtype(xdtype, "input")) || (rc = check_group(w, y, count, m, k, ydtype, ls))) return rc;
    if ((rc = check_fused_shape(k, 65536, "fused RMSNorm"))) return rc;
    if (m == 0) return BTL_OK;
    if (!x || !g) return fail(BTL_ERR_LAYOUT, "null input or norm weight");
    if (!aligned16(x) || !aligned16(g)) return fail(BTL_ERR_LAYOUT, "x and g must be 16-byte aligned");
    const Xform xf{btl::XF_RMSNORM, nullptr, g, eps, nullptr};
    return run_i8(ls, count, x, xdtype == BTL_BF16 ? btl::XK_BF16 : btl::XK_F32, nullptr, m, k,
                  ydtype == BTL_BF16 ? btl::YK_BF16 : btl::YK_F32, ws, ws_bytes, (hipStream_t)stream, &xf);
}

int btl_add_rmsnorm_linear_group(const btl_packed_t* const* w, void* const* y, int count, const float* h,
                                 const float* delta, float* h_out, const float* g, float eps, int64_t m, int64_t k,
                                 int ydtype, void* ws, size_t ws_bytes, void* stream)
{
    Layer ls[btl::kMaxGroup];
    int rc;
    if ((rc = check_group(w, y, count, m, k, ydtype, ls))) return rc;
    if ((rc = check_fused_shape(k, 65536, "fused residual + RMSNorm"))) return rc;
    if (m == 0) return BTL_OK;
    if (!h || !g) return fail(BTL_ERR_LAYOUT, "null residual or norm weight");
    if (!aligned16(h) || !aligned16(g) || (delta && !aligned16(delta)) || (delta && h_out && !aligned16(h_out)))
        return fail(BTL_ERR_LAYOUT, "h, delta, h_out and g must be 16-byte aligned");
    if (delta && h_out && h_out != h) {
        const uintptr_t a0 = (uintptr_t)h, a1 = (uintptr_t)h_out, nb = (uintptr_t)(m * k * 4);
        if (a0 < a1 + nb && a1 < a0 + nb) return fail(BTL_ERR_LAYOUT, "h_out overlaps h without being h");
    }
    const Xform xf{delta ? btl::XF_ADD_RMSNORM : btl::XF_RMSNORM, delta, g, eps, delta ? h_out : nullptr};
    return run_i8(ls, count, h, btl::XK_F32, nullptr, m, k, ydtype == BTL_BF16 ? btl::YK_BF16 : btl::YK_F32, ws,
                  ws_bytes, (hipStream_t)stream, &xf);
}

namespace {
// the reference-order group behind a transform (xf 1): f32 rows of k staged
// by the kernel itself (k % 64 == 0, 64 <= k <= 16384, 16-byte aligned rows)
int run_ref_xf(const btl_packed_t* const* w, void* const* y, int count, int64_t m, int64_t k, int xf,
               const btl::RefXf& t, const void* const* ins, int nin, void* stream)
{
    if (count < 1 || count > btl::kMaxGroup) return fail(BTL_ERR_ARG, "count %d not in 1..%d", count, btl::kMaxGroup);
    if (!w || !y) return fail(BTL_ERR_ARG, "null layer array");
    if (m < 0 || m > 65535) return fail(BTL_ERR_SHAPE, "m = %lld: need 0 <= m <= 65535", (long long)m);
    if (k < 64 || k % 64 || k > 16384)
        return fail(BTL_ERR_SHAPE, "k = %lld: need a multiple of 64 in [64, 16384]", (long long)k);
    const uint8_t* wd[btl::kMaxGroup];
    int64_t n[btl::kMaxGroup];
    float sc[btl::kMaxGroup];
    void* yy[btl::kMaxGroup];
    int64_t nsum = 0;
    int rc;
    for (int i = 0; i < count; ++i) {
        if ((rc = check_packed(w[i], m, k))) return rc;
        if (!aligned16(w[i]->data)) return fail(BTL_ERR_LAYOUT, "weights %d must be 16-byte aligned", i);
        if (!y[i] && m > 0 && w[i]->n > 0) return fail(BTL_ERR_LAYOUT, "null output %d", i);
        wd[i] = w[i]->data;
        n[i] = w[i]->n;
        sc[i] = w[i]->scale;
        yy[i] = y[i];
        nsum += w[i]->n;
    }
    if (m == 0 || nsum == 0) return BTL_OK;
    const uintptr_t rows = (uintptr_t)(m * k * 4);
    for (int j = 0; j < nin; ++j) {
        if (!ins[j] && j == 0) return fail(BTL_ERR_LAYOUT, "null input");
        if (ins[j] && !aligned16(ins[j])) return fail(BTL_ERR_LAYOUT, "inputs must be 16-byte aligned");
        for (int i = 0; i < count; ++i) {  // no output row overlaps an input the launch still reads
            const uintptr_t a = (uintptr_t)ins[j], b = (uintptr_t)yy[i], nb = (uintptr_t)(m * n[i] * 4);
            if (a && a < b + nb && b < a + rows) return fail(BTL_ERR_LAYOUT, "output %d overlaps an input", i);
        }
    }
    int dev;
    if ((rc = current_device(&dev))) return rc;
    const hipError_t e = btl::launch_ref_f32_group(nullptr, btl::XK_F32, m, k, wd, n, sc, yy, count, btl::YK_F32,
                                                   (hipStream_t)stream, xf, &t);
    if (e != hipSuccess) return hip_fail(e, "reference-order kernel launch");
    return BTL_OK;
}
}  // namespace

int btl_add_rmsnorm_linear_group_ref(const btl_packed_t* const* w, void* const* y, int count, const float* h,
                                     const float* delta, float* h_out, const float* g, float eps, int64_t m,
                                     int64_t k, void* stream)
{
    if (!h || !g) return fail(BTL_ERR_LAYOUT, "null residual or norm weight");
    if (!aligned16(g) || (h_out && !aligned16(h_out))) return fail(BTL_ERR_LAYOUT, "g and h_out must be 16-byte aligned");
    if (h_out) {  // the launch's other workgroups still read h and delta while h_out is written
        const uintptr_t o = (uintptr_t)h_out, nb = (uintptr_t)(m * k * 4);
        const uintptr_t ins[3] = {(uintptr_t)h, (uintptr_t)delta, (uintptr_t)g};
        const uintptr_t len[3] = {nb, nb, (uintptr_t)(k * 4)};
        for (int j = 0; j < 3; ++j)
            if (ins[j] && ins[j] < o + nb && o < ins[j] + len[j])
                return fail(BTL_ERR_LAYOUT, "h_out overlaps h, delta or g");
        for (int i = 0; i < count && y; ++i) {
            const uintptr_t b = (uintptr_t)y[i];
            if (b && w && w[i] && b < o + nb && o < b + (uintptr_t)(m * w[i]->n * 4))
                return fail(BTL_ERR_LAYOUT, "h_out overlaps output %d", i);
        }
    }
    const btl::RefXf t{h, delta, h_out, g, eps};
    const void* ins[4] = {h, delta, h_out, nullptr};
    return run_ref_xf(w, y, count, m, k, 1, t, ins, 3, stream);
}

int btl_linear_residual(const btl_packed_t* w, const void* x, int xdtype, int64_t m, int64_t k, const float* resid,
                        float* y, void* ws, size_t ws_bytes, void* stream)
{
    int rc;
    if ((rc = check_dtype(xdtype, "input")) || (rc = check_packed(w, m, k))) return rc;
    const int64_t n = w->n;
    if (m == 0 || n == 0) return BTL_OK;
    if (k > 0 && (!x || !resid || !y)) return fail(BTL_ERR_LAYOUT, "null input, residual or output");
    if (k == 0) return fail(BTL_ERR_SHAPE, "in_features must be positive");
    {
        const uintptr_t a0 = (uintptr_t)resid, a1 = (uintptr_t)y, nb = (uintptr_t)(m * n * 4);
        if (a0 < a1 + nb && a1 < a0 + nb) return fail(BTL_ERR_LAYOUT, "y overlaps resid");
        const uintptr_t ax = (uintptr_t)x, xb = (uintptr_t)(m * k * (xdtype == BTL_BF16 ? 2 : 4));
        if (ax < a1 + nb && a1 < ax + xb) return fail(BTL_ERR_LAYOUT, "y overlaps the input");
    }
    Layer l{w, y, nullptr};
    return run_i8(&l, 1, x, xdtype == BTL_BF16 ? btl::XK_BF16 : btl::XK_F32, nullptr, m, k, btl::YK_F32, ws, ws_bytes,
                  (hipStream_t)stream, nullptr, nullptr, resid);
}

int btl_add_rmsnorm_swiglu(const btl_packed_t* w_gate, const btl_packed_t* w_up, const float* h,
                           const float* delta, float* h_out, const float* g, float eps, int64_t m, int64_t k,
                           float* out, void* ws, size_t ws_bytes, void* stream)
{
    const btl_packed_t* w[2] = {w_gate, w_up};
    void* ydummy[2] = {out, out};
    Layer ls[2];
    int rc;
    if ((rc = check_group(w, ydummy, 2, m, k, BTL_F32, ls))) return rc;
    if (w_gate->n != w_up->n)
        return fail(BTL_ERR_SHAPE, "gate and up have %lld and %lld rows", (long long)w_gate->n, (long long)w_up->n);
    if ((rc = check_fused_shape(k, 65536, "fused residual + RMSNorm"))) return rc;
    const int64_t n = w_gate->n;
    if (m == 0 || n == 0) return BTL_OK;
    if (!h || !g || !out) return fail(BTL_ERR_LAYOUT, "null residual, norm weight or output");
    if (!aligned16(h) || !aligned16(g) || (delta && !aligned16(delta)) || (delta && h_out && !aligned16(h_out)))
        return fail(BTL_ERR_LAYOUT, "h, delta, h_out and g must be 16-byte aligned");
    if (delta && h_out && h_out != h) {
        const uintptr_t a0 = (uintptr_t)h, a1 = (uintptr_t)h_out, nb = (uintptr_t)(m * k * 4);
        if (a0 < a1 + nb && a1 < a0 + nb) return fail(BTL_ERR_LAYOUT, "h_out overlaps h without being h");
    }
    if (m > INT32_MAX / 2 || n * m > ((int64_t)1 << 40)) return fail(BTL_ERR_SHAPE, "dimension too large");
    const Xform xf{delta ? btl::XF_ADD_RMSNORM : btl::XF_RMSNORM, delta, g, eps, delta ? h_out : nullptr};
    int rbw = 1;
    const bool dec = env_int(btl::KN_GEMV_DEC) != 0 && dec_waves(m, k, &rbw) > 0 && dec_waves(m, k, &rbw) <= 8;
    const hipStream_t st = (hipStream_t)stream;
    if (dec) {
        // the decode kernel writes silu(gate) * up from its epilogue
        ls[0].y = nullptr;
        ls[1].y = nullptr;
        return run_i8(ls, 2, h, btl::XK_F32, nullptr, m, k, btl::YK_F32, ws, ws_bytes, st, &xf, out);
    }
    // many rows: gate and up into workspace scratch, then the elementwise SwiGLU
    int dev;
    if ((rc = current_device(&dev))) return rc;
    const size_t inner = btl_workspace_bytes(m, 2 * n, k, BTL_ACT_I8);
    const size_t ybytes = align_up((size_t)(m * n * 4), 256);
    void* wsp = nullptr;
    if ((rc = get_ws(dev, ws, ws_bytes, inner + 2 * ybytes, &wsp, st))) return rc;
    float* yg = (float*)((uint8_t*)wsp + inner);
    float* yu = (float*)((uint8_t*)wsp + inner + ybytes);
    ls[0].y = yg;
    ls[1].y = yu;
    if ((rc = run_i8(ls, 2, h, btl::XK_F32, nullptr, m, k, btl::YK_F32, wsp, inner, st, &xf))) return rc;
    hipError_t e = btl::launch_swiglu_f32(yg, yu, m * n, out, st);
    if (e != hipSuccess) return hip_fail(e, "swiglu kernel launch");
    return BTL_OK;
}

size_t btl_add_rmsnorm_swiglu_workspace_bytes(int64_t m, int64_t n, int64_t k)
{
    if (m < 0 || n < 0 || k < 0) return 0;
    return btl_workspace_bytes(m, 2 * n, k, BTL_ACT_I8) + 2 * align_up((size_t)(m * n * 4), 256);
}

int btl_adaptive_split(const uint8_t* packed, int64_t n, int64_t k, int nb, uint8_t* const* out, void* stream)
{
    if (nb < 1 || nb > btl::kMaxBases) return fail(BTL_ERR_ARG, "number of bases %d not in 1..%d", nb, btl::kMaxBases);
    if (n < 0 || k < 0) return fail(BTL_ERR_SHAPE, "negative size");
    if (k % 4 != 0) return fail(BTL_ERR_SHAPE, "in_features %lld is not a multiple of 4", (long long)k);
    if (n * (k / 4) == 0) return BTL_OK;
    if (!packed || !out) return fail(BTL_ERR_LAYOUT, "null pointer");
    btl::AdaptiveOut o;
    memset(&o, 0, sizeof(o));
    for (int b = 0; b < nb; ++b) {
        if (!out[b] || ((uintptr_t)out[b] & 3u)) return fail(BTL_ERR_LAYOUT, "base %d output null or not 4-byte aligned", b);
        o.p[b] = out[b];
    }
    int dev, rc;
    if ((rc = current_device(&dev))) return rc;
    hipError_t e = btl::launch_adaptive_split(packed, n, k, nb, o, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "adaptive split kernel launch");
    return BTL_OK;
}

int btl_adaptive_reconstruct(const uint8_t* packed, const float* scales, int nb, int64_t n, int64_t k, float* out,
                             void* stream)
{
    if (nb < 1 || nb > btl::kMaxBases) return fail(BTL_ERR_ARG, "number of bases %d not in 1..%d", nb, btl::kMaxBases);
    if (n < 0 || k < 0) return fail(BTL_ERR_SHAPE, "negative size");
    if (k % 4 != 0) return fail(BTL_ERR_SHAPE, "in_features %lld is not a multiple of 4", (long long)k);
    if (n * k == 0) return BTL_OK;
    if (!packed || !scales || !out) return fail(BTL_ERR_LAYOUT, "null pointer");
    if (!aligned16(out)) return fail(BTL_ERR_LAYOUT, "out must be 16-byte aligned");
    btl::AdaptiveScales sc;
    memset(&sc, 0, sizeof(sc));
    for (int b = 0; b < nb; ++b) sc.s[b] = scales[b];
    int dev, rc;
    if ((rc = current_device(&dev))) return rc;
    hipError_t e = btl::launch_adaptive_reconstruct(packed, n, k, nb, sc, out, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "adaptive reconstruct kernel launch");
    return BTL_OK;
}

size_t btl_adaptive_workspace_bytes(int64_t m, int64_t n, int64_t k, int nb)
{
    if (m < 0 || n < 0 || k < 0 || nb < 1 || nb > btl::kMaxBases) return 0;
    const int chunk = nb < btl::kMaxGroup ? nb : btl::kMaxGroup;
    return btl_workspace_bytes(m, chunk * n, k, BTL_ACT_I8) + (size_t)nb * align_up((size_t)(m * n * 4), 256);
}

int btl_adaptive_linear(const btl_packed_t* const* bases, int nb, const void* x, int xdtype, int64_t m, int64_t k,
                        void* y, int ydtype, void* ws, size_t ws_bytes, void* stream)
{
    if (nb < 1 || nb > btl::kMaxBases) return fail(BTL_ERR_ARG, "number of bases %d not in 1..%d", nb, btl::kMaxBases);
    if (!bases) return fail(BTL_ERR_ARG, "null base array");
    int rc;
    if ((rc = check_dtype(xdtype, "input")) || (rc = check_dtype(ydtype, "output"))) return rc;
    for (int b = 0; b < nb; ++b) {
        if ((rc = check_packed(bases[b], m, k))) return rc;
        if (bases[b]->n != bases[0]->n)
            return fail(BTL_ERR_SHAPE, "base %d has %lld rows, base 0 %lld", b, (long long)bases[b]->n,
                        (long long)bases[0]->n);
    }
    const int64_t n = bases[0]->n;
    if (m == 0 || n == 0) return BTL_OK;
    if (!x || !y) return fail(BTL_ERR_LAYOUT, "null input or output");
    int dev;
    if ((rc = current_device(&dev))) return rc;
    const int chunk = nb < btl::kMaxGroup ? nb : btl::kMaxGroup;
    const size_t inner = btl_workspace_bytes(m, chunk * n, k, BTL_ACT_I8);
    const size_t ybytes = align_up((size_t)(m * n * 4), 256);
    void* wsp = nullptr;
    const hipStream_t st = (hipStream_t)stream;
    if ((rc = get_ws(dev, ws, ws_bytes, inner + (size_t)nb * ybytes, &wsp, st))) return rc;
    btl::AdaptiveSum sum;
    memset(&sum, 0, sizeof(sum));
    // every base's f32 output y_b = (float)acc_b * (s_x * s_b), up to kMaxGroup bases per launch
    for (int b0 = 0; b0 < nb; b0 += btl::kMaxGroup) {
        const int cnt = nb - b0 < btl::kMaxGroup ? nb - b0 : btl::kMaxGroup;
        Layer ls[btl::kMaxGroup];
        for (int i = 0; i < cnt; ++i) {
            float* yb = (float*)((uint8_t*)wsp + inner + (size_t)(b0 + i) * ybytes);
            ls[i] = Layer{bases[b0 + i], yb, nullptr};
            sum.ys[b0 + i] = yb;
        }
        if ((rc = run_i8(ls, cnt, x, xdtype == BTL_BF16 ? btl::XK_BF16 : btl::XK_F32, nullptr, m, k, btl::YK_F32, wsp,
                         inner, st)))
            return rc;
    }
    // y = y_0 + y_1 + ... in base order
    sum.nb = nb;
    sum.count = m * n;
    sum.y = y;
    sum.ykind = ydtype == BTL_BF16 ? btl::YK_BF16 : btl::YK_F32;
    hipError_t e = btl::launch_base_sum(sum, st);
    if (e != hipSuccess) return hip_fail(e, "base sum kernel launch");
    return BTL_OK;
}

int btl_swiglu_linear_group(const btl_packed_t* const* w, void* const* y, int count, const void* gate,
                            const void* up, int xdtype, int64_t m, int64_t k, int ydtype, void* ws,
                            size_t ws_bytes, void* stream)
{
    Layer ls[btl::kMaxGroup];
    int rc;
    if ((rc = check_dtype(xdtype, "input")) || (rc = check_group(w, y, count, m, k, ydtype, ls))) return rc;
    if ((rc = check_fused_shape(k, 32768, "fused SwiGLU"))) return rc;
    if (m == 0) return BTL_OK;
    if (!gate || !up) return fail(BTL_ERR_LAYOUT, "null gate or up input");
    if (!aligned16(gate) || !aligned16(up)) return fail(BTL_ERR_LAYOUT, "gate and up must be 16-byte aligned");
    const Xform xf{btl::XF_SWIGLU, up, nullptr, 0.0f, nullptr};
    return run_i8(ls, count, gate, xdtype == BTL_BF16 ? btl::XK_BF16 : btl::XK_F32, nullptr, m, k,
                  ydtype == BTL_BF16 ? btl::YK_BF16 : btl::YK_F32, ws, ws_bytes, (hipStream_t)stream, &xf);
}

size_t btl_workspace_bytes(int64_t m, int64_t n, int64_t k, int mode)
{
    if (m < 0 || n < 0 || k < 0) return 0;
    if (mode == BTL_ACT_F32_REF || mode == BTL_ACT_F32_SEQ) return 0;
    // split-K partials of the GEMM / batched-decode routes; a group's layers
    // have at least ceil(n / 128) (ceil(n / 64)) output tiles in total and the
    // splits only fall as tiles are added, so this bounds them
    int splits = btl::gemm_splits(m, ceil_div(n, 128), k, nullptr);
    size_t q_bytes = 0;
    if (m <= 64) {  // any BTL_GEMV_BAT_MAX_M / BTL_GEMV_TR_MAX_M
        const int sb = btl::gemv_bat_plan(m, n, k).splits;
        splits = sb > splits ? sb : splits;
        // the token-register route: its splits depend on k alone, its token
        // layout pads m to 16, 32 or 64 rows and k to 512
        const btl::TrPlan tp = btl::gemv_tr_plan(m, ceil_div(n, 16), k, 0);
        splits = tp.splits > splits ? tp.splits : splits;
        q_bytes = (size_t)btl::tr_bytes(k, tp.mtb);
    }
    return ws_layout(m, k, splits > 1 ? (size_t)splits * m * n * 4 : 0, q_bytes).total;
}

int btl_workspace_clear(void* ws, size_t ws_bytes, void* stream)
{
    if (!ws && ws_bytes) return fail(BTL_ERR_ARG, "null workspace");
    if (((uintptr_t)ws & 255u) != 0) return fail(BTL_ERR_LAYOUT, "workspace must be 256-byte aligned");
    int dev;
    int rc = current_device(&dev);
    if (rc) return rc;
    hipError_t e = btl::launch_fill_zero(ws, ws_bytes, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "fill kernel launch");
    return BTL_OK;
}

}  // extern "C"

// Error reporting, device and workspace helpers for the other C-ABI source
// (btl_model_api.cpp), which shares this file's per-thread message and
// per-device workspace.
namespace btl {
namespace host {
int fail_msg(int code, const char* msg) { return fail(code, "%s", msg); }
int hip_error(hipError_t e, const char* what) { return hip_fail(e, what); }
int device(int* dev) { return current_device(dev); }
int workspace(int dev, void* ws, size_t ws_bytes, size_t need, void** out, hipStream_t st)
{
    return get_ws(dev, ws, ws_bytes, need, out, st);
}
}  // namespace host

int knob(Knob k)
{
    knobs_init();
    return g_knob[k].load(std::memory_order_relaxed);
}
}  // namespace btl
