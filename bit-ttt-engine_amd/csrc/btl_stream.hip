// btl_stream.hip -- the decode stream: the one-token linear chain of a Llama
// block's projections over every layer, in ONE persistent launch.
//
//   x_0 (bf16 [H]) -> for each layer l:
//     stage QKV:  [q | k | v] = W1.58-A8(W_q|W_k|W_v, x_l)     (K = H)
//     stage O:    o = W1.58-A8(W_o, q)                          (K = H = nq)
//     stage GU:   h = silu(W1.58-A8(W_gate, o)) * W1.58-A8(W_up, o)   (K = H)
//     stage D:    x_{l+1} = W1.58-A8(W_down, h)                 (K = I)
//   every stage output rounded to bf16 (the transport type); y = x_L.
//
// It replaces the per-layer calls of BitLinear::forward that a decoder step
// issues in dependency order (layers/bit_linear.rs:52-119 from
// model/block.rs:90-138, attention.rs:159-162, swiglu.rs:29-35) for one token:
// the arithmetic of every stage is btl_linear's W1.58-A8 (bit-identical), the
// launch boundaries between them are replaced by a device-side handoff.
//
// Why one launch: a launch boundary costs ~1.6 us and the next launch cannot
// start reading its weights before it begins; here every workgroup holds the
// packed weights of its rows for one whole layer in registers, issued one
// layer ahead, so HBM streams while stages wait for their inputs.
//
// Geometry: one workgroup per CU (grid = the CUs, every workgroup resident), 16
// waves: 2 control waves and 14 compute waves.  A stage's output rows are cut
// into groups of R rows (R = 4 for k <= 4096, 2 above); workgroup w owns a
// contiguous run of groups of every stage, one group per compute wave:
//   QKV groups -> waves 0..5, O -> waves 0..3, GU (gate and up rows of the same
//   indices) -> waves 0..13, D -> waves 6..13,
// so a wave holds at most 16 loads (64 VGPRs) of packed weights.  Each group
// is computed as in k_gemv_rq (one 16-byte load covers R rows, unpack16 + the
// MFMA trace trick, exact int32), then y = (float)acc * (s_x * s_w).
//
// Handoff (cross-workgroup, agent scope, no grid barrier):
//  - the compute waves leave a stage's outputs in LDS (they issue no global
//    memory operation but their weight loads, so the compiler's in-order wait
//    counts stay exact); control wave 0, once they are done, stores them as
//    tagged 32-bit words (bf16 << 16 | epoch tag) with sc1 stores, no wait for
//    their completion, and publishes a 64-bit flag (launch sequence number |
//    absmax of the workgroup's outputs that the next stage reads: q only, of
//    q|k|v) in 8 replicas (one per XCD, fewer pollers per line);
//  - the control waves of every workgroup poll their replica (2 KB), take the
//    global absmax from the flags (so the quantisation needs no pass of its
//    own), copy the tagged input into LDS (buffer_load ... lds, sc1), re-read
//    any word whose tag is still stale, and quantise it into the operand-order
//    int8 row (double-buffered by stage parity);
//  - compute waves wait for that row on an LDS counter (their own weight
//    loads stay in flight: vector memory counters are in order, so they issue
//    no other global loads).
// Every wait is bounded by a time budget (s_memrealtime); a wait that gives
// up sets kFaultStream and the workgroup skips every later wait, so the
// launch always finishes (its outputs are then not valid).
//
// The epoch (tags and sequence numbers) lives on the device: every workgroup
// reads it at start; workgroup 0 increments it when it is done (every other
// workgroup has read it by then: each stage needs all workgroups' outputs).
#include <hip/hip_runtime.h>

#include "btl_device.hpp"
#include "btl_internal.hpp"

namespace btl {

__device__ uint32_t g_stream_faults;

namespace {

constexpr int kSReplicas = 8;
constexpr int kSCtl = 2;       // control waves
constexpr int kSComp = 14;     // compute waves
constexpr int kSQkvWaves = 6;  // compute waves 0..5 may own a QKV group
constexpr int kSOWaves = 4;    // 0..3 an O group
constexpr int kSDWave0 = 6;    // 6..13 a D group

struct GroupPos {
    int g0, ng;  // first group of this workgroup, groups it owns
};

// contiguous split of G groups over nwg workgroups
__device__ __forceinline__ GroupPos group_pos(int G, int nwg, int w)
{
    // G * (w + 1) < 2^31 (checked by the host), so 32-bit unsigned division
    const uint32_t g0 = (uint32_t)G * (uint32_t)w / (uint32_t)nwg;
    const uint32_t g1 = (uint32_t)G * (uint32_t)(w + 1) / (uint32_t)nwg;
    return GroupPos{(int)g0, (int)(g1 - g0)};
}

__device__ __forceinline__ uint64_t now_ticks() { return __builtin_amdgcn_s_memrealtime(); }

struct Clock {
    uint64_t deadline;
    bool abort;
    __device__ __forceinline__ bool expired()
    {
        if (abort) return true;
        if (now_ticks() > deadline) abort = true;  // reported once, when the wave ends
        return abort;
    }
};

// wait until the LDS counter reaches target (or the budget runs out)
__device__ __forceinline__ void lds_wait(const uint32_t* c, uint32_t target, Clock& clk)
{
    while (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
        if (clk.expired()) break;
        __builtin_amdgcn_s_sleep(1);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ uint4 ld_sc1(__amdgpu_buffer_rsrc_t r, int off)
{
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16));
}

// stage j of layer l -> its input and output transport offsets (words)
struct StageIO {
    int k;        // input length
    int in_off;   // -1: x0
    int out_off;
    int n_out;    // output words
};

__device__ __forceinline__ StageIO stage_io(const StreamArgs& a, int l, int j)
{
    const int nqkv = a.nq + a.nk + a.nv;
    const int per = nqkv + a.H + a.I + a.H;
    const int base = l * per;
    StageIO io;
    switch (j) {
    case 0:
        io.k = a.H;
        io.in_off = l == 0 ? -1 : base - a.H;
        io.out_off = base;
        io.n_out = nqkv;
        break;
    case 1:
        io.k = a.nq;
        io.in_off = base;
        io.out_off = base + nqkv;
        io.n_out = a.H;
        break;
    case 2:
        io.k = a.H;
        io.in_off = base + nqkv;
        io.out_off = base + nqkv + a.H;
        io.n_out = a.I;
        break;
    default:
        io.k = a.I;
        io.in_off = base + nqkv + a.H;
        io.out_off = base + nqkv + a.H + a.I;
        io.n_out = a.H;
        break;
    }
    return io;
}

// groups of stage j (R rows each; GU: pairs of R gate + R up rows)
__device__ __forceinline__ int stage_groups(const StreamArgs& a, int j, int rd)
{
    if (j == 0) return (a.nq + a.nk + a.nv) / 4;
    if (j == 1) return a.H / 4;
    if (j == 2) return a.I / 4;
    return a.H / rd;
}

// ---------------------------------------------------------------------------
// compute waves
// ---------------------------------------------------------------------------
// One group: its weight rows (rsrc), row count, output rows, scale.
struct GroupW {
    __amdgpu_buffer_rsrc_t rs;
    int rows;
    int n0;     // first output row (index into the stage's output)
    float sw;
};

template <int R>
__device__ __forceinline__ GroupW group_w(const uint8_t* w, int layer_row0, int rows_layer, int out_row0, int K,
                                          float sw)
{
    GroupW g;
    const int rowb = K >> 2;
    g.rows = __builtin_amdgcn_readfirstlane(max(0, min(R, rows_layer - layer_row0)));
    g.rs = make_rsrc(w + (int64_t)max(layer_row0, 0) * rowb, (uint32_t)(g.rows * rowb));
    g.n0 = out_row0;
    g.sw = sw;
    return g;
}

template <int R, int ST>
__device__ __forceinline__ void issue_loads(uint4* buf, const GroupW& g, int K, int lane)
{
    constexpr int SUB = 16 / R, RB = 1024 / R;
    const int rowb = K >> 2;
    const int gq = lane >> 4, il = lane & 15;
    const int rho = il / SUB, sl = SUB * gq + (il - rho * SUB);
#pragma unroll
    for (int t = 0; t < ST; ++t) {
        const int b = t * RB + 16 * sl;
        buf[t] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                               g.rs, b < rowb && g.rows > 0 ? rho * rowb + b : kOOB, 0, kCachePolicyNT));
    }
}

// exact int32 dot products of the group's rows with the operand row sq; the
// lane with `own` set holds row `r`'s sum
template <int R, int ST>
__device__ __forceinline__ int group_dot(const uint4* buf, const uint8_t* sq, int K, int lane)
{
    constexpr int SUB = 16 / R, RB = 1024 / R;
    const int gq = lane >> 4, il = lane & 15;
    const int rho = il / SUB, sl = SUB * gq + (il - rho * SUB);
    (void)rho;
    v4i acc = v4i{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < ST; ++t) {
        const int ko = 4 * (t * RB + 16 * sl);
        const uint4 cur = buf[t];
        const uint32_t wv[4] = {cur.x, cur.y, cur.z, cur.w};
        const uint8_t* bj = sq + (ko < K ? ko : 0);
#pragma unroll
        for (int h = 0; h < 4; ++h)
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack16(wv[h]), *(const v4i*)(bj + 16 * h), acc, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);  // one load's unpack at a time (register pressure)
    }
    int d = acc[0] + __builtin_amdgcn_update_dpp(0, acc[1], 0x55, 0xF, 0xF, true);
    d += __builtin_amdgcn_update_dpp(0, acc[2], 0xAA, 0xF, 0xF, true);
    d += __builtin_amdgcn_update_dpp(0, acc[3], 0xFF, 0xF, 0xF, true);
    if (R == 2) d += __shfl_down(d, 20, 64);
    return d;
}

// gate and up of the same rows against one operand row: one B read per word
// feeds both products
__device__ __forceinline__ void group_dot_pair(const uint4* bg, const uint4* bu, const uint8_t* sq, int K, int lane,
                                               int* dg, int* du)
{
    constexpr int R = 4, SUB = 4, RB = 256;
    const int gq = lane >> 4, il = lane & 15;
    const int rho = il / SUB, sl = SUB * gq + (il - rho * SUB);
    v4i ag = v4i{0, 0, 0, 0}, au = v4i{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int ko = 4 * (t * RB + 16 * sl);
        const uint32_t wg[4] = {bg[t].x, bg[t].y, bg[t].z, bg[t].w};
        const uint32_t wu[4] = {bu[t].x, bu[t].y, bu[t].z, bu[t].w};
        const uint8_t* bj = sq + (ko < K ? ko : 0);
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const v4i b = *(const v4i*)(bj + 16 * h);
            ag = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack16(wg[h]), b, ag, 0, 0, 0);
            au = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack16(wu[h]), b, au, 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    (void)R;
    int g = ag[0] + __builtin_amdgcn_update_dpp(0, ag[1], 0x55, 0xF, 0xF, true);
    g += __builtin_amdgcn_update_dpp(0, ag[2], 0xAA, 0xF, 0xF, true);
    g += __builtin_amdgcn_update_dpp(0, ag[3], 0xFF, 0xF, 0xF, true);
    int u = au[0] + __builtin_amdgcn_update_dpp(0, au[1], 0x55, 0xF, 0xF, true);
    u += __builtin_amdgcn_update_dpp(0, au[2], 0xAA, 0xF, 0xF, true);
    u += __builtin_amdgcn_update_dpp(0, au[3], 0xFF, 0xF, 0xF, true);
    *dg = g;
    *du = u;
}

template <int R>
__device__ __forceinline__ int own_row(int lane, bool* own)
{
    const int r = R == 4 ? lane / 20 : lane / 40;
    *own = lane - (R == 4 ? 20 : 40) * r == 0;
    return r;
}

constexpr int kSOut = 64;  // outputs of one stage a workgroup computes at most (gate|up: 14 x 4)

struct Shared {
    uint32_t ready;            // operand rows posted (each control wave adds 1 per stage)
    uint32_t cdone;            // compute-wave arrivals (one per participating wave per stage)
    float scale[2];            // s_x of the operand row (by stage parity)
    float out[kSOut];          // this workgroup's outputs of the current stage (f32, before rounding)
    uint32_t ctl_amax[kSCtl];  // first stage: the control waves' absmax of x0
    uint32_t ctl_arrive;
    uint32_t ctl_copy;         // control waves whose input copies are in LDS (one per wave per stage)
};

__device__ __forceinline__ uint32_t tag_of(uint32_t epoch) { return epoch & 0xFFFFu; }

// A compute wave's group in one slot: which layer matrix (w index), the first
// row in that matrix, rows (0: none) and K.  Layer-independent.
struct Slot {
    int wi;
    int lrow0;
    int rows;
    int K;
};

// The layer table through the constant address space: read with scalar loads
// (lgkmcnt).  A vector load of it (the compiler's choice for a plain pointer,
// since the kernel also stores to global memory) would count in vmcnt, and
// waiting for it would wait for every weight load issued before it.
typedef const __attribute__((address_space(4))) StreamLayer* LayerTab;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t slot_rsrc(LayerTab layers, int l, const Slot& sl)
{
    // every field wave-uniform (readfirstlane): a descriptor in VGPRs turns each
    // load into a waterfall loop
    const int rowb = sl.K >> 2;
    const uint64_t base = (uint64_t)(layers[l].w[sl.wi] + (int64_t)sl.lrow0 * rowb);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)base);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(base >> 32));
    const uint32_t nb = (uint32_t)__builtin_amdgcn_readfirstlane(sl.rows * rowb);
    return make_rsrc((const void*)(((uint64_t)hi << 32) | lo), nb);
}

// The slot's loads for layer l, issued whether or not the wave owns a group
// (rows == 0: every offset is out of range, nothing is read): the compute
// waves issue no other vector memory instructions, so the order of their
// loads is the same on every path and the compiler's in-order wait counts
// (s_waitcnt vmcnt(N) before each use) stay exact across the layer loop.
template <int R, int ST>
__device__ __forceinline__ void slot_issue(uint4* buf, LayerTab layers, int l, const Slot& sl, int lane)
{
    GroupW g;
    g.rs = slot_rsrc(layers, l, sl);
    g.rows = sl.rows;
    issue_loads<R, ST>(buf, g, sl.K, lane);
    __builtin_amdgcn_sched_barrier(0);  // the slots' loads stay in the order they are issued
}

// a compute wave's end of stage s: its outputs are in sh.out; count it
__device__ __forceinline__ void compute_arrive(Shared& sh, int lane)
{
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the outputs are in LDS
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (lane == 0) __hip_atomic_fetch_add(&sh.cdone, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Compute wave c.  ROLE: 0 = QKV + O + GU (c 0..3), 1 = QKV + GU (c 4..5),
// 2 = D + GU (c 6..13).  Local output index of group g in a stage: g * R + r.
template <int ROLE, int RD, int STD>
__device__ void compute_wave(const StreamArgs& a, Shared& sh, const uint8_t* rows_lds, int c, int lane, Clock& clk)
{
    constexpr bool HQ = ROLE <= 1, HO = ROLE == 0, HD = ROLE == 2;
    const int w = blockIdx.x;
    const int kmax_row = a.kmax + 16;
    const int H = a.H, I = a.I, nqkv = a.nq + a.nk + a.nv;
    const GroupPos pq = group_pos(nqkv / 4, a.nwg, w);
    const GroupPos po = group_pos(H / 4, a.nwg, w);
    const GroupPos pg = group_pos(I / 4, a.nwg, w);
    const GroupPos pd = group_pos(H / RD, a.nwg, w);

    Slot sq_, so_, sg_, sd_;
    sq_.wi = 0; sq_.lrow0 = 0; sq_.rows = 0; sq_.K = H;
    so_.wi = 3; so_.lrow0 = 0; so_.rows = 0; so_.K = a.nq;
    sg_.wi = 4; sg_.lrow0 = 0; sg_.rows = 0; sg_.K = H;
    sd_.wi = 6; sd_.lrow0 = 0; sd_.rows = 0; sd_.K = I;
    if (HQ && c < pq.ng) {
        const int r0 = (pq.g0 + c) * 4;  // row in [q | k | v]
        const int li = r0 < a.nq ? 0 : (r0 < a.nq + a.nk ? 1 : 2);
        sq_.wi = li;
        sq_.lrow0 = li == 0 ? r0 : (li == 1 ? r0 - a.nq : r0 - a.nq - a.nk);
        sq_.rows = min(4, (li == 0 ? a.nq : (li == 1 ? a.nk : a.nv)) - sq_.lrow0);
    }
    if (HO && c < po.ng) {
        so_.lrow0 = (po.g0 + c) * 4;
        so_.rows = min(4, H - so_.lrow0);
    }
    if (c < pg.ng) {
        sg_.lrow0 = (pg.g0 + c) * 4;
        sg_.rows = min(4, I - sg_.lrow0);
    }
    if (HD && c - kSDWave0 < pd.ng) {
        sd_.lrow0 = (pd.g0 + c - kSDWave0) * RD;
        sd_.rows = min(RD, H - sd_.lrow0);
    }
    Slot su_ = sg_;
    su_.wi = 5;

    uint4 bq[HQ ? 4 : 1], bo[HO ? 4 : 1], bg[8], bd[HD ? STD : 1];
    const LayerTab layers = (LayerTab)a.layers;
    // layer 0, in the slot order the loop re-issues them
    if (HQ) slot_issue<4, 4>(bq, layers, 0, sq_, lane);
    if (HO) slot_issue<4, 4>(bo, layers, 0, so_, lane);
    slot_issue<4, 4>(bg, layers, 0, sg_, lane);
    slot_issue<4, 4>(bg + 4, layers, 0, su_, lane);
    if (HD) slot_issue<RD, STD>(bd, layers, 0, sd_, lane);

    bool own4, own_d;
    const int r4 = own_row<4>(lane, &own4);
    const int rdd = own_row<RD>(lane, &own_d);

    for (int l = 0; l < a.nl; ++l) {
        const int ln = l + 1 < a.nl ? l + 1 : l;  // the last layer re-reads its own weights (never used)
        if (HQ) {
            const int s = 4 * l;
            if (sq_.rows) {
                lds_wait(&sh.ready, 2u * (uint32_t)(s + 1), clk);
                const int d = group_dot<4, 4>(bq, rows_lds + (s & 1) * kmax_row, H, lane);
                if (own4 && r4 < sq_.rows)
                    sh.out[c * 4 + r4] = __fmul_rn((float)d, __fmul_rn(sh.scale[s & 1], layers[l].sw[sq_.wi]));
                compute_arrive(sh, lane);
            }
            slot_issue<4, 4>(bq, layers, ln, sq_, lane);
        }
        if (HO) {
            const int s = 4 * l + 1;
            if (so_.rows) {
                lds_wait(&sh.ready, 2u * (uint32_t)(s + 1), clk);
                const int d = group_dot<4, 4>(bo, rows_lds + (s & 1) * kmax_row, a.nq, lane);
                if (own4 && r4 < so_.rows)
                    sh.out[c * 4 + r4] = __fmul_rn((float)d, __fmul_rn(sh.scale[s & 1], layers[l].sw[3]));
                compute_arrive(sh, lane);
            }
            slot_issue<4, 4>(bo, layers, ln, so_, lane);
        }
        {
            const int s = 4 * l + 2;
            if (sg_.rows) {
                lds_wait(&sh.ready, 2u * (uint32_t)(s + 1), clk);
                int dg, du;
                group_dot_pair(bg, bg + 4, rows_lds + (s & 1) * kmax_row, H, lane, &dg, &du);
                if (own4 && r4 < sg_.rows) {
                    const float sx = sh.scale[s & 1];
                    const float yg = __fmul_rn((float)dg, __fmul_rn(sx, layers[l].sw[4]));
                    const float yu = __fmul_rn((float)du, __fmul_rn(sx, layers[l].sw[5]));
                    sh.out[c * 4 + r4] = __fmul_rn(__fdiv_rn(yg, __fadd_rn(1.0f, btl_expf(-yg))), yu);
                }
                compute_arrive(sh, lane);
            }
            slot_issue<4, 4>(bg, layers, ln, sg_, lane);
            slot_issue<4, 4>(bg + 4, layers, ln, su_, lane);
        }
        if (HD) {
            const int s = 4 * l + 3;
            if (sd_.rows) {
                lds_wait(&sh.ready, 2u * (uint32_t)(s + 1), clk);
                const int d = group_dot<RD, STD>(bd, rows_lds + (s & 1) * kmax_row, I, lane);
                if (own_d && rdd < sd_.rows)
                    sh.out[(c - kSDWave0) * RD + rdd] =
                        __fmul_rn((float)d, __fmul_rn(sh.scale[s & 1], layers[l].sw[6]));
                compute_arrive(sh, lane);
            }
            slot_issue<RD, STD>(bd, layers, ln, sd_, lane);
        }
    }
}

// ---------------------------------------------------------------------------
// control waves
// ---------------------------------------------------------------------------
// Quantise 16 values (f32) into one operand-order group of the row.
__device__ __forceinline__ void quant_group_to(uint8_t* sq, int g, const float* f, const QParams& qp)
{
    *(uint4*)(sq + 16 * g) = qp.ok ? group_quant_f(f, qp.r) : uint4{0u, 0u, 0u, 0u};
}

// Control wave 0 after the compute waves of stage s are done: the workgroup's
// outputs (n local rows from output row o0) as tagged bf16 words, plain copies
// where asked, then the flag replicas with the absmax of the rows the next
// stage reads (rows below amax_rows of the stage's output).
__device__ __forceinline__ void publish(const StreamArgs& a, Shared& sh, int out_off, int o0, int n, int amax_rows,
                                        bool last, uint32_t epoch, uint32_t seq, int lane)
{
    uint32_t am = 0;
    if (lane < n) {
        const uint16_t b = f32_to_bf16(sh.out[lane]);
        const int row = o0 + lane;
        __hip_atomic_store(a.tbuf + out_off + row, ((uint32_t)b << 16) | tag_of(epoch), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        if (a.dbg) a.dbg[out_off + row] = b;
        if (last) a.y[row] = b;
        if (row < amax_rows) am = ((uint32_t)b << 16) & 0x7FFFFFFFu;
    }
    am = wave_max_dpp(am);
    if (lane < kSReplicas)
        __hip_atomic_store(a.flags + (size_t)lane * a.nwg + blockIdx.x, ((uint64_t)am << 32) | seq, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

__device__ void control_wave(const StreamArgs& a, Shared& sh, uint8_t* rows_lds, uint8_t* stage_lds, int cw, int lane,
                             uint32_t epoch, Clock& clk, int rd)
{
    const int w = blockIdx.x;
    const int t = cw * 64 + lane;  // control thread
    constexpr int NT = kSCtl * 64;
    const uint32_t tag = tag_of(epoch);
    const int kmax_row = a.kmax + 16;
    const int S = 4 * a.nl;
    const int rep = w % kSReplicas;
    const int nqkv = a.nq + a.nk + a.nv;
    // this workgroup's groups per slot, their first output rows and counts
    // (selected by value, not indexed: a runtime index into a private array
    // would put it in scratch memory)
    const GroupPos gp0 = group_pos(nqkv / 4, a.nwg, w), gp1 = group_pos(a.H / 4, a.nwg, w),
                   gp2 = group_pos(a.I / 4, a.nwg, w), gp3 = group_pos(a.H / rd, a.nwg, w);
    uint32_t cum = 0;  // compute-wave arrivals expected through the current stage
    const __amdgpu_buffer_rsrc_t fr = make_rsrc(a.flags + (size_t)rep * a.nwg, (uint32_t)(a.nwg * 8));
    for (int s = 0; s < S; ++s) {
        const int l = s >> 2, j = s & 3;
        const StageIO io = stage_io(a, l, j);
        const int K = io.k, G = K >> 4;
        uint8_t* sq = rows_lds + (s & 1) * kmax_row;
        QParams qp;
        if (io.in_off < 0) {
            // the plain bf16 input: absmax over both control waves, then quantise
            const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x0, (uint32_t)(K * 2));
            uint32_t am = 0;
            for (int g = t; g < G; g += NT) {
                uint4 v[2] = {bload(xr, 32 * g), bload(xr, 32 * g + 16)};
                am = max(am, group_absmax<XK_BF16>(v));
            }
            am = wave_max_dpp(am);
            if (lane == 0) {
                sh.ctl_amax[cw] = am;
                __builtin_amdgcn_s_waitcnt(0xC07F);
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                __hip_atomic_fetch_add(&sh.ctl_arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
            lds_wait(&sh.ctl_arrive, (uint32_t)kSCtl, clk);
            uint32_t gam = 0;
#pragma unroll
            for (int i = 0; i < kSCtl; ++i) gam = max(gam, sh.ctl_amax[i]);
            qp = qparams(gam);
            for (int g = t; g < G; g += NT) {
                uint4 v[2] = {bload(xr, 32 * g), bload(xr, 32 * g + 16)};
                float f[16];
                widen16<XK_BF16>(v, f);
                quant_group_to(sq, g, f, qp);
            }
        } else {
            // 1. every workgroup's flag for stage s - 1 (seq and its outputs' absmax)
            const uint32_t want = (epoch << 10) + (uint32_t)s;  // stage s-1 done: seq = s
            uint32_t gam = 0;
            for (;;) {
                asm volatile("" ::: "memory");
                const uint4 f0 = ld_sc1(fr, lane * 32), f1 = ld_sc1(fr, lane * 32 + 16);
                const int i0 = 4 * lane;
                // sequence numbers compared modulo 2^32 (stale ones are at most a launch old)
                const bool ok = (i0 >= a.nwg || (int32_t)(f0.x - want) >= 0) &&
                                (i0 + 1 >= a.nwg || (int32_t)(f0.z - want) >= 0) &&
                                (i0 + 2 >= a.nwg || (int32_t)(f1.x - want) >= 0) &&
                                (i0 + 3 >= a.nwg || (int32_t)(f1.z - want) >= 0);
                if (__all(ok)) {
                    uint32_t m = 0;
                    if (i0 < a.nwg) m = max(m, f0.y);
                    if (i0 + 1 < a.nwg) m = max(m, f0.w);
                    if (i0 + 2 < a.nwg) m = max(m, f1.y);
                    if (i0 + 3 < a.nwg) m = max(m, f1.w);
                    gam = wave_max_dpp(m);
                    break;
                }
                if (clk.expired()) break;
            }
            qp = qparams(gam);
            // 2. the tagged input into LDS: this wave's 1 KB copies, then wait for the other's
            const __amdgpu_buffer_rsrc_t ir = make_rsrc(a.tbuf + io.in_off, (uint32_t)(K * 4));
            const int nch = (K * 4 + 1023) >> 10;
            for (int ch = cw; ch < nch; ch += kSCtl)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    ir, (__attribute__((address_space(3))) void*)(stage_lds + ch * 1024), 16, ch * 1024 + 16 * lane, 0,
                    0, 16);
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's copies are in LDS
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            if (lane == 0) __hip_atomic_fetch_add(&sh.ctl_copy, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            lds_wait(&sh.ctl_copy, (uint32_t)(kSCtl * s), clk);  // stages 1..s each counted once per wave
            // 3. quantise groups t, t + 128, ..., re-reading words whose tag is stale
            for (int g = t; g < G; g += NT) {
                uint4 v[4];
#pragma unroll
                for (int h = 0; h < 4; ++h) v[h] = *(const uint4*)(stage_lds + 64 * g + 16 * h);
                const uint32_t* u = (const uint32_t*)v;
                bool ok = true;
#pragma unroll
                for (int e = 0; e < 16; ++e) ok = ok && (u[e] & 0xFFFFu) == tag;
                if (!ok) {
                    const __amdgpu_buffer_rsrc_t gr_ = make_rsrc(a.tbuf + io.in_off + 16 * g, 64u);
                    for (;;) {
                        asm volatile("" ::: "memory");
#pragma unroll
                        for (int h = 0; h < 4; ++h) v[h] = ld_sc1(gr_, 16 * h);
                        ok = true;
#pragma unroll
                        for (int e = 0; e < 16; ++e) ok = ok && (u[e] & 0xFFFFu) == tag;
                        if (ok || clk.expired()) break;
                    }
                }
                float f[16];
#pragma unroll
                for (int e = 0; e < 16; ++e) f[e] = __uint_as_float(u[e] & 0xFFFF0000u);
                quant_group_to(sq, g, f, qp);
            }
        }
        // 4. post the row: s_x for the compute waves, one arrival per control wave
        if (lane == 0) sh.scale[s & 1] = qp.s;
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the row is in LDS
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (lane == 0) __hip_atomic_fetch_add(&sh.ready, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        // 5. wave 0: once this stage's compute waves are done, publish the outputs
        //    (q|k|v: the absmax of q only, the rows o reads)
        const int cap = j == 0 ? kSQkvWaves : (j == 1 ? kSOWaves : (j == 2 ? kSComp : kSComp - kSDWave0));
        const GroupPos gpj = j == 0 ? gp0 : (j == 1 ? gp1 : (j == 2 ? gp2 : gp3));
        const int grj = j == 3 ? rd : 4;
        const int np = min(gpj.ng, cap);
        cum += (uint32_t)np;
        if (cw == 0) {
            lds_wait(&sh.cdone, cum, clk);
            publish(a, sh, io.out_off, gpj.g0 * grj, np * grj < io.n_out - gpj.g0 * grj
                                                         ? np * grj
                                                         : io.n_out - gpj.g0 * grj,
                    j == 0 ? a.nq : io.n_out, j == 3 && l + 1 == a.nl, epoch, (epoch << 10) + (uint32_t)s + 1u, lane);
        }
    }
}

template <int RD, int STD>
__global__ __launch_bounds__(1024, 1) void k_dec_stream(StreamArgs a)
{
    extern __shared__ __align__(16) uint8_t lds[];  // [2][kmax + 16] operand rows, then the staging copy
    __shared__ Shared sh;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (tid == 0) {
        sh.ready = 0u;
        sh.cdone = 0u;
        sh.ctl_arrive = 0u;
        sh.ctl_copy = 0u;
    }
    const uint32_t epoch =
        (uint32_t)__builtin_amdgcn_readfirstlane((int)__hip_atomic_load(a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    __syncthreads();
    Clock clk{now_ticks() + (uint64_t)a.budget_ticks, false};
    uint8_t* rows_lds = lds;
    uint8_t* stage_lds = lds + 2 * (a.kmax + 16);
    if (wave < kSCtl) {
        control_wave(a, sh, rows_lds, stage_lds, wave, lane, epoch, clk, RD);
        // workgroup 0 ends the launch's epoch after its last stage (every
        // workgroup read the epoch before producing the outputs it consumed)
        if (blockIdx.x == 0 && wave == 0 && lane == 0)
            __hip_atomic_store(a.epoch, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        const int c = wave - kSCtl;
        if (c < kSOWaves) compute_wave<0, RD, STD>(a, sh, rows_lds, c, lane, clk);
        else if (c < kSQkvWaves) compute_wave<1, RD, STD>(a, sh, rows_lds, c, lane, clk);
        else compute_wave<2, RD, STD>(a, sh, rows_lds, c, lane, clk);
    }
    if (clk.abort && lane == 0)
        __hip_atomic_fetch_or(&g_stream_faults, kFaultStream, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

// two operand rows, then the staging copy of a tagged input (whole 1 KB copies)
size_t stream_lds_bytes(int kmax) { return (size_t)2 * (kmax + 16) + (((size_t)kmax * 4 + 1023) & ~(size_t)1023); }

// The stages of the stream wait on each other's workgroups, so every workgroup
// must be resident at once.  The occupancy of the instantiation is checked
// first (a grid that cannot be co-resident fails with
// hipErrorCooperativeLaunchTooLarge before anything runs); outside a stream
// capture the launch is cooperative, which makes the runtime guarantee that all
// workgroups run together (or fail the launch).  Under a capture it is a plain
// launch resting on the occupancy check, and a workgroup kept off the device by
// other work makes the bounded waits give up and set the fault word
// (btl_check_faults) instead of hanging.
hipError_t launch_dec_stream(const StreamArgs& a, hipStream_t s)
{
    const size_t lds = stream_lds_bytes(a.kmax);
    if (a.I > 14336 || a.H > 4096 || a.nwg > 256) return hipErrorInvalidValue;
    const void* fn = a.I > 4096 ? (const void*)k_dec_stream<2, 7> : (const void*)k_dec_stream<4, 4>;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    int dev = 0, cus = 0, per_cu = 0;
    if ((e = hipGetDevice(&dev)) != hipSuccess ||
        (e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess ||
        (e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 1024, lds)) != hipSuccess)
        return e;
    if ((int64_t)per_cu * cus < a.nwg) return hipErrorCooperativeLaunchTooLarge;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if ((e = hipStreamIsCapturing(s, &cap)) != hipSuccess) return e;
    if (cap == hipStreamCaptureStatusNone) {
        StreamArgs arg = a;
        void* params[] = {(void*)&arg};
        return hipLaunchCooperativeKernel(fn, dim3(a.nwg), dim3(1024), params, (unsigned)lds, s);
    }
    if (a.I > 4096) hipLaunchKernelGGL((k_dec_stream<2, 7>), dim3(a.nwg), dim3(1024), lds, s, a);
    else hipLaunchKernelGGL((k_dec_stream<4, 4>), dim3(a.nwg), dim3(1024), lds, s, a);
    return hipGetLastError();
}

hipError_t stream_faults(uint32_t* bits, hipStream_t st)
{
    hipError_t e = hipMemcpyFromSymbolAsync(bits, HIP_SYMBOL(g_stream_faults), sizeof(uint32_t), 0,
                                            hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess || !*bits) return e;
    static const uint32_t zero = 0;
    e = hipMemcpyToSymbolAsync(HIP_SYMBOL(g_stream_faults), &zero, sizeof(uint32_t), 0, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return e;
}

}  // namespace btl
