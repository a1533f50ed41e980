// btl_stream_api.cpp -- C ABI of the decode stream (include/bitllama.h,
// btl_stream_*): shape checks, the plan's device buffers, launch.
//
// Host-side counterpart of the per-layer loop of a one-token decoder step
// (model/llama.rs:201-271 forward_one -> model/block.rs:90-138 ->
// layers/bit_linear.rs:52-119 for q, k, v, o, w1, w3, w2), with the projections
// of every layer run by one persistent launch (btl_stream.hip).
#include "bitllama.h"

#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstring>
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

constexpr int kReplicas = 8;
constexpr int kCompWaves = 14;
constexpr uint32_t kPlanMagic = 0x5354524Du;  // "STRM"

struct Plan {
    uint32_t magic;
    int dev;
    int nl, H, I, nq, nk, nv, nwg, kmax;
    size_t words;  // tagged transport words
    btl::StreamLayer* d_layers;
    uint32_t* tbuf;
    uint64_t* flags;
    uint32_t* epoch;
};

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

int check_mat(const btl_packed_t& w, int64_t n, int64_t k, const char* name, int li)
{
    if (w.n != n || w.k != k)
        return failf(BTL_ERR_SHAPE, "layer %d %s is [%lld, %lld], the stream needs [%lld, %lld]", li, name,
                     (long long)w.n, (long long)w.k, (long long)n, (long long)k);
    if (!w.data || ((uintptr_t)w.data & 15u)) return failf(BTL_ERR_LAYOUT, "layer %d %s: null or unaligned data", li, name);
    return BTL_OK;
}

void free_plan(Plan* p)
{
    if (!p) return;
    if (p->d_layers) (void)hipFree(p->d_layers);
    if (p->tbuf) (void)hipFree(p->tbuf);
    if (p->flags) (void)hipFree(p->flags);
    if (p->epoch) (void)hipFree(p->epoch);
    p->magic = 0;
    delete p;
}

}  // namespace

extern "C" {

int btl_stream_create(const btl_stream_layer_t* layers, int n_layers, void** plan_out)
{
    if (!plan_out) return fail_msg(BTL_ERR_ARG, "null plan pointer");
    *plan_out = nullptr;
    if (!layers || n_layers < 1 || n_layers > 4096) return fail_msg(BTL_ERR_ARG, "need 1..4096 layers");
    int rc;
    const btl_stream_layer_t& L0 = layers[0];
    const int64_t H = L0.q.k, nq = L0.q.n, nk = L0.k.n, nv = L0.v.n, I = L0.gate.n;
    if (nq != H) return failf(BTL_ERR_SHAPE, "q has %lld rows, hidden is %lld: o reads q directly", (long long)nq, (long long)H);
    if (H < 64 || H % 64 || H > 4096)
        return failf(BTL_ERR_SHAPE, "hidden %lld: the stream needs a multiple of 64 up to 4096", (long long)H);
    if (I < 64 || I % 64 || I > 14336)
        return failf(BTL_ERR_SHAPE, "intermediate %lld: the stream needs a multiple of 64 up to 14336", (long long)I);
    if (nk % 4 || nv % 4 || nk < 4 || nv < 4) return fail_msg(BTL_ERR_SHAPE, "k and v rows must be positive multiples of 4");
    for (int l = 0; l < n_layers; ++l) {
        const btl_stream_layer_t& L = layers[l];
        if ((rc = check_mat(L.q, nq, H, "q", l)) || (rc = check_mat(L.k, nk, H, "k", l)) ||
            (rc = check_mat(L.v, nv, H, "v", l)) || (rc = check_mat(L.o, H, nq, "o", l)) ||
            (rc = check_mat(L.gate, I, H, "gate", l)) || (rc = check_mat(L.up, I, H, "up", l)) ||
            (rc = check_mat(L.down, H, I, "down", l)))
            return rc;
    }
    int dev;
    if ((rc = btl::host::device(&dev))) return rc;
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return hip_error(e, "hipGetDeviceProperties");
    const int nwg = prop.multiProcessorCount;
    if (nwg < 1 || nwg > 256) return failf(BTL_ERR_DEVICE, "the stream polls at most 256 workgroups, device has %d CUs", nwg);
    const int kmax = (int)(H > I ? H : I);
    if (btl::stream_lds_bytes(kmax) + 256 > (size_t)prop.sharedMemPerBlock)
        return failf(BTL_ERR_SHAPE, "the stream needs %zu bytes of LDS, the device gives %zu", btl::stream_lds_bytes(kmax),
                     (size_t)prop.sharedMemPerBlock);
    // one group per compute wave and slot (QKV <= 6, O <= 4, GU <= 14, D <= 8)
    const int rd = I > 4096 ? 2 : 4;
    const int64_t gq = cdiv((nq + nk + nv) / 4, nwg), go = cdiv(H / 4, nwg), gg = cdiv(I / 4, nwg), gd = cdiv(H / rd, nwg);
    if (gq > 6 || go > 4 || gg > kCompWaves || gd > 8)
        return failf(BTL_ERR_SHAPE,
                     "shapes too large for %d workgroups: per workgroup %lld q|k|v, %lld o, %lld gate|up, %lld down "
                     "row groups (at most 6, 4, 14, 8)",
                     nwg, (long long)gq, (long long)go, (long long)gg, (long long)gd);
    const int64_t per = nq + nk + nv + 2 * H + I;
    const int64_t words = per * n_layers;
    if (words > INT32_MAX / 2) return fail_msg(BTL_ERR_SHAPE, "too many layers for the transport buffer");

    Plan* p = new Plan();
    p->magic = kPlanMagic;
    p->dev = dev;
    p->nl = n_layers;
    p->H = (int)H;
    p->I = (int)I;
    p->nq = (int)nq;
    p->nk = (int)nk;
    p->nv = (int)nv;
    p->nwg = nwg;
    p->kmax = kmax;
    p->words = (size_t)words;
    std::vector<btl::StreamLayer> hl((size_t)n_layers);
    for (int l = 0; l < n_layers; ++l) {
        const btl_stream_layer_t& L = layers[l];
        const btl_packed_t* m[7] = {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down};
        for (int i = 0; i < 7; ++i) {
            hl[(size_t)l].w[i] = m[i]->data;
            hl[(size_t)l].sw[i] = m[i]->scale;
        }
    }
    if ((e = hipMalloc(&p->d_layers, sizeof(btl::StreamLayer) * (size_t)n_layers)) != hipSuccess ||
        (e = hipMalloc(&p->tbuf, p->words * 4)) != hipSuccess ||
        (e = hipMalloc(&p->flags, (size_t)kReplicas * nwg * 8)) != hipSuccess ||
        (e = hipMalloc(&p->epoch, 256)) != hipSuccess) {
        free_plan(p);
        return hip_error(e, "hipMalloc (stream plan)");
    }
    const uint32_t one = 1;
    if ((e = hipMemcpy(p->d_layers, hl.data(), sizeof(btl::StreamLayer) * (size_t)n_layers, hipMemcpyHostToDevice)) !=
            hipSuccess ||
        (e = hipMemset(p->tbuf, 0, p->words * 4)) != hipSuccess ||
        (e = hipMemset(p->flags, 0, (size_t)kReplicas * nwg * 8)) != hipSuccess ||
        (e = hipMemcpy(p->epoch, &one, 4, hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipDeviceSynchronize()) != hipSuccess) {
        free_plan(p);
        return hip_error(e, "stream plan initialisation");
    }
    *plan_out = p;
    return BTL_OK;
}

size_t btl_stream_stage_words(const void* plan)
{
    const Plan* p = (const Plan*)plan;
    return p && p->magic == kPlanMagic ? p->words : 0;
}

int btl_stream_run(void* plan, const void* x, void* y, void* stage_out, void* stream)
{
    Plan* p = (Plan*)plan;
    if (!p || p->magic != kPlanMagic) return fail_msg(BTL_ERR_ARG, "not a stream plan");
    if (!x || !y) return fail_msg(BTL_ERR_LAYOUT, "null input or output");
    if (((uintptr_t)x & 15u) || ((uintptr_t)y & 1u)) return fail_msg(BTL_ERR_LAYOUT, "x must be 16-byte aligned, y 2-byte");
    int dev;
    int rc = btl::host::device(&dev);
    if (rc) return rc;
    if (dev != p->dev) return failf(BTL_ERR_DEVICE, "plan made on device %d, current device %d", p->dev, dev);
    btl::StreamArgs a;
    memset(&a, 0, sizeof(a));
    a.layers = p->d_layers;
    a.nl = p->nl;
    a.H = p->H;
    a.I = p->I;
    a.nq = p->nq;
    a.nk = p->nk;
    a.nv = p->nv;
    a.nwg = p->nwg;
    a.kmax = p->kmax;
    a.x0 = (const uint16_t*)x;
    a.y = (uint16_t*)y;
    a.tbuf = p->tbuf;
    a.flags = p->flags;
    a.epoch = p->epoch;
    a.dbg = (uint16_t*)stage_out;
    // the waits' time budget follows BTL_WAIT_SPIN (polls of ~50 ns): 2^22 -> 0.21 s
    a.budget_ticks = (int64_t)btl::knob(btl::KN_WAIT_SPIN) * 5;
    hipError_t e = btl::launch_dec_stream(a, (hipStream_t)stream);
    if (e != hipSuccess) return hip_error(e, "decode stream launch");
    return BTL_OK;
}

int btl_stream_destroy(void* plan)
{
    Plan* p = (Plan*)plan;
    if (!p) return BTL_OK;
    if (p->magic != kPlanMagic) return fail_msg(BTL_ERR_ARG, "not a stream plan");
    hipError_t e = hipDeviceSynchronize();
    free_plan(p);
    if (e != hipSuccess) return hip_error(e, "hipDeviceSynchronize (stream destroy)");
    return BTL_OK;
}

}  // extern "C"
