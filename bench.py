"""BitLinear benchmark on one MI355X.

Default workload: the Llama-3-8B decode GEMV set at M=1.
32 distinct layers of absmean-ternarised N(0, 0.02) weights (1.745 GB packed, far
above the 256 MB Infinity Cache); per layer the dependency-ordered launches a
decoder issues:
    q|k|v  (one grouped launch, 4096 -> 4096+1024+1024)
    o      (4096 -> 4096)
    w1|w3  (one grouped launch, 4096 -> 2 x 14336)
    w2     (14336 -> 4096)
bf16 activations N(0,1) with 0.1% outliers at +-20 in, bf16 out, W1.58-A8 arithmetic
(per-token absmax int8 activations, exact int32 accumulation).  One step = one token
through all 32 layers (224 projections, 128 launches) replayed from a HIP graph.

The same line carries a "prefill" section (cfg4, M=2048 on the same 32 layers, its own
int8-MFMA roofline) and a "batched_decode" section (cfg3, M = 1..64 on the MLP shapes).

    python bench.py [--steps K] [--warmup W] [--no-cpu-baseline] [--no-prefill] [--no-sweep]
"""
import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "bit-ttt-engine_amd"))

import bitlinear as bl  # noqa: E402

HIDDEN, INTER, KV = 4096, 14336, 1024
LAYERS = 32
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
METRIC = "BitLinear GEMV/GEMM µs & % HBM/int8-MFMA roofline; tok/s, Llama-3-8B shapes"


def synth_packed(n, k, gen, device):
    """Absmean-ternarise N(0, 0.02) weights and pack them in the reference layout,
    on the GPU with torch (synthetic-data plumbing, mirrors PackedTensor::pack)."""
    w = torch.randn((n, k), device=device, generator=gen, dtype=torch.float32) * 0.02
    scale = np.float32(np.float32(w.abs().double().mean().item()) + np.float32(1e-6))
    inv = float(np.float32(1.0 / np.float64(scale)))
    v = w * inv
    del w
    t = (torch.sign(v) * torch.floor(v.abs() + 0.5)).clamp_(-1, 1)
    del v
    codes = torch.where(t > 0.5, 1, torch.where(t < -0.5, 2, 0)).to(torch.uint8).view(-1, 4)
    del t
    packed = codes[:, 0] | (codes[:, 1] << 2) | (codes[:, 2] << 4) | (codes[:, 3] << 6)
    return bl.PackedTensor(packed.contiguous(), float(scale), (n, k), device)


def synth_act(m, k, gen, device):
    """N(0,1) bf16 activations with 0.1% of each row set to +-20."""
    x = torch.randn((m, k), device=device, generator=gen, dtype=torch.float32)
    cnt = int(np.ceil(0.001 * k))
    pos = torch.rand((m, k), device=device, generator=gen).topk(cnt, dim=1).indices
    sign = torch.where(torch.rand((m, cnt), device=device, generator=gen) < 0.5, -20.0, 20.0)
    x.scatter_(1, pos, sign)
    return x.to(torch.bfloat16)


class Call:
    """A pre-bound C-ABI call (pointers resolved once, so graph capture and timing
    loops pay no Python argument handling)."""

    def __init__(self, layers, x, outs, mode=None):
        import ctypes
        # the call holds raw device pointers: keep the tensors they point into
        # alive for as long as the call (a graph capture empties torch's cache)
        self.layers, self.outs = list(layers), list(outs)
        self.cs = [l.as_c() for l in layers]
        self.n = len(layers)
        self.arr = (ctypes.POINTER(bl.BtlPacked) * self.n)(*[ctypes.pointer(c) for c in self.cs])
        self.ys = (ctypes.c_void_p * self.n)(*[o.data_ptr() for o in outs])
        self.x = x
        self.m, self.k = x.shape
        self.xdt = bl.BTL_BF16 if x.dtype == torch.bfloat16 else bl.BTL_F32
        self.ydt = bl.BTL_BF16 if outs[0].dtype == torch.bfloat16 else bl.BTL_F32
        self.mode = bl.BTL_ACT_I8 if mode is None else mode
        self.bytes = sum(l.data.numel() for l in layers) + x.numel() * x.element_size() + sum(
            o.numel() * o.element_size() for o in outs)

    def __call__(self, stream):
        bl.check(bl.lib.btl_linear_group_mode(self.arr, self.ys, self.n, self.x.data_ptr(), self.xdt,
                                              self.m, self.k, self.ydt, self.mode, None, 0, stream))


class OpCall:
    """A pre-bound btl_linear_i8_op call: the prefill GEMM alone (one launch for the
    layers of a group) on operand-order int8 activations."""

    def __init__(self, layers, q, s, outs):
        import ctypes
        self.layers, self.outs = list(layers), list(outs)  # kept alive: the call holds their pointers
        self.cs = [l.as_c() for l in layers]
        self.n = len(layers)
        self.arr = (ctypes.POINTER(bl.BtlPacked) * self.n)(*[ctypes.pointer(c) for c in self.cs])
        self.ys = (ctypes.c_void_p * self.n)(*[o.data_ptr() for o in outs])
        self.q, self.s = q, s
        self.m, self.k = q.shape
        self.ns = [l.dims2()[0] for l in layers]
        self.ops = 2.0 * self.m * self.k * sum(self.ns)

    def __call__(self, stream):
        bl.check(bl.lib.btl_linear_i8_op(self.arr, self.ys, None, self.n, self.q.data_ptr(), self.s.data_ptr(),
                                         self.m, self.k, bl.BTL_BF16, stream))


def time_launches(fn, reps, stream_obj):
    """Average µs of `fn(stream)` over `reps` back-to-back launches, HIP events
    recorded on the stream the kernels run on.  Synchronises first: the inputs
    were made on another stream, and memory that stream's pending kernels still
    use may already back tensors that `fn` reads or writes."""
    torch.cuda.synchronize()
    with torch.cuda.stream(stream_obj):
        s = stream_obj.cuda_stream
        fn(s)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream_obj)
        for _ in range(reps):
            fn(s)
        e1.record(stream_obj)
    torch.cuda.synchronize()
    return 1000.0 * e0.elapsed_time(e1) / reps


def profiled_trace_us(name):
    """The kernel-trace mean duration (us) of the roofline launch recorded in
    profiles/<name> (line "trace_mean_us_gate_up: X"); None if absent."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("trace_mean_us_gate_up:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def _trace_frac(trace_us, work, peak, unit_div):
    """trace_avg_us / achieved_trace / frac_trace of a roofline launch from its
    kernel-trace mean: work (bytes or ops) / trace_us / unit_div against peak."""
    if not trace_us:
        return {"trace_avg_us": None, "frac_trace": None}
    ach = work / trace_us / unit_div
    return {"trace_avg_us": trace_us, "achieved_trace": round(ach, 1), "frac_trace": round(ach / peak, 3),
            "trace_source": "kernel-trace mean of the committed rocprofv3 summary"}


def profiled_traffic(name):
    """HBM bytes per launch measured by the FETCH_SIZE / WRITE_SIZE counter runs
    summarised in profiles/<name> (see the commands there); None if absent."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_baseline(host_layers, seconds):
    """The reference's CPU BitLinear (cpu.rs, restated with AVX2 intrinsics and a
    thread pool, oracle/) on a bounded sample: whole tokens through the 7
    projections of all 32 layers (1.745 GB of packed weights, streamed from host
    DRAM: far beyond any CPU cache), fp32 activations, repeated for about
    `seconds`."""
    from oracle import oracle as orc
    threads = max(1, min(16, os.cpu_count() or 1))
    rng = np.random.default_rng(0)
    xs = {k: rng.standard_normal((1, k)).astype(np.float32) for k in (HIDDEN, INTER)}
    reps, t0 = 0, time.perf_counter()
    while True:
        for proj in host_layers:
            for (wb, n, k, s) in proj:
                orc.forward_f32_avx2(xs[k], wb, n, s, threads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds and reps >= 2:
            break
    per_token = el / reps * (LAYERS / len(host_layers))
    model = "unknown CPU"
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), model)
    except OSError:
        pass
    return {"value": round(1.0 / per_token, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "cpu": "%s, %d logical CPUs visible" % (model, os.cpu_count() or 0),
            "sample": "%d tokens through layers 0-%d of 32 (7 projections each, %.0f MB packed), M=1 fp32, "
                      "cpu.rs algorithm restated in C with AVX2+FMA intrinsics, %d threads; %.1f s"
                      % (reps, len(host_layers) - 1,
                         sum(wb.size for p in host_layers for (wb, _, _, _) in p) / 1e6, threads, el)}


def run_decode(args):
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    bl.check(bl.lib.btl_init(0))
    gen = torch.Generator(device=dev)
    gen.manual_seed(0xB17EB17E)
    shapes = {"q": (HIDDEN, HIDDEN), "k": (KV, HIDDEN), "v": (KV, HIDDEN), "o": (HIDDEN, HIDDEN),
              "gate": (INTER, HIDDEN), "up": (INTER, HIDDEN), "down": (HIDDEN, INTER)}
    layers = []
    for _ in range(LAYERS):
        layers.append({name: synth_packed(n, k, gen, dev) for name, (n, k) in shapes.items()})
    bf = dict(dtype=torch.bfloat16, device=dev)
    calls = {"qkv": [], "o": [], "gate_up": [], "down": []}
    for L in layers:
        xq, xo, xg, xd = (synth_act(1, HIDDEN, gen, dev), synth_act(1, HIDDEN, gen, dev),
                          synth_act(1, HIDDEN, gen, dev), synth_act(1, INTER, gen, dev))
        calls["qkv"].append(Call([L["q"], L["k"], L["v"]], xq,
                                 [torch.empty((1, HIDDEN), **bf), torch.empty((1, KV), **bf),
                                  torch.empty((1, KV), **bf)]))
        calls["o"].append(Call([L["o"]], xo, [torch.empty((1, HIDDEN), **bf)]))
        calls["gate_up"].append(Call([L["gate"], L["up"]], xg,
                                     [torch.empty((1, INTER), **bf), torch.empty((1, INTER), **bf)]))
        calls["down"].append(Call([L["down"]], xd, [torch.empty((1, HIDDEN), **bf)]))
    print("bench: %d layers of weights and inputs ready" % LAYERS, file=sys.stderr, flush=True)
    order = [calls[c][l] for l in range(LAYERS) for c in ("qkv", "o", "gate_up", "down")]
    step_bytes = sum(c.bytes for c in order)
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream().cuda_stream
    for c in order:  # sizes the library workspace before capture
        c(stream)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            s = torch.cuda.current_stream().cuda_stream
            for c in order:
                c(s)
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(args.steps):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    print("bench: %d graph replays, %.4f ms/step" % (args.steps, ms), file=sys.stderr, flush=True)

    # per-kernel durations: the 32 launches of one kind back to back in their
    # own HIP graph, HIP events on the stream the kernels run on
    kern = {}
    for name in ("qkv", "o", "gate_up", "down"):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(cap):
            with torch.cuda.graph(g, stream=cap):
                s2 = torch.cuda.current_stream().cuda_stream
                for l in range(LAYERS):
                    calls[name][l](s2)
        torch.cuda.synchronize()
        g.replay()
        reps = 10
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        us = 1000.0 * e0.elapsed_time(e1) / (reps * LAYERS)
        b = calls[name][0].bytes
        kern[name] = {"us": round(us, 2), "bytes": b, "GB_s": round(b / us / 1e3, 1),
                      "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 3)}
    f32_ref = run_decode_f32_ref(layers, gen, dev, args)
    ceilings = run_ceilings(dev, args)
    dom = kern["gate_up"]
    result = {
        "metric": METRIC, "value": round(1000.0 / ms, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "i8",
        "data": "synthetic (seeded N(0,0.02) weights absmean-ternarised on the GPU; N(0,1) bf16 "
                "activations with 0.1% +-20 outliers)",
        "config": {"workload": "cfg2: Llama-3-8B decode GEMV set, M=1, 32 distinct layers x "
                               "{q|k|v grouped, o, gate|up grouped, down}, bf16 in/out, W1.58-A8; "
                               "one step = one token (224 projections, 128 launches, HIP graph)",
                   "layers": LAYERS, "m": 1, "hidden": HIDDEN, "intermediate": INTER, "kv": KV,
                   "bytes_per_step": step_bytes,
                   "step_GB_s": round(step_bytes / ms / 1e6, 1),
                   "step_frac_hbm": round(step_bytes / ms / 1e6 / HBM_PEAK_GBS, 3)},
        "roofline": {"bound": "hbm", "kernel": "k_gemv_rq<XK_BF16, 4, 4> gate|up 4096->2x14336 (W1.58-A8)",
                     "achieved": dom["GB_s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": dom["frac_hbm"],
                     "traffic": profiled_traffic("k_gemv_rq_gate_up_decode_traffic.md"),
                     "traffic_source": "profiles/k_gemv_rq_gate_up_decode_traffic.md (FETCH_SIZE x copy-calibrated "
                                       "factor + WRITE_SIZE, bytes per launch)",
                     "algorithmic_bytes": dom["bytes"], "avg_us": dom["us"],
                     # the same launch's kernel-trace mean (rocprofv3, no launch gap) from the committed summary
                     **_trace_frac(profiled_trace_us("k_gemv_rq_decode_llama3-8b_m1.md"), dom["bytes"], HBM_PEAK_GBS,
                                   1e3)},
        "kernels": kern,
        "ceilings": ceilings,
        "f32_ref": f32_ref,
    }
    if args.prefill:
        result["prefill"] = run_prefill(layers, gen, dev, args)
    if args.sweep:
        result["batched_decode"] = run_sweep(layers, gen, dev, args)
    if args.pack:
        result["pack"] = run_pack(gen, dev)
    if args.cfg1:
        result["cfg1"] = run_cfg1(gen, dev, args)
    result["anchor"] = run_anchor(dev, args)
    if args.e2e:
        result["e2e"] = run_e2e(layers, gen, dev, args)
    if args.adaptive:
        result["adaptive"] = run_adaptive(gen, dev, args)
    if args.cpu_baseline:
        print("bench: timing the CPU baseline", file=sys.stderr, flush=True)
        host = []
        for L in layers:
            host.append([(L[nm].data.cpu().numpy(), shapes[nm][0], shapes[nm][1], L[nm].scale)
                         for nm in ("q", "k", "v", "o", "gate", "up", "down")])
        result["cpu_baseline"] = cpu_baseline(host, args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


def _graph_us(fns, reps, cap):
    """us per replay of one HIP graph holding fns (each fn(stream)) in order
    (synchronises first, as time_launches)."""
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap):
        with torch.cuda.graph(g, stream=cap):
            s = torch.cuda.current_stream().cuda_stream
            for fn in fns:
                fn(s)
    torch.cuda.synchronize()
    g.replay()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return 1000.0 * e0.elapsed_time(e1) / reps


def run_decode_f32_ref(layers, gen, dev, args):
    """The cfg2 step in the reference's own arithmetic (BTL_ACT_F32_REF: cpu.rs's
    fp32 semantics and 8-lane summation order, bit for bit), f32 in and out as the
    reference's BitLinearCpu takes them: q|k|v and gate|up through
    btl_linear_group_mode, o and down single, 32 layers in one HIP graph."""
    f32 = dict(dtype=torch.float32, device=dev)
    calls = {"qkv": [], "o": [], "gate_up": [], "down": []}
    for L in layers:
        xq, xo, xg, xd = (torch.randn((1, k), generator=gen, **f32) for k in (HIDDEN, HIDDEN, HIDDEN, INTER))
        calls["qkv"].append(Call([L["q"], L["k"], L["v"]], xq,
                                 [torch.empty((1, HIDDEN), **f32), torch.empty((1, KV), **f32),
                                  torch.empty((1, KV), **f32)], mode=bl.BTL_ACT_F32_REF))
        calls["o"].append(Call([L["o"]], xo, [torch.empty((1, HIDDEN), **f32)], mode=bl.BTL_ACT_F32_REF))
        calls["gate_up"].append(Call([L["gate"], L["up"]], xg,
                                     [torch.empty((1, INTER), **f32), torch.empty((1, INTER), **f32)],
                                     mode=bl.BTL_ACT_F32_REF))
        calls["down"].append(Call([L["down"]], xd, [torch.empty((1, HIDDEN), **f32)], mode=bl.BTL_ACT_F32_REF))
    order = [calls[c][l] for l in range(LAYERS) for c in ("qkv", "o", "gate_up", "down")]
    step_bytes = sum(c.bytes for c in order)
    cap = torch.cuda.Stream()
    for c in order:
        c(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    us = _graph_us(order, 10, cap)
    kern = {}
    for name in ("qkv", "o", "gate_up", "down"):
        kus = _graph_us(calls[name], 10, cap) / LAYERS
        b = calls[name][0].bytes
        kern[name] = {"us": round(kus, 2), "bytes": b, "GB_s": round(b / kus / 1e3, 1),
                      "frac_hbm": round(b / kus / 1e3 / HBM_PEAK_GBS, 3)}
    print("bench: cfg2 in f32_ref mode %.4f ms/step" % (us / 1000.0), file=sys.stderr, flush=True)
    return {"workload": "cfg2 in the reference's arithmetic (BTL_ACT_F32_REF, cpu.rs order bit for bit): "
                        "M=1, 32 layers x {q|k|v grouped, o, gate|up grouped, down}, f32 in/out, HIP graph",
            "ms_per_step": round(us / 1000.0, 4), "tok_s": round(1e6 / us, 1), "bytes_per_step": step_bytes,
            "step_GB_s": round(step_bytes / us / 1e3, 1),
            "step_frac_hbm": round(step_bytes / us / 1e3 / HBM_PEAK_GBS, 3), "kernels": kern}


def run_prefill(layers, gen, dev, args):
    """cfg4: M=2048 prefill on the seven Llama-3-8B projection shapes, the same 32
    layers of weights.  One step = the 7 projections of all 32 layers as a decoder
    issues them (btl_linear_group q|k|v, btl_linear o, btl_linear_group gate|up,
    btl_linear down: each quantises its bf16 input, then the GEMM), HIP graph.
    Per kernel kind: the GEMM alone (btl_linear_i8_op) and the quantiser alone."""
    M = args.prefill_m
    bf = dict(dtype=torch.bfloat16, device=dev)
    xh = synth_act(M, HIDDEN, gen, dev)
    xi = synth_act(M, INTER, gen, dev)
    groups = {"qkv": ("q", "k", "v"), "o": ("o",), "gate_up": ("gate", "up"), "down": ("down",)}
    outs = {g: [torch.empty((M, layers[0][nm].dims2()[0]), **bf) for nm in names] for g, names in groups.items()}
    calls = []
    for L in layers:
        for g, names in groups.items():
            calls.append(Call([L[nm] for nm in names], xi if g == "down" else xh, outs[g]))
    stream = torch.cuda.current_stream().cuda_stream
    for c in calls[:4]:  # sizes the library workspace before capture
        c(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            s = torch.cuda.current_stream().cuda_stream
            for c in calls:
                c(s)
    torch.cuda.synchronize()
    for _ in range(max(1, args.warmup // 2)):
        graph.replay()
    torch.cuda.synchronize()
    psteps = max(2, args.steps // 10)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(psteps):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / psteps
    print("bench: prefill M=%d, %d graph replays, %.3f ms/step" % (M, psteps, ms), file=sys.stderr, flush=True)

    # the GEMM alone per kind (layer 0's weights; operand-order activations)
    qh, sh = bl.quantize_act_op(xh)
    qi, si = bl.quantize_act_op(xi)
    kern = {}
    for g, names in groups.items():
        oc = OpCall([layers[0][nm] for nm in names], qi if g == "down" else qh,
                    si if g == "down" else sh, outs[g])
        us = time_launches(oc, 20, cap)
        kern[g] = {"us": round(us, 2), "TOPS": round(oc.ops / us / 1e6, 1),
                   "frac_int8": round(oc.ops / us / 1e6 / INT8_PEAK_TOPS, 3), "ops": oc.ops,
                   "n": oc.ns, "k": oc.k}
    for name, x in (("quant_op_k4096", xh), ("quant_op_k14336", xi)):
        qq, ss = (qh, sh) if x is xh else (qi, si)
        fn = lambda st, x=x, qq=qq, ss=ss: bl.check(bl.lib.btl_quantize_act_op(
            x.data_ptr(), bl.BTL_BF16, M, x.shape[1], qq.data_ptr(), ss.data_ptr(), st))
        us = time_launches(fn, 20, cap)
        b = x.numel() * 2 + qq.numel() + ss.numel() * 4
        kern[name] = {"us": round(us, 2), "bytes": b, "GB_s": round(b / us / 1e3, 1),
                      "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 3)}
    gemm_us = sum(kern[g]["us"] for g in groups)
    layer_ops = sum(kern[g]["ops"] for g in groups)
    dom = kern["gate_up"]
    return {
        "workload": "cfg4: Llama-3-8B prefill, M=%d tokens, 7 projections x 32 layers as 4 calls per "
                    "layer (q|k|v and gate|up grouped), bf16 in/out, W1.58-A8" % M,
        "value": round(M / ms * 1000.0, 1), "unit": "tok/s", "ms_per_step": round(ms, 3),
        "step_TOPS": round(LAYERS * layer_ops / ms / 1e9, 1),
        "step_frac_int8": round(LAYERS * layer_ops / ms / 1e9 / INT8_PEAK_TOPS, 3),
        "gemm_only_layer_us": round(gemm_us, 2),
        "gemm_only_frac_int8": round(layer_ops / gemm_us / 1e6 / INT8_PEAK_TOPS, 3),
        "roofline": {"bound": "mfma", "kernel": "k_gemm_i8 gate|up 2048 x (2 x 14336) x 4096, one launch",
                     "achieved": dom["TOPS"], "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
                     "frac": dom["frac_int8"],
                     "traffic": profiled_traffic("k_gemm_i8_gate_up_prefill_traffic.md"),
                     "traffic_source": "profiles/k_gemm_i8_gate_up_prefill_traffic.md (bytes per launch crossing "
                                       "the L2s; the 8 XCDs each fetch the weights once)",
                     "algorithmic_ops": dom["ops"], "avg_us": dom["us"],
                     **_trace_frac(profiled_trace_us("k_gemm_i8_prefill_llama3-8b_m2048.md"), dom["ops"],
                                   INT8_PEAK_TOPS, 1e6)},
        "kernels": kern,
    }


def run_sweep(layers, gen, dev, args):
    """cfg3: batched decode M in {1,2,4,8,16,32,64} on the MLP shapes (gate|up grouped
    4096 -> 2 x 14336, down 14336 -> 4096) of the same 32 layers, HIP graph per M.
    Locates where the HBM-bound GEMV hands over to the MFMA GEMM."""
    bf = dict(dtype=torch.bfloat16, device=dev)
    rows = []
    cap = torch.cuda.Stream()
    for m in (1, 2, 4, 8, 16, 32, 64):
        xg, xd = synth_act(m, HIDDEN, gen, dev), synth_act(m, INTER, gen, dev)
        og = [torch.empty((m, INTER), **bf), torch.empty((m, INTER), **bf)]
        od = [torch.empty((m, HIDDEN), **bf)]
        calls = []
        for L in layers:
            calls.append(Call([L["gate"], L["up"]], xg, og))
            calls.append(Call([L["down"]], xd, od))
        stream = torch.cuda.current_stream().cuda_stream
        for c in calls[:2]:
            c(stream)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(cap):
            with torch.cuda.graph(g, stream=cap):
                s = torch.cuda.current_stream().cuda_stream
                for c in calls:
                    c(s)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        reps = 10
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        us = 1000.0 * e0.elapsed_time(e1) / (reps * LAYERS)
        b = calls[0].bytes + calls[1].bytes
        ops = 2.0 * m * (2 * INTER * HIDDEN + HIDDEN * INTER)
        rows.append({"m": m, "mlp_us": round(us, 2), "tok_s": round(m * 1e6 / (us * LAYERS), 1),
                     "GB_s": round(b / us / 1e3, 1), "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 3),
                     "TOPS": round(ops / us / 1e6, 2)})
        del g
    print("bench: batched-decode sweep done", file=sys.stderr, flush=True)
    return {"workload": "cfg3: batched decode, MLP of 32 layers (gate|up grouped, down), bf16 in/out, "
                        "W1.58-A8; per M: µs per layer MLP, tokens/s through the 32 MLPs",
            "rows": rows}


def _e2e_run(model, prompt, gen_len):
    """Prefill (timed with HIP events), the first greedy pick, one eager decode
    step, capture, then gen_len - 2 graph replays (timed).  -> (prefill ms,
    decode ms per token, the generated ids)."""
    model.reset()
    model.prefill(prompt)  # warm-up (sizes the library workspace)
    torch.cuda.synchronize()
    model.reset()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    model.prefill(prompt)
    e1.record()
    torch.cuda.synchronize()
    prefill_ms = e0.elapsed_time(e1)
    model.greedy()
    start = model.pos
    model.start_decode()
    model.decode_steps(1, use_graph=False)
    model.capture_decode()
    torch.cuda.synchronize()
    e0.record()
    model.decode_steps(gen_len - 2, use_graph=True)
    e1.record()
    torch.cuda.synchronize()
    dec_ms = e0.elapsed_time(e1) / (gen_len - 2)
    return prefill_ms, dec_ms, model.log[start:start + gen_len].cpu().numpy()


def _dense_head_kernel(w, code, dev, reps=20):
    """btl_dense_linear alone at M=1 (the lm_head GEMV): launches over the same
    weights back to back on one stream (each reads far more than the caches hold);
    us per launch and the HBM fraction of its bytes."""
    x = torch.randn((1, w.shape[1]), device=dev)
    y = torch.empty((1, w.shape[0]), device=dev)

    def fn(stream):
        for _ in range(reps):
            bl.check(bl.lib.btl_dense_linear(w.data_ptr(), code, w.shape[0], w.shape[1], x.data_ptr(), 1,
                                             y.data_ptr(), stream))

    us = time_launches(fn, 5, torch.cuda.Stream()) / reps
    nbytes = w.numel() * w.element_size() + x.numel() * 4 + y.numel() * 4
    return {"us": round(us, 2), "bytes": int(nbytes), "GB_s": round(nbytes / us / 1e3, 1),
            "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 3)}


def run_e2e(layers, gen, dev, args):
    """cfg5: the end-to-end decoder (bitlinear.model.BitLlamaHip) with Llama-3-8B
    shapes on the same 32 layers of packed weights, plus seeded norm weights and an
    f32 embedding table (vocab 128256): a prompt of 512 uniform random ids
    prefilled in one batch, then 256 greedy decode steps at batch 1, each a
    HIP-graph replay of one step with the position and next id on the device (no
    host synchronisation between steps).  Timed separately: the prefill (HIP
    events around it) and the decode steps after the first (events around the
    replays).  Three heads: a ternary BitLinear lm_head (the headline), and the
    reference's dense lm_head (llama.rs:129-141) with f32 weights -- as the
    reference holds them -- and with bf16 weights."""
    from bitlinear.model import BitLlamaHip, LlamaConfig
    prompt_len, gen_len = args.e2e_prompt, args.e2e_tokens
    cfg = LlamaConfig.llama3_8b(max_seq=prompt_len + gen_len + 1)

    def norm():
        return (1.0 + 0.1 * torch.randn((HIDDEN,), generator=gen, device=dev)).contiguous()

    w = torch.randn((cfg.vocab, HIDDEN), generator=gen, device=dev) * 0.02
    head = bl.PackedTensor.pack_device(w)
    weights = {"embed": torch.randn((cfg.vocab, HIDDEN), generator=gen, device=dev), "norm_f": norm(),
               "lm_head": head,
               "layers": [dict(L, norm1=norm(), norm2=norm()) for L in layers]}
    prompt = torch.randint(0, cfg.vocab, (prompt_len,), generator=gen, device=dev).cpu().numpy()
    # per-step bytes: the 32 layers' packed weights + lm_head + the Q8 KV rows read at the mean context
    wbytes = sum(L[nm].data.numel() for L in layers for nm in ("q", "k", "v", "o", "gate", "up", "down"))
    mean_ctx = prompt_len + gen_len / 2
    kv_bytes = LAYERS * 2 * cfg.n_kv_heads * mean_ctx * (cfg.head_dim + 4)

    def summary(prefill_ms, dec_ms, head_bytes):
        step_bytes = wbytes + head_bytes + kv_bytes
        return {"prefill_tok_s": round(prompt_len / prefill_ms * 1000.0, 1), "prefill_ms": round(prefill_ms, 3),
                "decode_tok_s": round(1000.0 / dec_ms, 1), "decode_ms_per_token": round(dec_ms, 4),
                "decode_bytes_per_token": int(step_bytes),
                "decode_frac_hbm": round(step_bytes / dec_ms / 1e6 / HBM_PEAK_GBS, 3)}

    model = BitLlamaHip(cfg, weights, dev, max_rows=prompt_len)
    prefill_ms, dec_ms, toks = _e2e_run(model, prompt, gen_len)
    del model
    print("bench: e2e prefill %d tokens %.2f ms, decode %.3f ms/token" % (prompt_len, prefill_ms, dec_ms),
          file=sys.stderr, flush=True)
    out = {"workload": "cfg5: Llama-3-8B-shaped ternary decoder, 32 layers, hidden 4096, 32/8 heads x 128, "
                       "intermediate 14336, vocab 128256, every linear BitLinear W1.58-A8 (lm_head too), Q8 KV "
                       "cache; %d-token uniform random prompt prefilled in one batch, %d greedy tokens at batch 1 "
                       "(HIP-graph step, device-side position)" % (prompt_len, gen_len)}
    out.update(summary(prefill_ms, dec_ms, head.data.numel()))
    # embedding; per layer q|k|v (norm in the quantising waves), attention (RoPE,
    # append, chunks and their merge), o (+ residual), gate|up (norm; SwiGLU
    # epilogue), down (+ residual); final norm, lm_head, pick
    out["launches_per_token"] = 1 + LAYERS * 5 + 3
    out["first_tokens"] = [int(t) for t in toks[:8]]
    dense = {"workload": "the same decoder with the reference's dense lm_head (candle_nn::Linear, "
                         "llama.rs:129-141): final RMSNorm to f32 (btl_add_rmsnorm), then btl_dense_linear "
                         "(f32 sums) over f32 weights (as the reference holds them) or bf16 weights"}
    for name, dt, code in (("f32", torch.float32, bl.BTL_F32), ("bf16", torch.bfloat16, bl.BTL_BF16)):
        dw = w.to(dt).contiguous()
        weights["lm_head"] = dw
        model = BitLlamaHip(cfg, weights, dev, max_rows=prompt_len)
        p_ms, d_ms, _ = _e2e_run(model, prompt, gen_len)
        del model
        dense[name] = summary(p_ms, d_ms, dw.numel() * dw.element_size())
        dense[name]["lm_head_kernel"] = _dense_head_kernel(dw, code, dev)
        print("bench: e2e dense %s head: decode %.3f ms/token, head kernel %.1f us" %
              (name, d_ms, dense[name]["lm_head_kernel"]["us"]), file=sys.stderr, flush=True)
        del dw
    # the decoder in the reference's own arithmetic: fp32 BitLinears (cpu.rs order,
    # BTL_ACT_F32_REF) and the dense f32 lm_head -- what the reference computes on a CPU
    dw = w.contiguous()
    weights["lm_head"] = dw
    model = BitLlamaHip(cfg, weights, dev, max_rows=prompt_len, mode="f32_ref")
    ref_tokens = min(gen_len, 64)
    p_ms, d_ms, _ = _e2e_run(model, prompt, ref_tokens)
    del model, dw
    out["reference_arithmetic"] = dict(
        summary(p_ms, d_ms, cfg.vocab * HIDDEN * 4),
        workload="the same decoder with every BitLinear in the reference's fp32 order (mode f32_ref, "
                 "BitLinearCpu::forward bit for bit) and the dense f32 lm_head: the reference's own CPU "
                 "arithmetic; %d greedy tokens" % ref_tokens)
    print("bench: e2e in the reference's arithmetic: decode %.3f ms/token" % d_ms, file=sys.stderr, flush=True)
    weights["lm_head"] = head
    del w
    out["dense_head"] = dense
    return out


def run_adaptive(gen, dev, args):
    """The multi-base adaptive format (AdaptiveBitLinear, adaptive_linear.rs) with the
    reference converter's default of 3 bases (convert_llama_v2.py --n-bases 3), on the
    Llama-3-8B MLP gate shape 4096 -> 14336: 32 distinct layers of interleaved bytes
    (44 MB each, random codes, ~1/3 zeros), split once on the device
    (btl_adaptive_split), then W1.58-A8 btl_adaptive_linear at M=1 (the 32 calls
    back to back in a HIP graph) and at M=2048.  Algorithmic bytes at M=1: the 3
    bases' packed bytes + x (bf16) + y (bf16)."""
    nb, n, k = 3, INTER, HIDDEN
    layers = []
    for _ in range(LAYERS):
        codes = torch.randint(0, 3, (n * (k // 4) * nb, 4), generator=gen, device=dev, dtype=torch.uint8)
        packed = (codes[:, 0] | (codes[:, 1] << 2) | (codes[:, 2] << 4) | (codes[:, 3] << 6)).contiguous()
        del codes
        scales = [0.02, 0.007, 0.0025]
        layers.append(bl.AdaptiveBitLinear.load(k, n, packed, scales))
        del packed
    bf = dict(dtype=torch.bfloat16, device=dev)
    x1 = synth_act(1, k, gen, dev)
    y1 = torch.empty((1, n), **bf)
    stream = torch.cuda.current_stream().cuda_stream

    def call(L, x, y, st):
        if L._c is None:
            L.forward(x)  # binds the C arrays
        bl.check(bl.lib.btl_adaptive_linear(L._c[1], nb, x.data_ptr(), bl.BTL_BF16, x.shape[0], k, y.data_ptr(),
                                            bl.BTL_BF16, None, 0, st))
    for L in layers:
        call(L, x1, y1, stream)
    torch.cuda.synchronize()
    cap = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap):
        with torch.cuda.graph(g, stream=cap):
            s2 = torch.cuda.current_stream().cuda_stream
            for L in layers:
                call(L, x1, y1, s2)
    torch.cuda.synchronize()
    g.replay()
    reps = 10
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    us1 = 1000.0 * e0.elapsed_time(e1) / (reps * LAYERS)
    b1 = nb * n * k // 4 + k * 2 + n * 2
    M = args.prefill_m
    xm = synth_act(M, k, gen, dev)
    ym = torch.empty((M, n), **bf)
    usm = time_launches(lambda st: call(layers[0], xm, ym, st), 10, cap)
    ops = 2.0 * M * n * k * nb
    print("bench: adaptive nb=3 decode %.2f us, prefill %.1f us" % (us1, usm), file=sys.stderr, flush=True)
    return {"workload": "multi-base adaptive format, 3 bases, 4096 -> 14336 (Llama-3-8B gate), W1.58-A8, bf16 in/out; "
                        "split once on the device, then btl_adaptive_linear (one grouped launch over the bases + "
                        "the ordered base sum)",
            "decode_m1_us": round(us1, 2), "decode_bytes": b1, "decode_GB_s": round(b1 / us1 / 1e3, 1),
            "decode_frac_hbm": round(b1 / us1 / 1e3 / HBM_PEAK_GBS, 3),
            "prefill_m": M, "prefill_us": round(usm, 2), "prefill_TOPS": round(ops / usm / 1e6, 1),
            "prefill_frac_int8": round(ops / usm / 1e6 / INT8_PEAK_TOPS, 3)}


def run_cfg1(gen, dev, args):
    """cfg1 (the reference's own CPU-runnable case): one
    BitLinear forward, K=2048 -> N=5632, M=1, f32 N(0,1) in, f32 out, in both
    arithmetic modes -- BTL_ACT_F32_REF (the reference's fp32 semantics and
    summation order) and W1.58-A8.  16 distinct weight copies replayed back to
    back in a HIP graph (us per call); the reference's CPU algorithm (cpu.rs,
    restated with AVX2 intrinsics and a thread pool) on the same shape beside it.
    A parity configuration: launch-latency-bound, its roofline fraction is
    reported, not targeted."""
    import ctypes
    n, k, copies = 5632, 2048, 16
    ws = [synth_packed(n, k, gen, dev) for _ in range(copies)]
    x = torch.randn((1, k), generator=gen, device=dev, dtype=torch.float32)
    y = torch.empty((1, n), dtype=torch.float32, device=dev)
    cs = [w.as_c() for w in ws]
    out = {"workload": "cfg1: one BitLinear 2048 -> 5632, M=1, f32 in/out, 16 distinct weight copies "
                       "back to back in a HIP graph",
           "algorithmic_bytes": n * k // 4 + k * 4 + n * 4 + 4}
    b = out["algorithmic_bytes"]
    for mode_name, mode in (("f32_ref", bl.BTL_ACT_F32_REF), ("f32_seq", bl.BTL_ACT_F32_SEQ), ("i8", bl.BTL_ACT_I8)):
        def one(stream, c):
            bl.check(bl.lib.btl_linear(ctypes.byref(c), x.data_ptr(), bl.BTL_F32, 1, k, y.data_ptr(), bl.BTL_F32,
                                       mode, None, None, 0, stream))
        st = torch.cuda.current_stream().cuda_stream
        for c in cs:
            one(st, c)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        with torch.cuda.stream(cap):
            with torch.cuda.graph(g, stream=cap):
                s2 = torch.cuda.current_stream().cuda_stream
                for c in cs:
                    one(s2, c)
        torch.cuda.synchronize()
        g.replay()
        reps = 20
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        us = 1000.0 * e0.elapsed_time(e1) / (reps * copies)
        out[mode_name] = {"us": round(us, 2), "GB_s": round(b / us / 1e3, 1),
                          "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 3)}
    print("bench: cfg1 f32_ref %.2f us, f32_seq %.2f us, i8 %.2f us" % (out["f32_ref"]["us"], out["f32_seq"]["us"],
                                                                       out["i8"]["us"]), file=sys.stderr, flush=True)
    if args.cpu_baseline:
        from oracle import oracle as orc
        threads = max(1, min(16, os.cpu_count() or 1))
        xh = x.cpu().numpy()
        wb, sw = ws[0].data.cpu().numpy(), ws[0].scale
        orc.forward_f32_avx2(xh, wb, n, sw, threads=threads)
        reps, t0 = 0, time.perf_counter()
        while True:
            orc.forward_f32_avx2(xh, wb, n, sw, threads=threads)
            reps += 1
            el = time.perf_counter() - t0
            if el >= 2.0 and reps >= 10:
                break
        cus = 1e6 * el / reps
        out["cpu_baseline"] = {"us": round(cus, 2), "GB_s": round(b / cus / 1e3, 2), "cores": threads,
                               "kind": "port", "sample": "%d calls of the cfg1 shape on one weight copy, "
                                                         "%.1f s" % (reps, el)}
    return out


def run_anchor(dev, args):
    """The reference's own kernel benchmark (bench_cpu_kernel.rs:12-91): one
    BitLinear M=1, K=N=8192, x = 0.5, packed bytes i % 255, scale 1; 10 warm-up
    calls, then the mean of 100 timed calls; GOps/s = M*N*K/t and GB/s =
    (4MK + NK/4 + 4MN)/t, the reference's formulas.  On the GPU in both
    arithmetic modes (f32 in/out), and the reference's CPU algorithm (cpu.rs
    restated with AVX2 intrinsics) on the host cores.  gpu_f32_seq: the same in the
    order of a host without AVX2/FMA (one sequential chain of K adds per output)."""
    import ctypes
    m, k, n = 1, 8192, 8192
    wb = (np.arange(n * k // 4) % 255).astype(np.uint8)
    pt = bl.PackedTensor(torch.from_numpy(wb).to(dev), 1.0, (n, k), dev)
    c = pt.as_c()
    x = torch.full((m, k), 0.5, device=dev)
    y = torch.empty((m, n), device=dev)
    nbytes = 4 * m * k + n * k // 4 + 4 * m * n
    ops = m * n * k

    def rates(sec):
        return {"ms": round(sec * 1e3, 4), "GOps_s": round(ops / sec / 1e9, 2), "GB_s": round(nbytes / sec / 1e9, 2)}

    out = {"workload": "bench_cpu_kernel.rs: M=1, K=N=8192, x=0.5, weight bytes i % 255, scale 1; 10 warm-ups, "
                       "mean of 100 calls; GOps/s = M*N*K/t, GB/s = (4MK + NK/4 + 4MN)/t"}
    for name, mode in (("gpu_f32_ref", bl.BTL_ACT_F32_REF), ("gpu_f32_seq", bl.BTL_ACT_F32_SEQ),
                       ("gpu_i8", bl.BTL_ACT_I8)):
        def call(stream):
            bl.check(bl.lib.btl_linear(ctypes.byref(c), x.data_ptr(), bl.BTL_F32, m, k, y.data_ptr(), bl.BTL_F32,
                                       mode, None, None, 0, stream))
        st = torch.cuda.current_stream()
        for _ in range(10):
            call(st.cuda_stream)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(100):
            call(st.cuda_stream)
        e1.record()
        torch.cuda.synchronize()
        out[name] = rates(e0.elapsed_time(e1) / 1e3 / 100)
        out[name]["frac_hbm"] = round(nbytes / (e0.elapsed_time(e1) / 1e3 / 100) / 1e9 / HBM_PEAK_GBS, 4)
    if args.cpu_baseline:
        from oracle import oracle as orc
        threads = max(1, min(16, os.cpu_count() or 1))
        xh = np.full((m, k), 0.5, np.float32)
        for _ in range(10):
            orc.forward_f32_avx2(xh, wb, n, 1.0, threads=threads)
        t0 = time.perf_counter()
        for _ in range(100):
            orc.forward_f32_avx2(xh, wb, n, 1.0, threads=threads)
        out["cpu"] = dict(rates((time.perf_counter() - t0) / 100), cores=threads, kind="port",
                          nproc=os.cpu_count() or 0,
                          sample="cpu.rs restated in C with AVX2+FMA intrinsics, %d threads (the box's CPU share; "
                                 "the reference's rayon pool would take nproc)" % threads)
    print("bench: anchor (M=1, K=N=8192): gpu f32_ref %.4f ms, gpu f32_seq %.4f ms, gpu i8 %.4f ms%s" %
          (out["gpu_f32_ref"]["ms"], out["gpu_f32_seq"]["ms"], out["gpu_i8"]["ms"],
           ", cpu %.3f ms" % out["cpu"]["ms"] if "cpu" in out else ""), file=sys.stderr, flush=True)
    return out


def run_pack(gen, dev):
    """PackedTensor::pack on the device (btl_pack_device) of one f32 weight of the
    MLP up shape 14336 x 4096: the load-time quantisation a checkpoint loader
    runs once per layer.  Algorithmic bytes = the f32 read once + the packed
    bytes written; the kernels read the f32 tensor twice (the absmean reduction,
    then the code pass), so the HBM-bound ceiling is about half the peak."""
    n, k = INTER, HIDDEN
    w = torch.randn((n, k), generator=gen, device=dev, dtype=torch.float32) * 0.02
    out = torch.empty(((n * k + 3) // 4,), dtype=torch.uint8, device=dev)
    sc = torch.empty((1,), dtype=torch.float32, device=dev)
    wsb = bl.lib.btl_pack_workspace_bytes(n, k)
    ws = torch.empty((wsb,), dtype=torch.uint8, device=dev)

    def fn(stream):
        bl.check(bl.lib.btl_pack_device(w.data_ptr(), n, k, out.data_ptr(), sc.data_ptr(), ws.data_ptr(), wsb,
                                        stream))
    us = time_launches(fn, 20, torch.cuda.Stream())
    b = n * k * 4 + (n * k) // 4
    print("bench: device pack %.1f us" % us, file=sys.stderr, flush=True)
    return {"workload": "btl_pack_device, f32 [14336, 4096] -> packed 2-bit + absmean scale",
            "us": round(us, 2), "algorithmic_bytes": b, "GB_s": round(b / us / 1e3, 1),
            "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 3), "kernels": "k_abs_sum x2 levels + k_pack_codes"}


def run_ceilings(dev, args):
    """The ceilings of the cfg2 decode chain, from the probe kernels
    (bit-ttt-engine_amd/probe/btl_probe.hip, not part of the library): a plain
    streaming read (non-temporal 16-byte loads, every load in flight before the
    first use) of exactly the packed bytes of each launch of the step, over the
    same 32-layer footprint (1.745 GB, far beyond the 256 MB Infinity Cache), as
    the same 128 dependent launches in one HIP graph; the same per launch kind (32
    launches of one kind in a graph); and an empty kernel in a chain of 128
    dependent launches (1 and 1792 workgroups): the cost of a launch boundary.
    Then the int8 MFMA ceilings (mfma_ceilings)."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(ROOT, "bit-ttt-engine_amd", "probe", "libbtl_probe.so"))
    lib.probe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    lib.probe_stream_read_words.restype = ctypes.c_int64
    lib.probe_stream_read_words.argtypes = [ctypes.c_int64]
    lib.probe_empty.argtypes = [ctypes.c_int, ctypes.c_void_p]
    kinds = {"qkv": (HIDDEN + 2 * KV) * HIDDEN // 4, "o": HIDDEN * HIDDEN // 4, "gate_up": 2 * INTER * HIDDEN // 4,
             "down": HIDDEN * INTER // 4}
    per_layer = sum(kinds.values())
    buf = torch.empty(LAYERS * per_layer, dtype=torch.uint8, device=dev).fill_(0x5A)
    out = torch.empty(lib.probe_stream_read_words(max(kinds.values())), dtype=torch.int32, device=dev)
    reads = {k: [] for k in kinds}
    off = 0
    for _ in range(LAYERS):
        for k, b in kinds.items():
            reads[k].append(lambda st, o=off, b=b: lib.probe_stream_read(buf.data_ptr() + o, b, out.data_ptr(), st))
            off += b
    order = [reads[k][l] for l in range(LAYERS) for k in kinds]
    cap = torch.cuda.Stream()
    for fn in order:
        fn(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    chain_us = _graph_us(order, 10, cap)
    res = {"what": "probe kernels (bit-ttt-engine_amd/probe/btl_probe.hip): streaming read of each launch's packed "
                   "bytes over the 32-layer footprint, and empty launches; HIP graphs, HIP events",
           "stream_read_step_us": round(chain_us, 1),
           "stream_read_step_frac_hbm": round(LAYERS * per_layer / chain_us / 1e3 / HBM_PEAK_GBS, 3)}
    for k, b in kinds.items():
        us = _graph_us(reads[k], 10, cap) / LAYERS
        res["stream_read_" + k] = {"us": round(us, 2), "bytes": b, "GB_s": round(b / us / 1e3, 1),
                                   "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 3)}
    for wgs in (1, 1792):
        us = _graph_us([lambda st, w=wgs: lib.probe_empty(w, st)] * 128, 10, cap) / 128
        res["empty_launch_us_%dwg" % wgs] = round(us, 3)
    del buf
    res.update(mfma_ceilings(lib, dev, cap))
    print("bench: ceilings: streaming-read step %.1f us, empty launch %.2f us" % (
        chain_us, res["empty_launch_us_1wg"]), file=sys.stderr, flush=True)
    return res


PROBE_KINDS = {"qkv": ((HIDDEN, HIDDEN), (KV, HIDDEN), (KV, HIDDEN)), "o": ((HIDDEN, HIDDEN),),
               "gate_up": ((INTER, HIDDEN), (INTER, HIDDEN)), "down": ((HIDDEN, INTER),)}


def mfma_ceilings(lib, dev, cap):
    """What the int8 matrix cores and the vendor library reach on this box: the
    probe's MFMA loop (8 independent v_mfma_i32_16x16x64_i8 per round, two waves
    per SIMD on every CU, operands held in registers) with random int8 x ternary
    operands (the prefill GEMM's data), random x random, and one constant byte;
    and hipBLASLt's dense int8 GEMM (torch._int_mm) on the M=2048 gate|up shape
    with the weights stored as dense int8 {-1, 0, +1} (4x the packed bytes)."""
    import ctypes
    lib.probe_mfma_loop.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    wgs, iters = 2 * cus, 4000
    ops = wgs * 4 * 8 * iters * 2.0 * 16 * 16 * 64
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    rnd = torch.randint(-128, 128, (65536, 16), generator=g, device=dev, dtype=torch.int16).to(torch.int8)
    ter = torch.randint(-1, 2, (65536, 16), generator=g, device=dev, dtype=torch.int16).to(torch.int8)
    lane = torch.arange(65536, device=dev).unsqueeze(1) % 8
    srcs = {"random_x_ternary": torch.where(lane < 4, rnd, ter).contiguous(), "random_x_random": rnd,
            "constant": torch.full((65536, 16), 1, dtype=torch.int8, device=dev)}
    out = torch.empty(wgs * 256, dtype=torch.int32, device=dev)
    res = {}
    for name, src in srcs.items():
        fn = lambda st, src=src: lib.probe_mfma_loop(src.data_ptr(), iters, wgs, out.data_ptr(), st)
        us = time_launches(fn, 5, cap)
        res["mfma_loop_" + name] = {"TOPS": round(ops / us / 1e6, 1), "frac_int8": round(ops / us / 1e6 / INT8_PEAK_TOPS, 3)}
    m, k, n = 2048, HIDDEN, 2 * INTER
    a = torch.randint(-128, 128, (m, k), generator=g, device=dev, dtype=torch.int16).to(torch.int8)
    w = torch.randint(-1, 2, (n, k), generator=g, device=dev, dtype=torch.int16).to(torch.int8)
    best = None
    for layout, b in (("k-major", w.t()), ("n-major", w.t().contiguous())):
        try:
            us = time_launches(lambda st, b=b: torch._int_mm(a, b), 10, cap)
        except RuntimeError:
            continue
        if best is None or us < best[1]:
            best = (layout, us)
    if best is not None:
        op = 2.0 * m * n * k
        res["hipblaslt_int8_gate_up_m2048"] = {"us": round(best[1], 1), "TOPS": round(op / best[1] / 1e6, 1),
                                               "frac_int8": round(op / best[1] / 1e6 / INT8_PEAK_TOPS, 3),
                                               "weights": "dense int8 [28672, 4096], %s" % best[0]}
    return res


def run_probe(args):
    """A few launches of one workload, plus a plain copy of known size, for
    counter runs (rocprofv3 --pmc ...): --probe decode_<kind> is btl_linear_group
    at M=1 (the decode kernel), batched<M>_<kind> the same at M token rows (M up
    to 64: the batched-decode routes), prefill_<kind> btl_linear_i8_op at M=--prefill-m
    (the GEMM alone), kind one of qkv, o, gate_up, down (the Llama-3-8B calls of a
    layer).  The copy reads and writes 256 MiB per dispatch and calibrates the
    memory counters.  Prints what ran."""
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    bl.check(bl.lib.btl_init(0))
    gen = torch.Generator(device=dev)
    gen.manual_seed(0xB17EB17E)
    stream = torch.cuda.current_stream().cuda_stream
    phase, kind = args.probe.split("_", 1)
    shp = PROBE_KINDS[kind]
    k = shp[0][1]
    ws = [synth_packed(n, kk, gen, dev) for (n, kk) in shp]
    m = 1 if phase == "decode" else (int(phase[7:]) if phase.startswith("batched") else args.prefill_m)
    x = synth_act(m, k, gen, dev)
    outs = [torch.empty((m, n), dtype=torch.bfloat16, device=dev) for (n, _) in shp]
    if phase == "decode" or phase.startswith("batched"):
        call = Call(ws, x, outs)
        what = "btl_linear_group %s, M=%d, %d -> %s, bf16 (%s route)" % (
            kind, m, k, "+".join(str(n) for n, _ in shp), "decode" if m == 1 else "batched-decode")
    else:
        q, s = bl.quantize_act_op(x)
        call = OpCall(ws, q, s, outs)
        what = "btl_linear_i8_op %s, M=%d, %d -> %s, bf16 (k_gemm_i8)" % (kind, m, k, "+".join(str(n) for n, _ in shp))
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(7)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(args.steps):
        call(stream)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("probe: %d x %s; 3 x copy of 268435456 bytes" % (args.steps, what), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="decode", choices=["decode"])
    ap.add_argument("--no-cpu-baseline", dest="cpu_baseline", action="store_false")
    ap.add_argument("--no-prefill", dest="prefill", action="store_false",
                    help="skip the cfg4 prefill section of the JSON line")
    ap.add_argument("--prefill-m", type=int, default=2048)
    ap.add_argument("--no-pack", dest="pack", action="store_false",
                    help="skip the device-pack (PackedTensor::pack) timing")
    ap.add_argument("--no-sweep", dest="sweep", action="store_false",
                    help="skip the cfg3 batched-decode section of the JSON line")
    ap.add_argument("--probe", default=None,
                    choices=["ceilings"] + ["%s_%s" % (p, k) for p in ("decode", "prefill") + tuple(
                        "batched%d" % m for m in (2, 4, 8, 16, 32, 64)) for k in PROBE_KINDS],
                    help="decode_<kind> / batched<M>_<kind> / prefill_<kind> (kind qkv, o, gate_up, down): "
                         "counter-run mode, --steps "
                         "launches of one workload and a 256 MiB copy, no JSON; ceilings: the decode chain's "
                         "streaming-read and launch-floor probes alone, one JSON line")
    ap.add_argument("--no-e2e", dest="e2e", action="store_false",
                    help="skip the cfg5 end-to-end decoder section of the JSON line")
    ap.add_argument("--no-cfg1", dest="cfg1", action="store_false",
                    help="skip the cfg1 section (one 2048 -> 5632 forward in both modes, CPU beside it)")
    ap.add_argument("--no-adaptive", dest="adaptive", action="store_false",
                    help="skip the multi-base adaptive-format section of the JSON line")
    ap.add_argument("--e2e-prompt", type=int, default=512)
    ap.add_argument("--e2e-tokens", type=int, default=256)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(every box here has one GPU); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X GPU", file=sys.stderr)
        sys.exit(1)
    if args.probe == "ceilings":
        dev = torch.device("cuda:0")
        torch.cuda.set_device(dev)
        print(json.dumps({"probe": "ceilings", **run_ceilings(dev, args)}), flush=True)
        return
    if args.probe:
        run_probe(args)
        return
    run_decode(args)


if __name__ == "__main__":
    main()
