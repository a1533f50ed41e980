"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle on the same
seeded inputs.  Bar: int8 activations, int32 accumulators and the int-path fp32
outputs bit-exact; reference-mode fp32 outputs bit-exact (the kernel reproduces the
8-lane order of cpu.rs); bf16 outputs equal to the oracle's f32 rounded to nearest even
(tolerance 0, tighter than the 1e-2 the task allows)."""
import os

import numpy as np
import pytest
import torch

import bitlinear as bl
from datagen import activations, random_codes, ternary, weights
from oracle import oracle as orc

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]

DEV = "cuda"


def _bits(a):
    a = np.ascontiguousarray(a, np.float32).copy()
    a[np.isnan(a)] = np.float32("nan")  # canonical NaN
    return a.view(np.uint32)


def assert_f32_identical(got, ref):
    got = got.detach().cpu().numpy() if torch.is_tensor(got) else got
    g, r = _bits(got), _bits(ref)
    bad = np.flatnonzero(g != r)
    assert bad.size == 0, "%d mismatches, first at %d: %r vs %r" % (
        bad.size, bad[0], got.reshape(-1)[bad[0]], ref.reshape(-1)[bad[0]])


def assert_bf16_matches(got, ref_f32):
    g = got.detach().cpu().view(torch.int16).numpy().view(np.uint16)
    r = orc.f32_to_bf16(ref_f32)
    bad = np.flatnonzero(g.reshape(-1) != r.reshape(-1))
    assert bad.size == 0, "%d bf16 mismatches" % bad.size


def make_layer(n, k, seed, dev=DEV):
    wb, sw = orc.pack(weights(n, k, seed))
    return bl.PackedTensor(torch.from_numpy(wb).to(dev), sw, (n, k), dev), wb, sw


def to_dev(x, dtype):
    t = torch.from_numpy(x).to(DEV)
    return t.to(dtype)


def host_x(xt):
    return xt.float().cpu().numpy()


# --- activation quantisation ----------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("m,k", [(1, 4096), (3, 1000), (16, 14336), (5, 4)])
def test_quantize_act_bitexact(dtype, m, k):
    print("quantize", dtype, m, k, flush=True)
    x = activations(m, k, seed=m * 7 + k)
    if m >= 3:
        x[1] = 0.0
        x[2, 0] = np.nan
    xt = to_dev(x, dtype)
    q, s = bl.quantize_act(xt)
    qr, sr = orc.quantize_act(host_x(xt))
    assert np.array_equal(q.cpu().numpy(), qr)
    assert_f32_identical(s, sr)


# --- W1.58-A8 linear -------------------------------------------------------------

I8_SHAPES = [
    (1, 2048, 5632),   # config 1 (TinyLlama gate/up shape)
    (1, 4096, 1024),   # Llama-3-8B k/v
    (1, 14336, 4096),  # Llama-3-8B down
    (1, 100, 37),      # k % 64 != 0: generic path
    (3, 36, 5),
    (2, 68, 130),
    (5, 320, 70),      # k % 256 != 0: partial last wave-load
    (16, 512, 200),
    (17, 256, 64),     # two 16-token tiles
    (33, 1024, 300),
]


@pytest.mark.parametrize("m,k,n", I8_SHAPES)
@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                     (torch.bfloat16, torch.float32)])
def test_linear_i8_matches_oracle(m, k, n, xdt, ydt):
    print("linear_i8", m, k, n, xdt, ydt, flush=True)
    x = activations(m, k, seed=m + k + n)
    pt, wb, sw = make_layer(n, k, seed=k * 3 + n)
    xt = to_dev(x, xdt)
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    y = bl.BitLinearHip.forward(xt, pt, mode="i8", out_dtype=ydt, acc_out=acc)
    yr, qr, sr, accr = orc.forward_i8(host_x(xt), wb, n, sw)
    assert np.array_equal(acc.cpu().numpy(), accr)
    if ydt == torch.float32:
        assert_f32_identical(y, yr)
    else:
        assert_bf16_matches(y, yr)


def test_linear_i8_special_rows():
    m, k, n = 4, 4096, 256
    x = activations(m, k, seed=3)
    x[1] = 0.0
    x[2, 5] = np.inf
    x[3] *= np.float32(1e-35)
    pt, wb, sw = make_layer(n, k, seed=4)
    y = bl.BitLinearHip.forward(to_dev(x, torch.float32), pt, mode="i8")
    yr, _, _, _ = orc.forward_i8(x, wb, n, sw)
    assert_f32_identical(y, yr)
    assert np.all(np.isnan(y[2].cpu().numpy()))
    assert np.all(y[1].cpu().numpy() == 0)


@pytest.mark.parametrize("k,parts", [(4096, "2"), (4096, "3"), (4096, "4"), (4096, "16"), (1024, "1"),
                                     (1024, "4"), (320, "1"), (14336, "7"), (14336, "8"), (14336, "14")])
@pytest.mark.parametrize("m", [1, 2, 4])
def test_decode_k_parts_are_exact(parts, k, m, tune):
    # a decode workgroup: 4 / parts row blocks (when parts divides 4), each
    # split into `parts` K parts summed through LDS; n = 330 leaves a partial
    # row block and a workgroup with row blocks past the end.  Shapes whose
    # tokens do not fit the prologue take the batched route instead.  One
    # token row takes the K-part form here only with the row-contiguous form
    # switched off.
    n = 330
    x = activations(m, k, seed=11)
    pt, wb, sw = make_layer(n, k, seed=12)
    tune("BTL_GEMV_DEC_PARTS", parts)
    tune("BTL_DEC_ROW", "0")
    tune("BTL_DEC_RQ", "0")
    tune("BTL_GEMV_DEC_MAX_M", "4")
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    y = bl.BitLinearHip.forward(to_dev(x, torch.float32), pt, acc_out=acc)
    yr, _, _, accr = orc.forward_i8(x, wb, n, sw)
    assert np.array_equal(acc.cpu().numpy(), accr)
    assert_f32_identical(y, yr)


# One token row, k % 64 == 0 and 4096 <= k <= 16384: the row-contiguous decode
# form (whole rows per wave, 1 KB per load, the row's dot product as the trace
# of a 16x16 MFMA product).  k covers one chunk, two chunks with a 64-byte
# second one (only lane 0 loads), two full chunks, three of four chunks, three
# and a half (Llama-3-8B down) and four; n = 330 leaves rows past the end of
# the last row block.  rpw / rb override rows per wave and row blocks per
# workgroup (the tuning knobs); every variant must give the oracle's bits and
# those of the K-part form.
ROW_CASES = [(4096, None, None), (4096, "8", None), (4096, "16", None), (4096, None, "2"),
             (4160, None, None), (8192, None, None), (8192, "8", None), (12288, None, None),
             (14336, None, None), (14336, "4", None), (16384, None, None), (2048, None, None)]


@pytest.mark.parametrize("k,rpw,rb", ROW_CASES)
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_decode_row_form_exact(k, rpw, rb, xdt, tune):
    print("row form", k, rpw, rb, xdt, flush=True)
    n = 330
    x = activations(1, k, seed=k + 5)
    pt, wb, sw = make_layer(n, k, seed=k + 6)
    xt = to_dev(x, xdt)
    tune("BTL_DEC_RQ", "0")
    tune("BTL_DEC_ROW_MIN_K", "2048")
    if rpw:
        tune("BTL_DEC_ROW_RPW", rpw)
    if rb:
        tune("BTL_DEC_ROW_RB", rb)
    acc = torch.empty((1, n), dtype=torch.int32, device=DEV)
    y = bl.BitLinearHip.forward(xt, pt, out_dtype=torch.float32, acc_out=acc)
    yr, _, _, accr = orc.forward_i8(host_x(xt), wb, n, sw)
    assert np.array_equal(acc.cpu().numpy(), accr)
    assert_f32_identical(y, yr)
    tune("BTL_DEC_ROW", "0")
    acc2 = torch.empty((1, n), dtype=torch.int32, device=DEV)
    y2 = bl.BitLinearHip.forward(xt, pt, out_dtype=torch.float32, acc_out=acc2)
    assert torch.equal(acc, acc2) and torch.equal(y, y2)


@pytest.mark.parametrize("form", ["rq", "row"])
@pytest.mark.parametrize("case", ["zero", "inf", "nan", "tiny", "outliers"])
def test_decode_row_form_special_rows(case, form, tune):
    # the one-token quantiser's special rows through the row-group form and
    # the row-contiguous form
    if form == "row":
        tune("BTL_DEC_RQ", "0")
    k, n = 4096, 96
    x = activations(1, k, seed=21)
    if case == "zero":
        x[:] = 0.0
    elif case == "inf":
        x[0, 17] = -np.inf
    elif case == "nan":
        x[0, 4000] = np.nan
    elif case == "tiny":
        x *= np.float32(1e-35)
    else:
        x[0, ::97] = np.float32(3.0e4)
    pt, wb, sw = make_layer(n, k, seed=22)
    acc = torch.empty((1, n), dtype=torch.int32, device=DEV)
    y = bl.BitLinearHip.forward(to_dev(x, torch.float32), pt, acc_out=acc)
    yr, _, _, accr = orc.forward_i8(x, wb, n, sw)
    assert np.array_equal(acc.cpu().numpy(), accr)
    assert_f32_identical(y, yr)


@pytest.mark.parametrize("form", ["rq", "row"])
@pytest.mark.parametrize("k", [4096, 14336])
def test_decode_row_form_group_of_ragged_layers(k, form, tune):
    # three layers of one launch whose row counts are not multiples of 16
    if form == "row":
        tune("BTL_DEC_RQ", "0")
    x = activations(1, k, seed=31)
    ns = (100, 37, 250)
    layers = [make_layer(n, k, seed=32 + n) for n in ns]
    xt = to_dev(x, torch.bfloat16)
    ys = bl.linear_group([l[0] for l in layers], xt, out_dtype=torch.float32)
    for n, (pt, wb, sw), y in zip(ns, layers, ys):
        yr, _, _, _ = orc.forward_i8(host_x(xt), wb, n, sw)
        assert_f32_identical(y, yr)


# One token row, no transform: the row-group form (R = 4 rows per wave for
# k <= 4096, else 2; one load instruction covers R rows x 1024 / R bytes; the
# rows' dot products are diagonal sums of one MFMA accumulator; only the first
# waves of a workgroup quantise).  k covers partial last slices (1088, 4160,
# 5120), every loads-per-wave count (1024..4096 -> 1..4, 6144..16384 -> 3..8)
# and k below 1024 (one partial slice); wpc overrides the compute waves per
# workgroup (1 up to 16 minus the quantising waves).  n = 330 leaves a partial row
# block and waves past the end.  Every case must give the oracle's bits and
# those of the K-part form.
RQ_CASES = [(4096, None), (4096, "1"), (4096, "5"), (4096, "14"), (1024, None), (2048, None),
            (3072, None), (1088, None), (64, None), (960, "1"), (4160, None), (5120, None),
            (6144, None), (8192, None), (10240, None), (12288, None), (14336, None), (14336, "7"),
            (14336, "9"), (16384, None)]


@pytest.mark.parametrize("dg", ["auto", "2"])
@pytest.mark.parametrize("k,wpc", RQ_CASES)
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_decode_row_group_form_exact(k, wpc, xdt, dg, tune):
    # dg "2": two token groups per quantising thread even where the launch
    # would take one (k <= 4096 and room in the workgroup)
    print("row-group form", k, wpc, xdt, dg, flush=True)
    n = 330
    x = activations(1, k, seed=k + 7)
    pt, wb, sw = make_layer(n, k, seed=k + 8)
    xt = to_dev(x, xdt)
    tune("BTL_DEC_RQ_MIN_K", "64")
    if dg == "2":
        tune("BTL_DEC_RQ_DG", "2")
    if wpc:
        tune("BTL_DEC_RQ_WPC", wpc)
    acc = torch.empty((1, n), dtype=torch.int32, device=DEV)
    y = bl.BitLinearHip.forward(xt, pt, out_dtype=torch.float32, acc_out=acc)
    yr, _, _, accr = orc.forward_i8(host_x(xt), wb, n, sw)
    assert np.array_equal(acc.cpu().numpy(), accr)
    assert_f32_identical(y, yr)
    yb = bl.BitLinearHip.forward(xt, pt, out_dtype=torch.bfloat16)
    assert_bf16_matches(yb, yr)
    tune("BTL_DEC_RQ", "0")
    tune("BTL_DEC_ROW", "0")
    acc2 = torch.empty((1, n), dtype=torch.int32, device=DEV)
    y2 = bl.BitLinearHip.forward(xt, pt, out_dtype=torch.float32, acc_out=acc2)
    assert torch.equal(acc, acc2) and torch.equal(y, y2)


# Two token rows: the row-group form with one accumulator per token row (every
# unpacked weight word feeds each row's MFMA) and a per-row absmax over the
# quantising waves (two token groups per quantising thread for k <= 4096, four
# above: R = 2 rows per compute wave, 3..8 loads); three and four rows take the
# batched route.  Every route gives the oracle's bits and those of the K-part
# form.
@pytest.mark.parametrize("m", [2, 3, 4])
@pytest.mark.parametrize("k", [1024, 1088, 2048, 3072, 4096, 4160, 6144, 8192, 12352, 14336, 16384])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_decode_row_group_form_token_rows(m, k, xdt, tune):
    print("row-group form, token rows", m, k, xdt, flush=True)
    n = 330
    x = activations(m, k, seed=m * 100 + k)
    x[m - 1, 3] = np.float32(-25.0)
    if m == 3:
        x[1] = 0.0  # a zero row among others
    pt, wb, sw = make_layer(n, k, seed=k + m)
    xt = to_dev(x, xdt)
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    y = bl.BitLinearHip.forward(xt, pt, out_dtype=torch.float32, acc_out=acc)
    yr, _, _, accr = orc.forward_i8(host_x(xt), wb, n, sw)
    assert np.array_equal(acc.cpu().numpy(), accr)
    assert_f32_identical(y, yr)
    q, s = bl.quantize_act(xt)
    acc1 = torch.empty_like(acc)
    y1 = bl.linear_i8(q, s, pt, acc_out=acc1)
    assert torch.equal(acc, acc1) and torch.equal(y, y1)
    tune("BTL_DEC_RQ", "0")
    tune("BTL_GEMV_DEC_MAX_M", "4")
    acc2 = torch.empty_like(acc)
    y2 = bl.BitLinearHip.forward(xt, pt, out_dtype=torch.float32, acc_out=acc2)
    assert torch.equal(acc, acc2) and torch.equal(y, y2)


@pytest.mark.parametrize("k", [1024, 1088, 4096])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_decode_row_group_form_two_rows_four_groups(k, xdt, tune):
    # two token rows of k <= 4096 with four token groups per quantising thread
    # (half the quantising waves, room for twice the compute waves)
    m, n = 2, 330
    x = activations(m, k, seed=k + 41)
    x[1, 5] = np.float32(30.0)
    pt, wb, sw = make_layer(n, k, seed=k + 42)
    xt = to_dev(x, xdt)
    tune("BTL_DEC_RQ_DG", "4")
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    y = bl.BitLinearHip.forward(xt, pt, out_dtype=torch.float32, acc_out=acc)
    yr, _, _, accr = orc.forward_i8(host_x(xt), wb, n, sw)
    assert np.array_equal(acc.cpu().numpy(), accr)
    assert_f32_identical(y, yr)


@pytest.mark.parametrize("k", [4096, 14336])
def test_decode_row_group_form_prequantized(k, tune):
    # int8 inputs through the row-group form: natural order (btl_linear_i8)
    # and operand order (an RMSNorm group whose transform runs as its own
    # launch), against the fused quantisation, the GEMM on the same operand-
    # order rows and the transform fused into the K-part decode kernel
    n = 200
    g = torch.from_numpy(np.random.default_rng(k).uniform(0.5, 1.5, k).astype(np.float32)).to(DEV)
    xf = to_dev(activations(1, k, seed=k + 11), torch.float32)
    pn, _, _ = make_layer(n, k, seed=k + 12)
    yf = bl.rmsnorm_linear_group([pn], xf, g, 1e-5, out_dtype=torch.float32)[0]
    tune("BTL_FUSE_DEC", "0")
    yu = bl.rmsnorm_linear_group([pn], xf, g, 1e-5, out_dtype=torch.float32)[0]
    assert torch.equal(yf, yu)
    x = to_dev(activations(1, k, seed=k + 9), torch.bfloat16)
    pt, wb, sw = make_layer(n, k, seed=k + 10)
    acc0 = torch.empty((1, n), dtype=torch.int32, device=DEV)
    y0 = bl.BitLinearHip.forward(x, pt, out_dtype=torch.float32, acc_out=acc0)
    q, s = bl.quantize_act(x)
    acc1 = torch.empty_like(acc0)
    y1 = bl.linear_i8(q, s, pt, acc_out=acc1)
    qo, so = bl.quantize_act_op(x)
    y2 = bl.linear_i8_op(qo, so, [pt])[0]
    assert torch.equal(acc0, acc1) and torch.equal(y0, y1) and torch.equal(y0, y2)
    yr, _, _, accr = orc.forward_i8(host_x(x), wb, n, sw)
    assert np.array_equal(acc0.cpu().numpy(), accr)
    assert_f32_identical(y0, yr)


# batched decode / small prefill: k_gemv_bat (m <= 64) and the GEMM, both with
# K split over workgroups.  (m, k, n): many splits; a K range past k; a half
# last GEMM step; m = 2..4 where the decode kernel does not fit k = 14336;
# exactly one 128-row tile (unsplit above 64 rows at this k); 17..32 and 33..64
# token rows (2 and 4 B blocks); above 64 rows a long K on few tiles (split,
# a half last step)
SPLIT_SHAPES = [(16, 14336, 256), (5, 4096, 300), (64, 1088, 1000), (2, 14336, 130), (4, 14336, 64),
                (128, 2048, 130), (33, 256, 64), (20, 192, 70), (48, 8192, 200), (130, 8256, 300)]


@pytest.mark.parametrize("route", ["merge", "bat", "gemm"])
@pytest.mark.parametrize("m,k,n", SPLIT_SHAPES)
@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16)])
def test_split_k_matches_oracle(m, k, n, xdt, ydt, route, tune):
    # merge: the batched kernel adding its K splits in the launch; bat: the same
    # contraction with a reduce launch after it
    print("split-k", route, m, k, n, xdt, ydt, flush=True)
    tune("BTL_GEMV_TR", 0)  # the token-register kernel has tests of its own
    if route == "gemm":
        tune("BTL_GEMV_BAT", "0")
    else:
        tune("BTL_GEMV_BAT_MAX_M", "64")  # the 33..64-row blocks too
        tune("BTL_SPLIT_MERGE", 1 if route == "merge" else 0)
    x = activations(m, k, seed=m * 5 + k + n)
    pt, wb, sw = make_layer(n, k, seed=n * 3 + k)
    xt = to_dev(x, xdt)
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    y = bl.BitLinearHip.forward(xt, pt, out_dtype=ydt, acc_out=acc)
    yr, _, _, accr = orc.forward_i8(host_x(xt), wb, n, sw)
    assert np.array_equal(acc.cpu().numpy(), accr)
    if ydt == torch.float32:
        assert_f32_identical(y, yr)
    else:
        assert_bf16_matches(y, yr)


# the token-register batched decode kernel (k_gemv_tr, 3..64 token rows): one
# K split (k <= 4096), several (k = 8192: 2, 14336: 4, merged in the launch), a
# last K segment that ends inside its 512 weights (k = 1088, 576), ragged n; 16,
# 32 and 64 token columns per wave (m = 3 / 16, 17 / 32, 33 / 64); the row blocks
# per workgroup forced to 1, 3 (a workgroup with fewer blocks than its template
# holds) and 8, or the rule (0)
TR_SHAPES = [(4096, 300), (14336, 200), (1088, 70), (576, 33), (8192, 1000)]


def tr_everywhere(tune):
    # the token-register kernel for every m in 3..64 and every k (the routing
    # rule sends it only the shapes where it measured faster)
    tune("BTL_GEMV_TR", 1)
    tune("BTL_GEMV_TR_MIN_M", 3)
    tune("BTL_GEMV_TR_MAX_M", 64)
    tune("BTL_GEMV_TR_K16", 0)


@pytest.mark.parametrize("m", [3, 16, 17, 32, 33, 64])
@pytest.mark.parametrize("k,n", TR_SHAPES)
@pytest.mark.parametrize("rbpw", [0, 1, 3, 8])
def test_token_register_kernel_matches_oracle(m, k, n, rbpw, tune):
    print("token-register", m, k, n, rbpw, flush=True)
    tr_everywhere(tune)
    tune("BTL_GEMV_TR_RBPW", rbpw)
    xdt, ydt = (torch.bfloat16, torch.bfloat16) if (m + k + rbpw) % 2 else (torch.float32, torch.float32)
    x = activations(m, k, seed=7 * m + k + n)
    pt, wb, sw = make_layer(n, k, seed=n * 5 + k)
    xt = to_dev(x, xdt)
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    y = bl.BitLinearHip.forward(xt, pt, out_dtype=ydt, acc_out=acc)
    yr, _, _, accr = orc.forward_i8(host_x(xt), wb, n, sw)
    assert np.array_equal(acc.cpu().numpy(), accr)
    if ydt == torch.float32:
        assert_f32_identical(y, yr)
    else:
        assert_bf16_matches(y, yr)


@pytest.mark.parametrize("m,k,ns", [(64, 4096, (14336, 14336)), (24, 4096, (300, 130, 4096)), (48, 14336, (4096,)),
                                    (5, 2048, (100, 2000, 50, 7))])
def test_token_register_kernel_groups(m, k, ns, tune):
    # grouped layers (row blocks of a workgroup can cross a layer boundary): every
    # output against the oracle of its own layer; the Llama-3-8B MLP shapes at m = 64
    print("token-register group", m, k, ns, flush=True)
    tr_everywhere(tune)
    xt = to_dev(activations(m, k, seed=m + 3 * k), torch.bfloat16)
    layers = [make_layer(n, k, seed=n + 11 * i) for i, n in enumerate(ns)]
    outs = bl.linear_group([l[0] for l in layers], xt, out_dtype=torch.float32)
    xh = host_x(xt)
    for (pt, wb, sw), y in zip(layers, outs):
        n = pt.shape[0]
        if n * m * k > 2e9:  # the oracle on sampled token rows
            rows = [0, m // 2, m - 1]
            assert_f32_identical(y[rows], orc.forward_i8(xh[rows], wb, n, sw)[0])
        else:
            assert_f32_identical(y, orc.forward_i8(xh, wb, n, sw)[0])


# 21..64 token rows on a layer group of at least 192 tiles of 128 rows: the
# GEMM's 64-token tiles, unsplit, 4 LDS stages (steady loop of 4 steps + tail).
# k = 1088: 9 steps, the last one half; k = 4096: 32 steps; n ragged.  Checked
# bit for bit against the 128-token tiles (BTL_GEMM_TM64 = 0, the prefill
# kernel the oracle tests pin) and, on the smaller shape, against the oracle.
@pytest.mark.parametrize("m,k,ns", [(24, 1088, (24576 + 70,)), (64, 4096, (14336, 14336)), (40, 2048, (12288, 12288 + 130))])
def test_small_m_gemm_unsplit_stages(m, k, ns, tune):
    print("small-m gemm", m, k, ns, flush=True)
    tune("BTL_GEMV_TR", 0)
    x = to_dev(activations(m, k, seed=m + k), torch.bfloat16)
    layers = [make_layer(n, k, seed=n + 7 * i) for i, n in enumerate(ns)]

    def run():
        if len(ns) == 1:  # one layer: the int32 sums too
            acc = torch.empty((m, ns[0]), dtype=torch.int32, device=DEV)
            return [bl.BitLinearHip.forward(x, layers[0][0], out_dtype=torch.float32, acc_out=acc)], [acc]
        return bl.linear_group([l[0] for l in layers], x, out_dtype=torch.float32), []

    got, accs = run()
    tune("BTL_GEMM_TM64", 0)
    ref, accs0 = run()
    for y, y0 in zip(got, ref):
        assert torch.equal(y, y0)
    for a, a0 in zip(accs, accs0):
        assert torch.equal(a, a0)
    if len(ns) == 1:
        pt, wb, sw = layers[0]
        yr, _, _, accr = orc.forward_i8(host_x(x), wb, ns[0], sw)
        assert np.array_equal(accs[0].cpu().numpy(), accr)
        assert_f32_identical(got[0], yr)


# the 64-token tiles with a K split: 256-row tiles (2 stages by the rule, 4
# forced), and the 128-row tile forced; every form against the 128-token tiles
@pytest.mark.parametrize("m,k,n", [(48, 14336, 4096), (64, 1088, 1000), (33, 8192, 200)])
@pytest.mark.parametrize("stages,tile", [(0, 0), (4, 0), (2, 1), (4, 1)])
def test_small_m_gemm_split_forms(m, k, n, stages, tile, tune):
    print("small-m gemm split", m, k, n, stages, tile, flush=True)
    tune("BTL_GEMV_BAT", 0)
    tune("BTL_GEMV_TR", 0)
    x = to_dev(activations(m, k, seed=3 * m + k), torch.bfloat16)
    pt, wb, sw = make_layer(n, k, seed=n + k)
    tune("BTL_GEMM_TM64", 0)
    acc0 = torch.empty((m, n), dtype=torch.int32, device=DEV)
    y0 = bl.BitLinearHip.forward(x, pt, out_dtype=torch.float32, acc_out=acc0)
    tune("BTL_GEMM_TM64", 1)
    tune("BTL_GEMM_TM64_STAGES", stages)
    tune("BTL_GEMM_TILE", tile)
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    y = bl.BitLinearHip.forward(x, pt, out_dtype=torch.float32, acc_out=acc)
    assert torch.equal(acc, acc0)
    assert torch.equal(y, y0)


# the prefill GEMM's 128-row tiles with 2 and 3 LDS stages (2 x 2 waves, and 1 x 4
# waves of 128 tokens x 32 rows), and its 256-row tiles with 2 (the form the M = 2048
# gate|up launch takes) and 4 (a forced 3 takes 4: the 256-row tile has no 3-stage
# form): k = 1088 (9 steps, the last one half:
# unrolled rounds and a tail), k = 4096, k = 8256 (64.5 steps); ragged m and n;
# one split launch (m = 130 x 300 rows has few tiles)
@pytest.mark.parametrize("m,k,n", [(256, 1088, 1000), (130, 4096, 300), (300, 2048, 2560), (200, 8256, 700)])
def test_prefill_gemm_stages(m, k, n, tune):
    print("prefill gemm stages", m, k, n, flush=True)
    x = to_dev(activations(m, k, seed=m * 7 + k), torch.bfloat16)
    pt, wb, sw = make_layer(n, k, seed=n + 2 * k)
    ys, accs = [], []
    for tile, stages, form in ((1, 2, "<128,2,4,128,2>"), (1, 3, "<128,2,4,128,3>"), (2, 2, "<256,4,4,128,2>"),
                               (2, 3, "<256,4,4,128,4>"), (2, 4, "<256,4,4,128,4>"), (3, 2, "<128,4,4,128,2>"),
                               (3, 3, "<128,4,4,128,3>")):
        tune("BTL_GEMM_TILE", tile)
        tune("BTL_GEMM_STAGES", stages)
        acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
        ys.append(bl.BitLinearHip.forward(x, pt, out_dtype=torch.float32, acc_out=acc))
        assert bl.lib.btl_last_gemm_form().decode() == "k_gemm_i8" + form
        accs.append(acc)
    for a, y in zip(accs[1:], ys[1:]):
        assert torch.equal(accs[0], a) and torch.equal(ys[0], y)
    yr, _, _, accr = orc.forward_i8(host_x(x), wb, n, sw)
    assert np.array_equal(accs[1].cpu().numpy(), accr)
    assert_f32_identical(ys[1], yr)


@pytest.mark.parametrize("m,k,ns", [(20, 2048, (100, 64, 64)), (7, 14336, (300, 64)), (64, 4096, (1000, 200, 200))])
def test_split_k_group_with_exact_caller_workspace(m, k, ns):
    # a group's layers share one split-K launch; btl_workspace_bytes(m, sum n, k)
    # is enough for it
    x = to_dev(activations(m, k, seed=77), torch.bfloat16)
    layers = [make_layer(n, k, seed=n + i) for i, n in enumerate(ns)]
    ws = bl.Workspace(m, sum(ns), k, device=DEV)
    ws.buf.fill_(0x5A)
    outs = bl.linear_group([l[0] for l in layers], x, out_dtype=torch.float32, workspace=ws)
    for (pt, wb, sw), n, y in zip(layers, ns, outs):
        yr, _, _, _ = orc.forward_i8(host_x(x), wb, n, sw)
        assert_f32_identical(y, yr)


def test_caller_workspace_contents_do_not_matter():
    m, k, n = 40, 4096, 1000
    x = to_dev(activations(m, k, seed=1), torch.bfloat16)
    pt, wb, sw = make_layer(n, k, seed=2)
    ws = bl.Workspace(m, n, k, device=DEV)
    y1 = bl.BitLinearHip.forward(x, pt, workspace=ws)
    ws.buf.fill_(0xA5)
    y2 = bl.BitLinearHip.forward(x, pt, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    yr, _, _, _ = orc.forward_i8(host_x(x), wb, n, sw)
    assert_bf16_matches(y1, yr)


@pytest.mark.parametrize("use_caller_ws", [False, True])
def test_workspace_shared_across_shapes(use_caller_ws):
    # scratch users (ragged k, m > 16, prefill) and fused-prologue calls share
    # one workspace, which holds the previous call's bytes (or garbage)
    ws = bl.Workspace(300, 2048, 4096, device=DEV) if use_caller_ws else None
    for (m, k, n) in [(2, 68, 130), (40, 1024, 300), (16, 512, 200), (3, 36, 500), (16, 4096, 2048),
                      (300, 1024, 130), (33, 256, 64), (1, 4096, 1024), (130, 128, 70)]:
        x = activations(m, k, seed=m * k + n)
        pt, wb, sw = make_layer(n, k, seed=n)
        acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
        if ws is not None:
            ws.buf.fill_((m * 37 + k) & 0xFF)
        y = bl.BitLinearHip.forward(to_dev(x, torch.float32), pt, acc_out=acc, workspace=ws)
        yr, _, _, accr = orc.forward_i8(x, wb, n, sw)
        assert np.array_equal(acc.cpu().numpy(), accr), (m, k, n)
        assert_f32_identical(y, yr)


def test_linear_i8_prequantized_equals_fused():
    m, k, n = 2, 2048, 5632
    x = to_dev(activations(m, k, seed=5), torch.bfloat16)
    pt, wb, sw = make_layer(n, k, seed=6)
    q, s = bl.quantize_act(x)
    acc1 = torch.empty((m, n), dtype=torch.int32, device=DEV)
    acc2 = torch.empty_like(acc1)
    y1 = bl.linear_i8(q, s, pt, acc_out=acc1)
    y2 = bl.BitLinearHip.forward(x, pt, out_dtype=torch.float32, acc_out=acc2)
    assert torch.equal(acc1, acc2)
    assert torch.equal(y1, y2)


def test_group_matches_single_layers():
    m, k = 1, 4096
    x = to_dev(activations(m, k, seed=7), torch.bfloat16)
    layers = [make_layer(n, k, seed=20 + i) for i, n in enumerate((512, 128, 192))]
    outs = bl.linear_group([l[0] for l in layers], x)
    for (pt, wb, sw), y in zip(layers, outs):
        ys = bl.BitLinearHip.forward(x, pt)
        assert torch.equal(y, ys)
        yr, _, _, _ = orc.forward_i8(host_x(x), wb, pt.shape[0], sw)
        assert_bf16_matches(y, yr)


def test_codes_3_and_extremes():
    # code 3 decodes to 0; |acc| reaches 127*K without overflow
    m, k, n = 1, 14336, 64
    wb = random_codes(n, k, seed=1, p_zero=0.2, p3=0.3)
    pt = bl.PackedTensor(torch.from_numpy(wb).to(DEV), 0.02, (n, k), DEV)
    x = np.full((m, k), -3.0, np.float32)
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    bl.BitLinearHip.forward(to_dev(x, torch.float32), pt, acc_out=acc)
    t = ternary(wb, n * k).reshape(n, k).astype(np.int64)
    assert np.array_equal(acc.cpu().numpy()[0], (-127 * t.sum(axis=1)).astype(np.int32))


def test_large_m_sampled_rows():
    m, k, n = 256, 4096, 1024
    x = to_dev(activations(m, k, seed=9), torch.bfloat16)
    pt, wb, sw = make_layer(n, k, seed=10)
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    bl.BitLinearHip.forward(x, pt, acc_out=acc)
    rows = np.random.default_rng(0).choice(m, 12, replace=False)
    xs = host_x(x)[rows]
    _, _, _, accr = orc.forward_i8(xs, wb, n, sw)
    assert np.array_equal(acc.cpu().numpy()[rows], accr)


# --- reference fp32 semantics ---------------------------------------------------------

F32_SHAPES = [(1, 2048, 5632), (3, 100, 17), (2, 36, 9), (4, 4096, 64), (1, 4, 3), (2, 8192, 8)]


@pytest.mark.parametrize("m,k,n", F32_SHAPES)
def test_linear_f32_ref_bitexact(m, k, n):
    print("f32_ref", m, k, n, flush=True)
    x = activations(m, k, seed=k + n)
    pt, wb, sw = make_layer(n, k, seed=n + 1)
    y = bl.BitLinearHip.forward(to_dev(x, torch.float32), pt, mode="f32_ref")
    assert_f32_identical(y, orc.forward_f32(x, wb, n, sw))


def test_linear_f32_ref_order_cases():
    # the lane-order / lane-sum / tail known answers of the oracle tests
    k = 36
    x = np.zeros((2, k), np.float32)
    x[0, 0], x[0, 1], x[0, 2], x[0, 8] = 2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)
    x[1, 0], x[1, 1], x[1, 2], x[1, 32] = 2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)
    codes = np.zeros(2 * k, np.uint8)
    codes[[0, 1, 2, 8, 32]] = 1
    codes[k + np.array([0, 1, 2, 8, 32])] = 1
    from datagen import pack_codes
    wb = pack_codes(codes)
    pt = bl.PackedTensor(torch.from_numpy(wb).to(DEV), 1.0, (2, k), DEV)
    y = bl.BitLinearHip.forward(to_dev(x, torch.float32), pt, mode="f32_ref").cpu().numpy()
    assert_f32_identical(y, orc.forward_f32(x, wb, 2, 1.0))


# k % 64 == 0 and k <= 16384: the LDS-staged form of the reference-order kernel
# (inputs lane-major in LDS, weight rows streamed through LDS in stages of 1024
# weights).  Inputs spanning 40 binades make every sum order-sensitive, so a
# lane or step mismatch shows; codes 3 appear; m > 1 runs two token rows per
# workgroup (odd m: the last workgroup's second row is past m); bf16 in and
# out; the three LDS sizes of x (k <= 4096, 8192, 16384), a last stage of one
# 16-byte chunk (k = 64) and of half a stage (k = 5632), several stages per
# loop trip (k = 14336); k = 16448 takes the general form.
@pytest.mark.parametrize("m,k,n", [(1, 64, 40), (3, 192, 33), (2, 4096, 70), (1, 5632, 36), (2, 8192, 40),
                                   (1, 14336, 64), (1, 16384, 24), (2, 16448, 9), (9, 4096, 40), (5, 14336, 33)])
@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16)])
def test_linear_f32_ref_staged_form(m, k, n, xdt, ydt):
    print("f32 ref staged", m, k, n, xdt, ydt, flush=True)
    rng = np.random.default_rng(m * 7 + k + n)
    x = (rng.standard_normal((m, k)) * np.exp2(rng.integers(-20, 20, (m, k)))).astype(np.float32)
    wb = random_codes(n, k, seed=k + n, p3=0.1)
    sw = np.float32(0.0173)
    pt = bl.PackedTensor(torch.from_numpy(wb).to(DEV), float(sw), (n, k), DEV)
    xt = to_dev(x, xdt)
    y = bl.BitLinearHip.forward(xt, pt, mode="f32_ref", out_dtype=ydt)
    yr = orc.forward_f32(host_x(xt), wb, n, sw)
    if ydt == torch.float32:
        assert_f32_identical(y, yr)
    else:
        assert_bf16_matches(y, yr)


# special inputs in the reference's order: subnormal inputs and partial sums
# (fma keeps them), sums that overflow to inf, inf inputs (times a zero
# coefficient: NaN) and a NaN input; staged (k % 64 == 0) and general forms
@pytest.mark.parametrize("k", [4096, 14336, 100])
def test_linear_f32_ref_special_values(k):
    print("f32 ref special", k, flush=True)
    rng = np.random.default_rng(k)
    m, n = 3, 40
    x = np.empty((m, k), np.float32)
    x[0] = rng.standard_normal(k) * 1e-39                      # subnormal
    x[1] = rng.standard_normal(k) * 3e37                       # partial sums overflow (inf, NaN)
    x[2] = rng.standard_normal(k) * 1e-3
    x[2, 5], x[2, 61], x[2, 77] = np.inf, -np.inf, np.nan
    wb = random_codes(n, k, seed=k + 3, p3=0.1)
    sw = np.float32(0.5)
    pt = bl.PackedTensor(torch.from_numpy(wb).to(DEV), float(sw), (n, k), DEV)
    y = bl.BitLinearHip.forward(to_dev(x, torch.float32), pt, mode="f32_ref").cpu().numpy()
    yr = orc.forward_f32(x, wb, n, sw)
    assert np.isnan(yr[2]).any() and not np.isfinite(yr[1]).all() and (np.abs(yr[0][yr[0] != 0]) < 1.2e-38).any()
    nan = np.isnan(yr)
    assert np.array_equal(np.isnan(y), nan)
    assert_f32_identical(np.where(nan, 0, y).astype(np.float32), np.where(nan, 0, yr).astype(np.float32))


def test_linear_f32_ref_reference_bench_input():
    # bench_cpu_kernel.rs:33,47,50 at a reduced N: y[n] = 0.5 * sum_k t[n,k]
    k, n = 8192, 512
    wb = (np.arange(n * k // 4) % 255).astype(np.uint8)
    pt = bl.PackedTensor(torch.from_numpy(wb).to(DEV), 1.0, (n, k), DEV)
    y = bl.BitLinearHip.forward(torch.full((1, k), 0.5, device=DEV), pt, mode="f32_ref")
    t = ternary(wb, n * k).reshape(n, k).astype(np.int64)
    assert np.array_equal(y.cpu().numpy()[0].astype(np.float64), 0.5 * t.sum(axis=1))


# --- PackedTensor / BitLinear host mirror on the GPU ------------------------------------

def test_unpack_device_matches_host():
    pt, wb, sw = make_layer(37, 100, seed=3)
    dense = pt.unpack("cpu").numpy().reshape(-1)
    assert_f32_identical(dense, orc.unpack(wb, 3700, sw))


def test_bitlinear_layer_forward():
    w = torch.from_numpy(weights(96, 256, seed=4))
    layer = bl.BitLinear.load(256, 96, w, device=DEV)
    layer.precompute_packed()
    x = to_dev(activations(6, 256, seed=5), torch.float32).reshape(2, 3, 256)
    y = layer.forward(x)
    assert tuple(y.shape) == (2, 3, 96)
    wb, sw = orc.pack(w.numpy())
    yr, _, _, _ = orc.forward_i8(x.reshape(6, 256).cpu().numpy(), wb, 96, sw)
    assert_f32_identical(y.reshape(6, 96), yr)
    y_ref = layer.forward(x, mode="f32_ref")
    assert_f32_identical(y_ref.reshape(6, 96), orc.forward_f32(x.reshape(6, 256).cpu().numpy(), wb, 96, sw))


def test_shape_mismatch_raises_on_gpu():
    pt, _, _ = make_layer(8, 64, seed=1)
    with pytest.raises(bl.BitLinearError, match=r"Shape mismatch: Input \[1, 60\] vs Weight \[8, 64\]"):
        bl.BitLinearHip.forward(torch.zeros((1, 60), device=DEV), pt)


# --- prefill GEMM (many token rows) -------------------------------------------------

# k % 128 == 64 (a half last K step), ragged token / output tiles, exact tiles, long k
GEMM_SHAPES = [(65, 64, 100), (300, 320, 128), (129, 4096, 1000), (257, 1024, 130),
               (300, 1088, 257), (128, 192, 128), (131, 14336, 64)]


@pytest.mark.parametrize("m,k,n", GEMM_SHAPES)
@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16)])
def test_gemm_matches_oracle(m, k, n, xdt, ydt):
    print("gemm", m, k, n, xdt, ydt, flush=True)
    x = activations(m, k, seed=m * 3 + k + n)
    x[min(5, m - 1)] = 0.0
    pt, wb, sw = make_layer(n, k, seed=n * 7 + k)
    xt = to_dev(x, xdt)
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    y = bl.BitLinearHip.forward(xt, pt, out_dtype=ydt, acc_out=acc)
    yr, _, _, accr = orc.forward_i8(host_x(xt), wb, n, sw)
    assert np.array_equal(acc.cpu().numpy(), accr)
    if ydt == torch.float32:
        assert_f32_identical(y, yr)
    else:
        assert_bf16_matches(y, yr)


# Tiles of 256 output rows (1 x 4 waves of 128 x 64; chosen for launches of
# >= 512 such workgroups, forced here) and the whole-tile epilogue of both tile
# widths: ragged m / n / k (a half last K step), exact multiples, a group of
# layers whose tiles start mid-way through the launch.
WIDE_SHAPES = [(300, 1088, 257), (129, 4096, 1000), (256, 512, 512), (384, 1024, 768), (128, 192, 256),
               (131, 14336, 64)]


@pytest.mark.parametrize("tile", ["wide", "narrow"])
@pytest.mark.parametrize("m,k,n", WIDE_SHAPES)
@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16)])
def test_gemm_tile_widths_match_oracle(m, k, n, xdt, ydt, tile, tune):
    # narrow: 128-row tiles of 2 x 2 waves (64 x 64 each)
    print("gemm tiles", m, k, n, xdt, ydt, tile, flush=True)
    tune("BTL_GEMM_MAX_SPLITS", "1")
    tune("BTL_GEMM_WIDE_MIN_TILES", "1" if tile == "wide" else "1000000000")
    x = activations(m, k, seed=m + k * 5 + n)
    x[min(7, m - 1)] = 0.0
    pt, wb, sw = make_layer(n, k, seed=n * 11 + k)
    xt = to_dev(x, xdt)
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    y = bl.BitLinearHip.forward(xt, pt, out_dtype=ydt, acc_out=acc)
    yr, _, _, accr = orc.forward_i8(host_x(xt), wb, n, sw)
    assert np.array_equal(acc.cpu().numpy(), accr)
    if ydt == torch.float32:
        assert_f32_identical(y, yr)
    else:
        assert_bf16_matches(y, yr)


def test_gemm_wide_tiles_group_of_layers(tune):
    tune("BTL_GEMM_MAX_SPLITS", "1")
    tune("BTL_GEMM_WIDE_MIN_TILES", "1")
    m, k, ns = 256, 1024, (300, 512, 70)
    x = activations(m, k, seed=77)
    layers = [make_layer(n, k, seed=78 + n) for n in ns]
    xt = to_dev(x, torch.bfloat16)
    ys = bl.linear_group([l[0] for l in layers], xt, out_dtype=torch.float32)
    for n, (pt, wb, sw), y in zip(ns, layers, ys):
        yr, _, _, _ = orc.forward_i8(host_x(xt), wb, n, sw)
        assert_f32_identical(y, yr)


@pytest.mark.parametrize("m,k,n", [(200, 512, 96), (130, 1088, 200)])
def test_gemm_prequantized_natural_layout(m, k, n):
    # btl_linear_i8 hands the GEMM natural-order int8 rows
    x = to_dev(activations(m, k, seed=21 + k), torch.bfloat16)
    pt, wb, sw = make_layer(n, k, seed=22)
    q, s = bl.quantize_act(x)
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    y = bl.linear_i8(q, s, pt, acc_out=acc)
    yr, _, _, accr = orc.forward_i8(host_x(x), wb, n, sw)
    assert np.array_equal(acc.cpu().numpy(), accr)
    assert_f32_identical(y, yr)


OP_PERM = np.array([0, 4, 8, 12, 1, 5, 9, 13, 2, 6, 10, 14, 3, 7, 11, 15])


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_quantize_act_op_is_a_reordering(xdt):
    m, k = 37, 1088
    x = to_dev(activations(m, k, seed=41), xdt)
    x[3] = 0.0
    qo, so = bl.quantize_act_op(x)
    q, s = bl.quantize_act(x)
    assert torch.equal(so, s)
    qo = qo.cpu().numpy().reshape(m, k // 16, 16)
    assert np.array_equal(qo, q.cpu().numpy().reshape(m, k // 16, 16)[:, :, OP_PERM])
    _, qr, sr, _ = orc.forward_i8(host_x(x), make_layer(16, k, seed=1)[1], 16, 1.0)
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(s.cpu().numpy(), sr)


@pytest.mark.parametrize("m,k,ns", [(300, 1088, (130, 64, 64)), (129, 256, (256,)), (70, 4096, (100, 1000))])
def test_linear_i8_op_group_matches_oracle(m, k, ns):
    x = to_dev(activations(m, k, seed=m + k), torch.bfloat16)
    layers = [make_layer(n, k, seed=n * 5 + i) for i, n in enumerate(ns)]
    q, s = bl.quantize_act_op(x)
    accs = [torch.empty((m, n), dtype=torch.int32, device=DEV) for n in ns]
    ys = bl.linear_i8_op(q, s, [l[0] for l in layers], out_dtype=torch.bfloat16, acc_out=accs)
    # the grouped entry of the fused path gives the same bytes
    yg = bl.linear_group([l[0] for l in layers], x, out_dtype=torch.bfloat16)
    for (pt, wb, sw), n, y, acc, g in zip(layers, ns, ys, accs, yg):
        yr, _, _, accr = orc.forward_i8(host_x(x), wb, n, sw)
        assert np.array_equal(acc.cpu().numpy(), accr)
        assert_bf16_matches(y, yr)
        assert torch.equal(y, g)


def test_gemm_prefill_shape_sampled_rows():
    # config 4 shape class: M = 2048 tokens, q-proj 4096 -> 4096
    m, k, n = 2048, 4096, 4096
    x = to_dev(activations(m, k, seed=31), torch.bfloat16)
    pt, wb, sw = make_layer(n, k, seed=32)
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    y = bl.BitLinearHip.forward(x, pt, acc_out=acc)
    rows = np.random.default_rng(1).choice(m, 6, replace=False)
    rows = np.concatenate([rows, [0, 255, 256, 2047]])
    yr, _, _, accr = orc.forward_i8(host_x(x)[rows], wb, n, sw)
    assert np.array_equal(acc.cpu().numpy()[rows], accr)
    assert_bf16_matches(y[rows], yr)
    # cross-path property: the decode kernel on single rows gives the same accumulators
    acc1 = torch.empty((1, n), dtype=torch.int32, device=DEV)
    for r in (0, 1000, 2047):
        bl.BitLinearHip.forward(x[r:r + 1].contiguous(), pt, acc_out=acc1)
        assert torch.equal(acc1[0], acc[r])


# --- fused RMSNorm / SwiGLU ahead of the contraction ----------------------------

def _rms_reference(x, g, eps, layers):
    xn = orc.rmsnorm(x, g, eps)
    return [orc.forward_i8(xn, wb, pt.dims2()[0], sw)[0] for (pt, wb, sw) in layers]


# decode (m <= 4), batched (5..32), GEMM (> 32); k from one MFMA step to 2 groups per thread
FUSED_SHAPES = [(1, 4096, (256, 64, 64)), (2, 1024, (300,)), (4, 4096, (130,)), (7, 2048, (200, 100)),
                (32, 4096, (64,)), (65, 1024, (300,)), (300, 4096, (128,)), (3, 64, (80,)), (1, 16384, (64,)),
                (2, 32768, (32,))]


@pytest.mark.parametrize("m,k,ns", FUSED_SHAPES)
@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16)])
def test_rmsnorm_linear_group_matches_oracle(m, k, ns, xdt, ydt):
    print("rmsnorm", m, k, ns, xdt, ydt, flush=True)
    rng = np.random.default_rng(m * 7 + k)
    x = (rng.standard_normal((m, k)) * rng.uniform(0.2, 40, (m, 1))).astype(np.float32)
    x[m // 2, : k // 3] = 0.0
    g = rng.uniform(0.5, 1.5, k).astype(np.float32)
    eps = 1e-5
    layers = [make_layer(n, k, seed=n * 11 + i) for i, n in enumerate(ns)]
    xt = to_dev(x, xdt)
    ys = bl.rmsnorm_linear_group([l[0] for l in layers], xt, torch.from_numpy(g), eps, out_dtype=ydt)
    refs = _rms_reference(host_x(xt), g, eps, layers)
    for y, yr in zip(ys, refs):
        if ydt == torch.float32:
            assert_f32_identical(y, yr)
        else:
            assert_bf16_matches(y, yr)


def test_rmsnorm_many_rows_exercise_the_sqrt():
    # 256 rows whose mean squares span many binades: the per-row sqrt must be
    # correctly rounded (the hardware sqrt is not) for the scales to match
    m, k, n = 256, 64, 48
    rng = np.random.default_rng(21)
    x = (rng.standard_normal((m, k)) * np.exp(rng.uniform(-12, 12, (m, 1)))).astype(np.float32)
    g = rng.uniform(0.5, 1.5, k).astype(np.float32)
    pt, wb, sw = make_layer(n, k, seed=5)
    y = bl.rmsnorm_linear_group([pt], to_dev(x, torch.float32), torch.from_numpy(g), 1e-6,
                                out_dtype=torch.float32)[0]
    assert_f32_identical(y, _rms_reference(x, g, 1e-6, [(pt, wb, sw)])[0])


def test_rmsnorm_special_rows():
    # zero row (0 / sqrt(eps) = 0 -> scale 0), an inf row (non-finite -> NaN),
    # huge and tiny magnitudes; eps = 0 on a zero row gives 0/0 = NaN
    m, k, n = 4, 1024, 96
    x = np.random.default_rng(9).standard_normal((m, k)).astype(np.float32)
    x[0] = 0.0
    x[1, 5] = np.inf
    x[2] *= np.float32(1e30)
    x[3] *= np.float32(1e-30)
    g = np.ones(k, np.float32)
    pt, wb, sw = make_layer(n, k, seed=4)
    for eps in (1e-5, 0.0):
        y = bl.rmsnorm_linear_group([pt], to_dev(x, torch.float32), torch.from_numpy(g), eps,
                                    out_dtype=torch.float32)[0]
        yr = _rms_reference(x, g, eps, [(pt, wb, sw)])[0]
        assert_f32_identical(y, yr)


@pytest.mark.parametrize("m,k,ns", [(1, 14336, (4096,)), (2, 14336, (300,)), (4, 4096, (130, 64)),
                                    (16, 14336, (256,)), (64, 4096, (200,)), (130, 1024, (100,)),
                                    (3, 64, (80,)), (1, 32768, (64,))])
@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16)])
def test_swiglu_linear_group_matches_oracle(m, k, ns, xdt, ydt):
    print("swiglu", m, k, ns, xdt, ydt, flush=True)
    rng = np.random.default_rng(m * 13 + k)
    gate = (rng.standard_normal((m, k)) * 3).astype(np.float32)
    up = rng.standard_normal((m, k)).astype(np.float32)
    gate[0, :7] = np.array([0, -0.0, 90, -90, 200, -200, 1e-30], np.float32)
    layers = [make_layer(n, k, seed=n * 3 + i) for i, n in enumerate(ns)]
    gt, ut = to_dev(gate, xdt), to_dev(up, xdt)
    ys = bl.swiglu_linear_group([l[0] for l in layers], gt, ut, out_dtype=ydt)
    h = orc.swiglu(host_x(gt), host_x(ut))
    for y, (pt, wb, sw) in zip(ys, layers):
        yr = orc.forward_i8(h, wb, pt.dims2()[0], sw)[0]
        if ydt == torch.float32:
            assert_f32_identical(y, yr)
        else:
            assert_bf16_matches(y, yr)


def test_fused_with_caller_workspace_and_graph_replays():
    # caller workspace of exactly btl_workspace_bytes, garbage between calls,
    # and the same calls captured in a HIP graph and replayed
    m, k, n = 6, 4096, 512
    rng = np.random.default_rng(12)
    x = rng.standard_normal((m, k)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, k).astype(np.float32)
    pt, wb, sw = make_layer(n, k, seed=8)
    ws = bl.Workspace(m, n, k, device=DEV)
    ws.buf.fill_(0x77)
    xt = to_dev(x, torch.bfloat16)
    gt = torch.from_numpy(g).to(DEV)
    out = [torch.empty((m, n), dtype=torch.float32, device=DEV)]
    bl.rmsnorm_linear_group([pt], xt, gt, 1e-5, workspace=ws, outputs=out)
    torch.cuda.synchronize()
    yr = _rms_reference(host_x(xt), g, 1e-5, [(pt, wb, sw)])[0]
    assert_f32_identical(out[0], yr)
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            bl.rmsnorm_linear_group([pt], xt, gt, 1e-5, workspace=ws, outputs=out)
    for _ in range(3):
        out[0].zero_()
        ws.buf.fill_(0x33)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert_f32_identical(out[0], yr)


def test_library_workspace_growth_keeps_captured_graph_valid():
    # a call on the library's own workspace (ws = NULL) captured in a HIP graph, then
    # calls that need a larger library workspace: it is replaced and the old one
    # retired (never freed), so every replay, with eager work between the replays,
    # still gives the oracle's bits.  Growth while capturing fails cleanly.
    print("workspace growth under capture", flush=True)
    m, k, n = 6, 4096, 512
    x = activations(m, k, seed=31)
    pt, wb, sw = make_layer(n, k, seed=32)
    xt = to_dev(x, torch.float32)
    out = [torch.empty((m, n), dtype=torch.float32, device=DEV)]
    bl.linear_group([pt], xt, outputs=out)
    torch.cuda.synchronize()
    yr, _, _, _ = orc.forward_i8(x, wb, n, sw)
    assert_f32_identical(out[0], yr)
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            bl.linear_group([pt], xt, outputs=out)
    for i, (mb, kb, nb) in enumerate([(1024, 4096, 64), (2048, 8192, 64)]):
        xb = activations(mb, kb, seed=40 + i)
        pb, wbb, swb = make_layer(nb, kb, seed=50 + i)
        yb = bl.BitLinearHip.forward(to_dev(xb, torch.float32), pb)
        out[0].zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert_f32_identical(out[0], yr)
        ybr, _, _, _ = orc.forward_i8(xb, wbb, nb, swb)
        assert_f32_identical(yb, ybr)
    big = torch.zeros((4096, 16384), dtype=torch.float32, device=DEV)
    pbig, _, _ = make_layer(64, 16384, seed=60)
    g2 = torch.cuda.CUDAGraph()
    with pytest.raises(bl.BitLinearError) as ei:
        with torch.cuda.stream(s):
            with torch.cuda.graph(g2, stream=s):
                bl.BitLinearHip.forward(big, pbig)
    assert ei.value.status == bl.BTL_ERR_WORKSPACE
    torch.cuda.synchronize()
    bl.check_faults()
    graph.replay()
    torch.cuda.synchronize()
    assert_f32_identical(out[0], yr)


def test_wait_that_gives_up_is_reported(tune):
    # the one-token decode kernel's LDS waits bounded by BTL_WAIT_SPIN polls: with a
    # bound of 0 every wait gives up at once (the kernel still finishes, its output is
    # not valid) and btl_check_faults reports it; the default bound gives the exact
    # result and a clean check
    print("wait bound fault word", flush=True)
    k, n = 4096, 1024
    x = activations(1, k, seed=70)
    pt, wb, sw = make_layer(n, k, seed=71)
    xt = to_dev(x, torch.float32)
    bl.check_faults()
    tune("BTL_WAIT_SPIN", 0)
    bl.BitLinearHip.forward(xt, pt)
    with pytest.raises(bl.BitLinearError) as ei:
        bl.check_faults()
    assert ei.value.status == bl.BTL_ERR_FAULT
    assert "token row" in str(ei.value)
    bl.check_faults()  # cleared by the read
    tune("BTL_WAIT_SPIN", 1 << 22)
    y = bl.BitLinearHip.forward(xt, pt)
    bl.check_faults()
    yr, _, _, _ = orc.forward_i8(x, wb, n, sw)
    assert_f32_identical(y, yr)


# --- PackedTensor::pack on the device ---------------------------------------------

@pytest.mark.parametrize("shape", [(1, 4), (3, 5), (17, 33), (300, 4096), (4096, 14336)])
def test_pack_device_equals_pack_host(shape):
    print("pack_device", shape, flush=True)
    rng = np.random.default_rng(shape[0] + shape[1])
    w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    if w.size > 8:
        w.reshape(-1)[:4] = 0.0
    host = bl.PackedTensor.pack(torch.from_numpy(w))
    dev = bl.PackedTensor.pack_device(torch.from_numpy(w).to(DEV))
    assert np.float32(dev.scale).view(np.uint32) == np.float32(host.scale).view(np.uint32)
    assert torch.equal(dev.data.cpu(), host.data)
    if w.size <= 300 * 4096:
        wb, sw = orc.pack(w)
        assert np.array_equal(host.data.numpy(), wb) and np.float32(sw) == np.float32(host.scale)


def test_pack_device_clamps_and_zeros():
    # |w / s| beyond 1.5 clamps to +-1, small values go to 0 (exact ties: test_golden.py)
    w = np.array([[2.0, -2.0, 1.0, -1.0, 0.0, 6.0, -6.0, 4.0]], np.float32)
    host = bl.PackedTensor.pack(torch.from_numpy(w))
    dev = bl.PackedTensor.pack_device(torch.from_numpy(w).to(DEV))
    assert torch.equal(dev.data.cpu(), host.data) and dev.scale == host.scale
    wb, sw = orc.pack(w)
    assert np.array_equal(host.data.numpy(), wb)


# btl_linear_group_mode in the reference's fp32 order: the layers of one launch
# (and the per-layer fallback for k % 64 != 0) bit for bit with the oracle
@pytest.mark.parametrize("m,k,ns,xdt", [(1, 4096, (4096, 1024, 1024), torch.float32),
                                        (1, 4096, (14336, 14336), torch.bfloat16),
                                        (3, 512, (96, 40, 33, 7), torch.float32), (2, 100, (17, 9), torch.float32)])
def test_group_f32_ref_bitexact(m, k, ns, xdt):
    print("group f32_ref", m, k, ns, flush=True)
    rng = np.random.default_rng(m + k + len(ns))
    x = (rng.standard_normal((m, k)) * np.exp2(rng.integers(-10, 10, (m, k)))).astype(np.float32)
    xt = to_dev(x, xdt)
    layers = []
    for i, n in enumerate(ns):
        wb = random_codes(n, k, seed=31 * i + n, p3=0.1)
        layers.append((bl.PackedTensor(torch.from_numpy(wb).to(DEV), 0.01 * (i + 1), (n, k), DEV), wb))
    outs = bl.linear_group([l[0] for l in layers], xt, out_dtype=torch.float32, mode="f32_ref")
    for (pt, wb), y in zip(layers, outs):
        assert_f32_identical(y, orc.forward_f32(host_x(xt), wb, pt.shape[0], np.float32(pt.scale)))
        assert torch.equal(y, bl.BitLinearHip.forward(xt, pt, mode="f32_ref", out_dtype=torch.float32))


@pytest.mark.parametrize("kernel", ["bat", "tr"])
def test_batched_merge_counters_and_graph_replays(kernel, tune):
    # the in-launch split merge keeps its counters per workspace and every launch
    # leaves them at zero: calls of different m and K splits on one workspace, then
    # a captured call replayed with eager calls in between, all bit for bit
    # (k_gemv_bat, or the token-register kernel: 4 K splits at k = 14336)
    print("split merge counters / graph", kernel, flush=True)
    if kernel == "tr":
        tr_everywhere(tune)
    else:
        tune("BTL_GEMV_TR", 0)
    tune("BTL_GEMV_BAT_MAX_M", "64")
    tune("BTL_SPLIT_MERGE", 1)
    k, n = 14336, 384
    pt, wb, sw = make_layer(n, k, seed=90)
    ws = bl.Workspace(64, n, k, device=DEV)
    xs = {m: to_dev(activations(m, k, seed=91 + m), torch.bfloat16) for m in (3, 16, 40, 64)}
    ref = {m: orc.forward_i8(host_x(x), wb, n, sw)[0] for m, x in xs.items()}
    for m in (3, 16, 40, 64, 16, 3):
        assert_f32_identical(bl.BitLinearHip.forward(xs[m], pt, out_dtype=torch.float32, workspace=ws), ref[m])
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            y = bl.BitLinearHip.forward(xs[16], pt, out_dtype=torch.float32, workspace=ws)
    torch.cuda.synchronize()
    for i in range(3):
        y.fill_(-1.0)
        g.replay()
        torch.cuda.synchronize()
        assert_f32_identical(y, ref[16])
        assert_f32_identical(bl.BitLinearHip.forward(xs[40], pt, out_dtype=torch.float32, workspace=ws), ref[40])
