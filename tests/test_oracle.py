"""Pins the CPU oracle (oracle/bitlinear_oracle.c) before anything is checked against it.

What pins each oracle function (reference = imonoonoko/Bit-TTT-Engine, crates/rust_engine):
  orc_pack / orc_unpack   the reference's own unit tests, restated with their inputs and
                          tolerances (kernels/packing.rs:155-261); exhaustive 256-byte decode
                          table against the closed form (c&1)-(c>>1) (cpu.rs:161-166); the
                          half-away tie at |w/s| = 0.5; float64 semantic invariants.
                          The last ulp of the scale (candle's mean_all order) is parity unpinned.
  orc_forward_f32         integer-valued inputs (every partial sum exact) against numpy int64;
                          the reference bench's known input (bench_cpu_kernel.rs:33,47,50);
                          hand-built cases whose result depends on the lane order, the
                          sequential lane sum and the tail order (cpu.rs:105-123,192-238);
                          bit-identity with the AVX2-intrinsics restatement.
  orc_quantize_act        build-defined (no reference function): rounding-mode ties, the
                          outlier scale 20/127, zero/NaN/tiny rows, error bound |x/s - q| <= 1/2,
                          monotonicity.
  orc_contract_i8         numpy int64 matmul of the unpacked ternary matrix.
  orc_epilogue            numpy float32 arithmetic.
  bf16 helpers            torch's round-to-nearest-even bfloat16 conversion.
  orc_pairwise_sum        inputs whose float32 sum differs between the pairwise tree and a
                          sequential sum or another tree split (so only the defined order
                          passes); zero-padding invariance; exact integer sums.
  orc_expf                float64 exp rounded to float32: within 2 ulp over a dense sweep
                          of the whole range incl. subnormal results; exp(0) = 1; overflow,
                          underflow, NaN.  Rust's f32::exp (libm) is the reference's: the
                          last ulps are parity unpinned (a documented tolerance).
  orc_swiglu              float64 closed form silu(g)*u (relative 1e-6); limits.
  orc_rmsnorm             float64 closed form (relative 1e-6); a known answer; zero row;
                          the eps and weight terms; scale invariance.  Candle's own sum
                          order is not vendored: its last ulp is parity unpinned.
"""
import numpy as np
import pytest
import torch

from datagen import activations, pack_codes, random_codes, ternary, weights
from oracle import oracle as orc


# --- packing.rs tests, restated -------------------------------------------------

def test_packing_cycle_dense():
    # packing.rs:155-173
    w = np.array([1.0, -1.0, 1.0, -1.0, -1.0, 1.0, 1.0, 1.0], np.float32)
    b, s = orc.pack(w)
    assert abs(s - 1.0) < 1e-3
    np.testing.assert_allclose(orc.unpack(b, w.size, s), w, atol=1e-4, rtol=0)


def test_packing_cycle_sparse():
    # packing.rs:175-202
    w = np.array([1.0, -1.0, 0.0, 0.0, 1.0, -1.0, 0.0, 0.0], np.float32)
    b, s = orc.pack(w)
    assert abs(s - 0.5) < 1e-3
    np.testing.assert_allclose(orc.unpack(b, w.size, s), [0.5, -0.5, 0, 0, 0.5, -0.5, 0, 0], atol=1e-4, rtol=0)


def test_packing_manual():
    # packing.rs:204-233: byte 73 -> [1, -1, 0, 1]
    assert list(orc.unpack(np.array([73], np.uint8), 4, 1.0)) == [1.0, -1.0, 0.0, 1.0]


def test_packing_padding():
    # packing.rs:235-261: [1,1,1,1,-1] -> bytes [85, 2]
    w = np.array([1.0, 1.0, 1.0, 1.0, -1.0], np.float32)
    b, s = orc.pack(w)
    assert list(b) == [85, 2]
    np.testing.assert_allclose(orc.unpack(b, 5, s), w, atol=1e-4, rtol=0)


def test_decode_table_exhaustive():
    data = np.arange(256, dtype=np.uint8)
    got = orc.unpack(data, 1024, 1.0).astype(np.int8)
    assert np.array_equal(got, ternary(data, 1024))
    # code 3 (unused/padding) decodes to 0 (cpu.rs:59, packing.rs:121-123)
    assert np.all(got.reshape(256, 4)[data == 0xFF] == 0)


def test_pack_round_half_away():
    # w*inv == 0.5 exactly with s == 1.0: f32::round gives 1 (half-to-even would give 0)
    w = np.array([0.5, 1.4999979734420776], np.float32)
    b, s = orc.pack(w)
    assert s == 1.0
    assert list(b) == [0b0101]


@pytest.mark.parametrize("shape", [(64, 256), (7, 33), (1, 5), (3, 1)])
def test_pack_invariants(shape):
    w = weights(*shape, seed=11)
    b, s = orc.pack(w)
    numel = w.size
    assert b.size == (numel + 3) // 4
    ref_scale = np.abs(w.astype(np.float64)).mean() + 1e-6
    assert abs(s - ref_scale) <= 1e-6 * ref_scale
    codes = np.stack([(b >> (2 * i)) & 3 for i in range(4)], 1).reshape(-1)
    assert not np.any(codes == 3)
    assert np.all(codes[numel:] == 0)  # pad fields stay 00
    t = ternary(b, numel).astype(np.int64)
    v = w.reshape(-1).astype(np.float64) / float(s)
    clear = np.abs(np.abs(v) - 0.5) > 1e-5
    expect = np.where(v >= 0.5, 1, np.where(v <= -0.5, -1, 0))
    assert np.array_equal(t[clear], expect[clear])


def test_pack_ternary_input_roundtrip():
    rng = np.random.default_rng(3)
    t = rng.choice(np.array([-1.0, 1.0], np.float32), size=999)
    b, s = orc.pack(t)
    assert abs(s - 1.0) < 1e-5
    assert np.array_equal(ternary(b, t.size), t.astype(np.int8))


# --- cpu.rs forward, fp32 order ---------------------------------------------------

@pytest.mark.parametrize("k", [4, 8, 28, 32, 36, 64, 100, 260])
@pytest.mark.parametrize("avx2_order", [True, False])
def test_forward_f32_integer_inputs_exact(k, avx2_order):
    rng = np.random.default_rng(k)
    m, n = 3, 17
    x = rng.integers(-3, 4, size=(m, k)).astype(np.float32)
    w = random_codes(n, k, seed=k + 1, p3=0.1)
    t = ternary(w, n * k).reshape(n, k).astype(np.int64)
    for scale in (1.0, 0.25):
        y = orc.forward_f32(x, w, n, scale, avx2_order=avx2_order)
        exact = (x.astype(np.int64) @ t.T).astype(np.float64) * scale
        assert np.array_equal(y.astype(np.float64), exact)


def test_forward_f32_reference_bench_input():
    # bench_cpu_kernel.rs:33,47,50: x = 0.5, W bytes (i % 255), scale 1, M=1, K=N=8192
    k = n = 8192
    w = (np.arange(n * k // 4) % 255).astype(np.uint8)
    x = np.full((1, k), 0.5, np.float32)
    y = orc.forward_f32(x, w, n, 1.0)
    t = ternary(w, n * k).reshape(n, k).astype(np.int64)
    assert np.array_equal(y[0].astype(np.float64), 0.5 * t.sum(axis=1))


def _one_hot_codes(n, k, plus):
    codes = np.zeros(n * k, np.uint8)
    codes[list(plus)] = 1
    return pack_codes(codes)


def test_forward_f32_lane_order():
    # lane 0 gets x[0] and x[8]; lanes 1, 2 get x[1], x[2] (cpu.rs:205-220)
    k = 32
    x = np.zeros((1, k), np.float32)
    x[0, 0], x[0, 1], x[0, 2], x[0, 8] = 2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)
    w = _one_hot_codes(1, k, [0, 1, 2, 8])
    # lanes: l0 = 2^24 - 2^24 = 0, l1 = 1, l2 = 1 -> 2.  A sequential k loop gives
    # ((2^24 + 1) + 1) - 2^24 = 0 because 2^24 + 1 rounds back to 2^24.
    assert orc.forward_f32(x, w, 1, 1.0, avx2_order=True)[0, 0] == 2.0
    assert orc.forward_f32(x, w, 1, 1.0, avx2_order=False)[0, 0] == 0.0


def test_forward_f32_lane_sum_then_tail():
    # lanes 0,1,2 = 2^24, 1, 1; tail x[32] = -2^24.  Lane sum is sequential
    # (cpu.rs:236-238): ((2^24 + 1) + 1) = 2^24, then the tail (cpu.rs:105-122) -> 0.
    # Pairwise/reverse lane sums or folding the tail into the lanes give 2.
    k = 36
    x = np.zeros((1, k), np.float32)
    x[0, 0], x[0, 1], x[0, 2], x[0, 32] = 2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)
    w = _one_hot_codes(1, k, [0, 1, 2, 32])
    assert orc.forward_f32(x, w, 1, 1.0)[0, 0] == 0.0


def test_forward_f32_special_codes():
    m, k, n = 2, 64, 3
    x = np.arange(m * k, dtype=np.float32).reshape(m, k) - 50
    zero = pack_codes(np.zeros(n * k, np.uint8))
    three = pack_codes(np.full(n * k, 3, np.uint8))
    ones = pack_codes(np.ones(n * k, np.uint8))
    assert np.all(orc.forward_f32(x, zero, n, 1.5) == 0)
    assert np.all(orc.forward_f32(x, three, n, 1.5) == 0)
    y = orc.forward_f32(x, ones, n, 1.0)
    assert np.array_equal(y, np.repeat(x.sum(axis=1, keepdims=True), n, axis=1))


@pytest.mark.skipif(not orc.has_avx2(), reason="oracle built without AVX2")
@pytest.mark.parametrize("k", [32, 100, 2048, 4100])
def test_forward_f32_matches_avx2_intrinsics(k):
    m, n = 2, 129
    x = activations(m, k, seed=k)
    w = random_codes(n, k, seed=k + 7, p3=0.05)
    a = orc.forward_f32(x, w, n, 0.0173)
    b = orc.forward_f32_avx2(x, w, n, 0.0173, threads=4)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# --- W1.58-A8 path (build-defined) --------------------------------------------------

def test_quantize_rounding_ties():
    # absmax 127 -> r = 127/127 = 1 exactly, so q = round_half_away(x)
    x = np.array([[127.0, 2.5, -2.5, 0.5, -0.5, 0.49999997, 1.5, -126.5]], np.float32)
    q, s = orc.quantize_act(x)
    assert s[0] == 1.0
    assert list(q[0]) == [127, 3, -3, 1, -1, 0, 2, -127]


def test_quantize_outliers_and_special_rows():
    x = activations(4, 4096, seed=5)
    x[1] = 0.0
    x[2, 7] = np.nan
    x[3] = np.float32(1e-31)  # below 2^-100
    q, s = orc.quantize_act(x)
    assert s[0] == np.float32(20.0) / np.float32(127.0)
    assert s[1] == 0.0 and not q[1].any()
    assert np.isnan(s[2]) and not q[2].any()
    assert s[3] == 0.0 and not q[3].any()
    xi = x.copy()
    xi[0, 3] = np.inf
    q2, s2 = orc.quantize_act(xi[:1])
    assert np.isnan(s2[0]) and not q2.any()


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_quantize_properties(seed):
    x = activations(8, 1000, seed=seed, outlier_frac=0.0)
    x[3] *= 1e-20
    q, s = orc.quantize_act(x)
    a = np.abs(x).max(axis=1)
    for i in range(x.shape[0]):
        assert np.abs(q[i]).max() == 127
        assert q[i][np.argmax(np.abs(x[i]))] == np.sign(x[i][np.argmax(np.abs(x[i]))]) * 127
        err = np.abs(x[i].astype(np.float64) / float(s[i]) - q[i])
        assert err.max() <= 0.5 + 1e-4
        order = np.argsort(x[i], kind="stable")
        assert np.all(np.diff(q[i][order].astype(np.int32)) >= 0)
        assert np.all(np.sign(q[i]) * np.sign(x[i]) >= 0)
        assert s[i] == np.float32(a[i]) / np.float32(127.0)


def test_contract_matches_numpy():
    m, k, n = 5, 200, 33
    rng = np.random.default_rng(9)
    q = rng.integers(-127, 128, size=(m, k)).astype(np.int8)
    w = random_codes(n, k, seed=10, p3=0.1)
    acc = orc.contract_i8(q, w, n)
    t = ternary(w, n * k).reshape(n, k).astype(np.int64)
    assert np.array_equal(acc, (q.astype(np.int64) @ t.T).astype(np.int32))


def test_contract_extremes_no_overflow():
    k, n = 14336, 2
    q = np.full((1, k), -127, np.int8)
    w = pack_codes(np.concatenate([np.ones(k, np.uint8), np.full(k, 2, np.uint8)]))
    acc = orc.contract_i8(q, w, n)
    assert list(acc[0]) == [-127 * k, 127 * k]


def test_epilogue_float32():
    rng = np.random.default_rng(4)
    acc = rng.integers(-2_000_000, 2_000_000, size=(3, 50)).astype(np.int32)
    sx = np.array([0.1, 0.0, 17.25], np.float32)
    sw = np.float32(0.01596)
    y = orc.epilogue(acc, sx, float(sw))
    expect = acc.astype(np.float32) * (sx[:, None] * sw)
    assert np.array_equal(y.view(np.uint32), expect.astype(np.float32).view(np.uint32))


def test_forward_i8_composes():
    m, k, n = 3, 256, 40
    x = activations(m, k, seed=1)
    wb, sw = orc.pack(weights(n, k, seed=2))
    y, q, s, acc = orc.forward_i8(x, wb, n, sw)
    q2, s2 = orc.quantize_act(x)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)
    assert np.array_equal(acc, orc.contract_i8(q, wb, n))
    assert np.array_equal(y, orc.epilogue(acc, s, sw))
    # the int8 path approximates the fp32 path: rel. error well under 5%
    yf = orc.forward_f32(x, wb, n, sw)
    assert np.linalg.norm(y - yf) / np.linalg.norm(yf) < 0.05


def test_bf16_conversions_match_torch():
    rng = np.random.default_rng(8)
    f = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 100,
                        np.array([0.0, -0.0, np.inf, -np.inf, 3.0e38, 1e-40], np.float32)])
    got = orc.f32_to_bf16(f)
    ref = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    back = orc.bf16_to_f32(got)
    assert np.array_equal(back, torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16).float().numpy())
    assert orc.f32_to_bf16(np.array([np.nan], np.float32))[0] == 0x7FC0


# --- fused activation transforms (RMSNorm, SwiGLU) ------------------------------

def test_pairwise_sum_follows_the_pairwise_tree():
    # (1 + 1) + (1e8 - 1e8) = 2 in float32; a sequential sum loses the 2 in 1e8
    v4 = np.array([1, 1, 1e8, -1e8], np.float32)
    assert orc.pairwise_sum(v4) == np.float32(2.0)
    seq = np.float32(0)
    for v in v4:
        seq = np.float32(seq + v)
    assert seq == np.float32(0.0)
    # five leaves padded to eight: ((a+b)+(c+d)) + e.  A 3+2 split gives 0.
    v = np.array([1e8, 1, 1, -1e8, 1], np.float32)
    assert orc.pairwise_sum(v) == np.float32(1.0)
    three_two = np.float32(np.float32(np.float32(1e8) + np.float32(1)) + np.float32(1))
    three_two = np.float32(three_two + np.float32(np.float32(-1e8) + np.float32(1)))
    assert three_two == np.float32(0.0)
    # zero padding to a longer power of two changes nothing
    rng = np.random.default_rng(3)
    x = rng.standard_normal(1000).astype(np.float32)
    assert orc.pairwise_sum(x) == orc.pairwise_sum(np.concatenate([x, np.zeros(3000, np.float32)]))
    # exact for small integers, and close to float64 in general
    assert orc.pairwise_sum(np.arange(1000, dtype=np.float32)) == 499500.0
    assert abs(float(orc.pairwise_sum(x)) - float(x.astype(np.float64).sum())) < 1e-4


def _ulp_diff(a, b):
    ai = a.view(np.int32).astype(np.int64)
    bi = b.view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7FFFFFFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFFFFFF), bi)
    return np.abs(ai - bi)


def test_expf_within_two_ulp():
    x = np.concatenate([np.linspace(-103.9, 88.72, 200001, dtype=np.float32),
                        np.array([-1e-6, 1e-6, 0.34657359, -0.34657359, 1.0, -1.0, 10.0], np.float32)])
    got = orc.expf(x)
    ref = np.exp(x.astype(np.float64)).astype(np.float32)
    assert int(_ulp_diff(got, ref).max()) <= 2
    assert orc.expf(np.array([0.0], np.float32))[0] == 1.0
    assert np.isinf(orc.expf(np.array([88.8, 1e30, np.inf], np.float32))).all()
    assert (orc.expf(np.array([-104.0, -1e30, -np.inf], np.float32)) == 0).all()
    assert np.isnan(orc.expf(np.array([np.nan], np.float32)))[0]
    # largest finite result and a subnormal one
    assert np.isfinite(orc.expf(np.array([88.72283], np.float32)))[0]
    sub = orc.expf(np.array([-100.0], np.float32))[0]
    assert 0 < sub < np.finfo(np.float32).tiny and abs(float(sub) - np.exp(-100.0)) <= 1.5e-45


def test_swiglu_closed_form():
    rng = np.random.default_rng(5)
    g = (rng.standard_normal(50000) * 4).astype(np.float32)
    u = rng.standard_normal(50000).astype(np.float32)
    got = orc.swiglu(g, u).astype(np.float64)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    ref = g64 / (1 + np.exp(-g64)) * u64
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)) < 1e-6
    lim = orc.swiglu(np.array([0.0, 200.0, -200.0, 1e30], np.float32), np.ones(4, np.float32))
    assert lim[0] == 0 and lim[1] == 200.0 and lim[2] == 0 and lim[3] == np.float32(1e30)


def test_rmsnorm_closed_form_and_known_answer():
    # known answer: x = [3, 4], g = 1, eps = 0 -> ms = 12.5, d = sqrt(12.5)
    out = orc.rmsnorm(np.array([[3.0, 4.0]], np.float32), np.ones(2, np.float32), 0.0)
    d = np.sqrt(np.float32(12.5))
    assert np.array_equal(out[0], np.array([np.float32(3.0) / d, np.float32(4.0) / d], np.float32))
    rng = np.random.default_rng(6)
    m, k = 5, 4096
    x = (rng.standard_normal((m, k)) * rng.uniform(0.1, 30, (m, 1))).astype(np.float32)
    g = rng.uniform(0.5, 1.5, k).astype(np.float32)
    for eps in (1e-5, 1e-2):
        got = orc.rmsnorm(x, g, eps).astype(np.float64)
        x64 = x.astype(np.float64)
        ref = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + np.float32(eps)) * g
        assert np.max(np.abs(got - ref) / np.abs(ref).max()) < 1e-6
    # zero row: 0 / sqrt(eps) = 0; scale invariance when eps is negligible
    z = orc.rmsnorm(np.zeros((1, 64), np.float32), np.ones(64, np.float32), 1e-5)
    assert not z.any()
    a = orc.rmsnorm(x[:1], g, 1e-30)
    b = orc.rmsnorm(x[:1] * np.float32(4.0), g, 1e-30)
    assert np.array_equal(a, b)  # the factor 4 is exact in every step
