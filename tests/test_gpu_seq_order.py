"""GPU parity of BTL_ACT_F32_SEQ: the reference's contraction on a host without
AVX2/FMA (cpu.rs:62-66 then the scalar loop of cpu.rs:105-123), bit for bit against
the oracle's restatement of that branch (orc.forward_f32(..., avx2_order=False),
pinned in tests/test_oracle.py by integer-exact sums and a known answer that tells
the two orders apart).  Inputs spanning 40 binades make every sum order-sensitive."""
import numpy as np
import pytest
import torch

import bitlinear as bl
from datagen import pack_codes, random_codes
from oracle import oracle as orc
from test_gpu_parity import assert_bf16_matches, assert_f32_identical, host_x, to_dev

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]

DEV = "cuda"


def wide_x(m, k, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((m, k)) * np.exp2(rng.integers(-20, 20, (m, k)))).astype(np.float32)


def layer(n, k, seed, scale=0.0173):
    wb = random_codes(n, k, seed=seed, p3=0.1)
    return bl.PackedTensor(torch.from_numpy(wb).to(DEV), float(np.float32(scale)), (n, k), DEV), wb


def seq_ref(x, wb, n, scale):
    return orc.forward_f32(x, wb, n, np.float32(scale), avx2_order=False)


# k % 64 == 0 takes the vector form (a 64-weight block per load, two blocks per loop
# trip: k = 4160 ends on the first of a pair, k = 64 is one block); k = 100 and 36
# the byte form
@pytest.mark.parametrize("m,k,n", [(1, 2048, 300), (3, 100, 17), (2, 36, 9), (4, 4096, 64), (1, 4, 3),
                                   (1, 64, 257), (5, 4160, 33), (1, 14336, 40), (2, 8192, 8)])
@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                     (torch.bfloat16, torch.float32)])
def test_linear_f32_seq_bitexact(m, k, n, xdt, ydt):
    print("f32_seq", m, k, n, xdt, ydt, flush=True)
    pt, wb = layer(n, k, seed=k + n)
    xt = to_dev(wide_x(m, k, seed=m * 7 + k + n), xdt)
    y = bl.BitLinearHip.forward(xt, pt, mode="f32_seq", out_dtype=ydt)
    yr = seq_ref(host_x(xt), wb, n, pt.scale)
    if ydt == torch.float32:
        assert_f32_identical(y, yr)
    else:
        assert_bf16_matches(y, yr)


def test_linear_f32_seq_order_known_answer():
    # row 0: x[0] = 2^24, x[1] = x[2] = 1, x[8] = -2^24.  The AVX2 lanes give
    # (2^24 - 2^24) + 1 + 1 = 2; the sequential loop ((2^24 + 1) + 1) - 2^24 = 0
    # (2^24 + 1 rounds back to 2^24); at k = 36 the byte form, at k = 64 the vector form.
    for k in (36, 64):
        x = np.zeros((1, k), np.float32)
        x[0, 0], x[0, 1], x[0, 2], x[0, 8] = 2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)
        codes = np.zeros(k, np.uint8)
        codes[[0, 1, 2, 8]] = 1
        wb = pack_codes(codes)
        pt = bl.PackedTensor(torch.from_numpy(wb).to(DEV), 1.0, (1, k), DEV)
        xt = to_dev(x, torch.float32)
        assert bl.BitLinearHip.forward(xt, pt, mode="f32_seq").item() == 0.0
        assert bl.BitLinearHip.forward(xt, pt, mode="f32_ref").item() == 2.0


# subnormal inputs and sums, sums that overflow, inf inputs (times a zero
# coefficient: NaN) and a NaN input; vector and byte forms
@pytest.mark.parametrize("k", [4096, 100])
def test_linear_f32_seq_special_values(k):
    print("f32_seq special", k, flush=True)
    rng = np.random.default_rng(k)
    m, n = 3, 40
    x = np.empty((m, k), np.float32)
    x[0] = rng.standard_normal(k) * 1e-39
    x[1] = rng.standard_normal(k) * 3e37
    x[2] = rng.standard_normal(k) * 1e-3
    x[2, 5], x[2, 61], x[2, 77] = np.inf, -np.inf, np.nan
    pt, wb = layer(n, k, seed=k + 3, scale=0.5)
    y = bl.BitLinearHip.forward(to_dev(x, torch.float32), pt, mode="f32_seq").cpu().numpy()
    yr = seq_ref(x, wb, n, pt.scale)
    assert np.isnan(yr[2]).any() and not np.isfinite(yr[1]).all() and (np.abs(yr[0][yr[0] != 0]) < 1.2e-38).any()
    nan = np.isnan(yr)
    assert np.array_equal(np.isnan(y), nan)
    assert_f32_identical(np.where(nan, 0, y).astype(np.float32), np.where(nan, 0, yr).astype(np.float32))


def test_linear_f32_seq_rows_past_the_grid_and_misaligned_x():
    # m > 65535: the rows past grid.y are walked by the kernel's loop
    m, k, n = 65537, 64, 3
    pt, wb = layer(n, k, seed=5)
    x = wide_x(m, k, seed=6)
    y = bl.BitLinearHip.forward(to_dev(x, torch.float32), pt, mode="f32_seq")
    assert_f32_identical(y, seq_ref(x, wb, n, pt.scale))
    # x 4 bytes off a 16-byte boundary: the byte form
    m, k, n = 3, 256, 50
    pt, wb = layer(n, k, seed=7)
    x = wide_x(m, k, seed=8)
    buf = torch.zeros(m * k + 1, device=DEV)
    buf[1:] = torch.from_numpy(x.reshape(-1)).to(DEV)
    xv = buf[1:].view(m, k)
    assert xv.data_ptr() % 16 == 4
    assert_f32_identical(bl.BitLinearHip.forward(xv, pt, mode="f32_seq"), seq_ref(x, wb, n, pt.scale))


def test_group_and_layer_f32_seq():
    k = 512
    xt = to_dev(wide_x(3, k, seed=9), torch.float32)
    layers = [layer(n, k, seed=40 + n, scale=0.01 * (i + 1)) for i, n in enumerate((96, 40, 33))]
    outs = bl.linear_group([l[0] for l in layers], xt, out_dtype=torch.float32, mode="f32_seq")
    for (pt, wb), y in zip(layers, outs):
        assert_f32_identical(y, seq_ref(host_x(xt), wb, pt.shape[0], pt.scale))
    # the layer: rank 3 flattens, packed params run the kernel (bit_linear.rs:52-97)
    w = torch.from_numpy(wide_x(24, k, seed=10) * 1e-6)
    lay = bl.BitLinear.load(k, 24, w, device=DEV)
    lay.precompute_packed()
    x3 = to_dev(wide_x(6, k, seed=11), torch.float32).reshape(2, 3, k)
    y = lay.forward(x3, mode="f32_seq")
    assert y.shape == (2, 3, 24)
    pp = lay.packed_params
    assert_f32_identical(y.reshape(6, 24), seq_ref(host_x(x3.reshape(6, k)), pp.data.cpu().numpy(), 24, pp.scale))
