"""GPU parity of the multi-base adaptive format (btl_adaptive_*) against the oracle:
split bytes, the dense reconstruction and the W1.58-A8 forward bit-exact; bf16 outputs
equal to the oracle's f32 rounded to nearest even."""
import ctypes

import numpy as np
import pytest
import torch

import bitlinear as bl
from datagen import activations, pack_interleaved_2bit, rvq_bases, weights
from oracle import oracle as orc

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]

DEV = "cuda"


def model(n, k, nb, seed):
    t, s = rvq_bases(weights(n, k, seed=seed), nb)
    return pack_interleaved_2bit(t), s


@pytest.mark.parametrize("n,k,nb", [(16, 64, 1), (33, 100, 2), (64, 4096, 3), (7, 36, 5), (40, 256, 8)])
def test_split_and_reconstruct(n, k, nb):
    print("adaptive split", n, k, nb, flush=True)
    packed, s = model(n, k, nb, seed=n + nb)
    pt = torch.from_numpy(packed).to(DEV)
    bases = bl.split_bases(pt, n, k, list(s))
    exp = orc.adaptive_split(packed, nb, n, k)
    for b in range(nb):
        assert np.array_equal(bases[b].data.cpu().numpy(), exp[b])
        assert bases[b].scale == float(s[b])
    rec = bl.reconstruct_dense(pt, list(s), n, k).cpu().numpy()
    assert np.array_equal(rec.view(np.uint32), orc.adaptive_reconstruct(packed, s, n, k).view(np.uint32))


@pytest.mark.parametrize("m", [1, 3, 9, 70])
@pytest.mark.parametrize("nb", [1, 2, 3, 5])
def test_adaptive_linear_bitexact(m, nb):
    n, k = 200, 512
    print("adaptive linear", m, nb, flush=True)
    packed, s = model(n, k, nb, seed=m * 10 + nb)
    layer = bl.AdaptiveBitLinear.load(k, n, torch.from_numpy(packed), list(s))
    x = activations(m, k, seed=m + nb)
    y = layer.forward(torch.from_numpy(x).to(DEV))
    e = orc.adaptive_forward_i8(x, packed, s, n)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), e.view(np.uint32))


@pytest.mark.parametrize("m", [1, 40])
def test_adaptive_linear_bf16_and_llama_shape(m):
    n, k, nb = 1024, 4096, 3
    packed, s = model(n, k, nb, seed=m)
    layer = bl.AdaptiveBitLinear.load(k, n, torch.from_numpy(packed).to(DEV), list(s))
    x = activations(m, k, seed=3)
    xt = torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    y = layer.forward(xt)
    e = orc.adaptive_forward_i8(xt.float().cpu().numpy(), packed, s, n)
    got = y.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, orc.f32_to_bf16(e))
    # rank-3 input flattens like the reference (adaptive_linear.rs:137-143)
    y3 = layer.forward(xt.reshape(1, m, k))
    assert y3.shape == (1, m, n) and torch.equal(y3.reshape(m, n), y)


def test_adaptive_rejects_bad_shapes():
    packed, s = model(16, 64, 2, seed=1)
    with pytest.raises(bl.BitLinearError):
        bl.split_bases(torch.from_numpy(packed).to(DEV), 16, 60, list(s))
    pt = torch.from_numpy(packed).to(DEV)
    bases = bl.split_bases(pt, 16, 64, list(s))
    cs = [b.as_c() for b in bases]
    arr = (ctypes.POINTER(bl.BtlPacked) * 2)(*[ctypes.pointer(c) for c in cs])
    x = torch.zeros((1, 32), device=DEV)
    y = torch.zeros((1, 16), device=DEV)
    st = bl.lib.btl_adaptive_linear(arr, 2, x.data_ptr(), bl.BTL_F32, 1, 32, y.data_ptr(), bl.BTL_F32, None, 0, None)
    assert st == bl.BTL_ERR_SHAPE and b"Shape mismatch" in bl.lib.btl_last_error()


@pytest.mark.parametrize("m,nb", [(1, 1), (9, 3), (70, 5), (33, 8)])
def test_adaptive_f32_ref_forward(m, nb):
    # the reference's arithmetic: dense weights rebuilt at load (adaptive_linear.rs:86-124),
    # then x . w_recon^T per forward (:141-151); bit-exact against the oracle's
    # reconstruction and dense product, and within an fp32 sum's bound of float64
    n, k = 200, 512
    print("adaptive f32_ref", m, nb, flush=True)
    packed, s = model(n, k, nb, seed=m + 7 * nb)
    layer = bl.AdaptiveBitLinear.load(k, n, torch.from_numpy(packed), list(s), mode="f32_ref")
    assert layer.bases is None and layer.reconstructed_weight.device.type == "cuda"
    rec = orc.adaptive_reconstruct(packed, s, n, k)
    assert np.array_equal(layer.reconstructed_weight.cpu().numpy().view(np.uint32), rec.view(np.uint32))
    x = activations(m, k, seed=m + 1)
    y = layer.forward(torch.from_numpy(x).to(DEV))
    assert y.dtype == torch.float32 and tuple(y.shape) == (m, n)
    got = y.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), orc.dense_linear(x, rec).view(np.uint32))
    ref = x.astype(np.float64) @ rec.T.astype(np.float64)
    tol = k * 2.0 ** -24 * (np.abs(x.astype(np.float64)) @ np.abs(rec.T.astype(np.float64))) + 1e-30
    assert np.all(np.abs(got - ref) <= tol)


def test_adaptive_f32_ref_llama_shape_rank3_and_bf16():
    n, k, nb, m = 1024, 4096, 3, 6
    packed, s = model(n, k, nb, seed=11)
    layer = bl.AdaptiveBitLinear.load(k, n, torch.from_numpy(packed).to(DEV), list(s), mode="f32_ref")
    rec = orc.adaptive_reconstruct(packed, s, n, k)
    xt = torch.from_numpy(activations(m, k, seed=12)).to(DEV).to(torch.bfloat16)
    y = layer.forward(xt.reshape(2, 3, k))  # rank 3 flattens (adaptive_linear.rs:137-143)
    assert y.shape == (2, 3, n) and y.dtype == torch.float32
    e = orc.dense_linear(xt.float().cpu().numpy(), rec)  # bf16 widens exactly
    assert np.array_equal(y.reshape(m, n).cpu().numpy().view(np.uint32), e.view(np.uint32))
    with pytest.raises(bl.BitLinearError):
        layer.forward(xt, out_dtype=torch.bfloat16)
    with pytest.raises(bl.BitLinearError):
        layer.forward(torch.zeros((1, k - 4), device=DEV))
