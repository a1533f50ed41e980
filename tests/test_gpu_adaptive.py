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
