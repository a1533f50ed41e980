"""BitLinear's STE training path on the GPU (bit_linear.rs:98-118 with
TensorExt::matmul_robust, layers.rs:28-59): a layer that was never packed runs a dense
matmul with the straight-through weight on the device its tensors live on.  Checked
against the numpy float32 restatement of the straight-through weight (bit for bit:
its f32 multiply, round-half-away and two f32 adds are exactly rounded on the GPU
too) and a float64 matmul (tolerance: torch's fp32 GEMM sums in its own order,
|error| <= K * 2^-24 * sum |x w|), and the straight-through gradient
d(sum y)/dw = (1/scale) * sum_rows x."""
import warnings

import numpy as np
import pytest
import torch

import bitlinear as bl
from bitlinear.layer import matmul_robust, ste_weight
from datagen import weights
from test_layer_host import np_ste_weight

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]

DEV = "cuda"


def _tol(x, w):
    # bound of an fp32 sum of K products in any order, per output
    k = x.shape[-1]
    return k * 2.0 ** -24 * (np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T) + 1e-30


@pytest.mark.parametrize("n,k", [(40, 128), (300, 512), (64, 4096)])
def test_ste_weight_on_device_is_bitexact(n, k):
    w = weights(n, k, seed=n + k)
    got = ste_weight(torch.from_numpy(w).to(DEV))
    assert got.device.type == "cuda"
    exp, _, _ = np_ste_weight(w)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), exp.view(np.uint32))


def test_bitlinear_ste_forward_and_gradient_on_gpu():
    n, k = 96, 512
    w = torch.from_numpy(weights(n, k, seed=18)).to(DEV).requires_grad_(True)
    layer = bl.BitLinear(w, k, n)
    xh = np.random.default_rng(19).standard_normal((2, 5, k)).astype(np.float32)
    x = torch.from_numpy(xh).to(DEV)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        y = layer.forward(x)
    assert y.device.type == "cuda" and tuple(y.shape) == (2, 5, n)
    w_ste, inv, _ = np_ste_weight(w.detach().cpu().numpy())
    x2 = xh.reshape(10, k)
    ref = x2.astype(np.float64) @ w_ste.T.astype(np.float64)
    err = np.abs(y.detach().cpu().numpy().reshape(10, n).astype(np.float64) - ref)
    assert np.all(err <= _tol(x2, w_ste))
    # straight-through gradient, on the device
    y.sum().backward()
    assert w.grad.device.type == "cuda"
    g = np.broadcast_to(x2.astype(np.float64).sum(0) * np.float64(inv), (n, k))
    gerr = np.abs(w.grad.cpu().numpy().astype(np.float64) - g)
    assert np.all(gerr <= 16 * 2.0 ** -24 * (np.abs(x2.astype(np.float64)).sum(0) * np.float64(inv)) + 1e-30)
    # a packed layer on the same device takes the HIP kernel instead (no warning)
    layer.precompute_packed()
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        yp = layer.forward(x)
    assert yp.device.type == "cuda" and tuple(yp.shape) == (2, 5, n)


def test_matmul_robust_moves_rhs_to_the_lhs_device():
    lhs = torch.from_numpy(np.random.default_rng(3).standard_normal((3, 4, 64)).astype(np.float32)).to(DEV)
    rhs_cpu = torch.from_numpy(weights(64, 24, seed=4))
    out = matmul_robust(lhs, rhs_cpu)
    assert out.device.type == "cuda" and tuple(out.shape) == (3, 4, 24)
    ref = lhs.cpu().numpy().reshape(12, 64).astype(np.float64) @ rhs_cpu.numpy().astype(np.float64)
    err = np.abs(out.cpu().numpy().reshape(12, 24) - ref)
    assert np.all(err <= _tol(lhs.cpu().numpy().reshape(12, 64), rhs_cpu.numpy().T))
    v = matmul_robust(lhs[0, 0], rhs_cpu)
    assert tuple(v.shape) == (24,) and v.device.type == "cuda"
