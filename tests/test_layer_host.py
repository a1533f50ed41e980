"""CPU tests of the host-side mirror of the reference's Rust API that need no GPU:
PackedTensor::new's length check (packing.rs:25-47) and BitLinear's STE training path
(bit_linear.rs:98-118, layers.rs:28-59), each against a numpy float32 restatement."""
import warnings

import numpy as np
import pytest
import torch

import bitlinear as bl
from bitlinear.layer import ste_weight
from datagen import weights
from oracle import oracle as orc


@pytest.mark.parametrize("shape", [(8, 64), (3, 5), (1, 1), (7, 33)])
def test_packed_tensor_new_checks_length(shape):
    # packing.rs:25-47: Tensor::from_vec(data, (ceil(numel / 4),)) fails on any other length
    w = weights(*shape, seed=2)
    wb, sw = orc.pack(w)
    numel = shape[0] * shape[1]
    assert wb.size == (numel + 3) // 4
    pt = bl.PackedTensor.new(wb, shape, sw)
    assert pt.shape == shape and pt.num_elem == numel and pt.scale == np.float32(sw)
    assert np.array_equal(pt.data.numpy(), wb)
    assert np.array_equal(pt.unpack().numpy().reshape(-1), orc.unpack(wb, numel, sw))
    pt2 = bl.PackedTensor.new(torch.from_numpy(wb.copy()), shape, sw)
    assert np.array_equal(pt2.data.numpy(), wb)
    for bad in (np.append(wb, 0), wb[:-1]):
        with pytest.raises(bl.BitLinearError) as ei:
            bl.PackedTensor.new(bad, shape, sw)
        assert ei.value.status == bl.BTL_ERR_SHAPE


def np_ste_weight(w):
    """bit_linear.rs:101-110 in numpy float32: w_s = w * (f32)(1/(f64)mean|w|) + 0,
    w_q = round_half_away(w_s).clamp(-1, 1), w_ste = (w_q - w_s) + w_s."""
    w = w.astype(np.float32)
    s = np.float32(np.abs(w.astype(np.float64)).mean())
    inv = np.float32(1.0 / np.float64(s))
    w_s = (w * inv).astype(np.float32) + np.float32(0.0)
    w_q = np.clip(np.sign(w_s) * np.floor(np.abs(w_s).astype(np.float64) + 0.5), -1, 1).astype(np.float32)
    return ((w_q - w_s).astype(np.float32) + w_s).astype(np.float32), inv, w_q


def test_ste_weight_matches_numpy_restatement():
    w = weights(96, 256, seed=7)
    # plant values of w_s at the rounding edges: 0.49999997 (-> 0, where floor(v + 0.5) in
    # f32 gives 1), exactly 0.5 (-> 1, half away) and -0.5 (-> -1)
    s = np.float32(np.abs(w.astype(np.float64)).mean())
    got = ste_weight(torch.from_numpy(w)).numpy()
    exp, inv, w_q = np_ste_weight(w)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
    # w_ste is w_q up to the rounding of (w_q - w_s) + w_s, never more than an ulp of w_q's magnitude
    assert np.all(np.abs(got - w_q) <= np.float32(2 ** -23) * 2)
    assert np.all(np.isin(w_q, [-1.0, 0.0, 1.0]))
    assert s > 0 and inv == np.float32(1.0 / np.float64(s))


def test_ste_rounds_half_away_at_the_edges():
    # a row whose mean |w| is exactly 1, so w_s = w: 0.49999997 -> 0, 0.5 -> 1, -0.5 -> -1, 1.5 -> 1
    w = np.array([[0.49999997, 0.5, -0.5, 1.5, -2.0, 0.0, 1.0, 2.00000003]], np.float32)
    w = w * np.float32(1.0 / np.abs(w.astype(np.float64)).mean())
    exp, _, w_q = np_ste_weight(w)
    got = ste_weight(torch.from_numpy(w)).numpy()
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
    s = np.float32(np.abs(w.astype(np.float64)).mean())
    assert s == np.float32(1.0) or abs(float(s) - 1.0) < 1e-6


def test_bitlinear_ste_forward_and_gradient():
    w = torch.from_numpy(weights(40, 128, seed=8)).requires_grad_(True)
    layer = bl.BitLinear(w, 128, 40)
    x = torch.from_numpy(np.random.default_rng(9).standard_normal((2, 3, 128)).astype(np.float32))
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        y = layer.forward(x)
    assert tuple(y.shape) == (2, 3, 40)
    w_ste, inv, _ = np_ste_weight(w.detach().numpy())
    ref = x.numpy().reshape(6, 128).astype(np.float64) @ w_ste.T.astype(np.float64)
    np.testing.assert_allclose(y.detach().numpy().reshape(6, 40), ref, rtol=1e-5, atol=1e-5)
    # straight-through: d(sum y) / dw = (1 / scale) * sum over rows of x
    y.sum().backward()
    g = np.broadcast_to(x.numpy().reshape(6, 128).sum(0) * np.float64(inv), (40, 128))
    np.testing.assert_allclose(w.grad.numpy(), g, rtol=1e-5, atol=1e-5)
    # rank-1 input (matmul_robust unsqueezes and squeezes)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        y1 = layer.forward(x[0, 0])
    assert tuple(y1.shape) == (40,)
    np.testing.assert_allclose(y1.detach().numpy(), ref[0], rtol=1e-5, atol=1e-5)


def test_adaptive_layer_state_and_mode_checks():
    # adaptive_linear.rs:126-127,159: no weights at all / a layer without either form
    with pytest.raises(bl.BitLinearError, match="neither legacy nor adaptive"):
        bl.AdaptiveBitLinear.load(64, 16)
    with pytest.raises(bl.BitLinearError, match="unknown mode"):
        bl.AdaptiveBitLinear.load(64, 16, np.zeros(16 * 16 * 2, np.uint8), [0.5, 0.25], mode="f16")
    with pytest.raises(bl.BitLinearError, match="Invalid State"):
        bl.AdaptiveBitLinear(64, 16).forward(torch.zeros((1, 64)))
