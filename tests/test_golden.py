"""Committed golden vectors (tests/golden/bitlinear_golden.npz, written by
tests/golden/make_golden.py from the CPU oracle): the oracle must still reproduce
them, and the GPU kernels must match them bit for bit."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "bitlinear_golden.npz")


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_oracle_reproduces_golden(g):
    y, q, s, acc = orc.forward_i8(g["i8_x"], g["i8_w"], int(g["i8_n"]), float(g["i8_sw"]))
    assert np.array_equal(q, g["i8_q"]) and np.array_equal(acc, g["i8_acc"])
    assert np.array_equal(s.view(np.uint32), g["i8_s"].view(np.uint32))
    assert np.array_equal(y.view(np.uint32), g["i8_y"].view(np.uint32))
    yr = orc.forward_f32(g["ref_x"], g["ref_w"], int(g["ref_n"]), float(g["ref_sw"]))
    assert np.array_equal(yr.view(np.uint32), g["ref_y"].view(np.uint32))
    xf = orc.bf16_to_f32(g["dec_x_bf16"])
    y, _, _, acc = orc.forward_i8(xf, g["dec_w"], int(g["dec_n"]), float(g["dec_sw"]))
    assert np.array_equal(acc, g["dec_acc"])
    assert np.array_equal(orc.f32_to_bf16(y), g["dec_y_bf16"])


def test_pack_golden(g):
    w = g["pack_w"]
    wb, sw = orc.pack(w)
    assert np.array_equal(wb, g["pack_b"]) and np.float32(sw).view(np.uint32) == g["pack_s"].view(np.uint32)
    inv = np.float32(1.0 / np.float64(g["pack_s"]))
    # the planted ties: w * inv == +-0.5 exactly, which f32::round takes away from zero
    assert np.float32(w[1, 5] * inv) == 0.5 and np.float32(w[2, 7] * inv) == -0.5
    codes = lambda e: (int(g["pack_b"][e // 4]) >> (2 * (e % 4))) & 3
    assert codes(1 * 129 + 5) == 1 and codes(2 * 129 + 7) == 2 and codes(1) == 0 and codes(2) == 0
    # the last byte's unused fields stay 00
    assert w.size % 4 == 1 and int(g["pack_b"][-1]) >> 2 == 0
    import bitlinear as bl
    host = bl.PackedTensor.pack(torch.from_numpy(w))
    assert np.array_equal(host.data.numpy(), g["pack_b"]) and np.float32(host.scale) == g["pack_s"]


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
def test_gpu_pack_matches_golden(g):
    import bitlinear as bl
    dev = bl.PackedTensor.pack_device(torch.from_numpy(g["pack_w"]).to("cuda"))
    assert np.array_equal(dev.data.cpu().numpy(), g["pack_b"])
    assert np.float32(dev.scale).view(np.uint32) == g["pack_s"].view(np.uint32)


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
def test_gpu_matches_golden(g):
    import bitlinear as bl
    dev = "cuda"

    def layer(prefix):
        n = int(g[prefix + "_n"])
        wb = g[prefix + "_w"]
        k = wb.size * 4 // n
        return bl.PackedTensor(torch.from_numpy(wb).to(dev), float(g[prefix + "_sw"]), (n, k), dev)

    pt = layer("i8")
    x = torch.from_numpy(g["i8_x"]).to(dev)
    acc = torch.empty(g["i8_acc"].shape, dtype=torch.int32, device=dev)
    y = bl.BitLinearHip.forward(x, pt, acc_out=acc)
    assert np.array_equal(acc.cpu().numpy(), g["i8_acc"])
    assert np.array_equal(y.cpu().numpy().view(np.uint32), g["i8_y"].view(np.uint32))
    q, s = bl.quantize_act(x)
    assert np.array_equal(q.cpu().numpy(), g["i8_q"])

    pt = layer("ref")
    y = bl.BitLinearHip.forward(torch.from_numpy(g["ref_x"]).to(dev), pt, mode="f32_ref")
    assert np.array_equal(y.cpu().numpy().view(np.uint32), g["ref_y"].view(np.uint32))

    pt = layer("dec")
    xb = torch.from_numpy(g["dec_x_bf16"].view(np.int16)).to(dev).view(torch.bfloat16)
    acc = torch.empty(g["dec_acc"].shape, dtype=torch.int32, device=dev)
    y = bl.BitLinearHip.forward(xb, pt, acc_out=acc)
    assert np.array_equal(acc.cpu().numpy(), g["dec_acc"])
    assert np.array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16), g["dec_y_bf16"])
