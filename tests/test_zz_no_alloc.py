"""btl_linear_noalloc (no workspace, no allocation; scratch in a static device array)
against btl_linear through the C ABI: bit-identical outputs and int32 accumulators on
two calls in a row, the second with a smaller input, over the routes that use scratch
(batched decode, split-K, the prefill GEMM, ragged k) and one that does not (one-token
decode, the reference-order mode).  Shapes beyond the array fail cleanly."""
import ctypes

import numpy as np
import pytest
import torch

import bitlinear as bl
from datagen import activations, weights
from oracle import oracle as orc

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]

DEV = "cuda"


def _layer(n, k, seed):
    wb, sw = orc.pack(weights(n, k, seed))
    return bl.PackedTensor(torch.from_numpy(wb).to(DEV), sw, (n, k), DEV)


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _call(fn, pt, x, mode, ydt, with_acc):
    m, k = x.shape
    n = pt.shape[0]
    y = torch.full((m, n), float("nan"), dtype=ydt, device=DEV)
    acc = torch.full((m, n), -7, dtype=torch.int32, device=DEV) if with_acc else None
    c = pt.as_c()
    xdt = bl.BTL_BF16 if x.dtype == torch.bfloat16 else bl.BTL_F32
    ydc = bl.BTL_BF16 if ydt == torch.bfloat16 else bl.BTL_F32
    args = [ctypes.byref(c), x.data_ptr(), xdt, m, k, y.data_ptr(), ydc, mode,
            acc.data_ptr() if acc is not None else None]
    if fn == "linear":
        bl.check(bl.lib.btl_linear(*args, None, 0, _stream()))
    else:
        bl.check(bl.lib.btl_linear_noalloc(*args, _stream()))
    return y, acc


# (first call, second smaller call): m, k, n, input dtype, output dtype
PAIRS = [
    ((40, 4096, 1000), (6, 1024, 300)),        # batched decode (+ split-K), then a smaller one
    ((300, 2048, 1024), (130, 1088, 257)),     # prefill GEMM, then a ragged-tile GEMM
    ((2048, 4096, 4096), (64, 4096, 64)),      # a Llama-3-8B prefill projection, then split-K batched decode
    ((5, 1000, 200), (3, 36, 50)),             # ragged k (generic route, scratch), smaller
    ((1, 4096, 2048), (1, 1024, 100)),         # one-token decode (no scratch)
]


@pytest.mark.parametrize("first,second", PAIRS)
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_noalloc_equals_linear_twice(first, second, dt):
    print("noalloc", first, second, dt, flush=True)
    for i, (m, k, n) in enumerate((first, second)):
        wb, sw = orc.pack(weights(n, k, m + k + n))
        pt = bl.PackedTensor(torch.from_numpy(wb).to(DEV), sw, (n, k), DEV)
        x = torch.from_numpy(activations(m, k, seed=m * 3 + i)).to(DEV).to(dt)
        y1, a1 = _call("linear", pt, x, bl.BTL_ACT_I8, dt, True)
        y2, a2 = _call("noalloc", pt, x, bl.BTL_ACT_I8, dt, True)
        torch.cuda.synchronize()
        assert torch.equal(a1, a2), (m, k, n)
        assert torch.equal(y1.view(torch.int16) if dt == torch.bfloat16 else y1.view(torch.int32),
                           y2.view(torch.int16) if dt == torch.bfloat16 else y2.view(torch.int32)), (m, k, n)
        if m * n * k <= 300 * 2048 * 1024:
            _, _, _, accr = orc.forward_i8(x.float().cpu().numpy(), wb, n, sw)
            assert np.array_equal(a2.cpu().numpy(), accr)
    bl.check_faults()


def test_noalloc_reference_mode():
    pt = _layer(300, 2048, seed=5)
    x = torch.from_numpy(activations(2, 2048, seed=6)).to(DEV)
    y1, _ = _call("linear", pt, x, bl.BTL_ACT_F32_REF, torch.float32, False)
    y2, _ = _call("noalloc", pt, x, bl.BTL_ACT_F32_REF, torch.float32, False)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int32), y2.view(torch.int32))


def test_noalloc_rejects_shapes_beyond_the_array():
    m, k, n = 4096, 16384, 64  # 64 MiB of quantised activations
    pt = _layer(n, k, seed=9)
    x = torch.zeros((m, k), dtype=torch.bfloat16, device=DEV)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    c = pt.as_c()
    rc = bl.lib.btl_linear_noalloc(ctypes.byref(c), x.data_ptr(), bl.BTL_BF16, m, k, y.data_ptr(), bl.BTL_BF16,
                                   bl.BTL_ACT_I8, None, _stream())
    assert rc == bl.BTL_ERR_WORKSPACE
    assert b"scratch" in bl.lib.btl_last_error()
