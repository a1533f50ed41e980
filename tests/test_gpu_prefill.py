"""GPU parity of the prefill GEMM (k_gemm_i8) at the launches the cfg4 bench times:
M = 2048 bf16 tokens through the Llama-3-8B projection shapes, issued as the bench
issues them (the fused quantise + GEMM route of btl_linear_group_mode, and the GEMM
alone on operand-order int8 through btl_linear_i8_op), checked against the CPU oracle.

Every int32 accumulator of a launch is checked, not a sample: acc = q t^T is tested
as acc r == q (t^T r) for random integer vectors r with no zero entry (Freivalds'
check; a single wrong accumulator always changes acc r), and as l^T acc == (l^T q) t^T
for random l over the token rows.  Both sides are sums of integers below 2^53 in
float64 (t^T r, below 2^24, in float32), so the comparison is exact.  q is the
oracle's quantisation of the same bf16 rows, so the check also pins the GPU's
quantiser.  With the accumulators pinned, every bf16 output is compared with the
oracle's epilogue of them, and sampled token rows (first and last token tile, the
tile boundaries) with the oracle's whole forward (cpu.rs:73-124 contraction order is
irrelevant here: the int path is exact).  Shapes: models/Meta-Llama-3-8B/config.json:4-8.
"""
import numpy as np
import pytest
import torch

import bitlinear as bl
from datagen import activations, ternary, weights
from exactcheck import check_acc_exact
from oracle import oracle as orc

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]

DEV = "cuda"
M = 2048
HIDDEN, INTER, KV = 4096, 14336, 1024

# the four calls of a layer as bench.py's prefill section issues them, and the GEMM
# instantiation the default routing gives each on 256 CUs
KINDS = {
    "qkv": (HIDDEN, (HIDDEN, KV, KV), "k_gemm_i8<128,2,4,128,2>"),
    "o": (HIDDEN, (HIDDEN,), "k_gemm_i8<128,4,4,128,3>"),
    "gate_up": (HIDDEN, (INTER, INTER), "k_gemm_i8<256,4,4,128,2>"),
    "down": (INTER, (HIDDEN,), "k_gemm_i8<128,4,4,128,3>"),
}


def _form():
    return bl.lib.btl_last_gemm_form().decode()


def assert_bf16_equals(y, ref_f32, what):
    g = y.cpu().view(torch.int16).numpy().view(np.uint16)
    r = orc.f32_to_bf16(ref_f32)
    bad = np.flatnonzero(g.reshape(-1) != r.reshape(-1))
    assert bad.size == 0, "%s: %d bf16 mismatches, first at %d" % (what, bad.size, bad[0])


@pytest.mark.parametrize("kind", list(KINDS))
def test_cfg4_launch_matches_oracle(kind):
    k, ns, form = KINDS[kind]
    print("cfg4 launch", kind, M, k, ns, flush=True)
    x = activations(M, k, seed=401 + k)
    x[3] = 0.0                                   # a zero token row inside the first tile
    xt = torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    xh = xt.float().cpu().numpy()
    layers = []
    for i, n in enumerate(ns):
        wb, sw = orc.pack(weights(n, k, seed=4000 + 17 * i + n))
        layers.append((bl.PackedTensor(torch.from_numpy(wb).to(DEV), sw, (n, k), DEV), wb, sw))
    pts = [l[0] for l in layers]

    # the bench's Call: quantise + GEMM in one btl_linear_group_mode call
    ys_fused = bl.linear_group(pts, xt, out_dtype=torch.bfloat16)
    assert _form() == form
    # the bench's OpCall: the GEMM alone on operand-order int8, with accumulators
    qo, so = bl.quantize_act_op(xt)
    accs = [torch.empty((M, n), dtype=torch.int32, device=DEV) for n in ns]
    ys = bl.linear_i8_op(qo, so, pts, out_dtype=torch.bfloat16, acc_out=accs)
    assert _form() == form
    torch.cuda.synchronize()

    q, s = orc.quantize_act(xh)
    assert np.array_equal(so.cpu().numpy().view(np.uint32), s.view(np.uint32))
    rows = np.unique(np.concatenate([[0, 3, 127, 128, 1023, 1024, 1919, 1920, 2047],
                                     np.random.default_rng(k).choice(M, 4, replace=False)]))
    for i, ((pt, wb, sw), n) in enumerate(zip(layers, ns)):
        acc = accs[i].cpu().numpy()
        t32 = ternary(wb, n * k).reshape(n, k).astype(np.float32)
        check_acc_exact(acc, q, t32, seed=i)
        del t32
        assert_bf16_equals(ys[i], orc.epilogue(acc, s, sw), "%s layer %d outputs" % (kind, i))
        assert torch.equal(ys_fused[i], ys[i]), "fused route differs from the GEMM-alone route"
        yr, _, _, accr = orc.forward_i8(xh[rows], wb, n, sw)
        assert np.array_equal(acc[rows], accr)
        assert_bf16_equals(ys[i][rows], yr, "%s layer %d sampled rows" % (kind, i))
