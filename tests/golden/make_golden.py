"""Writes tests/golden/bitlinear_golden.npz: seeded inputs and the CPU oracle's outputs.

    python tests/golden/make_golden.py

The fixtures are data (inputs and expected outputs) so that the GPU can be checked
against fixed vectors as well as the live oracle.  Cases:
  i8_*   W1.58-A8 forward, f32 activations with outliers, zero and tiny rows
  ref_*  reference-semantics fp32 forward (cpu.rs order), k % 32 != 0 tail
  dec_*  a decode-shaped case (M=1, K=1024, N=96) in bf16
  pack_* PackedTensor::pack of a ragged 37 x 129 f32 weight (tail byte, exact ties
         w * (1 / scale) = +-0.5, zeros and denormal-range values), packed bytes and scale
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

from datagen import activations, weights  # noqa: E402
from oracle import oracle as orc  # noqa: E402


def main():
    out = {}
    # W1.58-A8, f32, odd shapes
    m, k, n = 5, 320, 70
    x = activations(m, k, seed=101)
    x[3] = 0.0
    x[4] *= np.float32(1e-32)
    wb, sw = orc.pack(weights(n, k, seed=102))
    y, q, s, acc = orc.forward_i8(x, wb, n, sw)
    out.update(i8_x=x, i8_w=wb, i8_sw=np.float32(sw), i8_n=np.int64(n), i8_y=y, i8_q=q, i8_s=s, i8_acc=acc)
    # reference fp32 order
    m, k, n = 3, 100, 17
    x = activations(m, k, seed=103)
    wb, sw = orc.pack(weights(n, k, seed=104))
    out.update(ref_x=x, ref_w=wb, ref_sw=np.float32(sw), ref_n=np.int64(n), ref_y=orc.forward_f32(x, wb, n, sw))
    # decode-shaped bf16 case
    m, k, n = 1, 1024, 96
    xb = orc.f32_to_bf16(activations(m, k, seed=105))
    xf = orc.bf16_to_f32(xb)
    wb, sw = orc.pack(weights(n, k, seed=106))
    y, q, s, acc = orc.forward_i8(xf, wb, n, sw)
    out.update(dec_x_bf16=xb, dec_w=wb, dec_sw=np.float32(sw), dec_n=np.int64(n), dec_acc=acc,
               dec_y_bf16=orc.f32_to_bf16(y))
    # pack: ragged numel, exact ties (w * (1 / scale) == +-0.5 in f32)
    w = weights(37, 129, seed=107)
    w[0, :3] = np.float32([0.0, 1e-30, -1e-30])
    for _ in range(8):
        _, sw = orc.pack(w)
        inv = np.float32(1.0 / np.float64(np.float32(sw)))
        t = np.float32(0.5) / inv
        while np.float32(t * inv) != np.float32(0.5):
            t = np.nextafter(t, np.float32(np.inf) if np.float32(t * inv) < 0.5 else np.float32(0))
        w[1, 5], w[2, 7] = t, -t
        if orc.pack(w)[1] == sw:
            break
    assert np.float32(w[1, 5] * inv) == 0.5 and orc.pack(w)[1] == sw
    wb, sw = orc.pack(w)
    out.update(pack_w=w, pack_b=wb, pack_s=np.float32(sw))
    path = os.path.join(HERE, "bitlinear_golden.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
