"""Pins the multi-base (AdaptiveBitLinear) oracle: orc_adaptive_reconstruct,
orc_adaptive_split, orc_adaptive_forward_i8 (oracle/bitllama_oracle.c).

  reconstruct   one base is the PackedTensor layout: equal bit for bit to
                orc_unpack (packing.rs:108-133); a hand-built known answer; against the
                float64 sum of scale * ternary over the bases (each f32 add rounds once,
                so within nb ulp-sized steps); the byte order [n, k/4, nb] of the
                reference's loader (adaptive_linear.rs:60,99-107) -- a transposed
                [nb, n, k/4] reading fails the known answer.
  split         every base's bytes decode (numpy bit ops) to that base's ternary
                values from the converter restatement.
  forward_i8    numpy int64 contraction per base and the stated f32 epilogue order.
"""
import numpy as np
import pytest

from datagen import pack_interleaved_2bit, rvq_bases, ternary, weights
from oracle import oracle as orc


def test_one_base_is_the_packed_tensor_layout():
    w = weights(24, 64, seed=1)
    b, s = orc.pack(w)
    rec = orc.adaptive_reconstruct(b, [s], 24, 64)
    assert np.array_equal(rec.view(np.uint32), orc.unpack(b, 24 * 64, s).reshape(24, 64).view(np.uint32))


def test_known_answer_two_bases():
    # row 0, columns 0..3: base 0 codes [1, 2, 0, 1] (byte 0b01_00_10_01 = 73), base 1 codes [2, 2, 1, 0]
    # (byte 0b00_01_10_10 = 26); interleaved as [cp][base]
    packed = np.array([73, 26], np.uint8)
    rec = orc.adaptive_reconstruct(packed, [0.5, 0.25], 1, 4)
    assert list(rec[0]) == [0.5 - 0.25, -0.5 - 0.25, 0.25, 0.5]
    # a [nb, n, k/4] (non-interleaved) reading of the same bytes would give base 0 = byte 73 only
    # for columns 0..3 and nothing else; the interleaved reading above is the reference's


@pytest.mark.parametrize("nb", [1, 2, 3, 5])
def test_reconstruct_against_float64(nb):
    n, k = 40, 128
    w = weights(n, k, seed=nb)
    t, s = rvq_bases(w, nb)
    packed = pack_interleaved_2bit(t)
    rec = orc.adaptive_reconstruct(packed, s, n, k)
    exact = np.tensordot(s.astype(np.float64), t.astype(np.float64), axes=(0, 0))
    assert np.all(np.abs(rec - exact) <= nb * np.spacing(np.abs(exact).astype(np.float32) + s.max()))
    # residual decomposition: more bases, closer to w
    if nb > 1:
        t1, s1 = rvq_bases(w, nb - 1)
        rec1 = orc.adaptive_reconstruct(pack_interleaved_2bit(t1), s1, n, k)
        assert np.abs(rec - w).mean() < np.abs(rec1 - w).mean()


@pytest.mark.parametrize("nb", [1, 3, 4])
def test_split_decodes_to_each_base(nb):
    n, k = 17, 96
    t, s = rvq_bases(weights(n, k, seed=7), nb)
    sp = orc.adaptive_split(pack_interleaved_2bit(t), nb, n, k)
    for b in range(nb):
        assert np.array_equal(ternary(sp[b], n * k).reshape(n, k), t[b])


@pytest.mark.parametrize("nb,m", [(1, 1), (2, 3), (3, 1), (3, 5)])
def test_forward_i8_per_base_order(nb, m):
    n, k = 33, 256
    t, s = rvq_bases(weights(n, k, seed=nb + m), nb)
    packed = pack_interleaved_2bit(t)
    x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
    y = orc.adaptive_forward_i8(x, packed, s, n)
    q, sx = orc.quantize_act(x)
    exp = None
    for b in range(nb):
        acc = (q.astype(np.int64) @ t[b].astype(np.int64).T).astype(np.float32)
        v = (acc * (sx[:, None] * s[b]).astype(np.float32)).astype(np.float32)
        exp = v if exp is None else (exp + v).astype(np.float32)
    assert np.array_equal(y.view(np.uint32), exp.view(np.uint32))
