"""Pins the decoder-op oracle (oracle/bitllama_oracle.c, oracle/llama_oracle.py)
before the GPU decoder is checked against it.

What pins each function (reference = imonoonoko/Bit-TTT-Engine, crates/rust_engine):
  orc_rope_table    float64 closed form of RotaryEmbedding::new (attention.rs:15-42):
                    inv_freq = 1.0f / (f32)theta^(2i/hd) (attention.rs:19: the cast binds
                    before the division, so the power is rounded to f32 and the reciprocal
                    is an f32 division; the reading that rounds 1/theta^e once in f64
                    differs at 18 of the 64 Llama-3 frequencies and is rejected below),
                    freq = (f32)p * inv_freq exactly, cos/sin
                    within 1 ulp of the float64 values (glibc cosf/sinf, which Rust's
                    f32::cos/sin call on Linux); the Llama-3 theta 500000.
  orc_rope_apply    float64 rotation (relative 1e-6), norm preservation, position 0 is
                    the identity, the half-split pairing (i, i + hd/2) of attention.rs:67-72
                    (an interleaved (2i, 2i+1) pairing fails).
  orc_q8_quant /    kv_cache.rs:95-128 closed form: the max element -> code 255 or 1, codes
  orc_q8_dequant    in [1, 255], |dequant - x| <= s/2, s = max|x| * (f32)(1/127) (candle's
                    Tensor / f64 is affine(1/rhs, 0), kv_cache.rs:101; rows where the IEEE
                    quotient max|x|/127 differs by an ulp are planted); the round-half-away
                    tie; a zero row (0/0 -> NaN -> code 0 by Rust's saturating cast,
                    dequantised to 0).
  orc_attn_decode   float64 softmax attention over the dequantised cache with the GQA map
                    of repeat_kv (attention.rs:227-239), relative 2e-6 of the output scale,
                    at chunk boundaries T = 1, 63, 64, 65, 129; per-head planted values
                    that a wrong head map (h % nkv instead of h // rep) gets wrong.
                    The reference's own summation order (candle gemm) is not vendored:
                    its last ulps are parity unpinned (tolerance above).  The fixed order
                    (orc_attn_dot: a sequential chain of fused multiply-adds for every
                    score and value sum) is pinned by known answers: a term whose
                    product is inexact (an fma and a multiply-then-add differ), a
                    cancelling sequence (the sequential order and the reversed one
                    differ), and a two-key attention whose output carries the score's
                    fma bit.
  orc_argmax        Iterator::max_by semantics: the last of equal maxima.
  orc_dense_linear  candle_nn::Linear::forward (the dense lm_head, llama.rs:129-141):
                    exact integer-valued products and sums (no dropped term, no
                    transposed operand: rectangular w with distinct rows), float64
                    matmul within 1e-5 relative, bf16 weights = their exact f32
                    widening, and the order itself: a row whose lane-0 partial sum
                    absorbs a small term only in the fixed order.  The reference's
                    gemm order is not vendored: its last ulps are parity unpinned.
  OracleLlama       composition only; pinned by the functions above and by
                    test_oracle.py (BitLinear, RMSNorm, SwiGLU); checked here for the
                    causal invariant that token t's logits do not depend on later tokens.
"""
import numpy as np
import pytest

from datagen import weights
from oracle import oracle as orc
from oracle.llama_oracle import OracleLlama


def _ulp_diff(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


def ref_inv_freq(theta, hd):
    """attention.rs:19 `1.0 / (theta.powf((2 * i) as f64 / head_dim as f64)) as f32`: the f64
    power cast to f32, then 1.0f32 / that (numpy float32 division is IEEE)."""
    return np.array([np.float32(1.0) / np.float32(theta ** ((2 * i) / hd)) for i in range(hd // 2)], np.float32)


def _table64(inv, S):
    freq = (np.arange(S, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    return (np.cos(freq.astype(np.float64)).astype(np.float32), np.sin(freq.astype(np.float64)).astype(np.float32))


def test_rope_inv_freq_rounds_the_power_first():
    # theta 500000, hd 128 (Llama-3), i = 2: fl32(1 / fl32(p)) != fl32(1 / p)
    theta, hd, S = 500000.0, 128, 769
    p = theta ** (4 / 128)
    assert np.float32(1.0) / np.float32(p) != np.float32(1.0 / p)
    wrong = np.array([np.float32(1.0 / theta ** ((2 * i) / hd)) for i in range(hd // 2)], np.float32)
    right = ref_inv_freq(theta, hd)
    assert (wrong != right).sum() == 18
    c, s = orc.rope_table(theta, hd, S)
    rc, rs = _table64(right, S)
    wc, ws = _table64(wrong, S)
    assert np.all(_ulp_diff(c, rc) <= 1) and np.all(_ulp_diff(s, rs) <= 1)
    # the double-rounded reading moves the table by far more than an ulp at most positions
    bad = (_ulp_diff(c, wc) > 1) | (_ulp_diff(s, ws) > 1)
    assert bad.any(axis=1).sum() > S // 2


@pytest.mark.parametrize("theta,hd", [(500000.0, 128), (10000.0, 64), (10000.0, 2)])
def test_rope_table_closed_form(theta, hd):
    S = 300
    c, s = orc.rope_table(theta, hd, S)
    half = hd // 2
    inv = ref_inv_freq(theta, hd)
    freq = (np.arange(S, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    assert np.all(_ulp_diff(c, np.cos(freq.astype(np.float64)).astype(np.float32)) <= 1)
    assert np.all(_ulp_diff(s, np.sin(freq.astype(np.float64)).astype(np.float32)) <= 1)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    # i = 0 is the fastest rotation: angle p radians
    np.testing.assert_allclose(c[:, 0], np.cos(np.arange(S)), rtol=0, atol=1e-6)


def test_rope_apply_rotation():
    hd = 128
    c, s = orc.rope_table(500000.0, hd, 64)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, hd)).astype(np.float32)
    for p in (0, 1, 37, 63):
        y = orc.rope_apply(x, c[p], s[p])
        x64, c64, s64 = x.astype(np.float64), c[p].astype(np.float64), s[p].astype(np.float64)
        h = hd // 2
        e1 = x64[:, :h] * c64 - x64[:, h:] * s64
        e2 = x64[:, :h] * s64 + x64[:, h:] * c64
        np.testing.assert_allclose(y, np.concatenate([e1, e2], 1), rtol=1e-6, atol=1e-6)
        np.testing.assert_allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x64, axis=1), rtol=1e-6)
        if p == 0:
            assert np.array_equal(y, x)
    # the pairing is (i, i + hd/2): a vector living in the first half rotates into the second
    e = np.zeros((1, hd), np.float32)
    e[0, 0] = 1.0
    y = orc.rope_apply(e, c[1], s[1])
    assert y[0, hd // 2] == s[1][0] and y[0, 1] == 0.0


def test_q8_quant_closed_form():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((50, 128)).astype(np.float32)
    q, s = orc.q8_quant(x)
    amax = np.abs(x).max(1)
    assert np.array_equal(s, (amax * np.float32(1.0 / 127.0)).astype(np.float32))
    assert q.min() >= 1 and q.max() <= 255
    idx = np.abs(x).argmax(1)
    top = q[np.arange(50), idx]
    assert np.all(np.where(x[np.arange(50), idx] > 0, top == 255, top == 1))
    d = orc.q8_dequant(q, s)
    assert np.all(np.abs(d - x) <= s[:, None] * 0.5000001)
    # codes: round half away of x/s, + 128
    r = x / s[:, None]
    exp_codes = (np.sign(r) * np.floor(np.abs(r) + 0.5) + 128).astype(np.uint8)
    assert np.array_equal(q, exp_codes)


def test_q8_scale_is_candle_affine_multiply():
    # kv_cache.rs:101: candle's `tensor / 127.0` multiplies by (f32)(1/127); pick row maxima
    # where the IEEE quotient amax / 127 is one ulp away from that product
    rng = np.random.default_rng(11)
    cand = np.abs(rng.standard_normal(20000)).astype(np.float32) + np.float32(0.01)
    div = (cand / np.float32(127)).astype(np.float32)
    mul = (cand * np.float32(1.0 / 127.0)).astype(np.float32)
    amax = cand[div != mul][:16]
    assert amax.size == 16
    x = rng.uniform(-1, 1, (16, 64)).astype(np.float32) * amax[:, None]
    x[np.arange(16), rng.integers(0, 64, 16)] = amax
    q, s = orc.q8_quant(x)
    assert np.array_equal(s, (amax * np.float32(1.0 / 127.0)).astype(np.float32))
    assert np.all(s != (amax / np.float32(127)).astype(np.float32))
    r = x / s[:, None]
    assert np.array_equal(q, (np.sign(r) * np.floor(np.abs(r) + 0.5) + 128).astype(np.uint8))


def test_q8_quant_tie_and_zero_row():
    # s = 127/127 = 1: x = 2.5 -> 3 (half away), -2.5 -> -3
    x = np.zeros((1, 8), np.float32)
    x[0, :4] = [127.0, 2.5, -2.5, 0.5]
    q, s = orc.q8_quant(x)
    assert s[0] == 1.0
    assert list(q[0, :4]) == [255, 131, 125, 129]
    z, zs = orc.q8_quant(np.zeros((1, 16), np.float32))
    assert zs[0] == 0.0 and np.all(z == 0)
    assert np.all(orc.q8_dequant(z, zs) == 0.0)


def _attn64(q, kq, ks, vq, vs, nh, T):
    nkv, _, hd = kq.shape
    rep = nh // nkv
    k = (kq[:, :T].astype(np.float64) - 128.0) * ks[:, :T, None]
    v = (vq[:, :T].astype(np.float64) - 128.0) * vs[:, :T, None]
    out = np.zeros((nh, hd))
    for h in range(nh):
        g = h // rep
        sc = (k[g] @ q.reshape(nh, hd)[h].astype(np.float64)) / np.sqrt(hd)
        p = np.exp(sc - sc.max())
        out[h] = (p / p.sum()) @ v[g]
    return out.reshape(-1)


def _cache(nkv, S, hd, seed):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((nkv, S, hd)).astype(np.float32) * 2
    v = rng.standard_normal((nkv, S, hd)).astype(np.float32)
    kq, ks = orc.q8_quant(k)
    vq, vs = orc.q8_quant(v)
    return kq, ks, vq, vs


@pytest.mark.parametrize("T", [1, 63, 64, 65, 129])
@pytest.mark.parametrize("nh,nkv,hd", [(8, 2, 64), (4, 4, 128), (32, 8, 128)])
def test_attn_decode_matches_float64(T, nh, nkv, hd):
    S = 160
    kq, ks, vq, vs = _cache(nkv, S, hd, seed=T + nh)
    q = np.random.default_rng(7).standard_normal(nh * hd).astype(np.float32)
    y = orc.attn_decode(q, kq, ks, vq, vs, nh, T)
    e = _attn64(q, kq, ks, vq, vs, nh, T)
    scale = np.abs(e).reshape(nh, hd).max(1, keepdims=True)
    assert np.all(np.abs(y.reshape(nh, hd) - e.reshape(nh, hd)) <= 2e-6 * scale + 1e-30)


def test_attn_dot_is_a_sequential_fma_chain():
    # s = 2 (1 + 2^-12): the product s * s = 4 + 2^-9 + 2^-22 is not a float; after
    # -2 s the fma keeps the 2^-22 (2^-10 + 2^-22 exactly), a rounded multiply then
    # an add gives 2^-10 (the product's tie rounds to 4 + 2^-9)
    sv = np.float32(2.0 * (1.0 + 2.0 ** -12))
    got = orc.attn_dot([-2.0, sv], [sv, sv])
    assert got == np.float32(2.0 ** -10 + 2.0 ** -22), got
    mul_add = np.float32(np.float32(-2.0 * sv) + np.float32(sv * sv))
    assert mul_add == np.float32(2.0 ** -10) and mul_add != got
    # sequential in index order: 2^24 + 1 rounds back to 2^24, so the sum is 0; the
    # reversed order keeps the 1
    assert orc.attn_dot([2.0 ** 24, 1.0, -2.0 ** 24], [1.0, 1.0, 1.0]) == 0.0
    assert orc.attn_dot([-2.0 ** 24, 1.0, 2.0 ** 24], [1.0, 1.0, 1.0]) == 1.0
    # from zero: a single term is the rounded product
    assert orc.attn_dot([3.0], [1.0 / 3.0]) == np.float32(3.0 * np.float32(1.0 / 3.0))


def test_attn_decode_scores_use_the_fma_chain():
    # key 0 = [s, s] (codes 129, scale s = 64 + 2^-6) against q = [-64, s]: -64 s = -4097
    # exactly, s * s = 4098 + 2^-12 is not a float (it rounds to 4098), so the fma chain
    # scores 1 + 2^-12 and a multiply-then-add 1.  Key 1 is zero; values 1 and 0 give
    # y = 1 / (1 + exp(-scal * s0)): the two scores differ in y by a relative 5.7e-5,
    # far above the exp's rounding
    hd, S, T = 2, 4, 2
    sv = np.float32(64.0 + 2.0 ** -6)
    kq = np.full((1, S, hd), 128, np.uint8)
    kq[0, 0] = 129
    ks = np.full((1, S), sv, np.float32)
    vq = np.full((1, S, hd), 128, np.uint8)
    vq[0, 0] = 129
    vs = np.ones((1, S), np.float32)
    q = np.array([-64.0, sv], np.float32)
    assert np.float32(-64.0 * sv) == -4097.0 and np.float32(sv * sv) == 4098.0
    y = orc.attn_decode(q, kq, ks, vq, vs, 1, T).astype(np.float64)
    scal = np.float32(1.0 / np.sqrt(2.0))

    def expect(s0):
        return 1.0 / (1.0 + np.exp(-float(np.float32(np.float32(s0) * scal))))

    e_fma, e_mul_add = expect(1.0 + 2.0 ** -12), expect(1.0)
    assert np.all(np.abs(y - e_fma) <= 1e-6 * e_fma), (y, e_fma)
    assert np.all(np.abs(y - e_mul_add) > 3e-5 * e_mul_add), (y, e_mul_add)


def test_attn_decode_score_order_known_answer():
    # the fixed order of a score: sequential over d.  With q = [2^24, 1, -2^24, 1, 1, 0, 0, 0]
    # against a key of ones the f32 sum is 2 (2^24 + 1 rounds to 2^24), where an order
    # of four interleaved chains combined pairwise would give 1 and the exact value is 3.
    # A second key of zeros scores 0, values 1 and 0: y = 1 / (1 + exp(-s0)).
    hd, S, T = 8, 4, 2
    kq = np.full((1, S, hd), 128, np.uint8)
    kq[0, 0] = 129                      # key 0: all ones (scale 1)
    ks = np.ones((1, S), np.float32)
    vq = np.full((1, S, hd), 128, np.uint8)
    vq[0, 0] = 129                      # value 0: ones, value 1: zeros
    vs = np.ones((1, S), np.float32)
    q = np.array([2.0 ** 24, 1, -2.0 ** 24, 1, 1, 0, 0, 0], np.float32)
    y = orc.attn_decode(q, kq, ks, vq, vs, 1, T)
    scal = float(np.float32(1.0 / np.sqrt(8.0)))
    for score, want in ((2.0, True), (1.0, False), (3.0, False)):
        e = 1.0 / (1.0 + np.exp(-score * scal))
        assert (abs(float(y[0]) - e) < 1e-6) == want, (score, float(y[0]), e)
    assert np.all(y == y[0])


def test_attn_decode_value_order_known_answer():
    # the fixed order of a chunk's value sum: sequential over the keys.  Five keys of
    # equal score (p = 1 each, l = 5) with values 2^24, 1, -2^24, 1, 1: the f32 sum is 2
    # (y = 0.4); four interleaved chains combined pairwise would give 1 (y = 0.2), the
    # exact value is 3 (y = 0.6)
    hd, S, T = 4, 8, 5
    kq = np.full((1, S, hd), 128, np.uint8)
    ks = np.ones((1, S), np.float32)
    vq = np.full((1, S, hd), 129, np.uint8)
    vs = np.array([[2.0 ** 24, 1, 2.0 ** 24, 1, 1, 1, 1, 1]], np.float32)
    vq[0, 2] = 127                       # -1 * 2^24 with a positive scale
    y = orc.attn_decode(np.ones(hd, np.float32), kq, ks, vq, vs, 1, T)
    assert np.all(y == np.float32(2.0) / np.float32(5.0)), y


def test_attn_decode_gqa_head_map():
    # each KV head holds one constant value vector: output of head h must be that of kv head h // rep
    nh, nkv, hd, S, T = 8, 2, 64, 70, 70
    kq = np.full((nkv, S, hd), 128, np.uint8)
    ks = np.ones((nkv, S), np.float32)
    vq = np.zeros((nkv, S, hd), np.uint8)
    vq[0] = 128 + 10
    vq[1] = 128 - 20
    vs = np.ones((nkv, S), np.float32)
    y = orc.attn_decode(np.ones(nh * hd, np.float32), kq, ks, vq, vs, nh, T).reshape(nh, hd)
    rep = nh // nkv
    for h in range(nh):
        assert np.all(y[h] == (10.0 if h // rep == 0 else -20.0)), h


def test_argmax_last_of_equal_maxima():
    assert orc.argmax(np.array([1, 5, 2, 5, 0], np.float32)) == 3
    assert orc.argmax(np.array([-3, -1, -1], np.float32)) == 2
    assert orc.argmax(np.array([7.0], np.float32)) == 0
    assert orc.argmax(np.array([0.0, -0.0], np.float32)) == 1


class TinyCfg:
    hidden, n_layers, n_heads, n_kv_heads, head_dim = 64, 2, 4, 2, 16
    intermediate, vocab, rope_theta, max_seq, eps = 128, 50, 10000.0, 80, 1e-5


def tiny_weights(cfg, seed=0):
    rng = np.random.default_rng(seed)

    def lin(n, k):
        return orc.pack(weights(n, k, int(rng.integers(1 << 30))))

    def norm(n):
        return (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)

    kvd = cfg.n_kv_heads * cfg.head_dim
    layers = [{"norm1": norm(cfg.hidden), "norm2": norm(cfg.hidden),
               "q": lin(cfg.n_heads * cfg.head_dim, cfg.hidden), "k": lin(kvd, cfg.hidden),
               "v": lin(kvd, cfg.hidden), "o": lin(cfg.hidden, cfg.n_heads * cfg.head_dim),
               "gate": lin(cfg.intermediate, cfg.hidden), "up": lin(cfg.intermediate, cfg.hidden),
               "down": lin(cfg.hidden, cfg.intermediate)} for _ in range(cfg.n_layers)]
    return {"embed": rng.standard_normal((cfg.vocab, cfg.hidden)).astype(np.float32),
            "norm_f": norm(cfg.hidden), "lm_head": lin(cfg.vocab, cfg.hidden), "layers": layers}


def test_oracle_llama_is_causal_and_deterministic():
    cfg = TinyCfg()
    w = tiny_weights(cfg)
    prompt = [3, 14, 15, 9, 26, 5]
    a = OracleLlama(cfg, w)
    la = [a.forward_one(t) for t in prompt]
    b = OracleLlama(cfg, w)
    lb = [b.forward_one(t) for t in prompt[:3] + [0, 0]]
    for i in range(3):
        assert np.array_equal(la[i], lb[i])   # later tokens do not change earlier logits
    assert not np.array_equal(la[3], lb[3])
    g1 = OracleLlama(cfg, w).generate(prompt, 5)
    g2 = OracleLlama(cfg, w).generate(prompt, 5)
    assert np.array_equal(g1, g2) and g1.shape == (5,)
    assert np.all((g1 >= 0) & (g1 < cfg.vocab))


def test_dense_linear_exact_small_integers():
    # products and partial sums are small integers: every order gives the exact dot
    rng = np.random.default_rng(3)
    for m, n, k in [(1, 1, 4), (2, 5, 12), (3, 7, 520)]:
        x = rng.integers(-8, 9, (m, k)).astype(np.float32)
        w = rng.integers(-8, 9, (n, k)).astype(np.float32)
        y = orc.dense_linear(x, w)
        assert np.array_equal(y, (x.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32))


def test_dense_linear_float64_and_bf16_widening():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 4096)).astype(np.float32)
    w = (rng.standard_normal((33, 4096)) * 0.02).astype(np.float32)
    y = orc.dense_linear(x, w)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()
    bits = (w.view(np.uint32) >> 16).astype(np.uint16)  # truncated to bf16 bits
    wide = (bits.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(orc.dense_linear(x, bits), orc.dense_linear(x, wide))


def test_dense_linear_lane_order():
    # B = 2^25 absorbs t = 2^-30 (t is far below half an ulp of B).  k = 512: lane 0
    # holds chunks 0 and 64 (elements 0-3, 256-259), lane 1 chunk 1 (elements 4-7),
    # lane 32 chunk 32 (elements 128-131).  A fold over k in index order gives
    # (B + t) - B = 0 in both cases below; the fixed order keeps t.
    k, B, t = 512, 2.0 ** 25, 2.0 ** -30
    x = np.ones((1, k), np.float32)
    # chunk-to-lane map: B and -B meet inside lane 0, t sits in lane 1
    w = np.zeros((1, k), np.float32)
    w[0, 0], w[0, 256], w[0, 4] = B, -B, t
    assert orc.dense_linear(x, w)[0, 0] == np.float32(t)
    # butterfly, xor 32 first: lane 0 (B) meets lane 32 (-B) before lane 1 (t)
    w = np.zeros((1, k), np.float32)
    w[0, 0], w[0, 128], w[0, 4] = B, -B, t
    assert orc.dense_linear(x, w)[0, 0] == np.float32(t)
    # and the fold that the order replaces loses it
    assert np.float32(np.float32(np.float32(B) + np.float32(t)) - np.float32(B)) == 0.0
