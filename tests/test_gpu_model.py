"""GPU parity of the decoder ops (include/bitllama.h) and of the end-to-end ternary
decoder (bitlinear.model.BitLlamaHip) against the CPU oracle.

Bar: everything bit-exact.  The RoPE rows, the Q8 cache codes and scales, the
attention outputs (the oracle restates the kernels' fixed summation order), the
residual stream, the logits and the greedy tokens.  The attention order itself is
pinned against float64 in test_model_oracle.py (relative 2e-6)."""
import ctypes

import numpy as np
import pytest
import torch

import bitlinear as bl
from bitlinear.model import BitLlamaHip
from oracle import oracle as orc
from oracle.llama_oracle import OracleLlama
from test_model_oracle import TinyCfg, tiny_weights

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]

DEV = "cuda"


def _bits(a):
    a = np.ascontiguousarray(a, np.float32).copy()
    a[np.isnan(a)] = np.float32("nan")
    return a.view(np.uint32)


def assert_same(got, ref, what=""):
    got = got.detach().cpu().numpy() if torch.is_tensor(got) else np.asarray(got)
    g, r = _bits(got), _bits(ref)
    bad = np.flatnonzero(g.reshape(-1) != r.reshape(-1))
    assert bad.size == 0, "%s: %d mismatches, first at %d: %r vs %r" % (
        what, bad.size, bad[0], got.reshape(-1)[bad[0]], np.asarray(ref).reshape(-1)[bad[0]])


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class Cache:
    def __init__(self, nkv, S, hd):
        self.k = torch.full((nkv, S, hd), 7, dtype=torch.uint8, device=DEV)
        self.v = torch.full((nkv, S, hd), 9, dtype=torch.uint8, device=DEV)
        self.ks = torch.full((nkv, S), 0.5, dtype=torch.float32, device=DEV)
        self.vs = torch.full((nkv, S), 0.25, dtype=torch.float32, device=DEV)
        self.c = bl.BtlKvQ8(self.k.data_ptr(), self.v.data_ptr(), self.ks.data_ptr(), self.vs.data_ptr(), nkv, S, hd)

    def host(self):
        return (self.k.cpu().numpy(), self.ks.cpu().numpy(), self.v.cpu().numpy(), self.vs.cpu().numpy())


def rope_dev(theta, hd, S):
    c = np.zeros((S, hd // 2), np.float32)
    s = np.zeros_like(c)
    bl.check(bl.lib.btl_rope_table(theta, hd, S, c.ctypes.data, s.ctypes.data))
    return c, s, torch.from_numpy(c).to(DEV), torch.from_numpy(s).to(DEV)


def test_rope_table_matches_oracle():
    c, s, _, _ = rope_dev(500000.0, 128, 700)
    oc, osn = orc.rope_table(500000.0, 128, 700)
    assert np.array_equal(c, oc) and np.array_equal(s, osn)


@pytest.mark.parametrize("nh,nkv,hd", [(4, 2, 64), (32, 8, 128), (3, 1, 2)])
@pytest.mark.parametrize("m,pos,dpos", [(1, 0, False), (1, 37, True), (5, 60, False), (70, 0, False)])
def test_rope_kv_append_bitexact(nh, nkv, hd, m, pos, dpos):
    print("rope_kv_append", nh, nkv, hd, m, pos, dpos, flush=True)
    S = 160
    rng = np.random.default_rng(m * 100 + pos + hd)
    q = rng.standard_normal((m, nh * hd)).astype(np.float32)
    k = (rng.standard_normal((m, nkv * hd)) * 3).astype(np.float32)
    v = rng.standard_normal((m, nkv * hd)).astype(np.float32)
    if m > 1:
        v[1, :hd] = 0.0  # a zero head row: codes 0, scale 0
    cos, sin, dc, ds = rope_dev(10000.0, hd, S)
    cache = Cache(nkv, S, hd)
    qt, kt, vt = (torch.from_numpy(a).to(DEV) for a in (q, k, v))
    qo = torch.empty_like(qt)
    d_pos = torch.tensor([pos], dtype=torch.int32, device=DEV) if dpos else None
    bl.check(bl.lib.btl_rope_kv_append(qt.data_ptr(), kt.data_ptr(), vt.data_ptr(), m, nh, ctypes.byref(cache.c),
                                       0 if dpos else pos, d_pos.data_ptr() if dpos else None, dc.data_ptr(),
                                       ds.data_ptr(), qo.data_ptr(), stream()))
    kq, ks, vq, vs = cache.host()
    for t in range(m):
        p = pos + t
        assert_same(qo[t], orc.rope_apply(q[t].reshape(nh, hd), cos[p], sin[p]).reshape(-1), "q rope")
        kr = orc.rope_apply(k[t].reshape(nkv, hd), cos[p], sin[p])
        ekq, eks = orc.q8_quant(kr)
        evq, evs = orc.q8_quant(v[t].reshape(nkv, hd))
        assert np.array_equal(kq[:, p], ekq) and np.array_equal(vq[:, p], evq)
        assert_same(ks[:, p], eks, "k scale")
        assert_same(vs[:, p], evs, "v scale")
    # rows outside [pos, pos + m) untouched
    untouched = [r for r in range(S) if not pos <= r < pos + m]
    assert np.all(kq[:, untouched] == 7) and np.all(ks[:, untouched] == 0.5)


def test_rope_kv_append_rejects_out_of_range_positions():
    cache = Cache(2, 16, 64)
    x = torch.zeros((4, 4 * 64), device=DEV)
    y = torch.zeros((4, 2 * 64), device=DEV)
    _, _, dc, ds = rope_dev(10000.0, 64, 16)
    st = bl.lib.btl_rope_kv_append(x.data_ptr(), y.data_ptr(), y.data_ptr(), 4, 4, ctypes.byref(cache.c), 14, None,
                                   dc.data_ptr(), ds.data_ptr(), x.data_ptr(), stream())
    assert st == bl.BTL_ERR_SHAPE
    assert b"outside the cache" in bl.lib.btl_last_error()


def _fill_cache(cache, T, seed):
    nkv, S, hd = cache.k.shape
    rng = np.random.default_rng(seed)
    k = (rng.standard_normal((nkv, S, hd)) * 2).astype(np.float32)
    v = rng.standard_normal((nkv, S, hd)).astype(np.float32)
    kq, ks = orc.q8_quant(k)
    vq, vs = orc.q8_quant(v)
    cache.k.copy_(torch.from_numpy(kq))
    cache.v.copy_(torch.from_numpy(vq))
    cache.ks.copy_(torch.from_numpy(ks))
    cache.vs.copy_(torch.from_numpy(vs))


@pytest.mark.parametrize("nh,nkv,hd", [(4, 2, 64), (32, 8, 128), (16, 1, 128)])
@pytest.mark.parametrize("m,pos", [(1, 0), (1, 63), (1, 64), (1, 199), (3, 61), (70, 0), (40, 100)])
def test_attention_bitexact(nh, nkv, hd, m, pos):
    print("attention", nh, nkv, hd, m, pos, flush=True)
    S = 256
    cache = Cache(nkv, S, hd)
    _fill_cache(cache, S, seed=nh + m + pos)
    q = np.random.default_rng(pos + 5).standard_normal((m, nh * hd)).astype(np.float32)
    qt = torch.from_numpy(q).to(DEV)
    out = torch.full((m, nh * hd), 3.0, device=DEV)
    ws_bytes = bl.lib.btl_attention_workspace_bytes(m, nh, ctypes.byref(cache.c))
    ws = torch.full((ws_bytes // 4 + 64,), 1234.5, dtype=torch.float32, device=DEV)  # garbage is fine
    bl.check(bl.lib.btl_attention(qt.data_ptr(), m, nh, ctypes.byref(cache.c), pos, None, out.data_ptr(),
                                  ws.data_ptr(), ws_bytes, stream()))
    kq, ks, vq, vs = cache.host()
    o = out.cpu().numpy()
    for i in range(m):
        e = orc.attn_decode(q[i], kq, ks, vq, vs, nh, pos + i + 1)
        assert_same(o[i], e, "query %d" % i)


def test_attention_device_position():
    nh, nkv, hd, S = 8, 2, 128, 300
    cache = Cache(nkv, S, hd)
    _fill_cache(cache, S, seed=11)
    q = np.random.default_rng(12).standard_normal((1, nh * hd)).astype(np.float32)
    qt = torch.from_numpy(q).to(DEV)
    kq, ks, vq, vs = cache.host()
    for p in (0, 130, 299):
        d_pos = torch.tensor([p], dtype=torch.int32, device=DEV)
        out = torch.empty((1, nh * hd), device=DEV)
        bl.check(bl.lib.btl_attention(qt.data_ptr(), 1, nh, ctypes.byref(cache.c), 0, d_pos.data_ptr(),
                                      out.data_ptr(), None, 0, stream()))
        assert_same(out[0], orc.attn_decode(q[0], kq, ks, vq, vs, nh, p + 1), "pos %d" % p)


@pytest.mark.parametrize("merge", [1, 0])
@pytest.mark.parametrize("nh,nkv,hd", [(4, 2, 64), (32, 8, 128), (4, 4, 128), (8, 1, 16)])
@pytest.mark.parametrize("pos,dpos", [(0, False), (63, True), (64, False), (130, True), (255, False)])
def test_rope_append_attention_one_token(nh, nkv, hd, pos, dpos, merge, tune):
    # m = 1: RoPE, the Q8 append and the attention in one kernel, the chunk
    # merge in the same launch (merge=1) or a second one; same bits as
    # btl_rope_kv_append + btl_attention and as the oracle
    print("rope_append_attention", nh, nkv, hd, pos, dpos, merge, flush=True)
    tune("BTL_ATTN_MERGE", merge)
    S = 256
    rng = np.random.default_rng(pos * 7 + hd + nh)
    q = rng.standard_normal((1, nh * hd)).astype(np.float32)
    k = (rng.standard_normal((1, nkv * hd)) * 2).astype(np.float32)
    v = rng.standard_normal((1, nkv * hd)).astype(np.float32)
    cos, sin, dc, ds = rope_dev(500000.0, hd, S)
    cache = Cache(nkv, S, hd)
    _fill_cache(cache, S, seed=pos + 1)
    kq0, ks0, vq0, vs0 = cache.host()
    qt, kt, vt = (torch.from_numpy(a).to(DEV) for a in (q, k, v))
    out = torch.full((1, nh * hd), 3.0, device=DEV)
    d_pos = torch.tensor([pos], dtype=torch.int32, device=DEV) if dpos else None
    bl.check(bl.lib.btl_rope_append_attention(qt.data_ptr(), kt.data_ptr(), vt.data_ptr(), 1, nh, ctypes.byref(cache.c),
                                              0 if dpos else pos, d_pos.data_ptr() if dpos else None, dc.data_ptr(),
                                              ds.data_ptr(), out.data_ptr(), None, 0, stream()))
    assert_same(qt, q, "q not modified")
    kq, ks, vq, vs = cache.host()
    ekq, eks = orc.q8_quant(orc.rope_apply(k[0].reshape(nkv, hd), cos[pos], sin[pos]))
    evq, evs = orc.q8_quant(v[0].reshape(nkv, hd))
    assert np.array_equal(kq[:, pos], ekq) and np.array_equal(vq[:, pos], evq)
    assert_same(ks[:, pos], eks, "k scale")
    assert_same(vs[:, pos], evs, "v scale")
    other = [r for r in range(S) if r != pos]
    assert np.array_equal(kq[:, other], kq0[:, other]) and np.array_equal(vs[:, other], vs0[:, other])
    qr = orc.rope_apply(q[0].reshape(nh, hd), cos[pos], sin[pos]).reshape(-1)
    assert_same(out[0], orc.attn_decode(qr, kq, ks, vq, vs, nh, pos + 1), "attention")


@pytest.mark.parametrize("pos", [4095, 8190])
def test_rope_append_attention_one_token_long_cache(pos, tune):
    # more than 64 key chunks (the merge walks them in several 64-chunk passes),
    # Llama-3-8B head layout; then repeated calls (the merge counters must be
    # back at zero after each launch) and a device position outside the cache
    nh, nkv, hd, S = 32, 8, 128, 8192
    print("rope_append_attention long", pos, flush=True)
    rng = np.random.default_rng(pos)
    q = rng.standard_normal((1, nh * hd)).astype(np.float32)
    k = rng.standard_normal((1, nkv * hd)).astype(np.float32)
    v = rng.standard_normal((1, nkv * hd)).astype(np.float32)
    cos, sin, dc, ds = rope_dev(500000.0, hd, S)
    cache = Cache(nkv, S, hd)
    _fill_cache(cache, S, seed=pos)
    qt, kt, vt = (torch.from_numpy(a).to(DEV) for a in (q, k, v))
    d_pos = torch.tensor([pos], dtype=torch.int32, device=DEV)
    outs = []
    for merge in (1, 1, 0, 1):
        tune("BTL_ATTN_MERGE", merge)
        out = torch.full((1, nh * hd), 3.0, device=DEV)
        bl.check(bl.lib.btl_rope_append_attention(qt.data_ptr(), kt.data_ptr(), vt.data_ptr(), 1, nh,
                                                  ctypes.byref(cache.c), 0, d_pos.data_ptr(), dc.data_ptr(),
                                                  ds.data_ptr(), out.data_ptr(), None, 0, stream()))
        outs.append(out.cpu().numpy())
    kq, ks, vq, vs = cache.host()
    qr = orc.rope_apply(q[0].reshape(nh, hd), cos[pos], sin[pos]).reshape(-1)
    ref = orc.attn_decode(qr, kq, ks, vq, vs, nh, pos + 1)
    for i, o in enumerate(outs):
        assert_same(o[0], ref, "call %d" % i)
    tune("BTL_ATTN_MERGE", 1)
    bad = torch.tensor([S], dtype=torch.int32, device=DEV)
    out = torch.full((1, nh * hd), 3.0, device=DEV)
    bl.check(bl.lib.btl_rope_append_attention(qt.data_ptr(), kt.data_ptr(), vt.data_ptr(), 1, nh,
                                              ctypes.byref(cache.c), 0, bad.data_ptr(), dc.data_ptr(),
                                              ds.data_ptr(), out.data_ptr(), None, 0, stream()))
    assert torch.isnan(out).all(), "a device position outside the cache gives NaN"
    kq2, ks2, _, _ = cache.host()
    assert np.array_equal(kq2, kq) and np.array_equal(ks2, ks), "no append"


@pytest.mark.parametrize("nh,nkv,hd", [(32, 8, 128), (32, 2, 64)])
def test_rope_append_attention_one_token_merge_sequence(nh, nkv, hd, tune):
    # The merge in the launch over a sequence of calls on one caller workspace:
    # falling and rising positions (the workspace keeps the partials of earlier
    # calls), the workspace overwritten with other bits between some calls,
    # more key chunks than the merge loads ahead (16), the last call repeated;
    # the counters must be back at zero after every launch, each call against
    # the oracle.
    print("rope_append_attention sequence", nh, nkv, hd, flush=True)
    tune("BTL_ATTN_MERGE", 1)
    S = 2048
    cos, sin, dc, ds = rope_dev(500000.0, hd, S)
    cache = Cache(nkv, S, hd)
    _fill_cache(cache, S, seed=nh + nkv)
    wn = bl.lib.btl_attention_workspace_bytes(1, nh, ctypes.byref(cache.c))
    ws = torch.zeros((wn,), dtype=torch.uint8, device=DEV)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(3)
    plan = [1500, 300, 1500, 64, 63, 2047, 1100, 1100]
    for i, pos in enumerate(plan):
        rng = np.random.default_rng(100 + i)
        q = rng.standard_normal((1, nh * hd)).astype(np.float32)
        k = rng.standard_normal((1, nkv * hd)).astype(np.float32)
        v = rng.standard_normal((1, nkv * hd)).astype(np.float32)
        if i in (3, 6):
            ws.random_(0, 256, generator=gen)
        qt, kt, vt = (torch.from_numpy(a).to(DEV) for a in (q, k, v))
        d_pos = torch.tensor([pos], dtype=torch.int32, device=DEV)
        out = torch.full((1, nh * hd), 3.0, device=DEV)
        bl.check(bl.lib.btl_rope_append_attention(qt.data_ptr(), kt.data_ptr(), vt.data_ptr(), 1, nh,
                                                  ctypes.byref(cache.c), 0, d_pos.data_ptr(), dc.data_ptr(),
                                                  ds.data_ptr(), out.data_ptr(), ctypes.c_void_p(ws.data_ptr()),
                                                  wn, stream()))
        bl.check(bl.lib.btl_check_faults(stream()))
        kq, ks, vq, vs = cache.host()
        qr = orc.rope_apply(q[0].reshape(nh, hd), cos[pos], sin[pos]).reshape(-1)
        assert_same(out[0], orc.attn_decode(qr, kq, ks, vq, vs, nh, pos + 1), "call %d pos %d" % (i, pos))


@pytest.mark.parametrize("m,pos", [(2, 0), (17, 40), (70, 60)])
def test_rope_append_attention_many_tokens(m, pos):
    nh, nkv, hd, S = 8, 2, 128, 200
    rng = np.random.default_rng(m + pos)
    q = rng.standard_normal((m, nh * hd)).astype(np.float32)
    k = rng.standard_normal((m, nkv * hd)).astype(np.float32)
    v = rng.standard_normal((m, nkv * hd)).astype(np.float32)
    cos, sin, dc, ds = rope_dev(10000.0, hd, S)
    a, b = Cache(nkv, S, hd), Cache(nkv, S, hd)
    _fill_cache(a, S, seed=3)
    _fill_cache(b, S, seed=3)
    qt, kt, vt = (torch.from_numpy(x).to(DEV) for x in (q, k, v))
    out = torch.empty((m, nh * hd), device=DEV)
    bl.check(bl.lib.btl_rope_append_attention(qt.data_ptr(), kt.data_ptr(), vt.data_ptr(), m, nh, ctypes.byref(a.c),
                                              pos, None, dc.data_ptr(), ds.data_ptr(), out.data_ptr(), None, 0,
                                              stream()))
    qr = torch.empty_like(qt)
    bl.check(bl.lib.btl_rope_kv_append(qt.data_ptr(), kt.data_ptr(), vt.data_ptr(), m, nh, ctypes.byref(b.c), pos,
                                       None, dc.data_ptr(), ds.data_ptr(), qr.data_ptr(), stream()))
    out2 = torch.empty_like(out)
    bl.check(bl.lib.btl_attention(qr.data_ptr(), m, nh, ctypes.byref(b.c), pos, None, out2.data_ptr(), None, 0,
                                  stream()))
    assert torch.equal(a.k, b.k) and torch.equal(a.vs, b.vs)
    assert_same(out, out2.cpu().numpy(), "two-call path")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("dim,off", [(320, 0), (4096, 0), (4100, 0), (322, 0), (4096, 1), (5, 0)])
def test_embedding(dtype, dim, off):
    # whole-row copies: 16-byte (f32) / 8-byte (bf16) loads when dim % 4 == 0 and
    # the pointers allow it, element loads otherwise (off: an output view one
    # float past an aligned start); several 1024-element blocks per row
    vocab = 1000
    table = torch.randn((vocab, dim), device=DEV).to(dtype)
    ids = torch.tensor([5, 999, 0, -1, 1000, 5], dtype=torch.int32, device=DEV)
    buf = torch.full((6 * dim + off,), 7.0, device=DEV)
    out = buf[off:].view(6, dim)
    bl.check(bl.lib.btl_embedding(table.data_ptr(), bl.BTL_BF16 if dtype == torch.bfloat16 else bl.BTL_F32, vocab,
                                  dim, ids.data_ptr(), 6, out.data_ptr(), stream()))
    t = table.float()
    exp = torch.stack([t[5], t[999], t[0], torch.zeros(dim, device=DEV), torch.zeros(dim, device=DEV), t[5]])
    assert torch.equal(out, exp)
    if off:
        assert float(buf[0]) == 7.0


def test_greedy_next():
    cases = [np.array([1, 5, 2, 5, 0], np.float32), np.array([-3, -1, -1, -7], np.float32),
             np.array([0.0, -0.0, -1.0, 0.0, -0.0], np.float32)]
    rng = np.random.default_rng(1)
    big = rng.standard_normal(128256).astype(np.float32)
    big[77777] = big[1234] = 9.0  # tie: the later index wins
    cases.append(big)
    cases.append(rng.standard_normal(1001).astype(np.float32))  # tail of n % 4
    cases += [np.array([2.0], np.float32), np.array([1.0, 3.0, 3.0], np.float32)]
    sp = rng.standard_normal(128256).astype(np.float32)
    sp[[3, 128255]] = np.inf  # equal infinities: the later one
    cases.append(sp)
    # many workgroups, several passes each; the maximum in the last element's
    # workgroup and a tie far apart
    huge = rng.standard_normal(10_000_003).astype(np.float32)
    huge[[17, 10_000_002]] = 50.0
    cases.append(huge)
    neg = -np.abs(rng.standard_normal(50_001)).astype(np.float32) - 1.0
    neg[49_999] = -0.5
    cases.append(neg)
    for x in cases:
        xt = torch.from_numpy(x).to(DEV)
        nid = torch.full((1,), -5, dtype=torch.int32, device=DEV)
        bl.check(bl.lib.btl_greedy_next(xt.data_ptr(), x.size, nid.data_ptr(), None, None, 0, stream()))
        assert int(nid.item()) == orc.argmax(x)
    # device bookkeeping: log[pos + 1] = id, ++pos
    x = torch.from_numpy(cases[0]).to(DEV)
    nid = torch.zeros((1,), dtype=torch.int32, device=DEV)
    pos = torch.tensor([4], dtype=torch.int32, device=DEV)
    log = torch.full((8,), -1, dtype=torch.int32, device=DEV)
    for _ in range(4):
        bl.check(bl.lib.btl_greedy_next(x.data_ptr(), 5, nid.data_ptr(), pos.data_ptr(), log.data_ptr(), 8, stream()))
    assert int(pos.item()) == 8
    assert log.cpu().tolist() == [-1, -1, -1, -1, -1, 3, 3, 3]  # log[8] is outside: not written


@pytest.mark.parametrize("m,k,ns", [(1, 256, (96, 40)), (1, 4096, (96, 40)), (1, 4096, (8192, 96)),
                                    (3, 4096, (96, 40)), (70, 512, (96, 40))])
@pytest.mark.parametrize("inplace", [False, True])
def test_add_rmsnorm_linear_group(m, k, ns, inplace):
    # (1, 4096, (8192, 96)): 518 row blocks, over the limit for the fused decode prologue
    print("add_rmsnorm", m, k, ns, inplace, flush=True)
    rng = np.random.default_rng(m + k)
    h = rng.standard_normal((m, k)).astype(np.float32)
    d = rng.standard_normal((m, k)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    layers = []
    for i, n in enumerate(ns):
        wb, sw = orc.pack((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        layers.append((bl.PackedTensor(torch.from_numpy(wb).to(DEV), sw, (n, k), DEV), wb, sw, n))
    ht, dt, gt = (torch.from_numpy(a).to(DEV) for a in (h, d, g))
    ho = ht if inplace else torch.full_like(ht, 5.0)
    outs = [torch.empty((m, n), device=DEV) for (_, _, _, n) in layers]
    cs = [L[0].as_c() for L in layers]
    arr = (ctypes.POINTER(bl.BtlPacked) * 2)(*[ctypes.pointer(c) for c in cs])
    ys = (ctypes.c_void_p * 2)(*[o.data_ptr() for o in outs])
    bl.check(bl.lib.btl_add_rmsnorm_linear_group(arr, ys, 2, ht.data_ptr(), dt.data_ptr(), ho.data_ptr(),
                                                 gt.data_ptr(), 1e-5, m, k, bl.BTL_F32, None, 0, stream()))
    hs = (h + d).astype(np.float32)
    assert_same(ho, hs, "residual")
    if not inplace:
        assert_same(ht, h, "input untouched")
    xn = orc.rmsnorm(hs, g, 1e-5)
    for o, (_, wb, sw, n) in zip(outs, layers):
        assert_same(o, orc.forward_i8(xn, wb, n, sw)[0], "layer")
    # delta = NULL: RMSNorm of h only, nothing written
    h2 = torch.from_numpy(h).to(DEV)
    bl.check(bl.lib.btl_add_rmsnorm_linear_group(arr, ys, 2, h2.data_ptr(), None, None, gt.data_ptr(), 1e-5, m, k,
                                                 bl.BTL_F32, None, 0, stream()))
    assert_same(h2, h, "h untouched")
    assert_same(outs[0], orc.forward_i8(orc.rmsnorm(h, g, 1e-5), layers[0][1], ns[0], layers[0][2])[0], "plain")


@pytest.mark.parametrize("m,k,n,fuse", [(1, 256, 512, "1"), (1, 4096, 14336, "1"), (2, 512, 96, "1"),
                                        (4, 4096, 1000, "1"), (9, 512, 256, "1"), (70, 256, 512, "1"),
                                        (1, 4096, 1000, "0"), (1, 14336, 300, "0"), (1, 2048, 7, "0"),
                                        (1, 1024, 300, "1"), (1, 3008, 150, "1"), (1, 2048, 4001, "1")])
@pytest.mark.parametrize("with_delta", [False, True])
def test_add_rmsnorm_swiglu(m, k, n, fuse, with_delta, tune):
    # decode rows (m <= 4): the gate/up kernel writes silu(gate) * up from its epilogue.
    # One row, 1024 <= k <= 4096: without delta the RMSNorm runs in the quantising
    # waves of the row-group form's gate/up pairing (two token groups per thread,
    # the norm weight copied into LDS at the start; k = 3008 leaves half-empty
    # groups and a zero block); with delta a separate one-workgroup transform runs
    # first.  fuse "0" forces the separate norm kernel (row-group pairing with
    # ragged n: rows past the end of a workgroup's span)
    print("add_rmsnorm_swiglu", m, k, n, fuse, with_delta, flush=True)
    tune("BTL_FUSE_DEC", fuse)
    rng = np.random.default_rng(m * 31 + k + n)
    h = rng.standard_normal((m, k)).astype(np.float32)
    d = rng.standard_normal((m, k)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    wg, sg = orc.pack((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    wu, su = orc.pack((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    pg = bl.PackedTensor(torch.from_numpy(wg).to(DEV), sg, (n, k), DEV)
    pu = bl.PackedTensor(torch.from_numpy(wu).to(DEV), su, (n, k), DEV)
    ht, dt, gt = (torch.from_numpy(a).to(DEV) for a in (h, d, g))
    ho = torch.zeros_like(ht)
    out = torch.full((m, n), 9.0, device=DEV)
    cg, cu = pg.as_c(), pu.as_c()
    bl.check(bl.lib.btl_add_rmsnorm_swiglu(ctypes.byref(cg), ctypes.byref(cu), ht.data_ptr(),
                                           dt.data_ptr() if with_delta else None, ho.data_ptr() if with_delta else None,
                                           gt.data_ptr(), 1e-5, m, k, out.data_ptr(), None, 0, stream()))
    hs = (h + d).astype(np.float32) if with_delta else h
    if with_delta:
        assert_same(ho, hs, "residual")
    xn = orc.rmsnorm(hs, g, 1e-5)
    e = orc.swiglu(orc.forward_i8(xn, wg, n, sg)[0], orc.forward_i8(xn, wu, n, su)[0])
    assert_same(out, e, "swiglu")


@pytest.mark.parametrize("k", [512, 4096, 14336])
def test_swiglu_group_one_token_fused(k):
    # m = 1, f32: the SwiGLU runs inside the decode kernel's prologue
    rng = np.random.default_rng(k)
    gte = (rng.standard_normal((1, k)) * 3).astype(np.float32)
    up = rng.standard_normal((1, k)).astype(np.float32)
    n = 200
    wb, sw = orc.pack((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    pt = bl.PackedTensor(torch.from_numpy(wb).to(DEV), sw, (n, k), DEV)
    y = bl.swiglu_linear_group([pt], torch.from_numpy(gte).to(DEV), torch.from_numpy(up).to(DEV))[0]
    assert_same(y, orc.forward_i8(orc.swiglu(gte, up), wb, n, sw)[0], "swiglu fused")


@pytest.mark.parametrize("form", ["rq", "dec"])
@pytest.mark.parametrize("kind", ["rmsnorm", "add_rmsnorm", "swiglu"])
@pytest.mark.parametrize("k", [1024, 1088, 2048, 3008, 4096])
def test_one_token_transforms_both_forms(k, kind, form, tune):
    # m = 1, f32, k <= 4096: the transform runs in the row-group form's
    # quantising waves (rq) or in the decode kernel's prologue (dec); both
    # must give the oracle's bits.  n = 150 leaves a partial row group.
    print("one-token transform", k, kind, form, flush=True)
    if form == "dec":
        tune("BTL_DEC_RQ", "0")
    rng = np.random.default_rng(k * 3 + len(kind))
    x = (rng.standard_normal((1, k)) * 2).astype(np.float32)
    x2 = rng.standard_normal((1, k)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    n = 150
    wb, sw = orc.pack((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    pt = bl.PackedTensor(torch.from_numpy(wb).to(DEV), sw, (n, k), DEV)
    xt, x2t, gt = (torch.from_numpy(a).to(DEV) for a in (x, x2, g))
    if kind == "swiglu":
        y = bl.swiglu_linear_group([pt], xt, x2t)[0]
        assert_same(y, orc.forward_i8(orc.swiglu(x, x2), wb, n, sw)[0], "swiglu")
        return
    out = torch.empty((1, n), device=DEV)
    c = pt.as_c()
    arr = (ctypes.POINTER(bl.BtlPacked) * 1)(ctypes.pointer(c))
    ys = (ctypes.c_void_p * 1)(out.data_ptr())
    ho = torch.full_like(xt, 5.0)
    add = kind == "add_rmsnorm"
    bl.check(bl.lib.btl_add_rmsnorm_linear_group(arr, ys, 1, xt.data_ptr(), x2t.data_ptr() if add else None,
                                                 ho.data_ptr() if add else None, gt.data_ptr(), 1e-5, 1, k,
                                                 bl.BTL_F32, None, 0, stream()))
    hs = (x + x2).astype(np.float32) if add else x
    if add:
        assert_same(ho, hs, "residual")
    assert_same(out, orc.forward_i8(orc.rmsnorm(hs, g, 1e-5), wb, n, sw)[0], kind)


@pytest.mark.parametrize("m,k,n,xdt", [(1, 4096, 4096, "f32"), (1, 14336, 4096, "f32"), (1, 4096, 1000, "f32"),
                                        (1, 1024, 150, "bf16"), (1, 512, 96, "f32"), (1, 1000, 40, "f32"),
                                        (2, 4096, 300, "f32"), (2, 2048, 200, "bf16"), (2, 14336, 300, "f32"),
                                        (2, 6144, 90, "bf16"), (3, 1024, 100, "f32"),
                                        (70, 512, 200, "f32")])
def test_linear_residual(m, k, n, xdt):
    # y = resid + x W^T.  One row, 1024 <= k <= 16384 (and two rows, k <= 4096):
    # the add runs in the row-group decode kernel's epilogue; k < 1024, k % 64 != 0,
    # three rows and the GEMM add in a launch after the product.
    print("linear_residual", m, k, n, xdt, flush=True)
    rng = np.random.default_rng(m * 7 + k + n)
    x = (rng.standard_normal((m, k)) * 2).astype(np.float32)
    if xdt == "bf16":
        xt = torch.from_numpy(x).to(DEV).to(torch.bfloat16)
        x = xt.float().cpu().numpy()
    else:
        xt = torch.from_numpy(x).to(DEV)
    r = rng.standard_normal((m, n)).astype(np.float32)
    wb, sw = orc.pack((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    pt = bl.PackedTensor(torch.from_numpy(wb).to(DEV), sw, (n, k), DEV)
    rt = torch.from_numpy(r).to(DEV)
    y = bl.linear_residual(pt, xt, rt)
    assert_same(rt, r, "residual untouched")
    assert_same(y, (r + orc.forward_i8(x, wb, n, sw)[0]).astype(np.float32), "resid + x W^T")


def test_linear_residual_rejects_overlap():
    k, n = 1024, 64
    pt = bl.PackedTensor(torch.zeros((n * k // 4,), dtype=torch.uint8, device=DEV), 1.0, (n, k), DEV)
    c = pt.as_c()
    x = torch.zeros((1, k), device=DEV)
    r = torch.zeros((1, 2 * n), device=DEV)
    for y, xx in ((r[:, 1:], x), (x[:, :n], x)):  # y over resid; y over the input
        st = bl.lib.btl_linear_residual(ctypes.byref(c), xx.data_ptr(), bl.BTL_F32, 1, k, r[:, :n].data_ptr(),
                                        y.data_ptr(), None, 0, stream())
        assert st == bl.BTL_ERR_LAYOUT


@pytest.mark.parametrize("case", ["tiny", "huge"])
@pytest.mark.parametrize("k", [2048, 4096])
def test_one_token_rmsnorm_special_values(k, case):
    # RMSNorm in the quantising waves of one token row with values at the
    # edges of f32: zeros of both signs, a subnormal, 2^-100 and a group of
    # zeros ("tiny"); one 2^62 entry that dominates the mean square ("huge").
    # Both the gate/up pairing (two token groups per thread) and a plain
    # launch (one group) must give the oracle's bits.
    print("rmsnorm special values", k, case, flush=True)
    rng = np.random.default_rng(k + len(case))
    x = rng.standard_normal((1, k)).astype(np.float32)
    if case == "tiny":
        x[0, 5] = 0.0
        x[0, 40] = -0.0
        x[0, 100] = np.float32(1e-40)   # subnormal
        x[0, 333] = np.float32(2.0 ** -100)
        x[0, 17 * 16:18 * 16] = 0.0     # a group of zeros
        x[0, 700] = np.float32(2.0 ** -60)  # the bottom of the range
    else:
        x[0, 9] = np.float32(2.0 ** 62)
    g = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    xn = orc.rmsnorm(x, g, 1e-5)
    xt, gt = torch.from_numpy(x).to(DEV), torch.from_numpy(g).to(DEV)
    n = 300
    wg, sg = orc.pack((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    wu, su = orc.pack((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    pg = bl.PackedTensor(torch.from_numpy(wg).to(DEV), sg, (n, k), DEV)
    pu = bl.PackedTensor(torch.from_numpy(wu).to(DEV), su, (n, k), DEV)
    out = torch.full((1, n), 9.0, device=DEV)
    cg, cu = pg.as_c(), pu.as_c()
    bl.check(bl.lib.btl_add_rmsnorm_swiglu(ctypes.byref(cg), ctypes.byref(cu), xt.data_ptr(), None, None,
                                           gt.data_ptr(), 1e-5, 1, k, out.data_ptr(), None, 0, stream()))
    e = orc.swiglu(orc.forward_i8(xn, wg, n, sg)[0], orc.forward_i8(xn, wu, n, su)[0])
    assert_same(out, e, "gate/up pairing")
    y = torch.empty((1, n), device=DEV)
    arr = (ctypes.POINTER(bl.BtlPacked) * 1)(ctypes.pointer(cg))
    ys = (ctypes.c_void_p * 1)(y.data_ptr())
    bl.check(bl.lib.btl_add_rmsnorm_linear_group(arr, ys, 1, xt.data_ptr(), None, None, gt.data_ptr(), 1e-5, 1, k,
                                                 bl.BTL_F32, None, 0, stream()))
    assert_same(y, orc.forward_i8(xn, wg, n, sg)[0], "one group per thread")


def test_add_rmsnorm_rejects_partial_overlap():
    k = 256
    h = torch.zeros((2, k), device=DEV)
    pt = bl.PackedTensor(torch.zeros((16 * k // 4,), dtype=torch.uint8, device=DEV), 1.0, (16, k), DEV)
    c = pt.as_c()
    arr = (ctypes.POINTER(bl.BtlPacked) * 1)(ctypes.pointer(c))
    y = torch.empty((2, 16), device=DEV)
    ys = (ctypes.c_void_p * 1)(y.data_ptr())
    g = torch.ones(k, device=DEV)
    st = bl.lib.btl_add_rmsnorm_linear_group(arr, ys, 1, h.data_ptr(), h.data_ptr(), h[1].data_ptr(), g.data_ptr(),
                                             1e-5, 2, k, bl.BTL_F32, None, 0, stream())
    assert st == bl.BTL_ERR_LAYOUT


# --- the decoder end to end ----------------------------------------------------

class Tiny2(TinyCfg):
    # hidden 128 = 1 head of 128 (GQA rep 1), odd vocab, a chunk boundary inside the prompt
    hidden, n_layers, n_heads, n_kv_heads, head_dim = 256, 2, 2, 1, 128
    intermediate, vocab, rope_theta, max_seq, eps = 512, 1001, 500000.0, 160, 1e-5


def gpu_model(cfg, w, max_rows=512):
    def lin(pk, n, k):
        return bl.PackedTensor(torch.from_numpy(pk[0]).to(DEV), pk[1], (n, k), DEV)

    kvd = cfg.n_kv_heads * cfg.head_dim
    qd = cfg.n_heads * cfg.head_dim
    layers = [{"norm1": torch.from_numpy(L["norm1"]).to(DEV), "norm2": torch.from_numpy(L["norm2"]).to(DEV),
               "q": lin(L["q"], qd, cfg.hidden), "k": lin(L["k"], kvd, cfg.hidden), "v": lin(L["v"], kvd, cfg.hidden),
               "o": lin(L["o"], cfg.hidden, qd), "gate": lin(L["gate"], cfg.intermediate, cfg.hidden),
               "up": lin(L["up"], cfg.intermediate, cfg.hidden), "down": lin(L["down"], cfg.hidden, cfg.intermediate)}
              for L in w["layers"]]
    gw = {"embed": torch.from_numpy(w["embed"]).to(DEV), "norm_f": torch.from_numpy(w["norm_f"]).to(DEV),
          "lm_head": lin(w["lm_head"], cfg.vocab, cfg.hidden), "layers": layers}
    return BitLlamaHip(cfg, gw, DEV, max_rows=max_rows)


class TinyA(TinyCfg):
    hidden, n_layers, n_heads, n_kv_heads, head_dim = 256, 2, 4, 2, 64
    intermediate, vocab, rope_theta, max_seq, eps = 512, 1000, 10000.0, 160, 1e-5


@pytest.mark.parametrize("cfg_cls", [TinyA, Tiny2])
def test_decoder_forward_one_matches_oracle(cfg_cls):
    cfg = cfg_cls()
    w = tiny_weights(cfg, seed=5)
    gm = gpu_model(cfg, w)
    om = OracleLlama(cfg, w)
    rng = np.random.default_rng(9)
    toks = rng.integers(0, cfg.vocab, 70)
    for i, t in enumerate(toks):
        print("forward_one step", i, flush=True)
        lg = gm.forward_one(int(t))
        lo = om.forward_one(int(t))
        assert_same(lg, lo, "step %d logits" % i)
    for li in range(cfg.n_layers):
        c = gm.caches[li]
        assert np.array_equal(c.k.cpu().numpy()[:, :70], om.caches[li]["kq"][:, :70])
        assert_same(c.v_scale.cpu().numpy()[:, :70], om.caches[li]["vs"][:, :70], "v scales")


@pytest.mark.parametrize("cfg_cls", [TinyA, Tiny2])
def test_decoder_prefill_equals_token_by_token(cfg_cls):
    cfg = cfg_cls()
    w = tiny_weights(cfg, seed=6)
    prompt = np.random.default_rng(2).integers(0, cfg.vocab, 75)
    a = gpu_model(cfg, w, max_rows=32)  # 75 tokens: batches of 32, 32, 11
    la = a.prefill(prompt).clone()
    b = gpu_model(cfg, w)
    for t in prompt:
        lb = b.forward_one(int(t))
    assert_same(la, lb.cpu().numpy(), "prefill vs token-by-token logits")
    for li in range(cfg.n_layers):
        assert torch.equal(a.caches[li].k, b.caches[li].k) and torch.equal(a.caches[li].v, b.caches[li].v)
        assert torch.equal(a.caches[li].k_scale, b.caches[li].k_scale)


@pytest.mark.parametrize("use_graph", [False, True])
def test_decoder_generate_matches_oracle(use_graph):
    cfg = TinyA()
    w = tiny_weights(cfg, seed=7)
    prompt = np.random.default_rng(3).integers(0, cfg.vocab, 66)
    gm = gpu_model(cfg, w)
    got = gm.generate(prompt, 24, use_graph=use_graph)
    exp = OracleLlama(cfg, w).generate(prompt, 24)
    assert np.array_equal(got, exp), (got, exp)
    if use_graph:
        # replays again after eager work in between: the same continuation as the oracle's
        torch.cuda.synchronize()
        again = gm.generate(prompt, 24, use_graph=True)
        assert np.array_equal(again, exp)


class Llama3Wide(TinyCfg):
    # Llama-3-8B's widths (hidden 4096, 32 / 8 heads of 128, intermediate 14336,
    # vocab 128256, theta 500000), two layers
    hidden, n_layers, n_heads, n_kv_heads, head_dim = 4096, 2, 32, 8, 128
    intermediate, vocab, rope_theta, max_seq, eps = 14336, 128256, 500000.0, 256, 1e-5


def _random_codes(rng, n, k):
    # packed ternary rows of valid codes (00 -> 0, 01 -> +1, 10 -> -1; the
    # unused 11 folded to 00) and a scale, as PackedTensor holds them
    b = rng.integers(0, 256, n * k // 4, dtype=np.uint8)
    m = b & (b >> 1) & 0x55
    b &= ~(m | (m << 1)).astype(np.uint8)
    return b, float(rng.uniform(0.005, 0.02))


class _RowsOnDevice:
    # the oracle's view of a device embedding table: the rows it asks for
    def __init__(self, t):
        self.t = t

    def __getitem__(self, i):
        return self.t[int(i)].float().cpu().numpy()


def test_decoder_llama3_width_matches_oracle():
    # full Llama-3-8B widths, two layers: five tokens one at a time (logits bit
    # for bit each step, then the KV caches), then a greedy continuation from a
    # two-token prefill (the batched path) replayed from a HIP graph
    cfg = Llama3Wide()
    rng = np.random.default_rng(11)
    kvd, qd = cfg.n_kv_heads * cfg.head_dim, cfg.n_heads * cfg.head_dim

    def norm(n):
        return (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)

    layers = [{"norm1": norm(cfg.hidden), "norm2": norm(cfg.hidden),
               "q": _random_codes(rng, qd, cfg.hidden), "k": _random_codes(rng, kvd, cfg.hidden),
               "v": _random_codes(rng, kvd, cfg.hidden), "o": _random_codes(rng, cfg.hidden, qd),
               "gate": _random_codes(rng, cfg.intermediate, cfg.hidden),
               "up": _random_codes(rng, cfg.intermediate, cfg.hidden),
               "down": _random_codes(rng, cfg.hidden, cfg.intermediate)} for _ in range(cfg.n_layers)]
    g = torch.Generator(device=DEV)
    g.manual_seed(5)
    embed = torch.randn((cfg.vocab, cfg.hidden), device=DEV, generator=g)
    w = {"embed": _RowsOnDevice(embed), "norm_f": norm(cfg.hidden),
         "lm_head": _random_codes(rng, cfg.vocab, cfg.hidden), "layers": layers}

    def lin(pk, n, k):
        return bl.PackedTensor(torch.from_numpy(pk[0]).to(DEV), pk[1], (n, k), DEV)

    gl = [{"norm1": torch.from_numpy(L["norm1"]).to(DEV), "norm2": torch.from_numpy(L["norm2"]).to(DEV),
           "q": lin(L["q"], qd, cfg.hidden), "k": lin(L["k"], kvd, cfg.hidden), "v": lin(L["v"], kvd, cfg.hidden),
           "o": lin(L["o"], cfg.hidden, qd), "gate": lin(L["gate"], cfg.intermediate, cfg.hidden),
           "up": lin(L["up"], cfg.intermediate, cfg.hidden), "down": lin(L["down"], cfg.hidden, cfg.intermediate)}
          for L in layers]
    gw = {"embed": embed, "norm_f": torch.from_numpy(w["norm_f"]).to(DEV),
          "lm_head": lin(w["lm_head"], cfg.vocab, cfg.hidden), "layers": gl}
    gm = BitLlamaHip(cfg, gw, DEV, max_rows=16)
    om = OracleLlama(cfg, w)
    toks = [int(t) for t in rng.integers(0, cfg.vocab, 5)]
    for i, t in enumerate(toks):
        print("llama3-width forward_one", i, flush=True)
        assert_same(gm.forward_one(t), om.forward_one(t), "step %d logits" % i)
    for li in range(cfg.n_layers):
        c = gm.caches[li]
        assert np.array_equal(c.k.cpu().numpy()[:, :5], om.caches[li]["kq"][:, :5])
        assert np.array_equal(c.v.cpu().numpy()[:, :5], om.caches[li]["vq"][:, :5])
        assert_same(c.k_scale.cpu().numpy()[:, :5], om.caches[li]["ks"][:, :5], "k scales")
    print("llama3-width generate", flush=True)
    gm2 = BitLlamaHip(cfg, gw, DEV, max_rows=16)
    got = gm2.generate(toks[:2], 3, use_graph=True)
    exp = OracleLlama(cfg, w).generate(toks[:2], 3)
    assert np.array_equal(got, exp), (got, exp)


@pytest.mark.parametrize("m,k", [(1, 64), (1, 4096), (3, 4160), (2, 65536)])
@pytest.mark.parametrize("mode", ["plain", "delta", "delta_out", "inplace"])
def test_add_rmsnorm_rows(m, k, mode):
    # RMSNorm into f32 rows, the sum of squares a pairwise tree over the row
    print("add_rmsnorm", m, k, mode, flush=True)
    rng = np.random.default_rng(k + m)
    h = (rng.standard_normal((m, k)) * 3).astype(np.float32)
    d = rng.standard_normal((m, k)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    ht, dt, gt = (torch.from_numpy(a).to(DEV) for a in (h, d, g))
    y = torch.full((m, k), 5.0, device=DEV)
    ho = torch.full((m, k), 5.0, device=DEV)
    delta = dt.data_ptr() if mode != "plain" else None
    hout = {"plain": None, "delta": None, "delta_out": ho.data_ptr(), "inplace": ht.data_ptr()}[mode]
    bl.check(bl.lib.btl_add_rmsnorm(ht.data_ptr(), delta, hout, gt.data_ptr(), 1e-5, m, k, y.data_ptr(), stream()))
    s = h + d if mode != "plain" else h
    assert_same(y, orc.rmsnorm(s, g, 1e-5), "rmsnorm rows")
    if mode == "delta_out":
        assert_same(ho, s, "h_out")
    if mode == "inplace":
        assert_same(ht, s, "h in place")


# the reference's arithmetic with the residual add + RMSNorm staged by the
# projections' own launch: the same bits as btl_add_rmsnorm followed by
# btl_linear_group_mode (BTL_ACT_F32_REF) and as the oracle; h_out from the
# first output tile's workgroups, h and delta untouched; m = 3 runs a second
# token-row pair with one row past m; k = 14336 stages four 4096-element blocks
@pytest.mark.parametrize("m,k,ns", [(1, 4096, (96, 40, 33)), (3, 4096, (700,)), (2, 14336, (64, 50)), (1, 64, (40,)),
                                    (3, 2112, (130, 33))])
@pytest.mark.parametrize("mode", ["plain", "delta", "delta_out", "plain_out"])
def test_add_rmsnorm_linear_group_ref(m, k, ns, mode):
    print("add_rmsnorm_linear_group_ref", m, k, ns, mode, flush=True)
    rng = np.random.default_rng(m * 3 + k + len(ns))
    h = (rng.standard_normal((m, k)) * np.exp2(rng.integers(-8, 8, (m, k)))).astype(np.float32)
    d = rng.standard_normal((m, k)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    layers = []
    for i, n in enumerate(ns):
        wb, sw = orc.pack((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        layers.append((bl.PackedTensor(torch.from_numpy(wb).to(DEV), sw, (n, k), DEV), wb, sw, n))
    ht, dt, gt = (torch.from_numpy(a).to(DEV) for a in (h, d, g))
    ho = torch.full_like(ht, 5.0)
    cnt = len(layers)
    cs = [L[0].as_c() for L in layers]
    arr = (ctypes.POINTER(bl.BtlPacked) * cnt)(*[ctypes.pointer(c) for c in cs])
    outs = [torch.full((m, n), 7.0, device=DEV) for (_, _, _, n) in layers]
    ys = (ctypes.c_void_p * cnt)(*[o.data_ptr() for o in outs])
    delta = dt.data_ptr() if mode.startswith("delta") else None
    hout = ho.data_ptr() if mode.endswith("_out") else None
    bl.check(bl.lib.btl_add_rmsnorm_linear_group_ref(arr, ys, cnt, ht.data_ptr(), delta, hout, gt.data_ptr(), 1e-5,
                                                     m, k, stream()))
    s_ = (h + d).astype(np.float32) if delta else h
    xn = orc.rmsnorm(s_, g, 1e-5)
    for o, (_, wb, sw, n) in zip(outs, layers):
        assert_same(o, orc.forward_f32(xn, wb, n, np.float32(sw)), "layer")
    assert_same(ht, h, "h untouched")
    assert_same(ho, s_ if hout else np.full((m, k), 5.0, np.float32), "h_out")
    # the two launches it replaces give the same bits
    xt = torch.empty((m, k), device=DEV)
    bl.check(bl.lib.btl_add_rmsnorm(ht.data_ptr(), delta, None, gt.data_ptr(), 1e-5, m, k, xt.data_ptr(), stream()))
    outs2 = [torch.empty((m, n), device=DEV) for (_, _, _, n) in layers]
    ys2 = (ctypes.c_void_p * cnt)(*[o.data_ptr() for o in outs2])
    bl.check(bl.lib.btl_linear_group_mode(arr, ys2, cnt, xt.data_ptr(), bl.BTL_F32, m, k, bl.BTL_F32,
                                          bl.BTL_ACT_F32_REF, None, 0, stream()))
    for a, b in zip(outs, outs2):
        assert torch.equal(a, b)


def test_fused_ref_rejects_bad_shapes_and_overlap():
    k, m = 4096, 2
    h = torch.zeros((m, k), device=DEV)
    g = torch.ones(k, device=DEV)
    wb, sw = orc.pack(np.full((8, k), 0.01, np.float32))
    pt = bl.PackedTensor(torch.from_numpy(wb).to(DEV), sw, (8, k), DEV)
    c = pt.as_c()
    arr = (ctypes.POINTER(bl.BtlPacked) * 1)(ctypes.pointer(c))
    y = torch.empty((m, 8), device=DEV)
    ys = (ctypes.c_void_p * 1)(y.data_ptr())
    # h_out over h: the launch's other workgroups still read h
    assert bl.lib.btl_add_rmsnorm_linear_group_ref(arr, ys, 1, h.data_ptr(), None, h.data_ptr(), g.data_ptr(), 1e-5,
                                                   m, k, stream()) == bl.BTL_ERR_LAYOUT
    # y over the input
    ys_bad = (ctypes.c_void_p * 1)(h.data_ptr())
    assert bl.lib.btl_add_rmsnorm_linear_group_ref(arr, ys_bad, 1, h.data_ptr(), None, None, g.data_ptr(), 1e-5,
                                                   m, k, stream()) == bl.BTL_ERR_LAYOUT
    # k past the staged form
    h2 = torch.zeros((1, 16448), device=DEV)
    g2 = torch.ones(16448, device=DEV)
    w2, s2 = orc.pack(np.full((8, 16448), 0.01, np.float32))
    p2 = bl.PackedTensor(torch.from_numpy(w2).to(DEV), s2, (8, 16448), DEV)
    c2 = p2.as_c()
    arr2 = (ctypes.POINTER(bl.BtlPacked) * 1)(ctypes.pointer(c2))
    assert bl.lib.btl_add_rmsnorm_linear_group_ref(arr2, ys, 1, h2.data_ptr(), None, None, g2.data_ptr(), 1e-5, 1,
                                                   16448, stream()) == bl.BTL_ERR_SHAPE


def test_add_rmsnorm_rejects_overlap():
    h = torch.zeros((2, 256), device=DEV)
    g = torch.ones(256, device=DEV)
    assert bl.lib.btl_add_rmsnorm(h.data_ptr(), None, None, g.data_ptr(), 1e-5, 2, 256, h.data_ptr(),
                                  stream()) == bl.BTL_ERR_LAYOUT
    assert bl.lib.btl_add_rmsnorm(h.data_ptr(), None, None, g.data_ptr(), 1e-5, 2, 100, h.data_ptr(),
                                  stream()) == bl.BTL_ERR_SHAPE


@pytest.mark.parametrize("n,k,m,dt", [(1000, 4096, 1, "f32"), (1000, 4096, 2, "bf16"), (333, 520, 3, "f32"),
                                      (77, 4100, 1, "bf16"), (128256, 4096, 1, "f32")])
def test_dense_linear(n, k, m, dt):
    # the dense lm_head: f32 sums in the fixed lane order (registers for k = 4096,
    # the generic chunk loop otherwise), bit for bit with the oracle
    print("dense_linear", n, k, m, dt, flush=True)
    rng = np.random.default_rng(n + k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    if dt == "bf16":
        wt = torch.from_numpy(w).to(DEV).to(torch.bfloat16)
        wh = wt.view(torch.int16).cpu().numpy().view(np.uint16)
        code = bl.BTL_BF16
    else:
        wt = torch.from_numpy(w).to(DEV)
        wh = w
        code = bl.BTL_F32
    xt = torch.from_numpy(x).to(DEV)
    y = torch.full((m, n), 9.0, device=DEV)
    bl.check(bl.lib.btl_dense_linear(wt.data_ptr(), code, n, k, xt.data_ptr(), m, y.data_ptr(), stream()))
    exp = orc.dense_linear(x, wh)
    assert_same(y, exp, "dense linear")
    ref = x.astype(np.float64) @ (wt.float().cpu().numpy().astype(np.float64)).T
    assert np.abs(y.cpu().numpy() - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())


def test_decoder_dense_head_matches_oracle():
    # the reference's dense lm_head (f32 and bf16 weights) after the ternary blocks
    cfg = TinyA()
    w = tiny_weights(cfg, seed=8)
    rng = np.random.default_rng(4)
    for dt in (torch.float32, torch.bfloat16):
        head = torch.from_numpy((rng.standard_normal((cfg.vocab, cfg.hidden)) * 0.05).astype(np.float32)).to(DEV)
        head = head.to(dt).contiguous()
        gm = gpu_model(cfg, w)
        gm.w["lm_head"] = head
        gm2 = BitLlamaHip(cfg, dict(gm.w), DEV)
        wo = dict(w)
        wo["lm_head"] = head.cpu().numpy() if dt == torch.float32 else head.view(torch.int16).cpu().numpy().view(np.uint16)
        om = OracleLlama(cfg, wo)
        for i, t in enumerate(rng.integers(0, cfg.vocab, 6)):
            assert_same(gm2.forward_one(int(t)), om.forward_one(int(t)), "%s step %d" % (dt, i))
        got = BitLlamaHip(cfg, dict(gm.w), DEV).generate([3, 9, 27], 8, use_graph=True)
        exp = OracleLlama(cfg, wo).generate([3, 9, 27], 8)
        assert np.array_equal(got, exp), (dt, got, exp)


def test_dense_linear_order_cases():
    # rows where only the fixed lane order keeps the small term (see the oracle
    # tests): the kernel must agree with it
    k, B, t = 512, 2.0 ** 25, 2.0 ** -30
    w = np.zeros((3, k), np.float32)
    w[0, [0, 256, 4]] = [B, -B, t]
    w[1, [0, 128, 4]] = [B, -B, t]
    w[2, [0, 1, 2]] = [B, t, -B]
    x = np.ones((1, k), np.float32)
    y = torch.zeros((1, 3), device=DEV)
    wt, xt = torch.from_numpy(w).to(DEV), torch.from_numpy(x).to(DEV)
    bl.check(bl.lib.btl_dense_linear(wt.data_ptr(), bl.BTL_F32, 3, k, xt.data_ptr(), 1, y.data_ptr(), stream()))
    assert y.cpu().numpy()[0].tolist() == [t, t, 0.0]
    assert_same(y, orc.dense_linear(x, w), "order cases")


@pytest.mark.parametrize("cfg_cls", [TinyA, Tiny2])
def test_decoder_f32_ref_matches_oracle(cfg_cls):
    # every BitLinear in the reference's own fp32 order (BTL_ACT_F32_REF): token by
    # token against the oracle in that mode, a batched prefill equal to it, and a
    # graph-replayed greedy continuation
    cfg = cfg_cls()
    w = tiny_weights(cfg, seed=12)
    gm = gpu_model(cfg, w)
    ref = BitLlamaHip(cfg, dict(gm.w), DEV, mode="f32_ref")
    om = OracleLlama(cfg, w, mode="f32_ref")
    toks = np.random.default_rng(13).integers(0, cfg.vocab, 40)
    for i, t in enumerate(toks):
        print("f32_ref forward_one", i, flush=True)
        assert_same(ref.forward_one(int(t)), om.forward_one(int(t)), "step %d logits" % i)
    b = BitLlamaHip(cfg, dict(gm.w), DEV, mode="f32_ref", max_rows=16)
    assert_same(b.prefill(toks), ref.logits[0].cpu().numpy(), "prefill in batches of 16")
    for li in range(cfg.n_layers):
        assert torch.equal(b.caches[li].k, ref.caches[li].k) and torch.equal(b.caches[li].v_scale, ref.caches[li].v_scale)
    got = BitLlamaHip(cfg, dict(gm.w), DEV, mode="f32_ref").generate(toks[:5], 10, use_graph=True)
    exp = OracleLlama(cfg, w, mode="f32_ref").generate(toks[:5], 10)
    assert np.array_equal(got, exp), (got, exp)


def test_decoder_reference_arithmetic_with_dense_head():
    # the decoder as the reference runs it on a CPU: fp32 BitLinears and a dense
    # f32 lm_head
    cfg = TinyA()
    w = tiny_weights(cfg, seed=14)
    gm = gpu_model(cfg, w)
    head = (np.random.default_rng(5).standard_normal((cfg.vocab, cfg.hidden)) * 0.05).astype(np.float32)
    gw = dict(gm.w)
    gw["lm_head"] = torch.from_numpy(head).to(DEV)
    wo = dict(w)
    wo["lm_head"] = head
    got = BitLlamaHip(cfg, gw, DEV, mode="f32_ref").generate([7, 1, 99, 5], 12, use_graph=True)
    exp = OracleLlama(cfg, wo, mode="f32_ref").generate([7, 1, 99, 5], 12)
    assert np.array_equal(got, exp), (got, exp)
