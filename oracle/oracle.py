"""ctypes binding of oracle/libbitlinear_oracle.so (see bitlinear_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py.  The product package never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbitlinear_oracle.so")


def build():
    """Compile the oracle with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", HERE, "-B"], check=True)
    return LIB_PATH


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    vp, i64, f32, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int
    sigs = {
        "orc_pack": (i32, [vp, i64, vp, ctypes.POINTER(f32)]),
        "orc_unpack": (None, [vp, i64, f32, vp]),
        "orc_forward_f32": (i32, [vp, i64, i64, vp, i64, i64, f32, vp, i32]),
        "orc_forward_f32_avx2": (i32, [vp, i64, i64, vp, i64, i64, f32, vp, i32]),
        "orc_has_avx2": (i32, []),
        "orc_quantize_act": (None, [vp, i64, i64, vp, vp]),
        "orc_contract_i8": (None, [vp, i64, i64, vp, i64, vp]),
        "orc_epilogue": (None, [vp, vp, f32, i64, i64, vp]),
        "orc_forward_i8": (i32, [vp, i64, i64, vp, i64, f32, vp, vp, vp, vp]),
        "orc_bf16_to_f32_array": (None, [vp, i64, vp]),
        "orc_pairwise_sum": (f32, [vp, i64]),
        "orc_rmsnorm": (None, [vp, i64, i64, vp, f32, vp]),
        "orc_expf": (f32, [f32]),
        "orc_swiglu": (None, [vp, vp, i64, vp]),
        "orc_f32_to_bf16_array": (None, [vp, i64, vp]),
        "orc_rope_table": (None, [ctypes.c_double, i64, i64, vp, vp]),
        "orc_rope_apply": (None, [vp, i64, vp, vp, vp]),
        "orc_q8_quant": (None, [vp, i64, vp, vp]),
        "orc_q8_dequant": (None, [vp, i64, f32, vp]),
        "orc_attn_decode": (None, [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, vp]),
        "orc_attn_dot": (ctypes.c_float, [vp, vp, i64, i64]),
        "orc_argmax": (i64, [vp, i64]),
        "orc_dense_linear": (None, [vp, i64, i64, vp, i32, i64, vp]),
        "orc_adaptive_reconstruct": (None, [vp, vp, i64, i64, i64, vp]),
        "orc_adaptive_split": (None, [vp, i64, i64, i64, vp]),
        "orc_adaptive_forward_i8": (i32, [vp, i64, i64, vp, vp, i64, i64, vp]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a.size else None


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def pack(w):
    """PackedTensor::pack -> (uint8 bytes, scale)."""
    w = _f32(w).reshape(-1)
    out = np.zeros(((w.size + 3) // 4,), dtype=np.uint8)
    s = ctypes.c_float(0)
    rc = lib.orc_pack(_p(w), w.size, _p(out), ctypes.byref(s))
    assert rc == 0
    return out, s.value


def unpack(data, numel, scale):
    out = np.zeros((numel,), dtype=np.float32)
    lib.orc_unpack(_p(np.ascontiguousarray(data, np.uint8)), numel, scale, _p(out))
    return out


def forward_f32(x, w, n, scale, avx2_order=True, wbytes=None):
    """BitLinearCpu::forward in the exact fp32 order; x [m,k] f32, w packed bytes."""
    x = _f32(x)
    m, k = x.shape
    w = np.ascontiguousarray(w, np.uint8)
    y = np.zeros((m, n), dtype=np.float32)
    rc = lib.orc_forward_f32(_p(x), m, k, _p(w), n, w.size if wbytes is None else wbytes, scale, _p(y),
                             1 if avx2_order else 0)
    if rc != 0:
        raise ValueError("orc_forward_f32 status %d" % rc)
    return y


def forward_f32_avx2(x, w, n, scale, threads=1):
    """Intrinsics + threads restatement (the timed baseline)."""
    x = _f32(x)
    m, k = x.shape
    w = np.ascontiguousarray(w, np.uint8)
    y = np.zeros((m, n), dtype=np.float32)
    rc = lib.orc_forward_f32_avx2(_p(x), m, k, _p(w), n, w.size, scale, _p(y), threads)
    if rc != 0:
        raise ValueError("orc_forward_f32_avx2 status %d" % rc)
    return y


def has_avx2():
    return bool(lib.orc_has_avx2())


def quantize_act(x):
    x = _f32(x)
    m, k = x.shape
    q = np.zeros((m, k), dtype=np.int8)
    s = np.zeros((m,), dtype=np.float32)
    lib.orc_quantize_act(_p(x), m, k, _p(q), _p(s))
    return q, s


def contract_i8(q, w, n):
    q = np.ascontiguousarray(q, np.int8)
    m, k = q.shape
    acc = np.zeros((m, n), dtype=np.int32)
    lib.orc_contract_i8(_p(q), m, k, _p(np.ascontiguousarray(w, np.uint8)), n, _p(acc))
    return acc


def epilogue(acc, sx, sw):
    acc = np.ascontiguousarray(acc, np.int32)
    m, n = acc.shape
    y = np.zeros((m, n), dtype=np.float32)
    lib.orc_epilogue(_p(acc), _p(_f32(sx)), sw, m, n, _p(y))
    return y


def forward_i8(x, w, n, sw):
    """W1.58-A8 forward -> (y f32, q int8, s_x f32, acc int32)."""
    x = _f32(x)
    m, k = x.shape
    y = np.zeros((m, n), dtype=np.float32)
    q = np.zeros((m, k), dtype=np.int8)
    s = np.zeros((m,), dtype=np.float32)
    acc = np.zeros((m, n), dtype=np.int32)
    rc = lib.orc_forward_i8(_p(x), m, k, _p(np.ascontiguousarray(w, np.uint8)), n, sw, _p(y), _p(q), _p(s),
                            _p(acc))
    assert rc == 0
    return y, q, s, acc


def bf16_to_f32(h):
    h = np.ascontiguousarray(h, np.uint16)
    out = np.zeros(h.shape, dtype=np.float32)
    lib.orc_bf16_to_f32_array(_p(h), h.size, _p(out))
    return out


def f32_to_bf16(f):
    f = _f32(f)
    out = np.zeros(f.shape, dtype=np.uint16)
    lib.orc_f32_to_bf16_array(_p(f), f.size, _p(out))
    return out


def pairwise_sum(v):
    """Pairwise-tree sum in index order, zero-padded to a power of two (float32)."""
    v = _f32(v).ravel()
    return np.float32(lib.orc_pairwise_sum(_p(v), v.size))


def rmsnorm(x, g, eps):
    """rms_norm.rs:33-56 restated (see the C header): float32 [M, K] -> [M, K]."""
    x = _f32(x)
    m, k = x.shape
    g = _f32(g).ravel()
    assert g.size == k
    out = np.empty_like(x)
    lib.orc_rmsnorm(_p(x), m, k, _p(g), float(np.float32(eps)), _p(out))
    return out


def expf(x):
    """The build's float32 exp (Cody-Waite + Taylor), elementwise."""
    x = _f32(x)
    return np.array([lib.orc_expf(float(v)) for v in x.ravel()], dtype=np.float32).reshape(x.shape)


def swiglu(g, u):
    """swiglu.rs:29-35: silu(g) * u, float32."""
    g, u = _f32(g), _f32(u)
    assert g.shape == u.shape
    out = np.empty_like(g)
    lib.orc_swiglu(_p(g), _p(u), g.size, _p(out))
    return out


# ---------------------------------------------------------------------------
# decoder ops around the BitLinear path (bitllama_oracle.c)
# ---------------------------------------------------------------------------
def rope_table(theta, head_dim, max_seq):
    """RotaryEmbedding::new (attention.rs:15-42): (cos, sin) float32 [max_seq, head_dim/2]."""
    half = head_dim // 2
    c = np.zeros((max_seq, half), dtype=np.float32)
    s = np.zeros((max_seq, half), dtype=np.float32)
    lib.orc_rope_table(float(theta), head_dim, max_seq, _p(c), _p(s))
    return c, s


def rope_apply(x, cos_row, sin_row):
    """RotaryEmbedding::apply (attention.rs:46-87) on the last axis of x at one position."""
    x = _f32(x)
    hd = x.shape[-1]
    out = np.empty_like(x)
    xf, of = x.reshape(-1, hd), out.reshape(-1, hd)
    c, s = _f32(cos_row), _f32(sin_row)
    for i in range(xf.shape[0]):
        row = np.ascontiguousarray(xf[i])
        o = np.empty_like(row)
        lib.orc_rope_apply(_p(row), hd, _p(c), _p(s), _p(o))
        of[i] = o
    return out


def q8_quant(x):
    """QuantizedKVCache::quantize_q8 (kv_cache.rs:95-119) per row of the last axis -> (u8 codes, f32 scales)."""
    x = _f32(x)
    hd = x.shape[-1]
    xf = x.reshape(-1, hd)
    q = np.zeros(xf.shape, dtype=np.uint8)
    s = np.zeros((xf.shape[0],), dtype=np.float32)
    for i in range(xf.shape[0]):
        row = np.ascontiguousarray(xf[i])
        qi = np.zeros((hd,), dtype=np.uint8)
        si = np.zeros((1,), dtype=np.float32)
        lib.orc_q8_quant(_p(row), hd, _p(qi), _p(si))
        q[i], s[i] = qi, si[0]
    return q.reshape(x.shape), s.reshape(x.shape[:-1])


def q8_dequant(q, s):
    """dequantize_q8 (kv_cache.rs:122-128): ((f32)q - 128) * s per row."""
    q = np.ascontiguousarray(q, np.uint8)
    hd = q.shape[-1]
    qf = q.reshape(-1, hd)
    sf = _f32(s).reshape(-1)
    out = np.zeros(qf.shape, dtype=np.float32)
    for i in range(qf.shape[0]):
        o = np.zeros((hd,), dtype=np.float32)
        lib.orc_q8_dequant(_p(np.ascontiguousarray(qf[i])), hd, float(sf[i]), _p(o))
        out[i] = o
    return out.reshape(q.shape)


def attn_decode(q, kq, ks, vq, vs, n_heads, T):
    """One query position of BitAttention::forward over a Q8 cache (fixed GPU order).
    q [nh*hd] f32; kq/vq [nkv, max_seq, hd] u8; ks/vs [nkv, max_seq] f32."""
    kq, vq = np.ascontiguousarray(kq, np.uint8), np.ascontiguousarray(vq, np.uint8)
    ks, vs = _f32(ks), _f32(vs)
    nkv, max_seq, hd = kq.shape
    q = _f32(q).reshape(-1)
    out = np.zeros((n_heads * hd,), dtype=np.float32)
    lib.orc_attn_decode(_p(q), _p(kq), _p(ks), _p(vq), _p(vs), n_heads, nkv, hd, max_seq, T, _p(out))
    return out


def attn_dot(a, b):
    """The attention's dot product: acc = fma(a[i], b[i], acc), sequential, from 0."""
    a, b = _f32(a).reshape(-1), _f32(b).reshape(-1)
    assert a.size == b.size
    return np.float32(lib.orc_attn_dot(_p(a), _p(b), a.size, 1))


def dense_linear(x, w):
    """candle_nn::Linear::forward without a bias (the dense lm_head, llama.rs:129-141)
    in the GPU kernel's fixed order.  x [m, k] f32; w [n, k] f32, or uint16 holding
    bf16 bits.  -> y [m, n] f32."""
    x = _f32(x)
    m, k = x.shape
    bf = w.dtype == np.uint16
    w = np.ascontiguousarray(w, np.uint16 if bf else np.float32)
    n = w.shape[0]
    assert w.shape[1] == k and k % 4 == 0
    y = np.zeros((m, n), dtype=np.float32)
    lib.orc_dense_linear(_p(x), m, k, _p(w), int(bf), n, _p(y))
    return y


def argmax(x):
    """Greedy pick of stream_completion (llama.rs:509-515): the last maximum."""
    x = _f32(x).reshape(-1)
    return int(lib.orc_argmax(_p(x), x.size))


# ---------------------------------------------------------------------------
# multi-base adaptive format (adaptive_linear.rs)
# ---------------------------------------------------------------------------
def adaptive_reconstruct(packed, scales, n, k):
    """AdaptiveBitLinear::load's dense f32 weights [n, k] (adaptive_linear.rs:86-117)."""
    packed = np.ascontiguousarray(packed, np.uint8).reshape(-1)
    scales = _f32(scales).reshape(-1)
    out = np.zeros((n, k), dtype=np.float32)
    lib.orc_adaptive_reconstruct(_p(packed), _p(scales), scales.size, n, k, _p(out))
    return out


def adaptive_split(packed, nb, n, k):
    """[n, k/4, nb] interleaved bytes -> [nb, n * k/4] PackedTensor byte arrays."""
    packed = np.ascontiguousarray(packed, np.uint8).reshape(-1)
    out = np.zeros((nb, n * (k // 4)), dtype=np.uint8)
    lib.orc_adaptive_split(_p(packed), nb, n, k, _p(out))
    return out


def adaptive_forward_i8(x, packed, scales, n):
    """W1.58-A8 multi-base forward: y = sum_b (float)acc_b * (s_x * s_b) in base order."""
    x = _f32(x)
    m, k = x.shape
    scales = _f32(scales).reshape(-1)
    y = np.zeros((m, n), dtype=np.float32)
    rc = lib.orc_adaptive_forward_i8(_p(x), m, k, _p(np.ascontiguousarray(packed, np.uint8).reshape(-1)), _p(scales),
                                     scales.size, n, _p(y))
    assert rc == 0
    return y
