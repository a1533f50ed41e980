"""CPU tests of the C ABI: the library loads, exports what include/bitlinear.h declares,
its host-side packing matches the oracle, and argument validation fails before any
device work with the reference's error texts."""
import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest
import torch

import bitlinear as bl
from datagen import weights
from oracle import oracle as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))
           if h.endswith(".h")]


def header_functions():
    text = "".join(open(h).read() for h in HEADERS)
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(btl_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_python_exports():
    assert header_functions() == sorted(bl.EXPORTS)


CRATE = os.path.join(ROOT, "bit-ttt-engine_amd", "crates", "bitlinear-hip-sys", "src", "lib.rs")


def _c_prototypes():
    text = "".join(open(h).read() for h in HEADERS)
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(btl_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_ffi_crate_mirrors_the_headers():
    # the Rust FFI crate (bitlinear-hip-sys, source only: no cargo in this image)
    # declares every function of include/*.h with the same arity, every struct
    # with the same fields and every BTL_ constant with the same value
    rs = open(CRATE).read()
    decls = {m.group(1): m.group(2) for m in re.finditer(r"pub fn (btl_[a-z0-9_]+)\(([^)]*)\)", rs, flags=re.S)}
    protos = _c_prototypes()
    assert sorted(protos) == sorted(header_functions())
    assert sorted(decls) == sorted(protos), set(decls) ^ set(protos)
    for name, n in protos.items():
        args = decls[name].strip()
        assert (0 if not args else args.count(":")) == n, name
    text = "".join(open(h).read() for h in HEADERS)
    for name, val in re.findall(r"#define\s+(BTL_[A-Z0-9_]+)\s+(-?\d+)", text):
        assert re.search(r"pub const %s: c_int = %s;" % (name, val), rs), name
    for body, tname in re.findall(r"typedef struct \w+ \{(.*?)\}\s*(\w+);", text, flags=re.S):
        fields = re.findall(r"(\w+)\s*(?:,|;)", re.sub(r"//.*", "", body))
        m = re.search(r"pub struct %s \{(.*?)\}" % tname, rs, flags=re.S)
        assert m, tname
        assert re.findall(r"pub (\w+):", m.group(1)) == fields, tname


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", bl.LIB_PATH], stdout=subprocess.PIPE, text=True,
                         check=True).stdout
    syms = set(l.split()[-1] for l in out.splitlines() if l.strip())
    missing = [f for f in header_functions() if f not in syms]
    assert not missing, missing
    for f in header_functions():
        assert hasattr(bl.lib, f)


def test_version_and_status_strings():
    assert bl.lib.btl_version() == 1
    assert bl.lib.btl_status_string(bl.BTL_ERR_SHAPE) == b"BTL_ERR_SHAPE"
    assert bl.lib.btl_status_string(99) == b"BTL_ERR_UNKNOWN"


def test_packed_bytes():
    assert bl.lib.btl_packed_bytes(5632, 2048) == 5632 * 2048 // 4
    assert bl.lib.btl_packed_bytes(1, 5) == 2
    assert bl.lib.btl_packed_bytes(-1, 5) == -1


@pytest.mark.parametrize("shape", [(40, 64), (7, 33), (1, 5), (256, 2048)])
def test_pack_host_matches_oracle(shape):
    w = weights(*shape, seed=21)
    out = np.zeros((w.size + 3) // 4, np.uint8)
    s = ctypes.c_float()
    bl.check(bl.lib.btl_pack_host(w.ctypes.data, shape[0], shape[1], out.ctypes.data, ctypes.byref(s)))
    ob, osc = orc.pack(w)
    assert np.array_equal(out, ob)
    assert s.value == osc


def test_unpack_host_matches_oracle():
    data = np.arange(256, dtype=np.uint8)
    out = np.zeros(1023, np.float32)
    bl.check(bl.lib.btl_unpack_host(data.ctypes.data, 3, 341, ctypes.c_float(0.37), out.ctypes.data))
    assert np.array_equal(out, orc.unpack(data, 1023, np.float32(0.37)))


def test_rope_table_host_matches_oracle():
    # btl_rope_table is host code: the same table as the oracle, bit for bit, at the Llama-3
    # theta over cfg5's positions (attention.rs:15-42)
    S, hd = 769, 128
    c = np.zeros((S, hd // 2), np.float32)
    s = np.zeros_like(c)
    bl.check(bl.lib.btl_rope_table(500000.0, hd, S, c.ctypes.data, s.ctypes.data))
    oc, osn = orc.rope_table(500000.0, hd, S)
    assert np.array_equal(c.view(np.uint32), oc.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), osn.view(np.uint32))


def test_tuning_knobs_set_get_and_unknown():
    old = bl.get_tuning("BTL_GEMV_BAT_MAX_M")
    try:
        assert bl.set_tuning("GEMV_BAT_MAX_M", 7) == old  # the prefix may be left out
        assert bl.get_tuning("BTL_GEMV_BAT_MAX_M") == 7
        with bl.tuning(BTL_GEMV_BAT_MAX_M=3, BTL_DEC_RQ=0):
            assert bl.get_tuning("BTL_GEMV_BAT_MAX_M") == 3 and bl.get_tuning("BTL_DEC_RQ") == 0
        assert bl.get_tuning("BTL_GEMV_BAT_MAX_M") == 7
    finally:
        bl.set_tuning("BTL_GEMV_BAT_MAX_M", old)
    v = ctypes.c_int()
    assert bl.lib.btl_get_tuning(b"BTL_NO_SUCH_KNOB", ctypes.byref(v)) == bl.BTL_ERR_ARG
    assert b"unknown tuning knob" in bl.lib.btl_last_error()
    assert bl.lib.btl_set_tuning(None, 1) == bl.BTL_ERR_ARG


def test_tuning_reads_the_environment_once():
    # the environment at the first library call sets a knob; later changes to the
    # process environment do not re-route calls
    code = ("import os, bitlinear as bl; a = bl.get_tuning('BTL_GEMV_BAT_MAX_M'); "
            "os.environ['BTL_GEMV_BAT_MAX_M'] = '5'; b = bl.get_tuning('BTL_GEMV_BAT_MAX_M'); "
            "c = bl.get_tuning('BTL_DEC_ROW_MIN_K'); print(a, b, c)")
    path = os.pathsep.join([ROOT, os.path.join(ROOT, "bit-ttt-engine_amd")])
    env = dict(os.environ, BTL_GEMV_BAT_MAX_M="9", PYTHONPATH=path)
    env.pop("BTL_DEC_ROW_MIN_K", None)
    out = subprocess.run([sys.executable, "-c", code], env=env, stdout=subprocess.PIPE, text=True, check=True).stdout
    assert out.split() == ["9", "9", "4096"]


def test_stream_create_rejects_bad_shapes():
    # shape checks of btl_stream_create run before any device work
    def layer(H, I, nkv, q_rows=None):
        L = bl.BtlStreamLayer()
        dims = {"q": (q_rows or H, H), "k": (nkv, H), "v": (nkv, H), "o": (H, q_rows or H), "gate": (I, H),
                "up": (I, H), "down": (H, I)}
        for nm, (n, k) in dims.items():
            setattr(L, nm, bl.BtlPacked(256, n, k, 1.0))
        return L
    h = ctypes.c_void_p()
    for L, frag in ((layer(4160, 512, 64), b"hidden"), (layer(256, 520, 64), b"intermediate"),
                    (layer(256, 512, 64, q_rows=512), b"o reads q"), (layer(256, 16384, 64), b"intermediate")):
        arr = (bl.BtlStreamLayer * 1)(L)
        assert bl.lib.btl_stream_create(arr, 1, ctypes.byref(h)) == bl.BTL_ERR_SHAPE
        assert frag in bl.lib.btl_last_error()
    arr = (bl.BtlStreamLayer * 2)(layer(256, 512, 64), layer(256, 1024, 64))
    assert bl.lib.btl_stream_create(arr, 2, ctypes.byref(h)) == bl.BTL_ERR_SHAPE
    assert bl.lib.btl_stream_create(arr, 0, ctypes.byref(h)) == bl.BTL_ERR_ARG
    assert bl.lib.btl_stream_stage_words(None) == 0
    assert bl.lib.btl_stream_destroy(None) == bl.BTL_OK


def test_workspace_bytes():
    assert bl.lib.btl_workspace_bytes(1, 4096, 4096, bl.BTL_ACT_F32_REF) == 0
    a = bl.lib.btl_workspace_bytes(1, 4096, 4096, bl.BTL_ACT_I8)
    b = bl.lib.btl_workspace_bytes(2048, 4096, 4096, bl.BTL_ACT_I8)
    assert 0 < a < b
    assert b >= 2048 * 4096 + 4 * 2048
    assert bl.lib.btl_workspace_bytes(-1, 1, 1, bl.BTL_ACT_I8) == 0


def _packed(n, k, data=1):
    return bl.BtlPacked(data, n, k, 1.0)


def _linear(w, m, k, xdt=bl.BTL_F32, ydt=bl.BTL_F32, mode=bl.BTL_ACT_I8, acc=None):
    return bl.lib.btl_linear(ctypes.byref(w), 16, xdt, m, k, 16, ydt, mode, acc, None, 0, None)


def test_shape_mismatch_message():
    # cpu.rs:22-30: "Shape mismatch: Input [m, k] vs Weight [n, k_w]"
    w = _packed(5632, 2048)
    rc = _linear(w, 1, 2044)
    assert rc == bl.BTL_ERR_SHAPE
    assert bl.lib.btl_last_error() == b"Shape mismatch: Input [1, 2044] vs Weight [5632, 2048]"
    with pytest.raises(bl.BitLinearError, match="Shape mismatch"):
        bl.check(rc)


def test_validation_errors_before_device_work():
    assert _linear(_packed(8, 6), 1, 6) == bl.BTL_ERR_SHAPE  # k % 4
    assert _linear(_packed(8, 8), -1, 8) == bl.BTL_ERR_SHAPE
    assert _linear(_packed(8, 8), 1, 8, xdt=7) == bl.BTL_ERR_DTYPE
    assert _linear(_packed(8, 8), 1, 8, ydt=3) == bl.BTL_ERR_DTYPE
    assert _linear(_packed(8, 8), 1, 8, mode=5) == bl.BTL_ERR_DTYPE
    assert _linear(_packed(8, 8), 1, 8, mode=bl.BTL_ACT_F32_REF, acc=16) == bl.BTL_ERR_ARG
    assert _linear(_packed(8, 8, data=None), 1, 8) == bl.BTL_ERR_LAYOUT
    assert bl.lib.btl_linear(None, 16, 0, 1, 8, 16, 0, 1, None, None, 0, None) == bl.BTL_ERR_ARG
    # empty problems are successful no-ops (nothing to launch)
    assert _linear(_packed(8, 8), 0, 8) == bl.BTL_OK
    assert _linear(_packed(0, 8), 3, 8) == bl.BTL_OK
    assert bl.lib.btl_linear_group(None, None, 0, 16, 0, 1, 8, 0, None, 0, None) == bl.BTL_ERR_ARG
    assert bl.lib.btl_linear_group(None, None, 5, 16, 0, 1, 8, 0, None, 0, None) == bl.BTL_ERR_ARG


def test_linear_residual_validation():
    # btl_linear_residual checks its arguments before any device work
    f = bl.lib.btl_linear_residual
    w = _packed(8, 64, data=16)
    assert f(ctypes.byref(w), 4096, 9, 1, 64, 8192, 12288, None, 0, None) == bl.BTL_ERR_DTYPE
    assert f(ctypes.byref(w), 4096, bl.BTL_F32, 1, 32, 8192, 12288, None, 0, None) == bl.BTL_ERR_SHAPE
    assert f(None, 4096, bl.BTL_F32, 1, 64, 8192, 12288, None, 0, None) == bl.BTL_ERR_ARG
    assert f(ctypes.byref(w), None, bl.BTL_F32, 1, 64, 8192, 12288, None, 0, None) == bl.BTL_ERR_LAYOUT
    assert f(ctypes.byref(w), 4096, bl.BTL_F32, 1, 64, None, 12288, None, 0, None) == bl.BTL_ERR_LAYOUT
    # y overlapping the residual (8 rows of f32 from 8192) or the input (64 f32 from 4096)
    assert f(ctypes.byref(w), 4096, bl.BTL_F32, 1, 64, 8192, 8196, None, 0, None) == bl.BTL_ERR_LAYOUT
    assert f(ctypes.byref(w), 4096, bl.BTL_F32, 1, 64, 8192, 4160, None, 0, None) == bl.BTL_ERR_LAYOUT
    # empty problems are no-ops
    assert f(ctypes.byref(w), 4096, bl.BTL_F32, 0, 64, 8192, 12288, None, 0, None) == bl.BTL_OK
    assert f(ctypes.byref(_packed(0, 64)), 4096, bl.BTL_F32, 1, 64, 8192, 12288, None, 0, None) == bl.BTL_OK


def test_operand_order_entry_validation():
    w = _packed(64, 128, data=16)
    arr = (ctypes.POINTER(bl.BtlPacked) * 1)(ctypes.pointer(w))
    ys = (ctypes.c_void_p * 1)(16)
    op = bl.lib.btl_linear_i8_op
    assert op(arr, ys, None, 0, 16, 16, 4, 128, 0, None) == bl.BTL_ERR_ARG       # count
    assert op(arr, ys, None, 5, 16, 16, 4, 128, 0, None) == bl.BTL_ERR_ARG
    assert op(None, ys, None, 1, 16, 16, 4, 128, 0, None) == bl.BTL_ERR_ARG
    assert op(arr, ys, None, 1, 16, 16, 4, 128, 9, None) == bl.BTL_ERR_DTYPE     # ydtype
    assert op(arr, ys, None, 1, 16, 16, 4, 124, 0, None) == bl.BTL_ERR_SHAPE     # k != w.k
    assert bl.lib.btl_last_error().startswith(b"Shape mismatch: Input [4, 124] vs Weight [64, 128]")
    w96 = _packed(64, 96, data=16)
    arr96 = (ctypes.POINTER(bl.BtlPacked) * 1)(ctypes.pointer(w96))
    assert op(arr96, ys, None, 1, 16, 16, 4, 96, 0, None) == bl.BTL_ERR_SHAPE    # k % 64
    w_mis = _packed(64, 128, data=24)
    arr_mis = (ctypes.POINTER(bl.BtlPacked) * 1)(ctypes.pointer(w_mis))
    assert op(arr_mis, ys, None, 1, 16, 16, 4, 128, 0, None) == bl.BTL_ERR_LAYOUT  # alignment
    assert op(arr, ys, None, 1, 24, 16, 4, 128, 0, None) == bl.BTL_ERR_LAYOUT
    assert op(arr, ys, None, 1, 16, 16, 0, 128, 0, None) == bl.BTL_OK             # m == 0
    q = bl.lib.btl_quantize_act_op
    assert q(16, 0, 4, 96, 16, 16, None) == bl.BTL_ERR_SHAPE                      # k % 64
    assert q(16, 3, 4, 128, 16, 16, None) == bl.BTL_ERR_DTYPE
    assert q(24, 0, 4, 128, 16, 16, None) == bl.BTL_ERR_LAYOUT                    # alignment
    assert q(None, 0, 4, 128, 16, 16, None) == bl.BTL_ERR_LAYOUT
    assert q(16, 0, 0, 128, 16, 16, None) == bl.BTL_OK


def test_fused_entry_validation():
    w = _packed(64, 128, data=16)
    arr = (ctypes.POINTER(bl.BtlPacked) * 1)(ctypes.pointer(w))
    ys = (ctypes.c_void_p * 1)(16)
    rms = bl.lib.btl_rmsnorm_linear_group
    swi = bl.lib.btl_swiglu_linear_group
    assert rms(arr, ys, 0, 16, 0, 16, 1e-5, 4, 128, 0, None, 0, None) == bl.BTL_ERR_ARG      # count
    assert rms(arr, ys, 1, 16, 5, 16, 1e-5, 4, 128, 0, None, 0, None) == bl.BTL_ERR_DTYPE    # xdtype
    assert rms(arr, ys, 1, 16, 0, 16, 1e-5, 4, 124, 0, None, 0, None) == bl.BTL_ERR_SHAPE    # k != w.k
    w96 = _packed(64, 96, data=16)
    arr96 = (ctypes.POINTER(bl.BtlPacked) * 1)(ctypes.pointer(w96))
    assert rms(arr96, ys, 1, 16, 0, 16, 1e-5, 4, 96, 0, None, 0, None) == bl.BTL_ERR_SHAPE   # k % 64
    big = _packed(64, 65600, data=16)
    arrb = (ctypes.POINTER(bl.BtlPacked) * 1)(ctypes.pointer(big))
    assert rms(arrb, ys, 1, 16, 0, 16, 1e-5, 4, 65600, 0, None, 0, None) == bl.BTL_ERR_SHAPE
    assert rms(arr, ys, 1, 16, 0, None, 1e-5, 4, 128, 0, None, 0, None) == bl.BTL_ERR_LAYOUT  # null g
    assert rms(arr, ys, 1, 24, 0, 16, 1e-5, 4, 128, 0, None, 0, None) == bl.BTL_ERR_LAYOUT    # alignment
    assert rms(arr, ys, 1, 16, 0, 16, 1e-5, 0, 128, 0, None, 0, None) == bl.BTL_OK           # m == 0
    assert swi(arr, ys, 1, 16, None, 0, 4, 128, 0, None, 0, None) == bl.BTL_ERR_LAYOUT       # null up
    assert swi(arr, ys, 1, 16, 24, 0, 4, 128, 0, None, 0, None) == bl.BTL_ERR_LAYOUT         # alignment
    wsw = _packed(64, 32832, data=16)
    arrs = (ctypes.POINTER(bl.BtlPacked) * 1)(ctypes.pointer(wsw))
    assert swi(arrs, ys, 1, 16, 16, 0, 4, 32832, 0, None, 0, None) == bl.BTL_ERR_SHAPE       # k > 32768
    assert swi(arr, ys, 1, 16, 16, 0, 0, 128, 0, None, 0, None) == bl.BTL_OK


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU error path")
def test_no_device_is_an_error():
    rc = bl.lib.btl_init(0)
    assert rc in (bl.BTL_ERR_HIP, bl.BTL_ERR_DEVICE)
    assert bl.lib.btl_last_error() != b""


def test_pack_device_validation():
    p = bl.lib.btl_pack_device
    assert p(16, -1, 4, 16, 16, None, 0, None) == bl.BTL_ERR_SHAPE
    assert p(None, 2, 4, 16, 16, None, 0, None) == bl.BTL_ERR_ARG                # w
    assert p(16, 2, 4, None, 16, None, 0, None) == bl.BTL_ERR_ARG                # out
    assert p(16, 2, 4, 16, None, None, 0, None) == bl.BTL_ERR_ARG                # scale
    assert p(20, 2, 4, 16, 16, None, 0, None) == bl.BTL_ERR_LAYOUT               # w 16 B
    assert p(16, 2, 4, 18, 16, None, 0, None) == bl.BTL_ERR_LAYOUT               # out 4 B
    ws = bl.lib.btl_pack_workspace_bytes
    assert ws(0, 5) == 0 and ws(-1, 5) == 0
    assert ws(1, 4096) == 8 and ws(1, 4097) == 3 * 8
    assert ws(4096, 14336) == (14336 + 4 + 1) * 8


def test_build_rejects_kernels_with_scratch():
    # build.py reads the compiler's kernel-resource-usage remarks and fails on any
    # kernel with scratch memory; its parser on remark lines of both kinds
    import importlib.util
    spec = importlib.util.spec_from_file_location("btl_build", os.path.join(ROOT, "bit-ttt-engine_amd", "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    tail = " [-Rpass-analysis=kernel-resource-usage]"
    lines = ["f.hip:1:1: remark: Function Name: _Z5k_onev" + tail,
             "f.hip:1:1: remark:     VGPRs Spill: 0" + tail,
             "f.hip:1:1: remark:     ScratchSize [bytes/lane]: 0" + tail,
             "f.hip:9:1: remark: Function Name: _Z5k_twov" + tail,
             "f.hip:9:1: remark:     VGPRs Spill: 4" + tail,
             "f.hip:9:1: remark:     ScratchSize [bytes/lane]: 20" + tail]
    assert mod.scratch_kernels(lines) == [("_Z5k_twov", 20, 4)]
    assert mod.scratch_kernels(lines[:3]) == []
