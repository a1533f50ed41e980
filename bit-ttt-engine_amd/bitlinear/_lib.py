"""ctypes binding of libbitlinear_hip.so (the C ABI declared in include/bitlinear.h).

The library is required: importing this module raises if it is missing, so no
code path can silently fall back to a CPU implementation.
"""
import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_PKG), "libbitlinear_hip.so")

BTL_OK = 0
BTL_ERR_SHAPE = 1
BTL_ERR_DTYPE = 2
BTL_ERR_LAYOUT = 3
BTL_ERR_DEVICE = 4
BTL_ERR_HIP = 5
BTL_ERR_ARG = 6
BTL_ERR_WORKSPACE = 7
BTL_ERR_FAULT = 8

BTL_F32 = 0
BTL_BF16 = 1

BTL_ACT_F32_REF = 0
BTL_ACT_I8 = 1
BTL_ACT_F32_SEQ = 2

# Every symbol include/bitlinear.h declares.
EXPORTS = (
    "btl_version", "btl_last_error", "btl_status_string", "btl_init", "btl_set_tuning", "btl_get_tuning",
    "btl_check_faults", "btl_last_gemm_form", "btl_packed_bytes",
    "btl_pack_host", "btl_unpack_host", "btl_pack_device", "btl_pack_workspace_bytes", "btl_unpack_device",
    "btl_quantize_act", "btl_linear", "btl_linear_noalloc",
    "btl_linear_i8", "btl_linear_group", "btl_linear_group_mode", "btl_quantize_act_op", "btl_linear_i8_op",
    "btl_rmsnorm_linear_group", "btl_swiglu_linear_group",
    "btl_workspace_bytes", "btl_workspace_clear",
    "btl_adaptive_split", "btl_adaptive_reconstruct", "btl_adaptive_linear", "btl_adaptive_workspace_bytes",
    # include/bitllama.h
    "btl_rope_table", "btl_rope_kv_append", "btl_attention_workspace_bytes", "btl_attention",
    "btl_rope_append_attention",
    "btl_embedding", "btl_greedy_next", "btl_add_rmsnorm", "btl_swiglu", "btl_dense_linear",
    "btl_add_rmsnorm_linear_group", "btl_add_rmsnorm_swiglu",
    "btl_add_rmsnorm_swiglu_workspace_bytes", "btl_linear_residual",
    "btl_add_rmsnorm_linear_group_ref",
    "btl_stream_create", "btl_stream_stage_words", "btl_stream_run", "btl_stream_destroy",
)


class BtlPacked(ctypes.Structure):
    """btl_packed_t: mirrors the reference's PackedTensor (kernels/packing.rs:14-21)."""
    _fields_ = [("data", ctypes.c_void_p), ("n", ctypes.c_int64), ("k", ctypes.c_int64),
                ("scale", ctypes.c_float)]


class BtlKvQ8(ctypes.Structure):
    """btl_kv_q8_t: one layer of the reference's QuantizedKVCache (kv_cache.rs:14-22)."""
    _fields_ = [("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("k_scale", ctypes.c_void_p),
                ("v_scale", ctypes.c_void_p), ("n_kv_heads", ctypes.c_int64), ("max_seq", ctypes.c_int64),
                ("head_dim", ctypes.c_int64)]


class BtlStreamLayer(ctypes.Structure):
    """btl_stream_layer_t: the seven packed projections of one decoder layer."""
    _fields_ = [(nm, BtlPacked) for nm in ("q", "k", "v", "o", "gate", "up", "down")]


class BitLinearError(RuntimeError):
    """A non-zero status from the C ABI; .status holds the code."""

    def __init__(self, status, message):
        super().__init__(message)
        self.status = status


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError("libbitlinear_hip.so not built at %s (run bit-ttt-engine_amd/build.py)" % LIB_PATH)
    lib = ctypes.CDLL(LIB_PATH)
    vp, i64, i32, f32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    P = ctypes.POINTER
    sig = {
        "btl_version": (i32, []),
        "btl_last_error": (ctypes.c_char_p, []),
        "btl_status_string": (ctypes.c_char_p, [i32]),
        "btl_init": (i32, [i32]),
        "btl_set_tuning": (i32, [ctypes.c_char_p, i32]),
        "btl_get_tuning": (i32, [ctypes.c_char_p, P(i32)]),
        "btl_check_faults": (i32, [vp]),
        "btl_last_gemm_form": (ctypes.c_char_p, []),
        "btl_packed_bytes": (i64, [i64, i64]),
        "btl_pack_host": (i32, [vp, i64, i64, vp, P(f32)]),
        "btl_unpack_host": (i32, [vp, i64, i64, f32, vp]),
        "btl_unpack_device": (i32, [P(BtlPacked), vp, vp]),
        "btl_pack_device": (i32, [vp, i64, i64, vp, vp, vp, sz, vp]),
        "btl_pack_workspace_bytes": (sz, [i64, i64]),
        "btl_quantize_act": (i32, [vp, i32, i64, i64, vp, vp, vp]),
        "btl_linear": (i32, [P(BtlPacked), vp, i32, i64, i64, vp, i32, i32, vp, vp, sz, vp]),
        "btl_linear_noalloc": (i32, [P(BtlPacked), vp, i32, i64, i64, vp, i32, i32, vp, vp]),
        "btl_linear_i8": (i32, [P(BtlPacked), vp, vp, i64, i64, vp, i32, vp, vp, sz, vp]),
        "btl_linear_group": (i32, [P(P(BtlPacked)), P(vp), i32, vp, i32, i64, i64, i32, vp, sz, vp]),
        "btl_linear_group_mode": (i32, [P(P(BtlPacked)), P(vp), i32, vp, i32, i64, i64, i32, i32, vp, sz, vp]),
        "btl_quantize_act_op": (i32, [vp, i32, i64, i64, vp, vp, vp]),
        "btl_linear_i8_op": (i32, [P(P(BtlPacked)), P(vp), P(vp), i32, vp, vp, i64, i64, i32, vp]),
        "btl_rmsnorm_linear_group": (i32, [P(P(BtlPacked)), P(vp), i32, vp, i32, vp, f32, i64, i64, i32, vp, sz,
                                           vp]),
        "btl_swiglu_linear_group": (i32, [P(P(BtlPacked)), P(vp), i32, vp, vp, i32, i64, i64, i32, vp, sz, vp]),
        "btl_workspace_bytes": (sz, [i64, i64, i64, i32]),
        "btl_workspace_clear": (i32, [vp, sz, vp]),
        "btl_adaptive_split": (i32, [vp, i64, i64, i32, P(vp), vp]),
        "btl_adaptive_reconstruct": (i32, [vp, P(f32), i32, i64, i64, vp, vp]),
        "btl_adaptive_linear": (i32, [P(P(BtlPacked)), i32, vp, i32, i64, i64, vp, i32, vp, sz, vp]),
        "btl_adaptive_workspace_bytes": (sz, [i64, i64, i64, i32]),
        "btl_rope_table": (i32, [ctypes.c_double, i64, i64, vp, vp]),
        "btl_rope_kv_append": (i32, [vp, vp, vp, i64, i64, P(BtlKvQ8), i64, vp, vp, vp, vp, vp]),
        "btl_attention_workspace_bytes": (sz, [i64, i64, P(BtlKvQ8)]),
        "btl_attention": (i32, [vp, i64, i64, P(BtlKvQ8), i64, vp, vp, vp, sz, vp]),
        "btl_rope_append_attention": (i32, [vp, vp, vp, i64, i64, P(BtlKvQ8), i64, vp, vp, vp, vp, vp, sz, vp]),
        "btl_embedding": (i32, [vp, i32, i64, i64, vp, i64, vp, vp]),
        "btl_greedy_next": (i32, [vp, i64, vp, vp, vp, i64, vp]),
        "btl_add_rmsnorm": (i32, [vp, vp, vp, vp, f32, i64, i64, vp, vp]),
        "btl_dense_linear": (i32, [vp, i32, i64, i64, vp, i64, vp, vp]),
        "btl_swiglu": (i32, [vp, vp, i64, vp, vp]),
        "btl_add_rmsnorm_linear_group_ref": (i32, [P(P(BtlPacked)), P(vp), i32, vp, vp, vp, vp, f32, i64, i64, vp]),
        "btl_add_rmsnorm_linear_group": (i32, [P(P(BtlPacked)), P(vp), i32, vp, vp, vp, vp, f32, i64, i64, i32, vp,
                                               sz, vp]),
        "btl_add_rmsnorm_swiglu": (i32, [P(BtlPacked), P(BtlPacked), vp, vp, vp, vp, f32, i64, i64, vp, vp, sz, vp]),
        "btl_add_rmsnorm_swiglu_workspace_bytes": (sz, [i64, i64, i64]),
        "btl_linear_residual": (i32, [P(BtlPacked), vp, i32, i64, i64, vp, vp, vp, sz, vp]),
        "btl_stream_create": (i32, [P(BtlStreamLayer), i32, P(vp)]),
        "btl_stream_stage_words": (sz, [vp]),
        "btl_stream_run": (i32, [vp, vp, vp, vp, vp]),
        "btl_stream_destroy": (i32, [vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def get_tuning(name):
    """Current value of a routing / tuning knob (btl_get_tuning)."""
    v = ctypes.c_int()
    check(lib.btl_get_tuning(name.encode(), ctypes.byref(v)))
    return v.value


def set_tuning(name, value):
    """Set a routing / tuning knob (btl_set_tuning); returns the previous value."""
    old = get_tuning(name)
    check(lib.btl_set_tuning(name.encode(), int(value)))
    return old


class tuning:
    """Context manager: knobs set for the body, restored afterwards.
    with tuning(BTL_DEC_RQ=0, BTL_DEC_ROW=0): ..."""

    def __init__(self, **knobs):
        self.knobs = knobs
        self.saved = {}

    def __enter__(self):
        for k, v in self.knobs.items():
            self.saved[k] = set_tuning(k, v)
        return self

    def __exit__(self, *exc):
        for k, v in self.saved.items():
            set_tuning(k, v)
        return False


def check_faults(stream=None):
    """btl_check_faults: synchronise the stream and raise if a kernel's bounded wait gave up."""
    check(lib.btl_check_faults(stream))


def check(status):
    """Raise BitLinearError for a non-zero status, with the library's message."""
    if status != BTL_OK:
        msg = lib.btl_last_error().decode("utf-8", "replace")
        name = lib.btl_status_string(status).decode()
        raise BitLinearError(status, "%s: %s" % (name, msg))
    return status
