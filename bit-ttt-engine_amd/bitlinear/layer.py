"""BitLinear layer and its HIP kernel arm (layers/bit_linear.rs, kernels/{cpu,cuda}.rs)."""
import ctypes
import warnings

import numpy as np
import torch

from ._lib import (
    BTL_ACT_F32_REF, BTL_ACT_F32_SEQ, BTL_ACT_I8, BTL_BF16, BTL_ERR_DEVICE, BTL_ERR_DTYPE, BTL_ERR_LAYOUT, BTL_F32,
    BitLinearError, BtlPacked, check, lib,
)
from .packed import PackedTensor

_DT = {torch.float32: BTL_F32, torch.bfloat16: BTL_BF16}
_MODES = {"i8": BTL_ACT_I8, "f32_ref": BTL_ACT_F32_REF, "f32_seq": BTL_ACT_F32_SEQ}


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _dtype_code(t, what):
    if t.dtype not in _DT:
        raise BitLinearError(BTL_ERR_DTYPE, "%s dtype %s is not float32/bfloat16" % (what, t.dtype))
    return _DT[t.dtype]


def _on_gpu(t, what):
    if t.device.type != "cuda":
        # bit_linear.rs:76-84: packed weights on a device without a kernel
        raise BitLinearError(BTL_ERR_DEVICE, "Packed params present but Custom Kernel not implemented "
                             "for this device (%s on %s)" % (what, t.device))
    if not t.is_contiguous():
        raise BitLinearError(BTL_ERR_LAYOUT, "%s must be contiguous" % what)


class Workspace:
    """A caller-owned workspace for btl_linear* (zeroed once at creation; the calls
    do not rely on its contents)."""

    def __init__(self, m, n, k, device="cuda", mode=BTL_ACT_I8):
        self.nbytes = int(lib.btl_workspace_bytes(m, n, k, mode))
        self.buf = torch.empty(max(self.nbytes, 256), dtype=torch.uint8, device=device)
        check(lib.btl_workspace_clear(self.buf.data_ptr(), self.nbytes, _stream(self.buf.device)))

    def args(self):
        return ctypes.c_void_p(self.buf.data_ptr()), self.nbytes


def _ws_args(ws):
    return (None, 0) if ws is None else ws.args()


class BitLinearHip:
    """The HIP arm next to BitLinearCpu::forward (cpu.rs:17) / BitLinearCuda::forward (cuda.rs:21)."""

    @staticmethod
    def forward(input, weights, mode="i8", out_dtype=None, acc_out=None, workspace=None):
        """Y = X W^T.  input [M, K] float32/bfloat16 on the GPU, weights a PackedTensor
        [N, K] on the GPU.  Returns a new [M, N] tensor (dtype out_dtype, default
        the input's).  mode "i8": W1.58-A8; mode "f32_ref": the reference's fp32
        semantics and summation order (its AVX2/FMA lanes); mode "f32_seq": the same
        semantics in the order of a host without AVX2/FMA.  acc_out: optional int32 [M, N] tensor that
        receives the exact accumulators (mode "i8")."""
        if input.dim() != 2:
            raise BitLinearError(1, "input must be 2-D, got %s" % (tuple(input.shape),))
        m, k = input.shape
        n, kw = weights.dims2()
        _on_gpu(input, "input")
        _on_gpu(weights.data, "weights")
        xdt = _dtype_code(input, "input")
        out_dtype = out_dtype or input.dtype
        y = torch.empty((m, n), dtype=out_dtype, device=input.device)
        ydt = _dtype_code(y, "output")
        if mode not in _MODES:
            raise BitLinearError(BTL_ERR_DTYPE, "unknown mode %r" % (mode,))
        acc_ptr = None
        if acc_out is not None:
            if acc_out.dtype != torch.int32 or tuple(acc_out.shape) != (m, n) or not acc_out.is_contiguous():
                raise BitLinearError(BTL_ERR_LAYOUT, "acc_out must be a contiguous int32 [M, N] tensor")
            acc_ptr = acc_out.data_ptr()
        c = weights.as_c()
        wsp, wsn = _ws_args(workspace)
        check(lib.btl_linear(ctypes.byref(c), input.data_ptr() if input.numel() else None, xdt, m, k,
                             y.data_ptr() if y.numel() else None, ydt, _MODES[mode], acc_ptr, wsp, wsn,
                             _stream(input.device)))
        return y


def quantize_act(x):
    """Per-token absmax int8 quantisation on the GPU -> (q int8 [M, K], s float32 [M])."""
    _on_gpu(x, "input")
    m, k = x.shape
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    s = torch.empty((m,), dtype=torch.float32, device=x.device)
    check(lib.btl_quantize_act(x.data_ptr() if x.numel() else None, _dtype_code(x, "input"), m, k,
                               q.data_ptr() if q.numel() else None, s.data_ptr() if m else None,
                               _stream(x.device)))
    return q, s


def linear_i8(q, s, weights, out_dtype=torch.float32, acc_out=None, workspace=None):
    """Contraction of pre-quantised activations (btl_linear_i8)."""
    _on_gpu(q, "input")
    m, k = q.shape
    n, _ = weights.dims2()
    y = torch.empty((m, n), dtype=out_dtype, device=q.device)
    c = weights.as_c()
    wsp, wsn = _ws_args(workspace)
    check(lib.btl_linear_i8(ctypes.byref(c), q.data_ptr() if q.numel() else None,
                            s.data_ptr() if s.numel() else None, m, k, y.data_ptr() if y.numel() else None,
                            _dtype_code(y, "output"), acc_out.data_ptr() if acc_out is not None else None,
                            wsp, wsn, _stream(q.device)))
    return y


def quantize_act_op(x):
    """btl_quantize_act_op: (q int8 [M, K] in operand order, s float32 [M])."""
    _on_gpu(x, "input")
    m, k = x.shape
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    s = torch.empty((m,), dtype=torch.float32, device=x.device)
    check(lib.btl_quantize_act_op(x.data_ptr() if x.numel() else None, _dtype_code(x, "input"), m, k,
                                  q.data_ptr() if q.numel() else None, s.data_ptr() if m else None,
                                  _stream(x.device)))
    return q, s


def linear_i8_op(q, s, weights, out_dtype=torch.float32, acc_out=None, outputs=None):
    """btl_linear_i8_op: the prefill GEMM on operand-order activations, one launch
    for the list of layers `weights` (1..4).  Returns the list of outputs."""
    _on_gpu(q, "input")
    m, k = q.shape
    if outputs is None:
        outputs = [torch.empty((m, w.dims2()[0]), dtype=out_dtype, device=q.device) for w in weights]
    cs = [w.as_c() for w in weights]
    arr = (ctypes.POINTER(BtlPacked) * len(cs))(*[ctypes.pointer(c) for c in cs])
    ys = (ctypes.c_void_p * len(cs))(*[o.data_ptr() if o.numel() else None for o in outputs])
    accs = None
    if acc_out is not None:
        accs = (ctypes.c_void_p * len(cs))(*[a.data_ptr() if a is not None else None for a in acc_out])
    check(lib.btl_linear_i8_op(arr, ys, accs, len(cs), q.data_ptr() if q.numel() else None,
                               s.data_ptr() if s.numel() else None, m, k, _dtype_code(outputs[0], "output"),
                               _stream(q.device)))
    return outputs


def _group_args(weights, m, dtype, device, outputs):
    if outputs is None:
        outputs = [torch.empty((m, w.dims2()[0]), dtype=dtype, device=device) for w in weights]
    cs = [w.as_c() for w in weights]
    arr = (ctypes.POINTER(BtlPacked) * len(cs))(*[ctypes.pointer(c) for c in cs])
    ys = (ctypes.c_void_p * len(cs))(*[o.data_ptr() if o.numel() else None for o in outputs])
    return outputs, cs, arr, ys


def rmsnorm_linear_group(weights, x, g, eps, out_dtype=None, workspace=None, outputs=None):
    """btl_rmsnorm_linear_group: BitLinear layers applied to RMSNorm(x) * g
    (rms_norm.rs:33-56) without materialising the normalised tensor."""
    _on_gpu(x, "input")
    m, k = x.shape
    out_dtype = out_dtype or x.dtype
    g = g.to(device=x.device, dtype=torch.float32).contiguous()
    outputs, cs, arr, ys = _group_args(weights, m, out_dtype, x.device, outputs)
    wsp, wsn = _ws_args(workspace)
    check(lib.btl_rmsnorm_linear_group(arr, ys, len(cs), x.data_ptr() if x.numel() else None,
                                       _dtype_code(x, "input"), g.data_ptr(), float(eps), m, k,
                                       _dtype_code(outputs[0], "output"), wsp, wsn, _stream(x.device)))
    return outputs


def swiglu_linear_group(weights, gate, up, out_dtype=None, workspace=None, outputs=None):
    """btl_swiglu_linear_group: BitLinear layers applied to silu(gate) * up
    (swiglu.rs:29-35) without materialising the hidden tensor."""
    _on_gpu(gate, "gate")
    _on_gpu(up, "up")
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise BitLinearError(1, "gate and up must have the same shape and dtype")
    m, k = gate.shape
    out_dtype = out_dtype or gate.dtype
    outputs, cs, arr, ys = _group_args(weights, m, out_dtype, gate.device, outputs)
    wsp, wsn = _ws_args(workspace)
    check(lib.btl_swiglu_linear_group(arr, ys, len(cs), gate.data_ptr() if gate.numel() else None,
                                      up.data_ptr() if up.numel() else None, _dtype_code(gate, "input"), m, k,
                                      _dtype_code(outputs[0], "output"), wsp, wsn, _stream(gate.device)))
    return outputs


def linear_group(weights, x, out_dtype=None, workspace=None, outputs=None, mode="i8"):
    """Several layers reading the same input in one launch (q|k|v, w1|w3), in
    W1.58-A8 (mode "i8") or the reference's fp32 order (mode "f32_ref", or "f32_seq"
    for its non-AVX2 order, one launch per layer)."""
    if mode not in _MODES:
        raise BitLinearError(BTL_ERR_DTYPE, "unknown mode %r" % (mode,))
    _on_gpu(x, "input")
    m, k = x.shape
    out_dtype = out_dtype or x.dtype
    if outputs is None:
        outputs = [torch.empty((m, w.dims2()[0]), dtype=out_dtype, device=x.device) for w in weights]
    cs = [w.as_c() for w in weights]
    arr = (ctypes.POINTER(BtlPacked) * len(cs))(*[ctypes.pointer(c) for c in cs])
    ys = (ctypes.c_void_p * len(cs))(*[o.data_ptr() for o in outputs])
    wsp, wsn = _ws_args(workspace)
    check(lib.btl_linear_group_mode(arr, ys, len(cs), x.data_ptr(), _dtype_code(x, "input"), m, k,
                                    _dtype_code(outputs[0], "output"), _MODES[mode], wsp, wsn, _stream(x.device)))
    return outputs


def linear_residual(weight, x, resid, out=None, workspace=None):
    """btl_linear_residual: resid + x W^T (the residual connection after a
    BitLinear, block.rs:119,131), f32 out; `out` must not overlap `resid`."""
    _on_gpu(x, "input")
    _on_gpu(resid, "residual")
    m, k = x.shape
    n = weight.dims2()[0]
    if resid.dtype != torch.float32 or tuple(resid.shape) != (m, n):
        raise BitLinearError(BTL_ERR_LAYOUT, "residual must be float32 [%d, %d]" % (m, n))
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=x.device)
    c = weight.as_c()
    wsp, wsn = _ws_args(workspace)
    check(lib.btl_linear_residual(ctypes.byref(c), x.data_ptr() if x.numel() else None, _dtype_code(x, "input"), m,
                                  k, resid.data_ptr() if resid.numel() else None,
                                  out.data_ptr() if out.numel() else None, wsp, wsn, _stream(x.device)))
    return out


class BitLinear:
    """1.58-bit linear layer (layers/bit_linear.rs:12-21)."""

    def __init__(self, weight, in_features, out_features):
        self.weight = weight
        self.in_features = in_features
        self.out_features = out_features
        self.packed_params = None

    @staticmethod
    def load(in_dim, out_dim, weight, device="cuda"):
        """bit_linear.rs:24-41, with the dense [out_dim, in_dim] weight given directly."""
        if tuple(weight.shape) != (out_dim, in_dim):
            raise BitLinearError(1, "weight shape %s is not [%d, %d]" % (tuple(weight.shape), out_dim, in_dim))
        return BitLinear(weight.to(device, torch.float32).contiguous(), in_dim, out_dim)

    def precompute_packed(self):
        """bit_linear.rs:44-50: absmean-ternarise and pack once."""
        self.packed_params = PackedTensor.pack(self.weight)

    def forward(self, x, mode="i8"):
        """bit_linear.rs:52-119: flatten rank > 2 to [B*T, K], run the packed kernel,
        reshape back.  Without packed params this is the reference's STE training
        path (bit_linear.rs:98-118): a dense matmul with ste_weight(W), no scale --
        the reference's path for layers that were never packed, not a fallback of
        the packed kernel (a packed layer always runs the HIP library)."""
        orig = None
        inp = x
        if x.dim() > 2:
            orig = list(x.shape)
            inp = x.reshape(-1, x.shape[-1])
        if self.packed_params is not None:
            y = BitLinearHip.forward(inp.contiguous(), self.packed_params, mode=mode)
            if orig is not None:
                orig[-1] = y.shape[1]
                return y.reshape(orig)
            return y
        warnings.warn("BitLinear: no packed params, using the STE training path", stacklevel=2)
        return matmul_robust(x.to(torch.float32), ste_weight(self.weight).t())


def ste_weight(w):
    """The straight-through weight of BitLinear's training path (bit_linear.rs:101-110):
        scale   = mean_all(|w|)                       (no epsilon here, unlike pack)
        w_s     = w / scale   -> candle's Tensor / f64 = affine(1/scale, 0):
                  w * (f32)(1 / (f64)scale) + 0
        w_q     = round(w_s).clamp(-1, 1)             (f32::round: half away from zero)
        w_ste   = (w_q - w_s).detach() + w_s          (f32 ops; differs from w_q by rounding)
    Gradients flow to w through w_s (d w_ste / d w = 1 / scale).  The mean is taken in
    float64 and rounded once; candle's own f32 reduction order is not vendored, so its
    last ulp is not pinned."""
    w = w.to(torch.float32)
    s = float(np.float32(w.detach().abs().double().mean().item())) if w.numel() else float("nan")
    inv = float(np.float32(1.0 / s)) if s != 0.0 else float("inf")
    w_s = w * inv + 0.0
    a = w_s.detach().abs().double()
    w_q = (torch.sign(w_s.detach()) * torch.floor(a + 0.5).to(torch.float32)).clamp(-1.0, 1.0)
    return (w_q - w_s).detach() + w_s


def matmul_robust(lhs, rhs):
    """TensorExt::matmul_robust (layers.rs:28-59): rhs moved to lhs's device, rank 1
    lhs as one row, rank > 2 flattened to [B*T, K] and reshaped back."""
    lhs = lhs.contiguous()
    rhs = rhs.contiguous().to(lhs.device)
    if lhs.dim() == 1:
        return (lhs.unsqueeze(0) @ rhs).squeeze(0)
    if lhs.dim() == 2:
        return lhs @ rhs
    out = lhs.reshape(-1, lhs.shape[-1]) @ rhs
    return out.reshape(*lhs.shape[:-1], out.shape[1])
