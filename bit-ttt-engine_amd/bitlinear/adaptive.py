"""AdaptiveBitLinear: the reference's multi-base ternary layer (layers/adaptive_linear.rs:31-169)
on the C ABI.

The reference loads weight_packed [out, in/4, nb] u8 + scales [nb] and rebuilds
dense f32 weights on the host at load time (adaptive_linear.rs:86-117), then runs
a dense matmul.  Here the interleaved bytes are split once on the device into nb
PackedTensors (btl_adaptive_split) and the forward is W1.58-A8 over the bases
(btl_adaptive_linear).  Mode "f32_ref" keeps the reference's own arithmetic
instead: the dense f32 weights rebuilt on the device at load (reconstruct_dense,
bit-identical to the reference's loop) and a dense f32 matmul per forward
(btl_dense_linear, in its fixed summation order).
"""
import ctypes

import numpy as np
import torch

from ._lib import BTL_ERR_DTYPE, BTL_ERR_SHAPE, BTL_F32, BitLinearError, BtlPacked, check, lib
from .layer import BitLinear, _dtype_code, _on_gpu, _stream, _ws_args
from .packed import PackedTensor


def split_bases(weight_packed, out_dim, in_dim, scales):
    """btl_adaptive_split: [out, in/4, nb] interleaved bytes (GPU) -> nb PackedTensors."""
    weight_packed = weight_packed.contiguous()
    _on_gpu(weight_packed, "weight_packed")
    nb = len(scales)
    if weight_packed.numel() != out_dim * (in_dim // 4) * nb or in_dim % 4:
        raise BitLinearError(BTL_ERR_SHAPE, "weight_packed has %d bytes, [%d, %d/4, %d] needs %d"
                             % (weight_packed.numel(), out_dim, in_dim, nb, out_dim * (in_dim // 4) * nb))
    dev = weight_packed.device
    outs = [torch.empty((out_dim * in_dim // 4,), dtype=torch.uint8, device=dev) for _ in range(nb)]
    ptrs = (ctypes.c_void_p * nb)(*[o.data_ptr() for o in outs])
    check(lib.btl_adaptive_split(weight_packed.contiguous().data_ptr(), out_dim, in_dim, nb, ptrs, _stream(dev)))
    return [PackedTensor(o, float(s), (out_dim, in_dim), dev) for o, s in zip(outs, scales)]


def reconstruct_dense(weight_packed, scales, out_dim, in_dim):
    """The reference's load-time reconstruction (adaptive_linear.rs:86-117) on the GPU:
    float32 [out, in], bases added in order."""
    weight_packed = weight_packed.contiguous()
    _on_gpu(weight_packed, "weight_packed")
    nb = len(scales)
    out = torch.empty((out_dim, in_dim), dtype=torch.float32, device=weight_packed.device)
    sc = (ctypes.c_float * nb)(*[float(s) for s in scales])
    check(lib.btl_adaptive_reconstruct(weight_packed.contiguous().data_ptr(), sc, nb, out_dim, in_dim,
                                       out.data_ptr(), _stream(out.device)))
    return out


class AdaptiveBitLinear:
    """adaptive_linear.rs:31-37: either a legacy BitLinear, or the multi-base weights as
    split bases (mode "i8") or as the reference's reconstructed dense weights (mode
    "f32_ref", the `reconstructed_weight` of adaptive_linear.rs:119-124)."""

    def __init__(self, in_features, out_features, bases=None, legacy_linear=None, reconstructed_weight=None):
        self.in_features = in_features
        self.out_features = out_features
        self.bases = bases
        self.legacy_linear = legacy_linear
        self.reconstructed_weight = reconstructed_weight
        self._c = None

    @staticmethod
    def load(in_dim, out_dim, weight_packed=None, scales=None, legacy_weight=None, device="cuda", mode="i8"):
        """adaptive_linear.rs:38-129: a legacy dense weight (BitLinear) if given, else the
        multi-base format with 1..8 bases: split into PackedTensor bases (mode "i8") or
        rebuilt into dense f32 weights on the device (mode "f32_ref", adaptive_linear.rs:86-117)."""
        if mode not in ("i8", "f32_ref"):
            raise BitLinearError(BTL_ERR_DTYPE, "unknown mode %r" % (mode,))
        if legacy_weight is not None:
            return AdaptiveBitLinear(in_dim, out_dim, legacy_linear=BitLinear.load(in_dim, out_dim, legacy_weight,
                                                                                  device))
        if weight_packed is None or scales is None or not 1 <= len(scales) <= 8:
            raise BitLinearError(6, "Failed to load layer: neither legacy nor adaptive weights found")
        wp = torch.as_tensor(np.asarray(weight_packed, np.uint8)) if not torch.is_tensor(weight_packed) \
            else weight_packed
        if wp.dtype != torch.uint8:  # adaptive_linear.rs:69-78: F32 packed bytes are cast
            wp = wp.to(torch.uint8)
        wp = wp.to(device).contiguous()
        if mode == "f32_ref":
            return AdaptiveBitLinear(in_dim, out_dim,
                                     reconstructed_weight=reconstruct_dense(wp, list(scales), out_dim, in_dim))
        return AdaptiveBitLinear(in_dim, out_dim, bases=split_bases(wp, out_dim, in_dim, list(scales)))

    def precompute_packed(self):
        """adaptive_linear.rs:162-168."""
        if self.legacy_linear is not None:
            self.legacy_linear.precompute_packed()

    def forward(self, x, out_dtype=None, workspace=None):
        """adaptive_linear.rs:131-160: rank-3 input flattened to [B*T, in]; y [.., out]."""
        if self.legacy_linear is not None:
            return self.legacy_linear.forward(x)
        if self.reconstructed_weight is None and self.bases is None:  # adaptive_linear.rs:159
            raise BitLinearError(6, "AdaptiveBitLinear: Invalid State")
        orig = None
        inp = x
        if x.dim() == 3:
            orig = x.shape[:2]
            inp = x.reshape(-1, x.shape[-1])
        _on_gpu(inp, "input")
        inp = inp.contiguous()
        m, k = inp.shape
        n = self.out_features
        if self.reconstructed_weight is not None:
            y = self._forward_dense(inp, out_dtype)
        else:
            y = torch.empty((m, n), dtype=out_dtype or inp.dtype, device=inp.device)
            if self._c is None:
                cs = [b.as_c() for b in self.bases]
                self._c = (cs, (ctypes.POINTER(BtlPacked) * len(cs))(*[ctypes.pointer(c) for c in cs]))
            wsp, wsn = _ws_args(workspace)
            check(lib.btl_adaptive_linear(self._c[1], len(self.bases), inp.data_ptr(), _dtype_code(inp, "input"),
                                          m, k, y.data_ptr(), _dtype_code(y, "output"), wsp, wsn,
                                          _stream(inp.device)))
        return y.reshape(*orig, n) if orig is not None else y

    def _forward_dense(self, inp, out_dtype):
        """x_flat.matmul(w_recon.t()) (adaptive_linear.rs:141-151) in f32: the weights
        follow the input's device, a bf16 input is widened exactly, y is f32."""
        if out_dtype not in (None, torch.float32):
            raise BitLinearError(BTL_ERR_DTYPE, "mode f32_ref produces float32 outputs, not %s" % (out_dtype,))
        _dtype_code(inp, "input")
        m, k = inp.shape
        n = self.out_features
        if k != self.in_features:
            raise BitLinearError(BTL_ERR_SHAPE, "input has %d features, the layer %d" % (k, self.in_features))
        w = self.reconstructed_weight
        if w.device != inp.device:  # adaptive_linear.rs:143-149
            w = w.to(inp.device)
        xf = inp.float().contiguous()
        y = torch.empty((m, n), dtype=torch.float32, device=inp.device)
        # btl_dense_linear takes at most 65535 rows per call
        for r0 in range(0, m, 65535):
            r = min(65535, m - r0)
            check(lib.btl_dense_linear(w.data_ptr(), BTL_F32, n, k, xf[r0:].data_ptr(), r, y[r0:].data_ptr(),
                                       _stream(inp.device)))
        return y
