"""PackedTensor: the reference's 2-bit ternary weight container (kernels/packing.rs:14-133)."""
import ctypes

import numpy as np
import torch

from ._lib import BitLinearError, BtlPacked, BTL_ERR_SHAPE, check, lib


class PackedTensor:
    """Packed ternary weights.

    data:     torch.uint8 [ceil(numel/4)], element e in byte e/4 at bits 2*(e%4),
              codes 00 = 0, 01 = +1, 10 = -1, 11 = 0 (packing.rs:6-13)
    scale:    float, mean|W| + 1e-6 (packing.rs:56-57)
    shape:    original shape, [out_dim, in_dim] for a linear layer
    num_elem: number of weights
    device:   torch.device of `data`
    """

    def __init__(self, data, scale, shape, device):
        self.data = data
        self.scale = float(scale)
        self.shape = tuple(int(s) for s in shape)
        self.num_elem = int(np.prod(self.shape)) if self.shape else 1
        self.device = torch.device(device)

    # packing.rs:25-47
    @staticmethod
    def new(data, shape, scale, device="cpu"):
        """Wrap raw packed bytes.  Like Tensor::from_vec in the reference, the
        byte count must equal ceil(numel/4)."""
        shape = tuple(int(s) for s in shape)
        numel = int(np.prod(shape)) if shape else 1
        buf = torch.as_tensor(np.asarray(data, dtype=np.uint8).reshape(-1)) if not torch.is_tensor(data) \
            else data.reshape(-1).to(torch.uint8)
        cap = (numel + 3) // 4
        if buf.numel() != cap:
            raise BitLinearError(BTL_ERR_SHAPE, "packed data has %d bytes, shape %s needs %d"
                                 % (buf.numel(), shape, cap))
        return PackedTensor(buf.to(device).contiguous(), scale, shape, device)

    # packing.rs:50-105
    @staticmethod
    def pack(tensor):
        """Absmean-ternarise and pack a float tensor (btl_pack_host); the result
        lives on the tensor's device."""
        device = tensor.device
        host = tensor.detach().to("cpu", torch.float32).contiguous()
        numel = host.numel()
        out = torch.empty(((numel + 3) // 4,), dtype=torch.uint8)
        scale = ctypes.c_float(0.0)
        n = host.shape[0] if host.dim() == 2 else 1
        k = host.shape[1] if host.dim() == 2 else numel
        check(lib.btl_pack_host(host.data_ptr() if numel else None, n, k,
                                out.data_ptr() if numel else None, ctypes.byref(scale)))
        return PackedTensor(out.to(device), scale.value, tuple(host.shape), device)

    @staticmethod
    def pack_device(tensor):
        """PackedTensor::pack on the GPU (btl_pack_device): bit-identical to pack()
        for a float32 tensor already on the device."""
        if tensor.device.type != "cuda":
            raise BitLinearError(2, "pack_device needs a GPU tensor")
        from .layer import _stream
        w = tensor.detach().to(torch.float32).contiguous()
        numel = w.numel()
        out = torch.empty(((numel + 3) // 4,), dtype=torch.uint8, device=w.device)
        scale = torch.empty((1,), dtype=torch.float32, device=w.device)
        n = w.shape[0] if w.dim() == 2 else 1
        k = w.shape[1] if w.dim() == 2 else numel
        check(lib.btl_pack_device(w.data_ptr() if numel else None, n, k, out.data_ptr() if numel else None,
                                  scale.data_ptr(), None, 0, _stream(w.device)))
        return PackedTensor(out, float(scale.item()), tuple(w.shape), w.device)

    # packing.rs:108-133
    def unpack(self, device=None):
        """Dense float32 weights t*scale with the original shape."""
        device = torch.device(device) if device is not None else self.device
        out = torch.empty(self.num_elem, dtype=torch.float32, device=self.data.device)
        if self.data.device.type == "cuda":
            if self.num_elem:
                from .layer import _stream
                c = self.as_c()
                check(lib.btl_unpack_device(ctypes.byref(c), out.data_ptr(), _stream(self.data.device)))
        else:
            if self.num_elem:
                check(lib.btl_unpack_host(self.data.data_ptr(), 1, self.num_elem, ctypes.c_float(self.scale),
                                          out.data_ptr()))
        return out.reshape(self.shape).to(device)

    def dims2(self):
        if len(self.shape) != 2:
            raise BitLinearError(BTL_ERR_SHAPE, "packed weight shape %s is not 2-D" % (self.shape,))
        return self.shape

    def as_c(self):
        n, k = self.shape if len(self.shape) == 2 else (1, self.num_elem)
        return BtlPacked(self.data.data_ptr() if self.data.numel() else None, n, k, self.scale)

    def to(self, device):
        return PackedTensor(self.data.to(device), self.scale, self.shape, device)

    def __repr__(self):
        return "PackedTensor(shape=%s, scale=%g, device=%s)" % (self.shape, self.scale, self.device)
