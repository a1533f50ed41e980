"""The decode stream (include/bitllama.h btl_stream_*): the one-token projection
chain of every layer -- q|k|v, o, silu(gate) * up, down -- in one persistent
launch, bf16 between the stages.

Reference: the per-layer BitLinear::forward calls of one decoder step
(crates/rust_engine/src/model/block.rs:90-138 -> layers/bit_linear.rs:52-119;
attention.rs:159-162, swiglu.rs:29-35), in dependency order.
"""
import ctypes

import torch

from ._lib import BtlStreamLayer, check, lib


class DecodeStream:
    """A plan over `layers`: a list of dicts of PackedTensor on the GPU with keys
    q, k, v, o, gate, up, down (every layer of the same shapes)."""

    def __init__(self, layers):
        self.layers = layers
        arr = (BtlStreamLayer * len(layers))()
        for i, L in enumerate(layers):
            for nm in ("q", "k", "v", "o", "gate", "up", "down"):
                setattr(arr[i], nm, L[nm].as_c())
        self._arr = arr
        h = ctypes.c_void_p()
        check(lib.btl_stream_create(arr, len(layers), ctypes.byref(h)))
        self.plan = h
        self.hidden = layers[0]["q"].dims2()[1]
        self.words = int(lib.btl_stream_stage_words(h))
        self.device = layers[0]["q"].data.device

    def run(self, x, y=None, stage_out=None, stream=None):
        """x: bf16 [hidden] on the GPU -> y (bf16 [hidden]); stage_out: optional bf16
        [stage_words] buffer for every stage's output."""
        if y is None:
            y = torch.empty((self.hidden,), dtype=torch.bfloat16, device=self.device)
        st = stream if stream is not None else torch.cuda.current_stream(self.device).cuda_stream
        check(lib.btl_stream_run(self.plan, x.data_ptr(), y.data_ptr(),
                                 stage_out.data_ptr() if stage_out is not None else None, ctypes.c_void_p(st)))
        return y

    def close(self):
        if self.plan:
            check(lib.btl_stream_destroy(self.plan))
            self.plan = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
