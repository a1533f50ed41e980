"""Host-side mirror of the reference's BitLinear interface, over the C ABI.

Reference (imonoonoko/Bit-TTT-Engine, crates/rust_engine/src):
  PackedTensor::{new, pack, unpack}         kernels/packing.rs:14-133
  BitLinearCpu / BitLinearCuda ::forward    kernels/cpu.rs:17, kernels/cuda.rs:21
  BitLinear::{load, precompute_packed, forward}   layers/bit_linear.rs:12-119

Here the device arm is BitLinearHip (libbitlinear_hip.so, gfx950).  Device
memory and streams come from torch; every computation on packed weights runs
in the HIP library, and there is no CPU implementation of the kernels in this
package (a CPU tensor reaching a packed forward is an error, as for an
unsupported device in bit_linear.rs:76-84).
"""
from ._lib import (  # noqa: F401
    BTL_ACT_F32_REF, BTL_ACT_F32_SEQ, BTL_ACT_I8, BTL_BF16, BTL_ERR_ARG, BTL_ERR_DEVICE, BTL_ERR_DTYPE, BTL_ERR_FAULT,
    BTL_ERR_HIP, BTL_ERR_LAYOUT, BTL_ERR_SHAPE, BTL_ERR_WORKSPACE, BTL_F32, BTL_OK, EXPORTS,
    LIB_PATH, BitLinearError, BtlKvQ8, BtlPacked, BtlStreamLayer, check, check_faults, get_tuning, lib, set_tuning, tuning,
)
from .packed import PackedTensor  # noqa: F401
from .layer import (  # noqa: F401
    BitLinear, BitLinearHip, Workspace, linear_group, linear_i8, linear_i8_op, linear_residual, quantize_act,
    quantize_act_op, rmsnorm_linear_group, swiglu_linear_group,
)
from .adaptive import AdaptiveBitLinear, reconstruct_dense, split_bases  # noqa: F401,E402
