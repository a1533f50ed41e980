//! The HIP arm of the reference's `BitLinear::forward`
//! (`crates/rust_engine/src/layers/bit_linear.rs:67-85`), behind the `candle`
//! feature.
//!
//! candle 0.8.4 has no HIP device, so the arm cannot match on a `Device::Hip`
//! tensor; it is taken when the layer holds a device copy of its packed weights
//! (made once, as the reference packs once in `precompute_packed`,
//! bit_linear.rs:44-50) and the activations arrive as CPU tensors.  The change a
//! maintainer makes in the reference:
//!
//! ```ignore
//! // layers/bit_linear.rs: BitLinear gains
//! #[cfg(feature = "hip")]
//! pub hip: Option<bitlinear_hip_sys::candle_arm::HipPackedTensor>,
//!
//! // precompute_packed (bit_linear.rs:44-50), after `PackedTensor::pack`:
//! #[cfg(feature = "hip")]
//! { self.hip = Some(HipPackedTensor::upload(&packed.data, packed.shape.dims2()?, packed.scale,
//!                                           Mode::F32Ref)?); }
//!
//! // forward (bit_linear.rs:67-85): one more arm ahead of the CPU one
//! let result = match input.device() {
//!     #[cfg(feature = "hip")]
//!     Device::Cpu if self.hip.is_some() => self.hip.as_ref().unwrap().forward(&input),
//!     Device::Cpu => BitLinearCpu::forward(&input, packed),
//!     Device::Cuda(_) => BitLinearCuda::forward(&input, packed),
//!     _ => candle_core::bail!("Packed params present but Custom Kernel not implemented for this device"),
//! }?;
//! ```
//!
//! The rank flattening before the match and the reshape after it
//! (bit_linear.rs:54-62, 88-95) stay as they are.  With `Mode::F32Ref` the
//! result equals BitLinearCpu::forward bit for bit.

use std::sync::Mutex;

use candle_core::{DType, Device, Result, Tensor};

use crate::safe::{self, BitLinearHip, Mode, PackedWeights};

fn to_candle(e: safe::Error) -> candle_core::Error {
    candle_core::Error::Msg(e.message)
}

/// A PackedTensor's bytes on the GPU plus the staging of one BitLinearHip.
pub struct HipPackedTensor {
    weights: PackedWeights,
    mode: Mode,
    engine: Mutex<BitLinearHip>,
}

impl HipPackedTensor {
    /// Upload a PackedTensor's `data` (u8 tensor of ceil(n k / 4) bytes), its
    /// [n, k] shape and scale.
    pub fn upload(data: &Tensor, (n, k): (usize, usize), scale: f32, mode: Mode) -> Result<Self> {
        let bytes = data.flatten_all()?.to_dtype(DType::U8)?.to_vec1::<u8>()?;
        let weights = PackedWeights::from_host_bytes(&bytes, n, k, scale).map_err(to_candle)?;
        let engine = BitLinearHip::new().map_err(to_candle)?;
        Ok(Self { weights, mode, engine: Mutex::new(engine) })
    }

    /// BitLinearCpu::forward's contract (cpu.rs:17-30): input [m, k] f32 on the
    /// CPU, output [m, n] f32 on the CPU; a wrong k fails with the reference's
    /// "Shape mismatch" message.
    pub fn forward(&self, input: &Tensor) -> Result<Tensor> {
        let (m, k) = input.dims2()?;
        let (n, kw) = self.weights.dims();
        if k != kw {
            candle_core::bail!("Shape mismatch: Input [{}, {}] vs Weight [{}, {}]", m, k, n, kw);
        }
        let x = input.to_dtype(DType::F32)?.flatten_all()?.to_vec1::<f32>()?;
        let mut engine = self.engine.lock().map_err(|_| candle_core::Error::Msg("HIP staging poisoned".into()))?;
        let y = engine.forward(&x, m, &self.weights, self.mode).map_err(to_candle)?;
        Tensor::from_vec(y, (m, n), &Device::Cpu)
    }
}

// HipPackedTensor becomes a field of the reference's BitLinear, which lives in
// AdaptiveBitLinear inside BitLlama inside the #[pyclass] PyBitLlama
// (python.rs:18): pyo3 requires Send there, and a model shared across threads
// needs Sync.  Fails to compile if a field loses either.
#[allow(dead_code)]
fn _assert_send_sync() {
    fn check<T: Send + Sync>() {}
    check::<HipPackedTensor>();
}
