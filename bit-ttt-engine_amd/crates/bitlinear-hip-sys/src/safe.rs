//! Safe wrapper over the raw bindings: owned device buffers and streams, packed
//! weights resident on the GPU, and BitLinear forwards that either stay on the
//! device or stage host slices the way `BitLinearCpu::forward` takes them
//! (cpu.rs:17-30: f32 [m, k] in, f32 [m, n] out).

use std::ffi::CStr;
use std::fmt;
use std::os::raw::{c_int, c_void};
use std::ptr;

use crate::*;

/// A failed call: the library's status and message (btl_last_error), or a HIP
/// runtime error (status BTL_ERR_HIP).
#[derive(Clone, Debug)]
pub struct Error {
    pub status: c_int,
    pub message: String,
}

impl fmt::Display for Error {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        let name = unsafe { CStr::from_ptr(btl_status_string(self.status)) }.to_string_lossy();
        write!(f, "{}: {}", name, self.message)
    }
}

impl std::error::Error for Error {}

pub type Result<T> = std::result::Result<T, Error>;

/// BTL_OK -> Ok; anything else -> Err with this thread's btl_last_error().  The
/// shape errors carry the reference's own strings ("Shape mismatch: Input [m, k]
/// vs Weight [n, k_w]", cpu.rs:24-29).
pub fn check(status: c_int) -> Result<()> {
    if status == BTL_OK {
        return Ok(());
    }
    let message = unsafe { CStr::from_ptr(btl_last_error()) }.to_string_lossy().into_owned();
    Err(Error { status, message })
}

fn hip(e: hipError_t, what: &str) -> Result<()> {
    if e == HIP_SUCCESS {
        return Ok(());
    }
    let s = unsafe { CStr::from_ptr(hipGetErrorString(e)) }.to_string_lossy().into_owned();
    Err(Error { status: BTL_ERR_HIP, message: format!("{}: {}", what, s) })
}

/// btl_init: select the device and set up the library there.
pub fn init(device: i32) -> Result<()> {
    hip(unsafe { hipSetDevice(device) }, "hipSetDevice")?;
    check(unsafe { btl_init(device) })
}

/// Device memory owned by the wrapper (hipMalloc / hipFree).
pub struct DeviceBuffer {
    ptr: *mut c_void,
    bytes: usize,
}

impl DeviceBuffer {
    pub fn new(bytes: usize) -> Result<Self> {
        let mut ptr = ptr::null_mut();
        if bytes > 0 {
            hip(unsafe { hipMalloc(&mut ptr, bytes) }, "hipMalloc")?;
        }
        Ok(Self { ptr, bytes })
    }

    pub fn from_slice<T: Copy>(data: &[T]) -> Result<Self> {
        let mut b = Self::new(std::mem::size_of_val(data))?;
        b.upload(data)?;
        Ok(b)
    }

    /// Synchronous host -> device copy into the start of the buffer.
    pub fn upload<T: Copy>(&mut self, data: &[T]) -> Result<()> {
        let n = std::mem::size_of_val(data);
        assert!(n <= self.bytes, "upload of {} bytes into a buffer of {}", n, self.bytes);
        if n == 0 {
            return Ok(());
        }
        hip(unsafe { hipMemcpy(self.ptr, data.as_ptr() as *const c_void, n, HIP_MEMCPY_HOST_TO_DEVICE) },
            "hipMemcpy (to device)")
    }

    /// Synchronous device -> host copy from the start of the buffer.
    pub fn download<T: Copy>(&self, out: &mut [T]) -> Result<()> {
        let n = std::mem::size_of_val(out);
        assert!(n <= self.bytes, "download of {} bytes from a buffer of {}", n, self.bytes);
        if n == 0 {
            return Ok(());
        }
        hip(unsafe { hipMemcpy(out.as_mut_ptr() as *mut c_void, self.ptr, n, HIP_MEMCPY_DEVICE_TO_HOST) },
            "hipMemcpy (to host)")
    }

    pub fn as_ptr(&self) -> *const c_void {
        self.ptr
    }

    pub fn as_mut_ptr(&mut self) -> *mut c_void {
        self.ptr
    }

    pub fn len(&self) -> usize {
        self.bytes
    }

    pub fn is_empty(&self) -> bool {
        self.bytes == 0
    }
}

// HIP device pointers and streams are plain handles that the HIP runtime lets
// any host thread use (its API is thread-safe), so the owning wrappers may move
// between threads and be shared: every method that writes through one takes
// `&mut self`, and shared `&self` use only reads device memory or enqueues work
// on a stream, which HIP orders itself.  The reference's BitLinear sits inside
// a #[pyclass] (python.rs:18), which pyo3 requires to be Send.
unsafe impl Send for DeviceBuffer {}
unsafe impl Sync for DeviceBuffer {}

impl Drop for DeviceBuffer {
    fn drop(&mut self) {
        if !self.ptr.is_null() {
            unsafe {
                hipFree(self.ptr);
            }
        }
    }
}

/// A HIP stream owned by the wrapper (default priority).
pub struct Stream(hipStream_t);

impl Stream {
    pub fn new() -> Result<Self> {
        let mut s = ptr::null_mut();
        hip(unsafe { hipStreamCreate(&mut s) }, "hipStreamCreate")?;
        Ok(Self(s))
    }

    pub fn raw(&self) -> *mut c_void {
        self.0
    }

    pub fn synchronize(&self) -> Result<()> {
        hip(unsafe { hipStreamSynchronize(self.0) }, "hipStreamSynchronize")
    }
}

unsafe impl Send for Stream {}
unsafe impl Sync for Stream {}

impl Drop for Stream {
    fn drop(&mut self) {
        unsafe {
            hipStreamDestroy(self.0);
        }
    }
}

/// Arithmetic of a BitLinear call.
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Mode {
    /// the reference's fp32 semantics and summation order (BitLinearCpu::forward, bit for bit)
    F32Ref,
    /// W1.58-A8: per-token absmax int8 activations, exact int32 sums
    I8,
}

impl Mode {
    fn code(self) -> c_int {
        match self {
            Mode::F32Ref => BTL_ACT_F32_REF,
            Mode::I8 => BTL_ACT_I8,
        }
    }
}

/// A PackedTensor (packing.rs:14-21) with its bytes resident on the GPU.
pub struct PackedWeights {
    buf: DeviceBuffer,
    raw: btl_packed_t,
}

// `raw` points into `buf`, which the value owns; the bytes are read-only after
// the upload.
unsafe impl Send for PackedWeights {}
unsafe impl Sync for PackedWeights {}

impl PackedWeights {
    /// Upload the bytes of a PackedTensor (its `data`, flat [ceil(n k / 4)] u8) and scale.
    pub fn from_host_bytes(bytes: &[u8], n: usize, k: usize, scale: f32) -> Result<Self> {
        let need = unsafe { btl_packed_bytes(n as i64, k as i64) };
        if need < 0 || bytes.len() as i64 != need {
            return Err(Error {
                status: BTL_ERR_SHAPE,
                message: format!("packed bytes: got {}, [{}, {}] needs {}", bytes.len(), n, k, need),
            });
        }
        let buf = DeviceBuffer::from_slice(bytes)?;
        let raw = btl_packed_t { data: buf.as_ptr() as *const u8, n: n as i64, k: k as i64, scale };
        Ok(Self { buf, raw })
    }

    /// PackedTensor::pack of host f32 weights [n, k] (packing.rs:50-105), then upload.
    pub fn pack_host(w: &[f32], n: usize, k: usize) -> Result<Self> {
        assert_eq!(w.len(), n * k, "weights are [n, k]");
        let need = unsafe { btl_packed_bytes(n as i64, k as i64) } as usize;
        let mut bytes = vec![0u8; need];
        let mut scale = 0.0f32;
        check(unsafe { btl_pack_host(w.as_ptr(), n as i64, k as i64, bytes.as_mut_ptr(), &mut scale) })?;
        Self::from_host_bytes(&bytes, n, k, scale)
    }

    /// Pack f32 weights [n, k] that already live on the device (btl_pack_device).
    pub fn pack_device(w: &DeviceBuffer, n: usize, k: usize, stream: &Stream) -> Result<Self> {
        assert!(w.len() >= n * k * 4, "weights are [n, k] f32");
        let need = unsafe { btl_packed_bytes(n as i64, k as i64) } as usize;
        let mut buf = DeviceBuffer::new(need)?;
        let mut scale_dev = DeviceBuffer::new(4)?;
        check(unsafe {
            btl_pack_device(w.as_ptr() as *const f32, n as i64, k as i64, buf.as_mut_ptr() as *mut u8,
                            scale_dev.as_mut_ptr() as *mut f32, ptr::null_mut(), 0, stream.raw())
        })?;
        stream.synchronize()?;
        let mut scale = [0.0f32];
        scale_dev.download(&mut scale)?;
        let raw = btl_packed_t { data: buf.as_ptr() as *const u8, n: n as i64, k: k as i64, scale: scale[0] };
        Ok(Self { buf, raw })
    }

    pub fn raw(&self) -> &btl_packed_t {
        &self.raw
    }

    pub fn dims(&self) -> (usize, usize) {
        (self.raw.n as usize, self.raw.k as usize)
    }

    pub fn bytes(&self) -> &DeviceBuffer {
        &self.buf
    }
}

/// y[m, n] = x[m, k] W^T on the device, f32 in and out (btl_linear; the library
/// workspace when the mode needs one).
pub fn linear(w: &PackedWeights, x: &DeviceBuffer, m: usize, y: &mut DeviceBuffer, mode: Mode, stream: &Stream)
              -> Result<()> {
    let (n, k) = w.dims();
    assert!(x.len() >= m * k * 4 && y.len() >= m * n * 4, "x is [m, k] and y [m, n] f32");
    check(unsafe {
        btl_linear(w.raw(), x.as_ptr(), BTL_F32, m as i64, k as i64, y.as_mut_ptr(), BTL_F32, mode.code(),
                   ptr::null_mut(), ptr::null_mut(), 0, stream.raw())
    })
}

/// Several layers reading the same x (q|k|v, w1|w3) in one launch
/// (btl_linear_group_mode), f32 in and out.
pub fn linear_group(ws: &[&PackedWeights], x: &DeviceBuffer, m: usize, ys: &mut [&mut DeviceBuffer], mode: Mode,
                    stream: &Stream) -> Result<()> {
    assert!(!ws.is_empty() && ws.len() == ys.len() && ws.len() <= 4, "1..4 layers, one output each");
    let k = ws[0].dims().1;
    let raws: Vec<*const btl_packed_t> = ws.iter().map(|w| w.raw() as *const btl_packed_t).collect();
    let outs: Vec<*mut c_void> = ys.iter_mut().map(|y| y.as_mut_ptr()).collect();
    for (w, y) in ws.iter().zip(ys.iter()) {
        assert!(y.len() >= m * w.dims().0 * 4, "each y is [m, n] f32");
    }
    assert!(x.len() >= m * k * 4, "x is [m, k] f32");
    check(unsafe {
        btl_linear_group_mode(raws.as_ptr(), outs.as_ptr(), ws.len() as c_int, x.as_ptr(), BTL_F32, m as i64,
                              k as i64, BTL_F32, mode.code(), ptr::null_mut(), 0, stream.raw())
    })
}

/// BitLinearCpu::forward's contract on the GPU (cpu.rs:17-127): host f32 [m, k]
/// in, host f32 [m, n] out, weights resident on the device.  Keeps its staging
/// buffers and stream between calls.
pub struct BitLinearHip {
    stream: Stream,
    x: DeviceBuffer,
    y: DeviceBuffer,
}

impl BitLinearHip {
    pub fn new() -> Result<Self> {
        Ok(Self { stream: Stream::new()?, x: DeviceBuffer::new(0)?, y: DeviceBuffer::new(0)? })
    }

    pub fn forward(&mut self, x: &[f32], m: usize, w: &PackedWeights, mode: Mode) -> Result<Vec<f32>> {
        let (n, k) = w.dims();
        if m * k != x.len() {
            // the library raises the reference's "Shape mismatch" for a wrong k; a
            // slice that is not [m, k] is the caller's error here
            return Err(Error { status: BTL_ERR_SHAPE, message: format!("input of {} floats is not [{}, {}]",
                                                                        x.len(), m, k) });
        }
        if self.x.len() < x.len() * 4 {
            self.x = DeviceBuffer::new(x.len() * 4)?;
        }
        if self.y.len() < m * n * 4 {
            self.y = DeviceBuffer::new(m * n * 4)?;
        }
        self.x.upload(x)?;
        linear(w, &self.x, m, &mut self.y, mode, &self.stream)?;
        self.stream.synchronize()?;
        check(unsafe { btl_check_faults(self.stream.raw()) })?;
        let mut out = vec![0.0f32; m * n];
        self.y.download(&mut out)?;
        Ok(out)
    }
}

// Compile-time check that the wrappers can live inside the reference's layers.
#[allow(dead_code)]
fn _assert_send_sync() {
    fn check<T: Send + Sync>() {}
    check::<DeviceBuffer>();
    check::<Stream>();
    check::<PackedWeights>();
    check::<BitLinearHip>();
}
