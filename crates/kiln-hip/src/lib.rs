//! kiln-hip: the MI355X (gfx950) affine-quantized linear path for kiln-models.
//!
//! A drop-in for the quantized calls kiln-models makes through kiln-mlx
//! (`kiln_mlx::ops::{quantized_matmul, dequantize, gather_qmm, take}`,
//! crates/kiln-mlx/src/ops.rs:249-484): the same argument lists and meaning,
//! over libkiln_hip's C ABI (`include/kiln_hip.h`). Unsafe code is confined
//! to this crate, as kiln-mlx confines its own.
//!
//! [`DeviceArray`] and [`HipStream`] play the roles of `kiln_mlx::Array` and
//! `kiln_mlx::Stream`: results are caller-allocated device arrays, and every
//! call is enqueued on the stream (synchronise at the step boundary, where
//! kiln-mlx calls `eval`).

pub mod ops;
pub mod sys;

use std::ffi::{c_int, c_void, CStr};

/// A failing library or runtime call, with its message (the role of
/// `kiln_mlx::MlxError`, crates/kiln-mlx/src/error.rs).
#[derive(Debug, Clone, thiserror::Error)]
#[error("kiln-hip error: {message}")]
pub struct HipError {
    pub status: i32,
    pub message: String,
}

/// Maps a kh_status to `Result`, reading the thread-local message as
/// `kiln_mlx::error::check` reads mlx-c's (error.rs:62-72).
pub(crate) fn check(status: c_int) -> Result<(), HipError> {
    if status == sys::KH_OK {
        return Ok(());
    }
    // SAFETY: kh_last_error returns a NUL-terminated thread-local string valid
    // until the next failing call on this thread; it is copied at once.
    let message = unsafe { CStr::from_ptr(sys::kh_last_error()) }.to_string_lossy().into_owned();
    Err(HipError { status, message })
}

pub(crate) fn check_hip(what: &str, e: sys::hipError_t) -> Result<(), HipError> {
    if e == 0 {
        return Ok(());
    }
    // SAFETY: hipGetErrorString returns a static NUL-terminated string.
    let s = unsafe { CStr::from_ptr(sys::hipGetErrorString(e)) }.to_string_lossy().into_owned();
    Err(HipError { status: sys::KH_ERR_DEVICE, message: format!("{what}: {s}") })
}

/// Element types (mlx_dtype numbering).
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum Dtype {
    Uint32,
    Int32,
    Float16,
    Float32,
    Bfloat16,
}

impl Dtype {
    pub fn code(self) -> i32 {
        match self {
            Dtype::Uint32 => sys::KH_UINT32,
            Dtype::Int32 => sys::KH_INT32,
            Dtype::Float16 => sys::KH_FLOAT16,
            Dtype::Float32 => sys::KH_FLOAT32,
            Dtype::Bfloat16 => sys::KH_BFLOAT16,
        }
    }
    pub fn size(self) -> usize {
        match self {
            Dtype::Float16 | Dtype::Bfloat16 => 2,
            _ => 4,
        }
    }
}

/// A HIP stream at default priority, destroyed on drop.
pub struct HipStream {
    raw: sys::kh_stream,
}

impl HipStream {
    pub fn new() -> Result<Self, HipError> {
        let mut raw: sys::kh_stream = std::ptr::null_mut();
        // SAFETY: hipStreamCreate writes a new stream handle into `raw`.
        check_hip("hipStreamCreate", unsafe { sys::hipStreamCreate(&mut raw) })?;
        Ok(Self { raw })
    }
    pub fn raw(&self) -> sys::kh_stream {
        self.raw
    }
    pub fn synchronize(&self) -> Result<(), HipError> {
        // SAFETY: the stream is valid for the lifetime of self.
        check_hip("hipStreamSynchronize", unsafe { sys::hipStreamSynchronize(self.raw) })
    }
}

impl Drop for HipStream {
    fn drop(&mut self) {
        // SAFETY: created by hipStreamCreate and destroyed once.
        unsafe {
            sys::hipStreamDestroy(self.raw);
        }
    }
}

/// Row-contiguous device memory with a shape and dtype; freed on drop.
pub struct DeviceArray {
    desc: sys::kh_array,
    dtype: Dtype,
}

impl DeviceArray {
    /// Uninitialised device memory of `shape` and `dtype`.
    pub fn empty(shape: &[i64], dtype: Dtype) -> Result<Self, HipError> {
        if shape.len() > sys::KH_MAX_NDIM || shape.iter().any(|&d| d < 0) {
            return Err(HipError { status: sys::KH_ERR_INVALID_ARGUMENT, message: format!("bad shape {shape:?}") });
        }
        let mut desc = sys::kh_array {
            data: std::ptr::null_mut(),
            dtype: dtype.code(),
            ndim: shape.len() as i32,
            shape: [0; sys::KH_MAX_NDIM],
        };
        desc.shape[..shape.len()].copy_from_slice(shape);
        let bytes = shape.iter().product::<i64>() as usize * dtype.size();
        if bytes > 0 {
            let mut p: *mut c_void = std::ptr::null_mut();
            // SAFETY: hipMalloc writes a device pointer of `bytes` bytes into p.
            check_hip("hipMalloc", unsafe { sys::hipMalloc(&mut p, bytes) })?;
            desc.data = p;
        }
        Ok(Self { desc, dtype })
    }

    /// Device copy of little-endian host bytes (e.g. a safetensors tensor).
    pub fn from_bytes(bytes: &[u8], shape: &[i64], dtype: Dtype) -> Result<Self, HipError> {
        let a = Self::empty(shape, dtype)?;
        if bytes.len() != a.nbytes() {
            return Err(HipError {
                status: sys::KH_ERR_INVALID_ARGUMENT,
                message: format!("{} bytes do not hold {shape:?} {dtype:?}", bytes.len()),
            });
        }
        if !bytes.is_empty() {
            // SAFETY: both ranges hold nbytes bytes.
            check_hip("hipMemcpy", unsafe {
                sys::hipMemcpy(a.desc.data, bytes.as_ptr().cast(), bytes.len(), sys::HIP_MEMCPY_HOST_TO_DEVICE)
            })?;
        }
        Ok(a)
    }

    /// Host copy of the contents (synchronises with all device work).
    pub fn to_bytes(&self) -> Result<Vec<u8>, HipError> {
        let mut out = vec![0u8; self.nbytes()];
        if !out.is_empty() {
            // SAFETY: both ranges hold nbytes bytes.
            check_hip("hipMemcpy", unsafe {
                sys::hipMemcpy(out.as_mut_ptr().cast(), self.desc.data, out.len(), sys::HIP_MEMCPY_DEVICE_TO_HOST)
            })?;
        }
        Ok(out)
    }

    pub fn shape(&self) -> &[i64] {
        &self.desc.shape[..self.desc.ndim as usize]
    }
    pub fn dtype(&self) -> Dtype {
        self.dtype
    }
    pub fn nbytes(&self) -> usize {
        self.shape().iter().product::<i64>() as usize * self.dtype.size()
    }
    pub(crate) fn raw(&self) -> *const sys::kh_array {
        &self.desc
    }
    pub(crate) fn raw_mut(&mut self) -> *mut sys::kh_array {
        &mut self.desc
    }
}

impl Drop for DeviceArray {
    fn drop(&mut self) {
        if !self.desc.data.is_null() {
            // SAFETY: allocated by hipMalloc and freed once.
            unsafe {
                sys::hipFree(self.desc.data);
            }
        }
    }
}

/// libkiln_hip's version string.
pub fn version() -> String {
    // SAFETY: kh_version returns a static NUL-terminated string.
    unsafe { CStr::from_ptr(sys::kh_version()) }.to_string_lossy().into_owned()
}
