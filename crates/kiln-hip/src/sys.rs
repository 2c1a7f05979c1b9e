//! Raw `extern "C"` bindings of `include/kiln_hip.h` (libkiln_hip.so) and the
//! few HIP runtime calls the safe layer needs. Hand-written: the surface is
//! small and every type mirrors the header field for field (checked against
//! the header by the repository's `tests/test_crate_sys.py`).
//!
//! Handles are plain structs: `kh_array` is a borrowed view of row-contiguous
//! device memory, `kh_optional_int` has the layout of mlx-c's
//! `mlx_optional_int`. Every call returns 0 or a non-zero `kh_status`; the
//! message of the last failing call on the calling thread comes from
//! `kh_last_error`.

#![allow(non_camel_case_types, dead_code)]

use std::ffi::{c_char, c_int, c_void};

pub const KH_MAX_NDIM: usize = 8;

// kh_dtype (mlx_dtype numbering)
pub const KH_BOOL: i32 = 0;
pub const KH_UINT8: i32 = 1;
pub const KH_UINT16: i32 = 2;
pub const KH_UINT32: i32 = 3;
pub const KH_UINT64: i32 = 4;
pub const KH_INT8: i32 = 5;
pub const KH_INT16: i32 = 6;
pub const KH_INT32: i32 = 7;
pub const KH_INT64: i32 = 8;
pub const KH_FLOAT16: i32 = 9;
pub const KH_FLOAT32: i32 = 10;
pub const KH_FLOAT64: i32 = 11;
pub const KH_BFLOAT16: i32 = 12;
pub const KH_COMPLEX64: i32 = 13;

// kh_status
pub const KH_OK: c_int = 0;
pub const KH_ERR_INVALID_ARGUMENT: c_int = 1;
pub const KH_ERR_UNSUPPORTED: c_int = 2;
pub const KH_ERR_DEVICE: c_int = 3;
pub const KH_ERR_NO_DEVICE: c_int = 4;

// kh_activation
pub const KH_ACT_SILU: c_int = 0;
pub const KH_ACT_GELU_APPROX: c_int = 1;

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct kh_array {
    pub data: *mut c_void,
    pub dtype: i32,
    pub ndim: i32,
    pub shape: [i64; KH_MAX_NDIM],
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct kh_optional_int {
    pub value: i32,
    pub has_value: bool,
}

pub type kh_stream = *mut c_void;

unsafe extern "C" {
    pub fn kh_quantized_matmul(res: *mut kh_array, x: *const kh_array, w: *const kh_array,
                               scales: *const kh_array, biases: *const kh_array, transpose: bool,
                               group_size: kh_optional_int, bits: kh_optional_int,
                               mode: *const c_char, stream: kh_stream) -> c_int;
    pub fn kh_quantize(w_q: *mut kh_array, scales: *mut kh_array, biases: *mut kh_array,
                       w: *const kh_array, group_size: kh_optional_int, bits: kh_optional_int,
                       mode: *const c_char, stream: kh_stream) -> c_int;
    pub fn kh_dequantize(res: *mut kh_array, w: *const kh_array, scales: *const kh_array,
                         biases: *const kh_array, group_size: kh_optional_int,
                         bits: kh_optional_int, mode: *const c_char, stream: kh_stream) -> c_int;
    pub fn kh_take(res: *mut kh_array, a: *const kh_array, indices: *const kh_array,
                   stream: kh_stream) -> c_int;
    pub fn kh_quantized_matmul_multi(n: c_int, res: *const *mut kh_array, x: *const kh_array,
                                     w: *const *const kh_array, scales: *const *const kh_array,
                                     biases: *const *const kh_array, transpose: bool,
                                     group_size: kh_optional_int, bits: kh_optional_int,
                                     mode: *const c_char, stream: kh_stream) -> c_int;
    pub fn kh_quantized_gate_up(res: *mut kh_array, x: *const kh_array, w_gate: *const kh_array,
                                scales_gate: *const kh_array, biases_gate: *const kh_array,
                                w_up: *const kh_array, scales_up: *const kh_array,
                                biases_up: *const kh_array, group_size: kh_optional_int,
                                bits: kh_optional_int, mode: *const c_char,
                                stream: kh_stream) -> c_int;
    pub fn kh_linear(res: *mut kh_array, x: *const kh_array, w: *const kh_array,
                     scales: *const kh_array, biases: *const kh_array, bias: *const kh_array,
                     group_size: kh_optional_int, bits: kh_optional_int, mode: *const c_char,
                     stream: kh_stream) -> c_int;
    pub fn kh_linear_multi(n: c_int, res: *const *mut kh_array, x: *const kh_array,
                           w: *const *const kh_array, scales: *const *const kh_array,
                           biases: *const *const kh_array, bias: *const *const kh_array,
                           group_size: kh_optional_int, bits: kh_optional_int,
                           mode: *const c_char, stream: kh_stream) -> c_int;
    pub fn kh_mlp_gate_up(res: *mut kh_array, x: *const kh_array, w_gate: *const kh_array,
                          scales_gate: *const kh_array, biases_gate: *const kh_array,
                          bias_gate: *const kh_array, w_up: *const kh_array,
                          scales_up: *const kh_array, biases_up: *const kh_array,
                          bias_up: *const kh_array, activation: c_int,
                          group_size: kh_optional_int, bits: kh_optional_int,
                          mode: *const c_char, stream: kh_stream) -> c_int;
    pub fn kh_gather_qmm(res: *mut kh_array, x: *const kh_array, w: *const kh_array,
                         scales: *const kh_array, biases: *const kh_array,
                         rhs_indices: *const kh_array, transpose: bool,
                         group_size: kh_optional_int, bits: kh_optional_int,
                         mode: *const c_char, sorted_indices: bool, stream: kh_stream) -> c_int;
    pub fn kh_quantized_embedding(res: *mut kh_array, ids: *const kh_array, w: *const kh_array,
                                  scales: *const kh_array, biases: *const kh_array,
                                  group_size: kh_optional_int, bits: kh_optional_int,
                                  mode: *const c_char, stream: kh_stream) -> c_int;
    pub fn kh_add(res: *mut kh_array, a: *const kh_array, b: *const kh_array,
                  stream: kh_stream) -> c_int;
    pub fn kh_quantized_matmul_noalloc(res: *mut kh_array, x: *const kh_array, w: *const kh_array,
                                       scales: *const kh_array, biases: *const kh_array,
                                       transpose: bool, group_size: kh_optional_int,
                                       bits: kh_optional_int, mode: *const c_char,
                                       stream: kh_stream) -> c_int;
    pub fn kh_noalloc_scratch_bytes() -> usize;
    pub fn kh_quantized_matmul_plan(m: i64, n: i64, k: i64, group_size: c_int, bits: c_int,
                                    x_dtype: c_int, scales_dtype: c_int, buf: *mut c_char,
                                    len: usize) -> c_int;
    pub fn kh_last_error() -> *const c_char;
    pub fn kh_version() -> *const c_char;
}

// HIP runtime (libamdhip64): device memory and streams for the safe layer.
pub type hipError_t = c_int;
pub const HIP_MEMCPY_HOST_TO_DEVICE: c_int = 1;
pub const HIP_MEMCPY_DEVICE_TO_HOST: c_int = 2;

unsafe extern "C" {
    pub fn hipMalloc(ptr: *mut *mut c_void, size: usize) -> hipError_t;
    pub fn hipFree(ptr: *mut c_void) -> hipError_t;
    pub fn hipMemcpy(dst: *mut c_void, src: *const c_void, size: usize, kind: c_int) -> hipError_t;
    pub fn hipStreamCreate(stream: *mut kh_stream) -> hipError_t;
    pub fn hipStreamDestroy(stream: kh_stream) -> hipError_t;
    pub fn hipStreamSynchronize(stream: kh_stream) -> hipError_t;
    pub fn hipGetErrorString(e: hipError_t) -> *const c_char;
}
