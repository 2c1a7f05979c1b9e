//! Safe wrappers with the signatures of `kiln_mlx::ops` (crates/kiln-mlx/src/
//! ops.rs) for the quantized path. Results are allocated here with the shape
//! and dtype the operation produces (MLX's promotion of the operand dtypes),
//! as kiln-mlx returns new arrays; work is enqueued on `s`.

use std::ffi::c_char;

use crate::sys::{self, kh_array, kh_optional_int};
use crate::{check, DeviceArray, Dtype, HipError, HipStream};

pub type Result<T> = std::result::Result<T, HipError>;

const AFFINE: *const c_char = c"affine".as_ptr();

fn opt(v: i32) -> kh_optional_int {
    kh_optional_int { value: v, has_value: true }
}

/// MLX's result dtype of two float operands: equal dtypes keep theirs,
/// anything else gives float32.
pub fn promote(a: Dtype, b: Dtype) -> Dtype {
    if a == b { a } else { Dtype::Float32 }
}

fn codes_per_word(bits: i32) -> i64 {
    if bits == 4 || bits == 8 { 32 / bits as i64 } else { 1 }
}

fn with_last(shape: &[i64], last: i64) -> Vec<i64> {
    let mut s = shape.to_vec();
    if let Some(l) = s.last_mut() {
        *l = last;
    }
    s
}

/// `kiln_mlx::ops::quantized_matmul` (ops.rs:359-388), mode "affine".
#[allow(clippy::too_many_arguments)] // mirrors the reference's parameter list
pub fn quantized_matmul(x: &DeviceArray, w: &DeviceArray, scales: &DeviceArray, biases: &DeviceArray,
                        transpose: bool, group_size: i32, bits: i32, s: &HipStream) -> Result<DeviceArray> {
    let n = if transpose { w.shape()[0] } else { w.shape()[w.shape().len() - 1] * codes_per_word(bits) };
    let mut out = DeviceArray::empty(&with_last(x.shape(), n), promote(x.dtype(), scales.dtype()))?;
    // SAFETY: every descriptor points at live device memory of its shape.
    check(unsafe {
        sys::kh_quantized_matmul(out.raw_mut(), x.raw(), w.raw(), scales.raw(), biases.raw(), transpose,
                                 opt(group_size), opt(bits), AFFINE, s.raw())
    })?;
    Ok(out)
}

/// `Linear::forward`'s quantized arm (crates/kiln-models/src/nn.rs:79-102):
/// the matmul (transpose = true) and the optional bias in one launch.
#[allow(clippy::too_many_arguments)]
pub fn linear(x: &DeviceArray, w: &DeviceArray, scales: &DeviceArray, biases: &DeviceArray,
              bias: Option<&DeviceArray>, group_size: i32, bits: i32, s: &HipStream) -> Result<DeviceArray> {
    let mut dt = promote(x.dtype(), scales.dtype());
    if let Some(b) = bias {
        dt = promote(dt, b.dtype());
    }
    let mut out = DeviceArray::empty(&with_last(x.shape(), w.shape()[0]), dt)?;
    let b = bias.map_or(std::ptr::null(), |b| b.raw());
    // SAFETY: as above; a null bias means none.
    check(unsafe {
        sys::kh_linear(out.raw_mut(), x.raw(), w.raw(), scales.raw(), biases.raw(), b, opt(group_size),
                       opt(bits), AFFINE, s.raw())
    })?;
    Ok(out)
}

/// One quantized projection: packed weights, scales, biases and an optional bias.
pub struct QuantizedProj<'a> {
    pub w: &'a DeviceArray,
    pub scales: &'a DeviceArray,
    pub biases: &'a DeviceArray,
    pub bias: Option<&'a DeviceArray>,
}

/// Several `Linear::forward` calls on one x (q/k/v, nn.rs:724-726).
pub fn linear_multi(x: &DeviceArray, parts: &[QuantizedProj<'_>], group_size: i32, bits: i32,
                    s: &HipStream) -> Result<Vec<DeviceArray>> {
    let mut outs = Vec::with_capacity(parts.len());
    for p in parts {
        let mut dt = promote(x.dtype(), p.scales.dtype());
        if let Some(b) = p.bias {
            dt = promote(dt, b.dtype());
        }
        outs.push(DeviceArray::empty(&with_last(x.shape(), p.w.shape()[0]), dt)?);
    }
    let res: Vec<*mut kh_array> = outs.iter_mut().map(|o| o.raw_mut()).collect();
    let w: Vec<*const kh_array> = parts.iter().map(|p| p.w.raw()).collect();
    let sc: Vec<*const kh_array> = parts.iter().map(|p| p.scales.raw()).collect();
    let bi: Vec<*const kh_array> = parts.iter().map(|p| p.biases.raw()).collect();
    let bs: Vec<*const kh_array> = parts.iter().map(|p| p.bias.map_or(std::ptr::null(), |b| b.raw())).collect();
    // SAFETY: the pointer vectors hold parts.len() live descriptors each.
    check(unsafe {
        sys::kh_linear_multi(parts.len() as i32, res.as_ptr(), x.raw(), w.as_ptr(), sc.as_ptr(), bi.as_ptr(),
                             bs.as_ptr(), opt(group_size), opt(bits), AFFINE, s.raw())
    })?;
    Ok(outs)
}

/// The gated MLP's activation (nn.rs:259-294).
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum Activation {
    Silu,
    GeluApprox,
}

/// `act(gate_proj(x)) * up_proj(x)` of `Mlp::forward` (nn.rs:284-294): the
/// input of down_proj, one launch at decode sizes.
pub fn mlp_gate_up(x: &DeviceArray, gate: &QuantizedProj<'_>, up: &QuantizedProj<'_>, activation: Activation,
                   group_size: i32, bits: i32, s: &HipStream) -> Result<DeviceArray> {
    let mut dt = promote(x.dtype(), gate.scales.dtype());
    if let Some(b) = gate.bias {
        dt = promote(dt, b.dtype());
    }
    let mut out = DeviceArray::empty(&with_last(x.shape(), gate.w.shape()[0]), dt)?;
    let act = match activation {
        Activation::Silu => sys::KH_ACT_SILU,
        Activation::GeluApprox => sys::KH_ACT_GELU_APPROX,
    };
    let bg = gate.bias.map_or(std::ptr::null(), |b| b.raw());
    let bu = up.bias.map_or(std::ptr::null(), |b| b.raw());
    // SAFETY: as above.
    check(unsafe {
        sys::kh_mlp_gate_up(out.raw_mut(), x.raw(), gate.w.raw(), gate.scales.raw(), gate.biases.raw(), bg,
                            up.w.raw(), up.scales.raw(), up.biases.raw(), bu, act, opt(group_size), opt(bits),
                            AFFINE, s.raw())
    })?;
    Ok(out)
}

/// `kiln_mlx::ops::gather_qmm` (ops.rs:390-429) with null lhs_indices.
#[allow(clippy::too_many_arguments)]
pub fn gather_qmm(x: &DeviceArray, w: &DeviceArray, scales: &DeviceArray, biases: &DeviceArray,
                  rhs_indices: &DeviceArray, transpose: bool, group_size: i32, bits: i32, sorted_indices: bool,
                  s: &HipStream) -> Result<DeviceArray> {
    // batch = broadcast(x.shape[:-2], rhs_indices.shape), numpy rules
    let xs = x.shape();
    let xb = &xs[..xs.len().saturating_sub(2)];
    let ib = rhs_indices.shape();
    let nd = xb.len().max(ib.len());
    let mut shape = vec![0i64; nd];
    for d in 0..nd {
        let ex = if d + xb.len() >= nd { xb[d + xb.len() - nd] } else { 1 };
        let ei = if d + ib.len() >= nd { ib[d + ib.len() - nd] } else { 1 };
        shape[d] = if ex == 1 { ei } else { ex };
    }
    shape.push(xs[xs.len() - 2]);
    shape.push(w.shape()[1]);
    let mut out = DeviceArray::empty(&shape, promote(x.dtype(), scales.dtype()))?;
    // SAFETY: as above.
    check(unsafe {
        sys::kh_gather_qmm(out.raw_mut(), x.raw(), w.raw(), scales.raw(), biases.raw(), rhs_indices.raw(),
                           transpose, opt(group_size), opt(bits), AFFINE, sorted_indices, s.raw())
    })?;
    Ok(out)
}

/// `kiln_mlx::ops::dequantize` (ops.rs:456-484); the result has the scales' dtype.
pub fn dequantize(w: &DeviceArray, scales: &DeviceArray, biases: &DeviceArray, group_size: i32, bits: i32,
                  s: &HipStream) -> Result<DeviceArray> {
    let ws = w.shape();
    let mut out = DeviceArray::empty(&with_last(ws, ws[ws.len() - 1] * codes_per_word(bits)), scales.dtype())?;
    // SAFETY: as above.
    check(unsafe {
        sys::kh_dequantize(out.raw_mut(), w.raw(), scales.raw(), biases.raw(), opt(group_size), opt(bits),
                           AFFINE, s.raw())
    })?;
    Ok(out)
}

/// `kiln_mlx::ops::take` (ops.rs:249-254), axis 0.
pub fn take(a: &DeviceArray, indices: &DeviceArray, axis: i32, s: &HipStream) -> Result<DeviceArray> {
    if axis != 0 {
        return Err(HipError { status: sys::KH_ERR_UNSUPPORTED, message: "[take] axis 0 only".into() });
    }
    let mut shape = indices.shape().to_vec();
    shape.extend_from_slice(&a.shape()[1..]);
    let mut out = DeviceArray::empty(&shape, a.dtype())?;
    // SAFETY: as above.
    check(unsafe { sys::kh_take(out.raw_mut(), a.raw(), indices.raw(), s.raw()) })?;
    Ok(out)
}

/// `Embedding::lookup`'s take x3 + dequantize (nn.rs:159-176) in one pass.
pub fn quantized_embedding(ids: &DeviceArray, w: &DeviceArray, scales: &DeviceArray, biases: &DeviceArray,
                           group_size: i32, bits: i32, s: &HipStream) -> Result<DeviceArray> {
    let mut shape = ids.shape().to_vec();
    shape.push(w.shape()[1] * codes_per_word(bits));
    let mut out = DeviceArray::empty(&shape, scales.dtype())?;
    // SAFETY: as above.
    check(unsafe {
        sys::kh_quantized_embedding(out.raw_mut(), ids.raw(), w.raw(), scales.raw(), biases.raw(),
                                    opt(group_size), opt(bits), AFFINE, s.raw())
    })?;
    Ok(out)
}

/// `kiln_mlx::ops::add` with numpy broadcasting.
pub fn add(a: &DeviceArray, b: &DeviceArray, s: &HipStream) -> Result<DeviceArray> {
    let (sa, sb) = (a.shape(), b.shape());
    let nd = sa.len().max(sb.len());
    let shape: Vec<i64> = (0..nd)
        .map(|d| {
            let ea = if d + sa.len() >= nd { sa[d + sa.len() - nd] } else { 1 };
            let eb = if d + sb.len() >= nd { sb[d + sb.len() - nd] } else { 1 };
            if ea == 1 { eb } else { ea }
        })
        .collect();
    let mut out = DeviceArray::empty(&shape, promote(a.dtype(), b.dtype()))?;
    // SAFETY: as above.
    check(unsafe { sys::kh_add(out.raw_mut(), a.raw(), b.raw(), s.raw()) })?;
    Ok(out)
}

/// The affine quantizer (mlx_quantize, the arithmetic of mlx_lm convert,
/// crates/kiln-jobs/src/quantize.rs:72-91): (packed codes, scales, biases).
pub fn quantize(w: &DeviceArray, group_size: i32, bits: i32, s: &HipStream)
                -> Result<(DeviceArray, DeviceArray, DeviceArray)> {
    let ws = w.shape();
    let k = ws[ws.len() - 1];
    let mut q = DeviceArray::empty(&with_last(ws, k * bits as i64 / 32), Dtype::Uint32)?;
    let mut sc = DeviceArray::empty(&with_last(ws, k / group_size as i64), w.dtype())?;
    let mut bi = DeviceArray::empty(&with_last(ws, k / group_size as i64), w.dtype())?;
    // SAFETY: as above.
    check(unsafe {
        sys::kh_quantize(q.raw_mut(), sc.raw_mut(), bi.raw_mut(), w.raw(), opt(group_size), opt(bits), AFFINE,
                         s.raw())
    })?;
    Ok((q, sc, bi))
}
