"""Host-side mirror of `kiln_mlx::ops` for the quantized path, over libkiln_hip.

Same names, argument order and meaning as the reference wrappers
(crates/kiln-mlx/src/ops.rs):

    quantized_matmul(x, w, scales, biases, transpose, group_size, bits)  ops.rs:359-388
    dequantize(w, scales, biases, group_size, bits)                      ops.rs:456-484
    take(a, indices, axis)                                                ops.rs:249-254

plus `quantized_embedding`, the fused take+dequantize of Embedding::lookup
(crates/kiln-models/src/nn.rs:159-176). Failures raise `KilnError` carrying
the library's message, as `check` turns mlx-c status codes into `MlxError`
(crates/kiln-mlx/src/error.rs:62-72).

Tensors are torch tensors resident on the GPU (torch is the device-memory and
stream plumbing here). Work is enqueued on torch's current stream for the
tensors' device, or on `stream` (a torch.cuda.Stream) when given; like MLX's
lazy evaluation, results are ready once that stream is synchronised.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

_TORCH_TO_KH = {
    torch.bfloat16: _lib.BFLOAT16,
    torch.float16: _lib.FLOAT16,
    torch.float32: _lib.FLOAT32,
    torch.uint32: _lib.UINT32,
    torch.int32: _lib.INT32,
    torch.uint8: _lib.UINT8,
    torch.int8: _lib.INT8,
    torch.int16: _lib.INT16,
    torch.uint16: _lib.UINT16,
    torch.int64: _lib.INT64,
    torch.float64: _lib.FLOAT64,
    torch.bool: _lib.BOOL,
}

_NAMES = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


class KilnError(RuntimeError):
    """A failing library call: `status` is the kh_status code."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status
        self.message = message


def _check(status: int) -> None:
    if status != 0:
        raise KilnError(status, _lib.last_error() or _lib.STATUS.get(status, str(status)))


def _desc(t: torch.Tensor, name: str, as_dtype: int | None = None) -> _lib.KhArray:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise KilnError(1, f"{name} must be a GPU tensor (got device {t.device}); "
                           "libkiln_hip runs on gfx950 only")
    if not t.is_contiguous():
        raise KilnError(1, f"{name} must be row-contiguous")
    dt = as_dtype if as_dtype is not None else _TORCH_TO_KH.get(t.dtype)
    if dt is None:
        raise KilnError(1, f"{name} has unsupported dtype {t.dtype}")
    return _lib.array(t.data_ptr(), dt, t.shape)


def _packed(w: torch.Tensor) -> _lib.KhArray:
    # Packed weights are uint32; an int32 tensor holding the same bits is
    # accepted and reinterpreted (torch has few uint32 kernels).
    if w.dtype in (torch.uint32, torch.int32):
        return _desc(w, "w", _lib.UINT32)
    return _desc(w, "w")


def _stream_handle(t: torch.Tensor, stream) -> int:
    s = stream if stream is not None else torch.cuda.current_stream(t.device)
    return s.cuda_stream


def result_dtype(x_dtype: torch.dtype, s_dtype: torch.dtype) -> torch.dtype:
    """MLX type promotion over (x, scales, biases): equal float types stay,
    bf16 with f16 (or anything with f32) promotes to float32."""
    return x_dtype if x_dtype == s_dtype else torch.float32


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                     biases: torch.Tensor, transpose: bool = True, group_size: int = 64,
                     bits: int = 4, *, mode: str = "affine", out_dtype=None,
                     out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """`x @ dequantize(w, scales, biases)^T` (transpose) or `x @ dequantize(...)`."""
    if isinstance(out_dtype, str):
        out_dtype = _NAMES[out_dtype]
    if transpose:
        N = w.shape[0]
    else:
        N = w.shape[-1] * (32 // bits) if bits in (4, 8) else w.shape[-1]
    if out is None:
        od = out_dtype or result_dtype(x.dtype, scales.dtype)
        out = torch.empty((*x.shape[:-1], N), dtype=od, device=x.device)
    _check(_lib.lib().kh_quantized_matmul(
        _desc(out, "res"), _desc(x, "x"), _packed(w), _desc(scales, "scales"),
        _desc(biases, "biases"), bool(transpose), _lib.opt(group_size), _lib.opt(bits),
        mode.encode() if mode is not None else None, _stream_handle(x, stream)))
    return out


def _ptrs(descs):
    P = ctypes.POINTER(_lib.KhArray)
    arr = (P * len(descs))(*[ctypes.pointer(d) for d in descs])
    return arr, descs  # keep the descriptors alive with the array


def quantized_matmul_multi(x: torch.Tensor, parts, transpose: bool = True, group_size: int = 64,
                           bits: int = 4, *, mode: str = "affine", out_dtype=None, outs=None,
                           stream=None):
    """[x @ dequantize(w_i, s_i, b_i)^T for (w_i, s_i, b_i) in parts], one
    launch where the decode GEMV applies (the q/k/v projections)."""
    if isinstance(out_dtype, str):
        out_dtype = _NAMES[out_dtype]
    if outs is None:
        outs = []
        for w, sc, _ in parts:
            N = w.shape[0] if transpose else w.shape[-1] * (32 // bits)
            od = out_dtype or result_dtype(x.dtype, sc.dtype)
            outs.append(torch.empty((*x.shape[:-1], N), dtype=od, device=x.device))
    res, k0 = _ptrs([_desc(o, "res") for o in outs])
    ws, k1 = _ptrs([_packed(w) for w, _, _ in parts])
    ss, k2 = _ptrs([_desc(sc, "scales") for _, sc, _ in parts])
    bs, k3 = _ptrs([_desc(b, "biases") for _, _, b in parts])
    _check(_lib.lib().kh_quantized_matmul_multi(
        len(parts), res, _desc(x, "x"), ws, ss, bs, bool(transpose), _lib.opt(group_size),
        _lib.opt(bits), mode.encode() if mode is not None else None, _stream_handle(x, stream)))
    return outs


def gather_qmm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               rhs_indices: torch.Tensor, transpose: bool = True, group_size: int = 64, bits: int = 4,
               sorted_indices: bool = False, *, mode: str = "affine", out_dtype=None,
               out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """res[b] = x[b] @ dequantize(w[e], ...)^T with e = rhs_indices[b] over
    batch = broadcast(x.shape[:-2], rhs_indices.shape) (MoE expert dispatch)."""
    if isinstance(out_dtype, str):
        out_dtype = _NAMES[out_dtype]
    if out is None:
        batch = torch.broadcast_shapes(tuple(x.shape[:-2]), tuple(rhs_indices.shape))
        od = out_dtype or result_dtype(x.dtype, scales.dtype)
        out = torch.empty((*batch, x.shape[-2], w.shape[-2]), dtype=od, device=x.device)
    idx = rhs_indices
    idx_desc = _desc(idx, "rhs_indices", _lib.UINT32 if idx.dtype == torch.uint32 else None)
    _check(_lib.lib().kh_gather_qmm(
        _desc(out, "res"), _desc(x, "x"), _packed(w), _desc(scales, "scales"),
        _desc(biases, "biases"), idx_desc, bool(transpose), _lib.opt(group_size), _lib.opt(bits),
        mode.encode() if mode is not None else None, bool(sorted_indices), _stream_handle(x, stream)))
    return out


def quantized_gate_up(x: torch.Tensor, gate, up, group_size: int = 64, bits: int = 4, *,
                      mode: str = "affine", out_dtype=None, out: torch.Tensor | None = None,
                      stream=None) -> torch.Tensor:
    """silu(x @ gate^T) * (x @ up^T) with gate = (w, scales, biases), likewise up."""
    if isinstance(out_dtype, str):
        out_dtype = _NAMES[out_dtype]
    if out is None:
        od = out_dtype or result_dtype(x.dtype, gate[1].dtype)
        out = torch.empty((*x.shape[:-1], gate[0].shape[0]), dtype=od, device=x.device)
    _check(_lib.lib().kh_quantized_gate_up(
        _desc(out, "res"), _desc(x, "x"), _packed(gate[0]), _desc(gate[1], "scales_gate"),
        _desc(gate[2], "biases_gate"), _packed(up[0]), _desc(up[1], "scales_up"),
        _desc(up[2], "biases_up"), _lib.opt(group_size), _lib.opt(bits),
        mode.encode() if mode is not None else None, _stream_handle(x, stream)))
    return out


def _bias_out_dtype(x, sc, bias):
    y = result_dtype(x.dtype, sc.dtype)
    return y if bias is None else result_dtype(y, bias.dtype)


def linear(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
           bias: torch.Tensor | None = None, group_size: int = 64, bits: int = 4, *,
           mode: str = "affine", out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Linear::forward (crates/kiln-models/src/nn.rs:79-102): the quantized
    matmul (transpose=true) plus the optional bias, in one launch."""
    if out is None:
        out = torch.empty((*x.shape[:-1], w.shape[0]), dtype=_bias_out_dtype(x, scales, bias),
                          device=x.device)
    _check(_lib.lib().kh_linear(
        _desc(out, "res"), _desc(x, "x"), _packed(w), _desc(scales, "scales"), _desc(biases, "biases"),
        None if bias is None else ctypes.byref(_desc(bias, "bias")), _lib.opt(group_size),
        _lib.opt(bits), mode.encode() if mode is not None else None, _stream_handle(x, stream)))
    return out


def linear_multi(x: torch.Tensor, parts, group_size: int = 64, bits: int = 4, *, mode: str = "affine",
                 outs=None, stream=None):
    """[Linear::forward(x) for (w, scales, biases, bias) in parts] (q/k/v)."""
    if outs is None:
        outs = [torch.empty((*x.shape[:-1], w.shape[0]), dtype=_bias_out_dtype(x, sc, bi), device=x.device)
                for w, sc, _, bi in parts]
    res, k0 = _ptrs([_desc(o, "res") for o in outs])
    ws, k1 = _ptrs([_packed(w) for w, _, _, _ in parts])
    ss, k2 = _ptrs([_desc(sc, "scales") for _, sc, _, _ in parts])
    bs, k3 = _ptrs([_desc(b, "biases") for _, _, b, _ in parts])
    descs = [None if bi is None else _desc(bi, "bias") for _, _, _, bi in parts]
    P = ctypes.POINTER(_lib.KhArray)
    barr = (P * len(parts))(*[P() if d is None else ctypes.pointer(d) for d in descs])
    _check(_lib.lib().kh_linear_multi(
        len(parts), res, _desc(x, "x"), ws, ss, bs, barr, _lib.opt(group_size), _lib.opt(bits),
        mode.encode() if mode is not None else None, _stream_handle(x, stream)))
    return outs


def mlp_gate_up(x: torch.Tensor, gate, up, activation: int = _lib.ACT_SILU, group_size: int = 64,
                bits: int = 4, *, mode: str = "affine", out: torch.Tensor | None = None,
                stream=None) -> torch.Tensor:
    """act(gate_proj(x)) * up_proj(x) of Mlp::forward (nn.rs:284-294); gate and
    up are (w, scales, biases, bias-or-None); activation ACT_SILU or
    ACT_GELU_APPROX."""
    if out is None:
        out = torch.empty((*x.shape[:-1], gate[0].shape[0]), dtype=_bias_out_dtype(x, gate[1], gate[3]),
                          device=x.device)
    opt_b = lambda t, n: None if t is None else ctypes.byref(_desc(t, n))
    _check(_lib.lib().kh_mlp_gate_up(
        _desc(out, "res"), _desc(x, "x"), _packed(gate[0]), _desc(gate[1], "scales_gate"),
        _desc(gate[2], "biases_gate"), opt_b(gate[3], "bias_gate"), _packed(up[0]), _desc(up[1], "scales_up"),
        _desc(up[2], "biases_up"), opt_b(up[3], "bias_up"), int(activation), _lib.opt(group_size),
        _lib.opt(bits), mode.encode() if mode is not None else None, _stream_handle(x, stream)))
    return out


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               group_size: int = 64, bits: int = 4, *, mode: str = "affine", out_dtype=None,
               out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Dense [..., K] values `scale*q + bias`; dtype defaults to the scales'."""
    if isinstance(out_dtype, str):
        out_dtype = _NAMES[out_dtype]
    if out is None:
        cols = w.shape[-1] * (32 // bits) if bits in (4, 8) else w.shape[-1]
        out = torch.empty((*w.shape[:-1], cols), dtype=out_dtype or scales.dtype, device=w.device)
    _check(_lib.lib().kh_dequantize(
        _desc(out, "res"), _packed(w), _desc(scales, "scales"), _desc(biases, "biases"),
        _lib.opt(group_size), _lib.opt(bits), mode.encode() if mode is not None else None,
        _stream_handle(w, stream)))
    return out


def quantize(w: torch.Tensor, group_size: int = 64, bits: int = 4, *, mode: str = "affine",
             stream=None):
    """mlx_quantize (affine): w [..., K] -> (w_q int32-held uint32 codes
    [..., K*bits/32], scales, biases [..., K/group_size] of w's dtype)."""
    lead, K = tuple(w.shape[:-1]), w.shape[-1] if w.dim() else 0
    per = 32 // bits if bits in (4, 8) else 1
    gs = group_size if group_size else 1
    wq = torch.empty((*lead, K // per), dtype=torch.int32, device=w.device)
    scales = torch.empty((*lead, K // gs), dtype=w.dtype, device=w.device)
    biases = torch.empty_like(scales)
    _check(_lib.lib().kh_quantize(
        _desc(wq, "w_q", _lib.UINT32), _desc(scales, "scales"), _desc(biases, "biases"),
        _desc(w, "w"), _lib.opt(group_size), _lib.opt(bits),
        mode.encode() if mode is not None else None, _stream_handle(w, stream)))
    return wq, scales, biases


def take(a: torch.Tensor, indices: torch.Tensor, axis: int = 0, *,
         out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Rows of `a` at `indices` along axis 0 (the embedding-lookup form)."""
    if axis != 0:
        raise KilnError(2, f"take along axis {axis} is not supported (axis 0 only)")
    if out is None:
        out = torch.empty((*indices.shape, *a.shape[1:]), dtype=a.dtype, device=a.device)
    _check(_lib.lib().kh_take(_desc(out, "res"), _desc(a, "a"), _desc(indices, "indices"),
                              _stream_handle(a, stream)))
    return out


def add(a: torch.Tensor, b: torch.Tensor, *, out: torch.Tensor | None = None,
        stream=None) -> torch.Tensor:
    """a + b with numpy broadcasting (ops::add; Linear's bias add,
    crates/kiln-models/src/nn.rs:98-100)."""
    if out is None:
        out = torch.empty(torch.broadcast_shapes(a.shape, b.shape), dtype=result_dtype(a.dtype, b.dtype),
                          device=a.device)
    _check(_lib.lib().kh_add(_desc(out, "res"), _desc(a, "a"), _desc(b, "b"),
                             _stream_handle(a, stream)))
    return out


def quantized_embedding(ids: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                        biases: torch.Tensor, group_size: int = 64, bits: int = 4, *,
                        mode: str = "affine", out_dtype=None, out: torch.Tensor | None = None,
                        stream=None) -> torch.Tensor:
    """dequantize(take(w, ids), take(scales, ids), take(biases, ids)) in one pass."""
    if isinstance(out_dtype, str):
        out_dtype = _NAMES[out_dtype]
    if out is None:
        cols = w.shape[-1] * (32 // bits) if bits in (4, 8) else w.shape[-1]
        out = torch.empty((*ids.shape, cols), dtype=out_dtype or scales.dtype, device=w.device)
    _check(_lib.lib().kh_quantized_embedding(
        _desc(out, "res"), _desc(ids, "ids"), _packed(w), _desc(scales, "scales"),
        _desc(biases, "biases"), _lib.opt(group_size), _lib.opt(bits),
        mode.encode() if mode is not None else None, _stream_handle(w, stream)))
    return out


def quantized_matmul_plan(M: int, N: int, K: int, group_size: int = 64, bits: int = 4,
                          x_dtype: torch.dtype = torch.bfloat16,
                          scales_dtype: torch.dtype = torch.float16) -> str:
    """Name of the kernel plan quantized_matmul runs for a transpose=true call
    of this shape (diagnostics; needs no GPU)."""
    buf = ctypes.create_string_buffer(96)
    _check(_lib.lib().kh_quantized_matmul_plan(M, N, K, group_size, bits, _TORCH_TO_KH[x_dtype],
                                                _TORCH_TO_KH[scales_dtype], buf, len(buf)))
    return buf.value.decode()
