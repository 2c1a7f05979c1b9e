"""CPU oracle for the affine-quantized linear path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, and only as the checker (or the timed CPU baseline); the product path
never imports it.

Two restatements live here:
  * the C oracle (oracle/kh_oracle.c, built by oracle/Makefile into
    oracle/_build/libkh_oracle.so), bound with ctypes: bit-exact unpack,
    dequantize, take and embedding, and a float32-accumulating
    quantized_matmul (the CPU baseline);
  * numpy functions written independently of the C code (vectorised shifts
    and masks, float64 matmul) that the tests use to cross-check it.

Reference semantics followed (paths relative to the reference repo):
  crates/kiln-mlx/src/ops.rs:359-388   quantized_matmul(x, w, scales, biases,
                                       transpose, group_size, bits), mode affine
  crates/kiln-mlx/src/ops.rs:456-484   dequantize, output dtype left unset
  crates/kiln-mlx/src/ops.rs:249-254   take(a, indices, axis)
  crates/kiln-models/src/nn.rs:159-176 Embedding::lookup = take x3 + dequantize
  crates/kiln-models/src/config.rs:137-148 bits in {4,8}, group_size in {32,64,128}
  crates/kiln-models/src/nn.rs:284-294 gated MLP input silu(gate(x)) * up(x)
  crates/kiln-jobs/src/quantize.rs:72-91 checkpoint conversion (mlx_lm
                                       convert -> MLX's affine quantize), restated
                                       as quantize / np_quantize; pinned by known
                                       answers and round-trip bounds, while
                                       bit-level agreement with MLX itself is
                                       "parity unpinned" (MLX is not importable)

Arrays: numpy containers; bf16 and f16 values travel as uint16 bit patterns
with an explicit dtype string ('bf16' | 'f16' | 'f32').
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libkh_oracle.so")

DT = {"f16": 9, "f32": 10, "bf16": 12, "u32": 3, "i32": 7}

_lib = None


def build() -> str:
    """Compile the C oracle (make -C oracle)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, ci = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.kho_unpack.argtypes = [vp, i64, i64, ci, vp]
        L.kho_pack.argtypes = [vp, i64, i64, ci, vp]
        L.kho_dequantize.argtypes = [vp, vp, vp, ci, i64, i64, ci, ci, vp, ci]
        L.kho_qmm_f32.argtypes = [vp, ci, vp, vp, vp, ci, i64, i64, i64, ci, ci, ci, vp]
        L.kho_qmm.argtypes = [vp, ci, vp, vp, vp, ci, i64, i64, i64, ci, ci, ci, vp, ci]
        L.kho_take.argtypes = [vp, i64, i64, vp, ci, i64, vp]
        L.kho_embedding.argtypes = [vp, ci, i64, vp, vp, vp, ci, i64, i64, ci, ci, vp, ci]
        L.kho_quantize.argtypes = [vp, ci, i64, i64, ci, ci, vp, vp, vp]
        L.kho_f32_to_bf16.argtypes = [ctypes.c_float]
        L.kho_f32_to_bf16.restype = ctypes.c_uint16
        L.kho_f32_to_f16.argtypes = [ctypes.c_float]
        L.kho_f32_to_f16.restype = ctypes.c_uint16
        L.kho_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.kho_bf16_to_f32.restype = ctypes.c_float
        L.kho_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.kho_f16_to_f32.restype = ctypes.c_float
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _out(shape, dt):
    return np.empty(shape, dtype=np.float32 if dt == "f32" else np.uint16)


# ----------------------------------------------------------------------------
# dtype helpers (numpy, independent of the C code)
# ----------------------------------------------------------------------------

def to_f32(a: np.ndarray, dt: str) -> np.ndarray:
    """Decode bf16/f16 bit patterns (uint16) or f32 values to float32."""
    if dt == "f32":
        return np.asarray(a, dtype=np.float32)
    if dt == "f16":
        return np.asarray(a, dtype=np.uint16).view(np.float16).astype(np.float32)
    if dt == "bf16":
        return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
    raise ValueError(dt)


def from_f32(a: np.ndarray, dt: str) -> np.ndarray:
    """Round float32 to dt (round-to-nearest-even), returned as stored bits."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    if dt == "f32":
        return a
    if dt == "f16":
        return a.astype(np.float16).view(np.uint16)
    if dt == "bf16":
        u = a.view(np.uint32).astype(np.uint64)
        nan = (u & 0x7FFFFFFF) > 0x7F800000
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
        return r
    raise ValueError(dt)


# ----------------------------------------------------------------------------
# numpy restatement (independent of kh_oracle.c)
# ----------------------------------------------------------------------------

def np_unpack(w: np.ndarray, bits: int) -> np.ndarray:
    """codes [rows, K] from packed uint32 [rows, K*bits/32]; lowest bits first."""
    per = 32 // bits
    w = np.asarray(w, dtype=np.uint32)
    shifts = (np.arange(per, dtype=np.uint32) * bits)
    codes = (w[..., None] >> shifts) & np.uint32((1 << bits) - 1)
    return codes.reshape(*w.shape[:-1], w.shape[-1] * per).astype(np.uint8)


def np_pack(codes: np.ndarray, bits: int) -> np.ndarray:
    per = 32 // bits
    c = np.asarray(codes, dtype=np.uint32).reshape(*codes.shape[:-1], codes.shape[-1] // per, per)
    shifts = (np.arange(per, dtype=np.uint32) * bits)
    return np.bitwise_or.reduce(c << shifts, axis=-1).astype(np.uint32)


def np_dequantize_f64(w, s, b, sdt, gs, bits) -> np.ndarray:
    """Exact real value of scale*q + bias in float64 (exact for f16/bf16
    scales: an 11-bit scale times an 8-bit code fits float64 without
    rounding, and so does the sum with an f16/bf16 bias)."""
    q = np_unpack(w, bits).astype(np.float64)
    sf = np.repeat(to_f32(s, sdt).astype(np.float64), gs, axis=-1)
    bf = np.repeat(to_f32(b, sdt).astype(np.float64), gs, axis=-1)
    return sf * q + bf


def np_qmm_f64(x, xdt, w, s, b, sdt, gs, bits, transpose=True) -> np.ndarray:
    """float64 reference of quantized_matmul (before output rounding)."""
    W = np_dequantize_f64(w, s, b, sdt, gs, bits).astype(np.float32).astype(np.float64)
    xf = to_f32(x, xdt).astype(np.float64)
    K = xf.shape[-1]
    x2 = xf.reshape(-1, K)
    y = x2 @ (W.T if transpose else W)
    return y.reshape(*xf.shape[:-1], y.shape[-1])


# ----------------------------------------------------------------------------
# C oracle bindings
# ----------------------------------------------------------------------------

def unpack(w: np.ndarray, bits: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint32)
    rows = int(np.prod(w.shape[:-1])) if w.ndim > 1 else 1
    K = w.shape[-1] * 32 // bits
    out = np.empty((*w.shape[:-1], K), dtype=np.uint8)
    lib().kho_unpack(_p(w), rows, K, bits, _p(out))
    return out


def pack(codes: np.ndarray, bits: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    rows = int(np.prod(codes.shape[:-1])) if codes.ndim > 1 else 1
    K = codes.shape[-1]
    out = np.empty((*codes.shape[:-1], K * bits // 32), dtype=np.uint32)
    lib().kho_pack(_p(codes), rows, K, bits, _p(out))
    return out


def dequantize(w, s, b, sdt, gs, bits, odt=None) -> np.ndarray:
    odt = odt or sdt
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s = np.ascontiguousarray(s)
    b = np.ascontiguousarray(b)
    K = w.shape[-1] * 32 // bits
    rows = int(np.prod(w.shape[:-1])) if w.ndim > 1 else 1
    out = _out((*w.shape[:-1], K), odt)
    lib().kho_dequantize(_p(w), _p(s), _p(b), DT[sdt], rows, K, gs, bits, _p(out), DT[odt])
    return out


def quantized_matmul_f32(x, xdt, w, s, b, sdt, gs, bits, transpose=True) -> np.ndarray:
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    K = x.shape[-1]
    M = int(np.prod(x.shape[:-1])) if x.ndim > 1 else 1
    N = w.shape[0] if transpose else w.shape[1] * 32 // bits
    y = np.empty((*x.shape[:-1], N), dtype=np.float32)
    lib().kho_qmm_f32(_p(x), DT[xdt], _p(w), _p(np.ascontiguousarray(s)),
                      _p(np.ascontiguousarray(b)), DT[sdt], M, N, K, gs, bits,
                      1 if transpose else 0, _p(y))
    return y


def quantized_matmul(x, xdt, w, s, b, sdt, gs, bits, transpose=True, odt="bf16"):
    return from_f32(quantized_matmul_f32(x, xdt, w, s, b, sdt, gs, bits, transpose), odt)


def take(a: np.ndarray, ids: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    ids = np.ascontiguousarray(ids)
    idt = "i32" if ids.dtype == np.int32 else "u32"
    ids_c = ids.astype(np.int32 if idt == "i32" else np.uint32)
    out = np.empty((*ids.shape, *a.shape[1:]), dtype=a.dtype)
    row_bytes = a.dtype.itemsize * int(np.prod(a.shape[1:]))
    lib().kho_take(_p(a), a.shape[0], row_bytes, _p(ids_c), DT[idt], ids.size, _p(out))
    return out


def embedding(ids, w, s, b, sdt, gs, bits, odt=None) -> np.ndarray:
    odt = odt or sdt
    ids = np.ascontiguousarray(ids)
    idt = "i32" if ids.dtype == np.int32 else "u32"
    ids_c = ids.astype(np.int32 if idt == "i32" else np.uint32)
    V = w.shape[0]
    H = w.shape[1] * 32 // bits
    out = _out((*ids.shape, H), odt)
    lib().kho_embedding(_p(ids_c), DT[idt], ids.size, _p(np.ascontiguousarray(w, dtype=np.uint32)),
                        _p(np.ascontiguousarray(s)), _p(np.ascontiguousarray(b)), DT[sdt], V, H,
                        gs, bits, _p(out), DT[odt])
    return out


def quantize(w: np.ndarray, wdt: str, gs: int, bits: int):
    """Affine quantization of w [..., K] (stored bits of dtype wdt, or float32
    values for "f32") -> (wq uint32 [..., K*bits/32], scales, biases [...,
    K/gs] as stored bits of wdt). MLX v0.31.1's affine rule, restated in
    oracle/kh_oracle.c (kho_quantize)."""
    w = np.ascontiguousarray(w)
    K = w.shape[-1]
    rows = int(np.prod(w.shape[:-1])) if w.ndim > 1 else 1
    wq = np.empty(w.shape[:-1] + (K * bits // 32,), dtype=np.uint32)
    s = _out(w.shape[:-1] + (K // gs,), wdt)
    b = _out(w.shape[:-1] + (K // gs,), wdt)
    lib().kho_quantize(_p(w), DT[wdt], rows, K, gs, bits, _p(wq), _p(s), _p(b))
    return wq, s, b


def np_quantize(w: np.ndarray, wdt: str, gs: int, bits: int):
    """numpy restatement of quantize (float32 arithmetic, round half away
    from zero evaluated in float64, where x + 0.5 is exact)."""
    v = to_f32(w, wdt).reshape(-1, gs)
    nb = np.float32((1 << bits) - 1)
    lo, hi = v.min(axis=1), v.max(axis=1)
    sc = np.maximum((hi - lo) / nb, np.float32(1e-7)).astype(np.float32)
    side = np.abs(lo) > np.abs(hi)
    sc = np.where(side, sc, -sc).astype(np.float32)
    edge = np.where(side, lo, hi).astype(np.float32)

    def rnd(x):
        x = np.asarray(x, dtype=np.float32).astype(np.float64)
        return (np.sign(x) * np.floor(np.abs(x) + 0.5)).astype(np.float32)

    q0 = rnd(edge / sc)
    nz = q0 != 0
    sc = np.where(nz, (edge / np.where(nz, q0, 1)).astype(np.float32), sc).astype(np.float32)
    bi = np.where(nz, edge, np.float32(0)).astype(np.float32)
    codes = np.clip(rnd((v - bi[:, None]) / sc[:, None]), 0, nb).astype(np.uint8)
    shape = w.shape
    wq = np_pack(codes.reshape(shape), bits)
    gshape = shape[:-1] + (shape[-1] // gs,)
    return wq, from_f32(sc.reshape(gshape), wdt), from_f32(bi.reshape(gshape), wdt)


def result_dtype(xdt: str, sdt: str) -> str:
    """MLX promotion of (x, scales, biases): equal float types stay, mixing
    bf16 with f16 or anything with f32 gives f32."""
    return xdt if xdt == sdt else "f32"


def silu_mul(g: np.ndarray, u: np.ndarray, dt: str) -> np.ndarray:
    """silu(gate) * up as the gated MLP forms it (crates/kiln-models/src/
    nn.rs:284-294: multiply(gate, sigmoid(gate)), then multiply by up), each
    op's result an array of dtype dt: g and u (stored values of dt) ->
    sigmoid evaluated in float32 and rounded to dt -> gate*sigmoid rounded ->
    times up, rounded. Returns stored values of dt."""
    gf, uf = to_f32(g, dt), to_f32(u, dt)
    with np.errstate(over="ignore"):
        sg = to_f32(from_f32(np.float32(1) / (np.float32(1) + np.exp(-gf)), dt), dt)
    a = to_f32(from_f32(gf * sg, dt), dt)
    return from_f32(a * uf, dt)


def gelu_mul(g: np.ndarray, u: np.ndarray, dt: str) -> np.ndarray:
    """gelu_approx(gate) * up as Kiln's gemma MLP forms it (crates/kiln-
    models/src/nn.rs:221-235 and 284-294), each op's result an array of
    dtype dt (weak scalars converted to dt first), every op evaluated in
    float32: cube = (g*g)*g; inner = g + c1*cube; scaled = c2*inner;
    gate = 1 + tanh(scaled); act = (0.5*g)*gate; result act*up. Returns
    stored values of dt."""
    f32 = np.float32
    r = lambda v: to_f32(from_f32(np.asarray(v, dtype=f32), dt), dt)
    gf, uf = to_f32(g, dt), to_f32(u, dt)
    c1, c2 = r(f32(0.044715)), r(f32(np.sqrt(2.0 / np.pi)))
    with np.errstate(over="ignore", invalid="ignore"):
        cube = r((gf * gf) * gf)
        inner = r(gf + r(c1 * cube))
        scaled = r(c2 * inner)
        gate = r(f32(1) + r(np.tanh(scaled)))
        act = r(r(f32(0.5) * gf) * gate)
    return from_f32(act * uf, dt)


def linear(x, xdt, w, s, b, sdt, gs, bits, bias=None, bdt=None, odt=None):
    """Linear::forward (nn.rs:79-102): the quantized matmul as an array of
    MLX's result dtype for (x, scales), then + bias (the sum of the rounded
    product and the bias formed in float32, rounded to the sum's dtype).
    Returns (stored values, dtype)."""
    ydt = result_dtype(xdt, sdt)
    y = quantized_matmul(x, xdt, w, s, b, sdt, gs, bits, True, ydt)
    if bias is None:
        return y, ydt
    rdt = odt or (ydt if ydt == bdt else "f32")
    return from_f32(to_f32(y, ydt) + to_f32(bias, bdt)[None, :], rdt), rdt
