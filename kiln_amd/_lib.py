"""ctypes binding of libkiln_hip.so (include/kiln_hip.h).

The library is the product: loading fails loudly when it has not been built
(`python -m kiln_amd.build`); there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkiln_hip.so")

KH_MAX_NDIM = 8

# kh_dtype values (mlx_dtype numbering)
BOOL, UINT8, UINT16, UINT32, UINT64, INT8, INT16, INT32, INT64 = range(9)
FLOAT16, FLOAT32, FLOAT64, BFLOAT16, COMPLEX64 = 9, 10, 11, 12, 13

STATUS = {0: "KH_OK", 1: "KH_ERR_INVALID_ARGUMENT", 2: "KH_ERR_UNSUPPORTED",
          3: "KH_ERR_DEVICE", 4: "KH_ERR_NO_DEVICE"}

# Every symbol include/kiln_hip.h declares.
EXPORTS = ("kh_quantized_matmul", "kh_quantized_matmul_multi", "kh_quantized_gate_up",
           "kh_gather_qmm", "kh_quantize",
           "kh_dequantize", "kh_take", "kh_quantized_embedding", "kh_add", "kh_last_error",
           "kh_version", "kh_quantized_matmul_plan", "kh_quantized_matmul_noalloc",
           "kh_noalloc_scratch_bytes", "kh_linear", "kh_linear_multi", "kh_mlp_gate_up")

# kh_activation
ACT_SILU, ACT_GELU_APPROX = 0, 1


class KhArray(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("ndim", ctypes.c_int32),
                ("shape", ctypes.c_int64 * KH_MAX_NDIM)]


class KhOptionalInt(ctypes.Structure):
    _fields_ = [("value", ctypes.c_int32), ("has_value", ctypes.c_bool)]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP library first (python -m kiln_amd.build)")
        # One HIP runtime per process: torch ships its own libamdhip64 (same
        # soname, libamdhip64.so.7) and loads it under the name
        # "libamdhip64.so". Loading torch first lets this library's
        # dependency resolve to that already-loaded copy; loading this library
        # first would pull in /opt/rocm's copy and torch would then load a
        # second runtime beside it.
        import torch  # noqa: F401

        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER(KhArray)
        L.kh_quantized_matmul.argtypes = [P, P, P, P, P, ctypes.c_bool, KhOptionalInt,
                                          KhOptionalInt, ctypes.c_char_p, ctypes.c_void_p]
        PP = ctypes.POINTER(P)
        L.kh_quantized_matmul_multi.argtypes = [ctypes.c_int, PP, P, PP, PP, PP, ctypes.c_bool,
                                                KhOptionalInt, KhOptionalInt, ctypes.c_char_p,
                                                ctypes.c_void_p]
        L.kh_gather_qmm.argtypes = [P, P, P, P, P, P, ctypes.c_bool, KhOptionalInt, KhOptionalInt,
                                    ctypes.c_char_p, ctypes.c_bool, ctypes.c_void_p]
        L.kh_quantized_gate_up.argtypes = [P, P, P, P, P, P, P, P, KhOptionalInt, KhOptionalInt,
                                           ctypes.c_char_p, ctypes.c_void_p]
        L.kh_linear.argtypes = [P, P, P, P, P, P, KhOptionalInt, KhOptionalInt, ctypes.c_char_p,
                                ctypes.c_void_p]
        L.kh_linear_multi.argtypes = [ctypes.c_int, PP, P, PP, PP, PP, PP, KhOptionalInt, KhOptionalInt,
                                      ctypes.c_char_p, ctypes.c_void_p]
        L.kh_mlp_gate_up.argtypes = [P, P, P, P, P, P, P, P, P, P, ctypes.c_int, KhOptionalInt,
                                     KhOptionalInt, ctypes.c_char_p, ctypes.c_void_p]
        L.kh_dequantize.argtypes = [P, P, P, P, KhOptionalInt, KhOptionalInt, ctypes.c_char_p,
                                    ctypes.c_void_p]
        L.kh_quantize.argtypes = [P, P, P, P, KhOptionalInt, KhOptionalInt, ctypes.c_char_p,
                                  ctypes.c_void_p]
        L.kh_take.argtypes = [P, P, P, ctypes.c_void_p]
        L.kh_add.argtypes = [P, P, P, ctypes.c_void_p]
        L.kh_quantized_embedding.argtypes = [P, P, P, P, P, KhOptionalInt, KhOptionalInt,
                                             ctypes.c_char_p, ctypes.c_void_p]
        for f in ("kh_quantized_matmul", "kh_quantized_matmul_multi", "kh_quantized_gate_up",
                  "kh_linear", "kh_linear_multi", "kh_mlp_gate_up",
                  "kh_gather_qmm", "kh_quantize",
                  "kh_dequantize", "kh_take", "kh_quantized_embedding", "kh_add"):
            getattr(L, f).restype = ctypes.c_int
        L.kh_quantized_matmul_noalloc.argtypes = L.kh_quantized_matmul.argtypes
        L.kh_quantized_matmul_noalloc.restype = ctypes.c_int
        L.kh_noalloc_scratch_bytes.restype = ctypes.c_size_t
        L.kh_quantized_matmul_plan.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                               ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_char_p, ctypes.c_size_t]
        L.kh_quantized_matmul_plan.restype = ctypes.c_int
        L.kh_last_error.restype = ctypes.c_char_p
        L.kh_version.restype = ctypes.c_char_p
        _lib = L
    return _lib


def array(data_ptr: int, dtype: int, shape) -> KhArray:
    shape = tuple(int(s) for s in shape)
    if len(shape) > KH_MAX_NDIM:
        raise ValueError(f"ndim {len(shape)} exceeds {KH_MAX_NDIM}")
    a = KhArray()
    a.data = data_ptr or None
    a.dtype = dtype
    a.ndim = len(shape)
    for i, s in enumerate(shape):
        a.shape[i] = s
    return a


def opt(v) -> KhOptionalInt:
    o = KhOptionalInt()
    if v is None:
        o.value, o.has_value = 0, False
    else:
        o.value, o.has_value = int(v), True
    return o


def last_error() -> str:
    return lib().kh_last_error().decode()
