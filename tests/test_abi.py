"""C-ABI tests that need no GPU: the library loads, exports every symbol the
header declares, and rejects bad arguments with a status and a message
instead of aborting (the contract of crates/kiln-mlx/src/error.rs:24-72,
tested in the reference by crates/kiln-mlx/tests/wrappers.rs:163-182)."""
import ctypes
import os
import re
import subprocess

import pytest

from kiln_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAKE = 0x10000  # never dereferenced: validation fails before any device access


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "kiln_hip.h")).read()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(kh_\w+)\s*\(", text, re.M)))


def test_header_declares_exports():
    assert set(_declared_symbols()) == set(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for name in _declared_symbols():
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (kh_\w+)", out))
    assert set(_declared_symbols()) <= exported
    assert _lib.lib().kh_version().decode().startswith("kiln-hip")


def A(dtype, shape, ptr=FAKE):
    return _lib.array(ptr, dtype, shape)


def qmm(res, x, w, s, b, transpose=True, gs=64, bits=4, mode=b"affine"):
    return _lib.lib().kh_quantized_matmul(ctypes.byref(res), ctypes.byref(x), ctypes.byref(w),
                                          ctypes.byref(s), ctypes.byref(b), transpose,
                                          _lib.opt(gs), _lib.opt(bits), mode, None)


def good(M=1, N=32, K=128, gs=64, bits=4):
    return (A(_lib.BFLOAT16, (M, N)), A(_lib.BFLOAT16, (M, K)),
            A(_lib.UINT32, (N, K * bits // 32)), A(_lib.FLOAT16, (N, K // gs)),
            A(_lib.FLOAT16, (N, K // gs)))


@pytest.mark.parametrize("kw,needle", [
    (dict(bits=3), "bits=3"),
    (dict(gs=48), "group_size=48"),
    (dict(mode=b"mxfp4"), "mode"),
])
def test_quant_domain_rejected(kw, needle):
    args = good()
    rc = qmm(*args, **kw)
    assert rc == 1
    assert needle in _lib.last_error()


def test_shape_errors_report_shapes():
    res, x, w, s, b = good()
    x_bad = A(_lib.BFLOAT16, (1, 96))
    assert qmm(res, x_bad, w, s, b) == 1
    assert "96" in _lib.last_error()
    res_bad = A(_lib.BFLOAT16, (1, 31))
    assert qmm(res_bad, x, w, s, b) == 1
    assert "expected (1,32)" in _lib.last_error()
    s_bad = A(_lib.FLOAT16, (32, 3))
    assert qmm(res, x, w, s_bad, s_bad) == 1


def test_dtype_errors():
    res, x, w, s, b = good()
    assert qmm(res, x, A(_lib.INT32, (32, 16)), s, b) == 1
    assert "uint32" in _lib.last_error()
    assert qmm(res, x, w, s, A(_lib.BFLOAT16, (32, 2))) == 1
    assert "share a dtype" in _lib.last_error()
    assert qmm(A(_lib.INT32, (1, 32)), x, w, s, b) == 1
    assert qmm(res, A(_lib.INT32, (1, 128)), w, s, b) == 1


def test_null_data_rejected():
    res, x, w, s, b = good()
    assert qmm(res, A(_lib.BFLOAT16, (1, 128), 0), w, s, b) == 1
    assert "NULL" in _lib.last_error()


def test_transpose_false_shapes():
    K, N = 64, 128
    res = A(_lib.FLOAT32, (2, N))
    x = A(_lib.BFLOAT16, (2, K))
    w = A(_lib.UINT32, (K, N // 8))
    s = A(_lib.FLOAT16, (K, N // 64))
    rc = qmm(res, x, w, s, s, transpose=False)
    assert rc in (0, 4)  # valid: reaches the device check (none here)


def test_valid_call_without_gpu_reports_no_device():
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        pytest.skip("a GPU is present")
    rc = qmm(*good())
    assert rc == 4
    assert _lib.last_error()


def test_dequantize_and_embedding_validation():
    L = _lib.lib()
    w = A(_lib.UINT32, (10, 16))
    s = A(_lib.FLOAT16, (10, 2))
    res = A(_lib.BFLOAT16, (10, 127))
    assert L.kh_dequantize(ctypes.byref(res), ctypes.byref(w), ctypes.byref(s), ctypes.byref(s),
                           _lib.opt(64), _lib.opt(4), None, None) == 1
    ids = A(_lib.INT64, (3,))
    res2 = A(_lib.BFLOAT16, (3, 128))
    assert L.kh_quantized_embedding(ctypes.byref(res2), ctypes.byref(ids), ctypes.byref(w),
                                    ctypes.byref(s), ctypes.byref(s), _lib.opt(64), _lib.opt(4),
                                    None, None) == 1
    assert "ids must be" in _lib.last_error()


def test_take_validation():
    L = _lib.lib()
    a = A(_lib.FLOAT16, (10, 4))
    ids = A(_lib.UINT32, (2, 3))
    res = A(_lib.FLOAT16, (2, 3, 5))
    assert L.kh_take(ctypes.byref(res), ctypes.byref(a), ctypes.byref(ids), None) == 1
    assert "expected (2,3,4)" in _lib.last_error()


def test_errors_are_thread_local():
    import threading
    args = good()
    assert qmm(*args, bits=3) == 1
    seen = []

    def other():
        seen.append(_lib.last_error())

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen == [""]
    assert "bits=3" in _lib.last_error()


def _pp(arrs):
    P = ctypes.POINTER(_lib.KhArray)
    return (P * len(arrs))(*[ctypes.pointer(a) for a in arrs])


def test_fused_entry_points_validation():
    L = _lib.lib()
    res, x, w, s, b = good(M=2, N=32, K=128)
    res2, _, w2, s2, b2 = good(M=2, N=16, K=128)
    # n out of range / null part arrays
    rc = L.kh_quantized_matmul_multi(0, _pp([res]), ctypes.byref(x), _pp([w]), _pp([s]), _pp([b]),
                                     True, _lib.opt(64), _lib.opt(4), b"affine", None)
    assert rc == 1 and "quantized_matmul_multi" in _lib.last_error()
    # a bad part is reported with its shapes
    bad_w = A(_lib.UINT32, (16, 8))  # K*bits/32 = 16 expected
    rc = L.kh_quantized_matmul_multi(2, _pp([res, res2]), ctypes.byref(x), _pp([w, bad_w]),
                                     _pp([s, s2]), _pp([b, b2]), True, _lib.opt(64), _lib.opt(4),
                                     b"affine", None)
    assert rc == 1 and "quantized_matmul_multi" in _lib.last_error()
    # gate/up of different N cannot share one result
    rc = L.kh_quantized_gate_up(ctypes.byref(res), ctypes.byref(x), ctypes.byref(w), ctypes.byref(s),
                                ctypes.byref(b), ctypes.byref(w2), ctypes.byref(s2), ctypes.byref(b2),
                                _lib.opt(64), _lib.opt(4), b"affine", None)
    assert rc == 1 and "quantized_gate_up" in _lib.last_error()


def test_fused_entry_points_without_gpu_report_no_device():
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        pytest.skip("a GPU is present")
    L = _lib.lib()
    res, x, w, s, b = good(M=2, N=32, K=128)
    rc = L.kh_quantized_matmul_multi(2, _pp([res, res]), ctypes.byref(x), _pp([w, w]), _pp([s, s]),
                                     _pp([b, b]), True, _lib.opt(64), _lib.opt(4), b"affine", None)
    assert rc == 4
    rc = L.kh_quantized_gate_up(ctypes.byref(res), ctypes.byref(x), ctypes.byref(w), ctypes.byref(s),
                                ctypes.byref(b), ctypes.byref(w), ctypes.byref(s), ctypes.byref(b),
                                _lib.opt(64), _lib.opt(4), b"affine", None)
    assert rc == 4


def test_gather_qmm_validation():
    L = _lib.lib()
    E, N, K = 4, 32, 128

    def call(res, x, w, s, b, idx, transpose=True):
        return L.kh_gather_qmm(ctypes.byref(res), ctypes.byref(x), ctypes.byref(w), ctypes.byref(s),
                               ctypes.byref(b), ctypes.byref(idx), transpose, _lib.opt(64), _lib.opt(4),
                               b"affine", False, None)
    w = A(_lib.UINT32, (E, N, K // 8))
    s = A(_lib.FLOAT16, (E, N, K // 64))
    x = A(_lib.BFLOAT16, (5, 1, 1, K))
    idx = A(_lib.UINT32, (5, 3))
    res = A(_lib.BFLOAT16, (5, 3, 1, N))
    # 2-D weights are not an expert stack
    assert call(res, x, A(_lib.UINT32, (N, K // 8)), A(_lib.FLOAT16, (N, 2)), A(_lib.FLOAT16, (N, 2)), idx) == 1
    assert "expert stack" in _lib.last_error()
    # float indices rejected
    assert call(res, x, w, s, s, A(_lib.FLOAT32, (5, 3))) == 1 and "rhs_indices" in _lib.last_error()
    # batch dims that do not broadcast
    assert call(res, x, w, s, s, A(_lib.UINT32, (4, 3))) == 1 and "broadcast" in _lib.last_error()
    # the result must have the broadcast batch shape
    assert call(A(_lib.BFLOAT16, (5, 1, N)), x, w, s, s, idx) == 1 and "res" in _lib.last_error()
    assert call(res, x, w, s, s, idx, transpose=False) == 2


def test_gather_qmm_without_gpu_reports_no_device():
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        pytest.skip("a GPU is present")
    L = _lib.lib()
    w = A(_lib.UINT32, (4, 32, 16))
    s = A(_lib.FLOAT16, (4, 32, 2))
    rc = L.kh_gather_qmm(ctypes.byref(A(_lib.BFLOAT16, (6, 1, 32))), ctypes.byref(A(_lib.BFLOAT16, (6, 1, 128))),
                         ctypes.byref(w), ctypes.byref(s), ctypes.byref(s),
                         ctypes.byref(A(_lib.INT32, (6,))), True, _lib.opt(64), _lib.opt(4), b"affine",
                         True, None)
    assert rc == 4


def _quantize(wq, s, b, w, gs=64, bits=4, mode=b"affine"):
    return _lib.lib().kh_quantize(ctypes.byref(wq), ctypes.byref(s), ctypes.byref(b),
                                  ctypes.byref(w), _lib.opt(gs), _lib.opt(bits), mode, None)


def test_quantize_validation():
    w = A(_lib.BFLOAT16, (6, 256))
    good = (A(_lib.UINT32, (6, 32)), A(_lib.BFLOAT16, (6, 4)), A(_lib.BFLOAT16, (6, 4)), w)
    # K not a multiple of the group size
    assert _quantize(A(_lib.UINT32, (6, 12)), A(_lib.BFLOAT16, (6, 1)), A(_lib.BFLOAT16, (6, 1)),
                     A(_lib.BFLOAT16, (6, 96)), gs=64) == 1
    assert "divisible by group_size" in _lib.last_error()
    # wrong packed width, wrong scale dtype, 1-d w, integer w, bad domain
    assert _quantize(A(_lib.UINT32, (6, 16)), *good[1:]) == 1
    assert "w_q is" in _lib.last_error()
    assert _quantize(good[0], A(_lib.FLOAT16, (6, 4)), good[2], w) == 1
    assert "scales is" in _lib.last_error()
    assert _quantize(A(_lib.UINT32, (32,)), A(_lib.BFLOAT16, (4,)), A(_lib.BFLOAT16, (4,)),
                     A(_lib.BFLOAT16, (256,))) == 1
    assert "ndim >= 2" in _lib.last_error()
    assert _quantize(good[0], good[1], good[2], A(_lib.UINT32, (6, 256))) == 1
    assert _quantize(*good, bits=3) == 1
    assert _quantize(*good, mode=b"mxfp4") in (1, 2)


def test_quantize_without_gpu_reports_no_device():
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        pytest.skip("a GPU is present")
    w = A(_lib.FLOAT32, (2, 3, 128))
    assert _quantize(A(_lib.UINT32, (2, 3, 32)), A(_lib.FLOAT32, (2, 3, 1)),
                     A(_lib.FLOAT32, (2, 3, 1)), w, gs=128, bits=8) == 4
    # empty inputs succeed without touching the device
    assert _quantize(A(_lib.UINT32, (0, 16)), A(_lib.FLOAT32, (0, 2)), A(_lib.FLOAT32, (0, 2)),
                     A(_lib.FLOAT32, (0, 128))) == 0


def _linear(res, x, w, s, b, bias, gs=64, bits=4):
    return _lib.lib().kh_linear(ctypes.byref(res), ctypes.byref(x), ctypes.byref(w), ctypes.byref(s),
                                ctypes.byref(b), None if bias is None else ctypes.byref(bias),
                                _lib.opt(gs), _lib.opt(bits), b"affine", None)


def test_linear_bias_validation():
    """kh_linear (Linear::forward, nn.rs:79-102): the bias is a float [N]
    vector and res has the dtype of product + bias (MLX promotion)."""
    res, x, w, s, b = good()          # bf16 x, f16 scales: the product is float32
    res32 = A(_lib.FLOAT32, (1, 32))
    assert _linear(res32, x, w, s, b, A(_lib.BFLOAT16, (31,))) == 1
    assert "bias has shape (31)" in _lib.last_error()
    assert _linear(res32, x, w, s, b, A(_lib.INT32, (32,))) == 1
    assert "bias must be" in _lib.last_error()
    assert _linear(res, x, w, s, b, A(_lib.BFLOAT16, (32,))) == 1   # res must be float32 here
    assert "float32" in _lib.last_error()
    xs = A(_lib.FLOAT16, (1, 128))                                    # f16 x, f16 scales: f16 product
    assert _linear(A(_lib.FLOAT16, (1, 32)), xs, w, s, b, A(_lib.FLOAT32, (32,))) == 1
    # valid calls reach the device check
    assert _linear(res32, x, w, s, b, A(_lib.BFLOAT16, (32,))) == 4
    assert _linear(A(_lib.FLOAT16, (1, 32)), xs, w, s, b, A(_lib.FLOAT16, (32,))) == 4
    assert _linear(res, x, w, s, b, None) == 4


def test_mlp_gate_up_validation():
    res, x, w, s, b = good()
    L = _lib.lib()

    def call(act, bg=None, bu=None, r=res):
        return L.kh_mlp_gate_up(ctypes.byref(r), ctypes.byref(x), ctypes.byref(w), ctypes.byref(s),
                                ctypes.byref(b), None if bg is None else ctypes.byref(bg), ctypes.byref(w),
                                ctypes.byref(s), ctypes.byref(b), None if bu is None else ctypes.byref(bu),
                                act, _lib.opt(64), _lib.opt(4), b"affine", None)
    assert call(7) == 1 and "activation 7" in _lib.last_error()
    assert call(_lib.ACT_GELU_APPROX, bu=A(_lib.FLOAT32, (33,))) == 1
    assert "bias_up" in _lib.last_error()
    assert call(_lib.ACT_GELU_APPROX) == 4
    assert call(_lib.ACT_SILU, A(_lib.FLOAT32, (32,)), A(_lib.FLOAT32, (32,)), A(_lib.FLOAT32, (1, 32))) == 4


def test_linear_multi_validation():
    res, x, w, s, b = good()
    L = _lib.lib()
    P = ctypes.POINTER(_lib.KhArray)
    arr = lambda *a: (P * len(a))(*[ctypes.pointer(v) if v is not None else P() for v in a])
    res32 = A(_lib.FLOAT32, (1, 32))
    call = lambda r, bias: L.kh_linear_multi(2, arr(r, r), ctypes.byref(x), arr(w, w), arr(s, s), arr(b, b),
                                             bias, _lib.opt(64), _lib.opt(4), b"affine", None)
    assert call(res32, arr(A(_lib.FLOAT32, (32,)), A(_lib.FLOAT32, (31,)))) == 1
    assert "(31)" in _lib.last_error()
    assert call(res32, arr(None, A(_lib.FLOAT32, (32,)))) == 4
    assert call(res, None) == 4


# Kernel choice for the benchmark's Llama-3-8B shapes (4-bit gs64, bf16 x,
# f16 scales), read from the library's own plan (host logic, no GPU): the
# decode GEMV at M = 1 and for the narrow k/v shape at M = 8, the small-batch
# MFMA kernel at M = 8..32 unless its x reads would exceed 150 MiB (down at
# M >= 22) or it would need more than three waves per SIMD (gate at M > 16),
# the GEMM above (split-K at decode sizes, the half-width tail at M = 2048).
@pytest.mark.parametrize("M,N,K,plan", [
    (1, 14336, 4096, "gemv"),
    (8, 1024, 4096, "gemv"),
    (8, 4096, 4096, "skinny"),
    (8, 14336, 4096, "skinny"),
    (21, 4096, 14336, "skinny"),
    (22, 4096, 14336, "gemm mt=2 nsplit=16 tail=0"),
    (32, 4096, 4096, "skinny"),
    (32, 14336, 4096, "gemm mt=2 nsplit=4 tail=0"),
    (64, 14336, 4096, "gemm mt=4 nsplit=4 tail=0"),
    (2048, 14336, 4096, "gemm mt=8 nsplit=1 tail=128"),
])
def test_kernel_choice_on_benchmark_shapes(M, N, K, plan):
    from kiln_amd import ops
    assert ops.quantized_matmul_plan(M, N, K, 64, 4) == plan
