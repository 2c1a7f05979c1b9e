"""kh_quantized_matmul_noalloc: the allocation-free variant of
kh_quantized_matmul (kernel scratch in a static per-GPU device array) gives
the same bits as kh_quantized_matmul, called through the C ABI, on two calls
in a row, the second with a smaller input, for plans that use the scratch
(the prefill GEMM with and without split-K, and the K % 128 != 0 GEMM) and
one that does not (the decode GEMV). Oversized calls are rejected before
anything is launched."""
import ctypes

import numpy as np
import pytest
import torch

from kiln_amd import _lib, ops
from kiln_amd.workloads import make_linear_device

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L = _lib.lib()
    L.kh_quantized_matmul_noalloc.argtypes = L.kh_quantized_matmul.argtypes
    L.kh_quantized_matmul_noalloc.restype = ctypes.c_int
    L.kh_noalloc_scratch_bytes.restype = ctypes.c_size_t


def _noalloc(x, L, gs, bits, out):
    lib = _lib.lib()
    st = torch.cuda.current_stream().cuda_stream
    rc = lib.kh_quantized_matmul_noalloc(
        ctypes.byref(ops._desc(out, "res")), ctypes.byref(ops._desc(x, "x")),
        ctypes.byref(ops._packed(L["w"])), ctypes.byref(ops._desc(L["scales"], "scales")),
        ctypes.byref(ops._desc(L["biases"], "biases")), True, _lib.opt(gs), _lib.opt(bits), b"affine",
        ctypes.c_void_p(st))
    return rc


# (N, K, gs, bits, M first, M second)
CASES = [(4096, 4096, 64, 4, 512, 200),     # GEMM, split-K 4 then split-K at a smaller tile class
         (14336, 4096, 64, 4, 2048, 64),    # GEMM without split-K, then with
         (1024, 4096, 64, 4, 96, 40),       # GEMM split-K
         (512, 3584, 32, 8, 300, 33),       # 8-bit gs32 GEMM
         (256, 1344, 64, 4, 100, 20),       # K % 128 != 0: qmm kernel (scratch) then qmv
         (8192, 2048, 64, 4, 4, 1)]         # decode GEMV (no scratch)


@pytest.mark.parametrize("N,K,gs,bits,M1,M2", CASES)
def test_noalloc_matches_quantized_matmul(N, K, gs, bits, M1, M2):
    print(f"case noalloc N={N} K={K} gs={gs} bits={bits} M={M1},{M2}", flush=True)
    L = make_linear_device(N, K, gs, "q4" if bits == 4 else "q8", seed=N + K)
    g = torch.Generator(device="cuda").manual_seed(M1)
    for M in (M1, M2):
        x = torch.randn((M, K), device="cuda", generator=g).bfloat16()
        ref = ops.quantized_matmul(x, L["w"], L["scales"], L["biases"], True, gs, bits, out_dtype=torch.bfloat16)
        out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        assert _noalloc(x, L, gs, bits, out) == 0, _lib.last_error()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), (M, ops.quantized_matmul_plan(M, N, K, gs, bits))


def test_noalloc_rejects_oversized_call():
    lib = _lib.lib()
    cap = lib.kh_noalloc_scratch_bytes()
    assert cap == 64 << 20
    N, K, M = 256, 16384, 4096  # M*K*2 = 128 MiB of float16 activations
    assert M * K * 2 > cap
    L = make_linear_device(N, K, 64, "q4", seed=1)
    x = torch.zeros((M, K), device="cuda", dtype=torch.bfloat16)
    out = torch.full((M, N), 7.0, dtype=torch.bfloat16, device="cuda")
    rc = _noalloc(x, L, 64, 4, out)
    assert rc == 2, rc  # KH_ERR_UNSUPPORTED
    assert "scratch" in _lib.last_error()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())  # nothing was launched
