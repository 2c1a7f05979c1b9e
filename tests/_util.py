"""Helpers shared by the GPU tests: numpy bit patterns <-> device tensors and
the parity metrics."""
import numpy as np
import torch

TORCH_DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def dev(a: np.ndarray, dt: str | None = None) -> torch.Tensor:
    """numpy -> cuda tensor; uint16 arrays are reinterpreted as dt (bf16/f16),
    uint32 as int32 bits."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).view(TORCH_DT[dt]).cuda()
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).cuda()
    return torch.from_numpy(a).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    """cuda tensor -> numpy bit patterns (uint16 for 16-bit floats)."""
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.int32:
        return t.numpy().view(np.uint32)
    return t.numpy()


def parity_metrics(y: np.ndarray, ref: np.ndarray):
    """(max|err| / max|ref|, mean|err| / mean|ref|) — the matmul tolerance:
    max|err| <= 2e-2 * max|ref| and mean relative error <= 1e-3, with both
    arrays as float64 values of the same output dtype."""
    y = y.astype(np.float64)
    ref = ref.astype(np.float64)
    err = np.abs(y - ref)
    return float(err.max() / max(np.abs(ref).max(), 1e-30)), float(err.mean() / max(np.abs(ref).mean(), 1e-30))


def gemv_max_m(K: int, bits: int) -> int:
    """Largest M the VALU decode GEMV serves for rows of K codes: each lane
    slot of a workgroup of at most 8 waves owns I 16-byte chunks per row, and
    M*I activation chunks must fit in registers (kh_gemv.hip, plan_gemv)."""
    nch = K * bits // 128
    I = 1
    while -(-nch // (64 * I)) > 8:
        I += 1
    return 8 if I == 1 else 2 if I == 2 else 1 if I <= 4 else 0


def decode_regime(M: int, K: int, bits: int, N: int, gs: int = 64):
    """Which kernel (and tiling class) kh_quantized_matmul uses for a
    transpose=true call with bf16 x and f16 scales, as the library's own plan
    names it (kh_quantized_matmul_plan, no GPU needed): rows of the result
    are bitwise identical for every M of one regime (kiln_hip.hip, run_qmm).
    The GEMM's class is its m-tile, and for 128-row tiles the number of
    row tiles (the split-K plan depends on them)."""
    from kiln_amd import ops
    plan = ops.quantized_matmul_plan(M, N, K, gs, bits)
    kind = plan.split()[0]
    if kind == "gemm":
        mt = int(dict(kv.split("=") for kv in plan.split()[1:])["mt"])
        return ("gemm", mt, -(-M // 128) if mt == 8 else 1)
    if kind == "qmm":
        return ("qmm", -(-M // 256))
    return (kind,)


def exact_weights(M: int, K: int, bits: int, N: int, gs: int = 64) -> bool:
    """True where every dequantised weight enters the products unrounded
    (the decode GEMV, the skinny MFMA kernel and qmv); the GEMM kernels round
    each weight once to fp16."""
    r = decode_regime(M, K, bits, N, gs)[0]
    return r in ("gemv", "skinny", "qmv")
