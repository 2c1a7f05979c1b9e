"""GPU parity at the benchmark configurations' own shapes.

Every configuration the benchmark is quoted on runs here at its real (N, K)
and at every batch size M it lists, so each kernel plan the benchmark times
(GEMV rows per workgroup, skinny tiling, GEMM tile class, split-K count and
the half-width tail launch) is compared with the CPU oracle:

  cfg0  8192x2048 4-bit gs64, M = 1
  cfg1  Llama-3.2-1B linears, 4-bit gs64, M in {1, 4, 16, 32}
  cfg2  Llama-3-8B linears, 4-bit gs64, M in {1, 8, 32, 64, 512, 2048, 4096}
  cfg3  Qwen2.5-7B linears, 8-bit gs32 and gs128, M in {1, 16, 2048}
  cfg4b tied 128256x4096 head, 4-bit gs128, M in {1, 32, 256}

Weights are generated in HBM (kiln_amd.workloads.make_linear_device); the
oracle (oracle/kh_oracle.c, the restatement of ops.rs:359-388) computes a
sample of >= 256 output columns for all M rows: the first and last columns,
one column in every 256-column tile, the rest random. The sampled rows of w,
scales and biases are copied back and passed to the oracle as an [n, K]
linear, so the check costs seconds at every size.

Bars on the sampled columns: bfloat16 output within the BASELINE tolerance
(max|err| <= 2e-2 max|ref|, mean rel err <= 1e-3) and float32 output within
the elementwise bound of the kernel class (exact weights: 3e-5 sum|x||w|;
float16-rounded weights: (2^-11 + 3e-5) sum|x||w|).
"""
import functools

import numpy as np
import pytest
import torch

from kiln_amd import ops
from kiln_amd.workloads import LAYER_SHAPES, make_linear_device, make_x_numpy

from _util import dev, host, parity_metrics
from test_gpu_parity import EXACT_REL, F16W_REL, MAX_TOL, MEAN_TOL

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _cases():
    out = [("cfg0", "gemv", 8192, 2048, 64, "q4", 1)]
    for cfg, model, dist, gss, Ms in (("cfg1", "llama-3.2-1b", "q4", (64,), (1, 4, 16, 32)),
                                      ("cfg2", "llama-3-8b", "q4", (64,), (1, 8, 32, 64, 512, 2048, 4096)),
                                      ("cfg3", "qwen2.5-7b", "q8", (32, 128), (1, 16, 2048))):
        seen = set()
        for name, N, K in LAYER_SHAPES[model]:
            if (N, K) in seen:  # k/v and gate/up share shapes
                continue
            seen.add((N, K))
            for gs in gss:
                for M in Ms:
                    out.append((cfg, name, N, K, gs, dist, M))
    for M in (1, 32, 256):
        out.append(("cfg4b", "head", 128256, 4096, 128, "emb", M))
    return out


CASES = _cases()


@functools.lru_cache(maxsize=2)
def _weights(N, K, gs, dist):
    torch.manual_seed(0)
    return make_linear_device(N, K, gs, dist, seed=N * 7 + K + gs)


def _sample_cols(N, seed):
    rng = np.random.default_rng(seed)
    cols = set(range(min(8, N))) | set(range(max(0, N - 8), N))
    for t in range(0, N, 256):
        cols.add(int(rng.integers(t, min(t + 256, N))))
    while len(cols) < min(256, N):
        cols.add(int(rng.integers(0, N)))
    return np.array(sorted(cols), dtype=np.int64)


def _to_np16(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("cfg,name,N,K,gs,dist,M", CASES,
                         ids=[f"{c[0]}-{c[1]}-{c[2]}x{c[3]}-gs{c[4]}-M{c[6]}" for c in CASES])
def test_baseline_shape(oracle, cfg, name, N, K, gs, dist, M):
    bits = 8 if dist == "q8" else 4
    plan = ops.quantized_matmul_plan(M, N, K, gs, bits)
    print(f"case {cfg} {name} N={N} K={K} gs={gs} bits={bits} M={M} plan={plan}", flush=True)
    L = _weights(N, K, gs, dist)
    x = make_x_numpy(M, K, seed=M + K)
    xd = dev(x, "bf16")
    y32 = ops.quantized_matmul(xd, L["w"], L["scales"], L["biases"], True, gs, bits, out_dtype=torch.float32)
    y16 = ops.quantized_matmul(xd, L["w"], L["scales"], L["biases"], True, gs, bits, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    cols = _sample_cols(N, seed=N + M)
    ci = torch.from_numpy(cols).cuda()
    w = L["w"].index_select(0, ci).cpu().numpy().view(np.uint32)
    s = _to_np16(L["scales"].index_select(0, ci))
    b = _to_np16(L["biases"].index_select(0, ci))
    y32 = y32.index_select(1, ci).cpu().numpy()
    y16 = host(y16.index_select(1, ci).contiguous())

    ref = oracle.quantized_matmul_f32(x, "bf16", w, s, b, "f16", gs, bits)
    # BASELINE tolerance on the bfloat16 result
    mx, mean = parity_metrics(oracle.to_f32(y16, "bf16"), oracle.to_f32(oracle.from_f32(ref, "bf16"), "bf16"))
    assert mx <= MAX_TOL and mean <= MEAN_TOL, (plan, mx, mean)
    # elementwise bound on the float32 result
    W = oracle.to_f32(oracle.dequantize(w, s, b, "f16", gs, bits, "f32"), "f32")
    mag = np.abs(oracle.to_f32(x, "bf16")).astype(np.float64) @ np.abs(W.T).astype(np.float64)
    rel = F16W_REL if plan.startswith(("gemm", "qmm")) else EXACT_REL
    bad = np.abs(y32.astype(np.float64) - ref) > rel * mag + 1e-30
    assert not bad.any(), f"{plan}: {bad.sum()} elements off; first at {np.argwhere(bad)[0]}"
    # the bfloat16 result is the float32 one rounded once
    assert np.array_equal(y16, oracle.from_f32(y32, "bf16")), plan


def test_baseline_shapes_cover_every_plan_kind():
    """The cases above reach every kernel the benchmark times: the GEMV, the
    skinny kernel, the GEMM with and without split-K and with the half-width
    tail launch, in every tile class."""
    plans = {ops.quantized_matmul_plan(M, N, K, gs, 8 if d == "q8" else 4) for _, _, N, K, gs, d, M in CASES}
    kinds = {p.split()[0] for p in plans}
    assert {"gemv", "skinny", "gemm"} <= kinds, plans
    gemm = [dict(kv.split("=") for kv in p.split()[1:]) for p in plans if p.startswith("gemm")]
    assert any(int(g["nsplit"]) > 1 for g in gemm), plans
    assert any(int(g["tail"]) > 0 for g in gemm), plans
    assert {int(g["mt"]) for g in gemm} >= {2, 4, 8}, plans


# Repeated calls on one input at Qwen2.5-7B's q/o shape, in every GEMM tile
# class and split-K plan the decode and prefill sizes reach: a load that a
# kernel's waits do not cover shows up as results that change from call to
# call (an 8-bit gs128 M = 64 case once returned a wrong 4x64 block in about
# half of the calls), so every repeat must be bitwise identical, and the
# result within the oracle's tolerance on sampled columns.
REPEAT_CASES = [(bits, gs, M) for bits in (4, 8) for gs in (32, 128) for M in (24, 40, 64, 65, 128, 512)]


@pytest.mark.parametrize("bits,gs,M", REPEAT_CASES, ids=[f"q{b}-gs{g}-M{m}" for b, g, m in REPEAT_CASES])
def test_repeated_calls_bitwise_identical(oracle, bits, gs, M):
    N = K = 3584
    plan = ops.quantized_matmul_plan(M, N, K, gs, bits)
    print(f"case repeat bits={bits} gs={gs} M={M} plan={plan}", flush=True)
    L = _weights(N, K, gs, "q8" if bits == 8 else "q4")
    x = make_x_numpy(M, K, seed=M + 1)
    xd = dev(x, "bf16")
    ys = [ops.quantized_matmul(xd, L["w"], L["scales"], L["biases"], True, gs, bits, out_dtype=torch.float32)
          for _ in range(8)]
    torch.cuda.synchronize()
    for i, y in enumerate(ys[1:], 1):
        diff = (y != ys[0]).nonzero()
        assert diff.numel() == 0, f"{plan}: repeat {i} differs at {diff[:4].tolist()} ({diff.shape[0]} elements)"
    cols = _sample_cols(N, seed=N + M)
    ci = torch.from_numpy(cols).cuda()
    w = L["w"].index_select(0, ci).cpu().numpy().view(np.uint32)
    s = _to_np16(L["scales"].index_select(0, ci))
    b = _to_np16(L["biases"].index_select(0, ci))
    ref = oracle.quantized_matmul_f32(x, "bf16", w, s, b, "f16", gs, bits)
    mx, mean = parity_metrics(ys[0].index_select(1, ci).cpu().numpy(), ref)
    assert mx <= MAX_TOL and mean <= MEAN_TOL, (plan, mx, mean)
