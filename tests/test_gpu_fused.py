"""GPU tests of the fused Linear::forward and gated-MLP entry points.

kh_linear / kh_linear_multi (crates/kiln-models/src/nn.rs:79-102, 724-726):
the product rounded to its own dtype, then the bias added in float32 — bit
for bit the composite kh_quantized_matmul + kh_add, in one launch, on every
kernel path (decode GEMV, skinny MFMA, prefill GEMM with and without split-K,
the K % 128 != 0 kernels, the general kernel), and within the matmul
tolerance of the oracle's Linear::forward.

kh_mlp_gate_up (nn.rs:221-235, 284-294): act(gate(x) [+ b]) * (up(x) [+ b])
with act silu or gelu_approx. The fused decode launch equals the composite
path (the two matmuls, then the activation kernel) bit for bit; both equal
the oracle's per-op sequence on the device's own gate/up values to one unit
in the last place (device tanhf/expf against the host's), and the oracle's
full result within the matmul tolerance.
"""
import numpy as np
import pytest
import torch

from kiln_amd import _lib, ops
from kiln_amd.workloads import make_linear_numpy, make_x_numpy

from _util import dev, host, parity_metrics

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _bias(N, dt, seed):
    b = np.random.default_rng(seed).standard_normal(N).astype(np.float32)
    return torch.from_numpy(b).to(dt).cuda()


# (M, N, K, gs, bits): decode GEMV, skinny MFMA, GEMM split-K, GEMM, GEMM with N % 4 != 0 (the
# element-by-element epilogue), K % 128 != 0 (qmv / qmm)
PATHS = [(1, 272, 2048, 64, 4), (3, 96, 512, 32, 8), (12, 4096, 1024, 64, 4), (40, 300, 2048, 64, 4),
         (200, 512, 512, 128, 4), (256, 1022, 512, 64, 4), (12, 96, 320, 64, 4), (40, 96, 320, 32, 8)]


@pytest.mark.parametrize("M,N,K,gs,bits", PATHS)
@pytest.mark.parametrize("xdt,sdt,bdt", [("bf16", "bf16", "bf16"), ("bf16", "f16", "f32"),
                                         ("f16", "f16", "bf16"), ("f16", "f16", "f16"), ("f32", "bf16", "bf16")])
def test_linear_equals_matmul_then_add(oracle, M, N, K, gs, bits, xdt, sdt, bdt):
    plan = ops.quantized_matmul_plan(M, N, K, gs, bits, ops._NAMES[xdt], ops._NAMES[sdt])
    print(f"case linear M={M} N={N} K={K} gs={gs} bits={bits} x={xdt} s={sdt} bias={bdt} {plan}", flush=True)
    L = make_linear_numpy(N, K, gs, "q4" if bits == 4 else "q8", seed=N + K, sdt=sdt)
    x = make_x_numpy(M, K, seed=M, xdt=xdt)
    xd, w, s, b = dev(x, xdt), dev(L["w"]), dev(L["scales"], sdt), dev(L["biases"], sdt)
    bias = _bias(N, ops._NAMES[bdt], N)
    fused = ops.linear(xd, w, s, b, bias, gs, bits)
    ydt = ops.result_dtype(xd.dtype, s.dtype)
    y = ops.quantized_matmul(xd, w, s, b, True, gs, bits, out_dtype=ydt)
    comp = ops.add(y, bias)
    assert fused.dtype == comp.dtype
    assert torch.equal(fused, comp), plan
    # without a bias it is quantized_matmul
    assert torch.equal(ops.linear(xd, w, s, b, None, gs, bits), y)
    # the oracle's Linear::forward
    ref, rdt = oracle.linear(x, xdt, L["w"], L["scales"], L["biases"], sdt, gs, bits,
                             host(bias) if bdt != "f32" else bias.cpu().numpy(), bdt)
    mx, mean = parity_metrics(oracle.to_f32(host(fused), rdt), oracle.to_f32(ref, rdt))
    assert mx <= 2e-2 and mean <= 1e-3, (plan, mx, mean)


@pytest.mark.parametrize("M", [1, 4, 40, 300])
def test_linear_multi_equals_linear(M):
    """q/k/v with Qwen2-style biases (the k part here has none): each part of
    the one call equals kh_linear's result, on the fused decode launch and the
    shared-activation prefill GEMMs."""
    print(f"case linear_multi M={M}", flush=True)
    K, gs, bits = 1024, 64, 4
    parts = []
    for i, N in enumerate((256, 64, 64)):
        L = make_linear_numpy(N, K, gs, "q4", seed=60 + i, sdt="bf16")
        bias = None if i == 1 else _bias(N, torch.bfloat16, i)
        parts.append((dev(L["w"]), dev(L["scales"], "bf16"), dev(L["biases"], "bf16"), bias))
    x = dev(make_x_numpy(M, K, seed=7), "bf16")
    outs = ops.linear_multi(x, parts, gs, bits)
    for (w, s, b, bias), o in zip(parts, outs):
        assert torch.equal(o, ops.linear(x, w, s, b, bias, gs, bits))


def _gate_up_case(M, N, K, seed, bias):
    gs, bits = 64, 4
    # scales exactly representable in both 16-bit formats (8 significant
    # bits): the up projection can run with bfloat16 scales of the same value
    Lg = make_linear_numpy(N, K, gs, "q4", seed=seed, sdt="bf16")
    Lu = make_linear_numpy(N, K, gs, "q4", seed=seed + 1, sdt="bf16")
    x = make_x_numpy(M, K, seed=seed + 2)
    as_f16 = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).cuda().to(torch.float16)
    gate = (dev(Lg["w"]), as_f16(Lg["scales"]), as_f16(Lg["biases"]), _bias(N, torch.float32, 1) if bias else None)
    up = (dev(Lu["w"]), as_f16(Lu["scales"]), as_f16(Lu["biases"]), _bias(N, torch.float32, 2) if bias else None)
    up_bf = (up[0], dev(Lu["scales"], "bf16"), dev(Lu["biases"], "bf16"), up[3])
    assert torch.equal(up_bf[1].float(), up[1].float()) and torch.equal(up_bf[2].float(), up[2].float())
    return dev(x, "bf16"), gate, up, up_bf, (Lg, Lu, x)


@pytest.mark.parametrize("act", [_lib.ACT_SILU, _lib.ACT_GELU_APPROX])
@pytest.mark.parametrize("M", [1, 4, 12, 24, 40, 300])
def test_mlp_gate_up_fused_equals_composite(act, M):
    """On the fused launch (gate and up with the same scale dtype: the decode
    GEMV at M = 1, 4, the small-batch MFMA kernel in paired mode at M = 12,
    24, two split-K GEMMs reduced together with the activation at M = 40,
    300) and on the composite path (up's scales in the other 16-bit dtype,
    same values: two matmul launches, then the activation kernel) the result
    is bit-identical."""
    print(f"case mlp_gate_up act={act} M={M}", flush=True)
    N, K = 272, 2048
    xd, gate, up, up_bf, _ = _gate_up_case(M, N, K, 70 + M, False)
    if M >= 40:
        plan = ops.quantized_matmul_plan(M, N, K, 64, 4)
        assert plan.startswith("gemm") and "nsplit=1 " not in plan, plan
    fused = ops.mlp_gate_up(xd, gate, up, act, 64, 4)
    comp = ops.mlp_gate_up(xd, gate, up_bf, act, 64, 4)
    assert fused.dtype == comp.dtype
    assert torch.equal(fused, comp)


@pytest.mark.parametrize("act", [_lib.ACT_SILU, _lib.ACT_GELU_APPROX])
@pytest.mark.parametrize("M", [1, 4, 12, 40])
def test_mlp_gate_up_biases(oracle, act, M):
    """With gate and up biases (mlp_bias models): the activation of the
    device's own kh_linear results, to one unit in the last place (host
    transcendental functions against the device's)."""
    print(f"case mlp_gate_up bias act={act} M={M}", flush=True)
    N, K = 272, 2048
    xd, gate, up, _, _ = _gate_up_case(M, N, K, 90 + M, True)
    y = ops.mlp_gate_up(xd, gate, up, act, 64, 4)
    assert y.dtype == torch.float32
    g = ops.linear(xd, *gate, 64, 4).cpu().numpy()
    u = ops.linear(xd, *up, 64, 4).cpu().numpy()
    fn = oracle.gelu_mul if act == _lib.ACT_GELU_APPROX else oracle.silu_mul
    sep = fn(g, u, "f32").astype(np.float64)
    # 1 + tanh(s) cancels for very negative s: one float32 unit of tanh there
    # is 2^-24 |g u| in absolute terms
    tol = 2.0 ** -20 * np.abs(sep) + 2.0 ** -22 * np.abs(g.astype(np.float64) * u) + 1e-30
    assert np.all(np.abs(y.cpu().numpy() - sep) <= tol)


@pytest.mark.parametrize("act", [_lib.ACT_SILU, _lib.ACT_GELU_APPROX])
@pytest.mark.parametrize("M", [1, 40, 300])
@pytest.mark.parametrize("odt", ["bf16", "f16"])
def test_mlp_gate_up_matches_oracle(oracle, act, M, odt):
    """The per-op sequence of the reference: on the device's own gate and up
    values (kh_linear) the activation equals the oracle's to one unit in the
    last place of odt; the whole result is within the matmul tolerance of the
    oracle's."""
    print(f"case mlp_gate_up oracle act={act} M={M} odt={odt}", flush=True)
    N, K, gs, bits = 272, 2048, 64, 4
    Lg = make_linear_numpy(N, K, gs, "q4", seed=80, sdt=odt)
    Lu = make_linear_numpy(N, K, gs, "q4", seed=81, sdt=odt)
    x = make_x_numpy(M, K, seed=82, xdt=odt)
    xd = dev(x, odt)
    gate = (dev(Lg["w"]), dev(Lg["scales"], odt), dev(Lg["biases"], odt), None)
    up = (dev(Lu["w"]), dev(Lu["scales"], odt), dev(Lu["biases"], odt), None)
    y = host(ops.mlp_gate_up(xd, gate, up, act, gs, bits))
    fn = oracle.gelu_mul if act == _lib.ACT_GELU_APPROX else oracle.silu_mul
    gd = host(ops.linear(xd, *gate, gs, bits))
    ud = host(ops.linear(xd, *up, gs, bits))
    sep = oracle.to_f32(fn(gd, ud, odt), odt).astype(np.float64)
    ulp = 2.0 ** (-7 if odt == "bf16" else -10)
    assert np.all(np.abs(oracle.to_f32(y, odt) - sep) <= ulp * np.abs(sep) + 1e-30)
    g_ref = oracle.quantized_matmul(x, odt, Lg["w"], Lg["scales"], Lg["biases"], odt, gs, bits, True, odt)
    u_ref = oracle.quantized_matmul(x, odt, Lu["w"], Lu["scales"], Lu["biases"], odt, gs, bits, True, odt)
    ref = fn(g_ref, u_ref, odt)
    mx, mean = parity_metrics(oracle.to_f32(y, odt), oracle.to_f32(ref, odt))
    # gelu's per-op rounding amplifies a one-ulp gate difference near the
    # tanh saturation: the mean tolerance holds, the max is relative to max|ref|
    assert mx <= 2e-2 and mean <= 1e-3, (mx, mean)
