"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each function of the oracle is checked against something that does not share
its code: hand-built known-answer words, the exact-rational golden fixtures
(tests/golden/make_golden.py), numpy/torch conversions, closed-form special
cases, and an independent numpy float64 restatement.
"""
import glob
import os
from fractions import Fraction

import numpy as np
import pytest
import torch

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# --------------------------------------------------------------------------- unpack / pack

def test_unpack_known_words(oracle):
    w = np.array([[0x76543210, 0xFEDCBA98]], dtype=np.uint32)
    assert oracle.unpack(w, 4).tolist() == [list(range(16))]
    w8 = np.array([[0x03020100, 0xFFFEFDFC]], dtype=np.uint32)
    assert oracle.unpack(w8, 8).tolist() == [[0, 1, 2, 3, 252, 253, 254, 255]]
    assert oracle.unpack(np.full((1, 1), 0xFFFFFFFF, np.uint32), 4).tolist() == [[15] * 8]
    assert oracle.unpack(np.zeros((1, 1), np.uint32), 8).tolist() == [[0] * 4]


@pytest.mark.parametrize("bits", [4, 8])
def test_unpack_one_hot_column_order(oracle, bits):
    per = 32 // bits
    for j in range(per):
        w = np.array([[1 << (bits * j)]], dtype=np.uint32)
        expect = [0] * per
        expect[j] = 1
        assert oracle.unpack(w, bits).tolist() == [expect]


@pytest.mark.parametrize("bits", [4, 8])
def test_pack_unpack_roundtrip_and_numpy(oracle, bits):
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, (13, 96), dtype=np.uint8)
    w = oracle.pack(codes, bits)
    assert np.array_equal(w, oracle.np_pack(codes, bits))
    assert np.array_equal(oracle.unpack(w, bits), codes)
    assert np.array_equal(oracle.np_unpack(w, bits), codes)


# --------------------------------------------------------------------------- rounding

def _sweep_f32():
    rng = np.random.default_rng(7)
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e-8, 6.1035156e-05, 6.0e-05,
            5.96e-08, 2.98e-08, 3.0e-08, np.inf, -np.inf, 3.4e38, 1.0000001, 1.00390625,
            1.005859375, 1.001953125]
    r = rng.standard_normal(4000).astype(np.float32) * (10.0 ** rng.integers(-9, 6, 4000))
    # exact bf16 ties: low half 0x8000
    ties = (rng.integers(0, 2 ** 16, 200).astype(np.uint32) << 16 | 0x8000).view(np.float32)
    return np.concatenate([np.array(vals, np.float32), r.astype(np.float32),
                           ties[np.isfinite(ties)]]).astype(np.float32)


def test_bf16_rounding_matches_torch(oracle):
    v = _sweep_f32()
    c = np.array([oracle.lib().kho_f32_to_bf16(float(f)) for f in v], dtype=np.uint16)
    t = torch.from_numpy(v).bfloat16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(c, t)
    assert np.array_equal(oracle.from_f32(v, "bf16"), t)


def test_f16_rounding_matches_numpy(oracle):
    v = _sweep_f32()
    c = np.array([oracle.lib().kho_f32_to_f16(float(f)) for f in v], dtype=np.uint16)
    n = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(c, n)
    back = np.array([oracle.lib().kho_f16_to_f32(int(h)) for h in n[:500]], dtype=np.float32)
    assert np.array_equal(back, n[:500].view(np.float16).astype(np.float32))


# --------------------------------------------------------------------------- dequantize

@pytest.mark.parametrize("sdt", ["f16", "bf16"])
@pytest.mark.parametrize("bits", [4, 8])
def test_dequant_special_cases(oracle, sdt, bits):
    half = 1 << (bits - 1)
    s = oracle.from_f32(np.array([[0.0125, 0.0, 0.01]], np.float32), sdt)
    sv = oracle.to_f32(s, sdt)
    b = oracle.from_f32(np.array([[-half * sv[0, 0], 0.75, -half * sv[0, 2]]], np.float32), sdt)
    bv = oracle.to_f32(b, sdt)
    per = 32 // bits
    codes = np.zeros((1, 96), np.uint8)
    codes[0, 0:32] = np.arange(32) % (1 << bits)
    codes[0, 32:64] = (1 << bits) - 1
    codes[0, 64:96] = half
    w = oracle.np_pack(codes, bits)
    d = oracle.to_f32(oracle.dequantize(w, s, b, sdt, 32, bits, "f32"), "f32")
    assert d[0, 0] == bv[0, 0]                           # q = 0 -> bias
    assert np.all(d[0, 32:64] == bv[0, 1])               # scale 0 -> bias broadcast
    assert np.all(d[0, 64:96] == 0.0)                    # q = zero point, b = -half*s -> 0
    assert per in (4, 8)


@pytest.mark.parametrize("sdt", ["f16", "bf16"])
@pytest.mark.parametrize("bits", [4, 8])
def test_dequant_every_code_against_exact(oracle, sdt, bits):
    rng = np.random.default_rng(3)
    K, gs = 256 * (bits // 4), 32
    codes = np.tile(np.arange(1 << bits, dtype=np.uint8), 40 * K // (1 << bits))[: 40 * K].reshape(40, K)
    s = oracle.from_f32(rng.uniform(-0.05, 0.05, (40, K // gs)).astype(np.float32), sdt)
    b = oracle.from_f32(rng.uniform(-2, 2, (40, K // gs)).astype(np.float32), sdt)
    w = oracle.np_pack(codes, bits)
    exact = oracle.np_dequantize_f64(w, s, b, sdt, gs, bits)
    for odt in ("f32", "bf16", "f16"):
        got = oracle.dequantize(w, s, b, sdt, gs, bits, odt)
        want = oracle.from_f32(exact.astype(np.float32), odt) if odt != "bf16" else \
            torch.from_numpy(exact.astype(np.float32)).bfloat16().view(torch.int16).numpy().view(np.uint16)
        # `exact` holds scale*q + bias without rounding (f64 has room for it), so
        # exact -> f32 is the single rounding of the fma; narrower outputs round
        # that f32 value once more, which is the dequantisation rule.
        assert np.array_equal(got, want), odt


def test_dequant_f32_scales_is_single_fma(oracle):
    rng = np.random.default_rng(5)
    s = rng.uniform(-1, 1, (3, 2)).astype(np.float32)
    b = rng.uniform(-1, 1, (3, 2)).astype(np.float32)
    codes = rng.integers(0, 16, (3, 64), dtype=np.uint8)
    got = oracle.dequantize(oracle.np_pack(codes, 4), s, b, "f32", 32, 4, "f32")
    for r in range(3):
        for k in range(64):
            exact = Fraction(float(s[r, k // 32])) * int(codes[r, k]) + Fraction(float(b[r, k // 32]))
            assert got[r, k] == np.float32(float(exact)) or \
                abs(Fraction(float(got[r, k])) - exact) <= abs(exact) * Fraction(1, 2 ** 24)


# --------------------------------------------------------------------------- golden fixtures

def _fixtures():
    return sorted(glob.glob(os.path.join(GOLDEN, "*.npz")))


@pytest.mark.parametrize("path", _fixtures(), ids=os.path.basename)
def test_oracle_against_golden(oracle, path):
    f = np.load(path)
    bits, gs, sdt = int(f["bits"]), int(f["gs"]), str(f["sdt"])
    assert np.array_equal(oracle.unpack(f["w"], bits), f["codes"])
    deq = oracle.dequantize(f["w"], f["scales"], f["biases"], sdt, gs, bits, "f32")
    assert np.array_equal(deq.view(np.uint32), f["deq_f32"])
    deqb = oracle.dequantize(f["w"], f["scales"], f["biases"], sdt, gs, bits, "bf16")
    assert np.array_equal(deqb, f["deq_bf16"])
    emb = oracle.embedding(f["ids"], f["w"], f["scales"], f["biases"], sdt, gs, bits, "bf16")
    assert np.array_equal(emb, f["emb_bf16"])
    y = oracle.quantized_matmul_f32(f["x"], "bf16", f["w"], f["scales"], f["biases"], sdt, gs, bits)
    y_exact = f["y_f32"].view(np.float32)
    scale = np.abs(oracle.to_f32(f["x"], "bf16")) @ np.abs(deq).T
    assert np.all(np.abs(y - y_exact) <= 1e-6 * scale + 1e-30)
    yb = oracle.from_f32(y, "bf16").astype(np.int32)
    assert np.max(np.abs(yb - f["y_bf16"].astype(np.int32))) <= 1


# --------------------------------------------------------------------------- matmul

@pytest.mark.parametrize("transpose", [True, False])
@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (8, 128)])
def test_qmm_c_vs_numpy_f64(oracle, transpose, bits, gs):
    from kiln_amd.workloads import make_linear_numpy, make_x_numpy
    M, N, K = 5, 128, 256
    if transpose:
        L = make_linear_numpy(N, K, gs, "q4" if bits == 4 else "q8", seed=11)
    else:
        L = make_linear_numpy(K, N, gs, "q4" if bits == 4 else "q8", seed=11)
    x = make_x_numpy(M, K, seed=2)
    y = oracle.quantized_matmul_f32(x, "bf16", L["w"], L["scales"], L["biases"], "f16", gs, bits,
                                    transpose)
    ref = oracle.np_qmm_f64(x, "bf16", L["w"], L["scales"], L["biases"], "f16", gs, bits, transpose)
    W = oracle.np_dequantize_f64(L["w"], L["scales"], L["biases"], "f16", gs, bits)
    mag = np.abs(oracle.to_f32(x, "bf16")).astype(np.float64) @ np.abs(W.T if transpose else W)
    assert np.all(np.abs(y - ref) <= 2e-6 * mag)


def test_qmm_linearity_and_row_independence(oracle):
    from kiln_amd.workloads import make_linear_numpy, make_x_numpy
    L = make_linear_numpy(48, 128, 64, "q4", seed=4)
    x = make_x_numpy(6, 128, seed=9)
    full = oracle.quantized_matmul_f32(x, "bf16", L["w"], L["scales"], L["biases"], "f16", 64, 4)
    for m in range(6):
        one = oracle.quantized_matmul_f32(x[m:m + 1], "bf16", L["w"], L["scales"], L["biases"], "f16", 64, 4)
        assert np.array_equal(one[0], full[m])
    # y(2x) == 2 y(x) exactly (power-of-two scaling commutes with rounding)
    x2 = oracle.from_f32(2 * oracle.to_f32(x, "bf16"), "bf16")
    y2 = oracle.quantized_matmul_f32(x2, "bf16", L["w"], L["scales"], L["biases"], "f16", 64, 4)
    assert np.array_equal(y2, 2 * full)


# --------------------------------------------------------------------------- take / embedding

def test_embedding_equals_take_then_dequantize(oracle):
    from kiln_amd.workloads import make_linear_numpy
    L = make_linear_numpy(300, 256, 128, "emb", seed=8)
    ids = np.array([[0, 299, 17], [17, 5, 250]], dtype=np.uint32)
    emb = oracle.embedding(ids, L["w"], L["scales"], L["biases"], "f16", 128, 4, "bf16")
    w, s, b = oracle.take(L["w"], ids), oracle.take(L["scales"], ids), oracle.take(L["biases"], ids)
    assert np.array_equal(emb, oracle.dequantize(w, s, b, "f16", 128, 4, "bf16"))
    assert np.array_equal(w, L["w"][ids.astype(np.int64)])


def test_take_out_of_range_and_negative(oracle):
    a = np.arange(40, dtype=np.uint32).reshape(10, 4)
    ids = np.array([-1, 3, 10, -11, 0], dtype=np.int32)
    got = oracle.take(a, ids)
    assert got[0].tolist() == a[9].tolist()
    assert got[1].tolist() == a[3].tolist()
    assert got[2].tolist() == [0, 0, 0, 0]
    assert got[3].tolist() == [0, 0, 0, 0]
    assert got[4].tolist() == a[0].tolist()


# --------------------------------------------------------------------------- gated MLP activation

def test_silu_mul_f32_is_the_closed_form(oracle):
    rng = np.random.default_rng(5)
    g = rng.standard_normal(4096).astype(np.float32) * 6
    u = rng.standard_normal(4096).astype(np.float32)
    got = oracle.silu_mul(g, u, "f32").astype(np.float64)
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(got, want, rtol=2e-6, atol=1e-30)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_silu_mul_special_values_and_rounding(oracle, dt):
    g = oracle.from_f32(np.array([0.0, -0.0, 30.0, -30.0, 1.0, -1.0], np.float32), dt)
    u = oracle.from_f32(np.array([3.0, 3.0, 2.0, 2.0, 1.0, 1.0], np.float32), dt)
    got = oracle.to_f32(oracle.silu_mul(g, u, dt), dt)
    assert got[0] == 0 and got[1] == 0          # silu(0) = 0
    assert got[2] == 60.0                       # sigmoid(30) rounds to 1 in 16 bits
    assert abs(got[3]) < 1e-9                   # silu(-30) ~ -2.8e-12
    # silu(1) = 0.7310586, silu(-1) = -0.2689414, each rounded to dt
    for i, v in ((4, 0.7310585786), (5, -0.2689414214)):
        assert abs(got[i] - v) <= 2 ** (-8 if dt == "bf16" else -11) * abs(v) * 2
    # rounding happens at each op: stored results are representable in dt
    assert np.array_equal(oracle.from_f32(got, dt), oracle.silu_mul(g, u, dt))


def test_gelu_mul_f32_is_the_closed_form(oracle):
    """In float32 the per-op roundings are float32's own: the result is the
    tanh approximation of GELU (0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3))),
    evaluated here in float64) times up, to float32 accuracy; torch's tanh-GELU
    agrees. A wrong constant, sign or missing term fails by far more."""
    rng = np.random.default_rng(6)
    g = (rng.standard_normal(4096) * 4).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    got = oracle.gelu_mul(g, u, "f32").astype(np.float64)
    gd = g.astype(np.float64)
    want = 0.5 * gd * (1 + np.tanh(np.sqrt(2 / np.pi) * (gd + 0.044715 * gd ** 3))) * u
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)
    import torch
    t = (torch.nn.functional.gelu(torch.from_numpy(g), approximate="tanh") * torch.from_numpy(u)).numpy()
    assert np.allclose(got, t, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_gelu_mul_special_values_and_rounding(oracle, dt):
    g = oracle.from_f32(np.array([0.0, 8.0, -8.0, 1.0, -1.0, 2.0], np.float32), dt)
    u = oracle.from_f32(np.ones(6, np.float32), dt)
    got = oracle.to_f32(oracle.gelu_mul(g, u, dt), dt)
    assert got[0] == 0                # gelu(0) = 0
    assert got[1] == 8.0              # tanh saturates: gate rounds to 2, act = x
    assert abs(got[2]) < 2e-2         # gelu(-8) ~ 0 (the gate 1 + tanh rounds in dt)
    # gelu(1) = 0.8411920, gelu(-1) = -0.1588080, gelu(2) = 1.9545977, within
    # the per-op roundings of dt
    for i, v in ((3, 0.8411920), (4, -0.1588080), (5, 1.9545977)):
        assert abs(got[i] - v) <= 2 ** (-8 if dt == "bf16" else -11) * 16 * max(abs(v), 1)
    assert np.array_equal(oracle.from_f32(got, dt), oracle.gelu_mul(g, u, dt))
    # the reference rounds every intermediate: with dt = bf16 the result
    # differs from the float32 evaluation rounded once somewhere in a sweep
    if dt == "bf16":
        xs = oracle.from_f32(np.linspace(-4, 4, 801).astype(np.float32), dt)
        once = oracle.from_f32(oracle.gelu_mul(oracle.to_f32(xs, dt), np.ones(801, np.float32), "f32"), dt)
        assert not np.array_equal(oracle.gelu_mul(xs, oracle.from_f32(np.ones(801, np.float32), dt), dt), once)


def test_linear_rounds_the_product_then_adds(oracle):
    """Linear::forward (nn.rs:79-102) is two arrays: the product in its own
    dtype, then + bias. The oracle's linear equals quantized_matmul rounded to
    the product's dtype followed by the float32 sum rounded to the result's."""
    from kiln_amd.workloads import make_linear_numpy, make_x_numpy
    L = make_linear_numpy(48, 256, 64, "q4", seed=3, sdt="bf16")
    x = make_x_numpy(5, 256, seed=4)
    bias = oracle.from_f32(np.random.default_rng(1).standard_normal(48).astype(np.float32), "bf16")
    y, ydt = oracle.linear(x, "bf16", L["w"], L["scales"], L["biases"], "bf16", 64, 4)
    assert ydt == "bf16"
    r, rdt = oracle.linear(x, "bf16", L["w"], L["scales"], L["biases"], "bf16", 64, 4, bias, "bf16")
    assert rdt == "bf16"
    assert np.array_equal(r, oracle.from_f32(oracle.to_f32(y, "bf16") + oracle.to_f32(bias, "bf16"), "bf16"))
    r32, rdt = oracle.linear(x, "bf16", L["w"], L["scales"], L["biases"], "bf16", 64, 4,
                             oracle.to_f32(bias, "bf16"), "f32")
    assert rdt == "f32"   # bf16 product + f32 bias -> f32, the product still rounded to bf16 first
    assert np.array_equal(r32, oracle.to_f32(y, "bf16") + oracle.to_f32(bias, "bf16"))
    # against float64: within the product's rounding plus the sum's
    exact = oracle.np_qmm_f64(x, "bf16", L["w"], L["scales"], L["biases"], "bf16", 64, 4) + \
        oracle.to_f32(bias, "bf16").astype(np.float64)
    assert np.allclose(oracle.to_f32(r, "bf16"), exact, rtol=2 ** -7, atol=2e-2)


# --------------------------------------------------------------------------- affine quantize

def _dq_f32(oracle, wq, s, b, dt, gs, bits):
    codes = oracle.unpack(wq.reshape(-1, wq.shape[-1]), bits).astype(np.float64)
    sv = np.repeat(oracle.to_f32(s, dt).reshape(codes.shape[0], -1).astype(np.float64), gs, axis=1)
    bv = np.repeat(oracle.to_f32(b, dt).reshape(codes.shape[0], -1).astype(np.float64), gs, axis=1)
    return codes, sv * codes + bv


def test_quantize_known_answers(oracle):
    # positive ramp 0, 0.25, ..., 3.75 (gs 32, 4-bit): the larger-magnitude
    # extreme (3.75) is the edge, scale -0.25, bias 3.75, code 15 - k
    k = np.arange(32) % 16
    w = (k * 0.25).astype(np.float32)[None]
    wq, s, b = oracle.quantize(w, "f32", 32, 4)
    assert s.tolist() == [[-0.25]] and b.tolist() == [[3.75]]
    assert oracle.unpack(wq, 4).tolist() == [(15 - k).tolist()]
    # negative ramp 0, -0.5, ..., -7.5: edge -7.5, scale 0.5, code 15 - k
    w = (-k * 0.5).astype(np.float32)[None]
    wq, s, b = oracle.quantize(w, "f32", 32, 4)
    assert s.tolist() == [[0.5]] and b.tolist() == [[-7.5]]
    assert oracle.unpack(wq, 4).tolist() == [(15 - k).tolist()]
    # ties round half away from zero: (3.625 - 3.75) / -0.25 = 0.5 -> 1,
    # (3.125 - 3.75) / -0.25 = 2.5 -> 3 (round-half-even would give 0 and 2)
    w = np.zeros(32, np.float32)
    w[1], w[2], w[3] = 3.75, 3.625, 3.125
    wq, s, b = oracle.quantize(w[None], "f32", 32, 4)
    assert s.tolist() == [[-0.25]] and b.tolist() == [[3.75]]
    assert oracle.unpack(wq, 4)[0, :4].tolist() == [15, 0, 1, 3]
    # all-zero group: scale -1e-7 (the floor, negated), bias 0, codes 0
    wq, s, b = oracle.quantize(np.zeros((1, 64), np.float32), "f32", 64, 8)
    assert s[0, 0] == np.float32(-1e-7) and b.tolist() == [[0.0]] and not wq.any()
    # constant group c: bias c and code 0 reproduce c exactly
    wq, s, b = oracle.quantize(np.full((1, 64), 0.375, np.float32), "f32", 64, 4)
    assert b.tolist() == [[0.375]] and not wq.any()


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (8, 64), (4, 128), (8, 128)])
def test_quantize_round_trip_bound(oracle, dt, bits, gs):
    rng = np.random.default_rng(bits * 1000 + gs)
    v = (rng.standard_normal((37, 4 * gs)) * rng.uniform(0.01, 3, (37, 1))).astype(np.float32)
    v[3] = np.abs(v[3])            # one-signed groups
    v[4] = -np.abs(v[4])
    w = oracle.from_f32(v, dt)
    x = oracle.to_f32(w, dt).astype(np.float64)
    wq, s, b = oracle.quantize(w, dt, gs, bits)
    codes, rec = _dq_f32(oracle, wq, s, b, dt, gs, bits)
    nb = (1 << bits) - 1
    assert codes.min() >= 0 and codes.max() <= nb
    g = x.reshape(x.shape[0], -1, gs)
    sa = np.repeat(np.abs(oracle.to_f32(s, dt).astype(np.float64)), gs, axis=1)
    rel = {"f32": 2.0 ** -22, "bf16": 2.0 ** -8, "f16": 2.0 ** -10}[dt]
    # half the stored scale from the nearest code, plus the rounding of scale
    # and bias to dt (scale error times up to nb codes, bias error). The
    # scale is edge / round(edge / step): at most (nb/2 + 1/2) / (nb/2) steps.
    mag = np.repeat(np.abs(g).max(axis=2), gs, axis=1)
    step = np.repeat((g.max(axis=2) - g.min(axis=2)) / nb, gs, axis=1)
    assert (sa <= step * (nb + 1) / nb * (1 + 2 * rel) + 1e-30).all()
    # Rounding edge/step to an integer can also shrink the scale so that
    # nb*|s| falls short of the group's range: the far extreme is then clipped
    # to code nb, by at most that shortfall (the rule keeps 0 at an exact
    # code instead of covering the whole range).
    span = np.repeat(g.max(axis=2) - g.min(axis=2), gs, axis=1)
    clip = np.maximum(span - nb * sa, 0)
    # edge / step >= nb / 2, so the far code is at most nb + 1 before clipping
    assert (clip <= sa * (1 + 4 * rel) + rel * mag).all()
    bound = 0.5 * sa * (1 + rel) + clip + rel * (nb * sa + mag) * 1.01 + 1e-30
    assert (np.abs(rec - x) <= bound).all()
    # every group reaches both ends of the code range except where rounding
    # the edge ratio moved the scale: the extremes map near 0 and nb
    cg = codes.reshape(codes.shape[0], -1, gs)
    assert (cg.min(axis=2) <= 1).all() and (cg.max(axis=2) >= nb - 1).all()


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("bits,gs", [(4, 32), (8, 64), (4, 128)])
def test_quantize_c_equals_numpy_restatement(oracle, dt, bits, gs):
    rng = np.random.default_rng(7 + bits + gs)
    v = (rng.standard_normal((19, 3 * gs)) * 0.05).astype(np.float32)
    v[0, :gs] = 0.0
    v[1, :gs] = 0.25
    w = oracle.from_f32(v, dt)
    a = oracle.quantize(w, dt, gs, bits)
    r = oracle.np_quantize(w, dt, gs, bits)
    for x, y in zip(a, r):
        assert np.array_equal(x, y)
