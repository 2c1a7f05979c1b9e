"""GPU parity: libkiln_hip (through the C ABI via kiln_amd.ops) against the
CPU oracle on the same seeded inputs.

Bars: unpack/dequantize/embedding/take are bit-exact; quantized_matmul meets
max|err| <= 2e-2 * max|ref| and mean|err| / mean|ref| <= 1e-3 against the
oracle's float32-accumulated result rounded to the same output dtype, and a
much tighter elementwise bound on float32 outputs that catches any layout
slip (a wrong code, group or scale costs far more than it allows).
"""
import os

import numpy as np
import pytest
import torch

from kiln_amd import ops
from kiln_amd.workloads import make_linear_numpy, make_x_numpy

from _util import decode_regime, dev, exact_weights, gemv_max_m, host, parity_metrics

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
MAX_TOL, MEAN_TOL = 2e-2, 1e-3


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _case(M, N, K, gs, bits, xdt="bf16", sdt="f16", seed=0):
    L = make_linear_numpy(N, K, gs, "q4" if bits == 4 else "q8", seed=seed, sdt=sdt)
    x = make_x_numpy(M, K, seed=seed + 100, xdt=xdt)
    return L, x


def _run(L, x, gs, bits, xdt, sdt, odt, transpose=True):
    y = ops.quantized_matmul(dev(x, xdt), dev(L["w"]), dev(L["scales"], sdt), dev(L["biases"], sdt),
                             transpose, gs, bits, out_dtype=odt)
    torch.cuda.synchronize()
    return host(y)


# Elementwise bounds on float32 outputs, relative to sum_k |x||w|: the decode
# path (M <= 16) keeps every dequantised weight exact (only float32
# accumulation differs); the prefill path rounds each weight once to float16,
# |err| <= 2^-11 * sum |x w| plus accumulation.
EXACT_REL, F16W_REL = 3e-5, 2.0 ** -11 + 3e-5


def rel_for(M, K, bits, transpose=True, N=1, gs=64):
    return EXACT_REL if (not transpose or exact_weights(M, K, bits, N, gs)) else F16W_REL


def _check_f32(oracle, L, x, gs, bits, xdt, sdt, y, transpose=True, rel=None):
    if rel is None:
        N = L["w"].shape[0] if transpose else L["w"].shape[1] * (32 // bits)
        rel = rel_for(x.reshape(-1, x.shape[-1]).shape[0], x.shape[-1], bits, transpose, N, gs)
    ref = oracle.quantized_matmul_f32(x, xdt, L["w"], L["scales"], L["biases"], sdt, gs, bits, transpose)
    W = oracle.to_f32(oracle.dequantize(L["w"], L["scales"], L["biases"], sdt, gs, bits, "f32"), "f32")
    mag = np.abs(oracle.to_f32(x, xdt)).astype(np.float64) @ np.abs(W.T if transpose else W).astype(np.float64)
    bad = np.abs(y.astype(np.float64) - ref) > rel * mag + 1e-30
    assert not bad.any(), f"{bad.sum()} elements off; first at {np.argwhere(bad)[0]}"
    return ref


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("M", [1, 3, 16, 17, 64, 65, 200])
def test_qmm_bf16_f32out(oracle, bits, gs, M):
    print(f"case qmm bits={bits} gs={gs} M={M}", flush=True)
    N, K = 80, 512
    L, x = _case(M, N, K, gs, bits, seed=M + bits + gs)
    y = _run(L, x, gs, bits, "bf16", "f16", "f32")
    _check_f32(oracle, L, x, gs, bits, "bf16", "f16", y)


@pytest.mark.parametrize("xdt,sdt,odt", [("bf16", "bf16", "bf16"), ("f16", "f16", "f16"),
                                         ("bf16", "f16", "bf16"), ("f16", "bf16", "f32"),
                                         ("bf16", "f32", "f32")])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [1, 7, 96])
def test_qmm_dtypes_tolerance(oracle, xdt, sdt, odt, bits, M):
    print(f"case qmm dtypes x={xdt} s={sdt} o={odt} bits={bits} M={M}", flush=True)
    gs, N, K = 64, 144, 384
    L, x = _case(M, N, K, gs, bits, xdt=xdt, sdt=sdt, seed=5)
    y = _run(L, x, gs, bits, xdt, sdt, odt)
    ref = oracle.quantized_matmul(x, xdt, L["w"], L["scales"], L["biases"], sdt, gs, bits, True, odt)
    mx, mean = parity_metrics(oracle.to_f32(y, odt), oracle.to_f32(ref, odt))
    assert mx <= MAX_TOL and mean <= MEAN_TOL, (mx, mean)


@pytest.mark.parametrize("bits,gs", [(4, 64), (8, 32)])
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_qmm_transpose_false(oracle, bits, gs, xdt):
    print(f"case qmm transpose=false bits={bits} gs={gs} x={xdt}", flush=True)
    M, N, K = 5, 128, 192
    L = make_linear_numpy(K, N, gs, "q4" if bits == 4 else "q8", seed=3)
    x = make_x_numpy(M, K, seed=4, xdt=xdt)
    y = _run(L, x, gs, bits, xdt, "f16", "f32", transpose=False)
    ref = oracle.quantized_matmul_f32(x, xdt, L["w"], L["scales"], L["biases"], "f16", gs, bits, False)
    # the general kernel performs the oracle's exact float32 operation sequence
    assert np.array_equal(y, ref)


@pytest.mark.parametrize("K", [512, 6144, 16384, 16512])
def test_gemm_activation_prep_row_lengths(oracle, K):
    """The activation conversion in front of the GEMM: rows held in registers
    by one wave (K <= 4096) or four waves (K <= 16384), a workgroup per row
    beyond; rows whose maximum needs the power-of-two scaling (|x| >= 2^15)
    included."""
    print(f"case gemm prep K={K}", flush=True)
    M, N, gs, bits = 40, 48, 64, 4
    L, x = _case(M, N, K, gs, bits, seed=K)
    xf = oracle.to_f32(x, "bf16").copy()
    xf[3] *= 3.0e5
    xf[17, 5] = -7.0e4
    x = oracle.from_f32(xf, "bf16")
    y = _run(L, x, gs, bits, "bf16", "f16", "f32")
    _check_f32(oracle, L, x, gs, bits, "bf16", "f16", y, rel=F16W_REL)


def test_qmm_f32_activations_bit_exact(oracle):
    M, N, K, gs = 3, 40, 256, 32
    L, x = _case(M, N, K, gs, 4, xdt="f32", seed=9)
    y = _run(L, x, gs, 4, "f32", "f16", "f32")
    assert np.array_equal(y, oracle.quantized_matmul_f32(x, "f32", L["w"], L["scales"], L["biases"], "f16", gs, 4))


def test_qmm_leading_dims_and_empty(oracle):
    L, x = _case(6, 32, 128, 64, 4, seed=1)
    x3 = x.reshape(2, 3, 128)
    y = ops.quantized_matmul(dev(x3, "bf16"), dev(L["w"]), dev(L["scales"], "f16"),
                             dev(L["biases"], "f16"), True, 64, 4, out_dtype="f32")
    torch.cuda.synchronize()
    assert tuple(y.shape) == (2, 3, 32)
    flat = _run(L, x, 64, 4, "bf16", "f16", "f32")
    assert np.array_equal(host(y).reshape(6, 32), flat)
    e = ops.quantized_matmul(torch.empty((0, 128), dtype=torch.bfloat16, device="cuda"),
                             dev(L["w"]), dev(L["scales"], "f16"), dev(L["biases"], "f16"), True, 64, 4)
    assert tuple(e.shape) == (0, 32)


@pytest.mark.parametrize("bits,gs,K", [(4, 64, 1024), (8, 128, 1024), (4, 32, 1024), (8, 64, 9216),
                                       (4, 32, 1056)])
def test_rows_are_m_invariant(bits, gs, K):
    """Row r of the result is bitwise the same for every M served by the same
    kernel and tiling class (decode_regime) — the property Kiln's calibration
    probes (crates/kiln-models/src/nn.rs:301-327)."""
    N = 272
    L, x = _case(200, N, K, gs, bits, seed=21)
    groups = {}
    for M in (1, 2, 3, 4, 5, 6, 15, 16, 17, 20, 31, 32, 33, 64, 65, 100, 128, 129, 200):
        groups.setdefault(decode_regime(M, K, bits, N, gs), []).append(M)
    for regime, Ms in groups.items():
        big = _run(L, x[:max(Ms)], gs, bits, "bf16", "f16", "bf16")
        for M in Ms[:-1]:
            assert np.array_equal(_run(L, x[:M], gs, bits, "bf16", "f16", "bf16"), big[:M]), (regime, M)


# Shapes that exercise every VALU-decode plan: I = 1..4 chunks per lane slot,
# chunk counts that leave lane slots idle, N not a multiple of the rows per
# workgroup, M = 3 through the M = 4 kernel, f16 activations, bf16 scales.
@pytest.mark.parametrize("N,K,bits,gs", [(37, 4096, 4, 64), (1000, 3584, 8, 32), (21, 14336, 4, 128),
                                         (19, 20480, 4, 64), (11, 18944, 8, 128), (9, 33792, 8, 64),
                                         (7, 65536, 4, 32), (130, 96, 4, 32), (64, 2048, 8, 64)])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("xdt,sdt", [("bf16", "f16"), ("f16", "bf16")])
def test_gemv_plans(oracle, N, K, bits, gs, M, xdt, sdt):
    L, x = _case(M, N, K, gs, bits, xdt=xdt, sdt=sdt, seed=N + K + M)
    y = _run(L, x, gs, bits, xdt, sdt, "f32")
    _check_f32(oracle, L, x, gs, bits, xdt, sdt, y.view(np.float32), rel=EXACT_REL)


@pytest.mark.parametrize("path", sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz")))
def test_golden_fixtures(path):
    f = np.load(os.path.join(GOLDEN, path))
    bits, gs, sdt = int(f["bits"]), int(f["gs"]), str(f["sdt"])
    w, s, b = dev(f["w"]), dev(f["scales"], sdt), dev(f["biases"], sdt)
    d32 = host(ops.dequantize(w, s, b, gs, bits, out_dtype="f32"))
    db = host(ops.dequantize(w, s, b, gs, bits, out_dtype="bf16"))
    emb = host(ops.quantized_embedding(dev(f["ids"]).view(torch.int32), w, s, b, gs, bits, out_dtype="bf16"))
    y = host(ops.quantized_matmul(dev(f["x"], "bf16"), w, s, b, True, gs, bits, out_dtype="f32"))
    torch.cuda.synchronize()
    assert np.array_equal(d32.view(np.uint32), f["deq_f32"])
    assert np.array_equal(db, f["deq_bf16"])
    assert np.array_equal(emb, f["emb_bf16"])
    y_exact = f["y_f32"].view(np.float32).astype(np.float64)
    mag = np.abs((f["x"].astype(np.uint32) << 16).view(np.float32)).astype(np.float64) @ \
        np.abs(f["deq_f32"].view(np.float32)).T.astype(np.float64)
    assert np.all(np.abs(y - y_exact) <= 3e-5 * mag)


@pytest.mark.parametrize("bits,gs,sdt,odt", [(4, 64, "f16", "bf16"), (8, 32, "bf16", "bf16"),
                                             (4, 128, "f32", "f32"), (8, 64, "f16", "f16")])
def test_dequantize_bit_exact(oracle, bits, gs, sdt, odt):
    L = make_linear_numpy(333, 1024, gs, "q4" if bits == 4 else "q8", seed=2, sdt=sdt)
    got = host(ops.dequantize(dev(L["w"]), dev(L["scales"], sdt), dev(L["biases"], sdt), gs, bits,
                              out_dtype=odt))
    want = oracle.dequantize(L["w"], L["scales"], L["biases"], sdt, gs, bits, odt)
    assert np.array_equal(got, want)


def test_dequantize_default_dtype_is_scales_dtype():
    L = make_linear_numpy(4, 64, 32, "q4", sdt="bf16")
    y = ops.dequantize(dev(L["w"]), dev(L["scales"], "bf16"), dev(L["biases"], "bf16"), 32, 4)
    assert y.dtype == torch.bfloat16


def test_embedding_full_table_zipf_bit_exact(oracle):
    """Config 4(a): tied 4-bit gs128 table [128256, 4096], 4096 Zipf(1.1) ids."""
    from kiln_amd.workloads import make_linear_device
    V, H, gs = 128256, 4096, 128
    T = make_linear_device(V, H, gs, "emb", seed=44)
    rng = np.random.default_rng(45)
    ids = np.minimum(rng.zipf(1.1, 4096) - 1, V - 1).astype(np.uint32)
    got = host(ops.quantized_embedding(dev(ids), T["w"], T["scales"],
                                       T["biases"], gs, 4, out_dtype="bf16"))
    # the oracle needs only the rows it gathers
    uniq, inv = np.unique(ids, return_inverse=True)
    sel = torch.from_numpy(uniq.astype(np.int64)).cuda()
    w = host(T["w"][sel])
    s = host(T["scales"][sel])
    b = host(T["biases"][sel])
    want = oracle.embedding(inv.astype(np.uint32), w, s, b, "f16", gs, 4, "bf16")
    assert np.array_equal(got, want)


def test_embedding_signed_ids_and_out_of_range():
    L = make_linear_numpy(50, 256, 64, "emb", seed=3)
    w, s, b = dev(L["w"]), dev(L["scales"], "f16"), dev(L["biases"], "f16")
    ids = torch.tensor([[-1, 0, 49], [50, -51, 7]], dtype=torch.int32, device="cuda")
    y = host(ops.quantized_embedding(ids, w, s, b, 64, 4, out_dtype="f32"))
    full = host(ops.dequantize(w, s, b, 64, 4, out_dtype="f32"))
    assert np.array_equal(y[0, 0], full[49]) and np.array_equal(y[0, 2], full[49])
    assert np.array_equal(y[0, 1], full[0]) and np.array_equal(y[1, 2], full[7])
    assert not y[1, 0].any() and not y[1, 1].any()


@pytest.mark.parametrize("H,bits,gs", [(4096, 8, 32), (96, 8, 32), (8320, 4, 128), (64, 4, 32)])
@pytest.mark.parametrize("sdt,odt", [("f16", "bf16"), ("bf16", "f32"), ("f16", "f16")])
@pytest.mark.parametrize("aligned", [True, False])
def test_embedding_rows_match_dequantize(H, bits, gs, sdt, odt, aligned):
    """The lookup equals the dequantized table's rows bit for bit, for 16-byte
    and 4-byte aligned tables, with signed and out-of-range ids."""
    V = 37
    L = make_linear_numpy(V, H, gs, "emb" if bits == 4 else "q8", seed=H + bits, sdt=sdt)
    w, s, b = dev(L["w"]), dev(L["scales"], sdt), dev(L["biases"], sdt)
    full = host(ops.dequantize(w, s, b, gs, bits, out_dtype=odt))
    if not aligned:  # the same words at a 4-byte (not 16-byte) aligned address
        buf = torch.zeros(w.numel() + 1, dtype=w.dtype, device="cuda")
        buf[1:] = w.reshape(-1)
        w = buf[1:].view(w.shape)
        assert w.data_ptr() % 16 != 0
    ids = np.array([5, 0, 36, -1, 37, 12, 5, -40, 20], dtype=np.int32)
    y = host(ops.quantized_embedding(torch.from_numpy(ids).cuda(), w, s, b, gs, bits, out_dtype=odt))
    for t, i in enumerate(ids):
        if -V <= i < V:
            assert np.array_equal(y[t], full[i % V]), t
        else:
            assert not y[t].astype(np.float64).any(), t


@pytest.mark.parametrize("dtype", [torch.float16, torch.int32, torch.uint8])
def test_take_rows(dtype):
    a = (torch.arange(10 * 6, device="cuda") % 251).to(dtype).reshape(10, 6)
    idx = torch.tensor([3, 0, 9, 3], dtype=torch.int32, device="cuda")
    got = ops.take(a, idx, 0)
    assert torch.equal(got, a[idx.long()])
    b = torch.arange(8 * 4 * 4, device="cuda", dtype=torch.float32).reshape(8, 4, 4)
    idx2 = torch.tensor([[1, 7], [0, 2]], dtype=torch.int32, device="cuda")
    assert torch.equal(ops.take(b, idx2), b[idx2.long()])


def test_errors_raise_kiln_error():
    L, x = _case(1, 32, 128, 64, 4)
    with pytest.raises(ops.KilnError) as e:
        ops.quantized_matmul(dev(x, "bf16"), dev(L["w"]), dev(L["scales"], "f16"),
                             dev(L["biases"], "f16"), True, 64, 3)
    assert e.value.status == 1 and "bits=3" in str(e.value)


@pytest.mark.parametrize("M,N,K", [(1, 1024, 4096), (3, 272, 1024), (130, 200, 512), (24, 1024, 4096),
                                   (64, 8200, 2048)])
def test_graph_capture_replays_match_eager(M, N, K):
    """The library's launches (split-K partials, workspace) are capturable in a
    HIP graph; every replay, with eager work in between, equals the eager call."""
    print(f"case graph M={M} N={N} K={K}", flush=True)
    L, x = _case(M, N, K, 64, 4, seed=13)
    xd, w, s, b = dev(x, "bf16"), dev(L["w"]), dev(L["scales"], "f16"), dev(L["biases"], "f16")
    eager = ops.quantized_matmul(xd, w, s, b, True, 64, 4, out_dtype="f32").clone()
    out = torch.empty_like(eager)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.quantized_matmul(xd, w, s, b, True, 64, 4, out=out)
    for r in range(4):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), r
        ops.quantized_matmul(xd, w, s, b, True, 64, 4, out_dtype="f32")  # eager work between
        torch.cuda.synchronize()


def test_graph_workspace_survives_eager_growth():
    """A graph captured on a stream keeps using that stream's workspace; an
    eager call afterwards on the same stream that needs a larger workspace
    must not free the buffer the graph refers to. Every replay after the
    growth still equals the eager result."""
    print("case graph workspace growth", flush=True)
    N, K = 1024, 2048
    L, x = _case(40, N, K, 64, 4, seed=17)  # M = 40: the GEMM path (workspace user)
    xd, w, s, b = dev(x, "bf16"), dev(L["w"]), dev(L["scales"], "f16"), dev(L["biases"], "f16")
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        eager = ops.quantized_matmul(xd, w, s, b, True, 64, 4, out_dtype="f32").clone()
        out = torch.empty_like(eager)
    st.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        ops.quantized_matmul(xd, w, s, b, True, 64, 4, out=out)
    Lb, xb = _case(2048, N, K, 64, 4, seed=18)  # needs a workspace several times larger
    big = [dev(xb, "bf16"), dev(Lb["w"]), dev(Lb["scales"], "f16"), dev(Lb["biases"], "f16")]
    for r in range(3):
        with torch.cuda.stream(st):
            ops.quantized_matmul(*big, True, 64, 4, out_dtype="f32")
            big[0] = torch.cat([big[0], big[0]])  # the next eager call grows it again
            out.fill_(float("nan"))
            g.replay()
        st.synchronize()
        assert torch.equal(out, eager), r


@pytest.mark.parametrize("bits,gs,K", [(4, 32, 224), (4, 64, 192), (8, 32, 96), (8, 64, 320), (4, 32, 32)])
@pytest.mark.parametrize("M", [1, 5, 16, 40])
def test_qmm_partial_blocks(oracle, bits, gs, K, M):
    """K that is a multiple of the group size but not of the 16-byte lane block."""
    print(f"case partial bits={bits} gs={gs} K={K} M={M}", flush=True)
    N = 48
    L, x = _case(M, N, K, gs, bits, seed=K + M)
    y = _run(L, x, gs, bits, "bf16", "f16", "f32")
    _check_f32(oracle, L, x, gs, bits, "bf16", "f16", y)


@pytest.mark.gpu
@pytest.mark.parametrize("adt,bdt,odt", [(torch.bfloat16, torch.bfloat16, torch.bfloat16),
                                         (torch.float16, torch.float16, torch.float16),
                                         (torch.bfloat16, torch.float32, torch.float32),
                                         (torch.float16, torch.bfloat16, torch.float16)])
@pytest.mark.parametrize("shape,bshape", [((5, 96), (96,)), ((2, 3, 4101), (4101,)),
                                          ((2, 3, 8), (3, 8)), ((0, 16), (16,)), ((4, 1, 8), (3, 8)),
                                          ((2, 3, 5, 7), (2, 3, 1, 7)), ((1, 5), (3, 1)), ((6,), (2, 4, 6))])
def test_add_broadcast_bit_exact(adt, bdt, odt, shape, bshape):
    """kh_add: numpy broadcasting (mlx_add), each sum formed in float32 and
    rounded once (RNE) to the output dtype — the same as IEEE float32
    addition followed by one cast."""
    g = torch.Generator().manual_seed(7)
    a = torch.randn(shape, generator=g).to(adt).cuda()
    b = torch.randn(bshape, generator=g).to(bdt).cuda()
    out = torch.empty(torch.broadcast_shapes(shape, bshape), dtype=odt, device="cuda")
    ops.add(a, b, out=out)
    ref = (a.float() + b.float()).to(odt)
    assert torch.equal(out.view(-1).cpu().view(torch.int16 if odt != torch.float32 else torch.int32),
                       ref.view(-1).cpu().view(torch.int16 if odt != torch.float32 else torch.int32))


@pytest.mark.gpu
def test_add_rejects_incompatible_shapes():
    a = torch.zeros((4, 8), dtype=torch.float16, device="cuda")
    with pytest.raises(ops.KilnError, match="cannot broadcast"):
        ops.add(a, torch.zeros((4,), dtype=torch.float16, device="cuda"), out=torch.empty_like(a))


# ----------------------------------------------------------------- fused neighbours (q/k/v, gate/up)

@pytest.mark.parametrize("M", [1, 3, 6, 8, 9, 12, 24, 40, 300])
@pytest.mark.parametrize("bits,gs", [(4, 64), (8, 128)])
def test_multi_equals_separate_calls(M, bits, gs):
    """kh_quantized_matmul_multi (the q/k/v triple on one x, nn.rs:724-726)
    returns, part by part, the bits of separate kh_quantized_matmul calls:
    one decode GEMV launch (M <= 8), one small-batch MFMA launch (M = 9..32),
    and at M = 6 the wide part on the MFMA kernel with the narrow parts'
    GEMV launch beside it; the prefill GEMM from M = 40."""
    K = 1024
    shapes = [(2048 if M == 6 else 256, K), (64, K), (64, K)]
    parts, host_parts = [], []
    for i, (N, _) in enumerate(shapes):
        L = make_linear_numpy(N, K, gs, "q4" if bits == 4 else "q8", seed=40 + i)
        host_parts.append(L)
        parts.append((dev(L["w"]), dev(L["scales"], "f16"), dev(L["biases"], "f16")))
    x = dev(make_x_numpy(M, K, seed=44), "bf16")
    outs = ops.quantized_matmul_multi(x, parts, True, gs, bits, out_dtype="bf16")
    if M == 6:
        plans = [ops.quantized_matmul_plan(M, N, K, gs, bits, torch.bfloat16, torch.float16) for N, _ in shapes]
        assert plans[0] == "skinny" and plans[1] == plans[2] == "gemv", plans
    for (w, s, b), o in zip(parts, outs):
        ref = ops.quantized_matmul(x, w, s, b, True, gs, bits, out_dtype="bf16")
        assert torch.equal(o.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("M", [1, 2, 4, 8, 17, 64])
@pytest.mark.parametrize("odt", ["bf16", "f16", "f32"])
def test_gate_up_matches_oracle(oracle, M, odt):
    """kh_quantized_gate_up = silu(x gate^T) * (x up^T) with the per-op
    roundings of nn.rs:284-294 (oracle.silu_mul), within the matmul tolerance
    of the oracle; and, on the fused decode launch, equal (to one unit in the
    last place: expf) to separate calls followed by the same activation."""
    N, K, gs, bits = 272, 2048, 64, 4
    Lg = make_linear_numpy(N, K, gs, "q4", seed=50)
    Lu = make_linear_numpy(N, K, gs, "q4", seed=51)
    x = make_x_numpy(M, K, seed=52, xdt="bf16")
    gate = (dev(Lg["w"]), dev(Lg["scales"], "f16"), dev(Lg["biases"], "f16"))
    up = (dev(Lu["w"]), dev(Lu["scales"], "f16"), dev(Lu["biases"], "f16"))
    y = host(ops.quantized_gate_up(dev(x, "bf16"), gate, up, gs, bits, out_dtype=odt))
    g_ref = oracle.quantized_matmul(x, "bf16", Lg["w"], Lg["scales"], Lg["biases"], "f16", gs, bits, True, odt)
    u_ref = oracle.quantized_matmul(x, "bf16", Lu["w"], Lu["scales"], Lu["biases"], "f16", gs, bits, True, odt)
    ref = oracle.silu_mul(g_ref, u_ref, odt)
    mx, mean = parity_metrics(oracle.to_f32(y, odt), oracle.to_f32(ref, odt))
    assert mx <= 2e-2 and mean <= 1e-3, (mx, mean)
    # separate device calls + the same activation on the host
    gd = host(ops.quantized_matmul(dev(x, "bf16"), *gate, True, gs, bits, out_dtype=odt))
    ud = host(ops.quantized_matmul(dev(x, "bf16"), *up, True, gs, bits, out_dtype=odt))
    sep = oracle.to_f32(oracle.silu_mul(gd, ud, odt), odt).astype(np.float64)
    # one unit of the 16-bit formats; for float32 a few units (device expf and
    # the float32 chain against numpy)
    ulp = 2.0 ** (-7 if odt == "bf16" else (-10 if odt == "f16" else -20))
    assert np.all(np.abs(oracle.to_f32(y, odt) - sep) <= ulp * np.abs(sep) + 1e-30)


def test_fused_entry_points_validate():
    L = make_linear_numpy(64, 256, 64, "q4", seed=3)
    w, s, b = dev(L["w"]), dev(L["scales"], "f16"), dev(L["biases"], "f16")
    L2 = make_linear_numpy(32, 256, 64, "q4", seed=4)
    w2, s2, b2 = dev(L2["w"]), dev(L2["scales"], "f16"), dev(L2["biases"], "f16")
    x = dev(make_x_numpy(2, 256, seed=5), "bf16")
    with pytest.raises(ops.KilnError, match="quantized_gate_up"):
        ops.quantized_gate_up(x, (w, s, b), (w2, s2, b2), 64, 4, out_dtype="bf16")
    with pytest.raises(ops.KilnError, match="quantized_matmul_multi"):
        ops.quantized_matmul_multi(x, [(w, s, b)], True, 48, 4, out_dtype="bf16")


# ----------------------------------------------------------------- gather_qmm (MoE expert dispatch)

def _experts(E, N, K, gs, bits, seed, sdt="f16"):
    Ls = [make_linear_numpy(N, K, gs, "q4" if bits == 4 else "q8", seed=seed + e, sdt=sdt) for e in range(E)]
    w = np.stack([L["w"] for L in Ls])
    s = np.stack([L["scales"] for L in Ls])
    b = np.stack([L["biases"] for L in Ls])
    return w, s, b


@pytest.mark.parametrize("layout", ["unsorted", "sorted"])
@pytest.mark.parametrize("bits,gs", [(4, 64), (8, 32)])
def test_gather_qmm_kiln_shapes(oracle, layout, bits, gs):
    """SwitchLinear::forward's two call shapes (moe.rs:124-176, 272-310):
    x [T,1,1,K] with indices [T,k] (no sort), and the sorted form x [T*k,1,K]
    with indices [T*k]. Each pair equals kh_quantized_matmul on its expert's
    slices, bit for bit, and the oracle to the decode bound."""
    E, N, K, T, k = 6, 96, 512, 5, 3
    w, s, b = _experts(E, N, K, gs, bits, seed=60)
    rng = np.random.default_rng(61)
    ids = rng.integers(0, E, (T, k)).astype(np.uint32)
    xs = make_x_numpy(T, K, seed=62, xdt="bf16")
    if layout == "unsorted":
        x = dev(xs.reshape(T, 1, 1, K), "bf16")
        idx = dev(ids)
        pairs = [(t, j) for t in range(T) for j in range(k)]
    else:
        order = np.argsort(ids.reshape(-1), kind="stable")
        x = dev(xs[order // k].reshape(T * k, 1, K), "bf16")
        idx = dev(ids.reshape(-1)[order])
        pairs = [(int(o) // k, int(o) % k) for o in order]
    y = ops.gather_qmm(x, dev(w), dev(s, "f16"), dev(b, "f16"), idx, True, gs, bits, layout == "sorted",
                       out_dtype="f32")
    torch.cuda.synchronize()
    yh = host(y).reshape(-1, N)
    for p, (t, j) in enumerate(pairs):
        e = int(ids[t, j])
        L = dict(w=w[e], scales=s[e], biases=b[e])
        xr = xs[t:t + 1]
        got = yh[p:p + 1]
        _check_f32(oracle, L, xr, gs, bits, "bf16", "f16", got, rel=EXACT_REL)
        single = host(ops.quantized_matmul(dev(xr, "bf16"), dev(w[e]), dev(s[e], "f16"), dev(b[e], "f16"),
                                           True, gs, bits, out_dtype="f32"))
        assert np.array_equal(single.view(np.uint32), got.view(np.uint32)), p


def test_gather_qmm_signed_and_out_of_range_ids(oracle):
    E, N, K = 4, 64, 256
    w, s, b = _experts(E, N, K, 64, 4, seed=70)
    xs = make_x_numpy(4, K, seed=71, xdt="bf16")
    ids = np.array([-1, 3, 7, -9], dtype=np.int32)  # -1 -> 3; 7 and -9 out of range
    y = host(ops.gather_qmm(dev(xs.reshape(4, 1, K), "bf16"), dev(w), dev(s, "f16"), dev(b, "f16"),
                            torch.from_numpy(ids).cuda(), True, 64, 4, out_dtype="f32")).reshape(4, N)
    ref3 = host(ops.quantized_matmul(dev(xs[0:1], "bf16"), dev(w[3]), dev(s[3], "f16"), dev(b[3], "f16"),
                                     True, 64, 4, out_dtype="f32"))
    assert np.array_equal(y[0:1].view(np.uint32), ref3.view(np.uint32))
    assert not y[2].any() and not y[3].any()


@pytest.mark.parametrize("M,xdt", [(2, "bf16"), (12, "bf16"), (3, "f32")])
def test_gather_qmm_rows_per_pair_and_fallback(oracle, M, xdt):
    """M rows per pair through the decode kernel (M in the GEMV range), the
    grouped GEMM (larger M) or the exact fallback (float32 x): per pair, the
    oracle's bound for that kernel (float32 x is the oracle's own chain:
    bit-exact)."""
    E, N, K, P = 3, 80, 256, 4
    w, s, b = _experts(E, N, K, 64, 4, seed=80)
    xs = make_x_numpy(P * M, K, seed=81, xdt=xdt).reshape(P, M, K)
    ids = np.array([2, 0, 2, 1], dtype=np.uint32)
    y = host(ops.gather_qmm(dev(xs, xdt if xdt != "f32" else None), dev(w), dev(s, "f16"), dev(b, "f16"),
                            dev(ids), True, 64, 4, out_dtype="f32"))
    for p in range(P):
        e = int(ids[p])
        L = dict(w=w[e], scales=s[e], biases=b[e])
        ref = oracle.quantized_matmul_f32(xs[p], xdt, w[e], s[e], b[e], "f16", 64, 4, True)
        if xdt == "f32":
            assert np.array_equal(y[p].astype(np.float32).view(np.uint32), ref.astype(np.float32).view(np.uint32))
        else:
            rel = EXACT_REL if M <= gemv_max_m(K, 4) else F16W_REL
            _check_f32(oracle, L, xs[p], 64, 4, xdt, "f16", y[p], rel=rel)


def _grouped_ids(T, k, E, seed):
    """[T, k] expert ids, k distinct per token, every expert used >= 33 times."""
    rng = np.random.default_rng(seed)
    base = np.arange(T * k).reshape(T, k) % E
    return ((base + rng.integers(0, E, (T, 1))) % E).astype(np.uint32)


@pytest.mark.parametrize("layout", ["sorted", "unsorted"])
@pytest.mark.parametrize("E,T,k", [(4, 80, 2), (2, 200, 1), (6, 100, 3)])
@pytest.mark.parametrize("bits,gs,sdt", [(4, 64, "f16"), (8, 32, "bf16"), (4, 128, "bf16")])
def test_gather_qmm_grouped_gemm(oracle, layout, E, T, k, bits, gs, sdt):
    """Prefill-size gather_qmm (SwitchGlu's T*k pairs, moe.rs:272-310) runs
    as one grouped GEMM: every row equals kh_quantized_matmul's GEMM path on
    its expert's rows bit for bit (K = 512 takes no split-K; a row's result
    depends neither on its tile nor its neighbours), and the oracle to the
    float16-weight bound. Tile heights 32, 128 and 64 rows by (E, T, k)."""
    N, K = 320, 512
    w, s, b = _experts(E, N, K, gs, bits, seed=100 + E, sdt=sdt)
    ids = _grouped_ids(T, k, E, seed=101)
    xs = make_x_numpy(T, K, seed=102, xdt="bf16")
    if layout == "unsorted":  # x [T,1,1,K] broadcast over the k slots
        x = dev(xs.reshape(T, 1, 1, K), "bf16")
        idx = dev(ids)
        pairs = [(t, j) for t in range(T) for j in range(k)]
    else:
        order = np.argsort(ids.reshape(-1), kind="stable")
        x = dev(xs[order // k].reshape(T * k, 1, K), "bf16")
        idx = dev(ids.reshape(-1)[order])
        pairs = [(int(o) // k, int(o) % k) for o in order]
    y = ops.gather_qmm(x, dev(w), dev(s, sdt), dev(b, sdt), idx, True, gs, bits, layout == "sorted",
                       out_dtype="f32")
    torch.cuda.synchronize()
    yh = host(y).reshape(-1, N)
    for e in range(E):
        sel = [p for p, (t, j) in enumerate(pairs) if ids[t, j] == e]
        toks = [pairs[p][0] for p in sel]
        assert len(sel) >= 33
        L = dict(w=w[e], scales=s[e], biases=b[e])
        ref = host(ops.quantized_matmul(dev(xs[toks], "bf16"), dev(w[e]), dev(s[e], sdt), dev(b[e], sdt),
                                        True, gs, bits, out_dtype="f32"))
        assert np.array_equal(yh[sel].view(np.uint32), ref.view(np.uint32)), e
        _check_f32(oracle, L, xs[toks[:8]], gs, bits, "bf16", sdt, yh[sel[:8]], rel=F16W_REL)


def test_gather_qmm_grouped_ids_out_of_range(oracle):
    """Grouped path with int32 ids: -1 counts from the end, ids outside
    [-E, E) give zero rows, and the valid rows are unchanged by them."""
    E, N, K, P = 5, 256, 256, 96
    w, s, b = _experts(E, N, K, 64, 4, seed=110)
    xs = make_x_numpy(P, K, seed=111, xdt="bf16")
    ids = (np.arange(P) % E).astype(np.int32)
    ids[::7] = -1      # expert 4
    ids[3::11] = 9     # out of range
    ids[5::13] = -6    # out of range
    y = host(ops.gather_qmm(dev(xs.reshape(P, 1, K), "bf16"), dev(w), dev(s, "f16"), dev(b, "f16"),
                            torch.from_numpy(ids).cuda(), True, 64, 4, out_dtype="f32")).reshape(P, N)
    bad = (ids >= E) | (ids < -E)
    assert bad.any() and not y[bad].any()
    for p in np.flatnonzero(~bad)[:12]:
        e = int(ids[p]) % E
        L = dict(w=w[e], scales=s[e], biases=b[e])
        _check_f32(oracle, L, xs[p:p + 1], 64, 4, "bf16", "f16", y[p:p + 1], rel=F16W_REL)


@pytest.mark.parametrize("E", [300, 1023, 1030])
def test_gather_qmm_many_experts(oracle, E):
    """Hundreds of experts through the grouped path (one scan thread per
    expert group, up to 1023 experts plus the out-of-range group), and past
    that limit the pair-by-pair kernels: every row equals
    kh_quantized_matmul on its expert within that kernel's bound."""
    N, K = 32, 256
    P = 2 * (E + 1) + 40  # enough rows per group for the grouped path where E allows it
    w, s, b = _experts(E, N, K, 64, 4, seed=120)
    rng = np.random.default_rng(121)
    ids = np.sort(rng.integers(0, E, P)).astype(np.int32)
    ids[::97] = E + 5  # out of range
    xs = make_x_numpy(P, K, seed=122, xdt="bf16")
    y = host(ops.gather_qmm(dev(xs.reshape(P, 1, K), "bf16"), dev(w), dev(s, "f16"), dev(b, "f16"),
                            torch.from_numpy(ids).cuda(), True, 64, 4, True, out_dtype="f32")).reshape(P, N)
    assert not y[::97].any()
    grouped = E <= 1023 and P >= 2 * min(E + 1, P)
    for p in [1, 2, 50, 333, P - 1]:
        if p % 97 == 0:
            continue
        e = int(ids[p])
        L = dict(w=w[e], scales=s[e], biases=b[e])
        _check_f32(oracle, L, xs[p:p + 1], 64, 4, "bf16", "f16", y[p:p + 1],
                   rel=F16W_REL if grouped else EXACT_REL)


def test_gather_qmm_empty_and_errors():
    w, s, b = _experts(2, 32, 256, 64, 4, seed=90)
    W = (dev(w), dev(s, "f16"), dev(b, "f16"))
    x1 = dev(make_x_numpy(1, 256, seed=91).reshape(1, 1, 256), "bf16")
    empty = ops.gather_qmm(x1, *W, torch.empty((0,), dtype=torch.int32, device="cuda"), True, 64, 4,
                           out_dtype="bf16")
    assert tuple(empty.shape) == (0, 1, 32)
    x3 = dev(make_x_numpy(3, 256, seed=92).reshape(3, 1, 256), "bf16")
    with pytest.raises(ops.KilnError, match="broadcast"):
        ops.gather_qmm(x3, *W, torch.zeros((2,), dtype=torch.int32, device="cuda"), True, 64, 4,
                       out=torch.empty((3, 1, 32), device="cuda", dtype=torch.bfloat16))
    with pytest.raises(ops.KilnError, match="transpose=false"):
        ops.gather_qmm(x3, *W, torch.zeros((3,), dtype=torch.int32, device="cuda"), False, 64, 4,
                       out=torch.empty((3, 1, 32), device="cuda", dtype=torch.bfloat16))


# --------------------------------------------------------------------------- affine quantize

def _quant_input(oracle, rows, K, gs, dt, seed):
    rng = np.random.default_rng(seed)
    v = (rng.standard_normal((rows, K)) * rng.uniform(0.001, 2, (rows, 1))).astype(np.float32)
    v[0, :gs] = 0.0                      # all-zero group
    v[1, :gs] = 0.375                    # constant group
    v[2] = np.abs(v[2])                  # one-signed rows
    v[3] = -np.abs(v[3])
    if gs >= 32 and rows > 4:            # ties of the code rounding
        v[4, :gs] = 0.0
        v[4, 1], v[4, 2], v[4, 3] = 3.75, 3.625, 3.125
    return oracle.from_f32(v, dt)


@pytest.mark.gpu
@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (4, 128), (8, 32), (8, 64), (8, 128)])
def test_quantize_bit_exact(oracle, dt, bits, gs):
    w = _quant_input(oracle, 37, 4 * gs + 2 * gs, gs, dt, seed=bits * 7 + gs)
    got = ops.quantize(dev(w, dt), gs, bits)
    want = oracle.quantize(w, dt, gs, bits)
    for g, x in zip(got, want):
        assert np.array_equal(host(g), x)


@pytest.mark.gpu
def test_quantize_leading_dims_and_round_trip(oracle):
    gs, bits, dt = 64, 4, "bf16"
    w = _quant_input(oracle, 2 * 3 * 5, 256, gs, dt, seed=11).reshape(2, 3, 5, 256)
    wq, s, b = ops.quantize(dev(w, dt), gs, bits)
    assert wq.shape == (2, 3, 5, 32) and s.shape == (2, 3, 5, 4)
    want = oracle.quantize(w, dt, gs, bits)
    for g, x in zip((wq, s, b), want):
        assert np.array_equal(host(g), x)
    # kh_dequantize of the result equals the oracle's dequantize of its own
    # quantization, bit for bit
    d = ops.dequantize(wq, s, b, gs, bits)
    assert np.array_equal(host(d), oracle.dequantize(*want, dt, gs, bits, dt))


@pytest.mark.gpu
def test_quantize_feeds_quantized_matmul(oracle):
    gs, bits, dt = 64, 4, "bf16"
    w = _quant_input(oracle, 512, 1024, gs, dt, seed=5)
    wq, s, b = ops.quantize(dev(w, dt), gs, bits)
    x = oracle.from_f32(np.random.default_rng(6).standard_normal((3, 1024)).astype(np.float32), "bf16")
    y = host(ops.quantized_matmul(dev(x, "bf16"), wq, s, b, True, gs, bits))
    ref = oracle.quantized_matmul(x, "bf16", host(wq), host(s), host(b), dt, gs, bits, True, "bf16")
    yf, rf = oracle.to_f32(y, "bf16"), oracle.to_f32(ref, "bf16")
    assert np.abs(yf - rf).max() <= 2e-2 * np.abs(rf).max()


@pytest.mark.gpu
def test_quantize_full_gate_shape(oracle):
    """BASELINE's gate shape 14336 x 4096, bf16 -> 4-bit gs64: rows quantize
    independently, so a sample of rows is checked bit-exact against the oracle,
    and every row against the round-trip bound."""
    N, K, gs, bits = 14336, 4096, 64, 4
    g = torch.Generator(device="cuda").manual_seed(3)
    w = (torch.randn((N, K), generator=g, device="cuda") * 0.02).bfloat16()
    wq, s, b = ops.quantize(w, gs, bits)
    rows = np.random.default_rng(4).choice(N, 64, replace=False)
    sel = torch.from_numpy(rows).cuda()
    want = oracle.quantize(host(w[sel]), "bf16", gs, bits)
    for got, x in zip((wq[sel], s[sel], b[sel]), want):
        assert np.array_equal(host(got), x)
    # round trip on the device: |dequant - w| <= |s| (half a step plus the
    # bounded clipping of the far extreme) plus bf16 rounding of s and b
    d = ops.dequantize(wq, s, b, gs, bits, out_dtype="f32")
    err = (d - w.float()).abs().view(N, K // gs, gs)
    sa = s.float().abs().unsqueeze(-1)
    mag = w.float().abs().view(N, K // gs, gs).amax(-1, keepdim=True)
    assert bool((err <= sa * 1.01 + 2.0 ** -8 * (15 * sa + mag)).all())


@pytest.mark.gpu
@pytest.mark.parametrize("bits,gs,odt", [(4, 64, "f32"), (8, 128, "bf16"), (4, 32, "f16")])
def test_gemm_partial_last_round_runs_half_tiles(oracle, bits, gs, odt):
    """17 column tiles x 16 row tiles of 128 = 272 tiles on 256 CUs: the last
    16 run as half-width workgroups in a second launch. Rows there must match
    the oracle and, bit for bit, the same rows computed by the full-width
    kernel (x's last 128 rows repeat its first 128)."""
    print(f"case gemm tail bits={bits} gs={gs} odt={odt}", flush=True)
    M, N, K = 2048, 17 * 256, 256
    L, x = _case(M, N, K, gs, bits, seed=31 + bits)
    x[-128:] = x[:128]
    y = _run(L, x, gs, bits, "bf16", "f16", odt)
    assert np.array_equal(y[-128:], y[:128])
    if odt == "f32":
        _check_f32(oracle, L, x, gs, bits, "bf16", "f16", y)
    else:
        ref = oracle.quantized_matmul(x, "bf16", L["w"], L["scales"], L["biases"], "f16", gs, bits, True, odt)
        mx, mean = parity_metrics(oracle.to_f32(y, odt), oracle.to_f32(ref, odt))
        assert mx <= 2e-2 and mean <= 1e-3


@pytest.mark.gpu
def test_quantize_unaligned_input(oracle):
    gs, bits = 32, 8
    w = _quant_input(oracle, 6, 128, gs, "bf16", seed=9)
    flat = torch.empty(w.size + 1, dtype=torch.bfloat16, device="cuda")
    view = flat[1:].view(6, 128)                       # 2 bytes off 16-byte alignment
    view.copy_(dev(w, "bf16"))
    for g, x in zip(ops.quantize(view, gs, bits), oracle.quantize(w, "bf16", gs, bits)):
        assert np.array_equal(host(g), x)


@pytest.mark.gpu
@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 64), (4, 128), (8, 32), (8, 64), (8, 128)])
@pytest.mark.parametrize("xdt", ["bf16", "f16"])
def test_skinny_kernel_exact(oracle, bits, gs, xdt):
    """The small-batch MFMA kernel (5 <= M <= 32, K % 128 == 0) keeps every
    dequantised weight exact: ragged N, one piece (K = 128, one wave), odd
    piece counts per wave (K = 896), one and two m-tiles, the 8-bit bf16
    nibble-split operands. Narrow shapes take it from M = 9 (below, the
    decode GEMV fills the chip better); M = 5 and 8 run on wide ones."""
    cases = [(N, K, M) for N, K in ((37, 128), (272, 896), (50, 4096)) for M in (13, 16, 17, 32)]
    cases += [(N, K, M) for N, K in ((16390, 128), (2360, 896), (2050, 4096)) for M in (5, 8)]
    for N, K, M in cases:
        print(f"case skinny bits={bits} gs={gs} xdt={xdt} N={N} K={K} M={M}", flush=True)
        assert decode_regime(M, K, bits, N, gs)[0] == "skinny"
        L, x = _case(M, N, K, gs, bits, xdt=xdt, seed=M + N + K + bits)
        y = _run(L, x, gs, bits, xdt, "f16", "f32")
        _check_f32(oracle, L, x, gs, bits, xdt, "f16", y, rel=EXACT_REL)


@pytest.mark.parametrize("odt", [torch.bfloat16, torch.float32])
def test_split_k_reduction_widths_agree(odt):
    """The split-K reduction serves four outputs per thread where the output
    is aligned for 4-element stores and the reduction is large (the
    Llama-3-8B gate shape at M = 64), one otherwise: both sum every output's
    slices in slice order, so an output buffer shifted by one element (one
    output per thread) holds the same bits."""
    from kiln_amd.workloads import make_linear_device
    M, N, K, gs = 64, 14336, 4096, 64
    plan = ops.quantized_matmul_plan(M, N, K, gs, 4)
    assert plan.startswith("gemm") and "nsplit=1 " not in plan, plan
    print(f"case split-K widths {plan} {odt}", flush=True)
    L = make_linear_device(N, K, gs, "q4", seed=5, device=torch.device("cuda"))
    x = torch.randn((M, K), generator=torch.Generator(device="cuda").manual_seed(6), device="cuda").bfloat16()
    a = torch.empty((M, N), dtype=odt, device="cuda")
    big = torch.empty(M * N + 1, dtype=odt, device="cuda")
    b = big[1:].view(M, N)
    ops.quantized_matmul(x, L["w"], L["scales"], L["biases"], True, gs, 4, out=a)
    ops.quantized_matmul(x, L["w"], L["scales"], L["biases"], True, gs, 4, out=b)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
