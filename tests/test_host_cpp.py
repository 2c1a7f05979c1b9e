"""The C++ host layer (kiln_amd/host, driven by tests/cpp/kiln_host_run.cpp):
safetensors loading (single file and sharded index, weights.rs:45-106),
config validation (config.rs:137-148, 735-760), Linear (nn.rs:51-114) with
its bias add, the gated Mlp (nn.rs:259-294, silu and gelu_approx), Embedding lookup and tied head (nn.rs:116-194), and the row
stability probe (nn.rs:301-327) — checked against the CPU oracle."""
import json
import os
import subprocess

import numpy as np
import pytest

from kiln_amd.workloads import make_linear_numpy, make_x_numpy

from _util import decode_regime

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RUNNER = os.path.join(ROOT, "kiln_amd", "kiln_host_run")


def _run(*args, timeout=120):
    r = subprocess.run([RUNNER, *args], capture_output=True, text=True, timeout=timeout)
    line = r.stdout.strip().splitlines()[-1] if r.stdout.strip() else "{}"
    return r.returncode, json.loads(line), r.stderr


def test_selftest_without_gpu():
    if not os.path.exists(RUNNER):
        pytest.skip("host test driver not built")
    rc, out, err = _run("selftest")
    assert rc == 0 and out["ok"], err


def _checkpoint(tmp_path, sharded):
    from safetensors.numpy import save_file
    gs, bits = 64, 4
    lin = make_linear_numpy(96, 256, gs, "q4", seed=31)
    emb = make_linear_numpy(200, 256, gs, "emb", seed=32)
    bias = (np.random.default_rng(33).standard_normal(96) * 0.1).astype(np.float16)
    tensors = {
        "model.layers.0.mlp.gate_proj.weight": lin["w"],
        "model.layers.0.mlp.gate_proj.scales": lin["scales"].view(np.float16),
        "model.layers.0.mlp.gate_proj.biases": lin["biases"].view(np.float16),
        "model.layers.0.mlp.gate_proj.bias": bias,
        "model.embed_tokens.weight": emb["w"],
        "model.embed_tokens.scales": emb["scales"].view(np.float16),
        "model.embed_tokens.biases": emb["biases"].view(np.float16),
        "model.norm.weight": np.ones(256, dtype=np.float16),
    }
    d = tmp_path / ("sharded" if sharded else "single")
    d.mkdir()
    if sharded:
        names = sorted(tensors)
        a, b = names[: len(names) // 2], names[len(names) // 2:]
        save_file({k: tensors[k] for k in a}, str(d / "model-00001-of-00002.safetensors"))
        save_file({k: tensors[k] for k in b}, str(d / "model-00002-of-00002.safetensors"))
        wm = {k: "model-00001-of-00002.safetensors" for k in a}
        wm.update({k: "model-00002-of-00002.safetensors" for k in b})
        (d / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    else:
        save_file(tensors, str(d / "model.safetensors"))
    (d / "config.json").write_text(json.dumps({"model_type": "llama",
                                               "quantization": {"group_size": gs, "bits": bits}}))
    return d, lin, emb, bias


def _job(tmp_path, **kw):
    p = tmp_path / f"job_{kw['op']}.json"
    p.write_text(json.dumps(kw))
    return _run("job", str(p))


@pytest.mark.gpu
@pytest.mark.parametrize("sharded", [False, True])
def test_linear_embedding_head_from_checkpoint(oracle, tmp_path, sharded):
    d, lin, emb, bias = _checkpoint(tmp_path, sharded)
    rc, out, err = _job(tmp_path, model_dir=str(d), op="load", prefix="model.layers.0.mlp.gate_proj")
    assert rc == 0 and out["ok"], (out, err)
    assert (out["in"], out["out"], out["quantized"]) == (256, 96, True)
    assert "model.norm.weight" in out["remaining"] and "model.embed_tokens.weight" in out["remaining"]

    # Linear::forward = quantized_matmul(transpose=true) + bias (f16 x -> f16 y)
    x = make_x_numpy(5, 256, seed=34, xdt="f16")
    (tmp_path / "x.bin").write_bytes(x.tobytes())
    rc, out, err = _job(tmp_path, model_dir=str(d), op="linear", prefix="model.layers.0.mlp.gate_proj",
                        input=str(tmp_path / "x.bin"), input_shape=[5, 256], input_dtype="float16",
                        output=str(tmp_path / "y.bin"))
    assert rc == 0 and out["ok"], (out, err)
    assert out["shape"] == [5, 96] and out["dtype"] == "float16"
    y = np.frombuffer((tmp_path / "y.bin").read_bytes(), dtype=np.float16).astype(np.float64).reshape(5, 96)
    ref16 = oracle.quantized_matmul(x, "f16", lin["w"], lin["scales"], lin["biases"], "f16", 64, 4, True, "f16")
    ref = (oracle.to_f32(ref16, "f16") + bias.astype(np.float32)).astype(np.float16).astype(np.float64)
    assert np.max(np.abs(y - ref)) <= 2e-2 * np.max(np.abs(ref))
    assert np.mean(np.abs(y - ref)) <= 1e-3 * np.mean(np.abs(ref))

    # Embedding::lookup, bit-exact (gather + dequantize)
    ids = np.array([[0, 199, 7], [7, 3, 100]], dtype=np.uint32)
    (tmp_path / "ids.bin").write_bytes(ids.tobytes())
    rc, out, err = _job(tmp_path, model_dir=str(d), op="embed", prefix="model.embed_tokens",
                        input=str(tmp_path / "ids.bin"), input_shape=[2, 3], input_dtype="uint32",
                        output=str(tmp_path / "e.bin"))
    assert rc == 0 and out["ok"] and out["shape"] == [2, 3, 256], (out, err)
    e = np.frombuffer((tmp_path / "e.bin").read_bytes(), dtype=np.uint16).reshape(2, 3, 256)
    assert np.array_equal(e, oracle.embedding(ids, emb["w"], emb["scales"], emb["biases"], "f16", 64, 4, "f16"))

    # Embedding::as_linear (tied head), f16 hidden -> f16 logits
    h = make_x_numpy(3, 256, seed=35, xdt="f16")
    (tmp_path / "h.bin").write_bytes(h.tobytes())
    rc, out, err = _job(tmp_path, model_dir=str(d), op="as_linear", prefix="model.embed_tokens",
                        input=str(tmp_path / "h.bin"), input_shape=[1, 3, 256], input_dtype="float16",
                        output=str(tmp_path / "l.bin"))
    assert rc == 0 and out["ok"] and out["shape"] == [1, 3, 200], (out, err)
    lg = np.frombuffer((tmp_path / "l.bin").read_bytes(), dtype=np.float16).astype(np.float64).reshape(3, 200)
    lref = oracle.to_f32(oracle.quantized_matmul(h, "f16", emb["w"], emb["scales"], emb["biases"], "f16",
                                                 64, 4, True, "f16"), "f16").astype(np.float64)
    assert np.mean(np.abs(lg - lref)) <= 1e-3 * np.mean(np.abs(lref))

    # probe_row_stability: row 0 stays bit-identical while M stays within the
    # kernel that serves M = 1, and first diverges where another takes over
    base = make_x_numpy(1, 64, seed=36, xdt="f16")
    (tmp_path / "b.bin").write_bytes(base.tobytes())
    rc, out, err = _job(tmp_path, model_dir=str(d), op="probe", prefix="model.embed_tokens", k=256,
                        input=str(tmp_path / "b.bin"), input_shape=[1, 1, 64], input_dtype="float16")
    assert rc == 0 and out["ok"], (out, err)
    first = next(m for m in range(2, 300) if decode_regime(m, 256, 4, 200) != decode_regime(1, 256, 4, 200))
    assert out["m"] == first


@pytest.mark.gpu
def test_missing_quantization_block_is_an_error(tmp_path):
    d, *_ = _checkpoint(tmp_path, False)
    (d / "config.json").write_text(json.dumps({"model_type": "llama"}))
    rc, out, err = _job(tmp_path, model_dir=str(d), op="load", prefix="model.layers.0.mlp.gate_proj")
    assert rc == 2 and not out["ok"]
    assert "no quantization block" in out["error"]


@pytest.mark.gpu
def test_switch_linear_bias_broadcasts(oracle, tmp_path):
    """SwitchLinear's expert bias is added as y + expand_dims(bias[indices], -2)
    (moe.rs:166-172) with numpy broadcasting: x [2, 1, 4, K] against indices
    [2, 3] gives y [2, 3, 4, N], and each pair's bias row is broadcast over
    its 4 rows."""
    from safetensors.numpy import save_file
    E, N, K, gs = 4, 48, 256, 64
    Ls = [make_linear_numpy(N, K, gs, "q4", seed=90 + e) for e in range(E)]
    bias = (np.random.default_rng(91).standard_normal((E, N)) * 0.1).astype(np.float16)
    pre = "model.layers.0.mlp"
    t = {f"{pre}.switch_mlp.up_proj.weight": np.stack([L["w"] for L in Ls]),
         f"{pre}.switch_mlp.up_proj.scales": np.stack([L["scales"] for L in Ls]).view(np.float16),
         f"{pre}.switch_mlp.up_proj.biases": np.stack([L["biases"] for L in Ls]).view(np.float16),
         f"{pre}.switch_mlp.up_proj.bias": bias}
    d = tmp_path / "bc"
    d.mkdir()
    save_file(t, str(d / "model.safetensors"))
    (d / "config.json").write_text(json.dumps({"model_type": "olmoe",
                                               "quantization": {"group_size": gs, "bits": 4}}))
    ids = np.array([[0, 3, 1], [2, 2, 0]], dtype=np.uint32)
    x = make_x_numpy(8, K, seed=92, xdt="f16").reshape(2, 1, 4, K)
    (tmp_path / "x.bin").write_bytes(x.tobytes())
    (tmp_path / "ids.bin").write_bytes(ids.tobytes())
    rc, out, err = _job(tmp_path, model_dir=str(d), op="switch", prefix=pre, proj="up_proj", experts=E,
                        input=str(tmp_path / "x.bin"), input_shape=[2, 1, 4, K], input_dtype="float16",
                        ids=str(tmp_path / "ids.bin"), ids_shape=[2, 3], sorted=False,
                        output=str(tmp_path / "y.bin"))
    assert rc == 0 and out["ok"], (out, err)
    assert out["shape"] == [2, 3, 4, N] and out["dtype"] == "float16"
    y = np.frombuffer((tmp_path / "y.bin").read_bytes(), dtype=np.float16).astype(np.float64).reshape(2, 3, 4, N)
    for i in range(2):
        for j in range(3):
            e = int(ids[i, j])
            r16 = oracle.quantized_matmul(x[i, 0], "f16", Ls[e]["w"], Ls[e]["scales"], Ls[e]["biases"], "f16",
                                          gs, 4, True, "f16")
            ref = (oracle.to_f32(r16, "f16") + bias[e].astype(np.float32)).astype(np.float16).astype(np.float64)
            assert np.max(np.abs(y[i, j] - ref)) <= 2e-2 * np.max(np.abs(ref)), (i, j)


@pytest.mark.gpu
@pytest.mark.parametrize("form", ["per_expert", "stacked"])
@pytest.mark.parametrize("P", [6, 80])
def test_switch_linear_from_checkpoint(oracle, tmp_path, form, P):
    """nn::SwitchLinear (moe.rs:47-176): experts stacked at load from
    `experts.{e}.{proj}` or taken as `switch_mlp.{proj}`, then x @ W[ids]^T
    (+ bias[ids]) through gather_qmm; each row against the oracle on its
    expert. P = 6 pairs run pair by pair, P = 80 through the grouped GEMM."""
    from safetensors.numpy import save_file
    E, N, K, gs = 4, 48, 256, 64
    Ls = [make_linear_numpy(N, K, gs, "q4", seed=60 + e) for e in range(E)]
    bias = (np.random.default_rng(61).standard_normal((E, N)) * 0.1).astype(np.float16)
    pre = "model.layers.0.mlp"
    t = {}
    if form == "stacked":
        t[f"{pre}.switch_mlp.up_proj.weight"] = np.stack([L["w"] for L in Ls])
        t[f"{pre}.switch_mlp.up_proj.scales"] = np.stack([L["scales"] for L in Ls]).view(np.float16)
        t[f"{pre}.switch_mlp.up_proj.biases"] = np.stack([L["biases"] for L in Ls]).view(np.float16)
        t[f"{pre}.switch_mlp.up_proj.bias"] = bias
    else:
        for e, L in enumerate(Ls):
            t[f"{pre}.experts.{e}.up_proj.weight"] = L["w"]
            t[f"{pre}.experts.{e}.up_proj.scales"] = L["scales"].view(np.float16)
            t[f"{pre}.experts.{e}.up_proj.biases"] = L["biases"].view(np.float16)
            t[f"{pre}.experts.{e}.up_proj.bias"] = bias[e]
    d = tmp_path / form
    d.mkdir()
    save_file(t, str(d / "model.safetensors"))
    (d / "config.json").write_text(json.dumps({"model_type": "olmoe",
                                               "quantization": {"group_size": gs, "bits": 4}}))
    ids = np.sort(np.random.default_rng(62).integers(0, E, P)).astype(np.uint32)
    x = make_x_numpy(P, K, seed=63, xdt="f16")
    (tmp_path / "x.bin").write_bytes(x.tobytes())
    (tmp_path / "ids.bin").write_bytes(ids.tobytes())
    rc, out, err = _job(tmp_path, model_dir=str(d), op="switch", prefix=pre, proj="up_proj", experts=E,
                        input=str(tmp_path / "x.bin"), input_shape=[P, 1, K], input_dtype="float16",
                        ids=str(tmp_path / "ids.bin"), ids_shape=[P], sorted=True,
                        output=str(tmp_path / "y.bin"))
    assert rc == 0 and out["ok"], (out, err)
    assert out["shape"] == [P, 1, N] and out["dtype"] == "float16"
    y = np.frombuffer((tmp_path / "y.bin").read_bytes(), dtype=np.float16).astype(np.float64).reshape(P, N)
    for p in range(P):
        e = int(ids[p])
        r16 = oracle.quantized_matmul(x[p:p + 1], "f16", Ls[e]["w"], Ls[e]["scales"], Ls[e]["biases"], "f16",
                                      gs, 4, True, "f16")
        ref = (oracle.to_f32(r16, "f16") + bias[e].astype(np.float32)).astype(np.float16).astype(np.float64)[0]
        assert np.max(np.abs(y[p] - ref)) <= 2e-2 * np.max(np.abs(ref)), p


@pytest.mark.gpu
@pytest.mark.parametrize("act", ["silu", "gelu_approx"])
@pytest.mark.parametrize("M", [1, 40])
def test_mlp_from_checkpoint(oracle, tmp_path, act, M):
    """nn::Mlp (nn.rs:259-294): down(act(gate(x) + b_g) * (up(x) + b_u)) + b_d
    with mlp_bias-style biases, the gate/up half in one kh_mlp_gate_up call;
    against the oracle's per-op composition (Linear::forward = matmul then
    bias; the activation with every intermediate in float16)."""
    from safetensors.numpy import save_file
    H, I, gs = 256, 192, 64
    pre = "model.layers.0.mlp"
    Ls = {p: make_linear_numpy(n, k, gs, "q4", seed=70 + i) for i, (p, n, k) in
          enumerate((("gate_proj", I, H), ("up_proj", I, H), ("down_proj", H, I)))}
    rng = np.random.default_rng(74)
    bias = {p: (rng.standard_normal(n) * 0.1).astype(np.float16) for p, n in
            (("gate_proj", I), ("up_proj", I), ("down_proj", H))}
    t = {}
    for p, L in Ls.items():
        t[f"{pre}.{p}.weight"] = L["w"]
        t[f"{pre}.{p}.scales"] = L["scales"].view(np.float16)
        t[f"{pre}.{p}.biases"] = L["biases"].view(np.float16)
        t[f"{pre}.{p}.bias"] = bias[p]
    d = tmp_path / "mlp"
    d.mkdir()
    save_file(t, str(d / "model.safetensors"))
    (d / "config.json").write_text(json.dumps({"model_type": "gemma2",
                                               "quantization": {"group_size": gs, "bits": 4}}))
    x = make_x_numpy(M, H, seed=75, xdt="f16")
    (tmp_path / "x.bin").write_bytes(x.tobytes())
    rc, out, err = _job(tmp_path, model_dir=str(d), op="mlp", prefix=pre, activation=act,
                        input=str(tmp_path / "x.bin"), input_shape=[1, M, H], input_dtype="float16",
                        output=str(tmp_path / "y.bin"))
    assert rc == 0 and out["ok"], (out, err)
    assert out["shape"] == [1, M, H] and out["dtype"] == "float16"
    y = np.frombuffer((tmp_path / "y.bin").read_bytes(), dtype=np.uint16).reshape(M, H)

    def lin(p, v):
        L = Ls[p]
        r, _ = oracle.linear(v, "f16", L["w"], L["scales"], L["biases"], "f16", gs, 4,
                             bias[p].view(np.uint16), "f16")
        return r
    fn = oracle.gelu_mul if act == "gelu_approx" else oracle.silu_mul
    ref = lin("down_proj", fn(lin("gate_proj", x), lin("up_proj", x), "f16"))
    yf, rf = oracle.to_f32(y, "f16").astype(np.float64), oracle.to_f32(ref, "f16").astype(np.float64)
    assert np.max(np.abs(yf - rf)) <= 2e-2 * np.max(np.abs(rf))
    assert np.mean(np.abs(yf - rf)) <= 1e-3 * np.mean(np.abs(rf))


@pytest.mark.gpu
def test_large_sharded_checkpoint_is_streamed(tmp_path):
    """WeightStore::from_model_dir maps each shard read-only and uploads it
    through a bounded pinned staging buffer (weights.rs:76 maps shards the same
    way, io.rs:22-30): loading a 1.2 GB checkpoint in two 600 MB shards raises
    the process's peak resident memory by far less than one shard, and every
    tensor arrives intact (hashes of its first and last 4 KiB)."""
    from safetensors.numpy import save_file
    rng = np.random.default_rng(5)
    d = tmp_path / "big"
    d.mkdir()
    wm, want = {}, {}
    per = 150 * 2 ** 20 // 4  # uint32 words per tensor
    for sh in range(2):
        fname = f"model-{sh + 1:05d}-of-00002.safetensors"
        t = {}
        for i in range(4):
            name = f"model.layers.{sh * 4 + i}.mlp.up_proj.weight"
            t[name] = rng.integers(0, 2 ** 32, size=(per // 4096, 4096), dtype=np.uint32)
            wm[name] = fname
        name = f"model.layers.{sh}.input_layernorm.weight"
        t[name] = rng.standard_normal(4096).astype(np.float16)
        wm[name] = fname
        for name, a in t.items():
            b = a.tobytes()
            k = min(len(b), 4096)
            h = 1469598103934665603
            for c in b[:k] + b[len(b) - k:]:
                h = ((h ^ c) * 1099511628211) % 2 ** 64
            want[name] = str(h)
        save_file(t, str(d / fname))
        del t
    (d / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    (d / "config.json").write_text(json.dumps({"model_type": "llama"}))
    shard = max(os.path.getsize(d / f) for f in set(wm.values()))
    assert shard > 600 * 2 ** 20
    rc, out, err = _job(tmp_path, model_dir=str(d), op="load_all", prefix="")
    assert rc == 0 and out["ok"], (out, err)
    assert out["hashes"] == want
    grew = (out["hwm_after_kib"] - out["rss_before_kib"]) * 1024
    print(f"peak resident growth {grew / 2 ** 20:.0f} MiB, shard {shard / 2 ** 20:.0f} MiB")
    assert grew <= 256 * 2 ** 20, grew   # two 32 MiB staging buffers and the mapped window
