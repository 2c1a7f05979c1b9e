"""Benchmark of the affine-quantized linear path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-sweep]

Headline (the JSON line's `value`): BASELINE configs[2], the seven
Llama-3-8B decoder linears (q/k/v/o 4096x4096|1024x4096, gate/up
14336x4096, down 4096x14336), 4-bit codes, group size 64, fp16
scales/biases, bf16 activations ~N(0,1), bf16 output, random-init
(synthetic) weights generated in HBM. A step is one decode pass of one
layer: the seven quantized_matmul calls at M = 1 through the C ABI
(kh_quantized_matmul), replayed from a HIP graph. Steps rotate over enough
distinct layer copies (> 512 MB) that the 256 MB MALL cannot serve the
weights: every call reads its weights from HBM.

value    = whole-step algorithmic bytes / step time (GB/s), bytes per call
           N*K*bits/8 + 2*N*(K/gs)*2 + M*K*2 + M*N*2.
roofline = the dominant kernel (decode GEMV at gate 14336x4096): its
           algorithmic bytes per launch / its average launch duration, from
           HIP events on the stream the library launches on.
sweep    = every BASELINE configuration: per-layer (or per-call) time, GB/s
           and TFLOP/s for each M the configuration lists.
cpu_baseline = the oracle's C restatement (OpenMP, float32 accumulate) on
           the host cores over the same M = 1 step, for about --cpu-seconds.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of `bench.py --profile traffic`:
# 16,212.5 KiB read x 1.99976 + 56 KiB written, per launch of the gate GEMV
GATE_TRAFFIC_BYTES = 33_289_353
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
MALL_BYTES = 600_000_000  # rotate over more distinct weight bytes than the 256 MB MALL


def call_bytes(N, K, M, bits, gs):
    """Algorithmic bytes of one call: packed codes + 16-bit scales and
    biases + bf16 activations + bf16 output."""
    return N * K * bits // 8 + 2 * N * (K // gs) * 2 + M * K * 2 + M * N * 2


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--m", type=int, default=None, help="batch rows of --profile decode|fused|qwen|head")
    ap.add_argument("--gs", type=int, default=None, help="group size of --profile qwen (32 or 128)")
    ap.add_argument("--profile", choices=["decode", "decode8", "fused", "prefill", "traffic", "moe", "qwen", "head",
                                          "embed"], default=None,
                    help="run one workload for a profiler and exit (no JSON line): the M=1 decode "
                         "step, the M=2048 Llama-3-8B layer, or a copy of known size followed by "
                         "gate-shape GEMV launches (counter calibration)")
    args = ap.parse_args()
    if args.steps < 1 or args.warmup < 0:
        ap.error("--steps must be >= 1 and --warmup >= 0")
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build runs the quantized linear path on a "
              f"single MI355X and has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from kiln_amd import ops
    from kiln_amd.workloads import LAYER_SHAPES, make_linear_device

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    g = torch.Generator(device=dev).manual_seed(7)

    def layer_copies(shapes, gs, dist, copies=None):
        bits = 4 if dist != "q8" else 8
        per = sum(N * K * bits // 8 for _, N, K in shapes)
        copies = copies or max(2, -(-MALL_BYTES // per))
        return [{name: make_linear_device(N, K, gs, dist, seed=1000 * c + i, device=dev)
                 for i, (name, N, K) in enumerate(shapes)} for c in range(copies)]

    def graph_us(fn, copies, reps):
        """Average µs of fn(c) over a graph holding fn(0..copies-1), replayed
        `reps` times; HIP events on the capture/replay stream. Untimed
        replays first (at least 5) bring the clocks back up after the host
        work of the capture."""
        for c in range(copies):
            fn(c)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for c in range(copies):
                fn(c)
        for _ in range(max(5, reps // 4)):
            graph.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        us = 1e3 * e0.elapsed_time(e1) / (reps * copies)
        del graph
        return us

    def layer_fns(layers, shapes, M, gs, bits):
        xs = {K: torch.randn((M, K), generator=g, device=dev).bfloat16() for _, _, K in shapes}
        outs = {name: torch.empty((M, N), dtype=torch.bfloat16, device=dev) for name, N, _ in shapes}

        def one(name, K):
            def f(c):
                W = layers[c][name]
                ops.quantized_matmul(xs[K], W["w"], W["scales"], W["biases"], True, gs, bits,
                                     out=outs[name])
            return f

        per = {name: one(name, K) for name, _, K in shapes}

        def step(c):
            for name, _, _ in shapes:
                per[name](c)
        return step, per

    if args.profile in ("qwen", "head", "embed"):
        profile_other(args.profile, torch, ops, layer_copies, layer_fns, dev, args.m or 1, args.gs or 32)
        return

    # ---------------- headline: Llama-3-8B decode step at M = 1
    gs, bits = 64, 4
    shapes = LAYER_SHAPES["llama-3-8b"]
    layers = layer_copies(shapes, gs, "q4")
    copies = len(layers)
    if args.profile:
        profile_run(args.profile, torch, ops, layers, shapes, layer_fns, dev, gs, bits, args.m)
        return
    step, per = layer_fns(layers, shapes, 1, gs, bits)
    step_us = timed_steps_us(torch, step, copies, args.steps, args.warmup, stream)
    nsteps = args.steps
    step_bytes = sum(call_bytes(N, K, 1, bits, gs) for _, N, K in shapes)
    value = step_bytes / (step_us * 1e-6) / 1e9
    per_shape_us = {name: graph_us(per[name], copies, 50) for name, _, _ in shapes}
    dN, dK = next((N, K) for n, N, K in shapes if n == "gate")
    dom_us = per_shape_us["gate"]
    dom_bytes = call_bytes(dN, dK, 1, bits, gs)
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9

    reps = max(1, -(-args.steps // copies))
    rot_us = graph_us(step, copies, reps)  # the same step, one graph of `copies` steps replayed
    fused = fused_step(torch, ops, layers, shapes, graph_us, dev, g, gs, bits, copies, reps)

    sweep = {} if args.no_sweep else run_sweep(torch, ops, layers, shapes, graph_us, layer_fns,
                                               layer_copies, make_linear_device, dev, g)

    cpu = None if args.no_cpu else cpu_baseline(shapes, gs, bits, args.cpu_seconds)

    line = {
        "metric": "q4 GEMV HBM GB/s (% of peak) at M=1; dequant-GEMM TFLOP/s at M=2048",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": nsteps,
        "warmup": args.warmup,
        "ms_per_step": round(step_us * 1e-3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 codes, bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded random codes/scales/biases in HBM, x ~ N(0,1))",
        "config": {"workload": "llama-3-8b decoder linears (q,k,v,o,gate,up,down), 4-bit gs64, M=1 "
                               "decode step (BASELINE configs[2])",
                   "m": 1, "group_size": gs, "bits": bits, "weight_copies": copies,
                   "weight_bytes_rotated": copies * sum(N * K // 2 for _, N, K in shapes)},
        "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     # HBM bytes per gate launch, FETCH_SIZE + WRITE_SIZE scaled by
                     # what they read for a 256 MiB copy (x1.99976 and x1.0), from
                     # the `--profile traffic` runs summarised in profiles/
                     "traffic": GATE_TRAFFIC_BYTES,
                     "traffic_source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of bench.py --profile "
                                       "traffic (profiles/gemv_traffic_llama3-8b_gate_m1.md)",
                     "kernel": "gemv_kernel<4,bf16,f16,M=1,R=4,I=1> at gate 14336x4096",
                     "bytes_per_launch": dom_bytes, "avg_launch_us": round(dom_us, 3)},
        "step_us_rotating_graph": round(rot_us, 3),
        "per_shape_us": {k: round(v, 2) for k, v in per_shape_us.items()},
        "per_shape_gbs": {n: round(call_bytes(N, K, 1, bits, gs) / (per_shape_us[n] * 1e-6) / 1e9, 1)
                          for n, N, K in shapes},
        "fused_step": fused,
        "prefill_m2048_tflops": sweep.get("llama-3-8b", {}).get("prefill", {}).get("2048", {}).get("tflops"),
        "sweep": sweep,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def timed_steps_us(torch, step, copies, steps, warmup, stream):
    """Average µs per step over exactly `steps` decode steps, after exactly
    `warmup` untimed ones. Each run is one HIP graph holding that many steps,
    step i on weight copy i % copies; HIP events on the replay stream, with a
    device synchronisation on both sides of the timed replay."""
    for c in range(copies):  # eager once per copy: every plan's workspace exists
        step(c)
    torch.cuda.synchronize()

    def capture(n):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(n):
                step(i % copies)
        return graph

    timed = capture(steps)
    if warmup:
        warm = capture(warmup)
        warm.replay()
        del warm
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    timed.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return 1e3 * e0.elapsed_time(e1) / steps


def profile_run(kind, torch, ops, layers, shapes, layer_fns, dev, gs, bits, m=None):
    """Workloads for rocprofv3 (kernel trace or counters), eager launches."""
    if kind == "decode":
        step, _ = layer_fns(layers, shapes, m or 1, gs, bits)
        for r in range(4 * len(layers)):
            step(r % len(layers))
    elif kind == "fused":
        # the layer through the fused entry points (q|k|v, gate_up) at M rows
        g = torch.Generator(device=dev)
        g.manual_seed(7)
        step, _ = fused_fns(torch, ops, layers, shapes, dev, g, gs, bits, m or 1)
        for r in range(4 * len(layers)):
            step(r % len(layers))
    elif kind == "decode8":
        # small-batch decode: the 7 linears at M = 8 over the rotated copies
        step, _ = layer_fns(layers, shapes, 8, gs, bits)
        for r in range(4 * len(layers)):
            step(r % len(layers))
    elif kind == "prefill":
        step, _ = layer_fns(layers[:2], shapes, 2048, gs, bits)
        for r in range(6):
            step(r % 2)
    elif kind == "moe":
        # gather_qmm as SwitchGlu issues it at prefill: OLMoE experts (E=64,
        # top-8), T = 2048 tokens -> 16384 one-row pairs sorted by expert,
        # gate/up shape then down shape, 5 calls each
        from kiln_amd.workloads import make_linear_device
        E, k, T = 64, 8, 2048
        g = torch.Generator(device=dev)
        g.manual_seed(T)
        ids = torch.stack([torch.randperm(E, device=dev, generator=g)[:k] for _ in range(T)]).to(torch.int32)
        order = torch.argsort(ids.reshape(-1), stable=True)
        idx = ids.reshape(-1)[order].contiguous()
        for Ne, Ke in ((1024, 2048), (2048, 1024)):
            Ls = [make_linear_device(Ne, Ke, 64, "q4", seed=e) for e in range(E)]
            we = torch.stack([L["w"] for L in Ls])
            se = torch.stack([L["scales"] for L in Ls])
            be = torch.stack([L["biases"] for L in Ls])
            del Ls
            xt = torch.randn((T, Ke), device=dev, generator=g).bfloat16()
            xg = xt[order // k].reshape(T * k, 1, Ke).contiguous()
            ye = torch.empty((T * k, 1, Ne), dtype=torch.bfloat16, device=dev)
            for _ in range(5):
                ops.gather_qmm(xg, we, se, be, idx, True, 64, 4, True, out=ye)
    else:
        # a device-to-device copy of 256 MiB (reads and writes exactly that
        # much: the calibration of FETCH_SIZE / WRITE_SIZE), then 12 launches
        # of the gate-shape GEMV over distinct weight copies
        a = torch.empty(64 << 20, dtype=torch.int32, device=dev).random_()
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        b.copy_(a)
        torch.cuda.synchronize()
        N, K = next((N, K) for n, N, K in shapes if n == "gate")
        x = torch.randn((1, K), device=dev).bfloat16()
        y = torch.empty((1, N), dtype=torch.bfloat16, device=dev)
        for r in range(12):
            W = layers[r % len(layers)]["gate"]
            ops.quantized_matmul(x, W["w"], W["scales"], W["biases"], True, gs, bits, out=y)
    torch.cuda.synchronize()


def profile_other(kind, torch, ops, layer_copies, layer_fns, dev, m, gs):
    """Workloads for rocprofv3 beyond the Llama-3-8B layer, eager launches over
    weight copies beyond the MALL: the Qwen2.5-7B 8-bit layer (group size gs)
    at M rows, the tied 128256x4096 gs128 LM head at M rows, and the
    embedding gather of 4096 Zipf ids."""
    from kiln_amd.workloads import LAYER_SHAPES
    if kind == "qwen":
        shapes = LAYER_SHAPES["qwen2.5-7b"]
        layers = layer_copies(shapes, gs, "q8")
        step, _ = layer_fns(layers, shapes, m, gs, 8)
    else:
        shapes = [("head", 128256, 4096)]
        layers = layer_copies(shapes, 128, "emb")
        if kind == "head":
            step, _ = layer_fns(layers, shapes, m, 128, 4)
        else:
            import numpy as np
            rng = np.random.default_rng(4000)
            ids = []
            while len(ids) < 4096:
                z = rng.zipf(1.1, 8192) - 1
                ids.extend(int(v) for v in z[z < 128256])
            idt = torch.tensor(ids[:4096], dtype=torch.int32, device=dev)
            eo = torch.empty((4096, 4096), dtype=torch.bfloat16, device=dev)

            def step(c):
                W = layers[c]["head"]
                ops.quantized_embedding(idt, W["w"], W["scales"], W["biases"], 128, 4, out=eo)
    for r in range(4 * len(layers)):
        step(r % len(layers))
    torch.cuda.synchronize()


def fused_fns(torch, ops, layers, shapes, dev, g, gs, bits, M=1):
    """The layer (M rows) through the fused entry points: q|k|v in one
    kh_quantized_matmul_multi call, o, silu(gate)*up in one
    kh_quantized_gate_up call, down. Returns (step(copy index), algorithmic
    bytes of one step: x counted once per call, the one activation output)."""
    Ns = {n: (N, K) for n, N, K in shapes}
    x = torch.randn((M, Ns["q"][1]), generator=g, device=dev).bfloat16()
    xd = torch.randn((M, Ns["down"][1]), generator=g, device=dev).bfloat16()
    qkv = [torch.empty((M, Ns[n][0]), dtype=torch.bfloat16, device=dev) for n in ("q", "k", "v")]
    o = torch.empty((M, Ns["o"][0]), dtype=torch.bfloat16, device=dev)
    act = torch.empty((M, Ns["gate"][0]), dtype=torch.bfloat16, device=dev)
    y = torch.empty((M, Ns["down"][0]), dtype=torch.bfloat16, device=dev)

    def step(c):
        L = layers[c]
        W = lambda n: (L[n]["w"], L[n]["scales"], L[n]["biases"])
        ops.quantized_matmul_multi(x, [W("q"), W("k"), W("v")], True, gs, bits, outs=qkv)
        ops.quantized_matmul(x, *W("o"), True, gs, bits, out=o)
        ops.quantized_gate_up(x, W("gate"), W("up"), gs, bits, out=act)
        ops.quantized_matmul(xd, *W("down"), True, gs, bits, out=y)

    wb = lambda n: Ns[n][0] * Ns[n][1] * bits // 8 + 2 * Ns[n][0] * (Ns[n][1] // gs) * 2
    nbytes = (sum(wb(n) for n in ("q", "k", "v", "o", "gate", "up", "down")) + 3 * 2 * M * Ns["q"][1]
              + 2 * M * Ns["down"][1]
              + 2 * M * (sum(Ns[n][0] for n in ("q", "k", "v", "o", "down")) + Ns["gate"][0]))
    return step, nbytes


def fused_step(torch, ops, layers, shapes, graph_us, dev, g, gs, bits, copies, reps, M=1):
    """Graph-replayed time of the fused layer of fused_fns (4 calls)."""
    step, nbytes = fused_fns(torch, ops, layers, shapes, dev, g, gs, bits, M)
    us = graph_us(step, copies, reps)
    return {"us": round(us, 2), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1), "calls": 4,
            "bytes": nbytes}


def run_sweep(torch, ops, l8_layers, l8_shapes, graph_us, layer_fns, layer_copies, make_linear_device,
              dev, g):
    """Every BASELINE configuration, one entry per M; per-layer figures sum the
    seven linears of one layer, replayed from a graph over > 512 MB of weights."""
    from kiln_amd.workloads import LAYER_SHAPES

    def entry(shapes, M, gs, bits, us):
        b = sum(call_bytes(N, K, M, bits, gs) for _, N, K in shapes)
        f = sum(2 * M * N * K for _, N, K in shapes)
        return {"us": round(us, 2), "gbs": round(b / (us * 1e-6) / 1e9, 1),
                "tflops": round(f / (us * 1e-6) / 1e12, 2)}

    def measure(layers, shapes, Ms, gs, bits, reps_for):
        res = {}
        for M in Ms:
            step, _ = layer_fns(layers, shapes, M, gs, bits)
            us = graph_us(step, len(layers), reps_for(M))
            res[str(M)] = entry(shapes, M, gs, bits, us)
            print(f"# sweep {shapes[0][1]}x{shapes[0][2]}.. M={M}: {res[str(M)]}", file=sys.stderr,
                  flush=True)
        return res

    out = {}
    # Llama-3-8B, decode M in {1,8,32,64}, prefill M in {512,2048,4096}
    out["llama-3-8b"] = {"decode": measure(l8_layers, l8_shapes, (1, 8, 32, 64), 64, 4, lambda M: 20),
                         "prefill": measure(l8_layers[:2], l8_shapes, (512, 2048, 4096), 64, 4,
                                            lambda M: 3)}
    out["llama-3-8b"]["decode_fused"] = {
        str(M): fused_step(torch, ops, l8_layers, l8_shapes, graph_us, dev, g, 64, 4, len(l8_layers), 20, M)
        for M in (1, 8, 32, 64)}
    print(f"# sweep fused decode: {out['llama-3-8b']['decode_fused']}", file=sys.stderr, flush=True)
    pf = out["llama-3-8b"]["prefill"]["2048"]
    pf["frac_of_bf16_peak"] = round(pf["tflops"] / BF16_PEAK_TFLOPS, 4)

    # one 8192x2048 matvec
    s0 = [("w", 8192, 2048)]
    L0 = layer_copies(s0, 64, "q4", copies=80)
    out["cfg0-8192x2048"] = measure(L0, s0, (1,), 64, 4, lambda M: 20)
    del L0

    # Llama-3.2-1B, M in {1,4,16,32}, per layer and x16 layers
    s1 = LAYER_SHAPES["llama-3.2-1b"]
    L1 = layer_copies(s1, 64, "q4")
    r1 = measure(L1, s1, (1, 4, 16, 32), 64, 4, lambda M: 20)
    for v in r1.values():
        v["us_16_layers"] = round(16 * v["us"], 1)
    out["llama-3.2-1b"] = r1
    del L1

    # Qwen2.5-7B 8-bit, gs 32 and 128, M in {1,16,2048}
    s3 = LAYER_SHAPES["qwen2.5-7b"]
    for gs3 in (32, 128):
        L3 = layer_copies(s3, gs3, "q8")
        r = measure(L3, s3, (1, 16), gs3, 8, lambda M: 10)
        r.update(measure(L3[:2], s3, (2048,), gs3, 8, lambda M: 3))
        out[f"qwen2.5-7b-q8-gs{gs3}"] = r
        del L3

    # tied head 128256x4096 4-bit gs128 at M in {1,32,256}; gather of 4096 Zipf ids
    s4 = [("head", 128256, 4096)]
    L4 = layer_copies(s4, 128, "emb")
    out["lm-head-128256x4096-gs128"] = measure(L4, s4, (1, 32, 256), 128, 4, lambda M: 10)
    import numpy as np
    rng = np.random.default_rng(4000)
    ids = []
    while len(ids) < 4096:
        z = rng.zipf(1.1, 8192) - 1
        ids.extend(int(v) for v in z[z < 128256])
    idt = torch.tensor(ids[:4096], dtype=torch.int32, device=dev).view(torch.int32)
    H, T = 4096, 4096
    eo = torch.empty((T, H), dtype=torch.bfloat16, device=dev)

    def gather(c):
        W = L4[c]["head"]
        ops.quantized_embedding(idt, W["w"], W["scales"], W["biases"], 128, 4, out=eo)

    us = graph_us(gather, len(L4), 20)
    eb = T * (H * 4 // 8 + 2 * (H // 128) * 2 + 2 * H) + 4 * T
    out["embedding-gather-4096-zipf"] = {"us": round(us, 2), "gbs": round(eb / (us * 1e-6) / 1e9, 1)}
    del L4

    # the affine quantizer (kh_quantize) on the gate shape, bf16 -> 4-bit gs64
    # (reads the bf16 matrix, writes codes, scales and biases)
    Nq, Kq = 14336, 4096
    wsrc = [(torch.randn((Nq, Kq), device=dev) * 0.02).bfloat16() for _ in range(2)]
    qo = [ops.quantize(w, 64, 4) for w in wsrc]
    lib = ops._lib.lib()

    def quant(c):
        wq, s, b = qo[c]
        ops._check(lib.kh_quantize(ops._desc(wq, "w_q", ops._lib.UINT32), ops._desc(s, "scales"),
                                   ops._desc(b, "biases"), ops._desc(wsrc[c], "w"), ops._lib.opt(64),
                                   ops._lib.opt(4), b"affine", ops._stream_handle(wsrc[c], None)))

    us = graph_us(quant, 2, 20)
    qb = Nq * Kq * 2 + Nq * Kq // 2 + 2 * Nq * (Kq // 64) * 2
    out["quantize-14336x4096-bf16-q4-gs64"] = {"us": round(us, 2), "gbs": round(qb / (us * 1e-6) / 1e9, 1)}
    del wsrc, qo

    # MoE expert dispatch (gather_qmm) as SwitchGlu issues it (moe.rs:272-310):
    # OLMoE experts (E=64, top-8, hidden 2048, intermediate 1024), 4-bit gs64,
    # T tokens -> T*8 one-row pairs sorted by expert; gate/up shape and down.
    E, k = 64, 8
    for name, Ne, Ke in (("gate", 1024, 2048), ("down", 2048, 1024)):
        Ls = [make_linear_device(Ne, Ke, 64, "q4", seed=e) for e in range(E)]
        we = torch.stack([L["w"] for L in Ls])
        se = torch.stack([L["scales"] for L in Ls])
        be = torch.stack([L["biases"] for L in Ls])
        del Ls
        for T in (8, 128, 2048):
            g = torch.Generator(device=dev)
            g.manual_seed(T)
            ids = torch.stack([torch.randperm(E, device=dev, generator=g)[:k] for _ in range(T)]).to(torch.int32)
            order = torch.argsort(ids.reshape(-1), stable=True)
            xt = torch.randn((T, Ke), device=dev, generator=g).bfloat16()
            xg = xt[order // k].reshape(T * k, 1, Ke).contiguous()
            idx = ids.reshape(-1)[order].contiguous()
            ye = torch.empty((T * k, 1, Ne), dtype=torch.bfloat16, device=dev)
            us = graph_us(lambda c: ops.gather_qmm(xg, we, se, be, idx, True, 64, 4, True, out=ye), 1, 20)
            touched = int(torch.unique(idx).numel())
            gb = touched * call_bytes(Ne, Ke, 0, 4, 64) + T * k * (Ke + Ne) * 2
            out[f"olmoe-gather_qmm-{name}-{Ne}x{Ke}-T{T}"] = {
                "us": round(us, 2), "tflops": round(2 * T * k * Ne * Ke / (us * 1e-6) / 1e12, 2),
                "gbs": round(gb / (us * 1e-6) / 1e9, 1), "experts_touched": touched}
        del we, se, be
    return out


def cpu_baseline(shapes, gs, bits, seconds):
    """The oracle's C restatement (OpenMP, float32 accumulate) over the same
    decode step on host cores, repeated for about `seconds`."""
    from kiln_amd.workloads import make_linear_numpy, make_x_numpy
    from oracle import oracle

    data = []
    for i, (name, N, K) in enumerate(shapes):
        L = make_linear_numpy(N, K, gs, "q4", seed=i)
        data.append((N, K, L, make_x_numpy(1, K, seed=i)))
    nbytes = 0
    reps = 0
    t0 = time.perf_counter()
    while True:
        for N, K, L, x in data:
            oracle.quantized_matmul(x, "bf16", L["w"], L["scales"], L["biases"], "f16", gs, bits, True, "bf16")
            nbytes += call_bytes(N, K, 1, bits, gs)
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": int(oracle.lib().kho_threads()),
            "kind": "port",
            "sample": f"{reps} x the 7-linear M=1 decode step (same shapes), oracle/kh_oracle.c kho_qmm, "
                      f"{dt:.1f} s"}


if __name__ == "__main__":
    main()
