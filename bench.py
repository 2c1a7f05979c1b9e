"""Benchmark of the affine-quantized linear path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--workload llama-3-8b]

Workload: the seven Llama-3-8B decoder linears
(q/k/v/o 4096x4096|1024x4096, gate/up 14336x4096, down 4096x14336), 4-bit
codes, group size 64, fp16 scales/biases, bf16 activations ~N(0,1), bf16
output, random-init (synthetic) weights generated in HBM.

A step is one decode pass of one layer: the seven quantized_matmul calls at
M = 1, each through the C ABI (kh_quantized_matmul). Steps rotate over
enough distinct layer copies (> 512 MB) that the 256 MB MALL cannot serve
the weights; every call reads its weights from HBM.

value = whole-step algorithmic bytes / step time (GB/s) at M = 1.
roofline = the dominant kernel (the decode GEMV at gate/up shape): algorithmic
bytes per launch / its average launch duration, measured with HIP events on
the stream the library launches on.
Also reported: prefill (M = 2048) dequant-GEMM TFLOP/s over the seven
linears, and the CPU baseline (the oracle's C restatement, OpenMP).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def layer_bytes(N, K, M, bits=4, gs=64):
    """Algorithmic bytes of one call: packed codes + fp16 scales and biases +
    bf16 activations + bf16 output."""
    return N * K * bits // 8 + 2 * N * (K // gs) * 2 + M * K * 2 + M * N * 2


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="llama-3-8b")
    ap.add_argument("--prefill-m", type=int, default=2048)
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    args = ap.parse_args()
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
    gs, bits = 64, 4
    shapes = LAYER_SHAPES[args.workload]
    per_layer = sum(N * K // 2 for _, N, K in shapes)
    copies = max(2, -(-600_000_000 // per_layer))  # > 512 MB of distinct weights
    layers = []
    for c in range(copies):
        layers.append({name: make_linear_device(N, K, gs, "q4", seed=1000 * c + i, device=dev)
                       for i, (name, N, K) in enumerate(shapes)})
    g = torch.Generator(device=dev).manual_seed(7)
    xs = {K: torch.randn((1, K), generator=g, device=dev).bfloat16() for _, _, K in shapes}
    outs = {name: torch.empty((1, N), dtype=torch.bfloat16, device=dev) for name, N, _ in shapes}
    stream = torch.cuda.current_stream(dev)

    def step(i):
        L = layers[i % copies]
        for name, N, K in shapes:
            W = L[name]
            ops.quantized_matmul(xs[K], W["w"], W["scales"], W["biases"], True, gs, bits,
                                 out=outs[name])

    def capture(fn):
        """Record fn's launches (made on torch's current stream, which is the
        capture stream inside the context) into a HIP graph."""
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        return graph

    # Eager warm-up, then one graph holding `copies` decode steps (one per
    # weight copy) so a replay walks > 512 MB of distinct weights.
    for i in range(copies):
        step(i)
    torch.cuda.synchronize()
    g_step = capture(lambda: [step(i) for i in range(copies)])
    reps = max(1, -(-args.steps // copies))
    wreps = max(1, -(-args.warmup // copies))
    for _ in range(wreps):
        g_step.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        g_step.replay()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    nsteps = reps * copies
    ms_per_step = wall * 1e3 / nsteps
    step_bytes = sum(layer_bytes(N, K, 1, bits, gs) for _, N, K in shapes)
    value = step_bytes / (wall / nsteps) / 1e9

    # Per-launch duration of each shape: a graph of that shape's launches over
    # every weight copy, bracketed by HIP events recorded on the replay stream.
    stream = torch.cuda.current_stream(dev)
    per_shape_us = {}
    for name, N, K in shapes:
        def one_shape(name=name, K=K):
            for i in range(copies):
                W = layers[i][name]
                ops.quantized_matmul(xs[K], W["w"], W["scales"], W["biases"], True, gs, bits,
                                     out=outs[name])
        gr = capture(one_shape)
        gr.replay()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        nrep = 20
        e0.record(stream)
        for _ in range(nrep):
            gr.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        per_shape_us[name] = 1e3 * e0.elapsed_time(e1) / (nrep * copies)
    dom = "gate"
    dN, dK = next((N, K) for n, N, K in shapes if n == dom)
    dom_us = per_shape_us[dom]
    dom_bytes = layer_bytes(dN, dK, 1, bits, gs)
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9
    per_shape_gbs = {n: round(layer_bytes(N, K, 1, bits, gs) / (per_shape_us[n] * 1e-6) / 1e9, 1)
                     for n, N, K in shapes}
    per_shape_us = {n: round(v, 2) for n, v in per_shape_us.items()}

    # Prefill: the seven linears at M = prefill_m, MFMA dequant-GEMM path.
    Mp = args.prefill_m
    xp = {K: torch.randn((Mp, K), generator=g, device=dev).bfloat16() for _, _, K in shapes}
    op = {name: torch.empty((Mp, N), dtype=torch.bfloat16, device=dev) for name, N, _ in shapes}

    def pstep(i, events=None):
        L = layers[i % copies]
        for name, N, K in shapes:
            W = L[name]
            if events is not None:
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record(stream)
            ops.quantized_matmul(xp[K], W["w"], W["scales"], W["biases"], True, gs, bits,
                                 out=op[name])
            if events is not None:
                e1.record(stream)
                events.append((name, e0, e1))

    for i in range(2):
        pstep(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.prefill_steps):
        pstep(i)
    torch.cuda.synchronize()
    pwall = (time.perf_counter() - t0) / args.prefill_steps
    flops = sum(2 * Mp * N * K for _, N, K in shapes)
    pevents = []
    for i in range(args.prefill_steps):
        pstep(i, pevents)
    torch.cuda.synchronize()
    pgate = [e0.elapsed_time(e1) for n, e0, e1 in pevents if n == dom]
    pgate_ms = sum(pgate) / len(pgate)
    prefill = {
        "m": Mp,
        "tflops": round(flops / pwall / 1e12, 1),
        "ms_per_layer": round(pwall * 1e3, 3),
        "gate_tflops": round(2 * Mp * dN * dK / (pgate_ms * 1e-3) / 1e12, 1),
        "gate_us": round(pgate_ms * 1e3, 1),
        "frac_of_bf16_peak": round(flops / pwall / 1e12 / BF16_PEAK_TFLOPS, 4),
    }

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(shapes, gs, bits, args.cpu_seconds)

    line = {
        "metric": "q4 GEMV HBM GB/s (% of peak) at M=1; dequant-GEMM TFLOP/s at M=2048",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": nsteps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 codes, bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded random codes/scales/biases in HBM, x ~ N(0,1))",
        "config": {"workload": f"{args.workload} decoder linears (q,k,v,o,gate,up,down), 4-bit gs64, M=1 decode step",
                   "m": 1, "group_size": gs, "bits": bits, "weight_copies": copies,
                   "weight_bytes_rotated": copies * per_layer},
        "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "qmv_kernel<4,64,bf16,1> at gate 14336x4096",
                     "bytes_per_launch": dom_bytes, "avg_launch_us": round(dom_us, 3)},
        "per_shape_us": per_shape_us,
        "per_shape_gbs": per_shape_gbs,
        "prefill": prefill,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def cpu_baseline(shapes, gs, bits, seconds):
    """The oracle's C restatement (OpenMP, float32 accumulate) over the same
    decode step on host cores, repeated for about `seconds`."""
    import numpy as np

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
            nbytes += layer_bytes(N, K, 1, bits, gs)
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    del np
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": int(oracle.lib().kho_threads()),
            "kind": "port",
            "sample": f"{reps} x the 7-linear M=1 decode step (same shapes), oracle/kh_oracle.c kho_qmm, "
                      f"{dt:.1f} s"}


if __name__ == "__main__":
    main()
