"""Run the hardware-ceiling probes on cuda:0 and print one JSON object.

    python -m kiln_amd.probes.run

- launch_floor_us: an empty kernel's time per launch inside a HIP graph of
  200 launches (the fixed cost every kernel of a decode step pays);
- stream_read: a plain one-pass read at the sizes of the benchmark's
  launches (cfg0 9.4 MB, a Llama-3-8B gate 33 MB, twice that, the 279 MB LM
  head, 600 MB), each replayed over enough distinct buffers (> 600 MB) that
  the 256 MB MALL cannot serve them: us per launch and GB/s;
- mfma: independent v_mfma_f32_16x16x32_f16 chains (and 32x32x16 chains) at
  one and two waves per SIMD on all 256 CUs: TFLOP/s against the 2.5 PFLOP/s
  dense fp16 peak.
"""
from __future__ import annotations

import ctypes
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libkh_probes.so")


def main():
    import torch

    if not os.path.exists(LIB):
        raise RuntimeError(f"{LIB} is missing: build it first (python -m kiln_amd.build)")
    L = ctypes.CDLL(LIB)
    L.kp_empty.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    L.kp_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    L.kp_mfma.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    out = torch.zeros(512 * 256, dtype=torch.float32, device=dev)
    st = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def graph_us(fn, n, reps=5):
        fn(0)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n):
                fn(i)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return 1e3 * e0.elapsed_time(e1) / (reps * n)

    res = {}
    res["launch_floor_us"] = round(graph_us(lambda i: L.kp_empty(ctypes.c_void_p(out.data_ptr()), st()), 200), 3)

    reads = {}
    for mb in (9.457664, 33.067008, 66.134016, 279.347, 600.0):
        nbytes = int(mb * 1e6) // 16 * 16
        copies = max(2, -(-600_000_000 // nbytes))
        bufs = [torch.empty(nbytes // 4, dtype=torch.int32, device=dev).random_() for _ in range(copies)]
        us = graph_us(lambda i: L.kp_stream_read(ctypes.c_void_p(bufs[i % copies].data_ptr()), nbytes,
                                                 ctypes.c_void_p(out.data_ptr()), st()), copies * 4)
        reads[f"{mb:.1f}MB"] = {"us": round(us, 3), "gbs": round(nbytes / us / 1e3, 1),
                                "frac_of_8TBs": round(nbytes / us / 1e3 / 8000, 4), "copies": copies}
        del bufs
    res["stream_read"] = reads

    L.kp_mfma32.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]

    def mfma_rate(fn, flops_per_wave_iter, iters=20000):
        r = {}
        for wgs in (256, 512, 1024):
            fn(ctypes.c_void_p(out.data_ptr()), wgs, 100, st())
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            assert fn(ctypes.c_void_p(out.data_ptr()), wgs, iters, st()) == 0
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1)
            tf = flops_per_wave_iter * iters * 4 * wgs / ms / 1e9
            r[f"{wgs // 256}_waves_per_simd"] = {"ms": round(ms, 3), "tflops": round(tf, 1),
                                                 "frac_of_2500": round(tf / 2500, 4)}
        return r

    res["mfma_f16_16x16x32"] = mfma_rate(L.kp_mfma, 2.0 * 16 * 16 * 32 * 8)      # 8 chains
    res["mfma_f16_32x32x16"] = mfma_rate(L.kp_mfma32, 2.0 * 32 * 32 * 16 * 4)     # 4 chains
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
