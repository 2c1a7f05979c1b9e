"""Seeded synthetic workloads of the benchmark configurations.

Distributions follow the five configurations the benchmark is quoted on:
  q4   4-bit codes U{0..15}; scales U[0.004, 0.02]; biases = -8*scale + N(0, 1e-3)
  q8   8-bit codes U{0..255}; scales U[2e-4, 1e-3]; biases = -128*scale
  emb  4-bit codes U{0..15}; scales U[0.004, 0.02]; biases = -8*scale
Scales and biases are float16; activations bf16 ~ N(0, 1).

Layer shapes (out x in) of the decoder linears in each configuration are in
LAYER_SHAPES. `make_linear_numpy` builds small cases on the CPU (numpy, for
parity tests); `make_linear_device` builds full-size cases directly in HBM
with torch's generator (benchmark inputs), packing with the same layout.
"""
from __future__ import annotations

import numpy as np

DISTS = {
    "q4": dict(bits=4, smin=0.004, smax=0.02, zero=8.0, noise=1e-3),
    "q8": dict(bits=8, smin=2e-4, smax=1e-3, zero=128.0, noise=0.0),
    "emb": dict(bits=4, smin=0.004, smax=0.02, zero=8.0, noise=0.0),
}

LAYER_SHAPES = {
    "llama-3.2-1b": [("q", 2048, 2048), ("k", 512, 2048), ("v", 512, 2048), ("o", 2048, 2048),
                     ("gate", 8192, 2048), ("up", 8192, 2048), ("down", 2048, 8192)],
    "llama-3-8b": [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
                   ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)],
    "qwen2.5-7b": [("q", 3584, 3584), ("k", 512, 3584), ("v", 512, 3584), ("o", 3584, 3584),
                   ("gate", 18944, 3584), ("up", 18944, 3584), ("down", 3584, 18944)],
}


def pack_numpy(codes: np.ndarray, bits: int) -> np.ndarray:
    per = 32 // bits
    c = codes.astype(np.uint32).reshape(*codes.shape[:-1], codes.shape[-1] // per, per)
    shifts = np.arange(per, dtype=np.uint32) * np.uint32(bits)
    return np.bitwise_or.reduce(c << shifts, axis=-1).astype(np.uint32)


def make_linear_numpy(N: int, K: int, gs: int, dist: str = "q4", seed: int = 0,
                      sdt: str = "f16"):
    """Return dict(codes, w, scales, biases) as numpy; scales/biases are
    uint16 bit patterns of sdt ('f16' | 'bf16') or float32 for 'f32'."""
    d = DISTS[dist]
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 1 << d["bits"], (N, K), dtype=np.uint8)
    s = rng.uniform(d["smin"], d["smax"], (N, K // gs)).astype(np.float32)
    b = -d["zero"] * s
    if d["noise"]:
        b = b + rng.normal(0, d["noise"], s.shape).astype(np.float32)
    if sdt == "f16":
        s16, b16 = s.astype(np.float16), b.astype(np.float16)
        sc, bi = s16.view(np.uint16), b16.view(np.uint16)
    elif sdt == "bf16":
        import torch
        sc = torch.from_numpy(s).bfloat16().view(torch.int16).numpy().view(np.uint16)
        bi = torch.from_numpy(b.astype(np.float32)).bfloat16().view(torch.int16).numpy().view(np.uint16)
    else:
        sc, bi = s, b.astype(np.float32)
    return dict(codes=codes, w=pack_numpy(codes, d["bits"]), scales=np.ascontiguousarray(sc),
                biases=np.ascontiguousarray(bi), bits=d["bits"])


def make_x_numpy(M: int, K: int, seed: int = 1, xdt: str = "bf16") -> np.ndarray:
    """Activations ~ N(0,1) as bf16/f16 bit patterns (uint16) or f32."""
    import torch
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    if xdt == "f32":
        return x.numpy()
    t = x.bfloat16() if xdt == "bf16" else x.half()
    return t.view(torch.int16).numpy().view(np.uint16)


def make_linear_device(N: int, K: int, gs: int, dist: str = "q4", seed: int = 0,
                       device="cuda", sdt=None):
    """Full-size weights generated in HBM: w int32 [N, K*bits/32] (uint32 bits),
    scales/biases float16 [N, K/gs]."""
    import torch
    d = DISTS[dist]
    sdt = sdt or torch.float16
    g = torch.Generator(device=device).manual_seed(seed)
    bits = d["bits"]
    per = 32 // bits
    words = torch.zeros((N, K // per), dtype=torch.int64, device=device)
    for j in range(per):
        c = torch.randint(0, 1 << bits, (N, K // per), generator=g, device=device, dtype=torch.int64)
        words |= c << (bits * j)
    w = torch.where(words >= (1 << 31), words - (1 << 32), words).to(torch.int32)
    s = torch.empty((N, K // gs), device=device, dtype=torch.float32).uniform_(d["smin"], d["smax"], generator=g)
    b = -d["zero"] * s
    if d["noise"]:
        b = b + torch.randn(s.shape, generator=g, device=device) * d["noise"]
    return dict(w=w.contiguous(), scales=s.to(sdt).contiguous(), biases=b.to(sdt).contiguous(), bits=bits)
