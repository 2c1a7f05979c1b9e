"""Write the small golden fixtures in tests/golden/ (run: python tests/golden/make_golden.py).

The reference holds no op-level vectors for this path (its only fixtures are
end-to-end token ids that need real checkpoints and Metal), so these vectors
are computed here by brute force, independently of oracle/:

  * codes are drawn first and packed with plain Python integer arithmetic
    (code j of word i at bits [bits*j, bits*j+bits), the mlx-lm layout);
  * every dequantised weight and every matmul output is evaluated with exact
    rational arithmetic (fractions.Fraction) from the decoded f16/bf16/f32
    inputs, then rounded to float32 (and to bf16) by explicit
    round-half-to-even on the exact rational — no floating-point shortcut.

Each fixture stores the inputs, the exact dequantised values rounded once
to f32, the exact matmul result rounded once to f32 and to bf16, and the
embedding rows. Cases cover 4/8 bits, group sizes 32/64/128, f16/bf16
scales, and hand-picked edge codes (all-zero, all-max, ramps).
"""
from __future__ import annotations

import os
import struct
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f16_value(h: int) -> Fraction:
    s = -1 if h & 0x8000 else 1
    e = (h >> 10) & 0x1F
    m = h & 0x3FF
    if e == 0:
        return s * Fraction(m, 1 << 24)
    return s * Fraction(1024 + m, 1024) * (Fraction(2) ** (e - 15))


def bf16_value(h: int) -> Fraction:
    return Fraction(struct.unpack("<f", struct.pack("<I", h << 16))[0])


def round_to_binary(v: Fraction, man_bits: int, emin: int) -> Fraction:
    """Round-half-to-even of v to a binary format with man_bits fraction bits
    and minimum normal exponent emin (no overflow handling needed here)."""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    ulp = Fraction(2) ** (e - man_bits)
    q = a / ulp
    fl = q.numerator // q.denominator
    rem = q - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return sign * fl * ulp


def to_f32_bits(v: Fraction) -> int:
    r = round_to_binary(v, 23, -126)
    return struct.unpack("<I", struct.pack("<f", float(r)))[0]


def to_bf16_bits(v: Fraction) -> int:
    r = round_to_binary(v, 7, -126)
    return struct.unpack("<I", struct.pack("<f", float(r)))[0] >> 16


def pack_codes(codes, bits):
    per = 32 // bits
    words = []
    for i in range(0, len(codes), per):
        w = 0
        for j in range(per):
            w |= int(codes[i + j]) << (bits * j)
        words.append(w)
    return words


def f32_bits_to_value(u: int) -> Fraction:
    return Fraction(struct.unpack("<f", struct.pack("<I", u))[0])


def make_case(name, rng, M, N, K, bits, gs, sdt, special=None):
    qmax = (1 << bits) - 1
    codes = rng.integers(0, qmax + 1, (N, K))
    if special == "edges":
        codes[0, :] = 0
        codes[1, :] = qmax
        codes[2, :] = np.arange(K) % (qmax + 1)
        codes[3, :] = (np.arange(K) * 7 + 3) % (qmax + 1)
    G = K // gs
    if sdt == "f16":
        s_f = rng.uniform(0.004, 0.02, (N, G)).astype(np.float16)
        b_f = (-(qmax + 1) / 2 * s_f.astype(np.float32)
               + rng.normal(0, 1e-3, (N, G))).astype(np.float16)
        s_bits, b_bits = s_f.view(np.uint16), b_f.view(np.uint16)
        dec = f16_value
    else:
        s32 = rng.uniform(0.004, 0.02, (N, G)).astype(np.float32)
        b32 = (-(qmax + 1) / 2 * s32 + rng.normal(0, 1e-3, (N, G))).astype(np.float32)
        s_bits = (s32.view(np.uint32) >> 16).astype(np.uint16)
        b_bits = (b32.view(np.uint32) >> 16).astype(np.uint16)
        dec = bf16_value
    if special == "edges":
        s_bits[4 % N, 0] = 0          # zero scale: the group is the bias
    x32 = rng.standard_normal((M, K)).astype(np.float32)
    x_bits = (x32.view(np.uint32) >> 16).astype(np.uint16)   # truncation to bf16 is fine for inputs

    w_words = np.array([pack_codes(codes[n], bits) for n in range(N)], dtype=np.uint32)
    Wq = [[dec(int(s_bits[n, k // gs])) * int(codes[n, k]) + dec(int(b_bits[n, k // gs]))
           for k in range(K)] for n in range(N)]
    # dequantised weights rounded once to f32 (the dequant rule)
    deq_f32 = np.array([[to_f32_bits(v) for v in row] for row in Wq], dtype=np.uint32)
    deq_bf16 = np.array([[to_bf16_bits(v) for v in row] for row in Wq], dtype=np.uint16)
    xv = [[bf16_value(int(x_bits[m, k])) for k in range(K)] for m in range(M)]
    # matmul against the f32-rounded weights, exact sum
    Wr = [[f32_bits_to_value(int(deq_f32[n, k])) for k in range(K)] for n in range(N)]
    y_exact = [[sum(xv[m][k] * Wr[n][k] for k in range(K)) for n in range(N)] for m in range(M)]
    y_f32 = np.array([[to_f32_bits(v) for v in row] for row in y_exact], dtype=np.uint32)
    y_bf16 = np.array([[to_bf16_bits(v) for v in row] for row in y_exact], dtype=np.uint16)
    ids = rng.integers(0, N, (7,)).astype(np.uint32)
    np.savez_compressed(
        os.path.join(HERE, f"{name}.npz"),
        bits=bits, gs=gs, sdt=sdt, codes=codes.astype(np.uint8), w=w_words, scales=s_bits,
        biases=b_bits, x=x_bits, deq_f32=deq_f32, deq_bf16=deq_bf16, y_f32=y_f32, y_bf16=y_bf16,
        ids=ids, emb_bf16=deq_bf16[ids.astype(np.int64)])


def main():
    rng = np.random.default_rng(20261201)
    make_case("q4_gs32_f16", rng, 3, 8, 64, 4, 32, "f16", special="edges")
    make_case("q4_gs64_bf16", rng, 2, 6, 128, 4, 64, "bf16", special="edges")
    make_case("q4_gs128_f16", rng, 2, 5, 256, 4, 128, "f16")
    make_case("q8_gs32_bf16", rng, 2, 6, 64, 8, 32, "bf16", special="edges")
    make_case("q8_gs64_f16", rng, 3, 5, 128, 8, 64, "f16")
    make_case("q8_gs128_bf16", rng, 2, 4, 256, 8, 128, "bf16")
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
