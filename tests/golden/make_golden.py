#!/usr/bin/env python3
"""Writes tests/golden/golden.json: known-answer vectors for the MLX affine
quantized format, produced WITHOUT the C oracle or the HIP library.

Nothing in the reference tree pins this path (it holds no quantized-matmul
fixture), so every vector here comes from an independent formulation:

* bitstreams: Python big-integer concatenation  stream = sum(c_i << bits*i),
  words = 32-bit slices of that integer (the layout implied by
  `model/3模块/模型加载-通用.swift:178-185` and the LSB-first shifts of
  `model/minimax h3/H3Common.swift:389-394`);
* bf16 rounding: exact rational arithmetic (fractions.Fraction), nearest
  representable value, ties to the even mantissa;
* generator: splitmix64 + Box-Muller written with Python ints and `math`;
* quantizer (min/max recipe): numpy float32 scalar arithmetic, plus grid
  inputs w = b0 + s0*q whose codes are known a priori;
* matmul: numpy float64 matmul of exactly dequantized weights s*q + b.

Run:  python tests/golden/make_golden.py   (deterministic; rewrites the file)
"""
import json
import math
import os
import random
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
MASK64 = (1 << 64) - 1
GAMMA = 0x9E3779B97F4A7C15


# --------------------------------------------------------------------------
# generator: splitmix64 stream, i-th output = mix(seed + (i+1)*gamma)
# --------------------------------------------------------------------------
def sm_mix(z):
    z &= MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def splitmix_outputs(seed, count):
    state = seed & MASK64
    out = []
    for _ in range(count):
        state = (state + GAMMA) & MASK64
        out.append(sm_mix(state))
    return out


def normals(seed, n, mean, std):
    raw = splitmix_outputs(seed, 2 * ((n + 1) // 2))
    vals = []
    for p in range(0, len(raw), 2):
        u1 = ((raw[p] >> 11) + 1) * (1.0 / 9007199254740992.0)
        u2 = (raw[p + 1] >> 11) * (1.0 / 9007199254740992.0)
        r = math.sqrt(-2.0 * math.log(u1))
        t = 6.283185307179586 * u2
        vals.append(mean + std * (r * math.cos(t)))
        vals.append(mean + std * (r * math.sin(t)))
    return vals[:n]


# --------------------------------------------------------------------------
# bf16 by exact rationals
# --------------------------------------------------------------------------
def bf16_value(bits16):
    """Exact value of a finite bf16 bit pattern as a Fraction."""
    s = -1 if bits16 & 0x8000 else 1
    e = (bits16 >> 7) & 0xFF
    m = bits16 & 0x7F
    if e == 0:
        return s * Fraction(m, 128) * Fraction(2) ** -126
    return s * (1 + Fraction(m, 128)) * Fraction(2) ** (e - 127)


def f32_round(x):
    """Python float (fp64) -> nearest fp32 value, as a Python float."""
    return float(np.float32(x))


def bf16_rne(x):
    """fp32 value x (Python float) -> bf16 bits, nearest, ties to even."""
    if math.isnan(x):
        raise ValueError("nan")
    if math.isinf(x):
        return 0x7F80 if x > 0 else 0xFF80
    sign = 0x8000 if (x < 0 or (x == 0 and math.copysign(1, x) < 0)) else 0
    a = Fraction(abs(x))
    if a == 0:
        return sign
    # candidates: all finite positive bf16 patterns around a
    e = max(min(math.floor(math.log2(a)), 127), -133) if a > 0 else 0
    cands = []
    for ee in (e - 1, e, e + 1):
        biased = ee + 127
        if biased <= 0:
            for m in range(128):
                cands.append(m)
        elif biased < 255:
            for m in range(128):
                cands.append((biased << 7) | m)
    cands = sorted(set(cands))
    best = min(cands, key=lambda b: (abs(bf16_value(b) - a), b & 1))
    # overflow: beyond the largest finite bf16 by at least half an ulp -> inf
    maxf = bf16_value(0x7F7F)
    if a >= maxf + (maxf - bf16_value(0x7F7E)) / 2:
        return sign | 0x7F80
    return sign | best


# --------------------------------------------------------------------------
# bitstream by big-integer concatenation
# --------------------------------------------------------------------------
def pack_row(codes, bits):
    stream = 0
    for i, c in enumerate(codes):
        stream |= (int(c) & ((1 << bits) - 1)) << (bits * i)
    nwords = len(codes) * bits // 32
    return [(stream >> (32 * w)) & 0xFFFFFFFF for w in range(nwords)]


def pack(codes2d, bits):
    return [pack_row(r, bits) for r in codes2d]


# --------------------------------------------------------------------------
# quantizer, min/max recipe, numpy float32 scalars
# --------------------------------------------------------------------------
def quantize_minmax(w, gs, bits):
    w = np.asarray(w, dtype=np.float32)
    N, K = w.shape
    nmax = np.float32((1 << bits) - 1)
    codes = np.zeros((N, K), dtype=np.int64)
    s_f32 = np.zeros((N, K // gs), dtype=np.float32)
    b_f32 = np.zeros((N, K // gs), dtype=np.float32)
    for n in range(N):
        for g in range(K // gs):
            grp = w[n, g * gs:(g + 1) * gs]
            mn, mx = grp.min(), grp.max()
            s = np.float32(mx - mn) / nmax
            if mx == mn:
                s = np.float32(1e-7)
            b = mn
            q = np.rint((grp - b) / s)
            q = np.clip(q, np.float32(0), nmax)
            codes[n, g * gs:(g + 1) * gs] = q.astype(np.int64)
            s_f32[n, g] = s
            b_f32[n, g] = b
    return codes, s_f32, b_f32


def main():
    out = {"format": 1}

    # ---- generator goldens ------------------------------------------------
    gen = []
    for seed, n, mean, std in [(0, 9, 0.0, 1.0), (1000, 8, 0.0, 1.0),
                               (2003, 7, 0.0, 0.02), (123456789, 6, 1.5, 3.0)]:
        vals = normals(seed, n, mean, std)
        gen.append({
            "seed": seed, "n": n, "mean": mean, "std": std,
            "f32": [f32_round(v) for v in vals],
            "bf16": [bf16_rne(f32_round(v)) for v in vals],
            "splitmix": [str(v) for v in splitmix_outputs(seed, 4)],
        })
    out["generator"] = gen

    # ---- bf16 rounding: closed-form corner cases ----------------------------
    cases = [1.0, -1.0, 0.0, -0.0, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8,
             1.0 + 2.0 ** -8 + 2.0 ** -20, 1.0 - 2.0 ** -9, 255.5, 256.0 + 1.0,
             3.0e38, -3.4028234663852886e38, 1.0e-40, 2.0 ** -126, 0.1, -0.3,
             65504.0, 1.0 / 3.0, float("inf"), float("-inf")]
    out["bf16"] = [{"f32": f32_round(c) if math.isfinite(c) else c,
                    "bits": bf16_rne(f32_round(c) if math.isfinite(c) else c)}
                   for c in cases]
    # json cannot hold inf; store as strings
    for e in out["bf16"]:
        if not math.isfinite(e["f32"]):
            e["f32"] = "inf" if e["f32"] > 0 else "-inf"

    # ---- packing ------------------------------------------------------------
    packs = []
    rng = random.Random(20240601)
    for bits in (2, 3, 4, 5, 6, 8):
        K = 64 if bits != 5 and bits != 3 else 64
        ramp = [[i % (1 << bits) for i in range(K)]]
        packs.append({"bits": bits, "N": 1, "K": K, "codes": ramp,
                      "words": pack(ramp, bits), "kind": "ramp"})
        N, K = 3, 128
        rnd = [[rng.randrange(1 << bits) for _ in range(K)] for _ in range(N)]
        packs.append({"bits": bits, "N": N, "K": K, "codes": rnd,
                      "words": pack(rnd, bits), "kind": "random"})
        allmax = [[(1 << bits) - 1] * 32]
        packs.append({"bits": bits, "N": 1, "K": 32, "codes": allmax,
                      "words": pack(allmax, bits), "kind": "all_ones"})
    out["pack"] = packs

    # ---- quantizer (min/max recipe) -----------------------------------------
    quants = []
    for (bits, gs, N, K, seed) in [(4, 64, 2, 128, 11), (6, 64, 2, 128, 12),
                                   (6, 32, 2, 96, 13), (4, 128, 1, 256, 14),
                                   (8, 64, 1, 64, 15), (2, 32, 2, 64, 16),
                                   (3, 32, 1, 64, 17), (5, 64, 1, 128, 18)]:
        w = np.array(normals(seed, N * K, 0.0, 0.02), dtype=np.float32).reshape(N, K)
        codes, s, b = quantize_minmax(w, gs, bits)
        quants.append({
            "bits": bits, "gs": gs, "N": N, "K": K, "kind": "normal",
            "w": [float(v) for v in w.ravel()],
            "codes": codes.ravel().tolist(),
            "scales_f32": [float(v) for v in s.ravel()],
            "biases_f32": [float(v) for v in b.ravel()],
            "scales_bf16": [bf16_rne(float(v)) for v in s.ravel()],
            "biases_bf16": [bf16_rne(float(v)) for v in b.ravel()],
        })
    # grid inputs: w = b0 + s0*q exactly, with 0 and 2^b-1 present in each group,
    # so min/max recovers s0, b0 and the codes are q (known a priori).
    gr = random.Random(777)
    for bits, gs in [(4, 64), (6, 64), (6, 32), (8, 128)]:
        N, K = 2, 2 * gs
        nmax = (1 << bits) - 1
        q = [[gr.randrange(nmax + 1) for _ in range(K)] for _ in range(N)]
        for n in range(N):
            for g in range(K // gs):
                q[n][g * gs] = 0
                q[n][g * gs + 1] = nmax
        s0 = [[2.0 ** -(gr.randrange(6, 12)) for _ in range(K // gs)] for _ in range(N)]
        b0 = [[-gr.randrange(1, 64) * 2.0 ** -8 for _ in range(K // gs)] for _ in range(N)]
        w = [[b0[n][k // gs] + s0[n][k // gs] * q[n][k] for k in range(K)] for n in range(N)]
        quants.append({
            "bits": bits, "gs": gs, "N": N, "K": K, "kind": "grid",
            "w": [v for r in w for v in r],
            "codes": [v for r in q for v in r],
            "scales_f32": [v for r in s0 for v in r],
            "biases_f32": [v for r in b0 for v in r],
            "scales_bf16": [bf16_rne(v) for r in s0 for v in r],
            "biases_bf16": [bf16_rne(v) for r in b0 for v in r],
        })
    out["quantize"] = quants

    # ---- matmul: fp64 numpy on exactly dequantized weights ------------------
    mms = []
    for (bits, gs, M, N, K, seed, with_bias) in [
            (6, 64, 3, 8, 128, 31, False), (4, 64, 2, 16, 256, 32, True),
            (6, 32, 5, 4, 96, 33, True), (4, 128, 1, 8, 256, 34, False),
            (8, 64, 2, 4, 128, 35, False), (2, 32, 2, 4, 64, 36, False),
            (3, 32, 2, 4, 64, 37, True), (5, 64, 2, 4, 128, 38, False)]:
        nmax = (1 << bits) - 1
        r = random.Random(seed)
        codes = [[r.randrange(nmax + 1) for _ in range(K)] for _ in range(N)]
        sb = [bf16_rne(f32_round(r.uniform(1e-3, 4e-3))) for _ in range(N * K // gs)]
        bb = [bf16_rne(f32_round(r.uniform(-0.1, 0.0))) for _ in range(N * K // gs)]
        xb = [bf16_rne(f32_round(v)) for v in normals(seed + 100, M * K, 0.0, 1.0)]
        bias = [bf16_rne(f32_round(r.uniform(-1, 1))) for _ in range(N)] if with_bias else None
        S = np.array([float(bf16_value(v)) for v in sb]).reshape(N, K // gs)
        B = np.array([float(bf16_value(v)) for v in bb]).reshape(N, K // gs)
        Q = np.array(codes, dtype=np.float64)
        Wd = Q * np.repeat(S, gs, axis=1) + np.repeat(B, gs, axis=1)  # exact in fp64
        X = np.array([float(bf16_value(v)) for v in xb]).reshape(M, K)
        Y = X @ Wd.T
        if bias is not None:
            Y = Y + np.array([float(bf16_value(v)) for v in bias])[None, :]
        mms.append({
            "bits": bits, "gs": gs, "M": M, "N": N, "K": K,
            "codes": [c for row in codes for c in row],
            "words": [w for row in pack(codes, bits) for w in row],
            "scales_bf16": sb, "biases_bf16": bb, "x_bf16": xb,
            "bias_bf16": bias, "y_f64": [float(v) for v in Y.ravel()],
        })
    out["qmm"] = mms

    path = os.path.join(HERE, "golden.json")
    with open(path, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
