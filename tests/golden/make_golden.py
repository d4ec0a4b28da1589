"""Writes tests/golden/qmv_golden.json: exact answers for tiny qmv problems.

The reference ships no numeric golden vectors for this path (its qmv tests all need
MLX: ironmule tests/engine/test_cuda_native.py:57-67, tests/runtime/
test_qmv_k3840_integration.py:83-96).  These fixtures are computed here from the
format's definition alone, in exact rational arithmetic (`fractions.Fraction`), with
inputs drawn from Python's own `random` module — nothing from the oracle or the
product is imported, so the fixtures check both independently.

Definition used (ironmule/cuda_native.py:54-56, 91; ironmule/numeric_plans.py:450-452):
  q[n][k] = (w[n][k // 8] >> 4*(k % 8)) & 0xF          (low nibble first)
  W[n][k] = s[n][k // 64] * q[n][k] + b[n][k // 64]      (bf16 s, b)
  y[m][n] = sum_k W[n][k] * x[m][k]                      (exact)
Each fixture stores y exactly as a float64 (nearest) and as its correctly rounded
bf16 bit pattern, plus fl32 of every dequantised weight.

Run:  python tests/golden/make_golden.py   (deterministic; rewrites the JSON)
"""

from __future__ import annotations

import json
import math
import os
import random
import struct
from fractions import Fraction

GS = 64
HERE = os.path.dirname(os.path.abspath(__file__))


def bf16_value(h: int) -> Fraction:
    return Fraction(struct.unpack("<f", struct.pack("<I", h << 16))[0])


def round_to_bits(v: Fraction, mant_bits: int, min_exp: int, max_exp: int) -> Fraction:
    """Correctly rounded (nearest, ties to even) binary value with `mant_bits`
    fraction bits, normal exponent range [min_exp, max_exp]; subnormals kept."""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    # fix floating log error
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, min_exp)
    ulp = Fraction(2) ** (e - mant_bits)
    q = a / ulp
    fl = q.numerator // q.denominator
    rem = q - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    r = fl * ulp
    if r >= Fraction(2) ** (max_exp + 1):
        return Fraction(sign) * Fraction(10) ** 400  # overflow marker (not produced here)
    return sign * r


def to_bf16_bits(v: Fraction) -> int:
    r = round_to_bits(v, 7, -126, 127)
    f = float(r)
    return struct.unpack("<I", struct.pack("<f", f))[0] >> 16


def to_f32(v: Fraction) -> float:
    return float(round_to_bits(v, 23, -126, 127))


def bf16_bits_of(x: float) -> int:
    return to_bf16_bits(Fraction(x))


def problem(rng: random.Random, name: str, n: int, k: int, m: int, *, q_mode="random",
            s_mode="random", x_mode="normal") -> dict:
    words = []
    for _ in range(n):
        row = []
        for _ in range(k // 8):
            if q_mode == "random":
                row.append(rng.getrandbits(32))
            elif q_mode == "zero":
                row.append(0)
            elif q_mode == "max":
                row.append(0xFFFFFFFF)
            elif q_mode == "ramp":
                row.append(0x76543210 if rng.random() < 0.5 else 0xFEDCBA98)
        words.append(row)
    g = k // GS
    if s_mode == "random":
        s = [[bf16_bits_of(rng.uniform(0.005, 0.02)) for _ in range(g)] for _ in range(n)]
    elif s_mode == "zero":
        s = [[0 for _ in range(g)] for _ in range(n)]
    b = [[bf16_bits_of(rng.uniform(-0.1, 0.1)) for _ in range(g)] for _ in range(n)]
    if x_mode == "normal":
        x = [[bf16_bits_of(rng.gauss(0.0, 1.0)) for _ in range(k)] for _ in range(m)]
    elif x_mode == "onehot":
        x = []
        for i in range(m):
            hot = rng.randrange(k)
            x.append([0x3F80 if j == hot else 0 for j in range(k)])
    elif x_mode == "wide":  # magnitudes spread over many binades
        x = [[bf16_bits_of(rng.choice([-1, 1]) * 2.0 ** rng.uniform(-20, 20)) for _ in range(k)]
             for _ in range(m)]
    q = [[(words[r][kk // 8] >> (4 * (kk % 8))) & 0xF for kk in range(k)] for r in range(n)]
    W = [[bf16_value(s[r][kk // GS]) * q[r][kk] + bf16_value(b[r][kk // GS]) for kk in range(k)]
         for r in range(n)]
    y = [[sum(W[r][kk] * bf16_value(x[mm][kk]) for kk in range(k)) for r in range(n)]
         for mm in range(m)]
    return {
        "name": name, "n": n, "k": k, "m": m,
        "w": [[f"{u:08x}" for u in row] for row in words],
        "scales": s, "biases": b, "x": x,
        "dequant_f32": [[to_f32(v) for v in row] for row in W],
        "y_f64": [[float(v) for v in row] for row in y],
        "y_bf16": [[to_bf16_bits(v) for v in row] for row in y],
    }


def main() -> None:
    rng = random.Random(20261201)
    problems = [
        problem(rng, "random_k64_m1", 8, 64, 1),
        problem(rng, "random_k128_m2", 8, 128, 2),
        problem(rng, "random_k192_m3", 5, 192, 3),
        problem(rng, "q_zero", 4, 128, 1, q_mode="zero"),
        problem(rng, "q_max", 4, 128, 1, q_mode="max"),
        problem(rng, "q_ramp", 4, 128, 2, q_mode="ramp"),
        problem(rng, "s_zero", 4, 128, 1, s_mode="zero"),
        problem(rng, "x_onehot", 6, 128, 3, x_mode="onehot"),
        problem(rng, "x_wide", 6, 256, 2, x_mode="wide"),
    ]
    known = {
        "unpack": [
            {"word": "76543210", "q": list(range(8))},
            {"word": "fedcba98", "q": list(range(8, 16))},
            {"word": "0000000f", "q": [15, 0, 0, 0, 0, 0, 0, 0]},
            {"word": "f0000000", "q": [0, 0, 0, 0, 0, 0, 0, 15]},
        ],
        "bf16_round": [  # float32 bits -> bf16 bits (nearest, ties to even; NaN -> 7fc0)
            {"f32": "3f800000", "bf16": "3f80"},
            {"f32": "3f808000", "bf16": "3f80"},
            {"f32": "3f818000", "bf16": "3f82"},
            {"f32": "3f808001", "bf16": "3f81"},
            {"f32": "bf80ffff", "bf16": "bf81"},
            {"f32": "7f7fffff", "bf16": "7f80"},
            {"f32": "7f800000", "bf16": "7f80"},
            {"f32": "ff800000", "bf16": "ff80"},
            {"f32": "7fc00001", "bf16": "7fc0"},
            {"f32": "ffffffff", "bf16": "7fc0"},
            {"f32": "00000001", "bf16": "0000"},
            {"f32": "00008000", "bf16": "0000"},
            {"f32": "00018000", "bf16": "0002"},
        ],
    }
    with open(os.path.join(HERE, "qmv_golden.json"), "w") as fh:
        json.dump({"generator": "tests/golden/make_golden.py", "group_size": GS,
                   "known_answers": known, "problems": problems}, fh, separators=(",", ":"))


if __name__ == "__main__":
    main()
