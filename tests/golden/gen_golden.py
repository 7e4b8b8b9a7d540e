"""Independent golden vectors for the MCKE kernel layer (this build's own).

Pure Python, no numpy and no C: inputs from a SplitMix64 stream, expected values
from the mathematical definitions with exact rational arithmetic
(``fractions.Fraction``) wherever the operation is exact, and ``math.fsum`` /
``math.exp`` / ``math.tanh`` / ``math.erf`` in double otherwise.  This is a second
derivation next to the C oracle and the reference's own fixture, with shapes that
the reference's fixture does not cover: tile- and vector-width boundaries, rows
that are not multiples of 4, an all-negative row, a one-column softmax and a
+30 spike.

Method (exactness): inputs are multiples of 0.25 in [-4, 4].  Every product of two
is a multiple of 1/16 with magnitude <= 16, so any sum of fewer than 2^20 of them
is an integer multiple of 1/16 below 2^24 units and therefore exact in f32 in ANY
summation order.  Such cases are marked "exact" and must match bit for bit.

Usage:  python tests/golden/gen_golden.py      (writes tests/golden/mcke_golden.json)
"""
from __future__ import annotations

import json
import math
import os
import struct
from fractions import Fraction

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "mcke_golden.json")
MASK = (1 << 64) - 1


class SplitMix64:
    def __init__(self, seed: int):
        self.s = seed & MASK

    def next(self) -> int:
        self.s = (self.s + 0x9E3779B97F4A7C15) & MASK
        z = self.s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK
        return z ^ (z >> 31)

    def quarter(self, lo: float = -4.0, hi: float = 4.0) -> float:
        steps = int(round((hi - lo) * 4)) + 1
        return lo + 0.25 * (self.next() % steps)

    def uniform(self, lo: float, hi: float) -> float:
        return lo + (hi - lo) * ((self.next() >> 11) / float(1 << 53))


def f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def hx(x: float) -> str:
    return "%08x" % struct.unpack("<I", struct.pack("<f", x))[0]


def exact_f32(q: Fraction) -> float:
    v = float(q)
    if Fraction(f32(v)) != q:
        raise AssertionError(f"value {q} is not exact in f32")
    return f32(v)


def case_gemm(name, m, n, k, alpha, beta, seed):
    g = SplitMix64(seed)
    a = [g.quarter() for _ in range(m * k)]
    b = [g.quarter() for _ in range(k * n)]
    c = [g.quarter() if beta != 0.0 else 0.0 for _ in range(m * n)]
    exp = []
    for i in range(m):
        for j in range(n):
            acc = sum((Fraction(a[i * k + p]) * Fraction(b[p * n + j]) for p in range(k)),
                      Fraction(0))
            exp.append(exact_f32(Fraction(alpha) * acc + Fraction(beta) * Fraction(c[i * n + j])))
    return {"name": name, "kind": "gemm", "mode": "exact",
            "ints": {"m": m, "n": n, "k": k}, "floats": {"alpha": hx(alpha), "beta": hx(beta)},
            "arrays": {"a": [hx(v) for v in a], "b": [hx(v) for v in b],
                       "c": [hx(v) for v in c], "expect": [hx(v) for v in exp]}}


def gelu_tanh(v: float) -> float:
    return 0.5 * v * (1.0 + math.tanh(0.79788456080286535588 * (v + 0.044715 * v * v * v)))


def gelu_erf(v: float) -> float:
    return 0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0)))


def case_bias_act(name, rows, cols, act, seed, exact):
    g = SplitMix64(seed)
    if exact:
        x = [g.quarter() for _ in range(rows * cols)]
        bias = [g.quarter(-2.0, 2.0) for _ in range(cols)]
    else:
        # A ramp across the GELU knee and both tails, plus random points.
        x = [f32(-8.0 + 16.0 * i / (rows * cols - 1)) for i in range(rows * cols)]
        bias = [f32(g.uniform(-0.5, 0.5)) for _ in range(cols)]
    exp = []
    for r in range(rows):
        for c in range(cols):
            v = x[r * cols + c] + bias[c]          # exact in double
            if act == 0:
                y = exact_f32(Fraction(x[r * cols + c]) + Fraction(bias[c])) if exact else f32(v)
            elif act == 1:
                y = f32(v if v > 0.0 else 0.0)
            elif act == 2:
                y = f32(gelu_erf(v))
            else:
                y = f32(gelu_tanh(v))
            exp.append(y)
    return {"name": name, "kind": "bias_act", "mode": "exact" if exact else "approx",
            "ints": {"rows": rows, "cols": cols, "act": act}, "floats": {},
            "arrays": {"x": [hx(v) for v in x], "bias": [hx(v) for v in bias],
                       "expect": [hx(v) for v in exp]}}


def case_row_reduce(name, rows, cols, kind, seed):
    g = SplitMix64(seed)
    x = [g.quarter() for _ in range(rows * cols)]
    # Row 1 all negative: the max identity must be -inf, not 0.
    for c in range(cols):
        x[cols + c] = -abs(x[cols + c]) - 0.25
    exp = []
    for r in range(rows):
        row = x[r * cols:(r + 1) * cols]
        if kind == 1:
            exp.append(f32(max(row)))
        else:
            s = sum((Fraction(v) for v in row), Fraction(0))
            if kind == 2:
                exp.append(f32(float(s / cols)))   # correctly rounded quotient
            else:
                exp.append(exact_f32(s))
    return {"name": name, "kind": "row_reduce", "mode": "exact",
            "ints": {"rows": rows, "cols": cols, "kind": kind}, "floats": {},
            "arrays": {"x": [hx(v) for v in x], "expect": [hx(v) for v in exp]}}


def case_softmax(name, rows, cols, seed, spike):
    g = SplitMix64(seed)
    x = [f32(g.uniform(-4.0, 4.0)) for _ in range(rows * cols)]
    if spike:
        for r in range(rows):
            c = g.next() % cols
            x[r * cols + c] = f32(x[r * cols + c] + 30.0)
    exp = []
    for r in range(rows):
        row = x[r * cols:(r + 1) * cols]
        m = max(row)
        e = [math.exp(v - m) for v in row]
        s = math.fsum(e)
        exp.extend(f32(v / s) for v in e)
    return {"name": name, "kind": "row_softmax", "mode": "approx",
            "ints": {"rows": rows, "cols": cols}, "floats": {},
            "arrays": {"x": [hx(v) for v in x], "expect": [hx(v) for v in exp]}}


def main() -> None:
    cases = [
        case_gemm("gemm_tall_skinny_1x40x48", 1, 40, 48, 1.0, 0.0, 11),
        case_gemm("gemm_column_40x1x48", 40, 1, 48, 1.0, 0.0, 12),
        case_gemm("gemm_k1_33x63x1", 33, 63, 1, 1.0, 0.0, 13),
        case_gemm("gemm_odd_19x21x37", 19, 21, 37, 1.0, 0.0, 14),
        case_gemm("gemm_alpha_beta_17x19x23", 17, 19, 23, 0.5, 2.0, 15),
        case_gemm("gemm_k0_beta_5x6x0", 5, 6, 0, 1.0, 2.0, 16),
        case_bias_act("bias_none_5x12", 5, 12, 0, 21, True),
        case_bias_act("bias_relu_3x10", 3, 10, 1, 22, True),
        case_bias_act("bias_gelu_tanh_ramp_4x64", 4, 64, 3, 23, False),
        case_bias_act("bias_gelu_erf_ramp_4x64", 4, 64, 2, 24, False),
        case_row_reduce("reduce_sum_4x37", 4, 37, 0, 31),
        case_row_reduce("reduce_max_4x37", 4, 37, 1, 32),
        case_row_reduce("reduce_mean_4x37", 4, 37, 2, 33),
        case_row_reduce("reduce_sum_3x300", 3, 300, 0, 34),
        case_softmax("softmax_spike_4x96", 4, 96, 41, True),
        case_softmax("softmax_one_col_3x1", 3, 1, 42, False),
        case_softmax("softmax_17x33", 17, 33, 43, False),
    ]
    doc = {"source": "tests/golden/gen_golden.py (independent derivation)",
           "encoding": "every float is an 8-hex-digit IEEE-754 binary32 bit pattern",
           "cases": cases}
    with open(OUT, "w") as f:
        json.dump(doc, f)
        f.write("\n")
    print(f"wrote {len(cases)} cases to {OUT}")


if __name__ == "__main__":
    main()
