"""Stage-wise checks of BASELINE config 5 -- the MLP block and the GEMM fan-out --
and of the reference graph bench's five topologies against the CPU oracle.  Test infrastructure: imported only by tests/ and by
bench.py's CPU leg, as the checker of what the GPU computed.

Every node is checked on the GPU's own input to that node (read back from a
per-tensor arena), so each tolerance covers one kernel's rounding:

  GEMM       the reference's spot check (tests/reference.hpp:401-426): 1024 output
             entries recomputed in double and judged at rel tol_gemm(K) + abs
             abs_tol_gemm(K, amax).  The reference derives its absolute floor from
             the typical term amax^2/3 of U(-amax, amax) inputs
             (reference.hpp:357-377), which is rms(a) * rms(b); for the normal
             inputs of the MLP the same floor is taken with amax^2/3 set to the
             measured rms(a) * rms(b) of the node's operands.
  bias+GELU  every element, abs 1e-6 + rel 1e-6 (BASELINE configs[3]'s abs 1e-6,
             with the reference's relative term for large outputs).
  bias add   every element bit-exact: one fp32 add, correctly rounded on both
             sides (reference.hpp:143-151).
  softmax    every element within BASELINE configs[2]'s abs 1e-6, and every row
             sum within 1e-5 of 1.
"""
from __future__ import annotations

import math

import numpy as np

from . import bias_act, compare, row_softmax, spot_check_gemm, abs_tol_gemm, tol_gemm

SPOT_SAMPLES = 1024
SPOT_SEED = 0x5A11E           # gemm_bench.cpp's spot-check seed


def gemm_amax(a: np.ndarray, b: np.ndarray) -> float:
    """The U(-amax, amax) scale whose typical term amax^2/3 equals rms(a) * rms(b)."""
    ra = math.sqrt(float(np.mean(np.square(a, dtype=np.float64))))
    rb = math.sqrt(float(np.mean(np.square(b, dtype=np.float64))))
    return math.sqrt(3.0 * ra * rb)


def check_gemm(a, b, got, m: int, n: int, k: int) -> dict:
    amax = gemm_amax(a, b)
    rel, floor = tol_gemm(k), abs_tol_gemm(k, amax)
    r = spot_check_gemm(a, b, got, m, n, k, 1.0, SPOT_SAMPLES, SPOT_SEED, rel, floor)
    finite = bool(np.isfinite(got).all())
    return {"ok": r.checked == SPOT_SAMPLES and r.mismatches == 0 and finite,
            "check": f"spot {SPOT_SAMPLES}", "checked": r.checked, "mismatches": r.mismatches,
            "max_abs_err": r.max_abs_err, "max_rel_err": r.max_rel_err,
            "tol": f"rel {rel:.3g} + abs {floor:.3g} (amax {amax:.3g})", "all_finite": finite}


def check_bias_act(x, bias, got, rows: int, cols: int, act: int) -> dict:
    want = bias_act(x, bias, rows, cols, act)
    if act == 0:
        same = bool(np.array_equal(np.asarray(got).view(np.uint32), want.view(np.uint32)))
        diff = np.abs(np.asarray(got, np.float64) - want.astype(np.float64))
        return {"ok": same, "check": "bit-exact", "max_abs_err": float(diff.max())}
    r = compare(got, want, 1e-6, 1e-6)
    return {"ok": r.ok, "check": "abs 1e-6 + rel 1e-6", "mismatches": r.mismatches,
            "max_abs_err": r.max_abs_err}


def check_softmax(x, got, rows: int, cols: int) -> dict:
    want = row_softmax(x, rows, cols)
    r = compare(got, want, 0.0, 1e-6)
    sums = np.asarray(got, np.float64).reshape(rows, cols).sum(axis=1)
    sum_err = float(np.max(np.abs(sums - 1.0)))
    return {"ok": r.ok and sum_err <= 1e-5, "check": "abs 1e-6, row sums 1e-5",
            "mismatches": r.mismatches, "max_abs_err": r.max_abs_err, "max_row_sum_err": sum_err}


def check_mlp(inp: dict, stages: dict, T: int, D: int, F: int) -> dict:
    """inp: x, W1, b1, W2, b2 (host arrays the GPU was given); stages: the GPU's
    gemm1 [T x F], h [T x F], gemm2 [T x D], z [T x D], y [T x D]."""
    res = {
        "gemm1": check_gemm(inp["x"], inp["W1"], stages["gemm1"], T, F, D),
        "bias_gelu": check_bias_act(stages["gemm1"], inp["b1"], stages["h"], T, F, 3),
        "gemm2": check_gemm(stages["h"], inp["W2"], stages["gemm2"], T, D, F),
        "bias_add": check_bias_act(stages["gemm2"], inp["b2"], stages["z"], T, D, 0),
        "softmax": check_softmax(stages["z"], stages["y"], T, D),
    }
    res["ok"] = all(v["ok"] for v in res.values())
    return res


def check_fanout(w, xs: list, nodes: list, n: int) -> dict:
    """nodes[k][d]: the GPU's output of GEMM d of chain k, whose input is xs[k]
    (d = 0) or nodes[k][d - 1]."""
    res = {}
    for k, chain in enumerate(nodes):
        cur = xs[k]
        for d, got in enumerate(chain):
            res[f"b{k}g{d}"] = check_gemm(cur, w, got, n, n, n)
            cur = got
    res["ok"] = all(v["ok"] for v in res.values())
    return res


def check_bias_chain(x, bias, outs: list, rows: int, cols: int, act: int = 3) -> dict:
    """outs[d]: the GPU's output of bias+act node d of a chain whose input is x
    (d = 0) or outs[d - 1] -- one chain of the reference's `chain` and `fanout`
    graphs (bench/graph_bench.cpp:155-194)."""
    res, cur = {}, x
    for d, got in enumerate(outs):
        res[f"n{d}"] = check_bias_act(cur, bias, got, rows, cols, act)
        cur = got
    res["ok"] = all(v["ok"] for v in res.values())
    return res


def check_transformer(inp: dict, stages: dict, T: int, D: int, F: int) -> dict:
    """The reference's transformer_block (bench/graph_bench.cpp:199-215): inp holds
    x [T x D], W1 [D x F], b1 [F], W2 [F x D]; stages the GPU's gemm1 [T x F],
    bias_gelu [T x F], gemm2 [T x D] and softmax [T x D]."""
    res = {
        "gemm1": check_gemm(inp["x"], inp["W1"], stages["gemm1"], T, F, D),
        "bias_gelu": check_bias_act(stages["gemm1"], inp["b1"], stages["bias_gelu"], T, F, 3),
        "gemm2": check_gemm(stages["bias_gelu"], inp["W2"], stages["gemm2"], T, D, F),
        "softmax": check_softmax(stages["gemm2"], stages["softmax"], T, D),
    }
    res["ok"] = all(v["ok"] for v in res.values())
    return res


def check_diamond_gemm(a, w, stages: dict, n: int) -> dict:
    """B = A W, C = A W, D = B C (bench/graph_bench.cpp:100-113) on the GPU's B and C."""
    res = {
        "B_gemm": check_gemm(a, w, stages["B_gemm"], n, n, n),
        "C_gemm": check_gemm(a, w, stages["C_gemm"], n, n, n),
        "D_gemm": check_gemm(stages["B_gemm"], stages["C_gemm"], stages["D_gemm"], n, n, n),
    }
    # B and C are the same product of the same operands under the same kernel.
    res["B_equals_C_bitwise"] = {"ok": bool(np.array_equal(
        np.asarray(stages["B_gemm"]).view(np.uint32), np.asarray(stages["C_gemm"]).view(np.uint32)))}
    res["ok"] = all(v["ok"] for v in res.values())
    return res


def check_diamond_starved(x, bias, stages: dict, rows: int, cols: int) -> dict:
    """B and C = bias+GELU(X), D = bias+GELU(B) (bench/graph_bench.cpp:138-153)."""
    res = {
        "B_starved": check_bias_act(x, bias, stages["B_starved"], rows, cols, 3),
        "C_starved": check_bias_act(x, bias, stages["C_starved"], rows, cols, 3),
        "D_join": check_bias_act(stages["B_starved"], bias, stages["D_join"], rows, cols, 3),
    }
    res["ok"] = all(v["ok"] for v in res.values())
    return res
