"""GPU parity over seeded random shapes: every launcher, through the C-ABI, against
the CPU oracle at shapes drawn from a fixed-seed generator (log-uniform extents,
random alpha / beta, activation, vector width, grid cap and operand alignment), so
that combinations the fixed shape lists do not name are covered too.

Bars are the ones the fixed-shape tests state:
  * fp32 GEMM: the reference's K-scaled tolerance tol_gemm(k) / abs_tol_gemm(k)
    (reference.hpp:344-374), the floor scaled by |alpha| and |beta|;
  * 16-bit GEMM: the same plus one ulp of a 16-bit output;
  * row reduce: max exact, sum / mean rel 1e-5 over the rows' magnitude floor;
  * softmax: rel 1e-5 + abs 1e-6, rows summing to 1 within 1e-5;
  * bias + activation: none / ReLU bit-exact, GELU rel 1e-6 + abs 1e-6, and every
    legal vector width and grid cap giving the same bits.
Each case prints its parameters on failure (the test id names the case index).
"""
from __future__ import annotations

import numpy as np
import pytest

from tests import golden_io
from tests.gpu_util import (cfg_id, f32, gemm_configs, run_bias_act, run_reduce,
                            run_softmax)
from tests.test_gpu_gemm_lp import BF16, F16, F32, OUT_ULP, run_lp
from tests.test_gpu_parity import _sum_abs_floor

pytestmark = pytest.mark.gpu

NCASES = 24


def _rng(op: str, case: int) -> np.random.Generator:
    return np.random.default_rng([0x5A4D, sum(map(ord, op)), case])


def _log_int(rng, lo: int, hi: int) -> int:
    """An integer in [lo, hi], log-uniform."""
    return int(min(hi, max(lo, round(float(np.exp(rng.uniform(np.log(lo), np.log(hi + 1))))))))


def _run_gemm_shift(m, a, b, c, M, N, K, alpha, beta, variant, tile, shift):
    """One fp32 launch on fresh buffers with `shift` floats of padding in front of
    every operand (shift = 1 breaks the 16-byte alignment of the vector paths)."""
    D = m.DeviceBuffer

    def up(arr):
        full = np.concatenate([np.zeros(shift, np.float32), f32(arr)]) if arr.size else \
            np.zeros(shift + 1, np.float32)
        buf = D.from_array(full)
        return buf, buf.ptr + 4 * shift

    ba, pa = up(a)
    bb, pb = up(b)
    bc, pc = up(c)
    st = m.launch_gemm_f32(pa, pb, pc, M, N, K, alpha, beta, variant, tile)
    assert st.ok(), str(st)
    m.device_synchronize()
    out = bc.download(shift + M * N)
    del ba, bb
    return out[shift:]


@pytest.mark.parametrize("case", range(NCASES))
def test_gemm_f32_random_shapes(gpu, orc, case):
    rng = _rng("gemm_f32", case)
    M, N, K = _log_int(rng, 1, 640), _log_int(rng, 1, 640), _log_int(rng, 1, 640)
    alpha = float(rng.choice([1.0, 0.5, -2.0]))
    beta = float(rng.choice([0.0, 0.0, 1.5]))
    shift = int(rng.integers(0, 2))
    a = orc.fill_random(M * K, 100 + case)
    b = orc.fill_random(K * N, 200 + case)
    c = orc.fill_random(M * N, 300 + case)
    want = orc.gemm(a, b, c, M, N, K, alpha, beta)
    rel = orc.tol_gemm(K)
    floor = max(1.0, abs(alpha)) * orc.abs_tol_gemm(K) + 2e-7 * max(1.0, abs(beta))
    params = f"M={M} N={N} K={K} alpha={alpha} beta={beta} shift={shift}"
    for variant, tile in gemm_configs(gpu):
        got = _run_gemm_shift(gpu, a, b, c, M, N, K, alpha, beta, variant, tile, shift)
        r = orc.compare(got, want, rel, floor)
        assert r.ok, f"{params} {cfg_id((variant, tile))}: {r}"


@pytest.mark.parametrize("case", range(NCASES))
def test_gemm_lp_random_shapes(gpu, orc, case):
    rng = _rng("gemm_lp", case)
    M, N, K = _log_int(rng, 1, 520), _log_int(rng, 1, 520), _log_int(rng, 1, 520)
    dt = int(rng.choice([BF16, F16]))
    cd = F32 if rng.integers(0, 2) else dt
    alpha = float(rng.choice([1.0, 0.5]))
    beta = float(rng.choice([0.0, 2.0]))
    shift = int(rng.integers(0, 2))
    a16 = orc.to_16(orc.fill_random(M * K, 400 + case), dt)
    b16 = orc.to_16(orc.fill_random(K * N, 500 + case), dt)
    cf = orc.fill_random(M * N, 600 + case)
    c = cf if cd == F32 else orc.to_16(cf, dt)
    want = orc.gemm_lp(a16, b16, c, M, N, K, alpha, beta, dt, cd)
    w = want if cd == F32 else orc.from_16(want, dt)
    rel = orc.tol_gemm(K) + (0.0 if cd == F32 else OUT_ULP[dt])
    floor = orc.abs_tol_gemm(K) + 2e-7 * max(1.0, beta)
    params = f"M={M} N={N} K={K} dt={dt} c={cd} alpha={alpha} beta={beta} shift={shift}"
    for tile in (gpu.gemm_lp_default_tile(M, N, K),) + tuple(gpu.LP_TILES):
        got = run_lp(gpu, a16, b16, c, M, N, K, alpha, beta, dt, cd, tile, shift=shift)
        g = got if cd == F32 else orc.from_16(got, dt)
        r = orc.compare(g, w, rel, floor)
        assert r.ok, f"{params} {tile}: {r}"


@pytest.mark.parametrize("case", range(NCASES))
def test_row_reduce_random_shapes(gpu, orc, case):
    rng = _rng("reduce", case)
    rows, cols = _log_int(rng, 1, 300), _log_int(rng, 1, 60000)
    x = orc.fill_normal(rows * cols, 700 + case, float(rng.uniform(-1, 1)), 1.0)
    for kind in (0, 1, 2):
        want = orc.row_reduce(x, rows, cols, kind)
        floor = _sum_abs_floor(x.reshape(rows, cols)) / (cols if kind == 2 else 1)
        for variant in (0, 1, 2):
            got = run_reduce(gpu, x, rows, cols, kind, variant)
            params = f"rows={rows} cols={cols} kind={kind} variant={variant}"
            if kind == 1:
                assert np.array_equal(got, want), params
            else:
                r = orc.compare(got, want, 1e-5, floor)
                assert r.ok, f"{params}: {r}"


@pytest.mark.parametrize("case", range(NCASES))
def test_softmax_random_shapes(gpu, orc, case):
    rng = _rng("softmax", case)
    rows, cols = _log_int(rng, 1, 200), _log_int(rng, 1, 12000)
    x = orc.fill_normal(rows * cols, 800 + case, 0.0, float(rng.uniform(0.5, 4.0)))
    want = orc.row_softmax(x, rows, cols)
    for variant in (0, 1):
        got = run_softmax(gpu, x, rows, cols, variant)
        params = f"rows={rows} cols={cols} variant={variant}"
        r = orc.compare(got, want, 1e-5, 1e-6)
        assert r.ok, f"{params}: {r}"
        sums = got.reshape(rows, cols).astype(np.float64).sum(axis=1)
        assert np.max(np.abs(sums - 1.0)) <= 1e-5, params


@pytest.mark.parametrize("case", range(NCASES))
def test_bias_act_random_shapes(gpu, orc, case):
    rng = _rng("bias_act", case)
    rows, cols = _log_int(rng, 1, 3000), _log_int(rng, 1, 5000)
    if rng.integers(0, 2):
        cols = max(4, cols // 4 * 4)          # half the cases admit the 16-byte path
    act = int(rng.integers(0, 4))
    x = orc.fill_normal(rows * cols, 900 + case, 0.0, 2.0)
    b = orc.fill_random(cols, 1000 + case, -0.5, 0.5)
    want = orc.bias_act(x, b, rows, cols, act)
    widths = [w for w in (4, 2, 1) if cols % w == 0]
    caps = [0, int(rng.integers(1, 12))]
    ref_bits = None
    for vw in widths:
        for mrb in caps:
            got = run_bias_act(gpu, x, b, rows, cols, act, vw, max_row_blocks=mrb)
            params = f"rows={rows} cols={cols} act={act} vw={vw} max_row_blocks={mrb}"
            if act in (0, 1):
                assert np.array_equal(golden_io.bits(got), golden_io.bits(want)), params
            else:
                r = orc.compare(got, want, 1e-6, 1e-6)
                assert r.ok, f"{params}: {r}"
            if ref_bits is None:
                ref_bits = golden_io.bits(got)
            assert np.array_equal(golden_io.bits(got), ref_bits), params
