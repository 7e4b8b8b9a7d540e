"""Parity at BASELINE.json's full shapes, on the same seeded inputs bench.py times.

  configs[0]  GEMM 1024^3 .. 8192^3 (MFMA, the tile bench.py uses): the reference's
              spot check (1024 sampled entries recomputed in double,
              reference.hpp:401-426) with the K-scaled tolerances
  configs[1]  row sum / row max of X[8192 x 8192] N(0,1): every row against the
              double-accumulating CPU reduce (max bit-exact); full sum of 2^26
              U[0,1) against the same reduce with rows = 1, and against its
              expectation N/2 within 6 sigma
  configs[2]  softmax of X[32768 x C], C in {128, 1024, 4096}, N(0, 2^2) with 1% of
              rows spiked by +30: every element within BASELINE's pure abs 1e-6
              (and the reference's mixed abs 1e-6 / rel 1e-5), every row sum
              (|sum - 1| <= 1e-5)
  configs[3]  bias + GELU_tanh of X[16384 x 4096] and X[4096 x 1024]: every
              element within abs 1e-6 + rel 1e-6
"""
from __future__ import annotations

import numpy as np
import pytest

from tests.gpu_util import run_bias_act, run_reduce, run_softmax

pytestmark = pytest.mark.gpu


def _sum_abs_floor(rms: float, cols: int) -> float:
    """Absolute floor for f32 sums from the magnitude of the terms (the
    reference's rule, reference.hpp:312-321), as in the smaller-shape tests."""
    return 5e-5 * (rms / 0.577) * max(1.0, np.sqrt(cols / 4096.0))


@pytest.mark.parametrize("n", [1024, 2048, 4096, 8192])
def test_gemm_spot_check_at_sweep_sizes(gpu, orc, n):
    m = gpu
    D = m.DeviceBuffer
    a = orc.fill_random(n * n, 0x6E33A)
    b = orc.fill_random(n * n, 0x8B10C)
    da, db, dc = D.from_array(a), D.from_array(b), D.zeros(n * n)
    tile = m.gemm_mfma_default_tile(n, n, n)
    m.launch_gemm_f32(da, db, dc, n, n, n, 1.0, 0.0, m.GemmVariant.kMfmaF32, tile).throw_if_error()
    m.device_synchronize()
    got = dc.download(n * n)
    assert np.isfinite(got).all()
    r = orc.spot_check_gemm(a, b, got, n, n, n, 1.0, 1024, 0x5A11E, orc.tol_gemm(n),
                            orc.abs_tol_gemm(n))
    assert r.checked == 1024 and r.mismatches == 0, f"tile {tile.astuple()}: {r}"


def test_row_sum_and_max_8192(gpu, orc):
    R = C = 8192
    x = orc.fill_normal(R * C, 0x5EED12345)
    floor = _sum_abs_floor(1.0, C)
    for variant in (gpu.ReduceVariant.kWarpShuffle, gpu.ReduceVariant.kTwoPass):
        got = run_reduce(gpu, x, R, C, 0, variant)
        r = orc.compare(got, orc.row_reduce(x, R, C, 0), 1e-5, floor)
        assert r.ok, f"sum variant {int(variant)}: {r}"
        got = run_reduce(gpu, x, R, C, 1, variant)
        assert np.array_equal(got, orc.row_reduce(x, R, C, 1)), f"max variant {int(variant)}"


def test_full_sum_2p26(gpu, orc):
    N = 1 << 26
    x = orc.fill_random(N, 0xF011, 0.0, 1.0)
    got = run_reduce(gpu, x, 1, N, 0, gpu.ReduceVariant.kTwoPass)
    want = orc.row_reduce(x, 1, N, 0)
    assert abs(float(got[0]) - float(want[0])) <= 1e-5 * abs(float(want[0]))
    assert abs(float(got[0]) - N / 2) <= 6.0 * np.sqrt(N / 12.0)


def _softmax_input(orc, rows, cols):
    """bench.py's softmax input: N(0, 2^2) plus a +30 spike in 1% of rows."""
    x = orc.fill_normal(rows * cols, 0x50F7A11 + cols, 0.0, 2.0)
    rng = np.random.default_rng(cols)
    spike_rows = rng.choice(rows, rows // 100, replace=False)
    x[spike_rows * cols + rng.integers(0, cols, spike_rows.size)] += 30.0
    return x, spike_rows


@pytest.mark.parametrize("cols", [128, 1024, 4096])
def test_softmax_32768_rows(gpu, orc, cols):
    rows = 32768
    x, spike_rows = _softmax_input(orc, rows, cols)
    got = run_softmax(gpu, x, rows, cols, gpu.SoftmaxVariant.kOnlineOnePass)
    want = orc.row_softmax(x, rows, cols)
    r = orc.compare(got, want, 0.0, 1e-6)          # abs 1e-6
    assert r.ok, str(r)
    r = orc.compare(got, want, 1e-5, 1e-6)         # reference.hpp's tol_softmax form
    assert r.ok, str(r)
    g2 = got.reshape(rows, cols)
    sums = g2.astype(np.float64).sum(axis=1)
    assert np.max(np.abs(sums - 1.0)) <= 1e-5
    # a +30 spike dominates its row: the spiked column carries almost all the mass
    assert np.all(g2[spike_rows].max(axis=1) > 0.99)


@pytest.mark.parametrize("shape", [(16384, 4096), (4096, 1024)])
def test_bias_gelu_baseline_shapes(gpu, orc, shape):
    rows, cols = shape
    x = orc.fill_normal(rows * cols, 0xB1A5AC7 + rows)
    b = orc.fill_random(cols, 0xB1A5B1A5, -0.5, 0.5)
    got = run_bias_act(gpu, x, b, rows, cols, 3, 4)
    r = orc.compare(got, orc.bias_act(x, b, rows, cols, 3), 1e-6, 1e-6)
    assert r.ok, str(r)
