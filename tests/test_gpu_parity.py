"""GPU parity: every launcher, through the C-ABI, against the CPU oracle.

Bars (stated per test):
  * golden "exact" cases: bit-for-bit (quarter-multiple inputs make every sum exact
    in f32, whatever the summation order -- so MFMA and FMA paths alike must match);
  * golden "approx" cases: rel 1e-6 + abs 1e-7 (the reference's fixture bar,
    test_host_core.cpp:2447-2449), GELU with its cancellation floor abs 1e-6;
  * seeded random inputs: the reference's mixed abs+rel tolerances
    (reference.hpp:292-374) and BASELINE's stated ones.
"""
from __future__ import annotations

import numpy as np
import pytest

from tests import golden_io
from tests.gpu_util import (cfg_id, gemm_configs, run_activation, run_bias_act, run_gemm,
                            run_reduce, run_softmax)

pytestmark = pytest.mark.gpu

CASES = golden_io.all_cases()


def _golden_ids(kind):
    return [c for c in CASES if c["kind"] == kind]


# ---------------------------------------------------------------------------
# Golden vectors
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("case", _golden_ids("bias_act"), ids=lambda c: c["name"])
@pytest.mark.parametrize("vw", [1, 2, 4])
def test_golden_bias_act(gpu, orc, case, vw):
    I, A = case["ints"], case["arrays"]
    if I["cols"] % vw:
        pytest.skip("cols not a multiple of the vector width")
    got = run_bias_act(gpu, A["x"], A["bias"], I["rows"], I["cols"], I["act"], vw)
    want = A["expect"]
    if case["mode"] == "exact":
        assert np.array_equal(golden_io.bits(got), golden_io.bits(want))
    else:
        r = orc.compare(got, want, 1e-6, 1e-6)
        assert r.ok, str(r)


@pytest.mark.parametrize("case", _golden_ids("row_reduce"), ids=lambda c: c["name"])
@pytest.mark.parametrize("variant", [0, 1, 2])
def test_golden_row_reduce(gpu, orc, case, variant):
    I, A = case["ints"], case["arrays"]
    got = run_reduce(gpu, A["x"], I["rows"], I["cols"], I["kind"], variant)
    assert np.array_equal(golden_io.bits(got), golden_io.bits(A["expect"]))


@pytest.mark.parametrize("case", _golden_ids("row_softmax"), ids=lambda c: c["name"])
@pytest.mark.parametrize("variant", [0, 1])
def test_golden_softmax(gpu, orc, case, variant):
    I, A = case["ints"], case["arrays"]
    got = run_softmax(gpu, A["x"], I["rows"], I["cols"], variant)
    r = orc.compare(got, A["expect"], 1e-6, 1e-7)
    assert r.ok, str(r)


@pytest.mark.parametrize("case", _golden_ids("gemm"), ids=lambda c: c["name"])
def test_golden_gemm_all_variants(gpu, case):
    I, A, F = case["ints"], case["arrays"], case["floats"]
    for cfg in gemm_configs(gpu):
        got = run_gemm(gpu, A["a"], A["b"], A["c"], I["m"], I["n"], I["k"], F["alpha"],
                       F["beta"], *cfg)
        assert np.array_equal(golden_io.bits(got), golden_io.bits(A["expect"])), cfg_id(cfg)


# ---------------------------------------------------------------------------
# Seeded random inputs
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("act", [0, 1, 2, 3])
@pytest.mark.parametrize("shape", [(37, 129), (64, 1024), (5, 4100)])
def test_bias_act_random(gpu, orc, act, shape):
    rows, cols = shape
    x = orc.fill_normal(rows * cols, 0xB1A5AC7, 0.0, 2.0)
    b = orc.fill_random(cols, 0xB1A5B1A5, -0.5, 0.5)
    want = orc.bias_act(x, b, rows, cols, act)
    for vw in (1, 2, 4):
        if cols % vw:
            continue
        got = run_bias_act(gpu, x, b, rows, cols, act, vw)
        if act in (0, 1):
            assert np.array_equal(golden_io.bits(got), golden_io.bits(want)), vw
        else:
            r = orc.compare(got, want, 1e-6, 1e-6)
            assert r.ok, f"vw={vw}: {r}"


def test_bias_act_row_streaming_path_and_starved_grid(gpu, orc):
    """More one-row workgroups than the small-launch limit: the row-per-workgroup
    kernel, also with its row dimension capped (rows walked with a stride)."""
    rows, cols = 4500, 1024
    x = orc.fill_normal(rows * cols, 15)
    b = orc.fill_random(cols, 16, -0.5, 0.5)
    want = orc.bias_act(x, b, rows, cols, 3)
    y4 = run_bias_act(gpu, x, b, rows, cols, 3, 4)
    r = orc.compare(y4, want, 1e-6, 1e-6)
    assert r.ok, str(r)
    for vw, mrb in ((4, 7), (4, 4000), (1, 0), (2, 13)):
        got = run_bias_act(gpu, x, b, rows, cols, 3, vw, max_row_blocks=mrb)
        assert np.array_equal(golden_io.bits(got), golden_io.bits(y4)), (vw, mrb)


@pytest.mark.parametrize("shape", [(4500, 1000), (50000, 12), (4097, 2052)],
                         ids=lambda s: "x".join(map(str, s)))
def test_bias_act_flat_grid_partial_strips(gpu, orc, shape):
    """The flat-grid kernel of VW = 4 (one workgroup per row strip, row and strip
    from a multiply-shift division) where a row's last strip is partial (1000 and
    2052 columns) or a row is narrower than one strip (12 columns), against the
    oracle and bit-equal to the 2-D grid that walks the rows (VW = 2 and 1, and
    VW = 4 with a capped grid)."""
    rows, cols = shape
    x = orc.fill_normal(rows * cols, 0xF1A7 + cols, 0.0, 2.0)
    b = orc.fill_random(cols, 0xF1A8, -0.5, 0.5)
    for act in (0, 3):
        want = orc.bias_act(x, b, rows, cols, act)
        ref_bits = None
        for vw, mrb in ((4, 0), (2, 0), (1, 0), (4, 9)):
            got = run_bias_act(gpu, x, b, rows, cols, act, vw, max_row_blocks=mrb)
            if act == 0:
                assert np.array_equal(golden_io.bits(got), golden_io.bits(want)), (vw, mrb)
            else:
                r = orc.compare(got, want, 1e-6, 1e-6)
                assert r.ok, f"vw={vw} mrb={mrb}: {r}"
            if ref_bits is None:
                ref_bits = golden_io.bits(got)
            assert np.array_equal(golden_io.bits(got), ref_bits), (act, vw, mrb)


def test_bias_act_width_invariance_and_starved_grid(gpu, orc):
    rows, cols = 300, 2048
    x = orc.fill_normal(rows * cols, 5)
    b = orc.fill_random(cols, 6, -0.5, 0.5)
    y1 = run_bias_act(gpu, x, b, rows, cols, 3, 1)
    y4 = run_bias_act(gpu, x, b, rows, cols, 3, 4)
    y4s = run_bias_act(gpu, x, b, rows, cols, 3, 4, max_row_blocks=7)
    assert np.array_equal(golden_io.bits(y1), golden_io.bits(y4))
    assert np.array_equal(golden_io.bits(y4), golden_io.bits(y4s))


@pytest.mark.parametrize("act", [0, 1, 2, 3])
def test_activation_special_values(gpu, orc, act):
    """Infinities, NaN, signed zeros, tiny and huge magnitudes, through the fused
    kernel with a zero bias and through the unfused activation kernel: the same
    values as the double-precision reference (reference.hpp:116-136 evaluated on
    x + b): NaN where it gives NaN (GELU of -inf is -inf * 0), +-inf where it
    gives +-inf, and finite values within abs 1e-6 + rel 1e-6."""
    vals = np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 1e-30, -1e-30, 1e-7, -1e-7, 3.0, -3.0,
                     9.5, -9.5, 30.0, -30.0, 88.0, -88.0, 1e3, -1e3, 1e30, -1e30, 3e38, -3e38,
                     0.5, -0.5, 6.0, -6.0, 12.0, -12.0, 1.0, -1.0, 2.0], np.float32)
    n = vals.size
    want = orc.bias_act(vals, np.zeros(n, np.float32), 1, n, act)
    for got in (run_bias_act(gpu, vals, np.zeros(n, np.float32), 1, n, act, 4),
                run_activation(gpu, vals, n, act, 4)):
        nan_w, nan_g = np.isnan(want), np.isnan(got)
        assert np.array_equal(nan_w, nan_g), (vals[nan_w != nan_g], got[nan_w != nan_g])
        fin = ~nan_w
        inf_w = np.isinf(want[fin])
        assert np.array_equal(got[fin][inf_w], want[fin][inf_w])
        r = orc.compare(got[fin][~inf_w], want[fin][~inf_w], 1e-6, 1e-6)
        assert r.ok, f"act {act}: {r}"


@pytest.mark.parametrize("act", [0, 1, 2, 3])
@pytest.mark.parametrize("n", [3 * 4096, 3 * 4096 + 20, 5])
def test_activation_unfused(gpu, orc, act, n):
    x = orc.fill_normal(n, 11, 0.0, 3.0)
    want = orc.bias_act(x, np.zeros(n, np.float32), 1, n, act)
    for vw in (4, 1):
        if n % vw:
            continue
        got = run_activation(gpu, x, n, act, vw)
        r = orc.compare(got, want, 1e-6, 1e-6)
        assert r.ok, f"vw={vw}: {r}"


def _sum_abs_floor(x2d):
    """Absolute floor for f32 sums of a row, from the magnitude of the terms
    (the reference's rule, reference.hpp:312-321): 5e-5 at 4096 terms of
    U[-1,1] (rms 0.577), scaled by the rows' rms and sqrt(cols/4096)."""
    rms = float(np.sqrt(np.mean(np.square(x2d.astype(np.float64)))))
    cols = x2d.shape[1]
    return 5e-5 * (rms / 0.577) * max(1.0, np.sqrt(cols / 4096.0))


@pytest.mark.parametrize("variant", [0, 1, 2])
@pytest.mark.parametrize("shape", [(1, 1), (3, 7), (17, 1000), (64, 4096), (2, 100003)])
def test_row_reduce_random(gpu, orc, variant, shape):
    rows, cols = shape
    x = orc.fill_normal(rows * cols, 0x5EED12345)
    for kind in (0, 1, 2):
        got = run_reduce(gpu, x, rows, cols, kind, variant)
        want = orc.row_reduce(x, rows, cols, kind)
        if kind == 1:
            assert np.array_equal(got, want)          # max: exact
        else:
            floor = _sum_abs_floor(x.reshape(rows, cols))
            if kind == 2:
                floor /= cols
            r = orc.compare(got, want, 1e-5, floor)
            assert r.ok, f"kind={kind}: {r}"


@pytest.mark.parametrize("cols", [5, 1000, 70000])
def test_row_reduce_special_values(gpu, orc, cols):
    """Sum, max and mean of rows holding +inf, -inf, both, NaN, or huge values, every
    variant: the same NaN / +-inf pattern as the double-precision reference
    (reference.hpp:154-172), finite results at its bar.  A row with +inf and -inf sums
    to NaN in any order; max skips NaN as fmaxf does (the reference kernel's MaxOp,
    reduce_ops.cuh:38-119) and as the reference's std::max(m, v) from -inf does, so
    an all-NaN row has max -inf."""
    rng = np.random.default_rng(cols)
    x = rng.normal(0.0, 1.0, (7, cols)).astype(np.float32)
    x[0, cols // 2] = np.inf
    x[1, 0] = -np.inf
    x[2, 1 % cols] = np.inf
    x[2, cols - 1] = -np.inf
    x[3, cols // 3] = np.nan
    x[4, 0] = 3e38                                # huge but finite: the double sum stays finite
    x[6, :] = np.nan                              # row 5 stays finite
    x = x.ravel()
    assert orc.row_reduce(x, 7, cols, 1)[6] == -np.inf
    for kind in (0, 1, 2):
        want = orc.row_reduce(x, 7, cols, kind)
        for variant in (0, 1, 2):
            got = run_reduce(gpu, x, 7, cols, kind, variant)
            params = f"kind={kind} variant={variant}"
            assert np.array_equal(np.isnan(got), np.isnan(want)), (params, got, want)
            inf_w = np.isinf(want)
            assert np.array_equal(got[inf_w], want[inf_w]), (params, got, want)
            fin = np.isfinite(want)
            if kind == 1:
                assert np.array_equal(got[fin], want[fin]), params
            else:
                floor = _sum_abs_floor(x.reshape(7, cols)[5:6]) / (cols if kind == 2 else 1)
                r = orc.compare(got[fin], want[fin], 1e-5, floor)
                assert r.ok, f"{params}: {r}"


def test_row_reduce_all_negative_and_inf_rows(gpu, orc):
    x = np.array([[-5, -1, -9, -3], [-np.inf] * 4, [1, np.nan, 3, 2]], np.float32)
    for variant in (0, 1, 2):
        got = run_reduce(gpu, x, 3, 4, 1, variant)
        assert got[0] == -1.0 and got[1] == -np.inf and got[2] == 3.0


@pytest.mark.parametrize("variant", [0, 1])
@pytest.mark.parametrize("cols", [1, 3, 4, 17, 64, 128, 131, 200, 256, 512, 1024, 2048, 4096,
                                  8192, 10000])
def test_softmax_random(gpu, orc, variant, cols):
    rows = 67 if cols <= 4096 else 8          # ragged against every rows-per-workgroup
    x = orc.fill_normal(rows * cols, 0x50F7A11, 0.0, 2.0)
    x[5 * cols] += 30.0                                  # a spike row
    got = run_softmax(gpu, x, rows, cols, variant)
    want = orc.row_softmax(x, rows, cols)
    r = orc.compare(got, want, 1e-5, 1e-6)
    assert r.ok, str(r)
    sums = got.reshape(rows, cols).astype(np.float64).sum(axis=1)
    assert np.max(np.abs(sums - 1.0)) <= 1e-5


@pytest.mark.parametrize("cols", [7, 8, 1024, 1031, 8200])
def test_softmax_special_values(gpu, orc, cols):
    """Rows with infinities, NaN, huge and tiny magnitudes against the double-precision
    reference (reference.hpp:175-191): its max keeps the running value against NaN
    (std::max(m, v)), so a NaN entry, a +inf entry or a row of -inf makes the whole
    row NaN through the sum, while -inf and -FLT_MAX entries beside finite ones get 0.
    Every kernel path: cols 7 and 1031 take the element path, 8 and 1024 the
    register-resident kernel, 8200 the one-pass online kernel on 16-byte data; both
    variants.  NaN positions must match; other entries rel 1e-5 + abs 1e-6."""
    fmax = np.finfo(np.float32).max
    rng = np.random.default_rng(cols)
    rows = []

    def row(specials):
        r = rng.normal(0.0, 2.0, cols).astype(np.float32)
        for j, v in specials.items():
            r[j % cols] = v
        rows.append(r)

    row({1: -np.inf})                                            # -inf beside finite values
    rows.append(np.full(cols, -np.inf, np.float32))              # all -inf: NaN
    row({cols // 2: np.nan})                                     # NaN: NaN row
    row({cols - 1: np.inf})                                      # +inf: NaN row
    row({0: 3e38, 2: -3e38, 3: 1e38})                            # huge: differences overflow to -inf
    row({0: 1e-30, 1: -1e-30, 2: 0.0, 3: -0.0})                  # tiny and signed zeros
    row({0: -fmax, 3: -fmax})                                    # -FLT_MAX beside finite values
    r = np.full(cols, -np.inf, np.float32)
    r[cols // 3] = -fmax                                         # one -FLT_MAX among -inf: 1 there
    rows.append(r)
    x = np.concatenate(rows)
    n_rows = len(rows)
    want = orc.row_softmax(x, n_rows, cols)
    nan_w = np.isnan(want)
    # The cases above pin the reference's semantics, not just this oracle's.
    assert nan_w.reshape(n_rows, cols).all(axis=1).tolist() == [False, True, True, True, False,
                                                                False, False, False]
    assert want[7 * cols + cols // 3] == 1.0
    for variant in (0, 1):
        got = run_softmax(gpu, x, n_rows, cols, variant)
        nan_g = np.isnan(got)
        assert np.array_equal(nan_w, nan_g), \
            f"variant {variant}: NaN rows {np.nonzero(nan_w != nan_g)[0] // cols}"
        r = orc.compare(got[~nan_w], want[~nan_w], 1e-5, 1e-6)
        assert r.ok, f"variant {variant}: {r}"


def test_softmax_overflow_ramp(gpu, orc):
    """Logits 0..90: without the max subtraction expf overflows (softmax_bench.cpp:172-199)."""
    cols = 1024
    x = np.linspace(0.0, 90.0, cols, dtype=np.float32)
    for variant in (0, 1):
        got = run_softmax(gpu, x, 1, cols, variant)
        assert np.isfinite(got).all()
        r = orc.compare(got, orc.row_softmax(x, 1, cols), 1e-5, 1e-6)
        assert r.ok, str(r)


@pytest.mark.parametrize("shape", [(1, 1, 1), (5, 7, 3), (129, 65, 257), (1, 64, 128),
                                   (64, 1, 128), (33, 63, 1), (253, 253, 253), (256, 256, 256),
                                   (300, 520, 36)])
def test_gemm_random(gpu, orc, shape):
    """The reference's validation shapes (gemm_bench.cpp:358-368), every variant."""
    M, N, K = shape
    a = orc.fill_random(M * K, 0x6E33A)
    b = orc.fill_random(K * N, 0x8B10C)
    c = np.zeros(M * N, np.float32)
    want = orc.gemm(a, b, c, M, N, K)
    rel, floor = orc.tol_gemm(K), orc.abs_tol_gemm(K)
    for cfg in gemm_configs(gpu):
        got = run_gemm(gpu, a, b, c, M, N, K, 1.0, 0.0, *cfg)
        r = orc.compare(got, want, rel, floor)
        assert r.ok, f"{cfg_id(cfg)}: {r}"


@pytest.mark.parametrize("shape", [(67, 45, 39), (256, 256, 64)], ids=lambda s: "x".join(map(str, s)))
def test_gemm_special_values(gpu, orc, shape):
    """Infinities and NaN in A and B, through every variant and tile: C holds NaN and
    +-inf exactly where the double-precision reference (reference.hpp:199-211) does,
    which no summation order changes (x + inf = inf for finite x, inf - inf = NaN,
    0 * inf = NaN); finite entries at the K-scaled bar.  Rows of A and columns of B
    each get one kind of special value, so every output pattern occurs: a single
    +inf or -inf, both signs in one dot product, a NaN, and inf times an exact zero."""
    M, N, K = shape
    rng = np.random.default_rng(M * N + K)
    a = rng.uniform(-1.0, 1.0, (M, K)).astype(np.float32)
    b = rng.uniform(-1.0, 1.0, (K, N)).astype(np.float32)
    a[0, 3] = np.inf                        # row 0: +inf times B row 3
    a[1, 5] = -np.inf                       # row 1: -inf times B row 5
    a[2, 1], a[2, 2] = np.inf, -np.inf      # row 2: both signs in one dot product
    a[3, K - 1] = np.nan                    # row 3: NaN
    a[4, 7] = np.inf                        # row 4: +inf times B row 7, which is
    b[7, : N // 2] = 0.0                    #   zero over half the columns (0 * inf)
    b[K - 2, N - 1] = np.inf                # column N-1: +inf down B
    b[9, N - 2] = np.nan                    # column N-2: NaN
    c = np.zeros(M * N, np.float32)
    want = orc.gemm(a.ravel(), b.ravel(), c, M, N, K, 1.0, 0.0)
    nan_w, inf_w = np.isnan(want), np.isinf(want)
    assert nan_w.any() and inf_w.any() and (~nan_w & ~inf_w).any()
    fin = ~nan_w & ~inf_w
    amax = 1.0
    for cfg in gemm_configs(gpu):
        got = run_gemm(gpu, a.ravel(), b.ravel(), c, M, N, K, 1.0, 0.0, *cfg)
        assert np.array_equal(np.isnan(got), nan_w), \
            f"{cfg_id(cfg)}: NaN at {np.argwhere((np.isnan(got) != nan_w).reshape(M, N))[:5]}"
        assert np.array_equal(got[inf_w], want[inf_w]), cfg_id(cfg)
        r = orc.compare(got[fin], want[fin], orc.tol_gemm(K), orc.abs_tol_gemm(K, amax))
        assert r.ok, f"{cfg_id(cfg)}: {r}"


def test_gemm_alpha_beta(gpu, orc):
    """beta != 0 at 129x65x257 with alpha 0.5, beta 2 (gemm_bench.cpp:408-437)."""
    M, N, K = 129, 65, 257
    a = orc.fill_random(M * K, 0x6E33A)
    b = orc.fill_random(K * N, 0x8B10C)
    c = orc.fill_random(M * N, 0xC0FFEE)
    want = orc.gemm(a, b, c, M, N, K, 0.5, 2.0)
    rel, floor = orc.tol_gemm(K), orc.abs_tol_gemm(K) + 2e-7
    for cfg in gemm_configs(gpu):
        got = run_gemm(gpu, a, b, c, M, N, K, 0.5, 2.0, *cfg)
        r = orc.compare(got, want, rel, floor)
        assert r.ok, f"{cfg_id(cfg)}: {r}"


def test_gemm_beta_zero_never_reads_c(gpu, orc):
    M, N, K = 70, 90, 40
    a = orc.fill_random(M * K, 1)
    b = orc.fill_random(K * N, 2)
    c = np.full(M * N, np.nan, np.float32)
    want = orc.gemm(a, b, np.zeros(M * N, np.float32), M, N, K)
    for cfg in gemm_configs(gpu):
        got = run_gemm(gpu, a, b, c, M, N, K, 1.0, 0.0, *cfg)
        assert not np.isnan(got).any(), cfg_id(cfg)
        r = orc.compare(got, want, orc.tol_gemm(K), orc.abs_tol_gemm(K))
        assert r.ok, f"{cfg_id(cfg)}: {r}"


@pytest.mark.parametrize("shape", [(256, 256), (70, 90)])
def test_gemm_k_zero(gpu, orc, shape):
    """k == 0 launches the kernel and gives C = beta * C (reference gemm.cu:867, no
    early return), for every variant and tile: beta = 2 doubles C exactly (also
    against the oracle), and beta = 0 on a NaN-poisoned C gives zeros (C is not
    read).  256 x 256 is whole tiles for every MFMA tile, 70 x 90 is ragged."""
    M, N = shape
    c = orc.fill_random(M * N, 0xC0FFEE)
    empty = np.zeros(0, np.float32)
    want = orc.gemm(empty, empty, c, M, N, 0, 1.0, 2.0)
    assert np.array_equal(golden_io.bits(want), golden_io.bits(c * np.float32(2.0)))
    poisoned = np.full(M * N, np.nan, np.float32)
    zeros = np.zeros(M * N, np.float32)
    for cfg in gemm_configs(gpu):
        got = run_gemm(gpu, empty, empty, c, M, N, 0, 1.0, 2.0, *cfg)
        assert np.array_equal(golden_io.bits(got), golden_io.bits(want)), cfg_id(cfg)
        got = run_gemm(gpu, empty, empty, poisoned, M, N, 0, 1.0, 0.0, *cfg)
        assert np.array_equal(golden_io.bits(got), golden_io.bits(zeros)), cfg_id(cfg)


@pytest.mark.parametrize("size", [512, 1024])
def test_gemm_quarter_exact_mfma(gpu, size):
    """Quarter-multiple inputs: the exact product is representable in f32 and any
    summation order reproduces it, so the MFMA path must match float64 bit for bit."""
    rng = np.random.default_rng(size)
    a = (rng.integers(-16, 17, size * size) * 0.25).astype(np.float32)
    b = (rng.integers(-16, 17, size * size) * 0.25).astype(np.float32)
    want = (a.reshape(size, size).astype(np.float64) @
            b.reshape(size, size).astype(np.float64)).astype(np.float32).ravel()
    for t in gpu.MFMA_TILES:
        got = run_gemm(gpu, a, b, np.zeros(size * size, np.float32), size, size, size, 1.0,
                       0.0, gpu.GemmVariant.kMfmaF32, t)
        assert np.array_equal(golden_io.bits(got), golden_io.bits(want)), repr(t)


def test_gemm_512_baseline_config(gpu, orc):
    """512^3, U[-1,1) from the reference seeds, rel tol 1e-4."""
    n = 512
    a = orc.fill_random(n * n, 0x6E33A)
    b = orc.fill_random(n * n, 0x8B10C)
    c = np.zeros(n * n, np.float32)
    want = orc.gemm(a, b, c, n, n, n)
    t = gpu.gemm_mfma_default_tile(n, n, n)
    got = run_gemm(gpu, a, b, c, n, n, n, 1.0, 0.0, gpu.GemmVariant.kMfmaF32, t)
    r = orc.compare(got, want, 1e-4, orc.abs_tol_gemm(n))
    assert r.ok, str(r)
    r2 = orc.compare(got, want, orc.tol_gemm(n), orc.abs_tol_gemm(n))
    assert r2.ok, str(r2)


def test_mfma_kernel_attrs_report_the_whole_tile_kernel(gpu):
    """gemm_kernel_attrs (kernels.hpp:293-302) describes the kernel that whole-tile
    shapes run: the 64x64, 128x128 and 256x256 tiles' direct-to-LDS kernels run
    one wave group of four waves (256 lanes), the 32x32 tile four one-wave groups
    (256 lanes)."""
    T = gpu.GemmTile
    for tile, threads in ((T(32, 32, 32, 2, 2), 256), (T(64, 64, 32, 4, 4), 256),
                          (T(128, 128, 32, 8, 8), 256), (T(256, 256, 32, 16, 16), 256)):
        st, at = gpu.gemm_kernel_attrs(gpu.GemmVariant.kMfmaF32, tile)
        assert st.ok(), str(st)
        assert at.threads_per_block == threads, tile.astuple()
        assert at.max_blocks_per_sm_api >= 1 and at.local_bytes == 0, tile.astuple()


_DMA_STEP_CASES = (
    [((64, 64, 32, 4, 4), mnk) for mnk in
     [(128, 128, 32), (128, 128, 96), (192, 64, 160), (64, 128, 224), (64, 64, 64)]] +
    [((32, 32, 32, 2, 2), mnk) for mnk in [(128, 128, 32), (128, 128, 96), (64, 96, 160)]] +
    [((256, 256, 32, 16, 16), mnk) for mnk in [(256, 256, 32), (256, 512, 96), (512, 256, 160)]] +
    [((128, 128, 32, 8, 8), mnk) for mnk in [(256, 256, 32), (128, 384, 96)]])


@pytest.mark.parametrize("tile,mnk", _DMA_STEP_CASES)
def test_gemm_dma_ring_step_counts(gpu, orc, tile, mnk):
    """Whole-tile launches take the direct-to-LDS kernel: the 4-stage ring of the
    64x64 and 32x32 tiles, whose barrier sits in the middle of a K step, and the
    2-stage ring of the 128x128 and 256x256 tiles, whose barrier opens each step.
    Odd and even K-step counts, down to a single step, against the full reference
    (reference.hpp:199-211), and the same bits on a second launch.  The whole-tile
    epilogue stores 16 bytes per lane (8 for the 128x128 tile, whose lanes hold two
    adjacent columns; the 64x64 and 32x32 tiles transpose 4x4 blocks across lane
    quads first), so alpha / beta are checked on every tile too."""
    m, n, k = mnk
    a = orc.fill_random(m * k, 0x51A7 + k)
    b = orc.fill_random(k * n, 0x7E57 + k)
    t = gpu.GemmTile(*tile)
    want = orc.gemm(a, b, np.zeros(m * n, np.float32), m, n, k)
    poisoned = np.full(m * n, np.nan, np.float32)
    got = run_gemm(gpu, a, b, poisoned, m, n, k, 1.0, 0.0, gpu.GemmVariant.kMfmaF32, t)
    r = orc.compare(got, want, orc.tol_gemm(k), orc.abs_tol_gemm(k))
    assert r.ok, str(r)
    again = run_gemm(gpu, a, b, poisoned, m, n, k, 1.0, 0.0, gpu.GemmVariant.kMfmaF32, t)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    c0 = orc.fill_random(m * n, 0xC0FFEE + k)
    got = run_gemm(gpu, a, b, c0, m, n, k, 0.5, 2.0, gpu.GemmVariant.kMfmaF32, t)
    want = orc.gemm(a, b, c0, m, n, k, 0.5, 2.0)
    r = orc.compare(got, want, orc.tol_gemm(k), orc.abs_tol_gemm(k) * 2.0)
    assert r.ok, str(r)


@pytest.mark.parametrize("tile", [(64, 64, 32, 4, 4), (32, 32, 32, 2, 2)])
@pytest.mark.parametrize("n", [32, 64, 192, 512, 1024, 100, 257])
def test_gemm_wave_group_tiles(gpu, orc, tile, n):
    """The small tiles: 64x64 (one wave group, 4-stage mid-step ring) and 32x32,
    which folds its four wave groups' shares of K in a fixed order (whole tiles on
    the direct-to-LDS kernel; n = 100 and 257 on the staged kernel, whose 32x32
    tile also runs four groups): the full reference (reference.hpp:199-211) at the
    K-scaled tolerance, the same bits on a second launch, and beta = 0 never
    reading a NaN-poisoned C."""
    a = orc.fill_random(n * n, 0x6E33A + n)
    b = orc.fill_random(n * n, 0x8B10C + n)
    t = gpu.GemmTile(*tile)
    want = orc.gemm(a, b, np.zeros(n * n, np.float32), n, n, n)
    poisoned = np.full(n * n, np.nan, np.float32)
    got = run_gemm(gpu, a, b, poisoned, n, n, n, 1.0, 0.0, gpu.GemmVariant.kMfmaF32, t)
    r = orc.compare(got, want, orc.tol_gemm(n), orc.abs_tol_gemm(n))
    assert r.ok, str(r)
    again = run_gemm(gpu, a, b, poisoned, n, n, n, 1.0, 0.0, gpu.GemmVariant.kMfmaF32, t)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    # alpha / beta epilogue on the same kernel
    c0 = orc.fill_random(n * n, 0xC0FFEE)
    got = run_gemm(gpu, a, b, c0, n, n, n, 0.5, 2.0, gpu.GemmVariant.kMfmaF32, t)
    want = orc.gemm(a, b, c0, n, n, n, 0.5, 2.0)
    r = orc.compare(got, want, orc.tol_gemm(n), orc.abs_tol_gemm(n) * 2.0)
    assert r.ok, str(r)
