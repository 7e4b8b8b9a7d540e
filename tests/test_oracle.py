"""Pins the CPU oracle (oracle/mcke_oracle.c) before anything is judged by it.

Checks, each chosen so that a plausible restatement mistake (dropped term, wrong
index, transposed operand, wrong identity, float-vs-double accumulation) fails:

* the reference's 19 golden vectors and this build's 17 independent ones
  (bit-exact for "exact" cases; rel 1e-6 / abs 1e-7 for "approx", the
  reference's own bar, test_host_core.cpp:2317-2455);
* the reference's hand KATs (test_host_core.cpp:1339-1445);
* bit-equality with the reference's own oracle compiled from its tree
  (oracle/_ref) on seeded random inputs;
* closed forms: the C++ standard's mt19937_64 known answer, tol_gemm(256),
  the online-softmax algebra (identity, commutativity, associativity);
* brute force on tiny inputs against math.fsum / numpy float64.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from tests import golden_io

# ---------------------------------------------------------------------------
# Golden vectors
# ---------------------------------------------------------------------------
CASES = golden_io.all_cases()


def _run_oracle(orc, c):
    I, A, F = c["ints"], c["arrays"], c["floats"]
    if c["kind"] == "gemm":
        return orc.gemm(A["a"], A["b"], A["c"], I["m"], I["n"], I["k"], F["alpha"], F["beta"])
    if c["kind"] == "bias_act":
        return orc.bias_act(A["x"], A["bias"], I["rows"], I["cols"], I["act"])
    if c["kind"] == "row_reduce":
        return orc.row_reduce(A["x"], I["rows"], I["cols"], I["kind"])
    if c["kind"] == "row_softmax":
        return orc.row_softmax(A["x"], I["rows"], I["cols"])
    raise AssertionError(c["kind"])


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_oracle_matches_golden(orc, case):
    got = _run_oracle(orc, case)
    want = case["arrays"]["expect"]
    if case["mode"] == "exact":
        assert np.array_equal(golden_io.bits(got), golden_io.bits(want)), case["name"]
    else:
        r = orc.compare(got, want, 1e-6, 1e-7)
        assert r.ok, f"{case['name']}: {r}"


def test_reference_fixture_has_enough_exact_cases():
    ref_cases = golden_io.load("reference_vectors.json")
    assert len(ref_cases) == 19
    assert sum(c["mode"] == "exact" for c in ref_cases) >= 10


# ---------------------------------------------------------------------------
# Hand KATs (test_host_core.cpp:1339-1445)
# ---------------------------------------------------------------------------
def test_kat_bias_act(orc):
    x = np.array([1.0, -1.0, 0.5, -0.5], np.float32)
    b = np.zeros(2, np.float32)
    y = orc.bias_act(x, b, 2, 2, orc.ACT_RELU)
    assert list(y) == [1.0, 0.0, 0.5, 0.0]
    y = orc.bias_act(x, b, 2, 2, orc.ACT_NONE)
    assert y[1] == -1.0
    ye = orc.bias_act(x, b, 2, 2, orc.ACT_GELU_ERF)
    yt = orc.bias_act(x, b, 2, 2, orc.ACT_GELU_TANH)
    assert orc.compare(yt, ye, 1e-2).ok          # the two GELUs agree loosely ...
    assert not orc.compare(yt, ye, 1e-7).ok      # ... but are different functions


def test_kat_row_reduce(orc):
    x = np.array([1, 2, 3, 4, -5, -1, -9, -3], np.float32)
    assert list(orc.row_reduce(x, 2, 4, orc.KIND_SUM)) == [10.0, -18.0]
    assert list(orc.row_reduce(x, 2, 4, orc.KIND_MEAN)) == [2.5, -4.5]
    assert list(orc.row_reduce(x, 2, 4, orc.KIND_MAX)) == [4.0, -1.0]   # not 0


def test_kat_softmax(orc):
    y = orc.row_softmax(np.array([1, 2, 3, 4], np.float32), 1, 4)
    assert abs(float(np.sum(y, dtype=np.float64)) - 1.0) < 1e-6
    assert y[3] > y[2] > y[1] > y[0]
    y = orc.row_softmax(np.array([1, 2, 3, 1000], np.float32), 1, 4)
    assert not np.isnan(y).any()
    assert abs(y[3] - 1.0) < 1e-6 and y[0] == 0.0 and y[1] == 0.0
    y = orc.row_softmax(np.full(4, 5.0, np.float32), 1, 4)
    assert np.all(np.abs(y - 0.25) < 1e-6)


def test_kat_gemm(orc):
    a = np.array([1, 2, 3, 4], np.float32)
    b = np.array([5, 6, 7, 8], np.float32)
    c = orc.gemm(a, b, np.zeros(4, np.float32), 2, 2, 2)
    assert list(c) == [19, 22, 43, 50]
    c2 = orc.gemm(a, b, np.ones(4, np.float32), 2, 2, 2, 2.0, 3.0)
    assert c2[0] == 2 * 19 + 3 and c2[3] == 2 * 50 + 3
    a3 = np.arange(1, 7, dtype=np.float32)
    b3 = np.arange(1, 7, dtype=np.float32)
    c3 = orc.gemm(a3, b3, np.zeros(4, np.float32), 2, 2, 3)
    assert c3[0] == 22 and c3[1] == 28


def test_gemm_reads_c_even_when_beta_zero(orc):
    """reference.hpp:207-209 computes beta*prev unconditionally: 0*NaN = NaN."""
    c = np.full(4, np.nan, np.float32)
    out = orc.gemm(np.ones(4, np.float32), np.ones(4, np.float32), c, 2, 2, 2, 1.0, 0.0)
    assert np.isnan(out).all()


# ---------------------------------------------------------------------------
# Generators
# ---------------------------------------------------------------------------
def test_mt19937_64_known_answer(orc):
    # C++ standard [rand.predef]: 10000th output of default-seeded mt19937_64.
    assert orc.mt64_nth(5489, 10000) == 9981545732273789042


def test_fill_random_range_and_determinism(orc):
    a = orc.fill_random(100000, 123, -1.0, 1.0)
    b = orc.fill_random(100000, 123, -1.0, 1.0)
    assert np.array_equal(a, b)
    assert a.min() >= -1.0 and a.max() < 1.0
    assert abs(float(a.mean())) < 0.01
    u = orc.fill_random(1000, 5, 0.0, 1.0)
    # u = (e >> 40) / 2^24 is a multiple of 2^-24: exact in f32.
    assert np.all(u * (1 << 24) == np.floor(u * (1 << 24)))


def test_fill_normal_moments(orc):
    z = orc.fill_normal(1 << 20, 77, 0.0, 1.0).astype(np.float64)
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1.0) < 5e-3
    s = orc.fill_normal(1 << 18, 78, 0.0, 2.0).astype(np.float64)
    assert abs(s.std() - 2.0) < 2e-2


def test_fill_normal_first_pair_closed_form(orc):
    e1 = orc.mt64_nth(99, 1)
    e2 = orc.mt64_nth(99, 2)
    u1 = ((e1 >> 11) + 0.5) * 2.0 ** -53
    u2 = (e2 >> 11) * 2.0 ** -53
    r = math.sqrt(-2.0 * math.log(u1))
    z = orc.fill_normal(2, 99, 0.0, 1.0)
    assert z[0] == np.float32(r * math.cos(2 * math.pi * u2))
    assert z[1] == np.float32(r * math.sin(2 * math.pi * u2))


# ---------------------------------------------------------------------------
# Brute force / closed forms
# ---------------------------------------------------------------------------
def test_row_reduce_brute_force(orc):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((7, 513)).astype(np.float32)
    s = orc.row_reduce(x, 7, 513, orc.KIND_SUM)
    want = np.array([math.fsum(map(float, r)) for r in x], np.float32)
    assert np.array_equal(s, want)           # double accumulation of 513 terms is exact-rounded here
    assert np.array_equal(orc.row_reduce(x, 7, 513, orc.KIND_MAX), x.max(axis=1))
    m = orc.row_reduce(x, 7, 513, orc.KIND_MEAN)
    assert np.allclose(m, want / 513, rtol=1e-6)


def test_softmax_brute_force(orc):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((5, 77)) * 3).astype(np.float32)
    y = orc.row_softmax(x, 5, 77).reshape(5, 77)
    xd = x.astype(np.float64)
    e = np.exp(xd - xd.max(axis=1, keepdims=True))
    want = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
    assert np.max(np.abs(y - want)) <= 1e-7


def test_gemm_brute_force_is_not_transposed(orc):
    rng = np.random.default_rng(5)
    m, n, k = 7, 5, 9
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    got = orc.gemm(a, b, np.zeros(m * n, np.float32), m, n, k).reshape(m, n)
    want = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
    assert np.max(np.abs(got - want)) <= 1e-6 * np.max(np.abs(want))


def test_gelu_closed_forms(orc):
    assert orc.gelu_tanh(0.0) == 0.0 and orc.gelu_erf(0.0) == 0.0
    for v in (-3.0, -0.5, 0.7, 2.0):
        assert abs(orc.gelu_erf(v) - 0.5 * v * (1 + math.erf(v / math.sqrt(2)))) < 1e-15
        z = math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3)
        assert abs(orc.gelu_tanh(v) - 0.5 * v * (1 + math.tanh(z))) < 1e-15
    # tanh-form and erf-form differ in the 3rd decimal at most on [-4, 4]
    diffs = [abs(orc.gelu_tanh(v) - orc.gelu_erf(v)) for v in np.linspace(-4, 4, 81)]
    assert 1e-7 < max(diffs) < 1e-2


def test_tolerance_closed_forms(orc):
    assert abs(orc.tol_gemm(256) - 4 * 16 * 1.1920929e-7) < 1e-18
    assert 0.7e-5 < orc.tol_gemm(256) < 1e-5
    ks = [1, 3, 257, 4096, 8192]
    t = [orc.tol_gemm(k) for k in ks]
    assert t == sorted(t)
    assert orc.tol_gemm(0) == orc.tol_gemm(1)
    assert abs(orc.abs_tol_gemm(4096) - 3 * 0.5 * 4096 * 1.1920929e-7 / 3) < 1e-15


def test_compare_semantics(orc):
    want = np.array([1.0, 2.0, 0.0, 5.0], np.float32)
    assert orc.compare(want, want, 0.0).ok
    got = want.copy()
    got[1] = np.nan
    r = orc.compare(got, want, 1e-6)
    assert not r.ok and r.any_nan and r.mismatches == 1
    got = want.copy()
    got[3] = np.inf
    r = orc.compare(got, want, 1e-6)
    assert r.any_inf and r.mismatches == 1
    # the worst FLAGGED element is reported, not the largest abs error
    want = np.array([1e6, 1e-3], np.float32)
    got = np.array([1e6 + 0.0625, 2e-3], np.float32)
    r = orc.compare(got, want, 1e-6, 1e-8)
    assert r.mismatches == 1 and r.worst_index == 1


def test_spot_check_detects_corruption(orc):
    rng = np.random.default_rng(6)
    m, n, k = 33, 17, 65
    a = rng.uniform(-1, 1, m * k).astype(np.float32)
    b = rng.uniform(-1, 1, k * n).astype(np.float32)
    c = orc.gemm(a, b, np.zeros(m * n, np.float32), m, n, k)
    r = orc.spot_check_gemm(a, b, c, m, n, k, 1.0, 256, 0x5A11E, orc.tol_gemm(k),
                            orc.abs_tol_gemm(k))
    assert r.ok and r.checked == 256
    bad = c.copy()
    bad[:] += 0.01
    r = orc.spot_check_gemm(a, b, bad, m, n, k, 1.0, 256, 0x5A11E, orc.tol_gemm(k),
                            orc.abs_tol_gemm(k))
    assert r.mismatches == 256


# ---------------------------------------------------------------------------
# Online softmax algebra (softmax_online.hpp:73-112)
# ---------------------------------------------------------------------------
def test_online_identity_and_combine(orc):
    ident = orc.online_identity()
    m, d = orc.online_combine(ident, ident)
    assert not math.isnan(m) and not math.isnan(d) and d == 0.0
    s = orc.online_update(*ident, 1.5)
    assert s == (1.5, 1.0)
    assert orc.online_combine(s, ident) == s and orc.online_combine(ident, s) == s


def test_online_fold_equals_three_pass(orc):
    rng = np.random.default_rng(7)
    for n in (1, 2, 17, 31, 32, 33, 255, 256, 1000):
        x = (rng.standard_normal(n) * 4).astype(np.float32)
        st = orc.online_identity()
        for v in x:
            st = orc.online_update(st[0], st[1], float(v))
        assert st[0] == float(x.max())
        want = math.fsum(math.exp(float(v) - float(x.max())) for v in x)
        assert abs(st[1] - want) <= 1e-5 * want


def test_online_combine_assoc_commut(orc):
    rng = np.random.default_rng(8)
    parts = []
    for _ in range(3):
        x = (rng.standard_normal(50) * 5).astype(np.float32)
        st = orc.online_identity()
        for v in x:
            st = orc.online_update(st[0], st[1], float(v))
        parts.append(st)
    a, b, c = parts
    l = orc.online_combine(orc.online_combine(a, b), c)
    r = orc.online_combine(a, orc.online_combine(b, c))
    assert l[0] == r[0] and abs(l[1] - r[1]) <= 1e-6 * l[1]
    ab, ba = orc.online_combine(a, b), orc.online_combine(b, a)
    assert ab[0] == ba[0] and abs(ab[1] - ba[1]) <= 1e-6 * ab[1]


# ---------------------------------------------------------------------------
# Bit-equality with the reference's own oracle (oracle/_ref), when built
# ---------------------------------------------------------------------------
needs_ref = pytest.mark.skipif(
    not __import__("oracle").ref_available(),
    reason="oracle/_ref not built (the reference tree was absent when building)")


@needs_ref
def test_ref_generators_bit_equal(orc):
    R = orc.Ref
    assert R.mt64_nth(5489, 10000) == orc.mt64_nth(5489, 10000)
    for seed, lo, hi in ((0x6E33A, -1.0, 1.0), (0xB1A5B1A5, -0.5, 0.5), (7, 0.0, 1.0),
                         (0x50F7A11, -8.0, 8.0)):
        assert np.array_equal(golden_io.bits(R.fill_random(4099, seed, lo, hi)),
                              golden_io.bits(orc.fill_random(4099, seed, lo, hi)))


@needs_ref
@pytest.mark.parametrize("act", [0, 1, 2, 3])
def test_ref_bias_act_bit_equal(orc, act):
    x = orc.fill_normal(37 * 129, 1)
    b = orc.fill_random(129, 2, -0.5, 0.5)
    assert np.array_equal(golden_io.bits(orc.Ref.bias_act(x, b, 37, 129, act)),
                          golden_io.bits(orc.bias_act(x, b, 37, 129, act)))


@needs_ref
@pytest.mark.parametrize("kind", [0, 1, 2])
def test_ref_row_reduce_bit_equal(orc, kind):
    x = orc.fill_normal(13 * 1031, 3)
    assert np.array_equal(golden_io.bits(orc.Ref.row_reduce(x, 13, 1031, kind)),
                          golden_io.bits(orc.row_reduce(x, 13, 1031, kind)))


@needs_ref
def test_ref_softmax_bit_equal(orc):
    x = orc.fill_normal(11 * 333, 4, 0.0, 2.0)
    x[5 * 333 + 17] += 30.0
    assert np.array_equal(golden_io.bits(orc.Ref.row_softmax(x, 11, 333)),
                          golden_io.bits(orc.row_softmax(x, 11, 333)))


@needs_ref
def test_ref_softmax_special_values_bit_equal(orc):
    """Rows with -inf, NaN, +inf, +-3e38, tiny values and -FLT_MAX: the restatement
    keeps the reference's NaN handling in the max (std::max(m, v) keeps m) bit for bit,
    including which rows come out NaN."""
    fmax = np.finfo(np.float32).max
    cols = 37
    base = orc.fill_normal(8 * cols, 5, 0.0, 2.0).reshape(8, cols)
    base[0, 1] = -np.inf
    base[1, :] = -np.inf
    base[2, 9] = np.nan
    base[3, 36] = np.inf
    base[4, :3] = (3e38, -3e38, 1e38)
    base[5, :4] = (1e-30, -1e-30, 0.0, -0.0)
    base[6, (0, 3)] = -fmax
    base[7, :] = -np.inf
    base[7, 12] = -fmax
    x = base.ravel()
    got = orc.row_softmax(x, 8, cols)
    assert np.array_equal(golden_io.bits(orc.Ref.row_softmax(x, 8, cols)), golden_io.bits(got))
    assert np.isnan(got.reshape(8, cols)).all(axis=1).tolist() == [False, True, True, True,
                                                                   False, False, False, False]
    assert got[7 * cols + 12] == 1.0


@needs_ref
def test_ref_gemm_bit_equal(orc):
    m, n, k = 29, 31, 37
    a = orc.fill_random(m * k, 0x6E33A)
    b = orc.fill_random(k * n, 0x8B10C)
    c = orc.fill_random(m * n, 0xC0FFEE)
    for alpha, beta in ((1.0, 0.0), (0.5, 2.0)):
        assert np.array_equal(golden_io.bits(orc.Ref.gemm(a, b, c, m, n, k, alpha, beta)),
                              golden_io.bits(orc.gemm(a, b, c, m, n, k, alpha, beta)))


@needs_ref
def test_ref_compare_tolerances_spot_equal(orc):
    R = orc.Ref
    for k in (0, 1, 3, 256, 257, 4096, 8192):
        assert R.tol_gemm(k) == orc.tol_gemm(k)
        assert R.abs_tol_gemm(k) == orc.abs_tol_gemm(k)
        assert R.abs_tol_gemm(k, 2.5) == orc.abs_tol_gemm(k, 2.5)
    rng = np.random.default_rng(9)
    want = rng.standard_normal(1000).astype(np.float32)
    got = want + rng.standard_normal(1000).astype(np.float32) * 1e-5
    got[10] = np.nan
    got[20] = np.inf
    assert R.compare(got, want, 1e-6, 1e-7) == orc.compare(got, want, 1e-6, 1e-7)
    m, n, k = 21, 23, 25
    a = orc.fill_random(m * k, 1)
    b = orc.fill_random(k * n, 2)
    c = orc.gemm(a, b, np.zeros(m * n, np.float32), m, n, k)
    c[::7] += 1e-3
    assert (R.spot_check_gemm(a, b, c, m, n, k, 1.0, 300, 0x5A11E, 1e-5, 1e-6) ==
            orc.spot_check_gemm(a, b, c, m, n, k, 1.0, 300, 0x5A11E, 1e-5, 1e-6))


@needs_ref
def test_ref_online_bit_equal(orc):
    rng = np.random.default_rng(10)
    vals = (rng.standard_normal(200) * 10).astype(np.float32)
    st_r = st_o = orc.online_identity()
    for v in vals:
        st_r = orc.Ref.online_update(st_r[0], st_r[1], float(v))
        st_o = orc.online_update(st_o[0], st_o[1], float(v))
        assert st_r == st_o
    a, b = (1.5, 3.0), (-2.0, 7.0)
    assert orc.Ref.online_combine(a, b) == orc.online_combine(a, b)
    ident = orc.online_identity()
    assert orc.Ref.online_combine(ident, ident) == orc.online_combine(ident, ident)
