"""TEST INFRASTRUCTURE ONLY: the CPU checker for the MCKE kernel layer.

ctypes bindings over two libraries built by ``oracle/Makefile``:

* ``liboracle.so`` -- the plain-C restatement in ``mcke_oracle.c`` of the
  reference's CPU oracle (tests/reference.hpp:101-426 and
  include/mcke/kernels/softmax_online.hpp:73-112 in the reference tree);
* ``_ref/libmcke_ref.so`` -- the reference's own header-only oracle compiled
  from the reference tree (optional; present when it was built here).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only to check or to time the CPU
reference.  The product library never calls it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libmcke_ref.so")

_F32P = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_I64 = C.c_int64
_U64 = C.c_uint64

# Enum values are the reference's (kernels.hpp:65,153,180,218).
ACT_NONE, ACT_RELU, ACT_GELU_ERF, ACT_GELU_TANH = 0, 1, 2, 3
KIND_SUM, KIND_MAX, KIND_MEAN = 0, 1, 2


class _CompareResult(C.Structure):
    _fields_ = [
        ("n", C.c_uint64),
        ("mismatches", C.c_uint64),
        ("max_abs_err", C.c_double),
        ("max_rel_err", C.c_double),
        ("worst_index", C.c_uint64),
        ("worst_got", C.c_double),
        ("worst_want", C.c_double),
        ("any_nan", C.c_int32),
        ("any_inf", C.c_int32),
    ]


class _SpotResult(C.Structure):
    _fields_ = [
        ("checked", C.c_uint64),
        ("mismatches", C.c_uint64),
        ("max_abs_err", C.c_double),
        ("max_rel_err", C.c_double),
    ]


@dataclass
class CompareResult:
    """Mirror of the reference's CompareResult (reference.hpp:215-241)."""

    n: int
    mismatches: int
    max_abs_err: float
    max_rel_err: float
    worst_index: int
    worst_got: float
    worst_want: float
    any_nan: bool
    any_inf: bool

    @property
    def ok(self) -> bool:
        return self.mismatches == 0 and not self.any_nan and not self.any_inf

    def __str__(self) -> str:
        s = f"{'OK' if self.ok else 'FAIL'}: {self.mismatches} / {self.n} mismatched"
        if self.any_nan:
            s += ", NaN present"
        if self.any_inf:
            s += ", Inf present"
        s += f"; max_abs={self.max_abs_err:.3g} max_rel={self.max_rel_err:.3g}"
        if self.mismatches:
            s += f"; worst at [{self.worst_index}] got {self.worst_got!r} want {self.worst_want!r}"
        return s


@dataclass
class SpotResult:
    checked: int
    mismatches: int
    max_abs_err: float
    max_rel_err: float

    @property
    def ok(self) -> bool:
        return self.mismatches == 0


def build() -> None:
    """Compile liboracle.so (and _ref/ when the reference tree is present)."""
    subprocess.run(["make", "-s", "-B", "-C", HERE], check=True)


def _load(path: str) -> C.CDLL:
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built; run `make -C {HERE}`")
    return C.CDLL(path)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        L = _load(LIB_PATH)
        L.orc_mt64_nth.argtypes = [_U64, _U64]
        L.orc_mt64_nth.restype = _U64
        L.orc_fill_random.argtypes = [_F32P, C.c_size_t, _U64, C.c_float, C.c_float]
        L.orc_fill_normal.argtypes = [_F32P, C.c_size_t, _U64, C.c_float, C.c_float]
        L.orc_gelu_erf.argtypes = [C.c_double]
        L.orc_gelu_erf.restype = C.c_double
        L.orc_gelu_tanh.argtypes = [C.c_double]
        L.orc_gelu_tanh.restype = C.c_double
        L.orc_bias_act.argtypes = [_F32P, _F32P, _F32P, _I64, _I64, C.c_int]
        L.orc_row_reduce.argtypes = [_F32P, _F32P, _I64, _I64, C.c_int]
        L.orc_row_softmax.argtypes = [_F32P, _F32P, _I64, _I64]
        L.orc_gemm.argtypes = [_F32P, _F32P, _F32P, _I64, _I64, _I64, C.c_float, C.c_float]
        L.orc_gemm_rows.argtypes = [_F32P, _F32P, _F32P, _I64, _I64, _I64, C.c_float,
                                    C.c_float, _I64, _I64]
        L.orc_compare.argtypes = [_F32P, _F32P, C.c_size_t, C.c_double, C.c_double,
                                  C.POINTER(_CompareResult)]
        L.orc_spot_check_gemm.argtypes = [_F32P, _F32P, _F32P, _I64, _I64, _I64, C.c_float,
                                          C.c_size_t, _U64, C.c_double, C.c_double,
                                          C.POINTER(_SpotResult)]
        for name in ("orc_tol_elementwise", "orc_tol_reduce4096", "orc_tol_softmax",
                     "orc_tol_gemm_k256", "orc_abs_tol_gelu_cancellation",
                     "orc_abs_tol_reduce_sum4096"):
            getattr(L, name).restype = C.c_double
            getattr(L, name).argtypes = []
        L.orc_tol_gemm.argtypes = [_I64]
        L.orc_tol_gemm.restype = C.c_double
        L.orc_abs_tol_gemm.argtypes = [_I64, C.c_double]
        L.orc_abs_tol_gemm.restype = C.c_double
        fp = C.POINTER(C.c_float)
        L.orc_online_update.argtypes = [C.c_float, C.c_float, C.c_float, fp, fp]
        L.orc_online_combine.argtypes = [C.c_float, C.c_float, C.c_float, C.c_float, fp, fp]
        L.orc_online_identity_m.restype = C.c_float
        u16 = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
        for name in ("orc_f32_to_bf16", "orc_f32_to_f16"):
            getattr(L, name).argtypes = [_F32P, u16, C.c_size_t]
        for name in ("orc_bf16_to_f32", "orc_f16_to_f32"):
            getattr(L, name).argtypes = [u16, _F32P, C.c_size_t]
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------------------
# Generators
# ---------------------------------------------------------------------------
def mt64_nth(seed: int, n: int) -> int:
    return int(lib().orc_mt64_nth(seed, n))


def fill_random(n: int, seed: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_random(out, n, seed, lo, hi)
    return out


def fill_normal(n: int, seed: int, mu: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_normal(out, n, seed, mu, sigma)
    return out


# ---------------------------------------------------------------------------
# References
# ---------------------------------------------------------------------------
def gelu_erf(x: float) -> float:
    return float(lib().orc_gelu_erf(x))


def gelu_tanh(x: float) -> float:
    return float(lib().orc_gelu_tanh(x))


def bias_act(x, bias, rows: int, cols: int, act: int) -> np.ndarray:
    x, bias = _f32(x), _f32(bias)
    y = np.empty(rows * cols, dtype=np.float32)
    lib().orc_bias_act(x, bias, y, rows, cols, act)
    return y


def row_reduce(x, rows: int, cols: int, kind: int) -> np.ndarray:
    x = _f32(x)
    out = np.empty(max(rows, 0), dtype=np.float32)
    lib().orc_row_reduce(x, out, rows, cols, kind)
    return out


def row_softmax(x, rows: int, cols: int) -> np.ndarray:
    x = _f32(x)
    y = np.empty(rows * cols, dtype=np.float32)
    lib().orc_row_softmax(x, y, rows, cols)
    return y


def gemm(a, b, c, m: int, n: int, k: int, alpha: float = 1.0, beta: float = 0.0) -> np.ndarray:
    """Returns a new array; `c` is the C input (read even when beta == 0)."""
    a, b = _f32(a), _f32(b)
    out = _f32(c).copy()
    lib().orc_gemm(a, b, out, m, n, k, alpha, beta)
    return out


def gemm_rows(a, b, c, m, n, k, alpha, beta, r0, r1) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    out = _f32(c).copy()
    lib().orc_gemm_rows(a, b, out, m, n, k, alpha, beta, r0, r1)
    return out


def compare(got, want, rel_tol: float, abs_tol: float = 1e-8) -> CompareResult:
    got, want = _f32(got).ravel(), _f32(want).ravel()
    assert got.size == want.size
    r = _CompareResult()
    lib().orc_compare(got, want, got.size, rel_tol, abs_tol, C.byref(r))
    return CompareResult(int(r.n), int(r.mismatches), r.max_abs_err, r.max_rel_err,
                         int(r.worst_index), r.worst_got, r.worst_want, bool(r.any_nan),
                         bool(r.any_inf))


def tol_gemm(k: int) -> float:
    return float(lib().orc_tol_gemm(k))


def abs_tol_gemm(k: int, amax: float = 1.0) -> float:
    return float(lib().orc_abs_tol_gemm(k, amax))


TOL = {}


def tolerances() -> dict:
    if not TOL:
        L = lib()
        TOL.update(
            elementwise=L.orc_tol_elementwise(),
            reduce4096=L.orc_tol_reduce4096(),
            softmax=L.orc_tol_softmax(),
            gemm_k256=L.orc_tol_gemm_k256(),
            abs_gelu=L.orc_abs_tol_gelu_cancellation(),
            abs_reduce_sum4096=L.orc_abs_tol_reduce_sum4096(),
        )
    return TOL


def spot_check_gemm(a, b, got, m, n, k, alpha, samples, seed, rel_tol, abs_tol) -> SpotResult:
    r = _SpotResult()
    lib().orc_spot_check_gemm(_f32(a), _f32(b), _f32(got), m, n, k, alpha, samples, seed,
                              rel_tol, abs_tol, C.byref(r))
    return SpotResult(int(r.checked), int(r.mismatches), r.max_abs_err, r.max_rel_err)


def online_update(m: float, d: float, x: float):
    om, od = C.c_float(), C.c_float()
    lib().orc_online_update(m, d, x, C.byref(om), C.byref(od))
    return om.value, od.value


def online_combine(a, b):
    om, od = C.c_float(), C.c_float()
    lib().orc_online_combine(a[0], a[1], b[0], b[1], C.byref(om), C.byref(od))
    return om.value, od.value


def online_identity():
    return float(lib().orc_online_identity_m()), 0.0


# ---------------------------------------------------------------------------
# 16-bit storage formats and the 16-bit-input GEMM
# ---------------------------------------------------------------------------
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2      # dtype.hpp:33-41


def to_16(x, dtype: int) -> np.ndarray:
    """float32 -> uint16 bit patterns of bf16 or fp16, rounded to nearest even."""
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    fn = lib().orc_f32_to_bf16 if dtype == DTYPE_BF16 else lib().orc_f32_to_f16
    fn(x.ravel(), out.ravel(), x.size)
    return out


def from_16(h, dtype: int) -> np.ndarray:
    """uint16 bit patterns of bf16 or fp16 -> float32 (exact)."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    fn = lib().orc_bf16_to_f32 if dtype == DTYPE_BF16 else lib().orc_f16_to_f32
    fn(h.ravel(), out.ravel(), h.size)
    return out


def gemm_lp(a16, b16, c, m, n, k, alpha, beta, ab_dtype: int, c_dtype: int) -> np.ndarray:
    """The reference GEMM (double accumulation, reference.hpp:199-211) over the
    decoded 16-bit inputs; C is read and returned in c_dtype (float32 array for
    DTYPE_F32, else uint16 bit patterns, rounded to nearest even from the float
    result)."""
    af, bf = from_16(a16, ab_dtype), from_16(b16, ab_dtype)
    cf = _f32(c) if c_dtype == DTYPE_F32 else from_16(c, c_dtype)
    out = gemm(af, bf, cf, m, n, k, alpha, beta)
    return out if c_dtype == DTYPE_F32 else to_16(out, c_dtype)


# ---------------------------------------------------------------------------
# The reference's own oracle (oracle/_ref), when it was built
# ---------------------------------------------------------------------------
_ref = None


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref() -> C.CDLL:
    global _ref
    if _ref is None:
        R = _load(REF_PATH)
        R.ref_mt64_nth.argtypes = [_U64, _U64]
        R.ref_mt64_nth.restype = _U64
        R.ref_fill_random.argtypes = [_F32P, C.c_size_t, _U64, C.c_float, C.c_float]
        R.ref_bias_act.argtypes = [_F32P, _F32P, _F32P, _I64, _I64, C.c_int]
        R.ref_row_reduce.argtypes = [_F32P, _F32P, _I64, _I64, C.c_int]
        R.ref_row_softmax.argtypes = [_F32P, _F32P, _I64, _I64]
        R.ref_gemm.argtypes = [_F32P, _F32P, _F32P, _I64, _I64, _I64, C.c_float, C.c_float]
        d9 = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
        R.ref_compare.argtypes = [_F32P, _F32P, C.c_size_t, C.c_double, C.c_double, d9]
        R.ref_tol_gemm.argtypes = [_I64]
        R.ref_tol_gemm.restype = C.c_double
        R.ref_abs_tol_gemm.argtypes = [_I64, C.c_double]
        R.ref_abs_tol_gemm.restype = C.c_double
        R.ref_spot_check_gemm.argtypes = [_F32P, _F32P, _F32P, _I64, _I64, _I64, C.c_float,
                                          C.c_size_t, _U64, C.c_double, C.c_double, d9]
        fp = C.POINTER(C.c_float)
        R.ref_online_update.argtypes = [C.c_float, C.c_float, C.c_float, fp, fp]
        R.ref_online_combine.argtypes = [C.c_float, C.c_float, C.c_float, C.c_float, fp, fp]
        _ref = R
    return _ref


class Ref:
    """Same call shapes as the module-level restatement, over oracle/_ref."""

    @staticmethod
    def mt64_nth(seed, n):
        return int(ref().ref_mt64_nth(seed, n))

    @staticmethod
    def fill_random(n, seed, lo=-1.0, hi=1.0):
        out = np.empty(n, dtype=np.float32)
        ref().ref_fill_random(out, n, seed, lo, hi)
        return out

    @staticmethod
    def bias_act(x, bias, rows, cols, act):
        y = np.empty(rows * cols, dtype=np.float32)
        ref().ref_bias_act(_f32(x), _f32(bias), y, rows, cols, act)
        return y

    @staticmethod
    def row_reduce(x, rows, cols, kind):
        out = np.empty(max(rows, 0), dtype=np.float32)
        ref().ref_row_reduce(_f32(x), out, rows, cols, kind)
        return out

    @staticmethod
    def row_softmax(x, rows, cols):
        y = np.empty(rows * cols, dtype=np.float32)
        ref().ref_row_softmax(_f32(x), y, rows, cols)
        return y

    @staticmethod
    def gemm(a, b, c, m, n, k, alpha=1.0, beta=0.0):
        out = _f32(c).copy()
        ref().ref_gemm(_f32(a), _f32(b), out, m, n, k, alpha, beta)
        return out

    @staticmethod
    def compare(got, want, rel_tol, abs_tol=1e-8):
        o = np.zeros(9, dtype=np.float64)
        got, want = _f32(got).ravel(), _f32(want).ravel()
        ref().ref_compare(got, want, got.size, rel_tol, abs_tol, o)
        return CompareResult(int(o[0]), int(o[1]), o[2], o[3], int(o[4]), o[5], o[6],
                             bool(o[7]), bool(o[8]))

    @staticmethod
    def tol_gemm(k):
        return float(ref().ref_tol_gemm(k))

    @staticmethod
    def abs_tol_gemm(k, amax=1.0):
        return float(ref().ref_abs_tol_gemm(k, amax))

    @staticmethod
    def spot_check_gemm(a, b, got, m, n, k, alpha, samples, seed, rel_tol, abs_tol):
        o = np.zeros(4, dtype=np.float64)
        ref().ref_spot_check_gemm(_f32(a), _f32(b), _f32(got), m, n, k, alpha, samples, seed,
                                  rel_tol, abs_tol, o)
        return SpotResult(int(o[0]), int(o[1]), o[2], o[3])

    @staticmethod
    def online_update(m, d, x):
        om, od = C.c_float(), C.c_float()
        ref().ref_online_update(m, d, x, C.byref(om), C.byref(od))
        return om.value, od.value

    @staticmethod
    def online_combine(a, b):
        om, od = C.c_float(), C.c_float()
        ref().ref_online_combine(a[0], a[1], b[0], b[1], C.byref(om), C.byref(od))
        return om.value, od.value
