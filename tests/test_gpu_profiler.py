"""Profiler::time_op, write_csv and summary_table on the GPU, through the C++
launcher API (tests/cpp/profiler_probe.cpp, run in-process through
tests/cpp/bin/libprofiler_probe.so).

The reference's benches time every kernel this way (include/mcke/profiling/
profiler.hpp:213-265; bench/bias_act_bench.cpp:182-184, bench/gemm_bench.cpp:312-316)
and write the 13-column CSV of src/core/profiler.cpp:95-113.  The checks: the
timed launches computed the right answer (against the CPU oracle), each record
carries its op's ideal cost and `iters` samples with min <= median, and every CSV
column is the function of those fields the reference defines."""
from __future__ import annotations

import csv
import ctypes as C
import os

import numpy as np
import pytest

from tests.gpu_util import f32

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "bin", "libprofiler_probe.so")

HEADER = ["kernel", "variant", "median_ms", "min_ms", "iterations", "ideal_flops", "ideal_bytes",
          "achieved_gb_s", "achieved_tflops", "arithmetic_intensity", "attainable_tflops",
          "efficiency_pct", "bound"]


def test_time_op_records_csv_and_outputs(gpu, orc, tmp_path):
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is missing: build with `make -C tests/cpp`")
    lib = C.CDLL(LIB)
    fn = lib.mcke_test_profiler_probe
    fn.restype = C.c_int
    fn.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64,
                   C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int, C.c_int,
                   C.c_char_p, C.POINTER(C.c_double), C.POINTER(C.c_double),
                   C.c_char_p, C.c_size_t]

    rows, cols, n, warmup, iters = 256, 1024, 256, 2, 9
    x = orc.fill_normal(rows * cols, 0xB1A5AC7, 0.0, 1.0)
    bias = orc.fill_random(cols, 0xB1A5B1A5, -0.5, 0.5)
    a = orc.fill_random(n * n, 0x6E33A)
    b = orc.fill_random(n * n, 0x8B10C)
    D = gpu.DeviceBuffer
    dx, db, dy = D.from_array(f32(x)), D.from_array(f32(bias)), D(rows * cols * 4)
    da, dbm, dc = D.from_array(f32(a)), D.from_array(f32(b)), D(n * n * 4)

    path = str(tmp_path / "records.csv")
    med, mn = (C.c_double * 2)(), (C.c_double * 2)()
    buf = C.create_string_buffer(8192)
    print(f"profiler probe: bias_act {rows}x{cols}, gemm {n}^3, warmup {warmup}, iters {iters}",
          flush=True)
    rc = fn(dx.ptr, db.ptr, dy.ptr, rows, cols, da.ptr, dbm.ptr, dc.ptr, n, warmup, iters,
            path.encode(), med, mn, buf, len(buf))
    table = buf.value.decode()
    assert rc == 0, table
    gpu.device_synchronize()
    print(table)

    # The timed launches did the work.
    r = orc.compare(dy.download(rows * cols), orc.bias_act(x, bias, rows, cols, 3), 1e-6, 1e-6)
    assert r.ok, r
    want = orc.gemm(a, b, np.zeros(n * n, np.float32), n, n, n)
    r = orc.compare(dc.download(n * n), want, orc.tol_gemm(n), orc.abs_tol_gemm(n))
    assert r.ok, r

    with open(path, newline="") as f:
        rowsd = list(csv.reader(f))
    assert rowsd[0] == HEADER
    assert len(rowsd) == 3, rowsd
    ideal = {
        "bias_act": (10 * rows * cols, (2 * rows * cols + cols) * 4),   # ops_bias_act.cpp:51-100
        "gemm": (2 * n ** 3, 3 * n * n * 4),                            # ops_gemm.cpp:58-72
    }
    peak_tflops, peak_gb_s = 157.3, 8000.0
    ridge = peak_tflops * 1e12 / (peak_gb_s * 1e9)
    for i, row in enumerate(rowsd[1:]):
        rec = dict(zip(HEADER, row))
        name = rec["kernel"]
        flops, nbytes = ideal[name]
        assert rec["variant"] == ("gelu_tanh_vw4" if name == "bias_act" else "mfma_f32")
        assert int(rec["iterations"]) == iters
        assert int(rec["ideal_flops"]) == flops and int(rec["ideal_bytes"]) == nbytes
        median, minimum = float(rec["median_ms"]), float(rec["min_ms"])
        # The CSV prints 6 significant digits of the record's fields.
        assert median == pytest.approx(med[i], rel=1e-5) and minimum == pytest.approx(mn[i], rel=1e-5)
        assert 0.0 < minimum <= median < 100.0, (minimum, median)
        s = med[i] * 1e-3
        ai = flops / nbytes
        assert float(rec["achieved_gb_s"]) == pytest.approx(nbytes / s / 1e9, rel=1e-5)
        assert float(rec["achieved_tflops"]) == pytest.approx(flops / s / 1e12, rel=1e-5)
        assert float(rec["arithmetic_intensity"]) == pytest.approx(ai, rel=1e-5)
        att = min(ai * peak_gb_s * 1e9 / 1e12, peak_tflops)
        assert float(rec["attainable_tflops"]) == pytest.approx(att, rel=1e-5)
        assert float(rec["efficiency_pct"]) == pytest.approx(100.0 * flops / s / 1e12 / att, rel=1e-5)
        assert rec["bound"] == ("memory" if ai < ridge else "compute")
    # bias+GELU is memory-bound (AI 1.25), the 256^3 GEMM compute-bound (AI 42.7 > 19.7).
    assert [r[-1] for r in rowsd[1:]] == ["memory", "compute"]
    # The summary table: one line per record after the header and its 117-wide rule.
    lines = table.splitlines()
    assert lines[1] == "-" * 117 and len(lines) == 4
    assert lines[2].startswith("bias_act") and lines[3].startswith("gemm")
