"""bench.py's contract with the driver, checked without a GPU.

* `--gpus N` above 1 exits non-zero with a message saying this build runs on one
  GPU (nothing is loaded on the device first);
* bad step counts are refused the same way;
* the HBM-traffic lines bench.py reads for `roofline.traffic` are present in the
  committed rocprof summary for every op of the step, and each is at least the
  op's algorithmic bytes (a plain copy calibrates the counters, so less would
  mean a miscalibration).
"""
from __future__ import annotations

import os
import re
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")

# Algorithmic bytes per launch of the step's memory-bound ops and the GEMM's
# compulsory A + B + C (fp32): the same formulas bench.py's numerators use.
ALGORITHMIC = {
    "gemm_mfma_f32": 3 * 8192 * 8192 * 4,
    "row_sum": (8192 * 8192 + 8192) * 4,
    "row_max": (8192 * 8192 + 8192) * 4,
    "full_sum": ((1 << 26) + 1) * 4,
    "softmax_c128": 2 * 32768 * 128 * 4,
    "softmax_c1024": 2 * 32768 * 1024 * 4,
    "softmax_c4096": 2 * 32768 * 4096 * 4,
    "bias_gelu_16384x4096": (2 * 16384 * 4096 + 4096) * 4,
    "bias_gelu_4096x1024": (2 * 4096 * 1024 + 1024) * 4,
}


def _run(*args):
    return subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True,
                          timeout=120)


def test_more_than_one_gpu_is_refused():
    p = _run("--gpus", "2")
    assert p.returncode != 0
    assert "one GPU" in p.stderr
    assert p.stdout.strip() == ""          # no JSON line for a refused run


def test_bad_step_counts_are_refused():
    assert _run("--steps", "0").returncode != 0
    assert _run("--warmup", "-1").returncode != 0


def test_committed_traffic_lines_cover_the_step():
    text = open(os.path.join(ROOT, "profiles", "bench_step_hbm_traffic.md")).read()
    traffic = {m.group(1): int(m.group(2))
               for m in re.finditer(r"^traffic\s+(\S+)\s+(\d+)\s*$", text, re.M)}
    for op, alg in ALGORITHMIC.items():
        assert op in traffic, f"no traffic line for {op}"
        assert traffic[op] >= alg * 0.999, f"{op}: {traffic[op]} < algorithmic {alg}"
