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


def _fake_detail():
    """A detail record shaped like a full default bench run, with every section
    filled (sizes as large as a real run's)."""
    ops = []
    for name, bound in [("gemm_mfma_f32", "mfma")] + [(n, "hbm") for n in ALGORITHMIC if n != "gemm_mfma_f32"]:
        ops.append({
            "name": name, "shape": "X[16384x4096] b[4096]", "bound": bound, "avg_ms": 7.38312,
            "launches": 20, "buffer_sets": 2, "single_launch_median_ms": 7.39, "single_launch_min_ms": 7.2,
            "achieved": 6378.12, "unit": "GB/s" if bound == "hbm" else "TFLOP/s",
            "peak": 8000.0 if bound == "hbm" else 157.3, "frac": 0.7972,
            "algorithmic_bytes": ALGORITHMIC[name], "measured_peak": 6696.1, "frac_of_measured": 0.95,
            "hbm_traffic_bytes": ALGORITHMIC[name] + 12345,
            "parity": {"ok": True, "max_abs_err": 1.1920928955078125e-07, "max_rel_err": 3.2e-07,
                       "check": "every element against the oracle at BASELINE's tolerances " * 3},
            "effective_resident": {"avg_ms": 0.04, "achieved": 6900.0, "unit": "GB/s", "frac": 0.86,
                                   "note": "x" * 200},
        })
    cpu_ops = [{"name": o["name"], "shape": o["shape"], "runs": 5, "median_ms": 30.6, "min_ms": 30.1,
                "gb_s": 8.87, "gpu_speedup": 123.4} for o in ops[1:]]
    big = {"rows": [{"k": "v" * 100, "n": i} for i in range(200)]}
    return {
        "metric": "fp32 GEMM TFLOP/s + reduce/softmax/bias-GELU HBM GB/s, % of roofline",
        "value": 148.9, "unit": "TFLOP/s", "n_gpus": 1, "steps": 20, "warmup": 5,
        "ms_per_step": 8.1234, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic: seeded fill_random U[-1,1) / Box-Muller N(mu,sigma^2) at "
                                "BASELINE.json shapes, resident in HBM",
        "config": {"workload": "fp32 GEMM 8192^3 (kMfmaF32) headline; step also runs row sum/max "
                               "8192x8192, full sum 2^26, softmax 32768x{128,1024,4096}, "
                               "bias+GELU_tanh 16384x4096 and 4096x1024",
                   "gemm_tile": [256, 256, 32, 16, 16], "device": "AMD Instinct MI355X"},
        "roofline": {"bound": "mfma", "achieved": 148.9, "peak": 157.3, "unit": "TFLOP/s",
                     "frac": 0.9466, "traffic": 3659354214},
        "measured_peaks": {"mfma_f32_tflops": 154.6, "mfma_f32_launch_ms": 7.5, "stream_triad_gb_s": 6696.1,
                           "stream_copy_gb_s": 6672.7, "stream_copy_32mib_gb_s": 4964.8, "note": "n" * 600},
        "cpu_baseline": {"value": 8.9e-05, "unit": "TFLOP/s", "cores": 1, "kind": "reference",
                         "sample": "rows 0..0 of C for the 8192^3 GEMM (1x8192x8192), median of 5 runs, "
                                   "1 thread of 16 host cores, double accumulation in the reference's "
                                   "i-j-p order",
                         "gemm_slab_seconds": {"median": 1.51, "min": 1.5, "runs": 5},
                         "extrapolated_8192_s": 12517.0,
                         "parity_on_sample": {"ok": True, "max_abs_err": 1e-5, "max_rel_err": 1e-6, "tol": "t"},
                         "full_reference": [big], "row_parallel": big, "ops": cpu_ops, "ops_note": "o" * 300},
        "ops": ops,
        "gemm_sweep": [{"n": n, "tile": [256, 256, 32, 16, 16],
                        "mfma": {"avg_ms": 1.0, "launches": 100, "tflops": 149.01, "frac": 0.947},
                        "rocblas": {"avg_ms": 1.1, "launches": 90, "tflops": 141.42, "frac": 0.9},
                        "avg_ms": 1.0, "tflops": 149.01, "frac": 0.947, "vs_rocblas": 1.054}
                       for n in (512, 1024, 2048, 4096, 8192)],
        "gemm_lp": {"runs": [{"n": n, "ab": ab, "c": c, "tflops": 1511.62, "filler": big}
                             for n in (8192, 4096, 2048, 1024) for ab in ("bf16", "f16")
                             for c in ("bf16", "f32")], "vendor_bf16_rocblas": big},
        "graph": {"mlp_block": {"wall_ms": 7.6694, "tflops": 143.46, "bound_over_wall": 0.9245,
                                "nodes": big}, "reference_graphs": big, "gates_passed": True,
                  "capture_choice": {k: {"captured": False, "eager_us_per_run": 28.12,
                                         "replay_us_per_run": 32.37, "trials": 100}
                                     for k in ("mlp_512x256x1024_2streams", "mlp_64x64x256_2streams",
                                               "fanout_4x4_256_4streams", "chain32_64x1024_1stream")}},
        "ladder": {"gemm_4096": big, "reduce": big},
    }


def test_headline_is_compact_and_carries_the_contract():
    sys.path.insert(0, ROOT)
    import json
    import bench
    detail = _fake_detail()
    assert len(json.dumps(detail)) > 4 * bench.HEADLINE_MAX_BYTES     # the detail itself is large
    line = bench.headline(detail, "gpurun_out/bench_detail.json")
    text = json.dumps(line, separators=(",", ":"))
    assert len(text.encode()) <= bench.HEADLINE_MAX_BYTES, len(text)
    assert "\n" not in text
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
              "higher_is_better", "scaling", "vs_baseline", "dtype", "config"):
        assert k in line, k
    assert line["config"]["workload"].startswith("fp32 GEMM 8192^3")
    assert set(line["roofline"]) == {"bound", "achieved", "peak", "unit", "frac", "traffic"}
    for k in ("value", "unit", "cores", "kind", "sample"):
        assert line["cpu_baseline"][k] is not None, k
    assert len(line["ops"]) == len(ALGORITHMIC)
    for row in line["ops"]:
        assert len(row) == len(line["ops_columns"]) and row[5] is True
    assert line["all_parity_ok"] is True
    assert line["parity_checks"] == len(ALGORITHMIC)
    assert line["detail_file"] == "gpurun_out/bench_detail.json"
    # One failed check anywhere in the record shows in the headline.
    detail["graph"]["reference_graphs"] = {"fanout4x4": {"parity": {"ok": False}}}
    bad = bench.headline(detail, None)
    assert bad["all_parity_ok"] is False and bad["parity_checks"] == len(ALGORITHMIC) + 1
    assert json.loads(text) == line


def test_headline_without_cpu_leg_or_sections():
    sys.path.insert(0, ROOT)
    import bench
    detail = _fake_detail()
    for k in ("cpu_baseline", "gemm_sweep", "gemm_lp", "graph", "ladder", "measured_peaks"):
        detail[k] = None
    for s in detail["ops"]:
        s.pop("parity")
    line = bench.headline(detail, None)
    assert line["cpu_baseline"] is None and line["all_parity_ok"] is None
    assert line["roofline"]["frac"] == 0.9466
