"""The reference's own graph-layer test suite run against this implementation.

oracle/_ref/test_graph_host is the reference's tests/test_graph_host.cpp compiled
unchanged against this repository's include/ (no reference header on the include
path) and linked to libmcke_host.so / libmcke_amd.so (`make -C oracle refsuite`,
run by build() where the reference tree is present; the binary travels to the GPU
box prebuilt).  It is the reference's build with MCKE_WITH_CUDA=1: its test op
validates its tensors and launches nothing, and its three numerics-gate tests that
need its host compute backend report themselves skipped.

What it covers here: Graph (finalize, depths, levels, liveness, dead nodes, errors,
seeded random DAGs), the three stream policies and their event counts, the
happens-before relation and its validation, the memory planner under the three
policies with its race verifier, the cost model, and the executor's plan, replay,
poisoning and preconditions.

* Without a GPU (the CPU suite) every test passes except the executor tests, which
  create HIP streams and so fail with "no device"; the test checks exactly that.
* On the GPU every test passes.
"""
from __future__ import annotations

import json
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "oracle", "_ref", "test_graph_host")
REF_SRC = "/root/reference/tests/test_graph_host.cpp"

# The tests that construct a GraphExecutor and plan on HIP streams.
NEEDS_DEVICE = {"test_executor_end_to_end", "test_executor_preconditions",
                "test_executor_poison_and_arena_alignment", "test_numerics_gate_preconditions"}
# Tests the suite must run (a changed or truncated binary would otherwise pass).
MUST_RUN = NEEDS_DEVICE | {
    "test_hb_sequential", "test_graph_chain_and_liveness", "test_graph_finalize_errors",
    "test_graph_random_dags", "test_cost_model_roofline", "test_bit_mismatch_helper",
    "test_numerics_gate_on_host", "test_numerics_gate_catches_nondeterminism"}


def _run():
    if not os.path.exists(BIN):
        if os.path.exists(REF_SRC):
            pytest.fail(f"{BIN} is missing: run `make -C oracle refsuite` (build() does)")
        pytest.skip("the reference's graph test suite was not built (no reference tree here)")
    print(f"running {BIN}", flush=True)
    p = subprocess.run([BIN], capture_output=True, text=True, timeout=300)
    out = p.stdout + p.stderr
    ran, fails, current = [], {}, None
    for line in out.splitlines():
        if re.match(r"^test_\w+$", line):
            current = line
            ran.append(line)
        elif line.strip().startswith("FAIL"):
            fails.setdefault(current, []).append(line.strip())
    m = re.search(r"=== (\d+) checks, (\d+) failures ===", out)
    assert m, out[-2000:]
    return p.returncode, ran, fails, int(m.group(1)), int(m.group(2)), out


def test_reference_graph_suite_without_device():
    """The CPU suite: everything but the executor tests passes."""
    rc, ran, fails, checks, nfail, out = _run()
    assert MUST_RUN <= set(ran), sorted(MUST_RUN - set(ran))
    assert len(ran) >= 32 and checks > 80000, (len(ran), checks)
    unexpected = {t: f for t, f in fails.items() if t not in NEEDS_DEVICE}
    assert not unexpected, unexpected
    if nfail:
        # Only for want of a device.
        assert "hipErrorNoDevice" in out or "no ROCm-capable device" in out, out[-3000:]
    print(f"{len(ran)} tests, {checks} checks; failing only for want of a device: {sorted(fails)}")


@pytest.mark.gpu
def test_reference_graph_suite_on_gpu(gpu):
    """On the GPU the reference's whole graph suite passes against this implementation."""
    rc, ran, fails, checks, nfail, out = _run()
    print(out[-1500:])
    assert MUST_RUN <= set(ran), sorted(MUST_RUN - set(ran))
    assert nfail == 0 and rc == 0, fails
    assert "(skipped: needs the host compute backend" in out


ALLOC_BENCH = os.path.join(ROOT, "oracle", "_ref", "alloc_bench")


@pytest.mark.gpu
def test_reference_alloc_bench_on_gpu(gpu, tmp_path):
    """The reference's allocator benchmark (bench/alloc_bench.cpp), built unchanged
    against include/ and linked to this build's allocators, replays its traces
    through RawDeviceAllocator (hipMalloc), BuddyAllocator and FreeListAllocator on
    the GPU and completes: its own invariant checks (FATAL + abort on any failed
    allocation or bookkeeping mismatch) all hold, and it writes its latency and
    fragmentation CSVs."""
    if not os.path.exists(ALLOC_BENCH):
        if os.path.exists(REF_SRC):
            pytest.fail(f"{ALLOC_BENCH} is missing: run `make -C oracle refsuite` (build() does)")
        pytest.skip("the reference's allocator bench was not built (no reference tree here)")
    print(f"running {ALLOC_BENCH} in {tmp_path}", flush=True)
    p = subprocess.run([ALLOC_BENCH], capture_output=True, text=True, timeout=240, cwd=tmp_path)
    out = p.stdout + p.stderr
    print(out[-4000:])
    assert p.returncode == 0, out[-3000:]
    assert "FATAL" not in out
    csvs = sorted(f.name for f in (tmp_path / "reports").iterdir())
    assert any(c.startswith("alloc_latency_") for c in csvs), csvs
    assert any(c.startswith("alloc_fragmentation_") for c in csvs), csvs
    # The fragmentation tables are deterministic (a fixed-seed trace): every pool
    # row must read what the reference published for its own allocators
    # (tests/golden/alloc_fragmentation.json, from its RESULTS.md section 2b).
    golden = json.load(open(os.path.join(ROOT, "tests", "golden", "alloc_fragmentation.json")))
    tables = _fragmentation_tables(out)
    assert list(tables) == ["uniform_pow2", "dl_transformer", "dl_transformer_bypass"], list(tables)
    compared = 0
    for trace, rows in tables.items():
        for name, got in rows.items():
            want = golden["traces"][trace][name.split("/")[0]]
            for col in ("peak_reserved", "peak_blocks", "peak_requested", "block_eff",
                        "reserv_eff", "utilisation", "internal_waste", "oom"):
                assert got[col] == want[col], (trace, name, col, got[col], want[col])
            if name != "raw":
                assert got["largest_free_at_end"] == want["largest_free_at_end"], (trace, name)
            compared += 1
    assert compared == 3 * 7, compared


def _fragmentation_tables(out: str) -> dict:
    """The alloc bench's '2b. Fragmentation' tables, one per trace in print order:
    {trace: {allocator: {column: "value unit"}}}."""
    traces = re.findall(r"^--- trace: (\S+) -", out, re.M)
    sections = out.split("=== 2b. Fragmentation")[1:]
    assert len(sections) == len(traces), (len(sections), traces)
    cols = ["peak_reserved", "peak_blocks", "peak_requested", "block_eff", "reserv_eff",
            "utilisation", "internal_waste", "largest_free_at_end", "oom"]
    tables = {}
    for trace, sec in zip(traces, sections):
        rows = {}
        for line in sec.splitlines()[2:]:
            tok = line.split()
            if not tok or not re.match(r"^(raw|buddy|freelist)\b", tok[0]):
                if rows:
                    break
                continue
            vals, i = [], 1
            for col in cols:
                if col in ("block_eff", "reserv_eff", "utilisation", "oom"):
                    vals.append(tok[i])
                    i += 1
                else:
                    vals.append(f"{tok[i]} {tok[i + 1]}")
                    i += 2
            rows[tok[0]] = dict(zip(cols, vals))
        tables[trace] = rows
    return tables
