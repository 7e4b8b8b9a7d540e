#!/usr/bin/env python3
"""Benchmark of the MCKE kernel layer on one MI355X.

One *step* runs every hot-path kernel once at its BASELINE.json shape:

  gemm      fp32 C = A B, M = N = K = 8192, MFMA variant        (the headline)
  reduce    row sum and row max of X[8192 x 8192]
  full_sum  sum of 2^26 values (kTwoPass with rows = 1)
  softmax   row softmax of X[32768 x C], C in {128, 1024, 4096}
  bias_gelu GELU_tanh(X + b) for X[16384 x 4096] and X[4096 x 1024]

Inputs are generated on the host from seeds and are resident in HBM before the
timed region.  Every memory-bound kernel rotates over enough copies of its
buffers that one rotation moves >= 768 MiB, three times the 256 MB Infinity
Cache, so each launch reads its input from HBM, not from the cache.

Timing: W untimed steps, then exactly K timed steps bracketed by device
synchronisation and a pair of HIP events.  Inside the timed region the K launches
of each kernel run back to back on one stream between their own event pair, so a
kernel's average launch duration is (that pair's elapsed time) / K: dispatch gaps
are included, per-launch event overhead is not.  After the timed region a
diagnostic pass brackets single launches with their own events for median/min.

Also measured in the same run: the denominators (fp32 MFMA peak sustained for
about the GEMM's duration, a STREAM triad), the GEMM size sweep, the 16-bit-input
GEMM (`gemm_lp`: bf16 / fp16 in, fp32 accumulation, against the published 2.5
PFLOP/s dense peak, the measured 16-bit MFMA peak and rocBLAS on the same
shapes), the config-5 graph section and the CPU baseline.

The CPU leg (skipped with --no-cpu) checks every op's output at its timed shape
against the CPU oracle (ops[*].parity: the GEMM by the reference's 1024-entry spot
check, the others element by element at BASELINE's tolerances), then times the
CPU reference of the same GEMM on a bounded row slab (`cpu_baseline`).

Printed: one compact JSON line (rank 0, N = 1, under 4 KB), the last line of
stdout.  `value` is the GEMM's TFLOP/s; `roofline` is the GEMM's; `ops` holds one
short row per kernel with its roofline fraction and parity verdict.  The full
record (every section above, per-op detail, CPU legs) is written beforehand to
--detail-out (default gpurun_out/bench_detail.json), named in the line's
`detail_file`.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from __graft_entry__ import load_package  # noqa: E402

PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, AMD published
PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense fp32 matrix, AMD published
ROTATION_BYTES = 768 << 20     # bytes one rotation of a memory-bound op's buffers moves
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "bench_step_hbm_traffic.md")

METRIC = "fp32 GEMM TFLOP/s + reduce/softmax/bias-GELU HBM GB/s, % of roofline"


def log(msg: str) -> None:
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def profiled_traffic() -> dict[str, int]:
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary (lines `traffic <op> <bytes>`), keyed by op name; {} if absent."""
    out = {}
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                mt = re.match(r"^traffic\s+(\S+)\s+(\d+)\s*$", line)
                if mt:
                    out[mt.group(1)] = int(mt.group(2))
    except OSError:
        pass
    return out


class Op:
    """One kernel of the step: `launch(i)` runs it on buffer set i % sets; `work`
    is its algorithmic bytes (hbm) or flops (mfma) per launch."""

    def __init__(self, name, launch, bound, work, unit, shape, sets=1):
        self.name, self.launch, self.bound = name, launch, bound
        self.work, self.unit, self.shape, self.sets = work, unit, shape, sets
        self.total_ms = 0.0
        self.launches = 0
        self.single_ms: list[float] = []
        self.verify = None       # callable(oracle) -> dict, run in the CPU leg
        self.cpu_ref = None      # callable(ref) -> output: the CPU reference on this op's input
        self.parity = None
        self.copy_peak = None    # measured 1R+1W ceiling (GB/s), when measured
        self.resident_ms = None  # one buffer set back to back (effective), when measured

    def summary(self, measured_peak=None, traffic=None):
        avg = self.total_ms / self.launches
        if self.bound == "mfma":
            achieved = self.work / (avg * 1e-3) / 1e12
            peak, unit = PEAK_FP32_MFMA_TFLOPS, "TFLOP/s"
        else:
            achieved = self.work / (avg * 1e-3) / 1e9
            peak, unit = PEAK_HBM_GBS, "GB/s"
        t = np.array(self.single_ms or [avg], dtype=np.float64)
        out = {
            "name": self.name, "shape": self.shape, "bound": self.bound,
            "avg_ms": round(avg, 5), "launches": self.launches, "buffer_sets": self.sets,
            "single_launch_median_ms": round(float(np.median(t)), 5),
            "single_launch_min_ms": round(float(t.min()), 5),
            "achieved": round(achieved, 2), "unit": unit, "peak": peak,
            "frac": round(achieved / peak, 4),
            "algorithmic_" + ("flops" if self.bound == "mfma" else "bytes"): self.work,
        }
        if measured_peak:
            out["measured_peak"] = round(measured_peak, 2)
            out["frac_of_measured"] = round(achieved / measured_peak, 4)
        if traffic is not None:
            out["hbm_traffic_bytes"] = traffic
        if self.parity is not None:
            out["parity"] = self.parity
        if self.copy_peak and self.name.startswith(("softmax", "bias_gelu")):
            out["measured_copy_peak"] = round(self.copy_peak, 1)
            out["frac_of_copy"] = round(achieved / self.copy_peak, 4)
        if self.resident_ms:
            eff = self.work / (self.resident_ms * 1e-3) / 1e9
            out["effective_resident"] = {
                "avg_ms": round(self.resident_ms, 5), "achieved": round(eff, 1), "unit": "GB/s",
                "frac": round(eff / PEAK_HBM_GBS, 4),
                "note": "one buffer set, back to back: the working set fits the 256 MB "
                        "Infinity Cache, so this is effective, not HBM, bandwidth"}
        return out


def rotation_sets(bytes_per_launch: int) -> int:
    return max(1, min(32, math.ceil(ROTATION_BYTES / bytes_per_launch)))


def build_ops(m, stream, only=None):
    """The step's kernels; `only` (a set of op-name prefixes) restricts the set,
    and also enables the calibration op `copy_256mib` (a plain 256 MiB copy)."""
    D = m.DeviceBuffer
    ops, keep = [], []
    st = stream

    def want(name):
        return only is None or any(name.startswith(p) for p in only)

    def ck(status):
        if not status.ok():
            raise RuntimeError(str(status))

    def copies(arr, sets):
        bufs = [D.from_array(arr) for _ in range(sets)]
        keep.extend(bufs)
        return bufs

    def outputs(nbytes, sets):
        bufs = [D(nbytes) for _ in range(sets)]
        keep.extend(bufs)
        return bufs

    # --- GEMM 8192^3 (BASELINE configs[0] at its largest sweep size) ---------
    # Compute-bound: one buffer set (A and B are re-read from L2/MALL tiles anyway).
    n = 8192
    a = b = c = None
    if want("gemm_mfma_f32"):
        log("generating GEMM inputs (2 x 8192^2 U[-1,1))")
        a = D.from_array(m.fill_random(n * n, 0x6E33A))
        b = D.from_array(m.fill_random(n * n, 0x8B10C))
        c = D.zeros(n * n)
        tile = m.gemm_mfma_default_tile(n, n, n)
        keep += [a, b, c]
        ops.append(Op("gemm_mfma_f32", lambda i: ck(m.launch_gemm_f32(
            a, b, c, n, n, n, 1.0, 0.0, m.GemmVariant.kMfmaF32, tile, st)),
            "mfma", 2 * n * n * n, "flop", f"{n}x{n}x{n} tile {tile.astuple()}"))

        def verify_gemm(orc):
            ha, hb, hc = a.download(n * n), b.download(n * n), c.download(n * n)
            r = orc.spot_check_gemm(ha, hb, hc, n, n, n, 1.0, 1024, 0x5A11E, orc.tol_gemm(n),
                                    orc.abs_tol_gemm(n))
            return {"ok": r.checked == 1024 and r.mismatches == 0, "max_abs_err": r.max_abs_err,
                    "max_rel_err": r.max_rel_err,
                    "check": "1024-entry spot check in double (reference.hpp:401-426), rel "
                             f"tol_gemm({n}) + abs abs_tol_gemm({n})"}
        ops[-1].verify = verify_gemm

    # --- reductions --------------------------------------------
    R = C_ = 8192
    if want("row_sum") or want("row_max"):
        log("generating reduce input (8192^2 N(0,1))")
        red_bytes = (R * C_ + R) * 4
        sets = rotation_sets(red_bytes)
        hx = m.fill_normal(R * C_, 0x5EED12345)
        xr = copies(hx, sets)
        for kind, nm in ((m.ReduceKind.kSum, "row_sum"), (m.ReduceKind.kMax, "row_max")):
            if want(nm):
                outr = outputs(R * 4, sets)
                ops.append(Op(nm, (lambda i, kind=kind, s=sets, outr=outr: ck(m.launch_row_reduce_f32(
                    xr[i % s], outr[i % s], R, C_, kind, m.ReduceVariant.kWarpShuffle, st))),
                    "hbm", red_bytes, "byte", f"{R}x{C_}", sets))

                def verify_reduce(orc, kind=kind, outr=outr):
                    got = outr[0].download(R)
                    want_ = orc.row_reduce(hx, R, C_, int(kind))
                    if int(kind) == 1:
                        ok = bool(np.array_equal(got, want_))
                        return {"ok": ok, "check": "bit-exact against the double-accumulating CPU max"}
                    # the reference's term-magnitude floor (reference.hpp:312-321) for N(0,1) rows
                    floor = 5e-5 * (1.0 / 0.577) * np.sqrt(C_ / 4096.0)
                    r = orc.compare(got, want_, 1e-5, floor)
                    return {"ok": bool(r.ok), "max_abs_err": r.max_abs_err,
                            "max_rel_err": r.max_rel_err,
                            "check": f"every row, rel 1e-5 + abs {floor:.3g}"}
                ops[-1].verify = verify_reduce
                ops[-1].cpu_ref = lambda ref, kind=kind: ref.row_reduce(hx, R, C_, int(kind))
    N26 = 1 << 26
    if want("full_sum"):
        log("generating full-sum input (2^26 U[0,1))")
        fs_bytes = (N26 + 1) * 4
        sets = rotation_sets(fs_bytes)
        hxs = m.fill_random(N26, 0xF011, 0.0, 1.0)
        xs = copies(hxs, sets)
        wsb = m.row_reduce_workspace_bytes(1, N26, m.ReduceVariant.kTwoPass)
        ws, outs = D(wsb), D(4)
        keep += [ws, outs]
        ops.append(Op("full_sum", lambda i, s=sets: ck(m.launch_row_reduce_f32(
            xs[i % s], outs, 1, N26, m.ReduceKind.kSum, m.ReduceVariant.kTwoPass, ws, wsb, st)),
            "hbm", fs_bytes, "byte", "1x2^26", sets))

        def verify_full(orc):
            got = float(outs.download(1)[0])
            want_ = float(orc.row_reduce(hxs, 1, N26, 0)[0])
            rel = abs(got - want_) / abs(want_)
            return {"ok": rel <= 1e-5, "max_rel_err": rel, "got": got, "want": want_,
                    "check": "rel 1e-5 against the double-accumulating CPU sum"}
        ops[-1].verify = verify_full
        ops[-1].cpu_ref = lambda ref: ref.row_reduce(hxs, 1, N26, 0)

    # --- softmax -----------------------------------------------
    rows = 32768
    for cols in (128, 1024, 4096):
        if not want(f"softmax_c{cols}"):
            continue
        log(f"generating softmax input (32768x{cols} N(0,4) + 1% spikes)")
        x = m.fill_normal(rows * cols, 0x50F7A11 + cols, 0.0, 2.0)
        rng = np.random.default_rng(cols)
        spike_rows = rng.choice(rows, rows // 100, replace=False)
        x[spike_rows * cols + rng.integers(0, cols, spike_rows.size)] += 30.0
        sm_bytes = 2 * rows * cols * 4
        sets = rotation_sets(sm_bytes)
        dx, dy = copies(x, sets), outputs(rows * cols * 4, sets)
        ops.append(Op(f"softmax_c{cols}", (lambda i, dx=dx, dy=dy, cols=cols, s=sets: ck(
            m.launch_row_softmax_f32(dx[i % s], dy[i % s], rows, cols,
                                     m.SoftmaxVariant.kOnlineOnePass, st))),
            "hbm", sm_bytes, "byte", f"{rows}x{cols}", sets))

        def verify_softmax(orc, x=x, dy=dy, cols=cols):
            got = dy[0].download(rows * cols)
            r = orc.compare(got, orc.row_softmax(x, rows, cols), 0.0, 1e-6)
            sums = got.reshape(rows, cols).astype(np.float64).sum(axis=1)
            dev = float(np.max(np.abs(sums - 1.0)))
            return {"ok": bool(r.ok) and dev <= 1e-5, "max_abs_err": r.max_abs_err,
                    "max_row_sum_dev": dev,
                    "check": "every element within abs 1e-6 (BASELINE configs[2]); every row "
                             "sum within 1e-5"}
        ops[-1].verify = verify_softmax
        ops[-1].cpu_ref = lambda ref, x=x, cols=cols: ref.row_softmax(x, rows, cols)

    # --- bias + GELU(tanh) -------------------------------------
    for (br, bc) in ((16384, 4096), (4096, 1024)):
        if not want(f"bias_gelu_{br}x{bc}"):
            continue
        log(f"generating bias+GELU input ({br}x{bc})")
        bg_bytes = (2 * br * bc + bc) * 4
        sets = rotation_sets(bg_bytes)
        hxb = m.fill_normal(br * bc, 0xB1A5AC7 + br)
        hbb = m.fill_random(bc, 0xB1A5B1A5, -0.5, 0.5)
        dx, db = copies(hxb, sets), copies(hbb, sets)
        dy = outputs(br * bc * 4, sets)
        ops.append(Op(f"bias_gelu_{br}x{bc}", (lambda i, dx=dx, db=db, dy=dy, br=br, bc=bc, s=sets: ck(
            m.launch_bias_act_f32(dx[i % s], db[i % s], dy[i % s], br, bc,
                                  m.Activation.kGeluTanh, 4, st))),
            "hbm", bg_bytes, "byte", f"{br}x{bc}", sets))

        def verify_bias(orc, hxb=hxb, hbb=hbb, dy=dy, br=br, bc=bc):
            r = orc.compare(dy[0].download(br * bc), orc.bias_act(hxb, hbb, br, bc, 3), 1e-6, 1e-6)
            return {"ok": bool(r.ok), "max_abs_err": r.max_abs_err, "max_rel_err": r.max_rel_err,
                    "check": "every element abs 1e-6 + rel 1e-6 against the double GELU_tanh"}
        ops[-1].verify = verify_bias
        ops[-1].cpu_ref = lambda ref, hxb=hxb, hbb=hbb, br=br, bc=bc: ref.bias_act(hxb, hbb, br,
                                                                                 bc, 3)

    # --- calibration: a plain copy of known size (only when asked for) -------
    if only is not None and want("copy_256mib"):
        nc = 1 << 26
        sets = rotation_sets(2 * nc * 4)
        dx, dy = copies(np.ones(nc, np.float32), sets), outputs(nc * 4, sets)
        ops.append(Op("copy_256mib", lambda i, s=sets: ck(m.launch_activation_f32(
            dx[i % s], dy[i % s], nc, m.Activation.kNone, 4, st)), "hbm", 2 * nc * 4, "byte",
            "2^26 floats", sets))
    m.device_synchronize()
    return ops, keep, (a, b, c, n)


def run_steps(m, stream, ops, steps, record):
    """`steps` steps: for each op, `steps` launches back to back on rotating
    buffers, between the op's own event pair when `record`.  Returns the elapsed
    time of the whole region (ms), bracketed by synchronisation and events."""
    t0, t1 = m.Event(), m.Event()
    marks = [(m.Event(), m.Event()) for _ in ops] if record else None
    stream.synchronize()
    t0.record(stream)
    for i, op in enumerate(ops):
        if record:
            marks[i][0].record(stream)
        for s in range(steps):
            op.launch(s)
        if record:
            marks[i][1].record(stream)
    t1.record(stream)
    stream.synchronize()
    if record:
        for i, op in enumerate(ops):
            op.total_ms += marks[i][0].elapsed_ms(marks[i][1])
            op.launches += steps
    return t0.elapsed_ms(t1)


def single_launches(m, stream, ops, count):
    """Diagnostic: `count` launches of each op, each between its own event pair."""
    for op in ops:
        pairs = [(m.Event(), m.Event()) for _ in range(count)]
        for s in range(count):
            pairs[s][0].record(stream)
            op.launch(s)
            pairs[s][1].record(stream)
        stream.synchronize()
        op.single_ms = [e0.elapsed_ms(e1) for e0, e1 in pairs]


# Working sets at or below this many bytes fit MI355X's 256 MB Infinity Cache; for
# them the bench also reports an effective (cache-resident) figure.
RESIDENT_MAX_BYTES = 270_000_000


def resident_pass(m, stream, ops, count=50, warm=10):
    """Effective bandwidth beside the cold figure for the memory-bound ops whose
    working set fits the Infinity Cache: `count` back-to-back launches on buffer
    set 0 only (after `warm` untimed ones), between one event pair.  Outside the
    timed region; the cold rotation stays the reported rate."""
    for op in ops:
        if op.bound != "hbm" or op.work > RESIDENT_MAX_BYTES:
            continue
        for _ in range(warm):
            op.launch(0)
        e0, e1 = m.Event(), m.Event()
        e0.record(stream)
        for _ in range(count):
            op.launch(0)
        e1.record(stream)
        stream.synchronize()
        op.resident_ms = e0.elapsed_ms(e1) / count


def measured_peaks(m, stream, gemm_ms, iters=5):
    """The measured denominators: fp32 MFMA throughput sustained for about
    `gemm_ms` per launch (4 waves per SIMD), and a STREAM triad over 3 x 256 MiB
    arrays rotating over two sets."""
    D = m.DeviceBuffer
    out = {}
    info = m.query_device(0)
    # Two waves per SIMD (2 workgroups of 4 waves per CU): 1, 2 and 8 waves per
    # SIMD all sustain the same rate; 4 workgroups per CU (1024 on 256 CUs)
    # measured ~20% lower, from uneven placement of workgroups on CUs.
    blocks = info.sm_count * 2
    seed = D.from_array((np.arange(256, dtype=np.float32) % 7 - 3) * 0.25)
    sink = D(blocks * 256 * 4)
    per_iter = m.mfma_peak_flops(blocks, 1)
    mfma_iters = max(1, int(gemm_ms * 1e-3 * PEAK_FP32_MFMA_TFLOPS * 1e12 / per_iter))
    ck = lambda st: st.throw_if_error()   # noqa: E731
    ck(m.launch_mfma_peak_f32(seed, sink, blocks, mfma_iters, stream))
    e0, e1 = m.Event(), m.Event()
    e0.record(stream)
    for _ in range(iters):
        m.launch_mfma_peak_f32(seed, sink, blocks, mfma_iters, stream)
    e1.record(stream)
    stream.synchronize()
    ms = e0.elapsed_ms(e1) / iters
    out["mfma_f32_tflops"] = round(m.mfma_peak_flops(blocks, mfma_iters) / (ms * 1e-3) / 1e12, 2)
    out["mfma_f32_launch_ms"] = round(ms, 4)
    # Random operands, like the ops' own inputs: HBM moves constant data measurably
    # faster (a 256 MiB copy of zeros took 79.7 us against 82.5-85 us for varied
    # data on one box), which would inflate the ceilings the ops are held to.
    nt = 1 << 26
    hb = m.fill_random(nt, 0x7A1AD, 0.0, 1.0)
    hc = m.fill_random(nt, 0x7A1AE, 0.0, 1.0)
    arrs = [(D.from_array(hb), D.from_array(hc), D(nt * 4)) for _ in range(2)]
    for s in range(2):
        ck(m.launch_stream_triad_f32(arrs[s][0], arrs[s][1], arrs[s][2], 3.0, nt, stream))
    reps = 20
    e0.record(stream)
    for s in range(reps):
        bb, cc, aa = arrs[s % 2]
        m.launch_stream_triad_f32(bb, cc, aa, 3.0, nt, stream)
    e1.record(stream)
    stream.synchronize()
    ms = e0.elapsed_ms(e1) / reps
    out["stream_triad_gb_s"] = round(3 * nt * 4 / (ms * 1e-3) / 1e9, 1)
    got = arrs[1][2].download(16)
    want = (np.float32(3.0) * hc[:16] + hb[:16]).astype(np.float32)
    if not np.allclose(got, want, rtol=1e-6, atol=0):
        raise RuntimeError(f"stream triad produced {got[:4]}, expected {want[:4]}")
    # The read+write ceiling (one read, one write per element), for softmax and bias+act.
    for s in range(2):
        ck(m.launch_stream_copy_f32(arrs[s][0], arrs[s][2], nt, stream))
    e0.record(stream)
    for s in range(reps):
        m.launch_stream_copy_f32(arrs[s % 2][0], arrs[s % 2][2], nt, stream)
    e1.record(stream)
    stream.synchronize()
    ms = e0.elapsed_ms(e1) / reps
    out["stream_copy_gb_s"] = round(2 * nt * 4 / (ms * 1e-3) / 1e9, 1)
    if not np.array_equal(arrs[1][2].download(16), hb[:16]):
        raise RuntimeError("stream copy produced wrong values")
    # The same copy at the size of the two ~33.5 MB ops (softmax 32768x128, bias+GELU
    # 4096x1024): 16 MiB in + 16 MiB out over 24 rotating sets (805 MB per rotation,
    # 3x the Infinity Cache), back to back.  At this size a launch's ramp and drain
    # weigh as much as its transfer, so this, not the 256 MiB copy, is those ops'
    # read+write ceiling.
    ns, nsets = 1 << 22, 24
    small = [(D.from_array(hb[:ns]), D(ns * 4)) for _ in range(nsets)]
    for s in range(nsets):
        ck(m.launch_stream_copy_f32(small[s][0], small[s][1], ns, stream))
    reps_small = 10 * nsets
    e0.record(stream)
    for s in range(reps_small):
        m.launch_stream_copy_f32(small[s % nsets][0], small[s % nsets][1], ns, stream)
    e1.record(stream)
    stream.synchronize()
    ms = e0.elapsed_ms(e1) / reps_small
    out["stream_copy_32mib_gb_s"] = round(2 * ns * 4 / (ms * 1e-3) / 1e9, 1)
    if not np.array_equal(small[-1][1].download(16), hb[:16]):
        raise RuntimeError("small stream copy produced wrong values")
    del small
    out["note"] = ("mfma: blocks = 2 x CUs, 4 waves each, 4 chains of v_mfma_f32_32x32x2_f32, "
                   f"{mfma_iters} iterations (~GEMM launch length); triad: a = 3c + b over "
                   "3 x 256 MiB of U[0,1) data, two rotating sets; copy: y = x over 2 x 256 MiB, one float4 "
                   "per lane, non-temporal, two rotating sets (the 1-read + 1-write ceiling "
                   "of softmax and bias+act, frac_of_copy); copy_32mib: the same copy of "
                   "16 MiB in + 16 MiB out over 24 rotating sets (the ceiling of the two "
                   "~33.5 MB ops)")
    log(f"measured peaks: MFMA fp32 {out['mfma_f32_tflops']} TFLOP/s, "
        f"triad {out['stream_triad_gb_s']} GB/s, copy {out['stream_copy_gb_s']} GB/s, "
        f"copy at 32 MiB {out['stream_copy_32mib_gb_s']} GB/s")
    return out


def gemm_sweep(m, stream, warm_ms=150.0, timed_ms=40.0, sizes=(512, 1024, 2048, 4096, 8192)):
    """configs[0]'s sweep sizes (reported, not the headline), each beside the vendor
    library's sgemm (rocBLAS, the kCublasRef ceiling row) on the same buffers.

    Steady state: the engine clock ramps up over the first ~10-30 ms of matrix
    work after the host pauses (input generation), so each (size, variant) first
    runs launches for about `warm_ms`, then times back-to-back launches covering
    about `timed_ms` between one event pair."""
    D = m.DeviceBuffer
    out = []

    def batch(launch, count):
        e0, e1 = m.Event(), m.Event()
        e0.record(stream)
        for _ in range(count):
            launch()
        e1.record(stream)
        stream.synchronize()
        return e0.elapsed_ms(e1) / count

    for n in sizes:
        a = D.from_array(m.fill_random(n * n, 0x6E33A))
        b = D.from_array(m.fill_random(n * n, 0x8B10C))
        c = D.zeros(n * n)
        tile = m.gemm_mfma_default_tile(n, n, n)
        row = {"n": n, "tile": tile.astuple()}
        for key, variant, t in (("mfma", m.GemmVariant.kMfmaF32, tile),
                                ("rocblas", m.GemmVariant.kCublasRef, None)):
            def launch(variant=variant, t=t):
                m.launch_gemm_f32(a, b, c, n, n, n, 1.0, 0.0, variant, t, stream).throw_if_error()
            batch(launch, 3)          # first calls carry one-time set-up (rocBLAS handle, code load)
            est = batch(launch, 3)
            batch(launch, max(1, int(warm_ms / max(est, 1e-3))))
            iters = max(10, int(timed_ms / max(est, 1e-3)))
            ms = batch(launch, iters)
            tf = 2 * n ** 3 / (ms * 1e-3) / 1e12
            row[key] = {"avg_ms": round(ms, 5), "launches": iters, "tflops": round(tf, 2),
                        "frac": round(tf / PEAK_FP32_MFMA_TFLOPS, 4)}
        # Keep the flat fields of the MFMA row for readers of earlier lines.
        row.update(avg_ms=row["mfma"]["avg_ms"], tflops=row["mfma"]["tflops"],
                   frac=row["mfma"]["frac"],
                   vs_rocblas=round(row["mfma"]["tflops"] / row["rocblas"]["tflops"], 3))
        out.append(row)
        log(f"gemm sweep {n}^3: mfma {row['mfma']['tflops']:.1f} TFLOP/s (tile {tile.astuple()[:2]}), "
            f"rocBLAS {row['rocblas']['tflops']:.1f}")
    return out


def ladder_section(m, stream, sm_count):
    """Every variant the reference's own benches time, on MI355X, at BASELINE shapes:

      gemm     every GemmVariant at 4096^3 with rocBLAS timed first and last
               (bench/gemm_bench.cpp:565-573);
      reduce   tree / shuffle x sum / max / mean and two-pass sum at 8192^2, and
               shuffle vs two-pass at the starved 64 x 524288 (reduce_bench.cpp:225-240);
      softmax  three-pass vs online at 32768 x {128, 1024, 4096}
               (softmax_bench.cpp:220-223);
      bias_act fused vs the unfused pair (bias_add + activation) for ReLU, GELU_tanh
               and GELU_erf, the fusion ratio, the vector-width sweep at full and at
               starved occupancy (one workgroup row per CU), and the cache-resident
               512 x 512 control (bias_act_bench.cpp:261-311) at 16384 x 4096;
      effective the two ~33.5 MB ops on one buffer set (the working set stays in the
               256 MB Infinity Cache), beside their cold figure (rotating sets).

    Memory-bound rows rotate over >= 768 MiB of buffers unless marked resident.
    Returns (results, verify): verify(oracle) checks every row's output in the CPU
    leg (GEMM rows by the 1024-entry spot check) and stores it under "parity"."""
    D = m.DeviceBuffer
    out, checks = {}, []

    def timed(launch, warmup, iters, sets=1):
        for i in range(warmup):
            launch(i % sets)
        e0, e1 = m.Event(), m.Event()
        e0.record(stream)
        for i in range(iters):
            launch(i % sets)
        e1.record(stream)
        stream.synchronize()
        return e0.elapsed_ms(e1) / iters

    def hbm_row(name, ms, nbytes, **extra):
        gbs = nbytes / (ms * 1e-3) / 1e9
        return {"name": name, "avg_ms": round(ms, 5), "gb_s": round(gbs, 1),
                "frac": round(gbs / PEAK_HBM_GBS, 4), **extra}

    # --- GEMM ladder at 4096^3 ------------------------------------------------
    n = 4096
    ha, hb = m.fill_random(n * n, 0x6E33A), m.fill_random(n * n, 0x8B10C)
    a, b = D.from_array(ha), D.from_array(hb)
    V, T = m.GemmVariant, m.GemmTile
    ladder = [("naive_uncoalesced", V.kNaiveUncoalesced, T(), 1, 2),
              ("naive", V.kNaive, T(), 1, 2),
              ("tiled_smem_32", V.kTiledSmem, T(32, 32, 32, 1, 1), 2, 5),
              ("tiled_regblock", V.kTiledRegBlock, T(128, 128, 8, 8, 8), 2, 5),
              ("warp_tile_nodbuf", V.kWarpTileNoDbuf, T(128, 128, 8, 8, 8), 2, 5),
              ("warp_tile", V.kWarpTile, T(128, 128, 8, 8, 8), 2, 5),
              ("warp_tile_vec4", V.kWarpTileVec4, T(128, 128, 8, 8, 8), 2, 5),
              ("mfma_f32", V.kMfmaF32, m.gemm_mfma_default_tile(n, n, n), 10, 20)]
    rows = []

    def gemm_row(label, variant, tile, warmup, iters):
        c = D.zeros(n * n)
        ms = timed(lambda _i: m.launch_gemm_f32(a, b, c, n, n, n, 1.0, 0.0, variant, tile,
                                                stream).throw_if_error(), warmup, iters)
        tf = 2 * n ** 3 / (ms * 1e-3) / 1e12
        row = {"name": label, "avg_ms": round(ms, 4), "tflops": round(tf, 3),
               "frac": round(tf / PEAK_FP32_MFMA_TFLOPS, 4)}
        host_c = c.download(n * n, stream=stream)
        checks.append(("gemm " + label, row, lambda orc, hc=host_c: spot(orc, hc)))
        log(f"ladder gemm {label}: {ms:.3f} ms, {tf:.2f} TFLOP/s")
        return row

    def spot(orc, hc):
        r = orc.spot_check_gemm(ha, hb, hc, n, n, n, 1.0, 1024, 0x5A11E, orc.tol_gemm(n),
                                orc.abs_tol_gemm(n))
        return {"ok": r.checked == 1024 and r.mismatches == 0, "max_abs_err": r.max_abs_err,
                "check": "1024-entry spot check, rel tol_gemm + abs abs_tol_gemm"}

    rows.append(gemm_row("rocblas_first", V.kCublasRef, None, 5, 20))
    for label, variant, tile, w, it in ladder:
        rows.append(gemm_row(label, variant, tile, w, it))
    rows.append(gemm_row("rocblas_last", V.kCublasRef, None, 5, 20))
    out["gemm_4096"] = rows
    del a, b

    # --- reduce ladder --------------------------------------------------------
    RV = m.ReduceVariant
    red = []
    for (R, Cc, label) in ((8192, 8192, "8192x8192"), (64, 524288, "64x524288_starved")):
        hx = m.fill_normal(R * Cc, 0x5EED12345)
        sets = rotation_sets((R * Cc + R) * 4)
        xs = [D.from_array(hx) for _ in range(sets)]
        combos = ([(v, k) for v in (RV.kSmemTree, RV.kWarpShuffle) for k in (0, 1, 2)] +
                  [(RV.kTwoPass, 0)]) if R == 8192 else [(RV.kWarpShuffle, 0), (RV.kTwoPass, 0)]
        for var, kind in combos:
            o = D(R * 4)
            wsb = max(m.row_reduce_workspace_bytes(R, Cc, var), 4)
            ws = D(wsb)
            ms = timed(lambda i, var=var, kind=kind, o=o, ws=ws, wsb=wsb: m.launch_row_reduce_f32(
                xs[i], o, R, Cc, kind, var, ws, wsb, stream).throw_if_error(), 3, 20, sets)
            row = hbm_row(f"{var.name}_{['sum', 'max', 'mean'][kind]}_{label}", ms, (R * Cc + R) * 4)
            got = o.download(R, stream=stream)

            def check(orc, got=got, kind=kind, R=R, Cc=Cc, hx=hx):
                want = orc.row_reduce(hx, R, Cc, kind)
                if kind == 1:
                    return {"ok": bool(np.array_equal(got, want)), "check": "max bit-exact"}
                floor = 5e-5 * (1.0 / 0.577) * max(1.0, np.sqrt(Cc / 4096.0)) / (Cc if kind == 2 else 1)
                r = orc.compare(got, want, 1e-5, floor)
                return {"ok": bool(r.ok), "max_rel_err": r.max_rel_err,
                        "check": f"rel 1e-5 + abs {floor:.3g}"}
            checks.append(("reduce " + row["name"], row, check))
            red.append(row)
            log(f"ladder reduce {row['name']}: {ms * 1e3:.1f} us, {row['gb_s']} GB/s")
        del xs
    out["reduce"] = red

    # --- softmax: three-pass vs online ------------------------------------------
    SV = m.SoftmaxVariant
    smx = []
    for cols in (128, 1024, 4096):
        R = 32768
        hx = m.fill_normal(R * cols, 0x50F7A11 + cols, 0.0, 2.0)
        sets = rotation_sets(2 * R * cols * 4)
        xs, ys = [D.from_array(hx) for _ in range(sets)], [D(R * cols * 4) for _ in range(sets)]
        for var in (SV.kThreePass, SV.kOnlineOnePass):
            ms = timed(lambda i, var=var: m.launch_row_softmax_f32(xs[i], ys[i], R, cols, var,
                                                                  stream).throw_if_error(),
                       3, 20, sets)
            row = hbm_row(f"{var.name}_32768x{cols}", ms, 2 * R * cols * 4)
            got = ys[0].download(R * cols, stream=stream)
            checks.append(("softmax " + row["name"], row,
                           lambda orc, got=got, hx=hx, cols=cols: _abs_check(
                               orc, got, orc.row_softmax(hx, 32768, cols), 1e-6)))
            smx.append(row)
            log(f"ladder softmax {row['name']}: {ms * 1e3:.1f} us, {row['gb_s']} GB/s")
        del xs, ys
    out["softmax"] = smx

    # --- bias + activation ------------------------------------------------------
    BR, BC = 16384, 4096
    hxb = m.fill_normal(BR * BC, 0xB1A5AC7 + BR)
    hbb = m.fill_random(BC, 0xB1A5B1A5, -0.5, 0.5)
    sets = rotation_sets((2 * BR * BC + BC) * 4)
    xs = [D.from_array(hxb) for _ in range(sets)]
    bs = [D.from_array(hbb) for _ in range(sets)]
    ys = [D(BR * BC * 4) for _ in range(sets)]
    tmp = [D(BR * BC * 4) for _ in range(sets)]
    fused_bytes, unfused_bytes = (2 * BR * BC + BC) * 4, (4 * BR * BC + BC) * 4
    A = m.Activation
    ba, results = [], {}

    def fused(act, vw, max_rows=0):
        return timed(lambda i: m.launch_bias_act_f32(xs[i], bs[i], ys[i], BR, BC, act, vw, stream,
                                                     max_rows).throw_if_error(), 3, 20, sets)

    def unfused(act, vw):
        def pair(i):
            m.launch_bias_add_f32(xs[i], bs[i], tmp[i], BR, BC, vw, stream).throw_if_error()
            m.launch_activation_f32(tmp[i], ys[i], BR * BC, act, vw, stream).throw_if_error()
        return timed(pair, 3, 20, sets)

    for act in (A.kRelu, A.kGeluTanh, A.kGeluErf):
        f_ms = fused(act, 4)
        got_f = ys[0].download(BR * BC, stream=stream)
        u_ms = unfused(act, 4)
        got_u = ys[0].download(BR * BC, stream=stream)
        row = hbm_row(f"fused_vw4_{act.name}", f_ms, fused_bytes,
                      unfused_pair_ms=round(u_ms, 5), fusion_speedup=round(u_ms / f_ms, 3),
                      unfused_pair_gb_s=round(unfused_bytes / (u_ms * 1e-3) / 1e9, 1))
        checks.append(("bias_act " + row["name"], row,
                       lambda orc, gf=got_f, gu=got_u, act=act: _bias_check(
                           orc, gf, gu, hxb, hbb, BR, BC, int(act))))
        results[int(act)] = got_f
        ba.append(row)
        log(f"ladder bias {row['name']}: {f_ms * 1e3:.1f} us fused, {u_ms * 1e3:.1f} us unfused "
            f"({u_ms / f_ms:.2f}x)")
    for vw in (1, 2, 4):
        for label, max_rows in (("full", 0), ("starved", sm_count)):
            ms = fused(A.kGeluTanh, vw, max_rows)
            got = ys[0].download(BR * BC, stream=stream)
            row = hbm_row(f"gelu_tanh_vw{vw}_{label}", ms, fused_bytes, max_row_blocks=max_rows)
            checks.append(("bias_act " + row["name"], row,
                           lambda orc, got=got: {"ok": bool(np.array_equal(
                               got.view(np.uint32), results[int(A.kGeluTanh)].view(np.uint32))),
                               "check": "bit-equal to the fused vw4 output"}))
            ba.append(row)
            log(f"ladder bias {row['name']}: {ms * 1e3:.1f} us, {row['gb_s']} GB/s")
    del xs, bs, ys, tmp
    # cache-resident control: 512 x 512, one buffer set
    s = 512
    cx, cb = D.from_array(hxb[:s * s]), D.from_array(hbb[:s])
    cy, ct = D(s * s * 4), D(s * s * 4)
    f_ms = timed(lambda _i: m.launch_bias_act_f32(cx, cb, cy, s, s, A.kGeluTanh, 4, stream,
                                                  0).throw_if_error(), 10, 200)

    def pair_small(_i):
        m.launch_bias_add_f32(cx, cb, ct, s, s, 4, stream).throw_if_error()
        m.launch_activation_f32(ct, cy, s * s, A.kGeluTanh, 4, stream).throw_if_error()
    u_ms = timed(pair_small, 10, 200)
    ba.append({"name": "gelu_tanh_512x512_resident", "avg_ms": round(f_ms, 5),
               "unfused_pair_ms": round(u_ms, 5), "fusion_speedup": round(u_ms / f_ms, 3),
               "note": "one buffer set: the working set stays in cache"})
    out["bias_act"] = ba

    # --- effective (cache-resident) figures of the two ~33.5 MB ops -------------
    eff = []
    R, cols = 32768, 128
    hx = m.fill_normal(R * cols, 0x50F7A11 + cols, 0.0, 2.0)
    x1, y1 = D.from_array(hx), D(R * cols * 4)
    ms = timed(lambda _i: m.launch_row_softmax_f32(x1, y1, R, cols, SV.kOnlineOnePass,
                                                  stream).throw_if_error(), 10, 200)
    eff.append(hbm_row("softmax_c128_resident", ms, 2 * R * cols * 4))
    br, bc = 4096, 1024
    hx2, hb2 = m.fill_normal(br * bc, 0xB1A5AC7 + br), m.fill_random(bc, 0xB1A5B1A5, -0.5, 0.5)
    x2, b2, y2 = D.from_array(hx2), D.from_array(hb2), D(br * bc * 4)
    ms = timed(lambda _i: m.launch_bias_act_f32(x2, b2, y2, br, bc, A.kGeluTanh, 4, stream,
                                                0).throw_if_error(), 10, 200)
    eff.append(hbm_row("bias_gelu_4096x1024_resident", ms, (2 * br * bc + bc) * 4))
    for e in eff:
        log(f"ladder effective {e['name']}: {e['avg_ms'] * 1e3:.1f} us, {e['gb_s']} GB/s")
    out["effective_resident"] = eff

    def verify(orc):
        ok = True
        for label, row, check in checks:
            row["parity"] = check(orc)
            ok = ok and row["parity"]["ok"]
            if not row["parity"]["ok"]:
                log(f"ladder parity FAILED: {label}: {row['parity']}")
        return {"ok": ok}

    return out, verify


def _abs_check(orc, got, want, tol):
    r = orc.compare(got, want, 0.0, tol)
    return {"ok": bool(r.ok), "max_abs_err": r.max_abs_err, "check": f"every element abs {tol:g}"}


def _bias_check(orc, got_fused, got_unfused, hx, hb, rows, cols, act):
    """The fused output and the unfused pair's, each against the CPU oracle at abs
    1e-6 + rel 1e-6.  Where the fused kernel rounds v = x + b to f32 before the
    activation (ReLU, GELU_tanh), as the pair's bias_add does, the two agree bit for
    bit; the fused GELU_erf carries v exactly and may differ in the last bits."""
    want = orc.bias_act(hx, hb, rows, cols, act)
    rf = orc.compare(got_fused, want, 1e-6, 1e-6)
    ru = orc.compare(got_unfused, want, 1e-6, 1e-6)
    same = bool(np.array_equal(got_fused.view(np.uint32), got_unfused.view(np.uint32)))
    need_same = act != 2
    return {"ok": bool(rf.ok and ru.ok and (same or not need_same)),
            "max_abs_err": rf.max_abs_err, "unfused_max_abs_err": ru.max_abs_err,
            "unfused_same_bits": same,
            "check": "fused and unfused pair: abs 1e-6 + rel 1e-6 against the CPU oracle; "
                     "the same bits except for GELU_erf"}


PEAK_16BIT_MFMA_TFLOPS = 2500.0   # MI355X dense bf16 / fp16 matrix, AMD published


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def gemm_lp_section(m, stream, iters=10, with_peak=True, vendor_sizes=(8192, 4096, 2048, 1024)):
    """The 16-bit-input GEMM (bf16 / fp16 A and B, fp32 accumulation) at 8192^3 for
    each output type, and bf16 -> bf16 at the sweep sizes; beside it the 16-bit
    MFMA peak sustained for about the 8192^3 launch length and the vendor library
    (rocBLAS gemm_ex, bf16 -> bf16) on the same shapes.  Returns (result dict,
    verify closures for the CPU leg)."""
    D, DT = m.DeviceBuffer, m.DType
    runs, verifies, bufs = [], [], {}
    traffic = profiled_traffic()
    names = {int(DT.kBF16): "bf16", int(DT.kF16): "f16", int(DT.kF32): "f32"}

    def inputs(n, ab):
        key = (n, int(ab))
        if key not in bufs:
            ha = m.fill_random(n * n, 0x6E33A)
            hb = m.fill_random(n * n, 0x8B10C)
            if int(ab) == int(DT.kBF16):
                ha16, hb16 = to_bf16_bits(ha), to_bf16_bits(hb)
            else:
                ha16 = ha.astype(np.float16).view(np.uint16)
                hb16 = hb.astype(np.float16).view(np.uint16)
            bufs[key] = (D.from_array(ha16), D.from_array(hb16), ha16, hb16)
        return bufs[key]

    def batch(fn, count):
        e0, e1 = m.Event(), m.Event()
        e0.record(stream)
        for _ in range(count):
            fn()
        e1.record(stream)
        stream.synchronize()
        return e0.elapsed_ms(e1) / count

    def time_launch(fn, warm_ms=150.0, timed_ms=40.0):
        """Steady clock, as in gemm_sweep: about `warm_ms` of launches first, then
        at least `iters` launches covering about `timed_ms`."""
        batch(fn, 3)                  # first calls carry one-time set-up
        est = batch(fn, 3)
        batch(fn, max(1, int(warm_ms / max(est, 1e-3))))
        return batch(fn, max(iters, int(timed_ms / max(est, 1e-3))))

    cases = [(8192, DT.kBF16, DT.kBF16), (8192, DT.kBF16, DT.kF32), (8192, DT.kF16, DT.kF16),
             (8192, DT.kF16, DT.kF32), (4096, DT.kBF16, DT.kBF16), (2048, DT.kBF16, DT.kBF16),
             (1024, DT.kBF16, DT.kBF16)]
    for n, ab, cd in cases:
        da, db, ha16, hb16 = inputs(n, ab)
        dc = D(n * n * (4 if int(cd) == int(DT.kF32) else 2))
        tile = m.gemm_lp_default_tile(n, n, n)

        def launch(da=da, db=db, dc=dc, n=n, ab=ab, cd=cd, tile=tile):
            st = m.launch_gemm_lp(da, db, dc, ab, cd, n, n, n, 1.0, 0.0, tile, stream)
            if not st.ok():
                raise RuntimeError(str(st))
        ms = time_launch(launch)
        tf = 2 * n ** 3 / (ms * 1e-3) / 1e12
        c_bytes = 4 if int(cd) == int(DT.kF32) else 2
        run = {"n": n, "ab": names[int(ab)], "c": names[int(cd)], "tile": tile.astuple(),
               "avg_ms": round(ms, 5), "tflops": round(tf, 1),
               "frac": round(tf / PEAK_16BIT_MFMA_TFLOPS, 4),
               "algorithmic_bytes": 2 * n * n * 2 + n * n * c_bytes}
        tr = traffic.get(f"gemm_lp_{run['ab']}_{run['c']}_{n}")
        if tr is not None:
            run["hbm_traffic_bytes"] = tr
        runs.append(run)
        log(f"gemm_lp {names[int(ab)]}->{names[int(cd)]} {n}^3: {ms:.4f} ms  {tf:.1f} TFLOP/s")
        if n == 8192:
            def verify(orc, run=run, dc=dc, ha16=ha16, hb16=hb16, n=n, ab=ab, cd=cd):
                af, bf = orc.from_16(ha16, int(ab)), orc.from_16(hb16, int(ab))
                if int(cd) == int(DT.kF32):
                    got, extra = dc.download(n * n), 0.0
                else:
                    got = orc.from_16(dc.download(n * n, np.uint16), int(cd))
                    extra = 2.0 ** -7 if int(cd) == int(DT.kBF16) else 2.0 ** -10
                r = orc.spot_check_gemm(af, bf, got, n, n, n, 1.0, 1024, 0x5A11E,
                                        orc.tol_gemm(n) + extra, orc.abs_tol_gemm(n))
                run["parity"] = {"ok": r.checked == 1024 and r.mismatches == 0,
                                 "max_abs_err": r.max_abs_err, "max_rel_err": r.max_rel_err,
                                 "check": "1024-entry spot check in double over the decoded "
                                          f"16-bit inputs, rel tol_gemm({n})"
                                          + (f" + {extra:g} (output ulp)" if extra else "")
                                          + f" + abs abs_tol_gemm({n})"}
                return run["parity"]
            verifies.append((f"gemm_lp {run['ab']}->{run['c']}", verify))

    out = {"peak_published_tflops": PEAK_16BIT_MFMA_TFLOPS, "runs": runs}
    if with_peak:
        info = m.query_device(0)
        blocks = info.sm_count * 2
        seed = D.from_array((np.arange(256, dtype=np.float32) % 7 - 3) * 0.25)
        sink = D(blocks * 256 * 4)
        ms8 = next(r["avg_ms"] for r in runs if r["n"] == 8192)
        iters_pk = max(1, int(ms8 * 1e-3 * 1.8e15 / m.mfma_peak_lp_flops(blocks, 1)))
        for dt in (DT.kBF16, DT.kF16):
            ms = time_launch(lambda dt=dt: m.launch_mfma_peak_lp(dt, seed, sink, blocks, iters_pk,
                                                                 stream).throw_if_error())
            out[f"measured_peak_{names[int(dt)]}_tflops"] = round(
                m.mfma_peak_lp_flops(blocks, iters_pk) / (ms * 1e-3) / 1e12, 1)
        for r in runs:
            pk = out[f"measured_peak_{r['ab']}_tflops"]
            r["frac_of_measured"] = round(r["tflops"] / pk, 4)
        out["peak_note"] = (f"blocks = 2 x CUs, 4 waves each, 4 chains of "
                            f"v_mfma_f32_32x32x16_{{bf16,f16}}, {iters_pk} iterations (~8192^3 "
                            "launch length)")
        # Engine clock under random operands that change with every MFMA, for the two
        # 16-bit MFMA forms at equal flops (mcke_launch_mfma_clock_lp): the reason the
        # GEMM's whole-tile kernel uses 16x16x32.  Alternating launches of ~45 ms.
        ticks = D(blocks * 16)
        rng = np.random.default_rng(0x51A7)
        probe = {}
        for dt in (DT.kBF16, DT.kF16):
            vals = rng.uniform(-1.0, 1.0, 256 * 8 * 8).astype(np.float32)
            bits = to_bf16_bits(vals) if int(dt) == int(DT.kBF16) else \
                vals.astype(np.float16).view(np.uint16)
            dbits = D.from_array(np.ascontiguousarray(bits))
            it_ck = max(1, int(0.045 * 2.0e15 / m.mfma_clock_lp_flops(blocks, 1)))
            res = {}
            for rep in range(3):
                for shape, label in ((0, "32x32x16"), (1, "16x16x32")):
                    e0, e1 = m.Event(), m.Event()
                    e0.record(stream)
                    m.launch_mfma_clock_lp(dt, shape, dbits, sink, ticks, blocks, it_ck,
                                           stream).throw_if_error()
                    e1.record(stream)
                    stream.synchronize()
                    ms = e0.elapsed_ms(e1)
                    tk = ticks.download(blocks * 2, np.uint64).reshape(blocks, 2).astype(np.float64)
                    if rep > 0:   # the first round warms the part
                        res.setdefault(label, []).append(
                            (m.mfma_clock_lp_flops(blocks, it_ck) / (ms * 1e-3) / 1e12,
                             float(np.mean(tk[:, 0] / (tk[:, 1] * 10.0)))))
            probe[names[int(dt)]] = {
                lab: {"tflops": round(float(np.median([v[0] for v in vs])), 1),
                      "clock_ghz": round(float(np.median([v[1] for v in vs])), 3)}
                for lab, vs in res.items()}
            log(f"16-bit MFMA clock probe {names[int(dt)]}: " + ", ".join(
                f"{lab} {v['tflops']} TFLOP/s at {v['clock_ghz']} GHz"
                for lab, v in probe[names[int(dt)]].items()))
        out["mfma_clock_probe"] = probe
        out["mfma_clock_probe_note"] = (
            f"blocks = 2 x CUs, 4 waves each; 8 (32x32x16) or 16 (16x16x32) MFMAs per "
            f"iteration over 8 operand registers of random 16-bit values, {it_ck} iterations "
            "(~45 ms); clock = s_memtime cycles / s_memrealtime span, mean over workgroups; "
            "median of 2 alternating rounds after one warm-up round")
        log(f"measured 16-bit MFMA peak: bf16 {out['measured_peak_bf16_tflops']} TFLOP/s, "
            f"f16 {out['measured_peak_f16_tflops']} TFLOP/s")
    # Vendor library on the same shapes (bf16 -> bf16, rocBLAS gemm_ex), for comparison
    # only.  The engine clock under 16-bit MFMA load follows the power drawn in the
    # last milliseconds, so the two kernels are timed in alternating blocks of about
    # 40 ms (8 each, median), after a warm-up of both: timed one after the other,
    # whichever runs second inherits the other's thermal state.
    vendor = []
    for n in vendor_sizes:
        da, db, _, _ = inputs(n, DT.kBF16)
        dc = D(n * n * 2)
        tile = m.gemm_lp_default_tile(n, n, n)

        def ours(da=da, db=db, dc=dc, n=n, tile=tile):
            m.launch_gemm_lp(da, db, dc, DT.kBF16, DT.kBF16, n, n, n, 1.0, 0.0, tile,
                             stream).throw_if_error()

        def theirs(da=da, db=db, dc=dc, n=n):
            m.launch_gemm_lp_vendor(da, db, dc, DT.kBF16, DT.kBF16, n, n, n, 1.0, 0.0,
                                    stream).throw_if_error()
        est = batch(ours, 3)
        cnt = max(iters, int(40.0 / max(est, 1e-3)))
        batch(ours, 2 * cnt)
        batch(theirs, 2 * cnt)
        a, b = [], []
        for r in range(8):
            pair = (ours, theirs) if r % 2 == 0 else (theirs, ours)
            for fn in pair:
                (a if fn is ours else b).append(batch(fn, cnt))
        ms_a, ms_b = sorted(a)[4], sorted(b)[4]
        tf = lambda ms, n=n: round(2 * n ** 3 / (ms * 1e-3) / 1e12, 1)
        vendor.append({"n": n, "avg_ms": round(ms_b, 5), "tflops": tf(ms_b),
                       "ours_interleaved_tflops": tf(ms_a),
                       "ours_over_vendor": round(ms_b / ms_a, 3)})
        log(f"vendor rocBLAS gemm_ex bf16->bf16 {n}^3: {ms_b:.4f} ms  {tf(ms_b)} TFLOP/s; "
            f"ours in the same alternating blocks {tf(ms_a)} TFLOP/s ({ms_b / ms_a:.3f}x)")
    out["vendor_bf16_rocblas"] = vendor
    out["vendor_note"] = ("ours and rocBLAS timed in alternating ~40 ms blocks, median of 8 "
                          "each; 'runs' above are the separate steady-state timings")
    return out, verifies


def graph_section(m, steps=5, warmup=2, gate_repeats=20, capture=True):
    """BASELINE config 5 through the GraphExecutor (buddy allocator, chain-greedy
    schedule, happens-before arena reuse):
      * the MLP block X[4096x4096] -> GEMM(W1 4096x16384) -> bias+GELU -> GEMM(W2)
        -> bias -> softmax, per-node times and roofline fractions;
      * a 4x4 fan-out of 2048^3 GEMM chains on 4 streams (chain-greedy and
        level-parallel) vs the same graph on one stream, with the overlap (sum of
        node medians / wall, both from a profiled run) and buddy statistics;
      * the reference graph bench's five graphs at its shapes (mcke_amd.graph.
        REFERENCE_GRAPHS: diamond of 2048^3 GEMMs, chain of 16 bias+GELU nodes,
        4x4 fan-out of starved bias+GELU chains, starved diamond, transformer
        block), under the three schedules, with the same overlap figure;
      * every wall time from an executor without timing events between the nodes
        (wall_ms), beside the profiled run's (wall_profiled_ms);
      * for every timed plan the launch-bound ratio (host enqueue time of one
        run / device time of one run, bench/graph_bench.cpp:437-441).
    Every one of these graphs also runs the numerics gate (3 schedules x 3 memory
    policies x `gate_repeats`, bench/graph_bench.cpp:444-471), and every node of
    a per-tensor plan is read back to the host.  Returns (results, verify), where
    verify(oracle) checks those stages in the CPU leg and stores the outcome under
    results[*]["parity"]."""
    from mcke_amd import graph as G

    out = {}
    host = {}

    def timed_runs(ex, n):
        """Average device ms per run over n back-to-back runs, and the median host
        time (us) one run_async call takes to enqueue its launches."""
        st = ex.stream()
        e0, e1 = m.Event(), m.Event()
        for _ in range(warmup):
            ex.run_async()
        ex.synchronize()
        enq = []
        e0.record(st)
        for _ in range(n):
            t0 = time.perf_counter()
            ex.run_async()
            enq.append(time.perf_counter() - t0)
        e1.record(st)
        ex.synchronize()
        return e0.elapsed_ms(e1) / n, float(np.median(enq)) * 1e6

    def launch_bound(wall_ms, enqueue_us):
        return round((enqueue_us / 1e3) / wall_ms, 4)

    T, D, F = 4096, 4096, 16384
    log("config 5: MLP block 4096x4096 -> 16384 -> 4096")
    mlp_in = {"x": m.fill_normal(T * D, 0x3001, 0.0, 1.0),
              "W1": m.fill_normal(D * F, 0x3002, 0.0, 0.02),
              "b1": m.fill_normal(F, 0x3003, 0.0, 0.01),
              "W2": m.fill_normal(F * D, 0x3004, 0.0, 0.02),
              "b2": m.fill_normal(D, 0x3005, 0.0, 0.01)}
    def mlp_executor(profile):
        g, t = G.mlp_block(T, D, F)
        ex = G.Executor(g, allocator=G.AllocatorKind.kBuddy, schedule=G.SchedulePolicy.kChainGreedy,
                        memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=4, profile=profile,
                        profile_slots=warmup + steps)
        ex.plan()
        for k, v in mlp_in.items():
            ex.set_input(t[k], v)
        return ex, t

    # The wall time comes from a plan without timing events; the per-node medians
    # from a second, profiled executor of the same plan (its events sit between
    # the nodes and cost the multi-stream plans measurable time).
    ex, t = mlp_executor(False)
    wall, enq = timed_runs(ex, steps)
    y_timed = ex.read(t["y"], T * D)
    info = ex.plan_info()
    ex.plan()     # re-plan: the new arena comes from the block the old one returned
    alloc_stats = ex.allocator_stats()
    ex.close()
    ex, _ = mlp_executor(True)
    wall_prof, _ = timed_runs(ex, steps)
    timings = ex.timings()
    ex.close()
    nodes = []
    for x in timings:
        is_gemm = x["name"].startswith("gemm")
        ach = (x["flops"] / (x["median_ms"] * 1e-3) / 1e12) if is_gemm else \
              (x["bytes"] / (x["median_ms"] * 1e-3) / 1e9)
        peak = PEAK_FP32_MFMA_TFLOPS if is_gemm else PEAK_HBM_GBS
        nodes.append({"name": x["name"], "median_ms": round(x["median_ms"], 4),
                      "achieved": round(ach, 1), "unit": "TFLOP/s" if is_gemm else "GB/s",
                      "frac": round(ach / peak, 4)})
    bound_ms = sum(max(x["flops"] / (PEAK_FP32_MFMA_TFLOPS * 1e12), x["bytes"] / (PEAK_HBM_GBS * 1e9))
                   for x in timings) * 1e3
    out["mlp_block"] = {
        "shape": f"X[{T}x{D}] W1[{D}x{F}] W2[{F}x{D}]", "wall_ms": round(wall, 4),
        "wall_profiled_ms": round(wall_prof, 4),
        "enqueue_us": round(enq, 2), "launch_bound_ratio": launch_bound(wall, enq),
        "tflops": round(info["total_flops"] / (wall * 1e-3) / 1e12, 2),
        "roofline_bound_ms": round(bound_ms, 4), "bound_over_wall": round(bound_ms / wall, 4),
        "nodes": nodes, "arena_bytes": info["arena_bytes"], "naive_bytes": info["naive_bytes"],
        "allocator": alloc_stats,
    }
    log(f"config 5 MLP: {wall:.3f} ms/run, {out['mlp_block']['tflops']} TFLOP/s")

    # Parity material: every stage of a per-tensor plan (checked in the CPU leg),
    # the timed plan's output bits against it, and the numerics gate.
    g, t = G.mlp_block(T, D, F)
    ex = G.Executor(g, schedule=G.SchedulePolicy.kSequential,
                    memory=G.MemoryPolicy.kAllocPerTensor, num_streams=1)
    ex.plan()
    for k, v in mlp_in.items():
        ex.set_input(t[k], v)
    ex.run_sync()
    host["mlp"] = {"gemm1": ex.read(t["gemm1"], T * F), "h": ex.read(t["h"], T * F),
                   "gemm2": ex.read(t["gemm2"], T * D), "z": ex.read(t["z"], T * D),
                   "y": ex.read(t["y"], T * D)}
    ex.close()
    same_bits = bool(np.array_equal(y_timed.view(np.uint32), host["mlp"]["y"].view(np.uint32)))
    del y_timed
    g, t = G.mlp_block(T, D, F)
    ex = G.Executor(g, num_streams=4, validate_numerics=True)
    ex.plan()
    for k, v in mlp_in.items():
        ex.set_input(t[k], v)
    gate = ex.validate_numerics(repeats=gate_repeats)
    ex.close()
    out["mlp_block"]["gate"] = {"passed": gate.passed, "configs": gate.configs_compared,
                                "repeats": gate_repeats, "detail": gate.detail}
    out["mlp_block"]["timed_plan_same_bits_as_per_tensor_plan"] = same_bits
    log(f"config 5 MLP: numerics gate {'PASS' if gate.passed else 'FAIL'}, timed plan same "
        f"bits: {same_bits}")

    # The same block with each GEMM -> bias+act pair fused into the GEMM's epilogue
    # (GemmBiasAct nodes): C never goes to memory and two launches go.  Same plan
    # settings; its H, Z and Y must carry the unfused per-tensor plan's bits.
    def mlp_fused_executor(**kw):
        g, t = G.mlp_block_fused(T, D, F)
        ex = G.Executor(g, **kw)
        ex.plan()
        for k, v in mlp_in.items():
            ex.set_input(t[k], v)
        return ex, t

    # Fused and unfused timed in alternating blocks (their difference, about 1%, is
    # below the run-to-run spread of two separate measurements).
    ex, t = mlp_fused_executor(allocator=G.AllocatorKind.kBuddy,
                               schedule=G.SchedulePolicy.kChainGreedy,
                               memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=4)
    ex_u, _ = mlp_executor(False)
    blocks_f, blocks_u, enq_fs = [], [], []
    for _ in range(4):
        w, e = timed_runs(ex, steps)
        blocks_f.append(w)
        enq_fs.append(e)
        blocks_u.append(timed_runs(ex_u, steps)[0])
    ex_u.close()
    wall_f, enq_f = float(np.median(blocks_f)), float(np.median(enq_fs))
    wall_u_alt = float(np.median(blocks_u))
    y_fused_timed = ex.read(t["y"], T * D)
    info_f = ex.plan_info()
    ex.close()
    ex, t = mlp_fused_executor(profile=True, profile_slots=warmup + steps, num_streams=4)
    timed_runs(ex, steps)
    timings_f = ex.timings()
    ex.close()
    ex, t = mlp_fused_executor(schedule=G.SchedulePolicy.kSequential,
                               memory=G.MemoryPolicy.kAllocPerTensor, num_streams=1)
    ex.run_sync()
    fused_same = {k: bool(np.array_equal(ex.read(t[k], T * (F if k == "h" else D)).view(np.uint32),
                                         host["mlp"][k].view(np.uint32))) for k in ("h", "z", "y")}
    ex.close()
    fused_same["y_timed_plan"] = bool(np.array_equal(y_fused_timed.view(np.uint32),
                                                     host["mlp"]["y"].view(np.uint32)))
    del y_fused_timed
    out["mlp_block_fused"] = {
        "shape": out["mlp_block"]["shape"], "nodes_in_graph": info_f["num_nodes"],
        "wall_ms": round(wall_f, 4), "enqueue_us": round(enq_f, 2),
        "tflops": round(info_f["total_flops"] / (wall_f * 1e-3) / 1e12, 2),
        "unfused_wall_ms_alternating": round(wall_u_alt, 4),
        "speedup_over_unfused": round(wall_u_alt / wall_f, 4),
        "blocks": f"4 alternating blocks of {steps} runs each, fused then unfused; medians",
        "nodes": [{"name": x["name"], "median_ms": round(x["median_ms"], 4)} for x in timings_f],
        "arena_bytes": info_f["arena_bytes"],
        "parity": {"ok": all(fused_same.values()), "same_bits_as_unfused": fused_same},
    }
    log(f"config 5 MLP, fused epilogues: {wall_f:.3f} ms/run against {wall_u_alt:.3f} unfused "
        f"in alternating blocks ({wall_u_alt / wall_f:.3f}x), "
        f"{out['mlp_block_fused']['tflops']} TFLOP/s, bits as unfused: {fused_same}")

    n, B, Dp = 2048, 4, 4
    fan_n = n
    fan_w = m.fill_random(n * n, 0x4000, -0.03125, 0.03125)
    fan_xs = [m.fill_random(n * n, 0x4001 + k) for k in range(B)]

    def fanout_executor(sched, streams, memory=G.MemoryPolicy.kReuseHappensBefore, **kw):
        g, t = G.gemm_fanout(B, Dp, n)
        ex = G.Executor(g, allocator=G.AllocatorKind.kBuddy, schedule=sched, memory=memory,
                        num_streams=streams, **kw)
        ex.plan()
        ex.set_input(t["W"], fan_w)
        for k in range(B):
            ex.set_input(t["xs"][k], fan_xs[k])
        return ex, t

    fan = {}
    for label, sched, streams in (("sequential", G.SchedulePolicy.kSequential, 1),
                                  ("level_parallel_4streams", G.SchedulePolicy.kLevelParallel, 4),
                                  ("chain_greedy_4streams", G.SchedulePolicy.kChainGreedy, 4)):
        ex, _ = fanout_executor(sched, streams)
        wall, enq = timed_runs(ex, steps)
        info = ex.plan_info()
        ex.plan()     # re-plan: exercises the allocator's reuse of the returned arena
        alloc_stats = ex.allocator_stats()
        ex.close()
        ex, _ = fanout_executor(sched, streams, profile=True, profile_slots=warmup + steps)
        wall_prof, _ = timed_runs(ex, steps)
        node_sum = sum(x["median_ms"] for x in ex.timings())
        fan[label] = {"wall_ms": round(wall, 4), "wall_profiled_ms": round(wall_prof, 4),
                      "node_sum_ms": round(node_sum, 4), "overlap": round(node_sum / wall_prof, 3),
                      "tflops": round(info["total_flops"] / (wall * 1e-3) / 1e12, 2),
                      "enqueue_us": round(enq, 2), "launch_bound_ratio": launch_bound(wall, enq),
                      "streams": info["num_streams_used"], "events": info["num_events"],
                      "waits": info["waits_dedup"], "arena_bytes": info["arena_bytes"],
                      "allocator": alloc_stats}
        log(f"config 5 fan-out {label}: {wall:.3f} ms, overlap {node_sum / wall_prof:.2f}")
        ex.close()
    for label in ("level_parallel_4streams", "chain_greedy_4streams"):
        fan[label]["speedup_vs_sequential"] = round(fan["sequential"]["wall_ms"] /
                                                    fan[label]["wall_ms"], 3)
    fan["speedup_vs_sequential"] = fan["chain_greedy_4streams"]["speedup_vs_sequential"]
    ex, t = fanout_executor(G.SchedulePolicy.kChainGreedy, 4, memory=G.MemoryPolicy.kAllocPerTensor)
    ex.run_sync()
    host["fan"] = [[ex.read(tid, n * n) for tid in chain] for chain in t["nodes"]]
    ex.close()
    ex, _ = fanout_executor(G.SchedulePolicy.kChainGreedy, 4, validate_numerics=True)
    gate = ex.validate_numerics(repeats=gate_repeats)
    ex.close()
    fan["gate"] = {"passed": gate.passed, "configs": gate.configs_compared,
                   "repeats": gate_repeats, "detail": gate.detail}
    log(f"config 5 fan-out: numerics gate {'PASS' if gate.passed else 'FAIL'}")
    out["fanout4x4_gemm2048"] = fan

    # The reference graph bench's five graphs at its shapes (bench/graph_bench.cpp:
    # 100-215, run at :477-481): a diamond of 2048^3 GEMMs, a chain of 16 bias+GELU
    # nodes over X[4096 x 4096], 4 chains of 4 bias+GELU nodes over X[2048 x 2048]
    # starved to 10 row blocks, a diamond whose middle nodes are bias+GELU starved
    # to 40 row blocks, and the transformer block (4096, 1024, 4096).  Each is
    # timed under the three schedules, then run through the numerics gate (3 x 3
    # x gate_repeats, :444-471), and every node is kept from a per-tensor plan
    # for the CPU leg's parity check.
    def numel(g, tid):
        k = 1
        for d in g.shape(tid):
            k *= d
        return k

    ref_graphs, ref_nodes = {}, {}
    ref_steps = max(steps, 20)     # these graphs run 0.2-0.8 ms
    for gname in G.REFERENCE_GRAPHS:
        rows = {}
        for label, sched, streams in (("sequential", G.SchedulePolicy.kSequential, 1),
                                      ("level_parallel", G.SchedulePolicy.kLevelParallel, 4),
                                      ("chain_greedy", G.SchedulePolicy.kChainGreedy, 4)):
            def ref_executor(profile):
                g, t, inputs = G.reference_graph(gname, m.fill_random, m.fill_normal)
                ex = G.Executor(g, allocator=G.AllocatorKind.kBuddy, schedule=sched,
                                memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=streams,
                                profile=profile, profile_slots=warmup + ref_steps)
                ex.plan()
                for tid, arr in inputs.items():
                    ex.set_input(tid, arr)
                return ex
            ex = ref_executor(False)
            wall, enq = timed_runs(ex, ref_steps)
            info = ex.plan_info()
            ex.close()
            ex = ref_executor(True)
            wall_prof, _ = timed_runs(ex, ref_steps)
            node_sum = sum(x["median_ms"] for x in ex.timings())
            rows[label] = {"wall_ms": round(wall, 4), "wall_profiled_ms": round(wall_prof, 4),
                           "node_sum_ms": round(node_sum, 4),
                           "overlap": round(node_sum / wall_prof, 3), "enqueue_us": round(enq, 2),
                           "launch_bound_ratio": launch_bound(wall, enq),
                           "streams": info["num_streams_used"], "events": info["num_events"],
                           "waits": info["waits_dedup"],
                           "arena_bytes": info["arena_bytes"], "naive_bytes": info["naive_bytes"]}
            ex.close()
        for label in ("level_parallel", "chain_greedy"):
            rows[label]["speedup_vs_sequential"] = round(rows["sequential"]["wall_ms"] /
                                                         rows[label]["wall_ms"], 3)
        # Every node from a per-tensor plan, for the CPU leg.
        g, t, inputs = G.reference_graph(gname, m.fill_random, m.fill_normal)
        sizes = {k: numel(g, v) for k, v in t.items() if k != "outs"}
        ex = G.Executor(g, schedule=G.SchedulePolicy.kSequential,
                        memory=G.MemoryPolicy.kAllocPerTensor, num_streams=1)
        ex.plan()
        for tid, arr in inputs.items():
            ex.set_input(tid, arr)
        ex.run_sync()
        ref_nodes[gname] = (
            {k: ex.read(v, sizes[k]) for k, v in t.items() if k != "outs" and v not in inputs},
            {k: inputs[v] for k, v in t.items() if k != "outs" and v in inputs})
        ex.close()
        g, t, inputs = G.reference_graph(gname, m.fill_random, m.fill_normal)
        ex = G.Executor(g, num_streams=4, validate_numerics=True)
        ex.plan()
        for tid, arr in inputs.items():
            ex.set_input(tid, arr)
        gate = ex.validate_numerics(repeats=gate_repeats)
        ex.close()
        rows["gate"] = {"passed": gate.passed, "configs": gate.configs_compared,
                        "repeats": gate_repeats, "detail": gate.detail}
        ref_graphs[gname] = rows
        log(f"graph {gname}: " + ", ".join(f"{k} {v['wall_ms']:.3f} ms" for k, v in rows.items()
                                          if k != "gate")
            + f"; numerics gate {'PASS' if gate.passed else 'FAIL'}")
    out["reference_graphs"] = ref_graphs

    # The reference's transformer_block with GEMM1 -> bias+GELU fused into one node,
    # against the unfused graph in alternating blocks (chain-greedy, 4 streams).
    tb_spec = G.REFERENCE_GRAPHS["transformer_block"][1]
    tb_inputs = {}

    def tb_executor(build):
        g, t = build(4096, 1024, 4096)
        for key, (kind, seed, p0, p1) in tb_spec.items():   # shapes before the executor takes g
            if key not in tb_inputs:
                n_el = int(np.prod(g.shape(t[key])))
                tb_inputs[key] = (m.fill_random(n_el, seed, p0, p1) if kind == "u"
                                  else m.fill_normal(n_el, seed, p0, p1))
        ex = G.Executor(g, allocator=G.AllocatorKind.kBuddy, schedule=G.SchedulePolicy.kChainGreedy,
                        memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=4)
        ex.plan()
        for key in tb_spec:
            ex.set_input(t[key], tb_inputs[key])
        return ex, t

    ex_u, t_u = tb_executor(G.transformer_block)
    ex_f, t_f = tb_executor(G.transformer_block_fused)
    tb_u, tb_f = [], []
    for _ in range(4):
        tb_f.append(timed_runs(ex_f, ref_steps)[0])
        tb_u.append(timed_runs(ex_u, ref_steps)[0])
    y_u = ex_u.read(t_u["softmax"], 4096 * 1024)
    y_f = ex_f.read(t_f["softmax"], 4096 * 1024)
    ex_u.close()
    ex_f.close()
    tb_same = bool(np.array_equal(y_u.view(np.uint32), y_f.view(np.uint32)))
    out["transformer_block_fused"] = {
        "shape": "transformer_block(4096, 1024, 4096), chain_greedy, 4 streams",
        "unfused_wall_ms": round(float(np.median(tb_u)), 4),
        "fused_wall_ms": round(float(np.median(tb_f)), 4),
        "speedup": round(float(np.median(tb_u)) / float(np.median(tb_f)), 4),
        "blocks": f"4 alternating blocks of {ref_steps} runs each; medians",
        "parity": {"ok": tb_same, "same_output_bits_as_unfused": tb_same},
    }
    log(f"transformer_block fused: {out['transformer_block_fused']['fused_wall_ms']} ms against "
        f"{out['transformer_block_fused']['unfused_wall_ms']} ms unfused "
        f"({out['transformer_block_fused']['speedup']}x), same bits: {tb_same}")

    # The HIP-graph capture part (skipped with capture=False: under rocprofv3's kernel
    # trace the host process crashed inside it, so profiling runs leave it out).
    if capture:
        # Launch-bound shapes: the same MLP chain at small sizes, replayed eagerly (the
        # plan's launches issued by the host each run) and as one captured HIP graph
        # launch per run.
        out["mlp_small_capture"] = []
        for (T2, D2, F2) in ((512, 256, 1024), (64, 64, 256)):
            cap = {}
            for label in ("eager", "hip_graph"):
                g, t = G.mlp_block(T2, D2, F2)
                ex = G.Executor(g, allocator=G.AllocatorKind.kFreeList,
                                schedule=G.SchedulePolicy.kChainGreedy,
                                memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=2)
                ex.plan()
                ex.set_input(t["x"], m.fill_normal(T2 * D2, 0x3101, 0.0, 1.0))
                ex.set_input(t["W1"], m.fill_normal(D2 * F2, 0x3102, 0.0, 0.02))
                ex.set_input(t["b1"], m.fill_normal(F2, 0x3103, 0.0, 0.01))
                ex.set_input(t["W2"], m.fill_normal(F2 * D2, 0x3104, 0.0, 0.02))
                ex.set_input(t["b2"], m.fill_normal(D2, 0x3105, 0.0, 0.01))
                if label == "hip_graph":
                    ex.capture()
                wall, _ = timed_runs(ex, 200)
                y = ex.read(t["y"], T2 * D2)
                cap[label] = {"us_per_run": round(wall * 1e3, 2), "y_bits": y.view(np.uint32)}
                ex.close()
            same = bool(np.array_equal(cap["eager"].pop("y_bits"), cap["hip_graph"].pop("y_bits")))
            entry = {"shape": f"X[{T2}x{D2}] W1[{D2}x{F2}] W2[{F2}x{D2}]", **cap,
                     "speedup": round(cap["eager"]["us_per_run"] / cap["hip_graph"]["us_per_run"], 3),
                     "same_bits": same}
            log(f"MLP {T2}x{D2}x{F2}: eager {cap['eager']['us_per_run']} us, "
                f"hipGraph {cap['hip_graph']['us_per_run']} us per run, same bits: {same}")
            out["mlp_small_capture"].append(entry)

        # A launch-bound plan, on 4 streams and on one: eager (the host issues the
        # launches, events and waits each run) vs one captured graph per run (on 4
        # streams assembled node by node from single-stream captures).
        n, B, Dp = 256, 4, 4
        fan_cap = {"shape": f"{B} chains x {Dp} GEMMs {n}^3"}
        bits_seen = []
        for plan_label, sched, streams in (("4_streams", G.SchedulePolicy.kChainGreedy, 4),
                                           ("1_stream", G.SchedulePolicy.kSequential, 1)):
            cap = {}
            for label in ("eager", "hip_graph"):
                g, t = G.gemm_fanout(B, Dp, n)
                ex = G.Executor(g, allocator=G.AllocatorKind.kFreeList, schedule=sched,
                                memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=streams)
                ex.plan()
                ex.set_input(t["W"], m.fill_random(n * n, 0x4100, -0.0625, 0.0625))
                for k in range(B):
                    ex.set_input(t["xs"][k], m.fill_random(n * n, 0x4101 + k))
                if label == "hip_graph":
                    ex.capture()
                wall, _ = timed_runs(ex, 200)
                bits_seen.append(np.concatenate([ex.read(o, n * n).view(np.uint32) for o in t["outs"]]))
                cap[label] = {"us_per_run": round(wall * 1e3, 2)}
                ex.close()
            cap["speedup"] = round(cap["eager"]["us_per_run"] / cap["hip_graph"]["us_per_run"], 3)
            fan_cap[plan_label] = cap
            log(f"fan-out {B}x{Dp} {n}^3 {plan_label}: eager {cap['eager']['us_per_run']} us, "
                f"hipGraph {cap['hip_graph']['us_per_run']} us per run")
        fan_cap["same_bits"] = all(np.array_equal(bits_seen[0], b) for b in bits_seen[1:])
        out["fanout_small_capture"] = fan_cap

        # A plan of many short nodes, where one graph launch replaces many eager ones: a
        # chain of 32 bias+GELU nodes over X[64 x 1024] (256 KiB, about a microsecond
        # of device work each) on one stream, eager vs replayed.
        chain_cap = {"shape": "chain of 32 bias+GELU nodes, X[64x1024], 1 stream"}
        chain_bits = []
        for label in ("eager", "hip_graph"):
            g, t = G.chain(32, 64, 1024)
            ex = G.Executor(g, allocator=G.AllocatorKind.kFreeList,
                            schedule=G.SchedulePolicy.kSequential,
                            memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=1)
            ex.plan()
            ex.set_input(t["x"], m.fill_normal(64 * 1024, 0x5100))
            ex.set_input(t["bias"], m.fill_random(1024, 0x5101, -0.5, 0.5))
            if label == "hip_graph":
                ex.capture()
            wall, enq = timed_runs(ex, 200)
            chain_bits.append(ex.read(t["outs"][0], 64 * 1024).view(np.uint32))
            chain_cap[label] = {"us_per_run": round(wall * 1e3, 2), "enqueue_us": round(enq, 2)}
            ex.close()
        chain_cap["speedup"] = round(chain_cap["eager"]["us_per_run"] /
                                     chain_cap["hip_graph"]["us_per_run"], 3)
        chain_cap["same_bits"] = bool(np.array_equal(chain_bits[0], chain_bits[1]))
        out["chain32_small_capture"] = chain_cap
        log(f"chain32 64x1024: eager {chain_cap['eager']['us_per_run']} us, hipGraph "
            f"{chain_cap['hip_graph']['us_per_run']} us per run")

        # The executor's measured choice (capture_if_faster) on each launch-bound plan:
        # it keeps the graph only where replay beat eager issue on that plan.
        def choice(build, set_inputs, **kw):
            g, t = build()
            ex = G.Executor(g, allocator=G.AllocatorKind.kFreeList,
                            memory=G.MemoryPolicy.kReuseHappensBefore, **kw)
            ex.plan()
            set_inputs(ex, t)
            d = ex.capture_if_faster(trials=100)
            ex.close()
            return {k: (round(v, 2) if isinstance(v, float) else v) for k, v in d.items()}

        def mlp_inputs_small(T2, D2, F2):
            def f(ex, t):
                ex.set_input(t["x"], m.fill_normal(T2 * D2, 0x3101, 0.0, 1.0))
                ex.set_input(t["W1"], m.fill_normal(D2 * F2, 0x3102, 0.0, 0.02))
                ex.set_input(t["b1"], m.fill_normal(F2, 0x3103, 0.0, 0.01))
                ex.set_input(t["W2"], m.fill_normal(F2 * D2, 0x3104, 0.0, 0.02))
                ex.set_input(t["b2"], m.fill_normal(D2, 0x3105, 0.0, 0.01))
            return f

        def fan_inputs_small(ex, t):
            ex.set_input(t["W"], m.fill_random(256 * 256, 0x4100, -0.0625, 0.0625))
            for k, x in enumerate(t["xs"]):
                ex.set_input(x, m.fill_random(256 * 256, 0x4101 + k))

        def chain_inputs(ex, t):
            ex.set_input(t["x"], m.fill_normal(64 * 1024, 0x5100))
            ex.set_input(t["bias"], m.fill_random(1024, 0x5101, -0.5, 0.5))

        out["capture_choice"] = {
            "mlp_512x256x1024_2streams": choice(lambda: G.mlp_block(512, 256, 1024),
                                                mlp_inputs_small(512, 256, 1024),
                                                schedule=G.SchedulePolicy.kChainGreedy, num_streams=2),
            "mlp_64x64x256_2streams": choice(lambda: G.mlp_block(64, 64, 256),
                                             mlp_inputs_small(64, 64, 256),
                                             schedule=G.SchedulePolicy.kChainGreedy, num_streams=2),
            "fanout_4x4_256_4streams": choice(lambda: G.gemm_fanout(4, 4, 256), fan_inputs_small,
                                              schedule=G.SchedulePolicy.kChainGreedy, num_streams=4),
            "chain32_64x1024_1stream": choice(lambda: G.chain(32, 64, 1024), chain_inputs,
                                              schedule=G.SchedulePolicy.kSequential, num_streams=1),
        }
        for k, v in out["capture_choice"].items():
            log(f"capture_if_faster {k}: eager {v['eager_us_per_run']} us, replay "
                f"{v['replay_us_per_run']} us -> {'graph' if v['captured'] else 'eager'}")

    out["gates_passed"] = bool(out["mlp_block"]["gate"]["passed"] and
                               out["fanout4x4_gemm2048"]["gate"]["passed"] and
                               all(r["gate"]["passed"] for r in ref_graphs.values()))

    def verify(orc):
        from oracle import graph_checks as gc
        mlp = gc.check_mlp(mlp_in, host["mlp"], T, D, F)
        mlp["ok"] = bool(mlp["ok"] and same_bits and out["mlp_block"]["gate"]["passed"])
        out["mlp_block"]["parity"] = mlp
        fp = gc.check_fanout(fan_w, fan_xs, host["fan"], fan_n)
        fp["ok"] = bool(fp["ok"] and out["fanout4x4_gemm2048"]["gate"]["passed"])
        out["fanout4x4_gemm2048"]["parity"] = fp
        ok = mlp["ok"] and fp["ok"]
        for gname, (nodes, inp) in ref_nodes.items():
            if gname == "diamond_gemm_2048":
                r = gc.check_diamond_gemm(inp["A"], inp["W"], nodes, 2048)
            elif gname == "chain16":
                r = gc.check_bias_chain(inp["x"], inp["bias"], [nodes[f"n{i}"] for i in range(16)],
                                        4096, 4096)
            elif gname == "fanout4x4":
                r = {f"b{k}": gc.check_bias_chain(inp["x"], inp["bias"],
                                                  [nodes[f"b{k}n{d}"] for d in range(4)], 2048, 2048)
                     for k in range(4)}
                r["ok"] = all(v["ok"] for v in r.values())
            elif gname == "diamond_starved":
                r = gc.check_diamond_starved(inp["X"], inp["bias"], nodes, 8192, 4096)
            else:
                r = gc.check_transformer(inp, nodes, 4096, 1024, 4096)
            r["ok"] = bool(r["ok"] and ref_graphs[gname]["gate"]["passed"])
            ref_graphs[gname]["parity"] = {"ok": r["ok"]}
            ok = ok and r["ok"]
        ref_nodes.clear()
        return {"ok": bool(ok)}

    return out, verify


def cpu_baseline(m, gemm_bufs, ops, seconds_target=10.0, stream=None, runs=5):
    """The CPU reference, one thread, timed on this host beside the GPU run.  Uses
    oracle/_ref (the reference's own tests/reference.hpp, compiled from its
    sources) when it was built, else the plain-C restatement.

    GEMM (reference.hpp:199-211: i-j-p loops, double accumulation): a row slab of
    the same 8192^3 problem, sized so that `runs` runs take about
    `seconds_target`, timed `runs` times (median and min), and the GPU's C
    checked on that slab.  Beside it: the full reference at 512^3 and 1024^3
    against the GPU's C at those sizes, and the slab's work split by rows over
    the host cores (one reference call per thread; ctypes releases the GIL),
    reported as a separate figure.

    Every memory-bound op of the step (row sum/max, full sum, softmax, bias+GELU)
    at its full BASELINE shape on the op's own input: reference_row_reduce,
    reference_row_softmax and reference_bias_act (reference.hpp:143-191), each
    timed `runs` times, median and min, with GB/s at the op's algorithmic bytes."""
    import concurrent.futures
    import oracle

    a, b, c, n = gemm_bufs
    ha = a.download(n * n)
    hb = b.download(n * n)
    hc = c.download(n * n)
    use_ref = oracle.ref_available()
    kind = "reference" if use_ref else "port"
    ref = oracle.Ref if use_ref else oracle
    host_cores = os.cpu_count()
    ref_gemm = ref.gemm

    # Size the slab from one row, then time the same slab `runs` times.
    t = time.perf_counter()
    ref_gemm(ha[:n], hb, np.zeros(n, np.float32), 1, n, n, 1.0, 0.0)
    per_row = time.perf_counter() - t
    rows_done = max(1, min(64, int(seconds_target / runs / per_row)))
    times, want = [], None
    for _ in range(runs):
        out = np.zeros(rows_done * n, np.float32)
        t = time.perf_counter()
        got_rows = ref_gemm(ha[:rows_done * n], hb, out, rows_done, n, n, 1.0, 0.0)
        times.append(time.perf_counter() - t)
        if want is None:
            want = got_rows
    tarr = np.array(times)
    elapsed = float(np.median(tarr))
    r = oracle.compare(hc[:rows_done * n], want, oracle.tol_gemm(n), oracle.abs_tol_gemm(n))
    flops = 2.0 * rows_done * n * n
    log(f"cpu baseline: GEMM slab {rows_done}x{n}x{n}: median {elapsed:.2f} s, min "
        f"{tarr.min():.2f} s over {runs} runs")

    # The memory-bound ops at their full shapes.
    op_rows = []
    for op in ops:
        if op.cpu_ref is None:
            continue
        ts = []
        for _ in range(runs):
            t = time.perf_counter()
            op.cpu_ref(ref)
            ts.append(time.perf_counter() - t)
        ts = np.array(ts)
        med = float(np.median(ts))
        op_rows.append({"name": op.name, "shape": op.shape, "runs": runs,
                        "median_ms": round(med * 1e3, 2), "min_ms": round(float(ts.min()) * 1e3, 2),
                        "gb_s": round(op.work / med / 1e9, 3),
                        "gpu_speedup": round(med * 1e3 / (op.total_ms / op.launches), 1)
                        if op.launches else None})
        log(f"cpu baseline: {op.name} median {med * 1e3:.1f} ms "
            f"({op.work / med / 1e9:.2f} GB/s), min {ts.min() * 1e3:.1f} ms")

    # The full reference at 512^3 and 1024^3, on bench inputs of those sizes.
    full = []
    D = m.DeviceBuffer
    for nn in (512, 1024):
        fa, fb = m.fill_random(nn * nn, 0x6E33A), m.fill_random(nn * nn, 0x8B10C)
        da, db, dc = D.from_array(fa), D.from_array(fb), D.zeros(nn * nn)
        m.launch_gemm_f32(da, db, dc, nn, nn, nn, 1.0, 0.0, m.GemmVariant.kMfmaF32,
                          m.gemm_mfma_default_tile(nn, nn, nn), stream).throw_if_error()
        gpu_c = dc.download(nn * nn, stream=stream)
        t = time.perf_counter()
        want_full = ref_gemm(fa, fb, np.zeros(nn * nn, np.float32), nn, nn, nn, 1.0, 0.0)
        dt = time.perf_counter() - t
        rf = oracle.compare(gpu_c, want_full, oracle.tol_gemm(nn), oracle.abs_tol_gemm(nn))
        full.append({"n": nn, "seconds": round(dt, 3), "tflops": round(2.0 * nn ** 3 / dt / 1e12, 6),
                     "parity_of_gpu_c": {"ok": bool(rf.ok), "max_abs_err": rf.max_abs_err,
                                         "max_rel_err": rf.max_rel_err,
                                         "check": "every element, rel tol_gemm + abs abs_tol_gemm"}})
        log(f"cpu baseline: full reference {nn}^3 in {dt:.2f} s; GPU C "
            f"{'matches' if rf.ok else 'DIFFERS'}")
        del da, db, dc

    # Row-parallel: the next rows of the same 8192^3 problem, one row per thread,
    # on the host cores this process may use (at most 16, the GPU box's share).
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    r0 = rows_done
    def one_row(i):
        row = r0 + i
        return ref_gemm(ha[row * n:(row + 1) * n], hb, np.zeros(n, np.float32), 1, n, n, 1.0, 0.0)
    t = time.perf_counter()
    with concurrent.futures.ThreadPoolExecutor(threads) as pool:
        par_rows = list(pool.map(one_row, range(threads)))
    dt_par = time.perf_counter() - t
    rp = oracle.compare(hc[r0 * n:(r0 + threads) * n], np.concatenate(par_rows),
                        oracle.tol_gemm(n), oracle.abs_tol_gemm(n))
    log(f"cpu baseline: row-parallel, {threads} threads: {threads} rows in {dt_par:.1f} s")
    return {
        "value": round(flops / elapsed / 1e12, 6), "unit": "TFLOP/s", "cores": 1,
        "kind": kind,
        "sample": f"rows 0..{rows_done - 1} of C for the 8192^3 GEMM ({rows_done}x8192x8192), "
                  f"median of {runs} runs, 1 thread of {host_cores} host cores, double "
                  f"accumulation in the reference's i-j-p order",
        "gemm_slab_seconds": {"median": round(elapsed, 3), "min": round(float(tarr.min()), 3),
                              "runs": runs},
        "extrapolated_8192_s": round(elapsed / rows_done * n, 1),
        "parity_on_sample": {"ok": bool(r.ok), "max_abs_err": r.max_abs_err,
                             "max_rel_err": r.max_rel_err,
                             "tol": f"rel tol_gemm(8192)={oracle.tol_gemm(n):.3g} + abs "
                                    f"abs_tol_gemm(8192)={oracle.abs_tol_gemm(n):.3g}"},
        "full_reference": full,
        "row_parallel": {"threads": threads, "rows": f"{r0}..{r0 + threads - 1}",
                         "seconds": round(dt_par, 2),
                         "tflops": round(2.0 * threads * n * n / dt_par / 1e12, 6),
                         "parity_ok": bool(rp.ok)},
        "ops": op_rows,
        "ops_note": f"memory-bound ops at their full BASELINE shapes on the ops' own inputs, "
                    f"1 thread of {host_cores} host cores, {runs} runs each; gpu_speedup = CPU "
                    f"median / GPU average launch",
    }


HEADLINE_MAX_BYTES = 4096


def headline(detail: dict, detail_file: str | None) -> dict:
    """The compact record printed as stdout's last line: the contract fields, the
    GEMM's roofline, the CPU baseline's summary and one short row per op, in the
    spirit of the reference's one-CSV-row-per-kernel profiler record
    (src/core/profiler.cpp:95-113).  Every other section stays in `detail`, which
    bench.py writes to `detail_file`.  Kept under HEADLINE_MAX_BYTES: the section
    summaries are dropped, least important first, until it fits."""
    keep = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
            "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config", "roofline")
    line = {k: detail.get(k) for k in keep}
    cpu = detail.get("cpu_baseline")
    if cpu:
        line["cpu_baseline"] = {
            "value": cpu.get("value"), "unit": cpu.get("unit"), "cores": cpu.get("cores"),
            "kind": cpu.get("kind"), "sample": cpu.get("sample"),
            "extrapolated_8192_s": cpu.get("extrapolated_8192_s"),
            "parity_ok": (cpu.get("parity_on_sample") or {}).get("ok"),
            "ops_gb_s": {r["name"]: r["gb_s"] for r in cpu.get("ops", [])},
        }
    else:
        line["cpu_baseline"] = None
    # One row per op: [name, avg_ms, achieved, unit, frac of the published peak, parity ok].
    line["ops"] = [[s["name"], s["avg_ms"], s["achieved"], s["unit"], s["frac"],
                    (s.get("parity") or {}).get("ok")] for s in detail.get("ops") or []]
    line["ops_columns"] = ["name", "avg_ms", "achieved", "unit", "frac", "parity_ok"]
    extra = {}
    peaks = detail.get("measured_peaks")
    if peaks:
        extra["measured_peaks"] = {k: peaks[k] for k in
                                   ("mfma_f32_tflops", "stream_triad_gb_s", "stream_copy_gb_s",
                                    "stream_copy_32mib_gb_s") if k in peaks}
    sweep = detail.get("gemm_sweep") or []
    if sweep:
        extra["gemm_sweep_tflops"] = {str(r["n"]): [r["mfma"]["tflops"], r["rocblas"]["tflops"]]
                                      for r in sweep}
    lp = detail.get("gemm_lp") or {}
    if lp.get("runs"):
        extra["gemm_lp_tflops"] = {f"{r['ab']}->{r['c']} {r['n']}": r["tflops"]
                                   for r in lp["runs"]}
    graph = detail.get("graph") or {}
    if graph.get("mlp_block"):
        g = graph["mlp_block"]
        extra["graph_mlp"] = {"wall_ms": g.get("wall_ms"), "tflops": g.get("tflops"),
                              "bound_over_wall": g.get("bound_over_wall")}
        fused = graph.get("mlp_block_fused")
        if fused:
            extra["graph_mlp"].update(fused_wall_ms=fused.get("wall_ms"),
                                      fused_tflops=fused.get("tflops"))
        tb = graph.get("transformer_block_fused")
        if tb:
            extra["graph_mlp"]["transformer_block_fused_speedup"] = tb.get("speedup")
    if graph.get("gates_passed") is not None:
        extra["graph_gates_passed"] = graph["gates_passed"]
    if graph.get("capture_choice"):
        # Per launch-bound plan: [eager us, replay us, graph kept].
        extra["graph_capture_choice"] = {
            k: [v["eager_us_per_run"], v["replay_us_per_run"], v["captured"]]
            for k, v in graph["capture_choice"].items()}
    # Every parity verdict in the record (ops, 16-bit GEMM, graphs, ladder, CPU legs).
    verdicts = []

    def walk(node):
        if isinstance(node, dict):
            p = node.get("parity")
            if isinstance(p, dict) and isinstance(p.get("ok"), bool):
                verdicts.append(p["ok"])
            for v in node.values():
                walk(v)
        elif isinstance(node, list):
            for v in node:
                walk(v)
    walk(detail)
    extra["all_parity_ok"] = all(verdicts) if verdicts else None
    extra["parity_checks"] = len(verdicts)
    extra["detail_file"] = detail_file
    line.update(extra)
    # Only the summaries may go; the contract fields always stay.
    for k in ("graph_capture_choice", "graph_mlp", "gemm_lp_tflops", "gemm_sweep_tflops",
              "measured_peaks"):
        if len(json.dumps(line, separators=(",", ":"))) <= HEADLINE_MAX_BYTES:
            break
        line.pop(k, None)
    return line


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-sweep", action="store_true", help="skip the GEMM size sweep")
    p.add_argument("--sweep-sizes", default="512,1024,2048,4096,8192",
                   help="square sizes of the GEMM sweep (with --only gemm_sweep it runs alone)")
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="target CPU time of the GEMM slab's timed runs together")
    p.add_argument("--no-graph", action="store_true", help="skip the config-5 graph section")
    p.add_argument("--no-peaks", action="store_true", help="skip the measured-peak microbenches")
    p.add_argument("--no-capture", action="store_true",
                   help="skip the graph section's HIP-graph capture part (for profiling runs)")
    p.add_argument("--no-lp", action="store_true", help="skip the 16-bit-input GEMM section")
    p.add_argument("--lp-vendor-sizes", default="8192,4096,2048,1024",
                   help="sizes of the 16-bit GEMM's interleaved rocBLAS comparison")
    p.add_argument("--no-ladder", action="store_true",
                   help="skip the variant ladder (every variant the reference's benches time)")
    p.add_argument("--only", default=None,
                   help="comma-separated op-name prefixes to run (profiling); enables "
                        "the copy_256mib calibration op; 'graph' keeps the graph section")
    p.add_argument("--detail-out", default=os.path.join(ROOT, "gpurun_out", "bench_detail.json"),
                   help="file that receives the full record (every section); stdout's last "
                        "line carries the compact headline")
    args = p.parse_args(argv)
    only = set(args.only.split(",")) if args.only else None

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the "
              "kernel layer has no multi-GPU path to measure.", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("bench.py: need --steps >= 1 and --warmup >= 0", file=sys.stderr)
        return 2

    # The graph section's multi-stream plans want a hardware queue per executor lane.
    # HIP hands streams out over GPU_MAX_HW_QUEUES queues per process (4 by default)
    # and, once each holds a stream, puts a new stream on a queue it shares, so two
    # lanes of a plan created after the bench's other streams can run one after the
    # other (fanout4x4 under chain-greedy: 1.48x over one stream with 4 queues, 2.13-2.17x
    # with 8 or 16, measured on MI355X).  HIP reads it when it initialises, i.e. before
    # the library loads.  The bench runs with 8 (MCKE_BENCH_HW_QUEUES picks another
    # value) and records it in config.hw_queues.
    os.environ["GPU_MAX_HW_QUEUES"] = os.environ.get("MCKE_BENCH_HW_QUEUES", "8")
    m = load_package()
    info = m.require_gpu()
    log(f"device: {info.name.decode()} {info.arch.decode()} CUs={info.sm_count} "
        f"hw_queues={os.environ['GPU_MAX_HW_QUEUES']}")
    stream = m.Stream()
    ops, keep, gemm_bufs = build_ops(m, stream, only)

    if only is not None and not ops and not any(x.startswith(("gemm_lp", "gemm_sweep", "graph")) for x in only):
        print(f"bench.py: --only {args.only} names no op", file=sys.stderr)
        return 2
    log(f"warmup: {args.warmup} steps")
    run_steps(m, stream, ops, args.warmup, record=False)
    log(f"timed: {args.steps} steps")
    total_ms = run_steps(m, stream, ops, args.steps, record=True)
    log("timed region done; single-launch diagnostic pass")
    single_launches(m, stream, ops, min(args.steps, 20))
    resident_pass(m, stream, ops)

    peaks = None
    if not args.no_peaks and only is None:
        gemm_ms = ops[0].total_ms / ops[0].launches if ops[0].bound == "mfma" else 8.0
        peaks = measured_peaks(m, stream, gemm_ms)
    traffic = profiled_traffic()
    summaries = []
    for op in ops:
        if peaks:
            # Ops of a few tens of MB are held to the copy of their own size.
            op.copy_peak = (peaks["stream_copy_32mib_gb_s"] if op.work < 64e6
                            else peaks["stream_copy_gb_s"])
        mp = None
        if peaks:
            mp = peaks["mfma_f32_tflops"] if op.bound == "mfma" else peaks["stream_triad_gb_s"]
        summaries.append(op.summary(mp, traffic.get(op.name)))
    for s in summaries:
        log(f"{s['name']:>20s} {s['avg_ms']:.4f} ms  {s['achieved']:.1f} {s['unit']}  "
            f"({100 * s['frac']:.1f}% of {s['peak']})")
        if "effective_resident" in s:
            e = s["effective_resident"]
            log(f"{'':>20s} resident {e['avg_ms']:.4f} ms  {e['achieved']:.1f} GB/s effective")

    run_sweep = not args.no_sweep and (only is None or any(x.startswith("gemm_sweep") for x in only))
    sweep = gemm_sweep(m, stream, sizes=tuple(int(x) for x in args.sweep_sizes.split(",") if x)) \
        if run_sweep else []
    lp_res, lp_verify = None, []
    if not args.no_lp and (only is None or any(x.startswith("gemm_lp") for x in only)):
        lp_res, lp_verify = gemm_lp_section(
            m, stream, with_peak=not args.no_peaks,
            vendor_sizes=tuple(int(x) for x in args.lp_vendor_sizes.split(",") if x))
    graph_res, graph_verify = None, None
    if not (args.no_graph or (only is not None and "graph" not in only)):
        graph_res, graph_verify = graph_section(m, capture=not args.no_capture)
    ladder_res, ladder_verify = None, None
    if not (args.no_ladder or only is not None):
        ladder_res, ladder_verify = ladder_section(m, stream, info.sm_count)
    cpu = None
    if not args.no_cpu:
        # The CPU checker on every timed op's output at its timed shape (the timed
        # launches wrote these buffers); results land in ops[*].parity.
        import oracle
        for op in ops:
            if op.verify is not None:
                t0 = time.perf_counter()
                op.parity = op.verify(oracle)
                log(f"parity {op.name}: {'OK' if op.parity['ok'] else 'FAILED'} "
                    f"({time.perf_counter() - t0:.1f} s)")
        extra = list(lp_verify)
        if graph_verify is not None:
            extra.append(("graph (config 5 stages, timed-plan bits, numerics gates)", graph_verify))
        if ladder_verify is not None:
            extra.append(("ladder (every variant's output)", ladder_verify))
        for name, verify in extra:
            t0 = time.perf_counter()
            res = verify(oracle)
            log(f"parity {name}: {'OK' if res['ok'] else 'FAILED'} "
                f"({time.perf_counter() - t0:.1f} s)")
    if not args.no_cpu and gemm_bufs[0] is not None:
        log(f"cpu baseline: reference GEMM on a row slab (~{args.cpu_seconds:.0f} s) and the "
            "memory-bound ops at full shape")
        cpu = cpu_baseline(m, gemm_bufs, ops, args.cpu_seconds, stream)
        log(f"cpu baseline: {cpu['value']} TFLOP/s ({cpu['sample']})")
    summaries = [op.summary(s["measured_peak"] if "measured_peak" in s else None,
                            s.get("hbm_traffic_bytes")) for op, s in zip(ops, summaries)]
    # A profiling run restricted by --only may hold no fp32 op at all.
    gemm = summaries[0] if summaries else {"achieved": None, "unit": None, "bound": None,
                                           "peak": None, "frac": None, "name": None}

    detail = {
        "metric": METRIC,
        "value": gemm["achieved"],
        "unit": gemm["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded fill_random U[-1,1) / Box-Muller N(mu,sigma^2) at "
                "BASELINE.json shapes, resident in HBM",
        "config": {
            "workload": "fp32 GEMM 8192^3 (kMfmaF32) headline; step also runs row sum/max "
                        "8192x8192, full sum 2^26, softmax 32768x{128,1024,4096}, "
                        "bias+GELU_tanh 16384x4096 and 4096x1024",
            "gemm_tile": list(m.gemm_mfma_default_tile(8192, 8192, 8192).astuple()),
            # The runtime leaves the marketing name empty on some boxes.
            "device": info.name.decode() or f"{info.arch.decode()} ({info.sm_count} CUs)",
            "hw_queues": os.environ.get("GPU_MAX_HW_QUEUES"),
        },
        "roofline": {
            "bound": gemm["bound"], "achieved": gemm["achieved"], "peak": gemm["peak"],
            "unit": gemm["unit"], "frac": gemm["frac"],
            "traffic": traffic.get(gemm["name"]),
        },
        "measured_peaks": peaks,
        "cpu_baseline": cpu,
        "ops": summaries,
        "gemm_sweep": sweep,
        "gemm_lp": lp_res,
        "graph": graph_res,
        "ladder": ladder_res,
    }
    # The full record goes to a file first; stdout's last line is the compact
    # headline, which must stay whole inside the few KB of stdout a driver keeps.
    detail_path = os.path.abspath(args.detail_out)
    os.makedirs(os.path.dirname(detail_path), exist_ok=True)
    with open(detail_path, "w") as f:
        json.dump(detail, f, indent=1)
    log(f"full record ({os.path.getsize(detail_path)} bytes) written to {detail_path}")
    line = headline(detail, os.path.relpath(detail_path, ROOT))
    print(json.dumps(line, separators=(",", ":")), flush=True)
    del keep
    return 0


if __name__ == "__main__":
    sys.exit(main())
