"""BASELINE config 5 at the size bench.py times, through GraphExecutor.

* The MLP block X[4096 x 4096] . W1[4096 x 16384] -> bias + GELU -> . W2[16384 x
  4096] -> bias add -> row softmax, on the bench's seeded inputs (X N(0,1), W1 and
  W2 N(0, 0.02^2), b1 and b2 N(0, 0.01^2)).  A per-tensor plan keeps every stage
  readable; each stage is checked on the GPU's own input to it
  (oracle/graph_checks.py: both GEMMs by the reference's 1024-entry spot check,
  GEMM2 with K = 16384; bias + GELU, bias add and softmax element by element).
  The plan bench.py times (chain-greedy on 4 streams, arena shared under
  happens-before, buddy allocator) must give the same output bits.
* The 4 x 4 fan-out of 2048^3 GEMM chains on 4 streams: every one of the 16
  nodes spot-checked on its own GPU input, under chain-greedy and level-parallel
  schedules (the latter with 12 cross-stream events).
* The numerics gate at both shapes, 3 schedules x 3 memory policies x 20
  repeats each, as the reference's graph bench runs it at its bench shapes
  (bench/graph_bench.cpp:444-471).
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

T, D, F = 4096, 4096, 16384
FAN_N, FAN_B, FAN_D = 2048, 4, 4


@pytest.fixture(scope="module")
def G(gpu):
    from mcke_amd import graph
    return graph


@pytest.fixture(scope="module")
def checks(orc):
    from oracle import graph_checks
    return graph_checks


@pytest.fixture(scope="module")
def mlp_inputs(orc):
    """bench.py's config-5 MLP inputs (its seeds 0x3001..0x3005)."""
    return {
        "x": orc.fill_normal(T * D, 0x3001, 0.0, 1.0),
        "W1": orc.fill_normal(D * F, 0x3002, 0.0, 0.02),
        "b1": orc.fill_normal(F, 0x3003, 0.0, 0.01),
        "W2": orc.fill_normal(F * D, 0x3004, 0.0, 0.02),
        "b2": orc.fill_normal(D, 0x3005, 0.0, 0.01),
    }


@pytest.fixture(scope="module")
def fan_inputs(orc):
    """bench.py's fan-out inputs (W U[-1/32, 1/32), chain inputs U[-1, 1))."""
    n = FAN_N
    w = orc.fill_random(n * n, 0x4000, -0.03125, 0.03125)
    xs = [orc.fill_random(n * n, 0x4001 + k) for k in range(FAN_B)]
    return w, xs


def _set_mlp(ex, t, inp):
    for k, v in inp.items():
        ex.set_input(t[k], v)


def test_mlp_full_size_stagewise(G, checks, mlp_inputs):
    g, t = G.mlp_block(T, D, F)
    ex = G.Executor(g, schedule=G.SchedulePolicy.kSequential,
                    memory=G.MemoryPolicy.kAllocPerTensor, num_streams=1)
    try:
        ex.plan()
        _set_mlp(ex, t, mlp_inputs)
        ex.run_sync()
        stages = {"gemm1": ex.read(t["gemm1"], T * F), "h": ex.read(t["h"], T * F),
                  "gemm2": ex.read(t["gemm2"], T * D), "z": ex.read(t["z"], T * D),
                  "y": ex.read(t["y"], T * D)}
    finally:
        ex.close()
    res = checks.check_mlp(mlp_inputs, stages, T, D, F)
    assert res["ok"], {k: v for k, v in res.items() if k != "ok" and not v["ok"]}

    # bench.py's timed plan: same bits as the per-tensor plan
    g, t = G.mlp_block(T, D, F)
    ex = G.Executor(g, allocator=G.AllocatorKind.kBuddy, schedule=G.SchedulePolicy.kChainGreedy,
                    memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=4)
    try:
        ex.plan()
        _set_mlp(ex, t, mlp_inputs)
        ex.run_sync()
        ex.run_sync()
        y = ex.read(t["y"], T * D)
        info = ex.plan_info()
    finally:
        ex.close()
    assert info["arena_bytes"] < info["naive_bytes"]
    assert np.array_equal(y.view(np.uint32), stages["y"].view(np.uint32))


def test_mlp_full_size_numerics_gate(G, mlp_inputs):
    g, t = G.mlp_block(T, D, F)
    ex = G.Executor(g, num_streams=4, validate_numerics=True)
    try:
        ex.plan()
        _set_mlp(ex, t, mlp_inputs)
        res = ex.validate_numerics(repeats=20)
    finally:
        ex.close()
    assert res.passed, res.detail
    assert res.configs_compared == 9


@pytest.mark.parametrize("schedule", ["kChainGreedy", "kLevelParallel"])
def test_fanout_2048_every_node(G, checks, fan_inputs, schedule):
    n = FAN_N
    w, xs = fan_inputs
    g, t = G.gemm_fanout(FAN_B, FAN_D, n)
    ex = G.Executor(g, allocator=G.AllocatorKind.kBuddy,
                    schedule=getattr(G.SchedulePolicy, schedule),
                    memory=G.MemoryPolicy.kAllocPerTensor, num_streams=4)
    try:
        ex.plan()
        info = ex.plan_info()
        assert info["num_nodes"] == 16 and info["num_streams_used"] == 4
        if schedule == "kLevelParallel":
            assert info["num_events"] == 12
        ex.set_input(t["W"], w)
        for k in range(FAN_B):
            ex.set_input(t["xs"][k], xs[k])
        ex.run_sync()
        nodes = [[ex.read(tid, n * n) for tid in chain] for chain in t["nodes"]]
    finally:
        ex.close()
    res = checks.check_fanout(w, xs, nodes, n)
    assert res["ok"], {k: v for k, v in res.items() if k != "ok" and not v["ok"]}


def test_fanout_2048_numerics_gate(G, fan_inputs):
    w, xs = fan_inputs
    g, t = G.gemm_fanout(FAN_B, FAN_D, FAN_N)
    ex = G.Executor(g, num_streams=4, validate_numerics=True)
    try:
        ex.plan()
        ex.set_input(t["W"], w)
        for k in range(FAN_B):
            ex.set_input(t["xs"][k], xs[k])
        res = ex.validate_numerics(repeats=20)
    finally:
        ex.close()
    assert res.passed, res.detail
    assert res.configs_compared == 9
