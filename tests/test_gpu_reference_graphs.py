"""The reference graph bench's five graphs (bench/graph_bench.cpp:100-215, run at
:477-481) at its shapes, through GraphExecutor on the GPU:

  diamond_gemm_2048   B = A W, C = A W, D = B C, 2048^3 GEMMs
  chain16             16 bias+GELU nodes over x[4096 x 4096]
  fanout4x4           4 chains of 4 bias+GELU nodes over x[2048 x 2048], grids
                      capped at 10 row blocks
  diamond_starved     bias+GELU of X[8192 x 4096] at 40 row blocks, twice, then a
                      join node
  transformer_block   GEMM [4096 x 1024 x 4096] -> bias+GELU -> GEMM -> softmax

For each: every node checked on its own GPU input against the CPU oracle from a
sequential per-tensor plan (oracle/graph_checks.py: GEMMs by the reference's
1024-entry spot check, bias+GELU element by element at abs 1e-6 + rel 1e-6,
softmax at abs 1e-6 with row sums within 1e-5); the plan bench.py times
(chain-greedy, 4 streams, arena shared under happens-before, buddy allocator)
giving the same output bits; and the numerics gate (3 schedules x 3 memory
policies, bitwise identical over repeats), as the reference's graph bench gates
every graph it times (:444-471)."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GRAPHS = ["diamond_gemm_2048", "chain16", "fanout4x4", "diamond_starved", "transformer_block"]


@pytest.fixture(scope="module")
def G(gpu):
    from mcke_amd import graph
    return graph


@pytest.fixture(scope="module")
def checks(orc):
    from oracle import graph_checks
    return graph_checks


def _numel(g, t):
    n = 1
    for d in g.shape(t):
        n *= d
    return n


def _executor(G, name, orc, **kw):
    g, t, inputs = G.reference_graph(name, orc.fill_random, orc.fill_normal)
    sizes = {k: _numel(g, v) for k, v in t.items() if k != "outs"}
    outs = list(t["outs"])
    ex = G.Executor(g, **kw)
    ex.plan()
    for tid, arr in inputs.items():
        ex.set_input(tid, arr)
    return ex, t, sizes, outs, inputs


def _host_inputs(t, inputs):
    return {k: inputs[v] for k, v in t.items() if k != "outs" and v in inputs}


def _check(checks, name, t, host, inp):
    if name == "diamond_gemm_2048":
        return checks.check_diamond_gemm(inp["A"], inp["W"], host, 2048)
    if name == "chain16":
        return checks.check_bias_chain(inp["x"], inp["bias"], [host[f"n{i}"] for i in range(16)],
                                       4096, 4096)
    if name == "fanout4x4":
        res = {f"b{k}": checks.check_bias_chain(inp["x"], inp["bias"],
                                                [host[f"b{k}n{d}"] for d in range(4)], 2048, 2048)
               for k in range(4)}
        res["ok"] = all(v["ok"] for v in res.values())
        return res
    if name == "diamond_starved":
        return checks.check_diamond_starved(inp["X"], inp["bias"], host, 8192, 4096)
    return checks.check_transformer(inp, host, 4096, 1024, 4096)


@pytest.mark.parametrize("name", GRAPHS)
def test_reference_graph_every_node_and_timed_plan_bits(G, orc, checks, name):
    print(f"reference graph {name}: per-tensor plan", flush=True)
    ex, t, sizes, outs, inputs = _executor(G, name, orc, schedule=G.SchedulePolicy.kSequential,
                                           memory=G.MemoryPolicy.kAllocPerTensor, num_streams=1)
    ex.run_sync()
    node_keys = [k for k in t if k != "outs" and t[k] not in inputs]
    host = {k: ex.read(t[k], sizes[k]) for k in node_keys}
    want_out = [ex.read(o, _numel_of(sizes, t, o)) for o in outs]
    ex.close()
    res = _check(checks, name, t, host, _host_inputs(t, inputs))
    assert res["ok"], res

    print(f"reference graph {name}: timed plan", flush=True)
    ex, t2, _, outs2, _ = _executor(G, name, orc, allocator=G.AllocatorKind.kBuddy,
                                    schedule=G.SchedulePolicy.kChainGreedy,
                                    memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=4)
    for _ in range(2):
        ex.run_sync()
        for o, w in zip(outs2, want_out):
            got = ex.read(o, w.size)
            assert np.array_equal(got.view(np.uint32), w.view(np.uint32)), name
    ex.close()


def _numel_of(sizes, t, tid):
    for k, v in t.items():
        if k != "outs" and v == tid:
            return sizes[k]
    raise KeyError(tid)


@pytest.mark.parametrize("name", GRAPHS)
def test_reference_graph_numerics_gate(G, orc, name):
    print(f"reference graph {name}: numerics gate", flush=True)
    ex, *_ = _executor(G, name, orc, num_streams=4, validate_numerics=True)
    gate = ex.validate_numerics(repeats=5)
    ex.close()
    assert gate.passed, gate.detail
    assert gate.configs_compared == 9, gate.detail


@pytest.mark.parametrize("name", GRAPHS)
def test_plan_statistics_match_the_reference_table(G, name):
    """Streams used, peak arena bytes and naive bytes of each reference graph under
    the three schedules, planned as the reference's bench plans them (happens-before
    reuse, 1 stream for sequential and 4 for the others, bench/graph_bench.cpp:333),
    equal the reference's published table (tests/golden/graph_plan_stats.json, from
    its RESULTS.md section 4).  Planning only: nothing is launched."""
    import json
    import os

    golden = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                                         "graph_plan_stats.json")))["graphs"][name]
    for label, sched, streams in (("sequential", G.SchedulePolicy.kSequential, 1),
                                  ("level_parallel", G.SchedulePolicy.kLevelParallel, 4),
                                  ("chain_greedy", G.SchedulePolicy.kChainGreedy, 4)):
        g, _ = G.REFERENCE_GRAPHS[name][0]()
        ex = G.Executor(g, allocator=G.AllocatorKind.kBuddy, schedule=sched,
                        memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=streams)
        ex.plan()
        info = ex.plan_info()
        ex.close()
        want = golden[label]
        got = {"streams_used": info["num_streams_used"],
               "streams_requested": info["num_streams_requested"],
               "arena_bytes": info["arena_bytes"], "naive_bytes": info["naive_bytes"]}
        assert got == want, (name, label, got, want)


def test_fused_transformer_block_has_the_unfused_bits(G, orc):
    """transformer_block_fused (GEMM1 + bias + GELU in one node) against the
    reference's transformer_block at a reduced shape: the same H and output bits on
    a per-tensor plan and on a 4-stream plan with reuse over poisoned buffers."""
    T, D, F = 512, 256, 1024
    inp = {"x": orc.fill_normal(T * D, 0x4500, 0.0, 1.0),
           "W1": orc.fill_normal(D * F, 0x4501, 0.0, 0.02),
           "b1": orc.fill_normal(F, 0x4502, 0.0, 0.01),
           "W2": orc.fill_normal(F * D, 0x4503, 0.0, 0.02)}

    def run(build, **kw):
        g, t = build(T, D, F)
        ex = G.Executor(g, **kw)
        ex.plan()
        for k, v in inp.items():
            ex.set_input(t[k], v)
        ex.run_sync()
        ex.run_sync()
        got = {k: ex.read(t[k], n) for k, n in (("bias_gelu", T * F), ("softmax", T * D))
               if kw.get("memory") == G.MemoryPolicy.kAllocPerTensor or k == "softmax"}
        ex.close()
        return got

    per = dict(schedule=G.SchedulePolicy.kSequential, memory=G.MemoryPolicy.kAllocPerTensor,
               num_streams=1)
    gold = run(G.transformer_block, **per)
    fused = run(G.transformer_block_fused, **per)
    for k in ("bias_gelu", "softmax"):
        assert np.array_equal(gold[k].view(np.uint32), fused[k].view(np.uint32)), k
    reuse = run(G.transformer_block_fused, schedule=G.SchedulePolicy.kChainGreedy,
                memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=4, poison_buffers=True)
    assert np.array_equal(gold["softmax"].view(np.uint32), reuse["softmax"].view(np.uint32))
