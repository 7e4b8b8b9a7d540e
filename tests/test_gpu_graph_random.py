"""Random DAGs through GraphExecutor on the GPU.

For each seed, a DAG of 6-14 nodes over square S x S f32 tensors: bias+activation
(activation and grid cap drawn), row softmax, and GEMMs of any two earlier tensors
(alpha = 1/S keeps magnitudes bounded), which make joins; then one or two row
reductions (any kind and variant) of computed tensors.  Every tensor no node reads
is an output.  The reference graph bench builds fixed shapes only
(bench/graph_bench.cpp:100-215); the host tests fuzz the planner without a GPU
(tests/cpp/test_host.cpp); this runs random plans for real, on several streams.

Checks:
  * a sequential plan with one buffer per tensor: every node's output against the
    CPU oracle on that node's own GPU inputs (GEMM at tol_gemm(S) / abs_tol_gemm(S),
    bias+activation none/ReLU exact and GELU at rel 1e-6 + abs 1e-6, softmax at
    rel 1e-5 + abs 1e-6, reductions as in test_gpu_parity.py);
  * six plans on 4 streams (each schedule with same-stream and happens-before arena
    reuse, the three allocators in turn), poisoned buffers, two runs each: the
    outputs' bits equal the per-tensor plan's;
  * a captured replay of the chain-greedy / happens-before plan: the same bits;
  * the numerics gate: 3 schedules x 3 memory policies, bitwise identical.
"""
from __future__ import annotations

import numpy as np
import pytest

from tests import golden_io
from tests.test_gpu_parity import _sum_abs_floor

pytestmark = pytest.mark.gpu

SEEDS = range(30)


@pytest.fixture(scope="module")
def G(gpu):
    from mcke_amd import graph
    return graph


def build(G, orc, seed):
    """The seed's graph (a fresh Graph each call: an executor consumes it), its
    nodes as (kind, out, inputs, params), its input arrays and its outputs."""
    rng = np.random.default_rng([0x6DA6, seed])
    S = int(rng.choice([64, 96, 128, 192, 256]))
    g = G.Graph()
    tensors, inputs, nodes = [], {}, []
    for i in range(int(rng.integers(2, 4))):
        t = g.add_input([S, S], f"in{i}")
        inputs[t] = orc.fill_random(S * S, 0x6DA60 + 16 * seed + i)
        tensors.append(t)
    bias = g.add_input([S], "bias")
    inputs[bias] = orc.fill_random(S, 0x6DA6F + seed, -0.5, 0.5)

    def pick():
        return tensors[int(rng.integers(0, len(tensors)))]

    for k in range(int(rng.integers(6, 15))):
        op = rng.choice(["bias_act", "softmax", "gemm"], p=[0.45, 0.2, 0.35])
        if op == "bias_act":
            x = pick()
            act, mrb = int(rng.integers(0, 4)), int(rng.choice([0, 0, 3, 7]))
            y = g.add_bias_act(x, bias, f"n{k}", act=act, max_row_blocks=mrb)
            nodes.append(("bias_act", y, (x, bias), {"act": act}))
        elif op == "softmax":
            x = pick()
            y = g.add_softmax(x, f"n{k}")
            nodes.append(("softmax", y, (x,), {}))
        else:
            a, b = pick(), pick()
            y = g.add_gemm(a, b, f"n{k}", alpha=1.0 / S)
            nodes.append(("gemm", y, (a, b), {"alpha": 1.0 / S}))
        tensors.append(y)
    computed = [n[1] for n in nodes]
    for k in range(int(rng.integers(1, 3))):
        x = computed[int(rng.integers(0, len(computed)))]
        kind, variant = int(rng.integers(0, 3)), int(rng.integers(0, 3))
        y = g.add_reduce(x, f"r{k}", kind=kind, variant=variant)
        nodes.append(("reduce", y, (x,), {"kind": kind}))
    consumed = {i for n in nodes for i in n[2]}
    outs = [n[1] for n in nodes if n[1] not in consumed]
    for y in outs:
        g.mark_output(y)
    sizes = {n[1]: (S if n[0] == "reduce" else S * S) for n in nodes}
    return g, nodes, inputs, outs, sizes, S


def _executor(G, orc, seed, **kw):
    g, nodes, inputs, outs, sizes, S = build(G, orc, seed)
    ex = G.Executor(g, **kw)
    ex.plan()
    for t, arr in inputs.items():
        ex.set_input(t, arr)
    return ex, nodes, inputs, outs, sizes, S


def _read_outputs(ex, outs, sizes):
    return {t: ex.read(t, sizes[t]) for t in outs}


def _check_node(orc, kind, got, ins, params, S):
    """The node's GPU output against the oracle on its GPU inputs; None if it passes."""
    if kind == "bias_act":
        x, b = ins
        want = orc.bias_act(x, b, S, S, params["act"])
        if params["act"] in (0, 1):
            return None if np.array_equal(golden_io.bits(got), golden_io.bits(want)) else "bits"
        r = orc.compare(got, want, 1e-6, 1e-6)
        return None if r.ok else str(r)
    if kind == "softmax":
        r = orc.compare(got, orc.row_softmax(ins[0], S, S), 1e-5, 1e-6)
        return None if r.ok else str(r)
    if kind == "gemm":
        a, b = ins
        alpha = params["alpha"]
        want = orc.gemm(a, b, np.zeros(S * S, np.float32), S, S, S, alpha, 0.0)
        amax = float(max(np.max(np.abs(a)), np.max(np.abs(b)), 1e-30))
        r = orc.compare(got, want, orc.tol_gemm(S), 2.0 * alpha * orc.abs_tol_gemm(S, amax) + 1e-30)
        return None if r.ok else str(r)
    kind_r = params["kind"]
    want = orc.row_reduce(ins[0], S, S, kind_r)
    if kind_r == 1:
        return None if np.array_equal(got, want) else "max differs"
    floor = _sum_abs_floor(ins[0].reshape(S, S)) / (S if kind_r == 2 else 1)
    r = orc.compare(got, want, 1e-5, floor)
    return None if r.ok else str(r)


@pytest.mark.parametrize("seed", SEEDS)
def test_random_dag_every_node_and_every_plan(G, orc, seed):
    # Per-tensor sequential plan: every tensor keeps its own buffer, so every node's
    # inputs and output can be read back and checked on their own.
    ex, nodes, inputs, outs, sizes, S = _executor(
        G, orc, seed, schedule=G.SchedulePolicy.kSequential, memory=G.MemoryPolicy.kAllocPerTensor,
        num_streams=1, allocator=G.AllocatorKind.kRaw)
    ex.run_sync()
    host = dict(inputs)
    for _, y, _, _ in nodes:
        host[y] = ex.read(y, sizes[y])
    for kind, y, ins, params in nodes:
        err = _check_node(orc, kind, host[y], [host[i] for i in ins], params, S)
        assert err is None, f"seed {seed} S={S}: {kind} node {y}: {err}"
    gold = {t: golden_io.bits(host[t]) for t in outs}
    ex.close()

    allocators = [G.AllocatorKind.kRaw, G.AllocatorKind.kBuddy, G.AllocatorKind.kFreeList]
    plans = [(s, m) for s in (G.SchedulePolicy.kSequential, G.SchedulePolicy.kLevelParallel,
                              G.SchedulePolicy.kChainGreedy)
             for m in (G.MemoryPolicy.kReuseSameStream, G.MemoryPolicy.kReuseHappensBefore)]
    for i, (sched, mem) in enumerate(plans):
        alloc = allocators[i % 3]
        ex, _, _, _, _, _ = _executor(G, orc, seed, schedule=sched, memory=mem, num_streams=4,
                                      allocator=alloc, poison_buffers=True)
        ex.run_sync()
        ex.run_sync()      # a second run over a re-poisoned arena
        got = _read_outputs(ex, outs, sizes)
        ex.close()
        for t in outs:
            assert np.array_equal(golden_io.bits(got[t]), gold[t]), \
                f"seed {seed}: {sched.name}/{mem.name}/{alloc.name} output {t} differs"

    # A captured replay of the plan the bench times.
    ex, _, _, _, _, _ = _executor(G, orc, seed, schedule=G.SchedulePolicy.kChainGreedy,
                                  memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=4)
    ex.capture()
    for _ in range(3):
        ex.run_sync()
        got = _read_outputs(ex, outs, sizes)
        for t in outs:
            assert np.array_equal(golden_io.bits(got[t]), gold[t]), \
                f"seed {seed}: captured replay, output {t} differs"
    ex.close()

    # The numerics gate over 3 schedules x 3 memory policies.
    ex, _, _, _, _, _ = _executor(G, orc, seed, num_streams=4, validate_numerics=True)
    res = ex.validate_numerics(repeats=2)
    ex.close()
    assert res.passed, f"seed {seed}: {res.detail}"
    assert res.configs_compared == 9
