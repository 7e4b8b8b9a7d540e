"""GPU tests of the graph layer through its C-ABI (include/mcke_graph.h):
BASELINE config 5's MLP block and GEMM fan-out at reduced sizes, stage by stage
against the CPU oracle, the bitwise numerics gate over 3 schedules x 3 memory
policies, plan statistics and the buddy allocator's reuse.

Stage-wise parity: each node's output is compared with the oracle applied to the
GPU's own input to that node (read back from a per-tensor arena), so a tolerance
only has to cover one kernel's rounding, as in the kernel tests."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def G(gpu):
    from mcke_amd import graph
    return graph


def _mlp_inputs(orc, tokens, d_model, d_ff):
    return {
        "x": orc.fill_normal(tokens * d_model, 1, 0.0, 1.0),
        "W1": orc.fill_normal(d_model * d_ff, 2, 0.0, 0.02),
        "b1": orc.fill_normal(d_ff, 3, 0.0, 0.01),
        "W2": orc.fill_normal(d_ff * d_model, 4, 0.0, 0.02),
        "b2": orc.fill_normal(d_model, 5, 0.0, 0.01),
    }


def test_mlp_block_stagewise_parity(G, orc):
    T, D, F = 256, 128, 512
    g, t = G.mlp_block(T, D, F)
    ex = G.Executor(g, schedule=G.SchedulePolicy.kSequential,
                    memory=G.MemoryPolicy.kAllocPerTensor, num_streams=1)
    ex.plan()
    inp = _mlp_inputs(orc, T, D, F)
    for k, v in inp.items():
        ex.set_input(t[k], v)
    ex.run_sync()
    g1 = ex.read(t["gemm1"], T * F)
    h = ex.read(t["h"], T * F)
    g2 = ex.read(t["gemm2"], T * D)
    z = ex.read(t["z"], T * D)
    y = ex.read(t["y"], T * D)
    # GEMMs: K-scaled tolerances with the inputs' magnitude (amax ~ 4 sigma).
    w = orc.gemm(inp["x"], inp["W1"], np.zeros(T * F, np.float32), T, F, D)
    r = orc.compare(g1, w, orc.tol_gemm(D), orc.abs_tol_gemm(D, 4.0 * 0.02 * 4.0))
    assert r.ok, f"gemm1: {r}"
    r = orc.compare(h, orc.bias_act(g1, inp["b1"], T, F, 3), 1e-6, 1e-6)
    assert r.ok, f"bias_gelu: {r}"
    w = orc.gemm(h, inp["W2"], np.zeros(T * D, np.float32), T, D, F)
    r = orc.compare(g2, w, orc.tol_gemm(F), orc.abs_tol_gemm(F, 0.1))
    assert r.ok, f"gemm2: {r}"
    assert np.array_equal(z, orc.bias_act(g2, inp["b2"], T, D, 0))      # bias add: exact
    r = orc.compare(y, orc.row_softmax(z, T, D), 1e-5, 1e-6)
    assert r.ok, f"softmax: {r}"
    # end to end against the oracle chain from the original inputs
    r1 = orc.gemm(inp["x"], inp["W1"], np.zeros(T * F, np.float32), T, F, D)
    r2 = orc.gemm(orc.bias_act(r1, inp["b1"], T, F, 3), inp["W2"], np.zeros(T * D, np.float32),
                  T, D, F)
    ref = orc.row_softmax(orc.bias_act(r2, inp["b2"], T, D, 0), T, D)
    assert np.max(np.abs(y - ref)) < 1e-5


@pytest.mark.parametrize("schedule", [0, 1, 2])
@pytest.mark.parametrize("memory", [0, 2, 3])
def test_mlp_block_same_bits_under_every_plan(G, orc, schedule, memory):
    T, D, F = 128, 64, 256
    inp = _mlp_inputs(orc, T, D, F)

    def run(sched, mem, streams):
        g, t = G.mlp_block(T, D, F)
        ex = G.Executor(g, schedule=sched, memory=mem, num_streams=streams, poison_buffers=True)
        ex.plan()
        for k, v in inp.items():
            ex.set_input(t[k], v)
        ex.run_sync()
        ex.run_sync()     # second run over a re-poisoned arena
        out = ex.read(t["y"], T * D)
        ex.close()
        return out

    gold = run(0, 0, 1)
    got = run(schedule, memory, 4)
    assert np.array_equal(gold.view(np.uint32), got.view(np.uint32))


@pytest.mark.parametrize("shape", [(256, 128, 512), (200, 96, 320)], ids=["whole", "ragged"])
def test_fused_mlp_block_has_the_unfused_bits(G, orc, shape):
    """mlp_block_fused (GemmBiasAct nodes: bias+GELU and the bias add in the GEMMs'
    epilogues) against mlp_block: H, Z and Y bit for bit, on a per-tensor plan and on
    a 4-stream chain-greedy plan with arena reuse over poisoned buffers; the fused
    graph has 3 nodes, and the numerics gate passes on it."""
    T, D, F = shape
    inp = _mlp_inputs(orc, T, D, F)

    def run(build, names, **kw):
        g, t = build(T, D, F)
        ex = G.Executor(g, **kw)
        ex.plan()
        for k, v in inp.items():
            ex.set_input(t[k], v)
        ex.run_sync()
        ex.run_sync()
        sizes = {"h": T * F, "z": T * D, "y": T * D}
        outs = {k: ex.read(t[k], sizes[k]) for k in names}
        info = ex.plan_info()
        ex.close()
        return outs, info

    per_tensor = dict(schedule=G.SchedulePolicy.kSequential, memory=G.MemoryPolicy.kAllocPerTensor,
                      num_streams=1)
    gold, _ = run(G.mlp_block, ("h", "z", "y"), **per_tensor)
    fused, info = run(G.mlp_block_fused, ("h", "z", "y"), **per_tensor)
    assert info["num_nodes"] == 3
    for k in ("h", "z", "y"):
        assert np.array_equal(gold[k].view(np.uint32), fused[k].view(np.uint32)), k
    reuse, _ = run(G.mlp_block_fused, ("y",), schedule=G.SchedulePolicy.kChainGreedy,
                   memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=4, poison_buffers=True)
    assert np.array_equal(gold["y"].view(np.uint32), reuse["y"].view(np.uint32))
    # And against the oracle chain from the original inputs.
    r1 = orc.gemm(inp["x"], inp["W1"], np.zeros(T * F, np.float32), T, F, D)
    r2 = orc.gemm(orc.bias_act(r1, inp["b1"], T, F, 3), inp["W2"], np.zeros(T * D, np.float32),
                  T, D, F)
    ref = orc.row_softmax(orc.bias_act(r2, inp["b2"], T, D, 0), T, D)
    assert np.max(np.abs(fused["y"] - ref)) < 1e-5
    g, t = G.mlp_block_fused(T, D, F)
    ex = G.Executor(g, num_streams=4, validate_numerics=True)
    ex.plan()
    for k, v in inp.items():
        ex.set_input(t[k], v)
    res = ex.validate_numerics(repeats=3)
    ex.close()
    assert res.passed and res.configs_compared == 9, res.detail


def test_numerics_gate_passes(G, orc):
    T, D, F = 128, 64, 256
    g, t = G.mlp_block(T, D, F)
    ex = G.Executor(g, num_streams=4, validate_numerics=True)
    ex.plan()
    for k, v in _mlp_inputs(orc, T, D, F).items():
        ex.set_input(t[k], v)
    res = ex.validate_numerics(repeats=3)
    assert res.passed, res.detail
    assert res.configs_compared == 9


def test_gemm_fanout_streams_and_parity(G, orc):
    n, B, Dp = 256, 4, 4
    g, t = G.gemm_fanout(B, Dp, n)
    ex = G.Executor(g, schedule=G.SchedulePolicy.kChainGreedy,
                    memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=4, profile=True)
    ex.plan()
    info = ex.plan_info()
    assert info["num_nodes"] == 16 and info["num_streams_used"] == 4
    assert info["num_events"] == 0 and info["waits_dedup"] == 0      # independent chains
    assert info["forkjoin_events"] == 4 + 2 * 3
    assert info["total_flops"] == 16 * 2 * n ** 3
    w = (orc.fill_random(n * n, 7) * 0.0625).astype(np.float32)
    xs = [orc.fill_random(n * n, 100 + k) for k in range(B)]
    ex.set_input(t["W"], w)
    for k in range(B):
        ex.set_input(t["xs"][k], xs[k])
    for _ in range(3):
        ex.run_async()
    ex.synchronize()
    for k in range(B):
        want = xs[k]
        for _ in range(Dp):
            want = orc.gemm(want, w, np.zeros(n * n, np.float32), n, n, n)
        got = ex.read(t["outs"][k], n * n)
        r = orc.compare(got, want, 1e-4, 1e-5)
        assert r.ok, f"branch {k}: {r}"
    tim = ex.timings()
    assert len(tim) == 16 and all(x["samples"] == 3 and x["median_ms"] > 0 for x in tim)
    assert {x["stream"] for x in tim} == {0, 1, 2, 3}


def test_starved_bias_act_diamond(G, orc):
    """The reference graph bench's starved diamond (graph_bench.cpp:138-153): two
    bias+GELU nodes whose grids are capped at a few workgroup rows and a join on
    the first.  Every output against the CPU oracle, and the same bits for caps of
    3 and 40 rows as without a cap (0)."""
    rows, cols = 1000, 512
    x = orc.fill_normal(rows * cols, 0x4400)
    b = orc.fill_random(cols, 0x4401, -0.5, 0.5)
    h = orc.bias_act(x, b, rows, cols, 3)
    seen = []
    for blocks in (0, 3, 40):
        g = G.Graph()
        tx = g.add_input((rows, cols), "X")
        tb = g.add_input((cols,), "bias")
        left = g.add_bias_act(tx, tb, "B_starved", act=3, max_row_blocks=blocks)
        right = g.add_bias_act(tx, tb, "C_starved", act=3, max_row_blocks=blocks)
        join = g.add_bias_act(left, tb, "D_join", act=3)
        g.mark_output(join)
        g.mark_output(right)
        ex = G.Executor(g, schedule=G.SchedulePolicy.kLevelParallel, num_streams=2)
        try:
            ex.plan()
            ex.set_input(tx, x)
            ex.set_input(tb, b)
            ex.run_sync()
            got_r = ex.read(right, rows * cols)
            got_d = ex.read(join, rows * cols)
        finally:
            ex.close()
        r = orc.compare(got_r, h, 1e-6, 1e-6)
        assert r.ok, f"cap {blocks}: {r}"
        # the join reads B's output, which C's output equals bit for bit
        r = orc.compare(got_d, orc.bias_act(got_r, b, rows, cols, 3), 1e-6, 1e-6)
        assert r.ok, f"cap {blocks}: {r}"
        seen.append(np.concatenate([got_r, got_d]).view(np.uint32))
    assert all(np.array_equal(seen[0], s_) for s_ in seen[1:])


def test_level_parallel_event_counts(G):
    g, _ = G.gemm_fanout(4, 4, 64)
    ex = G.Executor(g, schedule=G.SchedulePolicy.kLevelParallel, num_streams=4)
    ex.plan()
    info = ex.plan_info()
    assert info["num_events"] == 12 and info["waits_dedup"] == 36


def test_allocators_give_same_bits(G, orc):
    """The arena's allocator changes addresses, never results."""
    T, D, F = 128, 64, 256
    inp = _mlp_inputs(orc, T, D, F)
    outs = []
    for kind in (G.AllocatorKind.kRaw, G.AllocatorKind.kBuddy, G.AllocatorKind.kFreeList):
        g, t = G.mlp_block(T, D, F)
        ex = G.Executor(g, allocator=kind, schedule=G.SchedulePolicy.kChainGreedy,
                        memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=3,
                        poison_buffers=True)
        ex.plan()
        for k, v in inp.items():
            ex.set_input(t[k], v)
        ex.run_sync()
        outs.append(ex.read(t["y"], T * D))
        ex.close()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert np.array_equal(outs[0].view(np.uint32), outs[2].view(np.uint32))


@pytest.mark.parametrize("kind", ["kBuddy", "kFreeList"])
def test_allocator_reuses_across_plans(G, orc, kind):
    g, t = G.mlp_block(128, 64, 256)
    ex = G.Executor(g, allocator=getattr(G.AllocatorKind, kind), num_streams=2)
    ex.plan()
    first = ex.allocator_stats()
    ex.plan()                      # re-plan: the old arena returns, the new one reuses it
    ex.plan()
    s = ex.allocator_stats()
    assert s["raw_malloc_calls"] == first["raw_malloc_calls"]
    assert s["reuse_hits"] >= 2 and s["alloc_calls"] > first["alloc_calls"]
    info = ex.plan_info()
    assert info["arena_bytes"] <= info["naive_bytes"]
    assert s["bytes_in_use"] >= info["arena_bytes"]


# ---------------------------------------------------------------------------
# HIP graph capture of the replay loop
# ---------------------------------------------------------------------------
def _eager_y(G, inp, T, D, F, **kw):
    g, t = G.mlp_block(T, D, F)
    ex = G.Executor(g, **kw)
    ex.plan()
    for k, v in inp.items():
        ex.set_input(t[k], v)
    ex.run_sync()
    y = ex.read(t["y"], T * D)
    ex.close()
    return y


def test_memset_refused_under_capture(gpu):
    """mcke_rt_memset_async refuses a stream that is being captured (a memset node
    does not replay reliably on this stack) and names the fill kernel; the fill
    kernel captured in its place replays right, three times, with an eager memset
    of the same buffer between replays."""
    import ctypes as C

    m = gpu
    L = m.lib()
    VP = C.c_void_p
    for name, args in (("mcke_rt_stream_begin_capture", [VP]),
                       ("mcke_rt_stream_end_capture", [VP, C.POINTER(VP)]),
                       ("mcke_rt_graph_launch", [VP, VP]),
                       ("mcke_rt_graph_destroy", [VP]),
                       ("mcke_fill_u32_async", [VP, C.c_uint32, C.c_size_t, VP])):
        getattr(L, name).restype = C.c_int
        getattr(L, name).argtypes = args
    n = 4096
    buf = m.DeviceBuffer(n * 4)
    st = m.Stream()
    exe = VP()
    try:
        assert L.mcke_rt_stream_begin_capture(st.handle) == 0
        rc = L.mcke_rt_memset_async(buf.ptr, 0, n * 4, st.handle)
        msg = L.mcke_last_error().decode()
        assert L.mcke_fill_u32_async(buf.ptr, 0x3F800000, n, st.handle) == 0
        assert L.mcke_rt_stream_end_capture(st.handle, C.byref(exe)) == 0 and exe.value
        assert rc == int(m.StatusCode.kInvalidArgument), rc
        assert "mcke_fill_u32_async" in msg, msg
        for _ in range(3):
            buf.memset(0, st)                 # eager, not captured: allowed
            st.synchronize()
            assert L.mcke_rt_graph_launch(exe, st.handle) == 0
            got = buf.download(n, stream=st)
            assert np.all(got == 1.0)
    finally:
        if exe.value:
            L.mcke_rt_graph_destroy(exe)
        st.close()


@pytest.mark.parametrize("poison", [False, True])
def test_captured_replays_match_eager(G, orc, poison):
    """Every replay of the captured iteration gives the eager bits, with the
    program's own eager work and synchronisations between replays; new inputs
    written with set_input are seen by the replays."""
    import mcke_amd as m
    T, D, F = 256, 128, 512
    kw = dict(schedule=G.SchedulePolicy.kChainGreedy, memory=G.MemoryPolicy.kReuseHappensBefore,
              num_streams=4, poison_buffers=poison)
    inp = _mlp_inputs(orc, T, D, F)
    gold = _eager_y(G, inp, T, D, F, **kw)
    g, t = G.mlp_block(T, D, F)
    ex = G.Executor(g, **kw)
    ex.plan()
    for k, v in inp.items():
        ex.set_input(t[k], v)
    ex.capture()
    assert ex.captured
    scratch_x = m.DeviceBuffer.from_array(orc.fill_normal(4096, 9))
    scratch_y = m.DeviceBuffer(4096 * 4)
    for rep in range(4):
        ex.run_sync()
        got = ex.read(t["y"], T * D)
        assert np.array_equal(got.view(np.uint32), gold.view(np.uint32)), f"replay {rep}"
        # unrelated eager work between replays
        m.launch_activation_f32(scratch_x, scratch_y, 4096, m.Activation.kGeluTanh, 4).throw_if_error()
        m.device_synchronize()
    inp2 = dict(inp, x=orc.fill_normal(T * D, 77, 0.0, 1.0))
    gold2 = _eager_y(G, inp2, T, D, F, **kw)
    ex.set_input(t["x"], inp2["x"])
    for rep in range(2):
        ex.run_sync()
        assert np.array_equal(ex.read(t["y"], T * D).view(np.uint32), gold2.view(np.uint32))
    ex.plan()                              # a new plan binds new buffers: capture dropped
    assert not ex.captured
    ex.close()


@pytest.mark.parametrize("schedule,poison", [("kLevelParallel", False), ("kChainGreedy", True)])
def test_captured_fanout_across_streams(G, orc, schedule, poison):
    """A plan on several streams is assembled into one graph (one child graph per
    node, edges from stream order and cross-stream events).  Every replay, with
    the program's own eager work and synchronisations between replays, gives the
    eager bits, and the eager bits match the oracle chain of GEMMs."""
    import mcke_amd as m
    n, B, Dp = 128, 4, 3
    g, t = G.gemm_fanout(B, Dp, n)
    ex = G.Executor(g, schedule=getattr(G.SchedulePolicy, schedule),
                    memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=4, poison_buffers=poison)
    ex.plan()
    assert ex.plan_info()["num_streams_used"] > 1
    w = (orc.fill_random(n * n, 7) * 0.0625).astype(np.float32)
    xs = [orc.fill_random(n * n, 300 + k) for k in range(B)]
    ex.set_input(t["W"], w)
    for k in range(B):
        ex.set_input(t["xs"][k], xs[k])
    ex.run_sync()
    eager = [ex.read(t["outs"][k], n * n) for k in range(B)]
    ex.capture()
    assert ex.captured
    scratch_x = m.DeviceBuffer.from_array(orc.fill_normal(4096, 9))
    scratch_y = m.DeviceBuffer(4096 * 4)
    for rep in range(4):
        ex.run_sync()
        for k in range(B):
            got = ex.read(t["outs"][k], n * n)
            assert np.array_equal(got.view(np.uint32), eager[k].view(np.uint32)), (rep, k)
        m.launch_activation_f32(scratch_x, scratch_y, 4096, m.Activation.kGeluTanh, 4).throw_if_error()
        m.device_synchronize()
    # new inputs are seen by the replays
    xs2 = [orc.fill_random(n * n, 900 + k) for k in range(B)]
    for k in range(B):
        ex.set_input(t["xs"][k], xs2[k])
    ex.run_sync()
    for k in range(B):
        want = xs2[k]
        for _ in range(Dp):
            want = orc.gemm(want, w, np.zeros(n * n, np.float32), n, n, n)
        r = orc.compare(ex.read(t["outs"][k], n * n), want, 1e-4, 1e-5)
        assert r.ok, f"replay with new inputs, branch {k}: {r}"
    for k in range(B):
        want = xs[k]
        for _ in range(Dp):
            want = orc.gemm(want, w, np.zeros(n * n, np.float32), n, n, n)
        r = orc.compare(eager[k], want, 1e-4, 1e-5)
        assert r.ok, f"branch {k}: {r}"
    ex.close()


def test_captured_diamond_with_workspace_reduce(G, orc):
    """A GEMM feeding three branches (bias+GELU -> softmax, a two-pass row sum
    that uses its stream's workspace, a row max) on several streams, with
    poisoning: every replay of the assembled graph gives the eager bits."""
    T, D, F = 256, 128, 512
    g = G.Graph()
    x = g.add_input((T, D), "x")
    w1 = g.add_input((D, F), "W1")
    b1 = g.add_input((F,), "b1")
    g1 = g.add_gemm(x, w1, "gemm1")
    h = g.add_bias_act(g1, b1, "bias_gelu", act=3)
    y = g.add_softmax(h, "softmax")
    rs = g.add_reduce(g1, "row_sum", kind=0, variant=2)
    rm = g.add_reduce(g1, "row_max", kind=1, variant=1)
    for o in (y, rs, rm):
        g.mark_output(o)
    ex = G.Executor(g, schedule=G.SchedulePolicy.kLevelParallel,
                    memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=3, poison_buffers=True)
    ex.plan()
    assert ex.plan_info()["num_streams_used"] > 1
    ex.set_input(x, orc.fill_normal(T * D, 11, 0.0, 1.0))
    ex.set_input(w1, orc.fill_normal(D * F, 12, 0.0, 0.05))
    ex.set_input(b1, orc.fill_normal(F, 13, 0.0, 0.01))
    ex.run_sync()
    outs = ((y, T * F), (rs, T), (rm, T))
    eager = [ex.read(o, n) for o, n in outs]
    ex.capture()
    for rep in range(3):
        ex.run_sync()
        for (o, n), want in zip(outs, eager):
            assert np.array_equal(ex.read(o, n).view(np.uint32), want.view(np.uint32)), (rep, o)
    ex.close()


def test_capture_refused_with_timing_probes(G):
    g, _ = G.mlp_block(64, 64, 64)
    ex = G.Executor(g, num_streams=2, profile=True)
    ex.plan()
    with pytest.raises(Exception, match="FailedPrecondition|timing probes"):
        ex.capture()
    assert not ex.captured
    ex.close()


@pytest.mark.parametrize("dt", [2, 1], ids=["bf16", "f16"])
def test_16bit_gemm_node_feeds_f32_ops(G, orc, dt):
    """A GEMM node on 16-bit inputs (the 16-bit MFMA kernel) with f32 C feeding
    bias+GELU, and a second node writing 16-bit C, against the oracle on the
    decoded inputs."""
    T, D, F = 256, 128, 512
    g = G.Graph()
    x = g.add_input((T, D), "x", dtype=dt)
    w1 = g.add_input((D, F), "W1", dtype=dt)
    b1 = g.add_input((F,), "b1")
    h32 = g.add_gemm_lp(x, w1, "gemm_lp")
    h = g.add_bias_act(h32, b1, "bias_gelu", act=3)
    h16 = g.add_gemm_lp(x, w1, "gemm_lp16", out_dtype=dt)
    for t in (h32, h, h16):
        g.mark_output(t)
    ex = G.Executor(g, schedule=G.SchedulePolicy.kSequential,
                    memory=G.MemoryPolicy.kAllocPerTensor, num_streams=1)
    ex.plan()
    xq = orc.to_16(orc.fill_normal(T * D, 11, 0.0, 1.0), dt)
    wq = orc.to_16(orc.fill_normal(D * F, 12, 0.0, 0.02), dt)
    bias = orc.fill_normal(F, 13, 0.0, 0.01)
    ex.set_input(x, xq)
    ex.set_input(w1, wq)
    ex.set_input(b1, bias)
    ex.run_sync()
    got32 = ex.read(h32, T * F)
    want32 = orc.gemm_lp(xq, wq, np.zeros(T * F, np.float32), T, F, D, 1.0, 0.0, dt, 0)
    r = orc.compare(got32, want32, orc.tol_gemm(D), orc.abs_tol_gemm(D, 4.0 * 0.02 * 4.0))
    assert r.ok, f"gemm_lp: {r}"
    r = orc.compare(ex.read(h, T * F), orc.bias_act(got32, bias, T, F, 3), 1e-6, 1e-6)
    assert r.ok, f"bias_gelu: {r}"
    got16 = orc.from_16(ex.read(h16, T * F, np.uint16), dt)
    want16 = orc.from_16(orc.to_16(want32, dt), dt)
    ulp = 2.0 ** -7 if dt == 2 else 2.0 ** -10
    r = orc.compare(got16, want16, orc.tol_gemm(D) + ulp, orc.abs_tol_gemm(D, 4.0 * 0.02 * 4.0))
    assert r.ok, f"gemm_lp 16-bit C: {r}"


def test_captured_split_reduce_replays(G, orc):
    """kTwoPass nodes whose rows split over workgroups (captured, they take the
    two-launch path, partials then fold, since a graph may be replayed on any
    stream); two of them on different streams of one captured graph.  Every
    replay, also after new
    inputs, matches the eager launch's bits and the double-accumulating CPU
    reduce (reference tests/reference.hpp:154-172)."""
    g = G.Graph()
    a = g.add_input((2, 65536), "a")
    b = g.add_input((3, 40000), "b")
    ra = g.add_reduce(a, "sum_a", kind=0, variant=2)
    rb = g.add_reduce(b, "mean_b", kind=2, variant=2)
    g.mark_output(ra)
    g.mark_output(rb)
    ex = G.Executor(g, schedule=G.SchedulePolicy.kLevelParallel,
                    memory=G.MemoryPolicy.kReuseHappensBefore, num_streams=2)
    ex.plan()
    assert ex.plan_info()["num_streams_used"] == 2
    captured = False
    for rep in range(4):
        xa = orc.fill_normal(2 * 65536, 0x5A0 + rep, 0.0, 1.0)
        xb = orc.fill_normal(3 * 40000, 0x5B0 + rep, 0.0, 1.0)
        ex.set_input(a, xa)
        ex.set_input(b, xb)
        if not captured:
            ex.run_sync()
            eager = (ex.read(ra, 2).copy(), ex.read(rb, 3).copy())
            ex.capture()
            captured = True
            ex.run_sync()
            assert np.array_equal(ex.read(ra, 2).view(np.uint32), eager[0].view(np.uint32))
            assert np.array_equal(ex.read(rb, 3).view(np.uint32), eager[1].view(np.uint32))
        else:
            ex.run_sync()
        for out, x, rows, cols, kind in ((ra, xa, 2, 65536, 0), (rb, xb, 3, 40000, 2)):
            got = ex.read(out, rows)
            want = orc.row_reduce(x, rows, cols, kind)
            floor = 5e-5 * (1.0 / 0.577) * np.sqrt(cols / 4096.0)
            if kind == 2:
                floor /= cols
            r = orc.compare(got, want, 1e-5, floor)
            assert r.ok, f"replay {rep} kind {kind}: {r}"
    ex.close()


@pytest.mark.parametrize("plan", ["mlp_64x64x256_2streams", "chain32_64x1024_1stream",
                                  "fanout_4x4_256_4streams"])
def test_capture_if_faster_keeps_the_faster_path(G, orc, plan):
    """capture_if_faster measures eager issue against graph replay on the plan and
    keeps the graph only where replay was faster; either way the executor's
    outputs are the eager bits, before and after the choice, over several runs."""
    if plan.startswith("mlp"):
        T, D, F = 64, 64, 256
        g, t = G.mlp_block(T, D, F)
        kw = dict(schedule=G.SchedulePolicy.kChainGreedy, num_streams=2)
        inputs = {t[k]: v for k, v in _mlp_inputs(orc, T, D, F).items()}
        outs = [(t["y"], T * D)]
        build = lambda: G.mlp_block(T, D, F)  # noqa: E731
    elif plan.startswith("chain"):
        build = lambda: G.chain(32, 64, 1024)  # noqa: E731
        g, t = build()
        kw = dict(schedule=G.SchedulePolicy.kSequential, num_streams=1)
        inputs = {t["x"]: orc.fill_normal(64 * 1024, 0x5100), t["bias"]: orc.fill_random(1024, 0x5101, -0.5, 0.5)}
        outs = [(t["outs"][0], 64 * 1024)]
    else:
        n = 256
        build = lambda: G.gemm_fanout(4, 4, n)  # noqa: E731
        g, t = build()
        kw = dict(schedule=G.SchedulePolicy.kChainGreedy, num_streams=4)
        inputs = {t["W"]: orc.fill_random(n * n, 0x4100, -0.0625, 0.0625)}
        inputs.update({x: orc.fill_random(n * n, 0x4101 + k) for k, x in enumerate(t["xs"])})
        outs = [(o, n * n) for o in t["outs"]]

    def run(ex):
        ex.run_sync()
        return [ex.read(o, k).view(np.uint32) for o, k in outs]

    ref = G.Executor(g, **kw)
    ref.plan()
    for tid, arr in inputs.items():
        ref.set_input(tid, arr)
    gold = run(ref)
    ref.close()

    g, t2 = build()
    ex = G.Executor(g, **kw)
    ex.plan()
    for tid, arr in inputs.items():
        ex.set_input(tid, arr)
    d = ex.capture_if_faster(trials=40)
    print(plan, d)
    assert d["eager_us_per_run"] > 0 and d["replay_us_per_run"] > 0
    assert d["captured"] == (d["replay_us_per_run"] < d["eager_us_per_run"])
    assert ex.captured == d["captured"]
    for rep in range(3):
        for got, want in zip(run(ex), gold):
            assert np.array_equal(got, want), f"{plan} run {rep} (captured={d['captured']})"
    ex.close()


def test_captured_fused_mlp_replays_match_unfused_eager(G, orc):
    """The fused MLP (GemmBiasAct nodes) captured into one HIP graph: every replay,
    with unrelated eager work between them, gives the unfused graph's eager bits."""
    import mcke_amd as m
    T, D, F = 256, 128, 512
    kw = dict(schedule=G.SchedulePolicy.kChainGreedy, memory=G.MemoryPolicy.kReuseHappensBefore,
              num_streams=4, poison_buffers=True)
    inp = _mlp_inputs(orc, T, D, F)
    gold = _eager_y(G, inp, T, D, F, **kw)
    g, t = G.mlp_block_fused(T, D, F)
    ex = G.Executor(g, **kw)
    ex.plan()
    for k, v in inp.items():
        ex.set_input(t[k], v)
    ex.capture()
    assert ex.captured
    scratch_x = m.DeviceBuffer.from_array(orc.fill_normal(4096, 9))
    scratch_y = m.DeviceBuffer(4096 * 4)
    for rep in range(4):
        ex.run_sync()
        got = ex.read(t["y"], T * D)
        assert np.array_equal(got.view(np.uint32), gold.view(np.uint32)), f"replay {rep}"
        m.launch_activation_f32(scratch_x, scratch_y, 4096, m.Activation.kGeluTanh, 4).throw_if_error()
        m.device_synchronize()
    ex.close()
