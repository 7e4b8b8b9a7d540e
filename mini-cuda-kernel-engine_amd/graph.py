"""Graph layer of the MCKE kernel layer, over the C-ABI in include/mcke_graph.h.

Mirrors the reference's C++ Graph / GraphExecutor (reference
include/mcke/graph/graph.hpp and executor.hpp): build a DAG of Gemm / BiasAct /
Reduce / Softmax nodes, plan it onto HIP streams and one arena under a schedule
and memory policy, replay it, and read back outputs, plan statistics, per-node
timings, allocator statistics and the bitwise numerics gate.
"""
from __future__ import annotations

import ctypes as C
import enum
import os
from dataclasses import dataclass

import numpy as np

from . import (HERE, GemmTile, GemmVariant, MckeError, Status, StatusCode, _sh,
               lib as _amd_lib)

HOST_LIB_PATH = os.path.join(HERE, "lib", "libmcke_host.so")


class SchedulePolicy(enum.IntEnum):      # schedule.hpp:49
    kSequential = 0
    kLevelParallel = 1
    kChainGreedy = 2


class MemoryPolicy(enum.IntEnum):        # memory_plan.hpp
    kAllocPerTensor = 0
    kReuseTopoNaive = 1
    kReuseSameStream = 2
    kReuseHappensBefore = 3


class AllocatorKind(enum.IntEnum):
    kRaw = 0
    kBuddy = 1
    kFreeList = 2


class ExecutorOptions(C.Structure):
    _fields_ = [("schedule", C.c_int32), ("memory", C.c_int32), ("num_streams", C.c_int32),
                ("profile", C.c_int32), ("profile_slots", C.c_int32),
                ("validate_numerics", C.c_int32), ("poison_buffers", C.c_int32),
                ("poison_pattern", C.c_uint32)]


class PlanInfo(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "num_nodes", "num_streams_used", "num_streams_requested", "num_events", "waits_raw",
        "waits_dedup", "forkjoin_events", "arena_bytes", "naive_bytes", "buffers_used",
        "total_flops", "total_bytes")]

    def asdict(self):
        return {n: int(getattr(self, n)) for n, _ in self._fields_}


class NodeTiming(C.Structure):
    _fields_ = [("node", C.c_uint32), ("stream_idx", C.c_int32), ("median_ms", C.c_double),
                ("min_ms", C.c_double), ("flops", C.c_uint64), ("bytes", C.c_uint64),
                ("samples", C.c_int32), ("name", C.c_char * 64)]


class AllocatorStats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "alloc_calls", "free_calls", "raw_malloc_calls", "raw_free_calls", "oom_events",
        "deferred_reuses", "blocking_drains", "reuse_hits", "bytes_reserved", "bytes_in_use",
        "bytes_requested", "peak_bytes_in_use", "largest_free_block")]

    def asdict(self):
        return {n: int(getattr(self, n)) for n, _ in self._fields_}


_hl = None
_VP, _U32, _U32P = C.c_void_p, C.c_uint32, C.POINTER(C.c_uint32)


def host_lib() -> C.CDLL:
    global _hl
    if _hl is not None:
        return _hl
    _amd_lib()   # libmcke_amd.so first: libmcke_host.so links against it
    if not os.path.exists(HOST_LIB_PATH):
        raise RuntimeError(f"{HOST_LIB_PATH} is missing: run __graft_entry__.build()")
    L = C.CDLL(HOST_LIB_PATH)
    sig = {
        "mcke_graph_last_error": (C.c_char_p, []),
        "mcke_graph_create": (_VP, []),
        "mcke_graph_destroy": (None, [_VP]),
        "mcke_graph_add_input": (C.c_int, [_VP, C.POINTER(C.c_int64), C.c_int, C.c_char_p, _U32P]),
        "mcke_graph_add_input_typed": (C.c_int, [_VP, C.POINTER(C.c_int64), C.c_int, C.c_int,
                                                 C.c_char_p, _U32P]),
        "mcke_graph_add_gemm_lp": (C.c_int, [_VP, _U32, _U32, C.c_float, C.c_int,
                                             C.POINTER(GemmTile), C.c_char_p, _U32P]),
        "mcke_graph_add_gemm": (C.c_int, [_VP, _U32, _U32, C.c_float, C.c_int, C.POINTER(GemmTile),
                                          C.c_char_p, _U32P]),
        "mcke_graph_add_gemm_bias_act": (C.c_int, [_VP, _U32, _U32, _U32, C.c_float, C.c_int,
                                                   C.POINTER(GemmTile), C.c_char_p, _U32P]),
        "mcke_graph_add_bias_act": (C.c_int, [_VP, _U32, _U32, C.c_int, C.c_int, C.c_char_p, _U32P]),
        "mcke_graph_add_bias_act_rows": (C.c_int, [_VP, _U32, _U32, C.c_int, C.c_int, C.c_int,
                                                   C.c_char_p, _U32P]),
        "mcke_graph_add_reduce": (C.c_int, [_VP, _U32, C.c_int, C.c_int, C.c_char_p, _U32P]),
        "mcke_graph_add_softmax": (C.c_int, [_VP, _U32, C.c_int, C.c_char_p, _U32P]),
        "mcke_graph_mark_output": (C.c_int, [_VP, _U32]),
        "mcke_graph_num_nodes": (C.c_int, [_VP, C.POINTER(C.c_uint64)]),
        "mcke_graph_tensor_shape": (C.c_int, [_VP, _U32, C.POINTER(C.c_int64), C.POINTER(C.c_int)]),
        "mcke_executor_create": (C.c_int, [_VP, C.c_int, C.POINTER(ExecutorOptions), C.POINTER(_VP)]),
        "mcke_executor_destroy": (None, [_VP]),
        "mcke_executor_plan": (C.c_int, [_VP]),
        "mcke_executor_set_input": (C.c_int, [_VP, _U32, _VP, C.c_size_t]),
        "mcke_executor_run_async": (C.c_int, [_VP]),
        "mcke_executor_synchronize": (C.c_int, [_VP]),
        "mcke_executor_capture": (C.c_int, [_VP]),
        "mcke_executor_capture_if_faster": (C.c_int, [_VP, C.c_int, C.POINTER(C.c_int),
                                                      C.POINTER(C.c_double), C.POINTER(C.c_double)]),
        "mcke_executor_is_captured": (C.c_int, [_VP, C.POINTER(C.c_int)]),
        "mcke_executor_read_tensor": (C.c_int, [_VP, _U32, _VP, C.c_size_t]),
        "mcke_executor_plan_info": (C.c_int, [_VP, C.POINTER(PlanInfo)]),
        "mcke_executor_collect_timings": (C.c_int, [_VP, C.POINTER(NodeTiming), C.c_size_t,
                                                    C.POINTER(C.c_size_t)]),
        "mcke_executor_validate_numerics": (C.c_int, [_VP, C.c_int, C.POINTER(C.c_int),
                                                      C.POINTER(C.c_int), C.c_char_p, C.c_size_t]),
        "mcke_executor_allocator_stats": (C.c_int, [_VP, C.POINTER(AllocatorStats)]),
        "mcke_executor_stream": (C.c_int, [_VP, C.POINTER(_VP)]),
        "mcke_executor_describe": (C.c_int, [_VP, C.c_char_p, C.c_size_t]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _hl = L
    return L


def host_library_path() -> str:
    return HOST_LIB_PATH


def _check(rc: int) -> None:
    if rc == 0:
        return
    msg = host_lib().mcke_graph_last_error() or b""
    if not msg:
        msg = _amd_lib().mcke_last_error() or b""
    raise MckeError(Status(StatusCode(rc), msg.decode()))


class Graph:
    """A DAG of kernel-backed ops (reference Graph).  Tensors are f32 unless an
    input is declared bf16 / f16 (`dtype`); only GEMM nodes take 16-bit inputs."""

    def __init__(self):
        self.h = host_lib().mcke_graph_create()
        self.names: dict[int, str] = {}

    def _out(self, rc, out):
        _check(rc)
        return int(out.value)

    def add_input(self, shape, name: str, dtype: int = 0) -> int:
        """dtype: 0 f32 (the default), 1 f16, 2 bf16 (DType numbering)."""
        dims = (C.c_int64 * len(shape))(*shape)
        out = C.c_uint32()
        if int(dtype) == 0:
            rc = host_lib().mcke_graph_add_input(self.h, dims, len(shape), name.encode(),
                                                 C.byref(out))
        else:
            rc = host_lib().mcke_graph_add_input_typed(self.h, dims, len(shape), int(dtype),
                                                       name.encode(), C.byref(out))
        t = self._out(rc, out)
        self.names[t] = name
        return t

    def add_gemm_lp(self, a: int, b: int, name: str, out_dtype: int = 0,
                    tile: GemmTile | None = None, alpha: float = 1.0) -> int:
        """GEMM on 16-bit inputs (a, b both bf16 or both f16); C in out_dtype
        (0 = f32, or the input type).  tile None: the per-shape default."""
        out = C.c_uint32()
        tp = C.byref(tile) if tile is not None else None
        return self._out(host_lib().mcke_graph_add_gemm_lp(self.h, a, b, alpha, int(out_dtype), tp,
                                                           name.encode(), C.byref(out)), out)

    def add_gemm(self, a: int, b: int, name: str, variant=GemmVariant.kMfmaF32,
                 tile: GemmTile | None = None, alpha: float = 1.0) -> int:
        out = C.c_uint32()
        tp = C.byref(tile) if tile is not None else None
        return self._out(host_lib().mcke_graph_add_gemm(self.h, a, b, alpha, int(variant), tp,
                                                        name.encode(), C.byref(out)), out)

    def add_gemm_bias_act(self, a: int, b: int, bias: int, name: str, act=3,
                          tile: GemmTile | None = None, alpha: float = 1.0) -> int:
        """GEMM (kMfmaF32) with the bias + activation in its epilogue: one node with
        the bits of add_gemm -> add_bias_act.  tile None: the per-shape default."""
        out = C.c_uint32()
        tp = C.byref(tile) if tile is not None else None
        return self._out(host_lib().mcke_graph_add_gemm_bias_act(
            self.h, a, b, bias, alpha, int(act), tp, name.encode(), C.byref(out)), out)

    def add_bias_act(self, x: int, bias: int, name: str, act=3, vector_width: int = 0,
                     max_row_blocks: int = 0) -> int:
        """max_row_blocks caps the launch grid's row dimension (0 = automatic)."""
        out = C.c_uint32()
        return self._out(host_lib().mcke_graph_add_bias_act_rows(
            self.h, x, bias, int(act), vector_width, max_row_blocks, name.encode(),
            C.byref(out)), out)

    def add_reduce(self, x: int, name: str, kind=0, variant=1) -> int:
        out = C.c_uint32()
        return self._out(host_lib().mcke_graph_add_reduce(self.h, x, int(kind), int(variant),
                                                          name.encode(), C.byref(out)), out)

    def add_softmax(self, x: int, name: str, variant=1) -> int:
        out = C.c_uint32()
        return self._out(host_lib().mcke_graph_add_softmax(self.h, x, int(variant), name.encode(),
                                                           C.byref(out)), out)

    def mark_output(self, t: int) -> None:
        _check(host_lib().mcke_graph_mark_output(self.h, t))

    def shape(self, t: int) -> tuple:
        dims = (C.c_int64 * 5)()
        rank = C.c_int()
        _check(host_lib().mcke_graph_tensor_shape(self.h, t, dims, C.byref(rank)))
        return tuple(int(dims[i]) for i in range(rank.value))

    def __del__(self):
        if getattr(self, "h", None):
            host_lib().mcke_graph_destroy(self.h)
            self.h = None


@dataclass
class NumericsResult:
    passed: bool
    configs_compared: int
    detail: str


class Executor:
    """GraphExecutor over a Graph (which it consumes)."""

    def __init__(self, graph: Graph, allocator=AllocatorKind.kBuddy,
                 schedule=SchedulePolicy.kChainGreedy, memory=MemoryPolicy.kReuseHappensBefore,
                 num_streams: int = 4, profile: bool = False, profile_slots: int = 32,
                 validate_numerics: bool = False, poison_buffers: bool = False):
        opts = ExecutorOptions(int(schedule), int(memory), num_streams, int(profile), profile_slots,
                               int(validate_numerics), int(poison_buffers), 0)
        h = _VP()
        _check(host_lib().mcke_executor_create(graph.h, int(allocator), C.byref(opts), C.byref(h)))
        graph.h = None            # consumed
        self.h = h.value

    def plan(self) -> None:
        _check(host_lib().mcke_executor_plan(self.h))

    def set_input(self, t: int, arr: np.ndarray) -> None:
        """f32 tensors take float arrays; 16-bit tensors take uint16 bit patterns."""
        arr = np.ascontiguousarray(arr, dtype=np.uint16 if arr.dtype == np.uint16 else np.float32)
        _check(host_lib().mcke_executor_set_input(self.h, t, arr.ctypes.data, arr.nbytes))

    def run_async(self) -> None:
        _check(host_lib().mcke_executor_run_async(self.h))

    def synchronize(self) -> None:
        _check(host_lib().mcke_executor_synchronize(self.h))

    def run_sync(self) -> None:
        self.run_async()
        self.synchronize()

    def capture(self) -> None:
        """Capture one iteration into a HIP graph; later run_async() replays it."""
        _check(host_lib().mcke_executor_capture(self.h))

    def capture_if_faster(self, trials: int = 50) -> dict:
        """Capture, then keep the HIP graph only if replay measures faster than eager
        issue on this plan (GraphExecutor::capture_if_faster)."""
        cap, e_us, r_us = C.c_int(0), C.c_double(0.0), C.c_double(0.0)
        _check(host_lib().mcke_executor_capture_if_faster(self.h, trials, C.byref(cap), C.byref(e_us),
                                                          C.byref(r_us)))
        return {"captured": bool(cap.value), "eager_us_per_run": e_us.value,
                "replay_us_per_run": r_us.value, "trials": trials}

    @property
    def captured(self) -> bool:
        out = C.c_int(0)
        _check(host_lib().mcke_executor_is_captured(self.h, C.byref(out)))
        return bool(out.value)

    def read(self, t: int, numel: int, dtype=np.float32) -> np.ndarray:
        """dtype np.uint16 reads a 16-bit tensor's bit patterns."""
        out = np.empty(numel, dtype=dtype)
        _check(host_lib().mcke_executor_read_tensor(self.h, t, out.ctypes.data, out.nbytes))
        return out

    def plan_info(self) -> dict:
        info = PlanInfo()
        _check(host_lib().mcke_executor_plan_info(self.h, C.byref(info)))
        return info.asdict()

    def timings(self) -> list[dict]:
        n = C.c_size_t()
        _check(host_lib().mcke_executor_collect_timings(self.h, None, 0, C.byref(n)))
        arr = (NodeTiming * max(1, n.value))()
        _check(host_lib().mcke_executor_collect_timings(self.h, arr, n.value, C.byref(n)))
        return [{"node": t.node, "name": t.name.decode(), "stream": t.stream_idx,
                 "median_ms": t.median_ms, "min_ms": t.min_ms, "flops": t.flops,
                 "bytes": t.bytes, "samples": t.samples} for t in arr[:n.value]]

    def validate_numerics(self, repeats: int = 3) -> NumericsResult:
        passed, cfgs = C.c_int(), C.c_int()
        buf = C.create_string_buffer(2048)
        _check(host_lib().mcke_executor_validate_numerics(self.h, repeats, C.byref(passed),
                                                          C.byref(cfgs), buf, 2048))
        return NumericsResult(bool(passed.value), cfgs.value, buf.value.decode())

    def allocator_stats(self) -> dict:
        s = AllocatorStats()
        _check(host_lib().mcke_executor_allocator_stats(self.h, C.byref(s)))
        return s.asdict()

    def stream(self) -> int:
        s = _VP()
        _check(host_lib().mcke_executor_stream(self.h, C.byref(s)))
        return s.value

    def describe(self) -> str:
        buf = C.create_string_buffer(1 << 16)
        _check(host_lib().mcke_executor_describe(self.h, buf, 1 << 16))
        return buf.value.decode()

    def close(self) -> None:
        if getattr(self, "h", None):
            host_lib().mcke_executor_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def mlp_block(tokens: int, d_model: int, d_ff: int, gemm_variant=GemmVariant.kMfmaF32):
    """BASELINE config 5's main chain: H = GELU(X W1 + b1); Z = H W2 + b2; softmax(Z)
    (the reference's transformer_block, graph_bench.cpp:199-215, plus the b2 node)."""
    g = Graph()
    x = g.add_input((tokens, d_model), "x")
    w1 = g.add_input((d_model, d_ff), "W1")
    b1 = g.add_input((d_ff,), "b1")
    w2 = g.add_input((d_ff, d_model), "W2")
    b2 = g.add_input((d_model,), "b2")
    g1 = g.add_gemm(x, w1, "gemm1", gemm_variant)
    h = g.add_bias_act(g1, b1, "bias_gelu", act=3)
    g2 = g.add_gemm(h, w2, "gemm2", gemm_variant)
    z = g.add_bias_act(g2, b2, "bias_add", act=0)
    y = g.add_softmax(z, "softmax")
    g.mark_output(y)
    return g, {"x": x, "W1": w1, "b1": b1, "W2": w2, "b2": b2, "gemm1": g1, "h": h, "gemm2": g2,
               "z": z, "y": y}


def mlp_block_fused(tokens: int, d_model: int, d_ff: int):
    """mlp_block with each GEMM -> bias+act pair as one fused node:
    H = GELU(X W1 + b1) and Z = H W2 + b2 in the GEMMs' epilogues, then softmax(Z).
    The same tensors under the same names (no "gemm1"/"gemm2": C is never stored),
    and the same output bits."""
    g = Graph()
    x = g.add_input((tokens, d_model), "x")
    w1 = g.add_input((d_model, d_ff), "W1")
    b1 = g.add_input((d_ff,), "b1")
    w2 = g.add_input((d_ff, d_model), "W2")
    b2 = g.add_input((d_model,), "b2")
    h = g.add_gemm_bias_act(x, w1, b1, "gemm1_bias_gelu", act=3)
    z = g.add_gemm_bias_act(h, w2, b2, "gemm2_bias_add", act=0)
    y = g.add_softmax(z, "softmax")
    g.mark_output(y)
    return g, {"x": x, "W1": w1, "b1": b1, "W2": w2, "b2": b2, "h": h, "z": z, "y": y}


def gemm_fanout(branches: int, depth: int, n: int, gemm_variant=GemmVariant.kMfmaF32):
    """`branches` independent chains of `depth` n^3 GEMMs: chain k is
    C_k0 = X_k W, C_kd = C_k(d-1) W (the reference's fanout topology,
    graph_bench.cpp:176-194, with GEMM nodes).  The returned "nodes"[k][d] is the
    output of GEMM d of chain k."""
    g = Graph()
    w = g.add_input((n, n), "W")
    xs, outs, nodes = [], [], []
    for k in range(branches):
        cur = g.add_input((n, n), f"x{k}")
        xs.append(cur)
        chain = []
        for d in range(depth):
            cur = g.add_gemm(cur, w, f"b{k}g{d}", gemm_variant)
            chain.append(cur)
        g.mark_output(cur)
        outs.append(cur)
        nodes.append(chain)
    return g, {"W": w, "xs": xs, "outs": outs, "nodes": nodes}


# ---------------------------------------------------------------------------
# The reference graph bench's five topologies (bench/graph_bench.cpp:100-215, run at
# :477-481).  Each returns (graph, tensors): the graph's inputs, every node's output
# under its node name and "outs", the graph outputs.  Activations are GELU_tanh as
# in the reference's bias_act_op (:91-96).  GEMM nodes run this build's kMfmaF32
# kernel with the tile picked per shape, where the reference's run its
# register-blocked FFMA kernel (gemm_op, :85-90).
# ---------------------------------------------------------------------------

def diamond_gemm(n: int):
    """B = A W and C = A W, then D = B C (graph_bench.cpp:100-113)."""
    g = Graph()
    a = g.add_input((n, n), "A")
    w = g.add_input((n, n), "W")
    left = g.add_gemm(a, w, "B_gemm")
    right = g.add_gemm(a, w, "C_gemm")
    d = g.add_gemm(left, right, "D_gemm")
    g.mark_output(d)
    return g, {"A": a, "W": w, "B_gemm": left, "C_gemm": right, "D_gemm": d, "outs": [d]}


def chain(nodes: int, rows: int, cols: int):
    """`nodes` bias+GELU nodes in a row over x[rows x cols], all with one bias
    (graph_bench.cpp:155-171)."""
    g = Graph()
    x = g.add_input((rows, cols), "x")
    bias = g.add_input((cols,), "bias")
    t = {"x": x, "bias": bias}
    cur = x
    for i in range(nodes):
        cur = g.add_bias_act(cur, bias, f"n{i}", act=3)
        t[f"n{i}"] = cur
    g.mark_output(cur)
    t["outs"] = [cur]
    return g, t


def fanout(branches: int, depth: int, rows: int, cols: int, max_row_blocks: int):
    """`branches` chains of `depth` bias+GELU nodes, every chain starting from x and
    every node's grid capped at `max_row_blocks` row blocks (graph_bench.cpp:173-194;
    the reference benches fanout(4, 4, 2048, 2048, 10)).  Node d of chain k is
    "b{k}n{d}"."""
    g = Graph()
    x = g.add_input((rows, cols), "x")
    bias = g.add_input((cols,), "bias")
    t = {"x": x, "bias": bias, "outs": []}
    for k in range(branches):
        cur = x
        for d in range(depth):
            cur = g.add_bias_act(cur, bias, f"b{k}n{d}", act=3, max_row_blocks=max_row_blocks)
            t[f"b{k}n{d}"] = cur
        g.mark_output(cur)
        t["outs"].append(cur)
    return g, t


def diamond_starved(rows: int, cols: int, max_row_blocks: int):
    """B and C: bias+GELU of X with grids capped at `max_row_blocks` row blocks; D:
    bias+GELU of B, uncapped; outputs D and C (graph_bench.cpp:138-153)."""
    g = Graph()
    x = g.add_input((rows, cols), "X")
    bias = g.add_input((cols,), "bias")
    left = g.add_bias_act(x, bias, "B_starved", act=3, max_row_blocks=max_row_blocks)
    right = g.add_bias_act(x, bias, "C_starved", act=3, max_row_blocks=max_row_blocks)
    d = g.add_bias_act(left, bias, "D_join", act=3)
    g.mark_output(d)
    g.mark_output(right)
    return g, {"X": x, "bias": bias, "B_starved": left, "C_starved": right, "D_join": d,
               "outs": [d, right]}


def transformer_block(tokens: int, d_model: int, d_ff: int):
    """GEMM -> bias+GELU -> GEMM -> row softmax, no second bias
    (graph_bench.cpp:199-215; benched at (4096, 1024, 4096))."""
    g = Graph()
    x = g.add_input((tokens, d_model), "x")
    w1 = g.add_input((d_model, d_ff), "W1")
    b1 = g.add_input((d_ff,), "b1")
    w2 = g.add_input((d_ff, d_model), "W2")
    g1 = g.add_gemm(x, w1, "gemm1")
    h = g.add_bias_act(g1, b1, "bias_gelu", act=3)
    g2 = g.add_gemm(h, w2, "gemm2")
    y = g.add_softmax(g2, "softmax")
    g.mark_output(y)
    return g, {"x": x, "W1": w1, "b1": b1, "W2": w2, "gemm1": g1, "bias_gelu": h, "gemm2": g2,
               "softmax": y, "outs": [y]}


def transformer_block_fused(tokens: int, d_model: int, d_ff: int):
    """transformer_block with its GEMM -> bias+GELU pair as one GemmBiasAct node
    (the bias and GELU in GEMM1's epilogue): three nodes, the same tensors under
    the same names except "gemm1" (never stored), and the same output bits."""
    g = Graph()
    x = g.add_input((tokens, d_model), "x")
    w1 = g.add_input((d_model, d_ff), "W1")
    b1 = g.add_input((d_ff,), "b1")
    w2 = g.add_input((d_ff, d_model), "W2")
    h = g.add_gemm_bias_act(x, w1, b1, "gemm1_bias_gelu", act=3)
    g2 = g.add_gemm(h, w2, "gemm2")
    y = g.add_softmax(g2, "softmax")
    g.mark_output(y)
    return g, {"x": x, "W1": w1, "b1": b1, "W2": w2, "bias_gelu": h, "gemm2": g2,
               "softmax": y, "outs": [y]}


# name -> (builder, {input name: ("u", seed, lo, hi) | ("n", seed, mean, sigma)}): the
# five graphs the reference's graph bench runs, at its shapes (graph_bench.cpp:477-481),
# with seeded inputs drawn by fill_random (U[lo, hi)) or fill_normal (N(mean, sigma^2)).
REFERENCE_GRAPHS = {
    "diamond_gemm_2048": (lambda: diamond_gemm(2048),
                          {"A": ("u", 0x4200, -0.0625, 0.0625), "W": ("u", 0x4201, -0.0625, 0.0625)}),
    "chain16": (lambda: chain(16, 4096, 4096),
                {"x": ("n", 0x4300, 0.0, 1.0), "bias": ("u", 0x4301, -0.5, 0.5)}),
    "fanout4x4": (lambda: fanout(4, 4, 2048, 2048, 10),
                  {"x": ("n", 0x4600, 0.0, 1.0), "bias": ("u", 0x4601, -0.5, 0.5)}),
    "diamond_starved": (lambda: diamond_starved(8192, 4096, 40),
                        {"X": ("n", 0x4400, 0.0, 1.0), "bias": ("u", 0x4401, -0.5, 0.5)}),
    "transformer_block": (lambda: transformer_block(4096, 1024, 4096),
                          {"x": ("n", 0x4500, 0.0, 1.0), "W1": ("n", 0x4501, 0.0, 0.02),
                           "b1": ("n", 0x4502, 0.0, 0.01), "W2": ("n", 0x4503, 0.0, 0.02)}),
}


def reference_graph(name: str, fill_random, fill_normal):
    """(graph, tensors, {tensor id: host input}) for REFERENCE_GRAPHS[name], the
    inputs drawn with the given generators (the package's or the oracle's, which
    give the same bits)."""
    build, spec = REFERENCE_GRAPHS[name]
    g, t = build()
    inputs = {}
    for key, (kind, seed, p0, p1) in spec.items():
        n = 1
        for d in g.shape(t[key]):
            n *= d
        inputs[t[key]] = fill_random(n, seed, p0, p1) if kind == "u" else fill_normal(n, seed, p0, p1)
    return g, t, inputs
