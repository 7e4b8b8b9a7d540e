"""kTwoPass: split rows, partials in the caller's workspace, a fold launch.

A kTwoPass launch whose rows are split over several workgroups stores one partial
per workgroup in the caller's workspace, and a second launch on the same stream
folds each row's partials in a fixed order.  The launcher keeps no state between
calls (reference kernels.hpp:182-197).  These tests check what that has to
guarantee, each against the double-accumulating CPU reduce (reference
tests/reference.hpp:154-172; max bit-exact):

* back-to-back launches of different shapes and kinds on one stream, with no
  synchronisation between them and half of them sharing one workspace;
* the same full sum repeated gives the same bits;
* launches on several streams at once, each with its own workspace, and two
  host threads launching on the per-thread default stream;
* streams created and destroyed with plain hipStreamDestroy (not through this
  library) while their launches may still run, and launches on the fresh
  streams created after them, which may reuse the destroyed handles' values;
* a launch captured into a graph and replayed on another stream beside eager
  launches on the capture stream.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# (rows, cols, kind): every shape splits its rows (cols >= 8192 with fewer than
# 256 rows), except the last two, which cover split == 1 between split launches.
_SHAPES = [(1, 1 << 20, 0), (3, 40000, 1), (200, 8192, 2), (1, 8192, 0), (2, 100003, 0),
           (255, 8200, 1), (7, 65536, 2), (1, 1 << 18, 1), (300, 9000, 0), (1, 4096, 0)]


def _check(orc, x, rows, cols, kind, got):
    want = orc.row_reduce(x, rows, cols, kind)
    if kind == 1:
        assert np.array_equal(got, want), f"max rows={rows} cols={cols}"
        return
    rms = float(np.sqrt(np.mean(np.square(x.astype(np.float64)))))
    floor = 5e-5 * (rms / 0.577) * max(1.0, np.sqrt(cols / 4096.0))
    if kind == 2:
        floor /= cols
    r = orc.compare(got, want, 1e-5, floor)
    assert r.ok, f"kind={kind} rows={rows} cols={cols}: {r}"


def _launch(m, dx, dout, rows, cols, kind, ws, wsb, stream=None):
    m.launch_row_reduce_f32(dx, dout, rows, cols, kind, m.ReduceVariant.kTwoPass, ws, wsb,
                            stream).throw_if_error()


def test_back_to_back_on_one_stream(gpu, orc):
    """Ten launches queued without a synchronisation; half share one workspace."""
    m = gpu
    D = m.DeviceBuffer
    shared_wsb = max(m.row_reduce_workspace_bytes(r, c, m.ReduceVariant.kTwoPass)
                     for r, c, _ in _SHAPES)
    shared_ws = D(shared_wsb)
    keep = []
    for i, (rows, cols, kind) in enumerate(_SHAPES):
        x = orc.fill_normal(rows * cols, 0x5EED12345 + i)
        dx, dout = D.from_array(x), D(rows * 4)
        if i % 2:
            ws, wsb = shared_ws, shared_wsb
        else:
            wsb = max(m.row_reduce_workspace_bytes(rows, cols, m.ReduceVariant.kTwoPass), 4)
            ws = D(wsb)
        _launch(m, dx, dout, rows, cols, kind, ws, wsb)
        keep.append((x, rows, cols, kind, dx, dout, ws))
    m.device_synchronize()
    for x, rows, cols, kind, _dx, dout, _ws in keep:
        _check(orc, x, rows, cols, kind, dout.download(rows))


def test_repeated_full_sum_same_bits(gpu, orc):
    """The same full sum 20 times in a row on one stream: identical bits each time
    (the fold's order is fixed) and equal to the CPU sum."""
    m = gpu
    D = m.DeviceBuffer
    n = 1 << 24
    x = orc.fill_random(n, 0xF011, 0.0, 1.0)
    dx = D.from_array(x)
    wsb = m.row_reduce_workspace_bytes(1, n, m.ReduceVariant.kTwoPass)
    ws = D(wsb)
    outs = [D(4) for _ in range(20)]
    for o in outs:
        _launch(m, dx, o, 1, n, 0, ws, wsb)
    m.device_synchronize()
    got = np.array([o.download(1)[0] for o in outs], np.float32)
    assert np.all(got.view(np.uint32) == got.view(np.uint32)[0])
    _check(orc, x, 1, n, 0, got[:1])


def test_concurrent_streams(gpu, orc):
    """Four streams, each with its own workspace, launching interleaved."""
    m = gpu
    D = m.DeviceBuffer
    streams = [m.Stream() for _ in range(4)]
    try:
        work = []
        for i in range(12):
            rows, cols, kind = _SHAPES[i % 8]
            x = orc.fill_normal(rows * cols, 0xC0C0 + i)
            wsb = max(m.row_reduce_workspace_bytes(rows, cols, m.ReduceVariant.kTwoPass), 4)
            dx, dout, ws = D.from_array(x), D(rows * 4), D(wsb)
            work.append((x, rows, cols, kind, dx, dout, ws, wsb, streams[i % 4]))
        for x, rows, cols, kind, dx, dout, ws, wsb, st in work:
            _launch(m, dx, dout, rows, cols, kind, ws, wsb, st)
        for st in streams:
            st.synchronize()
        for x, rows, cols, kind, _dx, dout, _ws, _wsb, _st in work:
            _check(orc, x, rows, cols, kind, dout.download(rows))
    finally:
        for st in streams:
            st.close()


def _hip():
    """libamdhip64 through ctypes, for stream calls that bypass this library."""
    import ctypes as C

    h = C.CDLL("libamdhip64.so")
    h.hipStreamCreate.restype = C.c_int
    h.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
    h.hipStreamDestroy.restype = C.c_int
    h.hipStreamDestroy.argtypes = [C.c_void_p]
    return h


def test_raw_stream_destroy_then_fresh_streams(gpu, orc):
    """64 rounds: create a stream with hipStreamCreate, queue two split launches on
    it, destroy it with hipStreamDestroy before they complete, and queue the next
    round on a fresh stream (whose handle value may be the destroyed one's).  Every
    launch has its own output and workspace; all agree with the CPU and with each
    other bit for bit."""
    import ctypes as C

    m = gpu
    h = _hip()
    D = m.DeviceBuffer
    TP = m.ReduceVariant.kTwoPass
    rows, cols = 3, 1 << 16                   # 16 workgroups per row
    x = orc.fill_normal(rows * cols, 0xDE57)
    dx = D.from_array(x)
    wsb = m.row_reduce_workspace_bytes(rows, cols, TP)
    outs, keep, handles = [], [], set()
    for i in range(64):
        st = C.c_void_p()
        assert h.hipStreamCreate(C.byref(st)) == 0 and st.value
        handles.add(st.value)
        for kind in (0, 1):
            o, ws = D(rows * 4), D(wsb)
            _launch(m, dx, o, rows, cols, kind, ws, wsb, st.value)
            outs.append((kind, o))
            keep.append(ws)
        assert h.hipStreamDestroy(st) == 0
    m.device_synchronize()
    first = {}
    for kind, o in outs:
        got = o.download(rows)
        if kind not in first:
            _check(orc, x, rows, cols, kind, got)
            first[kind] = got
        assert np.array_equal(got.view(np.uint32), first[kind].view(np.uint32)), kind
    print(f"{len(handles)} distinct stream handles over 64 rounds")


def test_per_thread_default_stream_in_two_threads(gpu, orc):
    """hipStreamPerThread is one handle naming a different stream in each host
    thread: two threads launching on it at once, each with its own workspace (the
    launches are ctypes calls, which release the GIL, so they interleave)."""
    import threading

    m = gpu
    D = m.DeviceBuffer
    per_thread = 2                       # hipStreamPerThread
    n = 1 << 20
    inputs = [orc.fill_random(n, 0x7EAD + t, 0.0, 1.0) for t in range(2)]
    wsb = m.row_reduce_workspace_bytes(1, n, m.ReduceVariant.kTwoPass)
    dev = [(D.from_array(x), D(wsb), [D(4) for _ in range(16)]) for x in inputs]
    errors = []

    def worker(t):
        try:
            dx, ws, outs = dev[t]
            for o in outs:
                _launch(m, dx, o, 1, n, 0, ws, wsb, per_thread)
            assert m.lib().mcke_rt_stream_synchronize(per_thread) == 0
        except Exception as e:          # reported after join
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    m.device_synchronize()
    for t, (_dx, _ws, outs) in enumerate(dev):
        got = np.array([o.download(1)[0] for o in outs], np.float32)
        _check(orc, inputs[t], 1, n, 0, got[:1])
        assert np.all(got.view(np.uint32) == got.view(np.uint32)[0]), f"thread {t}"


def test_graph_replayed_beside_its_capture_stream(gpu, orc):
    """A split kTwoPass launch captured into a graph on stream S1 and replayed on
    stream S2 while eager kTwoPass launches of the same shape run on S1: every
    eager launch and the last replay give the CPU result, and a further launch
    on S1 is right too."""
    import ctypes as C

    m = gpu
    L = m.lib()
    VP = C.c_void_p
    for name, args in (("mcke_rt_stream_begin_capture", [VP]),
                       ("mcke_rt_stream_end_capture", [VP, C.POINTER(VP)]),
                       ("mcke_rt_graph_launch", [VP, VP]),
                       ("mcke_rt_graph_destroy", [VP])):
        getattr(L, name).restype = C.c_int
        getattr(L, name).argtypes = args
    D = m.DeviceBuffer
    TP = m.ReduceVariant.kTwoPass
    rows, cols = 2, 1 << 20                   # 128 workgroups per row
    wsb = m.row_reduce_workspace_bytes(rows, cols, TP)
    s1, s2 = m.Stream(), m.Stream()
    exe = VP()
    try:
        xg = orc.fill_normal(rows * cols, 0xCA97)
        dxg, outg, wsg = D.from_array(xg), D(rows * 4), D(wsb)
        assert L.mcke_rt_stream_begin_capture(s1.handle) == 0
        _launch(m, dxg, outg, rows, cols, 0, wsg, wsb, s1)
        assert L.mcke_rt_stream_end_capture(s1.handle, C.byref(exe)) == 0 and exe.value
        eager = []
        for i in range(8):
            x = orc.fill_normal(rows * cols, 0xE6E0 + i)
            eager.append((x, D.from_array(x), D(rows * 4), D(wsb)))
        for _x, dx, dout, ws in eager:
            assert L.mcke_rt_graph_launch(exe, s2.handle) == 0
            _launch(m, dx, dout, rows, cols, 0, ws, wsb, s1)
        s1.synchronize()
        s2.synchronize()
        for x, _dx, dout, _ws in eager:
            _check(orc, x, rows, cols, 0, dout.download(rows))
        _check(orc, xg, rows, cols, 0, outg.download(rows))
        x, dx, dout, ws = eager[0]
        _launch(m, dx, dout, rows, cols, 1, ws, wsb, s1)
        s1.synchronize()
        _check(orc, x, rows, cols, 1, dout.download(rows))
    finally:
        if exe.value:
            L.mcke_rt_graph_destroy(exe)
        s1.close()
        s2.close()
