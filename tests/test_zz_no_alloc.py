"""mcke_launch_row_reduce_noalloc_f32: kTwoPass without a workspace, allocating
nothing (its partials live in a per-GPU device array the library holds).

Checked through the C-ABI against the entry point it varies, the 9-argument
kTwoPass launch with a caller workspace (same kernels, so the same bits), and
against the double-accumulating CPU reduce (reference tests/reference.hpp:154-172;
max bit-exact).  The calls run in a row on one stream with no synchronisation
between them, each smaller than the one before, so every call reuses the scratch
its predecessor left behind.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# (rows, cols, kind), largest first: 255 rows x 2 chunks = 510 partials (the most
# this build's split needs), then fewer partials each time, then rows that are
# not split, then a full-tensor sum.
_CALLS = [(255, 8200, 0), (3, 1 << 20, 1), (2, 100003, 2), (1, 1 << 16, 0), (300, 9000, 1),
          (1, 8192, 2), (1, 1 << 22, 0)]


def _check_oracle(orc, x, rows, cols, kind, got):
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


def test_noalloc_matches_workspace_launch(gpu, orc):
    m = gpu
    D = m.DeviceBuffer
    TP = m.ReduceVariant.kTwoPass
    st = m.Stream()
    try:
        work = []
        for i, (rows, cols, kind) in enumerate(_CALLS):
            x = orc.fill_normal(rows * cols, 0x0A11C + i)
            wsb = max(m.row_reduce_workspace_bytes(rows, cols, TP), 4)
            work.append((x, rows, cols, kind, D.from_array(x), D(rows * 4), D(rows * 4), D(wsb),
                         wsb))
        for x, rows, cols, kind, dx, d_noalloc, d_ws, ws, wsb in work:
            m.launch_row_reduce_noalloc_f32(dx, d_noalloc, rows, cols, kind, st).throw_if_error()
            m.launch_row_reduce_f32(dx, d_ws, rows, cols, kind, TP, ws, wsb, st).throw_if_error()
        st.synchronize()
        for x, rows, cols, kind, _dx, d_noalloc, d_ws, _ws, _wsb in work:
            got, ref = d_noalloc.download(rows), d_ws.download(rows)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (rows, cols, kind)
            _check_oracle(orc, x, rows, cols, kind, got)
    finally:
        st.close()


def test_noalloc_second_call_smaller_after_sync(gpu, orc):
    """Two calls, each followed by a synchronisation, the second smaller: the
    scratch keeps the first call's partials, and the second call must not see
    them."""
    m = gpu
    D = m.DeviceBuffer
    TP = m.ReduceVariant.kTwoPass
    outs = []
    for rows, cols, kind, seed in ((4, 1 << 20, 0, 0x5C1), (1, 1 << 13, 0, 0x5C2)):
        x = orc.fill_random(rows * cols, seed, 0.0, 1.0)
        dx, got, ref = D.from_array(x), D(rows * 4), D(rows * 4)
        m.launch_row_reduce_noalloc_f32(dx, got, rows, cols, kind).throw_if_error()
        m.device_synchronize()
        wsb = m.row_reduce_workspace_bytes(rows, cols, TP)
        m.launch_row_reduce_f32(dx, ref, rows, cols, kind, TP, D(wsb), wsb, None).throw_if_error()
        m.device_synchronize()
        g, r = got.download(rows), ref.download(rows)
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), (rows, cols)
        _check_oracle(orc, x, rows, cols, kind, g)
        outs.append(g)
    assert outs[1][0] < outs[0][0]


def test_noalloc_rejections(gpu):
    """Host-side validation: nothing is launched for these."""
    m = gpu
    D = m.DeviceBuffer
    x, out = D(64), D(64)
    inval = int(m.StatusCode.kInvalidArgument)
    assert int(m.launch_row_reduce_noalloc_f32(x, out, 65536, 1, 0).code) == inval
    assert int(m.launch_row_reduce_noalloc_f32(x, out, -1, 4, 0).code) == inval
    assert int(m.launch_row_reduce_noalloc_f32(None, out, 1, 4, 0).code) == inval
    assert int(m.launch_row_reduce_noalloc_f32(x, out, 1, 4, 3).code) == inval
    assert m.launch_row_reduce_noalloc_f32(x, out, 0, 4, 0).ok()


def test_noalloc_first_call_under_capture_replays_same_bits(gpu):
    """The entry point's first call in a fresh process made under stream capture
    (so its per-device scratch lookup runs while the stream captures), then the
    graph replayed several times with eager calls on a smaller input in between:
    every replay gives the workspace launch's bits (tests/noalloc_capture_child.py)."""
    import os
    import subprocess
    import sys
    child = os.path.join(os.path.dirname(os.path.abspath(__file__)), "noalloc_capture_child.py")
    p = subprocess.run([sys.executable, "-u", child], capture_output=True, text=True, timeout=110)
    print(p.stdout)
    print(p.stderr[-4000:])
    assert p.returncode == 0, p.stdout + p.stderr[-4000:]
    assert "NOALLOC_CAPTURE_OK" in p.stdout
