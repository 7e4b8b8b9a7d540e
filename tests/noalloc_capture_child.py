"""Child process of tests/test_zz_no_alloc.py (not a test module): captures
mcke_launch_row_reduce_noalloc_f32 into a HIP graph as the entry point's first
call in this process -- so its per-device scratch lookup runs under capture --
then replays the graph several times on the capture stream and checks every
replay's bits against the kTwoPass launch with a caller workspace (same
kernels).  Between replays an eager noalloc call on a smaller input runs on the
same stream and leaves different partials in the shared scratch.

Prints one line per step, flushed, and NOALLOC_CAPTURE_OK at the end; exits 0 on
success, 1 on a mismatch or error."""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from __graft_entry__ import load_package  # noqa: E402

VP = C.c_void_p


def say(msg: str) -> None:
    print(f"[noalloc-capture] {msg}", flush=True)


def last_error(L) -> str:
    return (L.mcke_last_error() or b"").decode()


def main() -> int:
    import oracle

    m = load_package()
    m.require_gpu()
    L = m.lib()
    for name, args in (("mcke_rt_stream_begin_capture", [VP]),
                       ("mcke_rt_stream_end_capture", [VP, C.POINTER(VP)]),
                       ("mcke_rt_graph_launch", [VP, VP]),
                       ("mcke_rt_graph_destroy", [VP]),
                       ("mcke_fill_u32_async", [VP, C.c_uint32, C.c_size_t, VP])):
        getattr(L, name).argtypes = args
        getattr(L, name).restype = C.c_int
    D = m.DeviceBuffer
    TP = m.ReduceVariant.kTwoPass
    st = m.Stream()
    # 255 rows of 8200 split in 2 chunks: 510 partials, the most the scratch takes.
    rows, cols, kind = 255, 8200, 0
    x = oracle.fill_normal(rows * cols, 0x0CA97)
    dx, d_cap, d_ws = D.from_array(x), D(rows * 4), D(rows * 4)
    wsb = max(m.row_reduce_workspace_bytes(rows, cols, TP), 4)
    ws = D(wsb)
    # The smaller eager call that runs between replays.
    rows2, cols2 = 3, 1 << 18
    x2 = oracle.fill_normal(rows2 * cols2, 0x0CA98)
    dx2, d2_na, d2_ws = D.from_array(x2), D(rows2 * 4), D(rows2 * 4)
    ws2b = max(m.row_reduce_workspace_bytes(rows2, cols2, TP), 4)
    ws2 = D(ws2b)
    m.launch_row_reduce_f32(dx, d_ws, rows, cols, kind, TP, ws, wsb, st).throw_if_error()
    m.launch_row_reduce_f32(dx2, d2_ws, rows2, cols2, 1, TP, ws2, ws2b, st).throw_if_error()
    st.synchronize()
    want, want2 = d_ws.download(rows).view(np.uint32), d2_ws.download(rows2).view(np.uint32)

    say(f"capturing the first noalloc call of this process: rows={rows} cols={cols} kind={kind}")
    assert L.mcke_rt_stream_begin_capture(st.handle) == 0, last_error(L)
    rc = m.launch_row_reduce_noalloc_f32(dx, d_cap, rows, cols, kind, st)
    exe = VP()
    rc_end = L.mcke_rt_stream_end_capture(st.handle, C.byref(exe))
    if not rc.ok() or rc_end != 0 or not exe.value:
        say(f"capture failed: launch {rc}, end_capture rc {rc_end}: {last_error(L)}")
        return 1
    try:
        for r in range(4):
            # Poison the output (eager, same stream), replay, then disturb the scratch.
            assert L.mcke_fill_u32_async(d_cap.ptr, 0x7FC00000, rows, st.handle) == 0
            assert L.mcke_rt_graph_launch(exe, st.handle) == 0, last_error(L)
            st.synchronize()
            got = d_cap.download(rows).view(np.uint32)
            if not np.array_equal(got, want):
                say(f"replay {r}: bits differ from the workspace launch")
                return 1
            m.launch_row_reduce_noalloc_f32(dx2, d2_na, rows2, cols2, 1, st).throw_if_error()
            st.synchronize()
            if not np.array_equal(d2_na.download(rows2).view(np.uint32), want2):
                say(f"eager call after replay {r}: bits differ from the workspace launch")
                return 1
            say(f"replay {r}: same bits as the workspace launch")
    finally:
        L.mcke_rt_graph_destroy(exe)
        st.close()
    say("NOALLOC_CAPTURE_OK")
    return 0


if __name__ == "__main__":
    sys.exit(main())
