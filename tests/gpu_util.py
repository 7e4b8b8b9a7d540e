"""Helpers shared by the GPU parity tests: run one launcher on host arrays."""
from __future__ import annotations

import numpy as np


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).ravel()


def run_bias_act(m, x, bias, rows, cols, act, vw=None, max_row_blocks=0):
    D = m.DeviceBuffer
    dx, db = D.from_array(f32(x)), D.from_array(f32(bias))
    dy = D(rows * cols * 4)
    if vw is None:
        vw = min(m.max_vector_width_f32(dx, cols), m.max_vector_width_f32(dy, cols))
    st = m.launch_bias_act_f32(dx, db, dy, rows, cols, act, vw, None, max_row_blocks)
    assert st.ok(), str(st)
    m.device_synchronize()
    return dy.download(rows * cols)


def run_activation(m, x, n, act, vw=1):
    D = m.DeviceBuffer
    dx = D.from_array(f32(x))
    dy = D(n * 4)
    st = m.launch_activation_f32(dx, dy, n, act, vw)
    assert st.ok(), str(st)
    m.device_synchronize()
    return dy.download(n)


def run_reduce(m, x, rows, cols, kind, variant):
    D = m.DeviceBuffer
    dx = D.from_array(f32(x))
    dout = D(max(rows, 1) * 4)
    if int(variant) == int(m.ReduceVariant.kTwoPass):
        wsb = m.row_reduce_workspace_bytes(rows, cols, variant)
        ws = D(max(wsb, 4))
        st = m.launch_row_reduce_f32(dx, dout, rows, cols, kind, variant, ws, wsb, None)
    else:
        st = m.launch_row_reduce_f32(dx, dout, rows, cols, kind, variant, None)
    assert st.ok(), str(st)
    m.device_synchronize()
    return dout.download(rows)


def run_softmax(m, x, rows, cols, variant):
    D = m.DeviceBuffer
    dx = D.from_array(f32(x))
    dy = D(rows * cols * 4)
    st = m.launch_row_softmax_f32(dx, dy, rows, cols, variant)
    assert st.ok(), str(st)
    m.device_synchronize()
    return dy.download(rows * cols)


def run_gemm(m, a, b, c, M, N, K, alpha, beta, variant, tile=None):
    D = m.DeviceBuffer
    da = D.from_array(f32(a)) if M * K else D(4)
    db = D.from_array(f32(b)) if K * N else D(4)
    dc = D.from_array(f32(c))
    st = m.launch_gemm_f32(da, db, dc, M, N, K, alpha, beta, variant, tile)
    assert st.ok(), str(st)
    m.device_synchronize()
    return dc.download(M * N)


# (variant, tile) pairs that every GEMM parity test runs.
def gemm_configs(m):
    V, T = m.GemmVariant, m.GemmTile
    cfgs = [
        (V.kNaive, T()),
        (V.kNaiveUncoalesced, T()),
        (V.kTiledSmem, T(32, 32, 32, 1, 1)),
        (V.kTiledRegBlock, T(128, 128, 8, 8, 8)),
        (V.kWarpTileNoDbuf, T(128, 128, 8, 8, 8)),
        (V.kWarpTile, T(128, 128, 8, 8, 8)),
        (V.kWarpTileVec4, T(128, 128, 8, 8, 8)),
    ]
    cfgs += [(V.kMfmaF32, t) for t in m.MFMA_TILES]
    return cfgs


def cfg_id(cfg) -> str:
    v, t = cfg
    return f"{v.name}-{t.bm}x{t.bn}x{t.bk}"
