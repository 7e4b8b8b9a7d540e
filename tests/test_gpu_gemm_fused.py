"""The fused GEMM + bias + activation entry point (mcke_launch_gemm_bias_act_f32)
on the GPU, through the C-ABI.

Its contract is the pair it replaces: launch_gemm_f32 (kMfmaF32, beta = 0) into C,
then launch_bias_act_f32 on C (the reference's GemmOp -> BiasActOp chain,
src/graph/ops_gemm.cpp:74-96 and ops_bias_act.cpp:102-130).  So every case here is
checked bit for bit against that pair on the same tile -- every MFMA tile, whole
tiles (the direct-to-LDS kernel) and ragged or unaligned shapes (the staged
kernel), all four activations, several alphas, k = 0 and special values -- and
against the CPU oracle (oracle.gemm, then oracle.bias_act on its fp32 result)
within the GEMM tolerance tol_gemm(k) / abs_tol_gemm(k) plus the bias+act
tolerance (abs 1e-6 + rel 1e-6), the bars the two launches meet separately."""
from __future__ import annotations

import numpy as np
import pytest

from tests import golden_io
from tests.gpu_util import f32

pytestmark = pytest.mark.gpu

ACTS = [0, 1, 2, 3]


def _nan_aware_bits_equal(got, want):
    g, w = np.asarray(got, np.float32), np.asarray(want, np.float32)
    both_nan = np.isnan(g) & np.isnan(w)
    return bool(np.all(both_nan | (golden_io.bits(g) == golden_io.bits(w))))


def _run(m, a, b, bias, M, N, K, alpha, act, tile, offset=0):
    """Fused and unfused outputs on the same device inputs.  `offset` floats
    shift every operand off 16-byte alignment (the staged scalar kernel)."""
    D = m.DeviceBuffer

    def up(arr, n):
        buf = D((n + offset + 4) * 4)
        host = np.zeros(n + offset, np.float32)
        host[offset:] = f32(arr) if n else host[offset:]
        buf.upload(host)
        return buf

    da, db, dbias = up(a, M * K), up(b, K * N), up(bias, N)
    dy, dc, dy2 = D((M * N + offset + 4) * 4), D((M * N + offset + 4) * 4), D((M * N + 4) * 4)
    p = lambda buf: buf.ptr + 4 * offset   # noqa: E731
    st = m.launch_gemm_bias_act_f32(p(da), p(db), p(dbias), p(dy), M, N, K, alpha, act, tile)
    assert st.ok(), str(st)
    st = m.launch_gemm_f32(p(da), p(db), p(dc), M, N, K, alpha, 0.0, m.GemmVariant.kMfmaF32, tile)
    assert st.ok(), str(st)
    # bias_act needs aligned operands at vw > 1; vw = 1 takes any (every width gives the same bits).
    st = m.launch_bias_act_f32(p(dc), p(dbias), dy2.ptr, M, N, act, 1)
    assert st.ok(), str(st)
    m.device_synchronize()
    fused = dy.download(M * N + offset)[offset:]
    pair = dy2.download(M * N)
    return fused, pair


def _oracle(orc, a, b, bias, M, N, K, alpha, act):
    c = orc.gemm(a, b, np.zeros(M * N, np.float32), M, N, K, alpha, 0.0)
    return orc.bias_act(c, bias, M, N, act)


def _check_oracle(orc, got, want, K):
    r = orc.compare(got, want, orc.tol_gemm(K) + 1e-6, orc.abs_tol_gemm(K) + 1e-6)
    assert r.ok, r


def _inputs(orc, M, N, K, seed):
    a = orc.fill_random(M * K, 0x6E33A + seed)
    b = orc.fill_random(K * N, 0x8B10C + seed)
    bias = orc.fill_random(N, 0xB1A5B1A5 + seed, -0.5, 0.5)
    return a, b, bias


def _whole_shape(t):
    return (2 * t.bm, 3 * t.bn, 4 * t.bk) if t.bm <= 64 else (t.bm, 2 * t.bn, 8 * t.bk)


@pytest.mark.parametrize("ti", range(6), ids=lambda i: f"tile{i}")
@pytest.mark.parametrize("act", ACTS)
def test_whole_tiles_match_the_pair_and_the_oracle(gpu, orc, ti, act):
    t = gpu.MFMA_TILES[ti]
    M, N, K = _whole_shape(t)
    a, b, bias = _inputs(orc, M, N, K, ti)
    for alpha in (1.0, -0.75):
        fused, pair = _run(gpu, a, b, bias, M, N, K, alpha, act, t)
        assert _nan_aware_bits_equal(fused, pair), (t.astuple(), act, alpha)
        _check_oracle(orc, fused, _oracle(orc, a, b, bias, M, N, K, alpha, act), K)


@pytest.mark.parametrize("ti", range(6), ids=lambda i: f"tile{i}")
@pytest.mark.parametrize("shape", [(129, 65, 257), (33, 63, 1), (1, 64, 128), (253, 253, 253)],
                         ids=lambda s: "x".join(map(str, s)))
def test_ragged_shapes_match_the_pair(gpu, orc, ti, shape):
    t = gpu.MFMA_TILES[ti]
    M, N, K = shape
    a, b, bias = _inputs(orc, M, N, K, 7)
    for act in ACTS:
        fused, pair = _run(gpu, a, b, bias, M, N, K, 1.25, act, t)
        assert _nan_aware_bits_equal(fused, pair), (t.astuple(), shape, act)
    _check_oracle(orc, fused, _oracle(orc, a, b, bias, M, N, K, 1.25, 3), K)


@pytest.mark.parametrize("ti", [0, 2, 4, 5], ids=lambda i: f"tile{i}")
def test_unaligned_operands_take_the_scalar_kernel(gpu, orc, ti):
    t = gpu.MFMA_TILES[ti]
    M, N, K = 96, 80, 72
    a, b, bias = _inputs(orc, M, N, K, 11)
    for act in (1, 3):
        fused, pair = _run(gpu, a, b, bias, M, N, K, 1.0, act, t, offset=1)
        assert _nan_aware_bits_equal(fused, pair), (t.astuple(), act)
        _check_oracle(orc, fused, _oracle(orc, a, b, bias, M, N, K, 1.0, act), K)


@pytest.mark.parametrize("ti", [0, 4, 5], ids=lambda i: f"tile{i}")
def test_k0_gives_the_activation_of_the_bias(gpu, orc, ti):
    t = gpu.MFMA_TILES[ti]
    M, N = t.bm, t.bn
    bias = orc.fill_random(N, 0xB1A5, -2.0, 2.0)
    for act in ACTS:
        for alpha in (1.0, -2.0):
            fused, pair = _run(gpu, np.zeros(0), np.zeros(0), bias, M, N, 0, alpha, act, t)
            assert _nan_aware_bits_equal(fused, pair), (act, alpha)
            want = orc.bias_act(np.zeros(M * N, np.float32), bias, M, N, act)
            r = orc.compare(fused, want, 1e-6, 1e-6)
            assert r.ok, r


def test_special_values_match_the_pair(gpu, orc):
    """inf and NaN in A and in the bias, and products that overflow: the fused
    epilogue gives NaN and +-inf exactly where the pair does."""
    for t in (gpu.MFMA_TILES[0], gpu.MFMA_TILES[4], gpu.MFMA_TILES[5]):
        M, N, K = 2 * t.bm, t.bn, 64
        a, b, bias = _inputs(orc, M, N, K, 3)
        a = a.copy()
        bias = bias.copy()
        a[5] = np.inf
        a[K + 3] = -np.inf
        a[3 * K + 1] = np.nan
        a[7 * K:8 * K] = 3e38
        bias[2] = np.inf
        bias[9] = -np.inf
        bias[N - 1] = np.nan
        for act in ACTS:
            fused, pair = _run(gpu, a, b, bias, M, N, K, 1.0, act, t)
            assert _nan_aware_bits_equal(fused, pair), (t.astuple(), act)
            if act == 0:   # the plain bias add keeps both (ReLU maps NaN to 0)
                assert np.isnan(fused).any() and np.isinf(fused).any()


def test_bench_shape_mlp_stage(gpu, orc):
    """The MLP block's first stage at a quarter of its size, 1024 x 4096 x 1024
    with GELU(tanh), on the default tile: the same bits as the pair, and every
    97th row against the oracle."""
    M, N, K = 1024, 4096, 1024
    a = orc.fill_normal(M * K, 0x6E33A, 0.0, 1.0)
    b = orc.fill_normal(K * N, 0x8B10C, 0.0, 0.02)
    bias = orc.fill_normal(N, 0xB1A5, 0.0, 0.01)
    t = gpu.gemm_mfma_default_tile(M, N, K)
    fused, pair = _run(gpu, a, b, bias, M, N, K, 1.0, 3, t)
    assert _nan_aware_bits_equal(fused, pair)
    rows = np.arange(0, M, 97)
    a_rows = np.asarray(a, np.float32).reshape(M, K)[rows].ravel()
    want = _oracle(orc, a_rows, b, bias, len(rows), N, K, 1.0, 3)
    _check_oracle(orc, fused.reshape(M, N)[rows].ravel(), want, K)
