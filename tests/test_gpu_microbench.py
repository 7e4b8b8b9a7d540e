"""GPU tests of the measured-denominator kernels (mcke_launch_mfma_peak_f32,
mcke_launch_stream_triad_f32), the counterparts of the reference's
bench/fma_peak.cu and bench/stream_triad.cu, and of the 16-bit MFMA chains and the
read+write copy ceiling this build adds.

Both are checked for exact results, so a rate measured with them is a rate of
work that was really done: the triad on quarter-multiple inputs (every fma is
exact), the MFMA chains against the closed form of the 32x32x2 product that the
v_mfma_f32_32x32x2_f32 operand layout defines, on small integers (every partial
sum is an integer below 2^24)."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _mfma_peak_expected(seed: np.ndarray, blocks: int, iters: int) -> np.ndarray:
    """out[block*256 + t] for the kernel: per wave w, lane l holds A[l%32][l/32] =
    seed[64w + l] and B[l/32][l%32] = seed[(64w + l + 1) % 256]; accumulator
    register r of lane l is C[8(r/4) + 4(l/32) + r%4][l%32]; four identical
    chains, each C = iters * A @ B."""
    out = np.zeros(256, dtype=np.float64)
    for w in range(4):
        lanes = np.arange(64)
        a = np.zeros((32, 2))
        b = np.zeros((2, 32))
        for l in lanes:
            a[l % 32, l // 32] = seed[64 * w + l]
            b[l // 32, l % 32] = seed[(64 * w + l + 1) % 256]
        c = iters * (a @ b)
        for l in lanes:
            s = 0.0
            for r in range(16):
                s += c[8 * (r // 4) + 4 * (l // 32) + r % 4, l % 32]
            out[64 * w + l] = 4 * s
    return np.tile(out, blocks).astype(np.float32)


def test_mfma_peak_closed_form(mcke, gpu):
    m = mcke
    seed = (np.arange(256) % 7 - 3).astype(np.float32)
    blocks, iters = 8, 1000
    d_seed = m.DeviceBuffer.from_array(seed)
    out = m.DeviceBuffer(blocks * 256 * 4)
    m.launch_mfma_peak_f32(d_seed, out, blocks, iters).throw_if_error()
    m.device_synchronize()
    got = out.download(blocks * 256)
    want = _mfma_peak_expected(seed, blocks, iters)
    assert np.array_equal(got, want)
    assert m.mfma_peak_flops(blocks, iters) == blocks * 4 * iters * 4 * 4096


def test_mfma_peak_rejects_bad_arguments(mcke, gpu):
    m = mcke
    d = m.DeviceBuffer(1024 * 4)
    assert m.launch_mfma_peak_f32(d, d, 0, 10).code == m.StatusCode.kInvalidArgument
    assert m.launch_mfma_peak_f32(d, d, 4, 0).code == m.StatusCode.kInvalidArgument
    assert m.launch_mfma_peak_f32(None, d, 4, 10).code == m.StatusCode.kInvalidArgument
    assert m.mfma_peak_flops(0, 5) == 0


@pytest.mark.parametrize("n", [1, 3, 4, 7, 1000, 4097, 1 << 20])
def test_stream_triad_exact(mcke, gpu, n):
    m = mcke
    rng = np.random.default_rng(n)
    b = (rng.integers(-400, 400, n) * 0.25).astype(np.float32)
    c = (rng.integers(-400, 400, n) * 0.25).astype(np.float32)
    db, dc = m.DeviceBuffer.from_array(b), m.DeviceBuffer.from_array(c)
    da = m.DeviceBuffer(max(4, n) * 4)
    m.launch_stream_triad_f32(db, dc, da, 3.0, n).throw_if_error()
    m.device_synchronize()
    assert np.array_equal(da.download(n), (3.0 * c + b).astype(np.float32))


def test_stream_triad_rejects_alias_and_misalignment(mcke, gpu):
    m = mcke
    d = m.DeviceBuffer(4096)
    e = m.DeviceBuffer(4096)
    assert m.launch_stream_triad_f32(d, e, d, 1.0, 64).code == m.StatusCode.kInvalidArgument
    assert m.launch_stream_triad_f32(d.ptr + 4, e, e.ptr + 2048, 1.0, 64).code == \
        m.StatusCode.kInvalidArgument
    assert m.launch_stream_triad_f32(d, e, e, 1.0, 0).ok()


def _mfma_peak_lp_expected(seed: np.ndarray, blocks: int, iters: int) -> np.ndarray:
    """out[block*256 + t] for the 16-bit chains: thread t (wave w = t/64, lane
    l = t%64) feeds A values seed[(t + e) % 256] and B values seed[(t + 8 + e) % 256],
    e = 0..7.  Whatever k each (lane half h, element e) slot stands for, A and B
    share it, so C[i][j] = sum over h, e of A(lane i + 32h, e) * B(lane j + 32h, e);
    the accumulator layout is the 32x32 one of the fp32 chains."""
    out = np.zeros(256, dtype=np.float64)
    for w in range(4):
        c = np.zeros((32, 32))
        for i in range(32):
            for j in range(32):
                acc = 0.0
                for h in range(2):
                    ta, tb = 64 * w + i + 32 * h, 64 * w + j + 32 * h
                    for e in range(8):
                        acc += seed[(ta + e) % 256] * seed[(tb + 8 + e) % 256]
                c[i, j] = acc
        c *= iters
        for l in range(64):
            s = 0.0
            for r in range(16):
                s += c[8 * (r // 4) + 4 * (l // 32) + r % 4, l % 32]
            out[64 * w + l] = 4 * s
    return np.tile(out, blocks).astype(np.float32)


@pytest.mark.parametrize("dt", [2, 1], ids=["bf16", "f16"])
def test_mfma_peak_lp_closed_form(mcke, gpu, dt):
    m = mcke
    seed = (np.arange(256) % 7 - 3).astype(np.float32)     # exact in bf16 and fp16
    blocks, iters = 4, 500
    d_seed = m.DeviceBuffer.from_array(seed)
    out = m.DeviceBuffer(blocks * 256 * 4)
    m.launch_mfma_peak_lp(dt, d_seed, out, blocks, iters).throw_if_error()
    m.device_synchronize()
    assert np.array_equal(out.download(blocks * 256), _mfma_peak_lp_expected(seed, blocks, iters))
    assert m.mfma_peak_lp_flops(blocks, iters) == blocks * 4 * iters * 4 * 32768
    assert m.launch_mfma_peak_lp(0, d_seed, out, blocks, iters).code == \
        m.StatusCode.kInvalidArgument


# Operand-register pairs (A, B) of each chain's two MFMAs per iteration in the clock
# probe (mfma_clock_lp_kernel): 4 chains of 32x32x16, or 8 chains of 16x16x32.
_CLOCK_PAIRS = {
    0: [[(0, 1), (1, 2)], [(2, 3), (3, 4)], [(4, 5), (5, 6)], [(6, 7), (7, 0)]],
    1: [[(0, 1), (2, 5)], [(2, 3), (4, 7)], [(4, 5), (6, 1)], [(6, 7), (0, 3)],
        [(1, 2), (3, 6)], [(3, 4), (5, 0)], [(5, 6), (7, 2)], [(7, 0), (1, 4)]],
}


def _mfma_clock_lp_expected(vals: np.ndarray, shape: int, blocks: int, iters: int) -> np.ndarray:
    """out[block*256 + t] of the clock probe.  vals[t, k, e]: element e of operand
    register k of thread t.  Whatever k each (lane group, element) slot stands for, A
    and B share it.  32x32x16: C[i][j] = sum over h, e of A(lane i + 32h, e) B(lane
    j + 32h, e), lane l register r holding C[8 (r/4) + 4 (l/32) + r%4][l%32].
    16x16x32: C[i][j] = sum over g, e of A(lane i + 16g, e) B(lane j + 16g, e), lane l
    register r holding C[4 (l/16) + r][l%16]."""
    out = np.zeros(256, dtype=np.float64)
    n, groups = (32, 2) if shape == 0 else (16, 4)
    for w in range(4):
        v = vals[64 * w:64 * w + 64].astype(np.float64)          # [lane, k, e]
        for pairs in _CLOCK_PAIRS[shape]:
            c = np.zeros((n, n))
            for ka, kb in pairs:
                for g in range(groups):
                    a = v[n * g:n * g + n, ka, :]                  # [i, e]
                    b = v[n * g:n * g + n, kb, :]                  # [j, e]
                    c += a @ b.T
            c *= iters
            for l in range(64):
                if shape == 0:
                    out[64 * w + l] += sum(c[8 * (r // 4) + 4 * (l // 32) + r % 4, l % 32]
                                           for r in range(16))
                else:
                    out[64 * w + l] += sum(c[4 * (l // 16) + r, l % 16] for r in range(4))
    return np.tile(out, blocks).astype(np.float32)


@pytest.mark.parametrize("dt", [2, 1], ids=["bf16", "f16"])
@pytest.mark.parametrize("shape", [0, 1], ids=["32x32x16", "16x16x32"])
def test_mfma_clock_lp_closed_form_and_clock(mcke, gpu, dt, shape):
    """The clock probe computes what its operand rotation says (exact: small integers),
    and reports a plausible clock."""
    m = mcke
    vals = ((np.arange(256 * 8 * 8) * 5 + 3) % 7 - 3).astype(np.float32).reshape(256, 8, 8)
    if dt == 2:
        bits = (vals.reshape(-1).view(np.uint32) >> 16).astype(np.uint16)   # exact values
    else:
        bits = vals.reshape(-1).astype(np.float16).view(np.uint16)
    blocks, iters = 2, 50
    d_bits = m.DeviceBuffer.from_array(bits)
    out = m.DeviceBuffer(blocks * 256 * 4)
    ticks = m.DeviceBuffer(blocks * 16)
    m.launch_mfma_clock_lp(dt, shape, d_bits, out, ticks, blocks, iters).throw_if_error()
    m.device_synchronize()
    got = out.download(blocks * 256)
    assert np.array_equal(got, _mfma_clock_lp_expected(vals, shape, blocks, iters))
    tk = ticks.download(blocks * 2, np.uint64).reshape(blocks, 2).astype(np.float64)
    assert (tk > 0).all()
    ghz = tk[:, 0] / (tk[:, 1] * 10.0)
    assert ((ghz > 0.3) & (ghz < 4.0)).all(), ghz
    assert m.mfma_clock_lp_flops(blocks, iters) == blocks * 4 * iters * 8 * 32768


def test_mfma_clock_lp_rejects(mcke, gpu):
    m = mcke
    b, o, t = m.DeviceBuffer(32768), m.DeviceBuffer(4096), m.DeviceBuffer(64)
    IA = m.StatusCode.kInvalidArgument
    assert m.launch_mfma_clock_lp(0, 0, b, o, t, 1, 1).code == IA       # fp32
    assert m.launch_mfma_clock_lp(2, 2, b, o, t, 1, 1).code == IA       # no such shape
    assert m.launch_mfma_clock_lp(2, 0, b.ptr + 8, o, t, 1, 1).code == IA
    assert m.launch_mfma_clock_lp(2, 0, b, o, t, 0, 1).code == IA
    assert m.launch_mfma_clock_lp(2, 0, b, o, t, 1, 0).code == IA
    assert m.launch_mfma_clock_lp(2, 0, None, o, t, 1, 1).code == IA
    assert m.mfma_clock_lp_flops(0, 1) == 0


@pytest.mark.parametrize("n", [1, 3, 4, 7, 1000, 4097, 1 << 20])
def test_stream_copy_exact(mcke, gpu, n):
    m = mcke
    x = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    dx = m.DeviceBuffer.from_array(x)
    dy = m.DeviceBuffer(max(4, n) * 4)
    m.launch_stream_copy_f32(dx, dy, n).throw_if_error()
    m.device_synchronize()
    assert np.array_equal(dy.download(n), x)
    assert m.launch_stream_copy_f32(dx, dx, n).code == m.StatusCode.kInvalidArgument
    assert m.launch_stream_copy_f32(dx.ptr + 4, dy, 8).code == m.StatusCode.kInvalidArgument
