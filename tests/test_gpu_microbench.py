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
