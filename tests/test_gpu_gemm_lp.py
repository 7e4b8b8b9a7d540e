"""GPU parity of the 16-bit-input GEMM (mcke_launch_gemm_lp) through the C-ABI.

The reference reserves the kF16 / kBF16 DType tags (include/mcke/core/dtype.hpp:33-41)
without a kernel, so the oracle is the reference's fp32 GEMM (reference.hpp:199-211,
double accumulation) over the decoded 16-bit inputs (oracle.gemm_lp), with the
16-bit output rounded to nearest even.

Bars (stated per test):
  * quarter-multiple inputs: every product and partial sum is exact in fp32, so the
    result is bit-for-bit the oracle's -- fp32 out, and 16-bit out (both sides round
    the same exact value to nearest even) -- for every tile, dtype and path;
  * seeded U[-1,1) inputs rounded to 16 bits: the reference's K-scaled GEMM
    tolerance tol_gemm(k) / abs_tol_gemm(k) (reference.hpp:344-374), plus one ulp of
    the output format (2^-7 bf16, 2^-10 fp16) when C is 16-bit;
  * the 16-byte and per-element load paths give the same bits (same MFMA order).
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

BF16, F16, F32 = 2, 1, 0
DTS = [BF16, F16]
DT_ID = {BF16: "bf16", F16: "f16"}
OUT_ULP = {BF16: 2.0**-7, F16: 2.0**-10}


def _nan16(dt):
    return 0x7FC0 if dt == BF16 else 0x7E00


def run_lp(m, a16, b16, c, M, N, K, alpha, beta, ab, cd, tile=None, shift=0):
    """One launch on fresh buffers; `shift` elements of padding in front of every
    operand (shift = 1 breaks the 16-byte alignment)."""
    D = m.DeviceBuffer

    def up(arr, itemsize):
        arr = np.ascontiguousarray(arr).ravel()
        pad = np.zeros(shift, dtype=arr.dtype)
        full = np.concatenate([pad, arr]) if arr.size else np.zeros(shift + 1, arr.dtype)
        buf = D.from_array(full)
        return buf, buf.ptr + shift * itemsize

    ba, pa = up(a16, 2)
    bb, pb = up(b16, 2)
    c_item = 4 if cd == F32 else 2
    bc, pc = up(c, c_item)
    st = m.launch_gemm_lp(pa, pb, pc, ab, cd, M, N, K, alpha, beta, tile)
    assert st.ok(), str(st)
    m.device_synchronize()
    out = bc.download(shift + M * N, np.float32 if cd == F32 else np.uint16)
    del ba, bb
    return out[shift:]


def _quarters(rng, shape):
    return (rng.integers(-8, 9, size=shape) / 4.0).astype(np.float32)


# Whole tiles for the direct-to-LDS kernels (tiles with BN >= 128):
#   * K % 64 == 32 takes the 32x32x16 kernel; K = 32, 96, 160, 224 give it 1, 3, 5
#     and 7 K steps of 32 (its 4-stage ring's prologue and tail);
#   * K % 64 == 0 takes the 16x16x32 kernel, whose ring is 3 steps deep and clamps
#     the A pair and B step it fetches past the end; K = 64, 128, 192, 320 give it
#     2, 4, 6 and 10 steps (K = 64: fewer steps than the ring is deep).
QSHAPES = [(1, 1, 1), (5, 7, 3), (129, 65, 257), (1, 64, 128), (64, 1, 128), (33, 63, 1),
           (253, 253, 253), (256, 256, 256), (512, 512, 512),
           (256, 256, 32), (256, 256, 96), (256, 512, 160), (512, 256, 224),
           (256, 256, 64), (256, 512, 128), (512, 256, 192), (256, 256, 320)]


@pytest.mark.parametrize("dt", DTS, ids=DT_ID.get)
@pytest.mark.parametrize("out", ["f32", "same"])
@pytest.mark.parametrize("shape", QSHAPES, ids=lambda s: "x".join(map(str, s)))
def test_quarter_exact_bit_for_bit_every_tile(gpu, orc, dt, out, shape):
    M, N, K = shape
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    a16 = orc.to_16(_quarters(rng, (M, K)), dt)
    b16 = orc.to_16(_quarters(rng, (K, N)), dt)
    cf = _quarters(rng, (M, N))
    cd = F32 if out == "f32" else dt
    c = cf if cd == F32 else orc.to_16(cf, dt)
    for alpha, beta in ((1.0, 0.0), (0.5, 2.0)):
        want = orc.gemm_lp(a16, b16, c, M, N, K, alpha, beta, dt, cd)
        for tile in gpu.LP_TILES:
            got = run_lp(gpu, a16, b16, c, M, N, K, alpha, beta, dt, cd, tile)
            assert np.array_equal(got.view(np.uint32 if cd == F32 else np.uint16).ravel(),
                                  want.view(np.uint32 if cd == F32 else np.uint16).ravel()), \
                (tile, alpha, beta)


RSHAPES = [(129, 65, 257), (253, 253, 253), (300, 520, 1032), (1024, 1024, 1024)]


@pytest.mark.parametrize("dt", DTS, ids=DT_ID.get)
@pytest.mark.parametrize("out", ["f32", "same"])
@pytest.mark.parametrize("shape", RSHAPES, ids=lambda s: "x".join(map(str, s)))
def test_random_within_gemm_tolerance(gpu, orc, dt, out, shape):
    M, N, K = shape
    a16 = orc.to_16(orc.fill_random(M * K, 0x6E33A), dt)
    b16 = orc.to_16(orc.fill_random(K * N, 0x8B10C), dt)
    cd = F32 if out == "f32" else dt
    cf = orc.fill_random(M * N, 0xC0FFEE)
    c = cf if cd == F32 else orc.to_16(cf, dt)
    alpha, beta = 1.0, 0.5
    want = orc.gemm_lp(a16, b16, c, M, N, K, alpha, beta, dt, cd)
    rel = orc.tol_gemm(K) + (0.0 if cd == F32 else OUT_ULP[dt])
    for tile in (gpu.gemm_lp_default_tile(M, N, K),) + tuple(gpu.LP_TILES):
        got = run_lp(gpu, a16, b16, c, M, N, K, alpha, beta, dt, cd, tile)
        g = got if cd == F32 else orc.from_16(got, dt)
        w = want if cd == F32 else orc.from_16(want, dt)
        r = orc.compare(g, w, rel, orc.abs_tol_gemm(K))
        assert r.ok, f"{tile}: {r}"


@pytest.mark.parametrize("dt", DTS, ids=DT_ID.get)
def test_unaligned_and_ragged_take_the_element_path_with_same_bits(gpu, orc, dt):
    # K % 8 != 0 or a misaligned base forces per-element loads; the MFMA sequence
    # is the same, so the bits match the 16-byte path where both apply.
    M, N, K = 200, 136, 264
    a16 = orc.to_16(orc.fill_random(M * K, 11), dt)
    b16 = orc.to_16(orc.fill_random(K * N, 12), dt)
    c = np.zeros(M * N, np.float32)
    for tile in gpu.LP_TILES:
        aligned = run_lp(gpu, a16, b16, c, M, N, K, 1.0, 0.0, dt, F32, tile)
        shifted = run_lp(gpu, a16, b16, c, M, N, K, 1.0, 0.0, dt, F32, tile, shift=1)
        assert np.array_equal(aligned.view(np.uint32), shifted.view(np.uint32)), tile
    # Ragged K and N (not multiples of 8) against the oracle.
    M, N, K = 77, 45, 101
    a16 = orc.to_16(orc.fill_random(M * K, 13), dt)
    b16 = orc.to_16(orc.fill_random(K * N, 14), dt)
    c = np.zeros(M * N, np.float32)
    want = orc.gemm_lp(a16, b16, c, M, N, K, 1.0, 0.0, dt, F32)
    for tile in gpu.LP_TILES:
        got = run_lp(gpu, a16, b16, c, M, N, K, 1.0, 0.0, dt, F32, tile)
        r = orc.compare(got, want, orc.tol_gemm(K), orc.abs_tol_gemm(K))
        assert r.ok, f"{tile}: {r}"


@pytest.mark.parametrize("dt", DTS, ids=DT_ID.get)
@pytest.mark.parametrize("out", ["f32", "same"])
@pytest.mark.parametrize("shape", [(67, 45, 39), (256, 256, 64)], ids=lambda s: "x".join(map(str, s)))
def test_special_values(gpu, orc, dt, out, shape):
    """16-bit infinities and NaN in A and B, every tile, ragged (element path) and
    whole-tile (direct-to-LDS kernel) shapes: NaN and +-inf in C exactly where the
    oracle has them (no summation order changes those), finite entries within
    tol_gemm(k) plus one output ulp for 16-bit C."""
    M, N, K = shape
    cd = F32 if out == "f32" else dt
    rng = np.random.default_rng(M + N + K)
    a = rng.uniform(-1.0, 1.0, (M, K)).astype(np.float32)
    b = rng.uniform(-1.0, 1.0, (K, N)).astype(np.float32)
    a[0, 3] = np.inf
    a[1, 5] = -np.inf
    a[2, 1], a[2, 2] = np.inf, -np.inf
    a[3, K - 1] = np.nan
    a[4, 7] = np.inf
    b[7, : N // 2] = 0.0
    b[K - 2, N - 1] = np.inf
    b[9, N - 2] = np.nan
    a16, b16 = orc.to_16(a, dt), orc.to_16(b, dt)
    c = np.zeros(M * N, np.float32) if cd == F32 else np.zeros(M * N, np.uint16)
    want = orc.gemm_lp(a16, b16, c, M, N, K, 1.0, 0.0, dt, cd)
    w = want if cd == F32 else orc.from_16(want, dt)
    nan_w, inf_w = np.isnan(w), np.isinf(w)
    assert nan_w.any() and inf_w.any()
    fin = ~nan_w & ~inf_w
    rel = orc.tol_gemm(K) + (0.0 if cd == F32 else OUT_ULP[dt])
    for tile in (gpu.gemm_lp_default_tile(M, N, K),) + tuple(gpu.LP_TILES):
        got = run_lp(gpu, a16, b16, c, M, N, K, 1.0, 0.0, dt, cd, tile)
        g = got if cd == F32 else orc.from_16(got, dt)
        assert np.array_equal(np.isnan(g), nan_w), tile
        assert np.array_equal(g[inf_w], w[inf_w]), tile
        r = orc.compare(g[fin], w[fin], rel, orc.abs_tol_gemm(K))
        assert r.ok, f"{tile}: {r}"


@pytest.mark.parametrize("dt", DTS, ids=DT_ID.get)
@pytest.mark.parametrize("out", ["f32", "same"])
def test_beta_zero_does_not_read_c_and_k_zero_scales_c(gpu, orc, dt, out):
    M, N, K = 96, 80, 64
    cd = F32 if out == "f32" else dt
    rng = np.random.default_rng(5)
    a16 = orc.to_16(_quarters(rng, (M, K)), dt)
    b16 = orc.to_16(_quarters(rng, (K, N)), dt)
    nan_c = (np.full(M * N, np.nan, np.float32) if cd == F32
             else np.full(M * N, _nan16(dt), np.uint16))
    zero_c = np.zeros(M * N, np.float32) if cd == F32 else np.zeros(M * N, np.uint16)
    want = orc.gemm_lp(a16, b16, zero_c, M, N, K, 1.0, 0.0, dt, cd)
    got = run_lp(gpu, a16, b16, nan_c, M, N, K, 1.0, 0.0, dt, cd)
    assert np.array_equal(got, want)
    # k == 0: C = beta * C (no early return).
    cf = _quarters(rng, (M, N))
    c = cf if cd == F32 else orc.to_16(cf, dt)
    got = run_lp(gpu, np.zeros(0, np.uint16), np.zeros(0, np.uint16), c, M, N, 0, 1.0, 3.0,
                 dt, cd)
    want = (3.0 * cf).astype(np.float32).ravel()
    if cd != F32:
        want = orc.to_16(want, dt)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dt", DTS, ids=DT_ID.get)
def test_large_spot_check_and_determinism(gpu, orc, dt):
    M = N = K = 4096
    a16 = orc.to_16(orc.fill_random(M * K, 0x6E33A), dt)
    b16 = orc.to_16(orc.fill_random(K * N, 0x8B10C), dt)
    c = np.zeros(M * N, np.float32)
    tile = gpu.gemm_lp_default_tile(M, N, K)
    got = run_lp(gpu, a16, b16, c, M, N, K, 1.0, 0.0, dt, F32, tile)
    r = orc.spot_check_gemm(orc.from_16(a16, dt), orc.from_16(b16, dt), got, M, N, K, 1.0, 1024,
                            0x5A11E, orc.tol_gemm(K), orc.abs_tol_gemm(K))
    assert r.ok, r
    again = run_lp(gpu, a16, b16, c, M, N, K, 1.0, 0.0, dt, F32, tile)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))


def test_rejections_with_real_buffers(gpu):
    m = gpu
    D, IA = m.DType, m.StatusCode.kInvalidArgument
    a, b, c = m.DeviceBuffer(4096), m.DeviceBuffer(4096), m.DeviceBuffer(4096)
    t = m.LP_TILES[0]
    assert m.launch_gemm_lp(a, b, a, D.kBF16, D.kF32, 8, 8, 8, 1, 0, t).code == IA
    assert m.launch_gemm_lp(a, b, c, D.kF32, D.kF32, 8, 8, 8, 1, 0, t).code == IA
    assert m.launch_gemm_lp(a, b, c, D.kF16, D.kBF16, 8, 8, 8, 1, 0, t).code == IA
    assert m.launch_gemm_lp(a, b, c, D.kBF16, D.kF32, 8, 8, 8, 1, 0, m.MFMA_TILES[0]).code == IA
    assert m.launch_gemm_lp(a, b, c, D.kBF16, D.kF32, 0, 8, 8, 1, 0, t).ok()


def test_kernel_attrs(gpu):
    for tile in gpu.LP_TILES:
        for ab, cd in ((2, 0), (2, 2), (1, 0), (1, 1)):
            st, at = gpu.gemm_lp_kernel_attrs(ab, cd, tile)
            assert st.ok(), str(st)
            assert at.local_bytes == 0, (tile, ab, cd)        # no spills on the whole-tile path
            if tile.bn >= 128:
                # Direct-to-LDS kernel (K % 64 == 0): three A buffers of 64 k
                # (bm x 128 bytes) and four B steps of 32 k (32 x bn x 2 bytes).
                assert at.static_smem_bytes == 3 * tile.bm * 128 + 4 * 32 * tile.bn * 2
            else:
                assert at.static_smem_bytes == 2 * (tile.bm + tile.bn) * 128
            assert at.threads_per_block == 256 and at.max_blocks_per_sm_api >= 1


@pytest.mark.parametrize("dt", DTS, ids=DT_ID.get)
def test_vendor_ceiling_row_matches_oracle(gpu, orc, dt):
    # The rocBLAS row the benchmark compares against computes the same product.
    M, N, K = 192, 320, 256
    a16 = orc.to_16(orc.fill_random(M * K, 21), dt)
    b16 = orc.to_16(orc.fill_random(K * N, 22), dt)
    D = gpu.DeviceBuffer
    da, db, dc = D.from_array(a16), D.from_array(b16), D(M * N * 4)
    st = gpu.launch_gemm_lp_vendor(da, db, dc, dt, F32, M, N, K, 1.0, 0.0)
    assert st.ok(), str(st)
    gpu.device_synchronize()
    want = orc.gemm_lp(a16, b16, np.zeros(M * N, np.float32), M, N, K, 1.0, 0.0, dt, F32)
    r = orc.compare(dc.download(M * N), want, orc.tol_gemm(K), orc.abs_tol_gemm(K))
    assert r.ok, str(r)
