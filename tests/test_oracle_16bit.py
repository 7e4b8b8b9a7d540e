"""Pins the oracle's 16-bit storage conversions and its 16-bit-input GEMM.

The reference has no conversion code (it only reserves the kF16 / kBF16 DType
tags, include/mcke/core/dtype.hpp:33-41), so these functions are pinned by
library routines that implement the same IEEE rounding, and by closed forms:

* bfloat16: bit-equality with torch's CPU float32 <-> bfloat16 conversions
  (round to nearest even) on every 16-bit pattern and on ~10^6 floats chosen to
  hit ties, overflow, subnormals, signed zeros and NaN;
* binary16: bit-equality with numpy's float32 <-> float16 conversions on the
  same sets;
* hand values whose encodings are fixed by the formats;
* the 16-bit GEMM reference against an exact integer brute force (quarter-valued
  inputs, where every product and sum is exact), on a non-square shape so that a
  transposed operand or a wrong decode fails.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

BF16, F16, F32 = 2, 1, 0


def _float_probe_set() -> np.ndarray:
    rng = np.random.default_rng(0x16B17)
    bits = [rng.integers(0, 2**32, size=1_000_000, dtype=np.uint64).astype(np.uint32)]
    hi = rng.integers(0, 2**16, size=20000, dtype=np.uint64).astype(np.uint32) << 16
    bits.append(hi | 0x8000)                       # exact bf16 ties, odd and even kept parts
    bits.append(hi | 0x7FFF)
    bits.append(hi | 0x8001)
    # binary16 ties and neighbours: 13 dropped fraction bits == 0x1000 (normal range),
    # and exact halves of the subnormal unit.
    e = rng.integers(127 - 14, 127 + 16, size=20000, dtype=np.uint64).astype(np.uint32)
    f = rng.integers(0, 2**10, size=20000, dtype=np.uint64).astype(np.uint32) << 13
    for low in (0x1000, 0x0FFF, 0x1001):
        bits.append((e << 23) | f | low)
    sub = np.arange(1, 2**10, dtype=np.float64)
    vals = [np.concatenate([(sub + 0.5) * 2.0**-24, sub * 2.0**-24, (sub + 0.25) * 2.0**-24,
                            [2.0**-25, 2.0**-25 * 1.0000001, 2.0**-26, 65504.0, 65519.0,
                             65520.0, 65536.0, 3.4028234663852886e38, 1.0 + 2.0**-8,
                             1.0 + 3 * 2.0**-8, 0.0, -0.0, np.inf, -np.inf, np.nan]])
            .astype(np.float32)]
    out = np.concatenate([b.view(np.float32) for b in bits] + vals)
    return np.concatenate([out, -out])


FLOATS = _float_probe_set()
ALL16 = np.arange(2**16, dtype=np.uint32).astype(np.uint16)


def _same_bits_or_both_nan(got16: np.ndarray, want16: np.ndarray, dtype: int):
    if dtype == BF16:
        nan = lambda h: ((h & 0x7F80) == 0x7F80) & ((h & 0x7F) != 0)
    else:
        nan = lambda h: ((h & 0x7C00) == 0x7C00) & ((h & 0x3FF) != 0)
    gn, wn = nan(got16), nan(want16)
    np.testing.assert_array_equal(gn, wn)
    bad = np.nonzero((got16 != want16) & ~wn)[0]
    assert bad.size == 0, (f"{bad.size} mismatches, first: x={FLOATS[bad[0]]!r} "
                           f"got {got16[bad[0]]:#06x} want {want16[bad[0]]:#06x}")


def test_bf16_encode_matches_torch(orc):
    got = orc.to_16(FLOATS, BF16)
    want = torch.from_numpy(FLOATS).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    _same_bits_or_both_nan(got, want, BF16)


def test_bf16_decode_matches_torch_on_every_pattern(orc):
    got = orc.from_16(ALL16, BF16)
    want = torch.from_numpy(ALL16.view(np.int16)).view(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_f16_encode_matches_numpy(orc):
    got = orc.to_16(FLOATS, F16)
    with np.errstate(over="ignore", invalid="ignore"):
        want = FLOATS.astype(np.float16).view(np.uint16)
    _same_bits_or_both_nan(got, want, F16)


def test_f16_decode_matches_numpy_on_every_pattern(orc):
    got = orc.from_16(ALL16, F16)
    want = ALL16.view(np.float16).astype(np.float32)
    finite = np.isfinite(want) | np.isinf(want)
    np.testing.assert_array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))


@pytest.mark.parametrize("x,bf16,f16", [
    (1.0, 0x3F80, 0x3C00),
    (-2.0, 0xC000, 0xC000),
    (1.0 + 2.0**-8, 0x3F80, 0x3C04),        # bf16 tie, even neighbour kept
    (1.0 + 3 * 2.0**-8, 0x3F82, 0x3C0C),    # bf16 tie, odd kept part rounds up
    (65504.0, 0x4780, 0x7BFF),              # binary16 max (bf16 rounds up to 2^16)
    (65520.0, 0x4780, 0x7C00),              # binary16 tie at max -> inf
    (2.0**-24, 0x3380, 0x0001),             # smallest binary16 subnormal
    (2.0**-25, 0x3300, 0x0000),             # tie between 0 and 2^-24 -> 0
    (3 * 2.0**-25, 0x33C0, 0x0002),         # tie between 1 and 2 units -> 2
    (-0.0, 0x8000, 0x8000),
    (float("inf"), 0x7F80, 0x7C00),
])
def test_hand_encodings(orc, x, bf16, f16):
    v = np.array([x], dtype=np.float32)
    assert int(orc.to_16(v, BF16)[0]) == bf16
    assert int(orc.to_16(v, F16)[0]) == f16
    # Where the value is representable the decode gives it back exactly.
    for dt, code in ((BF16, bf16), (F16, f16)):
        back = orc.from_16(np.array([code], np.uint16), dt)[0]
        if int(orc.to_16(np.array([back], np.float32), dt)[0]) == code and back == v[0]:
            assert np.signbit(back) == np.signbit(v[0])
    assert orc.from_16(np.array([0x3C00], np.uint16), F16)[0] == 1.0
    assert orc.from_16(np.array([0x0001], np.uint16), F16)[0] == np.float32(2.0**-24)
    assert orc.from_16(np.array([0x3F80], np.uint16), BF16)[0] == 1.0


def test_nan_stays_quiet_nan(orc):
    v = np.array([np.nan, -np.nan], dtype=np.float32)
    for dt in (BF16, F16):
        back = orc.from_16(orc.to_16(v, dt), dt)
        assert np.isnan(back).all()


@pytest.mark.parametrize("dt", [BF16, F16])
@pytest.mark.parametrize("cdt", ["f32", "same"])
def test_gemm_lp_exact_against_integer_brute_force(orc, dt, cdt):
    m, n, k = 19, 23, 37
    rng = np.random.default_rng(dt * 10 + (cdt == "f32"))
    ai = rng.integers(-8, 9, size=(m, k))
    bi = rng.integers(-8, 9, size=(k, n))
    ci = rng.integers(-8, 9, size=(m, n))
    a16 = orc.to_16((ai / 4.0).astype(np.float32), dt)
    b16 = orc.to_16((bi / 4.0).astype(np.float32), dt)
    # Exact: products are multiples of 1/16 below 4, sums below 2^8.
    want = (ai @ bi) / 16.0 * 0.5 + 2.0 * (ci / 4.0)
    c_dt = F32 if cdt == "f32" else dt
    c_in = (ci / 4.0).astype(np.float32)
    c_arg = c_in if c_dt == F32 else orc.to_16(c_in, dt)
    got = orc.gemm_lp(a16, b16, c_arg, m, n, k, 0.5, 2.0, dt, c_dt)
    if c_dt == F32:
        np.testing.assert_array_equal(got.reshape(m, n), want.astype(np.float32))
    else:
        np.testing.assert_array_equal(got.reshape(m, n), orc.to_16(want.astype(np.float32), dt))
