"""Pins for the deterministic arithmetic in `oracle/numerics.py`.

exp_det is checked against float64 `math.exp` rounded to fp32 (a library
routine), for monotonicity (the nucleus order relies on it), and at its
special points; fixed62 / rn32 / uniform_threshold against exact rational
arithmetic.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

from oracle.numerics import (LN2_HI, exp_det, fixed62, fixed62_sum, rn32, rn32_u64,
                             uniform_threshold)


def _rn32_fraction(fr):
    """Reference fp32 rounding of an exact rational via float64 (exact when the
    rational has < 53 significant bits, as in these tests)."""
    return np.float32(float(fr))


def test_exp_det_matches_rounded_libm():
    rs = np.random.RandomState(0)
    d = np.concatenate([-np.abs(rs.randn(200000).astype(np.float32)) * 20,
                        -rs.uniform(0, 104, 100000).astype(np.float32),
                        np.float32([0.0, -1e-30, -1e-8, -0.5, -1.0, -87.3, -103.9])])
    got = exp_det(d)
    ref = np.array([math.exp(float(x)) for x in d]).astype(np.float32)
    diff = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert diff.max() <= 1
    assert (diff == 0).mean() > 0.9999


def test_exp_det_special_points():
    assert exp_det(np.float32([0.0]))[0] == np.float32(1.0)
    assert exp_det(np.float32([-104.01]))[0] == 0.0
    assert exp_det(np.float32([-np.inf]))[0] == 0.0
    # denormal range is produced, not flushed
    v = exp_det(np.float32([-100.0]))[0]
    assert 0 < v < np.finfo(np.float32).tiny


def test_exp_det_monotone():
    # dense sweep plus every fp32 input within +-64 ulps of each range-reduction
    # boundary (k + 1/2) * ln2, where a Cody-Waite evaluation could step backwards
    rs = np.random.RandomState(1)
    d = np.sort(-rs.uniform(0, 104, 400000).astype(np.float32))
    e = exp_det(d)
    assert np.all(np.diff(e) >= 0)
    pts = []
    for k in range(-151, 1):
        c = np.float32((k + 0.5) * math.log(2))
        base = c.view(np.int32)
        pts.append((base + np.arange(-64, 65, dtype=np.int32)).view(np.float32))
    d = np.sort(np.concatenate(pts))
    d = d[(d <= 0) & (d >= -104)]
    assert np.all(np.diff(exp_det(d)) >= 0)
    assert LN2_HI * 151 == float(Fraction(LN2_HI) * 151)   # k * LN2_HI is exact


def test_fixed62_and_rn32_exact():
    rs = np.random.RandomState(2)
    x = rs.uniform(2.0 ** -39, 1.0, 20000).astype(np.float32)
    f = fixed62(x)
    for xi, fi in zip(x[:500], f[:500]):
        assert Fraction(int(fi), 2 ** 62) == Fraction(float(xi))
    back = rn32_u64(f)
    assert np.array_equal(back, x)
    # sums: rn32 of an exact integer equals fp32 rounding of the rational
    s = fixed62_sum(x[:3])
    assert rn32(s) == _rn32_fraction(sum(Fraction(float(v)) for v in x[:3]))


def test_rn32_ties_to_even():
    one = 2 ** 62
    ulp = 2 ** (62 - 23)                   # fp32 ulp at 1.0 in fixed62 units
    assert rn32(one + ulp // 2) == np.float32(1.0)                    # tie -> even (1.0)
    assert rn32(one + ulp + ulp // 2) == np.float32(1.0 + 2 * 2.0 ** -23)   # tie -> even
    assert rn32(one + ulp // 2 + 1) == np.float32(1.0 + 2.0 ** -23)
    big = (3 << 62) + 12345
    assert rn32(big) == np.float32(3.0)
    a = np.array([one + ulp // 2, one + ulp + ulp // 2, 12345, 0], np.uint64)
    assert np.array_equal(rn32_u64(a), np.array([rn32(int(v)) for v in a], np.float32))


def test_uniform_threshold_exact():
    rs = np.random.RandomState(3)
    for _ in range(2000):
        u = np.float32(rs.uniform(0, 1))
        tot = int(rs.randint(1, 2 ** 62, dtype=np.int64))
        assert uniform_threshold(u, tot) == math.floor(Fraction(float(u)) * tot)
    assert uniform_threshold(np.float32(0.0), 10 ** 18) == 0
    with pytest.raises(ValueError):
        uniform_threshold(np.float32(1.0), 5)


def _all_codes16(fmt):
    c = np.arange(65536, dtype=np.uint32)
    if fmt == "bf16":
        return (c << 16).view(np.float32)
    return c.astype(np.uint16).view(np.float16).astype(np.float32)


@pytest.mark.parametrize("fmt", ["bf16", "f16"])
def test_scaled_logit_by_fp64_reciprocal_equals_fp32_division(fmt):
    """The kernels evaluate x / T as fl32(fl64(x) * fl64(1/T)). For every
    16-bit x and fp32 T this must equal numpy's correctly rounded fp32
    division (the reference's `logits / temperature`): checked here over all
    65,536 codes for a spread of temperatures, including ones whose inverse
    is not exact and huge / tiny ones that overflow or underflow the quotient."""
    x = _all_codes16(fmt)
    rs = np.random.RandomState(7)
    temps = [0.8, 0.7, 0.1, 1.0 / 3.0, 3.0, 1.5, 1e-3, 4e6, 1e-30, 3e38, 0.95, 2.0 ** -20,
             1.0 + 2.0 ** -23, 1.0 - 2.0 ** -24]
    temps += list(rs.uniform(0.05, 4.0, 40)) + list(np.exp(rs.uniform(-60, 60, 20)))
    with np.errstate(all="ignore"):
        for T in temps:
            T32 = np.float32(T)
            want = x / T32
            got = (x.astype(np.float64) * (1.0 / np.float64(T32))).astype(np.float32)
            same = (want == got) | (np.isnan(want) & np.isnan(got))
            assert same.all(), (fmt, T, x[~same][:4], want[~same][:4], got[~same][:4])


def test_fp32_quotient_by_fp64_reciprocal():
    """The kernels evaluate p = e / z (and p / totf) as fl32(fl64(e) * fl64(1/z)):
    equal to the correctly rounded fp32 quotient for fp32 operands (the exact
    quotient of two 24-bit significands is never within 2^-52 of an fp32
    rounding midpoint). Checked on random, denormal and edge operands."""
    rs = np.random.RandomState(11)
    e = np.concatenate([rs.uniform(0, 1, 400000), np.exp(rs.uniform(-104, 0, 400000)),
                        [1.0, 2.0 ** -149, 2.0 ** -126, 0.5, 1.0 - 2.0 ** -24]]).astype(np.float32)
    z = np.concatenate([rs.uniform(1, 3, 400000), np.exp(rs.uniform(0, 12, 400000)),
                        [1.0, 3.0, 1.0 + 2.0 ** -23, 7.0, 151936.0]]).astype(np.float32)
    with np.errstate(all="ignore"):
        want = e / z
        got = (e.astype(np.float64) * (1.0 / z.astype(np.float64))).astype(np.float32)
    assert np.array_equal(want, got)
