"""Pins for the deterministic arithmetic in `oracle/numerics.py`.

exp_det is checked against float64 `math.exp` rounded to fp32 (a library
routine), at its special points, and for monotonicity (the nucleus order
relies on it): the premises of the argument in `oracle/numerics.py` (Horner
value 1 at r = 0, at most 2 up to the largest reduced argument, r >= 0), a
dense sweep around every range-reduction step, and, with SDX_EXHAUSTIVE=1, all
1,120,927,745 fp32 inputs in [-104, 0]. fixed62 / rn32 / uniform_threshold are
checked against exact rational arithmetic.
"""
import math
import os
from fractions import Fraction

import numpy as np
import pytest

from oracle.numerics import (INV_LN2, LN2, exp_det, exp_det_poly, fixed62, fixed62_sum, rn32,
                             rn32_u64, uniform_threshold)


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
    assert diff.max() <= 2
    assert (diff == 0).mean() > 0.8


def test_exp_det_special_points():
    assert exp_det(np.float32([0.0]))[0] == np.float32(1.0)
    assert exp_det(np.float32([-104.01]))[0] == 0.0
    assert exp_det(np.float32([-np.inf]))[0] == 0.0
    assert exp_det(np.float32([np.nan]))[0] == 0.0
    # exact powers of two where the reduced argument is 0
    assert exp_det(np.float32([-np.log(2.0) * 0.0]))[0] == 1.0
    # denormal range is produced, not flushed, and rounded once
    v = exp_det(np.float32([-100.0]))[0]
    assert 0 < v < np.finfo(np.float32).tiny
    assert abs(float(v) - math.exp(-100.0)) <= 2.0 ** -150


def test_exp_det_monotone_premises():
    """The three facts the monotonicity argument needs, checked directly."""
    # Horner value exactly 1 at r = 0, so p >= 1 at the start of every interval
    assert exp_det_poly(np.float32([0.0]))[0] == np.float32(1.0)
    # the Horner value never exceeds 2: p is non-decreasing in r >= 0, so the
    # 2^20 fp32 values up to a few ulps past fl32(ln2) (the largest reduced
    # argument) cover the top; a sorted sample checks the order below them
    top = int(np.float32(math.log(2.0)).view(np.int32)) + 8
    r = np.arange(top - (1 << 20), top + 1, dtype=np.int32).view(np.float32)
    p = exp_det_poly(r)
    assert np.all(np.diff(p) >= 0) and p.max() <= 2.0
    rs = np.random.RandomState(4)
    r = np.sort(rs.uniform(0, math.log(2.0), 500000).astype(np.float32))
    assert np.all(np.diff(exp_det_poly(r)) >= 0)
    # the reduction never leaves r below 0 before the clamp by more than rounding
    rs = np.random.RandomState(3)
    d = -rs.uniform(0, 104, 200000)
    kf = np.floor(d * INV_LN2)
    assert np.all(d - kf * LN2 > -1e-12) and np.all(d - kf * LN2 < math.log(2.0) + 1e-12)


def test_exp_det_monotone():
    # dense sweep plus every fp32 input within +-4096 ulps of each range-reduction
    # step k * ln2, where the interval index changes
    rs = np.random.RandomState(1)
    d = np.sort(-rs.uniform(0, 104, 400000).astype(np.float32))
    assert np.all(np.diff(exp_det(d)) >= 0)
    pts = []
    for k in range(-151, 1):
        c = np.float32(k * math.log(2))
        base = c.view(np.int32)
        pts.append((base + np.arange(-4096, 4097, dtype=np.int32)).view(np.float32))
    d = np.unique(np.concatenate(pts))
    d = d[(d <= 0) & (d >= -104)]
    assert np.all(np.diff(exp_det(d)) >= 0)


@pytest.mark.skipif(os.environ.get("SDX_EXHAUSTIVE") != "1",
                    reason="all 1.12e9 fp32 inputs in [-104, 0]: about 5 minutes; SDX_EXHAUSTIVE=1")
def test_exp_det_monotone_exhaustive():
    """Every fp32 d in [-104, 0], in value order: exp_det never increases as d
    decreases (negative floats: a larger bit pattern is a smaller value)."""
    end = int(np.float32(-104.0).view(np.uint32))
    b, prev, bad = 0x80000000, None, 0
    while b <= end:
        e1 = min(b + (1 << 24), end + 1)
        v = exp_det(np.arange(b, e1, dtype=np.uint64).astype(np.uint32).view(np.float32))
        bad += int((np.diff(v) > 0).sum()) + int(prev is not None and v[0] > prev)
        prev, b = v[-1], e1
    assert bad == 0


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
