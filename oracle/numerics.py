"""Deterministic arithmetic shared by the oracle and (restated in HIP) the kernels.

The reference computes `softmax`, the top-p cumulative sum and the final
renormalisation with torch's CPU kernels (`specdec/sampling.py:50,58,66-67`).
Their fp32 results depend on the vector width and summation order of the
machine they run on (the fp32 softmax denominator carries ~1e-6 relative
noise), so "bit-exact" decisions need a rule that every implementation can
reproduce. The rule used throughout:

* exp_det(d):   fp32 exp(d) by one fixed sequence of IEEE operations:
                k = floor(fl64(d / ln2)) and r = fl32(d - k ln2) in float64
                (r clamped below at 0, so r lies in [0, ln2]); the degree-9
                Taylor polynomial of exp at r in fp32 Horner form (plain
                multiply, then add; coefficients fl32(1/n!)), clamped above at
                2; times 2**k (rounded once when the result is subnormal); 0
                for d < -104 (below half the smallest fp32 denormal). Within 2
                ulps of a correctly rounded expf, and non-decreasing in d: the
                Horner steps are monotone in r because r >= 0 and every
                coefficient is positive, and at each k -> k+1 step the left
                value is at most 2 * 2**k (the clamp) while the right one is at
                least 2**(k+1) (r >= 0 gives p >= 1).
* fixed62(x):   floor(x * 2**62) as an unsigned integer, for fp32 x in [0, 1].
                Exact for x >= 2**-39; every mass, cumulative sum and sampling
                CDF is accumulated in this fixed point, so it is exact and
                independent of summation order.
* rn32(I):      I * 2**-62 rounded once to fp32 (round to nearest, ties to
                even).

The torch reference accumulates `cumsum` in float64 (checked on torch 2.10
CPU: [2**24, 1, 1] -> [..., 16777218]); for probabilities >= 2**-29 that sum is
exact, so `rn32(fixed62 prefix)` equals the reference's `cum` value bit for bit.
"""
import numpy as np

# exp_det constants, written in hex so the HIP restatement uses the identical
# bits: 1/ln2 and ln2 in float64, and fl32(1/n!) for n = 9 .. 0 (Horner order).
INV_LN2 = float.fromhex("0x1.71547652b82fep+0")
LN2 = float.fromhex("0x1.62e42fefa39efp-1")
EXP_TAYLOR32 = [np.float32(float.fromhex(h)) for h in (
    "0x1.71de3ap-19",   # 1/9!
    "0x1.a01a02p-16",   # 1/8!
    "0x1.a01a02p-13",   # 1/7!
    "0x1.6c16c2p-10",   # 1/6!
    "0x1.111112p-7",    # 1/5!
    "0x1.555556p-5",    # 1/4!
    "0x1.555556p-3",    # 1/3!
    "0x1p-1",           # 1/2!
    "0x1p+0",           # 1/1!
    "0x1p+0",           # 1/0!
)]
EXP_CUTOFF = np.float32(-104.0)
TWO62 = float(2 ** 62)


def exp_det_poly(r):
    """The fp32 Horner evaluation of exp at r (fp32 array, r >= 0), clamped at 2."""
    r = np.asarray(r, np.float32)
    p = np.full(r.shape, EXP_TAYLOR32[0], np.float32)
    for c in EXP_TAYLOR32[1:]:
        p = (p * r).astype(np.float32)
        p = (p + c).astype(np.float32)
    return np.minimum(p, np.float32(2.0))


def exp_det(d):
    """fp32 exp(d) under the deterministic rule above. d: fp32 array."""
    d = np.asarray(d, dtype=np.float32)
    with np.errstate(all="ignore"):                 # -inf / NaN inputs go through the cutoff
        dd = d.astype(np.float64)
        kf = np.floor(dd * INV_LN2)
        r = np.maximum((dd - kf * LN2).astype(np.float32), np.float32(0.0))
        p = exp_det_poly(r)
        k = np.nan_to_num(np.clip(kf, -200, 200)).astype(np.int64)
        normal = k >= -126
        sh = np.where(normal, k, k + 64) + 127
        scale = (np.clip(sh, 1, 254).astype(np.uint32) << np.uint32(23)).view(np.float32)
        e = (p * scale).astype(np.float32)
        e = np.where(normal, e, (e * np.float32(2.0 ** -64)).astype(np.float32))
    out = np.where(d >= EXP_CUTOFF, e, np.float32(0.0))
    return out.astype(np.float32)


def fixed62(x):
    """floor(x * 2**62) as uint64 for fp32 x in [0, 1] (array)."""
    x = np.asarray(x, dtype=np.float32)
    if np.any(x < 0) or np.any(x > 1):
        raise ValueError("fixed62 expects values in [0, 1]")
    return np.floor(x.astype(np.float64) * TWO62).astype(np.uint64)


def fixed62_sum(x):
    """Exact sum of fixed62(x) as a Python int (safe beyond 2**64)."""
    f = fixed62(np.ravel(x))
    hi = (f >> np.uint64(31)).sum(dtype=np.uint64)
    lo = (f & np.uint64((1 << 31) - 1)).sum(dtype=np.uint64)
    return (int(hi) << 31) + int(lo)


def rn32(i):
    """Round the non-negative integer i * 2**-62 once to fp32 (nearest, ties even)."""
    i = int(i)
    if i < 0:
        raise ValueError("rn32 expects a non-negative integer")
    if i == 0:
        return np.float32(0.0)
    nb = i.bit_length()
    shift = nb - 24
    if shift <= 0:
        return np.float32(np.ldexp(np.float64(i), -62))
    mant = i >> shift
    rem = i & ((1 << shift) - 1)
    half = 1 << (shift - 1)
    if rem > half or (rem == half and (mant & 1)):
        mant += 1
        if mant == (1 << 24):
            mant >>= 1
            shift += 1
    return np.float32(np.ldexp(np.float64(mant), shift - 62))


def rn32_u64(a):
    """Vectorised rn32 for a uint64 array (values < 2**64)."""
    a = np.asarray(a, dtype=np.uint64)
    hi = (a >> np.uint64(32)).astype(np.float64)
    lo = (a & np.uint64(0xFFFFFFFF)).astype(np.float64)
    # exact bit length via frexp of the 32-bit halves (exact in float64)
    bl_hi = np.frexp(hi)[1]
    bl_lo = np.frexp(lo)[1]
    nb = np.where(hi > 0, 32 + bl_hi, bl_lo).astype(np.int64)
    shift = np.maximum(nb - 24, 0)
    sh = shift.astype(np.uint64)
    mant = a >> sh
    one = np.uint64(1)
    rem = a & ((one << sh) - one)
    half = np.where(shift > 0, one << (np.maximum(sh, one) - one), np.uint64(0))
    up = (shift > 0) & ((rem > half) | ((rem == half) & ((mant & one) == one)))
    mant = mant + up.astype(np.uint64)
    carry = mant == np.uint64(1 << 24)
    mant = np.where(carry, mant >> one, mant)
    shift = shift + carry.astype(np.int64)
    return np.ldexp(mant.astype(np.float64), shift - 62).astype(np.float32)


def uniform_threshold(u, total):
    """floor(u * total) for an fp32 u in [0, 1) and a non-negative integer total.

    Exact: u is split into its 24-bit integer significand and power of two.
    This is the inverse-CDF target used by every sampler in this build.
    """
    u = np.float32(u)
    if not (0.0 <= float(u) < 1.0):
        raise ValueError("uniform must lie in [0, 1)")
    if u == 0:
        return 0
    m, e = np.frexp(np.float64(u))          # u = m * 2**e, m in [0.5, 1)
    mant = int(np.ldexp(m, 24))             # 24-bit integer significand
    sh = 24 - int(e)                        # u = mant * 2**-sh
    return (mant * int(total)) >> sh
