"""Deterministic arithmetic shared by the oracle and (restated in HIP) the kernels.

The reference computes `softmax`, the top-p cumulative sum and the final
renormalisation with torch's CPU kernels (`specdec/sampling.py:50,58,66-67`).
Their fp32 results depend on the vector width and summation order of the
machine they run on (the fp32 softmax denominator carries ~1e-6 relative
noise), so "bit-exact" decisions need a rule that every implementation can
reproduce. The rule used throughout:

* exp_det(d):   fp32 result of exp(d) evaluated in float64 (Cody-Waite
                reduction + degree-13 Taylor, plain mul/add, no FMA) and
                rounded once to fp32; 0 for d < -104 (below half the
                smallest fp32 denormal). Differs from a correctly rounded
                expf only when exp(d) lies within ~1e-16 of an fp32 midpoint.
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

# exp_det constants (float64, written in hex so the HIP restatement uses the
# identical bits).
INV_LN2 = float.fromhex("0x1.71547652b82fep+0")
LN2_HI = float.fromhex("0x1.62e42fee00000p-1")   # 32 significant bits: k*LN2_HI exact
LN2_LO = float.fromhex("0x1.a39ef35793c76p-33")
# 1/n! for n = 13 .. 0 (Horner order)
EXP_TAYLOR = [float.fromhex(h) for h in (
    "0x1.6124613a86d09p-33",  # 1/13!
    "0x1.1eed8eff8d898p-29",  # 1/12!
    "0x1.ae64567f544e4p-26",  # 1/11!
    "0x1.27e4fb7789f5cp-22",  # 1/10!
    "0x1.71de3a556c734p-19",  # 1/9!
    "0x1.a01a01a01a01ap-16",  # 1/8!
    "0x1.a01a01a01a01ap-13",  # 1/7!
    "0x1.6c16c16c16c17p-10",  # 1/6!
    "0x1.1111111111111p-7",   # 1/5!
    "0x1.5555555555555p-5",   # 1/4!
    "0x1.5555555555555p-3",   # 1/3!
    "0x1.0000000000000p-1",   # 1/2!
    "0x1.0000000000000p+0",   # 1/1!
    "0x1.0000000000000p+0",   # 1/0!
)]
EXP_CUTOFF = np.float32(-104.0)
TWO62 = float(2 ** 62)


def exp_det(d):
    """fp32 exp(d) under the deterministic rule above. d: fp32 array."""
    d = np.asarray(d, dtype=np.float32)
    with np.errstate(all="ignore"):                 # -inf inputs go through the cutoff
        dd = d.astype(np.float64)
        k = np.rint(dd * INV_LN2)
        r = (dd - k * LN2_HI) - k * LN2_LO
        p = np.full_like(r, EXP_TAYLOR[0])
        for c in EXP_TAYLOR[1:]:
            p = p * r + c
        k_int = np.nan_to_num(np.clip(k, -2000, 2000)).astype(np.int64)
        out = np.ldexp(p, k_int).astype(np.float32)
    out = np.where(d < EXP_CUTOFF, np.float32(0.0), out)
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
