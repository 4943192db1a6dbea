// Shared device code for the gfx950 verify path: 16-bit logit keys, the
// deterministic exp / fixed-point rules, and wave64 reductions.
//
// The arithmetic here is restated, operation for operation, by the numpy
// oracle; every routine that feeds a discrete decision uses only IEEE
// operations (no FMA contraction, correctly rounded fp32 division) so the two
// agree bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/specdec_amd.h"

namespace sdx {

constexpr int kWave = 64;

// ---------------------------------------------------------------- 16-bit keys
// bf16 and fp16 are sign-magnitude: flipping all bits of negatives and the
// sign bit of positives gives an unsigned key whose order is the value order
// (-0 sorts just below +0; key 0 is the all-ones code, a negative NaN, which
// this build treats as padding/ignored).
__device__ __forceinline__ uint32_t key_of_code16(uint32_t c) {
  return (c & 0x8000u) ? (~c & 0xFFFFu) : (c | 0x8000u);
}
__device__ __forceinline__ uint32_t code_of_key16(uint32_t k) {
  return (k & 0x8000u) ? (k & 0x7FFFu) : (~k & 0xFFFFu);
}
// Two packed codes -> two packed keys.
__device__ __forceinline__ uint32_t keys2_of_codes2(uint32_t w) {
  const uint32_t neg = (w >> 15) & 0x00010001u;  // sign of each half at bit 0 / 16
  return w ^ ((neg * 0x7FFFu) | 0x80008000u);
}

template <int FMT>
__device__ __forceinline__ float decode16(uint32_t code) {
  if constexpr (FMT == SDX_BF16) {
    return __uint_as_float(code << 16);
  } else {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)code);
  }
}
// Key of +inf: keys at or above it are +inf / +NaN.
template <int FMT>
constexpr uint32_t kPosInfKey = FMT == SDX_BF16 ? 0xFF80u : 0xFC00u;

// 32-bit key for fp32 logits (same construction).
__device__ __forceinline__ uint32_t key_of_f32(float x) {
  const uint32_t b = __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// ---------------------------------------------------------------- exp_det
// Deterministic fp32 exp(d), one fixed sequence of IEEE operations:
//   k = floor(fl64(d * (1/ln2)))  and  r = fl32(fl64(d - fl64(k * ln2))),
//   clamped below at 0, so r lies in [0, ln2];
//   p = the degree-9 Taylor polynomial of exp at r in fp32 Horner form
//       (coefficients fl32(1/n!), plain multiply then add), clamped above at 2;
//   e = p * 2^k, rounded once when the result is subnormal;
//   0 for d < -104 (below half the smallest fp32 denormal) and for NaN.
// Within 2 ulps of a correctly rounded expf. Non-decreasing in d, which the
// value-ordered histogram walks rely on: inside one k every Horner step is
// monotone in r (r >= 0, positive coefficients), and across k -> k+1 the left
// value is at most 2 * 2^k (the clamp) while the right one is at least 2^(k+1)
// (r >= 0 gives p >= 1).
__device__ __forceinline__ float exp_det_core(float d) {
#pragma clang fp contract(off)
  const double kInvLn2 = 0x1.71547652b82fep+0;
  const double kLn2 = 0x1.62e42fefa39efp-1;
  const double dd = (double)d;
  const double kf = floor(dd * kInvLn2);
  const float r = fmaxf((float)(dd - kf * kLn2), 0.0f);
  float p = 0x1.71de3ap-19f;  // 1/9!
  p = p * r + 0x1.a01a02p-16f;  // 1/8!
  p = p * r + 0x1.a01a02p-13f;  // 1/7!
  p = p * r + 0x1.6c16c2p-10f;  // 1/6!
  p = p * r + 0x1.111112p-7f;   // 1/5!
  p = p * r + 0x1.555556p-5f;   // 1/4!
  p = p * r + 0x1.555556p-3f;   // 1/3!
  p = p * r + 0x1p-1f;          // 1/2!
  p = p * r + 1.0f;             // 1/1!
  p = p * r + 1.0f;             // 1/0!
  p = fminf(p, 2.0f);
  const int k = (int)kf;
  const bool normal = k >= -126;
  // 2^k, or 2^(k+64) then 2^-64 below the normal range (one rounding)
  const float e = p * __uint_as_float((uint32_t)((normal ? k : k + 64) + 127) << 23);
  return normal ? e : e * 0x1p-64f;
}
__device__ __forceinline__ float exp_det(float d) {
  if (!(d >= -104.0f)) return 0.0f;
  return exp_det_core(d);
}

// exp_det without the early exit: the same value, 0 below -104 (and for NaN)
// by a final select, so that independent evaluations can interleave.
__device__ __forceinline__ float exp_det_sel(float d) {
  const float e = exp_det_core(fmaxf(d, -105.0f));
  return d >= -104.0f ? e : 0.0f;
}

// ---------------------------------------------------------------- fixed point
// floor(x * 2^62) for fp32 x in [0, 1] (branch-free: both shifts, one select).
__device__ __forceinline__ uint64_t fixed62(float x) {
  const uint32_t b = __float_as_uint(x);
  const uint32_t e = b >> 23;
  const uint64_t mant = (uint64_t)((b & 0x7FFFFFu) | (e ? 0x800000u : 0u));
  const int sh = (int)(e ? e : 1u) - 88;  // value = mant * 2^(eff - 150), sh <= 39
  const uint64_t up = mant << (sh & 63);
  const uint64_t dn = mant >> ((-sh) & 63);
  return sh >= 0 ? up : (sh <= -64 ? 0ull : dn);
}

// i * 2^-62 rounded once to fp32 (nearest, ties to even).
__device__ __forceinline__ float rn32_u64(uint64_t i) {
  if (i == 0) return 0.0f;
  const int nb = 64 - __clzll((long long)i);
  int shift = nb - 24;
  if (shift <= 0) return ldexpf((float)(uint32_t)i, -62);
  uint64_t mant = i >> shift;
  const uint64_t rem = i & ((1ull << shift) - 1);
  const uint64_t half = 1ull << (shift - 1);
  if (rem > half || (rem == half && (mant & 1))) {
    ++mant;
    if (mant == (1ull << 24)) {
      mant >>= 1;
      ++shift;
    }
  }
  return ldexpf((float)(uint32_t)mant, shift - 62);
}

// 128-bit unsigned accumulator as two words (hi:lo).
struct U128 {
  uint64_t lo, hi;
};
__device__ __forceinline__ U128 u128_add(U128 a, U128 b) {
  U128 r;
  r.lo = a.lo + b.lo;
  r.hi = a.hi + b.hi + (r.lo < a.lo ? 1 : 0);
  return r;
}
// c * f with c < 2^32, f < 2^64.
__device__ __forceinline__ U128 u128_mul32(uint32_t c, uint64_t f) {
  const uint64_t lo = (uint64_t)c * (uint32_t)f;
  const uint64_t mid = (uint64_t)c * (uint32_t)(f >> 32);
  U128 r;
  r.lo = lo + (mid << 32);
  r.hi = (mid >> 32) + (r.lo < lo ? 1 : 0);
  return r;
}
__device__ __forceinline__ float rn32_u128(U128 v) {
  if (v.hi == 0) return rn32_u64(v.lo);
  const int nb = 128 - __clzll((long long)v.hi);
  int shift = nb - 24;  // > 40
  // mantissa = v >> shift (fits in 24 bits)
  uint64_t mant = (shift >= 64) ? (v.hi >> (shift - 64))
                                : ((v.hi << (64 - shift)) | (v.lo >> shift));
  // remainder vs half: bit (shift-1) and the bits below it
  const int hb = shift - 1;
  const uint64_t halfbit = hb >= 64 ? ((v.hi >> (hb - 64)) & 1) : ((v.lo >> hb) & 1);
  bool below_nonzero;
  if (hb >= 64) {
    const int h2 = hb - 64;
    below_nonzero = v.lo != 0 || (h2 > 0 && (v.hi & ((1ull << h2) - 1)) != 0);
  } else {
    below_nonzero = hb > 0 && (v.lo & ((1ull << hb) - 1)) != 0;
  }
  if (halfbit && (below_nonzero || (mant & 1))) {
    ++mant;
    if (mant == (1ull << 24)) {
      mant >>= 1;
      ++shift;
    }
  }
  return ldexpf((float)(uint32_t)mant, shift - 62);
}

// floor(u * total) for fp32 u in [0, 1): the inverse-CDF target.
__device__ __forceinline__ uint64_t uniform_threshold(float u, uint64_t total) {
  const uint32_t b = __float_as_uint(u);
  if ((b & 0x7FFFFFFFu) == 0) return 0;
  const uint32_t e = b >> 23;
  const uint32_t mant = (b & 0x7FFFFFu) | (e ? 0x800000u : 0u);
  const int s = 150 - (int)(e ? e : 1u);  // u = mant * 2^-s, s >= 24
  const U128 prod = u128_mul32(mant, total);
  if (s >= 128) return 0;
  if (s >= 64) return prod.hi >> (s - 64);
  return (prod.lo >> s) | (prod.hi << (64 - s));
}

// ---------------------------------------------------------------- reductions
// Wave-wide scans and sums: a Hillis-Steele scan inside each 16-lane row with
// DPP row shifts (lanes shifted in from outside the row read 0), then the row
// totals (lanes 15, 31, 47) are added through scalar registers.
__device__ __forceinline__ uint32_t dpp_shr(uint32_t v, int n) {
  switch (n) {
    case 1: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, true);
    case 2: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, true);
    case 4: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, true);
    default: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, true);
  }
}
__device__ __forceinline__ uint32_t rdlane(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
// Inclusive prefix sum across the 64 lanes.
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v, int lane) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v += dpp_shr(v, o);
  const uint32_t r0 = rdlane(v, 15), r1 = rdlane(v, 31), r2 = rdlane(v, 47);
  const int row = lane >> 4;
  v += row >= 1 ? r0 : 0u;
  v += row >= 2 ? r1 : 0u;
  v += row >= 3 ? r2 : 0u;
  return v;
}
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v, int lane) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) {
    const uint32_t tl = dpp_shr(lo, o), th = dpp_shr(hi, o);
    const uint32_t nl = lo + tl;
    hi += th + (nl < lo ? 1u : 0u);
    lo = nl;
  }
  const uint64_t r0 = ((uint64_t)rdlane(hi, 15) << 32) | rdlane(lo, 15);
  const uint64_t r1 = ((uint64_t)rdlane(hi, 31) << 32) | rdlane(lo, 31);
  const uint64_t r2 = ((uint64_t)rdlane(hi, 47) << 32) | rdlane(lo, 47);
  uint64_t x = ((uint64_t)hi << 32) | lo;
  const int row = lane >> 4;
  x += row >= 1 ? r0 : 0ull;
  x += row >= 2 ? r1 : 0ull;
  x += row >= 3 ? r2 : 0ull;
  return x;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v = max(v, dpp_shr(v, o));
  return max(max(rdlane(v, 15), rdlane(v, 31)), max(rdlane(v, 47), rdlane(v, 63)));
}
// Sums: the result is uniform across the wave.
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v += dpp_shr(v, o);
  return rdlane(v, 15) + rdlane(v, 31) + rdlane(v, 47) + rdlane(v, 63);
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
  const uint64_t x = wave_incl_scan_u64(v, (int)(threadIdx.x & 63));
  return ((uint64_t)rdlane((uint32_t)(x >> 32), 63) << 32) | rdlane((uint32_t)x, 63);
}
__device__ __forceinline__ int64_t wave_min_i64(int64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, (int64_t)__shfl_xor((long long)v, o, kWave));
  return v;
}
__device__ __forceinline__ U128 wave_sum_u128(U128 v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    U128 w;
    w.lo = (uint64_t)__shfl_xor((long long)v.lo, o, kWave);
    w.hi = (uint64_t)__shfl_xor((long long)v.hi, o, kWave);
    v = u128_add(v, w);
  }
  return v;
}

// Drafted id whose probability row `r` of group g gathers: target rows (g = 0)
// are [batch, k+1] with position i < k gathering ids[b k + i] (the bonus
// position none), or, with per-row k, tgt_idx[r] indexes ids (-1: bonus);
// draft rows (g = 1) gather ids[r]. -1 when there is none.
__device__ __forceinline__ int64_t draft_id_of_row(const int64_t* ids, const int64_t* tgt_idx,
                                                   int32_t k, int64_t ndrf, int g, int64_t r) {
  if (!ids) return -1;
  if (g) return ids[r];
  if (tgt_idx) {
    const int64_t x = tgt_idx[r];
    return (x >= 0 && x < ndrf) ? ids[x] : -1;
  }
  const int64_t b = r / (k + 1), i = r % (k + 1);
  return i < k ? ids[b * k + i] : -1;
}

}  // namespace sdx
