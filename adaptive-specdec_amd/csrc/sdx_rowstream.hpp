#pragma once
// Row statistics for bf16 logits, streaming: the fused to_probs of
// specdec/sampling.py:34-67 reduced to what the accept test and the final
// draw need, with every logit read from HBM once and nothing kept resident.
//
// The probability of a token depends only on its bf16 value, so the row is
// reduced to counts per value in an LDS histogram. The histogram uses a fixed
// value window, not one anchored at the row maximum, so the LDS atomics start
// as soon as the first 16-byte loads land and overlap the rest of the row:
//   bin 0               x <= -2^16, -inf, -NaN       (exp_det == 0, checked)
//   bins 1..5120        -2^16 < x <= -2^-24          (one bin per bf16 value)
//   bin 5121            |x| < 2^-24, +-0, denormals  (all share exp(-m), checked)
//   bins 5122..10241    2^-24 <= x < 2^16            (one bin per bf16 value)
//   bin 10242           x >= 2^16, +inf, +NaN        (row leaves the fixed window)
// The bins are in value order, and a bin follows from the raw code with
// packed 16-bit arithmetic on two codes at once (magnitude clamped into the
// window, mirrored for negative codes), about ten vector instructions per two
// logits; the running maximum is tracked on the bins. 40 KiB of LDS per
// 512-thread workgroup fits three workgroups per CU, so the 576 rows of a
// B=64, k=4 verify all stream at once and share HBM evenly.
//
// After the histogram, the whole block works on it: the exact fixed-point
// normaliser over occupied bins (the top bins' exp values kept in LDS); the
// top-k / top-p walk down from the maximum in rounds of one bin per thread,
// with a block scan of exact cumulative mass and the reference's fp32 keep
// test `cum - p < top_p`; the boundary tie group (occupied bins of equal
// probability) and the number of its members kept, lowest ids first. Block
// reductions cost one barrier each (partials go to alternating LDS slots).
// The index cut inside the tie group is left to the consumers, which count
// group members in id order as they stream the rows they need; a drafted
// token inside its row's group is ranked here when the group is its own value
// alone, else by the accept chain of the draw (or the rank kernel).
//
// x / T is evaluated as fl32(fl64(x) * fl64(1 / T)). For a 16-bit x (at most
// 11 significant bits) and fp32 T this equals the correctly rounded fp32
// quotient: the fp64 product is within 2^-52 (relative) of x / T, while x / T
// is never an fp32 rounding midpoint and stays at least 2^-49 (relative) away
// from every midpoint, its significand being a ratio of integers below 2^24.
//
// Elements in bin 0 that carry mass (huge negative logits at huge
// temperatures) are summed by one more pass. Rows the fixed window cannot
// represent (values >= 2^16, a maximum among the merged tiny values, tiny
// values of different probability) are re-streamed into a histogram anchored
// at the row maximum (keys [kmax - 10242, kmax]). A decision that needs the
// order of elements below either window marks the row unsupported.
#include <stdlib.h>

#include "sdx_draw16.hpp"

namespace sdx {

constexpr int SK_NT = 512;
constexpr int SK_NW = SK_NT / kWave;
constexpr uint32_t SK_MAG_LO = 0x3380u;   // magnitude code of 2^-24
constexpr int SK_WIN = 5120;              // window values per sign
constexpr uint32_t SK_NEG_LO = 0x3880u;   // key of -(2^16 - ulp)
constexpr uint32_t SK_ZERO_LO = 0x4C80u;  // first key of the merged tiny-magnitude bin
constexpr uint32_t SK_ZERO_HI = 0xB37Fu;  // its last key
constexpr uint32_t SK_POS_LO = 0xB380u;   // key of 2^-24
constexpr int SK_BIN_ZERO = SK_WIN + 1;
constexpr int SK_BIN_EXC = 2 * SK_WIN + 2;
constexpr int SK_NB = 2 * SK_WIN + 4;     // bins, the last one (SK_NB - 1) unused
constexpr int SK_ETOP = 1024;             // exp values cached for the top bins
constexpr int SK_ZQ = 3 * kWave;          // per-wave queue of occupied bins (normaliser)
constexpr int SK_PW = 8 * kWave;          // top bins the top-p walk covers with one wave
// Rows split over several blocks: each part publishes its histogram as u16
// counts, 8 bins per 16-byte chunk, then a header chunk (its largest bin
// offset, its count of equal-bin elements before the drafted token).
constexpr int SK_SPLIT_CHUNKS = (SK_NB + 7) / 8;
constexpr uint32_t SK_SPLIT_BYTES = ((SK_SPLIT_CHUNKS + 1) * 16 + 63) / 64 * 64;
constexpr int64_t SK_PART_MAX = 65535;          // logits per part (u16 counts)
constexpr int64_t SK_PART_MIN_GROUPS = 1024;    // 8-logit groups per part, at least
constexpr uint32_t SK_SC1 = 16;  // buffer-op cache policy: coherent across the device

__device__ __forceinline__ int sk_bin_of_key(uint32_t k) {
  const uint32_t c1 = min(k > SK_NEG_LO - 1 ? k - (SK_NEG_LO - 1) : 0u, (uint32_t)SK_WIN + 1);
  const uint32_t c2 = min(k > SK_ZERO_HI ? k - SK_ZERO_HI : 0u, (uint32_t)SK_WIN + 1);
  return (int)(c1 + c2);
}
// Two packed bf16 codes -> two packed byte offsets 4 * bin (each < 2^16):
// t = clamp(|code| - (SK_MAG_LO - 1), 0, SK_WIN + 1) is the magnitude's place
// in the window; bin = SK_WIN + 1 + t for a positive code, SK_WIN + 1 - t for
// a negative one, formed as 4 * (t ^ s) + (4 * (SK_WIN + 1) - 4 * s) with
// s = 0 or 0xFFFF (the sign spread over the half), all modulo 2^16.
typedef unsigned short us2 __attribute__((ext_vector_type(2)));
typedef short ss2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t sk_off2(uint32_t w) {
  const us2 c = __builtin_bit_cast(us2, w);
  const us2 mag = c & (us2){0x7FFF, 0x7FFF};
  const us2 t = __builtin_elementwise_min(
      __builtin_elementwise_sub_sat(mag, (us2){SK_MAG_LO - 1, SK_MAG_LO - 1}),
      (us2){SK_WIN + 1, SK_WIN + 1});
  const us2 s = __builtin_bit_cast(us2, __builtin_bit_cast(ss2, c) >> (ss2){15, 15});
  const us2 x = t ^ s;
  const us2 cs = s * (us2){0xFFFC, 0xFFFC} + (us2){4 * (SK_WIN + 1), 4 * (SK_WIN + 1)};
  return __builtin_bit_cast(uint32_t, x * (us2){4, 4} + cs);
}
__device__ __forceinline__ uint32_t max2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(us2, a),
                                                                __builtin_bit_cast(us2, b)));
}
__device__ __forceinline__ uint32_t min2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(us2, a),
                                                                __builtin_bit_cast(us2, b)));
}
__device__ __forceinline__ uint32_t add2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(us2, a) + __builtin_bit_cast(us2, b));
}

// Bin <-> key maps of the two window kinds. Fixed: as tabled above. Anchored:
// bin b >= 1 holds key lo + b - 1, bin 0 the keys below lo.
struct BinMap {
  bool anchored;
  uint32_t lo;
  uint32_t zrep;  // fixed window: a key of the merged tiny bin standing for all of it
  uint32_t zlo;   // the merged tiny bin's lowest key: SK_ZERO_LO, or its smallest key
                  // present when only its members (not its edges) share one exp value
  __device__ uint32_t key_lo(int b) const {
    if (anchored) return b <= 0 ? 0u : lo + (uint32_t)(b - 1);
    if (b <= 0) return 0u;
    if (b <= SK_WIN) return SK_NEG_LO + (uint32_t)(b - 1);
    if (b == SK_BIN_ZERO) return zlo;
    return SK_POS_LO + (uint32_t)(b - SK_BIN_ZERO - 1);
  }
  __device__ uint32_t key_hi(int b) const {
    if (!anchored && b == SK_BIN_ZERO) return SK_ZERO_HI;
    return key_lo(b);
  }
  // key whose value stands for the bin in exp
  __device__ uint32_t key_rep(int b) const {
    return (!anchored && b == SK_BIN_ZERO) ? zrep : key_lo(b);
  }
  // key_rep(b) for b >= 1 by selects alone (no divergent branches), for the
  // normaliser's per-bin evaluations; b = 0 gives a key whose exp is unused
  __device__ uint32_t key_rep_sel(int b) const {
    const uint32_t ub = (uint32_t)b;
    const uint32_t kf = ub <= (uint32_t)SK_WIN ? SK_NEG_LO - 1u + ub
                                               : SK_POS_LO - (uint32_t)SK_BIN_ZERO - 1u + ub;
    const uint32_t kz = ub == (uint32_t)SK_BIN_ZERO ? zrep : kf;
    return anchored ? lo - 1u + ub : kz;
  }
  __device__ int bin(uint32_t k) const {
    if (anchored) return k < lo ? 0 : (int)(k - lo) + 1;
    return sk_bin_of_key(k);
  }
};

// fl32(x / T) as fl32(fl64(x) * fl64(1/T)) (equal for 16-bit x, see above)
__device__ __forceinline__ float sk_s(uint32_t key, double invT) {
  return (float)((double)decode16<SDX_BF16>(code_of_key16(key)) * invT);
}
__device__ __forceinline__ float sk_d(uint32_t key, double invT, float m) {
  return sk_s(key, invT) - m;
}

// ---------------------------------------------------------------- block helpers
// All of them contain barriers: call them from every thread of the block.
// Partials go to LDS slot set `rs`, which then flips: a set is written again
// only after the next helper's barrier, which every thread passes after
// reading it, so each helper needs one barrier.
template <int NW>
struct SkRedT {
  uint64_t v[2][4][NW];
};
using SkRed = SkRedT<SK_NW>;
enum : int { kOpNone = 0, kOpSum64 = 1, kOpMin32 = 2, kOpMax32 = 3, kOpSum32 = 4 };
template <int O>
__device__ __forceinline__ uint64_t sk_wave_op(uint64_t v) {
  if constexpr (O == kOpSum64) return wave_sum_u64(v);
  else if constexpr (O == kOpMin32) return (uint64_t)(~wave_max_u32(~(uint32_t)v));
  else if constexpr (O == kOpMax32) return (uint64_t)wave_max_u32((uint32_t)v);
  else if constexpr (O == kOpSum32) return (uint64_t)wave_sum_u32((uint32_t)v);
  else return 0;
}
template <int O>
__device__ __forceinline__ uint64_t sk_comb(uint64_t a, uint64_t b) {
  if constexpr (O == kOpMin32) return min(a, b);
  else if constexpr (O == kOpMax32) return max(a, b);
  else return a + b;
}
template <int O>
__device__ __forceinline__ uint64_t sk_ident() {
  return O == kOpMin32 ? 0xFFFFFFFFull : 0ull;
}
struct Red4 {
  uint64_t v[4];
};
template <int O0, int O1 = kOpNone, int O2 = kOpNone, int O3 = kOpNone, int NW>
__device__ __forceinline__ Red4 blk_red(uint64_t a0, uint64_t a1, uint64_t a2, uint64_t a3,
                                        SkRedT<NW>& red, int& rs) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const uint64_t x0 = sk_wave_op<O0>(a0), x1 = sk_wave_op<O1>(a1);
  const uint64_t x2 = sk_wave_op<O2>(a2), x3 = sk_wave_op<O3>(a3);
  if (lane == 0) {
    red.v[rs][0][w] = x0;
    if (O1) red.v[rs][1][w] = x1;
    if (O2) red.v[rs][2][w] = x2;
    if (O3) red.v[rs][3][w] = x3;
  }
  __syncthreads();
  Red4 r = {{sk_ident<O0>(), sk_ident<O1>(), sk_ident<O2>(), sk_ident<O3>()}};
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    r.v[0] = sk_comb<O0>(r.v[0], red.v[rs][0][i]);
    if (O1) r.v[1] = sk_comb<O1>(r.v[1], red.v[rs][1][i]);
    if (O2) r.v[2] = sk_comb<O2>(r.v[2], red.v[rs][2][i]);
    if (O3) r.v[3] = sk_comb<O3>(r.v[3], red.v[rs][3][i]);
  }
  rs ^= 1;
  return r;
}
template <int NW>
__device__ __forceinline__ uint32_t blk_min_u32(uint32_t v, SkRedT<NW>& red, int& rs) {
  return (uint32_t)blk_red<kOpMin32>(v, 0, 0, 0, red, rs).v[0];
}
template <int NW>
__device__ __forceinline__ uint32_t blk_max_u32(uint32_t v, SkRedT<NW>& red, int& rs) {
  return (uint32_t)blk_red<kOpMax32>(v, 0, 0, 0, red, rs).v[0];
}
template <int NW>
__device__ __forceinline__ uint32_t blk_sum_u32(uint32_t v, SkRedT<NW>& red, int& rs) {
  return (uint32_t)blk_red<kOpSum32>(v, 0, 0, 0, red, rs).v[0];
}
template <int NW>
__device__ __forceinline__ uint64_t blk_sum_u64(uint64_t v, SkRedT<NW>& red, int& rs) {
  return blk_red<kOpSum64>(v, 0, 0, 0, red, rs).v[0];
}
// Inclusive block scan, one barrier; *total gets the block sum.
template <int NW>
__device__ __forceinline__ uint64_t blk_incl_u64(uint64_t v, SkRedT<NW>& red, int& rs,
                                                 uint64_t* total) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const uint64_t incl = wave_incl_scan_u64(v, lane);
  if (lane == kWave - 1) red.v[rs][0][w] = incl;
  __syncthreads();
  uint64_t off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const uint64_t x = red.v[rs][0][i];
    off += i < w ? x : 0ull;
    tot += x;
  }
  rs ^= 1;
  *total = tot;
  return off + incl;
}
template <int NW>
__device__ __forceinline__ uint32_t blk_incl_u32(uint32_t v, SkRedT<NW>& red, int& rs,
                                                 uint32_t* total) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const uint32_t incl = wave_incl_scan_u32(v, lane);
  if (lane == kWave - 1) red.v[rs][0][w] = incl;
  __syncthreads();
  uint32_t off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const uint32_t x = (uint32_t)red.v[rs][0][i];
    off += i < w ? x : 0u;
    tot += x;
  }
  rs ^= 1;
  *total = tot;
  return off + incl;
}

// Whole block: the largest key of the row (padding / -NaN code 0xFFFF has key 0).
template <int NW>
__device__ uint32_t exact_kmax(const uint16_t* __restrict__ ptr, int64_t V, SkRedT<NW>& red,
                               int& rs) {
  uint32_t mx = 0;
  for (int64_t i = threadIdx.x; i < V; i += NW * kWave) mx = max(mx, key_of_code16(ptr[i]));
  return blk_max_u32(mx, red, rs);
}
// Whole block: counts the row's elements into `hist` under an anchored map.
template <int NT>
__device__ void restream_anchored(const uint16_t* __restrict__ ptr, int64_t V, const BinMap& bm,
                                  uint32_t* hist) {
  for (int64_t e0 = (int64_t)threadIdx.x * 8; e0 < V; e0 += (int64_t)NT * 8) {
    uint32_t c[8];
    if (e0 + 8 <= V) {
      const uint4 v = *reinterpret_cast<const uint4*>(ptr + e0);
      c[0] = v.x & 0xFFFFu; c[1] = v.x >> 16; c[2] = v.y & 0xFFFFu; c[3] = v.y >> 16;
      c[4] = v.z & 0xFFFFu; c[5] = v.z >> 16; c[6] = v.w & 0xFFFFu; c[7] = v.w >> 16;
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) c[t] = e0 + t < V ? ptr[e0 + t] : 0u;
    }
#pragma unroll
    for (int t = 0; t < 8; ++t)
      if (e0 + t < V) atomicAdd(&hist[bm.bin(key_of_code16(c[t]))], 1u);
  }
}
// Whole block, one pass: the largest key below `lo` (0 if none); over the keys
// in [zlo, zhi], the smallest key (0xFFFF if none) and the smallest / largest
// exp_det(x/T - m) as fp32 bit patterns (exp values are >= 0).
struct Extremes {
  uint32_t below_max, zkey_min, ze_min, ze_max;
};
template <int NW>
__device__ Extremes key_extremes(const uint16_t* __restrict__ ptr, int64_t V, uint32_t lo,
                                 uint32_t zlo, uint32_t zhi, double invT, float m,
                                 SkRedT<NW>& red, int& rs) {
  uint32_t b = 0, z0 = 0xFFFFu, e0 = 0xFFFFFFFFu, e1 = 0;
  for (int64_t i = threadIdx.x; i < V; i += NW * kWave) {
    const uint32_t k = key_of_code16(ptr[i]);
    if (k < lo) b = max(b, k);
    if (k >= zlo && k <= zhi) {
      const uint32_t e = __float_as_uint(exp_det(sk_d(k, invT, m)));
      z0 = min(z0, k);
      e0 = min(e0, e);
      e1 = max(e1, e);
    }
  }
  const Red4 r = blk_red<kOpMax32, kOpMin32, kOpMin32, kOpMax32>(b, z0, e0, e1, red, rs);
  Extremes x;
  x.below_max = (uint32_t)r.v[0];
  x.zkey_min = (uint32_t)r.v[1];
  x.ze_min = (uint32_t)r.v[2];
  x.ze_max = (uint32_t)r.v[3];
  return x;
}
// Whole block: sum over elements with key < lo of fixed62(exp_det(x/T - m) / div),
// exact in 128 bits (split as sum lo32 + 2^32 sum hi32, each below 2^63).
template <int NW>
__device__ U128 below_sum(const uint16_t* __restrict__ ptr, int64_t V, uint32_t lo, double invT,
                          float m, float div, SkRedT<NW>& red, int& rs) {
  uint64_t slo = 0, shi = 0;
  for (int64_t i = threadIdx.x; i < V; i += NW * kWave) {
    const uint32_t k = key_of_code16(ptr[i]);
    if (k < lo) {
      const float e = exp_det(sk_d(k, invT, m));
      const uint64_t f = fixed62(div == 1.0f ? e : e / div);
      slo += (uint32_t)f;
      shi += (uint32_t)(f >> 32);
    }
  }
  const Red4 r = blk_red<kOpSum64, kOpSum64>(slo, shi, 0, 0, red, rs);
  return u128_add(U128{r.v[0], 0}, U128{r.v[1] << 32, r.v[1] >> 32});
}

// Rows split over P blocks. Every part publishes its histogram (u16 counts) and
// header with device-coherent stores, waits for them, then counts itself in on
// the row's arrival counter; the part that arrives last adds the other parts
// into its LDS histogram, their largest offsets into *omx and their token
// counts into *cp, resets the counter to zero and returns 1. The others return
// 0 (and leave the kernel). When the workspace header lacks its magic word the
// counters cannot be trusted: no part counts in and every part returns 2.
//
// Hand-off invariant: every store of a part's histogram and header and every
// load of them by the merging part carries the sc1 cache policy (device
// coherent: no XCD's L2 keeps a stale copy), and each part waits for its stores
// (vmcnt(0)) before its relaxed agent-scope counter increment. A plain store or
// load of the handed-off data added here would race across XCDs.
typedef uint32_t sk_u32x4 __attribute__((ext_vector_type(4)));
template <int NT>
__device__ __forceinline__ int split_merge(const uint32_t* magic, uint32_t* __restrict__ cnt,
                                           uint8_t* parts, int P, int64_t sidx, int part,
                                           uint32_t* hist, uint32_t* omx, uint32_t* cp,
                                           int32_t* flag) {
  const int tid = threadIdx.x;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      parts + sidx * P * (int64_t)SK_SPLIT_BYTES, (short)0, (int)(P * SK_SPLIT_BYTES), 0x00020000);
  const uint32_t mine = (uint32_t)part * SK_SPLIT_BYTES;
  for (int c = tid; c < SK_SPLIT_CHUNKS; c += NT) {
    const uint4 h0 = *reinterpret_cast<const uint4*>(hist + 8 * c);
    const uint4 h1 = *reinterpret_cast<const uint4*>(hist + 8 * c + 4);
    const sk_u32x4 w = {h0.x | (h0.y << 16), h0.z | (h0.w << 16), h1.x | (h1.y << 16),
                        h1.z | (h1.w << 16)};
    __builtin_amdgcn_raw_buffer_store_b128(w, rsrc, c * 16, (int)mine, SK_SC1);
  }
  if (tid == 0) {
    const sk_u32x4 h = {*omx, *cp, 0u, 0u};
    __builtin_amdgcn_raw_buffer_store_b128(h, rsrc, SK_SPLIT_CHUNKS * 16, (int)mine, SK_SC1);
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // gfx9 encoding: vmcnt(0) (stores done)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (tid == 0) {
    int f = 2;
    if (__hip_atomic_load(magic, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == kWsMagic) {
      const uint32_t prev =
          __hip_atomic_fetch_add(cnt + sidx, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool last = prev == (uint32_t)(P - 1);
      if (last) __hip_atomic_store(cnt + sidx, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      f = last ? 1 : 0;
    }
    flag[0] = f;
  }
  __syncthreads();
  if (flag[0] != 1) return flag[0];
  // thread t owns chunks t, t + NT, ... (KC of them)
  constexpr int KC = (SK_SPLIT_CHUNKS + NT - 1) / NT;
  static_assert(KC >= 1 && KC <= 3, "chunks per thread");
  uint32_t acc[KC][8];
#pragma unroll
  for (int k = 0; k < KC; ++k)
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[k][t] = 0u;
  uint32_t om = *omx, cc = *cp;
  for (int o = 0; o < P; ++o) {  // uniform
    if (o == part) continue;
    const int so = o * (int)SK_SPLIT_BYTES;
    sk_u32x4 x[KC];
#pragma unroll
    for (int k = 0; k < KC; ++k) {  // clamped: every thread loads, unowned chunks unused
      const int c = min(tid + k * NT, SK_SPLIT_CHUNKS - 1);
      x[k] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, c * 16, so, SK_SC1);
    }
    const sk_u32x4 h = __builtin_amdgcn_raw_buffer_load_b128(rsrc, SK_SPLIT_CHUNKS * 16, so, SK_SC1);
    om = max(om, h[0]);
    cc += h[1];
#pragma unroll
    for (int k = 0; k < KC; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[k][2 * j] += x[k][j] & 0xFFFFu;
        acc[k][2 * j + 1] += x[k][j] >> 16;
      }
  }
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int c = tid + k * NT;
    if (c < SK_SPLIT_CHUNKS) {
#pragma unroll
      for (int t = 0; t < 8; ++t) hist[8 * c + t] += acc[k][t];
    }
  }
  __syncthreads();
  *omx = om;
  *cp = cc;
  return 1;
}

// All LDS of the kernel in one object, histogram first (LDS address 0, so the
// streaming atomics address it by byte offset alone).
template <int NT>
struct SkLdsT {
  uint32_t hist[SK_SPLIT_CHUNKS * 8];  // SK_NB bins, zero padding to whole chunks
  float etop[SK_ETOP];  // exp values of the top SK_ETOP bins (bmax - i); occupied ones only
  uint32_t zq[NT / kWave][SK_ZQ];  // per-wave queues of occupied bins for the normaliser
  SkRedT<NT / kWave> red;
  int32_t i32[12];
  int32_t pw[5];  // top-p walk of wave 0: boundary bin (or -1), its group bins and counts
  uint64_t x64[2];
  uint32_t unit_ctr;  // next 4 KB unit of the row to stream
};
using SkLds = SkLdsT<SK_NT>;

// Outputs of a row: plain stores, or device-coherent ones (agent-scope atomic
// stores, which no XCD's L2 keeps back) when the draw that reads them runs in
// the same launch.
__device__ __forceinline__ void st_rowstat(RowStat* dst, const RowStat& st, bool coh) {
  if (coh) {
    const uint64_t* s = reinterpret_cast<const uint64_t*>(&st);
    uint64_t* d = reinterpret_cast<uint64_t*>(dst);
#pragma unroll
    for (int i = 0; i < 8; ++i) __hip_atomic_store(d + i, s[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    *dst = st;
  }
}
__device__ __forceinline__ void st_f32(float* dst, float v, bool coh) {
  if (coh)
    __hip_atomic_store(reinterpret_cast<uint32_t*>(dst), __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  else
    *dst = v;
}

// Rows in batch-row order (jm_k = k > 0): the q-th row taken is position
// q % (2k + 1) of batch row q / (2k + 1), target positions first, so the rows of
// one batch row finish close together. With `xcd` (batch % 8 == 0) the order is
// kept per XCD instead: block q runs on XCD q % 8 (blocks are dealt to the XCDs
// in index order), and the (q / 8)-th row taken there is position
// (q / 8) % (2k + 1) of batch row q % 8 + 8 ((q / 8) / (2k + 1)). A batch row's
// rows then stream on the XCD its draw blocks run on, which reads two of them
// again.
__device__ __forceinline__ int64_t jm_row(int64_t q, int32_t k, int64_t ntgt, bool xcd) {
  const int64_t n = 2 * k + 1;
  int64_t b, i;
  if (xcd) {
    const int64_t s = q >> 3;
    b = (q & 7) + 8 * (s / n);
    i = s % n;
  } else {
    b = q / n;
    i = q % n;
  }
  return i <= k ? b * (k + 1) + i : ntgt + b * k + (i - k - 1);
}

// One block's share of the row statistics (block blk of the launch). Returns
// the row whose statistics this block completed (written), or -1 (a split
// row's part that did not merge).
template <bool FUSED, int NT = SK_NT>
__device__ __forceinline__ int64_t rowstream_body(const RowStatArgs& a, SkLdsT<NT>& L,
                                                  int64_t blk) {
  uint32_t* const hist = L.hist;
  int rs = 0;

  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  // the row, and the part of it when rows after nwhole are split over nparts blocks
  const int P = a.nparts;
  int64_t row = blk, sidx = -1;
  int part = -1;
  if (blk >= a.nwhole) {
    const int64_t q = blk - a.nwhole;
    if (a.xcd_group) {
      const int64_t t = q >> 3;
      sidx = (t / P) * 8 + (q & 7);
      part = (int)(t % P);
    } else {
      sidx = q / P;
      part = (int)(q % P);
    }
    row = a.nwhole + sidx;
  }
  if (FUSED)
    row = a.jm_order ? (int64_t)a.jm_order[row] : jm_row(row, a.jm_k, a.nrows[0], a.jm_xcd != 0);
  const int g = row < a.nrows[0] ? 0 : 1;
  const int64_t r = g ? row - a.nrows[0] : row;
  const uint16_t* __restrict__ ptr = a.base[g] + r * a.ld[g];
  const int64_t gid = draft_id_of_row(a.ids, a.tgt_idx, a.k, a.nrows[1], g, r);
  const int64_t V = a.V;
  RowStat* st_out = a.stats + row;
  float* tbl_out = a.tables + row * kTbl;
  if (part <= 0 && row < a.nzero) {
    const int zpr = a.zero_per_row > 0 ? a.zero_per_row : 1;
    if (tid < zpr) a.zero[row * zpr + tid] = 0u;
  }
  if (tid == 0 && part <= 0 && a.rank_acc) a.rank_acc[row] = 0ull;

  for (int b = tid; b < SK_SPLIT_CHUNKS * 8; b += NT) hist[b] = 0u;
  if (tid == 0) L.unit_ctr = 0u;
  __syncthreads();

  // ---- 1. stream the row: 16-byte loads two stages deep, packed codes ->
  // packed bin offsets, LDS atomics; the running maximum on the offsets
  // Blocks dealt after two per CU share a CU with two older workgroups, whose
  // waves win instruction arbitration; raising this block's wave priority while
  // it streams lets all three stream side by side instead of this one last.
  if ((int64_t)blockIdx.x >= a.late_block) __builtin_amdgcn_s_setprio(3);
  uint32_t omx = 0;
  // The drafted token's member rank, when its tie group turns out to be its own
  // value alone: equal codes before it, counted while streaming (a token in the
  // last V % 8 elements: the histogram's count, read once every unit is in).
  const bool has_g = gid >= 0 && gid < V;
  const uint32_t cg = has_g ? (uint32_t)ptr[gid] : 0u;
  const int bin_g = sk_bin_of_key(key_of_code16(cg));
  uint32_t snap = 0, pre = 0;  // pre: per thread, equal codes before the token
  // this block's range: 8-element groups [g0, g1), then the last V % 8 elements
  // when it holds the row's end
  const uint32_t n4_all = (uint32_t)(V >> 3);  // whole 8-element groups (V < 2^31)
  uint32_t g0 = 0, g1 = n4_all;
  if (part >= 0) {
    g0 = (uint32_t)((int64_t)n4_all * part / P);
    g1 = (uint32_t)((int64_t)n4_all * (part + 1) / P);
  }
  const bool has_tail = g1 == n4_all;
  const int64_t gid_l = gid - (int64_t)g0 * 8;  // the token's place in the range
  const bool g_in_groups = has_g && gid_l >= 0 && gid_l < (int64_t)(g1 - g0) * 8;
  const bool g_in_tail = has_g && has_tail && gid >= (int64_t)n4_all * 8;
  {
    // Units of 4 KB (64 lanes x 4 x 16 bytes) are dealt to the waves from an LDS
    // counter, so a wave that streams faster takes more of them and the block's
    // waves finish together (with a fixed split the second wave on each SIMD
    // finished about 4 us after the first). Raw buffer loads: the lane offset
    // stays in a register, the unit offset is scalar; loads past the range read
    // zeros without touching memory (a wave's last grab), and are not processed.
    constexpr int U = 4;
    constexpr uint32_t kUnit = (uint32_t)kWave * U;  // 8-element groups per unit
    const uint32_t n4 = g1 - g0;
    const uint32_t nunits = (n4 + kUnit - 1) / kUnit;
    // the resource from scalar copies of its (uniform) fields: built from values the
    // compiler cannot prove uniform it would wrap every load in a readfirstlane loop
    const uint64_t rb = (uint64_t)(uintptr_t)(ptr + (int64_t)g0 * 8);
    const uint64_t rbu = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(rb >> 32))
                          << 32) |
                         (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)rb);
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(uintptr_t)rbu, (short)0, __builtin_amdgcn_readfirstlane((int)(n4 * 16u)),
        0x00020000);
    const uint32_t voff = (uint32_t)lane * 16u;
    char* const hb = reinterpret_cast<char*>(hist);
    // the drafted token's rank: every equal code in units before the token's unit,
    // and those before it inside that unit (bin_g holds its value alone whenever
    // the count is used, so equal bins are equal codes)
    const uint32_t u_tok = g_in_groups ? (uint32_t)((gid_l >> 3) / kUnit) : 0u;
    const uint32_t og = 4u * (uint32_t)bin_g;
    const uint32_t og2 = og | (og << 16);
    // per half of the packed bin offsets: words of counted units whose offset
    // differed from the token's (packed 16-bit counts, at most 4 per group and
    // row, so no half overflows), and the counted words
    uint32_t neq2 = 0, ncw = 0;
    auto grab = [&]() -> uint32_t {
      uint32_t u = 0;
      if (lane == 0) u = atomicAdd(&L.unit_ctr, 1u);
      return (uint32_t)__builtin_amdgcn_readfirstlane((int)u);
    };
    auto load = [&](uint4 (&d)[U], uint32_t u) {
#pragma unroll
      for (int k = 0; k < U; ++k) {
        const auto x = __builtin_amdgcn_raw_buffer_load_b128(
            rsrc, (int)voff, (int)((u * kUnit + (uint32_t)k * kWave) * 16u), 0);
        d[k] = make_uint4(x[0], x[1], x[2], x[3]);
      }
    };
    auto proc = [&](const uint4& v, bool cnt) {
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t o = sk_off2(w[t]);
        omx = max2(omx, o);
        atomicAdd(reinterpret_cast<uint32_t*>(hb + (o & 0xFFFFu)), 1u);
        atomicAdd(reinterpret_cast<uint32_t*>(hb + (o >> 16)), 1u);
        if (cnt) neq2 = add2(neq2, min2(o ^ og2, 0x00010001u));  // 0 per equal half
      }
      if (cnt) ncw += 4u;
    };
    auto proc_unit = [&](const uint4 (&d)[U], uint32_t u) {
      const bool full = (u + 1) * kUnit <= n4;  // uniform
      const bool cnt = u < u_tok;               // uniform
#pragma unroll
      for (int k = 0; k < U; ++k) {
        const uint32_t grp = u * kUnit + (uint32_t)k * kWave + (uint32_t)lane;
        if (full || grp < n4) {
          if (cnt) proc(d[k], true);
          else proc(d[k], false);
        }
      }
      if (g_in_groups && u == u_tok) {  // uniform: the token's unit, counted by hand
#pragma unroll
        for (int k = 0; k < U; ++k) {
          const int64_t e0 = (int64_t)(u * kUnit + (uint32_t)k * kWave + (uint32_t)lane) * 8;
          const uint32_t wd[4] = {d[k].x, d[k].y, d[k].z, d[k].w};
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            const uint32_t c = (t & 1) ? wd[t >> 1] >> 16 : wd[t >> 1] & 0xFFFFu;
            pre += (e0 + t < gid_l && c == cg) ? 1u : 0u;
          }
        }
      }
    };
    if (nunits > 0) {  // uniform
      uint4 A[U], B[U];
      uint32_t ua = grab();
      load(A, ua);
      for (;;) {  // grabs only grow, so a unit past the end ends the wave's work
        const uint32_t ub = grab();
        load(B, ub);
        if (ua >= nunits) break;
        proc_unit(A, ua);
        ua = grab();
        load(A, ua);
        if (ub >= nunits) break;
        proc_unit(B, ub);
      }
    }
    pre += 2u * ncw - (neq2 & 0xFFFFu) - (neq2 >> 16);
    if (g_in_tail) {  // the token among the last V % 8 elements
      __syncthreads();
      snap = hist[bin_g];
    }
    const int64_t t0 = (int64_t)n4_all * 8;  // the last V % 8 elements, one per thread
    if (has_tail && tid < V - t0) {
      const uint32_t c = ptr[t0 + tid];
      const uint32_t o = 4u * (uint32_t)sk_bin_of_key(key_of_code16(c));
      omx = max2(omx, o);
      atomicAdd(reinterpret_cast<uint32_t*>(hb + o), 1u);
      if (g_in_tail && t0 + tid < gid && c == cg) ++pre;
    }
  }
  __builtin_amdgcn_s_setprio(0);
  // (the reduction's barrier also completes the histogram)
  uint32_t omx_b = blk_max_u32(max(omx & 0xFFFFu, omx >> 16), L.red, rs);
  if (part >= 0) {  // uniform: publish this part; the last part of the row to finish goes on
    // its count of equal-bin elements before the token
    uint32_t cp = 0;
    if (g_in_groups || g_in_tail) cp = snap + blk_sum_u32(pre, L.red, rs);
    else if (has_g && gid >= (int64_t)g1 * 8) cp = hist[bin_g];
    const int mg = split_merge<NT>(a.ws_header, a.split_cnt, a.split_parts, P, sidx, part, hist,
                               &omx_b, &cp, L.i32 + 11);
    if (mg == 2 && part == 0 && tid == 0) {  // uninitialised workspace: flag the row
      RowStat st = {};
      st.flags = kRowBadWs | kRowUnsupported;
      st.zf = 1.0f; st.totf = 1.0f; st.klo = 0x7FFFFFFF; st.glo = 1; st.ghi = 0; st.argmax = -1;
      st_rowstat(st_out, st, FUSED);
    }
    if (mg != 1) return mg == 2 && part == 0 ? row : -1;
    snap = cp;  // every part's count, this one's included
    pre = 0;
  }
  const int bmx = (int)(omx_b >> 2);
  uint32_t kmax;
  if (bmx >= 1 && bmx <= 2 * SK_WIN + 1 && bmx != SK_BIN_ZERO) {
    kmax = bmx <= SK_WIN ? SK_NEG_LO + (uint32_t)(bmx - 1)
                         : SK_POS_LO + (uint32_t)(bmx - SK_BIN_ZERO - 1);
  } else {  // the maximum is not a single window value: find it (uniform branch)
    kmax = exact_kmax(ptr, V, L.red, rs);
  }

  if (kmax >= kPosInfKey<SDX_BF16> || kmax == 0) {  // +inf / NaN: flag, outputs unspecified
    if (tid == 0) {
      RowStat st = {};
      st.flags = kRowNonfinite;
      st.zf = 1.0f; st.totf = 1.0f; st.klo = 0x7FFFFFFF; st.glo = 1; st.ghi = 0; st.argmax = -1;
      st_rowstat(st_out, st, FUSED);
    }
    return row;
  }
  const float T = a.T;
  const double invT = 1.0 / (double)T;
  const float m = sk_s(kmax, invT);

  // ---- 2. fixed window valid for this row? else re-stream anchored at kmax.
  // Bin 0 ("below the window") may carry mass: then Z adds it by one more pass
  // and a decision that needs it marks the row unsupported. The quick checks
  // use the bins' edge keys; when they fail, one pass finds the actual extreme
  // keys (rare: huge negative logits at huge temperatures, tiny logits).
  BinMap bm{false, 0u, 0x8000u, SK_ZERO_LO};
  uint32_t rflags = 0;
  uint32_t below_lo = SK_NEG_LO;  // keys below it are below the window
  bool below_mass = false;        // ... and some of them have exp_det > 0
  uint32_t below_top = 0;         // the largest key below the window
  {
    const int b0 = sk_bin_of_key(kmax);
    bool ok = b0 >= 1 && b0 != SK_BIN_EXC;
    const bool maybe_below = ok && hist[0] != 0 && exp_det(sk_d(SK_NEG_LO - 1, invT, m)) > 0.0f;
    // the merged tiny bin needs one exp value for all its members: d equal at its
    // edges (fp32 division and subtraction are monotone), else checked per member
    const float dz = sk_d(0x8000u, invT, m);
    const bool check_zero = ok && hist[SK_BIN_ZERO] != 0 &&
                            !(sk_d(SK_ZERO_LO, invT, m) == dz && sk_d(SK_ZERO_HI, invT, m) == dz);
    if (maybe_below || check_zero) {  // uniform across the block
      const Extremes x =
          key_extremes(ptr, V, SK_NEG_LO, SK_ZERO_LO, SK_ZERO_HI, invT, m, L.red, rs);
      if (maybe_below) {
        below_top = x.below_max;
        below_mass = exp_det(sk_d(below_top, invT, m)) > 0.0f;
      }
      if (check_zero) {
        if (x.ze_min == x.ze_max) bm.zrep = bm.zlo = x.zkey_min;  // consumers read the
        else ok = false;                                            // group's p at its lo key
      }
    }
    if (!ok) {  // uniform across the block
      bm.anchored = true;
      bm.lo = kmax > (uint32_t)(SK_NB - 2) ? kmax - (uint32_t)(SK_NB - 2) : 0u;
      below_lo = bm.lo;
      below_mass = false;
      __syncthreads();
      for (int b = tid; b < SK_NB; b += NT) hist[b] = 0u;
      __syncthreads();
      restream_anchored<NT>(ptr, V, bm, hist);
      __syncthreads();
      if (bm.lo > 0 && hist[0] != 0 && exp_det(sk_d(bm.lo - 1, invT, m)) > 0.0f) {
        below_top = key_extremes(ptr, V, bm.lo, 1u, 0u, invT, m, L.red, rs).below_max;
        below_mass = exp_det(sk_d(below_top, invT, m)) > 0.0f;
      }
    }
    if (below_mass) rflags |= kRowBelowWindow;
  }
  const int bmax = bm.bin(kmax);
  auto e_of_bin = [&](int b) -> float { return exp_det(sk_d(bm.key_rep(b), invT, m)); };

  // ---- 3. exact normaliser: sum c * fixed62(e) as sum c * lo32 + 2^32 sum c * hi32
  // (sum c <= V < 2^31 keeps both below 2^63). Thread t reads bins bmax - t - j*NT;
  // each wave queues its occupied bins as (bin << 18 | count) in LDS and
  // evaluates them 128 at a time, two independent exp evaluations per lane
  // (sparse stretches of the window cost no idle lanes). The top SK_ETOP bins'
  // exp values stay in etop.
  float zf;
  uint32_t pre_all = 0;  // equal codes before the drafted token (when has_g)
  {
    uint64_t slo = 0, shi = 0;
    uint32_t* const q = L.zq[tid / kWave];
    uint32_t qn = 0;  // wave-uniform
    auto zterm2 = [&](uint32_t e0, uint32_t e1) {
      const uint32_t c0 = e0 & 0x3FFFFu, c1 = e1 & 0x3FFFFu;
      const int b0 = (int)(e0 >> 18), b1 = (int)(e1 >> 18);
      const float x0 = exp_det_sel(sk_d(bm.key_rep_sel(b0), invT, m));
      const float x1 = exp_det_sel(sk_d(bm.key_rep_sel(b1), invT, m));
      if (c0 != 0 && bmax - b0 < SK_ETOP) L.etop[bmax - b0] = x0;
      if (c1 != 0 && bmax - b1 < SK_ETOP) L.etop[bmax - b1] = x1;
      const uint64_t f0 = fixed62(x0), f1 = fixed62(x1);
      slo += (uint64_t)c0 * (uint32_t)f0 + (uint64_t)c1 * (uint32_t)f1;
      shi += (uint64_t)c0 * (uint32_t)(f0 >> 32) + (uint64_t)c1 * (uint32_t)(f1 >> 32);
    };
    const int nround = bmax >= 1 ? (bmax - 1) / NT + 1 : 0;
    for (int j0 = 0; j0 < nround; j0 += 4) {
      uint32_t cc[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int b = bmax - tid - NT * (j0 + u);
        cc[u] = b >= 1 ? hist[b] : 0u;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int b = bmax - tid - NT * (j0 + u);
        const uint64_t mk = __ballot(cc[u] != 0);
        const uint32_t below = __builtin_amdgcn_mbcnt_hi(
            (uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, 0u));
        if (cc[u] != 0) q[qn + below] = ((uint32_t)b << 18) | cc[u];
        qn += (uint32_t)__popcll(mk);
        if (qn >= 2 * kWave) {  // uniform
          const uint32_t e0 = q[qn - 2 * kWave + lane], e1 = q[qn - kWave + lane];
          qn -= 2 * kWave;
          zterm2(e0, e1);
        }
      }
    }
    if (qn > 0) {  // uniform: the rest, under 128 entries (0: no bin)
      const uint32_t e0 = (uint32_t)lane < qn ? q[lane] : 0u;
      const uint32_t e1 = (uint32_t)lane + kWave < qn ? q[lane + kWave] : 0u;
      zterm2(e0, e1);
    }
    const Red4 zr = blk_red<kOpSum64, kOpSum64, kOpSum32>(slo, shi, pre, 0, L.red, rs);
    pre_all = (uint32_t)zr.v[2];
    U128 z = u128_add(U128{zr.v[0], 0}, U128{zr.v[1] << 32, zr.v[1] >> 32});
    if (below_mass) z = u128_add(z, below_sum(ptr, V, below_lo, invT, m, 1.0f, L.red, rs));
    zf = rn32_u128(z);  // every thread, same value
  }
  // e / zf as fl32(fl64(e) * fl64(1 / zf)): the correctly rounded quotient
  // for fp32 operands (same argument as for x / T above)
  const double invz = 1.0 / (double)zf;
  auto p_of_bin = [&](int b) -> float {
    if (b < 1) return 0.0f;
    const int i = bmax - b;
    return (float)((double)(i < SK_ETOP ? L.etop[i] : e_of_bin(b)) * invz);
  };

  // ---- 4. top-k threshold: rounds of one bin per thread, descending from bmax
  int klo_bin = 1;
  bool k_cut = false;  // top-k dropped something
  if (a.use_k) {
    uint32_t before = 0;
    int kb = -1;
    for (int top = bmax; top >= 1; top -= NT) {
      const int b = top - tid;
      const uint32_t c = b >= 1 ? hist[b] : 0u;
      uint32_t tot;
      const uint32_t incl = blk_incl_u32(c, L.red, rs, &tot);
      const bool hit = c != 0 && before + incl >= (uint32_t)a.top_k;
      const uint32_t th = blk_min_u32(hit ? (uint32_t)tid : 0xFFFFFFFFu, L.red, rs);
      if (th != 0xFFFFFFFFu) { kb = top - (int)th; break; }
      before += tot;
    }
    if (kb < 0) {
      // the k-th largest lies in bin 0: below the anchored window, or p == 0
      if (below_mass) rflags |= kRowUnsupported;
      kb = 1;
    } else {
      k_cut = true;
    }
    // lower occupied bins of equal probability are ties at the k-th: kept
    if (tid < kWave) {  // wave 0; rarely more than one step
      const float p_kth = p_of_bin(kb);
      int lowb = kb;
      for (;;) {
        int nxt = 0;
        for (int b0 = lowb - 1; b0 >= 1; b0 -= kWave) {
          const int bb = b0 - lane;
          const uint64_t mm = __ballot(bb >= 1 && hist[bb] != 0);
          if (mm) { nxt = b0 - (__ffsll((unsigned long long)mm) - 1); break; }
        }
        if (nxt < 1 || p_of_bin(nxt) != p_kth) break;
        lowb = nxt;
      }
      if (tid == 0) L.i32[0] = lowb;
    }
    __syncthreads();
    klo_bin = L.i32[0];
    // ties at the k-th that continue below the window cannot be ordered here
    if (k_cut && below_mass && exp_det(sk_d(below_top, invT, m)) / zf == p_of_bin(kb))
      rflags |= kRowUnsupported;
  }

  // ---- 5. top-p boundary, its tie group and the kept count inside it
  int glo_b = klo_bin, ghi_b = klo_bin - 1, rstar = 0, gcount = 0;
  bool has_group = false;
  uint64_t kept_mass = 0;
  if (a.use_p) {
    const float tp = a.top_p;
    uint64_t S = 0;
    int bb = -1;
    float pb = 0.0f;
    int gtop0 = 0, gbot0 = 0;
    uint32_t above0 = 0, gcnt0 = 0;
    // Wave 0 walks the top SK_PW bins first, in chunks of 256: lane l holds bins
    // top - 4l - j (j = 0..3) of a chunk, sums them in order, one wave scan gives
    // every lane the mass above its bins, and every bin's keep test follows with
    // no further dependence. A nucleus of a few hundred values ends here in one
    // or two scans, and the other blocks on the CU keep their issue slots. Past
    // them the block takes over in rounds of NT bins.
    constexpr int PJ = 4;  // bins per lane and chunk (more spills at this register budget)
    static_assert(SK_PW % (PJ * kWave) == 0, "whole chunks");
    if (tid < kWave) {
      uint64_t Sw = 0;
      int fb = -1;
      uint64_t sb0 = 0;
      int g0 = 0, g1 = 0;
      uint32_t ab = 0, gc = 0;
      for (int top = bmax; top >= klo_bin && top > bmax - SK_PW; top -= PJ * kWave) {
        uint32_t c[PJ];
        float p[PJ];
        uint64_t f[PJ];
        uint64_t run = 0;
#pragma unroll
        for (int j = 0; j < PJ; ++j) {
          const int b = top - PJ * lane - j;
          c[j] = b >= klo_bin ? hist[b] : 0u;
        }
#pragma unroll
        for (int j = 0; j < PJ; ++j) {
          const int b = top - PJ * lane - j;
          p[j] = c[j] ? p_of_bin(b) : 0.0f;
          f[j] = (uint64_t)c[j] * fixed62(p[j]);
          run += f[j];
        }
        const uint64_t incl = wave_incl_scan_u64(run, lane);
        uint32_t fmask = 0;
        {
          uint64_t acc = Sw + incl - run;  // mass above this lane's bins
#pragma unroll
          for (int j = 0; j < PJ; ++j) {
            acc += f[j];
            const bool fail = c[j] != 0 && !((rn32_u64(acc) - p[j]) < tp);
            fmask |= (fail ? 1u : 0u) << j;
          }
        }
        const uint64_t fm = __ballot(fmask != 0);
        if (fm) {  // the boundary bin is in this chunk (uniform)
          const int tf = __ffsll((unsigned long long)fm) - 1;
          const int jf = __ffs((int)rdlane(fmask, tf)) - 1;
          fb = top - PJ * tf - jf;
          const float pbw = p_of_bin(fb);
          uint64_t acc = Sw + incl - run, exf = 0;
          uint32_t gmax = 0, gmin = 0xFFFFFFFFu, a1 = 0, a2 = 0;
#pragma unroll
          for (int j = 0; j < PJ; ++j) {
            const int b = top - PJ * lane - j;
            if (j == jf) exf = acc;  // mass before the boundary bin (on lane tf)
            acc += f[j];
            const bool in_g = c[j] != 0 && p[j] == pbw;
            gmax = in_g ? max(gmax, (uint32_t)b) : gmax;
            gmin = in_g ? min(gmin, (uint32_t)b) : gmin;
            a1 += in_g && b > fb ? c[j] : 0u;
            a2 += in_g ? c[j] : 0u;
          }
          sb0 = ((uint64_t)rdlane((uint32_t)(exf >> 32), tf) << 32) | rdlane((uint32_t)exf, tf);
          g0 = (int)wave_max_u32(gmax);
          g1 = (int)~wave_max_u32(~gmin);
          ab = wave_sum_u32(a1);
          gc = wave_sum_u32(a2);
          break;
        }
        Sw += ((uint64_t)rdlane((uint32_t)(incl >> 32), kWave - 1) << 32) |
              rdlane((uint32_t)incl, kWave - 1);
      }
      if (tid == 0) {
        L.pw[0] = fb; L.pw[1] = g0; L.pw[2] = g1; L.pw[3] = (int32_t)ab;
        L.pw[4] = (int32_t)gc;
        L.x64[0] = fb >= 0 ? sb0 : Sw;
      }
    }
    __syncthreads();
    if (L.pw[0] >= 0) {  // uniform
      bb = L.pw[0];
      pb = p_of_bin(bb);
      gtop0 = L.pw[1]; gbot0 = L.pw[2];
      above0 = (uint32_t)L.pw[3]; gcnt0 = (uint32_t)L.pw[4];
    } else {
      S = L.x64[0];
    }
    for (int top = bmax - SK_PW; bb < 0 && top >= klo_bin; top -= NT) {
      const int b = top - tid;
      const uint32_t c = b >= klo_bin ? hist[b] : 0u;
      const float p = c ? p_of_bin(b) : 0.0f;
      const uint64_t mi = (uint64_t)c * fixed62(p);
      uint64_t tot;
      const uint64_t incl = blk_incl_u64(mi, L.red, rs, &tot);
      // keep fails from the boundary bin on (cum grows, p shrinks, fp32 ops monotone)
      const bool fail = c != 0 && !((rn32_u64(S + incl) - p) < tp);
      const uint32_t tf = blk_min_u32(fail ? (uint32_t)tid : 0xFFFFFFFFu, L.red, rs);
      if (tf != 0xFFFFFFFFu) {  // the boundary bin is in this round (uniform)
        bb = top - (int)tf;
        pb = p_of_bin(bb);
        if (tid == (int)tf) L.x64[0] = S + incl - mi;  // mass before the boundary bin
        // group bins of this round: occupied, of the boundary's probability
        const bool in_g = c != 0 && p == pb;
        const Red4 gr = blk_red<kOpMax32, kOpMin32, kOpSum32, kOpSum32>(
            in_g ? (uint32_t)b : 0u, in_g ? (uint32_t)b : 0xFFFFFFFFu,
            in_g && b > bb ? c : 0u, in_g ? c : 0u, L.red, rs);
        gtop0 = (int)gr.v[0];
        gbot0 = (int)gr.v[1];
        above0 = (uint32_t)gr.v[2];
        gcnt0 = (uint32_t)gr.v[3];
        break;
      }
      S += tot;
    }
    if (bb >= 1) {  // uniform
      if (tid < kWave) {  // wave 0: the group beyond this round (rare), then the kept count
        const uint64_t Sb0 = L.x64[0];  // written before the group reduction's barrier
        const uint32_t cb = hist[bb];
        int gtop = gtop0, gbot = gbot0;
        uint32_t above = above0, gcnt = gcnt0;
        {  // occupied bins above the round's group bins: the first one differs unless
           // the group continues into earlier rounds
          for (;;) {
            int nxt = bmax + 1;
            for (int b0 = gtop + 1; b0 <= bmax; b0 += kWave) {
              const int b2 = b0 + lane;
              const uint64_t mm = __ballot(b2 <= bmax && hist[b2] != 0);
              if (mm) { nxt = b0 + (__ffsll((unsigned long long)mm) - 1); break; }
            }
            if (nxt > bmax || p_of_bin(nxt) != pb) break;
            gtop = nxt;
            above += hist[nxt];
            gcnt += hist[nxt];
          }
        }
        {  // ... or below them, into later rounds
          for (;;) {
            int nxt = 0;
            for (int b0 = gbot - 1; b0 >= klo_bin; b0 -= kWave) {
              const int b2 = b0 - lane;
              const uint64_t mm = __ballot(b2 >= klo_bin && hist[b2] != 0);
              if (mm) { nxt = b0 - (__ffsll((unsigned long long)mm) - 1); break; }
            }
            if (nxt < klo_bin || p_of_bin(nxt) != pb) break;
            gbot = nxt;
            gcnt += hist[nxt];
          }
        }
        // members kept in the boundary bin: keep_r = rn32(Sb0 + (r+1) P) - pb < tp
        // holds for a prefix of r and fails at r = cb - 1. 64-way search: the
        // answer stays in [lo_r, hi_r], members below lo_r pass, hi_r fails.
        const uint64_t P = fixed62(pb);
        uint32_t lo_r = 0, hi_r = cb - 1;
        while (lo_r < hi_r) {
          const uint32_t step = (hi_r - lo_r + kWave - 1) / kWave;
          const uint32_t cand = lo_r + (uint32_t)lane * step;
          const bool keep = cand < hi_r && (rn32_u64(Sb0 + (uint64_t)(cand + 1) * P) - pb) < tp;
          const int nk = __popcll(__ballot(keep));  // keeping candidates form a prefix
          if (nk == 0) break;                        // lo_r itself fails
          const uint32_t last = lo_r + (uint32_t)(nk - 1) * step;
          lo_r = last + 1;
          hi_r = min(hi_r, last + step);
        }
        uint32_t rr = lo_r;
        if (Sb0 == (uint64_t)above * P && above == 0 && rr == 0) rr = 1;  // keep[..., 0] = True
        if (tid == 0) {
          L.i32[7] = gtop; L.i32[8] = gbot; L.i32[9] = (int32_t)(above + rr);
          L.i32[10] = (int32_t)gcnt;
          L.x64[1] = Sb0 + (uint64_t)rr * P;
        }
      }
      __syncthreads();
      ghi_b = L.i32[7];
      glo_b = L.i32[8];
      rstar = L.i32[9];
      gcount = L.i32[10];
      kept_mass = L.x64[1];
      klo_bin = glo_b;
      has_group = true;
      // a tie group that continues below the window cannot be ordered here
      if (below_mass && exp_det(sk_d(below_top, invT, m)) / zf == pb) rflags |= kRowUnsupported;
    } else {
      kept_mass = S;
      if (below_mass && !k_cut) rflags |= kRowUnsupported;  // nucleus reaches below the window
    }
  }
  // keys below the window are kept only when neither filter cut inside it
  const bool keep_below = !k_cut && !has_group;
  if (!a.use_p) {  // no nucleus: the kept mass is every bin from klo_bin up
    uint64_t acc = 0;
    for (int b = bmax - tid; b >= klo_bin; b -= NT) {
      const uint32_t c = hist[b];
      if (c) acc += (uint64_t)c * fixed62(p_of_bin(b));
    }
    kept_mass = blk_sum_u64(acc, L.red, rs);
    if (below_mass && keep_below)
      kept_mass += below_sum(ptr, V, below_lo, invT, m, zf, L.red, rs).lo;
  }
  const float totf = fmaxf(rn32_u64(kept_mass), 1e-12f);
  const double invtot = 1.0 / (double)totf;
  const int32_t klo = keep_below ? 0 : (int32_t)bm.key_lo(klo_bin);
  const int32_t glo = has_group ? (int32_t)bm.key_lo(glo_b) : klo;
  const int32_t ghi = has_group ? (int32_t)bm.key_hi(ghi_b) : klo - 1;

  // ---- 6. table of final probabilities for the top keys
  const int32_t tbl_lo = max(klo, (int32_t)kmax - (kTbl - 1));
  const int32_t ntbl = (int32_t)kmax - tbl_lo + 1;
  for (int t = tid; t < ntbl; t += NT) {
    const uint32_t kk = kmax - (uint32_t)t;
    const int b = bm.bin(kk);
    float v;
    if (b >= 1) {
      v = hist[b] != 0 ? (float)((double)p_of_bin(b) * invtot) : 0.0f;
    } else {  // below the window: exact per key (zero in the fixed window)
      v = exp_det(sk_d(kk, invT, m)) / zf / totf;
    }
    st_f32(tbl_out + t, v, FUSED);
  }

  // ---- 7. probability of the drafted token. Inside a partial tie group it
  // depends on the token's member rank (members with lower ids): the rank
  // kernel counts it, spread over many blocks, and sets pgather.
  float pg = 0.0f;
  if (has_g) {
    const int32_t kk = (int32_t)key_of_code16(cg);
    bool kept = kk >= klo;
    if (kept && kk >= glo && kk <= ghi) {
      if (rstar <= 0) {
        kept = false;
      } else if (rstar < gcount) {
        rflags |= kRowGatherTie;
        // a single-value group whose bin holds that value alone: its member rank
        // is the count of equal codes before the token; otherwise the draw ranks it
        const bool one = glo == ghi && bin_g >= 1 && bin_g <= 2 * SK_WIN + 1 && bin_g != SK_BIN_ZERO;
        if (one) kept = (int32_t)(snap + pre_all) < rstar;
        else { kept = false; rflags |= kRowRank; }
      }
    }
    if (kept) pg = exp_det(sk_d((uint32_t)kk, invT, m)) / zf / totf;
  }
  if (tid == 0) {
    RowStat st;
    st.m = m;
    st.zf = zf;
    st.totf = totf;
    st.pgather = pg;
    st.kmax = (int32_t)kmax;
    st.klo = klo;
    st.glo = glo;
    st.ghi = ghi;
    st.rstar = rstar;
    st.gcount = gcount;
    st.mass = kept_mass;
    st.flags = rflags;
    st.ntbl = ntbl;
    st.argmax = -1;
    st_rowstat(st_out, st, FUSED);
  }
  return row;
}

// ---------------------------------------------------------------- fused verify
// Row statistics and the draw in one launch, for bf16 logits at one k per batch
// row (2k + 1 <= 64 rows). Blocks [0, nrow) are row blocks, taking rows in
// batch-row order; each publishes its row's statistics and table with
// device-coherent stores, waits for them, and counts the row in on its batch
// row (job_cnt). Blocks from nrow_pad on are draw blocks (draw16_body on
// SM_NT threads; the block's other waves retire at once, and a barrier waits
// only for the waves that have not): each waits until its batch row's 2k + 1
// rows are in, then draws. So the draw of the batch rows whose rows finish
// first overlaps the row statistics of the others.
//
// The wait ends: row blocks never wait, and on every XCD all row blocks are
// dispatched before any draw block (workgroups are dispatched in index order),
// so a draw block never holds a slot a row block still needs. It is bounded all
// the same: after wait_ticks of the 100 MHz real-time counter (by default 20 ms,
// some 250 times the whole launch) the block gives up. A block that gives up
// flags its batch row (SDX_FLAG_WORKSPACE, y -1; n_acc unspecified) and never
// counts in on the draw counter, so no block of that batch row draws. Its row
// arrivals may still land after it left, so the header's counters can no longer
// be trusted: the block overwrites the magic word with kWsDirty, and every later
// call on the workspace flags its rows until sdx_workspace_init runs again.
constexpr uint64_t kFusedWaitTicks = 2000000;

struct FusedArgs {
  RowStatArgs rs;
  int64_t nrow;      // row blocks
  int64_t nrow_pad;  // the first draw block (a multiple of 8: block % 8 keeps the XCD)
  Draw16Args<SDX_BF16> d;
  uint32_t need;     // rows per batch row (per-row k: 2 k_b + 1, from acc.cu_k)
  const int32_t* rowjob;  // per-row k: each row's batch row (-1: offsets inconsistent)
  uint64_t wait_ticks;    // a draw block's bound on its wait for the rows (100 MHz ticks)
};

// Host side (sdx_rowstream.hip): the blocks of a row-statistics launch over
// `rows` rows (whole and split rows, set in `a`), and the fused kernels' wait
// bound (SDX_VERIFY_WAIT_TICKS or kFusedWaitTicks).
int64_t rowstream_setup(RowStatArgs& a, int64_t rows);
uint64_t fused_wait_ticks();

}  // namespace sdx
