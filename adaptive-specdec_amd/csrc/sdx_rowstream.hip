// Row statistics for bf16 logits, streaming: the fused to_probs of
// specdec/sampling.py:34-67 reduced to what the accept test and the final
// draw need, with every logit read from HBM once and nothing kept resident.
//
// The probability of a token depends only on its bf16 value, so the row is
// reduced to counts per value in an LDS histogram. The histogram uses a fixed
// value window, not one anchored at the row maximum, so the LDS atomics start
// as soon as the first 16-byte loads land and overlap the rest of the row:
//   bin 0               x <= -2^18, -inf, -NaN       (exp_det == 0, checked)
//   bins 1..6400        -2^18 < x <= -2^-32          (one bin per bf16 value)
//   bin 6401            |x| < 2^-32, +-0, denormals  (all share exp(-m), checked)
//   bins 6402..12801    2^-32 <= x < 2^18            (one bin per bf16 value)
//   bin 12802           x >= 2^18, +inf, +NaN        (row leaves the fixed window)
// The bins are in value order. 52 KiB of LDS per 512-thread workgroup fits
// three workgroups per CU, so the 576 rows of a B=64, k=4 verify all stream at
// once and share HBM evenly; the row maximum is tracked in registers.
//
// After the histogram, the whole block works on it: the exact fixed-point
// normaliser over occupied bins (the top bins' exp values kept in LDS); the
// top-k / top-p walk down from the maximum in rounds of one bin per thread,
// with a block scan of exact cumulative mass and the reference's fp32 keep
// test `cum - p < top_p`; the boundary tie group (occupied bins of equal
// probability) and the number of its members kept, lowest ids first. The
// index cut inside that group is left to the consumers, which count group
// members in id order as they stream the rows they need; only a drafted token
// inside its row's group is ranked here, by a rescan of the row prefix.
//
// Elements in bin 0 that carry mass (huge negative logits at huge
// temperatures) are summed by one more pass. Rows the fixed window cannot
// represent (values >= 2^18, a maximum among the merged tiny values, tiny
// values of different probability) are re-streamed into a histogram anchored
// at the row maximum (keys [kmax - 12802, kmax]). A decision that needs the
// order of elements below either window marks the row unsupported.
#include "sdx_launch.hpp"

namespace sdx {

constexpr int SK_NT = 512;
constexpr int SK_NW = SK_NT / kWave;
constexpr uint32_t SK_NEG_LO = 0x3780u;   // key of -(2^18 - ulp)
constexpr uint32_t SK_ZERO_LO = 0x5080u;  // first key of the merged tiny-magnitude bin
constexpr uint32_t SK_ZERO_HI = 0xAF7Fu;
constexpr uint32_t SK_POS_LO = 0xAF80u;   // key of 2^-32
constexpr int SK_WIN = 6400;
constexpr int SK_BIN_ZERO = 6401;
constexpr int SK_BIN_EXC = 12802;
constexpr int SK_TRASH = 12803;           // padding ids past the row end
constexpr int SK_NB = 12804;

__device__ __forceinline__ int sk_bin_of_key(uint32_t k) {
  const uint32_t c1 = min(k > 0x377Fu ? k - 0x377Fu : 0u, 6401u);
  const uint32_t c2 = min(k > 0xAF7Fu ? k - 0xAF7Fu : 0u, 6401u);
  return (int)(c1 + c2);
}
// Two packed keys -> two packed bins (v_pk_sub_u16 with clamp, v_pk_min_u16, v_pk_add_u16).
typedef unsigned short us2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t sk_bins2(uint32_t keys2) {
  const us2 k = __builtin_bit_cast(us2, keys2);
  const us2 c1 = __builtin_elementwise_min(__builtin_elementwise_sub_sat(k, (us2){0x377F, 0x377F}),
                                           (us2){6401, 6401});
  const us2 c2 = __builtin_elementwise_min(__builtin_elementwise_sub_sat(k, (us2){0xAF7F, 0xAF7F}),
                                           (us2){6401, 6401});
  return __builtin_bit_cast(uint32_t, c1 + c2);
}
__device__ __forceinline__ uint32_t max2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(us2, a),
                                                                __builtin_bit_cast(us2, b)));
}

// Bin <-> key maps of the two window kinds. Fixed: as tabled above. Anchored:
// bin b >= 1 holds key lo + b - 1, bin 0 the keys below lo.
struct BinMap {
  bool anchored;
  uint32_t lo;
  uint32_t zrep;  // fixed window: a key of the merged tiny bin standing for all of it
  __device__ uint32_t key_lo(int b) const {
    if (anchored) return b <= 0 ? 0u : lo + (uint32_t)(b - 1);
    if (b <= 0) return 0u;
    if (b <= SK_WIN) return SK_NEG_LO + (uint32_t)(b - 1);
    if (b == SK_BIN_ZERO) return SK_ZERO_LO;
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
  __device__ int bin(uint32_t k) const {
    if (anchored) return k < lo ? 0 : (int)(k - lo) + 1;
    return sk_bin_of_key(k);
  }
};

__device__ __forceinline__ float sk_d(uint32_t key, float T, float m) {
  return decode16<SDX_BF16>(code_of_key16(key)) / T - m;
}

// ---------------------------------------------------------------- block helpers
// All of them contain barriers: call them from every thread of the block.
struct SkSmem {
  uint64_t u64[SK_NW];
  uint32_t u32[2 * SK_NW];
};
__device__ __forceinline__ uint64_t blk_incl_u64(uint64_t v, SkSmem& sm, uint64_t* total) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const uint64_t incl = wave_incl_scan_u64(v, lane);
  if (lane == kWave - 1) sm.u64[w] = incl;
  __syncthreads();
  uint64_t off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < SK_NW; ++i) {
    const uint64_t x = sm.u64[i];
    off += i < w ? x : 0ull;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return off + incl;
}
__device__ __forceinline__ uint32_t blk_incl_u32(uint32_t v, SkSmem& sm, uint32_t* total) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const uint32_t incl = wave_incl_scan_u32(v, lane);
  if (lane == kWave - 1) sm.u32[w] = incl;
  __syncthreads();
  uint32_t off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < SK_NW; ++i) {
    const uint32_t x = sm.u32[i];
    off += i < w ? x : 0u;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return off + incl;
}
__device__ __forceinline__ uint64_t blk_sum_u64(uint64_t v, SkSmem& sm) {
  uint64_t t;
  blk_incl_u64(v, sm, &t);
  return t;
}
__device__ __forceinline__ uint32_t blk_sum_u32(uint32_t v, SkSmem& sm) {
  uint32_t t;
  blk_incl_u32(v, sm, &t);
  return t;
}
__device__ __forceinline__ uint32_t blk_min_u32(uint32_t v, SkSmem& sm) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, (uint32_t)__shfl_xor((int)v, o, kWave));
  if (lane == 0) sm.u32[SK_NW + w] = v;
  __syncthreads();
  uint32_t r = 0xFFFFFFFFu;
#pragma unroll
  for (int i = 0; i < SK_NW; ++i) r = min(r, sm.u32[SK_NW + i]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ uint32_t blk_max_u32(uint32_t v, SkSmem& sm) {
  return ~blk_min_u32(~v, sm);
}

// Whole block: counts the row's elements into `hist` under an anchored map.
__device__ void restream_anchored(const uint16_t* __restrict__ ptr, int64_t V, const BinMap& bm,
                                  uint32_t* hist) {
  for (int64_t e0 = (int64_t)threadIdx.x * 8; e0 < V; e0 += (int64_t)SK_NT * 8) {
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
__device__ Extremes key_extremes(const uint16_t* __restrict__ ptr, int64_t V, uint32_t lo,
                                 uint32_t zlo, uint32_t zhi, float T, float m, SkSmem& sm) {
  uint32_t b = 0, z0 = 0xFFFFu, e0 = 0xFFFFFFFFu, e1 = 0;
  for (int64_t i = threadIdx.x; i < V; i += SK_NT) {
    const uint32_t k = key_of_code16(ptr[i]);
    if (k < lo) b = max(b, k);
    if (k >= zlo && k <= zhi) {
      const uint32_t e = __float_as_uint(exp_det(sk_d(k, T, m)));
      z0 = min(z0, k);
      e0 = min(e0, e);
      e1 = max(e1, e);
    }
  }
  Extremes x;
  x.below_max = blk_max_u32(b, sm);
  x.zkey_min = blk_min_u32(z0, sm);
  x.ze_min = blk_min_u32(e0, sm);
  x.ze_max = blk_max_u32(e1, sm);
  return x;
}
// Whole block: sum over elements with key < lo of fixed62(exp_det(x/T - m) / div),
// exact in 128 bits (split as sum lo32 + 2^32 sum hi32, each below 2^63).
__device__ U128 below_sum(const uint16_t* __restrict__ ptr, int64_t V, uint32_t lo, float T,
                          float m, float div, SkSmem& sm) {
  uint64_t slo = 0, shi = 0;
  for (int64_t i = threadIdx.x; i < V; i += SK_NT) {
    const uint32_t k = key_of_code16(ptr[i]);
    if (k < lo) {
      const float e = exp_det(sk_d(k, T, m));
      const uint64_t f = fixed62(div == 1.0f ? e : e / div);
      slo += (uint32_t)f;
      shi += (uint32_t)(f >> 32);
    }
  }
  slo = blk_sum_u64(slo, sm);
  shi = blk_sum_u64(shi, sm);
  return u128_add(U128{slo, 0}, U128{shi << 32, shi >> 32});
}

__global__ void __launch_bounds__(SK_NT) __attribute__((amdgpu_waves_per_eu(6)))
rowstream_bf16_kernel(RowStatArgs a) {
  __shared__ uint32_t hist[SK_NB];
  __shared__ float etop[SK_NT];  // exp values of the top SK_NT bins (0 if unoccupied)
  __shared__ SkSmem sm;
  __shared__ int32_t s_i32[12];
  __shared__ uint64_t s_x64[2];
  __shared__ float s_f[2];

  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int64_t row = blockIdx.x;
  const int g = row < a.nrows[0] ? 0 : 1;
  const int64_t r = g ? row - a.nrows[0] : row;
  const uint16_t* __restrict__ ptr = a.base[g] + r * a.ld[g];
  int64_t gid = -1;
  if (a.ids) {
    if (g == 0) {
      const int64_t b = r / (a.k + 1), i = r % (a.k + 1);
      if (i < a.k) gid = a.ids[b * a.k + i];
    } else {
      gid = a.ids[r];
    }
  }
  const int64_t V = a.V;
  RowStat* st_out = a.stats + row;
  float* tbl_out = a.tables + row * kTbl;
  if (tid == 0 && row < a.nzero) a.zero[row] = 0u;
  if (tid == 0 && a.rank_acc) a.rank_acc[row] = 0ull;

  for (int b = tid; b < SK_NB; b += SK_NT) hist[b] = 0u;
  __syncthreads();

  // ---- 1. stream the row: 16-byte loads, packed keys -> packed bins, LDS atomics
  uint32_t kmx2 = 0;  // packed running maximum of keys
  {
    constexpr int U = 4;  // 16-byte loads in flight per lane
    const int64_t stride = (int64_t)SK_NT * 8;
    for (int64_t i0 = (int64_t)tid * 8; i0 < V; i0 += stride * U) {
      uint4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t e0 = i0 + u * stride;
        if (e0 + 8 <= V) {
          v[u] = *reinterpret_cast<const uint4*>(ptr + e0);
        } else if (e0 < V) {  // the row's last partial group, element by element
          uint32_t w[4] = {0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu};
#pragma unroll
          for (int t = 0; t < 8; ++t)
            if (e0 + t < V)
              w[t >> 1] = (w[t >> 1] & ~(0xFFFFu << (16 * (t & 1)))) |
                          ((uint32_t)ptr[e0 + t] << (16 * (t & 1)));
          v[u] = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t e0 = i0 + u * stride;
        if (e0 < V) {
          const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
          uint32_t bins[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const uint32_t k2 = keys2_of_codes2(w[t]);  // padding code 0xFFFF -> key 0
            kmx2 = max2(kmx2, k2);
            bins[t] = sk_bins2(k2);
          }
          if (e0 + 8 <= V) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              atomicAdd(&hist[bins[t] & 0xFFFFu], 1u);
              atomicAdd(&hist[bins[t] >> 16], 1u);
            }
          } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
              const uint32_t bb = (t & 1) ? (bins[t >> 1] >> 16) : (bins[t >> 1] & 0xFFFFu);
              atomicAdd(&hist[e0 + t < V ? bb : (uint32_t)SK_TRASH], 1u);
            }
          }
        }
      }
    }
  }
  // (the reduction's barriers also complete the histogram)
  const uint32_t kmax = blk_max_u32(max(kmx2 & 0xFFFFu, kmx2 >> 16), sm);

  if (kmax >= kPosInfKey<SDX_BF16> || kmax == 0) {  // +inf / NaN: flag, outputs unspecified
    if (tid == 0) {
      RowStat st = {};
      st.flags = kRowNonfinite;
      st.zf = 1.0f; st.totf = 1.0f; st.klo = 0x7FFFFFFF; st.glo = 1; st.ghi = 0; st.argmax = -1;
      *st_out = st;
    }
    return;
  }
  const float T = a.T;
  const float m = decode16<SDX_BF16>(code_of_key16(kmax)) / T;

  // ---- 2. fixed window valid for this row? else re-stream anchored at kmax.
  // Bin 0 ("below the window") may carry mass: then Z adds it by one more pass
  // and a decision that needs it marks the row unsupported. The quick checks
  // use the bins' edge keys; when they fail, one pass finds the actual extreme
  // keys (rare: huge negative logits at huge temperatures, tiny logits).
  BinMap bm{false, 0u, 0x8000u};
  uint32_t rflags = 0;
  uint32_t below_lo = SK_NEG_LO;  // keys below it are below the window
  bool below_mass = false;        // ... and some of them have exp_det > 0
  uint32_t below_top = 0;         // the largest key below the window
  {
    const int b0 = sk_bin_of_key(kmax);
    bool ok = b0 >= 1 && b0 != SK_BIN_EXC;
    const bool maybe_below = ok && hist[0] != 0 && exp_det(sk_d(SK_NEG_LO - 1, T, m)) > 0.0f;
    // the merged tiny bin needs one exp value for all its members: d equal at its
    // edges (fp32 division and subtraction are monotone), else checked per member
    const float dz = sk_d(0x8000u, T, m);
    const bool check_zero = ok && hist[SK_BIN_ZERO] != 0 &&
                            !(sk_d(SK_ZERO_LO, T, m) == dz && sk_d(SK_ZERO_HI, T, m) == dz);
    if (maybe_below || check_zero) {  // uniform across the block
      const Extremes x = key_extremes(ptr, V, SK_NEG_LO, SK_ZERO_LO, SK_ZERO_HI, T, m, sm);
      if (maybe_below) {
        below_top = x.below_max;
        below_mass = exp_det(sk_d(below_top, T, m)) > 0.0f;
      }
      if (check_zero) {
        if (x.ze_min == x.ze_max) bm.zrep = x.zkey_min;
        else ok = false;
      }
    }
    if (!ok) {  // uniform across the block
      bm.anchored = true;
      bm.lo = kmax > (uint32_t)(SK_NB - 2) ? kmax - (uint32_t)(SK_NB - 2) : 0u;
      below_lo = bm.lo;
      below_mass = false;
      __syncthreads();
      for (int b = tid; b < SK_NB; b += SK_NT) hist[b] = 0u;
      __syncthreads();
      restream_anchored(ptr, V, bm, hist);
      __syncthreads();
      if (bm.lo > 0 && hist[0] != 0 && exp_det(sk_d(bm.lo - 1, T, m)) > 0.0f) {
        below_top = key_extremes(ptr, V, bm.lo, 1u, 0u, T, m, sm).below_max;
        below_mass = exp_det(sk_d(below_top, T, m)) > 0.0f;
      }
    }
    if (below_mass) rflags |= kRowBelowWindow;
  }
  const int bmax = bm.bin(kmax);
  auto e_of_bin = [&](int b) -> float { return exp_det(sk_d(bm.key_rep(b), T, m)); };

  // ---- 3. exact normaliser: sum c * fixed62(e) as sum c * lo32 + 2^32 sum c * hi32
  // (sum c <= V < 2^31 keeps both below 2^63). Thread t takes bins bmax - t - j*SK_NT,
  // so the first round covers the top bins and leaves their exp values in etop.
  {
    uint64_t slo = 0, shi = 0;
    for (int b = bmax - tid, j = 0; b >= 1; b -= SK_NT, ++j) {
      const uint32_t c = hist[b];
      const float e = c ? e_of_bin(b) : 0.0f;
      if (j == 0) etop[tid] = e;
      if (c) {
        const uint64_t f = fixed62(e);
        slo += (uint64_t)c * (uint32_t)f;
        shi += (uint64_t)c * (uint32_t)(f >> 32);
      }
    }
    if (bmax - tid < 1) etop[tid] = 0.0f;
    slo = blk_sum_u64(slo, sm);
    shi = blk_sum_u64(shi, sm);
    U128 z = u128_add(U128{slo, 0}, U128{shi << 32, shi >> 32});
    if (below_mass) z = u128_add(z, below_sum(ptr, V, below_lo, T, m, 1.0f, sm));
    if (tid == 0) s_f[0] = rn32_u128(z);
    __syncthreads();
  }
  const float zf = s_f[0];
  auto p_of_bin = [&](int b) -> float {
    if (b < 1) return 0.0f;
    const int i = bmax - b;
    return (i < SK_NT ? etop[i] : e_of_bin(b)) / zf;
  };

  // ---- 4. top-k threshold: rounds of one bin per thread, descending from bmax
  int klo_bin = 1;
  bool k_cut = false;  // top-k dropped something
  if (a.use_k) {
    uint32_t before = 0;
    int kb = -1;
    for (int top = bmax; top >= 1; top -= SK_NT) {
      const int b = top - tid;
      const uint32_t c = b >= 1 ? hist[b] : 0u;
      uint32_t tot;
      const uint32_t incl = blk_incl_u32(c, sm, &tot);
      const bool hit = c != 0 && before + incl >= (uint32_t)a.top_k;
      const uint32_t th = blk_min_u32(hit ? (uint32_t)tid : 0xFFFFFFFFu, sm);
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
      if (tid == 0) s_i32[0] = lowb;
    }
    __syncthreads();
    klo_bin = s_i32[0];
    __syncthreads();
    // ties at the k-th that continue below the window cannot be ordered here
    if (k_cut && below_mass && exp_det(sk_d(below_top, T, m)) / zf == p_of_bin(kb))
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
    for (int top = bmax; top >= klo_bin; top -= SK_NT) {
      const int b = top - tid;
      const uint32_t c = b >= klo_bin ? hist[b] : 0u;
      const float p = c ? p_of_bin(b) : 0.0f;
      const uint64_t mi = (uint64_t)c * fixed62(p);
      uint64_t tot;
      const uint64_t incl = blk_incl_u64(mi, sm, &tot);
      const bool fail = c != 0 && !((rn32_u64(S + incl) - p) < tp);
      const uint32_t tf = blk_min_u32(fail ? (uint32_t)tid : 0xFFFFFFFFu, sm);
      if (tf != 0xFFFFFFFFu) {  // the boundary bin is in this round
        if (tid == (int)tf) {
          s_x64[0] = S + incl - mi;  // mass before the boundary bin
          s_i32[1] = (int32_t)c;
          s_f[1] = p;
        }
        bb = top - (int)tf;
        __syncthreads();
        // group bins of this round: occupied, of the boundary's probability
        const bool in_g = c != 0 && p == s_f[1];
        const uint32_t gmax = blk_max_u32(in_g ? (uint32_t)b : 0u, sm);
        const uint32_t gmin = blk_min_u32(in_g ? (uint32_t)b : 0xFFFFFFFFu, sm);
        const uint32_t above = blk_sum_u32(in_g && b > bb ? c : 0u, sm);
        const uint32_t gsum = blk_sum_u32(in_g ? c : 0u, sm);
        if (tid == 0) {
          s_i32[2] = (int32_t)gmax; s_i32[3] = (int32_t)gmin;
          s_i32[4] = (int32_t)above; s_i32[5] = (int32_t)gsum;
          }
        break;
      }
      S += tot;
    }
    __syncthreads();
    if (bb >= 1) {
      const uint64_t Sb0 = s_x64[0];
      const uint32_t cb = (uint32_t)s_i32[1];
      const float pb = s_f[1];
      if (tid < kWave) {  // wave 0: the group beyond this round (rare), then the kept count
        int gtop = s_i32[2], gbot = s_i32[3];
        uint32_t above = (uint32_t)s_i32[4], gcnt = (uint32_t)s_i32[5];
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
          s_i32[7] = gtop; s_i32[8] = gbot; s_i32[9] = (int32_t)(above + rr);
          s_i32[10] = (int32_t)gcnt;
          s_x64[1] = Sb0 + (uint64_t)rr * P;
        }
      }
      __syncthreads();
      ghi_b = s_i32[7];
      glo_b = s_i32[8];
      rstar = s_i32[9];
      gcount = s_i32[10];
      kept_mass = s_x64[1];
      klo_bin = glo_b;
      has_group = true;
      // a tie group that continues below the window cannot be ordered here
      if (below_mass && exp_det(sk_d(below_top, T, m)) / zf == pb) rflags |= kRowUnsupported;
    } else {
      kept_mass = S;
      if (below_mass && !k_cut) rflags |= kRowUnsupported;  // nucleus reaches below the window
    }
  }
  // keys below the window are kept only when neither filter cut inside it
  const bool keep_below = !k_cut && !has_group;
  if (!a.use_p) {  // no nucleus: the kept mass is every bin from klo_bin up
    uint64_t acc = 0;
    for (int b = bmax - tid; b >= klo_bin; b -= SK_NT) {
      const uint32_t c = hist[b];
      if (c) acc += (uint64_t)c * fixed62(p_of_bin(b));
    }
    kept_mass = blk_sum_u64(acc, sm);
    if (below_mass && keep_below) kept_mass += below_sum(ptr, V, below_lo, T, m, zf, sm).lo;
  }
  const float totf = fmaxf(rn32_u64(kept_mass), 1e-12f);
  const int32_t klo = keep_below ? 0 : (int32_t)bm.key_lo(klo_bin);
  const int32_t glo = has_group ? (int32_t)bm.key_lo(glo_b) : klo;
  const int32_t ghi = has_group ? (int32_t)bm.key_hi(ghi_b) : klo - 1;

  // ---- 6. table of final probabilities for the top keys
  const int32_t tbl_lo = max(klo, (int32_t)kmax - (kTbl - 1));
  const int32_t ntbl = (int32_t)kmax - tbl_lo + 1;
  for (int t = tid; t < ntbl; t += SK_NT) {
    const uint32_t kk = kmax - (uint32_t)t;
    const int b = bm.bin(kk);
    float v;
    if (b >= 1) {
      v = hist[b] != 0 ? p_of_bin(b) / totf : 0.0f;
    } else {  // below the window: exact per key (zero in the fixed window)
      v = exp_det(sk_d(kk, T, m)) / zf / totf;
    }
    tbl_out[t] = v;
  }

  // ---- 7. probability of the drafted token. Inside a partial tie group it
  // depends on the token's member rank (members with lower ids): the rank
  // kernel counts it, spread over many blocks, and sets pgather.
  float pg = 0.0f;
  if (gid >= 0 && gid < V) {
    const int32_t kk = (int32_t)key_of_code16(ptr[gid]);
    bool kept = kk >= klo;
    if (kept && kk >= glo && kk <= ghi) {
      if (rstar <= 0) kept = false;
      else if (rstar < gcount) { kept = false; rflags |= kRowRank; }
    }
    if (kept) pg = exp_det(sk_d((uint32_t)kk, T, m)) / zf / totf;
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
    *st_out = st;
  }
}

hipError_t launch_rowstream_bf16(const RowStatArgs& a, int64_t rows, hipStream_t s) {
  hipLaunchKernelGGL(rowstream_bf16_kernel, dim3((unsigned)rows), dim3(SK_NT), 0, s, a);
  return hipGetLastError();
}

}  // namespace sdx
