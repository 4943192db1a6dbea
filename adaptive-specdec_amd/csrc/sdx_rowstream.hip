// Row statistics for bf16 logits, streaming: the fused to_probs of
// specdec/sampling.py:34-67 reduced to what the accept test and the final
// draw need, with every logit read from HBM exactly once and nothing kept
// resident.
//
// The probability of a token depends only on its bf16 value, so the row is
// reduced to counts per value. The histogram uses a fixed value window, not
// one anchored at the row maximum, so the LDS atomics start as soon as the
// first 16-byte loads land and overlap the rest of the row's traffic:
//   bin 0              x <= -2^21 and -inf           (exp_det == 0, checked)
//   bins 1..7808       -2^21 < x <= -2^-40           (one bin per bf16 value)
//   bin 7809           |x| < 2^-40, +-0, denormals   (all share exp(-m), checked)
//   bins 7810..15617   2^-40 <= x < 2^21             (one bin per bf16 value)
//   bin 15618          x >= 2^21, +inf, NaN          (row goes to the fallback)
// The bins are in value order. 62.5 KiB of LDS per 1024-thread workgroup
// leaves room for two workgroups per CU, so one row's normaliser / nucleus
// walk overlaps the other row's loads.
//
// After the histogram: the exact fixed-point normaliser over occupied bins,
// the top-k / top-p walk down from the maximum (cumulative mass exact, keep
// test `cum - p < top_p` in fp32 as the reference), and the boundary tie
// group with the number of its members kept (lowest ids first). The index
// cut inside that group is left to the consumers, which count group members
// in id order as they stream the rows they need; only a drafted token that
// falls inside its row's group is ranked here, by a rescan of the row prefix.
// Rows outside the window's assumptions are flagged kRowFallback and
// recomputed by the register-resident kernel (sdx_rowstat.hip).
#include "sdx_launch.hpp"

namespace sdx {

constexpr int SK_NT = 1024;
constexpr int SK_NW = SK_NT / kWave;
constexpr uint32_t SK_NEG_LO = 0x3600u;   // key of the most negative in-window value
constexpr uint32_t SK_ZERO_LO = 0x5480u;  // first key of the merged tiny-magnitude bin
constexpr uint32_t SK_ZERO_HI = 0xAB7Fu;
constexpr uint32_t SK_POS_LO = 0xAB80u;
constexpr uint32_t SK_POS_HI = 0xC9FFu;
constexpr int SK_WIN = 7808;
constexpr int SK_BIN_ZERO = 7809;
constexpr int SK_BIN_EXC = 15618;
constexpr int SK_TRASH = 15619;           // padding ids past the row end
constexpr int SK_NB = 15620;
constexpr int SK_PTOP = 1024;             // probabilities precomputed for the top bins

__device__ __forceinline__ int sk_bin_of_key(uint32_t k) {
  const uint32_t c1 = min(k > 0x35FFu ? k - 0x35FFu : 0u, 7809u);
  const uint32_t c2 = min(k > 0xAB7Fu ? k - 0xAB7Fu : 0u, 7809u);
  return (int)(c1 + c2);
}
// Two packed keys -> two packed bins (v_pk_sub_u16 with clamp, v_pk_min_u16, v_pk_add_u16).
typedef unsigned short us2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t sk_bins2(uint32_t keys2) {
  const us2 k = __builtin_bit_cast(us2, keys2);
  const us2 c1 = __builtin_elementwise_min(__builtin_elementwise_sub_sat(k, (us2){0x35FF, 0x35FF}),
                                           (us2){7809, 7809});
  const us2 c2 = __builtin_elementwise_min(__builtin_elementwise_sub_sat(k, (us2){0xAB7F, 0xAB7F}),
                                           (us2){7809, 7809});
  return __builtin_bit_cast(uint32_t, c1 + c2);
}
__device__ __forceinline__ uint32_t sk_lowkey(int b) {
  if (b <= 0) return 0u;
  if (b <= SK_WIN) return SK_NEG_LO + (uint32_t)(b - 1);
  if (b == SK_BIN_ZERO) return SK_ZERO_LO;
  if (b <= 2 * SK_WIN + 1) return SK_POS_LO + (uint32_t)(b - SK_BIN_ZERO - 1);
  return SK_POS_HI + 1;
}
__device__ __forceinline__ uint32_t sk_highkey(int b) {
  if (b == SK_BIN_ZERO) return SK_ZERO_HI;
  if (b <= 0) return SK_NEG_LO - 1;
  if (b >= SK_BIN_EXC) return 0xFFFFu;
  return sk_lowkey(b);
}
// Key whose value stands for the bin in exp (the merged tiny bin uses +0).
__device__ __forceinline__ uint32_t sk_repkey(int b) {
  return b == SK_BIN_ZERO ? 0x8000u : sk_lowkey(b);
}

__device__ __forceinline__ float sk_d(uint32_t key, float T, float m) {
  return decode16<SDX_BF16>(code_of_key16(key)) / T - m;
}

__global__ void __launch_bounds__(SK_NT, 2) rowstream_bf16_kernel(RowStatArgs a) {
  __shared__ uint32_t hist[SK_NB];
  __shared__ float ptop[SK_PTOP];
  __shared__ uint64_t s_u64[2 * SK_NW];
  __shared__ uint32_t s_u32[2 * SK_NW + 4];
  __shared__ float s_f[4];
  __shared__ int32_t s_i32[16];

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
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

  for (int b = tid; b < SK_NB; b += SK_NT) hist[b] = 0u;
  __syncthreads();

  // ---- 1. stream the row: 16-byte loads, packed keys -> packed bins, LDS atomics
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
          uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
          uint32_t bins[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) bins[t] = sk_bins2(keys2_of_codes2(w[t]));
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
  __syncthreads();

  // ---- 2. highest occupied bin, validity of the window assumptions
  {
    int hi = -1;
    for (int b = tid; b <= 2 * SK_WIN + 1; b += SK_NT)
      if (hist[b] != 0) hi = b;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) hi = max(hi, __shfl_xor(hi, o, kWave));
    if (lane == 0) s_i32[wave] = hi;
    __syncthreads();
    if (tid == 0) {
      int h = -1;
      for (int w2 = 0; w2 < SK_NW; ++w2) h = max(h, s_i32[w2]);
      s_i32[SK_NW] = h;
    }
    __syncthreads();
  }
  const int bmax = s_i32[SK_NW];
  const float T = a.T;
  bool ok = hist[SK_BIN_EXC] == 0 && bmax >= 1 && bmax != SK_BIN_ZERO;
  const uint32_t kmax = ok ? sk_lowkey(bmax) : 0u;
  const float m = ok ? decode16<SDX_BF16>(code_of_key16(kmax)) / T : 0.0f;
  if (ok && hist[0] != 0) ok = exp_det(sk_d(SK_NEG_LO - 1, T, m)) == 0.0f;
  if (ok && hist[SK_BIN_ZERO] != 0) {
    const float dz = sk_d(0x8000u, T, m);
    ok = sk_d(SK_ZERO_LO, T, m) == dz && sk_d(SK_ZERO_HI, T, m) == dz;
  }
  if (!ok) {  // uniform across the block: hand the row to the fallback kernel
    if (tid == 0) {
      RowStat st = {};
      st.flags = kRowFallback;
      st.zf = 1.0f; st.totf = 1.0f; st.glo = 1; st.ghi = 0; st.argmax = -1;
      *st_out = st;
    }
    return;
  }
  auto e_of_bin = [&](int b) -> float { return exp_det(sk_d(sk_repkey(b), T, m)); };

  // ---- 3. exact normaliser over occupied bins (bin 0 holds exp_det == 0)
  {
    U128 acc = {0, 0};
    for (int b = tid + 1; b <= bmax; b += SK_NT) {
      const uint32_t c = hist[b];
      if (c) acc = u128_add(acc, u128_mul32(c, fixed62(e_of_bin(b))));
    }
    acc = wave_sum_u128(acc);
    if (lane == 0) { s_u64[2 * wave] = acc.lo; s_u64[2 * wave + 1] = acc.hi; }
    __syncthreads();
    if (tid == 0) {
      U128 z = {0, 0};
      for (int w2 = 0; w2 < SK_NW; ++w2) z = u128_add(z, U128{s_u64[2 * w2], s_u64[2 * w2 + 1]});
      s_f[0] = rn32_u128(z);
    }
    __syncthreads();
  }
  const float zf = s_f[0];
  // probabilities of the top SK_PTOP bins (all waves), for the walk and the table
  for (int i = tid; i < SK_PTOP; i += SK_NT) {
    const int b = bmax - i;
    ptop[i] = (b >= 1 && hist[b] != 0) ? e_of_bin(b) / zf : 0.0f;
  }
  __syncthreads();
  auto p_of_bin = [&](int b) -> float {  // bin 0 holds exp_det == 0 (checked above)
    const int i = bmax - b;
    return b < 1 ? 0.0f : (i < SK_PTOP ? ptop[i] : e_of_bin(b) / zf);
  };

  // ---- 4. top-k threshold and top-p boundary (wave 0 walks down from bmax)
  // s_i32: 0 klo-bin, 1 glo-bin, 2 ghi-bin, 3 rstar, 4 gcount, 5 has-group
  if (wave == 0) {
    int klo_bin = 1;
    float p_kth = 0.0f;
    if (a.use_k) {
      uint32_t cnt = 0;
      int kb = 1;
      for (int b0 = bmax; b0 >= 1; b0 -= kWave) {
        const int b = b0 - lane;
        const uint32_t c = b >= 1 ? hist[b] : 0u;
        const uint32_t inc = wave_incl_scan_u32(c, lane);
        const uint64_t hit = __ballot(c != 0 && cnt + inc >= (uint32_t)a.top_k);
        if (hit) { kb = b0 - (__ffsll((unsigned long long)hit) - 1); break; }
        cnt += (uint32_t)__shfl((int)inc, kWave - 1, kWave);
      }
      p_kth = p_of_bin(kb);
      int lowb = kb;  // lower bins with the same probability are ties at kth: kept
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
      klo_bin = lowb;
    }
    int glo_b = klo_bin, ghi_b = klo_bin - 1, rstar = 0, gcount = 0, has_group = 0;
    uint64_t kept_mass = 0;
    if (a.use_p) {
      const float tp = a.top_p;
      uint64_t S = 0;
      bool found = false;
      int bb = 0;
      uint32_t cb = 0;
      float pb = 0.0f;
      uint64_t Sb = 0;
      for (int b0 = bmax; b0 >= klo_bin; b0 -= kWave) {
        const int b = b0 - lane;
        const uint32_t c = b >= klo_bin ? hist[b] : 0u;
        const float p = c ? p_of_bin(b) : 0.0f;
        const uint64_t mi = (uint64_t)c * fixed62(p);
        const uint64_t incl = wave_incl_scan_u64(mi, lane);
        bool fail = false;
        if (c) fail = !((rn32_u64(S + incl) - p) < tp);
        const uint64_t fb = __ballot(fail);
        if (fb) {
          const int L = __ffsll((unsigned long long)fb) - 1;
          bb = b0 - L;
          cb = (uint32_t)__shfl((int)c, L, kWave);
          pb = __shfl(p, L, kWave);
          Sb = S + (uint64_t)__shfl((long long)incl, L, kWave) -
               (uint64_t)__shfl((long long)mi, L, kWave);
          found = true;
          break;
        }
        S += (uint64_t)__shfl((long long)incl, kWave - 1, kWave);
      }
      if (found) {
        const uint64_t P = fixed62(pb);
        uint32_t lo_r = 0, hi_r = cb - 1;  // members kept in the boundary bin, in [0, cb-1]
        while (lo_r < hi_r) {
          const uint32_t mid = (lo_r + hi_r) / 2;
          if ((rn32_u64(Sb + (uint64_t)(mid + 1) * P) - pb) < tp) lo_r = mid + 1; else hi_r = mid;
        }
        uint32_t rr = lo_r;
        int gtop = bb, gbot = bb;
        uint32_t above = 0, gcnt = cb;
        for (;;) {  // neighbouring occupied bins with the same probability: one tie group
          int nxt = bmax + 1;
          for (int b0 = gtop + 1; b0 <= bmax; b0 += kWave) {
            const int b2 = b0 + lane;
            const uint64_t mm = __ballot(b2 <= bmax && hist[b2] != 0);
            if (mm) { nxt = b0 + (__ffsll((unsigned long long)mm) - 1); break; }
          }
          if (nxt > bmax || p_of_bin(nxt) != pb) break;
          gtop = nxt;
          above += hist[nxt];
        }
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
        gcnt += above;
        if (Sb == (uint64_t)above * P && above == 0 && rr == 0) rr = 1;  // keep[..., 0] = True
        rstar = (int)(above + rr);
        gcount = (int)gcnt;
        glo_b = gbot;
        ghi_b = gtop;
        klo_bin = gbot;
        kept_mass = Sb + (uint64_t)rr * P;
        has_group = 1;
      } else {
        kept_mass = S;
      }
    }
    if (lane == 0) {
      s_i32[0] = klo_bin; s_i32[1] = glo_b; s_i32[2] = ghi_b; s_i32[3] = rstar;
      s_i32[4] = gcount; s_i32[5] = has_group;
      s_u64[0] = kept_mass;
    }
  }
  __syncthreads();
  const int klo_bin = s_i32[0], glo_b = s_i32[1], ghi_b = s_i32[2];
  const int rstar = s_i32[3], gcount = s_i32[4], has_group = s_i32[5];
  uint64_t kept_mass = s_u64[0];
  __syncthreads();
  if (!a.use_p) {  // no nucleus: the kept mass is every bin from klo_bin up
    uint64_t acc = 0;
    for (int b = klo_bin + tid; b <= bmax; b += SK_NT) {
      const uint32_t c = hist[b];
      if (c) acc += (uint64_t)c * fixed62(p_of_bin(b));
    }
    acc = wave_sum_u64(acc);
    if (lane == 0) s_u64[SK_NW + wave] = acc;
    __syncthreads();
    if (tid == 0) {
      uint64_t t2 = 0;
      for (int w2 = 0; w2 < SK_NW; ++w2) t2 += s_u64[SK_NW + w2];
      s_u64[0] = t2;
    }
    __syncthreads();
    kept_mass = s_u64[0];
  }
  const float totf = fmaxf(rn32_u64(kept_mass), 1e-12f);
  const int32_t klo = (int32_t)(klo_bin <= 1 ? 0u : sk_lowkey(klo_bin));
  const int32_t glo = has_group ? (int32_t)sk_lowkey(glo_b) : klo;
  const int32_t ghi = has_group ? (int32_t)sk_highkey(ghi_b) : klo - 1;

  // ---- 5. table of final probabilities for the top keys
  const int32_t tbl_lo = max(klo, (int32_t)kmax - (kTbl - 1));
  const int32_t ntbl = (int32_t)kmax - tbl_lo + 1;
  for (int t = tid; t < ntbl; t += SK_NT) {
    const int b = sk_bin_of_key(kmax - (uint32_t)t);
    tbl_out[t] = hist[b] != 0 ? p_of_bin(b) / totf : 0.0f;
  }

  // ---- 6. probability of the drafted token (rank it if it sits in the tie group)
  float pg = 0.0f;
  if (gid >= 0 && gid < V) {
    const int32_t kk = (int32_t)key_of_code16(ptr[gid]);
    bool kept = kk >= klo;
    if (kept && kk >= glo && kk <= ghi) {
      if (rstar <= 0) {
        kept = false;
      } else if (rstar < gcount) {  // members before gid, in id order
        uint32_t cnt = 0;
        for (int64_t i = tid; i < gid; i += SK_NT) {
          const int32_t k2 = (int32_t)key_of_code16(ptr[i]);
          cnt += (k2 >= glo && k2 <= ghi) ? 1u : 0u;
        }
        cnt = wave_sum_u32(cnt);
        if (lane == 0) s_u32[wave] = cnt;
        __syncthreads();
        if (tid == 0) {
          uint32_t t2 = 0;
          for (int w2 = 0; w2 < SK_NW; ++w2) t2 += s_u32[w2];
          s_u32[2 * SK_NW] = t2;
        }
        __syncthreads();
        kept = s_u32[2 * SK_NW] < (uint32_t)rstar;
      }
    }
    if (kept) pg = p_of_bin(sk_bin_of_key((uint32_t)kk)) / totf;
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
    st.flags = 0;
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
