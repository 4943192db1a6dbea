// Row statistics for 16-bit (bf16 / fp16) logits: the fused to_probs of
// specdec/sampling.py:34-67 reduced to the facts later stages need.
//
// One 1024-thread workgroup owns one row and keeps it in VGPRs (16 waves, each
// a contiguous 1/16 of the row, 16-byte coalesced loads): at V = 151,936 that
// is 19 x 16 B per lane, so the row is read from HBM exactly once. Because a
// bf16 logit has only 65,536 possible values and the probability of a token
// depends only on its value, the row is reduced to an LDS histogram over
// order-preserving 16-bit keys (a window of 36,864 keys below the maximum,
// 144 KiB). Everything else runs on the histogram:
//   * normaliser Z = sum_keys count * fixed62(exp_det(x/T - m)), exact
//     (128-bit fixed point, order independent);
//   * top-k threshold and the top-p nucleus boundary, found by a wave-0
//     walk down from the maximum key with exact fixed-point cumulative mass
//     and the reference's fp32 keep test `cum - p < top_p`;
//   * the kept count inside the boundary tie group (lowest ids kept first);
//     consumers rank group members by id as they stream the row.
// Keys below the window (logits more than ~2^28 below the maximum at
// ordinary temperatures) carry exp_det == 0 and are checked to do so.
//
// This kernel serves fp16 rows; bf16 rows go through the streaming kernel
// (sdx_rowstream.hip).
#include "sdx_launch.hpp"

namespace sdx {

constexpr int RS_NT = 1024;
constexpr int RS_NW = RS_NT / kWave;
constexpr int RS_NBINS = 36864;


template <int FMT>
__device__ __forceinline__ float e_of_key(uint32_t key, float T, float m) {
  const float s = decode16<FMT>(code_of_key16(key)) / T;
  return exp_det(s - m);
}

// Re-issue the packed key registers as opaque values. Each stage then
// re-extracts the 16-bit halves it needs (two ALU ops) instead of the
// compiler keeping eight unpacked values per slot alive across stages, which
// would double the register footprint of the resident row.
template <int NSLOT>
__device__ __forceinline__ void launder_keys(uint32_t (&key)[NSLOT][4]) {
#pragma unroll
  for (int j = 0; j < NSLOT; ++j)
#pragma unroll
    for (int t = 0; t < 4; ++t) asm volatile("" : "+v"(key[j][t]));
}

// fixed62(exp_det(x/T - m) / div) for one element below the histogram window
// (rare path, kept out of line so the unrolled register scans stay small).
template <int FMT>
__device__ __noinline__ uint64_t below_fixed(uint32_t key, float T, float m, float div) {
  const float e = e_of_key<FMT>(key, T, m);
  return fixed62(div == 1.0f ? e : e / div);
}

// First occupied bin strictly below b (>= 1), or 0. Called by a whole wave.
__device__ __forceinline__ int wave_occ_below(const uint32_t* hist, int b, int lane) {
  for (int b0 = b - 1; b0 >= 1; b0 -= kWave) {
    const int bb = b0 - lane;
    const bool occ = bb >= 1 && hist[bb] != 0;
    const uint64_t m = __ballot(occ);
    if (m) return b0 - (__ffsll((unsigned long long)m) - 1);
  }
  return 0;
}
// First occupied bin strictly above b (< nb), or nb.
__device__ __forceinline__ int wave_occ_above(const uint32_t* hist, int b, int nb, int lane) {
  for (int b0 = b + 1; b0 < nb; b0 += kWave) {
    const int bb = b0 + lane;
    const bool occ = bb < nb && hist[bb] != 0;
    const uint64_t m = __ballot(occ);
    if (m) return b0 + (__ffsll((unsigned long long)m) - 1);
  }
  return nb;
}

template <int NSLOT, int FMT>
__global__ void __launch_bounds__(RS_NT) rowstat16_kernel(RowStatArgs a) {
  __shared__ uint32_t hist[RS_NBINS];
  __shared__ uint64_t s_u64[2 * RS_NW];
  __shared__ uint32_t s_u32[2 * RS_NW + 4];
  __shared__ int64_t s_i64[2];
  __shared__ float s_f[4];
  __shared__ int32_t s_i32[16];

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int64_t row = blockIdx.x;
  const int g = row < a.nrows[0] ? 0 : 1;
  const int64_t r = g ? row - a.nrows[0] : row;
  const uint16_t* __restrict__ ptr = a.base[g] + r * a.ld[g];
  const int64_t gid = draft_id_of_row(a.ids, a.tgt_idx, a.k, a.nrows[1], g, r);
  const int64_t V = a.V;
  const int64_t cw = ((V + RS_NW * 8 - 1) / (RS_NW * 8)) * 8;
  const int64_t wb = (int64_t)wave * cw;
  const int64_t we = min(V, wb + cw);
  RowStat* st_out = a.stats + row;
  float* tbl_out = a.tables + row * kTbl;
  if (row < a.nzero) {
    const int zpr = a.zero_per_row > 0 ? a.zero_per_row : 1;
    if (tid < zpr) a.zero[row * zpr + tid] = 0u;
  }

  // Element (j, t) of this lane is id wb + j*512 + lane*8 + t; it exists iff
  // j*512 + t < rem. All per-slot checks compare one register with constants.
  const int32_t rem = (int32_t)max<int64_t>(0, we - wb) - lane * 8;
  const uint16_t* __restrict__ lptr = ptr + wb + lane * 8;
  const int64_t lbase = wb + lane * 8;

  // ---- 1. load the row into registers as packed keys, track the max key
  uint32_t key[NSLOT][4];
  uint32_t kmx = 0;
#pragma unroll
  for (int j = 0; j < NSLOT; ++j) {
    // Whole 16-byte loads (rows start 16-byte aligned); the row's last partial
    // group is read element by element. Ids at or past the row end become
    // code 0xFFFF, key 0, and are excluded by the `< rem` checks of every stage.
    uint32_t w[4] = {0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu};
    if (j * 512 + 8 <= rem) {
      const uint4 v = *reinterpret_cast<const uint4*>(lptr + j * 512);
      w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if (j * 512 < rem) {
#pragma unroll
      for (int t = 0; t < 8; ++t)
        if (j * 512 + t < rem)
          w[t >> 1] = (w[t >> 1] & ~(0xFFFFu << (16 * (t & 1)))) |
                      ((uint32_t)lptr[j * 512 + t] << (16 * (t & 1)));
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      key[j][t] = keys2_of_codes2(w[t]);
      kmx = max(kmx, max(key[j][t] & 0xFFFFu, key[j][t] >> 16));
    }
  }
  kmx = wave_max_u32(kmx);
  if (lane == 0) s_u32[wave] = kmx;
  __syncthreads();
  if (tid < kWave) {
    uint32_t v = tid < RS_NW ? s_u32[tid] : 0u;
    v = wave_max_u32(v);
    if (tid == 0) s_u32[2 * RS_NW] = v;
  }
  __syncthreads();
  const uint32_t kmax = s_u32[2 * RS_NW];

  if (kmax >= kPosInfKey<FMT> || kmax == 0) {  // +inf / NaN: flag, outputs unspecified
    if (tid == 0) {
      RowStat st = {};
      st.flags = kRowNonfinite;
      st.zf = 1.0f; st.totf = 1.0f; st.klo = 0x7FFFFFFF; st.glo = 1; st.ghi = 0;
      *st_out = st;
    }
    return;
  }

  // (temperature <= 0 never reaches this kernel: greedy rows go through the
  // argmax kernel.)

  // ---- 2. histogram over the key window [lo, kmax]; bin 0 collects keys < lo
  const uint32_t lo = kmax > (uint32_t)(RS_NBINS - 2) ? kmax - (uint32_t)(RS_NBINS - 2) : 0u;
  const int nb = (int)(kmax - lo) + 2;
  for (int b = tid; b < nb; b += RS_NT) hist[b] = 0u;
  __syncthreads();
  launder_keys(key);
#pragma unroll
  for (int j = 0; j < NSLOT; ++j) {
    if (j * 512 + 8 <= rem) {
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint32_t kk = (t & 1) ? (key[j][t >> 1] >> 16) : (key[j][t >> 1] & 0xFFFFu);
        atomicAdd(&hist[kk < lo ? 0u : kk - lo + 1u], 1u);
      }
    } else if (j * 512 < rem) {
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint32_t kk = (t & 1) ? (key[j][t >> 1] >> 16) : (key[j][t >> 1] & 0xFFFFu);
        if (j * 512 + t < rem) atomicAdd(&hist[kk < lo ? 0u : kk - lo + 1u], 1u);
      }
    }
  }
  __syncthreads();

  const float T = a.T;
  const float m = decode16<FMT>(code_of_key16(kmax)) / T;
  // Elements below the window carry mass only if the largest key below it does.
  const bool below_mass = lo > 0 && hist[0] != 0 && e_of_key<FMT>(lo - 1, T, m) > 0.0f;

  // ---- 3. exact normaliser Z
  {
    U128 acc = {0, 0};
    for (int b = tid + 1; b < nb; b += RS_NT) {
      const uint32_t c = hist[b];
      if (c) acc = u128_add(acc, u128_mul32(c, fixed62(e_of_key<FMT>(lo + b - 1, T, m))));
    }
    launder_keys(key);
    if (below_mass) {
#pragma unroll
      for (int j = 0; j < NSLOT; ++j) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const uint32_t kk = (t & 1) ? (key[j][t >> 1] >> 16) : (key[j][t >> 1] & 0xFFFFu);
          if (j * 512 + t < rem && kk < lo)
            acc = u128_add(acc, U128{below_fixed<FMT>(kk, T, m, 1.0f), 0});
        }
      }
    }
    acc = wave_sum_u128(acc);
    if (lane == 0) { s_u64[2 * wave] = acc.lo; s_u64[2 * wave + 1] = acc.hi; }
    __syncthreads();
    if (tid == 0) {
      U128 z = {0, 0};
      for (int w2 = 0; w2 < RS_NW; ++w2) z = u128_add(z, U128{s_u64[2 * w2], s_u64[2 * w2 + 1]});
      s_f[0] = rn32_u128(z);
    }
    __syncthreads();
  }
  const float zf = s_f[0];
  auto p_of_key = [&](uint32_t kk) -> float { return e_of_key<FMT>(kk, T, m) / zf; };

  // ---- 4. top-k threshold and top-p boundary (wave 0 walks down from kmax)
  // s_i32: 0 klo, 1 glo, 2 ghi, 3 kept-in-group R*, 4 group count, 5 need cut,
  //        6 flags;  s_u64[0] kept mass (only when use_p)
  if (wave == 0) {
    uint32_t rflags = below_mass ? kRowBelowWindow : 0u;
    int klo_bin = 1;          // lowest bin that top-k keeps (1 = everything in window)
    float p_kth = 0.0f;
    bool k_all = true;        // top-k keeps every key (disabled)
    if (a.use_k) {
      uint32_t cnt = 0;
      int kb = -1;
      for (int b0 = nb - 1; b0 >= 1; b0 -= kWave) {
        const int b = b0 - lane;
        const uint32_t c = b >= 1 ? hist[b] : 0u;
        const uint32_t inc = wave_incl_scan_u32(c, lane);
        const uint64_t hit = __ballot(c != 0 && cnt + inc >= (uint32_t)a.top_k);
        if (hit) { kb = b0 - (__ffsll((unsigned long long)hit) - 1); break; }
        cnt += __shfl(inc, kWave - 1, kWave);
      }
      if (kb < 0) {
        rflags |= kRowUnsupported;  // k-th largest lies below the window
        kb = 1;
      }
      p_kth = p_of_key(lo + kb - 1);
      // keys below kb with the same probability are ties at kth: kept too
      int lowb = kb;
      for (;;) {
        const int nxt = wave_occ_below(hist, lowb, lane);
        if (nxt < 1 || p_of_key(lo + nxt - 1) != p_kth) break;
        lowb = nxt;
      }
      klo_bin = lowb;
      k_all = false;
    }
    int32_t klo = (int32_t)(lo + klo_bin - 1);
    if (k_all && !below_mass) klo = 0;      // everything kept
    if (k_all && below_mass) klo = 0;
    int32_t glo = klo, ghi = klo - 1, rstar = 0, gcount = 0, needcut = 0;
    uint64_t kept_mass = 0;

    if (a.use_p) {
      const float tp = a.top_p;
      uint64_t S = 0;
      bool found = false;
      int bb = 0;
      uint32_t cb = 0;
      float pb = 0.0f;
      uint64_t Sb = 0;
      for (int b0 = nb - 1; b0 >= klo_bin; b0 -= kWave) {
        const int b = b0 - lane;
        uint32_t c = b >= klo_bin ? hist[b] : 0u;
        const float p = c ? p_of_key(lo + b - 1) : 0.0f;
        const uint64_t mi = (uint64_t)c * fixed62(p);
        const uint64_t incl = wave_incl_scan_u64(mi, lane);
        bool fail = false;
        if (c) {
          const float cumf = rn32_u64(S + incl);
          fail = !((cumf - p) < tp);
        }
        const uint64_t fb = __ballot(fail);
        if (fb) {
          const int L = __ffsll((unsigned long long)fb) - 1;
          bb = b0 - L;
          cb = (uint32_t)__shfl((int)c, L, kWave);
          pb = __shfl(p, L, kWave);
          const uint64_t inclL = (uint64_t)__shfl((long long)incl, L, kWave);
          const uint64_t miL = (uint64_t)__shfl((long long)mi, L, kWave);
          Sb = S + inclL - miL;
          found = true;
          break;
        }
        S += (uint64_t)__shfl((long long)incl, kWave - 1, kWave);
      }
      if (found) {
        const uint64_t P = fixed62(pb);
        // kept members of the boundary bin: keep_r = rn32(Sb + (r+1) P) - pb < tp,
        // monotone in r; the last member (r = cb - 1) fails.
        uint32_t lo_r = 0, hi_r = cb - 1;  // answer in [0, cb-1]
        while (lo_r < hi_r) {
          const uint32_t mid = (lo_r + hi_r) / 2;  // test member mid
          const bool keep = (rn32_u64(Sb + (uint64_t)(mid + 1) * P) - pb) < tp;
          if (keep) lo_r = mid + 1; else hi_r = mid;
        }
        uint32_t rr = lo_r;
        // tie group = neighbouring occupied bins with the same probability
        int gtop = bb, gbot = bb;
        uint32_t above = 0, gcnt = cb;
        for (;;) {
          const int nxt = wave_occ_above(hist, gtop, nb, lane);
          if (nxt >= nb || p_of_key(lo + nxt - 1) != pb) break;
          gtop = nxt;
          above += hist[nxt];
        }
        for (;;) {
          const int nxt = wave_occ_below(hist, gbot, lane);
          if (nxt < klo_bin || p_of_key(lo + nxt - 1) != pb) break;
          gbot = nxt;
          gcnt += hist[nxt];
        }
        gcnt += above;
        if (Sb == (uint64_t)above * P && rr == 0 && above == 0) rr = 1;  // keep[..., 0] = True
        rstar = (int32_t)(above + rr);
        gcount = (int32_t)gcnt;
        glo = (int32_t)(lo + gbot - 1);
        ghi = (int32_t)(lo + gtop - 1);
        klo = glo;
        kept_mass = Sb + (uint64_t)rr * P;
        needcut = (rstar > 0 && rstar < gcount) ? 1 : 0;
      } else {
        kept_mass = S;
        if (below_mass && k_all) rflags |= kRowUnsupported;  // nucleus reaches below the window
      }
    }
    if (lane == 0) {
      s_i32[0] = klo; s_i32[1] = glo; s_i32[2] = ghi; s_i32[3] = rstar;
      s_i32[4] = gcount; s_i32[5] = needcut; s_i32[6] = (int32_t)rflags;
      s_u64[0] = kept_mass;
    }
  }
  __syncthreads();
  const int32_t klo = s_i32[0], glo = s_i32[1], ghi = s_i32[2];
  const int32_t rstar = s_i32[3];
  uint32_t rflags = (uint32_t)s_i32[6];

  // ---- 5. kept mass when there is no nucleus: sum over kept keys
  uint64_t kept_mass = s_u64[0];
  __syncthreads();
  if (!a.use_p) {
    uint64_t acc = 0;
    const int bstart = klo >= (int32_t)lo ? (int)(klo - (int32_t)lo) + 1 : 1;
    for (int b = bstart + tid; b < nb; b += RS_NT) {
      const uint32_t c = hist[b];
      if (c) acc += (uint64_t)c * fixed62(p_of_key(lo + b - 1));
    }
    launder_keys(key);
    if (below_mass && klo < (int32_t)lo) {
#pragma unroll
      for (int j = 0; j < NSLOT; ++j) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const uint32_t kk = (t & 1) ? (key[j][t >> 1] >> 16) : (key[j][t >> 1] & 0xFFFFu);
          if (j * 512 + t < rem && kk < lo && (int32_t)kk >= klo)
            acc += below_fixed<FMT>(kk, T, m, zf);
        }
      }
    }
    acc = wave_sum_u64(acc);
    if (lane == 0) s_u64[RS_NW + wave] = acc;
    __syncthreads();
    if (tid == 0) {
      uint64_t t2 = 0;
      for (int w2 = 0; w2 < RS_NW; ++w2) t2 += s_u64[RS_NW + w2];
      s_u64[0] = t2;
    }
    __syncthreads();
    kept_mass = s_u64[0];
  }
  const float totf = fmaxf(rn32_u64(kept_mass), 1e-12f);

  // ---- 6. drafted token inside a partial boundary group: its member rank
  // (members with lower ids) decides whether it is among the rstar kept.
  bool g_kept = true;
  if (gid >= 0 && gid < V && rstar > 0 && rstar < s_i32[4]) {
    const int32_t kg = (int32_t)key_of_code16(ptr[gid]);
    if (kg >= glo && kg <= ghi) {
      g_kept = block_count_members(ptr, gid, glo, ghi, s_u32) < (uint32_t)rstar;
      rflags |= kRowGatherTie;
    }
  }

  // ---- 7. table of final probabilities for the top keys, gathered token, record
  const int32_t tbl_lo = max(klo, (int32_t)kmax - (kTbl - 1));
  const int32_t ntbl = (int32_t)kmax - tbl_lo + 1;
  for (int t = tid; t < ntbl; t += RS_NT) {
    const uint32_t kk = kmax - (uint32_t)t;
    const bool occ = kk < lo || hist[kk - lo + 1] != 0;
    tbl_out[t] = occ ? p_of_key(kk) / totf : 0.0f;
  }
  if (tid == 0) {
    RowStat st;
    st.m = m;
    st.zf = zf;
    st.totf = totf;
    st.kmax = (int32_t)kmax;
    st.klo = klo;
    st.glo = glo;
    st.ghi = ghi;
    st.rstar = rstar;
    st.gcount = s_i32[4];
    st.mass = kept_mass;
    st.flags = rflags;
    st.ntbl = ntbl;
    st.argmax = -1;
    float pg = 0.0f;
    if (gid >= 0 && gid < V) {
      const uint32_t code = ptr[gid];
      const int32_t kk = (int32_t)key_of_code16(code);
      const bool kept = kk >= klo && (!(kk >= glo && kk <= ghi) || (rstar > 0 && g_kept));
      pg = kept ? p_of_key((uint32_t)kk) / totf : 0.0f;
    }
    st.pgather = pg;
    *st_out = st;
  }
}

// ---------------------------------------------------------------- launch
template <int FMT>
static hipError_t launch_rowstat16_fmt(const RowStatArgs& a, int64_t rows, int nslot,
                                       hipStream_t s) {
  const dim3 grid((unsigned)rows), block(RS_NT);
#define SDX_RS_CASE(N)                                                        \
  case N:                                                                     \
    hipLaunchKernelGGL((rowstat16_kernel<N, FMT>), grid, block, 0, s, a);     \
    break;
  switch (nslot) {
    SDX_RS_CASE(1)
    SDX_RS_CASE(2)
    SDX_RS_CASE(4)
    SDX_RS_CASE(8)
    SDX_RS_CASE(12)
    SDX_RS_CASE(16)
    SDX_RS_CASE(19)
    SDX_RS_CASE(20)
    default:
      return hipErrorInvalidValue;
  }
#undef SDX_RS_CASE
  return hipGetLastError();
}

int rowstat16_nslot(int64_t V) {
  const int64_t cw = ((V + RS_NW * 8 - 1) / (RS_NW * 8)) * 8;
  const int64_t need = (cw + 511) / 512;
  static const int sizes[] = {1, 2, 4, 8, 12, 16, 19, 20};
  for (int s : sizes)
    if (need <= s) return s;
  return -1;
}

hipError_t launch_rowstat16(int fmt, const RowStatArgs& a, int64_t rows, hipStream_t s) {
  const int nslot = rowstat16_nslot(a.V);
  if (nslot < 0) return hipErrorInvalidValue;
  return fmt == SDX_BF16 ? launch_rowstat16_fmt<SDX_BF16>(a, rows, nslot, s)
                         : launch_rowstat16_fmt<SDX_F16>(a, rows, nslot, s);
}

}  // namespace sdx
