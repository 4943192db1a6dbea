// to_probs for fp32 logits (specdec/sampling.py:34-67), vocabularies up to
// 8192: the literal algorithm on one 1024-thread workgroup per row.
//
// fp32 logits are not limited to 65,536 distinct values, so the histogram
// of the 16-bit path does not apply. The row is small enough to sort in LDS:
// (p descending, id ascending) as one 64-bit key, bitonic sort, then the
// exact fixed-point inclusive scan for the nucleus test, exactly the order of
// operations of the reference (sort, cumsum, `cum - srt < top_p`, first token
// kept, renormalise). Writes dense fp32 probabilities and a RowStat with the
// gathered probability of the row's draft token.
#include "sdx_launch.hpp"

namespace sdx {

constexpr int F32_NT = 1024;
constexpr int F32_MAXV = 8192;
constexpr int F32_PER = F32_MAXV / F32_NT;  // 8 elements per thread


__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, uint64_t* red) {
  v = wave_sum_u64(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) red[w] = v;
  __syncthreads();
  uint64_t t = 0;
  for (int i = 0; i < F32_NT / kWave; ++i) t += red[i];
  return t;
}

__global__ void __launch_bounds__(F32_NT) to_probs_f32_kernel(F32Args a) {
  __shared__ uint64_t skey[F32_MAXV];
  __shared__ uint64_t red[2 * (F32_NT / kWave)];
  __shared__ uint8_t keep[F32_MAXV];
  __shared__ float s_f[4];
  __shared__ int64_t s_i[2];

  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  if (tid == 0 && row < a.nzero) a.zero[row] = 0u;
  if (tid == 0) s_i[1] = 0;  // set when the gathered token is a tie-group member
  const int g = row < a.nrows[0] ? 0 : 1;
  const int64_t r = g ? row - a.nrows[0] : row;
  const float* x = a.base[g] + r * a.ld[g];
  const int V = (int)a.V;
  const int64_t gid = draft_id_of_row(a.ids, a.tgt_idx, a.k, a.nrows[1], g, r);
  float* o = a.out + row * a.ld_out;

  float v[F32_PER];
#pragma unroll
  for (int t = 0; t < F32_PER; ++t) {
    const int i = tid + t * F32_NT;
    v[t] = i < V ? x[i] : -INFINITY;
  }
  // ---- greedy: one-hot at the first maximum (-0 == +0)
  if (a.greedy) {
    uint64_t best = 0;
#pragma unroll
    for (int t = 0; t < F32_PER; ++t) {
      const int i = tid + t * F32_NT;
      if (i < V) {
        uint32_t k = key_of_f32(v[t]);
        if (k == 0x7FFFFFFFu) k = 0x80000000u;
        const uint64_t c = ((uint64_t)k << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)i);
        best = c > best ? c : best;
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const uint64_t w = (uint64_t)__shfl_xor((long long)best, off, kWave);
      best = w > best ? w : best;
    }
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = best;
    __syncthreads();
    uint64_t b = 0;
    for (int w = 0; w < F32_NT / kWave; ++w) b = red[w] > b ? red[w] : b;
    const int64_t am = (int64_t)(0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFu));
    for (int i = tid; i < V; i += F32_NT) o[i] = i == am ? 1.0f : 0.0f;
    if (a.tie_bits)  // no tie groups in a one-hot row
      for (int i = tid; i < (int)kF32TieWords; i += F32_NT) a.tie_bits[row * kF32TieWords + i] = 0u;
    if (tid == 0 && a.stats) {
      RowStat st = {};
      st.flags = kRowGreedy | kRowProbs;
      st.argmax = am;
      st.zf = 1.0f; st.totf = 1.0f; st.glo = 1; st.ghi = 0;
      st.pgather = gid >= 0 ? (gid == am ? 1.0f : 0.0f) : 0.0f;
      a.stats[row] = st;
    }
    return;
  }

  // ---- softmax numerator and exact normaliser
  float s[F32_PER];
  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < F32_PER; ++t) {
    s[t] = v[t] / a.T;
    if (tid + t * F32_NT < V) mx = fmaxf(mx, s[t]);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
  if ((tid & (kWave - 1)) == 0) red[tid / kWave] = __float_as_uint(mx);
  __syncthreads();
  if (tid == 0) {
    float m2 = -INFINITY;
    for (int w = 0; w < F32_NT / kWave; ++w) m2 = fmaxf(m2, __uint_as_float((uint32_t)red[w]));
    s_f[0] = m2;
  }
  __syncthreads();
  const float m = s_f[0];
  float p[F32_PER];
  U128 acc = {0, 0};
#pragma unroll
  for (int t = 0; t < F32_PER; ++t) {
    p[t] = tid + t * F32_NT < V ? exp_det(s[t] - m) : 0.0f;
    acc = u128_add(acc, U128{fixed62(p[t]), 0});
  }
  acc = wave_sum_u128(acc);
  __syncthreads();
  if ((tid & (kWave - 1)) == 0) { red[2 * (tid / kWave)] = acc.lo; red[2 * (tid / kWave) + 1] = acc.hi; }
  __syncthreads();
  if (tid == 0) {
    U128 z = {0, 0};
    for (int w = 0; w < F32_NT / kWave; ++w) z = u128_add(z, U128{red[2 * w], red[2 * w + 1]});
    s_f[1] = rn32_u128(z);
  }
  __syncthreads();
  const float zf = s_f[1];
#pragma unroll
  for (int t = 0; t < F32_PER; ++t) p[t] = p[t] / zf;

  // ---- sort (p desc, id asc) when a filter is active
  bool mask[F32_PER];
#pragma unroll
  for (int t = 0; t < F32_PER; ++t) mask[t] = true;
  // the partially kept boundary tie group: the tokens of the last kept
  // probability vb (after top-k zeroing) when the first dropped token has it too
  bool partial = false;
  float vb = 0.0f, kth_g = 0.0f;
  if (a.use_k || a.use_p) {
    int n2 = 1;
    while (n2 < V) n2 <<= 1;
    for (int i = tid; i < n2; i += F32_NT) {
      if (i < V) {
        const int t = i / F32_NT;  // i = tid + t*F32_NT
        float pv = 0.0f;
#pragma unroll
        for (int u = 0; u < F32_PER; ++u)
          if (u == t) pv = p[u];
        skey[i] = ((uint64_t)(~__float_as_uint(pv)) << 32) | (uint32_t)i;
      } else {
        skey[i] = ~0ull;
      }
    }
    __syncthreads();
    for (int size = 2; size <= n2; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int i = tid; i < n2; i += F32_NT) {
          const int jx = i ^ stride;
          if (jx > i) {
            const bool up = (i & size) == 0;
            const uint64_t ai = skey[i], aj = skey[jx];
            if ((ai > aj) == up) { skey[i] = aj; skey[jx] = ai; }
          }
        }
        __syncthreads();
      }
    }
    // sorted position i holds (p_i, id_i); top-k keeps positions with p >= kth
    const float kth = a.use_k ? __uint_as_float(~(uint32_t)(skey[a.top_k - 1] >> 32)) : 0.0f;
    // inclusive scan of fixed62 masses over sorted positions (8 per thread, contiguous)
    uint64_t mloc[F32_PER];
    uint64_t sum = 0;
#pragma unroll
    for (int t = 0; t < F32_PER; ++t) {
      const int i = tid * F32_PER + t;
      float pv = i < V ? __uint_as_float(~(uint32_t)(skey[i] >> 32)) : 0.0f;
      if (a.use_k && pv < kth) pv = 0.0f;
      mloc[t] = fixed62(pv);
      sum += mloc[t];
    }
    // block exclusive scan of thread sums
    uint64_t incl = wave_incl_scan_u64(sum, tid & (kWave - 1));
    __syncthreads();
    if ((tid & (kWave - 1)) == kWave - 1) red[tid / kWave] = incl;
    __syncthreads();
    uint64_t wbase = 0;
    for (int w = 0; w < tid / kWave; ++w) wbase += red[w];
    uint64_t run = wbase + incl - sum;
#pragma unroll
    for (int t = 0; t < F32_PER; ++t) {
      const int i = tid * F32_PER + t;
      if (i < V) {
        float pv = __uint_as_float(~(uint32_t)(skey[i] >> 32));
        bool kk = !(a.use_k && pv < kth);
        if (!kk) pv = 0.0f;
        run += mloc[t];
        if (a.use_p) {
          const float cumf = rn32_u64(run);
          kk = kk && (((cumf - pv) < a.top_p) || i == 0);
        }
        keep[(uint32_t)skey[i]] = kk ? 1 : 0;
      }
    }
    __syncthreads();
    uint64_t nkeep = 0;
#pragma unroll
    for (int t = 0; t < F32_PER; ++t) {
      const int i = tid + t * F32_NT;
      mask[t] = i < V && keep[i] != 0;
      nkeep += mask[t] ? 1u : 0u;
    }
    if (a.use_p) {  // keep is a prefix of the sorted order: its last position is nkeep - 1
      nkeep = block_sum_u64(nkeep, red);
      const int js = (int)nkeep - 1;
      auto masked = [&](int i) {
        const float pv = __uint_as_float(~(uint32_t)(skey[i] >> 32));
        return (a.use_k && pv < kth) ? 0.0f : pv;
      };
      vb = masked(js);
      partial = js + 1 < V && vb > 0.0f && masked(js + 1) == vb;
      kth_g = kth;
    }
  }
  bool gtie = false;
  if (a.tie_bits || gid >= 0) {
    const int lane = tid & (kWave - 1), wv = tid / kWave;
#pragma unroll
    for (int t = 0; t < F32_PER; ++t) {
      const int i = tid + t * F32_NT;
      const float pm = (a.use_k && p[t] < kth_g) ? 0.0f : p[t];
      const bool mem = partial && i < V && pm == vb;
      if (mem && i == gid) gtie = true;
      const uint64_t bm = __ballot(mem);
      if (a.tie_bits && lane == 0) {  // ids t*F32_NT + 64*wv + [0, 64): two words
        uint32_t* dst = a.tie_bits + row * kF32TieWords + ((t * F32_NT + wv * kWave) >> 5);
        dst[0] = (uint32_t)bm;
        dst[1] = (uint32_t)(bm >> 32);
      }
    }
    if (gtie) s_i[1] = 1;
  }
  // ---- renormalise
  uint64_t tot = 0;
#pragma unroll
  for (int t = 0; t < F32_PER; ++t) {
    if (!mask[t]) p[t] = 0.0f;
    tot += fixed62(p[t]);
  }
  tot = block_sum_u64(tot, red);
  const float totf = fmaxf(rn32_u64(tot), 1e-12f);
#pragma unroll
  for (int t = 0; t < F32_PER; ++t) {
    const int i = tid + t * F32_NT;
    if (i < V) {
      const float pf = p[t] / totf;
      o[i] = pf;
      if (i == gid) s_f[2] = pf;
    }
  }
  __syncthreads();
  if (tid == 0 && a.stats) {
    RowStat st = {};
    st.flags = kRowProbs | (s_i[1] ? kRowGatherTie : 0u);
    st.m = m; st.zf = zf; st.totf = totf; st.mass = tot;
    st.glo = 1; st.ghi = 0; st.argmax = -1;
    st.pgather = (gid >= 0 && gid < V) ? s_f[2] : 0.0f;
    a.stats[row] = st;
  }
}

hipError_t launch_to_probs_f32(const F32Args& a, int64_t rows, hipStream_t s) {
  hipLaunchKernelGGL(to_probs_f32_kernel, dim3((unsigned)rows), dim3(F32_NT), 0, s, a);
  return hipGetLastError();
}

}  // namespace sdx
