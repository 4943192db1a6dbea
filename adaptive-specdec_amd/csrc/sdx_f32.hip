// to_probs for fp32 logits (specdec/sampling.py:34-67): vocabularies up to 8192
// with the literal algorithm on one 1024-thread workgroup per row; larger ones
// with the multi-pass kernel below, which sorts only the nucleus boundary region.
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
      for (int i = tid; i < (int)a.tie_ld; i += F32_NT) a.tie_bits[row * a.tie_ld + i] = 0u;
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
        uint32_t* dst = a.tie_bits + row * a.tie_ld + ((t * F32_NT + wv * kWave) >> 5);
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

// ---------------------------------------------------------------- large vocabularies
// The same rule for rows longer than the LDS sort holds, in passes over the row
// by one 1024-thread workgroup. p is non-decreasing in s, so the reference's
// order (p descending, id ascending) visits the values of s in descending key
// order, ids ascending within each tie group of equal p:
//  1. m = max s (s = fl32(x / T)) and, per bucket of the top 12 bits of key(s),
//     the element count and the smallest and largest key present;
//  2. the exact normaliser Z (128-bit fixed point); with top-k, the k-th largest
//     key from the bucket counts and the distinct keys of its bucket;
//  3. per bucket the fixed-point mass of the top-k-zeroed p. The keep test
//     `cum - p < top_p` fails first inside the first bucket whose last element
//     fails it (cum: the buckets above plus its own mass; p: that of its smallest
//     key). That bucket, widened while a neighbouring bucket holds the same p at
//     the shared edge (so no tie group straddles the region's edge), is the
//     region;
//  4. the region's distinct probabilities with their counts (an LDS hash table:
//     one entry per tie group), sorted descending and walked with the exact
//     prefix of the buckets above: the first group whose last element fails is
//     the boundary group, and a 64-way search gives its members kept, lowest ids
//     first;
//  5. the output (p / totf where kept, 0 elsewhere; group members ranked by id,
//     from wave ballots per 4,096 ids when the rows are 16-byte aligned, else
//     with one block scan per 1024 ids), the tie-group bits and the statistics.
// Every element's exp is evaluated once: pass 2 leaves it in the output row,
// pass 3 replaces it by p = exp / Z, which passes 4 and 5 read back. The
// passes stream with 16-byte loads, several in flight per thread; the kernel
// is bound by VALU issue (about 220 instructions per element over the passes,
// 59% of one CU's issue rate with one row per CU).
// A region with more than FB_KEYS distinct probabilities marks the row
// unsupported and writes NaN probabilities. (The top-k bucket is read the same
// way: the k-th largest p is the group where the bucket's counts reach k.)
constexpr int FB_NT = 1024;
constexpr int FB_NB = 4096;
constexpr int FB_SHIFT = 20;  // bucket = key >> 20
constexpr int FB_TAB = 8192;  // hash slots for distinct keys
constexpr int FB_KEYS = 7168; // distinct probabilities a region may hold (87.5% of the slots)
constexpr int FB_NW = FB_NT / kWave;
constexpr int FB_PER = FB_TAB / FB_NT;  // sorted entries per thread

struct FbLds {
  uint32_t cnt[FB_NB];
  uint32_t kmin[FB_NB];
  uint32_t kmax[FB_NB];
  uint64_t mass[FB_NB];
  uint64_t ent[FB_TAB];  // hash table (key word, count word), then sorted (~key << 32 | count)
  uint64_t red[2 * FB_NW];
  uint32_t wt[2][FB_NW];  // output pass: members per wave, double-buffered by step
  uint32_t ndist, nfill;
  int32_t i32[8];
  float f32[8];
  uint64_t u64[4];
};

__device__ __forceinline__ float fb_of_key(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
__device__ __forceinline__ float fb_pmask(float p, bool use_k, float kth) {
  return (use_k && p < kth) ? 0.0f : p;
}
__device__ uint64_t fb_sum_u64(uint64_t v, FbLds& L) {
  v = wave_sum_u64(v);
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) L.red[threadIdx.x / kWave] = v;
  __syncthreads();
  uint64_t t = 0;
  for (int i = 0; i < FB_NW; ++i) t += L.red[i];
  return t;
}
__device__ uint32_t blk_min_u32_fb(int v, FbLds& L) {
  uint32_t x = (uint32_t)v;
  x = ~wave_max_u32(~x);
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) L.red[threadIdx.x / kWave] = x;
  __syncthreads();
  uint32_t t = 0xFFFFFFFFu;
  for (int i = 0; i < FB_NW; ++i) t = min(t, (uint32_t)L.red[i]);
  return t;
}
// Inclusive block scan (u64), one value per thread.
__device__ uint64_t fb_scan_u64(uint64_t v, FbLds& L, uint64_t* total) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const uint64_t incl = wave_incl_scan_u64(v, lane);
  __syncthreads();
  if (lane == kWave - 1) L.red[w] = incl;
  __syncthreads();
  uint64_t off = 0, tot = 0;
  for (int i = 0; i < FB_NW; ++i) {
    off += i < w ? L.red[i] : 0ull;
    tot += L.red[i];
  }
  *total = tot;
  return off + incl;
}
// Streams the row x[0, V) through f(i, x[i]), every element exactly once, in no
// particular order: 16-byte loads, FB_UN of them per thread issued before any is
// used (one scalar load per thread and pass left the passes waiting on memory),
// and the elements before the first 16-byte boundary and after the last whole
// vector one per thread.
constexpr int FB_UN = 4;
template <class F>
__device__ __forceinline__ void fb_stream(const float* __restrict__ x, int64_t V, F&& f) {
  const int tid = threadIdx.x;
  int64_t head = (int64_t)(((16u - ((uint32_t)(uintptr_t)x & 15u)) & 15u) >> 2);
  if (head > V) head = V;
  if (tid < head) f((int64_t)tid, x[tid]);
  const float4* __restrict__ x4 = reinterpret_cast<const float4*>(x + head);
  const int64_t n4 = (V - head) >> 2;
  int64_t j = tid;
  for (; j + (int64_t)(FB_UN - 1) * FB_NT < n4; j += (int64_t)FB_UN * FB_NT) {
    float4 v[FB_UN];
#pragma unroll
    for (int u = 0; u < FB_UN; ++u) v[u] = x4[j + (int64_t)u * FB_NT];
#pragma unroll
    for (int u = 0; u < FB_UN; ++u) {
      const int64_t i = head + 4 * (j + (int64_t)u * FB_NT);
      f(i, v[u].x);
      f(i + 1, v[u].y);
      f(i + 2, v[u].z);
      f(i + 3, v[u].w);
    }
  }
  for (; j < n4; j += FB_NT) {
    const float4 v = x4[j];
    const int64_t i = head + 4 * j;
    f(i, v.x);
    f(i + 1, v.y);
    f(i + 2, v.z);
    f(i + 3, v.w);
  }
  const int64_t t0 = head + 4 * n4;  // fewer than 4 elements left
  if (t0 + tid < V) f(t0 + tid, x[t0 + tid]);
}
// The same over the logits x and the output row o together: r = f(i, x[i], o[i])
// (o[i] is not read, 0 is passed, when READ_O is false), stored to o[i] when
// WRITE_O. The output row holds each element's exp, then its probability,
// between the passes, so the exp is evaluated once per element; it is read
// with the logits, 16 bytes at a time, rather than element by element (a load
// inside the element's work would wait for every load in flight). Rows whose x
// and o differ in 16-byte phase take one element per thread.
template <bool READ_O, bool WRITE_O, class F>
__device__ __forceinline__ void fb_stream_io(const float* __restrict__ x, float* __restrict__ o,
                                             int64_t V, F&& f) {
  const int tid = threadIdx.x;
  auto put = [&](int64_t i, float r) {
    if (WRITE_O) o[i] = r;
  };
  if ((((uint32_t)(uintptr_t)x ^ (uint32_t)(uintptr_t)o) & 15u) != 0) {  // uniform
    for (int64_t i = tid; i < V; i += FB_NT) put(i, f(i, x[i], READ_O ? o[i] : 0.0f));
    return;
  }
  int64_t head = (int64_t)(((16u - ((uint32_t)(uintptr_t)x & 15u)) & 15u) >> 2);
  if (head > V) head = V;
  if (tid < head) put((int64_t)tid, f((int64_t)tid, x[tid], READ_O ? o[tid] : 0.0f));
  const float4* __restrict__ x4 = reinterpret_cast<const float4*>(x + head);
  float4* __restrict__ o4 = reinterpret_cast<float4*>(o + head);
  const int64_t n4 = (V - head) >> 2;
  constexpr int UN = READ_O ? 2 : FB_UN;
  auto one = [&](int64_t j, const float4& v, const float4& w) {
    const int64_t i = head + 4 * j;
    float4 r;
    r.x = f(i, v.x, w.x);
    r.y = f(i + 1, v.y, w.y);
    r.z = f(i + 2, v.z, w.z);
    r.w = f(i + 3, v.w, w.w);
    if (WRITE_O) o4[j] = r;
  };
  int64_t j = tid;
  for (; j + (int64_t)(UN - 1) * FB_NT < n4; j += (int64_t)UN * FB_NT) {
    float4 v[UN], w[UN];
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      v[u] = x4[j + (int64_t)u * FB_NT];
      w[u] = READ_O ? o4[j + (int64_t)u * FB_NT] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int u = 0; u < UN; ++u) one(j + (int64_t)u * FB_NT, v[u], w[u]);
  }
  for (; j < n4; j += FB_NT)
    one(j, x4[j], READ_O ? o4[j] : make_float4(0.0f, 0.0f, 0.0f, 0.0f));
  const int64_t t0 = head + 4 * n4;  // fewer than 4 elements left
  if (t0 + tid < V) put(t0 + tid, f(t0 + tid, x[t0 + tid], READ_O ? o[t0 + tid] : 0.0f));
}

// The distinct probabilities of the row's elements in buckets [bd, bu] (with
// top-k zeroing when mask_k) and their counts, sorted descending as
// ent[i] = (~bits(p) << 32) | count (empty slots, ~0, last): each entry is one
// tie group of the reference's order. Returns their number, or -1 when more than
// FB_KEYS. The occupied hash slots are packed to the front first, so the sort
// covers the next power of two above their number, not the whole table.
// The output row o holds each element's exp (o_is_e) or its probability.
__device__ __forceinline__ int fb_distinct_p(FbLds& L, const float* __restrict__ x,
                                             const float* __restrict__ o, bool o_is_e, int64_t V,
                                             float T, int bd, int bu, float zf, bool mask_k,
                                             float kth) {
  uint32_t* const hk = reinterpret_cast<uint32_t*>(L.ent);
  uint32_t* const hc = hk + FB_TAB;
  for (int i = threadIdx.x; i < FB_TAB; i += FB_NT) { hk[i] = 0u; hc[i] = 0u; }  // 0: empty
  if (threadIdx.x == 0) { L.ndist = 0u; L.nfill = 0u; }
  __syncthreads();
  // (o is only read here: the cast serves the shared streaming helper)
  fb_stream_io<true, false>(x, const_cast<float*>(o), V, [&](int64_t, float xv, float ov) -> float {
    const float sv = xv / T;
    const int b = (int)(key_of_f32(sv) >> FB_SHIFT);
    if (b < bd || b > bu) return 0.0f;
    const uint32_t k = __float_as_uint(fb_pmask(o_is_e ? ov / zf : ov, mask_k, kth)) + 1u;
    uint32_t h = (k * 0x9E3779B1u) >> 19;  // 13 bits
#pragma nounroll
    for (int probe = 0; probe < FB_TAB; ++probe) {  // kept rolled: 16 copies sit in the stream
      const uint32_t old = atomicCAS(&hk[h], 0u, k);
      if (old == 0u || old == k) {
        if (old == 0u) atomicAdd(&L.ndist, 1u);
        atomicAdd(&hc[h], 1u);
        break;
      }
      h = (h + 1) & (FB_TAB - 1);
    }
    return 0.0f;
  });
  __syncthreads();
  const int nd = (int)L.ndist;
  uint64_t e[FB_PER];
#pragma unroll
  for (int t = 0; t < FB_PER; ++t) {
    const int i = threadIdx.x + t * FB_NT;
    e[t] = hk[i] ? (((uint64_t)(~(hk[i] - 1u)) << 32) | hc[i]) : ~0ull;
  }
  __syncthreads();  // the table is read: its words become the packed entries
  if (nd > FB_KEYS) return -1;
#pragma unroll
  for (int t = 0; t < FB_PER; ++t)
    if (e[t] != ~0ull) L.ent[atomicAdd(&L.nfill, 1u)] = e[t];  // slots [0, nd), any order
  for (int i = nd + threadIdx.x; i < FB_TAB; i += FB_NT) L.ent[i] = ~0ull;
  __syncthreads();
  int S = 2;
  while (S < nd) S <<= 1;
  for (int size = 2; size <= S; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < S; i += FB_NT) {
        const int jx = i ^ stride;
        if (jx > i) {
          const bool up = (i & size) == 0;
          const uint64_t ai = L.ent[i], aj = L.ent[jx];
          if ((ai > aj) == up) { L.ent[i] = aj; L.ent[jx] = ai; }
        }
      }
      __syncthreads();
    }
  }
  return nd;
}
__device__ __forceinline__ float fb_ent_p(uint64_t e) { return __uint_as_float(~(uint32_t)(e >> 32)); }

__global__ void __launch_bounds__(FB_NT) to_probs_f32_big_kernel(F32Args a) {
  __shared__ FbLds L;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
  const int64_t row = blockIdx.x;
  if (tid == 0 && row < a.nzero) a.zero[row] = 0u;
  const int g = row < a.nrows[0] ? 0 : 1;
  const int64_t r = g ? row - a.nrows[0] : row;
  const float* __restrict__ x = a.base[g] + r * a.ld[g];
  const int64_t V = a.V;
  const int64_t gid = draft_id_of_row(a.ids, a.tgt_idx, a.k, a.nrows[1], g, r);
  float* o = a.out + row * a.ld_out;
  uint32_t* bits = a.tie_bits ? a.tie_bits + row * a.tie_ld : nullptr;

  // ---- greedy: one-hot at the first maximum (-0 == +0)
  if (a.greedy) {
    uint64_t best = 0;
    fb_stream(x, V, [&](int64_t i, float xv) {
      uint32_t k = key_of_f32(xv);
      if (k == 0x7FFFFFFFu) k = 0x80000000u;
      const uint64_t c = ((uint64_t)k << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)i);
      best = c > best ? c : best;
    });
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const uint64_t w = (uint64_t)__shfl_xor((long long)best, off, kWave);
      best = w > best ? w : best;
    }
    if (lane == 0) L.red[wv] = best;
    __syncthreads();
    uint64_t b = 0;
    for (int w = 0; w < FB_NW; ++w) b = L.red[w] > b ? L.red[w] : b;
    const int64_t am = (int64_t)(0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFu));
    for (int64_t i = tid; i < V; i += FB_NT) o[i] = i == am ? 1.0f : 0.0f;
    if (bits)
      for (int64_t i = tid; i < a.tie_ld; i += FB_NT) bits[i] = 0u;
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
  const float T = a.T;
  const bool use_k = a.use_k, use_p = a.use_p;

  // ---- 1. m, bucket counts and key extremes
  for (int b = tid; b < FB_NB; b += FB_NT) {
    L.cnt[b] = 0u; L.kmin[b] = 0xFFFFFFFFu; L.kmax[b] = 0u; L.mass[b] = 0ull;
  }
  if (tid == 0) { L.i32[0] = 0; L.f32[2] = 0.0f; }
  __syncthreads();
  float mx = -INFINITY;
  fb_stream(x, V, [&](int64_t, float xv) {
    const float sv = xv / T;
    mx = fmaxf(mx, sv);
    const uint32_t k = key_of_f32(sv);
    const int b = (int)(k >> FB_SHIFT);
    atomicAdd(&L.cnt[b], 1u);
    atomicMin(&L.kmin[b], k);
    atomicMax(&L.kmax[b], k);
  });
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
  if (lane == 0) L.red[wv] = __float_as_uint(mx);
  __syncthreads();
  if (tid == 0) {
    float m2 = -INFINITY;
    for (int w = 0; w < FB_NW; ++w) m2 = fmaxf(m2, __uint_as_float((uint32_t)L.red[w]));
    L.f32[0] = m2;
  }
  __syncthreads();
  const float m = L.f32[0];

  // ---- 2. exact normaliser
  U128 acc = {0, 0};
  fb_stream_io<false, true>(x, o, V, [&](int64_t, float xv, float) -> float {
    const float e = exp_det(xv / T - m);
    acc = u128_add(acc, U128{fixed62(e), 0});
    return e;  // the output row holds the exp until the masses pass
  });
  acc = wave_sum_u128(acc);
  __syncthreads();
  if (lane == 0) { L.red[2 * wv] = acc.lo; L.red[2 * wv + 1] = acc.hi; }
  __syncthreads();
  if (tid == 0) {
    U128 z = {0, 0};
    for (int w = 0; w < FB_NW; ++w) z = u128_add(z, U128{L.red[2 * w], L.red[2 * w + 1]});
    L.f32[1] = rn32_u128(z);
  }
  __syncthreads();
  const float zf = L.f32[1];
  auto pfun = [&](uint32_t key) -> float { return exp_det(fb_of_key(key) - m) / zf; };

  // top-k: the k-th largest key. Wave 0 finds its bucket (lane l holds buckets
  // FB_NB - 1 - 64 l - j, j = 0..63, descending), then the bucket's distinct keys
  // give the key itself.
  float kth = 0.0f;
  if (use_k) {
    if (wv == 0) {
      uint32_t c = 0;
      for (int j = 0; j < 64; ++j) c += L.cnt[FB_NB - 1 - 64 * lane - j];
      const uint32_t incl = wave_incl_scan_u32(c, lane);
      const uint64_t hit = __ballot(incl >= (uint32_t)a.top_k);
      const int hl = __ffsll((unsigned long long)hit) - 1;  // top_k < V: some lane hits
      if (lane == hl) {
        uint32_t run = incl - c;
        for (int j = 0; j < 64; ++j) {
          const int b = FB_NB - 1 - 64 * lane - j;
          if (run + L.cnt[b] >= (uint32_t)a.top_k) {
            L.i32[1] = b;
            L.i32[2] = (int32_t)run;  // elements above the bucket
            break;
          }
          run += L.cnt[b];
        }
      }
    }
    __syncthreads();
    const int bk = L.i32[1];
    const uint32_t need = (uint32_t)a.top_k - (uint32_t)L.i32[2];
    const int nd = fb_distinct_p(L, x, o, true, V, T, bk, bk, zf, false, 0.0f);
    if (nd < 0) {
      if (tid == 0) L.i32[0] = 1;
    } else {
      uint64_t c = 0;
#pragma unroll
      for (int t = 0; t < FB_PER; ++t) {
        const uint64_t e = L.ent[tid * FB_PER + t];
        c += e == ~0ull ? 0u : (uint32_t)e;
      }
      uint64_t tot;
      const uint64_t incl = fb_scan_u64(c, L, &tot);
      uint64_t run = incl - c;
      for (int t = 0; t < FB_PER; ++t) {
        const uint64_t e = L.ent[tid * FB_PER + t];
        if (e == ~0ull) break;
        const uint64_t before = run;
        run += (uint32_t)e;
        if (before < need && run >= need) L.f32[2] = fb_ent_p(e);
      }
    }
    __syncthreads();
    kth = L.f32[2];
  }

  // ---- 3. per-bucket masses of the top-k-zeroed p, then the region
  fb_stream_io<true, true>(x, o, V, [&](int64_t, float xv, float e) -> float {
    const float sv = xv / T;
    const float p = e / zf;
    const float pv = fb_pmask(p, use_k, kth);
    if (pv > 0.0f) atomicAdd((unsigned long long*)&L.mass[key_of_f32(sv) >> FB_SHIFT],
                             (unsigned long long)fixed62(pv));
    return p;  // from here on the output row holds the probability
  });
  __syncthreads();
  bool cut = false;
  int bd = 0, bu = -1;
  if (use_p) {
    // every occupied bucket's smallest p, by the whole block (the walk below
    // would otherwise evaluate them one after another on each lane)
    float* const pmin_b = reinterpret_cast<float*>(L.ent);  // free until the region's keys
    for (int b = tid; b < FB_NB; b += FB_NT)
      pmin_b[b] = L.cnt[b] ? fb_pmask(pfun(L.kmin[b]), use_k, kth) : 0.0f;
    __syncthreads();
    if (wv == 0) {
      const float tp = a.top_p;
      uint64_t ms = 0;
      for (int j = 0; j < 64; ++j) ms += L.mass[FB_NB - 1 - 64 * lane - j];
      const uint64_t incl = wave_incl_scan_u64(ms, lane);
      uint64_t run = incl - ms;
      int fb = -1;
      for (int j = 0; j < 64; ++j) {
        const int b = FB_NB - 1 - 64 * lane - j;
        if (L.cnt[b] == 0) continue;
        run += L.mass[b];
        if (!((rn32_u64(run) - pmin_b[b]) < tp)) { fb = b; break; }
      }
      const uint64_t hit = __ballot(fb >= 0);
      if (hit) {
        if (lane == __ffsll((unsigned long long)hit) - 1) L.i32[3] = fb;
      } else if (lane == 0) {
        L.i32[3] = -1;
      }
    }
    __syncthreads();
    const int bs = L.i32[3];
    if (bs >= 0) {
      if (tid == 0) {  // widen while a neighbour holds the same (nonzero) p at the shared edge
        int lo = bs, hi = bs;
        for (;;) {
          int nx = hi + 1;
          while (nx < FB_NB && L.cnt[nx] == 0) ++nx;
          if (nx >= FB_NB) break;
          const float e = fb_pmask(pfun(L.kmax[hi]), use_k, kth);
          if (e > 0.0f && fb_pmask(pfun(L.kmin[nx]), use_k, kth) == e) hi = nx; else break;
        }
        for (;;) {
          int nx = lo - 1;
          while (nx >= 0 && L.cnt[nx] == 0) --nx;
          if (nx < 0) break;
          const float e = fb_pmask(pfun(L.kmin[lo]), use_k, kth);
          if (e > 0.0f && fb_pmask(pfun(L.kmax[nx]), use_k, kth) == e) lo = nx; else break;
        }
        L.i32[4] = lo;
        L.i32[5] = hi;
      }
      __syncthreads();
      cut = true;
      bd = L.i32[4];
      bu = L.i32[5];
    }
  }
  uint64_t nabove = 0, sabove = 0;
  if (cut) {
    for (int b = tid; b < FB_NB; b += FB_NT)
      if (b > bu) { nabove += L.cnt[b]; sabove += L.mass[b]; }
    nabove = fb_sum_u64(nabove, L);
    sabove = fb_sum_u64(sabove, L);
  }

  // ---- 4. the boundary tie group from the region's distinct keys
  // vb: the value of the last kept element; partial: its group keeps only its
  // rstar lowest ids; vb = +inf when no element of the region is kept
  float vb = 0.0f;
  bool partial = false;
  int64_t rstar = 0;
  uint64_t tot = 0;
  if (cut) {
    const int nd = fb_distinct_p(L, x, o, false, V, T, bd, bu, zf, use_k, kth);
    if (nd < 0) {
      if (tid == 0) L.i32[0] = 1;
    } else {
      const float tp = a.top_p;
      // masses and counts of the sorted distinct keys: thread t holds entries
      // FB_PER t .. FB_PER t + FB_PER - 1
      uint64_t mk = 0, ck = 0;
#pragma unroll
      for (int t = 0; t < FB_PER; ++t) {
        const uint64_t e = L.ent[tid * FB_PER + t];
        if (e != ~0ull) {
          const uint32_t c = (uint32_t)e;
          mk += (uint64_t)c * fixed62(fb_ent_p(e));
          ck += c;
        }
      }
      uint64_t mtot, ctot;
      const uint64_t mincl = fb_scan_u64(mk, L, &mtot);
      const uint64_t cincl = fb_scan_u64(ck, L, &ctot);
      // the first key whose last element fails (or is dropped by top-k)
      uint64_t mrun = sabove + mincl - mk;
      int first = 0x7FFFFFFF;
      for (int t = 0; t < FB_PER; ++t) {
        const int i = tid * FB_PER + t;
        const uint64_t e = L.ent[i];
        if (e == ~0ull) break;
        const float pv = fb_ent_p(e);
        mrun += (uint64_t)(uint32_t)e * fixed62(pv);
        const bool dropped = use_k && pv < kth;
        if (dropped || !((rn32_u64(mrun) - pv) < tp)) { first = i; break; }
      }
      const uint32_t f = blk_min_u32_fb(first, L);
      // entry f is the boundary tie group (one entry per distinct p)
      const int g0 = f == 0x7FFFFFFFu ? -1 : (int)f, g1 = g0;
      if (tid == 0 && g0 >= 0) L.f32[4] = fb_ent_p(L.ent[g0]);
      __syncthreads();
      // the mass and count before the group, and the group's count
      uint64_t sb = 0, nb = 0, gc = 0;
      if (g0 >= 0) {
#pragma unroll
        for (int t = 0; t < FB_PER; ++t) {
          const int i = tid * FB_PER + t;
          const uint64_t e = L.ent[i];
          if (e == ~0ull) continue;
          const uint32_t c = (uint32_t)e;
          if (i < g0) {
            sb += (uint64_t)c * fixed62(fb_ent_p(e));
            nb += c;
          } else if (i <= g1) {
            gc += c;
          }
        }
        sb = sabove + fb_sum_u64(sb, L);
        nb = nabove + fb_sum_u64(nb, L);
        gc = fb_sum_u64(gc, L);
      }
      if (g0 < 0) {
        vb = 0.0f;
        tot = sabove + mtot;
        cut = false;  // every region element is kept as the elements above it
      } else {
        const float vf = L.f32[4];
        // members kept: keep_j = rn32(sb + (j+1) f(vf)) - vf < tp holds for a prefix
        // of j (the position-0 rule keeps j = 0 when nothing precedes); top-k-dropped
        // members keep none
        uint64_t r0 = 0;
        if (!(use_k && vf < kth)) {
          const uint64_t P = fixed62(vf);
          if (wv == 0) {
            uint64_t lo = 0, hi = gc;  // answer in [lo, hi]
            while (lo < hi) {
              const uint64_t step = (hi - lo + kWave - 1) / kWave;
              const uint64_t cand = lo + (uint64_t)lane * step;
              const bool keep = cand < hi &&
                                (((rn32_u64(sb + (cand + 1) * P) - vf) < tp) || (nb + cand == 0));
              const int nk = __popcll(__ballot(keep));
              if (nk == 0) break;
              const uint64_t last = lo + (uint64_t)(nk - 1) * step;
              lo = last + 1;
              hi = min(hi, last + step);
            }
            if (lane == 0) L.u64[3] = lo;
          }
          __syncthreads();
          r0 = L.u64[3];
        }
        if (r0 > 0) {
          vb = vf;
          rstar = (int64_t)r0;
          partial = r0 < gc && vf > 0.0f;
          tot = sb + r0 * fixed62(vf);
        } else if (g0 > 0) {  // the last kept element is of the entry before the group
          vb = fb_ent_p(L.ent[g0 - 1]);
          tot = sb;
        } else {              // ... or above the region
          vb = INFINITY;
          tot = sb;
        }
      }
    }
    __syncthreads();
  } else {  // no top-p cut: every element top-k keeps
    uint64_t t0 = 0;
    fb_stream(o, V, [&](int64_t, float p) { t0 += fixed62(fb_pmask(p, use_k, kth)); });
    tot = fb_sum_u64(t0, L);
  }
  const bool unsupported = L.i32[0] != 0;
  const float totf = fmaxf(rn32_u64(tot), 1e-12f);

  // ---- 5. output, tie-group bits, statistics (members ranked by id, one block
  // scan per 1024 ids, only for a partially kept group)
  if (tid == 0) { L.f32[3] = 0.0f; L.i32[7] = 0; }
  __syncthreads();
  uint64_t mbase = 0;
  // Rows whose logits and probabilities both start 16-byte aligned: four
  // consecutive ids per thread, 4,096 per block step, 16-byte loads and stores;
  // member ranks from three ballots per wave (a thread holds at most 4 members)
  // and one barrier per step. Other rows: one id per thread and a block scan
  // per 1,024 ids.
  const bool vec = (((uintptr_t)x | (uintptr_t)o) & 15u) == 0;  // uniform
  const uint64_t lt_mask = (1ull << lane) - 1ull;
  for (int64_t base = 0, step = 0; vec && base < V; base += 4 * FB_NT, ++step) {  // uniform loop
    const int64_t i0 = base + 4 * tid;
    const bool whole = i0 + 3 < V;
    float xv[4], p[4];
    if (whole) {
      const float4 v = *reinterpret_cast<const float4*>(x + i0);
      const float4 w = *reinterpret_cast<const float4*>(o + i0);
      xv[0] = v.x; xv[1] = v.y; xv[2] = v.z; xv[3] = v.w;
      p[0] = w.x; p[1] = w.y; p[2] = w.z; p[3] = w.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xv[j] = i0 + j < V ? x[i0 + j] : 0.0f;
        p[j] = i0 + j < V ? o[i0 + j] : 0.0f;
      }
    }
    float pv[4];
    int b[4];
    uint32_t nib = 0;  // bit j: id i0 + j is a member of the partially kept group
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float sv = xv[j] / T;
      pv[j] = fb_pmask(p[j], use_k, kth);
      b[j] = (int)(key_of_f32(sv) >> FB_SHIFT);
      if (partial && i0 + j < V && pv[j] == vb) nib |= 1u << j;
    }
    uint64_t rank = 0;  // members before id i0
    if (partial) {      // uniform
      const uint32_t c = (uint32_t)__popc(nib);
      uint32_t ex = 0, wt = 0;
#pragma unroll
      for (int bit = 0; bit < 3; ++bit) {
        const uint64_t bb = __ballot((c >> bit) & 1u);
        ex += (uint32_t)__popcll(bb & lt_mask) << bit;
        wt += (uint32_t)__popcll(bb) << bit;
      }
      // slot parity alternates, so a wave a step ahead never overwrites a total
      // still being read: the step between them has its own barrier
      if (lane == 0) L.wt[step & 1][wv] = wt;
      __syncthreads();
      uint32_t off = 0, tot_m = 0;
#pragma unroll
      for (int w = 0; w < FB_NW; ++w) {
        const uint32_t t = L.wt[step & 1][w];
        off += w < wv ? t : 0u;
        tot_m += t;
      }
      rank = mbase + off + ex;
      mbase += tot_m;
    }
    float pf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool mem = (nib >> j) & 1u;
      bool kept = !(use_k && p[j] < kth);
      if (cut) {
        if (b[j] < bd) kept = false;
        else if (b[j] <= bu)
          kept = kept && (pv[j] > vb || (pv[j] == vb && (!partial || rank < (uint64_t)rstar)));
      }
      if (mem) ++rank;
      pf[j] = unsupported ? __builtin_nanf("") : (kept ? p[j] / totf : 0.0f);
      if (i0 + j == gid) {
        L.f32[3] = pf[j];
        if (mem) L.i32[7] = 1;
      }
    }
    if (whole) {
      *reinterpret_cast<float4*>(o + i0) = make_float4(pf[0], pf[1], pf[2], pf[3]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (i0 + j < V) o[i0 + j] = pf[j];
    }
    if (bits) {  // uniform: word q of the row holds ids 32q .. 32q + 31, from 8 lanes
      uint32_t wd = nib;
#pragma unroll
      for (int q = 1; q < 8; ++q) wd |= (uint32_t)__shfl(nib, lane + q, kWave) << (4 * q);
      const int64_t w0 = i0 >> 5;
      if ((lane & 7) == 0 && w0 < a.tie_ld) bits[w0] = wd;
    }
  }
  for (int64_t base = 0; !vec && base < V; base += FB_NT) {  // uniform loop
    const int64_t i = base + tid;
    float p = 0.0f, pv = 0.0f;
    int b = -1;
    if (i < V) {
      const float sv = x[i] / T;
      p = o[i];  // the probability, left by the masses pass
      pv = fb_pmask(p, use_k, kth);
      b = (int)(key_of_f32(sv) >> FB_SHIFT);
    }
    const bool mem = partial && i < V && pv == vb;
    uint64_t rank = 0;
    if (partial) {
      uint64_t tot_m;
      const uint64_t incl = fb_scan_u64(mem ? 1u : 0u, L, &tot_m);
      rank = mbase + incl - (mem ? 1u : 0u);
      mbase += tot_m;
    }
    if (i < V) {
      bool kept = !(use_k && p < kth);
      if (cut) {
        if (b < bd) kept = false;
        else if (b <= bu) kept = kept && (pv > vb || (pv == vb && (!partial || rank < (uint64_t)rstar)));
      }
      const float pf = unsupported ? __builtin_nanf("") : (kept ? p / totf : 0.0f);
      o[i] = pf;
      if (i == gid) {
        L.f32[3] = pf;
        if (mem) L.i32[7] = 1;
      }
    }
    const uint64_t bm = __ballot(mem);
    const int64_t w0 = (base + wv * kWave) >> 5;  // the wave's 64 ids: two words
    if (bits && lane == 0 && w0 < a.tie_ld) {
      bits[w0] = (uint32_t)bm;
      if (w0 + 1 < a.tie_ld) bits[w0 + 1] = (uint32_t)(bm >> 32);
    }
  }
  __syncthreads();
  if (tid == 0 && a.stats) {
    RowStat st = {};
    st.flags = kRowProbs | (L.i32[7] ? kRowGatherTie : 0u) | (unsupported ? kRowUnsupported : 0u);
    st.m = m; st.zf = zf; st.totf = totf; st.mass = tot;
    st.glo = 1; st.ghi = 0; st.argmax = -1;
    st.pgather = (gid >= 0 && gid < V) ? L.f32[3] : 0.0f;
    a.stats[row] = st;
  }
}

hipError_t launch_to_probs_f32(const F32Args& a, int64_t rows, hipStream_t s) {
  if (a.V <= F32_MAXV)
    hipLaunchKernelGGL(to_probs_f32_kernel, dim3((unsigned)rows), dim3(F32_NT), 0, s, a);
  else
    hipLaunchKernelGGL(to_probs_f32_big_kernel, dim3((unsigned)rows), dim3(FB_NT), 0, s, a);
  return hipGetLastError();
}

}  // namespace sdx
