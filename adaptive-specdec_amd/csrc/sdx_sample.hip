// Accept test, residual / bonus inverse-CDF sampling and to_probs output.
//
// Stages after the row statistics (specdec/engine.py:285-303):
//   chunk_kernel    (jobs x chunks) grid. With the accept chain fused in, each
//                   block first replays its batch row's accept chain
//                   u < min(1, p(x)/max(q(x), 1e-10)) with the first-reject
//                   scan (sampling.py:117-129; block 0 of the row publishes
//                   n_acc, flags and the draw: residual at the stop position
//                   or bonus from p_{k+1}), then reduces one chunk of ids to a
//                   ChunkRec: exact fixed62 partial sums that do not yet know
//                   which members of the rows' boundary tie groups are kept.
//   select_kernel   one workgroup per draw: prefix counts of group members
//                   over the chunks give every chunk its member ranks, hence
//                   its exact residual (p - q)_+ and p masses (at most two
//                   chunks per draw, the ones where a group's kept count runs
//                   out, are rescanned in id order); the degenerate-residual
//                   rule (sampling.py:85-88); target floor(u * total); the
//                   chunk holding it; a block scan in id order for the first
//                   id whose prefix mass exceeds it.
// Element probabilities come from an evaluator: codes + RowStat + table for
// 16-bit logits, or dense fp32 probability rows (which have no groups).
#include "sdx_launch.hpp"

namespace sdx {

constexpr int SM_NT = 256;
constexpr int SM_NW = SM_NT / kWave;
constexpr int SM_ROUND = SM_NT * 8;  // ids per block round, 8 per thread

// ---------------------------------------------------------------- block scans
// Exclusive scans over the SM_NT threads of a block; `s` holds SM_NW words.
__device__ inline uint32_t block_excl_u32(uint32_t v, uint32_t* s, uint32_t* total) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const uint32_t incl = wave_incl_scan_u32(v, lane);
  if (lane == kWave - 1) s[w] = incl;
  __syncthreads();
  uint32_t off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < SM_NW; ++i) {
    const uint32_t x = s[i];
    off += i < w ? x : 0u;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return off + incl - v;
}
__device__ inline uint64_t block_excl_u64(uint64_t v, uint64_t* s, uint64_t* total) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const uint64_t incl = wave_incl_scan_u64(v, lane);
  if (lane == kWave - 1) s[w] = incl;
  __syncthreads();
  uint64_t off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < SM_NW; ++i) {
    const uint64_t x = s[i];
    off += i < w ? x : 0ull;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return off + incl - v;
}

// ---------------------------------------------------------------- evaluators
// load8 returns the probabilities of ids idx..idx+7 (0 at or past `lim`) and
// the bitmask of the ids that belong to the row's boundary tie group; those
// carry the group value (the value of a kept member) and the caller zeroes
// the members whose rank is >= rstar.
template <int FMT>
struct Eval16 {
  static constexpr bool kGroups = true;
  const uint16_t* base;
  int64_t ld;
  const uint16_t* base2;
  int64_t ld2;
  int64_t split;
  const RowStat* stats;
  const float* tables;
  float T;

  struct Row {
    const uint16_t* ptr;
    RowStat st;
    const float* tbl;
    float vg;  // probability of a kept group member
  };
  // Whole block: copy the row's table to LDS (call before bind, then sync).
  __device__ void stage(int64_t row, float* lds) const {
    const int n = stats[row].ntbl;
    const float* src = tables + row * kTbl;
    for (int t = threadIdx.x; t < n; t += blockDim.x) lds[t] = src[t];
  }
  __device__ void bind(Row& r, int64_t row, const float* lds) const {
    r.ptr = row < split ? base + row * ld : base2 + (row - split) * ld2;
    r.st = stats[row];
    r.tbl = lds;
    r.vg = r.st.glo <= r.st.ghi ? val16<FMT>(r.st, lds, code_of_key16((uint32_t)r.st.glo), T)
                                : 0.0f;
  }
  __device__ static int32_t rstar(const Row& r) { return r.st.rstar; }
  __device__ uint32_t load8(const Row& r, int64_t idx, int64_t lim, float v[8]) const {
    uint32_t c[8];
    if (idx + 8 <= lim) {  // rows start 16-byte aligned and idx is a multiple of 8
      const uint4 w = *reinterpret_cast<const uint4*>(r.ptr + idx);
      c[0] = w.x & 0xFFFFu; c[1] = w.x >> 16; c[2] = w.y & 0xFFFFu; c[3] = w.y >> 16;
      c[4] = w.z & 0xFFFFu; c[5] = w.z >> 16; c[6] = w.w & 0xFFFFu; c[7] = w.w >> 16;
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) c[t] = idx + t < lim ? r.ptr[idx + t] : 0xFFFFu;
    }
    uint32_t mask = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int cl = idx + t < lim ? cls16(r.st, (int32_t)key_of_code16(c[t])) : 0;
      v[t] = cl == 2 ? val16<FMT>(r.st, r.tbl, c[t], T) : (cl == 1 ? r.vg : 0.0f);
      mask |= (cl == 1 ? 1u : 0u) << t;
    }
    return mask;
  }
};

struct EvalProb {
  static constexpr bool kGroups = false;
  const float* base;
  int64_t ld;
  const float* base2;
  int64_t ld2;
  int64_t split;
  bool vec;
  struct Row {
    const float* ptr;
  };
  __device__ void stage(int64_t, float*) const {}
  __device__ void bind(Row& r, int64_t row, const float*) const {
    r.ptr = row < split ? base + row * ld : base2 + (row - split) * ld2;
  }
  __device__ static int32_t rstar(const Row&) { return 0; }
  __device__ uint32_t load8(const Row& r, int64_t idx, int64_t lim, float v[8]) const {
    if (vec && idx + 8 <= lim) {
      const float4 a = *reinterpret_cast<const float4*>(r.ptr + idx);
      const float4 b = *reinterpret_cast<const float4*>(r.ptr + idx + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) v[t] = idx + t < lim ? r.ptr[idx + t] : 0.0f;
    }
    return 0u;
  }
};

// ---------------------------------------------------------------- accept chain
// The accept chain of batch row b (one thread): fills the draw and returns
// n_acc; *fl receives the row's SDX_FLAG bits.
__device__ inline int64_t accept_chain(const AcceptArgs& a, int64_t b, SampleJob* job,
                                       uint32_t* fl_out) {
  const int k = a.k;
  const int64_t trow0 = b * (k + 1);
  const int64_t drow0 = a.batch * (k + 1) + b * k;
  bool alive = a.active ? a.active[b] != 0 : true;
  int n = 0;
  uint32_t fl = 0;
  for (int i = 0; i < k; ++i) {
    const float px = a.stats[trow0 + i].pgather;
    const float qx = a.stats[drow0 + i].pgather;
    const float ratio = px / fmaxf(qx, 1e-10f);
    const float r1 = fminf(ratio, 1.0f);
    const float u = a.u_accept[b * k + i];
    const bool evaluated = alive && n == i;
    const bool ok = evaluated && (u < r1);
    if (evaluated && fabsf(u - r1) < 1e-5f) fl |= SDX_FLAG_ACCEPT_NEAR_TIE;
    n += ok ? 1 : 0;
    alive = alive && ok;
  }
  for (int i = 0; i <= k; ++i)
    if (a.stats[trow0 + i].flags & kRowNonfinite) fl |= SDX_FLAG_NONFINITE;
  for (int i = 0; i < k; ++i)
    if (a.stats[drow0 + i].flags & kRowNonfinite) fl |= SDX_FLAG_NONFINITE;
  job->prow = n == k ? trow0 + k : trow0 + n;
  job->qrow = n == k ? -1 : drow0 + n;
  job->u = a.u_final[b];
  job->pad = 0;
  *fl_out = fl;
  return n;
}

// ---------------------------------------------------------------- chunk records
struct ChunkArgs {
  AcceptArgs acc;   // acc.stats == null: jobs are given
  SampleJob* jobs;
  int64_t V;
  int64_t chunk;    // ids per chunk (multiple of 8)
  int32_t nchunk;
  ChunkRec* recs;   // [jobs, nchunk]
};

template <class Ev>
__global__ void __launch_bounds__(SM_NT) chunk_kernel(Ev ev, ChunkArgs a) {
  __shared__ float tbl_p[kTbl];
  __shared__ float tbl_q[kTbl];
  __shared__ SampleJob s_job;
  __shared__ uint64_t red64[5 * SM_NW];
  __shared__ uint32_t red32[3 * SM_NW];
  const int64_t j = (int64_t)blockIdx.x / a.nchunk;
  const int c = (int)((int64_t)blockIdx.x % a.nchunk);
  if (threadIdx.x == 0) {
    if (a.acc.stats) {
      SampleJob jb;
      uint32_t fl;
      const int64_t n = accept_chain(a.acc, j, &jb, &fl);
      if (c == 0) {
        a.jobs[j] = jb;
        if (a.acc.n_acc) a.acc.n_acc[j] = n;
        if (a.acc.flags) a.acc.flags[j] = (uint8_t)fl;
      }
      s_job = jb;
    } else {
      s_job = a.jobs[j];
    }
  }
  __syncthreads();
  const SampleJob job = s_job;
  const bool hasq = job.qrow >= 0;
  ev.stage(job.prow, tbl_p);
  if (hasq) ev.stage(job.qrow, tbl_q);
  __syncthreads();
  typename Ev::Row rp, rq;
  ev.bind(rp, job.prow, tbl_p);
  if (hasq) ev.bind(rq, job.qrow, tbl_q);
  const int64_t c0 = (int64_t)c * a.chunk;
  const int64_t c1 = min(a.V, c0 + a.chunk);
  uint64_t p2 = 0, r0 = 0, ra = 0, rb = 0, rpm = 0;
  uint32_t np = 0, nq = 0, ndbl = 0;
  for (int64_t idx = c0 + (int64_t)threadIdx.x * 8; idx < c1; idx += SM_ROUND) {
    float p[8], q[8];
    const uint32_t mp = ev.load8(rp, idx, c1, p);
    if (hasq) {
      const uint32_t mq = ev.load8(rq, idx, c1, q);
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const bool ip = (mp >> t) & 1u, iq = (mq >> t) & 1u;
        const uint64_t wr = fixed62(fmaxf(p[t] - q[t], 0.0f));
        if (!ip) {
          p2 += fixed62(p[t]);
          if (!iq) r0 += wr;
          else { ra += wr; rb += fixed62(p[t]); }
        } else {
          if (!iq) rpm += wr;
          else ++ndbl;
        }
      }
      nq += __popc(mq);
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t)
        if (!((mp >> t) & 1u)) p2 += fixed62(p[t]);
    }
    np += __popc(mp);
  }
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  p2 = wave_sum_u64(p2);
  r0 = wave_sum_u64(r0);
  ra = wave_sum_u64(ra);
  rb = wave_sum_u64(rb);
  rpm = wave_sum_u64(rpm);
  np = wave_sum_u32(np);
  nq = wave_sum_u32(nq);
  ndbl = wave_sum_u32(ndbl);
  if (lane == 0) {
    red64[w] = p2; red64[SM_NW + w] = r0; red64[2 * SM_NW + w] = ra;
    red64[3 * SM_NW + w] = rb; red64[4 * SM_NW + w] = rpm;
    red32[w] = np; red32[SM_NW + w] = nq; red32[2 * SM_NW + w] = ndbl;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    ChunkRec rec = {};
    for (int w2 = 0; w2 < SM_NW; ++w2) {
      rec.p2 += red64[w2]; rec.r0 += red64[SM_NW + w2]; rec.ra += red64[2 * SM_NW + w2];
      rec.rb += red64[3 * SM_NW + w2]; rec.rp += red64[4 * SM_NW + w2];
      rec.np += red32[w2]; rec.nq += red32[SM_NW + w2]; rec.ndbl += red32[2 * SM_NW + w2];
    }
    a.recs[j * a.nchunk + c] = rec;
  }
}

// ---------------------------------------------------------------- exact chunk walk
struct WalkSmem {
  uint32_t s32[SM_NW];
  uint64_t s64[SM_NW];
  int64_t found;
};

// Walks ids [c0, c1) in id order with the member ranks at c0 equal to (bp, bq)
// and returns the chunk's mass (residual when use_r, else p). With t given
// (base <= t), also sets sm.found to the first id whose prefix mass, counted
// from `base`, exceeds t. Whole block.
template <class Ev>
__device__ uint64_t chunk_walk(const Ev& ev, const typename Ev::Row& rp,
                               const typename Ev::Row& rq, bool hasq, bool use_r, int64_t c0,
                               int64_t c1, uint32_t bp, uint32_t bq, uint64_t base, bool find,
                               uint64_t t, WalkSmem& sm) {
  const int32_t sp = Ev::rstar(rp), sq = hasq ? Ev::rstar(rq) : 0;
  uint64_t run = base;
  for (int64_t r0 = c0; r0 < c1; r0 += SM_ROUND) {
    const int64_t idx = r0 + (int64_t)threadIdx.x * 8;
    float p[8], q[8];
    uint32_t mp = 0, mq = 0;
    if (idx < c1) {
      mp = ev.load8(rp, idx, c1, p);
      if (use_r) mq = ev.load8(rq, idx, c1, q);
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u) { p[u] = 0.0f; q[u] = 0.0f; }
    }
    uint32_t rk_p = bp, rk_q = bq;
    if (Ev::kGroups) {  // member ranks: block scan of packed (p count, q count)
      uint32_t tot;
      const uint32_t ex = block_excl_u32((uint32_t)__popc(mp) | ((uint32_t)__popc(mq) << 16),
                                         sm.s32, &tot);
      rk_p += ex & 0xFFFFu;
      rk_q += ex >> 16;
      bp += tot & 0xFFFFu;
      bq += tot >> 16;
    }
    uint64_t w[8], mine = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      float pv = p[u];
      if ((mp >> u) & 1u) { pv = (int32_t)rk_p < sp ? pv : 0.0f; ++rk_p; }
      if (use_r) {
        float qv = q[u];
        if ((mq >> u) & 1u) { qv = (int32_t)rk_q < sq ? qv : 0.0f; ++rk_q; }
        w[u] = fixed62(fmaxf(pv - qv, 0.0f));
      } else {
        w[u] = fixed62(pv);
      }
      mine += w[u];
    }
    uint64_t tot;
    const uint64_t ex = block_excl_u64(mine, sm.s64, &tot);
    if (find) {
      const uint64_t st = run + ex;
      if (st <= t && st + mine > t) {
        uint64_t acc = st;
        int64_t f = -1;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          acc += w[u];
          if (f < 0 && acc > t) f = idx + u;
        }
        sm.found = f;
      }
    }
    run += tot;
  }
  return run - base;
}

// ---------------------------------------------------------------- select
struct SelectArgs {
  const SampleJob* jobs;
  int64_t V;
  int64_t chunk;
  int32_t nchunk;
  const ChunkRec* recs;
  int64_t* y;
};

template <class Ev>
__global__ void __launch_bounds__(SM_NT) select_kernel(Ev ev, SelectArgs a) {
  __shared__ float tbl_p[kTbl];
  __shared__ float tbl_q[kTbl];
  __shared__ WalkSmem sm;
  __shared__ uint64_t s_r[kMaxChunks];
  __shared__ int32_t s_part[2];
  __shared__ int64_t s_pick[4];
  const int64_t j = blockIdx.x;
  const SampleJob job = a.jobs[j];
  const bool hasq = job.qrow >= 0;
  ev.stage(job.prow, tbl_p);
  if (hasq) ev.stage(job.qrow, tbl_q);
  if (threadIdx.x < 2) s_part[threadIdx.x] = -1;
  if (threadIdx.x == 0) s_pick[0] = -1;
  __syncthreads();
  typename Ev::Row rp, rq;
  ev.bind(rp, job.prow, tbl_p);
  if (hasq) ev.bind(rq, job.qrow, tbl_q);
  const int32_t sp = Ev::rstar(rp), sq = hasq ? Ev::rstar(rq) : 0;
  float vp = 0.0f, vq = 0.0f;
  if constexpr (Ev::kGroups) {
    vp = rp.vg;
    if (hasq) vq = rq.vg;
  }

  // ---- chunk c (thread c): member ranks at its start, exact p mass, and the
  // residual mass when both rows' kept members are all-or-nothing inside it
  const int c = threadIdx.x;
  ChunkRec rec = {};
  if (c < a.nchunk) rec = a.recs[j * a.nchunk + c];
  uint64_t tot_n;
  const uint64_t ex_n = block_excl_u64((uint64_t)rec.np | ((uint64_t)rec.nq << 32), sm.s64, &tot_n);
  const uint32_t bp = (uint32_t)ex_n, bq = (uint32_t)(ex_n >> 32);
  const uint32_t kp = (uint32_t)min<int64_t>(max<int64_t>((int64_t)sp - bp, 0), rec.np);
  const uint32_t kq = (uint32_t)min<int64_t>(max<int64_t>((int64_t)sq - bq, 0), rec.nq);
  const uint64_t pmass = rec.p2 + (uint64_t)kp * fixed62(vp);
  uint64_t rmass = 0;
  if (hasq && c < a.nchunk) {
    const bool pall = kp == rec.np, pnone = kp == 0, qall = kq == rec.nq, qnone = kq == 0;
    if ((pall || pnone) && (qall || qnone)) {
      rmass = rec.r0 + (qall ? rec.ra : rec.rb);
      if (pall && rec.np) {
        rmass += rec.rp;
        rmass += (uint64_t)rec.ndbl * fixed62(fmaxf(vp - (qall ? vq : 0.0f), 0.0f));
      }
    } else {
      if (!(pall || pnone)) s_part[0] = c;
      if (!(qall || qnone)) s_part[1] = c;
    }
  }
  __syncthreads();
  // ---- rescan the (at most two) chunks where a group's kept members run out
  if (hasq) {
    const int pa = s_part[0], pb = s_part[1];
    for (int i = 0; i < 2; ++i) {
      const int cc = i == 0 ? pa : pb;
      if (cc < 0 || (i == 1 && cc == pa)) continue;
      if (c == cc) s_pick[1] = ((int64_t)bq << 32) | bp;
      __syncthreads();
      const int64_t packed = s_pick[1];
      const int64_t c0 = (int64_t)cc * a.chunk;
      const uint64_t m = chunk_walk(ev, rp, rq, true, true, c0, min(a.V, c0 + a.chunk),
                                    (uint32_t)(packed & 0xFFFFFFFF), (uint32_t)(packed >> 32),
                                    0, false, 0, sm);
      if (c == cc) rmass = m;
      __syncthreads();
    }
  }
  // ---- totals, degenerate-residual rule, the chunk holding the target
  uint64_t tot_r, tot_p;
  const uint64_t ex_r = block_excl_u64(rmass, sm.s64, &tot_r);
  const uint64_t ex_p = block_excl_u64(pmass, sm.s64, &tot_p);
  const bool use_r = hasq && rn32_u64(tot_r) > 1e-9f;
  const uint64_t tot = use_r ? tot_r : tot_p;
  if (tot == 0) {
    if (threadIdx.x == 0) a.y[j] = -1;
    return;
  }
  const uint64_t t = uniform_threshold(job.u, tot);
  const uint64_t ex = use_r ? ex_r : ex_p, mine = use_r ? rmass : pmass;
  if (c < a.nchunk && ex <= t && ex + mine > t) {
    s_pick[0] = c;
    s_pick[1] = ((int64_t)bq << 32) | bp;
    s_pick[2] = (int64_t)ex;
  }
  __syncthreads();
  const int64_t cstar = s_pick[0];
  if (cstar < 0) {  // unreachable: masses sum to tot > t
    if (threadIdx.x == 0) a.y[j] = -1;
    return;
  }
  const int64_t packed = s_pick[1];
  const uint64_t base = (uint64_t)s_pick[2];
  if (threadIdx.x == 0) sm.found = -1;
  __syncthreads();
  const int64_t c0 = cstar * a.chunk;
  chunk_walk(ev, rp, rq, hasq, use_r, c0, min(a.V, c0 + a.chunk), (uint32_t)(packed & 0xFFFFFFFF),
             (uint32_t)(packed >> 32), base, true, t, sm);
  __syncthreads();
  if (threadIdx.x == 0) a.y[j] = sm.found;
}

// ---------------------------------------------------------------- to_probs output
struct MaterializeArgs {
  int64_t V;
  int64_t chunk;
  int32_t nchunk;
  uint32_t* counts;  // [rows, nchunk] group members per chunk (partial rows only)
  float* out;
  int64_t ld_out;
};

__device__ __forceinline__ bool partial_group(const RowStat& st) {
  return st.rstar > 0 && st.rstar < st.gcount;
}

template <int FMT>
__global__ void __launch_bounds__(SM_NT) member_count_kernel(Eval16<FMT> ev, MaterializeArgs a) {
  __shared__ uint32_t red[SM_NW];
  const int64_t row = (int64_t)blockIdx.x / a.nchunk;
  const int64_t cidx = (int64_t)blockIdx.x % a.nchunk;
  const RowStat st = ev.stats[row];
  if (!partial_group(st)) return;
  const uint16_t* ptr = row < ev.split ? ev.base + row * ev.ld : ev.base2 + (row - ev.split) * ev.ld2;
  const int64_t c0 = cidx * a.chunk;
  const int64_t c1 = min(a.V, c0 + a.chunk);
  uint32_t cnt = 0;
  for (int64_t i = c0 + threadIdx.x; i < c1; i += SM_NT) {
    const int32_t kk = (int32_t)key_of_code16(ptr[i]);
    cnt += (kk >= st.glo && kk <= st.ghi) ? 1u : 0u;
  }
  cnt = wave_sum_u32(cnt);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = cnt;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
    for (int w = 0; w < SM_NW; ++w) t += red[w];
    a.counts[row * a.nchunk + cidx] = t;
  }
}

template <int FMT>
__global__ void __launch_bounds__(SM_NT) materialize16_kernel(Eval16<FMT> ev, MaterializeArgs a) {
  __shared__ float tbl[kTbl];
  __shared__ uint32_t s32[SM_NW];
  const int64_t row = (int64_t)blockIdx.x / a.nchunk;
  const int64_t cidx = (int64_t)blockIdx.x % a.nchunk;
  ev.stage(row, tbl);
  __syncthreads();
  typename Eval16<FMT>::Row r;
  ev.bind(r, row, tbl);
  const bool part = partial_group(r.st);
  uint32_t rank = 0;
  if (part) {  // members in earlier chunks
    uint32_t v = 0;
    for (int64_t c = threadIdx.x; c < cidx; c += SM_NT) v += a.counts[row * a.nchunk + c];
    block_excl_u32(v, s32, &rank);
  }
  const int64_t c0 = cidx * a.chunk;
  const int64_t c1 = min(a.V, c0 + a.chunk);
  float* o = a.out + row * a.ld_out;
  for (int64_t r0 = c0; r0 < c1; r0 += SM_ROUND) {
    const int64_t idx = r0 + (int64_t)threadIdx.x * 8;
    float p[8];
    uint32_t m = 0;
    if (idx < c1) m = ev.load8(r, idx, c1, p);
    if (part) {
      uint32_t tot;
      uint32_t rk = rank + block_excl_u32((uint32_t)__popc(m), s32, &tot);
      rank += tot;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if ((m >> u) & 1u) { if ((int32_t)rk >= r.st.rstar) p[u] = 0.0f; ++rk; }
    } else if (r.st.rstar <= 0) {
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if ((m >> u) & 1u) p[u] = 0.0f;
    }
    if (idx < c1) {
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (idx + u < c1) o[idx + u] = p[u];
    }
  }
}

// ---------------------------------------------------------------- residual_probs output

__global__ void __launch_bounds__(SM_NT) residual_norm_kernel(ResidualNormArgs a) {
  __shared__ float s_tot;
  __shared__ int s_use_r;
  const int64_t row = (int64_t)blockIdx.x / a.nchunk;
  const int64_t cidx = (int64_t)blockIdx.x % a.nchunk;
  if (threadIdx.x == 0) {
    // dense fp32 rows have no tie groups: residual mass is r0, p mass p2
    uint64_t totR = 0, totP = 0;
    for (int c = 0; c < a.nchunk; ++c) {
      totR += a.recs[row * a.nchunk + c].r0;
      totP += a.recs[row * a.nchunk + c].p2;
    }
    const float fr = rn32_u64(totR);
    const bool use_r = fr > 1e-9f;
    s_use_r = use_r;
    s_tot = fmaxf(use_r ? fr : rn32_u64(totP), 1e-12f);
  }
  __syncthreads();
  const float tot = s_tot;
  const bool use_r = s_use_r != 0;
  const int64_t c0 = cidx * a.chunk;
  const int64_t c1 = min(a.V, c0 + a.chunk);
  const float* p = a.p + row * a.ld;
  const float* q = a.q + row * a.ld;
  float* o = a.out + row * a.ld_out;
  for (int64_t idx = c0 + threadIdx.x; idx < c1; idx += SM_NT) {
    const float r = use_r ? fmaxf(p[idx] - q[idx], 0.0f) : p[idx];
    o[idx] = r / tot;
  }
}

// gather_prob
__global__ void gather_kernel(const float* probs, int64_t rows, int64_t V, int64_t ld,
                              const int64_t* ids, float* out) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int64_t i = ids[r];
  out[r] = (i >= 0 && i < V) ? probs[r * ld + i] : 0.0f;
}

// ---------------------------------------------------------------- launch helpers
template <class Ev>
static hipError_t launch_chunks(const Ev& ev, const AcceptArgs* acc, SampleJob* jobs,
                                int64_t njobs, int64_t V, int64_t chunk, int nchunk,
                                ChunkRec* recs, hipStream_t s) {
  ChunkArgs ca = {};
  if (acc) ca.acc = *acc;
  ca.jobs = jobs;
  ca.V = V;
  ca.chunk = chunk;
  ca.nchunk = nchunk;
  ca.recs = recs;
  hipLaunchKernelGGL((chunk_kernel<Ev>), dim3((unsigned)(nchunk * njobs)), dim3(SM_NT), 0, s, ev,
                     ca);
  return hipGetLastError();
}

template <class Ev>
static hipError_t launch_draw(const Ev& ev, const AcceptArgs* acc, SampleJob* jobs,
                              int64_t njobs, int64_t V, int64_t chunk, int nchunk,
                              ChunkRec* recs, int64_t* y, hipStream_t s) {
  if (nchunk > kMaxChunks || nchunk > SM_NT) return hipErrorInvalidValue;
  hipError_t e = launch_chunks(ev, acc, jobs, njobs, V, chunk, nchunk, recs, s);
  if (e != hipSuccess) return e;
  SelectArgs sa{jobs, V, chunk, nchunk, recs, y};
  hipLaunchKernelGGL((select_kernel<Ev>), dim3((unsigned)njobs), dim3(SM_NT), 0, s, ev, sa);
  return hipGetLastError();
}

hipError_t launch_draw16(int fmt, const RowSource16& src, const RowStat* stats,
                         const float* tables, float T, const AcceptArgs* acc, SampleJob* jobs,
                         int64_t njobs, int64_t V, int64_t chunk, int nchunk, ChunkRec* recs,
                         int64_t* y, hipStream_t s) {
  if (!src.vec) return hipErrorInvalidValue;
  if (fmt == SDX_BF16) {
    Eval16<SDX_BF16> ev{src.base, src.ld, src.base2, src.ld2, src.split, stats, tables, T};
    return launch_draw(ev, acc, jobs, njobs, V, chunk, nchunk, recs, y, s);
  }
  Eval16<SDX_F16> ev{src.base, src.ld, src.base2, src.ld2, src.split, stats, tables, T};
  return launch_draw(ev, acc, jobs, njobs, V, chunk, nchunk, recs, y, s);
}

hipError_t launch_draw_probs(const RowSourceF32& src, const AcceptArgs* acc, SampleJob* jobs,
                             int64_t njobs, int64_t V, int64_t chunk, int nchunk, ChunkRec* recs,
                             int64_t* y, hipStream_t s) {
  EvalProb ev{src.base, src.ld, src.base2, src.ld2, src.split, src.vec};
  return launch_draw(ev, acc, jobs, njobs, V, chunk, nchunk, recs, y, s);
}

hipError_t launch_chunk_mass_probs(const RowSourceF32& src, SampleJob* jobs, int64_t njobs,
                                   int64_t V, int64_t chunk, int nchunk, ChunkRec* recs,
                                   hipStream_t s) {
  EvalProb ev{src.base, src.ld, src.base2, src.ld2, src.split, src.vec};
  return launch_chunks(ev, nullptr, jobs, njobs, V, chunk, nchunk, recs, s);
}

hipError_t launch_materialize16(int fmt, const RowSource16& src, const RowStat* stats,
                                const float* tables, float T, int64_t rows, int64_t V,
                                int64_t chunk, int nchunk, uint32_t* counts, float* out,
                                int64_t ld_out, hipStream_t s) {
  if (!src.vec) return hipErrorInvalidValue;
  MaterializeArgs ma{V, chunk, nchunk, counts, out, ld_out};
  const dim3 grid((unsigned)(nchunk * rows));
  if (fmt == SDX_BF16) {
    Eval16<SDX_BF16> ev{src.base, src.ld, src.base2, src.ld2, src.split, stats, tables, T};
    hipLaunchKernelGGL((member_count_kernel<SDX_BF16>), grid, dim3(SM_NT), 0, s, ev, ma);
    hipLaunchKernelGGL((materialize16_kernel<SDX_BF16>), grid, dim3(SM_NT), 0, s, ev, ma);
  } else {
    Eval16<SDX_F16> ev{src.base, src.ld, src.base2, src.ld2, src.split, stats, tables, T};
    hipLaunchKernelGGL((member_count_kernel<SDX_F16>), grid, dim3(SM_NT), 0, s, ev, ma);
    hipLaunchKernelGGL((materialize16_kernel<SDX_F16>), grid, dim3(SM_NT), 0, s, ev, ma);
  }
  return hipGetLastError();
}

hipError_t launch_residual_norm(const ResidualNormArgs& a, int64_t rows, hipStream_t s) {
  hipLaunchKernelGGL(residual_norm_kernel, dim3((unsigned)(a.nchunk * rows)), dim3(SM_NT), 0,
                     s, a);
  return hipGetLastError();
}

hipError_t launch_gather(const float* probs, int64_t rows, int64_t V, int64_t ld, const int64_t* ids,
                         float* out, hipStream_t s) {
  const int nt = 256;
  hipLaunchKernelGGL(gather_kernel, dim3((unsigned)((rows + nt - 1) / nt)), dim3(nt), 0, s, probs,
                     rows, V, ld, ids, out);
  return hipGetLastError();
}

}  // namespace sdx
