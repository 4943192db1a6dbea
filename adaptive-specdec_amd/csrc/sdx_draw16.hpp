// The verify draw over 16-bit logits and what the other draws share with it:
// block scans, the 16-bit evaluator, the accept chains, the record helpers,
// the record pass and walks, and the draw body (draw16_body). Included by
// sdx_sample.hip (the draw kernels) and sdx_rowstream.hip (the fused verify
// kernel, whose draw blocks run the same body once the row blocks of their
// batch row have published its statistics).
#pragma once
#include "sdx_launch.hpp"

namespace sdx {

constexpr int SM_NT = 256;
constexpr int SM_NW = SM_NT / kWave;
constexpr int SM_ROUND = SM_NT * 8;  // ids per block round, 8 per thread

// ---------------------------------------------------------------- block scans
// Exclusive scans over the SM_NT threads of a block; `s` holds SM_NW words.
template <int NW = SM_NW>
__device__ inline uint32_t block_excl_u32(uint32_t v, uint32_t* s, uint32_t* total) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const uint32_t incl = wave_incl_scan_u32(v, lane);
  if (lane == kWave - 1) s[w] = incl;
  __syncthreads();
  uint32_t off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const uint32_t x = s[i];
    off += i < w ? x : 0u;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return off + incl - v;
}
template <int NW = SM_NW>
__device__ inline uint64_t block_excl_u64(uint64_t v, uint64_t* s, uint64_t* total) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const uint64_t incl = wave_incl_scan_u64(v, lane);
  if (lane == kWave - 1) s[w] = incl;
  __syncthreads();
  uint64_t off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const uint64_t x = s[i];
    off += i < w ? x : 0ull;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return off + incl - v;
}

// ---------------------------------------------------------------- evaluators
// fetch() loads the raw data of ids idx..idx+7 (ids at or past `lim` read as
// nothing); eval() turns it into probabilities (0 past `lim`) and returns in
// bits 0..7 the ids in the row's boundary tie group (those carry the group
// value, the value of a kept member; the caller zeroes the members whose rank
// is >= rstar) and in bits 8..15 the ids that may carry probability. load8()
// is both, returning the group bits.
template <int FMT>
struct Eval16 {
  static constexpr bool kGroups = true;
  static constexpr int kFmt = FMT;
  static constexpr int kLdsTbl = kTbl;
  using Raw = uint4;
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
  // Whole block: copy the row's table to LDS (then sync, then bind with it).
  __device__ void stage(int64_t row, float* lds) const {
    const int n = stats[row].ntbl;
    const float* src = tables + row * kTbl;
    for (int t = threadIdx.x; t < n; t += blockDim.x) lds[t] = src[t];
  }
  // `tbl`: the staged LDS copy of the row's table.
  __device__ void bind(Row& r, int64_t row, const float* tbl) const {
    r.ptr = row < split ? base + row * ld : base2 + (row - split) * ld2;
    r.st = stats[row];
    r.tbl = tbl;
    r.vg = r.st.glo <= r.st.ghi
               ? val16<FMT>(r.st, r.tbl, code_of_key16((uint32_t)r.st.glo), T)
               : 0.0f;
  }
  __device__ static int32_t rstar(const Row& r) { return r.st.rstar; }
  // Is id a member of the row's partially kept boundary tie group?
  __device__ static bool in_tie_group(const Row& r, int64_t id) {
    if (!(r.st.rstar > 0 && r.st.rstar < r.st.gcount)) return false;
    const int32_t key = (int32_t)key_of_code16(r.ptr[id]);
    return key >= r.st.glo && key <= r.st.ghi;
  }
  __device__ Raw fetch(const Row& r, int64_t idx, int64_t lim) const {
    if (idx + 8 <= lim)  // rows start 16-byte aligned and idx is a multiple of 8
      return *reinterpret_cast<const uint4*>(r.ptr + idx);
    uint32_t w[4] = {0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu};
#pragma unroll
    for (int t = 0; t < 8; ++t)
      if (idx + t < lim)
        w[t >> 1] = (w[t >> 1] & ~(0xFFFFu << (16 * (t & 1)))) |
                    ((uint32_t)r.ptr[idx + t] << (16 * (t & 1)));
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
  // Branch-free: every id reads the table at a clamped index and selects;
  // kept keys below the table (rare) take the exp path under a wave vote.
  __device__ uint32_t eval(const Row& r, int64_t idx, int64_t lim, const Raw& raw,
                           float v[8]) const {
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    const int32_t klo = r.st.klo, glo = r.st.glo, ghi = r.st.ghi, kmax = r.st.kmax;
    const int32_t tmax = max(r.st.ntbl - 1, 0);
    // ids in range: idx + t < lim exactly when t < nv (a 32-bit count of at most 8)
    const int32_t nv = (int32_t)min(max(lim - idx, (int64_t)0), (int64_t)8);
    const uint32_t kw[4] = {keys2_of_codes2(w[0]), keys2_of_codes2(w[1]), keys2_of_codes2(w[2]),
                            keys2_of_codes2(w[3])};
    uint32_t mask = 0, slow = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int32_t key = (int32_t)((t & 1) ? (kw[t >> 1] >> 16) : (kw[t >> 1] & 0xFFFFu));
      const bool live = t < nv && key >= klo;
      const bool mem = live && key >= glo && key <= ghi;
      const int32_t tt = kmax - key;
      const float tv = r.tbl[min(max(tt, 0), tmax)];
      v[t] = live ? (mem ? r.vg : tv) : 0.0f;
      mask |= ((mem ? 1u : 0u) << t) | ((live ? 1u : 0u) << (8 + t));
      slow |= (live && !mem && tt > tmax ? 1u : 0u) << t;
    }
    if (__builtin_expect(__ballot(slow != 0) != 0, 0)) {
#pragma unroll
      for (int t = 0; t < 8; ++t)
        if ((slow >> t) & 1u) {
          const uint32_t code = (t & 1) ? (w[t >> 1] >> 16) : (w[t >> 1] & 0xFFFFu);
          v[t] = val16_exp<FMT>(code, T, r.st.m, r.st.zf, r.st.totf);
        }
    }
    return mask;
  }
  __device__ uint32_t load8(const Row& r, int64_t idx, int64_t lim, float v[8]) const {
    return eval(r, idx, lim, fetch(r, idx, lim), v) & 0xFFu;
  }
};

// ---------------------------------------------------------------- accept chain
// Wave 0, one lane per draft position (64 at a time): the accept chain of
// batch row b. Returns n_acc and fills the draw; *fl_out gets the SDX_FLAG bits.
// Position i is evaluated iff the row is active and every earlier position
// accepted, so the chain stops at the first rejection.
__device__ inline int64_t accept_chain_wave(const AcceptArgs& a, int64_t b, SampleJob* job,
                                            uint32_t* fl_out) {
  const int lane = threadIdx.x & (kWave - 1);
  const RowGeom gm = row_geom(a, b);
  const int k = gm.k;
  const int64_t trow0 = gm.trow0, drow0 = gm.drow0;
  const bool alive = (a.active ? a.active[b] != 0 : true) && !gm.bad;
  int n = alive ? k : 0;
  uint32_t fl = gm.bad ? (uint32_t)SDX_FLAG_BAD_ROW : 0u;
  for (int i0 = 0; alive && n == k && i0 < k; i0 += kWave) {  // uniform loop
    const int i = i0 + lane;
    bool ok = true, near = false;
    if (i < k) {
      const float px = a.stats[trow0 + i].pgather;
      const float qx = a.stats[drow0 + i].pgather;
      const float r1 = fminf(px / fmaxf(qx, 1e-10f), 1.0f);
      const float u = a.u_accept[gm.ibase + i];
      ok = u < r1;
      near = fabsf(u - r1) < 1e-5f;
    }
    const uint64_t fm = __ballot(!ok);
    const int first = fm ? __ffsll((unsigned long long)fm) - 1 : kWave;
    if (__ballot(near && lane <= first)) fl |= SDX_FLAG_ACCEPT_NEAR_TIE;
    if (fm) n = i0 + first;
  }
  // evaluated tests (positions 0..n, at most k - 1) whose drafted token sits in
  // a partially kept tie group of its target or draft row
  const int ne = alive ? (n < k ? n + 1 : k) : 0;
  for (int i0 = 0; i0 < ne; i0 += kWave) {
    const int i = i0 + lane;
    uint32_t rf = 0;
    if (i < ne) rf = a.stats[trow0 + i].flags | a.stats[drow0 + i].flags;
    if (__ballot((rf & kRowGatherTie) != 0)) fl |= SDX_FLAG_TIE_ORDER;
  }
  for (int i0 = 0; i0 < 2 * k + 1; i0 += kWave) {
    const int i = i0 + lane;
    uint32_t rf = 0;
    if (i < 2 * k + 1) rf = a.stats[i <= k ? trow0 + i : drow0 + (i - k - 1)].flags;
    if (__ballot((rf & kRowNonfinite) != 0)) fl |= SDX_FLAG_NONFINITE;
    if (__ballot((rf & kRowUnsupported) != 0)) fl |= SDX_FLAG_UNSUPPORTED;
    if (__ballot((rf & kRowBadWs) != 0)) fl |= SDX_FLAG_WORKSPACE;
  }
  job->prow = n == k ? trow0 + k : trow0 + n;
  job->qrow = n == k ? -1 : drow0 + n;
  job->u = a.u_final[b];
  job->pad = 0;
  *fl_out = fl;
  return n;
}

// ---------------------------------------------------------------- record helpers
// Records cross blocks on different XCDs: word-wise agent-scope atomics, which
// no XCD's L2 holds stale.
__device__ inline void store_rec(ChunkRec* dst, const ChunkRec& r) {
  uint64_t* d = reinterpret_cast<uint64_t*>(dst);
  const uint64_t* s = reinterpret_cast<const uint64_t*>(&r);
#pragma unroll
  for (int i = 0; i < 8; ++i)
    __hip_atomic_store(d + i, s[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline ChunkRec load_rec(const ChunkRec* src) {
  ChunkRec r;
  const uint64_t* s = reinterpret_cast<const uint64_t*>(src);
  uint64_t* d = reinterpret_cast<uint64_t*>(&r);
#pragma unroll
  for (int i = 0; i < 8; ++i)
    d[i] = __hip_atomic_load(s + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return r;
}

// Exact residual / p masses of a record once the member ranks at its start
// are known; false when a group's kept members run out inside it (then only
// an id-order walk gives the residual mass).
__device__ inline bool rec_masses(const ChunkRec& rec, uint32_t bp, uint32_t bq, int32_t sp,
                                  int32_t sq, float vp, float vq, bool hasq, uint64_t* pmass,
                                  uint64_t* rmass) {
  const uint32_t kp = (uint32_t)min<int64_t>(max<int64_t>((int64_t)sp - bp, 0), rec.np);
  const uint32_t kq = (uint32_t)min<int64_t>(max<int64_t>((int64_t)sq - bq, 0), rec.nq);
  *pmass = rec.p2 + (uint64_t)kp * fixed62(vp);
  *rmass = 0;
  if (!hasq) return true;
  const bool pall = kp == rec.np, pnone = kp == 0, qall = kq == rec.nq, qnone = kq == 0;
  if (!((pall || pnone) && (qall || qnone))) return false;
  uint64_t m = rec.r0 + (qall ? rec.ra : rec.rb);
  if (pall && rec.np) {
    m += rec.rp;
    m += (uint64_t)rec.ndbl * fixed62(fmaxf(vp - (qall ? vq : 0.0f), 0.0f));
  }
  *rmass = m;
  return true;
}

// Loads of what other blocks of the same launch published (COH: the fused
// verify kernel, where a row block's statistics and table reach the draw
// blocks of its batch row through device-coherent accesses; every XCD has its
// own L2, and agent-scope atomic loads read past a stale copy in it).
template <bool COH>
__device__ __forceinline__ void ld_rowstat(const RowStat* p, uint4& w0, uint4& w1, uint4& w2,
                                           uint4& w3) {
  if (COH) {
    const uint64_t* s = reinterpret_cast<const uint64_t*>(p);
    uint64_t x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = __hip_atomic_load(s + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    w0 = make_uint4((uint32_t)x[0], (uint32_t)(x[0] >> 32), (uint32_t)x[1], (uint32_t)(x[1] >> 32));
    w1 = make_uint4((uint32_t)x[2], (uint32_t)(x[2] >> 32), (uint32_t)x[3], (uint32_t)(x[3] >> 32));
    w2 = make_uint4((uint32_t)x[4], (uint32_t)(x[4] >> 32), (uint32_t)x[5], (uint32_t)(x[5] >> 32));
    w3 = make_uint4((uint32_t)x[6], (uint32_t)(x[6] >> 32), (uint32_t)x[7], (uint32_t)(x[7] >> 32));
  } else {
    const uint4* s = reinterpret_cast<const uint4*>(p);
    w0 = s[0]; w1 = s[1]; w2 = s[2]; w3 = s[3];
  }
}
template <bool COH>
__device__ __forceinline__ float ld_f32(const float* p) {
  if (COH)
    return __uint_as_float(__hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT));
  return *p;
}

// ---------------------------------------------------------------- verify draw, 16-bit rows
// The verify path's accept chain and draw over bf16 / fp16 logits, laid out
// for nucleus rows (few ids carry p mass):
//  - wave 0 of every block loads the RowStats of its batch row's 2k+1 rows at
//    once (one lane per row), replays the accept chain from them and leaves
//    the draw's two RowStats in LDS;
//  - every wave owns one record of kRec16 ids (four 512-id rounds) and issues
//    all of its loads at once; the draw's tables are staged meanwhile;
//  - common case (the nucleus cut at a positive value, q's tie group one
//    value or none, the record inside the row): the ids that may carry p mass
//    are found by a signed 16-bit compare of the raw code with the cut, q's
//    group members by a code compare; the p-live ids are compacted into a
//    per-wave LDS list and evaluated one per lane, their masses summed in
//    registers; one wave reduction per record;
//  - otherwise every id is evaluated in place.
// The block completing a job's records selects as draw_kernel does, with
// walks that issue a record's loads before scanning it.
constexpr int kRec16 = 4 * kDrawSub;
constexpr int kRec16Rounds = kRec16 / kDrawSub;
constexpr int kMaxRec16 = (int)((kMaxVocabBf16 + kRec16 - 1) / kRec16);  // records of the largest row
constexpr int kLst16 = kDrawSub + kWave;  // one round of ids plus a leftover below 64

template <int FMT>
struct Draw16Args {
  AcceptArgs acc;
  Eval16<FMT> ev;
  int64_t V;
  int32_t nrec;        // records per job, kRec16 ids each
  int32_t nblk;        // blocks per job
  int32_t xcd;         // jobs a multiple of 8: a job's blocks on one XCD
  ChunkRec* recs;      // [jobs, nrec]
  uint32_t* counters;  // [jobs], zero on entry; the completing block resets its job's
  uint32_t* job_cnt;   // fused kernel: [jobs] row arrivals, reset with the counter; or null
  int64_t* y;
};

// Wave 0: the accept chain of batch row b, as accept_chain_wave, from the
// RowStats of its 2k+1 rows (2k+1 <= 64): lane i holds row i (target
// positions 0..k, then the k draft rows). The draw's RowStats go to st[0] (p)
// and st[1] (q, for a residual draw).
template <int FMT, bool COH>
__device__ inline int64_t chain16_wave(const AcceptArgs& a, const Eval16<FMT>& ev, int64_t b,
                                       SampleJob* job, uint32_t* fl_out, RowStat* st) {
  const int lane = threadIdx.x & (kWave - 1);
  const RowGeom gm = row_geom(a, b);
  const int k = gm.k;
  const int64_t trow0 = gm.trow0, drow0 = gm.drow0;
  const int nr = 2 * k + 1;
  uint4 w0 = make_uint4(0, 0, 0, 0), w1 = w0, w2 = w0, w3 = w0;
  if (lane < nr) {
    const int64_t row = lane <= k ? trow0 + lane : drow0 + (lane - k - 1);
    ld_rowstat<COH>(a.stats + row, w0, w1, w2, w3);
  }
  const float u = lane < k ? a.u_accept[gm.ibase + lane] : 2.0f;
  const float uf = a.u_final[b];
  const bool alive = (a.active ? a.active[b] != 0 : true) && !gm.bad;
  // drafted tokens the row kernel left unranked (their tie group spans several
  // values; rare): the wave counts the group members before the token
  uint64_t todo = __ballot(lane < nr && lane != k && (w3.x & kRowRank) != 0);
  while (todo) {  // uniform
    const int l = __ffsll((unsigned long long)todo) - 1;
    todo &= todo - 1;
    const int i = l < k ? l : l - k - 1;  // draft position of that row
    const int64_t row = l <= k ? trow0 + l : drow0 + i;
    const uint16_t* ptr = row < ev.split ? ev.base + row * ev.ld : ev.base2 + (row - ev.split) * ev.ld2;
    const int64_t gid = a.draft_ids[gm.ibase + i];
    const int32_t glo = (int32_t)rdlane(w1.z, l), ghi = (int32_t)rdlane(w1.w, l);
    uint32_t cnt = 0;
    for (int64_t e = lane; e < gid; e += kWave) {
      const int32_t kk = (int32_t)key_of_code16(ptr[e]);
      cnt += (kk >= glo && kk <= ghi) ? 1u : 0u;
    }
    cnt = wave_sum_u32(cnt);
    const int32_t rstar = (int32_t)rdlane(w2.x, l);
    float v = 0.0f;
    if ((int32_t)cnt < rstar)
      v = val16_exp<FMT>(ptr[gid], ev.T, __uint_as_float(rdlane(w0.x, l)),
                         __uint_as_float(rdlane(w0.y, l)), __uint_as_float(rdlane(w0.z, l)));
    if (lane == l) w0.w = __float_as_uint(v);
  }
  const float pg = __uint_as_float(w0.w);                          // RowStat::pgather
  const float qx = __shfl(pg, min(lane + k + 1, kWave - 1), kWave);  // its draft row's
  bool ok = true, near = false;
  if (lane < k) {
    const float r1 = fminf(pg / fmaxf(qx, 1e-10f), 1.0f);
    ok = u < r1;
    near = fabsf(u - r1) < 1e-5f;
  }
  int n = alive ? k : 0;
  uint32_t fl = gm.bad ? (uint32_t)SDX_FLAG_BAD_ROW : 0u;
  if (alive) {
    const uint64_t fm = __ballot(!ok);
    const int first = fm ? __ffsll((unsigned long long)fm) - 1 : kWave;
    if (__ballot(near && lane <= first)) fl |= SDX_FLAG_ACCEPT_NEAR_TIE;
    if (fm) n = first;
  }
  const uint32_t rf = w3.x;  // RowStat::flags
  {  // evaluated tests (positions 0..n, at most k - 1): drafted token in a partial tie group
    const int ne = alive ? (n < k ? n + 1 : k) : 0;
    const int pos = lane < k ? lane : (lane > k && lane < nr ? lane - k - 1 : kWave);
    if (__ballot(pos < ne && (rf & kRowGatherTie) != 0)) fl |= SDX_FLAG_TIE_ORDER;
  }
  if (__ballot(lane < nr && (rf & kRowNonfinite) != 0)) fl |= SDX_FLAG_NONFINITE;
  if (__ballot(lane < nr && (rf & kRowUnsupported) != 0)) fl |= SDX_FLAG_UNSUPPORTED;
  if (__ballot(lane < nr && (rf & kRowBadWs) != 0)) fl |= SDX_FLAG_WORKSPACE;
  const int lp = n == k ? k : n, lq = n == k ? -1 : k + 1 + n;
  if (lane == lp || lane == lq) {
    uint4* d = reinterpret_cast<uint4*>(st + (lane == lp ? 0 : 1));
    d[0] = w0; d[1] = w1; d[2] = w2; d[3] = w3;
  }
  job->prow = trow0 + lp;
  job->qrow = lq < 0 ? -1 : drow0 + n;
  job->u = uf;
  job->pad = 0;
  *fl_out = fl;
  return n;
}

// A record's R (4 or 5) rounds of 16-byte loads as named registers; pick()
// selects one by value (an array indexed at run time would live in scratch).
template <int R>
struct QuadT {
  static_assert(R == 4 || R == 5, "records of four or five rounds");
  uint4 a, b, c, d, e;
};
using Quad4 = QuadT<4>;
__device__ __forceinline__ uint32_t pick1(uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3,
                                          int u) {
  return u == 0 ? x0 : (u == 1 ? x1 : (u == 2 ? x2 : x3));
}
__device__ __forceinline__ uint32_t pick1(uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3,
                                          uint32_t x4, int u) {
  return u == 0 ? x0 : (u == 1 ? x1 : (u == 2 ? x2 : (u == 3 ? x3 : x4)));
}
template <int R>
__device__ __forceinline__ uint4 pick(const QuadT<R>& q, int u) {
  if constexpr (R == 4)
    return make_uint4(pick1(q.a.x, q.b.x, q.c.x, q.d.x, u), pick1(q.a.y, q.b.y, q.c.y, q.d.y, u),
                      pick1(q.a.z, q.b.z, q.c.z, q.d.z, u), pick1(q.a.w, q.b.w, q.c.w, q.d.w, u));
  else
    return make_uint4(pick1(q.a.x, q.b.x, q.c.x, q.d.x, q.e.x, u),
                      pick1(q.a.y, q.b.y, q.c.y, q.d.y, q.e.y, u),
                      pick1(q.a.z, q.b.z, q.c.z, q.d.z, q.e.z, u),
                      pick1(q.a.w, q.b.w, q.c.w, q.d.w, q.e.w, u));
}
template <int R>
__device__ __forceinline__ void put(QuadT<R>& q, int u, const uint4& v) {
  if (u == 0) q.a = v;
  else if (u == 1) q.b = v;
  else if (u == 2) q.c = v;
  else if (R == 4 || u == 3) q.d = v;
  else q.e = v;
}
__device__ __forceinline__ uint32_t sel_word(const uint4& v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// Whole block: walks NR records (each at most kRec16 = SM_NW rounds of 512
// ids) in id order, wave w taking round w of each; the loads of all of them
// are issued first. Record i spans ids [i0[i], i1[i]) with member ranks
// (bp[i], bq[i]) at its start; returns its mass (residual when use_r, else p)
// in m[i]. With `find` (NR == 1, base <= t): the id whose prefix mass, counted
// from `base`, first exceeds t goes to *found. `s32` / `s64` hold SM_NW words.
// FP: the found id's p value (its final probability, member rank applied) goes
// to s32[0] as float bits, read after the walk's last barrier.
template <int FMT, int NR, int NW = SM_NW, bool FP = false>
__device__ __forceinline__ void block_walk16(const Eval16<FMT>& ev, const typename Eval16<FMT>::Row& rp,
                             const typename Eval16<FMT>::Row& rq, bool use_r,
                             const int64_t (&i0)[NR], const int64_t (&i1)[NR],
                             const uint32_t (&bp)[NR], const uint32_t (&bq)[NR], uint64_t (&m)[NR],
                             uint64_t base, bool find, uint64_t t, int64_t* found, uint32_t* s32,
                             uint64_t* s64) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const int32_t sp = rp.st.rstar, sq = use_r ? rq.st.rstar : 0;
  uint4 P[NR], Q[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int64_t idx = i0[i] + w * kDrawSub + (int64_t)lane * 8;
    P[i] = make_uint4(0, 0, 0, 0);
    Q[i] = P[i];
    if (idx < i1[i]) {
      P[i] = ev.fetch(rp, idx, i1[i]);
      if (use_r) Q[i] = ev.fetch(rq, idx, i1[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int64_t idx = i0[i] + w * kDrawSub + (int64_t)lane * 8;
    float p[8], q[8];
    uint32_t mp = 0, mq = 0;
#pragma unroll
    for (int x = 0; x < 8; ++x) { p[x] = 0.0f; q[x] = 0.0f; }
    if (idx < i1[i]) {
      mp = ev.eval(rp, idx, i1[i], P[i], p) & 0xFFu;
      if (use_r) mq = ev.eval(rq, idx, i1[i], Q[i], q) & 0xFFu;
    }
    // member ranks: block scan of packed (p count, q count)
    const uint32_t cnt = (uint32_t)__popc(mp) | ((uint32_t)__popc(mq) << 16);
    const uint32_t incl = wave_incl_scan_u32(cnt, lane);
    if (lane == kWave - 1) s32[w] = incl;
    __syncthreads();
    uint32_t off = 0;
#pragma unroll
    for (int v = 0; v < NW; ++v) off += v < w ? s32[v] : 0u;
    uint32_t rk_p = bp[i] + ((off + incl - cnt) & 0xFFFFu);
    uint32_t rk_q = bq[i] + ((off + incl - cnt) >> 16);
    uint64_t wv[8], mine = 0;
#pragma unroll
    for (int x = 0; x < 8; ++x) {
      float pv = p[x];
      if ((mp >> x) & 1u) { pv = (int32_t)rk_p < sp ? pv : 0.0f; ++rk_p; }
      if constexpr (FP) p[x] = pv;
      if (use_r) {
        float qv = q[x];
        if ((mq >> x) & 1u) { qv = (int32_t)rk_q < sq ? qv : 0.0f; ++rk_q; }
        wv[x] = fixed62(fmaxf(pv - qv, 0.0f));
      } else {
        wv[x] = fixed62(pv);
      }
      mine += wv[x];
    }
    const uint64_t inc = wave_incl_scan_u64(mine, lane);
    if (lane == kWave - 1) s64[w] = inc;
    __syncthreads();
    uint64_t before = 0, tot = 0;
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      const uint64_t x = s64[v];
      before += v < w ? x : 0ull;
      tot += x;
    }
    m[i] = tot;
    if (find) {
      const uint64_t s0 = base + before + inc - mine;
      if (s0 <= t && s0 + mine > t) {
        uint64_t acc = s0;
        int64_t f = -1;
        float fpv = 0.0f;
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          acc += wv[x];
          if (f < 0 && acc > t) {
            f = idx + x;
            if constexpr (FP) fpv = p[x];
          }
        }
        *found = f;
        if constexpr (FP) s32[0] = __float_as_uint(fpv);  // every thread has read s32
      }
    }
    __syncthreads();  // s32 / s64 reused
  }
}

// Table value of a non-member id of row r with key `key`, not past the row's
// end: block_walk16's value of it (Eval16::eval) when *slow comes back false;
// *slow: the key is kept but below the table (its value is val16_exp's).
template <int FMT>
__device__ __forceinline__ float tval_nonmember16(const typename Eval16<FMT>::Row& r, int32_t key,
                                                  bool* slow) {
  const bool live = key >= r.st.klo;
  const int32_t tt = r.st.kmax - key, tmax = max(r.st.ntbl - 1, 0);
  *slow = live && tt > tmax;
  return live ? r.tbl[min(max(tt, 0), tmax)] : 0.0f;
}

// Whole block, wave w < R taking round w (512 ids) of each: the residual
// masses m[i] of the NR <= 2 records [x0[i], x1[i]) in which p's or q's kept
// group members run out, with member ranks (bp[i], bq[i]) at their starts and
// r0[i] each record's mass of its ids in neither group. The members of either
// group are the only ids whose value depends on the ranks: each is evaluated
// with its rank applied and added to r0. Every term is block_walk16's term for
// the id and fixed-point sums are exact in any order, so m[i] is block_walk16's
// mass of the record. A term whose non-member side is kept below the table
// (the exp path) waits for a rare pass after the others, which reloads that
// id's codes and evaluates it inline: an out-of-line call there would make the
// values live across it spill to scratch.
// `cnt64`, `m0`, `m1`: LDS words (NW each) this call may overwrite; the other
// code of the block does not read them between this call's barriers.
template <int FMT, int R, int NW, int NR>
__device__ __forceinline__ void block_part_mass16(const Eval16<FMT>& ev,
                                                  const typename Eval16<FMT>::Row& rp,
                                                  const typename Eval16<FMT>::Row& rq,
                                                  const int64_t (&x0)[NR], const int64_t (&x1)[NR],
                                                  const uint32_t (&bp)[NR], const uint32_t (&bq)[NR],
                                                  const uint64_t (&r0)[NR], uint64_t (&m)[NR],
                                                  uint64_t* cnt64, uint64_t* m0, uint64_t* m1) {
  static_assert(R <= NW, "one wave per round");
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const int32_t sp = rp.st.rstar, sq = rq.st.rstar;
  static_assert(NR == 1 || NR == 2, "one or two records");
  uint4 P[NR], Q[NR];
  int32_t nv[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int64_t idx = x0[i] + w * kDrawSub + (int64_t)lane * 8;
    const bool on = w < R;  // uniform per wave
    nv[i] = on ? (int32_t)min(max(x1[i] - idx, (int64_t)0), (int64_t)8) : 0;
    P[i] = make_uint4(0, 0, 0, 0);
    Q[i] = P[i];
    if (nv[i] > 0) {
      P[i] = ev.fetch(rp, idx, x1[i]);
      Q[i] = ev.fetch(rq, idx, x1[i]);
    }
  }
  uint32_t mp[NR], mq[NR], cnt[NR], incl[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const uint32_t pw[4] = {P[i].x, P[i].y, P[i].z, P[i].w};
    const uint32_t qw[4] = {Q[i].x, Q[i].y, Q[i].z, Q[i].w};
    mp[i] = 0;
    mq[i] = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const uint32_t kp2 = keys2_of_codes2(pw[t >> 1]), kq2 = keys2_of_codes2(qw[t >> 1]);
      const int32_t kp = (int32_t)((t & 1) ? kp2 >> 16 : kp2 & 0xFFFFu);
      const int32_t kq = (int32_t)((t & 1) ? kq2 >> 16 : kq2 & 0xFFFFu);
      const bool in = t < nv[i];
      mp[i] |= (in && kp >= rp.st.klo && kp >= rp.st.glo && kp <= rp.st.ghi ? 1u : 0u) << t;
      mq[i] |= (in && kq >= rq.st.klo && kq >= rq.st.glo && kq <= rq.st.ghi ? 1u : 0u) << t;
    }
    cnt[i] = (uint32_t)__popc(mp[i]) | ((uint32_t)__popc(mq[i]) << 16);
    incl[i] = wave_incl_scan_u32(cnt[i], lane);
  }
  if (lane == kWave - 1) cnt64[w] = (uint64_t)incl[0] | ((uint64_t)incl[NR - 1] << 32);
  __syncthreads();
  uint32_t off[2] = {0, 0};
#pragma unroll
  for (int v = 0; v < NW; ++v) {
    const uint64_t x = cnt64[v];
    off[0] += v < w ? (uint32_t)x : 0u;
    off[1] += v < w ? (uint32_t)(x >> 32) : 0u;
  }
  uint64_t mine[2] = {0, 0};
  uint32_t ex[NR], slow = 0;  // slow: bit 8i + t
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    ex[i] = off[i] + incl[i] - cnt[i];
    if (mp[i] | mq[i]) {  // few lanes: the members of this lane's 8 ids, in id order
      const uint32_t pw[4] = {P[i].x, P[i].y, P[i].z, P[i].w};
      const uint32_t qw[4] = {Q[i].x, Q[i].y, Q[i].z, Q[i].w};
      uint32_t rk_p = bp[i] + (ex[i] & 0xFFFFu), rk_q = bq[i] + (ex[i] >> 16);
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const bool ip = (mp[i] >> t) & 1u, iq = (mq[i] >> t) & 1u;
        if (ip || iq) {
          const uint32_t kp2 = keys2_of_codes2(pw[t >> 1]), kq2 = keys2_of_codes2(qw[t >> 1]);
          const int32_t kp = (int32_t)((t & 1) ? kp2 >> 16 : kp2 & 0xFFFFu);
          const int32_t kq = (int32_t)((t & 1) ? kq2 >> 16 : kq2 & 0xFFFFu);
          bool sl_p = false, sl_q = false;
          const float pv = ip ? ((int32_t)rk_p < sp ? rp.vg : 0.0f)
                              : tval_nonmember16<FMT>(rp, kp, &sl_p);
          const float qv = iq ? ((int32_t)rk_q < sq ? rq.vg : 0.0f)
                              : tval_nonmember16<FMT>(rq, kq, &sl_q);
          if (sl_p || sl_q)
            slow |= 1u << (8 * i + t);
          else
            mine[i] += fixed62(fmaxf(pv - qv, 0.0f));
        }
        rk_p += ip ? 1u : 0u;
        rk_q += iq ? 1u : 0u;
      }
    }
  }
  if (__builtin_expect(__ballot(slow != 0) != 0, 0)) {  // rare: one term per pass
    while (slow) {
      const int b = __builtin_ctz(slow);
      slow &= slow - 1;
      const int i = NR == 2 ? b >> 3 : 0, t = b & 7;
      const int64_t id = (i ? x0[NR - 1] : x0[0]) + w * kDrawSub + (int64_t)lane * 8 + t;
      const uint32_t e = i ? ex[NR - 1] : ex[0], mpb = i ? mp[NR - 1] : mp[0];
      const uint32_t mqb = i ? mq[NR - 1] : mq[0];
      const uint32_t below = (1u << t) - 1u;
      const uint32_t rk_p = (i ? bp[NR - 1] : bp[0]) + (e & 0xFFFFu) + (uint32_t)__popc(mpb & below);
      const uint32_t rk_q = (i ? bq[NR - 1] : bq[0]) + (e >> 16) + (uint32_t)__popc(mqb & below);
      const bool ip = (mpb >> t) & 1u, iq = (mqb >> t) & 1u;
      const uint32_t cp = rp.ptr[id], cq = rq.ptr[id];
      bool sl = false;
      float pv = ip ? ((int32_t)rk_p < sp ? rp.vg : 0.0f)
                    : tval_nonmember16<FMT>(rp, (int32_t)key_of_code16(cp), &sl);
      if (sl) pv = val16_exp_inl<FMT>(cp, ev.T, rp.st.m, rp.st.zf, rp.st.totf);
      sl = false;
      float qv = iq ? ((int32_t)rk_q < sq ? rq.vg : 0.0f)
                    : tval_nonmember16<FMT>(rq, (int32_t)key_of_code16(cq), &sl);
      if (sl) qv = val16_exp_inl<FMT>(cq, ev.T, rq.st.m, rq.st.zf, rq.st.totf);
      const uint64_t term = fixed62(fmaxf(pv - qv, 0.0f));
      mine[0] += i ? 0ull : term;
      mine[1] += i ? term : 0ull;
    }
  }
  const uint64_t s0 = wave_sum_u64(mine[0]), s1 = wave_sum_u64(mine[1]);
  if (lane == 0) { m0[w] = s0; m1[w] = s1; }
  __syncthreads();
  m[0] = r0[0];
  if (NR == 2) m[NR - 1] = r0[NR - 1];
#pragma unroll
  for (int v = 0; v < NW; ++v) {
    m[0] += m0[v];
    if (NR == 2) m[NR - 1] += m1[v];
  }
}

// Per-lane sums of a draw16 record.
struct Rec16Acc {
  uint64_t p2, r0, ra, rb, rp;
  uint32_t cnt;  // (ids in both groups) | (p group members << 16)
};
// What the record pass needs of the draw's two rows.
struct Rec16Rows {
  const float* tbl_p;
  const float* tbl_q;
  int32_t kmax_p, ntbl_p, glo_p, ghi_p;
  float vg_p, m_p, zf_p, totf_p;
  int32_t kmax_q, ntbl_q, klo_q, glo_q, ghi_q;
  float vg_q, m_q, zf_q, totf_q;
  bool hasq;
  float T;
};
// Final probability of a kept (non-member) key: its table entry, or exp below the table.
template <int FMT>
__device__ __forceinline__ float rec16_val(const float* tbl, int32_t kmax, int32_t ntbl,
                                           int32_t key, uint32_t code, float T, float m, float zf,
                                           float totf) {
  const int32_t tt = kmax - key;
  if (tt < ntbl) return tbl[tt];
  return val16_exp<FMT>(code, T, m, zf, totf);
}
// One id whose p code cp is live (key >= klo_p), with q code cq: its masses.
template <int FMT>
__device__ __forceinline__ void rec16_entry(const Rec16Rows& R, Rec16Acc& A, uint32_t cp,
                                            uint32_t cq) {
  const int32_t kp = (int32_t)key_of_code16(cp);
  const bool ip = kp >= R.glo_p && kp <= R.ghi_p;
  const float pv = ip ? R.vg_p
                      : rec16_val<FMT>(R.tbl_p, R.kmax_p, R.ntbl_p, kp, cp, R.T, R.m_p, R.zf_p,
                                       R.totf_p);
  float qv = 0.0f;
  bool iq = false;
  if (R.hasq) {
    const int32_t kq = (int32_t)key_of_code16(cq);
    iq = kq >= R.glo_q && kq <= R.ghi_q;
    qv = iq ? R.vg_q
            : (kq >= R.klo_q ? rec16_val<FMT>(R.tbl_q, R.kmax_q, R.ntbl_q, kq, cq, R.T, R.m_q,
                                              R.zf_q, R.totf_q)
                             : 0.0f);
  }
  const uint64_t wr = fixed62(fmaxf(pv - qv, 0.0f));
  const uint64_t fp = fixed62(pv);
  A.p2 += ip ? 0ull : fp;
  A.r0 += (!ip && !iq) ? wr : 0ull;
  A.ra += (!ip && iq) ? wr : 0ull;
  A.rb += (!ip && iq) ? fp : 0ull;
  A.rp += (ip && !iq) ? wr : 0ull;
  A.cnt += (ip && iq ? 1u : 0u) + (ip ? 0x10000u : 0u);
}
// Common case: p-live ids by a signed 16-bit compare of the code with the cut
// (thp = klo_p - 0x8000 >= 0), q members (one code, cqg) counted per lane from
// the packed codes into nq_l (in the last record, TAIL, by a wave vote per id
// into nq_s); the p-live ids go through the wave's LDS list L, evaluated one per
// lane once 64 have gathered. TAIL: the record runs past V (ids past V are skipped).
template <int FMT, bool TAIL, int RD = kRec16Rounds>
__device__ __forceinline__ void rec16_fast(const QuadT<RD>& P, const QuadT<RD>& Q, int64_t x0,
                                           int64_t V,
                                           int lane, int32_t thp, bool hasgq, uint32_t cqg,
                                           uint32_t* L, const Rec16Rows& R, Rec16Acc& A,
                                           uint32_t& nq_s, uint32_t& nq_l) {
  typedef unsigned short pq_us2 __attribute__((ext_vector_type(2)));
  const uint32_t cqg2 = cqg | (cqg << 16);
  uint32_t off = 0;  // uniform
#pragma unroll
  for (int u = 0; u < RD; ++u) {
    const uint4 pu = pick(P, u), qu = pick(Q, u);
    const uint32_t pw[4] = {pu.x, pu.y, pu.z, pu.w};
    const uint32_t qw[4] = {qu.x, qu.y, qu.z, qu.w};
    const int64_t nv = TAIL ? V - (x0 + u * kDrawSub + (int64_t)lane * 8) : 8;
    if (!TAIL && hasgq) {  // q group members: equal halves of the packed codes
      pq_us2 ne = {0, 0};
#pragma unroll
      for (int k = 0; k < 4; ++k)
        ne += __builtin_elementwise_min(__builtin_bit_cast(pq_us2, qw[k] ^ cqg2), (pq_us2){1, 1});
      nq_l += 8u - (uint32_t)ne[0] - (uint32_t)ne[1];
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const uint32_t cp = (t & 1) ? pw[t >> 1] >> 16 : pw[t >> 1] & 0xFFFFu;
      const uint32_t cq = (t & 1) ? qw[t >> 1] >> 16 : qw[t >> 1] & 0xFFFFu;
      const bool in = !TAIL || t < nv;
      const bool live = (int32_t)(int16_t)cp >= thp && in;
      const uint64_t m = __ballot(live);
      if (TAIL && hasgq) nq_s += (uint32_t)__popcll(__ballot(cq == cqg && in));
      if (m) {
        if (live)
          L[off + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                            __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u))] =
              cp | (cq << 16);
        off += (uint32_t)__popcll(m);
      }
    }
    if (off >= kWave || u == RD - 1) {  // evaluate whole lanes' worth
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_wave_barrier();
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      const uint32_t full = u == RD - 1 ? off : (off & ~(uint32_t)(kWave - 1));
      for (uint32_t i = lane; i < full; i += kWave) {
        const uint32_t e = L[i];
        rec16_entry<FMT>(R, A, e & 0xFFFFu, e >> 16);
      }
      const uint32_t rem = off - full;
      uint32_t keep = 0;
      if ((uint32_t)lane < rem) keep = L[full + lane];
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_wave_barrier();
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      if ((uint32_t)lane < rem) L[lane] = keep;
      off = rem;
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_wave_barrier();
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
  }
}
// Any rows: every id evaluated in place (one loop body, words picked by selects).
template <int FMT, int RD = kRec16Rounds>
__device__ __forceinline__ void rec16_general(const QuadT<RD>& P, const QuadT<RD>& Q, int64_t x0,
                                              int64_t V, int lane, int32_t klo_p,
                                              const Rec16Rows& R, Rec16Acc& A, uint32_t& nqv) {
  static_assert(RD == 4, "the in-place path serves four-round records");
#pragma unroll 1
  for (int i = 0; i < RD * 8; ++i) {
    const int u = i >> 3, t = i & 7;
    const int64_t id = x0 + u * kDrawSub + (int64_t)lane * 8 + t;
    const uint32_t pw = sel_word(pick(P, u), t >> 1), qw = sel_word(pick(Q, u), t >> 1);
    const uint32_t cp = (t & 1) ? pw >> 16 : pw & 0xFFFFu;
    const uint32_t cq = (t & 1) ? qw >> 16 : qw & 0xFFFFu;
    if (id < V) {
      if (R.hasq) {
        const int32_t kq = (int32_t)key_of_code16(cq);
        nqv += (kq >= R.glo_q && kq <= R.ghi_q) ? 1u : 0u;
      }
      if ((int32_t)key_of_code16(cp) >= klo_p) rec16_entry<FMT>(R, A, cp, cq);
    }
  }
}


// The draw body's LDS (one object, so the fused kernel can overlay it on the
// row blocks' histogram).
template <int NW>
struct Draw16LdsT {
  float tbl_p[kTbl];
  float tbl_q[kTbl];
  // per-wave list of p-live ids' (p code, q code); the completing block keeps the
  // job's records here afterwards
  alignas(16) uint32_t lst[NW][kLst16];
  RowStat st[2];
  SampleJob job;
  uint64_t s64[NW];
  uint64_t rm2[NW];
  int32_t last;
  int32_t part[2];    // records where p's / q's kept group members run out
  uint32_t pbase[4];  // their member ranks (bp, bq) at the record start
  int64_t pick[3];
  int64_t found;
  uint32_t s32w[NW];
  uint64_t s64w[NW];
  uint64_t pmass[2][NW];  // partial records' masses, per wave
  uint32_t fl;
};
using Draw16Lds = Draw16LdsT<SM_NW>;

// One job's accept chain and draw, run by a block of SM_NT threads: block bi of
// the job's blocks (wave w of it owns record bi * SM_NW + w); the block that
// completes the job's records draws y. FP: that block also leaves the drawn
// id's p value in S.s32w[0] (float bits) when y >= 0. NOQ: the caller's jobs
// never have a q row (k = 0), so nothing of one is loaded or compiled in.
template <int FMT, bool COH, int NT = SM_NT, int R = kRec16Rounds, bool FP = false,
          bool NOQ = false>
__device__ __forceinline__ void draw16_body(const Draw16Args<FMT>& a,
                                            Draw16LdsT<NT / kWave>& S, int64_t j, int bi) {
  constexpr int NW = NT / kWave;
  constexpr int REC = R * kDrawSub;  // ids per record
  constexpr int MAXREC = (int)((kMaxVocabBf16 + REC - 1) / REC);
  static_assert(R <= NW, "the walks give each round of a record to one wave");
  float* const tbl_p = S.tbl_p;
  float* const tbl_q = S.tbl_q;
  uint32_t(&lst)[NW][kLst16] = S.lst;
  RowStat* const s_st = S.st;
  SampleJob& s_job = S.job;
  uint64_t* const s64 = S.s64;
  uint64_t* const s_rm2 = S.rm2;
  int32_t& s_last = S.last;
  int32_t* const s_part = S.part;
  uint32_t* const s_pbase = S.pbase;
  int64_t* const s_pick = S.pick;
  int64_t& s_found = S.found;
  uint32_t* const s32w = S.s32w;
  uint64_t* const s64w = S.s64w;
  uint32_t& s_fl = S.fl;
  const Eval16<FMT>& ev = a.ev;
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const int64_t V = a.V;

  // ---- 1. the accept chain and the draw's RowStats (wave 0)
  if (w == 0) {
    SampleJob jb;
    uint32_t fl;
    int64_t n;
    if (2 * a.acc.k + 1 <= kWave) {
      n = chain16_wave<FMT, COH>(a.acc, ev, j, &jb, &fl, s_st);
    } else {  // long drafts: the generic chain, then the two RowStats word by word
      n = accept_chain_wave(a.acc, j, &jb, &fl);
      if (lane < 32) {
        const int which = lane >> 4;
        const int64_t row = which ? jb.qrow : jb.prow;
        if (row >= 0)
          reinterpret_cast<uint32_t*>(s_st + which)[lane & 15] =
              reinterpret_cast<const uint32_t*>(a.acc.stats + row)[lane & 15];
      }
    }
    if (lane == 0) {
      if (bi == 0) {
        a.acc.jobs[j] = jb;
        if (a.acc.n_acc) a.acc.n_acc[j] = n;
      }
      s_job = jb;
      s_fl = fl;  // written with y by the block that draws it
    }
  }
  __syncthreads();
  const SampleJob job = s_job;
  const bool hasq = !NOQ && job.qrow >= 0;
  typename Eval16<FMT>::Row rp, rq;
  rp.ptr = job.prow < ev.split ? ev.base + job.prow * ev.ld : ev.base2 + (job.prow - ev.split) * ev.ld2;
  rp.st = s_st[0];
  rp.tbl = tbl_p;
  if (hasq) {
    rq.ptr = job.qrow < ev.split ? ev.base + job.qrow * ev.ld
                                 : ev.base2 + (job.qrow - ev.split) * ev.ld2;
    rq.st = s_st[1];
  } else {
    rq.ptr = rp.ptr;
    rq.st = RowStat{};
    rq.st.klo = 0x7FFFFFFF;
    rq.st.glo = 1;
    rq.st.ghi = 0;
  }
  rq.tbl = tbl_q;

  // ---- 2. the tables' loads, then this wave's record's loads (issued last, so
  // each round is used as soon as it lands), then the tables go to LDS
  // (loads without branches, so the waits before use count them exactly;
  // addresses stay inside the rows / tables, unused values are replaced)
  const int t0 = threadIdx.x;  // first NT entries now, the rest (wide nuclei) after
  const float tp0 = ld_f32<COH>(ev.tables + job.prow * kTbl + t0);
  const float tq0 = NOQ ? 0.0f : ld_f32<COH>(ev.tables + (hasq ? job.qrow : job.prow) * kTbl + t0);
  __builtin_amdgcn_sched_barrier(0);  // keep the issue order: tables, then rows
  const int rec = bi * NW + w;
  const bool has_rec = rec < a.nrec;  // uniform per wave
  const int64_t x0 = (int64_t)rec * REC;
  QuadT<R> P, Q;
#pragma unroll
  for (int u = 0; u < R; ++u) {
    const int64_t idx = x0 + u * kDrawSub + (int64_t)lane * 8;
    // ids at or past V (the last record) are skipped when read, and q codes
    // are read only when the draw has a q row
    const int64_t ic = has_rec && idx < V ? idx : 0;  // V % 8 == 0: whole 16-byte groups
    put(P, u, *reinterpret_cast<const uint4*>(rp.ptr + ic));
    put(Q, u, NOQ ? make_uint4(0, 0, 0, 0)
                  : *reinterpret_cast<const uint4*>((hasq ? rq.ptr : rp.ptr) + ic));
  }
  __builtin_amdgcn_sched_barrier(0);
  if (t0 < rp.st.ntbl) tbl_p[t0] = tp0;
  if (hasq && t0 < rq.st.ntbl) tbl_q[t0] = tq0;
  for (int t = t0 + NT; t < rp.st.ntbl; t += NT)
    tbl_p[t] = ld_f32<COH>(ev.tables + job.prow * kTbl + t);
  if (hasq)
    for (int t = t0 + NT; t < rq.st.ntbl; t += NT)
      tbl_q[t] = ld_f32<COH>(ev.tables + job.qrow * kTbl + t);
  __syncthreads();
  rp.vg = rp.st.glo <= rp.st.ghi
              ? val16<FMT>(rp.st, tbl_p, code_of_key16((uint32_t)rp.st.glo), ev.T) : 0.0f;
  rq.vg = hasq && rq.st.glo <= rq.st.ghi
              ? val16<FMT>(rq.st, tbl_q, code_of_key16((uint32_t)rq.st.glo), ev.T) : 0.0f;

  // ---- 3. the record
  if (has_rec) {
    Rec16Rows RR;
    RR.tbl_p = tbl_p; RR.tbl_q = tbl_q; RR.hasq = hasq; RR.T = ev.T;
    RR.kmax_p = rp.st.kmax; RR.ntbl_p = rp.st.ntbl; RR.glo_p = rp.st.glo; RR.ghi_p = rp.st.ghi;
    RR.vg_p = rp.vg; RR.m_p = rp.st.m; RR.zf_p = rp.st.zf; RR.totf_p = rp.st.totf;
    RR.kmax_q = rq.st.kmax; RR.ntbl_q = rq.st.ntbl; RR.klo_q = rq.st.klo; RR.glo_q = rq.st.glo;
    RR.ghi_q = rq.st.ghi; RR.vg_q = rq.vg; RR.m_q = rq.st.m; RR.zf_q = rq.st.zf;
    RR.totf_q = rq.st.totf;
    const int32_t klo_p = rp.st.klo;
    Rec16Acc A = {0, 0, 0, 0, 0, 0};
    uint32_t nqv = 0;   // per lane: q group members (in-place path, packed counts)
    uint32_t nq_s = 0;  // per wave: q group members (listed path)
    if (klo_p >= 0x8000 && (!hasq || RR.glo_q >= RR.ghi_q)) {
      const int32_t thp = klo_p - 0x8000;  // p-live: positive code >= this
      const bool hasgq = hasq && RR.glo_q == RR.ghi_q;
      const uint32_t cqg = hasgq ? code_of_key16((uint32_t)RR.glo_q) : 0u;
      if (x0 + REC <= V)
        rec16_fast<FMT, false, R>(P, Q, x0, V, lane, thp, hasgq, cqg, lst[w], RR, A, nq_s, nqv);
      else
        rec16_fast<FMT, true, R>(P, Q, x0, V, lane, thp, hasgq, cqg, lst[w], RR, A, nq_s, nqv);
    } else {
      rec16_general<FMT, R>(P, Q, x0, V, lane, klo_p, RR, A, nqv);
    }
    const uint64_t p2 = A.p2, r0 = A.r0, ra = A.ra, rb = A.rb, rpm = A.rp;
    const uint32_t cnt = A.cnt;
    ChunkRec rc;
    rc.p2 = wave_sum_u64(p2);
    rc.r0 = wave_sum_u64(r0);
    rc.ra = wave_sum_u64(ra);
    rc.rb = wave_sum_u64(rb);
    rc.rp = wave_sum_u64(rpm);
    const uint32_t c = wave_sum_u32(cnt);
    rc.np = c >> 16;
    rc.ndbl = c & 0xFFFFu;
    rc.nq = nq_s + wave_sum_u32(nqv);
    rc.pad = 0;
    rc.pad2 = 0;
    if (lane == 0) store_rec(a.recs + j * a.nrec + rec, rc);
  }

  // ---- 4. the block that completes the job's records draws (as draw_kernel)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // gfx9 encoding: vmcnt(0), expcnt / lgkmcnt untouched
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&a.counters[j], 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == (uint32_t)(a.nblk - 1) ? 1 : 0;
  }
  if (threadIdx.x < 2) s_part[threadIdx.x] = -1;
  if (threadIdx.x == 0) { s_pick[0] = -1; s_found = -1; }
  __syncthreads();
  if (!s_last) return;
  // every block of the job has counted in: the counters go back to zero for the
  // next call (the fused kernel's job arrivals too)
  if (threadIdx.x == 0) {
    __hip_atomic_store(&a.counters[j], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (a.job_cnt) __hip_atomic_store(&a.job_cnt[j], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  const int32_t sp = rp.st.rstar, sq = hasq ? rq.st.rstar : 0;
  const float vp = rp.vg, vq = hasq ? rq.vg : 0.0f;
  // the job's records (at most MAXREC <= NT) go to LDS, one per thread, in
  // the list space the record pass no longer needs: held in registers across the
  // walks below they spilled to scratch, and scratch slows every wave's launch
  static_assert(sizeof(lst) >= MAXREC * sizeof(ChunkRec) && MAXREC <= NT,
                "a job's records fit in the list space, one per thread");
  ChunkRec* const lrec = reinterpret_cast<ChunkRec*>(&lst[0][0]);
  const ChunkRec* jrecs = a.recs + j * a.nrec;
  if ((int)threadIdx.x < a.nrec) lrec[threadIdx.x] = load_rec(jrecs + threadIdx.x);
  __syncthreads();
  const int rb0 = min(a.nrec, (int)threadIdx.x), rb1 = min(a.nrec, rb0 + 1);
  auto rec_at = [&](int r) -> ChunkRec { return lrec[r]; };
  uint64_t cntn = 0;
  for (int r = rb0; r < rb1; ++r) {
    const ChunkRec rec = rec_at(r);
    cntn += (uint64_t)rec.np | ((uint64_t)rec.nq << 32);
  }
  uint64_t tot_n;
  const uint64_t ex_n = block_excl_u64<NW>(cntn, s64, &tot_n);
  {  // at most one record where p's kept members run out, one for q's
    uint32_t bp = (uint32_t)ex_n, bq = (uint32_t)(ex_n >> 32);
    for (int r = rb0; r < rb1; ++r) {
      const ChunkRec rec = rec_at(r);
      uint64_t pm, rm;
      if (!rec_masses(rec, bp, bq, sp, sq, vp, vq, hasq, &pm, &rm)) {
        const int64_t kp = min<int64_t>(max<int64_t>((int64_t)sp - bp, 0), rec.np);
        const int slot = (kp != 0 && kp != (int64_t)rec.np) ? 0 : 1;
        s_part[slot] = r;
        s_pbase[2 * slot] = bp;
        s_pbase[2 * slot + 1] = bq;
      }
      bp += rec.np;
      bq += rec.nq;
    }
  }
  __syncthreads();
  const int pa = s_part[0], pb = s_part[1];
  uint64_t rm_part[2] = {0, 0};
  if (!NOQ && (pa >= 0 || pb >= 0)) {  // uniform: the (at most two) records where kept members run out
    // (only with a q row: without one, every record's p mass is exact)
    const int ra_ = pa >= 0 ? pa : pb, rb_ = (pa >= 0 && pb >= 0 && pb != pa) ? pb : -1;
    const int sa = pa >= 0 ? 0 : 1;
    uint64_t mm[2] = {0, 0};
    // one record at a time: the codes of both at once would not fit the
    // registers left here
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int rr = i == 0 ? ra_ : rb_;
      if (rr >= 0) {  // uniform
        const int64_t a0[1] = {(int64_t)rr * REC}, a1[1] = {min(V, a0[0] + REC)};
        const int sl = i == 0 ? sa : 1;
        const uint32_t p1[1] = {s_pbase[2 * sl]}, q1[1] = {s_pbase[2 * sl + 1]};
        const uint64_t z1[1] = {lrec[rr].r0};
        uint64_t m1[1];
        block_part_mass16<FMT, R, NW, 1>(ev, rp, rq, a0, a1, p1, q1, z1, m1, s64w, S.pmass[0],
                                         S.pmass[1]);
        mm[i] = m1[0];
      }
    }
    if (pa >= 0) rm_part[0] = mm[0];
    if (pb >= 0) rm_part[1] = pb == pa ? mm[0] : (pa >= 0 ? mm[1] : mm[0]);
  }
  // this thread's record's masses (evaluated again from the LDS copy rather
  // than held in registers across the partial records' pass)
  uint64_t sum_r = 0, sum_p = 0;
  {
    uint32_t bp = (uint32_t)ex_n, bq = (uint32_t)(ex_n >> 32);
    for (int r = rb0; r < rb1; ++r) {
      const ChunkRec rec = rec_at(r);
      uint64_t pm, rm;
      if (!rec_masses(rec, bp, bq, sp, sq, vp, vq, hasq, &pm, &rm))
        rm = r == pa ? rm_part[0] : rm_part[1];
      sum_r += rm;
      sum_p += pm;
      bp += rec.np;
      bq += rec.nq;
    }
  }
  uint64_t ex_r, ex_p, tot_r, tot_p;
  {
    const uint64_t ir = wave_incl_scan_u64(sum_r, lane), ip = wave_incl_scan_u64(sum_p, lane);
    if (lane == kWave - 1) { s64[w] = ir; s_rm2[w] = ip; }
    __syncthreads();
    uint64_t orr = 0, opp = 0;
    tot_r = 0;
    tot_p = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      const uint64_t xr = s64[i], xp = s_rm2[i];
      orr += i < w ? xr : 0ull;
      opp += i < w ? xp : 0ull;
      tot_r += xr;
      tot_p += xp;
    }
    ex_r = orr + ir - sum_r;
    ex_p = opp + ip - sum_p;
  }
  const bool use_r = hasq && rn32_u64(tot_r) > 1e-9f;
  const uint64_t tot = use_r ? tot_r : tot_p;
  // y and the row's flags (the accept chain's, plus SDX_FLAG_TIE_ORDER when y
  // is a member of a partially kept tie group of a row it was drawn from)
  auto finish = [&](int64_t yv) {
    if (threadIdx.x != 0) return;
    a.y[j] = yv;
    if (a.acc.flags) {
      uint32_t fl = s_fl;
      if (yv >= 0 && (Eval16<FMT>::in_tie_group(rp, yv) ||
                      (use_r && Eval16<FMT>::in_tie_group(rq, yv))))
        fl |= SDX_FLAG_TIE_ORDER;
      a.acc.flags[j] = (uint8_t)fl;
    }
  };
  if (tot == 0) {
    finish(-1);
    return;
  }
  const uint64_t t = uniform_threshold(job.u, tot);
  {
    uint64_t run = use_r ? ex_r : ex_p;
    const uint64_t mine = use_r ? sum_r : sum_p;
    if (rb0 < rb1 && run <= t && run + mine > t) {  // exactly one thread
      uint32_t bp = (uint32_t)ex_n, bq = (uint32_t)(ex_n >> 32);
      for (int r = rb0; r < rb1; ++r) {
        const ChunkRec rec = rec_at(r);
        uint64_t pm, rm;
        if (!rec_masses(rec, bp, bq, sp, sq, vp, vq, hasq, &pm, &rm))
          rm = r == pa ? rm_part[0] : rm_part[1];
        const uint64_t m = use_r ? rm : pm;
        if (run + m > t) {
          s_pick[0] = r;
          s_pick[1] = ((int64_t)bq << 32) | bp;
          s_pick[2] = (int64_t)run;
          break;
        }
        run += m;
        bp += rec.np;
        bq += rec.nq;
      }
    }
  }
  __syncthreads();
  const int64_t rec_star = s_pick[0];
  if (rec_star < 0) {  // unreachable: record masses sum to tot > t
    finish(-1);
    return;
  }
  {
    const int64_t packed = s_pick[1];
    const int64_t i0[1] = {rec_star * REC}, i1[1] = {min(V, rec_star * REC + REC)};
    const uint32_t bp1[1] = {(uint32_t)(packed & 0xFFFFFFFF)}, bq1[1] = {(uint32_t)(packed >> 32)};
    uint64_t mm[1];
    block_walk16<FMT, 1, NW, FP>(ev, rp, rq, use_r, i0, i1, bp1, bq1, mm, (uint64_t)s_pick[2],
                                 true, t, &s_found, s32w, s64w);
  }
  finish(s_found);
}

}  // namespace sdx
