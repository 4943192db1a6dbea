// Accept test, residual / bonus inverse-CDF sampling and to_probs output.
//
// Stages after the row statistics (specdec/engine.py:285-303), one launch:
//   draw_kernel  (jobs x blocks-per-job) grid. With the accept chain fused in,
//                wave 0 of each block replays its batch row's accept chain
//                u < min(1, p(x)/max(q(x), 1e-10)) with the first-reject scan
//                (sampling.py:117-129), one lane per position; block 0 of the
//                row publishes n_acc, flags and the draw (residual at the stop
//                position or bonus from p_{k+1}). Every wave then reduces a run
//                of 512-id rounds of the draw's rows to ChunkRecs: exact fixed62
//                partial sums that do not yet know which members of the rows'
//                boundary tie groups are kept. The block that completes a job's
//                records (an agent-scope counter) draws: prefix counts of group
//                members over the records give each its member ranks, hence its
//                exact residual (p - q)_+ and p masses (at most two records,
//                where a group's kept count runs out, are rescanned in id order
//                by one wave each); the degenerate-residual rule
//                (sampling.py:85-88); target floor(u * total); the record
//                holding it; a wave scan in id order for the first id whose
//                prefix mass exceeds it.
// Element probabilities come from an evaluator: codes + RowStat + table for
// 16-bit logits, or dense fp32 probability rows (which have no groups).
#include "sdx_draw16.hpp"

#include <cstdlib>
#include <type_traits>

namespace sdx {



struct EvalProb {
  static constexpr bool kGroups = false;
  static constexpr int kFmt = SDX_F32;
  static constexpr int kLdsTbl = 1;
  struct Raw {
    float4 a, b;
  };
  const float* base;
  int64_t ld;
  const float* base2;
  int64_t ld2;
  int64_t split;
  bool vec;
  const uint32_t* tie_bits;  // per row bits_ld words: members of a partial
                             // boundary tie group (null: no membership known)
  int64_t bits_ld;
  struct Row {
    const float* ptr;
    float vg;
    const uint32_t* bits;
  };
  __device__ void stage(int64_t, float*) const {}
  __device__ void bind(Row& r, int64_t row, const float*) const {
    r.ptr = row < split ? base + row * ld : base2 + (row - split) * ld2;
    r.vg = 0.0f;
    r.bits = tie_bits ? tie_bits + row * bits_ld : nullptr;
  }
  __device__ static int32_t rstar(const Row&) { return 0; }
  __device__ static bool in_tie_group(const Row& r, int64_t id) {
    return r.bits && ((r.bits[id >> 5] >> (id & 31)) & 1u) != 0;
  }
  __device__ Raw fetch(const Row& r, int64_t idx, int64_t lim) const {
    Raw x;
    if (vec && idx + 8 <= lim) {
      x.a = *reinterpret_cast<const float4*>(r.ptr + idx);
      x.b = *reinterpret_cast<const float4*>(r.ptr + idx + 4);
    } else {
      float v[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) v[t] = idx + t < lim ? r.ptr[idx + t] : 0.0f;
      x.a = make_float4(v[0], v[1], v[2], v[3]);
      x.b = make_float4(v[4], v[5], v[6], v[7]);
    }
    return x;
  }
  __device__ uint32_t eval(const Row&, int64_t idx, int64_t lim, const Raw& x, float v[8]) const {
    v[0] = x.a.x; v[1] = x.a.y; v[2] = x.a.z; v[3] = x.a.w;
    v[4] = x.b.x; v[5] = x.b.y; v[6] = x.b.z; v[7] = x.b.w;
    uint32_t live = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      if (idx + t >= lim) v[t] = 0.0f;
      live |= (v[t] > 0.0f ? 1u : 0u) << (8 + t);
    }
    return live;  // no tie groups; bits 8..15: nonzero probabilities
  }
  __device__ uint32_t load8(const Row& r, int64_t idx, int64_t lim, float v[8]) const {
    return eval(r, idx, lim, fetch(r, idx, lim), v) & 0xFFu;
  }
};


// One wave walks ids [i0, i1) in id order, the member ranks at i0 being
// (bp, bq), and returns the mass (residual when use_r, else p). With `find`
// (base <= t), the lane holding the first id whose prefix mass, counted from
// `base`, exceeds t writes it to *found.
template <class Ev>
__device__ uint64_t wave_walk(const Ev& ev, const typename Ev::Row& rp, const typename Ev::Row& rq,
                              bool use_r, int64_t i0, int64_t i1, uint32_t bp, uint32_t bq,
                              uint64_t base, bool find, uint64_t t, int64_t* found) {
  const int lane = threadIdx.x & (kWave - 1);
  const int32_t sp = Ev::rstar(rp), sq = use_r ? Ev::rstar(rq) : 0;
  uint64_t run = base;
  for (int64_t r0 = i0; r0 < i1; r0 += kDrawSub) {
    const int64_t idx = r0 + (int64_t)lane * 8;
    float p[8], q[8];
    uint32_t mp = 0, mq = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) { p[u] = 0.0f; q[u] = 0.0f; }
    if (idx < i1) {
      mp = ev.load8(rp, idx, i1, p);
      if (use_r) mq = ev.load8(rq, idx, i1, q);
    }
    uint32_t rk_p = bp, rk_q = bq;
    if constexpr (Ev::kGroups) {  // member ranks: wave scan of packed (p count, q count)
      const uint32_t cnt = (uint32_t)__popc(mp) | ((uint32_t)__popc(mq) << 16);
      const uint32_t incl = wave_incl_scan_u32(cnt, lane);
      const uint32_t tot = rdlane(incl, kWave - 1);
      rk_p += (incl - cnt) & 0xFFFFu;
      rk_q += (incl - cnt) >> 16;
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
    const uint64_t incl = wave_incl_scan_u64(mine, lane);
    const uint64_t tot = ((uint64_t)rdlane((uint32_t)(incl >> 32), kWave - 1) << 32) |
                         rdlane((uint32_t)incl, kWave - 1);
    if (find) {
      const uint64_t st = run + incl - mine;
      if (st <= t && st + mine > t) {
        uint64_t acc = st;
        int64_t f = -1;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          acc += w[u];
          if (f < 0 && acc > t) f = idx + u;
        }
        *found = f;
      }
    }
    run += tot;
  }
  return run - base;
}

// ---------------------------------------------------------------- the draw
struct DrawArgs {
  AcceptArgs acc;      // acc.stats == null: the draws are given in `jobs`
  SampleJob* jobs;
  int64_t V;
  int64_t rec_ids;     // ids per record (a multiple of kDrawSub)
  int32_t nrec;        // records per job
  int32_t gw;          // consecutive records per wave
  int32_t nblk;        // blocks per job
  ChunkRec* recs;      // [jobs, nrec]
  uint32_t* counters;  // [jobs], zero on entry (cleared by the kernel before)
  int64_t* y;          // null: records only
};

template <class Ev>
__global__ void __launch_bounds__(SM_NT) draw_kernel(Ev ev, DrawArgs a) {
  __shared__ float tbl_p[Ev::kLdsTbl];
  __shared__ float tbl_q[Ev::kLdsTbl];
  __shared__ float lst_p[SM_NW][kDrawSub];  // per-wave lists of ids with p mass
  __shared__ float lst_q[SM_NW][kDrawSub];
  __shared__ unsigned long long acc[SM_NW][6];  // per-wave record sums (16-bit rows)
  __shared__ SampleJob s_job;
  __shared__ uint64_t s64[SM_NW];
  __shared__ int32_t s_last;
  __shared__ int32_t s_part[2];    // records where p's / q's kept group members run out
  __shared__ uint32_t s_pbase[4];  // their member ranks (bp, bq) at the record start
  __shared__ uint64_t s_rm[2];     // and their residual masses
  __shared__ uint64_t s_rm2[SM_NW];
  __shared__ int64_t s_pick[3];
  __shared__ int64_t s_found;
  __shared__ uint32_t s_fl;
  const int64_t j = (int64_t)blockIdx.x / a.nblk;
  const int bi = (int)((int64_t)blockIdx.x % a.nblk);
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;

  // ---- 1. the draw: from the accept chain (wave 0) or given
  if (threadIdx.x < kWave) {
    if (a.acc.stats) {
      SampleJob jb;
      uint32_t fl;
      const int64_t n = accept_chain_wave(a.acc, j, &jb, &fl);
      if (lane == 0) {
        if (bi == 0) {
          a.jobs[j] = jb;
          if (a.acc.n_acc) a.acc.n_acc[j] = n;
        }
        s_job = jb;
        s_fl = fl;  // written with y by the block that draws it
      }
    } else if (lane == 0) {
      s_job = a.jobs[j];
      s_fl = 0;
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

  // ---- 2. records: wave w reduces records [r_beg, r_end) in 512-id rounds,
  // software-pipelined two rounds deep (buffers A / B keep fixed roles, so no
  // register rotation waits on a load in flight).
  {
    const int r_beg = (bi * SM_NW + w) * a.gw;
    const int r_end = min(a.nrec, r_beg + a.gw);
    if (r_beg < r_end) {
      const int64_t x_beg = (int64_t)r_beg * a.rec_ids;
      const int64_t x_end = min(a.V, (int64_t)r_end * a.rec_ids);
      const int64_t nround = (x_end - x_beg + kDrawSub - 1) / kDrawSub;
      const int64_t rpr = a.rec_ids / kDrawSub;  // rounds per record
      const int64_t lane_off = (int64_t)lane * 8;
      uint64_t p2 = 0, r0 = 0, ra = 0, rb = 0, rpm = 0;
      uint32_t np = 0, nq = 0, ndbl = 0;
      // one round: evaluate, compact the ids that may carry p mass into this
      // wave's LDS list (sign bits mark group members), reduce one per lane;
      // a round that ends a record publishes it
      auto round = [&](const typename Ev::Raw& cp, const typename Ev::Raw& cq, int64_t ro) {
        const int64_t s0 = x_beg + ro * kDrawSub;
        const int64_t rec = s0 / a.rec_ids;
        const int64_t e1 = min(a.V, (rec + 1) * a.rec_ids);
        const int64_t cur = s0 + lane_off;
        float p[8], q[8];
        const uint32_t ep = ev.eval(rp, cur, e1, cp, p);
        const uint32_t mp = ep & 0xFFu, lp = (ep >> 8) & 0xFFu;
        uint32_t mq = 0;
        if (hasq) {
          mq = ev.eval(rq, cur, e1, cq, q) & 0xFFu;
        } else {
#pragma unroll
          for (int t = 0; t < 8; ++t) q[t] = 0.0f;
        }
        np += __popc(mp);
        nq += __popc(mq);
        const uint32_t c = __popc(lp);
        const uint32_t incl = wave_incl_scan_u32(c, lane);
        const uint32_t n = rdlane(incl, kWave - 1);
        uint32_t o = incl - c;
#pragma unroll
        for (int t = 0; t < 8; ++t)
          if ((lp >> t) & 1u) {
            lst_p[w][o] = __uint_as_float(__float_as_uint(p[t]) | (((mp >> t) & 1u) << 31));
            lst_q[w][o] = __uint_as_float(__float_as_uint(q[t]) | (((mq >> t) & 1u) << 31));
            ++o;
          }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_wave_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        for (uint32_t i = lane; i < n; i += kWave) {
          const uint32_t bp = __float_as_uint(lst_p[w][i]), bq = __float_as_uint(lst_q[w][i]);
          const bool ip = (bp >> 31) != 0, iq = (bq >> 31) != 0;
          const float pv = __uint_as_float(bp & 0x7FFFFFFFu);
          const float qv = __uint_as_float(bq & 0x7FFFFFFFu);
          const uint64_t wr = fixed62(fmaxf(pv - qv, 0.0f));
          const uint64_t fp = fixed62(pv);
          p2 += ip ? 0ull : fp;
          r0 += (!ip && !iq) ? wr : 0ull;
          ra += (!ip && iq) ? wr : 0ull;
          rb += (!ip && iq) ? fp : 0ull;
          rpm += (ip && !iq) ? wr : 0ull;
          ndbl += (ip && iq) ? 1u : 0u;
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_wave_barrier();  // list reads done before the next round's writes
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if ((ro + 1) % rpr == 0 || ro + 1 == nround) {
          ChunkRec rc;
          rc.p2 = wave_sum_u64(p2);
          rc.r0 = wave_sum_u64(r0);
          rc.ra = wave_sum_u64(ra);
          rc.rb = wave_sum_u64(rb);
          rc.rp = wave_sum_u64(rpm);
          rc.np = wave_sum_u32(np);
          rc.nq = wave_sum_u32(nq);
          rc.ndbl = wave_sum_u32(ndbl);
          rc.pad = 0;
          rc.pad2 = 0;
          if (lane == 0) store_rec(a.recs + j * a.nrec + rec, rc);
          p2 = r0 = ra = rb = rpm = 0;
          np = nq = ndbl = 0;
        }
      };
      // 16-bit rows, lean: keys from packed codes, group-member counts from
      // ballots (scalar popcounts), the ids that may carry p mass (p's kept
      // keys, ~2% under a nucleus) compacted by ballot into this wave's LDS list
      // as packed (p code, q code) and evaluated one per lane, sums
      // accumulated with LDS atomics (no per-record wave reductions).
      uint32_t np_s = 0, nq_s = 0;
      if constexpr (Ev::kGroups) {
        if (lane < 6) acc[w][lane] = 0ull;
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_wave_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
      }
      auto round16 = [&](const typename Ev::Raw& cp, const typename Ev::Raw& cq, int64_t ro) {
        if constexpr (Ev::kGroups) {
          const int64_t s0 = x_beg + ro * kDrawSub;
          const int64_t rec = s0 / a.rec_ids;
          const int64_t e1 = min(a.V, (rec + 1) * a.rec_ids);
          const int nvalid = (int)max<int64_t>(0, min<int64_t>(8, e1 - (s0 + lane_off)));
          const int32_t klo_p = rp.st.klo, glo_p = rp.st.glo, ghi_p = rp.st.ghi;
          const int32_t klo_q = hasq ? rq.st.klo : 0x7FFFFFFF;
          const int32_t glo_q = hasq ? rq.st.glo : 1, ghi_q = hasq ? rq.st.ghi : 0;
          const uint32_t pw[4] = {cp.x, cp.y, cp.z, cp.w};
          const uint32_t qw[4] = {cq.x, cq.y, cq.z, cq.w};
          uint32_t kp2[4], kq2[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            kp2[i] = keys2_of_codes2(pw[i]);
            kq2[i] = keys2_of_codes2(qw[i]);
          }
          uint32_t* lst = reinterpret_cast<uint32_t*>(&lst_p[w][0]);
          uint32_t off = 0;
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            const int sh = 16 * (t & 1);
            const int32_t kp = (int32_t)((kp2[t >> 1] >> sh) & 0xFFFFu);
            const int32_t kq = (int32_t)((kq2[t >> 1] >> sh) & 0xFFFFu);
            const bool valid = t < nvalid;
            const bool lv = valid && kp >= klo_p;
            const uint64_t bl = __ballot(lv);
            np_s += (uint32_t)__popcll(__ballot(valid && kp >= glo_p && kp <= ghi_p));
            nq_s += (uint32_t)__popcll(__ballot(valid && kq >= glo_q && kq <= ghi_q));
            if (lv) {
              const uint32_t pos =
                  off + __builtin_amdgcn_mbcnt_hi((uint32_t)(bl >> 32),
                                                  __builtin_amdgcn_mbcnt_lo((uint32_t)bl, 0u));
              lst[pos] = ((pw[t >> 1] >> sh) & 0xFFFFu) | (((qw[t >> 1] >> sh) & 0xFFFFu) << 16);
            }
            off += (uint32_t)__popcll(bl);
          }
          __atomic_signal_fence(__ATOMIC_SEQ_CST);
          __builtin_amdgcn_wave_barrier();
          __atomic_signal_fence(__ATOMIC_SEQ_CST);
          auto tval = [&](const RowStat& st, const float* tb, int32_t key, uint32_t code) -> float {
            const int32_t tt = st.kmax - key;
            if (tt < st.ntbl) return tb[tt];
            return val16_exp<Ev::kFmt>(code, ev.T, st.m, st.zf, st.totf);
          };
          for (uint32_t i = lane; i < off; i += kWave) {
            const uint32_t e = lst[i];
            const uint32_t cpd = e & 0xFFFFu, cqd = e >> 16;
            const int32_t kp = (int32_t)key_of_code16(cpd), kq = (int32_t)key_of_code16(cqd);
            const bool ip = kp >= glo_p && kp <= ghi_p;
            const bool iq = kq >= glo_q && kq <= ghi_q;
            const float pv = ip ? rp.vg : tval(rp.st, tbl_p, kp, cpd);
            float qv = 0.0f;
            if (hasq) qv = iq ? rq.vg : (kq >= klo_q ? tval(rq.st, tbl_q, kq, cqd) : 0.0f);
            const uint64_t wr = fixed62(fmaxf(pv - qv, 0.0f));
            const uint64_t fp = fixed62(pv);
            atomicAdd(&acc[w][0], ip ? 0ull : fp);
            atomicAdd(&acc[w][1], (!ip && !iq) ? wr : 0ull);
            atomicAdd(&acc[w][2], (!ip && iq) ? wr : 0ull);
            atomicAdd(&acc[w][3], (!ip && iq) ? fp : 0ull);
            atomicAdd(&acc[w][4], (ip && !iq) ? wr : 0ull);
            atomicAdd(&acc[w][5], (ip && iq) ? 1ull : 0ull);
          }
          __atomic_signal_fence(__ATOMIC_SEQ_CST);
          __builtin_amdgcn_wave_barrier();  // list / sums settled before reuse
          __atomic_signal_fence(__ATOMIC_SEQ_CST);
          if ((ro + 1) % rpr == 0 || ro + 1 == nround) {
            if (lane == 0) {
              ChunkRec rc;
              rc.p2 = acc[w][0];
              rc.r0 = acc[w][1];
              rc.ra = acc[w][2];
              rc.rb = acc[w][3];
              rc.rp = acc[w][4];
              rc.ndbl = (uint32_t)acc[w][5];
              rc.np = np_s;
              rc.nq = nq_s;
              rc.pad = 0;
              rc.pad2 = 0;
              store_rec(a.recs + j * a.nrec + rec, rc);
              for (int i = 0; i < 6; ++i) acc[w][i] = 0ull;
            }
            np_s = nq_s = 0;
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_wave_barrier();
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
          }
        } else {
          round(cp, cq, ro);
        }
      };
      typename Ev::Raw ap = {}, aq = {}, bp_ = {}, bq_ = {};
      ap = ev.fetch(rp, x_beg + lane_off, x_end);
      if (hasq) aq = ev.fetch(rq, x_beg + lane_off, x_end);
      if (nround > 1) {
        bp_ = ev.fetch(rp, x_beg + kDrawSub + lane_off, x_end);
        if (hasq) bq_ = ev.fetch(rq, x_beg + kDrawSub + lane_off, x_end);
      }
      for (int64_t ro = 0; ro < nround; ro += 2) {
        round16(ap, aq, ro);
        if (ro + 2 < nround) {
          const int64_t x = x_beg + (ro + 2) * kDrawSub + lane_off;
          ap = ev.fetch(rp, x, x_end);
          if (hasq) aq = ev.fetch(rq, x, x_end);
        }
        if (ro + 1 < nround) {
          round16(bp_, bq_, ro + 1);
          if (ro + 3 < nround) {
            const int64_t x = x_beg + (ro + 3) * kDrawSub + lane_off;
            bp_ = ev.fetch(rp, x, x_end);
            if (hasq) bq_ = ev.fetch(rq, x, x_end);
          }
        }
      }
    }
  }
  if (!a.y) return;

  // ---- 3. the block that completes the job's records draws. Each wave waits
  // for its record stores (vmcnt(0)) before the block's counter increment, so
  // the block that sees the last increment sees every record (agent-scope
  // fences would write back the whole L2 in every block).
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

  const int32_t sp = Ev::rstar(rp), sq = hasq ? Ev::rstar(rq) : 0;
  const float vp = rp.vg, vq = hasq ? rq.vg : 0.0f;
  // thread t owns records [rb0, rb1): member ranks at their starts, exact
  // masses where both groups' kept members are all-or-nothing. Up to two
  // records per thread (vocabularies up to 262,144) stay in registers.
  const int per = (a.nrec + SM_NT - 1) / SM_NT;
  const int rb0 = min(a.nrec, (int)threadIdx.x * per), rb1 = min(a.nrec, rb0 + per);
  const ChunkRec* jrecs = a.recs + j * a.nrec;
  ChunkRec cache[2];
  if (per <= 2) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      if (rb0 + i < rb1) cache[i] = load_rec(jrecs + rb0 + i);
  }
  auto rec_at = [&](int r) -> ChunkRec {
    if (per <= 2) return r == rb0 ? cache[0] : cache[1];
    return load_rec(jrecs + r);
  };
  uint64_t cnt = 0;
  for (int r = rb0; r < rb1; ++r) {
    const ChunkRec rec = rec_at(r);
    cnt += (uint64_t)rec.np | ((uint64_t)rec.nq << 32);
  }
  uint64_t tot_n;
  const uint64_t ex_n = block_excl_u64(cnt, s64, &tot_n);
  uint64_t sum_r = 0, sum_p = 0;
  {
    uint32_t bp = (uint32_t)ex_n, bq = (uint32_t)(ex_n >> 32);
    for (int r = rb0; r < rb1; ++r) {
      const ChunkRec rec = rec_at(r);
      uint64_t pm, rm;
      if (!rec_masses(rec, bp, bq, sp, sq, vp, vq, hasq, &pm, &rm)) {
        // at most one record where p's kept members run out, one for q's
        const int64_t kp = min<int64_t>(max<int64_t>((int64_t)sp - bp, 0), rec.np);
        const int slot = (kp != 0 && kp != (int64_t)rec.np) ? 0 : 1;
        s_part[slot] = r;
        s_pbase[2 * slot] = bp;
        s_pbase[2 * slot + 1] = bq;
      }
      sum_r += rm;
      sum_p += pm;
      bp += rec.np;
      bq += rec.nq;
    }
  }
  __syncthreads();
  // the (at most two) records where a group's kept members run out: one wave each
  const int pa = s_part[0], pb = s_part[1];
  if ((pa >= 0 || pb >= 0) && w < 2) {
    const int rr = w == 0 ? pa : pb;
    if (rr >= 0 && !(w == 1 && rr == pa)) {
      const int64_t i0 = (int64_t)rr * a.rec_ids, i1 = min(a.V, i0 + a.rec_ids);
      const uint64_t m = wave_walk(ev, rp, rq, true, i0, i1, s_pbase[2 * w], s_pbase[2 * w + 1], 0,
                                   false, 0, &s_found);
      if (lane == 0) s_rm[w] = m;
    }
  }
  if (pa >= 0 || pb >= 0) __syncthreads();
  for (int i = 0; i < 2; ++i) {
    const int rr = i == 0 ? pa : pb;
    if (rr >= rb0 && rr < rb1 && !(i == 1 && rr == pa)) sum_r += s_rm[i];
  }
  // totals (one paired scan), degenerate-residual rule (sampling.py:85-88),
  // the record holding the target
  uint64_t ex_r, ex_p, tot_r, tot_p;
  {
    const uint64_t ir = wave_incl_scan_u64(sum_r, lane), ip = wave_incl_scan_u64(sum_p, lane);
    if (lane == kWave - 1) { s64[w] = ir; s_rm2[w] = ip; }
    __syncthreads();
    uint64_t orr = 0, opp = 0;
    tot_r = 0;
    tot_p = 0;
#pragma unroll
    for (int i = 0; i < SM_NW; ++i) {
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
    if (a.acc.stats && a.acc.flags) {
      uint32_t fl = s_fl;
      if (yv >= 0 && (Ev::in_tie_group(rp, yv) || (use_r && Ev::in_tie_group(rq, yv))))
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
          rm = r == pa ? s_rm[0] : s_rm[1];
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
  if (w == 0) {
    const int64_t packed = s_pick[1];
    const int64_t i0 = rec_star * a.rec_ids, i1 = min(a.V, i0 + a.rec_ids);
    wave_walk(ev, rp, rq, use_r, i0, i1, (uint32_t)(packed & 0xFFFFFFFF),
              (uint32_t)(packed >> 32), (uint64_t)s_pick[2], true, t, &s_found);
  }
  __syncthreads();
  finish(s_found);
}

// ---------------------------------------------------------------- verify draw, 16-bit rows
// The draw body (sdx_draw16.hpp) on its own grid: nblk blocks per batch row.
// NOQ: k = 0 (draft steps), no job has a q row.
template <int FMT, bool NOQ = false>
__global__ void __launch_bounds__(SM_NT) __attribute__((amdgpu_waves_per_eu(5)))
draw16_kernel(Draw16Args<FMT> a) {
  __shared__ Draw16Lds S;
  // The blocks of one job share an XCD (consecutive block indices go to the 8
  // XCDs in turn, so block % 8 picks the XCD): the completing block then finds
  // the job's records and rows in its own L2.
  int64_t j;
  int bi;
  if (a.xcd) {
    const int64_t i = (int64_t)blockIdx.x >> 3;
    j = (int64_t)(blockIdx.x & 7) + 8 * (i / a.nblk);
    bi = (int)(i % a.nblk);
  } else {
    j = (int64_t)blockIdx.x / a.nblk;
    bi = (int)((int64_t)blockIdx.x % a.nblk);
  }
  draw16_body<FMT, false, SM_NT, kRec16Rounds, false, NOQ>(a, S, j, bi);
}

// ---------------------------------------------------------------- to_probs output
// Rows are cut into chunks of kMatRounds block rounds (SM_ROUND ids each), one
// workgroup each, which writes the chunk's probabilities. A row whose boundary
// tie group is partially kept needs, in every chunk, the number of group members
// before it (members are kept lowest ids first). One pass does both, with a
// decoupled look-back: each workgroup counts the members of its chunk from the
// codes it has loaded anyway, publishes the count (bit 31 marks it published),
// then sums the counts of the row's earlier chunks as they appear. The words are
// cleared by the row statistics kernel of the same call (zero_per_row = nchunk).
// The wait ends: a chunk waits only for chunks of lower workgroup index, which
// are dispatched before it and publish before they wait. It is bounded all the
// same (kMatWaitTicks of the 100 MHz counter, or the smaller bound the launcher
// passes); a chunk that gives up writes NaN.
constexpr int kMatRounds = (int)(kMatChunk / SM_ROUND);
static_assert(kMatChunk % SM_ROUND == 0, "whole block rounds per chunk");
constexpr uint64_t kMatWaitTicks = 2000000;  // 20 ms
constexpr uint32_t kMatPublished = 0x80000000u;

struct MaterializeArgs {
  int64_t V;
  int64_t chunk;     // ids per chunk, kMatRounds * SM_ROUND
  int32_t nchunk;
  uint32_t* counts;  // [rows, nchunk] group members per chunk | kMatPublished
  float* out;
  int64_t ld_out;
  bool vec_out;      // out 16-byte aligned and ld_out % 4 == 0
  uint64_t wait_ticks;  // look-back bound, at most kMatWaitTicks
};

__device__ __forceinline__ bool partial_group(const RowStat& st) {
  return st.rstar > 0 && st.rstar < st.gcount;
}

typedef unsigned short mat_us2 __attribute__((ext_vector_type(2)));
constexpr int kMatScans = (kMatRounds + 3) / 4;  // 64-bit scans of four 16-bit round counts

template <int FMT>
__global__ void __launch_bounds__(SM_NT) materialize16_kernel(Eval16<FMT> ev, MaterializeArgs a) {
  __shared__ float tbl[kTbl + 1];  // + the "not kept" entry of the one-lookup form
  __shared__ uint32_t s32[SM_NW];
  __shared__ uint64_t s64[SM_NW];
  __shared__ int32_t s_fail;
  const int64_t row = (int64_t)blockIdx.x / a.nchunk;
  const int64_t cidx = (int64_t)blockIdx.x % a.nchunk;
  const int64_t c0 = cidx * a.chunk;
  const int64_t c1 = min(a.V, c0 + a.chunk);
  typename Eval16<FMT>::Row r;
  r.ptr = row < ev.split ? ev.base + row * ev.ld : ev.base2 + (row - ev.split) * ev.ld2;
  // the chunk's loads first, then the table
  uint4 raw[kMatRounds];
#pragma unroll
  for (int u = 0; u < kMatRounds; ++u) {
    const int64_t idx = c0 + (int64_t)u * SM_ROUND + (int64_t)threadIdx.x * 8;
    raw[u] = idx < c1 ? ev.fetch(r, idx, c1) : make_uint4(0, 0, 0, 0);
  }
  ev.stage(row, tbl);
  if (threadIdx.x == 0) s_fail = 0;
  __syncthreads();
  ev.bind(r, row, tbl);
  float* o = a.out + row * a.ld_out;
  const bool part = partial_group(r.st);
  uint32_t* const cnt_row = a.counts + row * a.nchunk;
  if (part) {  // uniform: this chunk's members, published before anything waits
    // whole 8-id groups on packed keys: key - glo (mod 2^16) is at most ghi - glo
    // exactly for a member (a partial group is not empty), so the saturating
    // (ghi - glo + 1) - (key - glo), capped at 1, is 1 for a member and 0 otherwise;
    // the padding of fetch() past the row's end (code 0xFFFF, key 0) is no member
    typedef unsigned short mc_us2 __attribute__((ext_vector_type(2)));
    const mc_us2 glo2 = {(unsigned short)r.st.glo, (unsigned short)r.st.glo};
    const mc_us2 span2 = {(unsigned short)(r.st.ghi - r.st.glo + 1),
                          (unsigned short)(r.st.ghi - r.st.glo + 1)};
    uint32_t cnt = 0;
#pragma unroll
    for (int u = 0; u < kMatRounds; ++u) {
      const int64_t idx = c0 + (int64_t)u * SM_ROUND + (int64_t)threadIdx.x * 8;
      if (idx < c1) {
        mc_us2 pk = {0, 0};
        const uint32_t w[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const mc_us2 d = __builtin_bit_cast(mc_us2, keys2_of_codes2(w[t])) - glo2;
          pk += __builtin_elementwise_min(__builtin_elementwise_sub_sat(span2, d), (mc_us2){1, 1});
        }
        cnt += (uint32_t)pk[0] + (uint32_t)pk[1];
      }
    }
    uint32_t tot;
    block_excl_u32(cnt, s32, &tot);
    if (threadIdx.x == 0)
      __hip_atomic_store(cnt_row + cidx, tot | kMatPublished, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  if (r.st.flags & kRowUnsupported) {  // outside the row kernel's windows: mark, don't guess
    for (int64_t i = c0 + threadIdx.x; i < c1; i += SM_NT) o[i] = __builtin_nanf("");
    return;
  }
  uint32_t rank = 0;
  if (part) {  // uniform: members in earlier chunks, as they are published
    uint32_t v = 0;
    for (int64_t c = threadIdx.x; c < cidx; c += SM_NT) {
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      for (;;) {
        const uint32_t w =
            __hip_atomic_load(cnt_row + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (w & kMatPublished) {
          v += w & ~kMatPublished;
          break;
        }
        if (__builtin_amdgcn_s_memrealtime() - t0 > a.wait_ticks) {
          s_fail = 1;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    block_excl_u32(v, s32, &rank);
    if (s_fail) {  // uniform (read after the scan's barrier)
      for (int64_t i = c0 + threadIdx.x; i < c1; i += SM_NT) o[i] = __builtin_nanf("");
      return;
    }
  }
  // One lookup per id, for rows whose kept keys [klo, kmax] all lie in the table
  // (nearly every row; klo >= 1 keeps key 0, the padding past the row's end, out):
  // entry kmax - key holds the output of a kept non-member, the group's entries
  // hold the output of a kept member (its value, or 0 when no member is kept),
  // and entry Z = kmax - klo + 1, where every key below klo lands, holds 0. Packed
  // 16-bit: index = min(sat(kmax - key), Z) for two ids at once. Outputs equal
  // eval()'s: live ids take tbl[kmax - key] or the group value, the others 0.
  const int32_t kmax = r.st.kmax, klo = r.st.klo;
  if ((r.st.flags & kRowNonfinite) == 0 && klo >= 1 && klo <= kmax &&
      kmax - klo <= r.st.ntbl - 1) {  // uniform
    const int32_t Z = kmax - klo + 1;
    const int32_t gl = max(r.st.glo, klo), gh = min(r.st.ghi, kmax);
    const float bv = r.st.rstar <= 0 ? 0.0f : r.vg;
    __syncthreads();  // every bind() has read the table
    for (int32_t e = kmax - gh + (int32_t)threadIdx.x; e <= kmax - gl; e += SM_NT) tbl[e] = bv;
    if (threadIdx.x == 0) tbl[Z] = 0.0f;
    // member ranks (a partially kept group): bits per round (four rounds to a
    // word), then block scans of the per-thread counts packed four rounds to a
    // 64-bit word (16-bit fields: a round holds at most SM_ROUND members)
    uint32_t mk[kMatScans];
    uint64_t es[kMatScans], ts[kMatScans];
#pragma unroll
    for (int i = 0; i < kMatScans; ++i) mk[i] = 0u, es[i] = 0ull, ts[i] = 0ull;
    if (part) {  // uniform
      const mat_us2 gl2 = {(unsigned short)gl, (unsigned short)gl};
      const mat_us2 sp2 = {(unsigned short)(gh - gl + 1), (unsigned short)(gh - gl + 1)};
      uint64_t cs[kMatScans];
#pragma unroll
      for (int i = 0; i < kMatScans; ++i) cs[i] = 0ull;
#pragma unroll
      for (int u = 0; u < kMatRounds; ++u) {
        const int64_t idx = c0 + (int64_t)u * SM_ROUND + (int64_t)threadIdx.x * 8;
        uint32_t m = 0;
        if (idx < c1) {
          const uint32_t w[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const mat_us2 d = __builtin_bit_cast(mat_us2, keys2_of_codes2(w[i])) - gl2;
            const mat_us2 b = __builtin_elementwise_min(__builtin_elementwise_sub_sat(sp2, d),
                                                        (mat_us2){1, 1});
            m |= ((uint32_t)b[0] << (2 * i)) | ((uint32_t)b[1] << (2 * i + 1));
          }
        }
        mk[u >> 2] |= m << (8 * (u & 3));
        cs[u >> 2] |= (uint64_t)__popc(m) << (16 * (u & 3));
      }
#pragma unroll
      for (int i = 0; i < kMatScans; ++i)  // (the barriers also order the table's patch)
        es[i] = block_excl_u64(cs[i], s64, &ts[i]);
    } else {
      __syncthreads();
    }
    const mat_us2 kmax2 = {(unsigned short)kmax, (unsigned short)kmax};
    const mat_us2 z2 = {(unsigned short)Z, (unsigned short)Z};
    uint32_t base = rank;
#pragma unroll
    for (int u = 0; u < kMatRounds; ++u) {
      const int64_t r0 = c0 + (int64_t)u * SM_ROUND;
      if (r0 >= c1) break;  // uniform
      const int64_t idx = r0 + (int64_t)threadIdx.x * 8;
      float p[8];
      const uint32_t w[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const mat_us2 d = __builtin_elementwise_min(
            __builtin_elementwise_sub_sat(kmax2, __builtin_bit_cast(mat_us2, keys2_of_codes2(w[i]))),
            z2);
        p[2 * i] = tbl[d[0]];
        p[2 * i + 1] = tbl[d[1]];
      }
      if (part) {
        const int sh = 16 * (u & 3);
        uint32_t rk = base + (uint32_t)((es[u >> 2] >> sh) & 0xFFFFu);
        base += (uint32_t)((ts[u >> 2] >> sh) & 0xFFFFu);
        const uint32_t m = (mk[u >> 2] >> (8 * (u & 3))) & 0xFFu;
        if (m != 0u) {
#pragma unroll
          for (int t2 = 0; t2 < 8; ++t2)
            if ((m >> t2) & 1u) { if ((int32_t)rk >= r.st.rstar) p[t2] = 0.0f; ++rk; }
        }
      }
      if (a.vec_out && idx + 8 <= c1) {
        *reinterpret_cast<float4*>(o + idx) = make_float4(p[0], p[1], p[2], p[3]);
        *reinterpret_cast<float4*>(o + idx + 4) = make_float4(p[4], p[5], p[6], p[7]);
      } else if (idx < c1) {
#pragma unroll
        for (int t2 = 0; t2 < 8; ++t2)
          if (idx + t2 < c1) o[idx + t2] = p[t2];
      }
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < kMatRounds; ++u) {
    const int64_t r0 = c0 + (int64_t)u * SM_ROUND;
    if (r0 >= c1) break;  // uniform
    const int64_t idx = r0 + (int64_t)threadIdx.x * 8;
    float p[8];
    uint32_t m = 0;
    if (idx < c1) {
      m = ev.eval(r, idx, c1, raw[u], p) & 0xFFu;
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) p[t] = 0.0f;
    }
    if (part) {  // member ranks: a block scan per round (members kept lowest ids first)
      uint32_t tot;
      uint32_t rk = rank + block_excl_u32((uint32_t)__popc(m), s32, &tot);
      rank += tot;
      if (m != 0u) {  // few lanes hold members: the others (usually the whole wave) skip
#pragma unroll
        for (int t = 0; t < 8; ++t)
          if ((m >> t) & 1u) { if ((int32_t)rk >= r.st.rstar) p[t] = 0.0f; ++rk; }
      }
    } else if (r.st.rstar <= 0 && m != 0u) {
#pragma unroll
      for (int t = 0; t < 8; ++t)
        if ((m >> t) & 1u) p[t] = 0.0f;
    }
    if (a.vec_out && idx + 8 <= c1) {
      *reinterpret_cast<float4*>(o + idx) = make_float4(p[0], p[1], p[2], p[3]);
      *reinterpret_cast<float4*>(o + idx + 4) = make_float4(p[4], p[5], p[6], p[7]);
    } else if (idx < c1) {
#pragma unroll
      for (int t = 0; t < 8; ++t)
        if (idx + t < c1) o[idx + t] = p[t];
    }
  }
}

// ---------------------------------------------------------------- sample_from_probs
// Inverse-CDF draws from dense fp32 probability rows (no tie groups, no q), in
// two launches and with no counters: every wave sums the fixed62 weights of one
// record of kDenseRec ids (8 float4 loads per lane, all in flight at once);
// then one workgroup per row scans the row's record masses, takes the record
// holding floor(u * total) and walks its ids to the draw. A weight is
// fixed62(p) for p > 0 and 0 otherwise, in both passes, so the walked record's
// ids sum to the mass the first pass gave it.
constexpr int kDenseNT = 256;

__device__ __forceinline__ uint64_t dense_w(float v) { return v > 0.0f ? fixed62(v) : 0ull; }

__global__ void __launch_bounds__(kDenseNT) dense_mass_kernel(DenseArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t g = (int64_t)blockIdx.x * (kDenseNT / kWave) + threadIdx.x / kWave;
  if (g >= a.rows * a.nrec) return;  // whole waves (no block barrier below)
  const int64_t row = g / a.nrec;
  const int64_t x0 = (g % a.nrec) * kDenseRec;
  const int64_t x1 = min(a.V, x0 + kDenseRec);
  const float* src = a.p + row * a.ld;
  uint64_t s = 0;
  if (a.vec && x1 - x0 == kDenseRec) {
    float4 v[kDenseRec / (4 * kWave)];
#pragma unroll
    for (int i = 0; i < kDenseRec / (4 * kWave); ++i)
      v[i] = *reinterpret_cast<const float4*>(src + x0 + ((int64_t)i * kWave + lane) * 4);
#pragma unroll
    for (int i = 0; i < kDenseRec / (4 * kWave); ++i)
      s += dense_w(v[i].x) + dense_w(v[i].y) + dense_w(v[i].z) + dense_w(v[i].w);
  } else {
    for (int64_t i = x0 + lane; i < x1; i += kWave) s += dense_w(src[i]);
  }
  s = wave_sum_u64(s);
  if (lane == 0) a.mass[g] = s;
}

__global__ void __launch_bounds__(kDenseNT) dense_pick_kernel(DenseArgs a) {
  static_assert(kDenseNT == SM_NT, "the block scans span SM_NT threads");
  __shared__ uint64_t s64[SM_NW];
  __shared__ int64_t s_rec;
  __shared__ uint64_t s_base;
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  if (tid == 0) s_rec = -1;
  // ---- the record holding t: thread tid sums records [r0, r1)
  const int per = (a.nrec + kDenseNT - 1) / kDenseNT;
  const int r0 = min(a.nrec, tid * per), r1 = min(a.nrec, r0 + per);
  const uint64_t* m = a.mass + row * a.nrec;
  uint64_t mine = 0;
  for (int r = r0; r < r1; ++r) mine += m[r];
  uint64_t total;
  const uint64_t ex = block_excl_u64(mine, s64, &total);
  if (total == 0) {  // uniform: an all-zero row
    if (tid == 0) a.y[row] = -1;
    return;
  }
  const uint64_t t = uniform_threshold(a.u[row], total);  // < total
  if (ex <= t && t - ex < mine) {  // exactly one thread
    uint64_t run = ex;
    for (int r = r0; r < r1; ++r) {
      if (t - run < m[r]) {
        s_rec = r;
        s_base = run;
        break;
      }
      run += m[r];
    }
  }
  __syncthreads();
  // ---- walk it: thread tid takes 16 consecutive ids
  constexpr int kPer = kDenseRec / kDenseNT;
  const int64_t rs = s_rec;  // >= 0 for u in [0, 1): the record masses sum to total > t
  if (rs < 0) {              // uniform: u outside [0, 1) (a caller error) draws nothing
    if (tid == 0) a.y[row] = -1;
    return;
  }
  const int64_t e1 = min(a.V, rs * kDenseRec + kDenseRec);
  const int64_t i0 = rs * kDenseRec + (int64_t)tid * kPer;
  const float* src = a.p + row * a.ld;
  float v[kPer];
  if (a.vec && i0 + kPer <= e1) {
#pragma unroll
    for (int i = 0; i < kPer / 4; ++i) {
      const float4 x = *reinterpret_cast<const float4*>(src + i0 + 4 * i);
      v[4 * i] = x.x; v[4 * i + 1] = x.y; v[4 * i + 2] = x.z; v[4 * i + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kPer; ++i) v[i] = i0 + i < e1 ? src[i0 + i] : 0.0f;
  }
  uint64_t sum = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) sum += dense_w(v[i]);
  uint64_t tot2;
  const uint64_t st = s_base + block_excl_u64(sum, s64, &tot2);
  if (st <= t && t - st < sum) {  // exactly one thread
    uint64_t acc = st;
    int64_t f = -1;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      acc += dense_w(v[i]);
      if (f < 0 && acc > t) f = i0 + i;
    }
    a.y[row] = f;
  }
}

// ---------------------------------------------------------------- residual_probs output

__global__ void __launch_bounds__(SM_NT) residual_norm_kernel(ResidualNormArgs a) {
  __shared__ uint64_t s64[SM_NW];
  const int64_t row = (int64_t)blockIdx.x / a.nrec;
  const int64_t cidx = (int64_t)blockIdx.x % a.nrec;
  // dense fp32 rows have no tie groups: residual mass is r0, p mass p2
  uint64_t r = 0, p = 0;
  for (int c = threadIdx.x; c < a.nrec; c += SM_NT) {
    const ChunkRec rec = load_rec(a.recs + row * a.nrec + c);
    r += rec.r0;
    p += rec.p2;
  }
  uint64_t totR, totP;
  block_excl_u64(r, s64, &totR);
  block_excl_u64(p, s64, &totP);
  const float fr = rn32_u64(totR);
  const bool use_r = fr > 1e-9f;
  const float tot = fmaxf(use_r ? fr : rn32_u64(totP), 1e-12f);
  const int64_t c0 = cidx * a.rec_ids;
  const int64_t c1 = min(a.V, c0 + a.rec_ids);
  const float* pp = a.p + row * a.ld;
  const float* qq = a.q + row * a.ld;
  float* o = a.out + row * a.ld_out;
  for (int64_t idx = c0 + threadIdx.x; idx < c1; idx += SM_NT) {
    const float v = use_r ? fmaxf(pp[idx] - qq[idx], 0.0f) : pp[idx];
    o[idx] = v / tot;
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
static hipError_t launch_draw(const Ev& ev, const AcceptArgs* acc, SampleJob* jobs,
                              int64_t njobs, int64_t V, ChunkRec* recs, uint32_t* counters,
                              int64_t* y, hipStream_t s) {
  DrawArgs da = {};
  if (acc) da.acc = *acc;
  da.jobs = jobs;
  da.V = V;
  int nrec;
  draw_layout(V, &da.rec_ids, &nrec);
  da.nrec = nrec;
  // records per wave: enough waves to cover the CUs a few times over
  const int64_t waves_wanted = 4096;
  int64_t gw = (njobs * nrec + waves_wanted - 1) / waves_wanted;
  gw = gw < 1 ? 1 : (gw > 16 ? 16 : gw);
  da.gw = (int32_t)gw;
  da.nblk = (int32_t)((nrec + SM_NW * gw - 1) / (SM_NW * gw));
  da.recs = recs;
  da.counters = counters;
  da.y = y;
  hipLaunchKernelGGL((draw_kernel<Ev>), dim3((unsigned)(da.nblk * njobs)), dim3(SM_NT), 0, s, ev,
                     da);
  return hipGetLastError();
}

template <int FMT>
static hipError_t launch_draw16_fmt(const RowSource16& src, const RowStat* stats,
                                    const float* tables, float T, const AcceptArgs& acc,
                                    int64_t njobs, int64_t V, ChunkRec* recs, uint32_t* counters,
                                    int64_t* y, hipStream_t s) {
  Draw16Args<FMT> a = {};
  a.acc = acc;
  a.ev = Eval16<FMT>{src.base, src.ld, src.base2, src.ld2, src.split, stats, tables, T};
  a.V = V;
  a.nrec = (int32_t)((V + kRec16 - 1) / kRec16);
  if (a.nrec > kMaxRec16) return hipErrorInvalidValue;
  a.nblk = (a.nrec + SM_NW - 1) / SM_NW;
  a.xcd = njobs % 8 == 0 ? 1 : 0;
  a.recs = recs;
  a.counters = counters;
  a.y = y;
  if (acc.k == 0 && !acc.cu_k)  // every job draws from its one p row
    hipLaunchKernelGGL((draw16_kernel<FMT, true>), dim3((unsigned)(a.nblk * njobs)), dim3(SM_NT),
                       0, s, a);
  else
    hipLaunchKernelGGL((draw16_kernel<FMT>), dim3((unsigned)(a.nblk * njobs)), dim3(SM_NT), 0, s,
                       a);
  return hipGetLastError();
}

hipError_t launch_draw16(int fmt, const RowSource16& src, const RowStat* stats,
                         const float* tables, float T, const AcceptArgs* acc, SampleJob* jobs,
                         int64_t njobs, int64_t V, ChunkRec* recs, uint32_t* counters, int64_t* y,
                         hipStream_t s) {
  if (!src.vec || !acc || !y || V % 8 != 0) return hipErrorInvalidValue;
  (void)jobs;  // the kernel writes acc->jobs itself
  if (fmt == SDX_BF16)
    return launch_draw16_fmt<SDX_BF16>(src, stats, tables, T, *acc, njobs, V, recs, counters, y, s);
  return launch_draw16_fmt<SDX_F16>(src, stats, tables, T, *acc, njobs, V, recs, counters, y, s);
}

hipError_t launch_draw_rows16(int fmt, const RowSource16& src, const RowStat* stats,
                              const float* tables, float T, SampleJob* jobs, int64_t njobs,
                              int64_t V, ChunkRec* recs, uint32_t* counters, int64_t* y,
                              hipStream_t s) {
  if (!src.vec || V % 8 != 0) return hipErrorInvalidValue;
  if (fmt == SDX_BF16)
    return launch_draw(Eval16<SDX_BF16>{src.base, src.ld, src.base2, src.ld2, src.split, stats,
                                         tables, T},
                       nullptr, jobs, njobs, V, recs, counters, y, s);
  return launch_draw(Eval16<SDX_F16>{src.base, src.ld, src.base2, src.ld2, src.split, stats,
                                      tables, T},
                     nullptr, jobs, njobs, V, recs, counters, y, s);
}

hipError_t launch_draw_probs(const RowSourceF32& src, const AcceptArgs* acc, SampleJob* jobs,
                             int64_t njobs, int64_t V, ChunkRec* recs, uint32_t* counters,
                             int64_t* y, hipStream_t s, const uint32_t* tie_bits) {
  EvalProb ev{src.base, src.ld, src.base2, src.ld2, src.split, src.vec, tie_bits, f32_tie_words(V)};
  return launch_draw(ev, acc, jobs, njobs, V, recs, counters, y, s);
}

hipError_t launch_chunk_mass_probs(const RowSourceF32& src, SampleJob* jobs, int64_t njobs,
                                   int64_t V, ChunkRec* recs, hipStream_t s) {
  EvalProb ev{src.base, src.ld, src.base2, src.ld2, src.split, src.vec, nullptr, 0};
  return launch_draw(ev, nullptr, jobs, njobs, V, recs, nullptr, nullptr, s);
}

// The look-back bound: kMatWaitTicks, or a smaller bound from SDX_PROBS_WAIT_TICKS
// (read at every launch; tests set 0 so that a chunk whose earlier chunks have not
// all published at its first poll gives up, while every kernel exits normally).
static uint64_t mat_wait_ticks() {
  const char* e = getenv("SDX_PROBS_WAIT_TICKS");
  if (!e || !*e) return kMatWaitTicks;
  char* end = nullptr;
  const unsigned long long v = strtoull(e, &end, 10);
  if (!end || *end != '\0') return kMatWaitTicks;
  return v < kMatWaitTicks ? (uint64_t)v : kMatWaitTicks;
}

hipError_t launch_materialize16(int fmt, const RowSource16& src, const RowStat* stats,
                                const float* tables, float T, int64_t rows, int64_t V,
                                int64_t chunk, int nchunk, uint32_t* counts, float* out,
                                int64_t ld_out, hipStream_t s) {
  if (!src.vec) return hipErrorInvalidValue;
  if (chunk != (int64_t)kMatRounds * SM_ROUND) return hipErrorInvalidValue;
  MaterializeArgs ma{V, chunk, nchunk, counts, out, ld_out,
                     ((uintptr_t)out & 15u) == 0 && (ld_out % 4) == 0, mat_wait_ticks()};
  const dim3 grid((unsigned)(nchunk * rows));
  if (fmt == SDX_BF16) {
    Eval16<SDX_BF16> ev{src.base, src.ld, src.base2, src.ld2, src.split, stats, tables, T};
    hipLaunchKernelGGL((materialize16_kernel<SDX_BF16>), grid, dim3(SM_NT), 0, s, ev, ma);
  } else {
    Eval16<SDX_F16> ev{src.base, src.ld, src.base2, src.ld2, src.split, stats, tables, T};
    hipLaunchKernelGGL((materialize16_kernel<SDX_F16>), grid, dim3(SM_NT), 0, s, ev, ma);
  }
  return hipGetLastError();
}

hipError_t launch_sample_dense(const DenseArgs& a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  if (!a.p || !a.mass || !a.u || !a.y || a.V < 1 || a.ld < a.V ||
      a.nrec != dense_nrec(a.V))
    return hipErrorInvalidValue;
  const int64_t waves = a.rows * a.nrec;
  const int64_t wpb = kDenseNT / kWave;
  hipLaunchKernelGGL(dense_mass_kernel, dim3((unsigned)((waves + wpb - 1) / wpb)), dim3(kDenseNT),
                     0, s, a);
  hipLaunchKernelGGL(dense_pick_kernel, dim3((unsigned)a.rows), dim3(kDenseNT), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_residual_norm(const ResidualNormArgs& a, int64_t rows, hipStream_t s) {
  hipLaunchKernelGGL(residual_norm_kernel, dim3((unsigned)(a.nrec * rows)), dim3(SM_NT), 0, s, a);
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
