// Accept test, residual / bonus inverse-CDF sampling and to_probs output.
//
// Stages after the row statistics (specdec/engine.py:285-303):
//   verify_accept_kernel   one thread per batch row: the accept chain
//                          u < min(1, p(x)/max(q(x), 1e-10)) with the
//                          first-reject scan, and the job for the final draw
//                          (residual at the stop position, or bonus p_{k+1}).
//   chunk_mass_kernel      (rows x chunks) grid: exact fixed62 mass of the
//                          residual (p - q)_+ and of p per chunk of ids.
//   select_kernel          one workgroup per row: degenerate-residual rule
//                          (sampling.py:85-88), target floor(u * total), the
//                          chunk holding it, then an in-chunk block scan for
//                          the first id whose prefix mass exceeds it.
// Element probabilities come from an evaluator: codes + RowStat + table for
// 16-bit logits, or dense fp32 probability rows.
#include "sdx_launch.hpp"

namespace sdx {

constexpr int SM_NT = 256;


// ---------------------------------------------------------------- evaluators
// Rows [0, split) live at base + row*ld, rows [split, ...) at base2 + (row-split)*ld2
// (target rows then draft rows, or p rows then q rows).
template <int FMT>
struct Eval16 {
  const uint16_t* base;
  int64_t ld;
  const uint16_t* base2;
  int64_t ld2;
  int64_t split;
  const RowStat* stats;
  const float* tables;
  float T;
  bool vec;  // rows are 16-byte aligned

  struct Row {
    const uint16_t* ptr;
    RowStat st;
    const float* tbl;
  };
  __device__ void bind(Row& r, int64_t row, const float* lds_tbl) const {
    r.ptr = row < split ? base + row * ld : base2 + (row - split) * ld2;
    r.st = stats[row];
    r.tbl = lds_tbl;
  }
  __device__ static int tbl_len(const RowStat& st) { return (st.flags & kRowGreedy) ? 0 : st.ntbl; }
  __device__ void load8(const Row& r, int64_t idx, int64_t V, float out[8]) const {
    uint32_t c[8];
    if (vec && idx + 8 <= V) {
      const uint4 v = *reinterpret_cast<const uint4*>(r.ptr + idx);
      c[0] = v.x & 0xFFFFu; c[1] = v.x >> 16; c[2] = v.y & 0xFFFFu; c[3] = v.y >> 16;
      c[4] = v.z & 0xFFFFu; c[5] = v.z >> 16; c[6] = v.w & 0xFFFFu; c[7] = v.w >> 16;
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) c[t] = idx + t < V ? r.ptr[idx + t] : 0u;
    }
#pragma unroll
    for (int t = 0; t < 8; ++t)
      out[t] = idx + t < V ? pfinal16<FMT>(r.st, r.tbl, idx + t, c[t], T) : 0.0f;
  }
};

struct EvalProb {
  const float* base;
  int64_t ld;
  const float* base2;
  int64_t ld2;
  int64_t split;
  bool vec;
  struct Row {
    const float* ptr;
  };
  __device__ void bind(Row& r, int64_t row, const float*) const {
    r.ptr = row < split ? base + row * ld : base2 + (row - split) * ld2;
  }
  __device__ void load8(const Row& r, int64_t idx, int64_t V, float out[8]) const {
    if (vec && idx + 8 <= V) {
      const float4 a = *reinterpret_cast<const float4*>(r.ptr + idx);
      const float4 b = *reinterpret_cast<const float4*>(r.ptr + idx + 4);
      out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
      out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) out[t] = idx + t < V ? r.ptr[idx + t] : 0.0f;
    }
  }
};

// Load a row's table into LDS (16-bit evaluator only).
template <int FMT>
__device__ void stage_table(const Eval16<FMT>& ev, int64_t row, float* lds) {
  const RowStat st = ev.stats[row];
  const int n = Eval16<FMT>::tbl_len(st);
  for (int t = threadIdx.x; t < n; t += blockDim.x) lds[t] = ev.tables[row * kTbl + t];
}
__device__ inline void stage_table(const EvalProb&, int64_t, float*) {}

// ---------------------------------------------------------------- accept chain

__global__ void verify_accept_kernel(AcceptArgs a) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= a.batch) return;
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
  SampleJob j;
  if (n == k) {
    j.prow = trow0 + k;
    j.qrow = -1;
  } else {
    j.prow = trow0 + n;
    j.qrow = drow0 + n;
  }
  j.u = a.u_final[b];
  j.pad = 0;
  a.jobs[b] = j;
  a.n_acc[b] = n;
  a.flags[b] = (uint8_t)fl;
}

// ---------------------------------------------------------------- chunk masses
struct ChunkArgs {
  const SampleJob* jobs;
  int64_t V;
  int64_t chunk;      // ids per chunk (multiple of 8)
  int32_t nchunk;
  uint64_t* sums;     // [jobs, nchunk, 2]: residual mass, p mass
};

template <class Ev>
__global__ void __launch_bounds__(SM_NT) chunk_mass_kernel(Ev ev, ChunkArgs a) {
  __shared__ float tbl_p[kTbl];
  __shared__ float tbl_q[kTbl];
  __shared__ uint64_t red[2 * (SM_NT / kWave)];
  const int64_t j = (int64_t)blockIdx.x / a.nchunk;
  const int c = (int)((int64_t)blockIdx.x % a.nchunk);
  const SampleJob job = a.jobs[j];
  stage_table(ev, job.prow, tbl_p);
  if (job.qrow >= 0) stage_table(ev, job.qrow, tbl_q);
  __syncthreads();
  typename Ev::Row rp, rq;
  ev.bind(rp, job.prow, tbl_p);
  if (job.qrow >= 0) ev.bind(rq, job.qrow, tbl_q);
  const int64_t c0 = (int64_t)c * a.chunk;
  const int64_t c1 = min(a.V, c0 + a.chunk);
  uint64_t R = 0, P = 0;
  for (int64_t idx = c0 + (int64_t)threadIdx.x * 8; idx < c1; idx += (int64_t)SM_NT * 8) {
    float p[8], q[8];
    ev.load8(rp, idx, c1, p);
    if (job.qrow >= 0) {
      ev.load8(rq, idx, c1, q);
#pragma unroll
      for (int t = 0; t < 8; ++t) R += fixed62(fmaxf(p[t] - q[t], 0.0f));
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) P += fixed62(p[t]);
  }
  R = wave_sum_u64(R);
  P = wave_sum_u64(P);
  const int w = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) { red[2 * w] = R; red[2 * w + 1] = P; }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t r2 = 0, p2 = 0;
    for (int w2 = 0; w2 < SM_NT / kWave; ++w2) { r2 += red[2 * w2]; p2 += red[2 * w2 + 1]; }
    a.sums[(j * a.nchunk + c) * 2] = r2;
    a.sums[(j * a.nchunk + c) * 2 + 1] = p2;
  }
}

// ---------------------------------------------------------------- select
struct SelectArgs {
  const SampleJob* jobs;
  int64_t V;
  int64_t chunk;
  int32_t nchunk;
  const uint64_t* sums;
  int64_t* y;
};

template <class Ev>
__global__ void __launch_bounds__(SM_NT) select_kernel(Ev ev, SelectArgs a) {
  __shared__ float tbl_p[kTbl];
  __shared__ float tbl_q[kTbl];
  __shared__ uint64_t s_scan[SM_NT];
  __shared__ int64_t s_pick[4];
  __shared__ int32_t s_mode;
  const int64_t j = blockIdx.x;
  const SampleJob job = a.jobs[j];
  stage_table(ev, job.prow, tbl_p);
  if (job.qrow >= 0) stage_table(ev, job.qrow, tbl_q);
  if (threadIdx.x == 0) {
    // residual mass decides the mode (sampling.py:85-88); sums are exact
    uint64_t totR = 0, totP = 0;
    for (int c = 0; c < a.nchunk; ++c) {
      totR += a.sums[(j * a.nchunk + c) * 2];
      totP += a.sums[(j * a.nchunk + c) * 2 + 1];
    }
    const bool use_r = job.qrow >= 0 && rn32_u64(totR) > 1e-9f;
    const uint64_t tot = use_r ? totR : totP;
    int64_t pick = -1, cstar = -1;
    uint64_t base = 0, t = 0;
    if (tot > 0) {
      t = uniform_threshold(job.u, tot);
      for (int c = 0; c < a.nchunk; ++c) {
        const uint64_t w = a.sums[(j * a.nchunk + c) * 2 + (use_r ? 0 : 1)];
        if (base + w > t) { cstar = c; break; }
        base += w;
      }
    }
    s_mode = use_r ? 1 : 0;
    s_pick[0] = cstar;
    s_pick[1] = (int64_t)base;
    s_pick[2] = (int64_t)t;
    s_pick[3] = pick;
  }
  __syncthreads();
  const int64_t cstar = s_pick[0];
  if (cstar < 0) {
    if (threadIdx.x == 0) a.y[j] = -1;
    return;
  }
  const bool use_r = s_mode != 0;
  const uint64_t base = (uint64_t)s_pick[1], t = (uint64_t)s_pick[2];
  typename Ev::Row rp, rq;
  ev.bind(rp, job.prow, tbl_p);
  if (use_r) ev.bind(rq, job.qrow, tbl_q);
  const int64_t c0 = cstar * a.chunk;
  const int64_t c1 = min(a.V, c0 + a.chunk);
  // each thread owns a contiguous run of `per` ids (multiple of 8)
  const int64_t n = c1 - c0;
  const int64_t per = ((n + SM_NT - 1) / SM_NT + 7) / 8 * 8;
  const int64_t r0 = c0 + (int64_t)threadIdx.x * per;
  const int64_t r1 = min(c1, r0 + per);
  auto weights8 = [&](int64_t idx, uint64_t w[8]) {
    float p[8], q[8];
    ev.load8(rp, idx, r1, p);
    if (use_r) {
      ev.load8(rq, idx, r1, q);
#pragma unroll
      for (int u = 0; u < 8; ++u) w[u] = fixed62(fmaxf(p[u] - q[u], 0.0f));
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u) w[u] = fixed62(p[u]);
    }
  };
  uint64_t mine = 0;
  for (int64_t idx = r0; idx < r1; idx += 8) {
    uint64_t w[8];
    weights8(idx, w);
#pragma unroll
    for (int u = 0; u < 8; ++u) mine += w[u];
  }
  // block exclusive scan of per-thread masses (Hillis-Steele in LDS)
  s_scan[threadIdx.x] = mine;
  __syncthreads();
  for (int o = 1; o < SM_NT; o <<= 1) {
    const uint64_t v = threadIdx.x >= (unsigned)o ? s_scan[threadIdx.x - o] : 0;
    __syncthreads();
    s_scan[threadIdx.x] += v;
    __syncthreads();
  }
  const uint64_t excl = s_scan[threadIdx.x] - mine;
  const uint64_t start = base + excl;
  if (start <= t && start + mine > t) {
    uint64_t run = start;
    int64_t found = -1;
    for (int64_t idx = r0; idx < r1 && found < 0; idx += 8) {
      uint64_t w[8];
      weights8(idx, w);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (found < 0) {
          run += w[u];
          if (run > t) found = idx + u;
        }
      }
    }
    a.y[j] = found;
  }
}

// ---------------------------------------------------------------- to_probs output
struct MaterializeArgs {
  int64_t V;
  int64_t chunk;
  int32_t nchunk;
  float* out;
  int64_t ld_out;
};

template <int FMT>
__global__ void __launch_bounds__(SM_NT) materialize16_kernel(Eval16<FMT> ev, MaterializeArgs a) {
  __shared__ float tbl[kTbl];
  const int64_t row = (int64_t)blockIdx.x / a.nchunk;
  const int64_t cidx = (int64_t)blockIdx.x % a.nchunk;
  stage_table(ev, row, tbl);
  __syncthreads();
  typename Eval16<FMT>::Row r;
  ev.bind(r, row, tbl);
  const int64_t c0 = cidx * a.chunk;
  const int64_t c1 = min(a.V, c0 + a.chunk);
  float* o = a.out + row * a.ld_out;
  for (int64_t idx = c0 + (int64_t)threadIdx.x * 8; idx < c1; idx += (int64_t)SM_NT * 8) {
    float p[8];
    ev.load8(r, idx, c1, p);
#pragma unroll
    for (int t = 0; t < 8; ++t)
      if (idx + t < c1) o[idx + t] = p[t];
  }
}

// ---------------------------------------------------------------- residual_probs output

__global__ void __launch_bounds__(SM_NT) residual_norm_kernel(ResidualNormArgs a) {
  __shared__ float s_tot;
  __shared__ int s_use_r;
  const int64_t row = (int64_t)blockIdx.x / a.nchunk;
  const int64_t cidx = (int64_t)blockIdx.x % a.nchunk;
  if (threadIdx.x == 0) {
    uint64_t totR = 0, totP = 0;
    for (int c = 0; c < a.nchunk; ++c) {
      totR += a.sums[(row * a.nchunk + c) * 2];
      totP += a.sums[(row * a.nchunk + c) * 2 + 1];
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
hipError_t launch_accept(const AcceptArgs& a, hipStream_t s) {
  const int nt = 128;
  hipLaunchKernelGGL(verify_accept_kernel, dim3((unsigned)((a.batch + nt - 1) / nt)), dim3(nt), 0,
                     s, a);
  return hipGetLastError();
}

template <class Ev>
static hipError_t launch_draw(const Ev& ev, const SampleJob* jobs, int64_t njobs, int64_t V,
                              int64_t chunk, int nchunk, uint64_t* sums, int64_t* y,
                              hipStream_t s) {
  ChunkArgs ca{jobs, V, chunk, nchunk, sums};
  hipLaunchKernelGGL((chunk_mass_kernel<Ev>), dim3((unsigned)(nchunk * njobs)),
                     dim3(SM_NT), 0, s, ev, ca);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  SelectArgs sa{jobs, V, chunk, nchunk, sums, y};
  hipLaunchKernelGGL((select_kernel<Ev>), dim3((unsigned)njobs), dim3(SM_NT), 0, s, ev, sa);
  return hipGetLastError();
}

hipError_t launch_draw16(int fmt, const RowSource16& src, const RowStat* stats,
                         const float* tables, float T, const SampleJob* jobs, int64_t njobs,
                         int64_t V, int64_t chunk, int nchunk, uint64_t* sums, int64_t* y,
                         hipStream_t s) {
  if (fmt == SDX_BF16) {
    Eval16<SDX_BF16> ev{src.base, src.ld, src.base2, src.ld2, src.split, stats, tables, T, src.vec};
    return launch_draw(ev, jobs, njobs, V, chunk, nchunk, sums, y, s);
  }
  Eval16<SDX_F16> ev{src.base, src.ld, src.base2, src.ld2, src.split, stats, tables, T, src.vec};
  return launch_draw(ev, jobs, njobs, V, chunk, nchunk, sums, y, s);
}

hipError_t launch_draw_probs(const RowSourceF32& src, const SampleJob* jobs, int64_t njobs,
                             int64_t V, int64_t chunk, int nchunk, uint64_t* sums, int64_t* y,
                             hipStream_t s) {
  EvalProb ev{src.base, src.ld, src.base2, src.ld2, src.split, src.vec};
  return launch_draw(ev, jobs, njobs, V, chunk, nchunk, sums, y, s);
}

hipError_t launch_chunk_mass_probs(const RowSourceF32& src, const SampleJob* jobs, int64_t njobs,
                                   int64_t V, int64_t chunk, int nchunk, uint64_t* sums,
                                   hipStream_t s) {
  EvalProb ev{src.base, src.ld, src.base2, src.ld2, src.split, src.vec};
  ChunkArgs ca{jobs, V, chunk, nchunk, sums};
  hipLaunchKernelGGL((chunk_mass_kernel<EvalProb>), dim3((unsigned)(nchunk * njobs)),
                     dim3(SM_NT), 0, s, ev, ca);
  return hipGetLastError();
}

hipError_t launch_materialize16(int fmt, const RowSource16& src, const RowStat* stats,
                                const float* tables, float T, int64_t rows, int64_t V,
                                int64_t chunk, int nchunk, float* out, int64_t ld_out,
                                hipStream_t s) {
  MaterializeArgs ma{V, chunk, nchunk, out, ld_out};
  const dim3 grid((unsigned)(nchunk * rows));
  if (fmt == SDX_BF16) {
    Eval16<SDX_BF16> ev{src.base, src.ld, src.base2, src.ld2, src.split, stats, tables, T, src.vec};
    hipLaunchKernelGGL((materialize16_kernel<SDX_BF16>), grid, dim3(SM_NT), 0, s, ev, ma);
  } else {
    Eval16<SDX_F16> ev{src.base, src.ld, src.base2, src.ld2, src.split, stats, tables, T, src.vec};
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
