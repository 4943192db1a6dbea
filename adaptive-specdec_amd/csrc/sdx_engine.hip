// Device-side bookkeeping of a speculative round (specdec/engine.py:228-342),
// so a round needs no host synchronisation:
//   - the draft step's probability of the sampled token, the running
//     confidence product and the early-exit test (engine.py:252-258,
//     controller.py:184-187);
//   - the emission of accepted tokens with the EOS / length stops and the
//     rollback of both caches by k - n_acc (engine.py:305-339);
//   - the draft-length controller's update and choice of the next k
//     (controller.py:121-154), per batch or per row.
#include "sdx_launch.hpp"

namespace sdx {

// ---------------------------------------------------------------- draft step epilogue
// One workgroup. qx[b] = the final probability of the drafted token x[b] under
// its row's to_probs (the draw only picks kept ids, so a member of the row's
// boundary tie group carries the group value); conf[b] *= qx[b]; then the
// batch-shared early-exit test: step >= min_k and mean(conf) < tau, the mean a
// sequential fp32 sum in row order divided by B.
template <int FMT>
__device__ float drafted_prob16(const uint16_t* row, const RowStat& st, const float* tbl,
                                int64_t x, float T) {
  const uint32_t code = row[x];
  const int32_t key = (int32_t)key_of_code16(code);
  if (key < st.klo) return 0.0f;
  if (key >= st.glo && key <= st.ghi)
    return val16<FMT>(st, tbl, code_of_key16((uint32_t)st.glo), T);
  return val16<FMT>(st, tbl, code, T);
}

__global__ void __launch_bounds__(256) draft_epilogue_kernel(DraftEpiArgs a) {
  for (int64_t b = threadIdx.x; b < a.B; b += blockDim.x) {
    const int64_t x = a.x[b];
    float p = 0.0f;
    if (x >= 0 && x < a.V) {
      if (a.greedy) {
        p = 1.0f;
      } else if (a.probs) {
        p = a.probs[b * a.ldp + x];
      } else {
        const uint16_t* row = a.codes + b * a.ld;
        const float* tbl = a.tables + b * kTbl;
        p = a.fmt == SDX_BF16 ? drafted_prob16<SDX_BF16>(row, a.stats[b], tbl, x, a.T)
                              : drafted_prob16<SDX_F16>(row, a.stats[b], tbl, x, a.T);
      }
    }
    if (a.qx) a.qx[b] = p;
    if (a.conf) a.conf[b] = a.conf[b] * p;
    if (a.xcopy) a.xcopy[b] = x;
  }
  if (a.sig && threadIdx.x == 0) {
    const uint32_t w[kDraftSigWords] = {kDraftSig, (uint32_t)a.B, (uint32_t)a.V,
                                        __float_as_uint(a.T), __float_as_uint(a.top_p),
                                        (uint32_t)a.top_k};
    for (int i = 0; i < kDraftSigWords; ++i) a.sig[i] = w[i];
  }
  if (!a.stop) return;
  __threadfence_block();
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t stop = 0;
    if (a.conf && a.step >= a.min_k) {
      float s = 0.0f;
      for (int64_t b = 0; b < a.B; ++b) s = s + a.conf[b];
      stop = (s / (float)a.B) < a.tau ? 1 : 0;
    }
    a.stop[0] = stop;
  }
}

hipError_t launch_draft_epilogue(const DraftEpiArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(draft_epilogue_kernel, dim3(1), dim3(256), 0, s, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------- draft statistics gather
// Block (b, i): row b of draft step i. Its RowStat and table move to draft row
// ntgt + b k + i of the verify workspace; pgather and the tie flags are those the
// row kernel gives a drafted token x = ids[b k + i]: 0 below the cut; a member of
// a partially kept boundary group carries the group value when x is the id the
// draft step drew (a drawn id is kept), else it is ranked by the verify's accept
// chain (kRowRank); any other kept token gets its table (or exp) value.
__global__ void __launch_bounds__(256) draft_gather_kernel(DraftGatherArgs a) {
  const int64_t b = blockIdx.x;
  const int i = (int)blockIdx.y;
  const uint8_t* ws = a.ws[i];
  // the draft step's workspace must still be trusted (a draw wait that gave up
  // overwrote its magic word) and its statistics made for this configuration
  const uint32_t* sig = reinterpret_cast<const uint32_t*>(ws) + kWsDraftSigWord;
  bool ok = reinterpret_cast<const uint32_t*>(ws)[0] == kWsMagic;
  for (int w = 0; w < kDraftSigWords; ++w) ok = ok && sig[w] == a.sig[w];
  const int64_t row = a.ntgt + b * a.k + i;
  RowStat* dst = a.stats + row;
  float* dtb = a.tables + row * kTbl;
  if (!ok) {
    if (threadIdx.x == 0) {
      RowStat st = {};
      st.flags = kRowBadWs | kRowUnsupported;
      st.zf = 1.0f; st.totf = 1.0f; st.klo = 0x7FFFFFFF; st.glo = 1; st.ghi = 0; st.argmax = -1;
      *dst = st;
    }
    return;
  }
  const RowStat* sst = reinterpret_cast<const RowStat*>(ws + a.st_off) + b;
  const float* stb = reinterpret_cast<const float*>(ws + a.tb_off) + b * kTbl;
  RowStat st = *sst;
  for (int t = threadIdx.x; t < st.ntbl; t += blockDim.x) dtb[t] = stb[t];
  if (threadIdx.x != 0) return;
  const int64_t x = a.ids[b * a.k + i];
  float pg = 0.0f;
  st.flags &= ~(kRowRank | kRowGatherTie);
  if (x >= 0 && x < a.V) {
    const uint32_t code = a.dlog[(b * a.k + i) * a.ld + x];
    const int32_t key = (int32_t)key_of_code16(code);
    if (key >= st.klo) {
      if (key >= st.glo && key <= st.ghi) {
        const int64_t drawn = *(reinterpret_cast<const int64_t*>(ws + a.x_off) + b);
        if (st.rstar >= st.gcount) {
          pg = val16<SDX_BF16>(st, stb, code, a.T);
        } else if (st.rstar > 0) {  // partial group: kept if drawn, else ranked by the chain
          st.flags |= kRowGatherTie;
          if (x == drawn) pg = val16<SDX_BF16>(st, stb, code, a.T);
          else st.flags |= kRowRank;
        }
      } else {
        pg = val16<SDX_BF16>(st, stb, code, a.T);
      }
    }
  }
  st.pgather = pg;
  *dst = st;
}

hipError_t launch_draft_gather(const DraftGatherArgs& a, hipStream_t s) {
  if (a.k < 1 || a.k > kMaxDraftK || a.B < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(draft_gather_kernel, dim3((unsigned)a.B, (unsigned)a.k), dim3(256), 0, s, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------- round commit
// One thread per batch row. Row b drafted k_b tokens (k, or cu_k[b+1] - cu_k[b]),
// accepted n_acc[b] and drew y[b]. Both caches drop k_b - n_acc[b] positions
// (engine.py:310-312). Unless the row is done, its accepted drafts and then y
// are appended to out[b, len..] while they fit: a token equal to an EOS id, or
// the row reaching max_new tokens, marks it done and stops the row
// (engine.py:321-339). pending[b] = y[b] for every row (engine.py:340).
// Verify flags that leave a row's outcome unspecified.
constexpr uint32_t kCommitBadFlags =
    SDX_FLAG_NONFINITE | SDX_FLAG_UNSUPPORTED | SDX_FLAG_BAD_ROW | SDX_FLAG_WORKSPACE;

__global__ void round_commit_kernel(RoundCommitArgs a) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= a.B) return;
  int64_t kb, base;
  if (a.cu_k) {
    kb = a.cu_k[b + 1] - a.cu_k[b];
    base = a.cu_k[b];
  } else {
    kb = a.k;
    base = b * a.k;
  }
  // n_acc within [0, k_b], as the verify entry points produce it; the clamp
  // keeps the reads of draft_ids inside the row's k_b ids for any input.
  int64_t n = a.n_acc[b];
  n = n < 0 ? 0 : (n > kb ? kb : n);
  const int64_t drop = kb - n;
  if (a.len0) a.len0[b] -= drop;
  if (a.len1) a.len1[b] -= drop;
  int64_t yb = a.y[b];
  if (a.done[b]) {
    if (a.pending) a.pending[b] = yb;
    return;
  }
  // a live row the verify could not decide (its flags, or no token drawn) emits
  // nothing, ends, and raises the round's error word
  const uint32_t fl = a.flags ? (uint32_t)a.flags[b] : 0u;
  const uint32_t err = ((fl & kCommitBadFlags) ? 1u : 0u) | (yb < 0 ? 2u : 0u);
  if (err) {
    if (a.error) atomicOr(reinterpret_cast<uint32_t*>(a.error), err);
    if (a.pending) a.pending[b] = 0;
    a.done[b] = 1;
    return;
  }
  if (a.pending) a.pending[b] = yb;
  auto is_eos = [&](int64_t t) {
    for (int32_t i = 0; i < a.n_eos; ++i)
      if (a.eos[i] == t) return true;
    return false;
  };
  int64_t len = a.out_len[b];
  bool done = false;
  int64_t* out = a.out + b * a.max_new;
  for (int64_t j = 0; j < n; ++j) {
    const int64_t t = a.draft_ids[base + j];
    if (len < a.max_new) out[len] = t;
    ++len;
    if (is_eos(t) || len >= a.max_new) {
      done = true;
      break;
    }
  }
  if (!done) {
    if (len < a.max_new) out[len] = yb;
    ++len;
    done = is_eos(yb) || len >= a.max_new;
  }
  a.out_len[b] = len;
  a.done[b] = done ? 1 : 0;
}

hipError_t launch_round_commit(const RoundCommitArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(round_commit_kernel, dim3((unsigned)((a.B + 255) / 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------- controller
// EWMAAnalytic (controller.py:121-154) in float64, as the host controller
// computes it: every multiply and add rounded on its own (no fused
// multiply-add), so the state follows the host's arithmetic step for step. The expected speedup of k drafts at acceptance a and cost ratio c
// (controller.py:47-61) and its argmax over k in [1, k_max] (the smallest k on
// ties, as Python's max keeps the first).
__device__ double ctrl_speedup(int k, double alpha, double c, int extra_fwd) {
#pragma clang fp contract(off)
  const double tokens =
      alpha >= 1.0 - 1e-9 ? (double)(k + 1) : (1.0 - pow(alpha, (double)(k + 1))) / (1.0 - alpha);
  return tokens / ((double)(k + extra_fwd) * c + 1.0);
}
__device__ int ctrl_best_k(double alpha, double c, int k_max, int extra_fwd) {
  int best = 1;
  double bv = ctrl_speedup(1, alpha, c, extra_fwd);
  for (int k = 2; k <= k_max; ++k) {
    const double v = ctrl_speedup(k, alpha, c, extra_fwd);
    if (v > bv) {
      bv = v;
      best = k;
    }
  }
  return best;
}
// One state's update by this round's totals, then its k for the next round
// (controller.py:136-154: per-token decay beta^reached, EWMA of c, warmup).
__device__ int ctrl_step(CtrlState& st, int64_t acc, int64_t reached, const CtrlArgs& a,
                         double c_obs) {
#pragma clang fp contract(off)
  const double w = pow(a.beta, (double)reached);
  st.acc = w * st.acc + (double)acc;
  st.reached = w * st.reached + (double)reached;
  if (c_obs > 0.0) st.c = 0.9 * st.c + 0.1 * c_obs;
  st.rounds += 1;
  int k;
  if (st.rounds < a.warmup) {
    k = a.k_init;
  } else {
    double alpha = 0.7;
    if (st.reached > 0.0) alpha = fmin(0.999, fmax(0.0, st.acc / st.reached));
    k = ctrl_best_k(alpha, st.c, a.k_max, a.extra_fwd);
  }
  st.last_k = k;
  return k;
}

// Per batch (nstate == 1): one workgroup sums the round over all B rows
// (accepted = sum n_acc, reached = sum min(n_acc + 1, k), controller.py:145-146).
// Per row (nstate == B): row b's own state, its own k_b; cu_k (nullable) gets
// the exclusive prefix of the next k_b (the offsets of the next per-row-k verify).
__global__ void __launch_bounds__(256) controller_kernel(CtrlArgs a) {
  __shared__ int64_t s_red[2][256 / kWave];
  __shared__ int64_t s_carry;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const double c_obs = a.c_obs ? (double)a.c_obs[0] : 0.0;
  if (a.nstate == 1) {
    int64_t acc = 0, reached = 0;
    const int64_t k0 = a.k_used[0];
    for (int64_t b = tid; b < a.B; b += blockDim.x) {
      const int64_t n = a.n_acc[b];
      acc += n;
      reached += n + 1 < k0 ? n + 1 : k0;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      acc += __shfl_xor(acc, o, kWave);
      reached += __shfl_xor(reached, o, kWave);
    }
    if (lane == 0) {
      s_red[0][w] = acc;
      s_red[1][w] = reached;
    }
    __syncthreads();
    if (tid == 0) {
      int64_t ta = 0, tr = 0;
      for (int i = 0; i < (int)(blockDim.x / kWave); ++i) {
        ta += s_red[0][i];
        tr += s_red[1][i];
      }
      CtrlState st = a.state[0];
      const int k = ctrl_step(st, ta, tr, a, c_obs);
      a.state[0] = st;
      if (a.k_next) a.k_next[0] = k;
    }
    return;
  }
  // per row: rows in chunks of the block, a running prefix for cu_k
  if (tid == 0) s_carry = 0;
  __syncthreads();
  for (int64_t b0 = 0; b0 < a.B; b0 += blockDim.x) {
    const int64_t b = b0 + tid;
    int64_t k = 0;
    if (b < a.B) {
      CtrlState st = a.state[b];
      const int64_t n = a.n_acc[b];
      const int64_t kb = a.k_used[b];
      k = ctrl_step(st, n, n + 1 < kb ? n + 1 : kb, a, c_obs);
      a.state[b] = st;
      if (a.k_next) a.k_next[b] = k;
    }
    if (a.cu_k) {  // uniform
      int64_t incl = k;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const int64_t v = __shfl_up(incl, o, kWave);
        if (lane >= o) incl += v;
      }
      if (lane == kWave - 1) s_red[0][w] = incl;
      __syncthreads();
      int64_t off = s_carry, tot = 0;
      for (int i = 0; i < (int)(blockDim.x / kWave); ++i) {
        off += i < w ? s_red[0][i] : 0;
        tot += s_red[0][i];
      }
      if (b == 0) a.cu_k[0] = 0;
      if (b < a.B) a.cu_k[b + 1] = off + incl;
      __syncthreads();
      if (tid == 0) s_carry += tot;
      __syncthreads();
    }
  }
}

hipError_t launch_controller(const CtrlArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(controller_kernel, dim3(1), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace sdx
