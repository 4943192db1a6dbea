// The draft step in one launch, for bf16 rows (specdec/engine.py:246-258 and
// controller.py:184-187): the to_probs statistics of each batch row's one row,
// the draw x from q on the caller's uniform, and the step's epilogue (q(x),
// conf *= q(x), the early-exit flag) in the block that completes the draw.
//
// It is the fused verify kernel at k = 0 (sdx_rowstream.hip) with two changes
// that only pay at one row per batch row, kept in a translation unit of their
// own so that the verify kernel's code is not touched by them:
//   - draw blocks of SK_NT threads (SK_NW records each): with SM_NT-thread
//     draw blocks about half of them could not get a slot before the rows
//     were in (every block of the launch has the row blocks' LDS size);
//   - no separate epilogue launch: the block that completes a batch row's
//     draw writes qx, xcopy and conf of its row; the last row to count in on
//     a header word reads every conf, writes the early-exit flag and the
//     workspace signature, and resets the word.
#include "sdx_rowstream.hpp"

namespace sdx {

struct DraftFusedArgs {
  FusedArgs f;     // k = 0: row b is batch row b; the draw's y is x
  DraftEpiArgs e;  // the epilogue's outputs (e.x unused: x is f.d.y)
  uint32_t* done;  // header word: batch rows whose epilogue is written
};

// Wave 0 of the block that completed batch row j's draw. q(x) is the value the
// draw's final walk gave the drawn id (its final probability, a kept member of
// the boundary tie group carrying the group value): the epilogue kernel's
// value, read off the walk instead of the row's statistics and table. `conf0`
// is conf[j] as lane 0 loaded it before the draw. With a stop flag, lane 0
// counts the row in once its conf store is done; the wave of the last row
// loads every conf at once and lane 0 sums them in row order.
__device__ __forceinline__ void draft_epilogue_row(const DraftFusedArgs& a, int64_t j, float qfound,
                                                   float conf0) {
  const DraftEpiArgs& e = a.e;
  const int lane = threadIdx.x & (kWave - 1);
  uint32_t prev = 0;
  if (lane == 0) {
    const int64_t x = a.f.d.y[j];  // written by this thread
    const float p = x >= 0 && x < e.V ? qfound : 0.0f;
    if (e.stop) {
      if (e.conf)
        __hip_atomic_store(reinterpret_cast<uint32_t*>(e.conf + j), __float_as_uint(conf0 * p),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // the conf store is done before this row counts in (the last row reads it)
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // gfx9 encoding: vmcnt(0)
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      prev = __hip_atomic_fetch_add(a.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (e.conf) {
      e.conf[j] = conf0 * p;
    }
    if (e.qx) e.qx[j] = p;
    if (e.xcopy) e.xcopy[j] = x;
    if (e.sig) {  // every row writes the same words
      const uint32_t w[kDraftSigWords] = {kDraftSig, (uint32_t)e.B, (uint32_t)e.V,
                                          __float_as_uint(e.T), __float_as_uint(e.top_p),
                                          (uint32_t)e.top_k};
      for (int i = 0; i < kDraftSigWords; ++i) e.sig[i] = w[i];
    }
  }
  if (!e.stop) return;
  prev = (uint32_t)__builtin_amdgcn_readfirstlane((int)prev);
  if (prev != (uint32_t)(e.B - 1)) return;  // wave-uniform: not the last row
  if (lane == 0) __hip_atomic_store(a.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  int32_t stop = 0;
  if (e.conf && e.step >= e.min_k) {
    float s = 0.0f;  // sequential in row order, as the epilogue kernel sums
    for (int64_t b0 = 0; b0 < e.B; b0 += kWave) {
      const int64_t b = b0 + lane;
      const float c = b < e.B ? __uint_as_float(__hip_atomic_load(
                                    reinterpret_cast<const uint32_t*>(e.conf + b),
                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
                              : 0.0f;
      const int n = (int)min<int64_t>(kWave, e.B - b0);
      for (int l = 0; l < n; ++l)
        s = s + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(c), l));
    }
    stop = (s / (float)e.B) < e.tau ? 1 : 0;
  }
  if (lane == 0) e.stop[0] = stop;
}

// Thread 0 of a draw block whose wait for its row gave up: the row's outputs
// are those of a draw that picked nothing (x -1, q(x) 0) and the draft loop is
// told to stop. The header's magic word, which the wait overwrote, keeps a
// verify from taking these statistics over. No row of such a launch counts in
// on `done`, so no block writes the flag from the confidences.
__device__ __forceinline__ void draft_give_up_row(const DraftFusedArgs& a, int64_t j) {
  const DraftEpiArgs& e = a.e;
  a.f.d.y[j] = -1;
  if (e.qx) e.qx[j] = 0.0f;
  if (e.xcopy) e.xcopy[j] = -1;
  if (e.conf) e.conf[j] = e.conf[j] * 0.0f;
  if (e.stop) e.stop[0] = 1;
}

__global__ void __launch_bounds__(SK_NT) __attribute__((amdgpu_waves_per_eu(6)))
draft_fused_bf16_kernel(DraftFusedArgs a) {
  __shared__ union DraftLds {
    SkLds row;
    Draw16LdsT<SK_NW> draw;
  } U;
  const FusedArgs& f = a.f;
  const int64_t blk = blockIdx.x;
  if (blk < f.nrow_pad) {
    if (blk >= f.nrow) return;
    const int64_t row = rowstream_body<true>(f.rs, U.row, blk);
    if (row < 0) return;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // gfx9 encoding: vmcnt(0) (the row's stores done)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (threadIdx.x == 0)  // k = 0: row b is batch row b's only row
      __hip_atomic_fetch_add(&f.d.job_cnt[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  const int64_t t = blk - f.nrow_pad;
  int64_t j;
  int bi;
  if (f.d.xcd) {  // a batch row's blocks on one XCD
    const int64_t i = t >> 3;
    j = (t & 7) + 8 * (i / f.d.nblk);
    bi = (int)(i % f.d.nblk);
  } else {
    j = t / f.d.nblk;
    bi = (int)(t % f.d.nblk);
  }
  if (threadIdx.x == 0) {
    int ok = 0;
    if (__hip_atomic_load(f.rs.ws_header, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == kWsMagic) {
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      for (;;) {
        if (__hip_atomic_load(&f.d.job_cnt[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= 1u) {
          ok = 1;
          break;
        }
        if (__builtin_amdgcn_s_memrealtime() - t0 > f.wait_ticks) {
          __hip_atomic_store(f.rs.ws_header, kWsDirty, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    U.draw.last = ok;
  }
  __syncthreads();
  if (!U.draw.last) {
    if (threadIdx.x == 0) draft_give_up_row(a, j);
    return;
  }
  // conf[j] (written before this launch) loaded ahead of the draw, for the
  // block that completes it
  const float conf0 = threadIdx.x == 0 && a.e.conf ? a.e.conf[j] : 0.0f;
  draw16_body<SDX_BF16, true, SK_NT, kRec16Rounds, true, true>(f.d, U.draw, j, bi);
  // draw16_body leaves `last` set in the one block that completed the row's draw
  if (threadIdx.x < kWave && U.draw.last)
    draft_epilogue_row(a, j, __uint_as_float(U.draw.s32w[0]), conf0);
}

hipError_t launch_draft_fused_bf16(const RowStatArgs& rs, const RowSource16& src,
                                   const AcceptArgs& acc, int64_t batch, int64_t V, float T,
                                   ChunkRec* recs, uint32_t* counters, uint32_t* job_cnt,
                                   int64_t* x, const DraftEpiArgs& e, uint32_t* done,
                                   hipStream_t s) {
  if (!src.vec || !x || !job_cnt || !done || !rs.ws_header || V % 8 != 0 || rs.k != 0 ||
      rs.nrows[1] != 0 || acc.cu_k || acc.k != 0 || e.B != batch)
    return hipErrorInvalidValue;
  DraftFusedArgs a = {};
  FusedArgs& f = a.f;
  f.rs = rs;
  f.rs.jm_k = 0;
  f.rs.jm_order = nullptr;
  f.rowjob = nullptr;
  f.rs.zero = nullptr;  // the draw counters reset themselves
  f.rs.nzero = 0;
  f.nrow = rowstream_setup(f.rs, batch);
  f.nrow_pad = (f.nrow + 7) / 8 * 8;
  Draw16Args<SDX_BF16>& d = f.d;
  d.acc = acc;
  d.ev = Eval16<SDX_BF16>{src.base, src.ld, src.base2, src.ld2, src.split, rs.stats, rs.tables, T};
  d.V = V;
  d.nrec = (int32_t)((V + kRec16 - 1) / kRec16);
  if (d.nrec > kMaxRec16) return hipErrorInvalidValue;
  d.nblk = (d.nrec + SK_NW - 1) / SK_NW;
  d.xcd = batch % 8 == 0 ? 1 : 0;
  d.recs = recs;
  d.counters = counters;
  d.job_cnt = job_cnt;
  d.y = x;
  f.need = 1;
  f.wait_ticks = fused_wait_ticks();
  a.e = e;
  a.done = done;
  const int64_t grid = f.nrow_pad + batch * d.nblk;
  hipLaunchKernelGGL(draft_fused_bf16_kernel, dim3((unsigned)grid), dim3(SK_NT), 0, s, a);
  return hipGetLastError();
}

}  // namespace sdx
