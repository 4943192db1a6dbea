// Member rank of drafted tokens that fall inside their row's partial tie
// group (bf16 rows). Such a token is kept iff fewer than `rstar` group members
// (keys in [glo, ghi]) precede it in id order (specdec/sampling.py:56-64 keeps
// the first members of a tie in sort order, which is id order). The row
// kernel flags these rows (kRowRank); here each flagged row's prefix
// [0, gid) is split into RK_SEG segments, each counted by one block with
// 16-byte loads; a fixed grid of RK_GRID blocks reads the flags of all its
// (row, segment) items in one parallel pass and works only on flagged ones.
// Every segment adds (count << 32 | 1) to the row's 64-bit accumulator with
// one agent-scope atomic; the one that brings the tally to RK_SEG sets the
// row's pgather.
#include "sdx_launch.hpp"

namespace sdx {

constexpr int RK_NT = 256;
constexpr int RK_SEG = 16;     // segments per flagged row
constexpr int RK_GRID = 1024;  // blocks; each checks its (row, segment) items at once

__global__ void __launch_bounds__(RK_NT) rank_bf16_kernel(RowStatArgs a, int64_t rows) {
  __shared__ uint32_t red[RK_NT / kWave];
  __shared__ uint64_t s_flagged;
  const int64_t nitems = rows * RK_SEG;
  const int64_t per = (nitems + RK_GRID - 1) / RK_GRID;  // items of this block: b + i*GRID
  for (int64_t i0 = 0; i0 < per; i0 += kWave) {  // 64 items per parallel flag pass
  if (threadIdx.x < kWave) {
    bool f = false;
    const int64_t it = blockIdx.x + (i0 + threadIdx.x) * RK_GRID;
    if (i0 + threadIdx.x < per && it < nitems) f = (a.stats[it / RK_SEG].flags & kRowRank) != 0;
    const uint64_t m = __ballot(f);
    if (threadIdx.x == 0) s_flagged = m;
  }
  __syncthreads();
  uint64_t todo = s_flagged;
  __syncthreads();
  while (todo) {  // uniform
    const int i = __ffsll((unsigned long long)todo) - 1;
    todo &= todo - 1;
    const int64_t it = blockIdx.x + (i0 + i) * RK_GRID;
    const int64_t row = it / RK_SEG;
    const int s = (int)(it % RK_SEG);
    const RowStat st = a.stats[row];
    const int g = row < a.nrows[0] ? 0 : 1;
    const int64_t r = g ? row - a.nrows[0] : row;
    const uint16_t* __restrict__ ptr = a.base[g] + r * a.ld[g];
    // the row kernel flags only rows with a drafted token (gid >= 0)
    const int64_t gid = draft_id_of_row(a.ids, a.tgt_idx, a.k, a.nrows[1], g, r);
    const int64_t len = ((gid + RK_SEG - 1) / RK_SEG + 7) / 8 * 8;
    const int64_t x0 = min<int64_t>(gid, (int64_t)s * len), x1 = min<int64_t>(gid, x0 + len);
    const uint32_t glo = (uint32_t)st.glo, span = (uint32_t)(st.ghi - st.glo);
    uint32_t cnt = 0;
    for (int64_t e0 = x0 + (int64_t)threadIdx.x * 8; e0 < x1; e0 += (int64_t)RK_NT * 8) {
      if (e0 + 8 <= x1) {  // rows start 16-byte aligned; x0 is a multiple of 8
        const uint4 v = *reinterpret_cast<const uint4*>(ptr + e0);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const uint32_t k2 = keys2_of_codes2(w[t]);
          cnt += ((k2 & 0xFFFFu) - glo <= span ? 1u : 0u) + ((k2 >> 16) - glo <= span ? 1u : 0u);
        }
      } else {
        for (int64_t x = e0; x < x1; ++x) cnt += key_of_code16(ptr[x]) - glo <= span ? 1u : 0u;
      }
    }
    cnt = wave_sum_u32(cnt);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = cnt;
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t tot = 0;
      for (int w = 0; w < RK_NT / kWave; ++w) tot += red[w];
      const uint64_t prev = __hip_atomic_fetch_add(&a.rank_acc[row], ((uint64_t)tot << 32) | 1u,
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((uint32_t)prev == (uint32_t)(RK_SEG - 1)) {  // last segment: the full count is known
        const uint32_t rank = (uint32_t)(prev >> 32) + tot;
        float pg = 0.0f;
        if (gid >= 0 && rank < (uint32_t)st.rstar) {
          const float d = decode16<SDX_BF16>(ptr[gid]) / a.T - st.m;
          pg = exp_det(d) / st.zf / st.totf;
        }
        a.stats[row].pgather = pg;
      }
    }
    __syncthreads();
  }
  }
}

hipError_t launch_rank_bf16(const RowStatArgs& a, int64_t rows, hipStream_t s) {
  if (!a.ids || !a.rank_acc) return hipSuccess;  // nothing to rank without drafted tokens
  hipLaunchKernelGGL(rank_bf16_kernel, dim3(RK_GRID), dim3(RK_NT), 0, s, a, rows);
  return hipGetLastError();
}

}  // namespace sdx
