// Internal layout shared by the kernels and the C-ABI launch code.
//
// A "row" is one [vocab] logit vector (one target or draft position). The
// row-statistics kernel reduces it to a RowStat record plus a short table of
// final probabilities for the keys at the top of the row; every later stage
// (accept test, residual/bonus sampling, to_probs output) evaluates the final
// probability of any element from (record, table, element code, element id)
// without touching the rest of the row.
#pragma once

#include "sdx_common.hpp"

namespace sdx {

constexpr int kTbl = 2048;  // table entries per row (keys kmax, kmax-1, ...)

enum RowFlag : uint32_t {
  kRowGreedy = 1u << 0,      // temperature <= 0: one-hot at `argmax`
  kRowNonfinite = 1u << 1,   // +inf / +NaN in the row (results unspecified)
  kRowUnsupported = 1u << 2, // decision fell outside the histogram window
  kRowBelowWindow = 1u << 3, // elements below the histogram window carry mass
  kRowProbs = 1u << 4,       // final probabilities stored densely (fp32 path)
  kRowRank = 1u << 5,        // drafted token inside the partial tie group: pgather is
                             // set by the rank kernel from its member rank
  kRowBadWs = 1u << 6,       // split row whose workspace header was not initialised
                             // (sdx_workspace_init): statistics not computed
  kRowGatherTie = 1u << 7    // the gathered (drafted) token is a member of the row's
                             // partially kept boundary tie group
};

// 64 bytes per row. Keys in [glo, ghi] form the tie group that straddles the
// nucleus boundary: its first `rstar` members in id order are kept, the
// other gcount - rstar are dropped. Consumers count members as they stream.
struct RowStat {
  float m;          // max over s = fl32(x / T)
  float zf;         // rn32(sum fixed62(exp_det(s - m)))
  float totf;       // max(rn32(kept mass), 1e-12): the renormaliser
  float pgather;    // final probability of the row's gathered (draft) token
  int32_t kmax;     // largest key in the row
  int32_t klo;      // keys below klo are dropped (top-k / top-p)
  int32_t glo, ghi; // boundary tie group key range (empty when glo > ghi)
  int32_t rstar;    // group members kept, lowest ids first
  int32_t gcount;   // group members in the row
  uint64_t mass;    // exact kept mass, fixed62
  uint32_t flags;   // RowFlag bits
  int32_t ntbl;     // table holds keys [kmax - ntbl + 1, kmax]
  int64_t argmax;   // greedy rows: first index of the maximum
};
static_assert(sizeof(RowStat) == 64, "RowStat layout");

// Number of tie-group members (keys in [glo, ghi]) among ids [0, end) of a
// 16-bit row, counted by the whole block (blockDim a multiple of 64; `red`
// holds blockDim/64 + 1 words of LDS). Used to rank a drafted token that sits
// inside its row's boundary group.
__device__ inline uint32_t block_count_members(const uint16_t* ptr, int64_t end, int32_t glo,
                                               int32_t ghi, uint32_t* red) {
  uint32_t cnt = 0;
  for (int64_t i = threadIdx.x; i < end; i += blockDim.x) {
    const int32_t k2 = (int32_t)key_of_code16(ptr[i]);
    cnt += (k2 >= glo && k2 <= ghi) ? 1u : 0u;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) cnt += (uint32_t)__shfl_xor((int)cnt, o, kWave);
  const int nw = blockDim.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = cnt;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
    for (int w = 0; w < nw; ++w) t += red[w];
    red[nw] = t;
  }
  __syncthreads();
  const uint32_t total = red[nw];
  __syncthreads();
  return total;
}

// Class of an element under its row's statistics: 0 dropped, 1 member of the
// boundary tie group (kept iff its member rank < rstar), 2 kept.
__device__ __forceinline__ int cls16(const RowStat& st, int32_t key) {
  if (key < st.klo) return 0;
  return (key >= st.glo && key <= st.ghi) ? 1 : 2;
}
// Final probability of a key below the table (out of line, so the compiler
// cannot if-convert the fp64 exp into every table lookup).
template <int FMT>
__device__ __forceinline__ float val16_exp_inl(uint32_t code, float T, float m, float zf,
                                               float totf) {
  const float s = decode16<FMT>(code) / T;
  const float p = exp_det(s - m) / zf;
  return p / totf;
}
template <int FMT>
__device__ __noinline__ float val16_exp(uint32_t code, float T, float m, float zf, float totf) {
  return val16_exp_inl<FMT>(code, T, m, zf, totf);
}
// Final probability of a kept (class 2) or kept-member element.
template <int FMT>
__device__ __forceinline__ float val16(const RowStat& st, const float* tbl, uint32_t code,
                                       float T) {
  const int32_t t = st.kmax - (int32_t)key_of_code16(code);
  if (t < st.ntbl) return tbl[t];
  return val16_exp<FMT>(code, T, st.m, st.zf, st.totf);
}

// Where rows live: rows [0, split) at base + row*ld, the rest at
// base2 + (row - split)*ld2 (target then draft rows; p then q rows).
struct RowSource16 {
  const uint16_t* base;
  int64_t ld;
  const uint16_t* base2;
  int64_t ld2;
  int64_t split;
  bool vec;  // every row start is 16-byte aligned
};
struct RowSourceF32 {
  const float* base;
  int64_t ld;
  const float* base2;
  int64_t ld2;
  int64_t split;
  bool vec;
};

}  // namespace sdx
