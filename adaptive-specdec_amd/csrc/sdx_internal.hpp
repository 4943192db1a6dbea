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
  kRowProbs = 1u << 4        // final probabilities stored densely (fp32 path)
};

// 64 bytes per row.
struct RowStat {
  float m;          // max over s = fl32(x / T)
  float zf;         // rn32(sum fixed62(exp_det(s - m)))
  float totf;       // max(rn32(kept mass), 1e-12): the renormaliser
  float pgather;    // final probability of the row's gathered (draft) token
  int32_t kmax;     // largest key in the row
  int32_t klo;      // keys below klo are dropped (top-k / top-p)
  int32_t glo, ghi; // boundary tie group: keys in [glo, ghi] kept iff id <= cut
  int64_t cut;      // last kept id of the boundary group (-1: none kept)
  uint64_t mass;    // exact kept mass, fixed62
  uint32_t flags;   // RowFlag bits
  int32_t ntbl;     // table holds keys [kmax - ntbl + 1, kmax]
  int64_t argmax;   // greedy rows: first index of the maximum
};
static_assert(sizeof(RowStat) == 64, "RowStat layout");

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

// Final probability of a 16-bit-coded element under the row's statistics.
template <int FMT>
__device__ __forceinline__ float pfinal16(const RowStat& st, const float* tbl, int64_t idx,
                                          uint32_t code, float T) {
  if (st.flags & kRowGreedy) return idx == st.argmax ? 1.0f : 0.0f;
  const int32_t key = (int32_t)key_of_code16(code);
  if (key < st.klo) return 0.0f;
  if (key <= st.ghi && key >= st.glo && idx > st.cut) return 0.0f;
  const int32_t t = st.kmax - key;
  if (t < st.ntbl) return tbl[t];
  const float s = decode16<FMT>(code) / T;
  const float p = exp_det(s - st.m) / st.zf;
  return p / st.totf;
}

}  // namespace sdx
