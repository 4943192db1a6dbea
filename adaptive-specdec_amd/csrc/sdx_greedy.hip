// Greedy paths: row argmax (vllm_draft_spec/proposer.py:262-263,331-332 and the
// T = 0 one-hot of specdec/sampling.py:43-48) and the greedy verify that
// follows from it (specdec/engine.py:285-303 with one-hot p).
//
// A row is scanned with 16-byte loads; each lane keeps the best
// (key, first index) pair packed as (key << 32) | ~index so one max reduction
// gives the largest value and, among equal values, the lowest index. -0 is
// folded onto +0 so equal values compare equal, as torch.argmax does.
#include "sdx_launch.hpp"

namespace sdx {

constexpr int AM_NT = 512;
typedef unsigned short am_us2 __attribute__((ext_vector_type(2)));

template <int DT>
__device__ __forceinline__ uint64_t pack_best(uint32_t key, int64_t idx) {
  return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)idx);
}

template <int DT>
__global__ void __launch_bounds__(AM_NT) argmax_kernel(const void* data, int64_t V, int64_t ld,
                                                       bool vec, int64_t* out) {
  __shared__ uint64_t red[AM_NT / kWave];
  const int64_t row = blockIdx.x;
  uint64_t best = 0;
  if constexpr (DT == SDX_F32) {
    const float* p = static_cast<const float*>(data) + row * ld;
    for (int64_t i0 = (int64_t)threadIdx.x * 4; i0 < V; i0 += (int64_t)AM_NT * 4) {
      float x[4];
      if (vec && i0 + 4 <= V) {
        const float4 v = *reinterpret_cast<const float4*>(p + i0);
        x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
      } else {
        for (int t = 0; t < 4; ++t) x[t] = i0 + t < V ? p[i0 + t] : -INFINITY;
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (i0 + t < V) {
          uint32_t k = key_of_f32(x[t]);
          if (k == 0x7FFFFFFFu) k = 0x80000000u;  // -0 == +0
          const uint64_t c = pack_best<DT>(k, i0 + t);
          best = c > best ? c : best;
        }
      }
    }
  } else if (vec && V / ((int64_t)AM_NT * 8) < 0xFFF0) {
    // Whole 8-element chunks with packed 16-bit work: both keys of a word at
    // once (-0 folded onto +0), and per element slot e of the chunk a running
    // best (key << 16) | (0xFFFF - round), whose max keeps the largest key and,
    // among equal keys, the earliest round. Four rounds of loads in flight; the
    // last V % 8 elements go through the per-element form below.
    const uint16_t* p = static_cast<const uint16_t*>(data) + row * ld;
    constexpr int64_t kStep = (int64_t)AM_NT * 8;  // ids per block round
    const int64_t nround = (V + kStep - 1) / kStep;
    uint32_t bk[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) bk[e] = 0u;
    for (int64_t r0 = 0; r0 < nround; r0 += 4) {
      uint4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t i0 = (r0 + u) * kStep + (int64_t)threadIdx.x * 8;
        // past the whole chunks: all-ones codes (key 0, later rounds lose ties)
        v[u] = i0 + 8 <= V ? *reinterpret_cast<const uint4*>(p + i0)
                           : make_uint4(0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t inv = 0xFFFFu - (uint32_t)(r0 + u);
        const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          uint32_t k2 = keys2_of_codes2(w[t]);
          // -0 (key 0x7FFF) -> +0 (0x8000): add 1 to exactly those halves
          const uint32_t x = k2 ^ 0x7FFF7FFFu;
          const uint32_t nz = __builtin_bit_cast(
              uint32_t, __builtin_elementwise_min(__builtin_bit_cast(am_us2, x), (am_us2){1, 1}));
          k2 += 0x00010001u - nz;
          bk[2 * t] = max(bk[2 * t], (k2 << 16) | inv);
          bk[2 * t + 1] = max(bk[2 * t + 1], (k2 & 0xFFFF0000u) | inv);
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (bk[e] != 0u) {
        const int64_t rr = (int64_t)(0xFFFFu - (bk[e] & 0xFFFFu));
        const uint64_t c = pack_best<DT>(bk[e] >> 16, rr * kStep + (int64_t)threadIdx.x * 8 + e);
        best = c > best ? c : best;
      }
    }
    for (int64_t i = V / 8 * 8 + threadIdx.x; i < V; i += AM_NT) {  // the last V % 8
      uint32_t k = key_of_code16(p[i]);
      if (k == 0x7FFFu) k = 0x8000u;  // -0 == +0
      const uint64_t c = pack_best<DT>(k, i);
      best = c > best ? c : best;
    }
  } else {
    const uint16_t* p = static_cast<const uint16_t*>(data) + row * ld;
    for (int64_t i0 = (int64_t)threadIdx.x * 8; i0 < V; i0 += (int64_t)AM_NT * 8) {
      uint32_t w[4];
      if (vec && i0 + 8 <= V) {
        const uint4 v = *reinterpret_cast<const uint4*>(p + i0);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
      } else {
        for (int t = 0; t < 4; ++t) {
          const uint32_t c0 = i0 + 2 * t < V ? p[i0 + 2 * t] : 0xFFFFu;
          const uint32_t c1 = i0 + 2 * t + 1 < V ? p[i0 + 2 * t + 1] : 0xFFFFu;
          w[t] = c0 | (c1 << 16);
        }
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        if (i0 + t < V) {
          const uint32_t code = (t & 1) ? (w[t >> 1] >> 16) : (w[t >> 1] & 0xFFFFu);
          uint32_t k = key_of_code16(code);
          if (k == 0x7FFFu) k = 0x8000u;  // -0 == +0
          const uint64_t c = pack_best<DT>(k, i0 + t);
          best = c > best ? c : best;
        }
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t v = (uint64_t)__shfl_xor((long long)best, o, kWave);
    best = v > best ? v : best;
  }
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = 0;
    for (int w = 0; w < AM_NT / kWave; ++w) b = red[w] > b ? red[w] : b;
    out[row] = (int64_t)(0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFu));
  }
}

// Greedy accept: argmax of target rows [batch, k+1] already in `am`. With
// per-row k (cu_k non-null) row b has k_b = cu_k[b+1] - cu_k[b] positions, its
// target rows start at cu_k[b] + b and its drafted ids / uniforms at cu_k[b];
// bad[b] marks a row whose offsets failed the check (n_acc 0, y -1, flag set).
__global__ void greedy_accept_kernel(const int64_t* am, int64_t batch, int32_t k,
                                     const int64_t* ids, const float* u_accept,
                                     const uint8_t* active, int64_t* n_acc, int64_t* y,
                                     uint8_t* flags, const int64_t* cu_k, const uint8_t* bad) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  int64_t t0 = b * (k + 1), i0 = b * k;
  if (cu_k) {
    if (bad[b]) {
      n_acc[b] = 0;
      y[b] = -1;
      flags[b] = (uint8_t)SDX_FLAG_BAD_ROW;
      return;
    }
    i0 = cu_k[b];
    t0 = i0 + b;
    k = (int32_t)(cu_k[b + 1] - i0);
  }
  bool alive = active ? active[b] != 0 : true;
  int n = 0;
  uint32_t fl = 0;
  for (int i = 0; i < k; ++i) {
    // p is one-hot at the argmax, q(x) = 1: ratio = p(x) in {0, 1}
    const float r1 = ids[i0 + i] == am[t0 + i] ? 1.0f : 0.0f;
    const float u = u_accept ? u_accept[i0 + i] : 0.0f;
    const bool evaluated = alive && n == i;
    const bool ok = evaluated && (u < r1);
    if (evaluated && fabsf(u - r1) < 1e-5f) fl |= SDX_FLAG_ACCEPT_NEAR_TIE;
    n += ok ? 1 : 0;
    alive = alive && ok;
  }
  n_acc[b] = n;
  y[b] = am[t0 + n];
  flags[b] = (uint8_t)fl;
}

// Greedy to_probs output: one-hot at the row argmax (sampling.py:46-48).
__global__ void onehot_kernel(const int64_t* am, int64_t V, int64_t per_row, float* out,
                              int64_t ld_out) {
  const int64_t row = (int64_t)blockIdx.x / per_row;
  const int64_t i = ((int64_t)blockIdx.x % per_row) * blockDim.x + threadIdx.x;
  if (i < V) out[row * ld_out + i] = i == am[row] ? 1.0f : 0.0f;
}

hipError_t launch_onehot(const int64_t* am, int64_t rows, int64_t V, float* out, int64_t ld_out,
                         hipStream_t s) {
  const int nt = 256;
  const int64_t per_row = (V + nt - 1) / nt;
  hipLaunchKernelGGL(onehot_kernel, dim3((unsigned)(per_row * rows)), dim3(nt), 0, s, am, V,
                     per_row, out, ld_out);
  return hipGetLastError();
}

hipError_t launch_argmax(int dtype, const void* data, int64_t rows, int64_t V, int64_t ld,
                         bool vec, int64_t* out, hipStream_t s) {
  const dim3 grid((unsigned)rows), block(AM_NT);
  if (dtype == SDX_F32)
    hipLaunchKernelGGL((argmax_kernel<SDX_F32>), grid, block, 0, s, data, V, ld, vec, out);
  else if (dtype == SDX_BF16)
    hipLaunchKernelGGL((argmax_kernel<SDX_BF16>), grid, block, 0, s, data, V, ld, vec, out);
  else
    hipLaunchKernelGGL((argmax_kernel<SDX_F16>), grid, block, 0, s, data, V, ld, vec, out);
  return hipGetLastError();
}

hipError_t launch_greedy_accept(const int64_t* am, int64_t batch, int32_t k, const int64_t* ids,
                                const float* u_accept, const uint8_t* active, int64_t* n_acc,
                                int64_t* y, uint8_t* flags, hipStream_t s, const int64_t* cu_k,
                                const uint8_t* bad) {
  const int nt = 128;
  hipLaunchKernelGGL(greedy_accept_kernel, dim3((unsigned)((batch + nt - 1) / nt)), dim3(nt), 0,
                     s, am, batch, k, ids, u_accept, active, n_acc, y, flags, cu_k, bad);
  return hipGetLastError();
}

// Per-row k: one workgroup checks cu_k (cu_k[0] = 0, cu_k[batch] = ndrf, non-
// decreasing, every k_b <= k_max) and maps each target row to the drafted id
// it gathers. Inconsistent offsets mark every row bad: rows then overlap, so
// none of their row sets can be trusted. With `order` / `rowjob` (the fused
// verify kernel) it also lists the rows in batch-row order (batch row b's
// k_b + 1 target rows then its k_b draft rows, from q = 2 cu_k[b] + b) and gives
// each row its batch row; bad offsets: the identity order and no batch row (-1).
__global__ void __launch_bounds__(1024) ragged_rows_kernel(const int64_t* cu_k, int64_t batch,
                                                          int32_t k_max, int64_t ntgt,
                                                          int64_t ndrf, int64_t* tgt_idx,
                                                          uint8_t* bad, int32_t* order,
                                                          int32_t* rowjob) {
  int ok = cu_k[0] == 0 && cu_k[batch] == ndrf && ndrf + batch == ntgt;
  for (int64_t b = threadIdx.x; b < batch; b += blockDim.x) {
    const int64_t kb = cu_k[b + 1] - cu_k[b];
    ok &= kb >= 0 && kb <= k_max;
  }
  ok = __syncthreads_and(ok);
  if (!ok && order) {
    for (int64_t q = threadIdx.x; q < ntgt + ndrf; q += blockDim.x) {
      order[q] = (int32_t)q;
      rowjob[q] = -1;
    }
  }
  for (int64_t b = threadIdx.x; b < batch; b += blockDim.x) {
    bad[b] = ok ? 0 : 1;
    if (!ok) continue;
    const int64_t c0 = cu_k[b], kb = cu_k[b + 1] - c0;
    for (int64_t i = 0; i <= kb; ++i) tgt_idx[c0 + b + i] = i < kb ? c0 + i : -1;
    if (order) {
      const int64_t q0 = 2 * c0 + b;
      for (int64_t i = 0; i <= kb; ++i) {
        order[q0 + i] = (int32_t)(c0 + b + i);
        rowjob[c0 + b + i] = (int32_t)b;
      }
      for (int64_t i = 0; i < kb; ++i) {
        order[q0 + kb + 1 + i] = (int32_t)(ntgt + c0 + i);
        rowjob[ntgt + c0 + i] = (int32_t)b;
      }
    }
  }
}

hipError_t launch_ragged_rows(const int64_t* cu_k, int64_t batch, int32_t k_max, int64_t ntgt,
                              int64_t ndrf, int64_t* tgt_idx, uint8_t* bad, hipStream_t s,
                              int32_t* order, int32_t* rowjob) {
  hipLaunchKernelGGL(ragged_rows_kernel, dim3(1), dim3(1024), 0, s, cu_k, batch, k_max, ntgt, ndrf,
                     tgt_idx, bad, order, rowjob);
  return hipGetLastError();
}

}  // namespace sdx
