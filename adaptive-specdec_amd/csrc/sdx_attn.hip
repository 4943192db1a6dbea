// Multi-query verify attention over paged KV, on MFMA: the attention of the
// target's verify forward (the k+1 new positions of every batch row against
// the row's cached keys, bench/bench_engine.py:170-174 through
// specdec/engine.py:273-275), with the additive mask of
// specdec/kvcache.py:138-162 (query j of row b sees key s iff
// s <= lengths[b] + j) and grouped-query heads (query head h reads KV head
// h / group, the repeat_kv of the HF Qwen3 attention).
//
// One workgroup per (batch row, KV head), rows taken in the caller's order
// (longest context first balances the tail): its query rows are the q_b
// positions x group heads that share the KV head (q_b * group <= 64, padded to
// 16-row MFMA tiles; wave w owns rows 16w .. 16w + 15). The row's keys stream
// through LDS in tiles of 32 tokens gathered through the block table (each
// token's head slice is 256 contiguous bytes of its page), the next tile
// prefetched into registers while the current one is used:
//   S = Q K^T       16 x 32 per wave: 2 x 8 v_mfma_f32_16x16x16_bf16
//   online softmax  per row in fp32 (max and sum across the 16-lane rows)
//   O += P V        16 x 128 per wave: 8 x 2 MFMAs, P rounded to bf16
// Q operands stay in registers; V is stored transposed in LDS so both MFMA
// operands of P V are 8-byte reads.
// The kernel is bound by the KV bytes it streams (about 22 flop per byte),
// not by MFMA.
#include "sdx_launch.hpp"

namespace sdx {

constexpr int VA_NT = 256;
constexpr int VA_NW = VA_NT / kWave;
constexpr int VA_D = 128;     // head dim
constexpr int VA_TOK = 32;    // tokens per tile
constexpr int VA_MAXM = 64;   // query rows per workgroup (q_b * group)
constexpr int VA_KS = VA_D + 8;    // LDS row strides (bf16 elements), padded against
                                   // bank conflicts of the 16-row operand reads
constexpr int VA_VS = VA_TOK + 8;
constexpr int VA_PS = VA_TOK + 8;

typedef short va_s4 __attribute__((ext_vector_type(4)));
typedef float va_f4 __attribute__((ext_vector_type(4)));


__device__ __forceinline__ uint16_t va_bf16(float x) {  // round to nearest even
  const uint32_t u = __float_as_uint(x);
  if ((u & 0x7F800000u) == 0x7F800000u) return (uint16_t)((u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u));
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
// max / sum over the 16 lanes of a DPP row (lanes sharing lane / 16): rotations
// of the row by 1, 2, 4 and 8 lanes leave every lane with the row's result
template <int R>
__device__ __forceinline__ float va_ror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + R, 0xF, 0xF,
                                                    false));
}
__device__ __forceinline__ float va_rowmax16(float v) {
  v = fmaxf(v, va_ror<1>(v));
  v = fmaxf(v, va_ror<2>(v));
  v = fmaxf(v, va_ror<4>(v));
  return fmaxf(v, va_ror<8>(v));
}
__device__ __forceinline__ float va_rowsum16(float v) {
  v += va_ror<1>(v);
  v += va_ror<2>(v);
  v += va_ror<4>(v);
  return v + va_ror<8>(v);
}

__global__ void __launch_bounds__(VA_NT) __attribute__((amdgpu_waves_per_eu(3)))
verify_attn_kernel(AttnArgs a) {
  __shared__ uint16_t sK[VA_TOK][VA_KS];
  __shared__ uint16_t sVt[VA_D][VA_VS];
  __shared__ uint16_t sP[VA_NW][16][VA_PS];

  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int64_t b = a.row_order ? (int64_t)a.row_order[blockIdx.x / a.hkv] : blockIdx.x / a.hkv;
  const int kvh = (int)(blockIdx.x % a.hkv);
  if (b < 0 || b >= a.batch) {  // uniform: a row order outside [0, batch)
    if (tid == 0 && a.error) *a.error = 1;
    return;
  }
  const int64_t q0 = a.cu_q[b], qb = a.cu_q[b + 1] - q0;
  const int64_t kvl = a.kv_len[b], base = kvl - qb;
  if (qb < 0 || qb > a.max_q || base < 0 ||
      (kvl + a.bs - 1) / a.bs > a.max_blocks) {  // uniform: a row the launch cannot serve
    if (tid == 0 && a.error) *a.error = 1;
    return;
  }
  const int M = (int)qb * a.group;
  const int64_t rowB = (int64_t)a.hkv * VA_D * 2;  // bytes per token of a page row

  // ---- tile loads: thread t moves 16 bytes (8 dims) of tokens t / 16 and 16 + t / 16
  const int ltok = tid / 16, lpart = tid % 16;
  const int32_t* bt = a.block_table + b * a.max_blocks;
  int bad = 0;
  auto gather = [&](int64_t t0, uint4 (&kv)[4]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t pos = t0 + ltok + 16 * h;
      kv[2 * h] = make_uint4(0, 0, 0, 0);
      kv[2 * h + 1] = make_uint4(0, 0, 0, 0);
      if (pos < kvl) {
        const int32_t page = bt[pos / a.bs];
        if (page >= 0 && page < a.num_blocks) {
          const int64_t off = (((int64_t)page * a.bs + pos % a.bs) * rowB + kvh * (VA_D * 2) +
                               lpart * 16) / 2;
          kv[2 * h] = *reinterpret_cast<const uint4*>(a.k_pool + off);
          kv[2 * h + 1] = *reinterpret_cast<const uint4*>(a.v_pool + off);
        } else {
          bad = 1;
        }
      }
    }
  };
  auto stage = [&](const uint4 (&kv)[4]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int tok = ltok + 16 * h;
      *reinterpret_cast<uint4*>(&sK[tok][lpart * 8]) = kv[2 * h];
      const uint32_t vw[4] = {kv[2 * h + 1].x, kv[2 * h + 1].y, kv[2 * h + 1].z,
                              kv[2 * h + 1].w};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        sVt[lpart * 8 + e][tok] = (uint16_t)((e & 1) ? (vw[e >> 1] >> 16) : (vw[e >> 1] & 0xFFFFu));
    }
  };

  // ---- per-wave state: rows r0 + 4 * (lane / 16) + r, r < 4
  const int r0 = 16 * w;
  const bool active = r0 < M;  // uniform per wave
  const int lr = 4 * (lane / 16), lc = lane % 16;
  va_f4 o[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) o[n] = (va_f4){0.0f, 0.0f, 0.0f, 0.0f};
  float m_run[4], l_run[4];
  int64_t lim[4];  // last visible key of the lane's rows (-1: padding row)
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m_run[r] = -INFINITY;
    l_run[r] = 0.0f;
    const int i = r0 + lr + r;
    lim[r] = i < M ? base + i / a.group : -1;
  }

  // the wave's query operands, in registers: lane holds row r0 + lc, dims
  // 16 kc + lr .. + 3 (row i = j * group + g is head kvh * group + g of position j)
  va_s4 qa[VA_D / 16];
  {
    const int i = r0 + lc;
    const bool has = active && i < M;
    const uint16_t* src = a.q + (has ? ((q0 + i / a.group) * a.hq + kvh * a.group + i % a.group) * VA_D
                                     : 0);
#pragma unroll
    for (int kc = 0; kc < VA_D / 16; ++kc)
      qa[kc] = has ? *reinterpret_cast<const va_s4*>(src + kc * 16 + lr) : (va_s4){0, 0, 0, 0};
  }

  uint4 kv[4];
  gather(0, kv);
  for (int64_t t0 = 0; t0 < kvl; t0 += VA_TOK) {
    stage(kv);
    __syncthreads();
    if (t0 + VA_TOK < kvl) gather(t0 + VA_TOK, kv);  // next tile in flight meanwhile
    if (active) {
      // S = Q K^T for the wave's 16 rows x 32 tokens
      va_f4 s[2];
#pragma unroll
      for (int n = 0; n < 2; ++n) s[n] = (va_f4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kc = 0; kc < VA_D / 16; ++kc) {
#pragma unroll
        for (int n = 0; n < 2; ++n) {
          const va_s4 kb = *reinterpret_cast<const va_s4*>(&sK[n * 16 + lc][kc * 16 + lr]);
          s[n] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(qa[kc], kb, s[n], 0, 0, 0);
        }
      }
      // online softmax in base 2; s[n][r] is row lr + r, token t0 + 16 n + lc
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float x[2];
#pragma unroll
        for (int n = 0; n < 2; ++n) {
          const int64_t pos = t0 + 16 * n + lc;
          x[n] = pos <= lim[r] ? s[n][r] * a.scale_log2 : -INFINITY;
        }
        const float tmax = va_rowmax16(fmaxf(x[0], x[1]));
        const float mnew = fmaxf(m_run[r], tmax);
        const float alpha = mnew == -INFINITY ? 1.0f : exp2f(m_run[r] - mnew);
        float psum = 0.0f;
#pragma unroll
        for (int n = 0; n < 2; ++n) {
          const float p = x[n] == -INFINITY ? 0.0f : exp2f(x[n] - mnew);
          const uint16_t pb = va_bf16(p);
          psum += __uint_as_float((uint32_t)pb << 16);  // the sum of what P V uses
          sP[w][lr + r][16 * n + lc] = pb;
        }
        l_run[r] = l_run[r] * alpha + va_rowsum16(psum);
        m_run[r] = mnew;
#pragma unroll
        for (int n = 0; n < 8; ++n) o[n][r] *= alpha;
      }
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_wave_barrier();  // P written by the whole wave before it is read
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      // O += P V: K = the tile's 32 tokens
#pragma unroll
      for (int kc = 0; kc < VA_TOK / 16; ++kc) {
        const va_s4 pa = *reinterpret_cast<const va_s4*>(&sP[w][lc][kc * 16 + lr]);
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          const va_s4 vb = *reinterpret_cast<const va_s4*>(&sVt[n * 16 + lc][kc * 16 + lr]);
          o[n] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, vb, o[n], 0, 0, 0);
        }
      }
    }
    __syncthreads();  // the tile's LDS is rewritten next
  }
  if (bad && a.error) *a.error = 1;

  // ---- out[q0 + j, kvh * group + g, :] = O / l
  if (active) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + lr + r;
      if (i < M) {
        const int64_t j = i / a.group, g = i % a.group;
        uint16_t* dst = a.out + ((q0 + j) * a.hq + kvh * a.group + g) * VA_D;
        const float inv = l_run[r] > 0.0f ? 1.0f / l_run[r] : 0.0f;
#pragma unroll
        for (int n = 0; n < 8; ++n) dst[n * 16 + lc] = va_bf16(o[n][r] * inv);
      }
    }
  }
}

hipError_t launch_verify_attn(const AttnArgs& a, int64_t batch, hipStream_t s) {
  hipLaunchKernelGGL(verify_attn_kernel, dim3((unsigned)(batch * a.hkv)), dim3(VA_NT), 0, s, a);
  return hipGetLastError();
}

}  // namespace sdx
