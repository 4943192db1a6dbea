// Multi-query verify attention over paged KV, on MFMA: the attention of the
// target's verify forward (the k+1 new positions of every batch row against
// the row's cached keys, bench/bench_engine.py:170-174 through
// specdec/engine.py:273-275), with the additive mask of
// specdec/kvcache.py:138-162 (query j of row b sees key s iff
// s <= lengths[b] + j) and grouped-query heads (query head h reads KV head
// h / group, the repeat_kv of the HF Qwen3 attention).
//
// Split over the keys: one workgroup per (key chunk, KV head), so a long row
// spreads over many CUs. A plan kernel (one workgroup) lists the chunks longest
// first (all whole chunks, then the rows' last partial chunks by decreasing
// size), each with its row's shape, so the hardware's in-order dispatch ends on
// the shortest work and a workgroup learns everything about its chunk in one
// load; the KV heads of a chunk run on one XCD (workgroup index % 8) and stream
// the same page rows together, so each token's 2 KB row is read as eight
// 256-byte slices close in time. A workgroup's query rows are the q_b positions
// x group heads that share the KV head, up to 64 of them (padded to 16-row MFMA
// tiles; wave w owns rows 16w .. 16w + 15); a KV head with more query rows has a
// workgroup per block of 64, each streaming the chunk. The chunk's token -> pool slot map
// is built in LDS once from the block table (read alongside the row's shape);
// its keys then stream through LDS
// in tiles of 32 tokens (each token's head slice is 256 contiguous bytes of
// its page), two tiles in flight in registers while one is used:
//   S = Q K^T       16 x 32 per wave: 2 x 4 v_mfma_f32_16x16x32_bf16 (gfx950)
//   online softmax  per row in fp32 (max and sum across the 16-lane rows)
//   O += P V        16 x 128 per wave: 8 MFMAs (K = the tile's 32 tokens), P
//                   rounded to bf16
// Q operands stay in registers; V is stored transposed in LDS so both MFMA
// operands of P V are pairs of 8-byte reads. A row that fits one chunk writes its
// output directly; otherwise each chunk writes (O unnormalised, max, sum) in
// fp32 and a second kernel merges the chunks of the row.
// The kernels are bound by the KV bytes streamed (about 22 flop per byte),
// not by MFMA.
#include "sdx_launch.hpp"

namespace sdx {

constexpr int VA_NT = 256;
constexpr int VA_NW = VA_NT / kWave;
constexpr int VA_D = 128;     // largest head dim (workspace partial rows are sized for it)
constexpr int VA_TOK = 32;    // tokens per tile
constexpr int VA_MAXM = 64;   // query rows per workgroup (a block of the q_b * group)
// LDS row strides (bf16 elements): 2 mod 4 dwords, so the 8-byte MFMA operand
// reads of 16 consecutive rows hit 32 distinct banks
template <int D>
constexpr int va_ks() { return D + 4; }
constexpr int VA_VS = VA_TOK + 4;
constexpr int VA_PS = VA_TOK + 4;
constexpr int VA_CHMAX = 1024;  // most tokens per chunk (multiple of 2 tiles)

typedef short va_s4 __attribute__((ext_vector_type(4)));
typedef short va_s8 __attribute__((ext_vector_type(8)));
typedef __bf16 va_bf8 __attribute__((ext_vector_type(8)));
typedef float va_f4 __attribute__((ext_vector_type(4)));

// gfx950's v_mfma_f32_16x16x32_bf16: lane l holds A[l % 16][8 (l / 16) .. + 7] and
// B[8 (l / 16) .. + 7][l % 16] (eight bf16 each); D[4 (l / 16) + r][l % 16] in
// element r, as in the 16x16x16 form.
__device__ __forceinline__ va_f4 va_mfma32(va_s8 a, va_s8 b, va_f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(va_bf8, a),
                                                 __builtin_bit_cast(va_bf8, b), c, 0, 0, 0);
}
// Eight bf16 from two 8-byte LDS reads (the operand rows are 8-byte aligned).
__device__ __forceinline__ va_s8 va_ld8(const uint16_t* p) {
  const va_s4 lo = *reinterpret_cast<const va_s4*>(p);
  const va_s4 hi = *reinterpret_cast<const va_s4*>(p + 4);
  return (va_s8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}


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

constexpr uint32_t VA_NOSLOT = 0xFFFFFFFFu;  // a token whose page id is outside the pool

// the row checks both kernels make (uniform per workgroup): false for a row the
// launch cannot serve
__device__ __forceinline__ bool va_row(const AttnArgs& a, int64_t b, int64_t& q0, int64_t& qb,
                                       int64_t& kvl) {
  if (b < 0 || b >= a.batch) return false;
  q0 = a.cu_q[b];
  qb = a.cu_q[b + 1] - q0;
  kvl = a.kv_len[b];
  return qb >= 0 && qb <= a.max_q && kvl - qb >= 0 && (kvl + a.bs - 1) / a.bs <= a.max_blocks;
}

// ---- plan: one workgroup. Row b (valid, with queries) has kvl / chunk whole
// chunks and, if kvl % chunk > 0, one partial chunk. units[0 ..) = the whole
// chunks row by row, then the partial chunks by decreasing size, then b = -1 up
// to nunits. A row the launch cannot serve sets *error and gets no chunk.
constexpr int VA_PLAN_NT = 1024;

// exclusive scan over the workgroup of x (one value per thread); every thread
// gets the total
__device__ __forceinline__ long long va_block_scan(long long x, long long* sWave, long long& total) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
  long long inc = x;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const long long y = __shfl_up(inc, d, kWave);
    if (lane >= d) inc += y;
  }
  if (lane == kWave - 1) sWave[wv] = inc;
  __syncthreads();
  if (tid == 0) {
    long long run = 0;
    for (int k = 0; k < VA_PLAN_NT / kWave; ++k) {
      const long long t = sWave[k];
      sWave[k] = run;
      run += t;
    }
    sWave[VA_PLAN_NT / kWave] = run;
  }
  __syncthreads();
  const long long ex = sWave[wv] + inc - x;
  total = sWave[VA_PLAN_NT / kWave];
  __syncthreads();  // sWave is reused by the next scan
  return ex;
}

__global__ void __launch_bounds__(VA_PLAN_NT) verify_attn_plan_kernel(AttnArgs a) {
  __shared__ long long sWave[VA_PLAN_NT / kWave + 1];
  __shared__ int sBin[VA_CHMAX];  // partial chunks by size, then their first slot
  const int tid = threadIdx.x;
  for (int r = tid; r < VA_CHMAX; r += VA_PLAN_NT) sBin[r] = 0;
  if (a.arrive)  // the arrival counters of this call's chunk workgroups start at zero
    for (int64_t i = tid; i < a.batch * a.hkv; i += VA_PLAN_NT) a.arrive[i] = 0;
  __syncthreads();
  long long carry = 0;  // whole chunks so far
  // row tid's shape, kept for the partial chunks below (rows past VA_PLAN_NT are
  // read again there)
  bool ok0 = false;
  int64_t q00 = 0, qb0 = 0, kvl0 = 0;
  for (int64_t b0 = 0; b0 < a.batch; b0 += VA_PLAN_NT) {
    const int64_t b = b0 + tid;
    long long nfull = 0;
    int64_t q0 = 0, qb = 0, kvl = 0;
    if (b < a.batch) {
      const bool ok = va_row(a, b, q0, qb, kvl);
      if (b0 == 0) { ok0 = ok; q00 = q0; qb0 = qb; kvl0 = kvl; }
      if (ok) {
        if (qb > 0) {
          nfull = kvl / a.chunk;
          const int rem = (int)(kvl % a.chunk);
          if (rem > 0) atomicAdd(&sBin[rem], 1);
        }
      } else if (a.error) {
        *a.error = 1;
      }
    }
    long long tot;
    const long long f = carry + va_block_scan(nfull, sWave, tot);
    for (long long c = 0; c < nfull; ++c)
      a.units[f + c] = AttnUnit{(int32_t)b, (int32_t)c, a.chunk, (int32_t)qb, q0, kvl};
    carry += tot;
  }
  // first slot of each partial size, largest first: thread t takes size chunk - 1 - t
  {
    const int r = a.chunk - 1 - tid;
    const long long cnt = r >= 1 ? sBin[r] : 0;
    long long tot;
    const long long ex = va_block_scan(cnt, sWave, tot);
    if (r >= 1) sBin[r] = (int)(carry + ex);
    __syncthreads();
    carry += tot;  // all chunks
  }
  for (int64_t b = tid; b < a.batch; b += VA_PLAN_NT) {
    int64_t q0 = q00, qb = qb0, kvl = kvl0;
    const bool ok = b < VA_PLAN_NT ? ok0 : va_row(a, b, q0, qb, kvl);
    if (!ok || qb <= 0) continue;
    const int rem = (int)(kvl % a.chunk);
    if (rem == 0) continue;
    const int at = atomicAdd(&sBin[rem], 1);
    a.units[at] = AttnUnit{(int32_t)b, (int32_t)(kvl / a.chunk), rem, (int32_t)qb, q0, kvl};
  }
  for (int64_t u = carry + tid; u < a.nunits; u += VA_PLAN_NT) a.units[u].b = -1;
}

// Stores and loads of the chunk partials: agent-scope atomics, which go past
// the XCD's own L2 (each XCD has one), since the partials of a row are written
// by workgroups on several XCDs and read by one of them.
__device__ __forceinline__ void va_st_f32(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void va_st_f2(float* p, float x, float y) {  // p 8-byte aligned
  const uint64_t v = (uint64_t)__float_as_uint(x) | ((uint64_t)__float_as_uint(y) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 va_ld_f2(const float* p) {  // p 8-byte aligned
  const uint64_t v = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
}
__device__ __forceinline__ float4 va_ld_f4(const float* p) {  // p 16-byte aligned
  const float2 lo = va_ld_f2(p), hi = va_ld_f2(p + 2);
  return make_float4(lo.x, lo.y, hi.x, hi.y);
}

// Merge of the chunk partials of row b, KV head kvh (a row longer than one
// chunk) by the whole workgroup: out = sum_c w_c O_c with
// w_c = 2^(m_c - m) / sum_c' 2^(m_c' - m) l_c' and m the row's largest m_c. The
// (m, l) pairs go through LDS (sW, sL: `cap` floats each) and each query row's
// weights are formed once; the O partials are then read as float4 with the
// loads of several chunks in flight. With more chunks x rows than `cap` the
// weights are formed per element.
template <int D>
__device__ __forceinline__ void va_merge(const AttnArgs& a, int64_t b, int kvh, int64_t q0, int M,
                                         int nch, float* sW, float* sL, int cap) {
  const int64_t part0 = (b * a.hkv + kvh) * a.nchunk * a.max_m;
  const bool staged = nch * M <= cap;  // uniform
  if (staged) {
    for (int e = threadIdx.x; e < nch * M; e += VA_NT) {  // sW, sL [c * M + i] = m, l of (c, i)
      const int ch = e / M, i = e % M;
      const float2 ml = va_ld_f2(a.part_ml + (part0 + (int64_t)ch * a.max_m + i) * 2);
      sW[e] = ml.x;
      sL[e] = ml.y;
    }
    __syncthreads();
    if (threadIdx.x < M) {  // one thread per query row: weights in place of the maxima
      const int i = threadIdx.x;
      float mx = -INFINITY;
      for (int ch = 0; ch < nch; ++ch) mx = fmaxf(mx, sW[ch * M + i]);
      float den = 0.0f;
      for (int ch = 0; ch < nch; ++ch) {
        const float m = sW[ch * M + i];
        const float f = m == -INFINITY ? 0.0f : exp2f(m - mx);
        sW[ch * M + i] = f;
        den += f * sL[ch * M + i];
      }
      const float inv = den > 0.0f ? 1.0f / den : 0.0f;
      for (int ch = 0; ch < nch; ++ch) sW[ch * M + i] *= inv;
    }
    __syncthreads();
  }
  for (int e = threadIdx.x; e < M * (D / 4); e += VA_NT) {
    const int i = e / (D / 4), d4 = e % (D / 4);
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (staged) {
#pragma unroll 4
      for (int ch = 0; ch < nch; ++ch) {
        const float wgt = sW[ch * M + i];
        const float4 v = va_ld_f4(a.part_o + (part0 + (int64_t)ch * a.max_m + i) * D + d4 * 4);
        acc.x += wgt * v.x;
        acc.y += wgt * v.y;
        acc.z += wgt * v.z;
        acc.w += wgt * v.w;
      }
    } else {
      float mx = -INFINITY;
      for (int ch = 0; ch < nch; ++ch)
        mx = fmaxf(mx, va_ld_f2(a.part_ml + (part0 + (int64_t)ch * a.max_m + i) * 2).x);
      float den = 0.0f;
      for (int ch = 0; ch < nch; ++ch) {
        const int64_t p = part0 + (int64_t)ch * a.max_m + i;
        const float2 ml = va_ld_f2(a.part_ml + p * 2);
        if (ml.x == -INFINITY) continue;  // the chunk holds none of the row's visible keys
        const float f = exp2f(ml.x - mx);
        den += f * ml.y;
        const float4 v = va_ld_f4(a.part_o + p * D + d4 * 4);
        acc.x += f * v.x;
        acc.y += f * v.y;
        acc.z += f * v.z;
        acc.w += f * v.w;
      }
      const float inv = den > 0.0f ? 1.0f / den : 0.0f;
      acc.x *= inv;
      acc.y *= inv;
      acc.z *= inv;
      acc.w *= inv;
    }
    const int64_t j = i / a.group, g = i % a.group;
    uint16_t* dst = a.out + ((q0 + j) * a.hq + kvh * a.group + g) * D + d4 * 4;
    const uint32_t lo = (uint32_t)va_bf16(acc.x) | ((uint32_t)va_bf16(acc.y) << 16);
    const uint32_t hi = (uint32_t)va_bf16(acc.z) | ((uint32_t)va_bf16(acc.w) << 16);
    *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
  }
}

// D: head dim, 64 or 128.
template <int D>
__global__ void __launch_bounds__(VA_NT) __attribute__((amdgpu_waves_per_eu(3)))
verify_attn_kernel(AttnArgs a) {
  static_assert(D == 64 || D == 128, "head dims of 64 or 128");
  constexpr int TPT = D / 8;           // threads per token of a K tile (16 bytes each)
  constexpr int TPP = VA_NT / TPT;     // tokens per pass of the block
  constexpr int KH = VA_TOK / TPP;     // passes per K tile
  __shared__ __align__(16) uint16_t sK[VA_TOK][va_ks<D>()];
  __shared__ __align__(16) uint16_t sVt[D][VA_VS];
  __shared__ __align__(16) uint16_t sP[VA_NW][16][VA_PS];
  __shared__ __align__(16) uint32_t sSlot[VA_CHMAX];  // chunk token -> head slice (256 B) of the pool
  __shared__ int64_t sRow[VA_MAXM];  // query row i -> element offset of its q / out vector

  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  // a chunk's workgroups on one XCD (workgroup % 8): one per (KV head, block of
  // VA_MAXM query rows), hx = rb * hkv + kvh of nh = hkv * nrb; blocks 8 nh g ..
  // cover chunks 8g .. 8g + 7, chunk 8g + x's hx at 8 nh g + 8 hx + x
  const int64_t nh = (int64_t)a.hkv * a.nrb;
  const int64_t grp = blockIdx.x / (8 * nh), rem = blockIdx.x % (8 * nh);
  const int hx = (int)(rem / 8);
  const int kvh = hx % a.hkv, rb = hx / a.hkv;
  const int64_t unit = 8 * grp + rem % 8;
  if (unit >= a.nunits) return;
  const AttnUnit un = a.units[unit];
  if (un.b < 0) return;  // uniform: no chunk in this slot
  const int64_t b = un.b, q0 = un.q0, qb = un.qb, kvl = un.kvl;
  const int c = un.c, n = un.n;
  // the KV head's query rows of the row (qb positions x group heads), and this
  // workgroup's block of them: rows rofs .. rofs + M - 1
  const int Mt = (int)qb * a.group, rofs = VA_MAXM * rb;
  if (rofs >= Mt) return;  // uniform: the row has fewer row blocks
  const int M = min(Mt - rofs, VA_MAXM);
  const int64_t c0 = (int64_t)c * a.chunk;
  const int64_t p0 = c0 / a.bs;  // first page of the chunk
  const int np = (int)((c0 + n - 1) / a.bs - p0 + 1);
  // the chunk's page ids go to LDS (in the V tile's space, unused yet)
  int32_t* sPage = reinterpret_cast<int32_t*>(&sVt[0][0]);
  for (int i = tid; i < np; i += VA_NT) sPage[i] = a.block_table[b * a.max_blocks + p0 + i];
  const int64_t base = kvl - qb;
  const bool whole = kvl <= a.chunk;  // the row is one chunk: write the output directly
  // row i = j * group + g is query head kvh * group + g of position j; local row
  // il of the block is row rofs + il
  if (tid < M) {
    const int i = rofs + tid;
    sRow[tid] = ((q0 + i / a.group) * a.hq + kvh * a.group + i % a.group) * D;
  }
  __syncthreads();  // page ids and row offsets in LDS

  // ---- the chunk's slots: token t -> (page * bs + (c0 + t) % bs) * hkv + kvh
  int bad = 0;
  for (int t = tid; t < n; t += VA_NT) {
    const int64_t pos = c0 + t;
    const int32_t page = sPage[pos / a.bs - p0];
    const bool ok = page >= 0 && page < a.num_blocks;
    bad |= !ok;
    sSlot[t] = ok ? (uint32_t)((((int64_t)page * a.bs + pos % a.bs) * a.hkv) + kvh) : VA_NOSLOT;
  }

  // ---- tile loads. K: thread t moves 16 bytes (8 dims) of tokens t / TPT,
  // TPP + t / TPT, ... (two passes at D = 128, one at 64). V: wave w moves tokens
  // 8w .. 8w + 7, lane l < D / 2 dims 2l, 2l + 1 of each (a 2D-byte row per
  // load), so a lane can write V transposed in 8-byte runs of 4 tokens.
  const int ltok = tid / TPT, lpart = tid % TPT;
  const bool vlane = D >= 2 * kWave || 2 * lane < D;  // this lane holds V dims (all at D = 128)
  // Loads are unconditional, so they stay in flight across the tile loop: a
  // token past the chunk or with a page outside the pool reads slice 0 instead;
  // its K only meets masked scores (or an error-flagged row) and its V is zeroed
  // when staged.
  auto gather = [&](int t0, uint4 (&kk)[KH], uint32_t (&vv)[8], uint32_t& vok) {
#pragma unroll
    for (int h = 0; h < KH; ++h) {
      const int t = t0 + ltok + TPP * h;
      const uint32_t sl = sSlot[min(t, n - 1)];
      const bool ok = t < n && sl != VA_NOSLOT;
      kk[h] = *reinterpret_cast<const uint4*>(a.k_pool + (size_t)(ok ? sl : 0u) * D + lpart * 8);
    }
    const int tb = t0 + 8 * w;  // the wave's 8 tokens: slots read as two 16-byte words
    const int tr = min(tb, VA_CHMAX - 8);
    const uint4 s0 = *reinterpret_cast<const uint4*>(&sSlot[tr]);
    const uint4 s1 = *reinterpret_cast<const uint4*>(&sSlot[tr + 4]);
    const uint32_t sl[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    vok = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool ok = tb + e < n && sl[e] != VA_NOSLOT;
      vok |= (uint32_t)ok << e;
      vv[e] = *reinterpret_cast<const uint32_t*>(a.v_pool + (size_t)(ok ? sl[e] : 0u) * D +
                                                 (vlane ? 2 * lane : 0));
    }
  };
  auto stage = [&](const uint4 (&kk)[KH], const uint32_t (&vr)[8], uint32_t vok) {
#pragma unroll
    for (int h = 0; h < KH; ++h) {
      uint2* dst = reinterpret_cast<uint2*>(&sK[ltok + TPP * h][lpart * 8]);  // rows are 8-byte aligned
      dst[0] = make_uint2(kk[h].x, kk[h].y);
      dst[1] = make_uint2(kk[h].z, kk[h].w);
    }
    uint32_t vv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) vv[e] = (vok >> e) & 1u ? vr[e] : 0u;
    // dim 2l: the low halves of the 8 tokens, dim 2l + 1 the high halves
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lo[e] = (vv[2 * e] & 0xFFFFu) | (vv[2 * e + 1] << 16);
      hi[e] = (vv[2 * e] >> 16) | (vv[2 * e + 1] & 0xFFFF0000u);
    }
    if (vlane) {
      uint2* d0 = reinterpret_cast<uint2*>(&sVt[2 * lane][8 * w]);
      uint2* d1 = reinterpret_cast<uint2*>(&sVt[2 * lane + 1][8 * w]);
      d0[0] = make_uint2(lo[0], lo[1]);
      d0[1] = make_uint2(lo[2], lo[3]);
      d1[0] = make_uint2(hi[0], hi[1]);
      d1[1] = make_uint2(hi[2], hi[3]);
    }
  };

  // ---- per-wave state: rows r0 + 4 * (lane / 16) + r, r < 4
  const int r0 = 16 * w;
  const bool active = r0 < M;  // uniform per wave
  const int lr = 4 * (lane / 16), lc = lane % 16;
  constexpr int OJ = D / 16;  // 16-wide output column blocks per wave
  va_f4 o[OJ];
#pragma unroll
  for (int j = 0; j < OJ; ++j) o[j] = (va_f4){0.0f, 0.0f, 0.0f, 0.0f};
  float m_run[4], l_run[4];
  int lim[4];  // last visible key of the lane's rows, relative to the chunk (-1: none;
               // at most n - 1, so a tile past the chunk's end is all masked)
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m_run[r] = -INFINITY;
    l_run[r] = 0.0f;
    const int i = r0 + lr + r;
    const int64_t l = i < M ? base + (rofs + i) / a.group - c0 : -1;
    lim[r] = (int)max((int64_t)-1, min(l, (int64_t)n - 1));
  }

  // the wave's query operands, in registers: lane holds row r0 + lc, dims
  // 32 kc + lk .. + 7 (lk = 8 (lane / 16), the operand layout of the 16x16x32 form)
  const int lk = 8 * (lane / 16);
  va_s8 qa[D / 32];
  {
    const int i = r0 + lc;
    const bool has = active && i < M;
    const uint16_t* src = a.q + (has ? sRow[i] : 0);
#pragma unroll
    for (int kc = 0; kc < D / 32; ++kc)
      qa[kc] = has ? *reinterpret_cast<const va_s8*>(src + kc * 32 + lk)
                   : (va_s8){0, 0, 0, 0, 0, 0, 0, 0};
  }

  // one tile: the wave's rows against the 32 keys from chunk token t0 in LDS
  auto compute = [&](int t0) {
    // S = Q K^T for the wave's 16 rows x 32 tokens
    va_f4 s[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) s[j] = (va_f4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kc = 0; kc < D / 32; ++kc) {
#pragma unroll
      for (int j = 0; j < 2; ++j) s[j] = va_mfma32(qa[kc], va_ld8(&sK[j * 16 + lc][kc * 32 + lk]), s[j]);
    }
    // online softmax in base 2; s[j][r] is row lr + r, token t0 + 16 j + lc
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float x[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) x[j] = t0 + 16 * j + lc <= lim[r] ? s[j][r] * a.scale_log2 : -INFINITY;
      const float tmax = va_rowmax16(fmaxf(x[0], x[1]));
      const float mnew = fmaxf(m_run[r], tmax);
      const float alpha = mnew == -INFINITY ? 1.0f : exp2f(m_run[r] - mnew);
      float psum = 0.0f;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float p = x[j] == -INFINITY ? 0.0f : exp2f(x[j] - mnew);
        const uint16_t pb = va_bf16(p);
        psum += __uint_as_float((uint32_t)pb << 16);  // the sum of what P V uses
        sP[w][lr + r][16 * j + lc] = pb;
      }
      l_run[r] = l_run[r] * alpha + va_rowsum16(psum);
      m_run[r] = mnew;
#pragma unroll
      for (int j = 0; j < OJ; ++j) o[j][r] *= alpha;
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_wave_barrier();  // P written by the whole wave before it is read
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    // O += P V: K = the tile's 32 tokens, one 16x16x32 product per 16 output dims
    static_assert(VA_TOK == 32, "one K step of the 16x16x32 form per tile");
    const va_s8 pa = va_ld8(&sP[w][lc][lk]);
#pragma unroll
    for (int j = 0; j < OJ; ++j) o[j] = va_mfma32(pa, va_ld8(&sVt[j * 16 + lc][lk]), o[j]);
  };

  __syncthreads();  // the slot map is complete
  // two tiles in flight while one is used: A holds tiles 0, 2, 4, ..., B 1, 3, 5, ...
  uint4 kA[KH], kB[KH];
  uint32_t vA[8], vB[8], okA, okB;
  gather(0, kA, vA, okA);
  gather(VA_TOK, kB, vB, okB);
  // one exit, at the bottom: both register sets are then in flight in the same
  // order on every entry to the loop, so each stage waits for its own set only
  // (a second tile past the chunk's end is all masked, with V zeroed)
  for (int t0 = 0;; t0 += 2 * VA_TOK) {
    stage(kA, vA, okA);
    __syncthreads();
    gather(t0 + 2 * VA_TOK, kA, vA, okA);
    if (active) compute(t0);
    __syncthreads();  // the tile's LDS is rewritten next
    stage(kB, vB, okB);
    __syncthreads();
    gather(t0 + 3 * VA_TOK, kB, vB, okB);
    if (active) compute(t0 + VA_TOK);
    __syncthreads();
    if (t0 + 2 * VA_TOK >= n) break;
  }
  if (bad && a.error) *a.error = 1;
  // the row index is rebuilt here rather than kept live across the tile loop
  int lre = lr;
  asm volatile("" : "+v"(lre));

  if (whole) {  // out[q0 + j, kvh * group + g, :] = O / l
    if (!active) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + lre + r;
      if (i < M) {
        uint16_t* dst = a.out + sRow[i];
        const float inv = l_run[r] > 0.0f ? 1.0f / l_run[r] : 0.0f;
#pragma unroll
        for (int jj = 0; jj < OJ; ++jj) dst[jj * 16 + lc] = va_bf16(o[jj][r] * inv);
      }
    }
    return;
  }
  // the chunk's partial: O unnormalised and (max, sum) per query row, in the
  // part of (row b, KV head, chunk c); the block's rows from rofs
  const int64_t part = ((b * a.hkv + kvh) * a.nchunk + c) * a.max_m + rofs;
  if (active) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = r0 + lre + r;
      if (i < M) {
        float* po = a.part_o + (part + i) * D;
#pragma unroll
        for (int jj = 0; jj < OJ; ++jj) va_st_f32(po + jj * 16 + lc, o[jj][r]);
        if (lc == 0) va_st_f2(a.part_ml + (part + i) * 2, m_run[r], l_run[r]);
      }
    }
  }
  // the workgroup's stores are done before it counts in on the (row, KV head):
  // the one that counts in last merges the row's chunks
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // gfx9 encoding: vmcnt(0)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  const int nch = (int)((kvl + a.chunk - 1) / a.chunk);
  const int nrbr = (Mt + VA_MAXM - 1) / VA_MAXM;  // the row's blocks of query rows
  uint32_t* const flag = reinterpret_cast<uint32_t*>(&sRow[0]);  // row offsets no longer needed
  if (tid == 0)
    *flag = __hip_atomic_fetch_add(a.arrive + b * a.hkv + kvh, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(nch * nrbr - 1);
  __syncthreads();
  if (!*flag) return;  // uniform
  // the tile buffers hold the merge's weights
  static_assert(sizeof(sK) <= sizeof(sVt), "merge weights sized by the K tile");
  va_merge<D>(a, b, kvh, q0, Mt, nch, reinterpret_cast<float*>(&sK[0][0]),
              reinterpret_cast<float*>(&sVt[0][0]), (int)(sizeof(sK) / sizeof(float)));
}

int attn_chunk_tokens(int64_t batch, int32_t hkv, int64_t max_tokens, int32_t chunk) {
  if (chunk > 0) return chunk;
  // smallest chunk count that still leaves about 8 workgroups per CU of work
  int ch = VA_CHMAX;
  while (ch > 2 * VA_TOK && batch * hkv * ((max_tokens + ch - 1) / ch) < 8 * 256) ch /= 2;
  return ch;
}

template <int D>
static hipError_t launch_attn_d(const AttnArgs& a, hipStream_t s) {
  if (a.nchunk > 1 && !a.arrive) return hipErrorInvalidValue;
  hipLaunchKernelGGL(verify_attn_kernel<D>,
                     dim3((unsigned)((a.nunits + 7) / 8 * 8 * a.hkv * a.nrb)),
                     dim3(VA_NT), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_verify_attn(const AttnArgs& a, int64_t batch, hipStream_t s) {
  if (a.d != 64 && a.d != 128) return hipErrorInvalidValue;
  hipLaunchKernelGGL(verify_attn_plan_kernel, dim3(1), dim3(VA_PLAN_NT), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return a.d == 64 ? launch_attn_d<64>(a, s) : launch_attn_d<128>(a, s);
}

}  // namespace sdx
