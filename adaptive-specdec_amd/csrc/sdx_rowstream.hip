// Row statistics for bf16 logits, streaming (the device code is in
// sdx_rowstream.hpp): the row-statistics kernel, the fused verify kernel (row
// statistics + accept chain + draw in one launch) and their launchers.
#include "sdx_rowstream.hpp"

namespace sdx {

__global__ void __launch_bounds__(SK_NT) __attribute__((amdgpu_waves_per_eu(6)))
rowstream_bf16_kernel(RowStatArgs a) {
  __shared__ SkLds L;
  rowstream_body<false>(a, L, blockIdx.x);
}

// Compute units of the current device (cached per device; 0 if unknown).
static int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    cus[dev] = n;
  }
  return cus[dev];
}

// Rows beyond the last whole multiple of the CU count are split into parts so
// that every CU streams about the same number of bytes (576 rows on 256 CUs:
// 512 whole rows, 64 rows in 4 parts). Parts hold at least SK_PART_MIN_GROUPS
// groups and at most SK_PART_MAX logits; 0 parts: no split.
static int split_layout(int64_t rows, int64_t V, int cus, int64_t* nwhole) {
  *nwhole = rows;
  if (cus <= 0 || rows <= 0) return 0;
  const int64_t whole = rows / cus * cus, rest = rows - whole;
  if (rest == 0 || rest > kWsMaxCounters) return 0;
  const int64_t n4 = V >> 3;
  int64_t p = cus / rest;
  if (p > 8) p = 8;
  if (p > n4 / SK_PART_MIN_GROUPS) p = n4 / SK_PART_MIN_GROUPS;
  while (p >= 2 && p <= 8 && ((n4 + p - 1) / p) * 8 + 7 > SK_PART_MAX) ++p;
  if (p < 2 || p > 8 || n4 / p < SK_PART_MIN_GROUPS) return 0;
  *nwhole = whole;
  return (int)p;
}
static size_t split_need(int64_t rows, int64_t nwhole, int p) {
  if (p < 2) return 0;
  const int64_t rest = rows - nwhole;
  return (size_t)rest * p * SK_SPLIT_BYTES;
}

int64_t rowstream_split_rows(int64_t rows, int64_t V, int cus) {
  int64_t nwhole;
  const int p = split_layout(rows, V, cus, &nwhole);
  return p >= 2 ? rows - nwhole : 0;
}

size_t rowstream_split_bytes(int64_t rows, int64_t V) {
  int64_t nwhole;
  const int p = split_layout(rows, V, device_cus(), &nwhole);
  return split_need(rows, nwhole, p);
}

// The launch shape of the row statistics: sets late_block and the split layout
// of `a` and returns the number of blocks.
int64_t rowstream_setup(RowStatArgs& a, int64_t rows) {
  const int cus = device_cus();
  a.late_block = cus > 0 ? 2 * (int64_t)cus : INT64_MAX;
  int64_t nwhole;
  int p = split_layout(rows, a.V, cus, &nwhole);
  if (p >= 2 && (!a.split_ws || !a.ws_header || a.split_bytes < split_need(rows, nwhole, p)))
    p = 0;
  int64_t grid = rows;
  if (p >= 2) {
    const int64_t rest = rows - nwhole;
    a.nwhole = nwhole;
    a.nparts = p;
    a.xcd_group = (nwhole % 8 == 0 && rest % 8 == 0) ? 1 : 0;
    a.split_cnt = split_counter_words(a.ws_header);
    a.split_parts = a.split_ws;
    grid = nwhole + rest * p;
  } else {
    a.nwhole = rows;
    a.nparts = 1;
    a.xcd_group = 0;
    a.split_cnt = nullptr;
    a.split_parts = nullptr;
  }
  return grid;
}

hipError_t launch_rowstream_bf16(const RowStatArgs& args, int64_t rows, hipStream_t s) {
  RowStatArgs a = args;
  const int64_t grid = rowstream_setup(a, rows);
  hipLaunchKernelGGL(rowstream_bf16_kernel, dim3((unsigned)grid), dim3(SK_NT), 0, s, a);
  return hipGetLastError();
}


__global__ void __launch_bounds__(SK_NT) __attribute__((amdgpu_waves_per_eu(6)))
verify_fused_bf16_kernel(FusedArgs a) {
  __shared__ union FusedLds {
    SkLds row;
    Draw16Lds draw;
  } U;
  const int64_t blk = blockIdx.x;
  if (blk < a.nrow_pad) {
    if (blk >= a.nrow) return;
    const int64_t row = rowstream_body<true>(a.rs, U.row, blk);
    if (row < 0) return;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // gfx9 encoding: vmcnt(0) (the row's stores done)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (threadIdx.x == 0) {
      const int64_t nt = a.rs.nrows[0];
      const int64_t b = a.rowjob ? (int64_t)a.rowjob[row]
                                 : (row < nt ? row / (a.rs.k + 1) : (row - nt) / a.rs.k);
      if (b >= 0)
        __hip_atomic_fetch_add(&a.d.job_cnt[b], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  if (threadIdx.x >= SM_NT) return;
  const int64_t t = blk - a.nrow_pad;
  int64_t j;
  int bi;
  if (a.d.xcd) {  // a job's blocks on one XCD, as in draw16_kernel
    const int64_t i = t >> 3;
    j = (t & 7) + 8 * (i / a.d.nblk);
    bi = (int)(i % a.d.nblk);
  } else {
    j = t / a.d.nblk;
    bi = (int)(t % a.d.nblk);
  }
  // per-row k: a batch row with inconsistent offsets draws nothing (its rows
  // were not counted in); it gets n_acc 0 and SDX_FLAG_BAD_ROW
  const AcceptArgs& acc = a.d.acc;
  if (acc.cu_k && acc.bad[j]) {
    if (threadIdx.x == 0 && bi == 0) {
      if (acc.n_acc) acc.n_acc[j] = 0;
      if (acc.flags) acc.flags[j] = (uint8_t)SDX_FLAG_BAD_ROW;
      a.d.y[j] = -1;
    }
    return;
  }
  if (threadIdx.x == 0) {
    int ok = 0;
    const uint32_t need =
        acc.cu_k ? (uint32_t)(2 * (acc.cu_k[j + 1] - acc.cu_k[j]) + 1) : a.need;
    if (__hip_atomic_load(a.rs.ws_header, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == kWsMagic) {
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      for (;;) {
        if (__hip_atomic_load(&a.d.job_cnt[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= need) {
          ok = 1;
          break;
        }
        if (__builtin_amdgcn_s_memrealtime() - t0 > a.wait_ticks) {
          // the counters of this call may now be left behind: mark the header
          __hip_atomic_store(a.rs.ws_header, kWsDirty, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    U.draw.last = ok;
  }
  __syncthreads();
  if (!U.draw.last) {
    // every block that gives up flags its batch row; none of them counts in, so
    // no block of the row draws and these are the row's outputs
    if (threadIdx.x == 0) {
      if (a.d.acc.n_acc) a.d.acc.n_acc[j] = 0;
      if (a.d.acc.flags) a.d.acc.flags[j] = (uint8_t)SDX_FLAG_WORKSPACE;
      a.d.y[j] = -1;
    }
    return;
  }
  draw16_body<SDX_BF16, true>(a.d, U.draw, j, bi);
}

// The draw blocks' wait bound: kFusedWaitTicks, or a smaller bound from
// SDX_VERIFY_WAIT_TICKS (read at every launch; tests set 0 to make every wait give
// up from the host, so that the give-up path runs while every kernel exits normally).
uint64_t fused_wait_ticks() {
  const char* e = getenv("SDX_VERIFY_WAIT_TICKS");
  if (!e || !*e) return kFusedWaitTicks;
  char* end = nullptr;
  const unsigned long long v = strtoull(e, &end, 10);
  if (!end || *end != '\0') return kFusedWaitTicks;
  return v < kFusedWaitTicks ? (uint64_t)v : kFusedWaitTicks;
}

hipError_t launch_verify_fused_bf16(const RowStatArgs& rs, int64_t rows, const RowSource16& src,
                                    const AcceptArgs& acc, int64_t njobs, int64_t V, float T,
                                    ChunkRec* recs, uint32_t* counters, uint32_t* job_cnt,
                                    int64_t* y, hipStream_t s, const int32_t* rowjob) {
  const bool ragged = acc.cu_k != nullptr;
  const int64_t per_job = 2 * (int64_t)rs.k + 1;
  if (!src.vec || !y || !job_cnt || !rs.ws_header || V % 8 != 0 || rs.k < 0 ||
      2 * rs.k + 1 > kWave || (rs.k == 0 && (ragged || rs.nrows[1] != 0)) ||
      (ragged ? (!rowjob || !rs.jm_order || !acc.bad) : rows != njobs * per_job))
    return hipErrorInvalidValue;
  FusedArgs a = {};
  a.rs = rs;
  a.rs.jm_k = rs.k;
  a.rs.jm_xcd = !ragged && njobs % 8 == 0 ? 1 : 0;
  if (!ragged) a.rs.jm_order = nullptr;
  a.rowjob = ragged ? rowjob : nullptr;
  a.rs.zero = nullptr;  // the draw counters reset themselves (a row block could clear one late)
  a.rs.nzero = 0;
  a.nrow = rowstream_setup(a.rs, rows);
  a.nrow_pad = (a.nrow + 7) / 8 * 8;
  Draw16Args<SDX_BF16>& d = a.d;
  d.acc = acc;
  d.ev = Eval16<SDX_BF16>{src.base, src.ld, src.base2, src.ld2, src.split, rs.stats, rs.tables, T};
  d.V = V;
  d.nrec = (int32_t)((V + kRec16 - 1) / kRec16);
  if (d.nrec > kMaxRec16) return hipErrorInvalidValue;
  d.nblk = (d.nrec + SM_NW - 1) / SM_NW;
  d.xcd = njobs % 8 == 0 ? 1 : 0;
  d.recs = recs;
  d.counters = counters;
  d.job_cnt = job_cnt;
  d.y = y;
  a.need = (uint32_t)per_job;
  a.wait_ticks = fused_wait_ticks();
  const int64_t grid = a.nrow_pad + njobs * d.nblk;
  hipLaunchKernelGGL(verify_fused_bf16_kernel, dim3((unsigned)grid), dim3(SK_NT), 0, s, a);
  return hipGetLastError();
}

// Zero a workspace and write the header's magic word, in one kernel (no memset,
// so the call can sit in a captured graph).
__global__ void workspace_init_kernel(uint32_t* ws, int64_t words) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += stride)
    ws[i] = i == 0 ? kWsMagic : 0u;
}

__global__ void __launch_bounds__(256) workspace_rearm_kernel(uint32_t* hdr) {
  __shared__ int dirty;
  if (threadIdx.x == 0) dirty = hdr[0] != kWsMagic;
  __syncthreads();
  if (!dirty) return;
  for (int i = 1 + (int)threadIdx.x; i < (int)(kWsHeaderBytes / 4); i += 256) hdr[i] = 0u;
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();
    hdr[0] = kWsMagic;
  }
}

hipError_t launch_workspace_rearm(void* ws, hipStream_t s) {
  hipLaunchKernelGGL(workspace_rearm_kernel, dim3(1), dim3(256), 0, s, (uint32_t*)ws);
  return hipGetLastError();
}

hipError_t launch_workspace_init(void* ws, size_t bytes, hipStream_t s) {
  const int64_t words = (int64_t)(bytes / 4);
  if (words == 0) return hipSuccess;
  int64_t blocks = (words + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(workspace_init_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                     (uint32_t*)ws, words);
  return hipGetLastError();
}

}  // namespace sdx
