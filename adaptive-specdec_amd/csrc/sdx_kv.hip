// KV-cache bookkeeping and scatter (specdec/kvcache.py) and the paged slot
// mapping of the draft proposer (vllm_draft_spec/proposer.py:295-314).
//
// Lengths live on the device: advance / rollback are O(1) per row and never
// touch K/V bytes (a rolled-back tail is simply never attended again). The
// paged append moves each new (layer, side, row, position) vector of
// kv_heads * head_dim bf16 values (2 KiB for 8 x 128) with one wavefront of
// 16-byte stores into the slot named by the shared block table.
#include <string.h>

#include "sdx_launch.hpp"

namespace sdx {

__global__ void kv_advance_kernel(int64_t* lengths, int64_t batch, int64_t q) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b < batch) lengths[b] += q;
}

// Single workgroup: check every row first, then apply, so an invalid request
// leaves all lengths untouched (the error is reported through *error).
__global__ void __launch_bounds__(1024) kv_rollback_kernel(int64_t* lengths, int64_t batch,
                                                           const int64_t* n, int32_t* error) {
  __shared__ int bad;
  if (threadIdx.x == 0) bad = 0;
  __syncthreads();
  for (int64_t b = threadIdx.x; b < batch; b += blockDim.x)
    if (lengths[b] - n[b] < 0 || n[b] < 0) bad = 1;
  __syncthreads();
  if (bad) {
    if (threadIdx.x == 0 && error) *error = 1;
    return;
  }
  for (int64_t b = threadIdx.x; b < batch; b += blockDim.x) lengths[b] -= n[b];
}

// keys/values [B, H, C, D]; new [B, H, q, D]; one wavefront per (b, h, j) row.
template <typename T>
__global__ void ragged_update_kernel(T* keys, T* values, const T* kn, const T* vn, int64_t B,
                                     int64_t H, int64_t C, int64_t D, int64_t q,
                                     const int64_t* lengths, int32_t* error) {
  const int64_t w = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  if (w >= B * H * q) return;
  const int64_t j = w % q, h = (w / q) % H, b = w / (q * H);
  const int64_t slot = lengths[b] + j;
  if (slot < 0 || slot >= C) {
    if (lane == 0 && error) *error = 1;
    return;
  }
  const int64_t src = ((b * H + h) * q + j) * D;
  const int64_t dst = ((b * H + h) * C + slot) * D;
  for (int64_t d = lane; d < D; d += kWave) {
    keys[dst + d] = kn[src + d];
    values[dst + d] = vn[src + d];
  }
}

template <typename T>
__global__ void attn_mask_kernel(const int64_t* lengths, const int64_t* valid, int64_t B, int64_t q,
                                 int64_t kv, T zero, T neg, T* out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * q * kv) return;
  const int64_t s = i % kv, j = (i / kv) % q, b = i / (kv * q);
  bool ok = s <= lengths[b] + j;
  if (valid) ok = ok && s < valid[b];
  out[i] = ok ? zero : neg;
}

// Paged append: one wavefront per (layer, side, row, position) vector.
__global__ void kv_append_paged_kernel(uint8_t* pool, int64_t layer_stride_b,
                                       int64_t side_stride_b, const uint8_t* staged,
                                       int32_t layers, int64_t batch, int64_t q,
                                       int64_t row_bytes, const int32_t* block_table,
                                       int64_t max_blocks, int32_t bs, int64_t num_blocks,
                                       const int64_t* lengths, int32_t* error) {
  const int64_t w = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t total = (int64_t)layers * 2 * batch * q;
  if (w >= total) return;
  const int64_t j = w % q;
  const int64_t b = (w / q) % batch;
  const int64_t ls = w / (q * batch);  // layer * 2 + side
  const int64_t l = ls / 2, sd = ls % 2;
  const int64_t pos = lengths[b] + j;
  const int64_t blk_i = pos / bs;
  if (pos < 0 || blk_i >= max_blocks) {
    if (lane == 0 && error) *error = 1;
    return;
  }
  const int64_t blk = block_table[b * max_blocks + blk_i];
  if (blk < 0 || blk >= num_blocks) {
    if (lane == 0 && error) *error = 1;
    return;
  }
  const int64_t slot = blk * bs + pos % bs;
  const uint8_t* src = staged + w * row_bytes;
  uint8_t* dst = pool + l * layer_stride_b + sd * side_stride_b + slot * row_bytes;
  // row_bytes is a multiple of 16 (checked on the host)
  for (int64_t o = (int64_t)lane * 16; o < row_bytes; o += kWave * 16)
    *reinterpret_cast<uint4*>(dst + o) = *reinterpret_cast<const uint4*>(src + o);
}

__global__ void slot_mapping_kernel(const int32_t* bt, int64_t rows, int64_t max_blocks,
                                    const int64_t* positions, int32_t bs, int64_t max_len,
                                    int64_t pad_slot, int64_t* clamped, int64_t* slots) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int64_t pos = positions[r];
  const bool over = pos >= max_len;
  const int64_t cp = over ? 0 : pos;
  if (clamped) clamped[r] = cp;
  const int64_t bi = cp / bs;
  if (over || cp < 0 || bi >= max_blocks) {
    slots[r] = pad_slot;
    return;
  }
  slots[r] = (int64_t)bt[r * max_blocks + bi] * bs + cp % bs;
}

// ---------------------------------------------------------------- launches
hipError_t launch_kv_advance(int64_t* lengths, int64_t batch, int64_t q, hipStream_t s) {
  const int nt = 256;
  hipLaunchKernelGGL(kv_advance_kernel, dim3((unsigned)((batch + nt - 1) / nt)), dim3(nt), 0, s,
                     lengths, batch, q);
  return hipGetLastError();
}

hipError_t launch_kv_rollback(int64_t* lengths, int64_t batch, const int64_t* n, int32_t* error,
                              hipStream_t s) {
  hipLaunchKernelGGL(kv_rollback_kernel, dim3(1), dim3(1024), 0, s, lengths, batch, n, error);
  return hipGetLastError();
}

hipError_t launch_ragged_update(int dtype, void* keys, void* values, const void* kn,
                                const void* vn, int64_t B, int64_t H, int64_t C, int64_t D,
                                int64_t q, const int64_t* lengths, int32_t* error, hipStream_t s) {
  const int nt = 256;
  const int64_t waves = B * H * q;
  const dim3 grid((unsigned)((waves * kWave + nt - 1) / nt));
  if (dtype == SDX_F32)
    hipLaunchKernelGGL((ragged_update_kernel<float>), grid, dim3(nt), 0, s, (float*)keys,
                       (float*)values, (const float*)kn, (const float*)vn, B, H, C, D, q, lengths,
                       error);
  else
    hipLaunchKernelGGL((ragged_update_kernel<uint16_t>), grid, dim3(nt), 0, s, (uint16_t*)keys,
                       (uint16_t*)values, (const uint16_t*)kn, (const uint16_t*)vn, B, H, C, D, q,
                       lengths, error);
  return hipGetLastError();
}

hipError_t launch_attn_mask(const int64_t* lengths, const int64_t* valid, int64_t B, int64_t q,
                            int64_t kv, float neg, int dtype, void* out, hipStream_t s) {
  const int nt = 256;
  const int64_t n = B * q * kv;
  const dim3 grid((unsigned)((n + nt - 1) / nt));
  if (dtype == SDX_F32) {
    hipLaunchKernelGGL((attn_mask_kernel<float>), grid, dim3(nt), 0, s, lengths, valid, B, q, kv,
                       0.0f, neg, (float*)out);
  } else {
    uint16_t nz;
    if (dtype == SDX_BF16) {
      uint32_t bits;
      memcpy(&bits, &neg, 4);
      nz = (uint16_t)(bits >> 16);
    } else {
      const _Float16 h = (_Float16)neg;
      memcpy(&nz, &h, 2);
    }
    hipLaunchKernelGGL((attn_mask_kernel<uint16_t>), grid, dim3(nt), 0, s, lengths, valid, B, q,
                       kv, (uint16_t)0, nz, (uint16_t*)out);
  }
  return hipGetLastError();
}

hipError_t launch_kv_append_paged(void* pool, int64_t layer_stride_b, int64_t side_stride_b,
                                  const void* staged, int32_t layers, int64_t batch, int64_t q,
                                  int64_t row_bytes, const int32_t* bt, int64_t max_blocks,
                                  int32_t bs, int64_t num_blocks, const int64_t* lengths,
                                  int32_t* error, hipStream_t s) {
  const int nt = 256;
  const int64_t waves = (int64_t)layers * 2 * batch * q;
  const dim3 grid((unsigned)((waves * kWave + nt - 1) / nt));
  hipLaunchKernelGGL(kv_append_paged_kernel, grid, dim3(nt), 0, s, (uint8_t*)pool, layer_stride_b,
                     side_stride_b, (const uint8_t*)staged, layers, batch, q, row_bytes, bt,
                     max_blocks, bs, num_blocks, lengths, error);
  return hipGetLastError();
}

hipError_t launch_slot_mapping(const int32_t* bt, int64_t rows, int64_t max_blocks,
                               const int64_t* positions, int32_t bs, int64_t max_len,
                               int64_t pad_slot, int64_t* clamped, int64_t* slots, hipStream_t s) {
  const int nt = 256;
  hipLaunchKernelGGL(slot_mapping_kernel, dim3((unsigned)((rows + nt - 1) / nt)), dim3(nt), 0, s, bt,
                     rows, max_blocks, positions, bs, max_len, pad_slot, clamped, slots);
  return hipGetLastError();
}

}  // namespace sdx
