// extern "C" entry points of libspecdec_amd.so (declared in include/specdec_amd.h):
// argument checks, workspace carving and kernel launches. No allocation.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include <cstdlib>

#include "sdx_launch.hpp"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* where) {
  if (e == hipSuccess) return SDX_OK;
  return fail(SDX_EHIP, "%s: %s", where, hipGetErrorString(e));
}

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// Bump allocator over the caller's workspace.
struct Carve {
  uint8_t* base;
  size_t used = 0;
  template <typename T>
  T* take(size_t count) {
    T* p = base ? reinterpret_cast<T*>(base + used) : nullptr;
    used += align256(count * sizeof(T));
    return p;
  }
};

bool dtype_ok(int d) { return d == SDX_F32 || d == SDX_BF16 || d == SDX_F16; }
size_t dsize(int d) { return d == SDX_F32 ? 4 : 2; }
bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

struct Switches {
  bool greedy, use_p, use_k;
};
Switches switches(float T, float top_p, int32_t top_k, int64_t V) {
  Switches s;
  s.greedy = !(T > 0.0f);
  s.use_p = top_p > 0.0f && top_p < 1.0f;
  s.use_k = top_k > 0 && (int64_t)top_k < V;
  return s;
}

// Chunking of the id range for the to_probs output kernels: chunks of a
// multiple of 8 ids, at most 2048 ids (one block round) where the chunk count
// allows, at most 128 per row.
void chunking(int64_t V, int64_t* chunk, int* nchunk) {
  *chunk = sdx::kMatChunk;
  *nchunk = (int)((V + sdx::kMatChunk - 1) / sdx::kMatChunk);
}

// Workspace of the transform + draw pipeline over `rows` rows and `njobs` draws.
size_t transform_ws(Carve& c, int64_t rows, int64_t V, int dtype, int64_t njobs,
                    sdx::RowStat** stats, float** tables, float** dense, sdx::SampleJob** jobs,
                    sdx::ChunkRec** recs, uint32_t** counters, uint64_t** rank_acc = nullptr) {
  int64_t rec_ids;
  int nrec;
  sdx::draw_layout(V, &rec_ids, &nrec);
  *stats = c.take<sdx::RowStat>(rows);
  *tables = dtype == SDX_F32 ? nullptr : c.take<float>((size_t)rows * sdx::kTbl);
  *dense = dtype == SDX_F32 ? c.take<float>((size_t)rows * V) : nullptr;
  *jobs = njobs ? c.take<sdx::SampleJob>(njobs) : nullptr;
  *recs = njobs ? c.take<sdx::ChunkRec>((size_t)njobs * nrec) : nullptr;
  *counters = njobs ? c.take<uint32_t>((size_t)njobs) : nullptr;
  if (rank_acc) *rank_acc = njobs ? c.take<uint64_t>((size_t)rows) : nullptr;
  return c.used;
}

// Row statistics of 16-bit rows: bf16 rows stream through the histogram
// kernel, fp16 rows go to the register-resident kernel.
int row_stats16(int dtype, const sdx::RowStatArgs& a, int64_t rows, hipStream_t s) {
  if (dtype == SDX_BF16)
    return hip_status(sdx::launch_rowstream_bf16(a, rows, s), "rowstream_bf16");
  return hip_status(sdx::launch_rowstat16(dtype, a, rows, s), "rowstat16");
}

int check_vocab(int dtype, int64_t V) {
  if (V < 1) return fail(SDX_EINVAL, "vocab must be >= 1");
  if (dtype == SDX_F32 && V > sdx::kF32MaxVocab)
    return fail(SDX_EUNSUPPORTED, "fp32 logits support vocab <= %lld (got %lld)",
                (long long)sdx::kF32MaxVocab, (long long)V);
  const int64_t max16 = dtype == SDX_BF16 ? sdx::kMaxVocabBf16 : sdx::kMaxVocabF16;
  if (dtype != SDX_F32 && V > max16)
    return fail(SDX_EUNSUPPORTED, "%s logits support vocab <= %lld (got %lld)",
                dtype == SDX_BF16 ? "bf16" : "fp16", (long long)max16, (long long)V);
  return SDX_OK;
}

}  // namespace

extern "C" {

const char* sdx_last_error(void) { return g_err; }
int sdx_version(void) { return 2; }

int sdx_workspace_init(void* workspace, size_t bytes, sdx_stream_t stream) {
  if (!workspace && bytes) return fail(SDX_EINVAL, "sdx_workspace_init: null workspace");
  if (((uintptr_t)workspace & 3u) != 0)
    return fail(SDX_EINVAL, "sdx_workspace_init: workspace must be 4-byte aligned");
  return hip_status(sdx::launch_workspace_init(workspace, bytes, (hipStream_t)stream),
                    "workspace_init");
}

// ------------------------------------------------------------------ to_probs
size_t sdx_to_probs_workspace(int64_t rows, int64_t vocab, int dtype) {
  Carve c{nullptr};
  sdx::RowStat* st; float* tb; float* dn; sdx::SampleJob* jb; sdx::ChunkRec* rc; uint32_t* ct;
  // fp32 rows are written straight to the output: no dense scratch
  transform_ws(c, rows, vocab, dtype == SDX_F32 ? SDX_BF16 : dtype, 0, &st, &tb, &dn, &jb, &rc, &ct);
  int64_t chunk;
  int nchunk;
  chunking(vocab, &chunk, &nchunk);
  c.take<uint32_t>((size_t)rows * nchunk);  // group members per chunk
  return dtype == SDX_F32 ? align256(rows * sizeof(sdx::RowStat)) : c.used;
}

int sdx_to_probs(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                 float temperature, float top_p, int32_t top_k, float* probs, int64_t ld_out,
                 void* workspace, size_t workspace_bytes, sdx_stream_t stream) {
  if (!logits || !probs || rows < 0 || ld < vocab || ld_out < vocab || !dtype_ok(dtype))
    return fail(SDX_EINVAL, "sdx_to_probs: bad arguments");
  if (int e = check_vocab(dtype, vocab)) return e;
  if (rows == 0) return SDX_OK;
  const size_t need = sdx_to_probs_workspace(rows, vocab, dtype);
  if (!workspace || workspace_bytes < need)
    return fail(SDX_EWORKSPACE, "sdx_to_probs: workspace %zu < %zu", workspace_bytes, need);
  hipStream_t s = (hipStream_t)stream;
  const Switches sw = switches(temperature, top_p, top_k, vocab);
  Carve c{(uint8_t*)workspace};
  if (dtype == SDX_F32) {
    // the large-vocabulary kernel keeps per-element intermediates in the output
    // rows between its passes, so the output may not overlap the logits
    const uintptr_t l0 = (uintptr_t)logits, l1 = l0 + (uintptr_t)(((rows - 1) * ld + vocab) * 4);
    const uintptr_t p0 = (uintptr_t)probs, p1 = p0 + (uintptr_t)(((rows - 1) * ld_out + vocab) * 4);
    if (l0 < p1 && p0 < l1)
      return fail(SDX_EINVAL, "sdx_to_probs: probs overlap the fp32 logits");
    sdx::F32Args a = {};
    a.base[0] = (const float*)logits; a.nrows[0] = rows; a.ld[0] = ld;
    a.base[1] = a.base[0]; a.nrows[1] = 0; a.ld[1] = ld;
    a.V = vocab; a.ids = nullptr; a.k = 0;
    a.T = temperature; a.top_p = top_p; a.top_k = top_k;
    a.use_p = sw.use_p; a.use_k = sw.use_k; a.greedy = sw.greedy;
    a.out = probs; a.ld_out = ld_out;
    a.stats = c.take<sdx::RowStat>(rows);
    return hip_status(sdx::launch_to_probs_f32(a, rows, s), "to_probs_f32");
  }
  if (!aligned16(logits) || (ld % 8) != 0)
    return fail(SDX_EINVAL, "sdx_to_probs: 16-bit rows must start 16-byte aligned (ld %% 8 == 0)");
  if (sw.greedy) {
    int64_t* am = c.take<int64_t>(rows);
    if (int e = hip_status(sdx::launch_argmax(dtype, logits, rows, vocab, ld, true, am, s), "argmax"))
      return e;
    return hip_status(sdx::launch_onehot(am, rows, vocab, probs, ld_out, s), "onehot");
  }
  sdx::RowStat* st; float* tb; float* dn; sdx::SampleJob* jb; sdx::ChunkRec* rc; uint32_t* ct;
  transform_ws(c, rows, vocab, dtype, 0, &st, &tb, &dn, &jb, &rc, &ct);
  int64_t chunk;
  int nchunk;
  chunking(vocab, &chunk, &nchunk);
  uint32_t* counts = c.take<uint32_t>((size_t)rows * nchunk);
  sdx::RowStatArgs a = {};
  a.base[0] = (const uint16_t*)logits; a.nrows[0] = rows; a.ld[0] = ld;
  a.base[1] = a.base[0]; a.nrows[1] = 0; a.ld[1] = ld;
  a.V = vocab; a.ids = nullptr; a.k = 0;
  a.T = temperature; a.top_p = top_p; a.top_k = top_k;
  a.use_p = sw.use_p; a.use_k = sw.use_k; a.greedy = sw.greedy;
  a.stats = st; a.tables = tb;
  // the output kernel's per-chunk member counts start at zero in every call
  a.zero = counts; a.nzero = rows; a.zero_per_row = nchunk;
  if (int e = row_stats16(dtype, a, rows, s)) return e;
  sdx::RowSource16 src{(const uint16_t*)logits, ld, (const uint16_t*)logits, ld, rows, true};
  return hip_status(sdx::launch_materialize16(dtype, src, st, tb, temperature, rows, vocab, chunk,
                                              nchunk, counts, probs, ld_out, s),
                    "materialize16");
}

// ------------------------------------------------------------------ sample_from_probs
size_t sdx_sample_probs_workspace(int64_t rows, int64_t vocab) {
  Carve c{nullptr};
  c.take<uint64_t>((size_t)rows * sdx::dense_nrec(vocab));  // record masses
  return c.used;
}

__global__ void sdx_jobs_from_u(sdx::SampleJob* jobs, const float* u, int64_t rows,
                                int64_t qsplit, uint32_t* counters) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  if (counters) counters[r] = 0u;
  sdx::SampleJob j;
  j.prow = r;
  j.qrow = qsplit >= 0 ? qsplit + r : -1;
  j.u = u ? u[r] : 0.0f;
  j.pad = 0;
  jobs[r] = j;
}

int sdx_sample_probs(const float* probs, int64_t rows, int64_t vocab, int64_t ld, const float* u,
                     int64_t* ids, void* workspace, size_t workspace_bytes, sdx_stream_t stream) {
  if (!probs || !u || !ids || rows < 0 || vocab < 1 || ld < vocab)
    return fail(SDX_EINVAL, "sdx_sample_probs: bad arguments");
  if (rows == 0) return SDX_OK;
  const size_t need = sdx_sample_probs_workspace(rows, vocab);
  if (!workspace || workspace_bytes < need)
    return fail(SDX_EWORKSPACE, "sdx_sample_probs: workspace %zu < %zu", workspace_bytes, need);
  Carve c{(uint8_t*)workspace};
  sdx::DenseArgs a = {};
  a.p = probs;
  a.ld = ld;
  a.rows = rows;
  a.V = vocab;
  a.nrec = sdx::dense_nrec(vocab);
  a.vec = aligned16(probs) && (ld % 4) == 0;
  a.mass = c.take<uint64_t>((size_t)rows * a.nrec);
  a.u = u;
  a.y = ids;
  return hip_status(sdx::launch_sample_dense(a, (hipStream_t)stream), "sample_dense");
}

// ------------------------------------------------------------------ residual_probs
size_t sdx_residual_probs_workspace(int64_t rows, int64_t vocab) {
  int64_t rec_ids;
  int nrec;
  sdx::draw_layout(vocab, &rec_ids, &nrec);
  Carve c{nullptr};
  c.take<sdx::SampleJob>(rows);
  c.take<sdx::ChunkRec>((size_t)rows * nrec);
  return c.used;
}

int sdx_residual_probs(const float* p, const float* q, int64_t rows, int64_t vocab, int64_t ld,
                       float* out, int64_t ld_out, void* workspace, size_t workspace_bytes,
                       sdx_stream_t stream) {
  if (!p || !q || !out || rows < 0 || vocab < 1 || ld < vocab || ld_out < vocab)
    return fail(SDX_EINVAL, "sdx_residual_probs: bad arguments");
  if (rows == 0) return SDX_OK;
  const size_t need = sdx_residual_probs_workspace(rows, vocab);
  if (!workspace || workspace_bytes < need)
    return fail(SDX_EWORKSPACE, "sdx_residual_probs: workspace %zu < %zu", workspace_bytes, need);
  hipStream_t s = (hipStream_t)stream;
  int64_t rec_ids;
  int nrec;
  sdx::draw_layout(vocab, &rec_ids, &nrec);
  Carve c{(uint8_t*)workspace};
  sdx::SampleJob* jobs = c.take<sdx::SampleJob>(rows);
  sdx::ChunkRec* recs = c.take<sdx::ChunkRec>((size_t)rows * nrec);
  hipLaunchKernelGGL(sdx_jobs_from_u, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, jobs,
                     (const float*)nullptr, rows, rows, (uint32_t*)nullptr);
  if (int e = hip_status(hipGetLastError(), "jobs")) return e;
  const bool vec = aligned16(p) && aligned16(q) && (ld % 4) == 0;
  sdx::RowSourceF32 src{p, ld, q, ld, rows, vec};
  if (int e = hip_status(sdx::launch_chunk_mass_probs(src, jobs, rows, vocab, recs, s),
                         "chunk_mass"))
    return e;
  sdx::ResidualNormArgs a{p, q, ld, vocab, rec_ids, nrec, recs, out, ld_out};
  return hip_status(sdx::launch_residual_norm(a, rows, s), "residual_norm");
}

// ------------------------------------------------------------------ gather_prob
int sdx_gather_prob(const float* probs, int64_t rows, int64_t vocab, int64_t ld, const int64_t* ids,
                    float* out, sdx_stream_t stream) {
  if (!probs || !ids || !out || rows < 0 || vocab < 1 || ld < vocab)
    return fail(SDX_EINVAL, "sdx_gather_prob: bad arguments");
  if (rows == 0) return SDX_OK;
  return hip_status(sdx::launch_gather(probs, rows, vocab, ld, ids, out, (hipStream_t)stream),
                    "gather");
}

// ------------------------------------------------------------------ allocation-free verify
// sdx_verify_noalloc runs sdx_verify on a library-owned device array instead of
// a caller workspace. Each GPU the library runs on holds its own copy of the
// array until the process ends. In host code `scratch` names a host-side
// stand-in, not device memory: the device address comes from
// hipGetSymbolAddress, once per device (with that device current), and only
// that address is ever handed to kernels.
namespace {
constexpr size_t kScratchBytes = (size_t)24 << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch address; on a device's first use, looked up and
// prepared (zero-filled, header word written) by a kernel queued on `s`.
int scratch_for_current_device(hipStream_t s, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(SDX_EHIP, "sdx_verify_noalloc: no current device (or device index >= %d)",
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    // preparing the scratch queues a kernel: under graph capture it would be
    // recorded into the graph instead of run, and every replay would redo it
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (int e = hip_status(hipStreamIsCapturing(s, &cs), "sdx_verify_noalloc: hipStreamIsCapturing"))
      return e;
    if (cs != hipStreamCaptureStatusNone)
      return fail(SDX_EINVAL,
                  "sdx_verify_noalloc: the first call on device %d is being captured; make one "
                  "call outside graph capture first (it prepares the device's scratch)", dev);
    void* p = nullptr;
    if (int e = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                           "sdx_verify_noalloc: hipGetSymbolAddress"))
      return e;
    if (!p) return fail(SDX_EHIP, "sdx_verify_noalloc: scratch has no device address");
    if (int e = hip_status(sdx::launch_workspace_init(p, kScratchBytes, s),
                           "sdx_verify_noalloc: scratch init"))
      return e;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SDX_OK;
}
}  // namespace

// ------------------------------------------------------------------ verify
static size_t verify_split_bytes(int dtype, int64_t rows, int64_t ntgt, int64_t vocab) {
  if (dtype != SDX_BF16) return 0;
  const size_t a = sdx::rowstream_split_bytes(rows, vocab), b = sdx::rowstream_split_bytes(ntgt, vocab);
  return a > b ? a : b;
}

// Byte offsets of the row statistics and tables in a draft-step workspace (the
// carve of sdx_draft_step: header, then RowStat[batch], then tables).
static void draft_ws_offsets(int64_t batch, size_t* st_off, size_t* tb_off) {
  Carve c{nullptr};
  c.take<uint8_t>(sdx::kWsHeaderBytes);
  *st_off = c.used;
  c.take<sdx::RowStat>(batch);
  *tb_off = c.used;
}

static size_t draft_ws_x_offset(int64_t batch, int64_t vocab, int dtype);

// The signature a bf16 draft step leaves in its workspace header (the words its
// epilogue writes): the verify that takes its statistics over compares it.
static void draft_sig(int64_t batch, int64_t vocab, float T, float top_p, int32_t top_k,
                      uint32_t* sig) {
  const Switches sw = switches(T, top_p, top_k, vocab);
  const float tp = sw.use_p ? top_p : 1.0f;
  const int32_t tk = sw.use_k ? top_k : 0;
  uint32_t tb, pb;
  memcpy(&tb, &T, 4);
  memcpy(&pb, &tp, 4);
  sig[0] = sdx::kDraftSig; sig[1] = (uint32_t)batch; sig[2] = (uint32_t)vocab;
  sig[3] = tb; sig[4] = pb; sig[5] = (uint32_t)tk;
}

// verify workspace for ntgt target and ndrf draft rows (per-row k adds the
// target row map and the bad-row bytes)
static size_t verify_ws_bytes(int64_t batch, int64_t ntgt, int64_t ndrf, int64_t vocab, int dtype,
                              bool ragged) {
  Carve c{nullptr};
  sdx::RowStat* st; float* tb; float* dn; sdx::SampleJob* jb; sdx::ChunkRec* rc; uint32_t* ct;
  uint64_t* ra;
  const int64_t rows = ntgt + ndrf;
  c.take<uint8_t>(sdx::kWsHeaderBytes);  // magic word + split-row counters, fixed offsets
  transform_ws(c, rows, vocab, dtype, batch, &st, &tb, &dn, &jb, &rc, &ct, &ra);
  c.take<int64_t>(ntgt);  // greedy argmax
  // part histograms of rows split over blocks (all rows, or the target rows alone
  // when the draft rows' statistics come from the draft steps)
  c.take<uint8_t>(verify_split_bytes(dtype, rows, ntgt, vocab));
  if (ragged) {
    c.take<int64_t>(ntgt);
    c.take<uint8_t>(batch);
    c.take<int32_t>(rows);  // the rows in batch-row order (fused kernel)
    c.take<int32_t>(rows);  // each row's batch row
  }
  if (dtype == SDX_F32) c.take<uint32_t>((size_t)rows * sdx::f32_tie_words(vocab));  // tie bits
  return c.used;
}

// The fused verify kernel (row statistics and draw in one launch) serves bf16
// logits, at one k or per-row k (2 k_max + 1 <= 64, batch <= 1024);
// SDX_VERIFY_FUSED=0 in the environment selects the two-launch path instead.
static bool fused_enabled() {
  static const bool on = [] {
    const char* e = getenv("SDX_VERIFY_FUSED");
    return !(e && e[0] == '0');
  }();
  return on;
}

size_t sdx_verify_workspace(int64_t batch, int32_t k, int64_t vocab, int dtype) {
  return verify_ws_bytes(batch, batch * ((int64_t)k + 1), batch * (int64_t)k, vocab, dtype, false);
}

size_t sdx_verify_ragged_workspace(int64_t batch, int64_t target_rows, int64_t vocab, int dtype) {
  if (batch < 0 || target_rows < batch) return 0;
  return verify_ws_bytes(batch, target_rows, target_rows - batch, vocab, dtype, true);
}

static int verify_impl(const void* target_logits, const void* draft_logits, int dtype,
                       int64_t batch, int32_t k, int64_t vocab, const int64_t* draft_ids,
                       const float* u_accept, const float* u_final, const uint8_t* active,
                       float temperature, float top_p, int32_t top_k, int64_t* n_acc, int64_t* y,
                       uint8_t* flags, void* workspace, size_t workspace_bytes,
                       sdx_stream_t stream, bool stats_only, const int64_t* cu_k = nullptr,
                       int64_t target_rows = 0, const void* const* draft_ws = nullptr);

int sdx_verify(const void* target_logits, const void* draft_logits, int dtype, int64_t batch,
               int32_t k, int64_t vocab, const int64_t* draft_ids, const float* u_accept,
               const float* u_final, const uint8_t* active, float temperature, float top_p,
               int32_t top_k, int64_t* n_acc, int64_t* y, uint8_t* flags, void* workspace,
               size_t workspace_bytes, sdx_stream_t stream) {
  if (!n_acc || !y || !flags) return fail(SDX_EINVAL, "sdx_verify: bad arguments");
  return verify_impl(target_logits, draft_logits, dtype, batch, k, vocab, draft_ids, u_accept,
                     u_final, active, temperature, top_p, top_k, n_acc, y, flags, workspace,
                     workspace_bytes, stream, false);
}

int sdx_verify_drafted(const void* target_logits, const void* draft_logits, int dtype,
                       int64_t batch, int32_t k, int64_t vocab, const int64_t* draft_ids,
                       const float* u_accept, const float* u_final, const uint8_t* active,
                       float temperature, float top_p, int32_t top_k,
                       const void* const* draft_workspaces, int64_t* n_acc, int64_t* y,
                       uint8_t* flags, void* workspace, size_t workspace_bytes,
                       sdx_stream_t stream) {
  if (!n_acc || !y || !flags || !draft_workspaces || k < 1)
    return fail(SDX_EINVAL, "sdx_verify_drafted: bad arguments");
  const bool takes_stats = dtype == SDX_BF16 && temperature > 0.0f && k <= sdx::kMaxDraftK;
  if (takes_stats)
    for (int i = 0; i < k; ++i)
      if (!draft_workspaces[i]) return fail(SDX_EINVAL, "sdx_verify_drafted: null draft workspace");
  return verify_impl(target_logits, draft_logits, dtype, batch, k, vocab, draft_ids, u_accept,
                     u_final, active, temperature, top_p, top_k, n_acc, y, flags, workspace,
                     workspace_bytes, stream, false, nullptr, 0,
                     takes_stats ? draft_workspaces : nullptr);
}

int sdx_verify_ragged(const void* target_logits, const void* draft_logits, int dtype,
                      int64_t batch, int32_t k_max, int64_t target_rows, int64_t vocab,
                      const int64_t* cu_k, const int64_t* draft_ids, const float* u_accept,
                      const float* u_final, const uint8_t* active, float temperature,
                      float top_p, int32_t top_k, int64_t* n_acc, int64_t* y, uint8_t* flags,
                      void* workspace, size_t workspace_bytes, sdx_stream_t stream) {
  if (!n_acc || !y || !flags || !cu_k || target_rows < batch || k_max < 1)
    return fail(SDX_EINVAL, "sdx_verify_ragged: bad arguments");
  if (target_rows - batch > batch * (int64_t)k_max)
    return fail(SDX_EINVAL, "sdx_verify_ragged: %lld draft rows exceed batch * k_max",
                (long long)(target_rows - batch));
  return verify_impl(target_logits, draft_logits, dtype, batch, k_max, vocab, draft_ids, u_accept,
                     u_final, active, temperature, top_p, top_k, n_acc, y, flags, workspace,
                     workspace_bytes, stream, false, cu_k, target_rows);
}

int sdx_verify_stats(const void* target_logits, const void* draft_logits, int dtype,
                     int64_t batch, int32_t k, int64_t vocab, const int64_t* draft_ids,
                     float temperature, float top_p, int32_t top_k, void* workspace,
                     size_t workspace_bytes, sdx_stream_t stream) {
  static const float dummy_u = 0.0f;
  if (!(temperature > 0.0f))
    return fail(SDX_EINVAL, "sdx_verify_stats: temperature must be > 0 (greedy has no phase 1)");
  return verify_impl(target_logits, draft_logits, dtype, batch, k, vocab, draft_ids, &dummy_u,
                     &dummy_u, nullptr, temperature, top_p, top_k, nullptr, nullptr, nullptr,
                     workspace, workspace_bytes, stream, true);
}

static int verify_impl(const void* target_logits, const void* draft_logits, int dtype,
                       int64_t batch, int32_t k, int64_t vocab, const int64_t* draft_ids,
                       const float* u_accept, const float* u_final, const uint8_t* active,
                       float temperature, float top_p, int32_t top_k, int64_t* n_acc, int64_t* y,
                       uint8_t* flags, void* workspace, size_t workspace_bytes,
                       sdx_stream_t stream, bool stats_only, const int64_t* cu_k,
                       int64_t target_rows, const void* const* draft_ws) {
  if (!target_logits || (!draft_ids && !stats_only) || !u_accept || !u_final || batch < 0 ||
      k < 1 || !dtype_ok(dtype))
    return fail(SDX_EINVAL, "sdx_verify: bad arguments");
  if (int e = check_vocab(dtype, vocab)) return e;
  if (batch == 0) return SDX_OK;
  // per-row k: target rows [sum (k_b + 1)], draft rows [sum k_b]
  const int64_t ntgt = cu_k ? target_rows : batch * ((int64_t)k + 1);
  const int64_t ndrf = cu_k ? target_rows - batch : batch * (int64_t)k;
  const size_t need = verify_ws_bytes(batch, ntgt, ndrf, vocab, dtype, cu_k != nullptr);
  if (!workspace || workspace_bytes < need)
    return fail(SDX_EWORKSPACE, "sdx_verify: workspace %zu < %zu", workspace_bytes, need);
  hipStream_t s = (hipStream_t)stream;
  const Switches sw = switches(temperature, top_p, top_k, vocab);
  Carve c{(uint8_t*)workspace};
  sdx::RowStat* st; float* tb; float* dn; sdx::SampleJob* jobs; sdx::ChunkRec* recs;
  uint32_t* counters;
  uint64_t* rank_acc;
  const int64_t rows = ntgt + ndrf;
  uint32_t* header = c.take<uint32_t>(sdx::kWsHeaderBytes / 4);
  transform_ws(c, rows, vocab, dtype, batch, &st, &tb, &dn, &jobs, &recs, &counters, &rank_acc);
  int64_t* am = c.take<int64_t>(ntgt);
  const size_t split_bytes = verify_split_bytes(dtype, rows, ntgt, vocab);
  uint8_t* split_ws = c.take<uint8_t>(split_bytes);
  int64_t* tgt_idx = nullptr;
  uint8_t* bad = nullptr;
  int32_t* order = nullptr;
  int32_t* rowjob = nullptr;
  if (cu_k) {
    tgt_idx = c.take<int64_t>(ntgt);
    bad = c.take<uint8_t>(batch);
    order = c.take<int32_t>(rows);
    rowjob = c.take<int32_t>(rows);
    if (int e = hip_status(sdx::launch_ragged_rows(cu_k, batch, k, ntgt, ndrf, tgt_idx, bad, s,
                                                   order, rowjob),
                           "ragged_rows"))
      return e;
  }
  uint32_t* tie_bits =
      dtype == SDX_F32 ? c.take<uint32_t>((size_t)rows * sdx::f32_tie_words(vocab)) : nullptr;

  if (sw.greedy) {
    // one-hot p: only the target argmax matters (see sdx_verify_greedy)
    const bool vec = aligned16(target_logits) && (vocab % (dtype == SDX_F32 ? 4 : 8)) == 0;
    if (int e = hip_status(sdx::launch_argmax(dtype, target_logits, ntgt, vocab, vocab, vec, am, s),
                           "argmax"))
      return e;
    return hip_status(sdx::launch_greedy_accept(am, batch, k, draft_ids, u_accept, active, n_acc,
                                                y, flags, s, cu_k, bad),
                      "greedy_accept");
  }
  if (!draft_logits) return fail(SDX_EINVAL, "sdx_verify: draft_logits required when T > 0");
  if (dtype == SDX_F32) {
    sdx::F32Args a = {};
    a.base[0] = (const float*)target_logits; a.nrows[0] = ntgt; a.ld[0] = vocab;
    a.base[1] = (const float*)draft_logits; a.nrows[1] = ndrf; a.ld[1] = vocab;
    a.V = vocab; a.ids = draft_ids; a.k = k; a.tgt_idx = tgt_idx;
    a.T = temperature; a.top_p = top_p; a.top_k = top_k;
    a.use_p = sw.use_p; a.use_k = sw.use_k; a.greedy = 0;
    a.out = dn; a.ld_out = vocab; a.stats = st;
    a.zero = counters; a.nzero = batch;
    a.tie_bits = tie_bits;
    a.tie_ld = sdx::f32_tie_words(vocab);
    if (int e = hip_status(sdx::launch_to_probs_f32(a, rows, s), "to_probs_f32")) return e;
  } else {
    if (!aligned16(target_logits) || !aligned16(draft_logits) || (vocab % 8) != 0)
      return fail(SDX_EINVAL,
                  "sdx_verify: 16-bit logits must be 16-byte aligned with vocab %% 8 == 0");
    sdx::RowStatArgs a = {};
    a.base[0] = (const uint16_t*)target_logits; a.nrows[0] = ntgt; a.ld[0] = vocab;
    a.base[1] = (const uint16_t*)draft_logits; a.nrows[1] = ndrf; a.ld[1] = vocab;
    a.V = vocab; a.ids = draft_ids; a.k = k; a.tgt_idx = tgt_idx;
    a.T = temperature; a.top_p = top_p; a.top_k = top_k;
    a.use_p = sw.use_p; a.use_k = sw.use_k; a.greedy = 0;
    a.stats = st; a.tables = tb;
    a.zero = counters; a.nzero = batch;
    a.rank_acc = dtype == SDX_BF16 ? rank_acc : nullptr;
    a.split_ws = split_ws;
    a.split_bytes = split_bytes;
    a.ws_header = header;
    int64_t stream_rows = rows;
    if (draft_ws) {
      // the draft rows' statistics from the draft steps' workspaces: only the
      // target rows stream, then the draw of the two-launch form. (The fused
      // kernel with target rows alone was measured slower: at 320 rows its row
      // workgroups stream one whole row each at the per-workgroup rate.)
      sdx::DraftGatherArgs g = {};
      for (int i = 0; i < k; ++i) g.ws[i] = (const uint8_t*)draft_ws[i];
      g.k = k; g.B = batch; g.V = vocab;
      draft_ws_offsets(batch, &g.st_off, &g.tb_off);
      g.x_off = draft_ws_x_offset(batch, vocab, SDX_BF16);
      g.stats = st; g.tables = tb; g.ntgt = ntgt;
      g.dlog = (const uint16_t*)draft_logits; g.ld = vocab; g.ids = draft_ids;
      draft_sig(batch, vocab, temperature, top_p, top_k, g.sig);
      g.T = temperature;
      if (int e = hip_status(sdx::launch_draft_gather(g, s), "draft_gather")) return e;
      stream_rows = ntgt;
    } else if (dtype == SDX_BF16 && !stats_only && 2 * (int64_t)k + 1 <= 64 &&
               batch <= sdx::kWsFusedMaxJobs && fused_enabled()) {
      // one launch: the draw of each batch row starts as soon as its rows are in.
      // Its counters sit at fixed header offsets (every call leaves them at zero),
      // so a workspace reused across shapes never hands it stale counts. Per-row
      // k takes the rows in the batch-row order ragged_rows_kernel listed.
      sdx::AcceptArgs aa{st,    batch, k,         u_accept, u_final, active, jobs,
                         n_acc, flags, draft_ids, cu_k,     bad,     ntgt};
      sdx::RowSource16 src{(const uint16_t*)target_logits, vocab, (const uint16_t*)draft_logits,
                           vocab, ntgt, true};
      a.jm_order = order;
      return hip_status(
          sdx::launch_verify_fused_bf16(a, rows, src, aa, batch, vocab, temperature, recs,
                                        sdx::fused_draw_words(header),
                                        sdx::fused_job_words(header), y, s, rowjob),
          "verify_fused_bf16");
    }
    if (int e = row_stats16(dtype, a, stream_rows, s)) return e;
    // bf16: drafted tokens the row kernel could not rank (a tie group of several
    // values) are ranked by the draw's accept chain; the statistics-only call
    // (and drafts too long for the one-wave chain) complete them with the rank kernel
    if (dtype == SDX_BF16 && (stats_only || 2 * (int64_t)k + 1 > 64))
      if (int e = hip_status(sdx::launch_rank_bf16(a, rows, s), "rank_bf16")) return e;
  }
  if (stats_only) return SDX_OK;
  sdx::AcceptArgs aa{st,    batch, k,         u_accept, u_final, active, jobs,
                     n_acc, flags, draft_ids, cu_k,     bad,     ntgt};
  if (dtype == SDX_F32) {
    sdx::RowSourceF32 src{dn, vocab, dn, vocab, rows, (vocab % 4) == 0};
    return hip_status(sdx::launch_draw_probs(src, &aa, jobs, batch, vocab, recs,
                                             counters, y, s, tie_bits),
                      "draw_probs");
  }
  sdx::RowSource16 src{(const uint16_t*)target_logits, vocab, (const uint16_t*)draft_logits, vocab,
                       ntgt, true};
  return hip_status(sdx::launch_draw16(dtype, src, st, tb, temperature, &aa, jobs, batch, vocab,
                                       recs, counters, y, s),
                    "draw16");
}

int sdx_verify_counter_layout(int64_t batch, int64_t target_rows, int32_t k, int64_t vocab,
                              int dtype, int32_t cus, int64_t* ranges, int32_t max_ranges) {
  if (batch < 1 || k < 1 || vocab < 1 || cus < 0 || !dtype_ok(dtype) || !ranges ||
      max_ranges < 4)
    return fail(SDX_EINVAL, "sdx_verify_counter_layout: bad arguments");
  const bool ragged = target_rows > 0;
  const int64_t ntgt = ragged ? target_rows : batch * ((int64_t)k + 1);
  const int64_t ndrf = ragged ? target_rows - batch : batch * (int64_t)k;
  const int64_t rows = ntgt + ndrf;
  // the carve of verify_impl: the header comes first
  Carve c{(uint8_t*)nullptr};
  c.take<uint8_t>(0);
  const size_t header_at = c.used;
  c.take<uint32_t>(sdx::kWsHeaderBytes / 4);
  uint32_t* const h = reinterpret_cast<uint32_t*>((uintptr_t)4096);  // a stand-in base
  auto off = [&](const uint32_t* p) {
    return (int64_t)header_at + (int64_t)((const uint8_t*)p - (const uint8_t*)h);
  };
  int n = 0;
  int64_t nsplit = dtype == SDX_BF16 ? sdx::rowstream_split_rows(rows, vocab, cus) : 0;
  if (dtype == SDX_BF16 && !ragged) {  // sdx_verify_drafted streams the target rows alone
    const int64_t n2 = sdx::rowstream_split_rows(ntgt, vocab, cus);
    nsplit = n2 > nsplit ? n2 : nsplit;
  }
  ranges[2 * n] = off(sdx::split_counter_words(h));
  ranges[2 * n + 1] = off(sdx::split_counter_words(h) + nsplit);
  ++n;
  const bool fused = dtype == SDX_BF16 && 2 * (int64_t)k + 1 <= 64 && batch <= sdx::kWsFusedMaxJobs;
  ranges[2 * n] = off(sdx::fused_job_words(h));
  ranges[2 * n + 1] = off(sdx::fused_job_words(h) + (fused ? batch : 0));
  ++n;
  ranges[2 * n] = off(sdx::fused_draw_words(h));
  ranges[2 * n + 1] = off(sdx::fused_draw_words(h) + (fused ? batch : 0));
  ++n;
  ranges[2 * n] = (int64_t)header_at;
  ranges[2 * n + 1] = (int64_t)(header_at + sdx::kWsHeaderBytes);
  ++n;
  return n;
}

int sdx_verify_noalloc(const void* target_logits, const void* draft_logits, int dtype,
                       int64_t batch, int32_t k, int64_t vocab, const int64_t* draft_ids,
                       const float* u_accept, const float* u_final, const uint8_t* active,
                       float temperature, float top_p, int32_t top_k, int64_t* n_acc, int64_t* y,
                       uint8_t* flags, sdx_stream_t stream) {
  if (batch < 0 || k < 1 || !dtype_ok(dtype))
    return fail(SDX_EINVAL, "sdx_verify_noalloc: bad arguments");
  const size_t need = sdx_verify_workspace(batch, k, vocab, dtype);
  if (need > kScratchBytes)
    return fail(SDX_EWORKSPACE,
                "sdx_verify_noalloc: batch %lld, k %d, vocab %lld need %zu bytes of scratch, more "
                "than its %zu; use sdx_verify with a workspace",
                (long long)batch, k, (long long)vocab, need, kScratchBytes);
  void* ws = nullptr;
  if (int e = scratch_for_current_device((hipStream_t)stream, &ws)) return e;
  // a draw whose wait gave up in an earlier call left the header marked: prepare
  // it again (a one-block kernel that returns at once when the header is intact)
  if (int e = hip_status(sdx::launch_workspace_rearm(ws, (hipStream_t)stream),
                         "sdx_verify_noalloc: scratch re-arm"))
    return e;
  return sdx_verify(target_logits, draft_logits, dtype, batch, k, vocab, draft_ids, u_accept,
                    u_final, active, temperature, top_p, top_k, n_acc, y, flags, ws,
                    kScratchBytes, stream);
}

size_t sdx_verify_greedy_workspace(int64_t batch, int32_t k) {
  return align256((size_t)batch * ((size_t)k + 1) * sizeof(int64_t));
}

int sdx_verify_greedy(const void* target_logits, int dtype, int64_t batch, int32_t k,
                      int64_t vocab, const int64_t* draft_ids, const float* u_accept,
                      const uint8_t* active, int64_t* n_acc, int64_t* y, uint8_t* flags,
                      void* workspace, size_t workspace_bytes, sdx_stream_t stream) {
  if (!target_logits || !draft_ids || !n_acc || !y || !flags || batch < 0 || k < 1 ||
      vocab < 1 || !dtype_ok(dtype))
    return fail(SDX_EINVAL, "sdx_verify_greedy: bad arguments");
  if (batch == 0) return SDX_OK;
  const size_t need = sdx_verify_greedy_workspace(batch, k);
  if (!workspace || workspace_bytes < need)
    return fail(SDX_EWORKSPACE, "sdx_verify_greedy: workspace %zu < %zu", workspace_bytes, need);
  hipStream_t s = (hipStream_t)stream;
  int64_t* am = (int64_t*)workspace;
  const int64_t ntgt = batch * ((int64_t)k + 1);
  const bool vec = aligned16(target_logits) && (vocab % (dtype == SDX_F32 ? 4 : 8)) == 0;
  if (int e = hip_status(sdx::launch_argmax(dtype, target_logits, ntgt, vocab, vocab, vec, am, s),
                         "argmax"))
    return e;
  return hip_status(
      sdx::launch_greedy_accept(am, batch, k, draft_ids, u_accept, active, n_acc, y, flags, s),
      "greedy_accept");
}

// ------------------------------------------------------------------ draft step
// workspace: header, the row statistics / tables (dense probabilities for fp32),
// the draws' jobs, records and counters, the split parts of bf16 rows
static size_t draft_ws_bytes(int64_t batch, int64_t vocab, int dtype) {
  Carve c{nullptr};
  sdx::RowStat* st; float* tb; float* dn; sdx::SampleJob* jb; sdx::ChunkRec* rc; uint32_t* ct;
  c.take<uint8_t>(sdx::kWsHeaderBytes);
  transform_ws(c, batch, vocab, dtype, batch, &st, &tb, &dn, &jb, &rc, &ct);
  c.take<uint8_t>(dtype == SDX_BF16 ? sdx::rowstream_split_bytes(batch, vocab) : 0);
  c.take<int64_t>(batch);  // the drawn ids, kept for sdx_verify_drafted
  return c.used;
}

// Byte offset of the drawn ids in a draft-step workspace (its last piece).
static size_t draft_ws_x_offset(int64_t batch, int64_t vocab, int dtype) {
  return draft_ws_bytes(batch, vocab, dtype) - align256((size_t)batch * sizeof(int64_t));
}

size_t sdx_draft_step_workspace(int64_t batch, int64_t vocab, int dtype) {
  if (batch < 0 || vocab < 1 || !dtype_ok(dtype)) return 0;
  return draft_ws_bytes(batch, vocab, dtype);
}

int sdx_draft_step(const void* logits, int dtype, int64_t batch, int64_t vocab, int64_t ld,
                   float temperature, float top_p, int32_t top_k, const float* u, int64_t* x,
                   float* qx, float* conf, float tau, int32_t step, int32_t min_k, int32_t* stop,
                   void* workspace, size_t workspace_bytes, sdx_stream_t stream) {
  if (!logits || !x || batch < 0 || ld < vocab || !dtype_ok(dtype))
    return fail(SDX_EINVAL, "sdx_draft_step: bad arguments");
  const Switches sw = switches(temperature, top_p, top_k, vocab);
  if (!sw.greedy) {  // the argmax of T <= 0 takes any vocabulary
    if (int e = check_vocab(dtype, vocab)) return e;
    if (!u) return fail(SDX_EINVAL, "sdx_draft_step: uniforms required when T > 0");
  }
  if (batch == 0) return SDX_OK;
  const size_t need = draft_ws_bytes(batch, vocab, dtype);
  if (!workspace || workspace_bytes < need)
    return fail(SDX_EWORKSPACE, "sdx_draft_step: workspace %zu < %zu", workspace_bytes, need);
  hipStream_t s = (hipStream_t)stream;
  Carve c{(uint8_t*)workspace};
  uint32_t* header = c.take<uint32_t>(sdx::kWsHeaderBytes / 4);
  sdx::RowStat* st; float* tb; float* dn; sdx::SampleJob* jobs; sdx::ChunkRec* recs;
  uint32_t* counters;
  transform_ws(c, batch, vocab, dtype, batch, &st, &tb, &dn, &jobs, &recs, &counters);
  const size_t split_bytes = dtype == SDX_BF16 ? sdx::rowstream_split_bytes(batch, vocab) : 0;
  uint8_t* split_ws = c.take<uint8_t>(split_bytes);
  sdx::DraftEpiArgs e = {};
  e.B = batch; e.V = vocab; e.x = x; e.qx = qx; e.conf = conf; e.tau = tau;
  e.step = step; e.min_k = min_k; e.stop = stop; e.T = temperature;
  if (sw.greedy) {  // sampling.py:43-48: one-hot at the first maximum
    const bool vec = aligned16(logits) && (ld % (dtype == SDX_F32 ? 4 : 8)) == 0;
    if (int r = hip_status(sdx::launch_argmax(dtype, logits, batch, vocab, ld, vec, x, s), "argmax"))
      return r;
    e.greedy = true;
    return hip_status(sdx::launch_draft_epilogue(e, s), "draft_epilogue");
  }
  if (dtype == SDX_F32) {
    hipLaunchKernelGGL(sdx_jobs_from_u, dim3((unsigned)((batch + 255) / 256)), dim3(256), 0, s,
                       jobs, u, batch, (int64_t)-1, counters);
    if (int r = hip_status(hipGetLastError(), "jobs")) return r;
    sdx::F32Args a = {};
    a.base[0] = (const float*)logits; a.nrows[0] = batch; a.ld[0] = ld;
    a.base[1] = a.base[0]; a.nrows[1] = 0; a.ld[1] = ld;
    a.V = vocab; a.ids = nullptr; a.k = 0;
    a.T = temperature; a.top_p = top_p; a.top_k = top_k;
    a.use_p = sw.use_p; a.use_k = sw.use_k; a.greedy = 0;
    a.out = dn; a.ld_out = vocab; a.stats = st;
    if (int r = hip_status(sdx::launch_to_probs_f32(a, batch, s), "to_probs_f32")) return r;
    sdx::RowSourceF32 src{dn, vocab, dn, vocab, batch, (vocab % 4) == 0};
    if (int r = hip_status(sdx::launch_draw_probs(src, nullptr, jobs, batch, vocab, recs, counters,
                                                  x, s),
                           "draw_probs"))
      return r;
    e.probs = dn;
    e.ldp = vocab;
    return hip_status(sdx::launch_draft_epilogue(e, s), "draft_epilogue");
  }
  if (!aligned16(logits) || (ld % 8) != 0 || (vocab % 8) != 0)
    return fail(SDX_EINVAL,
                "sdx_draft_step: 16-bit rows must start 16-byte aligned, ld %% 8 == 0, vocab %% 8 == 0");
  sdx::RowStatArgs a = {};
  a.base[0] = (const uint16_t*)logits; a.nrows[0] = batch; a.ld[0] = ld;
  a.base[1] = a.base[0]; a.nrows[1] = 0; a.ld[1] = ld;
  a.V = vocab; a.ids = nullptr; a.k = 0;
  a.T = temperature; a.top_p = top_p; a.top_k = top_k;
  a.use_p = sw.use_p; a.use_k = sw.use_k; a.greedy = 0;
  a.stats = st; a.tables = tb;
  a.split_ws = split_ws; a.split_bytes = split_bytes; a.ws_header = header;
  sdx::RowSource16 src{(const uint16_t*)logits, ld, (const uint16_t*)logits, ld, batch, true};
  e.fmt = dtype;
  e.codes = (const uint16_t*)logits;
  e.ld = ld;
  e.stats = st;
  e.tables = tb;
  if (dtype == SDX_BF16) {  // what sdx_verify_drafted checks before it takes these statistics
    e.xcopy = (int64_t*)((uint8_t*)workspace + draft_ws_x_offset(batch, vocab, dtype));
    uint32_t sig[sdx::kDraftSigWords];
    draft_sig(batch, vocab, temperature, top_p, top_k, sig);
    float tp;
    memcpy(&tp, &sig[4], 4);
    e.sig = header + sdx::kWsDraftSigWord;
    e.top_p = tp;
    e.top_k = (int32_t)sig[5];
  }
  if (dtype == SDX_BF16 && batch <= sdx::kWsFusedMaxJobs && fused_enabled()) {
    // one launch: the fused verify at k = 0 (one row per batch row, no accept
    // test: its bonus draw from the row is the draft's draw on u), whose row
    // counters sit in the workspace header like the verify's, with the
    // epilogue done by the blocks that complete the draws
    sdx::AcceptArgs aa{st,      batch,   0,       u,       u,       nullptr, jobs,
                       nullptr, nullptr, nullptr, nullptr, nullptr, batch};
    return hip_status(sdx::launch_draft_fused_bf16(a, src, aa, batch, vocab, temperature, recs,
                                                   sdx::fused_draw_words(header),
                                                   sdx::fused_job_words(header), x, e,
                                                   header + sdx::kWsDraftDoneWord, s),
                      "draft_fused_bf16");
  } else {
    if (int r = row_stats16(dtype, a, batch, s)) return r;
    hipLaunchKernelGGL(sdx_jobs_from_u, dim3((unsigned)((batch + 255) / 256)), dim3(256), 0, s,
                       jobs, u, batch, (int64_t)-1, counters);
    if (int r = hip_status(hipGetLastError(), "jobs")) return r;
    if (int r = hip_status(sdx::launch_draw_rows16(dtype, src, st, tb, temperature, jobs, batch,
                                                   vocab, recs, counters, x, s),
                           "draw_rows16"))
      return r;
  }
  return hip_status(sdx::launch_draft_epilogue(e, s), "draft_epilogue");
}

// ------------------------------------------------------------------ round bookkeeping
int sdx_round_commit(int64_t batch, int32_t k, const int64_t* cu_k, const int64_t* n_acc,
                     const int64_t* y, const int64_t* draft_ids, uint8_t* done,
                     int64_t* out_tokens, int64_t* out_len, int64_t max_new,
                     const int64_t* eos_ids, int32_t n_eos, int64_t* lengths0, int64_t* lengths1,
                     int64_t* pending, const uint8_t* flags, int32_t* error,
                     sdx_stream_t stream) {
  if (batch < 0 || !n_acc || !y || !done || !out_tokens || !out_len || max_new < 1 ||
      n_eos < 0 || (n_eos > 0 && !eos_ids) || (!cu_k && k < 0) || (!draft_ids && (cu_k || k > 0)))
    return fail(SDX_EINVAL, "sdx_round_commit: bad arguments");
  if (batch == 0) return SDX_OK;
  sdx::RoundCommitArgs a{batch, k,       cu_k,   n_acc, y,        draft_ids, done, out_tokens,
                         out_len, max_new, eos_ids, n_eos, lengths0, lengths1, pending,
                         flags,   error};
  return hip_status(sdx::launch_round_commit(a, (hipStream_t)stream), "round_commit");
}

int sdx_controller_update(sdx_ctrl_state* state, int64_t nstate, const int64_t* n_acc,
                          int64_t batch, const int64_t* k_used, double beta, int32_t k_max,
                          int32_t k_init, int32_t warmup, int32_t extra_fwd, const float* c_obs,
                          int64_t* k_next, int64_t* cu_k, sdx_stream_t stream) {
  if (!state || !n_acc || !k_used || batch < 1 || k_max < 1 || k_init < 1 ||
      !(nstate == 1 || nstate == batch) || !(beta > 0.0 && beta <= 1.0))
    return fail(SDX_EINVAL, "sdx_controller_update: bad arguments");
  if (cu_k && nstate != batch)
    return fail(SDX_EINVAL, "sdx_controller_update: cu_k needs one state per row");
  sdx::CtrlArgs a{reinterpret_cast<sdx::CtrlState*>(state), nstate, n_acc, batch, k_used, beta,
                  k_max, k_init, warmup, extra_fwd, c_obs, k_next, cu_k};
  return hip_status(sdx::launch_controller(a, (hipStream_t)stream), "controller");
}

// ------------------------------------------------------------------ proposer
int sdx_argmax(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
               int64_t* ids, sdx_stream_t stream) {
  if (!logits || !ids || rows < 0 || vocab < 1 || ld < vocab || !dtype_ok(dtype))
    return fail(SDX_EINVAL, "sdx_argmax: bad arguments");
  if (rows == 0) return SDX_OK;
  const bool vec = aligned16(logits) && (ld % (dtype == SDX_F32 ? 4 : 8)) == 0;
  return hip_status(sdx::launch_argmax(dtype, logits, rows, vocab, ld, vec, ids, (hipStream_t)stream),
                    "argmax");
}

int sdx_slot_mapping(const int32_t* block_table, int64_t rows, int64_t max_blocks,
                     const int64_t* positions, int32_t block_size, int64_t max_model_len,
                     int64_t padding_slot, int64_t* clamped_positions, int64_t* slots,
                     sdx_stream_t stream) {
  if (!block_table || !positions || !slots || rows < 0 || max_blocks < 1 || block_size < 1)
    return fail(SDX_EINVAL, "sdx_slot_mapping: bad arguments");
  if (rows == 0) return SDX_OK;
  return hip_status(sdx::launch_slot_mapping(block_table, rows, max_blocks, positions, block_size,
                                             max_model_len, padding_slot, clamped_positions, slots,
                                             (hipStream_t)stream),
                    "slot_mapping");
}

// ------------------------------------------------------------------ KV cache
int sdx_kv_advance(int64_t* lengths, int64_t batch, int64_t q, sdx_stream_t stream) {
  if (!lengths || batch < 0) return fail(SDX_EINVAL, "sdx_kv_advance: bad arguments");
  if (batch == 0) return SDX_OK;
  return hip_status(sdx::launch_kv_advance(lengths, batch, q, (hipStream_t)stream), "kv_advance");
}

int sdx_kv_rollback(int64_t* lengths, int64_t batch, const int64_t* n, int32_t* error,
                    sdx_stream_t stream) {
  if (!lengths || !n || batch < 0) return fail(SDX_EINVAL, "sdx_kv_rollback: bad arguments");
  if (batch == 0) return SDX_OK;
  return hip_status(sdx::launch_kv_rollback(lengths, batch, n, error, (hipStream_t)stream),
                    "kv_rollback");
}

int sdx_ragged_update(void* keys, void* values, const void* k_new, const void* v_new, int dtype,
                      int64_t batch, int64_t heads, int64_t capacity, int64_t head_dim, int64_t q,
                      const int64_t* lengths, int32_t* error, sdx_stream_t stream) {
  if (!keys || !values || !k_new || !v_new || !lengths || !dtype_ok(dtype) || batch < 0 ||
      heads < 1 || capacity < 1 || head_dim < 1 || q < 0)
    return fail(SDX_EINVAL, "sdx_ragged_update: bad arguments");
  if (batch == 0 || q == 0) return SDX_OK;
  return hip_status(sdx::launch_ragged_update(dtype, keys, values, k_new, v_new, batch, heads,
                                              capacity, head_dim, q, lengths, error,
                                              (hipStream_t)stream),
                    "ragged_update");
}

int sdx_attn_mask(const int64_t* lengths, const int64_t* valid, int64_t batch, int64_t q,
                  int64_t kv_len, float neg, int dtype, void* out, sdx_stream_t stream) {
  if (!lengths || !out || batch < 0 || q < 0 || kv_len < 0 || !dtype_ok(dtype))
    return fail(SDX_EINVAL, "sdx_attn_mask: bad arguments");
  if (batch * q * kv_len == 0) return SDX_OK;
  return hip_status(
      sdx::launch_attn_mask(lengths, valid, batch, q, kv_len, neg, dtype, out, (hipStream_t)stream),
      "attn_mask");
}

int sdx_kv_append_paged(void* pool, int64_t layer_stride, int64_t side_stride, const void* staged,
                        int dtype, int32_t layers, int64_t batch, int64_t q, int64_t row_elems,
                        const int32_t* block_table, int64_t max_blocks, int32_t block_size,
                        int64_t num_blocks, const int64_t* lengths, int32_t* error,
                        sdx_stream_t stream) {
  if (!pool || !staged || !block_table || !lengths || !dtype_ok(dtype) || layers < 1 ||
      batch < 0 || q < 0 || row_elems < 1 || max_blocks < 1 || block_size < 1 || num_blocks < 1)
    return fail(SDX_EINVAL, "sdx_kv_append_paged: bad arguments");
  const int64_t es = (int64_t)dsize(dtype);
  if ((row_elems * es) % 16 != 0 || !aligned16(pool) || !aligned16(staged) ||
      (layer_stride * es) % 16 != 0 || (side_stride * es) % 16 != 0)
    return fail(SDX_EINVAL, "sdx_kv_append_paged: rows and strides must be 16-byte multiples");
  if (batch == 0 || q == 0) return SDX_OK;
  return hip_status(sdx::launch_kv_append_paged(pool, layer_stride * es, side_stride * es, staged,
                                                layers, batch, q, row_elems * es, block_table,
                                                max_blocks, block_size, num_blocks, lengths, error,
                                                (hipStream_t)stream),
                    "kv_append_paged");
}

// ------------------------------------------------------------------ verify attention
// chunking of the keys shared by the workspace query and the launch
static int attn_plan(int64_t batch, int32_t max_q, int32_t num_q_heads, int32_t num_kv_heads,
                     int32_t block_size, int64_t max_blocks, int32_t chunk_tokens, int32_t* chunk,
                     int32_t* nchunk, size_t* bytes) {
  if (batch < 0 || max_q < 1 || num_q_heads < 1 || num_kv_heads < 1 || block_size < 1 ||
      max_blocks < 1 || chunk_tokens < 0)
    return fail(SDX_EINVAL, "sdx_verify_attention: bad arguments");
  if (chunk_tokens != 0 && (chunk_tokens % 64 != 0 || chunk_tokens > 1024))
    return fail(SDX_EINVAL, "sdx_verify_attention: chunk_tokens must be 0 or a multiple of 64 "
                            "up to 1024 (got %d)", chunk_tokens);
  if (num_q_heads % num_kv_heads != 0)
    return fail(SDX_EINVAL, "sdx_verify_attention: query heads must be a multiple of KV heads");
  const int64_t max_tokens = max_blocks * block_size;
  if (max_tokens > ((int64_t)1 << 31) - 1)
    return fail(SDX_EUNSUPPORTED, "sdx_verify_attention: max_blocks * block_size >= 2^31");
  const int32_t ch = sdx::attn_chunk_tokens(batch, num_kv_heads, max_tokens, chunk_tokens);
  const int64_t nch = (max_tokens + ch - 1) / ch;
  const int64_t m = (int64_t)max_q * (num_q_heads / num_kv_heads);
  const int64_t nrb = (m + 63) / 64;  // workgroups per (chunk, KV head): 64 query rows each
  if (m > 0x7FFFFFFF / 64 || nch * batch * num_kv_heads * nrb > 0x7FFFFFFF)
    return fail(SDX_EUNSUPPORTED, "sdx_verify_attention: grid of %lld chunk workgroups is too large",
                (long long)(nch * batch * num_kv_heads * nrb));
  *chunk = ch;
  *nchunk = (int32_t)nch;
  // the chunk list, then (rows of several chunks) the parts and the per-(row,
  // KV head) arrival counters
  const size_t units = ((size_t)(batch * nch) * sizeof(sdx::AttnUnit) + 15) & ~(size_t)15;
  *bytes = units + (nch > 1 ? (size_t)(batch * num_kv_heads * nch * m) * (128 + 2) * sizeof(float) +
                                  (size_t)(batch * num_kv_heads) * sizeof(uint32_t)
                            : 0);
  return SDX_OK;
}

size_t sdx_verify_attention_workspace(int64_t batch, int32_t max_q, int32_t num_q_heads,
                                      int32_t num_kv_heads, int32_t block_size,
                                      int64_t max_blocks, int32_t chunk_tokens) {
  int32_t ch, nch;
  size_t bytes = 0;
  if (attn_plan(batch, max_q, num_q_heads, num_kv_heads, block_size, max_blocks, chunk_tokens,
                &ch, &nch, &bytes) != SDX_OK)
    return 0;
  return bytes;
}

int sdx_verify_attention_paged(const void* q, int dtype, int64_t batch, const int64_t* cu_q,
                               int32_t max_q, int32_t num_q_heads, int32_t num_kv_heads,
                               int32_t head_dim, const void* k_pool, const void* v_pool,
                               int64_t num_blocks, int32_t block_size, const int32_t* block_table,
                               int64_t max_blocks, const int64_t* kv_len, float scale,
                               int32_t chunk_tokens, void* workspace,
                               size_t workspace_bytes, void* out, int32_t* error,
                               sdx_stream_t stream) {
  if (!q || !cu_q || !k_pool || !v_pool || !block_table || !kv_len || !out || num_blocks < 1 ||
      !(scale > 0.0f))
    return fail(SDX_EINVAL, "sdx_verify_attention_paged: bad arguments");
  if (dtype != SDX_BF16 || (head_dim != 64 && head_dim != 128))
    return fail(SDX_EUNSUPPORTED, "sdx_verify_attention_paged: bf16 with head_dim 64 or 128 only");
  int32_t ch = 0, nch = 0;
  size_t need = 0;
  const int rc = attn_plan(batch, max_q, num_q_heads, num_kv_heads, block_size, max_blocks,
                           chunk_tokens, &ch, &nch, &need);
  if (rc != SDX_OK) return rc;
  const int32_t group = num_q_heads / num_kv_heads;
  if (num_blocks * block_size * num_kv_heads >= (int64_t)0xFFFFFFFF)
    return fail(SDX_EUNSUPPORTED, "sdx_verify_attention_paged: pool of 2^32 or more head slices");
  if (!aligned16(q) || !aligned16(k_pool) || !aligned16(v_pool) || !aligned16(out))
    return fail(SDX_EINVAL, "sdx_verify_attention_paged: tensors must be 16-byte aligned");
  if (!workspace || !aligned16(workspace))
    return fail(SDX_EINVAL, "sdx_verify_attention_paged: needs a 16-byte aligned workspace");
  if (workspace_bytes < need)
    return fail(SDX_EWORKSPACE, "sdx_verify_attention_paged: needs a workspace of %zu bytes "
                                "(got %zu)", need, workspace_bytes);
  if (batch == 0) return SDX_OK;
  sdx::AttnArgs a = {};
  a.q = (const uint16_t*)q;
  a.cu_q = cu_q;
  a.k_pool = (const uint16_t*)k_pool;
  a.v_pool = (const uint16_t*)v_pool;
  a.block_table = block_table;
  a.kv_len = kv_len;
  a.batch = batch;
  a.out = (uint16_t*)out;
  a.error = error;
  a.max_blocks = max_blocks;
  a.num_blocks = num_blocks;
  a.hq = num_q_heads;
  a.hkv = num_kv_heads;
  a.group = group;
  a.bs = block_size;
  a.max_q = max_q;
  a.d = head_dim;
  a.chunk = ch;
  a.nchunk = nch;
  a.max_m = max_q * group;
  a.nrb = (a.max_m + 63) / 64;
  a.nunits = batch * (int64_t)nch;
  const size_t ubytes = ((size_t)a.nunits * sizeof(sdx::AttnUnit) + 15) & ~(size_t)15;
  a.units = (sdx::AttnUnit*)workspace;
  const int64_t nparts = batch * num_kv_heads * (int64_t)nch * a.max_m;
  a.part_o = nch > 1 ? (float*)((char*)workspace + ubytes) : nullptr;
  a.part_ml = nch > 1 ? a.part_o + nparts * head_dim : nullptr;
  a.arrive = nch > 1 ? (uint32_t*)(a.part_ml + nparts * 2) : nullptr;
  a.scale_log2 = scale * 1.4426950408889634f;
  return hip_status(sdx::launch_verify_attn(a, batch, (hipStream_t)stream), "verify_attn");
}

}  // extern "C"
