// Kernel argument records and launch entry points shared between the kernel
// translation units and the C-ABI layer (sdx_capi.hip).
#pragma once

#include "sdx_internal.hpp"

namespace sdx {

// Workspaces of the verify entry points start with a fixed header: a magic
// word that sdx_workspace_init writes, then the arrival counters of rows split
// over several blocks. The counters sit at fixed offsets, so a workspace reused
// for other shapes finds them where the last call left them, at zero.
constexpr size_t kWsHeaderBytes = 16384;
constexpr uint32_t kWsMagic = 0x53445857u;
// Written over the magic word by a fused-verify draw whose bounded wait gave up:
// the header's counters may then hold counts of that call, so every later call
// flags its rows (SDX_FLAG_WORKSPACE) until sdx_workspace_init prepares it again.
constexpr uint32_t kWsDirty = 0x44495254u;
constexpr int kWsCounterWord = 64;  // split-row arrival counters (256-byte aligned)
constexpr int kWsMaxCounters = 1024 - kWsCounterWord;
constexpr int kWsFusedJobWord = 1024;   // fused verify: row arrivals per batch row
constexpr int kWsFusedDrawWord = 2048;  // fused verify: the draw's counters per batch row
constexpr int kWsFusedMaxJobs = 1024;   // batch rows the fused verify serves
static_assert(kWsCounterWord + kWsMaxCounters <= kWsFusedJobWord &&
                  kWsFusedJobWord + kWsFusedMaxJobs <= kWsFusedDrawWord &&
                  kWsFusedDrawWord + kWsFusedMaxJobs <= (int)(kWsHeaderBytes / 4),
              "header word ranges in order, inside the header");

struct RowStatArgs {
  const uint16_t* base[2];  // group 0: target rows, group 1: draft rows
  int64_t nrows[2];
  int64_t ld[2];
  int64_t V;
  const int64_t* ids;  // draft ids [batch, k] (gather source), or null
  int32_t k;           // target rows are [batch, k+1], draft rows [batch, k]
  const int64_t* tgt_idx;  // per-row k: target row -> index into ids (-1: bonus), or null
  float T;
  float top_p;
  int32_t top_k;
  int32_t use_p, use_k, greedy;
  RowStat* stats;
  float* tables;  // [rows, kTbl]
  uint32_t* zero;  // rows [0, nzero) of zero_per_row words (0 meaning 1) cleared by the
  int64_t nzero;   // block of the row, or null
  int32_t zero_per_row;
  uint64_t* rank_acc;  // [rows] rank accumulators, cleared by the row kernel, or null
  int64_t late_block;  // bf16 streaming kernel: blocks from here stream at raised wave
                       // priority (set by launch_rowstream_bf16)
  // bf16 streaming kernel, rows split over several blocks (set by launch_rowstream_bf16
  // from split_ws / split_bytes): blocks [0, nwhole) take whole rows, the rows after
  // nwhole are taken by nparts blocks each, the last of which to finish merges them
  uint8_t* split_ws;   // caller region for the parts' packed histograms; null / too
  size_t split_bytes;  // small: no split
  uint32_t* ws_header;  // the workspace header (magic, then the arrival counters), or null
  int64_t nwhole;
  int32_t nparts;
  int32_t xcd_group;  // a row's parts on blocks of one XCD (block index mod 8)
  uint32_t* split_cnt;  // the header's counters (set by launch_rowstream_bf16)
  uint8_t* split_parts;
  int32_t jm_k;  // fused verify kernel: rows are taken in batch-row order at this k
  int32_t jm_xcd;  // ... with batch row b's rows on blocks of XCD b % 8 (batch % 8 == 0)
  const int32_t* jm_order;  // ... or, at per-row k, in this order (block's q -> row)
};

struct F32Args {
  const float* base[2];
  int64_t nrows[2];
  int64_t ld[2];
  int64_t V;
  const int64_t* ids;
  int32_t k;
  const int64_t* tgt_idx;  // per-row k: target row -> index into ids (-1: bonus), or null
  float T, top_p;
  int32_t top_k, use_p, use_k, greedy;
  float* out;  // dense probabilities [rows, ld_out]
  int64_t ld_out;
  RowStat* stats;  // may be null
  uint32_t* zero;  // words [0, nzero) cleared (block `row` clears word `row`), or null
  int64_t nzero;
  int64_t tie_ld;      // words per row of tie_bits (f32_tie_words(V))
  uint32_t* tie_bits;  // [rows, tie_ld]: members of the row's partially kept
                       // boundary tie group, one bit per id (null: not written)
};

// One final draw: weights from row `prow` (and `qrow` for a residual).
struct SampleJob {
  int64_t prow;     // row whose probabilities are p
  int64_t qrow;     // row of q for a residual draw, -1 for a draw from p
  float u;          // the uniform
  int32_t pad;
};

struct AcceptArgs {
  const RowStat* stats;  // target rows [batch*(k+1)] then draft rows [batch*k]
  int64_t batch;
  int32_t k;              // k, or with per-row k its maximum
  const float* u_accept;  // [batch, k] (per-row k: [sum k_b], row b from cu_k[b])
  const float* u_final;   // [batch]
  const uint8_t* active;  // [batch] or null
  SampleJob* jobs;        // [batch]
  int64_t* n_acc;
  uint8_t* flags;
  const int64_t* draft_ids;  // [batch, k] (16-bit rows: ranks of flagged drafted tokens)
  // per-row k (null: uniform k): row b drafts k_b = cu_k[b+1] - cu_k[b] tokens; its
  // target rows start at cu_k[b] + b, its draft rows at ntgt + cu_k[b]; bad[b] marks
  // a row whose offsets are inconsistent (checked by ragged_rows_kernel)
  const int64_t* cu_k;
  const uint8_t* bad;
  int64_t ntgt;  // target rows (the draft rows' RowStats follow them)
};
// Where batch row b's rows are: its k, first target and draft rows, the offset of
// its drafted ids / accept uniforms; bad rows get k = 0 on row 0
struct RowGeom {
  int k;
  int64_t trow0, drow0, ibase;
  bool bad;
};
__device__ __forceinline__ RowGeom row_geom(const AcceptArgs& a, int64_t b) {
  if (!a.cu_k) return RowGeom{a.k, b * (a.k + 1), a.ntgt + b * a.k, b * a.k, false};
  if (a.bad[b]) return RowGeom{0, 0, a.ntgt, 0, true};
  const int64_t c0 = a.cu_k[b];
  return RowGeom{(int)(a.cu_k[b + 1] - c0), c0 + b, a.ntgt + c0, c0, false};
}

// Partial sums of one draw over one chunk of ids, before the member ranks of
// the boundary tie groups are known (f = fixed62, vp / vq = group values of
// the p / q rows, "member" = element of its row's boundary tie group):
struct ChunkRec {
  uint64_t p2;  // sum f(p) over non-members of p
  uint64_t r0;  // sum f(max(p - q, 0)) over non-members of p and of q
  uint64_t ra;  // sum f(max(p - vq, 0)) over non-members of p that are members of q
  uint64_t rb;  // sum f(p) over the same elements (their q member dropped)
  uint64_t rp;  // sum f(max(vp - q, 0)) over members of p that are non-members of q
  uint32_t np;  // members of p
  uint32_t nq;  // members of q
  uint32_t ndbl;  // members of both
  uint32_t pad;
  uint64_t pad2;
};
static_assert(sizeof(ChunkRec) == 64, "ChunkRec layout");

// Draw records: one ChunkRec per `rec_ids` consecutive ids of a job's rows, a
// multiple of one wave round (64 lanes x 8 ids); at most kMaxRecs per job.
constexpr int kDrawSub = 512;
constexpr int kMaxRecs = 4096;
inline void draw_layout(int64_t V, int64_t* rec_ids, int* nrec) {
  const int64_t span = (int64_t)kDrawSub * kMaxRecs;
  const int64_t rounds = V > span ? (V + span - 1) / span : 1;
  *rec_ids = rounds * kDrawSub;
  *nrec = (int)((V + *rec_ids - 1) / *rec_ids);
}

struct ResidualNormArgs {
  const float* p;
  const float* q;
  int64_t ld;
  int64_t V;
  int64_t rec_ids;
  int32_t nrec;
  const ChunkRec* recs;  // draw records of the rows (one job per row)
  float* out;
  int64_t ld_out;
};

// sdx_rowstat.hip
int rowstat16_nslot(int64_t V);
hipError_t launch_rowstat16(int fmt, const RowStatArgs& a, int64_t rows, hipStream_t s);
// sdx_rowstream.hip
hipError_t launch_rowstream_bf16(const RowStatArgs& a, int64_t rows, hipStream_t s);
// The verify at one k per batch row over bf16 logits (2k + 1 <= 64) in one launch:
// row statistics and the draw (see sdx_rowstream.hip). `job_cnt` ([njobs] words)
// and `counters` must be zero on entry; the launch leaves them at zero.
struct AcceptArgs;
struct RowSource16;
struct ChunkRec;
// per-row k (acc.cu_k): `rowjob` gives each row its batch row (-1: none) and
// rs.jm_order the rows' batch-row order, both from launch_ragged_rows
// k = 0 (no draft rows): each batch row's one row gets the bonus draw, the draft
// step's draw.
hipError_t launch_verify_fused_bf16(const RowStatArgs& rs, int64_t rows, const RowSource16& src,
                                    const AcceptArgs& acc, int64_t njobs, int64_t V, float T,
                                    ChunkRec* recs, uint32_t* counters, uint32_t* job_cnt,
                                    int64_t* y, hipStream_t s, const int32_t* rowjob = nullptr);
// bytes of RowStatArgs::split_ws that let launch_rowstream_bf16 split rows over
// several blocks on the current device (0: it would not split)
size_t rowstream_split_bytes(int64_t rows, int64_t V);
// Rows of a launch over `rows` rows split over several blocks on a device of `cus`
// compute units (each has an arrival counter at header word kWsCounterWord + its
// index; split_layout keeps them below kWsMaxCounters).
int64_t rowstream_split_rows(int64_t rows, int64_t V, int cus);
// The header words the fused verify's per-batch-row counters start at: the row
// arrivals (job_cnt) and the draw counters, one word per batch row each.
inline uint32_t* fused_job_words(uint32_t* header) { return header + kWsFusedJobWord; }
inline uint32_t* fused_draw_words(uint32_t* header) { return header + kWsFusedDrawWord; }
inline uint32_t* split_counter_words(uint32_t* header) { return header + kWsCounterWord; }
// zero `bytes` of a workspace and write the header's magic word
hipError_t launch_workspace_init(void* ws, size_t bytes, hipStream_t s);
// One block: if the header's magic word is not kWsMagic (a draw's wait gave up,
// kWsDirty), zero the header's counter words and write the magic word again.
// Stream order makes it safe: every kernel of earlier calls on the stream has
// ended, so no late arrival can still land in the counters.
hipError_t launch_workspace_rearm(void* ws, hipStream_t s);
// sdx_rank.hip: pgather of drafted tokens inside a partial tie group (after rowstream)
hipError_t launch_rank_bf16(const RowStatArgs& a, int64_t rows, hipStream_t s);
// sdx_f32.hip
// Largest vocabularies of 16-bit rows. bf16 rows stream through the histogram
// kernel, whose normaliser queues a bin as (bin << 18 | count): counts, so the
// vocabulary, stay below 2^18 (the largest multiple of 8 below it, as rows are
// read in 16-byte groups). fp16 rows are held in the registers of one 1024-thread
// workgroup: 16 x 20 x 512 values.
constexpr int64_t kMaxVocabBf16 = (1 << 18) - 8;
constexpr int64_t kMaxVocabF16 = 16 * 20 * 512;
constexpr int64_t kF32MaxVocab = 262144;
// tie-group bit words per fp32 row: one bit per id, whole 64-id wave rounds
inline int64_t f32_tie_words(int64_t V) { return (V + 63) / 64 * 2; }
hipError_t launch_to_probs_f32(const F32Args& a, int64_t rows, hipStream_t s);
// sdx_sample.hip
// Draw: chunk records and the per-job select in one launch (with the accept
// chain when `acc` is given: jobs are then written by the kernel). Without
// `acc`, `jobs` must hold the draws already.
// `counters` ([njobs] words) must be zero on entry: the kernel launched just
// before the draw clears them (RowStatArgs / F32Args `zero`).
// `recs` holds njobs * nrec records (draw_layout).
hipError_t launch_draw16(int fmt, const RowSource16& src, const RowStat* stats,
                         const float* tables, float T, const AcceptArgs* acc, SampleJob* jobs,
                         int64_t njobs, int64_t V, ChunkRec* recs, uint32_t* counters, int64_t* y,
                         hipStream_t s);
hipError_t launch_draw_probs(const RowSourceF32& src, const AcceptArgs* acc, SampleJob* jobs,
                             int64_t njobs, int64_t V, ChunkRec* recs, uint32_t* counters,
                             int64_t* y, hipStream_t s, const uint32_t* tie_bits = nullptr);
hipError_t launch_chunk_mass_probs(const RowSourceF32& src, SampleJob* jobs, int64_t njobs,
                                   int64_t V, ChunkRec* recs, hipStream_t s);
// to_probs output of 16-bit rows: ids per chunk (one workgroup each).
constexpr int64_t kMatChunk = 16384;

// sample_from_probs over dense fp32 rows: record masses (mass[rows * nrec]
// words, nrec = dense_nrec(V)), then one workgroup per row draws y.
constexpr int kDenseRec = 2048;
inline int32_t dense_nrec(int64_t V) { return (int32_t)((V + kDenseRec - 1) / kDenseRec); }
struct DenseArgs {
  const float* p;
  int64_t ld;
  int64_t rows;
  int64_t V;
  int32_t nrec;
  bool vec;        // p 16-byte aligned and ld % 4 == 0
  uint64_t* mass;  // [rows, nrec]
  const float* u;  // [rows]
  int64_t* y;      // [rows]
};
hipError_t launch_sample_dense(const DenseArgs& a, hipStream_t s);
// to_probs output of 16-bit rows: the group members per chunk of partial rows
// into `counts` (rows * nchunk words), then the output.
hipError_t launch_materialize16(int fmt, const RowSource16& src, const RowStat* stats,
                                const float* tables, float T, int64_t rows, int64_t V,
                                int64_t chunk, int nchunk, uint32_t* counts, float* out,
                                int64_t ld_out, hipStream_t s);
hipError_t launch_residual_norm(const ResidualNormArgs& a, int64_t rows, hipStream_t s);
hipError_t launch_gather(const float* probs, int64_t rows, int64_t V, int64_t ld,
                         const int64_t* ids, float* out, hipStream_t s);
// sdx_greedy.hip
hipError_t launch_argmax(int dtype, const void* data, int64_t rows, int64_t V, int64_t ld,
                         bool vec, int64_t* out, hipStream_t s);
hipError_t launch_onehot(const int64_t* am, int64_t rows, int64_t V, float* out, int64_t ld_out,
                         hipStream_t s);
// per-row k: validates cu_k [batch+1] against k_max and the row counts; writes
// tgt_idx [ntgt] (target row -> index into the drafted ids, -1: bonus) and bad [batch]
hipError_t launch_ragged_rows(const int64_t* cu_k, int64_t batch, int32_t k_max, int64_t ntgt,
                              int64_t ndrf, int64_t* tgt_idx, uint8_t* bad, hipStream_t s,
                              int32_t* order = nullptr, int32_t* rowjob = nullptr);
hipError_t launch_greedy_accept(const int64_t* am, int64_t batch, int32_t k, const int64_t* ids,
                                const float* u_accept, const uint8_t* active, int64_t* n_acc,
                                int64_t* y, uint8_t* flags, hipStream_t s,
                                const int64_t* cu_k = nullptr, const uint8_t* bad = nullptr);
// draw from 16-bit rows with the draws given in `jobs` (no accept chain); the
// counters must be zero on entry
hipError_t launch_draw_rows16(int fmt, const RowSource16& src, const RowStat* stats,
                              const float* tables, float T, SampleJob* jobs, int64_t njobs,
                              int64_t V, ChunkRec* recs, uint32_t* counters, int64_t* y,
                              hipStream_t s);
// sdx_engine.hip: the device-side bookkeeping of a speculative round
// A draft step leaves in its workspace header, at word kWsDraftSigWord, what its
// statistics were computed with: kDraftSig, batch, vocab, temperature, top_p and
// top_k (as 32-bit patterns). The verify that takes them over checks it.
constexpr int kWsDraftSigWord = 3072;
constexpr uint32_t kDraftSig = 0x44524654u;
constexpr int kDraftSigWords = 6;
// The fused draft step's count of batch rows whose epilogue is written (the
// last one resets it to zero).
constexpr int kWsDraftDoneWord = kWsDraftSigWord + kDraftSigWords;
static_assert(kWsDraftSigWord >= kWsFusedDrawWord + kWsFusedMaxJobs &&
                  kWsDraftDoneWord < (int)(kWsHeaderBytes / 4),
              "the draft step's header words past the fused verify's, inside the header");
constexpr int kMaxDraftK = 31;  // the fused verify's 2k + 1 <= 64
struct DraftEpiArgs {
  int fmt;                 // SDX_BF16 / SDX_F16 (16-bit rows)
  bool greedy;             // temperature <= 0: the drafted token has probability 1
  const uint16_t* codes;   // 16-bit rows [B, ld]
  int64_t ld;
  const float* probs;      // fp32 path: dense probabilities [B, ldp] (else null)
  int64_t ldp;
  const RowStat* stats;
  const float* tables;
  float T;
  int64_t B, V;
  const int64_t* x;        // drafted tokens [B]
  float* qx;               // [B] or null
  float* conf;             // [B] running product, or null
  float tau;
  int32_t step, min_k;
  int32_t* stop;           // [1] or null
  uint32_t* sig;           // the workspace's signature words (kWsDraftSigWord), or null
  float top_p;
  int32_t top_k;
  int64_t* xcopy;          // [B] the drawn ids kept in the workspace, or null
};
hipError_t launch_draft_epilogue(const DraftEpiArgs& a, hipStream_t s);
// sdx_draft_fused.hip: the draft step for bf16 rows in one launch (the fused
// verify at k = 0 with the epilogue folded into the blocks that complete the
// draws); x is the draw's output, `done` the header word kWsDraftDoneWord.
hipError_t launch_draft_fused_bf16(const RowStatArgs& rs, const RowSource16& src,
                                   const AcceptArgs& acc, int64_t batch, int64_t V, float T,
                                   ChunkRec* recs, uint32_t* counters, uint32_t* job_cnt,
                                   int64_t* x, const DraftEpiArgs& e, uint32_t* done,
                                   hipStream_t s);
// The statistics of k draft steps (their workspaces ws[i]: RowStat[B] at st_off,
// tables [B][kTbl] at tb_off) copied to the verify workspace's draft rows
// (row ntgt + b k + i), with the drafted token's probability and tie flags set as
// the row kernel sets them. A workspace whose signature does not match flags its
// rows kRowBadWs (the verify then reports SDX_FLAG_WORKSPACE).
struct DraftGatherArgs {
  const uint8_t* ws[kMaxDraftK];
  int32_t k;
  int64_t B, V;
  size_t st_off, tb_off, x_off;  // RowStat[B], tables [B][kTbl], the drawn ids [B]
  RowStat* stats;
  float* tables;
  int64_t ntgt;
  const uint16_t* dlog;    // draft logits, row b k + i at dlog + (b k + i) ld
  int64_t ld;
  const int64_t* ids;      // draft ids [B, k]
  uint32_t sig[kDraftSigWords];
  float T;
};
hipError_t launch_draft_gather(const DraftGatherArgs& a, hipStream_t s);
struct RoundCommitArgs {
  int64_t B;
  int32_t k;               // drafts per row (uniform), or with cu_k the rows' own
  const int64_t* cu_k;     // [B+1] or null
  const int64_t* n_acc;
  const int64_t* y;
  const int64_t* draft_ids;  // [B, k] (or packed at cu_k)
  uint8_t* done;
  int64_t* out;            // [B, max_new]
  int64_t* out_len;        // [B]
  int64_t max_new;
  const int64_t* eos;      // [n_eos]
  int32_t n_eos;
  int64_t* len0;           // cache lengths rolled back by k - n_acc (nullable)
  int64_t* len1;
  int64_t* pending;        // [B] <- y (nullable)
  const uint8_t* flags;    // [B] the verify's flags (nullable)
  int32_t* error;          // OR-ed: 1 a live row flagged NONFINITE / UNSUPPORTED /
                           // BAD_ROW / WORKSPACE, 2 a live row with y < 0 (nullable)
};
hipError_t launch_round_commit(const RoundCommitArgs& a, hipStream_t s);
struct CtrlState {         // one EWMAAnalytic controller, 32 bytes (sdx_ctrl_state)
  double acc, reached, c;
  int32_t rounds, last_k;
};
static_assert(sizeof(CtrlState) == 32, "CtrlState layout");
struct CtrlArgs {
  CtrlState* state;
  int64_t nstate;          // 1: one controller for the batch; B: one per row
  const int64_t* n_acc;    // [B]
  int64_t B;
  const int64_t* k_used;   // [nstate]: the k each state's rows drafted this round
  double beta;
  int32_t k_max, k_init, warmup, extra_fwd;
  const float* c_obs;      // [1] observed draft / target forward time, or null
  int64_t* k_next;         // [nstate] or null
  int64_t* cu_k;           // per row: [B+1] exclusive prefix of k_next, or null
};
hipError_t launch_controller(const CtrlArgs& a, hipStream_t s);

// sdx_attn.hip: multi-query verify attention over paged KV (bf16, head_dim 128)
struct AttnUnit {   // one key chunk of one row (b < 0: no chunk)
  int32_t b, c, n, qb;  // row, chunk index, tokens in the chunk, query positions of the row
  int64_t q0, kvl;      // the row's first query row and its keys
};
struct AttnArgs {
  const uint16_t* q;        // [T, hq, d] bf16
  const int64_t* cu_q;      // [B + 1] query-row offsets
  const uint16_t* k_pool;   // [num_blocks, bs, hkv * d] bf16
  const uint16_t* v_pool;
  const int32_t* block_table;  // [B, max_blocks]
  const int64_t* kv_len;    // [B] keys per row, the new positions included
  uint16_t* out;            // [T, hq, d] bf16
  int32_t* error;           // set when a row's shape or pages are out of range
  AttnUnit* units;          // [nunits] the chunks in launch order (written by the plan kernel)
  float* part_o;            // [B, hkv, nchunk, max_m, d] chunk partials (nchunk > 1)
  float* part_ml;           // [B, hkv, nchunk, max_m, 2] their (max, sum)
  int64_t max_blocks, num_blocks, batch;
  int32_t hq, hkv, group, bs, max_q;
  int32_t chunk, nchunk, max_m;  // tokens per chunk, chunks of the longest row, max_q * group
  int64_t nunits;           // batch * nchunk: the launch's chunk slots
  float scale_log2;         // softmax scale * log2(e)
  int32_t d;                // head dim: 64 or 128
  uint32_t* arrive;         // [B, hkv] chunks of the row written so far (nchunk > 1; zeroed
                            // by the plan kernel)
  int32_t nrb;              // blocks of 64 query rows per (chunk, KV head): ceil(max_m / 64)
};
// tokens per key chunk (chunk > 0: that value, else the default for the shape)
int attn_chunk_tokens(int64_t batch, int32_t hkv, int64_t max_tokens, int32_t chunk);
hipError_t launch_verify_attn(const AttnArgs& a, int64_t batch, hipStream_t s);
// sdx_kv.hip
hipError_t launch_kv_advance(int64_t* lengths, int64_t batch, int64_t q, hipStream_t s);
hipError_t launch_kv_rollback(int64_t* lengths, int64_t batch, const int64_t* n, int32_t* error,
                              hipStream_t s);
hipError_t launch_ragged_update(int dtype, void* keys, void* values, const void* kn,
                                const void* vn, int64_t B, int64_t H, int64_t C, int64_t D,
                                int64_t q, const int64_t* lengths, int32_t* error, hipStream_t s);
hipError_t launch_attn_mask(const int64_t* lengths, const int64_t* valid, int64_t B, int64_t q,
                            int64_t kv, float neg, int dtype, void* out, hipStream_t s);
hipError_t launch_kv_append_paged(void* pool, int64_t layer_stride_b, int64_t side_stride_b,
                                  const void* staged, int32_t layers, int64_t batch, int64_t q,
                                  int64_t row_bytes, const int32_t* bt, int64_t max_blocks,
                                  int32_t bs, int64_t num_blocks, const int64_t* lengths,
                                  int32_t* error, hipStream_t s);
hipError_t launch_slot_mapping(const int32_t* bt, int64_t rows, int64_t max_blocks,
                               const int64_t* positions, int32_t bs, int64_t max_len,
                               int64_t pad_slot, int64_t* clamped, int64_t* slots, hipStream_t s);

}  // namespace sdx
