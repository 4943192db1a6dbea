/*
 * specdec_amd.h -- C ABI of the MI355X (gfx950) speculative-decoding verify path.
 *
 * One shared library, libspecdec_amd.so, built from adaptive-specdec_amd/csrc.
 * Every entry point:
 *   - takes plain device pointers, element counts and an explicit stream
 *     (a hipStream_t; NULL means the null stream) and is asynchronous;
 *   - returns 0 on success or a negative SDX_E* status, with a message
 *     retrievable from sdx_last_error() (thread-local);
 *   - never allocates: scratch comes from a caller workspace sized by the
 *     matching *_workspace() query.
 * Token ids are int64 (torch's index type); block tables are int32. All
 * tensors are row-major; a row stride ("ld") is given in elements.
 *
 * Numerics. Every discrete decision (nucleus membership, top-k threshold,
 * accept/reject, sampled id) is computed with a fixed deterministic rule:
 * s = fl32(x / T), m = max s, softmax numerator e = exp_det(s - m) where exp_det
 * is a Cody-Waite reduction in float64 (k = floor(d / ln 2), r = fl32(d - k ln 2)
 * clamped to [0, ln 2]) followed by the degree-9 Taylor polynomial of exp at r in
 * fp32 Horner form (plain multiply then add, coefficients fl32(1/n!), clamped at
 * 2) scaled by 2^k; the normaliser and every mass/CDF accumulated exactly in 2^-62
 * fixed point; stable (lowest id first) tie order; inverse-CDF sampling on
 * caller uniforms. Identical inputs give identical ids on every run and launch
 * configuration.
 */
#ifndef SPECDEC_AMD_H
#define SPECDEC_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* sdx_stream_t; /* == hipStream_t */

enum sdx_dtype { SDX_F32 = 0, SDX_BF16 = 1, SDX_F16 = 2 };

enum sdx_status {
  SDX_OK = 0,
  SDX_EINVAL = -1,       /* bad argument (null pointer, bad shape, misaligned) */
  SDX_EUNSUPPORTED = -2, /* valid request outside what this build implements */
  SDX_EHIP = -3,         /* a HIP runtime call failed */
  SDX_EWORKSPACE = -4    /* workspace smaller than the *_workspace() query */
};

/* Per-row flag bits written by the verify entry points. */
enum sdx_flag {
  SDX_FLAG_ACCEPT_NEAR_TIE = 1, /* an evaluated accept test had |u - min(p/q,1)| < 1e-5 */
  SDX_FLAG_NONFINITE = 2,       /* a logit row held +inf or NaN: results unspecified */
  SDX_FLAG_UNSUPPORTED = 4,     /* a row's probability mass spans more distinct logit values
                                   than the row kernels' histogram windows cover (only with
                                   |logit| >= 2^18 at temperatures above ~2500, or fp16 rows
                                   spanning over 36 binades of mass): results unspecified */
  SDX_FLAG_BAD_ROW = 8,         /* per-row k: the row offsets (cu_k) were inconsistent with
                                   k_max or the row counts; n_acc 0, y unspecified */
  SDX_FLAG_WORKSPACE = 16,      /* the verify workspace was not prepared by
                                   sdx_workspace_init, or a draw of the fused bf16
                                   verify gave up its bounded wait (20 ms) for the row
                                   statistics: y -1, n_acc unspecified. After a give-up
                                   the workspace header is marked and every later call
                                   flags its rows until sdx_workspace_init runs again
                                   (sdx_verify_noalloc prepares its scratch again by
                                   itself at its next call) */
  SDX_FLAG_TIE_ORDER = 32       /* an evaluated accept test's drafted token, or the final
                                   draw, is a member of a partially kept top-p boundary tie
                                   group (tokens of equal probability of which the nucleus
                                   keeps only some, specdec/sampling.py:57-64): the literal
                                   reference's unstable sort may keep other members, so the
                                   row's outcome is fixed here by the lowest-ids-first rule
                                   and may differ from a run of the reference */
};

const char* sdx_last_error(void);
int sdx_version(void);

/* Prepare a workspace for the entry points below: zero-fill `bytes` and write the
 * header word the verify kernels check. Required once for a workspace of
 * sdx_verify / sdx_verify_ragged / sdx_verify_stats (which keep arrival counters
 * at fixed offsets of its first 16 KB and leave them at zero after every call);
 * harmless for the others. Asynchronous on `stream`; no memset, so it may be
 * captured in a graph. A verify call on a workspace that was never prepared does
 * not trust its counters: the rows that would use them get SDX_FLAG_WORKSPACE.
 * No reference counterpart (the reference allocates per call in torch). */
int sdx_workspace_init(void* workspace, size_t bytes, sdx_stream_t stream);

/* ---- sampling transforms: specdec/sampling.py ---------------------------
 * Switches follow sampling.py:43,52,56: temperature <= 0 -> greedy one-hot
 * (first index among maxima); top_p outside (0, 1) -> no nucleus; top_k <= 0
 * or >= vocab -> no top-k.
 * Vocabularies: bf16 rows up to 262,136 (2^18 - 8), fp16 up to 163,840, fp32 up
 * to 262,144 (above 8,192 the fp32 rows take a multi-pass kernel that sorts only
 * the nucleus boundary region, at most 7,168 distinct probabilities: a row whose region is
 * larger is flagged SDX_FLAG_UNSUPPORTED with NaN probabilities); larger ones
 * return SDX_EUNSUPPORTED (here and in the verify entry points) before anything
 * is launched. (The Python entry points widen longer fp16 rows to fp32, which
 * is exact, and call the fp32 path.) */

/* to_probs (sampling.py:34-67): logits [rows, vocab] (dtype) -> probs [rows, vocab] fp32.
 * probs may not overlap fp32 logits (SDX_EINVAL): above 8,192 tokens the fp32 kernel
 * keeps each element's exp, then its probability, in the output row between passes. */
size_t sdx_to_probs_workspace(int64_t rows, int64_t vocab, int dtype);
int sdx_to_probs(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                 float temperature, float top_p, int32_t top_k,
                 float* probs, int64_t ld_out, void* workspace, size_t workspace_bytes,
                 sdx_stream_t stream);

/* sample_from_probs (sampling.py:70-74): one inverse-CDF draw per row on u[rows] in [0,1).
 * ids[r] = first j with prefix(fixed62(probs[r]))[j] > floor(u[r] * sum); -1 for an all-zero row. */
size_t sdx_sample_probs_workspace(int64_t rows, int64_t vocab);
int sdx_sample_probs(const float* probs, int64_t rows, int64_t vocab, int64_t ld, const float* u,
                     int64_t* ids, void* workspace, size_t workspace_bytes, sdx_stream_t stream);

/* residual_probs (sampling.py:77-90): out = norm((p - q)_+), or p when that mass <= 1e-9. */
size_t sdx_residual_probs_workspace(int64_t rows, int64_t vocab);
int sdx_residual_probs(const float* p, const float* q, int64_t rows, int64_t vocab, int64_t ld,
                       float* out, int64_t ld_out, void* workspace, size_t workspace_bytes,
                       sdx_stream_t stream);

/* gather_prob (sampling.py:93-95): out[r] = probs[r, ids[r]]. */
int sdx_gather_prob(const float* probs, int64_t rows, int64_t vocab, int64_t ld, const int64_t* ids,
                    float* out, sdx_stream_t stream);

/* ---- verify: specdec/engine.py:281-312 ----------------------------------
 * The engine's accept block factored out as one call. Inputs:
 *   target_logits [batch, k+1, vocab], draft_logits [batch, k, vocab] (dtype, contiguous),
 *   draft_ids [batch, k], u_accept [batch, k] (the per-position uniforms of engine.py:291),
 *   u_final [batch] (the residual/bonus uniform), active [batch] (nullable; 0 = row done,
 *   the engine's ~done, engine.py:287).
 * Outputs: n_acc [batch] accepted drafts, y [batch] the token emitted after them
 * (residual draw at position n_acc, or the bonus draw from p_{k+1} when n_acc == k),
 * flags [batch] (sdx_flag bits). Emitted tokens of row b: draft_ids[b, :n_acc[b]] then y[b];
 * KV rows to drop: k - n_acc[b] (engine.py:310).
 * Workspace: sized by sdx_verify_workspace for the current device and prepared once
 * by sdx_workspace_init: with bf16 logits it carries arrival counters of rows split
 * over several blocks at fixed offsets, which every call leaves at zero, so one
 * workspace serves calls of any shape that fits it. Calls that share a workspace
 * must not overlap. */
size_t sdx_verify_workspace(int64_t batch, int32_t k, int64_t vocab, int dtype);
int sdx_verify(const void* target_logits, const void* draft_logits, int dtype,
               int64_t batch, int32_t k, int64_t vocab,
               const int64_t* draft_ids, const float* u_accept, const float* u_final,
               const uint8_t* active, float temperature, float top_p, int32_t top_k,
               int64_t* n_acc, int64_t* y, uint8_t* flags,
               void* workspace, size_t workspace_bytes, sdx_stream_t stream);

/* sdx_verify without a workspace, for callers that cannot allocate device memory
 * (code under graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. Same arguments, outputs and
 * rules as sdx_verify; the scratch is a 24 MiB device array inside the library,
 * one per GPU, held until the process ends, prepared by a kernel queued on
 * `stream` at the first call on each device. Nothing is allocated. Requests
 * whose sdx_verify_workspace exceeds 24 MiB (more than about 1,152 logit rows
 * at vocab 151,936, e.g. batch 128 at k = 4) return SDX_EWORKSPACE. All calls on
 * one GPU share its array: calls that may overlap (other streams, other host
 * threads) race and must be serialised by the caller. */
int sdx_verify_noalloc(const void* target_logits, const void* draft_logits, int dtype,
                       int64_t batch, int32_t k, int64_t vocab,
                       const int64_t* draft_ids, const float* u_accept, const float* u_final,
                       const uint8_t* active, float temperature, float top_p, int32_t top_k,
                       int64_t* n_acc, int64_t* y, uint8_t* flags, sdx_stream_t stream);

/* sdx_verify for a round whose draft rows already went through sdx_draft_step:
 * draft_workspaces (a host array of k device pointers) holds, for each draft
 * position i, the workspace of the sdx_draft_step call that sampled draft_ids[:, i]
 * from draft_logits[:, i] (batch rows, same vocab, temperature, top_p and top_k).
 * The draft rows' to_probs statistics are taken from those workspaces instead of
 * streaming draft_logits again: only the k + 1 target rows per batch row are read
 * in full, plus the draft rows of the final residual draws (the row statistics
 * then the draw, two launches). Outputs, rules and workspace as sdx_verify, and
 * the same results as sdx_verify on the same inputs. A draft workspace whose
 * statistics were made for another shape or sampling configuration, or whose draft
 * step's wait gave up, flags its rows SDX_FLAG_WORKSPACE. Other dtypes, temperature <= 0 and k > 31 run
 * sdx_verify and ignore the draft workspaces. No reference counterpart: the
 * reference's verify recomputes q from the draft logits (engine.py:250,288). */
int sdx_verify_drafted(const void* target_logits, const void* draft_logits, int dtype,
                       int64_t batch, int32_t k, int64_t vocab, const int64_t* draft_ids,
                       const float* u_accept, const float* u_final, const uint8_t* active,
                       float temperature, float top_p, int32_t top_k,
                       const void* const* draft_workspaces, int64_t* n_acc, int64_t* y,
                       uint8_t* flags, void* workspace, size_t workspace_bytes,
                       sdx_stream_t stream);

/* Verify with a different k per batch row (config 5's adaptive k): row b drafts
 * k_b = cu_k[b+1] - cu_k[b] tokens, 0 <= k_b <= k_max (cu_k int64 [batch+1] on the
 * device, cu_k[0] = 0). Rows are packed: target_logits [target_rows, vocab] with
 * row b's k_b + 1 positions at cu_k[b] + b (target_rows = sum (k_b + 1), known to the
 * caller from the tensor's shape), draft_logits / draft_ids / u_accept
 * [target_rows - batch] with row b's at cu_k[b]. Same rules and outputs as
 * sdx_verify (emitted tokens of row b: draft_ids[cu_k[b] .. + n_acc[b]] then y[b]; KV
 * rows to drop: k_b - n_acc[b]). The offsets are checked on the device: if they are
 * inconsistent (not non-decreasing from 0 to target_rows - batch, or a k_b > k_max),
 * every row gets SDX_FLAG_BAD_ROW and n_acc 0. Workspace: sdx_verify_ragged_workspace,
 * prepared once by sdx_workspace_init, as for sdx_verify. No reference counterpart: the reference engine
 * verifies one k for the whole batch (engine.py:281-312). */
size_t sdx_verify_ragged_workspace(int64_t batch, int64_t target_rows, int64_t vocab, int dtype);
int sdx_verify_ragged(const void* target_logits, const void* draft_logits, int dtype,
                      int64_t batch, int32_t k_max, int64_t target_rows, int64_t vocab,
                      const int64_t* cu_k, const int64_t* draft_ids, const float* u_accept,
                      const float* u_final, const uint8_t* active, float temperature,
                      float top_p, int32_t top_k, int64_t* n_acc, int64_t* y, uint8_t* flags,
                      void* workspace, size_t workspace_bytes, sdx_stream_t stream);

/* Where the verify kernels keep their cross-workgroup counters (split-row arrivals,
 * the fused kernel's per-batch-row row arrivals and draw counters) in a workspace of
 * this shape (target_rows 0: one k for all rows; else per-row k with target_rows
 * target rows) on a device of `cus` compute units: ranges[2i], ranges[2i+1] are the
 * byte offsets [begin, end) of range i, from the same helpers the launches use;
 * the last range is the header itself. Returns the number of ranges (4), or a
 * negative status. Pure host arithmetic, for checking that every counter a kernel
 * is handed lies in the fixed header, which every call leaves at zero. No reference
 * counterpart. */
int sdx_verify_counter_layout(int64_t batch, int64_t target_rows, int32_t k, int64_t vocab,
                              int dtype, int32_t cus, int64_t* ranges, int32_t max_ranges);

/* Phase 1 of sdx_verify alone: the fused to_probs statistics of every target and draft
 * row (normaliser, top-k/top-p boundary, drafted-token probabilities) into the workspace,
 * without the accept test or the final draw. Lets a caller time or overlap the
 * vocabulary pass; temperature must be > 0. Same workspace as sdx_verify.
 * draft_ids may be NULL: then only the row statistics (no gathered probabilities). */
int sdx_verify_stats(const void* target_logits, const void* draft_logits, int dtype,
                     int64_t batch, int32_t k, int64_t vocab, const int64_t* draft_ids,
                     float temperature, float top_p, int32_t top_k, void* workspace,
                     size_t workspace_bytes, sdx_stream_t stream);

/* Greedy verify (temperature 0): row b accepts position i iff draft_ids[b,i] ==
 * argmax(target[b,i]) and u_accept[b,i] < 1 (u_accept nullable = all zero); y[b] =
 * argmax(target[b, n_acc[b]]). Draft logits are not needed: with one-hot p the accept
 * ratio is 0 or >= 1 whatever q is. Same outputs as sdx_verify at temperature 0. */
size_t sdx_verify_greedy_workspace(int64_t batch, int32_t k);
int sdx_verify_greedy(const void* target_logits, int dtype, int64_t batch, int32_t k,
                      int64_t vocab, const int64_t* draft_ids, const float* u_accept,
                      const uint8_t* active, int64_t* n_acc, int64_t* y, uint8_t* flags,
                      void* workspace, size_t workspace_bytes, sdx_stream_t stream);

/* ---- one speculative round on the device: specdec/engine.py:228-342 ------- */

/* One draft step (engine.py:246-258 with the early exit of controller.py:184-187).
 * Its workspace keeps the rows' statistics until the next call on it, for
 * sdx_verify_drafted:
 * q = to_probs(logits[b]) (sampling.py:34-67); x[b] = the inverse-CDF draw from q on
 * u[b] (the rule of sdx_sample_probs; temperature <= 0: the first argmax, u unused);
 * qx[b] = q(x[b]) (nullable); conf[b] *= qx[b] (nullable, the running product of
 * engine.py:256); *stop (nullable) = 1 if step >= min_k and mean(conf) < tau, the mean
 * a sequential fp32 sum in row order over batch (ConfidenceEarlyExit.
 * should_stop_drafting), else 0. logits [batch, ld] (dtype); workspace from
 * sdx_draft_step_workspace, prepared once by sdx_workspace_init. Every output stays on
 * the device: the reference's float(conf.mean()) host sync becomes a device flag.
 * With bf16 rows the call is one launch, whose draw blocks wait (bounded) for their
 * row's statistics; a wait that gives up leaves that row x -1, qx 0, conf *= 0 and
 * *stop = 1, and marks the workspace (its statistics are no longer taken over by
 * sdx_verify_drafted) until sdx_workspace_init prepares it again. */
size_t sdx_draft_step_workspace(int64_t batch, int64_t vocab, int dtype);
int sdx_draft_step(const void* logits, int dtype, int64_t batch, int64_t vocab, int64_t ld,
                   float temperature, float top_p, int32_t top_k, const float* u, int64_t* x,
                   float* qx, float* conf, float tau, int32_t step, int32_t min_k, int32_t* stop,
                   void* workspace, size_t workspace_bytes, sdx_stream_t stream);

/* The end of a round (engine.py:305-340) without its n_acc.tolist() host sync:
 * row b drafted k (or, with cu_k [batch+1], cu_k[b+1] - cu_k[b]) tokens draft_ids
 * [batch, k] (or packed at cu_k[b]), accepted n_acc[b] and drew y[b]. lengths0 and
 * lengths1 (the two caches' device lengths, nullable) drop k_b - n_acc[b] positions.
 * Unless done[b], the accepted drafts and then y[b] are appended to
 * out_tokens[b, out_len[b]..] (capacity max_new per row); a token in eos_ids
 * [n_eos], or the row reaching max_new tokens, sets done[b] and ends the row's
 * emission. pending[b] (nullable) = y[b], the next round's first input.
 * flags (nullable) are the verify's per-row flags: a row that is not done and is
 * flagged NONFINITE, UNSUPPORTED, BAD_ROW or WORKSPACE, or whose y is negative,
 * emits nothing, is set done, gets pending 0 and ORs into *error (nullable, device
 * int32) 1 (a flag) or 2 (y < 0): the caller reads it where it syncs anyway (the
 * reference fails loudly there: torch.multinomial raises on NaN probabilities).
 * draft_ids may be NULL only when no row drafted (k == 0 and no cu_k). */
int sdx_round_commit(int64_t batch, int32_t k, const int64_t* cu_k, const int64_t* n_acc,
                     const int64_t* y, const int64_t* draft_ids, uint8_t* done,
                     int64_t* out_tokens, int64_t* out_len, int64_t max_new,
                     const int64_t* eos_ids, int32_t n_eos, int64_t* lengths0, int64_t* lengths1,
                     int64_t* pending, const uint8_t* flags, int32_t* error,
                     sdx_stream_t stream);

/* EWMAAnalytic (controller.py:121-154) on the device. One state per batch
 * (nstate 1: accepted = sum n_acc, reached = sum min(n_acc + 1, k_used[0]), as
 * update() computes them) or per row (nstate == batch: row b's n_acc[b] and its
 * own k_used[b]). Each state: w = beta^reached; acc = w acc + accepted; reached =
 * w reached + reached; c = 0.9 c + 0.1 c_obs when c_obs (nullable, [1]) is > 0;
 * rounds += 1; then the next k (propose_k): k_init while rounds < warmup, else
 * best_k(clamp(acc / reached, 0, 0.999) (0.7 before any token), c, k_max,
 * extra_fwd) (controller.py:47-67) into k_next [nstate] (nullable) and, per row,
 * its exclusive prefix into cu_k [batch + 1] (nullable: the offsets of the next
 * sdx_verify_ragged). All in float64, as the host controller computes it. */
typedef struct {
  double acc, reached, c;
  int32_t rounds, last_k;
} sdx_ctrl_state;
int sdx_controller_update(sdx_ctrl_state* state, int64_t nstate, const int64_t* n_acc,
                          int64_t batch, const int64_t* k_used, double beta, int32_t k_max,
                          int32_t k_init, int32_t warmup, int32_t extra_fwd, const float* c_obs,
                          int64_t* k_next, int64_t* cu_k, sdx_stream_t stream);

/* ---- proposer-side calls: vllm_draft_spec/proposer.py -------------------- */

/* Greedy draft token, logits.argmax(dim=-1) (proposer.py:262-263,331-332): first index
 * among maxima, -0 == +0. logits [rows, vocab] (dtype) -> ids [rows]. */
int sdx_argmax(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
               int64_t* ids, sdx_stream_t stream);

/* Drafting-step slot mapping (proposer.py:295-314): positions >= max_model_len are parked
 * at 0 with slot padding_slot; else slot = block_table[r, pos / bs] * bs + pos % bs.
 * block_table [rows, max_blocks] int32. clamped_positions may be NULL. */
int sdx_slot_mapping(const int32_t* block_table, int64_t rows, int64_t max_blocks,
                     const int64_t* positions, int32_t block_size, int64_t max_model_len,
                     int64_t padding_slot, int64_t* clamped_positions, int64_t* slots,
                     sdx_stream_t stream);

/* ---- KV cache: specdec/kvcache.py ---------------------------------------- */

/* RaggedCache.advance (kvcache.py:165-168): lengths[b] += q. */
int sdx_kv_advance(int64_t* lengths, int64_t batch, int64_t q, sdx_stream_t stream);

/* RaggedCache.rollback (kvcache.py:174-190) with device counts: lengths[b] -= n[b]. If any
 * row would go below zero no length changes and *error (device int32) is set to 1;
 * otherwise *error is left untouched. error may be NULL. */
int sdx_kv_rollback(int64_t* lengths, int64_t batch, const int64_t* n, int32_t* error,
                    sdx_stream_t stream);

/* _RaggedLayer.update (kvcache.py:61-74): write k_new/v_new [batch, heads, q, head_dim]
 * into keys/values [batch, heads, capacity, head_dim] at slots lengths[b] + j.
 * dtype is the element type of all four tensors (SDX_BF16, SDX_F16 or SDX_F32). Rows that
 * would overflow capacity set *error (nullable) and are not written. */
int sdx_ragged_update(void* keys, void* values, const void* k_new, const void* v_new,
                      int dtype, int64_t batch, int64_t heads, int64_t capacity,
                      int64_t head_dim, int64_t q, const int64_t* lengths, int32_t* error,
                      sdx_stream_t stream);

/* RaggedCache.attn_mask (kvcache.py:138-162): out [batch, 1, q, kv_len] (dtype) with 0
 * where slot s <= lengths[b] + j and s < valid[b] (valid nullable), else `neg`. */
int sdx_attn_mask(const int64_t* lengths, const int64_t* valid, int64_t batch, int64_t q,
                  int64_t kv_len, float neg, int dtype, void* out, sdx_stream_t stream);

/* Paged append of q candidate positions per row into L layers that share one block
 * table (the 36 target + 28 draft layers of one vLLM KV group, proposer.py:18-22).
 * Pool of layer l, side s (0 = K, 1 = V): pool + l*layer_stride + s*side_stride, laid
 * out [num_blocks, block_size, row_elems] (row_elems = kv_heads * head_dim, bf16/f16).
 * New rows: staged + ((l*2 + s)*batch + b)*q*row_elems + j*row_elems.
 * Position of (b, j) is lengths[b] + j; block_table [batch, max_blocks] int32 with ids
 * in [0, num_blocks). Out-of-range positions or block ids set *error (nullable) and are
 * skipped. Strides are in elements; row_elems * sizeof(dtype) must be a multiple of 16. */
int sdx_kv_append_paged(void* pool, int64_t layer_stride, int64_t side_stride,
                        const void* staged, int dtype, int32_t layers, int64_t batch,
                        int64_t q, int64_t row_elems, const int32_t* block_table,
                        int64_t max_blocks, int32_t block_size, int64_t num_blocks,
                        const int64_t* lengths, int32_t* error, sdx_stream_t stream);

/* ---- verify attention: the target's multi-query attention of one verify
 * forward (bench/bench_engine.py:170-174 -> specdec/engine.py:273-275 through
 * HF SDPA with the mask of specdec/kvcache.py:138-162), one layer.
 * Row b has q_b = cu_q[b+1] - cu_q[b] <= max_q new positions (its k_b + 1
 * verify positions), already appended to the paged cache; kv_len[b] counts
 * the row's keys including them. Query j of row b sees keys
 * s <= kv_len[b] - q_b + j. q / out: [cu_q[B], num_q_heads, head_dim] bf16;
 * query head h reads KV head h / (num_q_heads / num_kv_heads). Pools: [num_blocks,
 * block_size, num_kv_heads * head_dim] bf16 (the K and V sides of one layer of
 * sdx_kv_append_paged's pool); block_table [batch, max_blocks] int32; cu_q and
 * kv_len int64 on the device. softmax(q k^T * scale) v in fp32, P rounded to
 * bf16 for the P V product, output rounded to bf16. The keys of a row are split
 * in chunks of chunk_tokens (0: the library's default for the shape; else a
 * multiple of 64, at most 1024) handled by separate workgroups, longest chunks
 * first; rows of more than one chunk merge fp32 partials (the row's last chunk
 * to finish merges it). `workspace` holds the chunk list, the partials and the
 * rows' arrival counters (sdx_verify_attention_workspace bytes, 16-byte aligned,
 * no initial contents). Two kernels are queued on `stream`. A row
 * whose shape is out of range sets *error (nullable) and is skipped; page ids
 * outside the pool set *error and the row's output is unspecified. bf16,
 * head_dim 64 or 128. A KV head with more than 64 query rows (max_q x query heads
 * per KV head) takes a workgroup per block of 64 rows for each key chunk. */
int sdx_verify_attention_paged(const void* q, int dtype, int64_t batch, const int64_t* cu_q,
                               int32_t max_q, int32_t num_q_heads, int32_t num_kv_heads,
                               int32_t head_dim, const void* k_pool, const void* v_pool,
                               int64_t num_blocks, int32_t block_size, const int32_t* block_table,
                               int64_t max_blocks, const int64_t* kv_len, float scale,
                               int32_t chunk_tokens, void* workspace, size_t workspace_bytes,
                               void* out, int32_t* error, sdx_stream_t stream);

/* Workspace bytes sdx_verify_attention_paged needs for these sizes and chunk_tokens
 * (0 on invalid arguments). */
size_t sdx_verify_attention_workspace(int64_t batch, int32_t max_q, int32_t num_q_heads,
                                      int32_t num_kv_heads, int32_t block_size,
                                      int64_t max_blocks, int32_t chunk_tokens);

#ifdef __cplusplus
}
#endif
#endif /* SPECDEC_AMD_H */
