/*
 * voidinfer_sampling.h — C ABI of the MI355X (gfx950) token-sampling library.
 *
 * Plain pointers and sizes only; every entry point returns a vi_status and never
 * throws.  Device pointers are HIP device memory; `stream` is a hipStream_t passed
 * as void* (NULL = the default stream).  All launches are stream-ordered and
 * asynchronous: no entry point synchronizes the host, so they are safe to record
 * into a HIP graph (workspaces are carved, never allocated, inside a call).
 *
 * Each entry point names the reference interface it replaces
 * (The8Darkness/voidinfer, file:line).
 */
#ifndef VOIDINFER_SAMPLING_H
#define VOIDINFER_SAMPLING_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
typedef int vi_status;
enum {
    VI_OK = 0,
    VI_ERR_INVALID = 1,      /* bad argument (extent, null pointer, range)          */
    VI_ERR_UNSUPPORTED = 2,  /* valid request outside what the kernels implement     */
    VI_ERR_WORKSPACE = 3,    /* workspace missing, too small or misaligned           */
    VI_ERR_LAUNCH = 4,       /* HIP launch / runtime error                           */
    VI_ERR_DEVICE = 5        /* device query failed / not gfx950                     */
};

/* ---- logit storage types ----------------------------------------------- */
enum { VI_BF16 = 0, VI_F16 = 1, VI_F32 = 2 };

/* ---- per-row output flags (vi_sample_rows / vi_verify_rows) ------------ */
enum {
    VI_FLAG_NONFINITE = 1u,     /* a non-finite logit was skipped                       */
    VI_FLAG_EMPTY = 2u,         /* no finite logit: token = vocabulary (invalid)        */
    VI_FLAG_ZERO_Q = 4u,        /* verify: drafted token has zero draft probability     */
    VI_FLAG_NO_RESIDUAL = 8u,   /* verify: residual mass <= 1e-9, corrected from p      */
    VI_FLAG_BAD_HISTORY = 16u,  /* a history token outside [0, vocabulary) was ignored  */
    VI_FLAG_ERROR = 0x80000000u /* the kernel could not finish this row (see status)    */
};

/* 16-byte decision row; identical layout to Exl3GreedyRow
 * (src/exl3/greedy_packet.h:22-26). */
typedef struct vi_greedy_row {
    uint64_t serial;
    int32_t token;
    uint32_t nonfinite;
} vi_greedy_row;

/* Request sampling configuration of the coupled (reference-semantics) route;
 * field-for-field Exl3DeviceSampling (src/exl3/sampled_select.h:17-28). */
typedef struct vi_device_sampling {
    float temperature;
    int32_t top_k;
    float top_p;
    float min_p;
    uint64_t seed;
    float presence_penalty;
    int32_t reserved;
    const int32_t* first_occurrence; /* device int32[vocabulary] or NULL */
} vi_device_sampling;

/* First-occurrence value of a token that was never generated
 * (kExl3AbsentOccurrence, src/exl3/sampled_select.h:16). */
#define VI_ABSENT_OCCURRENCE 0x7f7f7f7f

/* Per-row parameters of the batched (extended-semantics) sampler.  One row is
 * one lane's next-token distribution.  Per row: history tokens get
 * x' = (x>0 ? x/rep : x*rep) - freq*count - presence, stored back in the logit
 * dtype; z = x' * (1/T); tokens sorted by (z desc, id asc); the first
 * min(top_k, finite) form the cap set; weights w = exp(z - z_max); the support
 * is the cap-set prefix cut at the first w < min_p and after the first
 * cumulative w >= top_p * sum(cap set); the token is the first support entry
 * whose cumulative w exceeds u * sum(support), u the Philox uniform of
 * (seed, lane, position).  48 bytes. */
typedef struct vi_row_params {
    float temperature;        /* 0 = (penalized) argmax                               */
    float top_p;              /* (0,1]; 1 disables                                    */
    float min_p;              /* [0,1]; 0 disables                                    */
    float repetition_penalty; /* > 0; 1 disables (HF convention)                      */
    float presence_penalty;   /* OpenAI convention; 0 disables                        */
    float frequency_penalty;  /* OpenAI convention; 0 disables                        */
    int32_t top_k;            /* 0 disables                                           */
    uint32_t lane;            /* Philox counter word: request lane                    */
    uint64_t seed;            /* Philox key                                           */
    int32_t position;         /* Philox counter word: absolute position of the token  */
    uint32_t reserved;
} vi_row_params;

/* Optional per-row diagnostics of vi_sample_rows. */
typedef struct vi_sample_stats {
    uint32_t flags;           /* VI_FLAG_*                                            */
    uint32_t support;         /* tokens in the truncated support                      */
    uint32_t finite;          /* finite logits in the row                             */
    uint32_t reserved;
    double support_mass;      /* sum of exp(z - z_max) over the support               */
    double uniform;           /* the Philox uniform the draw consumed                 */
} vi_sample_stats;

/* ---- device / library ----------------------------------------------------
 * Workspaces are caller-owned device memory of the size the matching
 * *_workspace_bytes returns.  A workspace must be zero-filled once before its
 * first use (its arrival counters and barriers start at zero); every kernel
 * leaves it reusable (self-resetting counters), so no per-call memset is needed.
 * Calls that share one workspace must be ordered on one stream. */

/* Fails with VI_ERR_DEVICE unless the current HIP device is gfx950. */
vi_status vi_init(void);
const char* vi_status_string(vi_status status);
/* Version of this ABI (bumped on any layout change). */
uint32_t vi_abi_version(void);

/* ---- greedy argmax --------------------------------------------------------
 * Replaces exl3_launch_greedy_packet (src/exl3/greedy_packet.cuh:256-272) and
 * the exact_row_score_kernel argmax (src/exl3/text_model.cu:11393-11420).
 * Per row: largest finite value, lowest id on ties, any non-finite flagged and
 * skipped; token = vocabulary when no value is finite.  Rows are unbounded
 * (the reference caps at 16). */
size_t vi_greedy_workspace_bytes(int rows, int vocabulary);
vi_status vi_greedy_rows(const void* logits, int dtype, int rows, int vocabulary,
                         int64_t row_stride, uint64_t serial, vi_greedy_row* out,
                         void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free variant of vi_greedy_rows, with no counterpart in the
 * reference: for callers that cannot allocate (code under HIP graph capture,
 * serving loops that forbid hipMalloc).  Same results as vi_greedy_rows; the
 * slice partials and arrival counters live in a 64 KiB device array of the
 * library (one per GPU, held until the process ends), which holds the
 * workspace of every shape (VI_ERR_WORKSPACE otherwise).  No call allocates
 * memory.  Every call on one GPU shares that array and leaves its contents
 * behind: calls that overlap on one GPU (other streams, other threads) race,
 * so order them on one stream.  `stream` must belong to the current device. */
vi_status vi_greedy_rows_noalloc(const void* logits, int dtype, int rows, int vocabulary,
                                 int64_t row_stride, uint64_t serial, vi_greedy_row* out,
                                 void* stream);

/* ---- exact top-k ------------------------------------------------------------
 * Replaces dflash2_topk16_for_test / launch_dflash_topk16_segmented
 * (src/exl3/dflash2_draft.cu:2366-2420; dflash2_draft.h:198-202).
 * Exact top-k (1 <= k <= 64, k <= vocabulary) in (value desc, id asc) order;
 * rows containing NaN keep the reference's serial-insertion semantics
 * (dflash2_draft.cu:1827-1862).  `logprobs` (optional) receives
 * value - logsumexp(row) (NaN for rows with a non-finite value);
 * `nonfinite_flag` (optional) is set to 1 when any value of any row is
 * non-finite (dflash_nonfinite_flag_kernel, dflash2_draft.cu:2473-2485). */
size_t vi_topk_workspace_bytes(int rows, int vocabulary, int k);
vi_status vi_topk_rows(const void* logits, int dtype, int rows, int vocabulary,
                       int64_t row_stride, int k, int64_t* ids, float* values,
                       float* logprobs, uint32_t* nonfinite_flag,
                       void* workspace, size_t workspace_bytes, void* stream);
/* The qualification entry with the reference's own shape
 * (dflash2_topk16_for_test, src/exl3/dflash2_draft.cu:2390-2420): top-16 of
 * fp16 rows [rows][vocab] (stride vocab) into ids / values [rows][16].  Like
 * the reference's, its scratch is the library's: allocated and zero-filled on
 * the first call on a device (again, larger, when a larger shape comes) and
 * kept until the process ends.  Calls on one device share that scratch (its
 * self-resetting counters too), so they must be ordered on one stream; the
 * library holds a lock from the choice of the buffer to the launch, so a call
 * from another thread that grows it cannot free it under a queued launch.
 * rows 0 is a no-op. */
vi_status vi_topk16_for_test(const uint16_t* logits, int rows, int vocab, int64_t* ids, float* values,
                             uint32_t* nonfinite_flag, void* stream);

/* ---- coupled sampled packet (reference semantics) ----------------------------
 * Replaces exl3_launch_sampled_packet (src/exl3/sampled_select.cuh:362-377):
 * presence-penalized top-min(top_k,20) candidates, min_p / top_p truncation and
 * the Gumbel-max draw keyed by (seed, first_key + depth[r], token).  `depths`
 * and `inputs` are host arrays of `rows` entries or NULL, exactly as the
 * reference's spans.  rows <= 16 (the reference's packet capacity). */
size_t vi_sampled_packet_workspace_bytes(int rows, int vocabulary);
vi_status vi_sampled_packet(const void* scores, int dtype, int rows, int vocabulary,
                            int64_t row_stride, const vi_device_sampling* cfg,
                            int first_key, const int32_t* depths, int n_depths,
                            const int32_t* inputs, int n_inputs, uint64_t serial,
                            vi_greedy_row* out, void* workspace, size_t workspace_bytes,
                            void* stream);

/* First-occurrence table maintenance; replaces exl3_presence_reset /
 * _truncate / _record (src/exl3/sampled_select.h:33-35,
 * src/exl3/text_model.cu:12139-12173). */
vi_status vi_presence_reset(int32_t* table, int vocabulary, void* stream);
vi_status vi_presence_truncate(int32_t* table, int vocabulary, int from, void* stream);
vi_status vi_presence_record(int32_t* table, int vocabulary, int first,
                             const int64_t* tokens, size_t count, void* stream);

/* ---- greedy-packet transport ------------------------------------------------
 * Replaces the engine's pending-packet readback (Exl3GreedyPacketTransfer and
 * submit_greedy_packet / finish_greedy_packet, src/exl3/text_model.cu:779-900,
 * 12225-12355) and its cross-context batch (Exl3EngineGreedyPacketBatch,
 * src/exl3/engine_greedy_packet_batch.h:17-60): a pool of `slots` pinned host
 * buffers of `max_rows` packet rows, each with a completion event.  submit
 * enqueues one device-to-host copy of `rows` contiguous device rows on `stream`
 * (the packets of any number of lanes laid end to end travel as one copy) and
 * returns the slot; query reports whether the copy completed; finish waits for
 * it, copies the rows to `out` (host) and frees the slot.  Every slot in flight:
 * VI_ERR_WORKSPACE.  A failed copy or wait returns VI_ERR_LAUNCH and retires
 * the slot.  Host-side allocation happens in create only; destroy waits for
 * copies still in flight.  Slots are guarded by a mutex (thread-safe). */
typedef struct vi_packet_transport vi_packet_transport;
vi_status vi_packet_transport_create(int slots, int max_rows, vi_packet_transport** out);
vi_status vi_packet_transport_destroy(vi_packet_transport* transport);
vi_status vi_packet_submit(vi_packet_transport* transport, const vi_greedy_row* device_rows, int rows,
                           void* stream, int* slot);
vi_status vi_packet_query(vi_packet_transport* transport, int slot, int* ready);
vi_status vi_packet_finish(vi_packet_transport* transport, int slot, vi_greedy_row* out, int rows);

/* ---- VeriCache row scores -----------------------------------------------------
 * Scoring of a verified block: per row r, the exact choice and the gap, in
 * logit units, by which the drafted token next[r] trails it (next < 0: gap 0).
 *
 * vi_row_scores replaces exact_row_score_kernel (src/exl3/text_model.cu:11393-11420):
 * greedy[r] = argmax over values greater than -Inf (NaN and -Inf never win, +Inf
 * can; lowest id on ties; vocabulary if none); gap[r] = max - logit(next[r]) for
 * next in [0, vocabulary) other than the argmax, else 0.
 *
 * vi_sampled_scores replaces exl3_sampled_score_kernel
 * (src/exl3/sampled_select.cuh:300-360): chosen[r] = the coupled draw of row r
 * at key first_key + r (no drafted path); gap[r] = T x the perturbed-value gap
 * when next[r] is in the support; outside it, infinite unless raising next's
 * logit by `tolerance` (>= 0) brings it into the support, then measured against
 * the best other support entry; temperature 0: max(0, best - penalized
 * logit(next)).  next[r] >= vocabulary gives an infinite gap.  Rows unbounded. */
size_t vi_row_scores_workspace_bytes(int rows, int vocabulary);
vi_status vi_row_scores(const void* logits, int dtype, int rows, int vocabulary, int64_t row_stride,
                        const int64_t* next, int64_t* greedy, float* gap,
                        void* workspace, size_t workspace_bytes, void* stream);
size_t vi_sampled_scores_workspace_bytes(int rows, int vocabulary);
vi_status vi_sampled_scores(const void* scores, int dtype, int rows, int vocabulary, int64_t row_stride,
                            const vi_device_sampling* cfg, int first_key, float tolerance,
                            const int64_t* next, int64_t* chosen, float* gap,
                            void* workspace, size_t workspace_bytes, void* stream);

/* ---- DFlash2 draft coupled proposal ---------------------------------------------
 * Replaces dflash_sampled_choice with DraftSelectSampling
 * (src/exl3/dflash2_draft.cu:2554-2610) for many lanes: per lane, draft positions
 * 0..positions-1 in order, position p choosing among its 16 candidates.  With
 * inv_temperature > 0: candidates equal to the lane's seed token, generated
 * before key = key_base + p (first_occurrence[token] < key) or proposed at an
 * earlier position lose presence_penalty; the penalized scores are ordered
 * (stable, descending), capped at top_k, cut by min_p / top_p over
 * exp(score/T - max) and the argmax of score/T + Gumbel(seed, key, token) over
 * that support is proposed.  Otherwise the first maximum of the scores wins (the
 * reference feeds its selector scores there).  scores: f32 [lanes][positions][16];
 * candidates: int64 [lanes][positions][16]; seed_tokens: int64 [lanes] (or
 * NULL); sampling: one record per lane (device memory); proposals: int64
 * [lanes][positions].  first_occurrence lookups are bounded by `vocabulary`. */
typedef struct vi_draft_sampling {   /* field-for-field DraftSelectSampling */
    float inv_temperature, top_p, min_p;
    int32_t top_k;
    uint64_t seed;
    int32_t key_base, reserved;
    float presence_penalty;
    int32_t reserved2;
    const int32_t* first_occurrence;   /* device int32[vocabulary] or NULL */
} vi_draft_sampling;
vi_status vi_draft_choice(int lanes, int positions, int vocabulary, const float* scores,
                          const int64_t* candidates, const int64_t* seed_tokens,
                          const vi_draft_sampling* sampling, int64_t* proposals, void* stream);

/* Fused selector chain; replaces dflash_selector_fused_chain_kernel
 * (src/exl3/dflash2_draft.cu:2615-2678), batched over lanes.  Lane l's anchor
 * starts at anchors[l]; at each position p the score of candidate c is
 * unary[l][p][c] + sum over r < 256 of pred[anchor][r] * hidden[l][p][r] *
 * succ[candidates[l][p][c]][r] (fp16 codebooks pred / succ [vocabulary][256],
 * fp16 hidden [lanes][positions][256], fp32 products (pred * hidden) * succ
 * summed across one 64-lane wave in a fixed order of this library's, so that a
 * near tie within the fp32 sums' rounding may resolve differently from the
 * reference's order), the first maximum is proposed and becomes the anchor.  A
 * lane whose sampling record has inv_temperature > 0 (sampling may be NULL: all
 * greedy) proposes by the coupled sampled choice over the unary scores instead,
 * as vi_draft_choice does, with anchors[l] as its seed token.  An anchor or a
 * candidate outside [0, vocabulary) ends the lane's chain: that position and
 * every later one get -1.  All pointers are device memory. */
vi_status vi_selector_chain(int lanes, int positions, int vocabulary, const int64_t* anchors,
                            const int64_t* candidates, const float* unary, const void* hidden,
                            const void* pred_codebook, const void* succ_codebook,
                            const vi_draft_sampling* sampling, int64_t* proposals, void* stream);

/* ---- verification tree (host function, no device work) ---------------------
 * Replaces exl3_build_verification_tree (src/exl3/verification_tree.h:44-112):
 * a chain prefix of the drafts plus sibling leaves chosen to maximise
 * (1 + expected accepted tokens) / (1 + row_cost * rows) from the draft's
 * top-16 unary softmax.  Host pointers: drafts int64[depth]; candidate_ids
 * int64[depth][16] and candidate_unary float[depth][16] in unary order (the
 * top-16 output of vi_topk_rows after D2H); budget = verifier rows besides
 * the anchor.  Outputs: *chain_drafts, and *sibling_count (<= budget) leaves
 * in sibling_tokens / sibling_offsets (capacity `budget` each).  row_cost:
 * the reference default is 0.0141 (0 for batched multi-agent rounds). */
vi_status vi_build_verification_tree(const int64_t* drafts, int depth, const int64_t* candidate_ids,
                                     const float* candidate_unary, int budget, int max_siblings, float row_cost,
                                     int32_t* chain_drafts, int64_t* sibling_tokens, int32_t* sibling_offsets,
                                     int32_t* sibling_count);

/* ---- batched sampler (extended semantics) ----------------------------------
 * New batched entry for many lanes (the reference's packet stops at 16 rows,
 * sampled_select.cuh:200-216): per-row temperature, top-k, top-p, min-p,
 * repetition / presence / frequency penalties over the lane's int32 history
 * histories[history_offsets[r] .. history_offsets[r+1]), and a Philox4x32-10
 * inverse-CDF draw keyed by (seed, lane, position).  `params`, `histories`,
 * `history_offsets` and every output are device pointers.  Optional outputs:
 * `uniforms` (double[rows]), `probs` (float[rows][probs_stride], the filtered
 * distribution), `stats`.  `max_history` bounds every row's history length
 * (it sizes the workspace); a longer history fails that row.  Supported:
 * bf16, fp16 and fp32 logits, vocabularies up to 524,288 on the
 * full-vocabulary route (top_k 0 or > 64 with temperature > 0).  A row the
 * kernels cannot finish gets token -1 and VI_FLAG_ERROR in its stats. */
/* route_mask: which kernels run.  VI_ROUTE_TOPK serves rows with temperature 0
 * or 1 <= top_k <= 64, VI_ROUTE_FULL every other row; rows whose route is not in
 * the mask are left unwritten.  VI_ROUTE_ALL (or 0) runs both. */
enum { VI_ROUTE_TOPK = 1u, VI_ROUTE_FULL = 2u, VI_ROUTE_ALL = 3u };
size_t vi_sample_workspace_bytes(int rows, int vocabulary, int64_t max_history);
vi_status vi_sample_rows(const void* logits, int dtype, int rows, int vocabulary,
                         int64_t row_stride, const vi_row_params* params,
                         const int32_t* histories, const int64_t* history_offsets,
                         int64_t max_history, int32_t* tokens, double* uniforms, float* probs,
                         int64_t probs_stride, vi_sample_stats* stats, uint32_t route_mask,
                         void* workspace, size_t workspace_bytes, void* stream);

/* ---- per-lane penalty state --------------------------------------------------
 * Occurrence counts of each lane's generated tokens, kept current on the device
 * so that the sampler reads them instead of scanning the lane's history at
 * every step.  Generalizes the reference's incremental first-occurrence table
 * (exl3_presence_reset / _truncate / _record, src/exl3/sampled_select.h:33-35,
 * src/exl3/text_model.cu:12139-12173, driven by PresenceTrack::sync,
 * src/exl3/exl3_engine_core.cpp:106-133) from presence to counts, which the
 * repetition and frequency penalties need.
 *
 * One lane's state is vi_penalty_state_bytes(vocabulary, slots) bytes; `states`
 * holds `lanes` of them back to back (lane l at l * bytes), in device memory.
 * slots: power of two >= 64, at least twice the distinct tokens a lane records
 * between resets (a removed token keeps its slot).  reset: every lane empty.
 * update: sign +1 records, -1 removes, per lane the tokens
 * tokens[offsets[l] .. offsets[l+1]) (device int32 / int64 arrays), or, with
 * offsets NULL, the single token tokens[l] (a negative one is skipped: the
 * sampler's output of a failed row).  Recording a token outside
 * [0, vocabulary) sets VI_FLAG_BAD_HISTORY on the lane (the token is ignored,
 * as in a history); a full table or removing a token that is not there sets
 * VI_FLAG_ERROR.  Both flags stay until reset and are reported by every row
 * that takes penalties from the lane (such a row fails on ERROR).  Calls on one set of
 * states run in stream order; vocabulary and slots must be the same in every
 * call on a state, the sampler's included. */
size_t vi_penalty_state_bytes(int vocabulary, int slots);
vi_status vi_penalty_state_reset(void* states, int lanes, int vocabulary, int slots, void* stream);
vi_status vi_penalty_state_update(void* states, int lanes, int vocabulary, int slots, const int32_t* tokens,
                                  const int64_t* offsets, int sign, void* stream);
/* vi_sample_rows with the penalties taken from the lanes' penalty states (row r
 * uses lane r's state) instead of histories: results are those of vi_sample_rows
 * over any history with the same occurrence counts.  record = 1 also appends
 * each row's sampled token (when it is in [0, vocabulary)) to its lane's state,
 * in the same launch: a decode step is then one call.  Workspace:
 * vi_sample_workspace_bytes(rows, vocabulary, 0).  No limit on a lane's
 * distinct tokens or counts beyond the state's own (its hash slots). */
vi_status vi_sample_rows_state(const void* logits, int dtype, int rows, int vocabulary, int64_t row_stride,
                               const vi_row_params* params, void* states, int slots, int record, int32_t* tokens,
                               double* uniforms, float* probs, int64_t probs_stride, vi_sample_stats* stats,
                               uint32_t route_mask, void* workspace, size_t workspace_bytes, void* stream);

/* ---- DFlash2 verification ---------------------------------------------------
 * Replaces the host decisions decide_exl3_outer_prefix
 * (src/exl3/exact_outer_reference.h:68-82) in greedy mode and
 * Exl3IndependentAcceptanceReference::evaluate
 * (src/exl3/sampled_acceptance_reference.h:48-88) in sampled mode, applied per
 * lane over `drafts` drafted positions with the target softmax fused in.
 * target: [lanes][target_rows][target_stride], target_rows = drafts or
 * drafts + 1 (bonus row); draft: [lanes][drafts][draft_stride];
 * drafted: int32 [lanes][drafts]; params: one vi_row_params per lane (its
 * `position` is the absolute position of drafted row 0); terminal: optional
 * device list of stop tokens.  Outputs: accepted[lanes], committed
 * [lanes][drafts + 1] (unused slots = -1), committed_count[lanes],
 * lane_flags[lanes] (optional).  Sampled mode takes p and q from top-k lists
 * on lanes with 1 <= top_k <= 64 and from the full-vocabulary sampler's
 * filtered distributions on the others (top_k 0 or above 64; vocabularies up
 * to 524,288, 16-byte aligned 16-bit rows or 4-byte aligned fp32 rows).
 * VI_VERIFY_SAMPLED_TOPK is sampled mode for batches whose sampled lanes all
 * have 1 <= top_k <= 64 (the full-vocabulary launches are skipped): any other
 * sampled lane is then refused on the device (accepted 0, committed_count 0,
 * every committed slot -1, lane_flags VI_FLAG_ERROR), as it is when the
 * full-vocabulary path cannot take the rows. */
enum { VI_VERIFY_GREEDY = 0, VI_VERIFY_SAMPLED = 1, VI_VERIFY_SAMPLED_TOPK = 2 };
size_t vi_verify_workspace_bytes(int lanes, int drafts, int vocabulary);
vi_status vi_verify_rows(int mode, const void* target, int target_dtype,
                         int64_t target_stride, int target_rows,
                         const void* draft, int draft_dtype, int64_t draft_stride,
                         int lanes, int drafts, int vocabulary,
                         const int32_t* drafted, const vi_row_params* params,
                         const int64_t* terminal, int n_terminal,
                         int32_t* accepted, int32_t* committed,
                         int32_t* committed_count, uint32_t* lane_flags,
                         void* workspace, size_t workspace_bytes, void* stream);

/* ---- measurement helpers ------------------------------------------------------
 * Stream-read probe (the gfx950 analogue of tools/hbm_bandwidth_probe.cu:1-45):
 * reads `bytes` from `src` with 16-byte loads and writes one word per
 * workgroup to `sink` (2048 words). */
vi_status vi_probe_read(const void* src, size_t bytes, uint32_t* sink, void* stream);
/* Plain device copy of `bytes` (16-byte aligned), the FETCH_SIZE calibration
 * kernel. */
vi_status vi_probe_copy(void* dst, const void* src, size_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VOIDINFER_SAMPLING_H */
