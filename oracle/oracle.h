/*
 * oracle.h — CPU restatement of The8Darkness/voidinfer's token-sampling path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: tests/, the smoke()
 * entry of __graft_entry__.py and the cpu_baseline leg of bench.py may load it;
 * the product library (voidinfer_amd) never does.  Every function cites the
 * reference file:line whose behaviour it restates.  Semantic extensions that the
 * reference does not implement (full-vocabulary filtering, repetition and
 * frequency penalties, Philox inverse-CDF draws, log-probs, device verification)
 * are marked EXTENSION; the tests under tests/ name what pins each of them.
 */
#ifndef VOIDINFER_ORACLE_H
#define VOIDINFER_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/voidinfer_sampling.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Element decode to fp32 (exact for bf16 / fp16). */
float or_decode(int dtype, uint32_t bits);
/* fp32 -> storage dtype, round to nearest even (EXTENSION helper). */
uint32_t or_round_to_dtype(int dtype, float value);
/* Order-preserving 32-bit key of an fp32 value (-0 folded onto +0). */
uint32_t or_order_key(float value);

/* SplitMix64 finalizer (sampled_select.cuh:41-46; request_sampling_state.h:113-118). */
uint64_t or_splitmix64(uint64_t x);
/* Gumbel(0,1) of (seed, key, token) (sampled_select.cuh:47-54). */
float or_gumbel(uint64_t seed, int32_t key, int32_t token);
/* Philox4x32-10 (Salmon et al., SC'11) — EXTENSION RNG. */
void or_philox4x32_10(const uint32_t counter[4], const uint32_t key[2], uint32_t out[4]);
/* 53-bit uniform of (seed, lane, position, purpose); counter =
 * (position, 0, lane, purpose), key = seed.  Purpose 0 = sampler draw,
 * 1 = acceptance draw, 2 = correction draw. */
double or_uniform(uint64_t seed, uint32_t lane, int32_t position, uint32_t purpose);

/* Greedy packet rows (greedy_packet.cuh:15-77). */
int or_greedy_rows(const void* logits, int dtype, int rows, int vocabulary,
                   int64_t row_stride, uint64_t serial, vi_greedy_row* out);
/* Host-logit CPU greedy (branch_reference.h:23-31): first maximum; -1 when a
 * value is non-finite (the reference throws std::runtime_error). */
int64_t or_cpu_greedy(const float* logits, int64_t vocabulary);

/* Exact top-k, (value desc, id asc), NaN rows in serial insertion order
 * (dflash2_draft.cu:1827-1862; test_exl3_dflash2_topk.h:11-37).  logprobs:
 * EXTENSION (value - fp64 logsumexp; NaN on rows with a non-finite value). */
int or_topk_rows(const void* logits, int dtype, int rows, int vocabulary, int64_t row_stride,
                 int k, int64_t* ids, float* values, float* logprobs, uint32_t* nonfinite);

/* Reference-mode coupled packet (sampled_select.cuh:79-116,121-193,218-279,362-377).
 * cfg->first_occurrence is a HOST pointer here.  detail (optional, rows
 * entries) exposes the candidate list and support for tests. */
typedef struct or_packet_detail {
    int32_t cap, support, selected, key;
    float cand_val[20];
    int32_t cand_idx[20];
    float value[20];
    float prob[20];
    float sum;
} or_packet_detail;
int or_sampled_packet(const void* scores, int dtype, int rows, int vocabulary, int64_t row_stride,
                      const vi_device_sampling* cfg, int first_key, const int32_t* depths,
                      int n_depths, const int32_t* inputs, int n_inputs, uint64_t serial,
                      vi_greedy_row* out, or_packet_detail* detail);

/* VeriCache sampled row scores (exl3_sampled_score_kernel,
 * sampled_select.cuh:300-360): chosen token and gap of next[r] in logit units;
 * row r uses key first_key + r.  cfg->first_occurrence is a HOST pointer. */
int or_sampled_scores(const void* scores, int dtype, int rows, int vocabulary, int64_t row_stride,
                      const vi_device_sampling* cfg, int first_key, float tolerance, const int64_t* next,
                      int64_t* chosen, float* gap);
/* DFlash2 draft coupled proposal (dflash_sampled_choice, dflash2_draft.cu:2554-2610);
 * host pointers (first_occurrence included), layouts as vi_draft_choice. */
/* Fused selector chain (dflash_selector_fused_chain_kernel, dflash2_draft.cu:2615-2678), layouts as
 * vi_selector_chain; fp16 arrays as uint16 bit patterns; sampling may be NULL. */
int or_selector_chain(int lanes, int positions, int vocabulary, const int64_t* anchors, const int64_t* candidates,
                      const float* unary, const uint16_t* hidden, const uint16_t* pred_codebook,
                      const uint16_t* succ_codebook, const vi_draft_sampling* sampling, int64_t* proposals);
int or_draft_choice(int lanes, int positions, int vocabulary, const float* scores, const int64_t* candidates,
                    const int64_t* seed_tokens, const vi_draft_sampling* sampling, int64_t* proposals);
/* VeriCache exact row scores (exact_row_score_kernel, text_model.cu:11393-11420). */
int or_row_scores(const void* logits, int dtype, int rows, int vocabulary, int64_t row_stride,
                  const int64_t* next, int64_t* greedy, float* gap);

/* EXTENSION: batched sampler.  margins (optional, 4 doubles per row):
 * [0] draw margin  |cum - u*S_n| / S_n at the chosen token's boundaries,
 * [1] top-p margin |cum - top_p*S_cap| / S_cap at the cut,
 * [2] min-p margin |w - min_p| at the cut,
 * [3] the index of the chosen token in the sorted support.
 * threads <= 0 uses hardware_concurrency(). */
int or_sample_rows(const void* logits, int dtype, int rows, int vocabulary, int64_t row_stride,
                   const vi_row_params* params, const int32_t* histories,
                   const int64_t* history_offsets, int32_t* tokens, double* uniforms,
                   float* probs, int64_t probs_stride, vi_sample_stats* stats,
                   double* margins, int threads);

/* FP64 rejection-sampling acceptance (sampled_acceptance_reference.h:48-88).
 * Returns 0 on success, 1 for std::invalid_argument, 2 for std::logic_error. */
typedef struct or_accept_outcome {
    int32_t accepted, correction_draw_used;
    uint32_t token, reserved;
    double acceptance_probability;
} or_accept_outcome;
int or_accept(const double* target_p, const double* draft_q, int64_t vocabulary,
              uint32_t proposed_token, double acceptance_draw, double correction_draw,
              or_accept_outcome* out, double* residual /* optional [vocabulary] */);

/* Greedy longest-prefix decision (exact_outer_reference.h:68-82).  Returns 1
 * for std::invalid_argument. */
int or_outer_prefix(const int64_t* target_path, const int64_t* tentative, int n,
                    const int64_t* terminal, int n_terminal, int64_t* committed,
                    int* n_committed, int* accepted, int* rejected, int* stopped);

/* DFlash2 verification tree (verification_tree.h:44-112): chain length and
 * sibling leaves (tokens, offsets; *n_siblings of them, capacity `budget`). */
int or_build_verification_tree(const int64_t* drafts, int depth, const int64_t* candidate_ids,
                               const float* candidate_unary, int budget, int max_siblings, float row_cost,
                               int* chain_drafts, int64_t* sibling_tokens, int* sibling_offsets, int* n_siblings);

/* EXTENSION: lane verification (greedy prefix / sampled rejection with the
 * target distribution computed from logits), same arguments as
 * vi_verify_rows but host pointers. */
int or_verify_rows(int mode, const void* target, int target_dtype, int64_t target_stride,
                   int target_rows, const void* draft, int draft_dtype, int64_t draft_stride,
                   int lanes, int drafts, int vocabulary, const int32_t* drafted,
                   const vi_row_params* params, const int64_t* terminal, int n_terminal,
                   int32_t* accepted, int32_t* committed, int32_t* committed_count,
                   uint32_t* lane_flags, double* accept_margins /* optional [lanes][drafts] */,
                   int threads);
/* accept_margins (sampled mode): per decided position, the smallest distance
 * at which the outcome would turn: |u_a - min(1, p/q)|, the top-p / min-p cut
 * margins of the target and draft rows, at a rejection |u_c - cumulative
 * residual| on either side of the correction, and on the last position of a
 * lane that reached the bonus row, that draw's margins. */

/* EXTENSION: filtered distribution of one row (the sampler's p), dense fp64. */
int or_row_distribution(const void* row, int dtype, int vocabulary, const vi_row_params* params,
                        double* p_out, uint32_t* support);

#ifdef __cplusplus
}
#endif

#endif
