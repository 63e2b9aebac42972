// draft.hip — the DFlash2 draft's proposals: the coupled sampled choice
// (DraftSelectSampling / dflash_sampled_choice, src/exl3/dflash2_draft.cu:2554-2610)
// over given scores, and the fused selector chain that computes the scores
// (dflash_selector_fused_chain_kernel, :2615-2678).
//
// Each lane proposes one token per draft position from that position's 16
// candidates, in position order (an earlier proposal is part of the presence
// history of the later ones).  With inv_temperature > 0 the proposal is the
// token the target's coupled sampler most likely picks: the candidates'
// presence-penalized scores are ordered (stable, score descending), truncated
// like the target sampler (top_k, then min_p / top_p of exp(score/T - max))
// and the argmax of score/T + Gumbel(seed, key_base + position, token) over the
// support wins.  Otherwise the raw scores' first maximum wins.  One thread per
// lane; the per-thread candidate arrays live in LDS.
#include <math.h>

#include "vi_device.h"
#include "vi_internal.h"

namespace vi {
namespace {

constexpr int kDraftK = 16;       // candidates per draft position
constexpr int kDraftLanes = 64;   // lanes per workgroup

// The coupled sampled choice at one draft position (dflash_sampled_choice,
// src/exl3/dflash2_draft.cu:2570-2610): index of the chosen candidate.  `chain`
// holds the `pos` earlier proposals; val / prob / order are per-thread LDS rows.
__device__ __forceinline__ int sampled_pick(const vi_draft_sampling& s, int pos, int vocabulary, const float* sc,
                                            const int64_t* cd, int64_t seed_token, const int64_t* chain, float* val,
                                            float* prob, int* order) {
    const int key = s.key_base + pos;
    for (int c = 0; c < kDraftK; ++c) {
        float v = sc[c];
        if (s.presence_penalty != 0.0f) {
            const int64_t token = cd[c];
            bool seen = token == seed_token ||
                        (s.first_occurrence && token >= 0 && token < vocabulary && s.first_occurrence[token] < key);
            for (int i = 0; i < pos && !seen; ++i) seen = chain[i] == token;
            if (seen) v -= s.presence_penalty;
        }
        val[c] = v;
        order[c] = c;
    }
    for (int i = 1; i < kDraftK; ++i) {   // stable insertion sort, score descending
        const int o = order[i];
        int j = i;
        while (j > 0 && val[o] > val[order[j - 1]]) { order[j] = order[j - 1]; --j; }
        order[j] = o;
    }
    int cap = kDraftK;
    if (s.top_k > 0 && s.top_k < cap) cap = s.top_k;
    const float m = val[order[0]] * s.inv_temperature;
    float sum = 0.0f;
    for (int j = 0; j < cap; ++j) { prob[j] = expf(fmaf(val[order[j]], s.inv_temperature, -m)); sum += prob[j]; }
    const float min_p_thresh = s.min_p > 0.0f ? s.min_p * prob[0] : -1.0f;
    float cum = 0.0f;
    int support = 0;
    for (int j = 0; j < cap; ++j) {
        if (min_p_thresh >= 0.0f && prob[j] < min_p_thresh) break;
        cum += prob[j];
        support = j + 1;
        if (s.top_p < 1.0f && cum >= s.top_p * sum) break;
    }
    if (support < 1) support = 1;
    int best = order[0];
    float best_value = -kInfF;
    for (int j = 0; j < support; ++j) {
        const int c = order[j];
        const float v = fmaf(val[c], s.inv_temperature, gumbel(s.seed, key, int(cd[c])));
        if (v > best_value) { best_value = v; best = c; }
    }
    return best;
}

// First maximum of 16 scores (NaN never replaces the incumbent).
__device__ __forceinline__ int first_max16(const float* sc) {
    int best = 0;
    float bs = sc[0];
    for (int c = 1; c < kDraftK; ++c)
        if (sc[c] > bs) { bs = sc[c]; best = c; }
    return best;
}

__global__ __launch_bounds__(kDraftLanes) void draft_choice_kernel(int lanes, int positions, int vocabulary,
                                                                  const float* scores, const int64_t* candidates,
                                                                  const int64_t* seed_tokens,
                                                                  const vi_draft_sampling* sampling,
                                                                  int64_t* proposals) {
    __shared__ float s_val[kDraftLanes][kDraftK + 1];
    __shared__ float s_prob[kDraftLanes][kDraftK + 1];
    __shared__ int s_ord[kDraftLanes][kDraftK + 1];
    const int t = threadIdx.x, l = blockIdx.x * kDraftLanes + t;
    if (l >= lanes) return;
    const vi_draft_sampling s = sampling[l];
    const int64_t seed_token = seed_tokens ? seed_tokens[l] : -1;
    int64_t* out = proposals + size_t(l) * positions;
    for (int pos = 0; pos < positions; ++pos) {
        const size_t at = (size_t(l) * positions + pos) * kDraftK;
        const float* sc = scores + at;
        const int64_t* cd = candidates + at;
        const int best = s.inv_temperature > 0.0f
                             ? sampled_pick(s, pos, vocabulary, sc, cd, seed_token, out, s_val[t], s_prob[t], s_ord[t])
                             : first_max16(sc);
        out[pos] = cd[best];
    }
}

// The fused selector chain (dflash_selector_fused_chain_kernel,
// src/exl3/dflash2_draft.cu:2615-2678): per draft position, candidate c's
// score is unary[c] + sum_r pred[anchor][r] * hidden[pos][r] * succ[cand_c][r]
// (rank 256, fp16 codebooks, fp32 arithmetic), and the first maximum becomes
// the proposal and the next position's anchor.  With inv_temperature > 0 the
// coupled sampled choice over the unary scores decides instead (the selector's
// terms are not calibrated as logits).  One workgroup per lane; candidate c is
// reduced by 32 lanes (half a wave), in the order the reference reduces it:
// each lane sums its 8 products pairwise (k, k+4), (k, k+2), (0, 1), then a
// shuffle-down tree over offsets 16 .. 1.
constexpr int kRank = 256;
constexpr int kChainThreads = kDraftK * 32;

__global__ __launch_bounds__(kChainThreads) void selector_chain_kernel(
    int lanes, int positions, int vocabulary, const int64_t* anchors, const int64_t* candidates, const float* unary,
    const uint16_t* hidden, const uint16_t* pred_cb, const uint16_t* succ_cb, const vi_draft_sampling* sampling,
    int64_t* proposals) {
    __shared__ float s_score[kDraftK];
    __shared__ float s_val[kDraftK + 1], s_prob[kDraftK + 1];
    __shared__ int s_ord[kDraftK + 1];
    __shared__ int64_t s_anchor;
    __shared__ int s_bad;
    const int l = blockIdx.x, t = threadIdx.x, c = t >> 5, sub = t & 31;
    if (l >= lanes) return;
    const int64_t seed_token = anchors[l];
    const vi_draft_sampling s = sampling ? sampling[l] : vi_draft_sampling{};
    const bool sampled = sampling && s.inv_temperature > 0.0f;
    int64_t* out = proposals + size_t(l) * positions;
    if (t == 0) { s_anchor = seed_token; s_bad = seed_token < 0 || seed_token >= vocabulary; }
    __syncthreads();
    for (int pos = 0; pos < positions; ++pos) {
        const size_t at = size_t(l) * positions + pos;
        const int64_t cand = candidates[at * kDraftK + c];
        if (sub == 0 && (cand < 0 || cand >= vocabulary)) atomicOr(&s_bad, 1);
        __syncthreads();
        if (s_bad) {   // an anchor or a candidate outside the codebooks: no proposal from here on
            if (t == 0) out[pos] = -1;
            continue;
        }
        if (!sampled) {
            const uint16_t* pr = pred_cb + size_t(s_anchor) * kRank;
            const uint16_t* hr = hidden + at * kRank;
            const uint16_t* sr = succ_cb + size_t(cand) * kRank;
            float r[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int rank = sub + 32 * k;
                r[k] = Elem<VI_F16>::decode(pr[rank]) * Elem<VI_F16>::decode(hr[rank]) * Elem<VI_F16>::decode(sr[rank]);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) r[k] += r[k + 4];
#pragma unroll
            for (int k = 0; k < 2; ++k) r[k] += r[k + 2];
            float v = r[0] + r[1];
            for (int off = 16; off > 0; off >>= 1) v += __shfl_down(v, off, 32);
            if (sub == 0) s_score[c] = unary[at * kDraftK + c] + v;
        }
        __syncthreads();
        if (t == 0) {
            const int best = sampled ? sampled_pick(s, pos, vocabulary, unary + at * kDraftK, candidates + at * kDraftK,
                                                    seed_token, out, s_val, s_prob, s_ord)
                                     : first_max16(s_score);
            const int64_t chosen = candidates[at * kDraftK + best];
            out[pos] = chosen;
            s_anchor = chosen;
        }
        __syncthreads();
    }
}

}  // namespace

vi_status launch_draft_choice(int lanes, int positions, int vocabulary, const float* scores,
                              const int64_t* candidates, const int64_t* seed_tokens,
                              const vi_draft_sampling* sampling, int64_t* proposals, hipStream_t stream) {
    hipLaunchKernelGGL(draft_choice_kernel, dim3((lanes + kDraftLanes - 1) / kDraftLanes), dim3(kDraftLanes), 0,
                       stream, lanes, positions, vocabulary, scores, candidates, seed_tokens, sampling, proposals);
    return launch_status();
}

vi_status launch_selector_chain(int lanes, int positions, int vocabulary, const int64_t* anchors,
                                const int64_t* candidates, const float* unary, const void* hidden,
                                const void* pred_codebook, const void* succ_codebook,
                                const vi_draft_sampling* sampling, int64_t* proposals, hipStream_t stream) {
    hipLaunchKernelGGL(selector_chain_kernel, dim3(lanes), dim3(kChainThreads), 0, stream, lanes, positions, vocabulary,
                       anchors, candidates, unary, static_cast<const uint16_t*>(hidden),
                       static_cast<const uint16_t*>(pred_codebook), static_cast<const uint16_t*>(succ_codebook),
                       sampling, proposals);
    return launch_status();
}

}  // namespace vi
