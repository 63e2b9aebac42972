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
// (rank 256, fp16 codebooks, fp32 arithmetic, each product rounded as
// (pred * hidden) * succ), and the first maximum becomes the proposal and the
// next position's anchor.  With inv_temperature > 0 the coupled sampled choice
// over the unary scores decides instead (the selector's terms are not
// calibrated as logits).
//
// One wave per lane, the rank-256 dot in registers: lane k holds ranks
// 4k .. 4k + 3 of pred[anchor] * hidden[pos] and of every candidate's succ row
// (8-byte loads, each candidate row read by the wave in one 512-byte sweep);
// the 16 candidate sums are reduced across the wave with DPP in a fixed order.
// The next anchor is one of this position's candidates, so their pred rows are
// loaded with their succ rows and the chosen one is kept: no load waits on the
// choice.  The order of the fp32 sums is this kernel's own; near ties may
// therefore resolve differently from another order, within the sums'
// rounding.
constexpr int kRank = 256;
constexpr int kChainWaves = 4;                     // lanes per workgroup, one wave each
constexpr int kChainThreads = kChainWaves * kWave;
constexpr int kRanksPerLane = kRank / kWave;       // 4
static_assert(kRanksPerLane == 4, "four fp16 ranks = one 8-byte load");

// ranks 4k .. 4k + 3 of an fp16 row, as fp32
__device__ __forceinline__ float4 rank4(const uint16_t* row, int k) {
    const uint2 v = *reinterpret_cast<const uint2*>(row + kRanksPerLane * k);
    return make_float4(Elem<VI_F16>::decode(v.x & 0xffffu), Elem<VI_F16>::decode(v.x >> 16),
                       Elem<VI_F16>::decode(v.y & 0xffffu), Elem<VI_F16>::decode(v.y >> 16));
}

__global__ __launch_bounds__(kChainThreads) void selector_chain_kernel(
    int lanes, int positions, int vocabulary, const int64_t* anchors, const int64_t* candidates, const float* unary,
    const uint16_t* hidden, const uint16_t* pred_cb, const uint16_t* succ_cb, const vi_draft_sampling* sampling,
    int64_t* proposals) {
    __shared__ float s_val[kChainWaves][kDraftK + 1], s_prob[kChainWaves][kDraftK + 1];
    __shared__ int s_ord[kChainWaves][kDraftK + 1];
    const int w = threadIdx.x / kWave, k = lane_id();
    const int l = blockIdx.x * kChainWaves + w;
    if (l >= lanes) return;   // (a whole wave)
    const int64_t seed_token = anchors[l];
    const vi_draft_sampling smp = sampling ? sampling[l] : vi_draft_sampling{};
    const bool sampled = sampling && smp.inv_temperature > 0.0f;
    int64_t* out = proposals + size_t(l) * positions;
    bool bad = seed_token < 0 || seed_token >= vocabulary;
    // pred[anchor] of the current position (ranks 4k .. 4k + 3)
    float4 pa = bad || sampled ? make_float4(0.f, 0.f, 0.f, 0.f) : rank4(pred_cb + size_t(seed_token) * kRank, k);
    for (int pos = 0; pos < positions; ++pos) {
        const size_t at = size_t(l) * positions + pos;
        const int64_t* cd = candidates + at * kDraftK;
        int64_t cand[kDraftK];
#pragma unroll
        for (int c = 0; c < kDraftK; ++c) {
            cand[c] = cd[c];
            bad = bad || cand[c] < 0 || cand[c] >= vocabulary;
        }
        if (bad) {   // an anchor or a candidate outside the codebooks: no proposal from here on
            if (k == 0) out[pos] = -1;
            continue;
        }
        int best = 0;
        if (sampled) {
            if (k == 0)
                best = sampled_pick(smp, pos, vocabulary, unary + at * kDraftK, cd, seed_token, out, s_val[w],
                                    s_prob[w], s_ord[w]);
            best = __builtin_amdgcn_readfirstlane(best);
        } else {
            // every load of this position first: hidden, the candidates' succ rows
            // and their pred rows (the next anchor's)
            const float4 h = rank4(hidden + at * kRank, k);
            float4 sv[kDraftK], pv[kDraftK];
#pragma unroll
            for (int c = 0; c < kDraftK; ++c) {
                sv[c] = rank4(succ_cb + size_t(cand[c]) * kRank, k);
                pv[c] = rank4(pred_cb + size_t(cand[c]) * kRank, k);
            }
            const float4 ah = make_float4(pa.x * h.x, pa.y * h.y, pa.z * h.z, pa.w * h.w);
            float score[kDraftK];
#pragma unroll
            for (int c = 0; c < kDraftK; ++c) {
                const float part = (ah.x * sv[c].x + ah.y * sv[c].y) + (ah.z * sv[c].z + ah.w * sv[c].w);
                score[c] = unary[at * kDraftK + c] + wave_sum_f32(part);
            }
            // first maximum (NaN never replaces the incumbent); scores are wave-uniform
            float bs = score[0];
#pragma unroll
            for (int c = 1; c < kDraftK; ++c)
                if (score[c] > bs) { bs = score[c]; best = c; }
            // the chosen candidate's pred row is the next position's anchor row
#pragma unroll
            for (int c = 0; c < kDraftK; ++c)
                if (c == best) pa = pv[c];
        }
        if (k == 0) out[pos] = cand[best];
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
    hipLaunchKernelGGL(selector_chain_kernel, dim3((lanes + kChainWaves - 1) / kChainWaves), dim3(kChainThreads), 0,
                       stream, lanes, positions, vocabulary,
                       anchors, candidates, unary, static_cast<const uint16_t*>(hidden),
                       static_cast<const uint16_t*>(pred_codebook), static_cast<const uint16_t*>(succ_codebook),
                       sampling, proposals);
    return launch_status();
}

}  // namespace vi
