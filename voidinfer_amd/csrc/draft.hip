// draft.hip — the DFlash2 draft's coupled sampled proposal
// (DraftSelectSampling / dflash_sampled_choice, src/exl3/dflash2_draft.cu:2554-2610).
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
    float* val = s_val[t];
    float* prob = s_prob[t];
    int* order = s_ord[t];
    int64_t* out = proposals + size_t(l) * positions;
    for (int pos = 0; pos < positions; ++pos) {
        const size_t at = (size_t(l) * positions + pos) * kDraftK;
        const float* sc = scores + at;
        const int64_t* cd = candidates + at;
        int best = 0;
        if (!(s.inv_temperature > 0.0f)) {
            float bs = sc[0];
            for (int c = 1; c < kDraftK; ++c)
                if (sc[c] > bs) { bs = sc[c]; best = c; }
        } else {
            const int key = s.key_base + pos;
            for (int c = 0; c < kDraftK; ++c) {
                float v = sc[c];
                if (s.presence_penalty != 0.0f) {
                    const int64_t token = cd[c];
                    bool seen = token == seed_token ||
                                (s.first_occurrence && token >= 0 && token < vocabulary && s.first_occurrence[token] < key);
                    for (int i = 0; i < pos && !seen; ++i) seen = out[i] == token;
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
            best = order[0];
            float best_value = -kInfF;
            for (int j = 0; j < support; ++j) {
                const int c = order[j];
                const float v = fmaf(val[c], s.inv_temperature, gumbel(s.seed, key, int(cd[c])));
                if (v > best_value) { best_value = v; best = c; }
            }
        }
        out[pos] = cd[best];
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

}  // namespace vi
