// topk.hip — exact top-k selection over logit rows and the samplers built on it.
//
// One kernel family, four consumers:
//  * kModeTopk   — DFlash2 draft top-k (dflash2_draft.cu:1827-2342): ids and raw
//                  values in (value desc, id asc) order, NaN rows in the serial
//                  insertion order of dflash_topk16_serial_row, plus log-probs.
//  * kModePacket — the coupled reference sampler (sampled_select.cuh:79-279):
//                  presence-penalized top-min(top_k,20) candidates, min_p/top_p
//                  truncation and the Gumbel-max draw.
//  * kModeSample — rows of the batched sampler whose support lies in a top-k
//                  list (1 <= top_k <= 64, or temperature 0).
//  * kModeVerify — the sorted lists of sampled verification's target and draft
//                  rows.
//
// Shape: grid (slices, rows), 256 threads (4 waves), at most 32 slices per row.
// Each wave keeps a sorted top-K list distributed over its lanes (lane i = rank
// i, K <= 64).  The slice is read a batch at a time (four 16-byte vectors per
// lane, the next batch requested first); a batch's vector maxima are compared
// with a gate — the list's K-th entry, and a lower bound on the row's K-th best
// taken from the workgroup's first batch — and only vectors that reach it are
// looked at element by element.  Candidates are inserted with a ballot and a
// DPP wave shift (top-k and verification modes) or staged per wave and merged
// in bulk (sampler rows).  Lists merge by bitonic networks (ds_bpermute lane
// exchanges): the four wave lists as a tree through LDS, each workgroup
// publishes its slice list, and the last workgroup of a row to arrive
// (self-resetting counter) tree-merges the slice lists and finishes the row.
// Roofline: HBM, V x sizeof(logit) per row (+ the history for penalties); the
// kernels are VALU-issue bound in practice (decode, maxima, the log-sum-exp).
#include <math.h>

#include <algorithm>
#include <cstdlib>

#include "penalty_state.h"
#include "row_scan.h"
#include "verify_decide.h"
#include "vi_internal.h"

namespace vi {
namespace {

constexpr int kTopkThreads = 256;
constexpr int kTopkWaves = kTopkThreads / kWave;
constexpr int kInvalidId = 0x7fffffff;

struct SliceHeader {
    uint32_t flags;     // bit0 non-finite seen, bit1 NaN seen, bit2 bad history, bit3 error
    uint32_t valid;     // finite elements (sampler rows)
    float lse_max;      // log-sum-exp partial (top-k mode; base-2 units, see the kernel)
    float pad;
    double lse_sum;
};
constexpr uint32_t kSliceNonfinite = 1u, kSliceNan = 2u, kSliceBadHistory = 4u, kSliceError = 8u;
constexpr size_t kHistCountLds = 32768;   // most dynamic LDS for a slice's history counts

struct TopkArgs {
    const void* logits;
    int vocabulary;
    int64_t stride;
    int slice_len;
    float* pval;            // [rows][slices][kMaxK]
    int* pidx;
    SliceHeader* phdr;      // [rows][slices]
    uint32_t* arrivals;     // [rows]
    // kModeTopk
    int k;
    int64_t* ids;
    float* values;
    float* logprobs;
    uint32_t* nonfinite_flag;
    // kModePacket
    vi_device_sampling cfg;
    PacketKeys keys;
    uint64_t serial;
    vi_greedy_row* out_rows;
    int score;              // VeriCache sampled scores instead of packet rows
    float tolerance;
    const int64_t* next;
    int64_t* chosen;
    float* score_gap;
    // kModeSample
    const vi_row_params* params;
    const uint2* hash;      // [rows][hash_slots] (token+1, count)
    const uint32_t* row_flags;  // [rows] from the hash builder (bad history / error)
    int hash_shift;         // 32 - log2(hash_slots)
    int hash_slots;
    const int64_t* offsets;
    const int32_t* histories;
    unsigned char* pstate;   // per-lane penalty states (hash and flags) instead of the above
    PenaltyLayout pl;
    int record;              // append each row's sampled token to its lane's state
    int32_t* tokens;
    double* uniforms;
    float* probs;
    int64_t probs_stride;
    vi_sample_stats* stats;
    int full_rows_unsupported;  // fp32 logits: rows outside the top-k route fail
    int pres_words;         // dynamic LDS words for the slice's history-presence bitmap (0: none)
    int hist_counts;        // the dynamic words are the slice's history counts, one per token, counted
                            // from the histories by every workgroup of the row (no hash)
    int64_t max_history;
    // kModeVerify: sorted lists of the filtered rows
    int params_div;         // params index = row / params_div
    float* lval;            // [rows][kMaxK]
    int* lidx;
    uint32_t* lvalid;       // [rows]
    uint32_t* lflags;       // [rows]
    int skip_unlisted;      // rows of lanes without a top-k list are left to the full-vocabulary path
    // kModeVerify with the decisions taken as the rows finish: decide == 1 over
    // the draft rows (each position's decision, each lane's chain), decide == 2
    // over the target rows (the bonus rows' draws); in the paired launch
    // decide == 3 (target rows) and 4 (draft rows): each position's later row
    // decides.  larr: the lanes' arrival counters, zero between calls
    int decide;
    VerifyDecideArgs dv;
    int pair_rows;          // (the paired launch: rows of the target half)
};

// ----------------------------------------------------------- wave-resident list
struct WaveList {
    float v = -kInfF;   // this lane's entry (rank = lane)
    int i = kInvalidId;
    float kv = -kInfF;  // entry K-1, wave-uniform
    int ki = kInvalidId;
};

__device__ __forceinline__ void list_insert(WaveList& L, int K, float cv, int ci) {
    const int lane = lane_id();
    const uint64_t m = ballot(lane < K && better(cv, ci, L.v, L.i));
    if (!m) return;
    const int pos = __builtin_ctzll(m);
    const float pv = shift_up_f(L.v);
    const int pi = shift_up_i(L.i);
    if (lane == pos) { L.v = cv; L.i = ci; }
    else if (lane > pos && lane < K) { L.v = pv; L.i = pi; }
    L.kv = readlane_f(L.v, K - 1);
    L.ki = readlane_i(L.i, K - 1);
}

// Lane exchanges: ds_bpermute by default (off the VALU's issue slots, for the
// VALU-bound scans), DPP / permlane moves when D (the sampler's few-row
// launches, whose list merges are latency-bound chains of one wave).
template <bool D> __device__ __forceinline__ float xor_f(float v, int m) {
    if constexpr (D) return __builtin_bit_cast(float, lanes_xor_dpp(__builtin_bit_cast(uint32_t, v), m));
    else return shfl_xor_f(v, m);
}
template <bool D> __device__ __forceinline__ int xor_i(int v, int m) {
    if constexpr (D) return int(lanes_xor_dpp(uint32_t(v), m));
    else return shfl_xor_i(v, m);
}
template <bool D> __device__ __forceinline__ uint32_t reverse_u(uint32_t v) {
    if constexpr (D) return lanes_reverse_dpp(v);
    else return lanes_reverse(v);
}

// Merge of two sorted lists (lane = rank, (value desc, id asc), unused ranks
// (-inf, kInvalidId)): the better of each entry and the other list's entry of
// rank 63 - lane forms a bitonic sequence holding the best 64 of both, which a
// descending bitonic merge puts in order (into av, ai).
template <bool D = false>
__device__ __forceinline__ void merge_pair(float& av, int& ai, float bv, int bi) {
    const int lane = lane_id();
    const float rv = __builtin_bit_cast(float, reverse_u<D>(__builtin_bit_cast(uint32_t, bv)));
    const int ri = int(reverse_u<D>(uint32_t(bi)));
    float v = av;
    int i = ai;
    if (better(rv, ri, v, i)) { v = rv; i = ri; }
#pragma unroll
    for (int stride = kWave / 2; stride > 0; stride >>= 1) {
        const float pv = xor_f<D>(v, stride);
        const int pi = xor_i<D>(i, stride);
        const bool low = (lane & stride) == 0;
        const bool take = low ? better(pv, pi, v, i) : better(v, i, pv, pi);
        if (take) { v = pv; i = pi; }
    }
    av = v;
    ai = i;
}

// A sorted list merged into the wave list; ranks >= K are cleared afterwards,
// so the list keeps its form.
template <bool D = false>
__device__ __forceinline__ void list_merge(WaveList& L, int K, float bv, int bi) {
    const int lane = lane_id();
    float v = L.v;
    int i = L.i;
    merge_pair<D>(v, i, bv, bi);
    L.v = lane < K ? v : -kInfF;
    L.i = lane < K ? i : kInvalidId;
    L.kv = readlane_f(L.v, K - 1);
    L.ki = readlane_i(L.i, K - 1);
}

// The wave's 64 values (none NaN) sorted descending across the lanes: a
// bitonic sort.
template <bool D = false>
__device__ __forceinline__ float wave_sort_desc(float x) {
    const int lane = lane_id();
#pragma unroll
    for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const float y = xor_f<D>(x, stride);
            const bool desc = (lane & size) == 0 || size == kWave;   // the last merge runs descending
            const bool low = (lane & stride) == 0;
            x = (low == desc) ? fmaxf(x, y) : fminf(x, y);
        }
    }
    return x;
}

// The 64 largest of two descending lane-sorted lists, sorted descending: the
// larger of each entry and the other list's entry of rank 63 - lane forms a
// bitonic sequence, which a descending bitonic merge puts in order.
template <bool D = false>
__device__ __forceinline__ float merge_desc_f(float a, float b) {
    const int lane = lane_id();
    float x = fmaxf(a, __builtin_bit_cast(float, reverse_u<D>(__builtin_bit_cast(uint32_t, b))));
#pragma unroll
    for (int stride = kWave / 2; stride > 0; stride >>= 1) {
        const float y = xor_f<D>(x, stride);
        x = (lane & stride) ? fminf(x, y) : fmaxf(x, y);
    }
    return x;
}

// The wave's 64 (value, id) pairs sorted (value desc, id asc) across the
// lanes: a bitonic sort (pairs are distinct except (-inf, kInvalidId) padding).
template <bool D = false>
__device__ __forceinline__ void wave_sort_pairs(float& v, int& i) {
    const int lane = lane_id();
#pragma unroll
    for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const float pv = xor_f<D>(v, stride);
            const int pi = xor_i<D>(i, stride);
            const bool desc = (lane & size) == 0 || size == kWave;
            const bool low = (lane & stride) == 0;
            const bool take = (low == desc) ? better(pv, pi, v, i) : better(v, i, pv, pi);
            if (take) { v = pv; i = pi; }
        }
    }
}

// Offer one candidate per lane (wave-uniform call).
__device__ __forceinline__ void list_offer(WaveList& L, int K, bool ok, float v, int id) {
    uint64_t m = ballot(ok && better(v, id, L.kv, L.ki));
    while (m) {
        const int src = __builtin_ctzll(m);
        m &= m - 1;
        const float cv = readlane_f(v, src);
        const int ci = readlane_i(id, src);
        if (better(cv, ci, L.kv, L.ki)) list_insert(L, K, cv, ci);
    }
}

// Largest finite magnitude a penalty could push past the dtype's range.
template <int DT> __device__ __forceinline__ float overflow_guard() {
    if constexpr (DT == VI_F16) return 16384.0f;
    else return 1.0e37f;
}

// ------------------------------------------------------- NaN rows (top-k mode)
// dflash_topk16_serial_row (dflash2_draft.cu:1827-1862), generalized to k.
template <int DT>
__device__ void serial_topk_row(const void* row, int vocabulary, int k, float* vals, int* ids) {
    int count = 0;
    for (int c = 0; c < vocabulary; ++c) {
        const float value = Elem<DT>::decode(load_bits<DT>(row, c));
        if (count < k) {
            int j = count;
            while (j > 0 && vals[j - 1] < value) { vals[j] = vals[j - 1]; ids[j] = ids[j - 1]; --j; }
            vals[j] = value; ids[j] = c; ++count;
        } else if (value > vals[k - 1]) {
            int j = k - 1;
            while (j > 0 && vals[j - 1] < value) { vals[j] = vals[j - 1]; ids[j] = ids[j - 1]; --j; }
            vals[j] = value; ids[j] = c;
        }
    }
}

// ------------------------------------------------------------- finishing steps
// Support size of candidates sorted by value (exl3_sampled_support,
// sampled_select.cuh:283-298).  nvcc's default contraction fuses the
// multiply-adds of the coupled sampler; they are restated with fmaf.
// Tail work of one lane: its arrays live in LDS (`prob`, `v2`, `i2`) rather than
// in per-lane scratch.
__device__ __forceinline__ int packet_support(const vi_device_sampling& cfg, int cap, const float* value, float* prob) {
    const float inv_temp = 1.0f / cfg.temperature;
    const float m = value[0] * inv_temp;
    float sum = 0.0f;
    for (int j = 0; j < cap; ++j) { prob[j] = expf(fmaf(value[j], inv_temp, -m)); sum += prob[j]; }
    const float min_p_thresh = cfg.min_p > 0.0f ? cfg.min_p * prob[0] : -1.0f;
    const bool top_p_active = cfg.top_p < 1.0f;
    const float top_p_target = cfg.top_p * sum;
    float cum = 0.0f;
    int support = 0;
    for (int j = 0; j < cap; ++j) {
        if (min_p_thresh >= 0.0f && prob[j] < min_p_thresh) break;
        cum += prob[j];
        support = j + 1;
        if (top_p_active && cum >= top_p_target) break;
    }
    return support < 1 ? 1 : support;
}

// Coupled draw over the sorted candidates (sampled_select.cuh:79-116): the
// selected index; value[0..support) receives the perturbed values l/T + G.
__device__ __forceinline__ int packet_draw(const vi_device_sampling& cfg, int key, int cap, const float* cand_val,
                           const int* cand_idx, float* value, float* prob, int* support_out) {
    if (!(cfg.temperature > 0.0f)) {
        value[0] = cand_val[0];
        *support_out = 1;
        return 0;
    }
    const float inv_temp = 1.0f / cfg.temperature;
    const int support = packet_support(cfg, cap, cand_val, prob);
    int best = 0;
    for (int j = 0; j < support; ++j) {
        value[j] = fmaf(cand_val[j], inv_temp, gumbel(cfg.seed, key, cand_idx[j]));
        if (j > 0 && value[j] > value[best]) best = j;
    }
    *support_out = support;
    return best;
}

// VeriCache sampled gap (exl3_sampled_score_kernel, sampled_select.cuh:300-360):
// how far, in logit units, next trails the selected token.  In the support:
// T times the perturbed-value gap.  Outside it: infinite, unless raising next's
// logit by `tolerance` re-ranks it into the support of the same sampler; then
// the gap is taken against the best other support entry.  A next at or past
// the vocabulary end is infinite.
template <int DT>
__device__ __forceinline__ float sampled_gap(const vi_device_sampling& cfg, int key, const void* row, int vocabulary,
                             float tolerance, int64_t want, int selected, int support, const float* cand_val,
                             const int* cand_idx, const float* value, float* prob, float* v2, int* i2) {
    const int token = cand_idx[selected];
    if (want < 0 || want == token) return 0.0f;
    if (want >= vocabulary) return kInfF;
    if (!(cfg.temperature > 0.0f)) {
        float own = Elem<DT>::decode(static_cast<const typename Elem<DT>::Bits*>(row)[want]);
        if (cfg.presence_penalty != 0.0f && cfg.first_occurrence && cfg.first_occurrence[want] < key)
            own -= cfg.presence_penalty;
        return fmaxf(0.0f, cand_val[selected] - own);
    }
    int cap = 20;
    if (cfg.top_k > 0 && cfg.top_k < cap) cap = cfg.top_k;
    int rank = -1;
    for (int j = 0; j < cap; ++j)
        if (cand_idx[j] == want) { rank = j; break; }
    if (rank >= 0 && rank < support) return (value[selected] - value[rank]) * cfg.temperature;
    if (rank < 0 || !(tolerance > 0.0f)) return kInfF;
    const float boosted = cand_val[rank] + tolerance;
    int at = 0;
    for (int j = 0; j < cap; ++j) {
        if (j == rank) continue;
        v2[at] = cand_val[j];
        i2[at] = cand_idx[j];
        ++at;
    }
    int pos = at;
    while (pos > 0 && boosted > v2[pos - 1]) { v2[pos] = v2[pos - 1]; i2[pos] = i2[pos - 1]; --pos; }
    v2[pos] = boosted;
    i2[pos] = int(want);
    const int s2 = packet_support(cfg, cap, v2, prob);
    if (pos >= s2) return kInfF;
    const float inv_temp = 1.0f / cfg.temperature;
    float best = -kInfF;
    for (int j = 0; j < s2; ++j)
        if (j != pos) best = fmaxf(best, fmaf(v2[j], inv_temp, gumbel(cfg.seed, key, i2[j])));
    const float own = fmaf(cand_val[rank], inv_temp, gumbel(cfg.seed, key, int(want)));
    return fmaxf(0.0f, (best - own) * cfg.temperature);
}

// Extended sampler finish over the sorted top-`cap` list (fp64 weights,
// min_p / top_p prefix cuts, Philox inverse CDF in sorted order), run by a
// whole wave.  The one order-dependent chain, the running sums of the weights
// w[j] = exp(z[j] - z[0]) in candidate order, is taken once by lane 0 into
// cum[]; every later sum of the serial rule is one of them (the total, the
// support's mass, the draw's running sums), and the cuts and the draw are the
// first candidates whose tests hold, found by ballots.  Lane 0 writes the
// outputs.
__device__ __forceinline__ void sample_finish(const vi_row_params& p, int cap, const int* ids, int vocabulary,
                              int32_t* token_out, double* uniform_out, float* probs_row,
                              vi_sample_stats* stats_out, uint32_t flags, uint32_t valid, const double* w,
                              double* cum) {
    const int lane = lane_id();
    int32_t token = vocabulary;
    double u = 0.0, sn = 0.0;
    int support = 0;
    if (valid == 0) {
        flags |= VI_FLAG_EMPTY;
    } else if (!(p.temperature > 0.0f)) {
        token = ids[0]; support = 1; sn = 1.0;
        if (probs_row && lane == 0) probs_row[token] = 1.0f;
    } else {
        if (lane == 0) {
            double c = 0.0;
            for (int j = 0; j < cap; ++j) { c += w[j]; cum[j] = c; }
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        const double s = cum[cap - 1], w0 = w[0];
        const double minp = double(p.min_p), target = double(p.top_p) * s;
        const bool in = lane < cap;
        const double wj = in ? w[lane] : 0.0, cj = in ? cum[lane] : 0.0;
        // the serial rule stops at the first candidate under min_p (support
        // j) or the first whose running sum reaches top_p's (support j + 1)
        const uint64_t fm = ballot(in && p.min_p > 0.0f && wj < minp * w0);
        const uint64_t hm = ballot(in && p.top_p < 1.0f && cj >= target);
        const int jf = fm ? __builtin_ctzll(fm) : cap, jh = hm ? __builtin_ctzll(hm) : cap;
        support = jf <= jh ? jf : jh + 1;
        if (support < 1) support = 1;
        sn = cum[support - 1];
        u = philox_uniform(p.seed, p.lane, p.position, 0u);
        const double t = u * sn;
        const uint64_t pm = ballot(lane < support && cj > t);
        const int pick = pm ? __builtin_ctzll(pm) : support - 1;
        token = ids[pick];
        if (probs_row && lane < support) probs_row[ids[lane]] = float(wj / sn);
    }
    if (lane == 0) {
        *token_out = token;
        if (uniform_out) *uniform_out = u;
        if (stats_out) {
            stats_out->flags = flags;
            stats_out->support = uint32_t(support);
            stats_out->finite = valid;
            stats_out->reserved = 0u;
            stats_out->support_mass = sn;
            stats_out->uniform = u;
        }
    }
}

// ------------------------------------------------------------------- the kernel
// The work of one workgroup: slice `slice` of `slices` of row r.
template <int DT, bool VEC, int MODE>
__device__ __forceinline__ void topk_body(const TopkArgs& a, const int slice, const int slices, const int r) {
    constexpr bool kD = MODE == kModeSample;   // DPP lane exchanges in the list merges
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    const void* row = static_cast<const unsigned char*>(a.logits) + size_t(r) * size_t(a.stride) * sizeof(typename Elem<DT>::Bits);
    const int begin = slice * a.slice_len, end = min(a.vocabulary, begin + a.slice_len);

    // ---- per-row configuration
    int K = 1;
    vi_row_params p{};
    float inv_t = 1.0f;
    bool lookups = false, lookup_all = false;
    const uint2* table = nullptr;
    int key = 0, path[17], path_count = 0;
    float slack = 0.0f;
    if constexpr (MODE == kModeTopk) {
        K = a.k;
    } else if constexpr (MODE == kModePacket) {
        K = 20;
        if (a.cfg.top_k > 0 && a.cfg.top_k < K) K = a.cfg.top_k;
        if (a.vocabulary < K) K = a.vocabulary;
        key = a.keys.first + (a.score ? r : a.keys.depth[r]);
        if (!a.score && a.keys.inputs > r) {
            for (int j = 0; j < a.keys.depth[r] && j < a.keys.inputs; ++j) path[path_count++] = a.keys.input[j];
            path[path_count++] = a.keys.input[r];
        }
        slack = a.cfg.presence_penalty < 0.0f ? -a.cfg.presence_penalty : 0.0f;
    } else if constexpr (MODE == kModeVerify) {
        p = a.params[r / a.params_div];
        // a sampled lane whose top_k lies outside [1, 64] has no list here: its
        // rows are the full-vocabulary path's, or scanned with K = 1 and reported
        // refused (VI_FLAG_ERROR)
        if (a.skip_unlisted && verify_list_refused(p)) return;
        if (p.temperature > 0.0f) { K = verify_list_k(p); inv_t = 1.0f / p.temperature; }
    } else {
        p = a.params[r];
        if (!topk_route(p)) {
            if (a.full_rows_unsupported && slice == 0 && threadIdx.x == 0) {
                a.tokens[r] = -1;
                if (a.stats) { a.stats[r] = vi_sample_stats{}; a.stats[r].flags = VI_FLAG_ERROR; }
            }
            return;
        }
        if (p.temperature > 0.0f) { K = p.top_k; inv_t = 1.0f / p.temperature; }
        if (a.pstate) {
            lookups = penalties_active(p);
            if (lookups) table = reinterpret_cast<const uint2*>(a.pstate + size_t(r) * a.pl.lane_bytes + a.pl.off_hash);
        } else {
            const int64_t hn = a.offsets ? a.offsets[r + 1] - a.offsets[r] : 0;
            lookups = penalties_active(p) && hn > 0 && (a.hash || a.hist_counts);
            if (lookups && a.hash) table = a.hash + size_t(r) * size_t(a.hash_slots);
        }
        lookup_all = lookups && !penalties_lower_only(p);
        if (a.probs) {   // (the row's last arriver writes the support over these zeros:
                         // they are written through, and drained before the arrival)
            float* pr = a.probs + size_t(r) * size_t(a.probs_stride);
            for (int i = begin + threadIdx.x; i < end; i += kTopkThreads) put_agent(&pr[i], 0.0f);
        }
    }

    // ---- sample mode: the slice's history tokens as a presence bitmap in LDS
    // (from the lane's penalty state, or set from its history), so the penalty
    // lookups of absent tokens (nearly all) never leave the CU
    extern __shared__ uint32_t s_dyn[];
    const uint32_t* pres = nullptr;
    const uint32_t* hcnt = nullptr;
    uint32_t hist_flags = 0;   // (this thread's share of the history's check)
    uint4 pre[4] = {};         // (sample mode with history counts: the scan's first batch)
    bool have_pre = false;
    if constexpr (MODE == kModeSample) {
        if (lookups && a.hist_counts) {
            // the slice's first batch of logits requested before the counting
            // (its latency and the history's overlap)
            if constexpr (VEC) {
                constexpr int P = Elem<DT>::kPerVec;
                const int nvec = (end - begin) / P;
                const unsigned char* base = static_cast<const unsigned char*>(row) + size_t(begin) * (16 / P);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int v = u * kTopkThreads + int(threadIdx.x);
                    pre[u] = v < nvec ? load16(base + size_t(v) * 16) : make_uint4(0, 0, 0, 0);
                }
                have_pre = nvec > 0;
            }
            // the slice's tokens' counts in the lane's history, in LDS; the
            // history checked as the hash builder checks it
            uint32_t* cnt = s_dyn;
            for (int w = threadIdx.x; w < end - begin; w += kTopkThreads) cnt[w] = 0u;
            __syncthreads();
            const int64_t hb = a.offsets[r], hn = a.offsets[r + 1] - hb;
            if (hn > a.max_history) {
                hist_flags = kSliceError;
            } else {
                constexpr int kU = 8;   // (eight loads in flight per thread)
                for (int64_t i0 = 0; i0 < hn; i0 += kU * kTopkThreads) {
                    int32_t t[kU];
#pragma unroll
                    for (int u = 0; u < kU; ++u) {
                        const int64_t i = i0 + u * kTopkThreads + threadIdx.x;
                        t[u] = i < hn ? a.histories[hb + i] : begin - 1;
                    }
#pragma unroll
                    for (int u = 0; u < kU; ++u) {
                        if (i0 + u * kTopkThreads + threadIdx.x < hn && (t[u] < 0 || t[u] >= a.vocabulary))
                            hist_flags |= kSliceBadHistory;
                        else if (t[u] >= begin && t[u] < end)
                            atomicAdd(&cnt[t[u] - begin], 1u);
                    }
                }
            }
            __syncthreads();
            hcnt = cnt;
        } else if (lookups && a.pres_words > 0) {
            uint32_t* bm = s_dyn;
            const int words = (end - begin + 31) / 32;
            if (a.pstate) {
                const uint32_t* b1 = reinterpret_cast<const uint32_t*>(a.pstate + size_t(r) * a.pl.lane_bytes +
                                                                       a.pl.off_b1);
                for (int w = threadIdx.x; w < words; w += kTopkThreads) bm[w] = b1[begin / 32 + w];
            } else {
                for (int w = threadIdx.x; w < words; w += kTopkThreads) bm[w] = 0u;
                __syncthreads();
                const int64_t hb = a.offsets[r], hn = a.offsets[r + 1] - hb;
                constexpr int kU = 8;   // (eight loads in flight per thread)
                for (int64_t i0 = 0; i0 < hn; i0 += kU * kTopkThreads) {
                    int32_t t[kU];
#pragma unroll
                    for (int u = 0; u < kU; ++u) {
                        const int64_t i = i0 + u * kTopkThreads + threadIdx.x;
                        t[u] = i < hn ? a.histories[hb + i] : -1;
                    }
#pragma unroll
                    for (int u = 0; u < kU; ++u)
                        if (t[u] >= begin && t[u] < end) atomicOr(&bm[(t[u] - begin) >> 5], 1u << ((t[u] - begin) & 31));
                }
            }
            __syncthreads();
            pres = bm;
        }
    }
    // penalty count of a token of this slice (0 without lookups, or when the
    // bitmap says the token is absent)
    auto count_of = [&](int id) -> uint32_t {
        if (!lookups) return 0u;
        if (hcnt) return hcnt[id - begin];
        if (pres) {
            const int o = id - begin;
            if (!((pres[o >> 5] >> (o & 31)) & 1u)) return 0u;
        }
        return hash_count(table, a.hash_shift, a.hash_slots, id);
    };

    // Candidate pool of the workgroup (the held scan's and the sample mode's
    // batched scan's), and the held scan's staging
    constexpr int kHeld = 16;
    constexpr int kPool = 256;
    __shared__ uint4 s_hv[kTopkWaves][kWave];
    __shared__ int s_hid[kTopkWaves][kWave];
    __shared__ float s_pv[kPool];
    __shared__ int s_pi[kPool];
    __shared__ float s_selv[kMaxK];
    __shared__ int s_seli[kMaxK];
    __shared__ float s_tw[kTopkWaves];
    __shared__ int s_np, s_over;
    constexpr int kMergeHeld = 4;   // slice-list entries per thread in the last arriver's filter
    __shared__ float s_tauv;
    bool pooled = false;   // (workgroup-uniform) the slice's top K is wave 0's list
    // ---- scan the slice
    // Each wave's list K-th value, shared: an element below another wave's K-th
    // entry has K better elements in the row and cannot be in its top k, so
    // every wave gates on the largest of them (read without ordering: a stale
    // value is smaller, so it only prunes less).
    WaveList L;
    __shared__ float s_kth[kTopkWaves];
    if (threadIdx.x < kTopkWaves) s_kth[threadIdx.x] = -kInfF;
    __syncthreads();
    auto shared_kth = [&]() {   // (top-k mode; verification keeps its per-wave gate)
        float g = -kInfF;
        if constexpr (MODE != kModeTopk) return g;
#pragma unroll
        for (int w = 0; w < kTopkWaves; ++w)
            g = fmaxf(g, __hip_atomic_load(&s_kth[w], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        return g;
    };
    auto publish_kth = [&]() {
        if (MODE == kModeTopk && lane_id() == 0) __hip_atomic_store(&s_kth[threadIdx.x / kWave], L.kv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    };
    uint32_t flags = hist_flags, valid = 0;
    float lse_m = -kInfF, lse_s = 0.0f;
    const bool want_lse = MODE == kModeTopk && a.logprobs != nullptr;
    // Log-sum-exp state in base-2 units: lse_m is the exact f32 value m2 that the
    // terms 2^(x log2(e) - m2) are taken against (x log2(e) as x * kL2E + x *
    // kL2ELo, the second the rounding residual of the first), so the row's
    // log-sum-exp is ln 2 * (m2 + log2(sum)) with no rounding of m2 left over.
    constexpr float kL2E = 1.4426950408889634f;
    constexpr float kL2ELo = 1.925963e-8f;
    auto lse_term = [&](float x) { return __builtin_amdgcn_exp2f(fmaf(x, kL2ELo, fmaf(x, kL2E, -lse_m))); };
    auto lse_rebase = [&](float xmax) {   // (per lane)
        const float m2 = xmax * kL2E;
        if (m2 > lse_m) {
            lse_s = lse_s * __builtin_amdgcn_exp2f(lse_m - m2);
            lse_m = m2;
        }
    };
    // Whole vectors (top-k and verify modes): flags, counts and the running
    // log-sum-exp per vector (one rescale by the vector's maximum, then one exp
    // per element), and the list offered the vector's elements only when some
    // lane's vector maximum reaches the list's K-th entry (no element of a vector
    // below it can enter: it is exact).
    // Threshold from the first batch: the K-th largest of the workgroup's 256
    // lane maxima over their first four vectors (the four waves' sorted maxima
    // merged).  At least K of the row's elements reach it, so it never exceeds
    // the row's K-th best: elements below it are never offered.  (Pooling the
    // bounds of a row's workgroups through a global atomic maximum was measured
    // slower: the same-address atomics and reads contend.)
    float tau = -kInfF;
    __shared__ float s_first[kTopkWaves][kWave];
    auto first_fn = [&](const uint4 (&dv)[4], const bool (&okv)[4]) {
        constexpr int P = Elem<DT>::kPerVec;
        float lm = -kInfF;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
#pragma unroll
            for (int j = 0; j < P; ++j) {
                const uint32_t bits = vec_bits<DT>(dv[u], j);
                const float x = Elem<DT>::decode(bits);
                if constexpr (MODE == kModeTopk) {
                    lm = (okv[u] & !Elem<DT>::nan_bits(bits)) ? fmaxf(lm, x) : lm;
                } else {
                    const float v2 = p.temperature > 0.0f ? x * inv_t : x;
                    lm = (okv[u] & Elem<DT>::finite_bits(bits) & isfinite(v2)) ? fmaxf(lm, v2) : lm;
                }
            }
        }
        s_first[wave][lane] = wave_sort_desc<kD>(lm);
        __syncthreads();
        float t = s_first[0][lane];
#pragma unroll
        for (int w = 1; w < kTopkWaves; ++w) t = merge_desc_f<kD>(t, s_first[w][lane]);
        tau = readlane_f(t, K - 1);
    };
    auto vec_exact = [&](const uint4& dv, int id0, bool ok) {
        constexpr int P = Elem<DT>::kPerVec;
        float xs[P];
        uint32_t candm = 0;
        float vmax = -kInfF;
        if constexpr (MODE == kModeTopk) {
            uint32_t finm = 0;
#pragma unroll
            for (int j = 0; j < P; ++j) {
                const uint32_t bits = vec_bits<DT>(dv, j);
                xs[j] = Elem<DT>::decode(bits);
                const bool finite = Elem<DT>::finite_bits(bits), nan = Elem<DT>::nan_bits(bits);
                flags |= (ok & !finite) ? (nan ? (kSliceNan | kSliceNonfinite) : kSliceNonfinite) : 0u;
                finm |= uint32_t(ok & finite) << j;
                candm |= uint32_t(ok & !nan) << j;
                vmax = (ok & !nan) ? fmaxf(vmax, xs[j]) : vmax;
            }
            if (want_lse && finm) {   // (per lane)
                float m8 = -kInfF;
#pragma unroll
                for (int j = 0; j < P; ++j) m8 = ((finm >> j) & 1u) ? fmaxf(m8, xs[j]) : m8;
                lse_rebase(m8);
#pragma unroll
                for (int j = 0; j < P; ++j)
                    lse_s += ((finm >> j) & 1u) ? lse_term(xs[j]) : 0.0f;
            }
        } else {   // kModeVerify
#pragma unroll
            for (int j = 0; j < P; ++j) {
                const uint32_t bits = vec_bits<DT>(dv, j);
                const float x = Elem<DT>::decode(bits);
                const bool finite = Elem<DT>::finite_bits(bits);
                const float v = p.temperature > 0.0f ? x * inv_t : x;
                const bool live = ok & finite & isfinite(v);
                flags |= (ok & !live) ? kSliceNonfinite : 0u;
                valid += live ? 1u : 0u;
                xs[j] = v;
                candm |= uint32_t(live) << j;
                vmax = live ? fmaxf(vmax, v) : vmax;
            }
        }
        const float gate = fmaxf(fmaxf(L.kv, tau), shared_kth());
        if (ballot(candm != 0u && vmax >= gate) == 0) return;
        // rare: offer the vector's elements, one list insertion site per vector
        // (the element is taken again from the vector: a rolled loop keeps the
        // register count, and with it the occupancy, down)
#pragma unroll 1
        for (int j = 0; j < P; ++j) {
            const uint32_t bits = vec_bits<DT>(dv, j);
            float v = Elem<DT>::decode(bits);
            if constexpr (MODE == kModeVerify) v = p.temperature > 0.0f ? v * inv_t : v;
            list_offer(L, K, ((candm >> j) & 1u) && v >= gate, v, id0 + j);
        }
        publish_kth();
    };
    // The (lane, element) pairs of a clean vector reaching the gate, offered one
    // at a time as wave-uniform values (the list only rises meanwhile: each is
    // checked again against it; the final list does not depend on the order).
    auto vec_offer = [&](const uint4& dv, int id0, bool ok, float gate) {
        constexpr int P = Elem<DT>::kPerVec;
        const bool scaled = MODE == kModeVerify && p.temperature > 0.0f;
        uint32_t cm = 0;
#pragma unroll
        for (int j = 0; j < P; ++j) {
            const float x = Elem<DT>::decode(vec_bits<DT>(dv, j));
            cm |= uint32_t(ok && (scaled ? x * inv_t : x) >= gate) << j;
        }
        uint64_t lanes = ballot(cm != 0u);
        if (!lanes) return;
        if (__builtin_popcountll(lanes) > 8) {   // many (large k, early in the slice): element-wise
#pragma unroll 1
            for (int j = 0; j < P; ++j) {
                float v = Elem<DT>::decode(vec_bits<DT>(dv, j));
                if (scaled) v = v * inv_t;
                list_offer(L, K, ((cm >> j) & 1u) != 0u, v, id0 + j);
            }
            publish_kth();
            return;
        }
        while (lanes) {
            const int src = __builtin_ctzll(lanes);
            lanes &= lanes - 1;
            uint32_t m = uint32_t(readlane_i(int(cm), src));
            const uint4 w = make_uint4(uint32_t(readlane_i(int(dv.x), src)), uint32_t(readlane_i(int(dv.y), src)),
                                       uint32_t(readlane_i(int(dv.z), src)), uint32_t(readlane_i(int(dv.w), src)));
            const int base = readlane_i(id0, src);
            while (m) {
                const int j = __builtin_ctz(m);
                m &= m - 1;
                float v = Elem<DT>::decode(vec_bits<DT>(w, j));
                if (scaled) v = v * inv_t;
                if (better(v, base + j, L.kv, L.ki)) list_insert(L, K, v, base + j);
            }
        }
        publish_kth();
    };
    // Top-k and verification modes, a whole batch of clean vectors at a time:
    // the vector maxima bound the gate test and the log-sum-exp rescale, one
    // exp per element (top-k mode's log-probs), the shared K-th entries read
    // once; a batch holding a non-finite element (or, in verification, a scaled
    // value that overflows) goes vector by vector through vec_exact.
    auto batch_fn = [&](const uint4 (&dv)[4], int vb, const bool (&okv)[4]) {
        constexpr int P = Elem<DT>::kPerVec;
        const int id_base = begin + (vb + int(threadIdx.x)) * P;
        // verification scales by 1/T: a vector whose scaled maximum or minimum
        // overflows goes through vec_exact like one holding a non-finite element
        const bool scaled = MODE == kModeVerify && p.temperature > 0.0f;
        bool bad = false;
        // (maxima per vector, masked once per vector; the vectors of invalid
        // lanes are zeros)
        float vm[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            float m, mn = 0.0f;
            if constexpr (DT == VI_F16) {   // packed half maxima (used only when clean: no NaN)
                typedef _Float16 h2 __attribute__((ext_vector_type(2)));
                auto H = [](uint32_t w) { return __builtin_bit_cast(h2, w); };
                const h2 t = __builtin_elementwise_max(__builtin_elementwise_max(H(dv[u].x), H(dv[u].y)),
                                                       __builtin_elementwise_max(H(dv[u].z), H(dv[u].w)));
                m = float(t[0] > t[1] ? t[0] : t[1]);
                if (scaled) {
                    const h2 q = __builtin_elementwise_min(__builtin_elementwise_min(H(dv[u].x), H(dv[u].y)),
                                                           __builtin_elementwise_min(H(dv[u].z), H(dv[u].w)));
                    mn = float(q[0] < q[1] ? q[0] : q[1]);
                }
            } else {
                m = Elem<DT>::decode(vec_bits<DT>(dv[u], 0));
                mn = m;
#pragma unroll
                for (int j = 1; j < P; ++j) {
                    const float x = Elem<DT>::decode(vec_bits<DT>(dv[u], j));
                    m = fmaxf(m, x);
                    mn = fminf(mn, x);
                }
            }
            bool b = any_nonfinite<DT>(dv[u]);
            if (scaled) b = b || !isfinite(m * inv_t) || !isfinite(mn * inv_t);
            bad |= okv[u] && b;
            vm[u] = okv[u] ? (scaled ? m * inv_t : m) : -kInfF;
        }
        if (ballot(bad) != 0) {
#pragma unroll
            for (int u = 0; u < 4; ++u) vec_exact(dv[u], id_base + u * kTopkThreads * P, okv[u]);
            return;
        }
        if constexpr (MODE == kModeVerify) {
#pragma unroll
            for (int u = 0; u < 4; ++u) valid += okv[u] ? uint32_t(P) : 0u;
        }
        const float bm = fmaxf(fmaxf(vm[0], vm[1]), fmaxf(vm[2], vm[3]));
        if (want_lse) {
            lse_rebase(bm);
            float acc[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                float a = 0.0f;
#pragma unroll
                for (int j = 0; j < P; ++j)
                    a += lse_term(Elem<DT>::decode(vec_bits<DT>(dv[u], j)));
                acc[u] = okv[u] ? a : 0.0f;
            }
            lse_s += (acc[0] + acc[1]) + (acc[2] + acc[3]);
        }
        const float gate = fmaxf(fmaxf(L.kv, tau), shared_kth());
        if (ballot(bm >= gate) == 0) return;
        // only the vectors some lane's maximum says hold a candidate
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (ballot(vm[u] >= gate) != 0) vec_offer(dv[u], id_base + u * kTopkThreads * P, okv[u], gate);
    };
    auto elem_fn = [&](uint32_t bits, int id, bool ok) {
        const float x = Elem<DT>::decode(bits);
        const bool finite = Elem<DT>::finite_bits(bits);
        if constexpr (MODE == kModeTopk) {
            // straight-line per element: flags, running log-sum-exp, then the list
            const bool nan = Elem<DT>::nan_bits(bits);
            flags |= (ok & !finite) ? (nan ? (kSliceNan | kSliceNonfinite) : kSliceNonfinite) : 0u;
            const bool cand = ok & !nan;
            if (want_lse) {   // (uniform)
                const bool use = ok & finite;
                if (use) lse_rebase(x);
                lse_s += use ? lse_term(x) : 0.0f;
            }
            list_offer(L, K, cand, x, id);
        } else if constexpr (MODE == kModePacket) {
            if (ok && !finite) flags |= kSliceNonfinite;
            bool cand = ok && finite && better(x + slack, id, L.kv, L.ki);
            float v = x;
            if (cand && a.cfg.presence_penalty != 0.0f) {
                bool seen = a.cfg.first_occurrence && a.cfg.first_occurrence[id] < key;
                for (int j = 0; j < path_count && !seen; ++j) seen = path[j] == id;
                if (seen) v = x - a.cfg.presence_penalty;
            }
            list_offer(L, K, cand, v, id);
        } else if constexpr (MODE == kModeVerify) {
            if (ok && !finite) flags |= kSliceNonfinite;
            const float v = p.temperature > 0.0f ? x * inv_t : x;
            const bool live = ok && finite && isfinite(v);
            if (ok && finite && !live) flags |= kSliceNonfinite;
            valid += live ? 1u : 0u;
            list_offer(L, K, live, v, id);
        } else {
            if (ok && !finite) flags |= kSliceNonfinite;
            bool live = ok && finite;
            float v = p.temperature > 0.0f ? x * inv_t : x;
            bool cand = live && better(v, id, L.kv, L.ki);
            if (lookups && live && (cand || lookup_all || fabsf(x) >= overflow_guard<DT>() || !isfinite(v))) {
                const uint32_t c = count_of(id);
                if (c) {
                    const uint32_t pb = penalize_bits<DT>(bits, c, p);
                    if (!Elem<DT>::finite_bits(pb)) { flags |= kSliceNonfinite; live = false; }
                    else {
                        float xp = Elem<DT>::decode(pb);
                        if (xp == 0.0f) xp = 0.0f;
                        v = p.temperature > 0.0f ? xp * inv_t : xp;
                    }
                }
                if (live && p.temperature > 0.0f && !isfinite(v)) { flags |= kSliceNonfinite; live = false; }
                cand = live && better(v, id, L.kv, L.ki);
            } else if (live && p.temperature > 0.0f && !isfinite(v)) {
                flags |= kSliceNonfinite; live = false; cand = false;
            }
            valid += live ? 1u : 0u;
            list_offer(L, K, cand, v, id);
        }
    };
    // ---- sample mode, batches.  A row qualifies when its penalties only lower a
    // logit and cannot carry one with |x| below the overflow guard out of the
    // dtype's range (guard * repetition + frequency * history length + presence
    // under half the largest finite value): then, as in elem_fn, only elements
    // whose raw scaled value reaches the gate need their penalty looked up (the
    // penalized value is never larger), and every finite raw element of a clean
    // batch stays finite.  A batch holding a non-finite element, an element at
    // or past the guard or a scaled value that overflows goes element by element
    // through elem_fn.  Other rows take elem_fn throughout, and a row whose
    // penalties fail the range check has every element looked up (a penalty
    // could then turn a finite logit that no gate would look at non-finite,
    // which the row's finite count and flags must see).
    bool batched = false;
    if constexpr (MODE == kModeSample) {
        if (!lookups) {
            batched = true;
        } else if (!lookup_all) {
            const double hmax = a.pstate ? double(reinterpret_cast<const PenaltyHeader*>(
                                               a.pstate + size_t(r) * a.pl.lane_bytes)->total)
                                         : double(a.offsets[r + 1] - a.offsets[r]);
            const double top = DT == VI_F16 ? 65504.0 : 3.3895313892515355e38;
            batched = double(overflow_guard<DT>()) * double(p.repetition_penalty) +
                      double(p.frequency_penalty) * hmax + double(p.presence_penalty) < 0.5 * top;
            lookup_all = !batched;
        }
    }
    // live and value of a finite raw element after its penalty (the looked-up
    // counts given)
    auto penalized = [&](uint32_t bits, uint32_t c, float& v) -> bool {
        const float x = Elem<DT>::decode(bits);
        v = p.temperature > 0.0f ? x * inv_t : x;
        if (c) {
            const uint32_t pb = penalize_bits<DT>(bits, c, p);
            if (!Elem<DT>::finite_bits(pb)) return false;
            float xp = Elem<DT>::decode(pb);
            if (xp == 0.0f) xp = 0.0f;
            v = p.temperature > 0.0f ? xp * inv_t : xp;
        }
        return !(p.temperature > 0.0f) || isfinite(v);
    };
    // first batch: each lane's largest finite raw element, its penalty looked up
    // (one lookup per lane, all in flight together), gives one exact penalized
    // value per lane; the workgroup's K-th largest of these 256 values, from 256
    // distinct elements, bounds the row's K-th best from below
    auto first_sample = [&](const uint4 (&dv)[4], const bool (&okv)[4]) {
        constexpr int P = Elem<DT>::kPerVec;
        const int id_base = begin + int(threadIdx.x) * P;
        float mx = -kInfF;
        uint32_t mbits = 0u;
        int mid = -1;
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int j = 0; j < P; ++j) {
                const uint32_t bits = vec_bits<DT>(dv[u], j);
                const float x = Elem<DT>::decode(bits);
                const bool take = okv[u] && Elem<DT>::finite_bits(bits) && (mid < 0 || x > mx);
                mx = take ? x : mx;
                mbits = take ? bits : mbits;
                mid = take ? id_base + u * kTopkThreads * P + j : mid;
            }
        float lm = -kInfF;
        if (mid >= 0) {
            const uint32_t c = count_of(mid);
            float v;
            if (penalized(mbits, c, v)) lm = v;
        }
        s_first[wave][lane] = wave_sort_desc<kD>(lm);
        __syncthreads();
        float t = s_first[0][lane];
#pragma unroll
        for (int w = 1; w < kTopkWaves; ++w) t = merge_desc_f<kD>(t, s_first[w][lane]);
        tau = readlane_f(t, K - 1);
    };
    // Candidates of a batch are staged per wave in LDS and go into the list
    // together: sorted (bitonic, across the lanes), then merged (no insertion
    // one element at a time; a batch can hold the row's whole top-k early on).
    __shared__ float s_cv[kTopkWaves][kWave];
    __shared__ int s_ci[kTopkWaves][kWave];
    int fill = 0;   // (wave-uniform)
    auto flush = [&]() {
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        float cv = lane < fill ? s_cv[wave][lane] : -kInfF;
        int ci = lane < fill ? s_ci[wave][lane] : kInvalidId;
        wave_sort_pairs<kD>(cv, ci);
        list_merge<kD>(L, K, cv, ci);
        fill = 0;
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    };
    auto stage = [&](bool c, float v, int id) {
        const uint64_t m = ballot(c);
        if (!m) return;
        const int n = __builtin_popcountll(m);
        if (fill + n > kWave) flush();
        if (c) {
            const int pos = fill + int(__builtin_popcountll(m & ((uint64_t(1) << lane) - 1)));
            s_cv[wave][pos] = v;
            s_ci[wave][pos] = id;
        }
        fill += n;
    };
    // a candidate into the workgroup's pool (past the pool: into the wave's list)
    auto pool_put = [&](bool c, float v, int id) {
        const uint64_t m = ballot(c);
        if (!m) return;
        int at = 0;
        if (lane == 0) at = atomicAdd(&s_np, int(__builtin_popcountll(m)));
        at = __builtin_amdgcn_readfirstlane(at);
        const int pos = at + int(__builtin_popcountll(m & ((uint64_t(1) << lane) - 1)));
        const bool fit = c && pos < kPool;
        if (fit) { s_pv[pos] = v; s_pi[pos] = id; }
        stage(c && !fit, v, id);
    };
    auto sample_batch = [&](const uint4 (&dv)[4], int vb, const bool (&okv)[4]) {
        constexpr int P = Elem<DT>::kPerVec;
        const int id_base = begin + (vb + int(threadIdx.x)) * P;
        bool bad = false;
        float vm[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            float mx = -kInfF, mn = kInfF;
#pragma unroll
            for (int j = 0; j < P; ++j) {
                const float x = Elem<DT>::decode(vec_bits<DT>(dv[u], j));
                mx = fmaxf(mx, x);
                mn = fminf(mn, x);
            }
            bool b = any_nonfinite<DT>(dv[u]);
            if (lookups) b = b || fmaxf(mx, -mn) >= overflow_guard<DT>();
            if (p.temperature > 0.0f) b = b || !isfinite(mx * inv_t) || !isfinite(mn * inv_t);
            bad |= okv[u] && b;
            vm[u] = okv[u] ? (p.temperature > 0.0f ? mx * inv_t : mx) : -kInfF;
        }
        if (ballot(bad) != 0) {
            // (one call per vector with a constant index, each a rolled loop over
            // its elements: no indexed copy of the batch in scratch memory)
            auto exact_vec = [&](const uint4& v, int u, bool ok) {
#pragma unroll 1
                for (int j = 0; j < P; ++j) elem_fn(vec_bits<DT>(v, j), id_base + u * kTopkThreads * P + j, ok);
            };
            exact_vec(dv[0], 0, okv[0]);
            exact_vec(dv[1], 1, okv[1]);
            exact_vec(dv[2], 2, okv[2]);
            exact_vec(dv[3], 3, okv[3]);
            return;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) valid += okv[u] ? uint32_t(P) : 0u;
        const float gate = fmaxf(L.kv, tau);
        if (ballot(fmaxf(fmaxf(vm[0], vm[1]), fmaxf(vm[2], vm[3])) >= gate) == 0) return;
        // (one call per vector with a constant index: an indexed batch would be
        // copied to scratch memory)
        auto cand_vec = [&](const uint4& dvu, int u, bool ok, float vmu) {
            if (ballot(vmu >= gate) == 0) return;
            const int id0 = id_base + u * kTopkThreads * P;
#pragma unroll
            for (int j = 0; j < P; ++j) {
                const uint32_t bits = vec_bits<DT>(dvu, j);
                const float x = Elem<DT>::decode(bits);
                const bool want = ok && (p.temperature > 0.0f ? x * inv_t : x) >= gate;
                if (ballot(want) == 0) continue;
                float v = -kInfF;
                const bool c = want && penalized(bits, want ? count_of(id0 + j) : 0u, v) && v >= gate;
                pool_put(c, v, id0 + j);
            }
        };
        cand_vec(dv[0], 0, okv[0], vm[0]);
        cand_vec(dv[1], 1, okv[1], vm[1]);
        cand_vec(dv[2], 2, okv[2], vm[2]);
        cand_vec(dv[3], 3, okv[3], vm[3]);
        if (fill) flush();
    };
    // ---- held scan (top-k and verification modes, 16-bit rows whose slice
    // gives each lane at most kHeld vectors).  Every vector of the lane is
    // requested at once and kept in registers, and the scan is one light pass
    // per vector: its maximum (NaN-propagating packed f16 / f32 maxima) and a
    // running minimum; the log-sum-exp is one exp per logit against the lane's
    // own maximum.  A workgroup with a NaN or an infinity (or, in verification,
    // a logit whose scaled value overflows) takes the exact path, vec_exact
    // vector by vector into the wave lists.  Otherwise the gate is the largest
    // of the four waves' K-th largest lane maxima (distinct logits: at least K
    // logits of the slice reach it, and every logit of the slice's top K does);
    // the vectors whose maximum reaches it are staged in LDS, one per lane,
    // their logits that reach it are pooled for the workgroup, and each pooled
    // logit's rank among them (value desc, id asc) places the slice's top K.
    // per-wave partials of the slice header (flags, finite count, log-sum-exp)
    __shared__ uint32_t s_flags[kTopkWaves], s_valid[kTopkWaves];
    __shared__ float s_lm[kTopkWaves];
    __shared__ double s_ls[kTopkWaves];
    auto wave_partials = [&]() {
        uint32_t f = flags;
#pragma unroll
        for (int o = 32; o; o >>= 1) f |= shfl_xor_u(f, o);
        uint32_t c = valid;
#pragma unroll
        for (int o = 32; o; o >>= 1) c += shfl_xor_u(c, o);
        float m = lse_m;
#pragma unroll
        for (int o = 32; o; o >>= 1) m = fmaxf(m, shfl_xor_f(m, o));
        double s = (lse_m == -kInfF) ? 0.0 : double(lse_s) * double(__builtin_amdgcn_exp2f(lse_m - m));
#pragma unroll
        for (int o = 32; o; o >>= 1) s += shfl_xor_d(s, o);
        if (lane == 0) { s_flags[wave] = f; s_valid[wave] = c; s_lm[wave] = m; s_ls[wave] = s; }
    };
    // (16-bit vector rows; bf16 rows in top-k mode keep the batch scan: their
    // held scan with the log-sum-exp does not fit 128 registers)
    constexpr bool kHeldMode = VEC && (DT == VI_F16 || (DT == VI_BF16 && MODE == kModeVerify));
    auto held_scan = [&](int nvec) {
      if constexpr (kHeldMode) {
        constexpr int P = Elem<DT>::kPerVec;
        constexpr int kBatch = kHeld * kTopkThreads;   // vectors of one held batch
        typedef _Float16 h2t __attribute__((ext_vector_type(2)));
        auto H = [](uint32_t w) { return __builtin_bit_cast(h2t, w); };
        const int tid = int(threadIdx.x);
        const unsigned char* base = static_cast<const unsigned char*>(row) + size_t(begin) * 2;
        const int nb = (nvec + kBatch - 1) / kBatch;   // (one or two batches; uniform)
        if (threadIdx.x == 0) { s_np = 0; s_over = 0; }
        const bool scaled = MODE == kModeVerify && p.temperature > 0.0f;
        uint32_t vadd = 0;      // (the fast path's finite logits, counted once every batch passed)
        float tau_g = -kInfF;   // the workgroup's gate, from the first batch
        bool exact = false;
#pragma unroll 1
        for (int bt = 0; bt < nb; ++bt) {
            const int v0 = bt * kBatch;
            // (unconditional loads at clamped in-bounds addresses: past the end a
            // lane reads the slice's last vector again and leaves it out below)
            uint4 d[kHeld];
#pragma unroll
            for (int u = 0; u < kHeld; ++u)
                d[u] = load16(base + size_t(min(v0 + u * kTopkThreads + tid, nvec - 1)) * 16);
            // (vector maxima kept as their 16-bit patterns, two to a register)
            uint32_t vm2[kHeld / 2];
            float lmax = -kInfF, amin = kInfF;
            h2t hmin = H(0x7c007c00u);
            int nok = 0;
#pragma unroll
            for (int u = 0; u < kHeld; ++u) {
                const bool ok = v0 + u * kTopkThreads + tid < nvec;
                float mx;
                uint32_t mb;
                if constexpr (DT == VI_F16) {
                    const h2t hx = H(d[u].x), hy = H(d[u].y), hz = H(d[u].z), hw = H(d[u].w);
                    const h2t t = __builtin_elementwise_maximum(__builtin_elementwise_maximum(hx, hy),
                                                                __builtin_elementwise_maximum(hz, hw));
                    hmin = __builtin_elementwise_minimum(
                        __builtin_elementwise_minimum(hmin, __builtin_elementwise_minimum(hx, hy)),
                        __builtin_elementwise_minimum(hz, hw));
                    const _Float16 hm = __builtin_elementwise_maximum(t[0], t[1]);
                    mx = float(hm);
                    mb = uint32_t(__builtin_bit_cast(uint16_t, hm));
                } else {   // (a word at a time: its two logits as floats, one three-way max / min each)
                    const uint32_t w4[4] = {d[u].x, d[u].y, d[u].z, d[u].w};
                    mx = -kInfF;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float lo = __builtin_bit_cast(float, w4[q] << 16);
                        const float hi = __builtin_bit_cast(float, w4[q] & 0xffff0000u);
                        mx = __builtin_elementwise_maximum(__builtin_elementwise_maximum(mx, lo), hi);
                        amin = __builtin_elementwise_minimum(__builtin_elementwise_minimum(amin, lo), hi);
                    }
                    mb = __builtin_bit_cast(uint32_t, mx) >> 16;
                }
                constexpr uint32_t kNegInf = DT == VI_F16 ? 0xfc00u : 0xff80u;
                mb = ok ? mb : kNegInf;
                if (want_lse) {   // (against the largest vector maximum so far, as it arrives)
                    lse_rebase(ok ? mx : -kInfF);
                    float sm = 0.0f;
#pragma unroll
                    for (int j = 0; j < P; ++j) sm += lse_term(Elem<DT>::decode(vec_bits<DT>(d[u], j)));
                    lse_s += ok ? sm : 0.0f;
                }
                if (u & 1) vm2[u / 2] |= mb << 16;
                else vm2[u / 2] = mb;
                lmax = ok ? __builtin_elementwise_maximum(lmax, mx) : lmax;
                nok += ok ? 1 : 0;
            }
            if constexpr (DT == VI_F16) amin = float(__builtin_elementwise_minimum(hmin[0], hmin[1]));
            // (the minimum also covers re-read vectors: they belong to the slice, so
            // at worst another lane's non-finite logit sends the workgroup the exact way)
            bool bad = !isfinite(amin) || lmax == kInfF || __builtin_isnan(lmax);
            if (scaled) bad = bad || !isfinite(amin * inv_t) || (lmax > -kInfF && !isfinite(lmax * inv_t));
            if (bt == 0) s_first[wave][lane] = scaled ? lmax * inv_t : lmax;
            if (__syncthreads_or(bad ? 1 : 0)) {
                exact = true;
                break;
            }
            if (bt == 0) {
                // The workgroup's gate: the K-th largest of its 256 lane maxima
                // (distinct logits: at least K logits of the first batch reach
                // it, so it gates the later batch as well), by a radix select
                // over their order keys that every wave runs on the same four
                // values per lane (one ballot per value and bit, no barrier).
                uint32_t key[kTopkWaves];
#pragma unroll
                for (int w = 0; w < kTopkWaves; ++w) {
                    const uint32_t kb = __builtin_bit_cast(uint32_t, s_first[w][lane]);
                    key[w] = (kb & 0x80000000u) ? ~kb : (kb | 0x80000000u);
                }
                uint32_t t = 0;
#pragma unroll
                for (int bit = 31; bit >= 0; --bit) {
                    const uint32_t c = t | (1u << bit);
                    int cnt = 0;
#pragma unroll
                    for (int w = 0; w < kTopkWaves; ++w) cnt += __builtin_popcountll(ballot(key[w] >= c));
                    if (cnt >= K) t = c;
                }
                tau_g = __builtin_bit_cast(float, (t & 0x80000000u) ? (t & 0x7fffffffu) : ~t);
            }
            vadd += uint32_t(nok * P);
            // the vectors reaching it, staged per wave (at most one per lane: the
            // loop stays small enough to unroll, which keeps the vectors in registers)
            int nst = 0;   // (wave-uniform)
#pragma unroll
            for (int u = 0; u < kHeld; ++u) {
                const float vr = Elem<DT>::decode((u & 1) ? vm2[u / 2] >> 16 : vm2[u / 2] & 0xffffu);
                const float vs = scaled ? vr * inv_t : vr;
                const bool c = v0 + u * kTopkThreads + tid < nvec && vs >= tau_g;
                const uint64_t m = ballot(c);
                if (m) {   // (uniform: most vectors have no candidate in the wave)
                    const int pos = nst + int(__builtin_popcountll(m & ((uint64_t(1) << lane) - 1)));
                    if (c && pos < kWave) {
                        s_hv[wave][pos] = d[u];
                        s_hid[wave][pos] = begin + (v0 + u * kTopkThreads + tid) * P;
                    }
                    nst += int(__builtin_popcountll(m));
                }
            }
            // their logits reaching it, pooled for the workgroup
            if (nst <= kWave) {
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                const bool have = lane < nst;
                const uint4 v = s_hv[wave][lane];
                const int id0 = s_hid[wave][lane];
#pragma unroll
                for (int j = 0; j < P; ++j) {
                    float x = Elem<DT>::decode(vec_bits<DT>(v, j));
                    if (scaled) x = x * inv_t;
                    const bool c = have && x >= tau_g;
                    const uint64_t m = ballot(c);
                    if (m) {
                        int at = 0;
                        if (lane == 0) at = atomicAdd(&s_np, int(__builtin_popcountll(m)));
                        at = __builtin_amdgcn_readfirstlane(at);
                        const int pos = at + int(__builtin_popcountll(m & ((uint64_t(1) << lane) - 1)));
                        if (c && pos < kPool) { s_pv[pos] = x; s_pi[pos] = id0 + j; }
                    }
                }
                // (the staging area is written again by the next batch)
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            } else if (lane == 0) {
                s_over = 1;
            }
        }
        if (exact) {   // the element-exact path over every vector, the log-sum-exp started again
            lse_m = -kInfF;
            lse_s = 0.0f;
#pragma unroll 1
            for (int v = tid; v < nb * kBatch; v += kTopkThreads)
                vec_exact(load16(base + size_t(min(v, nvec - 1)) * 16), begin + v * P, v < nvec);
            return;
        }
        if constexpr (MODE == kModeVerify) valid += vadd;
        wave_partials();
        __syncthreads();
        const int n = s_np;
        if (s_over || n > kPool) {
            // too many candidates to pool: read again, offered into the wave lists
#pragma unroll 1
            for (int vi = tid; vi < nb * kBatch; vi += kTopkThreads) {
                const uint4 v = load16(base + size_t(min(vi, nvec - 1)) * 16);
                float vm = -kInfF;
#pragma unroll
                for (int j = 0; j < P; ++j) vm = fmaxf(vm, Elem<DT>::decode(vec_bits<DT>(v, j)));
                if (scaled) vm = vm * inv_t;
                const float gate = fmaxf(tau_g, L.kv);
                if (ballot(vi < nvec && vm >= gate) != 0) vec_offer(v, begin + vi * P, vi < nvec, gate);
            }
            return;
        }
        // each pooled logit placed by its rank among them (one per thread, the
        // others read with broadcast LDS reads; ids are distinct, so the ranks
        // are), then wave 0 takes the list
        for (int t = tid; t - lane < n; t += kTopkThreads) {   // (wave-uniform)
            const float v = s_pv[min(t, n - 1)];
            const int i = s_pi[min(t, n - 1)];
            int rank = 0;
#pragma unroll 8
            for (int q = 0; q < n; ++q) rank += better(s_pv[q], s_pi[q], v, i) ? 1 : 0;
            if (t < n && rank < K) { s_selv[rank] = v; s_seli[rank] = i; }
        }
        __syncthreads();
        if (wave == 0) {
            const bool h = lane < min(K, n);
            L.v = h ? s_selv[lane] : -kInfF;
            L.i = h ? s_seli[lane] : kInvalidId;
            L.kv = readlane_f(L.v, K - 1);
            L.ki = readlane_i(L.i, K - 1);
        }
        pooled = true;
      }
    };
    // (the held scan when the slice gives each lane at most kHeld vectors)
    auto held_fits = [&]() {
        if constexpr (kHeldMode) {
            const int nvec = (end - begin) / Elem<DT>::kPerVec;
            return nvec > 0 && nvec <= 2 * kHeld * kTopkThreads;   // (one or two held batches)
        }
        return false;
    };
    auto held_then_tail = [&]() {
        constexpr int P = Elem<DT>::kPerVec;
        const int nvec = (end - begin) / P;
        held_scan(nvec);
        if (begin + nvec * P < end) pooled = false;   // (the tail enters every wave's list)
        for (int ib = begin + nvec * P; ib < end; ib += kTopkThreads) {
            const int i = ib + int(threadIdx.x);
            const bool ok = i < end;
            elem_fn(ok ? load_bits<DT>(row, i) : 0u, i, ok);
        }
    };
    // Sample mode, batched scan: the pooled candidates ranked into wave 0's
    // list (merged with what that wave's list holds: exact-path elements and
    // candidates past the pool); the other waves' lists join in the tree merge
    // only when they hold anything.
    __shared__ int s_used[kTopkWaves];
    auto sample_pool_finish = [&]() {
        wave_partials();
        handoff_stores_done();   // every wave's probability zeros
        if (lane == 0) s_used[wave] = L.v != -kInfF ? 1 : 0;   // (lane 0 holds the list's best)
        __syncthreads();
        // each pooled candidate placed by its rank among them (one per thread;
        // ids are distinct, so the ranks are)
        const int n = min(s_np, kPool);
        for (int t = int(threadIdx.x); t - lane < n; t += kTopkThreads) {   // (wave-uniform)
            const float v = s_pv[min(t, n - 1)];
            const int i = s_pi[min(t, n - 1)];
            int rank = 0;
#pragma unroll 8
            for (int q = 0; q < n; ++q) rank += better(s_pv[q], s_pi[q], v, i) ? 1 : 0;   // (broadcast reads)
            if (t < n && rank < K) { s_selv[rank] = v; s_seli[rank] = i; }
        }
        __syncthreads();
        if (wave == 0) {
            const bool h = lane < min(K, n);
            const float pv = h ? s_selv[lane] : -kInfF;
            const int pi = h ? s_seli[lane] : kInvalidId;
            if (s_used[0]) {
                list_merge<kD>(L, K, pv, pi);
            } else {
                L.v = pv;
                L.i = pi;
                L.kv = readlane_f(L.v, K - 1);
                L.ki = readlane_i(L.i, K - 1);
            }
        }
        pooled = !(s_used[1] | s_used[2] | s_used[3]);
    };
    if constexpr (MODE == kModeTopk || MODE == kModeVerify) {
        if (held_fits()) held_then_tail();
        else scan_slice_batches<DT, VEC, kTopkThreads>(row, begin, end, first_fn, batch_fn, elem_fn);
    } else if constexpr (MODE == kModeSample) {
        if (batched) {
            if (threadIdx.x == 0) s_np = 0;   // (ordered by the first batch's barrier)
            scan_slice_batches_from<DT, VEC, kTopkThreads>(row, begin, end, pre, have_pre, first_sample, sample_batch,
                                                           elem_fn);
            sample_pool_finish();
        } else {
            scan_slice<DT, VEC, kTopkThreads>(row, begin, end, elem_fn);
        }
    } else {
        scan_slice<DT, VEC, kTopkThreads>(row, begin, end, elem_fn);
    }

    // Verification with decisions over the draft rows: the position's target
    // list (entries, finite count, flags), loaded by wave 0 as early as the row's
    // last workgroup is known
    float tl_v = -kInfF;
    int tl_i = kInvalidId;
    uint32_t tl_valid = 0, tl_flags = 0;
    bool tl_have = false;
    auto tl_fetch = [&]() {
        if constexpr (MODE == kModeVerify) {
            const int l = r / a.dv.drafts, j = r - l * a.dv.drafts;
            const size_t tr = size_t(l) * a.dv.target_rows + j;
            tl_v = a.dv.tlval[tr * kMaxK + lane];
            tl_i = a.dv.tlidx[tr * kMaxK + lane];
            tl_valid = a.dv.tlvalid[tr];
            tl_flags = a.dv.tlflags[tr];
            tl_have = true;
        }
    };
    // ---- merge the wave lists in LDS
    __shared__ float s_val[kTopkWaves][kMaxK];
    __shared__ int s_idx[kTopkWaves][kMaxK];
    // the four wave lists merged as a tree: waves 0 and 2 take waves 1 and 3's
    // lists, then wave 0 takes wave 2's
    auto tree_merge = [&]() {
        if (!(wave & 1))
            list_merge<kD>(L, K, lane < K ? s_val[wave + 1][lane] : -kInfF, lane < K ? s_idx[wave + 1][lane] : kInvalidId);
        if (wave == 2) { s_val[2][lane] = L.v; s_idx[2][lane] = L.i; }
        __syncthreads();
        if (wave == 0) list_merge<kD>(L, K, lane < K ? s_val[2][lane] : -kInfF, lane < K ? s_idx[2][lane] : kInvalidId);
    };
    // (a pooled slice has its list in wave 0 and the partials in LDS already)
    if (!pooled) {
        s_val[wave][lane] = L.v;
        s_idx[wave][lane] = L.i;
        wave_partials();
        if constexpr (MODE == kModeSample) handoff_stores_done();   // every wave's probability zeros
        __syncthreads();
        tree_merge();
    }
    uint32_t f = 0, c = 0;
    float m = -kInfF;
    double s = 0.0;
    if (wave == 0) {
        for (int w = 0; w < kTopkWaves; ++w) { f |= s_flags[w]; c += s_valid[w]; m = fmaxf(m, s_lm[w]); }
        for (int w = 0; w < kTopkWaves; ++w)
            if (s_lm[w] != -kInfF) s += s_ls[w] * double(__builtin_amdgcn_exp2f(s_lm[w] - m));
    }

    if (slices > 1) {
        // ---- publish the slice, last arriver merges
        __shared__ int s_last;
        if (wave == 0) {
            const size_t at = (size_t(r) * slices + slice) * kMaxK;
            if (lane < K) { put_agent(&a.pval[at + lane], L.v); put_agent(&a.pidx[at + lane], L.i); }
            if (lane == 0) {
                SliceHeader& h = a.phdr[size_t(r) * slices + slice];
                put_agent(&h.flags, f); put_agent(&h.valid, c); put_agent(&h.lse_max, m); put_agent(&h.lse_sum, s);
            }
            handoff_stores_done();
            if (lane == 0) s_last = atomicAdd(&a.arrivals[r], 1u) == uint32_t(slices - 1) ? 1 : 0;
        }
        __syncthreads();
        if (!s_last) return;
        handoff_acquire();
        if constexpr (MODE == kModeVerify) {   // (the target row's list, loaded under the merge below)
            if (a.decide == 1 && wave == 0) tl_fetch();
        }
        // the headers (wave 0, lane sl holds slice sl's; slices <= 64), loaded
        // now so that their latency overlaps the list loads and merges
        // (loads unconditional, at clamped in-bounds addresses, and selected
        // afterwards: predicated loads would each wait before the next is issued)
        const SliceHeader& h = a.phdr[size_t(r) * slices + min(lane, slices - 1)];
        const bool hl = lane < slices;
        const uint32_t hf = hl ? get_agent(&h.flags) : 0u, hc = hl ? get_agent(&h.valid) : 0u;
        const float hm = hl ? get_agent(&h.lse_max) : -kInfF;
        const double hs = hl ? get_agent(&h.lse_sum) : 0.0;
        L = WaveList{};
        {
            // The row's top K by each entry's rank among the pooled entries of
            // the slice lists: every entry when they fit the pool, else those
            // whose value reaches the K-th largest of the lists' first entries
            // (K entries of the row reach it, so the row's top K all do); past
            // the pool, the lists are merged as a tree below.
            const int t = int(threadIdx.x);
            int n = slices * K;
            bool pooled_all = true;
            if (n <= kPool) {
                // (padding pairs (-inf, kInvalidId) are equal and rank after every entry)
                if (t < n) {
                    const int sl = t / K;
                    const size_t src = (size_t(r) * slices + size_t(sl)) * kMaxK + size_t(t - sl * K);
                    s_pv[t] = get_agent(&a.pval[src]);
                    s_pi[t] = get_agent(&a.pidx[src]);
                }
                __syncthreads();
            } else if (MODE == kModeSample && n <= kMergeHeld * kTopkThreads) {
                // this thread's entries (loads at clamped addresses, selected after)
                float ev[kMergeHeld];
                int ei[kMergeHeld];
#pragma unroll
                for (int u = 0; u < kMergeHeld; ++u) {
                    const int e = min(t + u * kTopkThreads, n - 1), sl = e / K;
                    const size_t src = (size_t(r) * slices + size_t(sl)) * kMaxK + size_t(e - sl * K);
                    ev[u] = get_agent(&a.pval[src]);
                    ei[u] = get_agent(&a.pidx[src]);
                }
                if (wave == 0) {
                    // the K-th largest value among the lists' first m entries
                    // (at least K entries of the row reach it)
                    const int m = max(1, kWave / slices), sl = lane / m, q = lane - sl * m;
                    const bool ok = sl < slices && q < K;
                    const size_t src = (size_t(r) * slices + size_t(min(sl, slices - 1))) * kMaxK + size_t(min(q, K - 1));
                    const float v = get_agent(&a.pval[src]);
                    const float tv = readlane_f(wave_sort_desc<kD>(ok ? v : -kInfF), K - 1);
                    if (lane == 0) { s_tauv = tv; s_np = 0; }
                }
                __syncthreads();
                const float tv = s_tauv;
#pragma unroll
                for (int u = 0; u < kMergeHeld; ++u) {
                    if (t + u * kTopkThreads < n && ei[u] != kInvalidId && ev[u] >= tv) {
                        const int pos = atomicAdd(&s_np, 1);
                        if (pos < kPool) { s_pv[pos] = ev[u]; s_pi[pos] = ei[u]; }
                    }
                }
                __syncthreads();
                n = s_np;
                pooled_all = n <= kPool;
            } else {
                pooled_all = false;
            }
            if (pooled_all) {
                // (one entry per thread: more than a wave's worth of entries are
                // ranked by every wave, then handed to wave 0 through LDS)
                if (n > kWave || wave == 0) {
                    if (t < n) {
                        const float v = s_pv[t];
                        const int i = s_pi[t];
                        int rank = 0;
#pragma unroll 8
                        for (int q = 0; q < n; ++q) rank += better(s_pv[q], s_pi[q], v, i) ? 1 : 0;
                        if (i != kInvalidId && rank < K) { s_selv[rank] = v; s_seli[rank] = i; }
                    }
                }
                if (n > kWave) __syncthreads();
                if (wave != 0) return;
                wave_sync();
                int real = 0;   // (entries other than padding: every rank below it is placed)
                for (int t0 = 0; t0 < n; t0 += kWave)
                    real += int(__builtin_popcountll(ballot(t0 + lane < n && s_pi[min(t0 + lane, n - 1)] != kInvalidId)));
                L.v = lane < min(K, real) ? s_selv[lane] : -kInfF;
                L.i = lane < min(K, real) ? s_seli[lane] : kInvalidId;
                L.kv = readlane_f(L.v, K - 1);
                L.ki = readlane_i(L.i, K - 1);
                goto merged;
            }
        }
        {
        // every slice's sorted list, merged in: wave w takes a quarter of the
        // slices (the loads of eight in flight together), then the tree above
        const int per = (slices + kTopkWaves - 1) / kTopkWaves;
        const int s_lo = wave * per, s_hi = min(slices, s_lo + per);
        for (int sl0 = s_lo; sl0 < s_hi; sl0 += 8) {
            float bv[8];
            int bi[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const size_t src = (size_t(r) * slices + size_t(min(sl0 + u, slices - 1))) * kMaxK + lane;
                const float lv = get_agent(&a.pval[src]);
                const int li = get_agent(&a.pidx[src]);
                const bool ld = sl0 + u < s_hi && lane < K;
                bv[u] = ld ? lv : -kInfF;
                bi[u] = ld ? li : kInvalidId;
            }
            // the batch's lists merged as a tree (independent merges interleave),
            // then the result into the wave list
            const int n = min(8, s_hi - sl0);
#pragma unroll
            for (int step = 1; step < 8; step <<= 1)
#pragma unroll
                for (int u = 0; u + step < 8; u += 2 * step)
                    if (u + step < n) merge_pair<kD>(bv[u], bi[u], bv[u + step], bi[u + step]);
            list_merge<kD>(L, K, bv[0], bi[0]);
        }
        if (wave & 1) { s_val[wave][lane] = L.v; s_idx[wave][lane] = L.i; }
        __syncthreads();
        tree_merge();
        if (wave != 0) return;
        }
    merged:
        // reductions of the headers across the lanes (the log-sum-exp partials
        // summed in a fixed order)
        f = hf; c = hc; m = hm;
#pragma unroll
        for (int o = 32; o; o >>= 1) {
            f |= shfl_xor_u(f, o);
            c += shfl_xor_u(c, o);
            m = fmaxf(m, shfl_xor_f(m, o));
        }
        s = (hm != -kInfF) ? hs * double(__builtin_amdgcn_exp2f(hm - m)) : 0.0;
#pragma unroll
        for (int o = 32; o; o >>= 1) s += shfl_xor_d(s, o);
        if (lane == 0) a.arrivals[r] = 0u;
    } else if (wave != 0) {
        return;
    }

    // ---- finish the row (wave 0 of the last workgroup)
    s_val[0][lane] = L.v;
    s_idx[0][lane] = L.i;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
    if constexpr (MODE == kModeTopk) {
        if (f & kSliceNan) {
            if (lane == 0) {
                // the other waves' merged lists are dead here: their LDS holds the serial list
                float* vals = s_val[1];
                int* idsl = s_idx[1];
                serial_topk_row<DT>(row, a.vocabulary, K, vals, idsl);
                for (int j = 0; j < K; ++j) {
                    a.ids[size_t(r) * K + j] = idsl[j];
                    a.values[size_t(r) * K + j] = vals[j];
                    if (a.logprobs) a.logprobs[size_t(r) * K + j] = __builtin_nanf("");
                }
            }
        } else if (lane < K) {
            a.ids[size_t(r) * K + lane] = L.i;
            a.values[size_t(r) * K + lane] = L.v;
            if (a.logprobs) {
                const double lse = (double(m) + double(__builtin_amdgcn_logf(float(s)))) * 0.6931471805599453;
                a.logprobs[size_t(r) * K + lane] = (f & kSliceNonfinite) ? __builtin_nanf("") : float(double(L.v) - lse);
            }
        }
        if (lane == 0 && (f & kSliceNonfinite) && a.nonfinite_flag) atomicOr(a.nonfinite_flag, 1u);
    } else if constexpr (MODE == kModePacket) {
        __shared__ float s_tail[3][20];
        __shared__ int s_tail_i[20];
        if (lane == 0) {
            int support = 1;
            const int sel = packet_draw(a.cfg, key, K, s_val[0], s_idx[0], s_tail[0], s_tail[1], &support);
            if (a.score) {
                a.chosen[r] = s_idx[0][sel];
                a.score_gap[r] = sampled_gap<DT>(a.cfg, key, row, a.vocabulary, a.tolerance, a.next[r], sel, support,
                                                 s_val[0], s_idx[0], s_tail[0], s_tail[1], s_tail[2], s_tail_i);
            } else {
                a.out_rows[r].serial = a.serial;
                a.out_rows[r].token = s_idx[0][sel];
                a.out_rows[r].nonfinite = (f & kSliceNonfinite) ? 1u : 0u;
            }
        }
    } else if constexpr (MODE == kModeVerify) {
        const bool refused = verify_list_refused(p);
        const uint32_t rvalid = refused ? 0u : c;
        const uint32_t rflags = ((f & kSliceNonfinite) ? VI_FLAG_NONFINITE : 0u) | (refused ? VI_FLAG_ERROR : 0u);
        if (a.decide >= 3) {   // (read by the position's other row, in this launch)
            if (lane < K) { put_agent(&a.lval[size_t(r) * kMaxK + lane], L.v); put_agent(&a.lidx[size_t(r) * kMaxK + lane], L.i); }
            if (lane == 0) { put_agent(&a.lvalid[r], rvalid); put_agent(&a.lflags[r], rflags); }
        } else {
            if (lane < K) { a.lval[size_t(r) * kMaxK + lane] = L.v; a.lidx[size_t(r) * kMaxK + lane] = L.i; }
            if (lane == 0) { a.lvalid[r] = rvalid; a.lflags[r] = rflags; }
        }
        // the lane's decided positions counted; its last walks the chain
        auto lane_arrive = [&](int l, uint32_t total) {
            uint32_t old = 0;
            if (lane == 0) {
                handoff_stores_done();
                old = __hip_atomic_fetch_add(&a.dv.larr[l], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (uint32_t(__builtin_amdgcn_readfirstlane(old)) != total - 1u) return;
            handoff_acquire();
            const PosDecision* D = a.dv.dec + size_t(l) * (a.dv.drafts + 1);
            lane_chain_wave(l, [&](int q) {
                return PosDecision{get_agent(&D[q].token), get_agent(&D[q].flags), get_agent(&D[q].accept), 0};
            }, a.dv.drafts, a.dv.target_rows, a.dv.drafted, a.params, a.dv.terminal, a.dv.n_terminal, 0,
                            a.dv.accepted, a.dv.committed, a.dv.committed_count, a.dv.lane_flags);
            if (lane == 0) put_agent(&a.dv.larr[l], 0u);
        };
        if (a.decide >= 3) {
            // paired launch: target row (l, j) or draft row (l, j); the later of
            // the two takes position j's decision with the other's list read back
            // (a bonus row decides alone)
            const bool tside = a.decide == 3;
            const int per = tside ? a.dv.target_rows : a.dv.drafts;
            const int l = r / per, j = r - l * per;
            const bool bonus = tside && j == a.dv.drafts;
            bool here = bonus;
            if (!bonus) {
                uint32_t old = 0;
                uint32_t* pc = &a.dv.parr[size_t(l) * (a.dv.drafts + 1) + j];
                if (lane == 0) {
                    handoff_stores_done();
                    old = __hip_atomic_fetch_add(pc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (old == 1u) put_agent(pc, 0u);   // (both rows arrived: reset for the next call)
                }
                here = __builtin_amdgcn_readfirstlane(old) == 1;
            }
            if (here) {
                handoff_acquire();
                if (bonus) {
                    position_decision(p, j, l, a.dv.drafts, a.dv.target_rows, s_val[0], s_idx[0], rvalid, rflags,
                                      nullptr, nullptr, 0u, 0u, a.dv.drafted, a.vocabulary, 0, a.dv.dec);
                } else {
                    const size_t pr = tside ? size_t(l) * a.dv.drafts + j : size_t(l) * a.dv.target_rows + j;
                    const float* ov = tside ? a.dv.dlval : a.dv.tlval;
                    const int* oi = tside ? a.dv.dlidx : a.dv.tlidx;
                    __shared__ float s_ov[kMaxK];
                    __shared__ int s_oi[kMaxK];
                    s_ov[lane] = get_agent(&ov[pr * kMaxK + lane]);
                    s_oi[lane] = get_agent(&oi[pr * kMaxK + lane]);
                    const uint32_t ovalid = get_agent(tside ? &a.dv.dlvalid[pr] : &a.dv.tlvalid[pr]);
                    const uint32_t oflags = get_agent(tside ? &a.dv.dlflags[pr] : &a.dv.tlflags[pr]);
                    wave_sync();
                    if (tside)
                        position_decision(p, j, l, a.dv.drafts, a.dv.target_rows, s_val[0], s_idx[0], rvalid, rflags,
                                          s_ov, s_oi, ovalid, oflags, a.dv.drafted, a.vocabulary, 0, a.dv.dec);
                    else
                        position_decision(p, j, l, a.dv.drafts, a.dv.target_rows, s_ov, s_oi, ovalid, oflags, s_val[0],
                                          s_idx[0], rvalid, rflags, a.dv.drafted, a.vocabulary, 0, a.dv.dec);
                }
                lane_arrive(l, uint32_t(a.dv.drafts + (a.dv.target_rows == a.dv.drafts + 1 ? 1 : 0)));
            }
        } else if (a.decide == 2) {
            // target row r: position j of lane l; a bonus row draws the lane's
            // bonus token from its own list (in LDS)
            const int l = r / a.dv.target_rows, j = r - l * a.dv.target_rows;
            if (j == a.dv.drafts)
                position_decision(p, j, l, a.dv.drafts, a.dv.target_rows, s_val[0], s_idx[0], rvalid, rflags,
                                  nullptr, nullptr, 0u, 0u, a.dv.drafted, a.vocabulary, 0, a.dv.dec);
        } else if (a.decide == 1) {
            // draft row r is position j of lane l: its decision, from the target
            // row's list (in LDS) and this row's (in LDS; entries past K are never
            // read); the lane's last position to finish walks the chain (the
            // bonus draw is the target launch's; agent-scope hand-off of the
            // decisions, the lane's counter reset for the next call)
            const int l = r / a.dv.drafts, j = r - l * a.dv.drafts;
            if (!tl_have) tl_fetch();
            __shared__ float s_tv[kMaxK];
            __shared__ int s_ti[kMaxK];
            s_tv[lane] = tl_v;
            s_ti[lane] = tl_i;
            wave_sync();
            position_decision(p, j, l, a.dv.drafts, a.dv.target_rows, s_tv, s_ti, tl_valid, tl_flags, s_val[0],
                              s_idx[0], rvalid, rflags, a.dv.drafted, a.vocabulary, 0, a.dv.dec);
            lane_arrive(l, uint32_t(a.dv.drafts));
        }
    } else {
        // the candidates' fp64 weights, one per lane (into LDS for the running sums)
        __shared__ double s_w[kMaxK], s_cum[kMaxK];
        const int wcap = (p.temperature > 0.0f) ? min(K, int(c)) : 1;
        if (p.temperature > 0.0f && lane < wcap) s_w[lane] = exp(double(s_val[0][lane]) - double(s_val[0][0]));
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
        uint32_t flags_out = 0;
        if (f & kSliceNonfinite) flags_out |= VI_FLAG_NONFINITE;
        if (lookups)
            flags_out |= a.pstate        ? reinterpret_cast<const PenaltyHeader*>(a.pstate + size_t(r) * a.pl.lane_bytes)->flags
                         : a.hist_counts ? ((f & kSliceBadHistory) ? uint32_t(VI_FLAG_BAD_HISTORY) : 0u) |
                                               ((f & kSliceError) ? uint32_t(VI_FLAG_ERROR) : 0u)
                                         : a.row_flags[r];
        flags_out = uint32_t(__builtin_amdgcn_readfirstlane(int(flags_out)));
        if (flags_out & VI_FLAG_ERROR) {
            if (lane == 0) {
                a.tokens[r] = -1;
                if (a.uniforms) a.uniforms[r] = 0.0;
                if (a.stats) { a.stats[r] = vi_sample_stats{}; a.stats[r].flags = flags_out; }
            }
            return;
        }
        float* pr = a.probs ? a.probs + size_t(r) * size_t(a.probs_stride) : nullptr;
        sample_finish(p, wcap, s_idx[0], a.vocabulary, &a.tokens[r], a.uniforms ? &a.uniforms[r] : nullptr, pr,
                      a.stats ? &a.stats[r] : nullptr, flags_out, c, s_w, s_cum);
        if (a.record && lane == 0) {   // every slice of this row has finished reading the state (last arriver)
            const int32_t t = a.tokens[r];
            if (t >= 0 && t < a.vocabulary) {
                const LaneState ls = lane_state(a.pstate + size_t(r) * a.pl.lane_bytes, a.pl);
                state_record_one(ls, a.pl, a.vocabulary, t);
            }
        }
    }
}

template <int DT, bool VEC, int MODE>
__global__ __launch_bounds__(kTopkThreads, 4) void topk_kernel(TopkArgs a) {
    topk_body<DT, VEC, MODE>(a, int(blockIdx.x), int(gridDim.x), int(blockIdx.y));
}

// Verification's target rows (first t.pair_rows rows of the grid) and draft
// rows in one launch.
template <int DTT, int DTD>
__global__ __launch_bounds__(kTopkThreads, 4) void verify_pair_kernel(TopkArgs t, TopkArgs d) {
    const int y = int(blockIdx.y);
    if (y < t.pair_rows) topk_body<DTT, true, kModeVerify>(t, int(blockIdx.x), int(gridDim.x), y);
    else topk_body<DTD, true, kModeVerify>(d, int(blockIdx.x), int(gridDim.x), y - t.pair_rows);
}

// History hash builder: one workgroup per row.  Each history token is
// inserted with compare-and-swap (open addressing, linear probing), in LDS when
// the table fits (kHashLds slots: the CAS round trips stay on the CU), then
// copied out; larger tables are built in place in global memory.  row_flags[r]
// receives VI_FLAG_BAD_HISTORY for out-of-range tokens and VI_FLAG_ERROR when
// the history exceeds the workspace's max_history.
constexpr int kHashThreads = 512;
constexpr int kHashLds = 8192;   // 64 KB of (token + 1, count)
__global__ __launch_bounds__(kHashThreads) void history_hash_kernel(
    const vi_row_params* params, const int32_t* histories, const int64_t* offsets, int vocabulary,
    uint2* hash, int hash_shift, int hash_slots, uint32_t* row_flags, int64_t max_history) {
    const int r = blockIdx.x;
    const vi_row_params p = params[r];
    if (!topk_route(p) || !penalties_active(p)) return;
    const int64_t b = offsets[r], n = offsets[r + 1] - b;
    __shared__ uint32_t s_flags;
    __shared__ uint2 s_table[kHashLds];
    if (threadIdx.x == 0) s_flags = 0;
    const bool in_lds = hash_slots <= kHashLds;
    uint2* out = hash + size_t(r) * size_t(hash_slots);
    auto build = [&](uint2* table) {
        for (int i = threadIdx.x; i < hash_slots; i += kHashThreads) table[i] = make_uint2(0u, 0u);
        __syncthreads();
        if (n > max_history) {
            if (threadIdx.x == 0) s_flags = VI_FLAG_ERROR;
            return;
        }
        constexpr int kU = 8;   // (the history loads of a round issued together)
        for (int64_t i0 = 0; i0 < n; i0 += int64_t(kU) * kHashThreads) {
            int32_t tk[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const int64_t i = i0 + int64_t(u) * kHashThreads + threadIdx.x;
                tk[u] = i < n ? histories[b + i] : 0;
            }
#pragma unroll 1
            for (int u = 0; u < kU; ++u) {
                if (i0 + int64_t(u) * kHashThreads + threadIdx.x >= n) break;   // (past the history's end)
                const int32_t t = tk[u];
                if (t < 0 || t >= vocabulary) { atomicOr(&s_flags, uint32_t(VI_FLAG_BAD_HISTORY)); continue; }
                uint32_t s = (uint32_t(t) * 0x9E3779B1u) >> hash_shift;
                for (int probe = 0; probe < hash_slots; ++probe) {
                    const uint32_t old = atomicCAS(&table[s].x, 0u, uint32_t(t) + 1u);
                    if (old == 0u || old == uint32_t(t) + 1u) { atomicAdd(&table[s].y, 1u); break; }
                    s = (s + 1u) & uint32_t(hash_slots - 1);
                }
            }
        }
    };
    if (in_lds) build(s_table);
    else build(out);
    __syncthreads();
    if (in_lds)
        for (int i = threadIdx.x; i < hash_slots; i += kHashThreads) out[i] = s_table[i];
    if (threadIdx.x == 0) row_flags[r] = s_flags;
}

template <int MODE>
vi_status launch_mode(const TopkArgs& args, int dtype, bool vec, int rows, int slices, hipStream_t stream) {
    if (slices < 1 || slices > 64) return VI_ERR_INVALID;   // the merge reads one slice header per lane
    const dim3 grid(slices, rows), block(kTopkThreads);
    const size_t dyn = size_t(args.pres_words) * 4;
#define VI_TOPK_LAUNCH(DT, V) hipLaunchKernelGGL((topk_kernel<DT, V, MODE>), grid, block, dyn, stream, args)
    switch (dtype) {
        case VI_BF16: if (vec) VI_TOPK_LAUNCH(VI_BF16, true); else VI_TOPK_LAUNCH(VI_BF16, false); break;
        case VI_F16: if (vec) VI_TOPK_LAUNCH(VI_F16, true); else VI_TOPK_LAUNCH(VI_F16, false); break;
        default: if (vec) VI_TOPK_LAUNCH(VI_F32, true); else VI_TOPK_LAUNCH(VI_F32, false); break;
    }
#undef VI_TOPK_LAUNCH
    return launch_status();
}

bool aligned16(const void* p, int64_t stride, int dtype) {
    return (reinterpret_cast<uintptr_t>(p) % 16 == 0) && ((stride * elem_size(dtype)) % 16 == 0);
}

struct Partials {
    float* pval;
    int* pidx;
    SliceHeader* phdr;
    uint32_t* arrivals;
};
Partials carve_partials(Carver& c, int rows, int slices) {
    Partials p{};
    p.arrivals = c.take<uint32_t>(size_t(rows));
    p.pval = c.take<float>(size_t(rows) * slices * kMaxK);
    p.pidx = c.take<int>(size_t(rows) * slices * kMaxK);
    p.phdr = c.take<SliceHeader>(size_t(rows) * slices);
    return p;
}

}  // namespace

TopkPlan topk_plan(int rows, int vocabulary) {
    // ~1024 workgroups (4 per CU: every one resident at once — the kernels are
    // held to 4 waves per SIMD, and a second round of stragglers would double
    // the time) where the row count allows, slices >= 2048 logits, at most 32
    // slices per row (the row's last workgroup merges every slice list: for
    // one or a few rows, 32 slices measured faster than 64 or 16).
    int slices = rows >= 1024 ? 1 : (1024 + rows - 1) / rows;
    slices = std::min(slices, std::max(1, vocabulary / 2048));
    slices = std::max(1, std::min(slices, 32));
    const int len = slice_len_for(vocabulary, slices);
    slices = (vocabulary + len - 1) / len;
    return {slices, len};
}

size_t topk_partials_bytes_slices(int rows, int slices) {
    return align_up(size_t(rows) * 4, 256) + 2 * align_up(size_t(rows) * slices * kMaxK * 4, 256) +
           align_up(size_t(rows) * slices * sizeof(SliceHeader), 256) + 256;
}

size_t topk_partials_bytes(int rows, int vocabulary) {
    return topk_partials_bytes_slices(rows, topk_plan(rows, vocabulary).slices);
}

vi_status launch_topk_rows(const void* logits, int dtype, int rows, int vocabulary, int64_t stride,
                           int k, int64_t* ids, float* values, float* logprobs,
                           uint32_t* nonfinite_flag, void* ws, size_t ws_bytes, hipStream_t stream) {
    const TopkPlan plan = topk_plan(rows, vocabulary);
    Carver c(ws, ws_bytes);
    const Partials part = carve_partials(c, rows, plan.slices);
    if (!c.ok) return VI_ERR_WORKSPACE;
    TopkArgs a{};
    a.logits = logits; a.vocabulary = vocabulary; a.stride = stride; a.slice_len = plan.slice_len;
    a.pval = part.pval; a.pidx = part.pidx; a.phdr = part.phdr; a.arrivals = part.arrivals;
    a.k = k; a.ids = ids; a.values = values; a.logprobs = logprobs; a.nonfinite_flag = nonfinite_flag;
    return launch_mode<kModeTopk>(a, dtype, aligned16(logits, stride, dtype), rows, plan.slices, stream);
}

vi_status launch_packet(const void* scores, int dtype, int rows, int vocabulary, int64_t stride,
                        const vi_device_sampling& cfg, const PacketKeys& keys, uint64_t serial,
                        vi_greedy_row* out, void* ws, size_t ws_bytes, hipStream_t stream) {
    const TopkPlan plan = topk_plan(rows, vocabulary);
    Carver c(ws, ws_bytes);
    const Partials part = carve_partials(c, rows, plan.slices);
    if (!c.ok) return VI_ERR_WORKSPACE;
    TopkArgs a{};
    a.logits = scores; a.vocabulary = vocabulary; a.stride = stride; a.slice_len = plan.slice_len;
    a.pval = part.pval; a.pidx = part.pidx; a.phdr = part.phdr; a.arrivals = part.arrivals;
    a.cfg = cfg; a.keys = keys; a.serial = serial; a.out_rows = out;
    return launch_mode<kModePacket>(a, dtype, aligned16(scores, stride, dtype), rows, plan.slices, stream);
}

vi_status launch_sampled_scores(const void* scores, int dtype, int rows, int vocabulary, int64_t stride,
                                const vi_device_sampling& cfg, int first_key, float tolerance,
                                const int64_t* next, int64_t* chosen, float* gap, void* ws, size_t ws_bytes,
                                hipStream_t stream) {
    const TopkPlan plan = topk_plan(rows, vocabulary);
    Carver c(ws, ws_bytes);
    const Partials part = carve_partials(c, rows, plan.slices);
    if (!c.ok) return VI_ERR_WORKSPACE;
    TopkArgs a{};
    a.logits = scores; a.vocabulary = vocabulary; a.stride = stride; a.slice_len = plan.slice_len;
    a.pval = part.pval; a.pidx = part.pidx; a.phdr = part.phdr; a.arrivals = part.arrivals;
    a.cfg = cfg; a.keys.first = first_key; a.score = 1; a.tolerance = tolerance;
    a.next = next; a.chosen = chosen; a.score_gap = gap;
    return launch_mode<kModePacket>(a, dtype, aligned16(scores, stride, dtype), rows, plan.slices, stream);
}

vi_status launch_verify_lists(const void* logits, int dtype, int rows, int layout_rows, int layout_slices,
                              int vocabulary, int64_t stride, const vi_row_params* params, int params_div,
                              float* lval, int* lidx, uint32_t* lvalid, uint32_t* lflags, int skip_unlisted,
                              void* ws, size_t ws_bytes, hipStream_t stream, const VerifyDecideArgs* decide,
                              int decide_mode) {
    // Partials carved for (layout_rows, layout_slices) so that launches over
    // different row counts share one counter layout in one workspace.
    const TopkPlan plan = topk_plan(rows, vocabulary);
    if (rows > layout_rows || plan.slices > layout_slices) return VI_ERR_WORKSPACE;
    Carver c(ws, ws_bytes);
    const Partials part = carve_partials(c, layout_rows, layout_slices);
    if (!c.ok) return VI_ERR_WORKSPACE;
    TopkArgs a{};
    a.logits = logits; a.vocabulary = vocabulary; a.stride = stride; a.slice_len = plan.slice_len;
    a.pval = part.pval; a.pidx = part.pidx; a.phdr = part.phdr; a.arrivals = part.arrivals;
    a.params = params; a.params_div = params_div;
    a.lval = lval; a.lidx = lidx; a.lvalid = lvalid; a.lflags = lflags; a.skip_unlisted = skip_unlisted;
    if (decide) { a.decide = decide_mode; a.dv = *decide; }
    return launch_mode<kModeVerify>(a, dtype, aligned16(logits, stride, dtype), rows, plan.slices, stream);
}

bool verify_pair_supported(const void* target, int target_dtype, int64_t target_stride, const void* draft,
                           int draft_dtype, int64_t draft_stride) {
    auto ok = [](const void* p, int dt, int64_t stride) {
        return (dt == VI_BF16 || dt == VI_F16) && aligned16(p, stride, dt);
    };
    return ok(target, target_dtype, target_stride) && ok(draft, draft_dtype, draft_stride);
}

vi_status launch_verify_pair(const void* target, int target_dtype, int64_t target_stride, const void* draft,
                             int draft_dtype, int64_t draft_stride, int lanes, int vocabulary,
                             const vi_row_params* params, int layout_rows, int layout_slices, float* tval, int* tidx,
                             uint32_t* tvalid, uint32_t* tflags, float* dval, int* didx, uint32_t* dvalid,
                             uint32_t* dflags, const VerifyDecideArgs& decide, void* ws, size_t ws_bytes,
                             hipStream_t stream, int skip_unlisted) {
    if (!verify_pair_supported(target, target_dtype, target_stride, draft, draft_dtype, draft_stride))
        return VI_ERR_UNSUPPORTED;
    const int trows = lanes * decide.target_rows, drows = lanes * decide.drafts;
    // one slicing for both halves, about 1,024 workgroups for the two row sets
    // together (one round at four per CU; a slice of up to two held batches)
    TopkPlan plan;
    plan.slices = std::max(1, std::min({32, (1024 + trows + drows - 1) / (trows + drows), vocabulary / 2048}));
    plan.slice_len = slice_len_for(vocabulary, plan.slices);
    plan.slices = (vocabulary + plan.slice_len - 1) / plan.slice_len;
    if (trows + drows > layout_rows || plan.slices > layout_slices) return VI_ERR_WORKSPACE;
    Carver c(ws, ws_bytes);
    const Partials part = carve_partials(c, layout_rows, layout_slices);
    if (!c.ok) return VI_ERR_WORKSPACE;
    TopkArgs t{};
    t.logits = target; t.vocabulary = vocabulary; t.stride = target_stride; t.slice_len = plan.slice_len;
    t.pval = part.pval; t.pidx = part.pidx; t.phdr = part.phdr; t.arrivals = part.arrivals;
    t.params = params; t.params_div = decide.target_rows;
    t.lval = tval; t.lidx = tidx; t.lvalid = tvalid; t.lflags = tflags;
    t.decide = 3; t.dv = decide; t.pair_rows = trows; t.skip_unlisted = skip_unlisted;
    TopkArgs d = t;   // (the draft half: its rows' partials after the target half's)
    const size_t off = size_t(trows) * plan.slices;
    d.logits = draft; d.stride = draft_stride;
    d.pval = part.pval + off * kMaxK; d.pidx = part.pidx + off * kMaxK; d.phdr = part.phdr + off;
    d.arrivals = part.arrivals + trows;
    d.params_div = decide.drafts;
    d.lval = dval; d.lidx = didx; d.lvalid = dvalid; d.lflags = dflags;
    d.decide = 4;
    const dim3 grid(plan.slices, trows + drows), block(kTopkThreads);
#define VI_PAIR(A, B) hipLaunchKernelGGL((verify_pair_kernel<A, B>), grid, block, 0, stream, t, d)
    if (target_dtype == VI_BF16) {
        if (draft_dtype == VI_BF16) VI_PAIR(VI_BF16, VI_BF16); else VI_PAIR(VI_BF16, VI_F16);
    } else {
        if (draft_dtype == VI_BF16) VI_PAIR(VI_F16, VI_BF16); else VI_PAIR(VI_F16, VI_F16);
    }
#undef VI_PAIR
    return launch_status();
}

size_t history_hash_slots(int64_t max_history) {
    size_t slots = 64;
    while (slots < size_t(2 * std::max<int64_t>(max_history, 1))) slots <<= 1;
    return slots;
}

size_t sample_workspace(int rows, int vocabulary, int64_t max_history) {
    size_t bytes = topk_partials_bytes(rows, vocabulary);
    bytes += align_up(size_t(rows) * 4, 256);
    if (max_history > 0) bytes += align_up(size_t(rows) * history_hash_slots(max_history) * 8, 256);
    bytes += std::max({full_workspace(rows, vocabulary), wide_workspace(rows, vocabulary),
                       stream_workspace(rows, vocabulary, max_history)});
    return bytes + 1024;
}

vi_status launch_sample(const SampleArgs& s, void* ws, size_t ws_bytes, hipStream_t stream) {
    const TopkPlan plan = topk_plan(s.rows, s.vocabulary);
    Carver c(ws, ws_bytes);
    const Partials part = carve_partials(c, s.rows, plan.slices);
    uint2* hash = nullptr;
    uint32_t* row_flags = c.take<uint32_t>(size_t(s.rows));
    int slots = 0, shift = 0;
    if (s.pstate) {   // the lanes' own hashes
        slots = s.playout.slots;
        shift = s.playout.shift;
    } else if (s.max_history > 0 && s.histories && s.offsets) {
        slots = int(history_hash_slots(s.max_history));
        shift = 32 - __builtin_ctz(unsigned(slots));
        hash = c.take<uint2>(size_t(s.rows) * slots);
    }
    const size_t full_bytes = s.dtype == VI_F32 ? wide_workspace(s.rows, s.vocabulary)
                                                 : std::max(full_workspace(s.rows, s.vocabulary),
                                                            stream_workspace(s.rows, s.vocabulary, s.max_history));
    unsigned char* full_ws = c.take<unsigned char>(full_bytes);
    if (!c.ok) return VI_ERR_WORKSPACE;
    const bool run_topk = (s.route_mask & VI_ROUTE_TOPK) != 0;
    const bool full_ok = s.dtype == VI_F32 ? wide_supported(s.vocabulary, s.stride)
                                           : full_supported(s.dtype, s.vocabulary, s.stride);
    vi_status st = VI_OK;
    // Histories counted straight into each slice's LDS when the slice's counts
    // fit and no fp32 full-route row needs the hash: no hash launch
    const bool lds_counts = hash && size_t(plan.slice_len) * 4 <= kHistCountLds &&
                            !(s.dtype == VI_F32 && (s.route_mask & VI_ROUTE_FULL) && full_ok);
    if (run_topk && hash && !lds_counts) {
        hipLaunchKernelGGL(history_hash_kernel, dim3(s.rows), dim3(kHashThreads), 0, stream, s.params, s.histories,
                           s.offsets, s.vocabulary, hash, shift, slots, row_flags, s.max_history);
        if (launch_status() != VI_OK) return VI_ERR_LAUNCH;
    }
    // Rows of both routes: the top-k launch (the shorter of the two) runs on
    // the side stream beside the full-vocabulary route's launch chain, which
    // stays on the caller's stream, so neither cross-stream hand-over sits on
    // the chain's path; the side stream is joined back into the caller's before
    // the call returns.  The two routes' rows, outputs and workspace are
    // disjoint (each kernel skips the other route's rows).
    const bool full_run = (s.route_mask & VI_ROUTE_FULL) && full_ok;
    SideStream* side = (run_topk && full_run) ? side_stream() : nullptr;
    if (side && (hipEventRecord(side->fork, stream) != hipSuccess ||
                 hipStreamWaitEvent(side->stream, side->fork, 0) != hipSuccess)) {
        (void)hipGetLastError();
        side = nullptr;
    }
    const hipStream_t topk_stream = side ? side->stream : stream;
    if (run_topk) {
        TopkArgs a{};
        a.logits = s.logits; a.vocabulary = s.vocabulary; a.stride = s.stride; a.slice_len = plan.slice_len;
        a.pval = part.pval; a.pidx = part.pidx; a.phdr = part.phdr; a.arrivals = part.arrivals;
        a.params = s.params; a.hash = lds_counts ? nullptr : hash; a.row_flags = row_flags; a.hash_shift = shift;
        a.hash_slots = slots; a.offsets = s.offsets; a.histories = s.histories; a.max_history = s.max_history;
        // the presence bitmap (one bit per token of a slice, in dynamic LDS) when
        // penalties are read: up to 64 KB (a slice of up to 524,288 tokens); or
        // the slice's history counts
        if (lds_counts) {
            a.hist_counts = 1;
            a.pres_words = plan.slice_len;
        } else if (hash || s.pstate) {
            const size_t words = size_t(plan.slice_len + 31) / 32;
            a.pres_words = words * 4 <= 65536 ? int(words) : 0;
        }
        a.pstate = s.pstate; a.pl = s.playout; a.record = s.record;
        a.tokens = s.tokens; a.uniforms = s.uniforms; a.probs = s.probs; a.probs_stride = s.probs_stride;
        a.stats = s.stats;
        // fp32 logits / unaligned rows: full-route rows fail loudly in the top-k launch
        a.full_rows_unsupported = (full_ok && (s.route_mask & VI_ROUTE_FULL)) ? 0 : (full_ok ? 0 : 1);
        st = launch_mode<kModeSample>(a, s.dtype, aligned16(s.logits, s.stride, s.dtype), s.rows, plan.slices,
                                      topk_stream);
        if (st != VI_OK && !side) return st;
    }
    if (full_run) {
        if (st == VI_OK)
            st = s.dtype == VI_F32     ? launch_wide(s, full_ws, full_bytes, hash, shift, slots, row_flags, stream)
                 : stream_supported(s) ? launch_stream(s, full_ws, full_bytes, stream)
                                       : launch_full(s, full_ws, full_bytes, stream);
    } else if ((s.route_mask & VI_ROUTE_FULL) && !run_topk) {
        return VI_ERR_UNSUPPORTED;
    }
    // joined also when a launch failed: the side work uses the caller's workspace
    if (side && (hipEventRecord(side->join, side->stream) != hipSuccess ||
                 hipStreamWaitEvent(stream, side->join, 0) != hipSuccess))
        return VI_ERR_LAUNCH;
    return st;
}

}  // namespace vi
