// oracle.cpp — CPU restatement of The8Darkness/voidinfer's token-sampling path.
//
// TEST INFRASTRUCTURE ONLY: the checker for the HIP library, never linked into it.
// Build: oracle/Makefile (g++ -O3 -ffp-contract=off; no fast-math).  Every routine
// cites the reference lines it restates; EXTENSION marks semantics the reference
// does not implement (they follow the build's own specification and are pinned by
// closed forms in tests/).
#include "oracle.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <limits>
#include <numeric>
#include <thread>
#include <vector>

namespace {

constexpr float kInf = std::numeric_limits<float>::infinity();

inline float from_bits(uint32_t b) { float f; std::memcpy(&f, &b, 4); return f; }
inline uint32_t to_bits(float f) { uint32_t b; std::memcpy(&b, &f, 4); return b; }

// Independent binary16 decode, the mathematical form of
// tests/test_exl3_greedy_device.cu:11-17 (no bit-twiddling converter).
float half_value(uint16_t h) {
    const int exp = (h >> 10) & 31, mant = h & 1023;
    if (exp == 31) return mant ? std::numeric_limits<float>::quiet_NaN() : ((h & 0x8000) ? -kInf : kInf);
    const float magnitude = exp ? std::ldexp(float(1024 + mant), exp - 25) : std::ldexp(float(mant), -24);
    return (h & 0x8000) ? -magnitude : magnitude;
}
inline float bf16_value(uint16_t b) { return from_bits(uint32_t(b) << 16); }

inline float element(const void* row, int dtype, int64_t i) {
    switch (dtype) {
        case VI_BF16: return bf16_value(static_cast<const uint16_t*>(row)[i]);
        case VI_F16: return half_value(static_cast<const uint16_t*>(row)[i]);
        default: return static_cast<const float*>(row)[i];
    }
}
inline size_t elem_bytes(int dtype) { return dtype == VI_F32 ? 4 : 2; }
inline const void* row_ptr(const void* base, int dtype, int64_t row, int64_t stride) {
    return static_cast<const unsigned char*>(base) + size_t(row) * size_t(stride) * elem_bytes(dtype);
}

// Round to nearest even, fp32 -> bfloat16 bits.
uint16_t to_bf16(float f) {
    uint32_t u = to_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);  // quiet NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}
// Round to nearest even, fp32 -> binary16 bits (subnormals and overflow to inf).
uint16_t to_f16(float f) {
    uint32_t x = to_bits(f);
    const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
    x &= 0x7fffffffu;
    if (x >= 0x7f800000u) return sign | (x > 0x7f800000u ? 0x7e00u : 0x7c00u);
    if (x >= 0x477ff000u) return sign | 0x7c00u;  // >= 65520 rounds to infinity
    if (x < 0x38800000u) {                         // below 2^-14: subnormal grid 2^-24
        const float scaled = from_bits(x) * 16777216.0f;  // exact power-of-two scaling
        return sign | uint16_t(std::nearbyint(scaled));
    }
    const uint32_t mant = x & 0x7fffffu;
    uint32_t h = ((((x >> 23) & 0xffu) - 127u + 15u) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return sign | uint16_t(h);
}

inline uint32_t order_key(float v) {
    uint32_t u = to_bits(v);
    if (v == 0.0f) u = 0;  // +0 and -0 compare equal
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// exl3_sampled_better (sampled_select.cuh:55-57): value desc, lower id wins ties.
inline bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

// ---------------------------------------------------------------- extended rows
// EXTENSION: the batched sampler's filtered distribution of one row.
struct RowDist {
    uint32_t flags = 0;
    int n_valid = 0;
    bool greedy = false;
    int32_t greedy_token = -1;
    std::vector<int32_t> ids;   // sorted (z desc, id asc), first `sorted` entries
    std::vector<float> z;
    std::vector<double> w;      // exp(z - z0), fp64
    int cap = 0, support = 0;
    double s_cap = 0, s_n = 0;
    double topp_margin = INFINITY, minp_margin = INFINITY;
};

// Penalty of one history token (EXTENSION; conventions: HF repetition
// penalty `x>0 ? x/r : x*r`, then OpenAI frequency and presence
// `x - f*count - p`).  Arithmetic in fp32 without contraction, then the
// penalized logit is stored in the logits' own dtype (round to nearest even).
inline float penalize(float x, uint32_t count, const vi_row_params& p, int dtype) {
    float y = x;
    if (p.repetition_penalty != 1.0f) y = (y > 0.0f) ? y / p.repetition_penalty : y * p.repetition_penalty;
    if (p.frequency_penalty != 0.0f) {
        const float t = p.frequency_penalty * float(count);
        y = y - t;
    }
    if (p.presence_penalty != 0.0f) y = y - p.presence_penalty;
    if (dtype == VI_BF16) return bf16_value(to_bf16(y));
    if (dtype == VI_F16) return half_value(to_f16(y));
    return y;
}

inline bool penalties_active(const vi_row_params& p) {
    return p.repetition_penalty != 1.0f || p.presence_penalty != 0.0f || p.frequency_penalty != 0.0f;
}

void build_row(const void* row, int dtype, int vocabulary, const vi_row_params& p,
               const int32_t* history, int64_t history_len, RowDist& d,
               std::vector<uint32_t>& counts) {
    d = RowDist{};
    const bool pen = penalties_active(p) && history_len > 0;
    if (pen) {
        counts.assign(size_t(vocabulary), 0u);
        for (int64_t i = 0; i < history_len; ++i) {
            const int32_t t = history[i];
            if (t < 0 || t >= vocabulary) { d.flags |= VI_FLAG_BAD_HISTORY; continue; }
            ++counts[size_t(t)];
        }
    }
    std::vector<std::pair<int32_t, float>> valid;
    valid.reserve(size_t(vocabulary));
    for (int v = 0; v < vocabulary; ++v) {
        float x = element(row, dtype, v);
        if (!std::isfinite(x)) { d.flags |= VI_FLAG_NONFINITE; continue; }
        if (pen && counts[size_t(v)]) {
            x = penalize(x, counts[size_t(v)], p, dtype);
            if (!std::isfinite(x)) { d.flags |= VI_FLAG_NONFINITE; continue; }
        }
        if (x == 0.0f) x = 0.0f;
        valid.emplace_back(v, x);
    }
    if (valid.empty()) { d.flags |= VI_FLAG_EMPTY; return; }
    if (!(p.temperature > 0.0f)) {
        // Temperature 0: (penalized) argmax, first maximum.
        d.greedy = true;
        float best = -kInf; int32_t id = -1;
        for (auto& e : valid) if (id < 0 || e.second > best) { best = e.second; id = e.first; }
        d.n_valid = int(valid.size());
        d.greedy_token = id;
        d.support = 1;
        return;
    }
    const float inv_t = 1.0f / p.temperature;
    std::vector<uint64_t> keys;
    keys.reserve(valid.size());
    for (auto& e : valid) {
        const float z = e.second * inv_t;
        if (!std::isfinite(z)) { d.flags |= VI_FLAG_NONFINITE; continue; }
        keys.push_back((uint64_t(order_key(z)) << 32) | uint64_t(0xffffffffu - uint32_t(e.first)));
    }
    if (keys.empty()) { d.flags |= VI_FLAG_EMPTY; return; }
    d.n_valid = int(keys.size());
    d.cap = (p.top_k > 0) ? std::min(p.top_k, d.n_valid) : d.n_valid;
    auto desc = [](uint64_t a, uint64_t b) { return a > b; };
    if (d.cap < d.n_valid) std::partial_sort(keys.begin(), keys.begin() + d.cap, keys.end(), desc);
    else std::sort(keys.begin(), keys.end(), desc);
    d.ids.resize(size_t(d.cap)); d.z.resize(size_t(d.cap)); d.w.resize(size_t(d.cap));
    for (int j = 0; j < d.cap; ++j) {
        const int32_t id = int32_t(0xffffffffu - uint32_t(keys[size_t(j)]));
        d.ids[size_t(j)] = id;
        d.z[size_t(j)] = element(row, dtype, id);  // placeholder, replaced below
    }
    // z of the sorted ids (recomputed from the stored penalized values).
    {
        std::vector<float> xp(static_cast<size_t>(vocabulary), 0.0f);
        for (auto& e : valid) xp[size_t(e.first)] = e.second;
        for (int j = 0; j < d.cap; ++j) d.z[size_t(j)] = xp[size_t(d.ids[size_t(j)])] * inv_t;
    }
    const double z0 = double(d.z[0]);
    for (int j = 0; j < d.cap; ++j) d.w[size_t(j)] = std::exp(double(d.z[size_t(j)]) - z0);
    double s = 0;
    for (int j = 0; j < d.cap; ++j) s += d.w[size_t(j)];
    d.s_cap = s;
    // Truncation (the reference's loop, sampled_select.cuh:100-108, over the
    // whole cap set): min_p cut before accumulating, top_p cut after.
    const double minp = double(p.min_p), target = double(p.top_p) * s;
    double cum = 0; int n = 0;
    for (int j = 0; j < d.cap; ++j) {
        if (p.min_p > 0.0f && d.w[size_t(j)] < minp * d.w[0]) {
            d.minp_margin = std::fabs(d.w[size_t(j)] - minp);
            if (j > 0) d.minp_margin = std::min(d.minp_margin, std::fabs(d.w[size_t(j - 1)] - minp));
            break;
        }
        const double before = cum;
        cum += d.w[size_t(j)]; n = j + 1;
        if (p.top_p < 1.0f && cum >= target) {
            d.topp_margin = std::min(std::fabs(cum - target), std::fabs(before - target)) / s;
            break;
        }
    }
    if (n < 1) n = 1;
    d.support = n;
    double sn = 0;
    for (int j = 0; j < n; ++j) sn += d.w[size_t(j)];
    d.s_n = sn;
}

// Inverse CDF in sorted order: first support entry whose inclusive cumulative
// weight exceeds u * S_n (fallback: the last support entry).
int draw_sorted(const RowDist& d, double u, double* margin) {
    const double target = u * d.s_n;
    double cum = 0, before = 0;
    int pick = d.support - 1;
    for (int j = 0; j < d.support; ++j) {
        before = cum;
        cum += d.w[size_t(j)];
        if (cum > target) { pick = j; break; }
    }
    if (margin) *margin = std::min(std::fabs(cum - target), std::fabs(before - target)) / d.s_n;
    return pick;
}

template <class F>
void parallel_rows(int rows, int threads, F&& fn) {
    if (threads <= 0) threads = int(std::max(1u, std::thread::hardware_concurrency()));
    threads = std::max(1, std::min(threads, rows));
    if (threads == 1) { for (int r = 0; r < rows; ++r) fn(r); return; }
    std::atomic<int> next{0};
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; ++t)
        pool.emplace_back([&] { for (int r; (r = next.fetch_add(1)) < rows;) fn(r); });
    for (auto& th : pool) th.join();
}

}  // namespace

extern "C" {

float or_decode(int dtype, uint32_t bits) {
    if (dtype == VI_BF16) return bf16_value(uint16_t(bits));
    if (dtype == VI_F16) return half_value(uint16_t(bits));
    return from_bits(bits);
}

uint32_t or_round_to_dtype(int dtype, float value) {
    if (dtype == VI_BF16) return to_bf16(value);
    if (dtype == VI_F16) return to_f16(value);
    return to_bits(value);
}

uint32_t or_order_key(float value) { return order_key(value); }

// SplitMix64 finalizer (sampled_select.cuh:41-46, request_sampling_state.h:113-118).
uint64_t or_splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// exl3_sampled_gumbel (sampled_select.cuh:47-54).
float or_gumbel(uint64_t seed, int32_t key, int32_t token) {
    uint64_t h = or_splitmix64(seed ^ (uint64_t(uint32_t(key)) * 0xD1B54A32D192ED03ull));
    h = or_splitmix64(h ^ (uint64_t(uint32_t(token)) * 0x2545F4914F6CDD1Dull));
    const float u = (float(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
    return -std::log(-std::log(u));
}

// Philox4x32-10, Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as
// 1, 2, 3" (SC'11): multipliers 0xD2511F53 / 0xCD9E8D57, Weyl key bumps
// 0x9E3779B9 / 0xBB67AE85, 10 rounds.  Word order as rocRAND's
// philox4x32_10_engine (counter = x,y,z,w; key = x,y).
void or_philox4x32_10(const uint32_t counter[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = counter[0], c1 = counter[1], c2 = counter[2], c3 = counter[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int round = 0; round < 10; ++round) {
        if (round) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        const uint64_t p0 = uint64_t(0xD2511F53u) * c0;
        const uint64_t p1 = uint64_t(0xCD9E8D57u) * c2;
        const uint32_t n0 = uint32_t(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n1 = uint32_t(p1);
        const uint32_t n2 = uint32_t(p0 >> 32) ^ c3 ^ k1;
        const uint32_t n3 = uint32_t(p0);
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

double or_uniform(uint64_t seed, uint32_t lane, int32_t position, uint32_t purpose) {
    const uint32_t ctr[4] = {uint32_t(position), 0u, lane, purpose};
    const uint32_t key[2] = {uint32_t(seed), uint32_t(seed >> 32)};
    uint32_t out[4];
    or_philox4x32_10(ctr, key, out);
    const uint64_t m = (uint64_t(out[0]) << 21) | uint64_t(out[1] >> 11);
    return double(m) * 0x1p-53;
}

// exl3_greedy_packet_kernel (greedy_packet.cuh:15-77): largest finite value,
// lowest index on ties, non-finite skipped and flagged, index = V if none.
int or_greedy_rows(const void* logits, int dtype, int rows, int vocabulary, int64_t row_stride,
                   uint64_t serial, vi_greedy_row* out) {
    if (rows < 0 || vocabulary <= 0 || row_stride < vocabulary) return VI_ERR_INVALID;
    for (int r = 0; r < rows; ++r) {
        const void* row = row_ptr(logits, dtype, r, row_stride);
        float best = -kInf; int index = vocabulary; uint32_t bad = 0;
        for (int i = 0; i < vocabulary; ++i) {
            const float x = element(row, dtype, i);
            if (!std::isfinite(x)) { bad = 1; continue; }
            if (x > best || (x == best && i < index)) { best = x; index = i; }
        }
        out[r].serial = serial; out[r].token = index; out[r].nonfinite = bad;
    }
    return VI_OK;
}

// exl3_branch_greedy host path (branch_reference.h:23-31).
int64_t or_cpu_greedy(const float* logits, int64_t vocabulary) {
    if (vocabulary <= 0) return -1;
    for (int64_t i = 0; i < vocabulary; ++i) if (!std::isfinite(logits[i])) return -1;
    return std::max_element(logits, logits + vocabulary) - logits;
}

// Top-k (dflash2_draft.cu:1827-1862 serial NaN order; test_exl3_dflash2_topk.h:11-37
// partial_sort order otherwise), generalized from 16 to k.
int or_topk_rows(const void* logits, int dtype, int rows, int vocabulary, int64_t row_stride,
                 int k, int64_t* ids, float* values, float* logprobs, uint32_t* nonfinite) {
    if (rows < 0 || k < 1 || k > vocabulary || row_stride < vocabulary) return VI_ERR_INVALID;
    uint32_t any_nonfinite = 0;
    std::vector<float> x(static_cast<size_t>(vocabulary));
    for (int r = 0; r < rows; ++r) {
        const void* row = row_ptr(logits, dtype, r, row_stride);
        bool nan = false, finite = true;
        for (int i = 0; i < vocabulary; ++i) {
            x[size_t(i)] = element(row, dtype, i);
            nan = nan || std::isnan(x[size_t(i)]);
            finite = finite && std::isfinite(x[size_t(i)]);
        }
        if (!finite) any_nonfinite = 1;
        std::vector<int> sel;
        if (!nan) {
            std::vector<int> order(static_cast<size_t>(vocabulary));
            std::iota(order.begin(), order.end(), 0);
            std::partial_sort(order.begin(), order.begin() + k, order.end(), [&](int a, int b) {
                return x[size_t(a)] > x[size_t(b)] || (x[size_t(a)] == x[size_t(b)] && a < b);
            });
            sel.assign(order.begin(), order.begin() + k);
        } else {
            for (int i = 0; i < vocabulary; ++i) {
                if (int(sel.size()) == k && !(x[size_t(i)] > x[size_t(sel.back())])) continue;
                if (int(sel.size()) == k) sel.pop_back();
                auto position = sel.end();
                while (position != sel.begin() && x[size_t(*(position - 1))] < x[size_t(i)]) --position;
                sel.insert(position, i);
            }
        }
        double lse = std::numeric_limits<double>::quiet_NaN();
        if (finite) {
            double m = -INFINITY;
            for (int i = 0; i < vocabulary; ++i) m = std::max(m, double(x[size_t(i)]));
            double s = 0;
            for (int i = 0; i < vocabulary; ++i) s += std::exp(double(x[size_t(i)]) - m);
            lse = m + std::log(s);
        }
        for (int j = 0; j < k; ++j) {
            const int id = sel[size_t(j)];
            ids[size_t(r) * k + j] = id;
            values[size_t(r) * k + j] = x[size_t(id)];
            if (logprobs) logprobs[size_t(r) * k + j] = float(double(x[size_t(id)]) - lse);
        }
    }
    if (nonfinite) *nonfinite = any_nonfinite;
    return VI_OK;
}

}  // extern "C"

namespace {

// One row of the coupled sampler (sampled_select.cuh:79-116, 121-193): the
// presence-penalized top-cap candidates, the truncated support and the
// perturbed values.  The reference compiles with nvcc's default --fmad=true;
// the two multiply-add expressions of the draw (cand*inv_temp - m,
// cand*inv_temp + G) are therefore fused, as here.
struct PacketRow {
    int cap = 0, support = 1, selected = 0;
    float val[20], value[20] = {}, prob[20] = {}, sum = 0.0f;
    int idx[20];
    uint32_t bad = 0;
};

int packet_cap(const vi_device_sampling& cfg) {
    int cap = 20;
    if (cfg.top_k > 0 && cfg.top_k < cap) cap = cfg.top_k;
    return cap;
}

bool packet_seen(const vi_device_sampling& cfg, int key, const int* path, int path_count, int v) {
    bool seen = cfg.first_occurrence && cfg.first_occurrence[v] < key;
    for (int i = 0; i < path_count && !seen; ++i) seen = path[i] == v;
    return seen;
}

// exl3_sampled_support (sampled_select.cuh:283-298).
int packet_support(const float* value, int cap, const vi_device_sampling& cfg, float* prob, float* sum_out) {
    const float inv_temp = 1.0f / cfg.temperature;
    const float m = value[0] * inv_temp;
    float sum = 0.0f;
    for (int j = 0; j < cap; ++j) { prob[j] = std::exp(std::fmaf(value[j], inv_temp, -m)); sum += prob[j]; }
    const float min_p_thresh = cfg.min_p > 0.0f ? cfg.min_p * prob[0] : -1.0f;
    const bool top_p_active = cfg.top_p < 1.0f;
    const float top_p_target = cfg.top_p * sum;
    float cum = 0.0f; int support = 0;
    for (int j = 0; j < cap; ++j) {
        if (min_p_thresh >= 0.0f && prob[j] < min_p_thresh) break;
        cum += prob[j]; support = j + 1;
        if (top_p_active && cum >= top_p_target) break;
    }
    if (sum_out) *sum_out = sum;
    return support < 1 ? 1 : support;
}

void packet_row(const void* row, int dtype, int vocabulary, const vi_device_sampling& cfg, int key,
                const int* path, int path_count, PacketRow& o) {
    o = PacketRow{};
    o.cap = std::min(packet_cap(cfg), vocabulary);
    for (int j = 0; j < 20; ++j) { o.val[j] = -kInf; o.idx[j] = 0x7fffffff; }
    const int cap = o.cap;
    for (int v = 0; v < vocabulary; ++v) {
        float x = element(row, dtype, v);
        if (!std::isfinite(x)) { o.bad = 1; continue; }
        if (cfg.presence_penalty != 0.0f && packet_seen(cfg, key, path, path_count, v)) x -= cfg.presence_penalty;
        if (!better(x, v, o.val[cap - 1], o.idx[cap - 1])) continue;
        int pos = cap - 1;
        while (pos > 0 && better(x, v, o.val[pos - 1], o.idx[pos - 1])) {
            o.val[pos] = o.val[pos - 1]; o.idx[pos] = o.idx[pos - 1]; --pos;
        }
        o.val[pos] = x; o.idx[pos] = v;
    }
    if (!(cfg.temperature > 0.0f)) {
        o.value[0] = o.val[0];
        return;
    }
    const float inv_temp = 1.0f / cfg.temperature;
    o.support = packet_support(o.val, cap, cfg, o.prob, &o.sum);
    int best = 0;
    for (int j = 0; j < o.support; ++j) {
        o.value[j] = std::fmaf(o.val[j], inv_temp, or_gumbel(cfg.seed, key, o.idx[j]));
        if (o.value[j] > o.value[best]) best = j;
    }
    o.selected = best;
}

}  // namespace

extern "C" {

// exl3_launch_sampled_packet with one-CTA semantics (sampled_select.cuh:79-116,
// 121-193, 218-225, 283-298, 362-377).
int or_sampled_packet(const void* scores, int dtype, int rows, int vocabulary, int64_t row_stride,
                      const vi_device_sampling* cfg, int first_key, const int32_t* depths,
                      int n_depths, const int32_t* inputs, int n_inputs, uint64_t serial,
                      vi_greedy_row* out, or_packet_detail* detail) {
    if (rows <= 0 || rows > 16 || vocabulary <= 0 || row_stride < vocabulary || !cfg) return VI_ERR_INVALID;
    int depth[16]; int input_count = 0; int input[16];
    const bool tree = n_depths == rows && depths;
    for (int r = 0; r < rows; ++r) depth[r] = tree ? depths[r] : r;
    if (n_inputs == rows && inputs) { input_count = rows; for (int r = 0; r < rows; ++r) input[r] = inputs[r]; }
    for (int r = 0; r < rows; ++r) {
        const int key = first_key + depth[r];
        int path[17]; int path_count = 0;
        if (input_count > r) {
            for (int j = 0; j < depth[r] && j < input_count; ++j) path[path_count++] = input[j];
            path[path_count++] = input[r];
        }
        PacketRow o;
        packet_row(row_ptr(scores, dtype, r, row_stride), dtype, vocabulary, *cfg, key, path, path_count, o);
        out[r].serial = serial; out[r].token = o.idx[o.selected]; out[r].nonfinite = o.bad;
        if (detail) {
            or_packet_detail& d = detail[r];
            d.cap = o.cap; d.support = o.support; d.selected = o.selected; d.key = key; d.sum = o.sum;
            for (int j = 0; j < 20; ++j) {
                d.cand_val[j] = o.val[j]; d.cand_idx[j] = o.idx[j]; d.value[j] = o.value[j]; d.prob[j] = o.prob[j];
            }
        }
    }
    return VI_OK;
}

// exl3_sampled_score_kernel (sampled_select.cuh:300-360): row r chooses key
// first_key + r with no drafted path; gap in logit units by which next[r]
// trails the choice.  A next[r] outside [0, vocabulary) gets an infinite gap
// (the reference reads past the row there).
int or_sampled_scores(const void* scores, int dtype, int rows, int vocabulary, int64_t row_stride,
                      const vi_device_sampling* cfg, int first_key, float tolerance, const int64_t* next,
                      int64_t* chosen, float* gap) {
    if (rows < 0 || vocabulary <= 0 || row_stride < vocabulary || !cfg || !next || !chosen || !gap)
        return VI_ERR_INVALID;
    for (int r = 0; r < rows; ++r) {
        const void* row = row_ptr(scores, dtype, r, row_stride);
        const int key = first_key + r;
        PacketRow o;
        packet_row(row, dtype, vocabulary, *cfg, key, nullptr, 0, o);
        const int token = o.idx[o.selected];
        chosen[r] = token;
        const int64_t want = next[r];
        float g = 0.0f;
        if (want >= vocabulary && want != token) {
            g = kInf;
        } else if (want >= 0 && want != token && !(cfg->temperature > 0.0f)) {
            float own = element(row, dtype, int(want));
            if (cfg->presence_penalty != 0.0f && packet_seen(*cfg, key, nullptr, 0, int(want)))
                own -= cfg->presence_penalty;
            g = std::fmax(0.0f, o.val[o.selected] - own);
        } else if (want >= 0 && want != token) {
            g = kInf;
            const int cap = packet_cap(*cfg);
            int rank = -1;
            for (int j = 0; j < cap; ++j) if (o.idx[j] == want) { rank = j; break; }
            if (rank >= 0 && rank < o.support) {
                g = (o.value[o.selected] - o.value[rank]) * cfg->temperature;
            } else if (rank >= 0 && tolerance > 0.0f) {
                float value[20]; int index[20];
                const float boosted = o.val[rank] + tolerance;
                int at = 0;
                for (int j = 0; j < cap; ++j) {
                    if (j == rank) continue;
                    value[at] = o.val[j]; index[at] = o.idx[j]; ++at;
                }
                int pos = at;
                while (pos > 0 && boosted > value[pos - 1]) { value[pos] = value[pos - 1]; index[pos] = index[pos - 1]; --pos; }
                value[pos] = boosted; index[pos] = int(want);
                float prob[20];
                const int support = packet_support(value, cap, *cfg, prob, nullptr);
                if (pos < support) {
                    const float inv_temp = 1.0f / cfg->temperature;
                    float best = -kInf;
                    for (int j = 0; j < support; ++j)
                        if (j != pos) best = std::fmax(best, std::fmaf(value[j], inv_temp, or_gumbel(cfg->seed, key, index[j])));
                    const float own = std::fmaf(o.val[rank], inv_temp, or_gumbel(cfg->seed, key, int(want)));
                    g = std::fmax(0.0f, (best - own) * cfg->temperature);
                }
            }
        }
        gap[r] = g;
    }
    return VI_OK;
}

// dflash_sampled_choice with DraftSelectSampling (dflash2_draft.cu:2554-2610),
// applied to every position of every lane in position order; the inv_temperature
// <= 0 branch is the first maximum of the given scores (the reference's selector
// argmax).  As in the reference build, the two multiply-adds are fused.
int or_draft_choice(int lanes, int positions, int vocabulary, const float* scores, const int64_t* candidates,
                    const int64_t* seed_tokens, const vi_draft_sampling* sampling, int64_t* proposals) {
    if (lanes < 0 || positions < 0 || vocabulary <= 0 || !scores || !candidates || !sampling || !proposals)
        return VI_ERR_INVALID;
    constexpr int K = 16;
    for (int l = 0; l < lanes; ++l) {
        const vi_draft_sampling& s = sampling[l];
        const int64_t seed_token = seed_tokens ? seed_tokens[l] : -1;
        int64_t* out = proposals + size_t(l) * positions;
        for (int pos = 0; pos < positions; ++pos) {
            const size_t at = (size_t(l) * positions + pos) * K;
            const float* sc = scores + at;
            const int64_t* cd = candidates + at;
            int best = 0;
            if (!(s.inv_temperature > 0.0f)) {
                for (int c = 1; c < K; ++c) if (sc[c] > sc[best]) best = c;
            } else {
                const int key = s.key_base + pos;
                float v[K];
                int order[K];
                for (int c = 0; c < K; ++c) {
                    v[c] = sc[c];
                    order[c] = c;
                    if (s.presence_penalty == 0.0f) continue;
                    const int64_t token = cd[c];
                    bool seen = token == seed_token ||
                                (s.first_occurrence && token >= 0 && token < vocabulary && s.first_occurrence[token] < key);
                    for (int i = 0; i < pos && !seen; ++i) seen = out[i] == token;
                    if (seen) v[c] -= s.presence_penalty;
                }
                for (int i = 1; i < K; ++i) {
                    const int o = order[i];
                    int j = i;
                    while (j > 0 && v[o] > v[order[j - 1]]) { order[j] = order[j - 1]; --j; }
                    order[j] = o;
                }
                int cap = K;
                if (s.top_k > 0 && s.top_k < cap) cap = s.top_k;
                const float m = v[order[0]] * s.inv_temperature;
                float prob[K], sum = 0.0f;
                for (int j = 0; j < cap; ++j) { prob[j] = std::exp(std::fmaf(v[order[j]], s.inv_temperature, -m)); sum += prob[j]; }
                const float thresh = s.min_p > 0.0f ? s.min_p * prob[0] : -1.0f;
                float cum = 0.0f;
                int support = 0;
                for (int j = 0; j < cap; ++j) {
                    if (thresh >= 0.0f && prob[j] < thresh) break;
                    cum += prob[j]; support = j + 1;
                    if (s.top_p < 1.0f && cum >= s.top_p * sum) break;
                }
                if (support < 1) support = 1;
                best = order[0];
                float best_value = -kInf;
                for (int j = 0; j < support; ++j) {
                    const int c = order[j];
                    const float val = std::fmaf(v[c], s.inv_temperature, or_gumbel(s.seed, key, int32_t(cd[c])));
                    if (val > best_value) { best_value = val; best = c; }
                }
            }
            out[pos] = cd[best];
        }
    }
    return VI_OK;
}

// dflash_selector_fused_chain_kernel (src/exl3/dflash2_draft.cu:2615-2678):
// candidate c's selector value is reduced as 32 lanes of 8 products each
// (lane `sub` holds ranks sub + 32k), r[k] += r[k+4], r[k] += r[k+2],
// r[0] + r[1] per lane (:2640-2651), then a shuffle-down tree over offsets
// 16 .. 1 (:2652-2653); score = unary + value (:2655-2656); the first maximum
// is proposed and becomes the anchor (:2659-2673).  A sampled lane takes
// dflash_sampled_choice over the unary scores (:2661-2666), which is
// or_draft_choice with those scores and the initial anchor as seed token.
int or_selector_chain(int lanes, int positions, int vocabulary, const int64_t* anchors, const int64_t* candidates,
                      const float* unary, const uint16_t* hidden, const uint16_t* pred_codebook,
                      const uint16_t* succ_codebook, const vi_draft_sampling* sampling, int64_t* proposals) {
    if (lanes < 0 || positions < 0 || vocabulary <= 0 || !anchors || !candidates || !unary || !hidden ||
        !pred_codebook || !succ_codebook || !proposals)
        return VI_ERR_INVALID;
    constexpr int K = 16, R = 256;
    for (int l = 0; l < lanes; ++l) {
        int64_t* out = proposals + size_t(l) * positions;
        int64_t anchor = anchors[l];
        bool bad = anchor < 0 || anchor >= vocabulary;
        const bool sampled = sampling && sampling[l].inv_temperature > 0.0f;
        std::vector<int64_t> chain(size_t(positions), 0);
        if (sampled && !bad) {
            // the sampled proposals do not depend on the anchors; the chain ends at
            // the first position holding an invalid candidate
            or_draft_choice(1, positions, vocabulary, unary + size_t(l) * positions * K,
                            candidates + size_t(l) * positions * K, &anchors[l], &sampling[l], chain.data());
        }
        for (int pos = 0; pos < positions; ++pos) {
            const size_t at = size_t(l) * positions + pos;
            const int64_t* cd = candidates + at * K;
            for (int c = 0; c < K; ++c) bad = bad || cd[c] < 0 || cd[c] >= vocabulary;
            if (bad) { out[pos] = -1; continue; }
            if (sampled) { out[pos] = chain[size_t(pos)]; continue; }
            float score[K];
            for (int c = 0; c < K; ++c) {
                float lane_v[32];
                for (int sub = 0; sub < 32; ++sub) {
                    float r[8];
                    for (int k = 0; k < 8; ++k) {
                        const int rank = sub + 32 * k;
                        const float a = or_decode(VI_F16, pred_codebook[size_t(anchor) * R + rank]);
                        const float h = or_decode(VI_F16, hidden[at * R + rank]);
                        const float b = or_decode(VI_F16, succ_codebook[size_t(cd[c]) * R + rank]);
                        r[k] = a * h * b;
                    }
                    for (int k = 0; k < 4; ++k) r[k] += r[k + 4];
                    for (int k = 0; k < 2; ++k) r[k] += r[k + 2];
                    lane_v[sub] = r[0] + r[1];
                }
                for (int off = 16; off > 0; off >>= 1)
                    for (int sub = 0; sub < off; ++sub) lane_v[sub] += lane_v[sub + off];
                score[c] = unary[at * K + c] + lane_v[0];
            }
            int best = 0;
            for (int c = 1; c < K; ++c) if (score[c] > score[best]) best = c;
            out[pos] = cd[best];
            anchor = cd[best];
        }
    }
    return VI_OK;
}

// exact_row_score_kernel (text_model.cu:11393-11420): argmax over the values
// that compare greater than -Inf (NaN and -Inf never win, +Inf can), lowest
// index on ties, index = vocabulary when none; gap = max - logit(next) for a
// next in [0, vocabulary) other than the argmax, else 0.
int or_row_scores(const void* logits, int dtype, int rows, int vocabulary, int64_t row_stride,
                  const int64_t* next, int64_t* greedy, float* gap) {
    if (rows < 0 || vocabulary <= 0 || row_stride < vocabulary || !next || !greedy || !gap) return VI_ERR_INVALID;
    for (int r = 0; r < rows; ++r) {
        const void* row = row_ptr(logits, dtype, r, row_stride);
        float value = -kInf; int index = vocabulary;
        for (int i = 0; i < vocabulary; ++i) {
            const float v = element(row, dtype, i);
            if (v > value) { value = v; index = i; }
        }
        greedy[r] = index;
        const int64_t t = next[r];
        gap[r] = (t >= 0 && t < vocabulary && t != index) ? value - element(row, dtype, int(t)) : 0.0f;
    }
    return VI_OK;
}

int or_sample_rows(const void* logits, int dtype, int rows, int vocabulary, int64_t row_stride,
                   const vi_row_params* params, const int32_t* histories,
                   const int64_t* history_offsets, int32_t* tokens, double* uniforms,
                   float* probs, int64_t probs_stride, vi_sample_stats* stats,
                   double* margins, int threads) {
    if (rows < 0 || vocabulary <= 0 || row_stride < vocabulary || !params || !tokens) return VI_ERR_INVALID;
    if (probs && probs_stride < vocabulary) return VI_ERR_INVALID;
    parallel_rows(rows, threads, [&](int r) {
        thread_local std::vector<uint32_t> counts;
        const vi_row_params& p = params[r];
        const int32_t* h = nullptr; int64_t hn = 0;
        if (histories && history_offsets) { h = histories + history_offsets[r]; hn = history_offsets[r + 1] - history_offsets[r]; }
        RowDist d;
        build_row(row_ptr(logits, dtype, r, row_stride), dtype, vocabulary, p, h, hn, d, counts);
        double u = 0, margin = INFINITY; int pick = -1; int32_t token = vocabulary;
        if (!(d.flags & VI_FLAG_EMPTY)) {
            if (d.greedy) token = d.greedy_token;
            else {
                u = or_uniform(p.seed, p.lane, p.position, 0);
                pick = draw_sorted(d, u, &margin);
                token = d.ids[size_t(pick)];
            }
        }
        tokens[r] = token;
        if (uniforms) uniforms[r] = u;
        if (probs) {
            float* pr = probs + size_t(r) * size_t(probs_stride);
            std::fill(pr, pr + vocabulary, 0.0f);
            if (!(d.flags & VI_FLAG_EMPTY)) {
                if (d.greedy) pr[token] = 1.0f;
                else for (int j = 0; j < d.support; ++j) pr[d.ids[size_t(j)]] = float(d.w[size_t(j)] / d.s_n);
            }
        }
        if (stats) {
            stats[r].flags = d.flags; stats[r].support = uint32_t(d.support);
            stats[r].finite = uint32_t(d.n_valid); stats[r].reserved = 0;
            stats[r].support_mass = d.greedy ? 1.0 : d.s_n; stats[r].uniform = u;
        }
        if (margins) {
            margins[4 * r + 0] = margin; margins[4 * r + 1] = d.topp_margin;
            margins[4 * r + 2] = d.minp_margin; margins[4 * r + 3] = pick;
        }
    });
    return VI_OK;
}

int or_row_distribution(const void* row, int dtype, int vocabulary, const vi_row_params* params,
                        double* p_out, uint32_t* support) {
    std::vector<uint32_t> counts;
    RowDist d;
    build_row(row, dtype, vocabulary, *params, nullptr, 0, d, counts);
    std::fill(p_out, p_out + vocabulary, 0.0);
    if (d.flags & VI_FLAG_EMPTY) return VI_ERR_INVALID;
    if (d.greedy) { p_out[d.greedy_token] = 1.0; if (support) *support = 1; return VI_OK; }
    for (int j = 0; j < d.support; ++j) p_out[d.ids[size_t(j)]] = d.w[size_t(j)] / d.s_n;
    if (support) *support = uint32_t(d.support);
    return VI_OK;
}

// Exl3IndependentAcceptanceReference::evaluate (sampled_acceptance_reference.h:27-89).
int or_accept(const double* target_p, const double* draft_q, int64_t vocabulary,
              uint32_t proposed_token, double acceptance_draw, double correction_draw,
              or_accept_outcome* out, double* residual) {
    constexpr double tol = 1e-9;
    auto distribution_ok = [&](const double* v) {
        if (vocabulary <= 0) return false;
        double s = 0;
        for (int64_t i = 0; i < vocabulary; ++i) {
            if (!std::isfinite(v[i]) || v[i] < 0 || v[i] > 1) return false;
            s += v[i];
        }
        return std::isfinite(s) && std::abs(s - 1) <= tol;
    };
    auto uniform_ok = [](double u) { return std::isfinite(u) && u >= 0 && u < 1; };
    if (!distribution_ok(target_p) || !distribution_ok(draft_q) || !uniform_ok(acceptance_draw) ||
        !uniform_ok(correction_draw) || int64_t(proposed_token) >= vocabulary)
        return 1;
    const double q = draft_q[proposed_token];
    if (q == 0) return 1;
    *out = or_accept_outcome{};
    out->acceptance_probability = std::min(1.0, target_p[proposed_token] / q);
    if (acceptance_draw < out->acceptance_probability) {
        out->accepted = 1; out->token = proposed_token;
        return 0;
    }
    std::vector<double> res(static_cast<size_t>(vocabulary));
    double sum = 0;
    for (int64_t i = 0; i < vocabulary; ++i) { res[size_t(i)] = std::max(0.0, target_p[i] - draft_q[i]); sum += res[size_t(i)]; }
    if (!std::isfinite(sum) || sum <= tol) return 2;
    for (auto& v : res) v /= sum;
    out->correction_draw_used = 1;
    double cum = 0; uint32_t last_positive = 0; bool found = false;
    for (uint32_t t = 0; t < uint32_t(vocabulary); ++t) {
        if (res[t] > 0) last_positive = t;
        cum += res[t];
        if (correction_draw < cum) { out->token = t; found = true; break; }
    }
    if (!found) out->token = last_positive;
    if (residual) std::copy(res.begin(), res.end(), residual);
    return 0;
}

// decide_exl3_outer_prefix (exact_outer_reference.h:68-82).
int or_outer_prefix(const int64_t* target_path, const int64_t* tentative, int n,
                    const int64_t* terminal, int n_terminal, int64_t* committed,
                    int* n_committed, int* accepted, int* rejected, int* stopped) {
    if (n <= 0) return 1;
    int c = 0, acc = 0; bool rej = false, stop = false;
    for (int row = 0; row < n; ++row) {
        const int64_t authorized = target_path[row];
        committed[c++] = authorized;
        if (tentative[row] == authorized) ++acc; else rej = true;
        stop = std::find(terminal, terminal + n_terminal, authorized) != terminal + n_terminal;
        if (rej || stop) break;
    }
    *n_committed = c; *accepted = acc; *rejected = rej; *stopped = stop;
    return 0;
}

// EXTENSION: per-lane verification with the target / draft distributions of the
// batched sampler (no penalties).  Greedy mode = decide_exl3_outer_prefix over the
// target rows' greedy packets; sampled mode = the FP64 acceptance rule above with
// p, q the filtered distributions, the residual resampled in token-id order.
// exl3_build_verification_tree (verification_tree.h:44-112), restated in the
// reference's own loop shape: per depth the top-16 softmax in float, the chain
// token's hit rate by decile (:53-68), up to three sibling leaves in stable
// unary order skipping the chain token (:69-77); then every (rows, chain) pair
// in order, the leaf pool rebuilt and partially sorted each time (:81-97), and
// the first strict maximum of (1 + value) / (1 + row_cost * rows) kept (:99-109).
int or_build_verification_tree(const int64_t* drafts, int depth_in, const int64_t* candidate_ids,
                               const float* candidate_unary, int budget, int max_siblings, float row_cost,
                               int* chain_drafts, int64_t* sibling_tokens, int* sibling_offsets, int* n_siblings) {
    static const float kChainHit[10] = {0.32f, 0.38f, 0.35f, 0.44f, 0.42f, 0.49f, 0.57f, 0.67f, 0.78f, 0.97f};
    static const float kSiblingHit[3][10] = {
        {0.04f, 0.13f, 0.18f, 0.23f, 0.26f, 0.27f, 0.13f, 0.09f, 0.06f, 0.07f},
        {0.03f, 0.10f, 0.15f, 0.09f, 0.12f, 0.12f, 0.12f, 0.12f, 0.12f, 0.12f},
        {0.03f, 0.10f, 0.15f, 0.15f, 0.15f, 0.15f, 0.15f, 0.15f, 0.15f, 0.15f}};
    if (depth_in < 0 || budget < 0) return 1;
    const int depth = std::min(depth_in, budget);
    struct Leaf { float value; int offset; int64_t token; };
    auto decile = [](float pr) { int k = int(pr * 10.0f); return k < 0 ? 0 : (k > 9 ? 9 : k); };
    std::vector<float> chain_hit(static_cast<size_t>(depth));
    std::vector<Leaf> leaves(static_cast<size_t>(depth) * 3);
    for (int d = 0; d < depth; ++d) {
        const int64_t* ids = candidate_ids + size_t(d) * 16;
        const float* un = candidate_unary + size_t(d) * 16;
        float top = un[0];
        for (int c = 1; c < 16; ++c) if (un[c] > top) top = un[c];
        float p[16], sum = 0.0f;
        for (int c = 0; c < 16; ++c) { p[c] = std::exp(un[c] - top); sum += p[c]; }
        int order[16];
        for (int c = 0; c < 16; ++c) order[c] = c;
        std::stable_sort(order, order + 16, [&](int a, int b) { return un[a] > un[b]; });
        float chain_p = 0.0f;
        for (int c = 0; c < 16; ++c) if (ids[c] == drafts[d]) chain_p = p[c] / sum;
        chain_hit[size_t(d)] = kChainHit[decile(chain_p)];
        int rank = 0;
        for (int i = 0; i < 16 && rank < 3; ++i) {
            const int c = order[i];
            if (ids[c] == drafts[d]) continue;
            leaves[size_t(d) * 3 + size_t(rank)] = {kSiblingHit[rank][decile(p[c] / sum)], d + 1, ids[c]};
            ++rank;
        }
        for (; rank < 3; ++rank) leaves[size_t(d) * 3 + size_t(rank)] = {0.0f, d + 1, -1};
    }
    float best_rate = -1.0f;
    *chain_drafts = 0;
    *n_siblings = 0;
    for (int nodes = 1; nodes <= budget; ++nodes) {
        for (int chain = std::max(1, nodes - std::max(0, max_siblings)); chain <= std::min(depth, nodes); ++chain) {
            float survive = 1.0f, value = 0.0f;
            std::vector<Leaf> pool;
            for (int d = 0; d < chain; ++d) {
                for (int r = 0; r < 3; ++r) {
                    const Leaf& l = leaves[size_t(d) * 3 + size_t(r)];
                    if (l.token >= 0) pool.push_back({survive * l.value, l.offset, l.token});
                }
                survive *= chain_hit[size_t(d)];
                value += survive;
            }
            const int count = nodes - chain;
            if (count > int(pool.size())) continue;
            std::partial_sort(pool.begin(), pool.begin() + count, pool.end(),
                              [](const Leaf& a, const Leaf& b) { return a.value > b.value; });
            for (int i = 0; i < count; ++i) value += pool[size_t(i)].value;
            const float rate = (1.0f + value) / (1.0f + row_cost * float(nodes));
            if (rate > best_rate) {
                best_rate = rate;
                *chain_drafts = chain;
                *n_siblings = count;
                for (int i = 0; i < count; ++i) {
                    sibling_tokens[i] = pool[size_t(i)].token;
                    sibling_offsets[i] = pool[size_t(i)].offset;
                }
            }
        }
    }
    return 0;
}

int or_verify_rows(int mode, const void* target, int target_dtype, int64_t target_stride,
                   int target_rows, const void* draft, int draft_dtype, int64_t draft_stride,
                   int lanes, int drafts, int vocabulary, const int32_t* drafted,
                   const vi_row_params* params, const int64_t* terminal, int n_terminal,
                   int32_t* accepted, int32_t* committed, int32_t* committed_count,
                   uint32_t* lane_flags, double* accept_margins, int threads) {
    if (lanes < 0 || drafts <= 0 || vocabulary <= 0 || (target_rows != drafts && target_rows != drafts + 1))
        return VI_ERR_INVALID;
    auto is_terminal = [&](int64_t t) {
        return terminal && std::find(terminal, terminal + n_terminal, t) != terminal + n_terminal;
    };
    parallel_rows(lanes, threads, [&](int l) {
        int32_t* out = committed + size_t(l) * (drafts + 1);
        std::fill(out, out + drafts + 1, -1);
        uint32_t flags = 0; int c = 0, acc = 0;
        if (accept_margins) for (int j = 0; j < drafts; ++j) accept_margins[size_t(l) * drafts + j] = INFINITY;
        auto target_row = [&](int j) { return row_ptr(target, target_dtype, int64_t(l) * target_rows + j, target_stride); };
        if (mode == VI_VERIFY_GREEDY) {
            std::vector<int64_t> path(static_cast<size_t>(target_rows)), tent(static_cast<size_t>(drafts));
            for (int j = 0; j < target_rows; ++j) {
                vi_greedy_row g;
                or_greedy_rows(target_row(j), target_dtype, 1, vocabulary, vocabulary, 0, &g);
                if (g.nonfinite) flags |= VI_FLAG_NONFINITE;
                path[size_t(j)] = g.token;
            }
            for (int j = 0; j < drafts; ++j) tent[size_t(j)] = drafted[size_t(l) * drafts + j];
            std::vector<int64_t> com(static_cast<size_t>(drafts));
            int nc = 0, a = 0, rej = 0, stop = 0;
            or_outer_prefix(path.data(), tent.data(), drafts, terminal, n_terminal, com.data(), &nc, &a, &rej, &stop);
            for (int j = 0; j < nc; ++j) out[c++] = int32_t(com[size_t(j)]);
            acc = a;
            if (!rej && !stop && target_rows == drafts + 1) out[c++] = int32_t(path[size_t(drafts)]);
        } else {
            const vi_row_params& p = params[l];
            std::vector<uint32_t> counts;
            std::vector<double> pd(static_cast<size_t>(vocabulary)), qd(static_cast<size_t>(vocabulary));
            bool stopped = false;
            int j = 0;
            for (; j < drafts && !stopped; ++j) {
                RowDist tp, dq;
                build_row(target_row(j), target_dtype, vocabulary, p, nullptr, 0, tp, counts);
                build_row(row_ptr(draft, draft_dtype, int64_t(l) * drafts + j, draft_stride), draft_dtype,
                          vocabulary, p, nullptr, 0, dq, counts);
                flags |= (tp.flags | dq.flags) & (VI_FLAG_NONFINITE | VI_FLAG_EMPTY);
                std::fill(pd.begin(), pd.end(), 0.0); std::fill(qd.begin(), qd.end(), 0.0);
                if (tp.greedy) pd[size_t(tp.greedy_token)] = 1.0;
                else for (int i = 0; i < tp.support; ++i) pd[size_t(tp.ids[size_t(i)])] = tp.w[size_t(i)] / tp.s_n;
                if (dq.greedy) qd[size_t(dq.greedy_token)] = 1.0;
                else for (int i = 0; i < dq.support; ++i) qd[size_t(dq.ids[size_t(i)])] = dq.w[size_t(i)] / dq.s_n;
                const int32_t d = drafted[size_t(l) * drafts + j];
                const int pos = p.position + j;
                const double ua = or_uniform(p.seed, p.lane, pos, 1), uc = or_uniform(p.seed, p.lane, pos, 2);
                const double q = (d >= 0 && d < vocabulary) ? qd[size_t(d)] : 0.0;
                double a = 0;
                if (q == 0) flags |= VI_FLAG_ZERO_Q;
                else a = std::min(1.0, pd[size_t(d)] / q);
                // how close this position's decision came to turning: the accept
                // test, and the top-p / min-p cuts of both rows (which decide p, q)
                double margin = std::fabs(ua - a);
                margin = std::min({margin, tp.topp_margin, tp.minp_margin, dq.topp_margin, dq.minp_margin});
                if (accept_margins) accept_margins[size_t(l) * drafts + j] = margin;
                if (q != 0 && ua < a) {
                    out[c++] = d; ++acc;
                    stopped = is_terminal(d);
                    continue;
                }
                double sum = 0;
                for (int v = 0; v < vocabulary; ++v) sum += std::max(0.0, pd[size_t(v)] - qd[size_t(v)]);
                int32_t corr = 0;
                if (!std::isfinite(sum) || sum <= 1e-9) {
                    flags |= VI_FLAG_NO_RESIDUAL;
                    double cum = 0; int32_t last = 0; bool found = false;
                    for (int v = 0; v < vocabulary; ++v) {
                        if (pd[size_t(v)] > 0) last = v;
                        cum += pd[size_t(v)];
                        if (uc < cum) { corr = v; found = true; break; }
                    }
                    if (!found) corr = last;
                } else {
                    double cum = 0, before = 0; int32_t last = 0; bool found = false;
                    for (int v = 0; v < vocabulary; ++v) {
                        const double rv = std::max(0.0, pd[size_t(v)] - qd[size_t(v)]) / sum;
                        if (rv > 0) last = v;
                        before = cum;
                        cum += rv;
                        if (uc < cum) { corr = v; found = true; break; }
                    }
                    if (!found) corr = last;
                    // ... and of the correction: u_c against the cumulative residual
                    if (accept_margins) {
                        double& m = accept_margins[size_t(l) * drafts + j];
                        m = std::min({m, std::fabs(cum - uc), std::fabs(before - uc)});
                    }
                }
                out[c++] = corr;
                break;
            }
            if (acc == drafts && !stopped && target_rows == drafts + 1) {
                RowDist tp;
                build_row(target_row(drafts), target_dtype, vocabulary, p, nullptr, 0, tp, counts);
                if (!(tp.flags & VI_FLAG_EMPTY)) {
                    if (tp.greedy) {
                        out[c++] = tp.greedy_token;
                    } else {
                        double dm = INFINITY;
                        out[c++] = tp.ids[size_t(draw_sorted(tp, or_uniform(p.seed, p.lane, p.position + drafts, 0), &dm))];
                        if (accept_margins) {   // (the bonus draw's margins join the last position's)
                            double& m = accept_margins[size_t(l) * drafts + drafts - 1];
                            m = std::min({m, dm, tp.topp_margin, tp.minp_margin});
                        }
                    }
                }
            }
        }
        accepted[l] = acc;
        committed_count[l] = c;
        if (lane_flags) lane_flags[l] = flags;
    });
    return VI_OK;
}

}  // extern "C"
