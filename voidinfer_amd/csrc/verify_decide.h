// verify_decide.h — the per-position decision and per-lane accept chain of
// sampled verification over top-k lists (one wave each), shared by the
// position kernel (verify.hip) and the draft-row list scan that takes the
// decisions as its rows finish (topk.hip).
#pragma once
#include "vi_device.h"
#include "vi_internal.h"

namespace vi {

constexpr int kMaxK = 64;   // the longest list (top_k <= 64)

// Wave-level barrier for the one-wave steps below (LDS written by one lane and
// read by another).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
}

__device__ inline bool is_terminal(const int64_t* terminal, int n, int64_t t) {
    for (int i = 0; i < n; ++i) if (terminal[i] == t) return true;
    return false;
}

// Filtered distribution of one sorted list: entry k's weight and id (in LDS,
// and held by lane k as w, id), the support after the cap / min-p / top-p cuts
// and its mass.
struct ListDist {
    double w[kMaxK];
    double cum[kMaxK];   // running sums of w in entry order (entries below the cap)
    int id[kMaxK];
    int support;
    double sn;
};

// Lane j's value, on every lane (j wave-uniform).
__device__ __forceinline__ double readlane_d(double v, int j) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(b)), j));
    const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(b >> 32)), j));
    return __builtin_bit_cast(double, (uint64_t(hi) << 32) | lo);
}

// One wave per list: lane k computes the weight of list entry k; lane 0 takes
// the running sums in entry order (the one order-dependent chain: every sum of
// the one-thread rule is one of them), and the cuts are the first entries
// whose tests hold, found by ballots (the fp64 results are that rule's, bit for
// bit).  Returns lane k's weight (0 past the cap) in w.
__device__ inline void list_dist(const vi_row_params& p, const float* z, const int* id, uint32_t valid, ListDist& d,
                                 double& w) {
    const int k = lane_id();
    const bool greedy = !(p.temperature > 0.0f);
    // (callers refuse lanes with top_k outside [1, kMaxK]; the clamp keeps every
    // index inside the 64-entry lists regardless)
    const int cap = valid == 0 ? 0 : (greedy ? 1 : min(min(max(p.top_k, 0), kMaxK), int(valid)));
    w = 0.0;
    if (k < cap) {
        w = greedy ? 1.0 : exp(double(z[k]) - double(z[0]));
        d.id[k] = id[k];
        d.w[k] = w;
    }
    int n = 0;
    double sn = 0.0;
    if (cap > 0 && greedy) {
        n = 1;
        sn = 1.0;
        if (k == 0) d.cum[0] = 1.0;
    } else if (cap > 0) {
        wave_sync();
        if (k == 0) {
            double c = 0.0;
            for (int j = 0; j < cap; ++j) { c += d.w[j]; d.cum[j] = c; }
        }
        wave_sync();
        const double s = d.cum[cap - 1], w0 = d.w[0];
        const double minp = double(p.min_p), target = double(p.top_p) * s;
        const bool in = k < cap;
        const double ck = in ? d.cum[k] : 0.0;
        // the rule stops at the first entry under min_p (support j) or the
        // first whose running sum reaches top_p's (support j + 1)
        const uint64_t fm = ballot(in && p.min_p > 0.0f && w < minp * w0);
        const uint64_t hm = ballot(in && p.top_p < 1.0f && ck >= target);
        const int jf = fm ? __builtin_ctzll(fm) : cap, jh = hm ? __builtin_ctzll(hm) : cap;
        n = jf <= jh ? jf : jh + 1;
        // the support's mass: the running sum through its last entry, unless
        // no entry was taken
        if (n < 1) {
            n = 1;
            sn = w0;
        } else {
            sn = d.cum[n - 1];
        }
    }
    if (k == 0) {
        d.support = n;
        d.sn = sn;
    }
    wave_sync();
}

// Index of `token` in the support (first match), or -1: a ballot over the lanes.
__device__ __forceinline__ int list_find(const ListDist& d, int64_t token) {
    const int k = lane_id();
    const uint64_t m = ballot(k < d.support && int64_t(d.id[k]) == token);
    return m ? __builtin_ctzll(m) : -1;
}

constexpr int kFinalizeThreads = kMaxK;   // one wave: lane k <-> list entry k

// The decision at one drafted position, which depends on that position's rows
// and Philox draws only: accept (u_a < min(1, p(d)/q(d)), q(d) > 0) or the
// correction token drawn from the residual; position `drafts` of a lane with a
// bonus row holds the bonus draw.  Flags are the position's own.
struct PosDecision {
    int32_t token;    // correction / bonus token (-1: none)
    uint32_t flags;
    int32_t accept;
    int32_t pad;
};

// A position's decision, stored with agent-scope stores (another workgroup of
// the launch may read it: the lane's chain runs in its last position).
__device__ __forceinline__ void put_dec(PosDecision* o, PosDecision v) {
    put_agent(&o->token, v.token);
    put_agent(&o->flags, v.flags);
    put_agent(&o->accept, v.accept);
}

// The decision of position j of lane l, by one wave, from the position's
// target list (tv, ti: entries in (value desc, id asc) order, tvalid finite
// logits, tflags) and draft list (dv, di, dvalid, dflags; unused for the bonus
// position j == drafts).
__device__ inline void position_decision(const vi_row_params& p, int j, int l, int drafts, int target_rows,
                                         const float* tv, const int* ti, uint32_t tvalid, uint32_t tflags,
                                         const float* dv, const int* di, uint32_t dvalid, uint32_t dflags,
                                         const int32_t* drafted, int vocabulary, int full_ok, PosDecision* dec) {
    __shared__ ListDist P, Q;
    __shared__ double s_rv[kMaxK], s_pv[kMaxK], s_rs[kMaxK], s_rc[kMaxK];
    __shared__ double s_sum;
    __shared__ int s_rid[kMaxK];
    __shared__ int s_accept;
    const int k = lane_id();
    PosDecision* out = dec + size_t(l) * (drafts + 1) + j;
    if (verify_list_refused(p)) {   // no list of this lane's top_k: the full-vocabulary path, or refused
        if (!full_ok && k == 0 && (j < drafts || target_rows == drafts + 1)) put_dec(out, PosDecision{-1, VI_FLAG_ERROR, 0, 0});
        return;
    }
    if (j == drafts) {   // the bonus row's draw (used when every draft is accepted)
        if (target_rows != drafts + 1) return;
        double pw;
        list_dist(p, tv, ti, tvalid, P, pw);
        int32_t tok = -1;
        if (tvalid) {
            if (!(p.temperature > 0.0f)) tok = P.id[0];
            else {
                // the first support entry whose running sum passes u * s_n
                const double t = philox_uniform(p.seed, p.lane, p.position + drafts, 0u) * P.sn;
                const uint64_t pm = ballot(k < P.support && P.cum[min(k, kMaxK - 1)] > t);
                tok = P.id[pm ? __builtin_ctzll(pm) : P.support - 1];
            }
        }
        if (k == 0) put_dec(out, PosDecision{tok, 0u, 0, 0});
        return;
    }
    const size_t dr = size_t(l) * drafts + j;
    const int32_t d = drafted[dr];   // (issued first: its latency and the draws' work overlap the lists')
    const double ua = philox_uniform(p.seed, p.lane, p.position + j, 1u);
    const double uc = philox_uniform(p.seed, p.lane, p.position + j, 2u);
    double pw, qw;
    list_dist(p, tv, ti, tvalid, P, pw);
    list_dist(p, dv, di, dvalid, Q, qw);
    const int iq = (d >= 0 && d < vocabulary) ? list_find(Q, d) : -1;
    const int ip = list_find(P, d);
    uint32_t flags = 0;   // (lane 0's)
    if (k == 0) {
        flags = tflags | dflags;
        if (tvalid == 0 || dvalid == 0) flags |= VI_FLAG_EMPTY;
        const double q = iq >= 0 ? Q.w[iq] / Q.sn : 0.0;
        double acc_p = 0.0;
        if (q == 0.0) flags |= VI_FLAG_ZERO_Q;
        else acc_p = fmin(1.0, (ip >= 0 ? P.w[ip] / P.sn : 0.0) / q);
        s_accept = (q != 0.0 && ua < acc_p) ? 1 : 0;
        if (s_accept) put_dec(out, PosDecision{-1, flags, 1, 0});
    }
    wave_sync();
    if (s_accept) return;
    // residual max(0, p - q) over p's support, placed in token-id order by rank
    // (ids within a list are distinct); the lists' ids read back from LDS by
    // every lane (broadcast reads)
    const int m = P.support, qs = Q.support;
    const int pid = k < m ? P.id[k] : 0;
    int rank = 0;
#pragma unroll 8
    for (int i = 0; i < m; ++i) rank += P.id[i] < pid ? 1 : 0;
    int at = -1;   // (the first match: ids within a list are distinct)
#pragma unroll 8
    for (int i = qs - 1; i >= 0; --i) at = Q.id[i] == pid ? i : at;
    const double qt = at >= 0 ? Q.w[at] / Q.sn : 0.0;
    if (k < m) {
        const double pk = pw / P.sn;
        s_rid[rank] = pid;
        s_pv[rank] = pk;
        s_rv[rank] = fmax(0.0, pk - qt);
    }
    wave_sync();
    flags = uint32_t(__builtin_amdgcn_readfirstlane(int(flags)));
    if (k == 0) {
        double c = 0.0;
        for (int i = 0; i < m; ++i) c += s_rv[i];
        s_sum = c;
    }
    wave_sync();
    const double sum = s_sum;
    // The inverse CDF in id order: the first entry whose running sum exceeds
    // u_c, else the last entry with a positive share (0 if none).  The shares
    // are each lane's value over the sum (divided in parallel) or, with no
    // residual mass, p itself; their running sums are lane 0's chain.
    const bool nores = !(sum > 1e-9) || !isfinite(sum);
    if (nores) flags |= VI_FLAG_NO_RESIDUAL;
    const double share = k < m ? (nores ? s_pv[k] : s_rv[k] / sum) : 0.0;
    if (k < m) s_rs[k] = share;
    wave_sync();
    if (k == 0) {
        double c = 0.0;
        for (int i = 0; i < m; ++i) { c += s_rs[i]; s_rc[i] = c; }
    }
    wave_sync();
    const uint64_t fm = ballot(k < m && uc < s_rc[min(k, kMaxK - 1)]);
    const uint64_t pm = ballot(k < m && share > 0.0);
    const int32_t corr = fm ? s_rid[__builtin_ctzll(fm)] : pm ? s_rid[63 - __builtin_clzll(pm)] : 0;
    if (k == 0) put_dec(out, PosDecision{corr, flags, 0, 0});
}

// The accept chain of lane l over its position decisions (load(j)), in order:
// accepted drafts are committed until the first rejection (its correction is
// committed and ends the chain) or a terminal token; a lane that accepted
// every draft commits the bonus draw.  Flags of the positions visited (and the
// bonus row).
template <class Load>
__device__ __forceinline__ void lane_chain(int l, Load load, int drafts, int target_rows, const int32_t* drafted,
                                           const vi_row_params* params, const int64_t* terminal, int n_terminal,
                                           int full_ok, int32_t* accepted, int32_t* committed,
                                           int32_t* committed_count, uint32_t* lane_flags) {
    int32_t* out = committed + size_t(l) * (drafts + 1);
    for (int j = 0; j <= drafts; ++j) out[j] = -1;
    if (verify_list_refused(params[l]) && !full_ok) {   // refused lane: nothing accepted, nothing committed
        accepted[l] = 0;
        committed_count[l] = 0;
        if (lane_flags) lane_flags[l] = VI_FLAG_ERROR;
        return;
    }
    uint32_t flags = 0;
    int c = 0, acc = 0;
    bool stopped = false, rejected = false;
    for (int j = 0; j < drafts; ++j) {
        const PosDecision e = load(j);
        flags |= e.flags;
        if (e.accept) {
            const int32_t d = drafted[size_t(l) * drafts + j];
            out[c++] = d;
            ++acc;
            stopped = is_terminal(terminal, n_terminal, d);
            if (stopped) break;
            continue;
        }
        out[c++] = e.token;
        rejected = true;
        break;
    }
    if (!rejected && !stopped && acc == drafts && target_rows == drafts + 1) {
        const PosDecision b = load(drafts);
        flags |= b.flags;
        if (b.token >= 0) out[c++] = b.token;
    }
    accepted[l] = acc;
    committed_count[l] = c;
    if (lane_flags) lane_flags[l] = flags;
}

// The same chain walked by one wave: 64 positions' decisions and drafted tokens
// read at once (load(j) with a different j on every lane), the first position
// that stops the chain (a rejection, or an accepted terminal token) found by a
// ballot, the visited positions' flags OR-reduced; the committed entries are
// written by the lanes that hold them.
template <class Load>
__device__ inline void lane_chain_wave(int l, Load load, int drafts, int target_rows, const int32_t* drafted,
                                       const vi_row_params* params, const int64_t* terminal, int n_terminal,
                                       int full_ok, int32_t* accepted, int32_t* committed,
                                       int32_t* committed_count, uint32_t* lane_flags) {
    const int k = lane_id();
    int32_t* out = committed + size_t(l) * (drafts + 1);
    const int32_t* dl = drafted + size_t(l) * drafts;
    if (verify_list_refused(params[l]) && !full_ok) {   // refused lane: nothing accepted, nothing committed
        for (int j = k; j <= drafts; j += kMaxK) out[j] = -1;
        if (k == 0) {
            accepted[l] = 0;
            committed_count[l] = 0;
            if (lane_flags) lane_flags[l] = VI_FLAG_ERROR;
        }
        return;
    }
    uint32_t flags = 0;   // (wave-uniform)
    int c = -1, acc = 0;  // (wave-uniform; c < 0: no stop yet)
    for (int c0 = 0; c0 < drafts && c < 0; c0 += kMaxK) {
        const int j = c0 + k;
        const bool in = j < drafts;
        const PosDecision e = in ? load(j) : PosDecision{-1, 0u, 0, 0};
        const int32_t d = in ? dl[j] : -1;
        const bool st = in && (!e.accept || is_terminal(terminal, n_terminal, d));
        const uint64_t m = ballot(st);
        const int s = m ? __builtin_ctzll(m) : kMaxK;
        uint32_t f = (in && k <= s) ? e.flags : 0u;
#pragma unroll
        for (int o = 32; o; o >>= 1) f |= uint32_t(__shfl_xor(int(f), o, kMaxK));
        flags |= f;
        if (in && k < s) out[j] = d;                     // accepted, the chain goes on
        if (m) {
            const bool sa = __builtin_amdgcn_readlane(e.accept, s) != 0;
            if (k == s) out[j] = e.accept ? d : e.token;   // an accepted terminal token, or the correction
            c = c0 + s + 1;
            acc = c0 + s + (sa ? 1 : 0);
        }
    }
    if (c < 0) {   // every draft accepted: the bonus draw, if the lane has a bonus row
        c = drafts;
        acc = drafts;
        if (target_rows == drafts + 1) {
            const PosDecision b = load(drafts);
            flags |= b.flags;
            if (b.token >= 0) {
                if (k == 0) out[drafts] = b.token;
                c = drafts + 1;
            }
        }
    }
    for (int j = c + k; j <= drafts; j += kMaxK) out[j] = -1;
    if (k == 0) {
        accepted[l] = acc;
        committed_count[l] = c;
        if (lane_flags) lane_flags[l] = flags;
    }
}

}  // namespace vi
