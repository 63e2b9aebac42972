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

// Filtered distribution of one sorted list (in LDS): the lane's weights, the
// support after the cap / min-p / top-p cuts and its mass.
struct ListDist {
    double w[kMaxK];
    int id[kMaxK];
    int support;
    double sn;
};

// One wave per list: lane k computes the weight of list entry k; lane 0 then
// takes the cuts and sums sequentially, in the order of the one-thread rule
// (the fp64 results are that rule's, bit for bit).
__device__ inline void list_dist(const vi_row_params& p, const float* z, const int* id, uint32_t valid, ListDist& d) {
    const int k = lane_id();
    const bool greedy = !(p.temperature > 0.0f);
    // (callers refuse lanes with top_k outside [1, kMaxK]; the clamp keeps every
    // index inside the 64-entry lists regardless)
    const int cap = valid == 0 ? 0 : (greedy ? 1 : min(min(max(p.top_k, 0), kMaxK), int(valid)));
    if (k < cap) {
        d.id[k] = id[k];
        d.w[k] = greedy ? 1.0 : exp(double(z[k]) - double(z[0]));
    }
    wave_sync();
    if (k == 0) {
        int n = 0;
        double sn = 0.0;
        if (cap > 0 && greedy) {
            n = 1;
            sn = 1.0;
        } else if (cap > 0) {
            double s = 0.0;
            for (int j = 0; j < cap; ++j) s += d.w[j];
            const double minp = double(p.min_p), target = double(p.top_p) * s;
            double cum = 0.0;
            for (int j = 0; j < cap; ++j) {
                if (p.min_p > 0.0f && d.w[j] < minp * d.w[0]) break;
                cum += d.w[j];
                n = j + 1;
                if (p.top_p < 1.0f && cum >= target) break;
            }
            if (n < 1) n = 1;
            for (int j = 0; j < n; ++j) sn += d.w[j];
        }
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
    __shared__ double s_rv[kMaxK], s_pv[kMaxK];
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
        list_dist(p, tv, ti, tvalid, P);
        if (k == 0) {
            int32_t tok = -1;
            if (tvalid) {
                if (!(p.temperature > 0.0f)) tok = P.id[0];
                else {
                    const double t = philox_uniform(p.seed, p.lane, p.position + drafts, 0u) * P.sn;
                    double cum = 0.0;
                    int pick = P.support - 1;
                    for (int i = 0; i < P.support; ++i) { cum += P.w[i]; if (cum > t) { pick = i; break; } }
                    tok = P.id[pick];
                }
            }
            put_dec(out, PosDecision{tok, 0u, 0, 0});
        }
        return;
    }
    const size_t dr = size_t(l) * drafts + j;
    list_dist(p, tv, ti, tvalid, P);
    list_dist(p, dv, di, dvalid, Q);
    const int32_t d = drafted[dr];
    const int iq = (d >= 0 && d < vocabulary) ? list_find(Q, d) : -1;
    const int ip = list_find(P, d);
    uint32_t flags = 0;   // (lane 0's)
    if (k == 0) {
        flags = tflags | dflags;
        if (tvalid == 0 || dvalid == 0) flags |= VI_FLAG_EMPTY;
        const double ua = philox_uniform(p.seed, p.lane, p.position + j, 1u);
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
    // (ids within a list are distinct)
    if (k < P.support) {
        const int t = P.id[k];
        int rank = 0;
        for (int i = 0; i < P.support; ++i) rank += P.id[i] < t ? 1 : 0;
        double qt = 0.0;
        for (int i = 0; i < Q.support; ++i)
            if (Q.id[i] == t) { qt = Q.w[i] / Q.sn; break; }
        const double pk = P.w[k] / P.sn;
        s_rid[rank] = t;
        s_pv[rank] = pk;
        s_rv[rank] = fmax(0.0, pk - qt);
    }
    wave_sync();
    if (k == 0) {
        const int m = P.support;
        const double uc = philox_uniform(p.seed, p.lane, p.position + j, 2u);
        double sum = 0.0;
        for (int i = 0; i < m; ++i) sum += s_rv[i];
        int32_t corr = 0;
        if (!(sum > 1e-9) || !isfinite(sum)) {
            // No residual mass: correct from p itself (inverse CDF, id order).
            flags |= VI_FLAG_NO_RESIDUAL;
            double cum = 0.0;
            int32_t last = 0;
            bool found = false;
            for (int i = 0; i < m; ++i) {
                const double pv = s_pv[i];
                if (pv > 0.0) last = s_rid[i];
                cum += pv;
                if (uc < cum) { corr = s_rid[i]; found = true; break; }
            }
            if (!found) corr = last;
        } else {
            double cum = 0.0;
            int32_t last = 0;
            bool found = false;
            for (int i = 0; i < m; ++i) {
                const double r = s_rv[i] / sum;
                if (r > 0.0) last = s_rid[i];
                cum += r;
                if (uc < cum) { corr = s_rid[i]; found = true; break; }
            }
            if (!found) corr = last;
        }
        put_dec(out, PosDecision{corr, flags, 0, 0});
    }
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

}  // namespace vi
