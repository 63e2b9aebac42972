// verify.hip — DFlash2 draft verification on the device.
//
// Greedy mode: the target rows' greedy packets (greedy.hip) feed
// decide_exl3_outer_prefix (src/exl3/exact_outer_reference.h:68-82) per lane:
// the committed tokens are the target path through the first mismatch or
// terminal token, `accepted` counts the matches; with a bonus row (target_rows
// = drafts + 1) a fully accepted lane also commits the bonus row's argmax.
//
// Sampled mode: the target and draft rows are filtered with the lane's
// temperature / top-k / top-p / min-p (top-k lists from topk.hip, so
// 1 <= top_k <= 64), giving p and q.  Per position, in order, the rule of
// Exl3IndependentAcceptanceReference::evaluate
// (src/exl3/sampled_acceptance_reference.h:48-88): accept iff
// u_a < min(1, p[d]/q[d]); at the first rejection draw the correction from the
// residual max(0, p - q) normalised, inverse CDF in token-id order with u_c
// (last positive id on round-off).  u_a, u_c are Philox draws keyed by
// (seed, lane, position + j, purpose 1 / 2).  Every (lane, position) decision
// is taken at once, one wave each over the <= 64-entry lists (fp64): entry-wise
// work on the lanes, the order-dependent sums on lane 0; a per-lane pass then
// walks the accept chain in order.
#include <math.h>

#include "vi_device.h"
#include "vi_internal.h"

namespace vi {
namespace {

constexpr int kMaxK = 64;

__device__ bool is_terminal(const int64_t* terminal, int n, int64_t t) {
    for (int i = 0; i < n; ++i) if (terminal[i] == t) return true;
    return false;
}

__global__ void verify_greedy_kernel(const vi_greedy_row* rows, int lanes, int drafts, int target_rows,
                                     const int32_t* drafted, const int64_t* terminal, int n_terminal,
                                     int32_t* accepted, int32_t* committed, int32_t* committed_count,
                                     uint32_t* lane_flags) {
    const int l = blockIdx.x * blockDim.x + threadIdx.x;
    if (l >= lanes) return;
    const vi_greedy_row* g = rows + size_t(l) * target_rows;
    int32_t* out = committed + size_t(l) * (drafts + 1);
    for (int j = 0; j <= drafts; ++j) out[j] = -1;
    uint32_t flags = 0;
    for (int j = 0; j < target_rows; ++j) if (g[j].nonfinite) flags |= VI_FLAG_NONFINITE;
    int c = 0, acc = 0;
    bool rejected = false, stopped = false;
    for (int j = 0; j < drafts; ++j) {
        const int32_t authorized = g[j].token;
        out[c++] = authorized;
        if (drafted[size_t(l) * drafts + j] == authorized) ++acc; else rejected = true;
        stopped = is_terminal(terminal, n_terminal, authorized);
        if (rejected || stopped) break;
    }
    if (!rejected && !stopped && target_rows == drafts + 1) out[c++] = g[drafts].token;
    accepted[l] = acc;
    committed_count[l] = c;
    if (lane_flags) lane_flags[l] = flags;
}

// Filtered distribution of one sorted list (in LDS): the lane's weights, the
// support after the cap / min-p / top-p cuts and its mass.
struct ListDist {
    double w[kMaxK];
    int id[kMaxK];
    int support;
    double sn;
};

// One 64-lane workgroup per batch lane: lane k computes the weight of list
// entry k; lane 0 then takes the cuts and sums sequentially, in the order of
// the one-thread rule (the fp64 results are that rule's, bit for bit).
__device__ void list_dist(const vi_row_params& p, const float* z, const int* id, uint32_t valid, ListDist& d) {
    const int k = threadIdx.x;
    const bool greedy = !(p.temperature > 0.0f);
    // (callers refuse lanes with top_k outside [1, kMaxK]; the clamp keeps every
    // index inside the 64-entry lists regardless)
    const int cap = valid == 0 ? 0 : (greedy ? 1 : min(min(max(p.top_k, 0), kMaxK), int(valid)));
    if (k < cap) {
        d.id[k] = id[k];
        d.w[k] = greedy ? 1.0 : exp(double(z[k]) - double(z[0]));
    }
    __syncthreads();
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
    __syncthreads();
}

// Index of `token` in the support (first match), or -1: a ballot over the lanes.
__device__ __forceinline__ int list_find(const ListDist& d, int64_t token) {
    const int k = threadIdx.x;
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

// One wave per (position, lane): every position of every lane at once; the
// accept chain is resolved afterwards by verify_chain_kernel.
__global__ __launch_bounds__(kFinalizeThreads) void verify_position_kernel(
    const float* tval, const int* tidx, const uint32_t* tvalid, const uint32_t* tflags, const float* dval,
    const int* didx, const uint32_t* dvalid, const uint32_t* dflags, int drafts, int target_rows,
    const int32_t* drafted, const vi_row_params* params, int vocabulary, PosDecision* dec) {
    __shared__ ListDist P, Q;
    __shared__ double s_rv[kMaxK], s_pv[kMaxK];
    __shared__ int s_rid[kMaxK];
    __shared__ int s_accept;
    const int j = blockIdx.x, l = blockIdx.y, k = threadIdx.x;
    const vi_row_params p = params[l];
    PosDecision* out = dec + size_t(l) * (drafts + 1) + j;
    const size_t tr = size_t(l) * target_rows + j;
    if (verify_list_refused(p)) {   // no list of this lane's top_k: refused, nothing decided
        if (k == 0 && (j < drafts || target_rows == drafts + 1)) *out = PosDecision{-1, VI_FLAG_ERROR, 0, 0};
        return;
    }
    if (j == drafts) {   // the bonus row's draw (used when every draft is accepted)
        if (target_rows != drafts + 1) return;
        list_dist(p, tval + tr * kMaxK, tidx + tr * kMaxK, tvalid[tr], P);
        if (k == 0) {
            int32_t tok = -1;
            if (tvalid[tr]) {
                if (!(p.temperature > 0.0f)) tok = P.id[0];
                else {
                    const double t = philox_uniform(p.seed, p.lane, p.position + drafts, 0u) * P.sn;
                    double cum = 0.0;
                    int pick = P.support - 1;
                    for (int i = 0; i < P.support; ++i) { cum += P.w[i]; if (cum > t) { pick = i; break; } }
                    tok = P.id[pick];
                }
            }
            *out = PosDecision{tok, tflags[tr], 0, 0};
        }
        return;
    }
    const size_t dr = size_t(l) * drafts + j;
    list_dist(p, tval + tr * kMaxK, tidx + tr * kMaxK, tvalid[tr], P);
    list_dist(p, dval + dr * kMaxK, didx + dr * kMaxK, dvalid[dr], Q);
    const int32_t d = drafted[dr];
    const int iq = (d >= 0 && d < vocabulary) ? list_find(Q, d) : -1;
    const int ip = list_find(P, d);
    uint32_t flags = 0;   // (lane 0's)
    if (k == 0) {
        flags = tflags[tr] | dflags[dr];
        if (tvalid[tr] == 0 || dvalid[dr] == 0) flags |= VI_FLAG_EMPTY;
        const double ua = philox_uniform(p.seed, p.lane, p.position + j, 1u);
        const double q = iq >= 0 ? Q.w[iq] / Q.sn : 0.0;
        double acc_p = 0.0;
        if (q == 0.0) flags |= VI_FLAG_ZERO_Q;
        else acc_p = fmin(1.0, (ip >= 0 ? P.w[ip] / P.sn : 0.0) / q);
        s_accept = (q != 0.0 && ua < acc_p) ? 1 : 0;
        if (s_accept) *out = PosDecision{-1, flags, 1, 0};
    }
    __syncthreads();
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
    __syncthreads();
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
        *out = PosDecision{corr, flags, 0, 0};
    }
}

// The accept chain of each lane over its position decisions, in order: accepted
// drafts are committed until the first rejection (its correction is committed
// and ends the chain) or a terminal token; a lane that accepted every draft
// commits the bonus draw.  Flags of the positions visited (and the bonus row).
__global__ void verify_chain_kernel(const PosDecision* dec, int lanes, int drafts, int target_rows,
                                    const int32_t* drafted, const vi_row_params* params, const int64_t* terminal,
                                    int n_terminal, int32_t* accepted, int32_t* committed,
                                    int32_t* committed_count, uint32_t* lane_flags) {
    const int l = blockIdx.x * blockDim.x + threadIdx.x;
    if (l >= lanes) return;
    const PosDecision* D = dec + size_t(l) * (drafts + 1);
    int32_t* out = committed + size_t(l) * (drafts + 1);
    for (int j = 0; j <= drafts; ++j) out[j] = -1;
    if (verify_list_refused(params[l])) {   // refused lane: nothing accepted, nothing committed
        accepted[l] = 0;
        committed_count[l] = 0;
        if (lane_flags) lane_flags[l] = VI_FLAG_ERROR;
        return;
    }
    uint32_t flags = 0;
    int c = 0, acc = 0;
    bool stopped = false, rejected = false;
    for (int j = 0; j < drafts; ++j) {
        const PosDecision e = D[j];
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
        const PosDecision b = D[drafts];
        flags |= b.flags;
        if (b.token >= 0) out[c++] = b.token;
    }
    accepted[l] = acc;
    committed_count[l] = c;
    if (lane_flags) lane_flags[l] = flags;
}

}  // namespace

namespace {
struct VerifyLayout {
    int trows, drows, lrows, lslices;
};
VerifyLayout verify_layout(int lanes, int drafts, int vocabulary) {
    VerifyLayout v;
    v.trows = lanes * (drafts + 1);
    v.drows = lanes * drafts;
    v.lrows = v.trows;
    v.lslices = std::max(topk_plan(v.trows, vocabulary).slices, topk_plan(v.drows, vocabulary).slices);
    v.lslices = std::max(v.lslices, topk_plan(lanes * drafts, vocabulary).slices);
    return v;
}
}  // namespace

size_t verify_workspace(int lanes, int drafts, int vocabulary) {
    const VerifyLayout v = verify_layout(lanes, drafts, vocabulary);
    size_t b = align_up(size_t(v.trows) * sizeof(vi_greedy_row), 256);
    b += 2 * align_up(size_t(v.trows + v.drows) * kMaxK * 4, 256) + 2 * align_up(size_t(v.trows + v.drows) * 4, 256);
    b += align_up(greedy_workspace(v.trows, vocabulary), 256);
    b += topk_partials_bytes_slices(v.lrows, v.lslices);
    b += align_up(size_t(v.trows) * sizeof(PosDecision), 256);
    return b + 4096;
}

// Workspace layout (fixed for a (lanes, drafts, vocabulary) shape, whichever
// mode runs): greedy rows | lists | greedy partials | top-k partials.
vi_status launch_verify(const VerifyArgs& a, void* ws, size_t ws_bytes, hipStream_t stream) {
    const VerifyLayout v = verify_layout(a.lanes, a.drafts, a.vocabulary);
    const int trows = a.lanes * a.target_rows, drows = a.lanes * a.drafts;
    Carver c(ws, ws_bytes);
    vi_greedy_row* grows = c.take<vi_greedy_row>(size_t(v.trows));
    float* tval = c.take<float>(size_t(v.trows) * kMaxK);
    int* tidx = c.take<int>(size_t(v.trows) * kMaxK);
    float* dval = c.take<float>(size_t(v.drows) * kMaxK);
    int* didx = c.take<int>(size_t(v.drows) * kMaxK);
    uint32_t* tvalid = c.take<uint32_t>(size_t(v.trows));
    uint32_t* tflags = c.take<uint32_t>(size_t(v.trows));
    uint32_t* dvalid = c.take<uint32_t>(size_t(v.drows));
    uint32_t* dflags = c.take<uint32_t>(size_t(v.drows));
    PosDecision* dec = c.take<PosDecision>(size_t(v.trows));
    const size_t gbytes = greedy_workspace(v.trows, a.vocabulary);
    unsigned char* gws = gbytes ? c.take<unsigned char>(gbytes) : nullptr;
    const size_t lbytes = topk_partials_bytes_slices(v.lrows, v.lslices);
    unsigned char* lws = c.take<unsigned char>(lbytes);
    if (!c.ok) return VI_ERR_WORKSPACE;
    const int threads = 64, blocks = (a.lanes + threads - 1) / threads;
    vi_status st;
    if (a.mode == VI_VERIFY_GREEDY) {
        // greedy partials are carved for v.trows rows; a launch over fewer rows
        // (no bonus row) uses a prefix of the same arrival counters.
        st = launch_greedy(a.target, a.target_dtype, trows, a.vocabulary, a.target_stride, 0, grows, gws, gbytes,
                           stream);
        if (st != VI_OK) return st;
        hipLaunchKernelGGL(verify_greedy_kernel, dim3(blocks), dim3(threads), 0, stream, grows, a.lanes, a.drafts,
                           a.target_rows, a.drafted, a.terminal, a.n_terminal, a.accepted, a.committed,
                           a.committed_count, a.lane_flags);
        return launch_status();
    }
    st = launch_verify_lists(a.target, a.target_dtype, trows, v.lrows, v.lslices, a.vocabulary, a.target_stride,
                             a.params, a.target_rows, tval, tidx, tvalid, tflags, lws, lbytes, stream);
    if (st != VI_OK) return st;
    st = launch_verify_lists(a.draft, a.draft_dtype, drows, v.lrows, v.lslices, a.vocabulary, a.draft_stride,
                             a.params, a.drafts, dval, didx, dvalid, dflags, lws, lbytes, stream);
    if (st != VI_OK) return st;
    hipLaunchKernelGGL(verify_position_kernel, dim3(a.drafts + 1, a.lanes), dim3(kFinalizeThreads), 0, stream, tval,
                       tidx, tvalid, tflags, dval, didx, dvalid, dflags, a.drafts, a.target_rows, a.drafted, a.params,
                       a.vocabulary, dec);
    st = launch_status();
    if (st != VI_OK) return st;
    hipLaunchKernelGGL(verify_chain_kernel, dim3(blocks), dim3(threads), 0, stream, dec, a.lanes, a.drafts,
                       a.target_rows, a.drafted, a.params, a.terminal, a.n_terminal, a.accepted, a.committed,
                       a.committed_count, a.lane_flags);
    return launch_status();
}

}  // namespace vi
