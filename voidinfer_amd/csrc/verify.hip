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
// (seed, lane, position + j, purpose 1 / 2).  The finalize kernel runs one
// thread per lane over the <= 64-entry lists (fp64).
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

// Filtered distribution of one sorted list: support size and weights.
struct ListDist {
    const float* z;
    const int* id;
    int support;
    bool greedy;
    double w[kMaxK];
    double sn;
};

__device__ void list_dist(const vi_row_params& p, const float* z, const int* id, uint32_t valid, ListDist& d) {
    d.z = z; d.id = id; d.support = 0; d.sn = 0.0; d.greedy = !(p.temperature > 0.0f);
    if (valid == 0) return;
    if (d.greedy) { d.support = 1; d.w[0] = 1.0; d.sn = 1.0; return; }
    const int cap = min(p.top_k, int(valid));
    const double z0 = double(z[0]);
    double s = 0.0;
    for (int j = 0; j < cap; ++j) { d.w[j] = exp(double(z[j]) - z0); s += d.w[j]; }
    const double minp = double(p.min_p), target = double(p.top_p) * s;
    double cum = 0.0;
    int n = 0;
    for (int j = 0; j < cap; ++j) {
        if (p.min_p > 0.0f && d.w[j] < minp * d.w[0]) break;
        cum += d.w[j];
        n = j + 1;
        if (p.top_p < 1.0f && cum >= target) break;
    }
    if (n < 1) n = 1;
    d.support = n;
    for (int j = 0; j < n; ++j) d.sn += d.w[j];
}

__device__ double list_prob(const ListDist& d, int token) {
    for (int j = 0; j < d.support; ++j) if (d.id[j] == token) return d.w[j] / d.sn;
    return 0.0;
}

__global__ void verify_sampled_kernel(const float* tval, const int* tidx, const uint32_t* tvalid,
                                      const uint32_t* tflags, const float* dval, const int* didx,
                                      const uint32_t* dvalid, const uint32_t* dflags, int lanes, int drafts,
                                      int target_rows, const int32_t* drafted, const vi_row_params* params,
                                      const int64_t* terminal, int n_terminal, int vocabulary,
                                      int32_t* accepted, int32_t* committed, int32_t* committed_count,
                                      uint32_t* lane_flags) {
    const int l = blockIdx.x * blockDim.x + threadIdx.x;
    if (l >= lanes) return;
    const vi_row_params p = params[l];
    int32_t* out = committed + size_t(l) * (drafts + 1);
    for (int j = 0; j <= drafts; ++j) out[j] = -1;
    uint32_t flags = 0;
    int c = 0, acc = 0;
    bool stopped = false, rejected = false;
    ListDist P, Q;
    for (int j = 0; j < drafts && !stopped; ++j) {
        const size_t tr = size_t(l) * target_rows + j, dr = size_t(l) * drafts + j;
        flags |= tflags[tr] | dflags[dr];
        list_dist(p, tval + tr * kMaxK, tidx + tr * kMaxK, tvalid[tr], P);
        list_dist(p, dval + dr * kMaxK, didx + dr * kMaxK, dvalid[dr], Q);
        if (tvalid[tr] == 0 || dvalid[dr] == 0) flags |= VI_FLAG_EMPTY;
        const int32_t d = drafted[dr];
        const int pos = p.position + j;
        const double ua = philox_uniform(p.seed, p.lane, pos, 1u), uc = philox_uniform(p.seed, p.lane, pos, 2u);
        const double q = (d >= 0 && d < vocabulary) ? list_prob(Q, d) : 0.0;
        double acc_p = 0.0;
        if (q == 0.0) flags |= VI_FLAG_ZERO_Q;
        else acc_p = fmin(1.0, list_prob(P, d) / q);
        if (q != 0.0 && ua < acc_p) {
            out[c++] = d;
            ++acc;
            stopped = is_terminal(terminal, n_terminal, d);
            continue;
        }
        // residual max(0, p - q) over p's support, in token-id order
        int rid[kMaxK];
        double rv[kMaxK];
        int m = 0;
        for (int k = 0; k < P.support; ++k) {
            const int t = P.id[k];
            int at = m++;
            while (at > 0 && rid[at - 1] > t) { rid[at] = rid[at - 1]; rv[at] = rv[at - 1]; --at; }
            rid[at] = t;
            rv[at] = P.w[k] / P.sn;
        }
        double sum = 0.0;
        for (int k = 0; k < m; ++k) { rv[k] = fmax(0.0, rv[k] - list_prob(Q, rid[k])); sum += rv[k]; }
        int32_t corr = 0;
        if (!(sum > 1e-9) || !isfinite(sum)) {
            // No residual mass: correct from p itself (inverse CDF, id order).
            flags |= VI_FLAG_NO_RESIDUAL;
            double cum = 0.0;
            int32_t last = 0;
            bool found = false;
            for (int k = 0; k < m; ++k) {
                const double pv = list_prob(P, rid[k]);
                if (pv > 0.0) last = rid[k];
                cum += pv;
                if (uc < cum) { corr = rid[k]; found = true; break; }
            }
            if (!found) corr = last;
        } else {
            double cum = 0.0;
            int32_t last = 0;
            bool found = false;
            for (int k = 0; k < m; ++k) {
                const double r = rv[k] / sum;
                if (r > 0.0) last = rid[k];
                cum += r;
                if (uc < cum) { corr = rid[k]; found = true; break; }
            }
            if (!found) corr = last;
        }
        out[c++] = corr;
        rejected = true;
        break;
    }
    if (!rejected && !stopped && acc == drafts && target_rows == drafts + 1) {
        const size_t tr = size_t(l) * target_rows + drafts;
        flags |= tflags[tr];
        list_dist(p, tval + tr * kMaxK, tidx + tr * kMaxK, tvalid[tr], P);
        if (tvalid[tr]) {
            if (P.greedy) out[c++] = P.id[0];
            else {
                const double t = philox_uniform(p.seed, p.lane, p.position + drafts, 0u) * P.sn;
                double cum = 0.0;
                int pick = P.support - 1;
                for (int k = 0; k < P.support; ++k) { cum += P.w[k]; if (cum > t) { pick = k; break; } }
                out[c++] = P.id[pick];
            }
        }
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
    hipLaunchKernelGGL(verify_sampled_kernel, dim3(blocks), dim3(threads), 0, stream, tval, tidx, tvalid, tflags,
                       dval, didx, dvalid, dflags, a.lanes, a.drafts, a.target_rows, a.drafted, a.params,
                       a.terminal, a.n_terminal, a.vocabulary, a.accepted, a.committed, a.committed_count,
                       a.lane_flags);
    return launch_status();
}

}  // namespace vi
