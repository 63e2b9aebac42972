// verify.hip — DFlash2 draft verification on the device.
//
// Greedy mode: the target rows' greedy packets (greedy.hip) feed
// decide_exl3_outer_prefix (src/exl3/exact_outer_reference.h:68-82) per lane:
// the committed tokens are the target path through the first mismatch or
// terminal token, `accepted` counts the matches; with a bonus row (target_rows
// = drafts + 1) a fully accepted lane also commits the bonus row's argmax.
//
// Sampled mode: the target and draft rows are filtered with the lane's
// temperature / top-k / top-p / min-p, giving p and q: from top-k lists
// (topk.hip) for lanes with 1 <= top_k <= 64, from the full-vocabulary
// sampler's row distributions (sample_slices.hip / sample_wide.hip) for the
// others.  Per position, in order, the rule of
// Exl3IndependentAcceptanceReference::evaluate
// (src/exl3/sampled_acceptance_reference.h:48-88): accept iff
// u_a < min(1, p[d]/q[d]); at the first rejection draw the correction from the
// residual max(0, p - q) normalised, inverse CDF in token-id order with u_c
// (last positive id on round-off).  u_a, u_c are Philox draws keyed by
// (seed, lane, position + j, purpose 1 / 2).  Every (lane, position) decision
// is taken at once, one wave each over the <= 64-entry lists (fp64): entry-wise
// work on the lanes, the order-dependent sums on lane 0; the last position of
// a lane to finish then walks its accept chain in order (after the
// full-vocabulary kernels, a separate per-lane pass does).  Full-vocabulary lanes: the accept test
// evaluates the target softmax p and the draft q at the drafted token from the
// rows' supports, and the correction walks the target softmax, the draft q and
// their residual over the whole vocabulary in id order (ranges of 16,384
// tokens summed in parallel, then the crossing range scanned again).
#include <algorithm>
#include <math.h>

#include "verify_decide.h"
#include "vi_device.h"
#include "vi_internal.h"

namespace vi {
namespace {

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

// Every position of every lane at once; with `arrivals` (list lanes only) the
// last position of a lane to finish runs its chain (agent-scope hand-off of the
// decisions, the lane's counter reset for the next call), else
// verify_chain_kernel does after the full-vocabulary kernels.
__global__ __launch_bounds__(kFinalizeThreads) void verify_position_kernel(
    const float* tval, const int* tidx, const uint32_t* tvalid, const uint32_t* tflags, const float* dval,
    const int* didx, const uint32_t* dvalid, const uint32_t* dflags, int drafts, int target_rows,
    const int32_t* drafted, const vi_row_params* params, int vocabulary, int full_ok, PosDecision* dec,
    uint32_t* arrivals, const int64_t* terminal, int n_terminal, int32_t* accepted, int32_t* committed,
    int32_t* committed_count, uint32_t* lane_flags) {
    const int j = blockIdx.x, l = blockIdx.y;
    // (position `drafts` is the bonus row's, which has no draft row, and exists
    // only when target_rows == drafts + 1)
    const bool has_t = j < target_rows, has_d = j < drafts;
    const size_t tr = has_t ? size_t(l) * target_rows + j : 0, dr = has_d ? size_t(l) * drafts + j : 0;
    position_decision(params[l], j, l, drafts, target_rows, tval + tr * kMaxK, tidx + tr * kMaxK,
                      has_t ? tvalid[tr] : 0u, has_t ? tflags[tr] : 0u, dval + dr * kMaxK, didx + dr * kMaxK,
                      has_d ? dvalid[dr] : 0u, has_d ? dflags[dr] : 0u, drafted, vocabulary, full_ok, dec);
    if (!arrivals) return;
    uint32_t old = 0;
    if (threadIdx.x == 0) {
        handoff_stores_done();
        old = __hip_atomic_fetch_add(&arrivals[l], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (__builtin_amdgcn_readfirstlane(old) != uint32_t(drafts)) return;   // (drafts + 1 positions per lane)
    handoff_acquire();
    const PosDecision* D = dec + size_t(l) * (drafts + 1);
    lane_chain_wave(l, [&](int q) {
        return PosDecision{get_agent(&D[q].token), get_agent(&D[q].flags), get_agent(&D[q].accept), 0};
    }, drafts, target_rows, drafted, params, terminal, n_terminal, full_ok, accepted, committed, committed_count,
                    lane_flags);
    if (threadIdx.x == 0) put_agent(&arrivals[l], 0u);
}

// The accept chains after the full-vocabulary kernels (one thread per lane).
__global__ void verify_chain_kernel(const PosDecision* dec, int lanes, int drafts, int target_rows,
                                    const int32_t* drafted, const vi_row_params* params, const int64_t* terminal,
                                    int n_terminal, int full_ok, int32_t* accepted, int32_t* committed,
                                    int32_t* committed_count, uint32_t* lane_flags) {
    const int l = blockIdx.x * blockDim.x + threadIdx.x;
    if (l >= lanes) return;
    const PosDecision* D = dec + size_t(l) * (drafts + 1);
    lane_chain(l, [&](int j) { return D[j]; }, drafts, target_rows, drafted, params, terminal, n_terminal, full_ok,
               accepted, committed, committed_count, lane_flags);
}

// ------------------------------------------------------- full-vocabulary lanes
// Lanes with temperature > 0 and top_k outside [1, 64].  The full-route sampler
// leaves every target and draft row's filtered distribution (FullBound: the
// support's end and mass; bases: end-key logits before each slice) and every
// target row's own draw (the bonus token); p and q are read off them.

constexpr int kFT = 1024;                // accept kernel threads
constexpr int kRT = 1024;                // residual kernels' threads
constexpr int kRange = 16384;            // residual range (divides both routes' slices)
constexpr int kREPT = kRange / kRT;      // tokens per thread and range
constexpr int kW = kRT / kWave;
static_assert(kFullSlice16 % kRange == 0 && kFullSlice32 % kRange == 0, "residual ranges");

struct FullRows {
    const void* row0;
    int dtype;
    int64_t stride;
    const FullBound* bound;          // [rows]
    const uint32_t* bases;           // [rows][kFullBaseSlots]
    const vi_sample_stats* stats;    // [rows]
    int slice;                       // logits per slice (bases granularity)
};

struct FullVerifyArgs {
    FullRows t, d;                   // target rows [lanes][target_rows], draft rows [lanes][drafts]
    const int32_t* ttok;             // the target rows' draws
    int lanes, drafts, target_rows, vocabulary;
    const int32_t* drafted;
    const vi_row_params* params;
    const int64_t* terminal;
    int n_terminal;
    PosDecision* dec;
    double* rsum;                    // [lanes][ranges][2]: residual mass, p mass of each range
    int* rlast;                      // [lanes][ranges][2]: last id with residual / with p (-1: none)
    int ranges;
};

__device__ __forceinline__ const void* row_at(const FullRows& R, size_t r) {
    return static_cast<const unsigned char*>(R.row0) + r * size_t(R.stride) * (R.dtype == VI_F32 ? 4u : 2u);
}

// Order key of a logit (0: not valid) in the full routes' convention: key16 of
// the 16-bit pattern, or the 32-bit key of z for fp32 logits; and z of a key.
template <int DT>
__device__ __forceinline__ uint32_t dist_key(uint32_t b, float inv_t) {
    if constexpr (DT == VI_F32) {
        float x = __builtin_bit_cast(float, b);
        if (!isfinite(x)) return 0u;
        if (x == 0.0f) x = 0.0f;
        const float z = x * inv_t;
        if (!isfinite(z)) return 0u;
        uint32_t u = __builtin_bit_cast(uint32_t, z);
        if (z == 0.0f) u = 0u;
        return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    } else {
        if (!Elem<DT>::finite_bits(b) || !isfinite(Elem<DT>::decode(b) * inv_t)) return 0u;
        return key16(b);
    }
}
template <int DT>
__device__ __forceinline__ float dist_z(uint32_t k, float inv_t) {
    if constexpr (DT == VI_F32) return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
    else return Elem<DT>::decode(unkey16(k)) * inv_t;
}

// Support membership of a logit of key k; rank: its place among the row's
// end-key logits in id order (used only when k is the end key).
__device__ __forceinline__ bool in_support(uint32_t k, const FullBound& B, uint32_t rank) {
    if (!k || !B.valid) return false;
    if (k != B.end_key) return k > B.end_key;
    return B.end_take == 0xffffffffu || rank < B.end_take;
}
__device__ __forceinline__ bool counts_rank(uint32_t k, const FullBound& B) {
    return k && B.valid && k == B.end_key && B.end_take != 0xffffffffu;
}

// End-key logits of ids [lo, hi) of a row; all threads (NT of them).
template <int DT, int NT>
__device__ uint32_t end_key_count(const void* row, int64_t lo, int64_t hi, const FullBound& B, uint32_t* tmp) {
    uint32_t c = 0u;
    constexpr int U = 8;   // loads in flight per thread
    for (int64_t i0 = lo + threadIdx.x; i0 < hi; i0 += int64_t(U) * NT) {
        uint32_t b[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + int64_t(u) * NT;
            b[u] = i < hi ? load_bits<DT>(row, i) : 0u;
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            c += (i0 + int64_t(u) * NT < hi && counts_rank(dist_key<DT>(b[u], B.inv_t), B)) ? 1u : 0u;
    }
    uint32_t tot = 0u;
    (void)block_exclusive_scan_u32<NT>(c, tmp, &tot);
    return tot;
}

// p (or q) of token x in row r; all threads.
template <int DT, int NT>
__device__ double prob_at(const FullRows& R, size_t r, int x, uint32_t* tmp) {
    const FullBound B = R.bound[r];
    const void* row = row_at(R, r);
    const uint32_t k = dist_key<DT>(load_bits<DT>(row, x), B.inv_t);
    uint32_t rank = 0u;
    if (counts_rank(k, B)) {   // (uniform)
        const int s = x / R.slice;
        rank = R.bases[r * kFullBaseSlots + s] + end_key_count<DT, NT>(row, int64_t(s) * R.slice, x, B, tmp);
    }
    return in_support(k, B, rank) ? exp(double(dist_z<DT>(k, B.inv_t)) - B.z0) / B.s_n : 0.0;
}

// The accept test of every (lane, position) of the full-vocabulary lanes:
// u_a < min(1, p(d) / q(d)) with the target softmax p and the draft q at the
// drafted token; position `drafts` takes the bonus row's draw.
template <int TDT, int DDT>
__global__ __launch_bounds__(kFT) void verify_full_accept_kernel(FullVerifyArgs a) {
    __shared__ uint32_t tmp[kFT / kWave + 1];
    const int j = blockIdx.x, l = blockIdx.y;
    const vi_row_params p = a.params[l];
    if (!verify_list_refused(p)) return;
    PosDecision* out = a.dec + size_t(l) * (a.drafts + 1) + j;
    if (j == a.drafts) {
        if (a.target_rows != a.drafts + 1 || threadIdx.x != 0) return;
        const size_t tr = size_t(l) * a.target_rows + j;
        const uint32_t f = a.t.stats[tr].flags;
        const int32_t tok = a.ttok[tr];
        const bool bad = (f & VI_FLAG_ERROR) || tok < 0 || tok >= a.vocabulary;
        *out = PosDecision{bad ? -1 : tok, (f & VI_FLAG_ERROR) ? uint32_t(VI_FLAG_ERROR) : 0u, 0, 0};
        return;
    }
    const size_t tr = size_t(l) * a.target_rows + j, dr = size_t(l) * a.drafts + j;
    const int32_t x = a.drafted[dr];
    uint32_t flags = (a.t.stats[tr].flags | a.d.stats[dr].flags) &
                     uint32_t(VI_FLAG_NONFINITE | VI_FLAG_EMPTY | VI_FLAG_ERROR);
    double q = 0.0, pv = 0.0;
    if (x >= 0 && x < a.vocabulary) {
        q = prob_at<DDT, kFT>(a.d, dr, x, tmp);
        pv = prob_at<TDT, kFT>(a.t, tr, x, tmp);
    }
    if (threadIdx.x == 0) {
        const double ua = philox_uniform(p.seed, p.lane, p.position + j, 1u);
        double acc = 0.0;
        if (q == 0.0) flags |= VI_FLAG_ZERO_Q;
        else acc = fmin(1.0, pv / q);
        const int accept = (!(flags & VI_FLAG_ERROR) && q != 0.0 && ua < acc) ? 1 : 0;
        *out = PosDecision{-1, flags, accept, 0};
    }
}

// The lane's first rejected position before any accepted terminal token, or -1:
// 64 positions per round, one per lane of the wave (every wave alike).
__device__ int first_rejection(const FullVerifyArgs& a, int l) {
    const int lane = lane_id();
    for (int j0 = 0; j0 < a.drafts; j0 += kWave) {
        const int j = j0 + lane;
        bool ends = false, usable = false;
        if (j < a.drafts) {
            const PosDecision e = a.dec[size_t(l) * (a.drafts + 1) + j];
            ends = e.accept ? is_terminal(a.terminal, a.n_terminal, a.drafted[size_t(l) * a.drafts + j]) : true;
            usable = !e.accept && !(e.flags & VI_FLAG_ERROR);
        }
        const uint64_t m = ballot(ends);
        if (m) {
            const int f = __builtin_ctzll(m);
            return (ballot(usable) >> f) & 1ull ? j0 + f : -1;
        }
    }
    return -1;
}

// exp(z - z0) of a support logit (z <= z0), one hardware exp2.
__device__ __forceinline__ float weight_f(float z, float z0) {
    return __builtin_amdgcn_exp2f((z - z0) * 1.44269504088896340736f);
}

// End-key logits of the row before id r0 (a range start).
template <int DT>
__device__ uint32_t range_base(const FullRows& R, size_t r, const FullBound& B, int r0, uint32_t* tmp) {
    if (!B.valid || B.end_take == 0xffffffffu) return 0u;   // (uniform)
    const int s = r0 / R.slice, in = r0 - s * R.slice;
    return R.bases[r * kFullBaseSlots + s] +
           (in ? end_key_count<DT, kRT>(row_at(R, r), int64_t(s) * R.slice, r0, B, tmp) : 0u);
}

// Tokens [r0, r1) of the target and draft rows of one position: fn(e, id, p, q)
// for this thread's tokens r0 + kREPT t + e, in id order; all threads.
template <int TDT, int DDT, class F>
__device__ __forceinline__ void range_pass(const FullVerifyArgs& a, size_t tr, size_t dr, int r0, int r1,
                                           uint32_t* tmp, F&& fn) {
    const FullBound TB = a.t.bound[tr], DB = a.d.bound[dr];
    const void* trow = row_at(a.t, tr);
    const void* drow = row_at(a.d, dr);
    // weights exp(z - z0) in single precision (z0 is a float z); 1 / S_n in double
    const float tz0 = float(TB.z0), dz0 = float(DB.z0);
    const double tinv = TB.valid ? 1.0 / TB.s_n : 0.0, dinv = DB.valid ? 1.0 / DB.s_n : 0.0;
    const uint32_t bt = range_base<TDT>(a.t, tr, TB, r0, tmp), bd = range_base<DDT>(a.d, dr, DB, r0, tmp);
    const int e0 = r0 + kREPT * int(threadIdx.x);
    // this thread's kREPT consecutive logits of each row: whole 16-byte vectors
    // when the row is aligned and they are all inside the range (the pass is
    // latency bound: a few wide loads instead of one 2- or 4-byte load each)
    uint32_t bt_[kREPT], bd_[kREPT];
    auto fetch = [&](const void* rowp, auto dt, uint32_t (&b)[kREPT]) {
        constexpr int DT = decltype(dt)::value;
        constexpr int PV = Elem<DT>::kPerVec;
        const unsigned char* p = static_cast<const unsigned char*>(rowp) + size_t(e0) * (DT == VI_F32 ? 4 : 2);
        if (e0 + kREPT <= r1 && (reinterpret_cast<uintptr_t>(p) & 15u) == 0) {
#pragma unroll
            for (int q = 0; q < kREPT / PV; ++q) {
                const uint4 v = load16_cached(p + 16 * q);
#pragma unroll
                for (int j = 0; j < PV; ++j) b[q * PV + j] = vec_bits<DT>(v, j);
            }
        } else {
#pragma unroll
            for (int e = 0; e < kREPT; ++e) b[e] = e0 + e < r1 ? load_bits<DT>(rowp, e0 + e) : 0u;
        }
    };
    fetch(trow, std::integral_constant<int, TDT>{}, bt_);
    fetch(drow, std::integral_constant<int, DDT>{}, bd_);
    uint32_t kt[kREPT], kd[kREPT], ct = 0u, cd = 0u;
#pragma unroll
    for (int e = 0; e < kREPT; ++e) {
        const int i = e0 + e;
        kt[e] = i < r1 ? dist_key<TDT>(bt_[e], TB.inv_t) : 0u;
        kd[e] = i < r1 ? dist_key<DDT>(bd_[e], DB.inv_t) : 0u;
        ct += counts_rank(kt[e], TB) ? 1u : 0u;
        cd += counts_rank(kd[e], DB) ? 1u : 0u;
    }
    uint32_t tot = 0u;
    uint32_t rt = bt + block_exclusive_scan_u32<kRT>(ct, tmp, &tot);
    uint32_t rd = bd + block_exclusive_scan_u32<kRT>(cd, tmp, &tot);
#pragma unroll
    for (int e = 0; e < kREPT; ++e) {
        const bool it = in_support(kt[e], TB, rt), id = in_support(kd[e], DB, rd);
        rt += counts_rank(kt[e], TB) ? 1u : 0u;
        rd += counts_rank(kd[e], DB) ? 1u : 0u;
        const double pv = it ? double(weight_f(dist_z<TDT>(kt[e], TB.inv_t), tz0)) * tinv : 0.0;
        const double qv = id ? double(weight_f(dist_z<DDT>(kd[e], DB.inv_t), dz0)) * dinv : 0.0;
        fn(e, e0 + e, pv, qv);
    }
}

// Sum over the block in a fixed order (the threads' order); every thread gets it.
__device__ double block_sum_f64(double v, double* tmp) {
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    const double x = wave_incl_scan_f64(v);
    if (lane == kWave - 1) tmp[wave] = x;
    __syncthreads();
    double s = 0.0;
    for (int w = 0; w < int(blockDim.x) / kWave; ++w) s += tmp[w];
    __syncthreads();
    return s;
}
__device__ int block_max_i(int v, int* tmp) {
#pragma unroll
    for (int o = 32; o; o >>= 1) v = max(v, __shfl_xor(v, o, kWave));
    if (lane_id() == 0) tmp[threadIdx.x / kWave] = v;
    __syncthreads();
    int m = -1;
    for (int w = 0; w < int(blockDim.x) / kWave; ++w) m = max(m, tmp[w]);
    __syncthreads();
    return m;
}

// Residual and p mass of each range of each lane's rejected position.
template <int TDT, int DDT>
__global__ __launch_bounds__(kRT) void verify_full_ranges_kernel(FullVerifyArgs a) {
    __shared__ uint32_t tmp[kW + 1];
    __shared__ double dtmp[kW];
    __shared__ int itmp[kW];
    const int rg = blockIdx.x, l = blockIdx.y;
    if (!verify_list_refused(a.params[l])) return;
    const int js = first_rejection(a, l);
    if (js < 0) return;
    const size_t tr = size_t(l) * a.target_rows + js, dr = size_t(l) * a.drafts + js;
    const int r0 = rg * kRange, r1 = min(a.vocabulary, r0 + kRange);
    double R = 0.0, P = 0.0;
    int lr = -1, lp = -1;
    range_pass<TDT, DDT>(a, tr, dr, r0, r1, tmp, [&](int, int i, double pv, double qv) {
        const double rv = fmax(0.0, pv - qv);
        R += rv;
        P += pv;
        if (rv > 0.0) lr = i;
        if (pv > 0.0) lp = i;
    });
    const double Rt = block_sum_f64(R, dtmp), Pt = block_sum_f64(P, dtmp);
    const int lrt = block_max_i(lr, itmp), lpt = block_max_i(lp, itmp);
    if (threadIdx.x == 0) {
        const size_t at = (size_t(l) * a.ranges + rg) * 2;
        a.rsum[at] = Rt;
        a.rsum[at + 1] = Pt;
        a.rlast[at] = lrt;
        a.rlast[at + 1] = lpt;
    }
}

// The correction of each lane's rejected position: the first token (id order)
// whose cumulative residual exceeds u_c times the residual mass, or, with no
// residual mass (<= 1e-9), the first whose cumulative p exceeds u_c; past the
// end by round-off, the last token with mass.
template <int TDT, int DDT>
__global__ __launch_bounds__(kRT) void verify_full_correction_kernel(FullVerifyArgs a) {
    __shared__ uint32_t tmp[kW + 1];
    __shared__ double dtmp[kW + 1];
    __shared__ int s_range, s_tok;
    __shared__ double s_before, s_target;
    __shared__ uint32_t s_nores;
    const int l = blockIdx.x, tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const vi_row_params p = a.params[l];
    if (!verify_list_refused(p)) return;
    const int js = first_rejection(a, l);
    if (js < 0) return;
    if (wave == 0) {   // the ranges in order (each lane loads a range's sums; the sums read lane by lane)
        double R = 0.0, P = 0.0;
        int lr = -1, lp = -1;
        for (int r0 = 0; r0 < a.ranges; r0 += kWave) {
            const int r = min(r0 + lane, a.ranges - 1);
            const size_t at = (size_t(l) * a.ranges + r) * 2;
            const double rs = a.rsum[at], ps = a.rsum[at + 1];
            const int rl = a.rlast[at], pl = a.rlast[at + 1];
            for (int q = 0; q < min(kWave, a.ranges - r0); ++q) {
                R += readlane_d(rs, q);
                P += readlane_d(ps, q);
                lr = max(lr, __builtin_amdgcn_readlane(rl, q));
                lp = max(lp, __builtin_amdgcn_readlane(pl, q));
            }
        }
        const double uc = philox_uniform(p.seed, p.lane, p.position + js, 2u);
        const bool nores = !(R > 1e-9) || !isfinite(R);
        const double target = nores ? uc : uc * R;
        int range = -1;
        double cum = 0.0;
        for (int r0 = 0; r0 < a.ranges && range < 0; r0 += kWave) {
            const double mv = a.rsum[(size_t(l) * a.ranges + min(r0 + lane, a.ranges - 1)) * 2 + (nores ? 1 : 0)];
            for (int q = 0; q < min(kWave, a.ranges - r0) && range < 0; ++q) {
                const double m = readlane_d(mv, q);
                if (cum + m > target) range = r0 + q;
                else cum += m;
            }
        }
        if (lane == 0) {
            s_range = range;
            s_before = cum;
            s_target = target;
            s_nores = nores ? 1u : 0u;
            s_tok = max(0, nores ? lp : lr);   // (round-off past the end)
        }
    }
    __syncthreads();
    const int range = s_range;
    if (range >= 0) {   // (uniform) the crossing range again, token by token
        const size_t tr = size_t(l) * a.target_rows + js, dr = size_t(l) * a.drafts + js;
        const int r0 = range * kRange, r1 = min(a.vocabulary, r0 + kRange);
        const bool nores = s_nores != 0u;
        double v[kREPT], own = 0.0;
        int last = -1;
        range_pass<TDT, DDT>(a, tr, dr, r0, r1, tmp, [&](int e, int i, double pv, double qv) {
            v[e] = nores ? pv : fmax(0.0, pv - qv);
            own += v[e];
            if (v[e] > 0.0) last = i;
        });
        // exclusive prefix of the threads' sums (the order block_sum_f64 sums in)
        const double incl = wave_incl_scan_f64(own);
        if (lane == kWave - 1) dtmp[wave] = incl;
        __syncthreads();
        double wb = 0.0;
        for (int w = 0; w < wave; ++w) wb += dtmp[w];
        const int src = max(lane - 1, 0) << 2;
        const uint64_t ib = __builtin_bit_cast(uint64_t, incl);
        const uint32_t lo = uint32_t(__builtin_amdgcn_ds_bpermute(src, int(uint32_t(ib))));
        const uint32_t hi = uint32_t(__builtin_amdgcn_ds_bpermute(src, int(uint32_t(ib >> 32))));
        const double ex = wb + (lane ? __builtin_bit_cast(double, (uint64_t(hi) << 32) | lo) : 0.0);
        const double t = s_target - s_before;
        if (own > 0.0 && ex <= t && ex + own > t) {   // this thread's tokens hold the crossing
            double cum = ex;
            int pick = last;
            bool found = false;
            const int e0 = r0 + kREPT * tid;
#pragma unroll
            for (int e = 0; e < kREPT; ++e) {
                cum += v[e];
                if (!found && cum > t && v[e] > 0.0) { pick = e0 + e; found = true; }
            }
            if (pick >= 0) s_tok = pick;
        }
        __syncthreads();
    }
    if (tid == 0) {
        PosDecision* out = a.dec + size_t(l) * (a.drafts + 1) + js;
        out->token = s_tok;
        if (s_nores) out->flags |= VI_FLAG_NO_RESIDUAL;
    }
}

// Per-row sampler parameters of the full-vocabulary lanes' rows: the lane's,
// without penalties, at position + j.
__global__ void verify_row_params_kernel(const vi_row_params* params, int lanes, int per_lane,
                                         vi_row_params* out, int per_lane2, vi_row_params* out2) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= lanes * per_lane) {   // (the second row set's rows follow the first's)
        i -= lanes * per_lane;
        if (i >= lanes * per_lane2) return;
        per_lane = per_lane2;
        out = out2;
    }
    vi_row_params p = params[i / per_lane];
    p.repetition_penalty = 1.0f;
    p.presence_penalty = 0.0f;
    p.frequency_penalty = 0.0f;
    p.position += i % per_lane;
    if (!verify_list_refused(p)) p.temperature = 0.0f;   // (list lanes: not the full route's rows)
    out[i] = p;
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
    v.lrows = v.trows + v.drows;   // (the paired launch carves both row sets' partials)
    v.lslices = std::max(topk_plan(v.trows, vocabulary).slices, topk_plan(v.drows, vocabulary).slices);
    v.lslices = std::max(v.lslices, topk_plan(lanes * drafts, vocabulary).slices);
    return v;
}
}  // namespace

namespace {
inline int full_ranges(int vocabulary) { return (vocabulary + kRange - 1) / kRange; }
inline size_t full_sampler_bytes(int rows, int vocabulary) {
    return std::max(full_workspace(rows, vocabulary), wide_workspace(rows, vocabulary));
}
// The full-vocabulary path's part of the workspace (after the list path's).
size_t full_verify_bytes(int lanes, int drafts, int vocabulary) {
    const size_t rows = size_t(lanes) * size_t(2 * drafts + 1);   // target (with bonus) and draft rows
    size_t b = align_up(rows * sizeof(vi_row_params), 256) + align_up(rows * sizeof(FullBound), 256);
    b += align_up(rows * kFullBaseSlots * 4, 256) + align_up(rows * sizeof(vi_sample_stats), 256);
    b += align_up(rows * 4, 256);
    b += align_up(size_t(lanes) * full_ranges(vocabulary) * 2 * 8, 256) +
         align_up(size_t(lanes) * full_ranges(vocabulary) * 2 * 4, 256);
    // (one sampler workspace per row set: the two sets are sampled side by side)
    return b + full_sampler_bytes(lanes * (drafts + 1), vocabulary) + full_sampler_bytes(lanes * drafts, vocabulary) +
           2304;
}
bool full_path_ok(const void* logits, int dtype, int vocabulary, int64_t stride) {
    if (dtype == VI_F32) return wide_supported(vocabulary, stride) && reinterpret_cast<uintptr_t>(logits) % 4 == 0;
    return full_supported(dtype, vocabulary, stride) && reinterpret_cast<uintptr_t>(logits) % 16 == 0;
}

template <int TDT, int DDT>
void launch_full_verify(const FullVerifyArgs& f, hipStream_t stream) {
    hipLaunchKernelGGL((verify_full_accept_kernel<TDT, DDT>), dim3(f.drafts + 1, f.lanes), dim3(kFT), 0, stream, f);
    hipLaunchKernelGGL((verify_full_ranges_kernel<TDT, DDT>), dim3(f.ranges, f.lanes), dim3(kRT), 0, stream, f);
    hipLaunchKernelGGL((verify_full_correction_kernel<TDT, DDT>), dim3(f.lanes), dim3(kRT), 0, stream, f);
}
template <int TDT>
void launch_full_verify_d(const FullVerifyArgs& f, hipStream_t stream) {
    switch (f.d.dtype) {
        case VI_BF16: launch_full_verify<TDT, VI_BF16>(f, stream); break;
        case VI_F16: launch_full_verify<TDT, VI_F16>(f, stream); break;
        default: launch_full_verify<TDT, VI_F32>(f, stream); break;
    }
}
}  // namespace

// The greedy launch's workspace: arrival counters for v.trows rows (the
// bonus row's count) ahead of the partials of either row count.
static size_t verify_greedy_bytes(const VerifyLayout& v, int lanes, int drafts, int vocabulary) {
    const size_t with = greedy_workspace(v.trows, vocabulary), without = greedy_workspace(lanes * drafts, vocabulary);
    if (!with && !without) return 0;
    return align_up(size_t(v.trows) * 4, 256) + std::max(with, without);
}

size_t verify_workspace(int lanes, int drafts, int vocabulary) {
    const VerifyLayout v = verify_layout(lanes, drafts, vocabulary);
    size_t b = align_up(size_t(v.trows) * sizeof(vi_greedy_row), 256);
    b += 2 * align_up(size_t(v.trows + v.drows) * kMaxK * 4, 256) + 2 * align_up(size_t(v.trows + v.drows) * 4, 256);
    b += align_up(verify_greedy_bytes(v, lanes, drafts, vocabulary), 256);
    b += topk_partials_bytes_slices(v.lrows, v.lslices);
    b += align_up(size_t(v.trows) * sizeof(PosDecision), 256) + align_up(size_t(lanes) * 4, 256);
    b += align_up(size_t(lanes) * (drafts + 1) * 4, 256);
    b += full_verify_bytes(lanes, drafts, vocabulary);
    return b + 4096;
}

// Workspace layout (fixed for a (lanes, drafts, vocabulary) shape, whichever
// mode runs): greedy rows | lists | decisions | greedy partials | top-k
// partials | the full-vocabulary path's rows and sampler workspace.
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
    uint32_t* larr = c.take<uint32_t>(size_t(a.lanes));   // positions of a lane decided (zero between calls)
    uint32_t* parr = c.take<uint32_t>(size_t(a.lanes) * (a.drafts + 1));   // rows of a position listed (the same)
    const size_t gbytes = verify_greedy_bytes(v, a.lanes, a.drafts, a.vocabulary);
    unsigned char* gws = gbytes ? c.take<unsigned char>(gbytes) : nullptr;
    const size_t lbytes = topk_partials_bytes_slices(v.lrows, v.lslices);
    unsigned char* lws = c.take<unsigned char>(lbytes);
    if (!c.ok) return VI_ERR_WORKSPACE;
    const int threads = 64, blocks = (a.lanes + threads - 1) / threads;
    vi_status st;
    if (a.mode == VI_VERIFY_GREEDY) {
        // the greedy workspace is carved for v.trows rows (with the bonus row):
        // its arrival counters stay where they are for either row count
        st = launch_greedy(a.target, a.target_dtype, trows, a.vocabulary, a.target_stride, 0, grows, gws, gbytes,
                           stream, v.trows);
        if (st != VI_OK) return st;
        hipLaunchKernelGGL(verify_greedy_kernel, dim3(blocks), dim3(threads), 0, stream, grows, a.lanes, a.drafts,
                           a.target_rows, a.drafted, a.terminal, a.n_terminal, a.accepted, a.committed,
                           a.committed_count, a.lane_flags);
        return launch_status();
    }
    // full-vocabulary lanes run unless the caller vouches that every sampled
    // lane has 1 <= top_k <= 64 (VI_VERIFY_SAMPLED_TOPK), and both row sets fit
    // the full routes
    const int full_ok = (a.mode == VI_VERIFY_SAMPLED &&
                         full_path_ok(a.target, a.target_dtype, a.vocabulary, a.target_stride) &&
                         full_path_ok(a.draft, a.draft_dtype, a.vocabulary, a.draft_stride)) ? 1 : 0;
    // every lane listed: the target rows' scan draws the bonus tokens as its
    // bonus rows finish, the draft rows' scan takes each position's decision as
    // its row finishes, and each lane's last position walks the chain (two
    // launches in all)
    const bool fused = !full_ok;
    VerifyDecideArgs dv{};
    dv.drafts = a.drafts; dv.target_rows = a.target_rows;
    dv.tlval = tval; dv.tlidx = tidx; dv.tlvalid = tvalid; dv.tlflags = tflags;
    dv.dlval = dval; dv.dlidx = didx; dv.dlvalid = dvalid; dv.dlflags = dflags; dv.parr = parr;
    dv.drafted = a.drafted; dv.dec = dec; dv.larr = larr;
    dv.terminal = a.terminal; dv.n_terminal = a.n_terminal;
    dv.accepted = a.accepted; dv.committed = a.committed; dv.committed_count = a.committed_count;
    dv.lane_flags = a.lane_flags;
    const bool paired = verify_pair_supported(a.target, a.target_dtype, a.target_stride, a.draft, a.draft_dtype,
                                              a.draft_stride);
    if (paired) {
        // both row sets in one launch: each listed position decided by its later
        // row, each listed lane's chain walked by its last position (the lanes
        // without a list, when the full path runs, are left to it)
        st = launch_verify_pair(a.target, a.target_dtype, a.target_stride, a.draft, a.draft_dtype, a.draft_stride,
                                a.lanes, a.vocabulary, a.params, v.lrows, v.lslices, tval, tidx, tvalid, tflags, dval,
                                didx, dvalid, dflags, dv, lws, lbytes, stream, full_ok);
        if (st != VI_OK || !full_ok) return st;
    } else {
    st = launch_verify_lists(a.target, a.target_dtype, trows, v.lrows, v.lslices, a.vocabulary, a.target_stride,
                             a.params, a.target_rows, tval, tidx, tvalid, tflags, full_ok, lws, lbytes, stream,
                             fused ? &dv : nullptr, 2);
    if (st != VI_OK) return st;
    if (fused)
        return launch_verify_lists(a.draft, a.draft_dtype, drows, v.lrows, v.lslices, a.vocabulary, a.draft_stride,
                                   a.params, a.drafts, dval, didx, dvalid, dflags, 0, lws, lbytes, stream, &dv, 1);
    st = launch_verify_lists(a.draft, a.draft_dtype, drows, v.lrows, v.lslices, a.vocabulary, a.draft_stride,
                             a.params, a.drafts, dval, didx, dvalid, dflags, full_ok, lws, lbytes, stream);
    if (st != VI_OK) return st;
    hipLaunchKernelGGL(verify_position_kernel, dim3(a.drafts + 1, a.lanes), dim3(kFinalizeThreads), 0, stream, tval,
                       tidx, tvalid, tflags, dval, didx, dvalid, dflags, a.drafts, a.target_rows, a.drafted, a.params,
                       a.vocabulary, full_ok, dec, full_ok ? nullptr : larr, a.terminal, a.n_terminal, a.accepted,
                       a.committed, a.committed_count, a.lane_flags);
    st = launch_status();
    if (st != VI_OK) return st;
    }
    if (full_ok) {
        const size_t tn = size_t(trows), dn = size_t(drows);
        vi_row_params* tpar = c.take<vi_row_params>(tn);
        vi_row_params* dpar = c.take<vi_row_params>(dn);
        FullBound* tb = c.take<FullBound>(tn);
        FullBound* db = c.take<FullBound>(dn);
        uint32_t* tbase = c.take<uint32_t>(tn * kFullBaseSlots);
        uint32_t* dbase = c.take<uint32_t>(dn * kFullBaseSlots);
        vi_sample_stats* tst = c.take<vi_sample_stats>(tn);
        vi_sample_stats* dst = c.take<vi_sample_stats>(dn);
        int32_t* ttok = c.take<int32_t>(tn);
        int32_t* dtok = c.take<int32_t>(dn);
        const int ranges = full_ranges(a.vocabulary);
        double* rsum = c.take<double>(size_t(a.lanes) * ranges * 2);
        int* rlast = c.take<int>(size_t(a.lanes) * ranges * 2);
        const size_t fbytes = full_sampler_bytes(v.trows, a.vocabulary);
        const size_t dbytes = full_sampler_bytes(a.lanes * a.drafts, a.vocabulary);
        unsigned char* fws = c.take<unsigned char>(fbytes);
        unsigned char* dws = c.take<unsigned char>(dbytes);
        if (!c.ok) return VI_ERR_WORKSPACE;
        hipLaunchKernelGGL(verify_row_params_kernel, dim3((trows + drows + 255) / 256), dim3(256), 0, stream,
                           a.params, a.lanes, a.target_rows, tpar, a.drafts, dpar);
        // the rows' filtered distributions (and the target rows' draws) from the
        // full-vocabulary sampler, each row set in its own workspace: the draft
        // rows on the side stream beside the target rows on the caller's, joined
        // back before the accept launch
        auto sample = [&](const void* logits, int dtype, int rows, int64_t stride, const vi_row_params* par,
                          int32_t* tok, vi_sample_stats* stats, const FullOut* out, unsigned char* w, size_t wb,
                          hipStream_t on) {
            SampleArgs s{};
            s.logits = logits; s.dtype = dtype; s.rows = rows; s.vocabulary = a.vocabulary; s.stride = stride;
            s.params = par; s.tokens = tok; s.stats = stats; s.route_mask = VI_ROUTE_FULL; s.full_out = out;
            return dtype == VI_F32 ? launch_wide(s, w, wb, nullptr, 0, 0, nullptr, on) : launch_full(s, w, wb, on);
        };
        const FullOut tout{tb, tbase}, dout{db, dbase};
        SideStream* side = drows > 0 ? side_stream() : nullptr;
        if (side && (hipEventRecord(side->fork, stream) != hipSuccess ||
                     hipStreamWaitEvent(side->stream, side->fork, 0) != hipSuccess)) {
            (void)hipGetLastError();
            side = nullptr;
        }
        st = sample(a.draft, a.draft_dtype, drows, a.draft_stride, dpar, dtok, dst, &dout, dws, dbytes,
                    side ? side->stream : stream);
        if (st == VI_OK)
            st = sample(a.target, a.target_dtype, trows, a.target_stride, tpar, ttok, tst, &tout, fws, fbytes, stream);
        // joined also when a launch failed: the side work uses the caller's workspace
        if (side && (hipEventRecord(side->join, side->stream) != hipSuccess ||
                     hipStreamWaitEvent(stream, side->join, 0) != hipSuccess))
            return VI_ERR_LAUNCH;
        if (st != VI_OK) return st;
        FullVerifyArgs f{};
        f.t = FullRows{a.target, a.target_dtype, a.target_stride, tb, tbase, tst,
                       a.target_dtype == VI_F32 ? kFullSlice32 : kFullSlice16};
        f.d = FullRows{a.draft, a.draft_dtype, a.draft_stride, db, dbase, dst,
                       a.draft_dtype == VI_F32 ? kFullSlice32 : kFullSlice16};
        f.ttok = ttok; f.lanes = a.lanes; f.drafts = a.drafts; f.target_rows = a.target_rows;
        f.vocabulary = a.vocabulary; f.drafted = a.drafted; f.params = a.params; f.terminal = a.terminal;
        f.n_terminal = a.n_terminal; f.dec = dec; f.rsum = rsum; f.rlast = rlast; f.ranges = ranges;
        switch (a.target_dtype) {
            case VI_BF16: launch_full_verify_d<VI_BF16>(f, stream); break;
            case VI_F16: launch_full_verify_d<VI_F16>(f, stream); break;
            default: launch_full_verify_d<VI_F32>(f, stream); break;
        }
        st = launch_status();
        if (st != VI_OK) return st;
    }
    if (!full_ok) return VI_OK;   // (the position launch ran every lane's chain)
    hipLaunchKernelGGL(verify_chain_kernel, dim3(blocks), dim3(threads), 0, stream, dec, a.lanes, a.drafts,
                       a.target_rows, a.drafted, a.params, a.terminal, a.n_terminal, full_ok, a.accepted, a.committed,
                       a.committed_count, a.lane_flags);
    return launch_status();
}

}  // namespace vi
