// sample_full.hip — full-vocabulary rows of the batched sampler (top_k = 0 or
// > 64): penalties, temperature, top-k / top-p / min-p over the whole
// vocabulary and the Philox inverse-CDF draw, with one HBM read of the row.
//
// Key fact used: with bf16 / fp16 logits (and penalized logits stored back in
// the same dtype) every scaled logit z = x' / T is a strictly monotone function
// of the logit's 16-bit pattern.  The multiset of z over a row is therefore
// exactly a 65,536-bin count histogram over order-preserving 16-bit keys, and
// every truncation (top-k count, top-p mass, min-p ratio) and the draw reduce to
// prefix sums over the occupied bins; the float work (one exp per bin, fp64) is
// per distinct key, not per token.
//
// Shape: each row is owned by a PAIR of 1024-thread workgroups (one per half of
// the vocabulary, placed on the same XCD), which keep their half of the row in
// registers (16 x 16-byte vectors per thread):
//   A. history -> LDS u8 occurrence counts of the half (saturating, exact side
//      table), penalties applied to the register-resident logits in place;
//   B. LDS u16 key histogram -> sorted (key, count) list published to HBM;
//   C. one pair barrier; both workgroups merge the two lists (merge path) into
//      cumulative counts / masses in LDS and take identical decisions;
//   D. the half owning the drawn (key, rank) finds the token in its registers.
// The pair barrier spins on an agent-scope counter with an iteration cap, so a
// missing partner becomes VI_FLAG_ERROR, never a hang.  Roofline: HBM,
// V x 2 + L x 4 bytes per row (logits once, history once per pair via L2).
#include <math.h>

#include "vi_device.h"
#include "vi_internal.h"

namespace vi {
namespace {

constexpr int kFT = 1024;                 // threads per workgroup
constexpr int kFW = kFT / kWave;          // waves per workgroup
constexpr int kFV = 16;                   // 16-byte vectors per thread
constexpr int kHalfMax = kFT * kFV * 8;   // logits per half (131,072)
constexpr int kListMax = 8192;            // merged (key, half) entries
constexpr int kOvfMax = 512;              // history tokens with >= 255 occurrences per half
constexpr uint32_t kSpinLimit = 1u << 22;

struct FullHeader {
    uint32_t n_list;
    uint32_t n_finite;
    uint32_t flags;
    uint32_t pad;
};
struct alignas(256) PairBarrier {
    uint32_t count;
    uint32_t gen;
    uint32_t pad[62];
};

struct FullArgs {
    const void* logits;
    int rows, vocabulary, half_len;
    int64_t stride;
    const vi_row_params* params;
    const int32_t* histories;
    const int64_t* offsets;
    int32_t* tokens;
    double* uniforms;
    float* probs;
    int64_t probs_stride;
    vi_sample_stats* stats;
    PairBarrier* barriers;   // [pairs]
    FullHeader* headers;     // [rows][2]
    uint32_t* lists;         // [rows][2][kListMax]
};

constexpr uint32_t kHdrNonfinite = 1u, kHdrBadHistory = 2u, kHdrError = 4u, kHdrOverflow = 8u;

// LDS map (bytes).  Phase A: u8 counts [0, 128 KiB) + saturated side table.
// Phase B: u16 histogram [0, 128 KiB).  Phase C: lists [0, 32 KiB), C u32
// [32 KiB, 64 KiB + 4), W f64 [64 KiB + 256, 128 KiB + 264).
constexpr int kLdsBytes = 131072 + 8 * kOvfMax + 1024;
constexpr int kOffC = 32768, kOffW = 65536 + 256;

struct Shared {
    uint32_t u[kFW + 1];
    double d[kFW + 1];
    uint32_t ovf_n, flags, minp_pos, found;
    int32_t sel_pos, sel_key, sel_half, sel_count;
    double sel_w;
};

template <int NT>
__device__ __forceinline__ double block_exclusive_scan_f64(double v, double* tmp, double* total) {
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    double x = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const double y = __shfl_up(x, o, kWave);
        if (lane >= o) x += y;
    }
    if (lane == kWave - 1) tmp[wave] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        double s = 0;
        for (int w = 0; w < NT / kWave; ++w) { const double t = tmp[w]; tmp[w] = s; s += t; }
        tmp[NT / kWave] = s;
    }
    __syncthreads();
    const double r = tmp[wave] + (x - v);
    *total = tmp[NT / kWave];
    __syncthreads();
    return r;
}

template <int NT>
__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, uint32_t* tmp) {
    uint32_t t;
    (void)block_exclusive_scan_u32<NT>(v, tmp, &t);
    return t;
}

template <int DT>
__device__ __forceinline__ float key_z(uint32_t key, float inv_t) {
    return Elem<DT>::decode(unkey16(key)) * inv_t;
}

// Sequential merge state of the two descending lists (half 0 first on ties).
struct Merge {
    const uint32_t* A;  // ascending in memory; read reversed
    const uint32_t* B;
    int n0, n1, i, j;
    __device__ uint32_t a(int k) const { return A[n0 - 1 - k]; }
    __device__ uint32_t b(int k) const { return B[n1 - 1 - k]; }
    __device__ void seek(int d) {  // merge path: i + j = d
        int lo = max(0, d - n1), hi = min(d, n0);
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if ((a(mid) >> 16) >= (b(d - 1 - mid) >> 16)) lo = mid + 1; else hi = mid;
        }
        i = lo; j = d - lo;
    }
    // Next entry: (key << 16 | count) and its half.
    __device__ uint32_t next(int& half) {
        if (i < n0 && (j >= n1 || (a(i) >> 16) >= (b(j) >> 16))) { half = 0; return a(i++); }
        half = 1;
        return b(j++);
    }
};

template <int DT>
__global__ __launch_bounds__(kFT) void full_kernel(FullArgs a) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[kLdsBytes];
    __shared__ Shared sh;
    uint32_t* lds32 = reinterpret_cast<uint32_t*>(lds);
    const int tid = threadIdx.x;
    const int b = blockIdx.x, xcd = b & 7, slot = b >> 3, half = slot & 1;
    const int row = (slot >> 1) * 8 + xcd;
    if (row >= a.rows) return;
    const vi_row_params p = a.params[row];
    if (topk_route(p)) return;

    const int V = a.vocabulary, H = a.half_len;
    const int h0 = half * H, h1 = min(V, h0 + H);
    const int n_el = max(0, h1 - h0);
    const int nvec = n_el / 8, tail = n_el - nvec * 8;
    const unsigned char* rowp = static_cast<const unsigned char*>(a.logits) + (size_t(row) * size_t(a.stride) + size_t(h0)) * 2;

    // ---- issue every load of this half up front (one HBM read of the row)
    uint4 d[kFV];
#pragma unroll
    for (int i = 0; i < kFV; ++i) {
        const int v = i * kFT + tid;
        d[i] = v < nvec ? load16(rowp + size_t(v) * 16) : make_uint4(0, 0, 0, 0);
    }
    uint32_t tbits = tid < tail ? uint32_t(reinterpret_cast<const uint16_t*>(rowp)[nvec * 8 + tid]) : 0u;

    if (tid == 0) { sh.ovf_n = 0; sh.flags = 0; sh.minp_pos = 0xffffffffu; sh.found = 0; }
    const int64_t hb = a.offsets ? a.offsets[row] : 0;
    const int64_t hn = a.offsets ? a.offsets[row + 1] - hb : 0;
    const bool pen = penalties_active(p) && hn > 0 && a.histories;

    // ---- A. occurrence counts of this half, penalties in place
    if (pen) {
        for (int w = tid; w < (H + 3) / 4; w += kFT) lds32[w] = 0u;
        __syncthreads();
        const int32_t* hist = a.histories + hb;
        uint32_t* ovf_tok = lds32 + (131072 / 4);
        uint32_t* ovf_cnt = ovf_tok + kOvfMax;
        for (int64_t i = tid; i < hn; i += kFT) {
            const int32_t t = hist[i];
            if (t < 0 || t >= V) { atomicOr(&sh.flags, kHdrBadHistory); continue; }
            if (t < h0 || t >= h1) continue;
            const int off = t - h0, word = off >> 2, sh8 = (off & 3) * 8;
            uint32_t old = lds32[word];
            for (;;) {
                const uint32_t c = (old >> sh8) & 255u;
                if (c == 255u) break;
                const uint32_t prev = atomicCAS(&lds32[word], old, old + (1u << sh8));
                if (prev == old) {
                    if (c == 254u) {
                        const uint32_t k = atomicAdd(&sh.ovf_n, 1u);
                        if (k < uint32_t(kOvfMax)) ovf_tok[k] = uint32_t(t); else atomicOr(&sh.flags, kHdrError);
                    }
                    break;
                }
                old = prev;
            }
        }
        __syncthreads();
        const uint32_t n_ovf = min(sh.ovf_n, uint32_t(kOvfMax));
        if (n_ovf) {
            for (uint32_t k = tid; k < n_ovf; k += kFT) ovf_cnt[k] = 0u;
            __syncthreads();
            for (int64_t i = tid; i < hn; i += kFT) {
                const int32_t t = hist[i];
                if (t < h0 || t >= h1) continue;
                for (uint32_t k = 0; k < n_ovf; ++k)
                    if (ovf_tok[k] == uint32_t(t)) { atomicAdd(&ovf_cnt[k], 1u); break; }
            }
            __syncthreads();
        }
        auto count_of = [&](int off, uint32_t c) -> uint32_t {
            if (c != 255u) return c;
            for (uint32_t k = 0; k < n_ovf; ++k) if (ovf_tok[k] == uint32_t(h0 + off)) return ovf_cnt[k];
            return c;
        };
#pragma unroll
        for (int i = 0; i < kFV; ++i) {
            const int v = i * kFT + tid;
            if (v < nvec) {
                const uint2 cc = *reinterpret_cast<const uint2*>(lds + size_t(v) * 8);
                if (cc.x | cc.y) {
                    uint32_t w4[4] = {d[i].x, d[i].y, d[i].z, d[i].w};
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const uint32_t c = ((j < 4 ? cc.x : cc.y) >> ((j & 3) * 8)) & 255u;
                        if (c) {
                            uint32_t& w = w4[j >> 1];
                            const uint32_t bits = (j & 1) ? (w >> 16) : (w & 0xffffu);
                            if (Elem<DT>::finite_bits(bits)) {
                                const uint32_t nb = penalize_bits<DT>(bits, count_of(v * 8 + j, c), p) & 0xffffu;
                                w = (j & 1) ? ((w & 0xffffu) | (nb << 16)) : ((w & 0xffff0000u) | nb);
                            }
                        }
                    }
                    d[i] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
                }
            }
        }
        if (tid < tail) {
            const int off = nvec * 8 + tid;
            const uint32_t c = (lds32[off >> 2] >> ((off & 3) * 8)) & 255u;
            if (c && Elem<DT>::finite_bits(tbits)) tbits = penalize_bits<DT>(tbits, count_of(off, c), p) & 0xffffu;
        }
        __syncthreads();
    }

    // ---- B. key histogram (u16 counts packed in pairs) and the sorted list
    const float inv_t = 1.0f / p.temperature;
    uint32_t n_fin = 0;
    bool nonfinite = false;
    for (int w = tid; w < 32768; w += kFT) lds32[w] = 0u;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kFV; ++i) {
        if (i * kFT + tid < nvec) {
            const uint32_t w4[4] = {d[i].x, d[i].y, d[i].z, d[i].w};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t bits = (j & 1) ? (w4[j >> 1] >> 16) : (w4[j >> 1] & 0xffffu);
                if (Elem<DT>::finite_bits(bits)) {
                    const uint32_t k = key16(bits);
                    atomicAdd(&lds32[k >> 1], (k & 1u) ? 0x10000u : 1u);
                    ++n_fin;
                } else {
                    nonfinite = true;
                }
            }
        }
    }
    if (tid < tail) {
        if (Elem<DT>::finite_bits(tbits)) { const uint32_t k = key16(tbits); atomicAdd(&lds32[k >> 1], (k & 1u) ? 0x10000u : 1u); ++n_fin; }
        else nonfinite = true;
    }
    if (nonfinite) atomicOr(&sh.flags, kHdrNonfinite);
    __syncthreads();
    // thread t owns keys [64t, 64t + 64)
    uint32_t my_n = 0, my_sum = 0;
    for (int w = 0; w < 32; ++w) {
        const uint32_t x = lds32[tid * 32 + w];
        my_n += ((x & 0xffffu) != 0u) + ((x >> 16) != 0u);
        my_sum += (x & 0xffffu) + (x >> 16);
    }
    uint32_t n_list;
    const uint32_t base = block_exclusive_scan_u32<kFT>(my_n, sh.u, &n_list);
    const uint32_t tot_fin = block_sum_u32<kFT>(n_fin, sh.u);
    const uint32_t tot_sum = block_sum_u32<kFT>(my_sum, sh.u);
    uint32_t* my_list = a.lists + (size_t(row) * 2 + half) * kListMax;
    {
        uint32_t at = base;
        for (int w = 0; w < 32; ++w) {
            const uint32_t x = lds32[tid * 32 + w];
            const uint32_t k0 = uint32_t(tid * 64 + 2 * w);
            if ((x & 0xffffu) && at < uint32_t(kListMax)) my_list[at] = (k0 << 16) | (x & 0xffffu);
            at += (x & 0xffffu) != 0u;
            if ((x >> 16) && at < uint32_t(kListMax)) my_list[at] = ((k0 + 1u) << 16) | (x >> 16);
            at += (x >> 16) != 0u;
        }
    }
    if (tid == 0) {
        uint32_t f = sh.flags;
        if (tot_sum != tot_fin) f |= kHdrOverflow;  // a key held >= 65,536 logits of this half
        if (n_list > uint32_t(kListMax)) f |= kHdrOverflow;
        a.headers[size_t(row) * 2 + half] = FullHeader{n_list, tot_fin, f, 0u};
    }

    // ---- C. pair barrier (self-resetting; generation counter)
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        PairBarrier* bar = &a.barriers[row];
        const uint32_t gen = __hip_atomic_load(&bar->gen, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t arrived = __hip_atomic_fetch_add(&bar->count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (arrived == 1u) {
            __hip_atomic_store(&bar->count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_add(&bar->gen, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            uint32_t it = 0;
            while (__hip_atomic_load(&bar->gen, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) == gen) {
                __builtin_amdgcn_s_sleep(2);
                if (++it > kSpinLimit) { sh.flags |= kHdrError; break; }
            }
        }
    }
    __syncthreads();
    __threadfence();
    const FullHeader H0 = a.headers[size_t(row) * 2 + 0], H1 = a.headers[size_t(row) * 2 + 1];
    const uint32_t hflags = H0.flags | H1.flags | (sh.flags & kHdrError);
    const int n0 = int(H0.n_list), n1 = int(H1.n_list), n = n0 + n1;
    const uint32_t N_f = H0.n_finite + H1.n_finite;
    uint32_t out_flags = 0;
    if (hflags & kHdrNonfinite) out_flags |= VI_FLAG_NONFINITE;
    if (hflags & kHdrBadHistory) out_flags |= VI_FLAG_BAD_HISTORY;
    const bool fail = (hflags & (kHdrError | kHdrOverflow)) || n > kListMax;
    if (fail || N_f == 0) {
        if (half == 0 && tid == 0) {
            a.tokens[row] = fail ? -1 : V;
            if (a.uniforms) a.uniforms[row] = 0.0;
            if (a.stats) {
                vi_sample_stats s{};
                s.flags = out_flags | (fail ? VI_FLAG_ERROR : VI_FLAG_EMPTY);
                a.stats[row] = s;
            }
        }
        if (a.probs) {
            float* pr = a.probs + size_t(row) * size_t(a.probs_stride);
            for (int i = h0 + tid; i < h1; i += kFT) pr[i] = 0.0f;
        }
        return;
    }

    // ---- C'. merged cumulative counts / masses
    uint32_t* LA = lds32;
    uint32_t* LB = lds32 + n0;
    uint32_t* C = reinterpret_cast<uint32_t*>(lds + kOffC);
    double* W = reinterpret_cast<double*>(lds + kOffW);
    {
        const uint32_t* g0 = a.lists + (size_t(row) * 2 + 0) * kListMax;
        const uint32_t* g1 = a.lists + (size_t(row) * 2 + 1) * kListMax;
        for (int i = tid; i < n0; i += kFT) LA[i] = g0[i];
        for (int i = tid; i < n1; i += kFT) LB[i] = g1[i];
    }
    __syncthreads();
    Merge M{LA, LB, n0, n1, 0, 0};
    const uint32_t top_key = max(n0 ? LA[n0 - 1] >> 16 : 0u, n1 ? LB[n1 - 1] >> 16 : 0u);
    const double z0 = double(key_z<DT>(top_key, inv_t));
    const int E = (n + kFT - 1) / kFT;
    const int d0 = min(tid * E, n), d1 = min(d0 + E, n);
    uint32_t lc = 0;
    double lw = 0.0;
    M.seek(d0);
    const int mi = M.i, mj = M.j;
    for (int pos = d0; pos < d1; ++pos) {
        int hh;
        const uint32_t e = M.next(hh);
        const float z = key_z<DT>(e >> 16, inv_t);
        uint32_t cnt = e & 0xffffu;
        double w = 0.0;
        if (!isfinite(z)) { cnt = 0; atomicOr(&sh.flags, kHdrNonfinite); }
        else w = exp(double(z) - z0);
        if (p.min_p > 0.0f && w < double(p.min_p) && cnt) atomicMin(&sh.minp_pos, uint32_t(pos));
        C[pos] = lc;
        W[pos] = lw;
        lc += cnt;
        lw += double(cnt) * w;
    }
    uint32_t ctot;
    double wtot;
    const uint32_t coff = block_exclusive_scan_u32<kFT>(lc, sh.u, &ctot);
    const double woff = block_exclusive_scan_f64<kFT>(lw, sh.d, &wtot);
    for (int pos = d0; pos < d1; ++pos) { C[pos] += coff; W[pos] += woff; }
    if (tid == 0) { C[n] = ctot; W[n] = wtot; }
    __syncthreads();
    if (sh.flags & kHdrNonfinite) out_flags |= VI_FLAG_NONFINITE;
    const uint32_t Nv = C[n];

    // Parallel search: the first merged entry whose predicate holds; its
    // (pos, key, half, count, w) land in sh.sel_*.  pred(pos, C[pos], W[pos],
    // count, w) must be monotone in pos.
    auto find_first = [&](auto pred) -> bool {
        if (tid == 0) { sh.found = 0; sh.sel_pos = 0x7fffffff; }
        __syncthreads();
        Merge m2 = M;
        m2.i = mi; m2.j = mj;
        int hit = -1;
        for (int pos = d0; pos < d1 && hit < 0; ++pos) {
            int hh;
            const uint32_t e = m2.next(hh);
            const float z = key_z<DT>(e >> 16, inv_t);
            const uint32_t cnt = isfinite(z) ? (e & 0xffffu) : 0u;
            const double w = isfinite(z) ? exp(double(z) - z0) : 0.0;
            if (pred(pos, C[pos], W[pos], cnt, w)) hit = pos;
        }
        if (hit >= 0) atomicMin(reinterpret_cast<unsigned*>(&sh.sel_pos), unsigned(hit));
        __syncthreads();
        if (hit >= 0 && hit == sh.sel_pos) {
            Merge m3 = M;
            m3.seek(hit);
            int hh;
            const uint32_t e = m3.next(hh);
            const float z = key_z<DT>(e >> 16, inv_t);
            sh.sel_key = int(e >> 16);
            sh.sel_half = hh;
            sh.sel_count = isfinite(z) ? int(e & 0xffffu) : 0;
            sh.sel_w = isfinite(z) ? exp(double(z) - z0) : 0.0;
            sh.found = 1;
        }
        __syncthreads();
        return sh.found != 0;
    };

    // ---- decisions (identical in both workgroups)
    const uint32_t cap = (p.top_k > 0 && uint32_t(p.top_k) < Nv) ? uint32_t(p.top_k) : Nv;
    double s_cap = W[n];
    if (cap < Nv) {
        find_first([&](int, uint32_t c, double, uint32_t cnt, double) { return c + cnt >= cap; });
        s_cap = W[sh.sel_pos] + double(cap - C[sh.sel_pos]) * sh.sel_w;
    }
    uint32_t n_sup = cap;
    if (p.min_p > 0.0f && sh.minp_pos != 0xffffffffu) n_sup = min(n_sup, C[sh.minp_pos]);
    if (p.top_p < 1.0f) {
        const double target = double(p.top_p) * s_cap;
        if (find_first([&](int, uint32_t c, double wc, uint32_t cnt, double w) {
                if (c >= cap) return true;
                const uint32_t ce = min(cnt, cap - c);
                return wc + double(ce) * w >= target;
            })) {
            const uint32_t c = C[sh.sel_pos];
            if (c < cap) {
                const double wc = W[sh.sel_pos], w = sh.sel_w;
                const uint32_t ce = min(uint32_t(sh.sel_count), cap - c);
                // smallest i with wc + (i + 1) w >= target
                double q = (target - wc) / w;
                int i = q > 0.0 ? int(fmin(ceil(q), double(ce))) - 1 : 0;
                i = max(0, min(i, int(ce) - 1));
                while (i > 0 && wc + double(i) * w >= target) --i;
                while (i < int(ce) - 1 && wc + double(i + 1) * w < target) ++i;
                n_sup = min(n_sup, c + uint32_t(i) + 1u);
            }
        }
    }
    if (n_sup < 1u) n_sup = 1u;
    // S_n: entry holding element n_sup
    find_first([&](int, uint32_t c, double, uint32_t cnt, double) { return c + cnt >= n_sup; });
    const double s_n = W[sh.sel_pos] + double(n_sup - C[sh.sel_pos]) * sh.sel_w;
    const int pn_pos = sh.sel_pos, pn_key = sh.sel_key, pn_half = sh.sel_half;
    const uint32_t pn_take = n_sup - C[pn_pos];
    // draw
    const double u = philox_uniform(p.seed, p.lane, p.position, 0u);
    const double t = u * s_n;
    int r_pos, r_key, r_half;
    uint32_t rank;
    const bool hit = find_first([&](int, uint32_t c, double wc, uint32_t cnt, double w) {
        if (c >= n_sup) return true;
        const uint32_t ce = min(cnt, n_sup - c);
        return wc + double(ce) * w > t;
    });
    if (hit && C[sh.sel_pos] < n_sup) {
        r_pos = sh.sel_pos; r_key = sh.sel_key; r_half = sh.sel_half;
        const double wc = W[r_pos], w = sh.sel_w;
        const uint32_t ce = min(uint32_t(sh.sel_count), n_sup - C[r_pos]);
        // smallest i with wc + (i + 1) w > t
        const double q = (t - wc) / w;
        int i = q > 0.0 ? int(fmin(floor(q), double(ce - 1))) : 0;
        i = max(0, min(i, int(ce) - 1));
        while (i > 0 && wc + double(i) * w > t) --i;
        while (i < int(ce) - 1 && wc + double(i + 1) * w <= t) ++i;
        rank = uint32_t(i);
    } else {
        r_pos = pn_pos; r_key = pn_key; r_half = pn_half; rank = pn_take - 1u;
    }

    // ---- D. the owning half finds the rank-th logit of key r_key (id order)
    auto count_key = [&](const uint4& v, int key) -> uint32_t {
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
        uint32_t c = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t bits = (j & 1) ? (w4[j >> 1] >> 16) : (w4[j >> 1] & 0xffffu);
            c += (Elem<DT>::finite_bits(bits) && key16(bits) == uint32_t(key)) ? 1u : 0u;
        }
        return c;
    };
    // exclusive id-order rank, within this half, of the first logit of key `key`
    // held by (vector i, this thread): per-vector totals, then one block scan.
    uint32_t* vt = sh.u;  // reused: kFV + 1 <= kFW + 1 counters
    if (half == r_half) {
        if (tid <= kFV) vt[tid] = 0u;
        __syncthreads();
        uint32_t mine[kFV + 1];
#pragma unroll
        for (int i = 0; i < kFV; ++i) {
            mine[i] = (i * kFT + tid < nvec) ? count_key(d[i], r_key) : 0u;
            if (mine[i]) atomicAdd(&vt[i], mine[i]);
        }
        mine[kFV] = (tid < tail && Elem<DT>::finite_bits(tbits) && key16(tbits) == uint32_t(r_key)) ? 1u : 0u;
        if (mine[kFV]) atomicAdd(&vt[kFV], 1u);
        __syncthreads();
        int vi = kFV;
        uint32_t before = 0;
        {
            uint32_t acc = 0;
            for (int i = 0; i <= kFV; ++i) {
                if (rank < acc + vt[i]) { vi = i; before = acc; break; }
                acc += vt[i];
            }
        }
        uint32_t sel = 0;
#pragma unroll
        for (int i = 0; i <= kFV; ++i) if (i == vi) sel = mine[i];
        uint32_t tot;
        const uint32_t ex = block_exclusive_scan_u32<kFT>(sel, reinterpret_cast<uint32_t*>(sh.d), &tot);
        const uint32_t want = rank - before;
        if (sel && want >= ex && want < ex + sel) {
            int32_t token = -1;
            if (vi == kFV) {
                token = h0 + nvec * 8 + tid;
            } else {
                uint4 v = d[0];
#pragma unroll
                for (int i = 1; i < kFV; ++i) if (i == vi) v = d[i];
                const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
                uint32_t k = want - ex;
                for (int j = 0; j < 8; ++j) {
                    const uint32_t bits = (j & 1) ? (w4[j >> 1] >> 16) : (w4[j >> 1] & 0xffffu);
                    if (Elem<DT>::finite_bits(bits) && key16(bits) == uint32_t(r_key)) {
                        if (k == 0) { token = h0 + (vi * kFT + tid) * 8 + j; break; }
                        --k;
                    }
                }
            }
            a.tokens[row] = token;
            if (a.uniforms) a.uniforms[row] = u;
            if (a.stats) {
                vi_sample_stats s{};
                s.flags = out_flags; s.support = n_sup; s.finite = Nv; s.support_mass = s_n; s.uniform = u;
                a.stats[row] = s;
            }
        }
    }

    // ---- optional filtered distribution of this half
    if (a.probs) {
        float* pr = a.probs + size_t(row) * size_t(a.probs_stride);
        // rank of each boundary-key logit within this half, id order
        const bool boundary_half = half == pn_half;
        uint32_t running = 0;
        for (int i = 0; i <= kFV; ++i) {
            uint32_t c = 0;
            if (boundary_half) {
#pragma unroll
                for (int ii = 0; ii < kFV; ++ii) if (ii == i && i * kFT + tid < nvec) c = count_key(d[ii], pn_key);
                if (i == kFV) c = (tid < tail && Elem<DT>::finite_bits(tbits) && key16(tbits) == uint32_t(pn_key)) ? 1u : 0u;
            }
            uint32_t tot;
            uint32_t ex = block_exclusive_scan_u32<kFT>(c, sh.u, &tot);
            ex += running;
            running += tot;
            auto emit = [&](uint32_t bits, int id, uint32_t& k) {
                float pv = 0.0f;
                if (Elem<DT>::finite_bits(bits)) {
                    const uint32_t key = key16(bits);
                    bool in = key > uint32_t(pn_key);
                    if (key == uint32_t(pn_key)) {
                        if (half < pn_half) in = true;
                        else if (half == pn_half) { in = k < pn_take; ++k; }
                    }
                    const float z = key_z<DT>(key, inv_t);
                    if (in && isfinite(z)) pv = float(exp(double(z) - z0) / s_n);
                }
                pr[id] = pv;
            };
            uint32_t k = ex;
            if (i < kFV) {
                if (i * kFT + tid < nvec) {
                    uint4 v = d[0];
#pragma unroll
                    for (int ii = 1; ii < kFV; ++ii) if (ii == i) v = d[ii];
                    const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
                    for (int j = 0; j < 8; ++j) {
                        const uint32_t bits = (j & 1) ? (w4[j >> 1] >> 16) : (w4[j >> 1] & 0xffffu);
                        emit(bits, h0 + (i * kFT + tid) * 8 + j, k);
                    }
                }
            } else if (tid < tail) {
                emit(tbits, h0 + nvec * 8 + tid, k);
            }
        }
    }
}

}  // namespace

bool full_supported(int dtype, int vocabulary, int64_t stride) {
    if (dtype != VI_BF16 && dtype != VI_F16) return false;
    const int H = (((vocabulary + 1) / 2) + 63) / 64 * 64;
    return H <= kHalfMax && (stride * 2) % 16 == 0;
}

size_t full_workspace(int rows) {
    const size_t pairs = size_t(rows);
    return align_up(pairs * sizeof(PairBarrier), 256) + align_up(size_t(rows) * 2 * sizeof(FullHeader), 256) +
           align_up(size_t(rows) * 2 * kListMax * 4, 256) + 256;
}

vi_status launch_full(const SampleArgs& s, unsigned char* ws, size_t ws_bytes, hipStream_t stream) {
    if (reinterpret_cast<uintptr_t>(s.logits) % 16) return VI_ERR_UNSUPPORTED;
    Carver c(ws, ws_bytes);
    FullArgs a{};
    a.barriers = c.take<PairBarrier>(size_t(s.rows));
    a.headers = c.take<FullHeader>(size_t(s.rows) * 2);
    a.lists = c.take<uint32_t>(size_t(s.rows) * 2 * kListMax);
    if (!c.ok) return VI_ERR_WORKSPACE;
    a.logits = s.logits; a.rows = s.rows; a.vocabulary = s.vocabulary;
    a.half_len = (((s.vocabulary + 1) / 2) + 63) / 64 * 64;
    a.stride = s.stride; a.params = s.params; a.histories = s.histories; a.offsets = s.offsets;
    a.tokens = s.tokens; a.uniforms = s.uniforms; a.probs = s.probs; a.probs_stride = s.probs_stride;
    a.stats = s.stats;
    const int groups = (s.rows + 7) / 8;
    const dim3 grid(groups * 16), block(kFT);
    if (s.dtype == VI_BF16) hipLaunchKernelGGL(full_kernel<VI_BF16>, grid, block, 0, stream, a);
    else hipLaunchKernelGGL(full_kernel<VI_F16>, grid, block, 0, stream, a);
    return launch_status();
}

}  // namespace vi
