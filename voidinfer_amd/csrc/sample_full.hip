// sample_full.hip — full-vocabulary rows of the batched sampler (top_k = 0 or
// > 64): penalties, temperature, top-k / top-p / min-p over the whole
// vocabulary and the Philox inverse-CDF draw, with one HBM read of the row.
//
// Key fact used: with bf16 / fp16 logits (and penalized logits stored back in
// the same dtype) every scaled logit z = x' / T is a strictly monotone function
// of the logit's 16-bit pattern.  The multiset of z over a row is therefore
// exactly a 65,536-bin count histogram over order-preserving 16-bit keys, and
// every truncation (top-k count, top-p mass, min-p ratio) and the draw reduce to
// prefix sums over the occupied bins; the float work (one fp64 exp per bin) is
// per distinct key, not per token.
//
// Shape: each row is owned by a PAIR of 1024-thread workgroups (one per half of
// the vocabulary, both on one XCD), which keep their half of the row in
// registers (16 x 16-byte vectors per thread, plus <= 7 head / tail logits when
// the half does not start 16-byte aligned):
//   A. history -> LDS u8 occurrence counts of the half (saturating, exact side
//      table), penalties applied to the register-resident logits in place;
//   B. LDS u16 key histogram -> sorted (key, count) list published to HBM;
//   C. one pair barrier; both workgroups merge the two lists (merge path) into
//      cumulative counts / masses in LDS and take identical decisions with
//      wave-wide 64-ary searches;
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
constexpr int kVecMax = kFT * kFV;        // vectors per half
constexpr int kListMax = 8192;            // merged (key, half) entries
constexpr int kOvfMax = 512;              // history tokens with >= 255 occurrences per half
constexpr int kHB = 8;                    // history entries per thread per load round
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
// What the probs kernel needs to rebuild the filtered distribution.
struct alignas(16) RowBoundary {
    double z0, s_n;
    float inv_t;
    int32_t pn_key, pn_half;
    uint32_t pn_take, valid;
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
    float* probs;            // optional; doubles as scratch for penalized bits
    int64_t probs_stride;
    vi_sample_stats* stats;
    PairBarrier* barriers;   // [rows]
    FullHeader* headers;     // [rows][2]
    uint32_t* lists;         // [rows][2][kListMax]
    RowBoundary* bounds;     // [rows]
};

constexpr uint32_t kHdrNonfinite = 1u, kHdrBadHistory = 2u, kHdrError = 4u, kHdrOverflow = 8u;

// LDS map (bytes).  Phase A: u8 counts [0, 128 KiB) + saturated side table.
// Phase B: u16 histogram [0, 128 KiB).  Phase C: lists A|B [0, 32 KiB) (then
// cumulative counts C), merged entries M [32, 64 KiB), cumulative masses W
// [64 KiB, 128 KiB + 8), half bits after.
constexpr int kOffM = 4 * kListMax, kOffW = 8 * kListMax, kOffH = 16 * kListMax + 256;
constexpr int kLdsBytes = 131072 + 8 * kOvfMax + 1280;
static_assert(kOffH + kListMax / 8 <= kLdsBytes, "LDS map");

struct Shared {
    uint32_t u[kFW + 1];
    double d[kFW + 1];
    uint32_t ovf_n, flags, minp_pos;
    // decisions (written by wave 0)
    int32_t r_key, r_half, pn_key, pn_half;
    uint32_t rank, pn_take, n_sup, slot, slot_rank;
    double s_n, draw_u;
    uint32_t slot_tot[kFV + 2];
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

// Smallest i in [lo, hi) with pred(i) (pred monotone false -> true), or hi.
// Wave-uniform call; 64 probes per round.
template <class P>
__device__ int wave_search(int lo, int hi, P pred) {
    const int lane = lane_id();
    while (hi > lo) {
        const int n = hi - lo;
        if (n <= kWave) {
            const uint64_t m = ballot(lane < n && pred(lo + lane));
            return m ? lo + __builtin_ctzll(m) : hi;
        }
        const int step = (n + kWave - 1) / kWave;
        const int p = lo + lane * step;
        const uint64_t valid = ballot(p < hi);
        const uint64_t m = ballot(p < hi && pred(p));
        if (!m) {
            const int last = 63 - __builtin_clzll(valid);
            lo = lo + last * step + 1;
            continue;
        }
        const int f = __builtin_ctzll(m);
        if (f == 0) return lo;
        const int nlo = lo + (f - 1) * step + 1;
        hi = lo + f * step;
        lo = nlo;
        if (lo == hi) return lo;
    }
    return lo;
}

// Element j (0..7) of a 16-byte vector held as two 64-bit halves.
__device__ __forceinline__ uint32_t bits_of(uint64_t q0, uint64_t q1, int j) {
    return uint32_t(((j < 4 ? q0 : q1) >> ((j & 3) * 16)) & 0xffffu);
}

template <int DT>
__device__ __forceinline__ uint32_t count_key8(const uint4& v, uint32_t key) {
    uint32_t c = 0;
    const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t b = (j & 1) ? (w4[j >> 1] >> 16) : (w4[j >> 1] & 0xffffu);
        c += (Elem<DT>::finite_bits(b) && key16(b) == key) ? 1u : 0u;
    }
    return c;
}

template <int DT>
__global__ __launch_bounds__(kFT) void full_kernel(FullArgs a) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[kLdsBytes];
    __shared__ Shared sh;
    uint32_t* lds32 = reinterpret_cast<uint32_t*>(lds);
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const int b = blockIdx.x, xcd = b & 7, slot = b >> 3, half = slot & 1;
    const int row = (slot >> 1) * 8 + xcd;
    if (row >= a.rows) return;
    const vi_row_params p = a.params[row];
    if (topk_route(p)) return;

    const int V = a.vocabulary, H = a.half_len;
    const int h0 = half * H, h1 = min(V, h0 + H);
    const int n_el = max(0, h1 - h0);
    const int64_t g0 = int64_t(row) * a.stride + h0;     // element offset of this half
    const int head = min(n_el, int((8 - (g0 & 7)) & 7));
    const int nvec = (n_el - head) / 8, tail = n_el - head - nvec * 8;
    const uint16_t* base16 = static_cast<const uint16_t*>(a.logits) + g0;
    const unsigned char* vbase = reinterpret_cast<const unsigned char*>(base16 + head);
    const int vid0 = h0 + head;                          // token id of vector 0, element 0

    // ---- issue every load of this half up front (one HBM read of the row)
    // Branch-free: out-of-range slots re-load the half's last vector (an L2
    // hit) and are masked wherever the data is consumed (v < nvec).
    uint4 d[kFV];
    const int vlast = max(nvec - 1, 0);
    if (nvec > 0) {
#pragma unroll
        for (int i = 0; i < kFV; ++i) d[i] = load16(vbase + size_t(min(i * kFT + tid, vlast)) * 16);
    } else {
#pragma unroll
        for (int i = 0; i < kFV; ++i) d[i] = make_uint4(0, 0, 0, 0);
    }
    uint32_t hbits = tid < head ? uint32_t(base16[tid]) : 0u;
    uint32_t tbits = tid < tail ? uint32_t(base16[head + nvec * 8 + tid]) : 0u;

    if (tid == 0) { sh.ovf_n = 0; sh.flags = 0; sh.minp_pos = 0xffffffffu; }
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
        // kHB history entries per thread per round, all loads issued before any
        // is consumed (clamped indices keep them branch-free).
        const int64_t hlast = hn - 1;
        for (int64_t base = 0; base < hn; base += int64_t(kFT) * kHB) {
            int32_t t[kHB];
#pragma unroll
            for (int j = 0; j < kHB; ++j) t[j] = hist[min(base + int64_t(j) * kFT + tid, hlast)];
#pragma unroll
            for (int j = 0; j < kHB; ++j) {
                if (base + int64_t(j) * kFT + tid > hlast) continue;
                const int32_t tk = t[j];
                if (tk < 0 || tk >= V) { atomicOr(&sh.flags, kHdrBadHistory); continue; }
                if (tk < h0 || tk >= h1) continue;
                const int off = tk - h0, word = off >> 2, sh8 = (off & 3) * 8;
                uint32_t old = lds32[word];
                for (;;) {
                    const uint32_t c = (old >> sh8) & 255u;
                    if (c == 255u) break;
                    const uint32_t prev = atomicCAS(&lds32[word], old, old + (1u << sh8));
                    if (prev == old) {
                        if (c == 254u) {
                            const uint32_t k = atomicAdd(&sh.ovf_n, 1u);
                            if (k < uint32_t(kOvfMax)) ovf_tok[k] = uint32_t(tk); else atomicOr(&sh.flags, kHdrError);
                        }
                        break;
                    }
                    old = prev;
                }
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
        const unsigned char* cnt8 = lds;
        auto count_at = [&](int off) -> uint32_t {   // occurrences of token h0 + off
            const uint32_t c = cnt8[off];
            if (c != 255u) return c;
            for (uint32_t k = 0; k < n_ovf; ++k) if (ovf_tok[k] == uint32_t(h0 + off)) return ovf_cnt[k];
            return c;
        };
#pragma unroll
        for (int i = 0; i < kFV; ++i) {
            const int v = i * kFT + tid;
            if (v < nvec) {
                const int off0 = head + v * 8;
                // the 8 counts of this vector (two LDS words when the half starts aligned)
                uint64_t cc = 0;
                if ((head & 3) == 0) {
                    const uint32_t* c32 = reinterpret_cast<const uint32_t*>(cnt8 + off0);
                    cc = uint64_t(c32[0]) | (uint64_t(c32[1]) << 32);
                } else {
                    for (int j = 0; j < 8; ++j) cc |= uint64_t(cnt8[off0 + j]) << (8 * j);
                }
                if (cc) {
                    uint64_t q0 = uint64_t(d[i].x) | (uint64_t(d[i].y) << 32);
                    uint64_t q1 = uint64_t(d[i].z) | (uint64_t(d[i].w) << 32);
                    for (int j = 0; j < 8; ++j) {                     // rolled: low register use
                        if (!((cc >> (8 * j)) & 255u)) continue;
                        const uint32_t bits = bits_of(q0, q1, j);
                        if (!Elem<DT>::finite_bits(bits)) continue;
                        const uint64_t nb = penalize_bits<DT>(bits, count_at(off0 + j), p) & 0xffffu;
                        const int s = (j & 3) * 16;
                        if (j < 4) q0 = (q0 & ~(0xffffull << s)) | (nb << s);
                        else q1 = (q1 & ~(0xffffull << s)) | (nb << s);
                    }
                    d[i] = make_uint4(uint32_t(q0), uint32_t(q0 >> 32), uint32_t(q1), uint32_t(q1 >> 32));
                }
            }
        }
        if (tid < head) {
            const uint32_t c = count_at(tid);
            if (c && Elem<DT>::finite_bits(hbits)) hbits = penalize_bits<DT>(hbits, c, p) & 0xffffu;
        }
        if (tid < tail) {
            const int off = head + nvec * 8 + tid;
            const uint32_t c = count_at(off);
            if (c && Elem<DT>::finite_bits(tbits)) tbits = penalize_bits<DT>(tbits, c, p) & 0xffffu;
        }
        __syncthreads();
    }

    // ---- B. key histogram (u16 counts packed in pairs) and the sorted list
    const float inv_t = 1.0f / p.temperature;
    uint32_t n_fin = 0;
    bool nonfinite = false;
    for (int w = tid; w < 32768; w += kFT) lds32[w] = 0u;
    __syncthreads();
    auto hist_add = [&](uint32_t bits) {
        if (Elem<DT>::finite_bits(bits)) {
            const uint32_t k = key16(bits);
            atomicAdd(&lds32[k >> 1], (k & 1u) ? 0x10000u : 1u);
            ++n_fin;
        } else {
            nonfinite = true;
        }
    };
#pragma unroll
    for (int i = 0; i < kFV; ++i) {
        if (i * kFT + tid < nvec) {
            const uint32_t w4[4] = {d[i].x, d[i].y, d[i].z, d[i].w};
#pragma unroll
            for (int j = 0; j < 8; ++j) hist_add((j & 1) ? (w4[j >> 1] >> 16) : (w4[j >> 1] & 0xffffu));
        }
    }
    if (tid < head) hist_add(hbits);
    if (tid < tail) hist_add(tbits);
    if (nonfinite) atomicOr(&sh.flags, kHdrNonfinite);
    __syncthreads();
    // thread t owns keys [64t, 64t + 64)
    uint32_t my_n = 0, my_sum = 0;
#pragma unroll 2  // fully unrolled, the 32 LDS reads in flight spill the register-resident row
    for (int w = 0; w < 32; ++w) {
        const uint32_t x = lds32[tid * 32 + w];
        my_n += ((x & 0xffffu) != 0u) + ((x >> 16) != 0u);
        my_sum += (x & 0xffffu) + (x >> 16);
    }
    uint32_t n_list;
    const uint32_t lbase = block_exclusive_scan_u32<kFT>(my_n, sh.u, &n_list);
    const uint32_t tot_fin = block_sum_u32<kFT>(n_fin, sh.u);
    const uint32_t tot_sum = block_sum_u32<kFT>(my_sum, sh.u);
    uint32_t* my_list = a.lists + (size_t(row) * 2 + half) * kListMax;
    {
        uint32_t at = lbase;
#pragma unroll 2
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

    // ---- C. pair barrier (self-resetting; generation counter).  Every wave
    // drains its own list / header stores to L2 (s_waitcnt); one wave then
    // publishes with a single agent-scope release (L2 write-back) and, after
    // the partner arrived, takes a single agent-scope acquire (L1/L2
    // invalidate) on behalf of the workgroup; the spin itself polls with
    // relaxed loads so it does not invalidate caches each round.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        PairBarrier* bar = &a.barriers[row];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const uint32_t gen = __hip_atomic_load(&bar->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t arrived = __hip_atomic_fetch_add(&bar->count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (arrived == 1u) {
            __hip_atomic_store(&bar->count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_add(&bar->gen, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            uint32_t it = 0;
            while (__hip_atomic_load(&bar->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gen) {
                __builtin_amdgcn_s_sleep(1);
                if (++it > kSpinLimit) { sh.flags |= kHdrError; break; }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    const FullHeader H0 = a.headers[size_t(row) * 2 + 0], H1 = a.headers[size_t(row) * 2 + 1];
    const uint32_t hflags = H0.flags | H1.flags | (sh.flags & kHdrError);
    const int n0 = int(H0.n_list), n1 = int(H1.n_list), n = n0 + n1;
    uint32_t out_flags = 0;
    if (hflags & kHdrNonfinite) out_flags |= VI_FLAG_NONFINITE;
    if (hflags & kHdrBadHistory) out_flags |= VI_FLAG_BAD_HISTORY;
    const bool fail = (hflags & (kHdrError | kHdrOverflow)) || n > kListMax;
    if (fail || H0.n_finite + H1.n_finite == 0) {
        if (half == 0 && tid == 0) {
            a.tokens[row] = fail ? -1 : V;
            if (a.uniforms) a.uniforms[row] = 0.0;
            if (a.stats) {
                vi_sample_stats s{};
                s.flags = out_flags | (fail ? VI_FLAG_ERROR : VI_FLAG_EMPTY);
                a.stats[row] = s;
            }
            if (a.bounds) a.bounds[row] = RowBoundary{0.0, 0.0, 0.0f, -1, 0, 0u, 0u};
        }
        if (a.probs) {
            float* pr = a.probs + size_t(row) * size_t(a.probs_stride);
            for (int i = h0 + tid; i < h1; i += kFT) pr[i] = 0.0f;
        }
        return;
    }

    // ---- C'. merge: M (entries, merged order), W (exclusive masses), C (counts)
    uint32_t* LA = lds32;
    uint32_t* LB = lds32 + n0;
    uint32_t* M = reinterpret_cast<uint32_t*>(lds + kOffM);
    double* W = reinterpret_cast<double*>(lds + kOffW);
    uint32_t* HB = reinterpret_cast<uint32_t*>(lds + kOffH);
    uint32_t* C = lds32;   // reuses the list region after the merge
    {
        const uint32_t* gl0 = a.lists + (size_t(row) * 2 + 0) * kListMax;
        const uint32_t* gl1 = a.lists + (size_t(row) * 2 + 1) * kListMax;
        for (int i = tid; i < n0; i += kFT) LA[i] = gl0[i];
        for (int i = tid; i < n1; i += kFT) LB[i] = gl1[i];
        for (int i = tid; i < (n + 31) / 32; i += kFT) HB[i] = 0u;
    }
    __syncthreads();
    const uint32_t top_key = max(n0 ? LA[n0 - 1] >> 16 : 0u, n1 ? LB[n1 - 1] >> 16 : 0u);
    const double z0 = double(key_z<DT>(top_key, inv_t));
    const int E = (n + kFT - 1) / kFT;
    const int d0 = min(tid * E, n), d1 = min(d0 + E, n);
    uint32_t lc = 0;
    double lw = 0.0;
    {
        // merge path over the two lists read in descending key order (half 0 first on ties)
        auto A = [&](int k) { return LA[n0 - 1 - k]; };
        auto B = [&](int k) { return LB[n1 - 1 - k]; };
        int lo = max(0, d0 - n1), hi = min(d0, n0);
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if ((A(mid) >> 16) >= (B(d0 - 1 - mid) >> 16)) lo = mid + 1; else hi = mid;
        }
        int i = lo, j = d0 - lo;
        for (int pos = d0; pos < d1; ++pos) {
            uint32_t e;
            if (i < n0 && (j >= n1 || (A(i) >> 16) >= (B(j) >> 16))) e = A(i++);
            else { e = B(j++); atomicOr(&HB[pos >> 5], 1u << (pos & 31)); }
            const float z = key_z<DT>(e >> 16, inv_t);
            uint32_t cnt = e & 0xffffu;
            double w = 0.0;
            if (!isfinite(z) || !isfinite(z0)) { cnt = 0; atomicOr(&sh.flags, kHdrNonfinite); }
            else w = exp(double(z) - z0);
            if (p.min_p > 0.0f && cnt && w < double(p.min_p)) atomicMin(&sh.minp_pos, uint32_t(pos));
            M[pos] = (e & 0xffff0000u) | cnt;
            W[pos] = lw;
            lc += cnt;
            lw += double(cnt) * w;
        }
    }
    uint32_t ctot;
    double wtot;
    const uint32_t coff = block_exclusive_scan_u32<kFT>(lc, sh.u, &ctot);   // (barriers inside: merge done)
    const double woff = block_exclusive_scan_f64<kFT>(lw, sh.d, &wtot);
    {
        uint32_t c = coff;
        for (int pos = d0; pos < d1; ++pos) {
            W[pos] += woff;
            C[pos] = c;
            c += M[pos] & 0xffffu;
        }
    }
    if (tid == 0) { C[n] = ctot; W[n] = wtot; }
    __syncthreads();
    if (sh.flags & kHdrNonfinite) out_flags |= VI_FLAG_NONFINITE;

    // ---- decisions, identical in both workgroups (wave 0, 64-ary searches)
    if (wave == 0) {
        const uint32_t Nv = C[n];
        auto wt = [&](int pos) -> double {
            const float z = key_z<DT>(M[pos] >> 16, inv_t);
            return isfinite(z) ? exp(double(z) - z0) : 0.0;
        };
        auto cnt = [&](int pos) -> uint32_t { return M[pos] & 0xffffu; };
        const uint32_t cap = (p.top_k > 0 && uint32_t(p.top_k) < Nv) ? uint32_t(p.top_k) : Nv;
        double s_cap = W[n];
        if (cap < Nv) {
            const int pk = wave_search(0, n, [&](int pos) { return C[pos + 1] >= cap; });
            s_cap = W[pk] + double(cap - C[pk]) * wt(pk);
        }
        uint32_t n_sup = cap;
        if (p.min_p > 0.0f && sh.minp_pos != 0xffffffffu) n_sup = min(n_sup, C[sh.minp_pos]);
        if (p.top_p < 1.0f) {
            const double target = double(p.top_p) * s_cap;
            const int pt = wave_search(0, n, [&](int pos) {
                const uint32_t c = C[pos];
                if (c >= cap) return true;
                return W[pos] + double(min(cnt(pos), cap - c)) * wt(pos) >= target;
            });
            if (pt < n && C[pt] < cap) {
                const uint32_t c = C[pt];
                const double wc = W[pt], w = wt(pt);
                const uint32_t ce = min(cnt(pt), cap - c);
                // smallest i with wc + (i + 1) w >= target
                const double q = (target - wc) / w;
                int i = q > 0.0 ? int(fmin(ceil(q), double(ce))) - 1 : 0;
                i = max(0, min(i, int(ce) - 1));
                while (i > 0 && wc + double(i) * w >= target) --i;
                while (i < int(ce) - 1 && wc + double(i + 1) * w < target) ++i;
                n_sup = min(n_sup, c + uint32_t(i) + 1u);
            }
        }
        if (n_sup < 1u) n_sup = 1u;
        const int pn = wave_search(0, n, [&](int pos) { return C[pos + 1] >= n_sup; });
        const uint32_t pn_take = n_sup - C[pn];
        const double w_pn = wt(pn);
        const double s_n = W[pn] + double(pn_take) * w_pn;
        const double u = philox_uniform(p.seed, p.lane, p.position, 0u);
        const double t = u * s_n;
        int ru = wave_search(0, pn + 1, [&](int pos) {
            const uint32_t c = C[pos];
            const uint32_t ce = pos == pn ? pn_take : cnt(pos);
            return W[pos] + double(ce) * wt(pos) > t && c < n_sup;
        });
        uint32_t rank;
        if (ru <= pn) {
            const double wc = W[ru], w = wt(ru);
            const uint32_t ce = ru == pn ? pn_take : cnt(ru);
            // smallest i with wc + (i + 1) w > t
            const double q = (t - wc) / w;
            int i = q > 0.0 ? int(fmin(floor(q), double(ce - 1))) : 0;
            i = max(0, min(i, int(ce) - 1));
            while (i > 0 && wc + double(i) * w > t) --i;
            while (i < int(ce) - 1 && wc + double(i + 1) * w <= t) ++i;
            rank = uint32_t(i);
        } else {
            ru = pn;
            rank = pn_take - 1u;
        }
        if (lane == 0) {
            sh.r_key = int(M[ru] >> 16);
            sh.r_half = int((HB[ru >> 5] >> (ru & 31)) & 1u);
            sh.rank = rank;
            sh.pn_key = int(M[pn] >> 16);
            sh.pn_half = int((HB[pn >> 5] >> (pn & 31)) & 1u);
            sh.pn_take = pn_take;
            sh.n_sup = n_sup;
            sh.s_n = s_n;
            sh.draw_u = u;
            sh.slot = 0xffffffffu;
        }
    }
    if (tid < kFV + 2) sh.slot_tot[tid] = 0u;
    __syncthreads();
    const int r_half = sh.r_half;
    const uint32_t r_key = uint32_t(sh.r_key);

    // ---- D. the owning half finds the rank-th logit of key r_key (id order:
    // head slot, vector slots 0..15 (thread-major inside a slot), tail slot)
    if (half == r_half) {
        // per-slot totals
        uint32_t c_head = (tid < head && Elem<DT>::finite_bits(hbits) && key16(hbits) == r_key) ? 1u : 0u;
        uint32_t c_tail = (tid < tail && Elem<DT>::finite_bits(tbits) && key16(tbits) == r_key) ? 1u : 0u;
        if (c_head) atomicAdd(&sh.slot_tot[0], 1u);
#pragma unroll
        for (int i = 0; i < kFV; ++i) {
            const uint32_t c = (i * kFT + tid < nvec) ? count_key8<DT>(d[i], r_key) : 0u;
            if (c) atomicAdd(&sh.slot_tot[1 + i], c);
        }
        if (c_tail) atomicAdd(&sh.slot_tot[kFV + 1], 1u);
        __syncthreads();
        if (tid == 0) {
            uint32_t acc = 0;
            for (int s = 0; s < kFV + 2; ++s) {
                if (sh.rank < acc + sh.slot_tot[s]) { sh.slot = uint32_t(s); sh.slot_rank = sh.rank - acc; break; }
                acc += sh.slot_tot[s];
            }
        }
        __syncthreads();
        const int s = int(sh.slot);
        uint32_t mine = 0;
        if (s == 0) mine = c_head;
        else if (s == kFV + 1) mine = c_tail;
        else {
#pragma unroll
            for (int i = 0; i < kFV; ++i)
                if (s == 1 + i && i * kFT + tid < nvec) mine = count_key8<DT>(d[i], r_key);
        }
        uint32_t tot;
        const uint32_t ex = block_exclusive_scan_u32<kFT>(mine, sh.u, &tot);
        const uint32_t want = sh.slot_rank;
        if (mine && want >= ex && want < ex + mine) {
            int32_t token = -1;
            if (s == 0) token = h0 + tid;
            else if (s == kFV + 1) token = vid0 + nvec * 8 + tid;
            else {
                uint4 v = d[0];
#pragma unroll
                for (int i = 1; i < kFV; ++i) if (s == 1 + i) v = d[i];
                const uint64_t q0 = uint64_t(v.x) | (uint64_t(v.y) << 32), q1 = uint64_t(v.z) | (uint64_t(v.w) << 32);
                uint32_t k = want - ex;
                for (int j = 0; j < 8; ++j) {
                    const uint32_t bits = bits_of(q0, q1, j);
                    if (Elem<DT>::finite_bits(bits) && key16(bits) == r_key) {
                        if (k == 0) { token = vid0 + ((s - 1) * kFT + tid) * 8 + j; break; }
                        --k;
                    }
                }
            }
            a.tokens[row] = token;
            if (a.uniforms) a.uniforms[row] = sh.draw_u;
            if (a.stats) {
                vi_sample_stats st{};
                st.flags = out_flags; st.support = sh.n_sup; st.finite = C[n]; st.support_mass = sh.s_n;
                st.uniform = sh.draw_u;
                a.stats[row] = st;
            }
        }
    }

    // ---- optional: hand the penalized bits and the support boundary to the
    // probs kernel (probs row = scratch for the bits until it overwrites them)
    if (a.probs) {
        uint32_t* pr = reinterpret_cast<uint32_t*>(a.probs + size_t(row) * size_t(a.probs_stride));
        if (tid < head) pr[h0 + tid] = hbits;
        if (tid < tail) pr[vid0 + nvec * 8 + tid] = tbits;
#pragma unroll
        for (int i = 0; i < kFV; ++i) {
            const int v = i * kFT + tid;
            if (v < nvec) {
                const uint32_t w4[4] = {d[i].x, d[i].y, d[i].z, d[i].w};
#pragma unroll
                for (int j = 0; j < 8; ++j) pr[vid0 + v * 8 + j] = (j & 1) ? (w4[j >> 1] >> 16) : (w4[j >> 1] & 0xffffu);
            }
        }
        if (half == 0 && tid == 0)
            a.bounds[row] = RowBoundary{z0, sh.s_n, inv_t, sh.pn_key, sh.pn_half, sh.pn_take, 1u};
    }
}

// Filtered distribution of the full-route rows: one workgroup per (half, row)
// walks its half in id order, ranks the boundary-key logits with block scans
// and writes w / S_n for the support (0 elsewhere).  Test / diagnostics path.
template <int DT>
__global__ __launch_bounds__(kFT) void full_probs_kernel(const vi_row_params* params, int rows, int vocabulary,
                                                       int half_len, float* probs, int64_t probs_stride,
                                                       const RowBoundary* bounds) {
    __shared__ uint32_t tmp[kFW + 1];
    const int half = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    if (row >= rows || topk_route(params[row])) return;
    const RowBoundary bd = bounds[row];
    const int h0 = half * half_len, h1 = min(vocabulary, h0 + half_len);
    float* pr = probs + size_t(row) * size_t(probs_stride);
    if (!bd.valid) {
        for (int i = h0 + tid; i < h1; i += kFT) pr[i] = 0.0f;
        return;
    }
    const uint32_t pkey = uint32_t(bd.pn_key);
    uint32_t running = 0;
    for (int c0 = h0; c0 < h1; c0 += kFT * 8) {
        const int e0 = c0 + tid * 8;
        uint32_t bits[8];
        uint32_t mine = 0;
        for (int j = 0; j < 8; ++j) {
            const int e = e0 + j;
            bits[j] = e < h1 ? reinterpret_cast<const uint32_t*>(pr)[e] : 0x7fffu;
            if (e < h1 && half == bd.pn_half && Elem<DT>::finite_bits(bits[j]) && key16(bits[j]) == pkey) ++mine;
        }
        uint32_t tot;
        uint32_t k = block_exclusive_scan_u32<kFT>(mine, tmp, &tot) + running;
        running += tot;
        for (int j = 0; j < 8; ++j) {
            const int e = e0 + j;
            if (e >= h1) break;
            float pv = 0.0f;
            if (Elem<DT>::finite_bits(bits[j])) {
                const uint32_t key = key16(bits[j]);
                bool in = key > pkey;
                if (key == pkey) {
                    if (half < bd.pn_half) in = true;
                    else if (half == bd.pn_half) { in = k < bd.pn_take; ++k; }
                }
                const float z = Elem<DT>::decode(unkey16(key)) * bd.inv_t;
                if (in && isfinite(z)) pv = float(exp(double(z) - bd.z0) / bd.s_n);
            }
            pr[e] = pv;
        }
    }
}

}  // namespace

bool full_supported(int dtype, int vocabulary, int64_t stride) {
    if (dtype != VI_BF16 && dtype != VI_F16) return false;
    const int H = (((vocabulary + 1) / 2) + 63) / 64 * 64;
    return H <= kVecMax * 8 && stride >= vocabulary;
}

size_t full_workspace(int rows) {
    return align_up(size_t(rows) * sizeof(PairBarrier), 256) + align_up(size_t(rows) * 2 * sizeof(FullHeader), 256) +
           align_up(size_t(rows) * 2 * kListMax * 4, 256) + align_up(size_t(rows) * sizeof(RowBoundary), 256) + 256;
}

vi_status launch_full(const SampleArgs& s, unsigned char* ws, size_t ws_bytes, hipStream_t stream) {
    if (reinterpret_cast<uintptr_t>(s.logits) % 16) return VI_ERR_UNSUPPORTED;
    Carver c(ws, ws_bytes);
    FullArgs a{};
    a.barriers = c.take<PairBarrier>(size_t(s.rows));
    a.headers = c.take<FullHeader>(size_t(s.rows) * 2);
    a.lists = c.take<uint32_t>(size_t(s.rows) * 2 * kListMax);
    a.bounds = c.take<RowBoundary>(size_t(s.rows));
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
    vi_status st = launch_status();
    if (st != VI_OK || !s.probs) return st;
    const dim3 pgrid(2, s.rows);
    if (s.dtype == VI_BF16)
        hipLaunchKernelGGL(full_probs_kernel<VI_BF16>, pgrid, block, 0, stream, s.params, s.rows, s.vocabulary,
                           a.half_len, s.probs, s.probs_stride, a.bounds);
    else
        hipLaunchKernelGGL(full_probs_kernel<VI_F16>, pgrid, block, 0, stream, s.params, s.rows, s.vocabulary,
                           a.half_len, s.probs, s.probs_stride, a.bounds);
    return launch_status();
}

}  // namespace vi
