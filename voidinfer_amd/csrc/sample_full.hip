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
// the half does not start 16-byte aligned).
//
// Penalties (dense path, histories <= 32,768 tokens): the history is loaded
// first and turned into a bitmap of the half's history tokens, a rank prefix
// per bitmap word and a rank-ordered u16 count array; each thread takes 32
// consecutive ranks, gathers those logits from the (cache-hot) row and keeps
// (count, logit) in registers.  The streaming histogram then skips every
// history token (one bitmap byte per 8 logits) and the dense pass penalizes the
// gathered tokens, 32 per thread with no divergence, and adds them.  Longer
// histories take the general path: a u8 occurrence table of the half and
// penalties applied to the register-resident logits in place.
//
//   B. LDS u16 key histogram -> sorted (key, count) list published to HBM;
//   C. one pair barrier; both workgroups merge the two lists (merge path) into
//      cumulative counts / masses in LDS and take identical decisions with
//      wave-wide 64-ary searches;
//   D. the half owning the drawn (key, rank) finds the token in its registers
//      (history tokens: from the dense registers).
// The pair barrier spins on an agent-scope counter with an iteration cap, so a
// missing partner becomes VI_FLAG_ERROR, never a hang.  Roofline: HBM,
// V x 2 + L x 4 bytes per row (logits once, history once per pair via L2).
#include <math.h>

#include "penalty_state.h"
#include "vi_device.h"
#include "vi_internal.h"

namespace vi {
namespace {

constexpr int kFT = 1024;                 // threads per workgroup
constexpr int kFW = kFT / kWave;          // waves per workgroup
constexpr int kFV = 16;                   // 16-byte vectors per thread
constexpr int kVecMax = kFT * kFV;        // vectors per half
constexpr int kListMax = 65536;           // list slots of one half: 16 wave segments of 4096 keys
constexpr uint32_t kSpinLimit = 1u << 22;
// general path
constexpr int kOvfMax = 512;              // history tokens with >= 255 occurrences per half
constexpr int kHB = 8;                    // history entries per thread per load round
// dense path
constexpr int kHistMax = 32768;           // history tokens per row
// one-pass history counting: a second-occurrence bitmap and a list of the
// offsets of further occurrences, in the P16 region [64 KiB, 128 KiB) until the
// exchange overwrites it
constexpr int kList3 = 4096;              // list capacity; a longer list takes a second pass
constexpr int kOffB2 = 65536, kOffL3 = kOffB2 + 4 * 4096;
constexpr int kHT = kHistMax / kFT;       // history tokens per thread
// state route: the first kStage repeat-list entries are staged in LDS [64, 96) KiB
// (the one-pass counting's region, unused on this route) before the row arrives
constexpr int kStage = 4096, kOffStage = kOffB2;
constexpr int kDR = kHistMax / kFT;       // dense ranks (distinct history tokens) per thread
constexpr int kBmapWords = kVecMax * 8 / 32;

constexpr int kCoarse = 256;              // coarse bins of 256 keys
constexpr int kNfBins = 4;                // coarse bins at each end holding non-finite keys
// What a half publishes for its partner: header, its sorted (key << 16 | count)
// list's first index per coarse bin, and per coarse bin the count of valid
// logits and their mass sum count * exp(z(key) - z(top_key)).
struct alignas(16) HalfSummary {
    uint32_t n_list, n_finite, flags, top_key;   // top_key: largest valid key, ~0u if none
    uint32_t first[kCoarse], end[kCoarse];       // list slots of each coarse bin's entries
    uint32_t ccnt[kCoarse];                      // valid logits of the bin
    uint32_t bref[kCoarse];                      // the bin's largest valid key (its mass reference)
    double cmass[kCoarse];                       // sum of count * exp(z(key) - z(bref))
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
    unsigned char* pstate;   // per-lane penalty states instead of histories (or null)
    PenaltyLayout pl;
    int record;              // append the sampled token to the lane's state
    int32_t* tokens;
    double* uniforms;
    float* probs;            // optional; doubles as scratch for penalized bits
    int64_t probs_stride;
    vi_sample_stats* stats;
    PairBarrier* barriers;   // [rows]
    HalfSummary* summaries;  // [rows][2]
    uint32_t* lists;         // [rows][2][kListMax]
    RowBoundary* bounds;     // [rows]
    uint16_t* dense;         // [rows][2][kHistMax] penalized history-token logits by rank
};

constexpr uint32_t kHdrNonfinite = 1u, kHdrBadHistory = 2u, kHdrError = 4u, kHdrOverflow = 8u;

// LDS map (bytes).  u16 key histogram [0, 128 KiB); merge: lists A|B (then
// cumulative counts C) [0, 32 KiB), merged entries M [32, 64 KiB), exclusive
// masses W [64, 128 KiB).  Dense path: u16 rank-ordered counts [0, 64 KiB)
// before the histogram, history bitmap and rank prefix above 128 KiB for the
// whole kernel.  General path: u8 occurrence table [0, 128 KiB) before the
// histogram, saturated-token side table above it.
// decisions (after the histogram): coarse tables of both halves, coarse
// prefix, one 256-key window
constexpr int kOffDM = 2048, kOffDF = kOffDM + 4096, kOffPC = kOffDF + 16 * kCoarse;
constexpr int kOffPM = kOffPC + 4 * (kCoarse + 4), kOffWC = kOffPM + 8 * (kCoarse + 4);
constexpr int kOffWW = kOffWC + 8 * kCoarse, kOffWN = kOffWW + 8 * kCoarse, kOffWM = kOffWN + 4 * (kCoarse + 4);
constexpr int kOffDecEnd = kOffWM + 8 * (kCoarse + 4);
constexpr int kOffBmap = 131072;
constexpr int kOffPref = kOffBmap + 4 * (kBmapWords + 4);
constexpr int kLdsDense = kOffPref + 2 * kBmapWords;
constexpr int kOffP = 24576;              // D: penalized history bits by rank (u16), filled during the
                                          // decisions (past their tables), read by the owner
constexpr int kOffML = kOffP + 2 * kHistMax;   // D: history tokens matching the drawn key
constexpr int kMatchMax = 2048;
static_assert(kOffML + 4 * kMatchMax <= 131072, "owner LDS");
static_assert(4 * kFT <= kOffP, "owner candidate masks below the penalized bits");
constexpr int kLdsGeneral = 131072 + 8 * kOvfMax;
static_assert(kOffDecEnd <= kOffP && kOffDM % 8 == 0 && kOffPM % 8 == 0 && kOffWW % 8 == 0 && kOffWM % 8 == 0, "LDS map");
static_assert(kHistMax / 2 * 4 <= 131072, "dense counts");
static_assert(kOffL3 + 4 * kList3 <= 131072 && kHistMax * 2 <= kOffB2, "one-pass history counting");

struct Shared {
    uint32_t u[kFW + 1];
    double d[kFW + 1];
    uint32_t ovf_n, flags, top1;
    // decisions (written by wave 0)
    int32_t r_key, r_half, pn_key, pn_half;
    uint32_t rank, pn_take, n_sup, slot, slot_rank, ctot;
    double s_n, draw_u;
    uint32_t slot_tot[kFV + 2];
    uint32_t n_sum, n_fin, n_match, n3, wcount[kFW];
    uint32_t first[kCoarse], bend[kCoarse];   // this half's list slots of each coarse bin
};

// Orders one wave's LDS accesses around an exchange between its lanes (a
// wave's LDS operations execute in order; this keeps the compiler from moving
// them across).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int NT>
__device__ __forceinline__ double block_exclusive_scan_f64(double v, double* tmp, double* total) {
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    const double x = wave_incl_scan_f64(v);
    if (lane == kWave - 1) tmp[wave] = x;
    __syncthreads();
    if (wave == 0) {   // scan of the wave totals in wave 0
        const double t = lane < NT / kWave ? tmp[lane] : 0.0;
        const double it = wave_incl_scan_f64(t);
        const double ex = __shfl_up(it, 1, kWave);
        if (lane < NT / kWave) tmp[lane] = lane == 0 ? 0.0 : ex;
        if (lane == NT / kWave - 1) tmp[NT / kWave] = it;
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
__device__ __forceinline__ int wave_search(int lo, int hi, P pred) {
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

// The 16-bit patterns whose order key is `key`, for pattern compares in place
// of computing keys: key16 is one-to-one on finite patterns except that -0
// shares +0's key.  Both halves of each word hold the pattern (t2; alt2 also
// admits -0 for the key of zero); nothing matches a non-finite key or 0x7fff
// (the key only -0 would have before the fold): valid = false.
struct KeyPattern {
    uint32_t t2, alt2;
    bool valid;
};
template <int DT>
__device__ __forceinline__ KeyPattern key_pattern(uint32_t key) {
    if (Elem<DT>::nonfinite_key(key) || key == 0x7fffu) return KeyPattern{0u, 0u, false};
    const uint32_t t = unkey16(key);
    return KeyPattern{t | (t << 16), t == 0u ? 0x80008000u : t | (t << 16), true};
}
template <int DT>
__device__ __forceinline__ bool has_key(uint32_t b, const KeyPattern& k) {
    return k.valid && (b == (k.t2 & 0xffffu) || b == (k.alt2 & 0xffffu));
}

// Bit j set: element j of the vector is finite and has order key `key`, two
// elements per 32-bit word.
template <int DT>
__device__ __forceinline__ uint32_t match_mask8(const uint4& v, const KeyPattern& kp) {
    const uint32_t t2 = kp.t2, alt = kp.alt2;
    const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
    uint32_t m = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t x = w4[q] ^ t2, y = w4[q] ^ alt;
        const uint32_t lo = ((x & 0xffffu) == 0u) | ((y & 0xffffu) == 0u);
        const uint32_t hi = ((x >> 16) == 0u) | ((y >> 16) == 0u);
        m |= (lo << (2 * q)) | (hi << (2 * q + 1));
    }
    return kp.valid ? m : 0u;
}

typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

// A lane state's sticky flags as this kernel's header bits.
__device__ __forceinline__ uint32_t state_flags(const unsigned char* lstate) {
    const uint32_t f = reinterpret_cast<const PenaltyHeader*>(lstate)->flags;
    return ((f & VI_FLAG_BAD_HISTORY) ? kHdrBadHistory : 0u) | ((f & VI_FLAG_ERROR) ? kHdrError : 0u);
}

template <int DT, bool kDense>
__global__ __launch_bounds__(kFT) void full_kernel(FullArgs a) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[kDense ? kLdsDense : kLdsGeneral];
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

    if (tid == 0) { sh.ovf_n = 0; sh.flags = 0; sh.top1 = 0; sh.n_sum = 0; sh.n_fin = 0; }
    // penalties from the lane's penalty state (bitmaps and hash) or from its history
    const unsigned char* lstate = a.pstate ? a.pstate + size_t(row) * a.pl.lane_bytes : nullptr;
    const int64_t hb = (!lstate && a.offsets) ? a.offsets[row] : 0;
    const int64_t hn = (!lstate && a.offsets) ? a.offsets[row + 1] - hb : 0;
    const bool pen = penalties_active(p) && (lstate || (hn > 0 && a.histories));
    const int32_t* hist = (pen && !lstate) ? a.histories + hb : nullptr;
    // state route: this half's presence bitmap words 4 * tid .. 4 * tid + 3 and
    // repeat-list entries q * kFT + tid (the first kStage, zero past the list's
    // end), requested before the row: they are consumed first, and a wave's
    // loads complete in the order they were issued
    uint32_t sb1[4] = {0u, 0u, 0u, 0u};
    uint2 le[kStage / kFT];
    if constexpr (kDense) {
        if (pen && lstate) {
            const uint32_t* b1 = reinterpret_cast<const uint32_t*>(lstate + a.pl.off_b1) + (h0 >> 5);
            const uint2* list = reinterpret_cast<const uint2*>(lstate + a.pl.off_list);
            const int nw = (n_el + 31) >> 5;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int w = 4 * tid + q;
                if (w < nw) sb1[q] = b1[w];
            }
#pragma unroll
            for (int q = 0; q < kStage / kFT; ++q) {
                const int k = q * kFT + tid;
                le[q] = k < a.pl.slots ? list[k] : make_uint2(0u, 0u);
            }
        }
    }

    // ---- issue every load of this half up front (one HBM read of the row)
    // Branch-free: out-of-range slots re-load the half's last vector (an L2
    // hit) and are masked wherever the data is consumed (v < nvec).
    // (dense path with a history: vectors kFV/2 .. kFV-1 are requested after
    // the history work, which keeps the history and the row in registers together
    // within the 128-VGPR budget)
    uint4 d[kFV];
    const int vlast = max(nvec - 1, 0);
    auto load_vectors = [&](int i0, int i1) {
#pragma unroll
        for (int i = 0; i < kFV; ++i)
            if (i >= i0 && i < i1)
                d[i] = nvec > 0 ? load16_cached(vbase + size_t(min(i * kFT + tid, vlast)) * 16) : make_uint4(0, 0, 0, 0);
    };
    load_vectors(0, kFV);
    uint32_t hbits = tid < head ? uint32_t(base16[tid]) : 0u;
    uint32_t tbits = tid < tail ? uint32_t(base16[head + nvec * 8 + tid]) : 0u;

    // Flag bits of the half's tokens off0 .. off0 + 7 (bit j: token h0 + off0 + j
    // is in the history), read from the LDS bitmap; dense path only.
    auto flags8_lds = [&](int off0) -> uint32_t {
        if constexpr (kDense) {
            const uint32_t* bmap = reinterpret_cast<const uint32_t*>(lds + kOffBmap);
            const int w = off0 >> 5, s = off0 & 31;
            const uint64_t pr = uint64_t(bmap[w]) | (uint64_t(bmap[w + 1]) << 32);
            return uint32_t(pr >> s) & 0xffu;
        } else {
            return 0u;
        }
    };
    // the same for this thread's 16 vectors, kept in registers (8 bits each)
    uint32_t vfl[kFV / 4] = {0u, 0u, 0u, 0u};
    bool fl_head = false, fl_tail = false;
    auto vflags = [&](int i) -> uint32_t { return (vfl[i >> 2] >> (8 * (i & 3))) & 0xffu; };
    // Vector slot i of this thread after the histogram: the dense path reads it
    // again (an L2 / MALL hit; history tokens are taken from the dense ranks,
    // so the raw bits are what is wanted), which frees the registers the row
    // occupied while streaming; the general path kept it, penalized, in d[].
    auto row_vec = [&](int i) -> uint4 {
        if constexpr (kDense) return nvec > 0 ? load16_cached(vbase + size_t(min(i * kFT + tid, vlast)) * 16) : make_uint4(0, 0, 0, 0);
        else return d[i];
    };

    // ---- A (dense). bitmap of the half's history tokens, exclusive rank
    // prefix per bitmap word, rank-ordered entries (offset << 15 | count) in
    // LDS; then the history tokens' logits are gathered (consecutive lanes take
    // consecutive ranks: nearby tokens) and penalized into registers, rank
    // k * kFT + tid in slot k.
    uint32_t n_flag = 0;
    uint32_t dkeep[kDR / 2] = {};   // dense path: penalized bits of ranks k * kFT + tid, two per register
    // the history tokens' penalized logits by rank: this half's slice of the
    // workspace (written once, read back from L2; not kept in registers)
    uint16_t* dpen = kDense ? a.dense + (size_t(row) * 2 + half) * kHistMax : nullptr;
    // fn(rank, off) for every history token of this thread's 4 bitmap words
    // (rows with penalties only: the bitmap is not built otherwise)
    auto walk_words = [&](auto&& fn) {
        if constexpr (kDense) {
            if (!pen) return;
            const uint32_t* bmap = reinterpret_cast<const uint32_t*>(lds + kOffBmap);
            const uint16_t* pref = reinterpret_cast<const uint16_t*>(lds + kOffPref);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int w = 4 * tid + q;
                uint32_t bits = bmap[w];
                uint32_t rank = pref[w];
                while (bits) {
                    const int bpos = __builtin_ctz(bits);
                    bits &= bits - 1u;
                    fn(rank++, w * 32 + bpos);
                }
            }
        }
    };
    // fn(token) for each of the row's first kHistMax history tokens; the history
    // is read in rounds of kHR tokens per thread (bounded registers)
    auto for_history = [&](auto&& fn) {
        constexpr int kHR = 8;
        const int hl = int(min(hn, int64_t(kHistMax)));   // (32-bit offsets: one VGPR per load)
#pragma unroll
        for (int r0 = 0; r0 < kHT; r0 += kHR) {
            if (r0 * kFT >= hl) break;   // (uniform)
            int32_t t[kHR];
#pragma unroll
            for (int j = 0; j < kHR; ++j) t[j] = hist[min((r0 + j) * kFT + tid, hl - 1)];
#pragma unroll
            for (int j = 0; j < kHR; ++j)
                if ((r0 + j) * kFT + tid < hl) fn(t[j]);
        }
    };
    if constexpr (kDense) {
        if (pen) {
            uint32_t* bmap = reinterpret_cast<uint32_t*>(lds + kOffBmap);
            uint16_t* pref = reinterpret_cast<uint16_t*>(lds + kOffPref);
            // One history pass: a bitmap of first occurrences, a second bitmap of
            // second occurrences and a short list of the offsets of all further
            // occurrences, in the P16 region (free until the exchange); a long list
            // falls back to a second pass over the history.
            uint32_t* bmap2 = lds32 + kOffB2 / 4;
            uint32_t* list3 = lds32 + kOffL3 / 4;
            if (tid == 0) sh.n3 = 0u;
            if (lstate) {   // the state's bitmap (the last word masked to the half), the staged list
                const int nw = (n_el + 31) >> 5;
                const uint32_t lastm = (n_el & 31) ? (1u << (n_el & 31)) - 1u : ~0u;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int w = 4 * tid + q;
                    bmap[w] = sb1[q] & (w == nw - 1 ? lastm : ~0u);
                }
                if (tid < 4) bmap[kBmapWords + tid] = 0u;
                uint2* stage = reinterpret_cast<uint2*>(lds + kOffStage);
#pragma unroll
                for (int q = 0; q < kStage / kFT; ++q) stage[q * kFT + tid] = le[q];
                if (tid == 0) atomicOr(&sh.flags, state_flags(lstate));
            } else {
                for (int w = tid; w < kBmapWords + 4; w += kFT) bmap[w] = 0u;
                for (int w = tid; w < kBmapWords; w += kFT) bmap2[w] = 0u;
            }
            __syncthreads();
            if (tid == 0 && hn > kHistMax) atomicOr(&sh.flags, kHdrError);   // callers promise hn <= max_history
            if (!lstate) {
                // rounds of kHR tokens per thread; each stage's LDS atomics of a
                // round are issued together (their results are awaited once)
                constexpr int kHR = 8;
                const int hl = int(min(hn, int64_t(kHistMax)));
#pragma unroll
                for (int r0 = 0; r0 < kHT; r0 += kHR) {
                    if (r0 * kFT >= hl) break;   // (uniform)
                    int32_t t[kHR];
#pragma unroll
                    for (int j = 0; j < kHR; ++j) t[j] = hist[min((r0 + j) * kFT + tid, hl - 1)];
                    uint32_t in = 0, dup = 0, dup2 = 0;
#pragma unroll
                    for (int j = 0; j < kHR; ++j) {
                        if ((r0 + j) * kFT + tid >= hl) continue;
                        if (t[j] < 0 || t[j] >= V) atomicOr(&sh.flags, kHdrBadHistory);
                        else if (t[j] >= h0 && t[j] < h1) in |= 1u << j;
                    }
                    uint32_t old[kHR];
#pragma unroll
                    for (int j = 0; j < kHR; ++j) {
                        const int off = t[j] - h0;
                        old[j] = ((in >> j) & 1u) ? atomicOr(&bmap[off >> 5], 1u << (off & 31)) : 0u;
                    }
#pragma unroll
                    for (int j = 0; j < kHR; ++j) dup |= ((old[j] >> ((t[j] - h0) & 31)) & ((in >> j) & 1u)) << j;
                    if (dup) {
#pragma unroll
                        for (int j = 0; j < kHR; ++j) {
                            const int off = t[j] - h0;
                            old[j] = ((dup >> j) & 1u) ? atomicOr(&bmap2[off >> 5], 1u << (off & 31)) : 0u;
                        }
#pragma unroll
                        for (int j = 0; j < kHR; ++j) dup2 |= ((old[j] >> ((t[j] - h0) & 31)) & ((dup >> j) & 1u)) << j;
                        while (dup2) {
                            const int j = __builtin_ctz(dup2);
                            dup2 &= dup2 - 1u;
                            const uint32_t k = atomicAdd(&sh.n3, 1u);
                            if (k < uint32_t(kList3)) list3[k] = uint32_t(t[j] - h0);
                        }
                    }
                }
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < kFV; ++i) {
                const int v = i * kFT + tid;
                if (v < nvec) vfl[i >> 2] |= flags8_lds(head + v * 8) << (8 * (i & 3));
            }
            fl_head = tid < head && (flags8_lds(tid) & 1u);
            fl_tail = tid < tail && (flags8_lds(head + nvec * 8 + tid) & 1u);
            // thread t owns bitmap words 4t .. 4t + 3
            uint32_t c4[4], s4 = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) { c4[k] = __builtin_popcount(bmap[4 * tid + k]); s4 += c4[k]; }
            uint32_t ex = block_exclusive_scan_u32<kFT>(s4, sh.u, &n_flag);
            if (n_flag > uint32_t(kHistMax)) {   // (uniform; state route only) more distinct tokens than
                // the dense ranks hold: the row fails, and the rest runs as if without history
                if (tid == 0) atomicOr(&sh.flags, kHdrError);
                n_flag = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) { bmap[4 * tid + k] = 0u; c4[k] = 0; }
#pragma unroll
                for (int k = 0; k < kFV / 4; ++k) vfl[k] = 0u;
                fl_head = fl_tail = false;
                ex = 0;
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) { pref[4 * tid + k] = uint16_t(ex); ex += c4[k]; }
            __syncthreads();
            // u16 occurrence counts by rank, C16 = [0, 64 KiB) (a count reaches at
            // most kHistMax = 32,768: no carry between the packed halves)
            const uint32_t n3 = sh.n3;
            if (n3 <= uint32_t(kList3)) {   // (uniform) counts from the bitmaps, then the list, by rank
                uint16_t* c16 = reinterpret_cast<uint16_t*>(lds);
                if (lstate) {   // count 1 by rank, then the repeat list's counts (>= 2) of this half's tokens
                    walk_words([&](uint32_t rank, int off) { c16[rank] = uint16_t(1u); });
                    __syncthreads();
                    auto put = [&](uint2 e) {
                        const int off = int(e.x) - h0;
                        if (e.y < 2u || off < 0 || off >= n_el) return;
                        const int w = off >> 5;
                        if (!((bmap[w] >> (off & 31)) & 1u) || e.y > 0xffffu) {   // inconsistent / too many
                            atomicOr(&sh.flags, kHdrError);
                            return;
                        }
                        c16[pref[w] + __builtin_popcount(bmap[w] & ((1u << (off & 31)) - 1u))] = uint16_t(e.y);
                    };
                    const uint2* stage = reinterpret_cast<const uint2*>(lds + kOffStage);
                    for (int k = tid; k < kStage; k += kFT) put(stage[k]);
                    const int nrep = int(min(reinterpret_cast<const PenaltyHeader*>(lstate)->nrep, uint32_t(a.pl.slots)));
                    const uint2* list = reinterpret_cast<const uint2*>(lstate + a.pl.off_list);
                    for (int k = kStage + tid; k < nrep; k += kFT) put(list[k]);
                } else {
                    walk_words([&](uint32_t rank, int off) { c16[rank] = uint16_t(1u + ((bmap2[off >> 5] >> (off & 31)) & 1u)); });
                }
                __syncthreads();
                for (uint32_t k = tid; k < n3; k += kFT) {
                    const int off = int(list3[k]), w = off >> 5;
                    const uint32_t rank = pref[w] + __builtin_popcount(bmap[w] & ((1u << (off & 31)) - 1u));
                    atomicAdd(&lds32[rank >> 1], (rank & 1u) ? 0x10000u : 1u);
                }
            } else {   // a second pass over the history (L2 hits now)
                for (int w = tid; w < kHistMax / 2; w += kFT) lds32[w] = 0u;
                __syncthreads();
                for_history([&](int32_t t) {
                    if (t < h0 || t >= h1) return;
                    const int off = t - h0, w = off >> 5;
                    const uint32_t rank = pref[w] + __builtin_popcount(bmap[w] & ((1u << (off & 31)) - 1u));
                    atomicAdd(&lds32[rank >> 1], (rank & 1u) ? 0x10000u : 1u);
                });
            }
            __syncthreads();   // the bitmaps and the list are read before the exchange overwrites them
            // the history tokens' logits by rank, P16 = [64 KiB, 128 KiB), written by
            // the threads holding them (a vector's history tokens have consecutive ranks)
            uint16_t* P16 = reinterpret_cast<uint16_t*>(lds + 65536);
            auto rank_of = [&](int off) -> uint32_t {
                const int w = off >> 5;
                return pref[w] + __builtin_popcount(bmap[w] & ((1u << (off & 31)) - 1u));
            };
#pragma unroll
            for (int i = 0; i < kFV; ++i) {
                const uint32_t fl = vflags(i);
                if (fl) {
                    const uint32_t r0 = rank_of(head + (i * kFT + tid) * 8);
                    const uint32_t w4[4] = {d[i].x, d[i].y, d[i].z, d[i].w};
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        if ((fl >> j) & 1u)
                            P16[r0 + __builtin_popcount(fl & ((1u << j) - 1u))] =
                                uint16_t((j & 1) ? (w4[j >> 1] >> 16) : (w4[j >> 1] & 0xffffu));
                }
            }
            if (fl_head) P16[rank_of(tid)] = uint16_t(hbits);
            if (fl_tail) P16[rank_of(head + nvec * 8 + tid)] = uint16_t(tbits);
            __syncthreads();
            // penalized, rank k * kFT + tid into slot k (ranks past n_flag skipped:
            // n_flag is uniform)
#pragma unroll
            for (int k = 0; k < kDR; ++k) {
                const uint32_t r = uint32_t(k) * kFT + tid;
                if (uint32_t(k) * kFT >= n_flag) break;
                if (r < n_flag) {
                    const uint32_t bits = P16[r];
                    const uint32_t c = (lds32[r >> 1] >> (16 * (r & 1u))) & 0xffffu;
                    const uint32_t pb = Elem<DT>::finite_bits(bits) ? penalize_bits<DT>(bits, c, p) & 0xffffu : bits;
                    dpen[r] = uint16_t(pb);
                    dkeep[k >> 1] |= pb << (16 * (k & 1));
                }
            }
            __syncthreads();   // entries read before the histogram overwrites them
        }
    }

    // ---- A (general). occurrence counts of this half, penalties in place
    if constexpr (!kDense) {
        if (pen) {
            for (int w = tid; w < (H + 3) / 4; w += kFT) lds32[w] = 0u;
            __syncthreads();
            uint32_t* ovf_tok = lds32 + (131072 / 4);
            uint32_t* ovf_cnt = ovf_tok + kOvfMax;
            // kHB history entries per thread per round, all loads issued before any
            // is consumed (clamped indices keep them branch-free).
            // (32-bit offsets, one VGPR per load; a row's history is < 2^31 tokens)
            const int hlast = int(min(hn, int64_t(0x7fffffff))) - 1;
            if (tid == 0 && hn > 0x7fffffff) atomicOr(&sh.flags, kHdrError);
            for (int base = 0; base <= hlast; base += kFT * kHB) {
                int32_t t[kHB];
#pragma unroll
                for (int j = 0; j < kHB; ++j) t[j] = hist[min(base + j * kFT + tid, hlast)];
#pragma unroll
                for (int j = 0; j < kHB; ++j) {
                    if (base + j * kFT + tid > hlast) continue;
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
                for (int i = tid; i <= hlast; i += kFT) {
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
                        // visit only the elements with a count
                        uint64_t nz = (cc | (cc >> 4)) & 0x0f0f0f0f0f0f0f0full;
                        nz = (nz | (nz >> 2)) & 0x0303030303030303ull;
                        nz = (nz | (nz >> 1)) & 0x0101010101010101ull;
                        while (nz) {
                            const int j = __builtin_ctzll(nz) >> 3;
                            nz &= nz - 1u;
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
    }

    // ---- B. key histogram (u16 counts packed in pairs, key k in word k >> 1).
    // Every logit is counted under its order key, non-finite ones included (their
    // keys form the ends of the key range and are split off at compaction);
    // history tokens (dense path) count 0 here and are added by the dense pass.
    const float inv_t = 1.0f / p.temperature;
    for (int w = tid; w < 32768; w += kFT) lds32[w] = 0u;
    __syncthreads();
    auto hist_key = [&](uint32_t k, bool skip) {
        atomicAdd(&lds32[k >> 1], skip ? 0u : ((k & 1u) ? 0x10000u : 1u));
    };
    // both logits of a 32-bit word: key16 on the two halves at once (without
    // key16's -0 -> +0 fold: -0 lands on key 0x7fff, folded into 0x8000 below)
    auto hist_word = [&](uint32_t w, uint32_t skip2) {
        const uint32_t s2 = (w >> 15) & 0x00010001u;
        const uint32_t k2 = w ^ ((s2 * 0x7fffu) | 0x80008000u);
        hist_key(k2 & 0xffffu, skip2 & 1u);
        hist_key(k2 >> 16, skip2 & 2u);
    };
#pragma unroll
    for (int i = 0; i < kFV; ++i) {
        const int v = i * kFT + tid;
        if (v < nvec) {
            const uint32_t fl = vflags(i);
            hist_word(d[i].x, fl);
            hist_word(d[i].y, fl >> 2);
            hist_word(d[i].z, fl >> 4);
            hist_word(d[i].w, fl >> 6);
        }
    }
    if (tid < head) hist_key(key16(hbits), fl_head);
    if (tid < tail) hist_key(key16(tbits), fl_tail);
    if constexpr (kDense) {
        // the history tokens, penalized (ranks k * kFT + tid, kept in registers)
#pragma unroll
        for (int k = 0; k < kDR; ++k) {
            if (uint32_t(k) * kFT >= n_flag) break;
            if (uint32_t(k) * kFT + tid < n_flag) hist_key(key16((dkeep[k >> 1] >> (16 * (k & 1))) & 0xffffu), false);
        }
    }
    __syncthreads();
    if (tid == 0) {   // -0 counts as +0 (key 0x7fff is only ever -0)
        const uint32_t x = lds32[0x7fff >> 1];
        lds32[0x7fff >> 1] = x & 0xffffu;
        lds32[0x8000 >> 1] += x >> 16;
    }
    __syncthreads();
    // ---- B'. compaction and this half's summary.  Wave w owns the coarse bins
    // w, w + 16, w + 32, ... (256 keys = 128 histogram words each; neighbouring
    // bins go to different waves, which spreads a narrow key range over the
    // block).  It reads a bin as two 64-word rows (lane = word: no bank
    // conflicts), writes the bin's (key << 16 | count) entries in ascending key
    // order to its own 4096-entry segment of the half's list (slots from
    // ballots) and sums the bin's valid count and its mass relative to the
    // bin's largest valid key (bref).  A listed key whose scaled logit
    // z = x' / T is not finite is not valid: it is neither counted nor weighted
    // (the reference drops such logits).
    uint32_t* my_list = a.lists + (size_t(row) * 2 + half) * kListMax;
    HalfSummary* my_summary = a.summaries + size_t(row) * 2 + half;
    {
        uint32_t my_sum = 0, my_nf = 0;
        uint32_t at = uint32_t(wave) * 4096u;                 // (wave-uniform) next list slot
        uint32_t v_first = 0, v_end = 0, v_cnt = 0, v_ref = 0;   // lane b: bin b * 16 + wave
        double v_mass = 0.0;
        uint32_t wtop1 = 0;                                    // largest valid key + 1
        bool bad_z = false;
        constexpr int kBU = kDense ? 4 : 1;   // bins read ahead (the general path keeps its row live)
#pragma unroll
        for (int b0 = 0; b0 < kCoarse / kFW; b0 += kBU) {
            uint32_t xs[2 * kBU];
#pragma unroll
            for (int u = 0; u < 2 * kBU; ++u) xs[u] = lds32[((b0 + u / 2) * kFW + wave) * 128 + (u & 1) * 64 + lane];
#pragma unroll
            for (int ub = 0; ub < kBU; ++ub) {
                const int bb = b0 + ub, bin = bb * kFW + wave;
                uint32_t cnt[4];   // keys kb + 2 lane + {0, 1} (row 0) and kb + 128 + 2 lane + {0, 1} (row 1)
                cnt[0] = xs[2 * ub] & 0xffffu; cnt[1] = xs[2 * ub] >> 16;
                cnt[2] = xs[2 * ub + 1] & 0xffffu; cnt[3] = xs[2 * ub + 1] >> 16;
                my_sum += cnt[0] + cnt[1] + cnt[2] + cnt[3];
                if (bin < kNfBins || bin >= kCoarse - kNfBins) {   // the non-finite logits' keys
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t k = uint32_t(bin * 256) + 2u * uint32_t(lane) + uint32_t(e & 1) + 128u * uint32_t(e >> 1);
                        if (Elem<DT>::nonfinite_key(k)) { my_nf += cnt[e]; cnt[e] = 0u; }
                    }
                }
                uint64_t bal[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) bal[e] = ballot(cnt[e] != 0u);
                const uint32_t first = at;
                const uint32_t kb = uint32_t(bin * 256);
                if (bal[0] | bal[1] | bal[2] | bal[3]) {
                    // list slots: row 0's entries, then row 1's (ascending keys)
                    const uint32_t r0 = at + __builtin_amdgcn_mbcnt_hi(uint32_t(bal[0] >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(bal[0]), 0u)) +
                                        __builtin_amdgcn_mbcnt_hi(uint32_t(bal[1] >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(bal[1]), 0u));
                    const uint32_t at1 = at + uint32_t(__builtin_popcountll(bal[0]) + __builtin_popcountll(bal[1]));
                    const uint32_t r1 = at1 + __builtin_amdgcn_mbcnt_hi(uint32_t(bal[2] >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(bal[2]), 0u)) +
                                        __builtin_amdgcn_mbcnt_hi(uint32_t(bal[3] >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(bal[3]), 0u));
                    uint32_t key[4];
                    key[0] = kb + 2u * uint32_t(lane); key[1] = key[0] + 1u;
                    key[2] = key[0] + 128u; key[3] = key[0] + 129u;
                    if (cnt[0]) put_agent(&my_list[r0], (key[0] << 16) | cnt[0]);
                    if (cnt[1]) put_agent(&my_list[r0 + (cnt[0] != 0u)], (key[1] << 16) | cnt[1]);
                    if (cnt[2]) put_agent(&my_list[r1], (key[2] << 16) | cnt[2]);
                    if (cnt[3]) put_agent(&my_list[r1 + (cnt[2] != 0u)], (key[3] << 16) | cnt[3]);
                    at = at1 + uint32_t(__builtin_popcountll(bal[2]) + __builtin_popcountll(bal[3]));
                    // validity and the bin's reference key (largest valid key)
                    float z[4];
                    uint64_t vb[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        z[e] = key_z<DT>(key[e], inv_t);
                        const bool ok = cnt[e] != 0u && isfinite(z[e]);
                        bad_z |= cnt[e] != 0u && !ok;
                        if (!ok) cnt[e] = 0u;
                        vb[e] = ballot(ok);
                    }
                    uint32_t ref1 = 0;   // largest valid key + 1 (0: none)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (vb[e]) ref1 = max(ref1, kb + 2u * uint32_t(63 - __builtin_clzll(vb[e])) + uint32_t(e & 1) + 128u * uint32_t(e >> 1) + 1u);
                    if (ref1) {
                        const double zr = double(key_z<DT>(ref1 - 1u, inv_t));
                        double m = 0.0;
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (cnt[e]) m += double(cnt[e]) * exp(double(z[e]) - zr);
                        const uint32_t bc = wave_sum_u32(cnt[0] + cnt[1] + cnt[2] + cnt[3]);
                        const double bm = wave_sum_f64(m);
                        if (lane == bb) { v_cnt = bc; v_mass = bm; v_ref = ref1 - 1u; }
                        wtop1 = max(wtop1, ref1);
                    }
                }
                if (lane == bb) { v_first = first; v_end = at; }
            }
        }
        if (lane < kCoarse / kFW) {
            const int bin = lane * kFW + wave;
            put_agent(&my_summary->first[bin], v_first);
            put_agent(&my_summary->end[bin], v_end);
            put_agent(&my_summary->ccnt[bin], v_cnt);
            put_agent(&my_summary->bref[bin], v_ref);
            put_agent(&my_summary->cmass[bin], v_mass);
        }
        const uint32_t wsum = wave_sum_u32(my_sum), wnf = wave_sum_u32(my_nf);
        const uint32_t wfin = wsum - wnf;
        if (bad_z || wnf) atomicOr(&sh.flags, kHdrNonfinite);
        if (lane == 0) {
            sh.wcount[wave] = at - uint32_t(wave) * 4096u;
            atomicAdd(&sh.n_sum, wsum);
            atomicAdd(&sh.n_fin, wfin);
            if (wtop1) atomicMax(&sh.top1, wtop1);
        }
    }

    // ---- C. pair barrier (self-resetting; generation counter).  The list and
    // the summary were written through (put_agent); every wave drains its own
    // stores (s_waitcnt), one thread writes the header, drains it and arrives;
    // the partner's data is then read with agent-scope loads (get_agent), so
    // neither L2 is written back or invalidated.  The spin polls with relaxed
    // loads.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        uint32_t f = sh.flags;
        if (sh.n_sum != uint32_t(n_el)) f |= kHdrOverflow;  // a key held >= 65,536 logits of this half
        uint32_t n_list = 0;
        for (int w = 0; w < kFW; ++w) n_list += sh.wcount[w];
        put_agent(&my_summary->n_list, n_list);
        put_agent(&my_summary->n_finite, uint32_t(sh.n_fin));
        put_agent(&my_summary->flags, f);
        put_agent(&my_summary->top_key, sh.top1 ? sh.top1 - 1u : 0xffffffffu);
        PairBarrier* bar = &a.barriers[row];
        handoff_stores_done();
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
        handoff_acquire();
    }
    __syncthreads();
    const HalfSummary* S0 = a.summaries + size_t(row) * 2;
    const HalfSummary* S1 = S0 + 1;
    const uint32_t hflags = get_agent(&S0->flags) | get_agent(&S1->flags) | (sh.flags & kHdrError);
    const uint32_t tk0 = get_agent(&S0->top_key), tk1 = get_agent(&S1->top_key);
    uint32_t out_flags = 0;
    if (hflags & kHdrNonfinite) out_flags |= VI_FLAG_NONFINITE;
    if (hflags & kHdrBadHistory) out_flags |= VI_FLAG_BAD_HISTORY;
    const bool fail = (hflags & (kHdrError | kHdrOverflow)) != 0u;
    if (fail || (tk0 == 0xffffffffu && tk1 == 0xffffffffu)) {   // error, or no valid logit
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

    // ---- C'. decisions, identical in both workgroups.  Coarse bins in
    // descending key order (q = 255 - bin) carry merged counts and masses; a
    // boundary is located on them, then resolved inside its bin on a 256-key
    // window built from both halves' lists.
    const uint32_t tkmax = (tk0 == 0xffffffffu) ? tk1 : (tk1 == 0xffffffffu ? tk0 : max(tk0, tk1));
    const double z0 = double(key_z<DT>(tkmax, inv_t));
    uint32_t* DC = lds32;                                             // [2][256] valid counts
    double* DM = reinterpret_cast<double*>(lds + kOffDM);              // [2][256] masses (own reference)
    uint32_t* DF = reinterpret_cast<uint32_t*>(lds + kOffDF);          // [2][first, end][256] list slots
    uint32_t* PC = reinterpret_cast<uint32_t*>(lds + kOffPC);          // [257] count before q
    double* PM = reinterpret_cast<double*>(lds + kOffPM);              // [257] mass before q
    uint32_t* WC = reinterpret_cast<uint32_t*>(lds + kOffWC);          // [2][256] window counts by slot
    double* WW = reinterpret_cast<double*>(lds + kOffWW);              // [256] slot weight
    uint32_t* WN = reinterpret_cast<uint32_t*>(lds + kOffWN);          // [257] window count before slot
    double* WM = reinterpret_cast<double*>(lds + kOffWM);              // [257] window mass before slot
    for (int i = tid; i < 2 * kCoarse; i += kFT) {   // masses rescaled to z0
        const HalfSummary* Sh = i < kCoarse ? S0 : S1;
        const int c = i & (kCoarse - 1);
        const uint32_t cc = get_agent(&Sh->ccnt[c]);
        DC[i] = cc;
        DM[i] = cc ? get_agent(&Sh->cmass[c]) * exp(double(key_z<DT>(get_agent(&Sh->bref[c]), inv_t)) - z0) : 0.0;
    }
    for (int i = tid; i < 2 * kCoarse; i += kFT) {
        const HalfSummary* Sh = i < kCoarse ? S0 : S1;
        const int c = i & (kCoarse - 1);
        DF[2 * (i & ~(kCoarse - 1)) + c] = get_agent(&Sh->first[c]);
        DF[2 * (i & ~(kCoarse - 1)) + kCoarse + c] = get_agent(&Sh->end[c]);
    }
    __syncthreads();
    if (wave != 0) {
        // meanwhile the other waves bring this half's penalized history bits by
        // rank into LDS for the owner search (16-byte copies; the slice holds
        // kHistMax entries, so rounding n_flag up stays inside it)
        if constexpr (kDense) {
            if (pen) {
                const uint4* src = reinterpret_cast<const uint4*>(dpen);
                uint4* dst = reinterpret_cast<uint4*>(lds + kOffP);
                const int n16 = int((n_flag + 7u) >> 3);
                for (int i = tid - kWave; i < n16; i += kFT - kWave) dst[i] = src[i];
            }
        }
    } else {
        // merged coarse prefix: lane l owns q = 4l .. 4l + 3
        {
            uint32_t cq[4];
            double mq[4];
            uint32_t cs = 0;
            double ms = 0.0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int c = kCoarse - 1 - (4 * lane + e);
                cq[e] = DC[c] + DC[kCoarse + c];
                mq[e] = DM[c] + DM[kCoarse + c];
                cs += cq[e];
                ms += mq[e];
            }
            const uint32_t cx = wave_incl_scan_u32(cs);
            const double mx = wave_incl_scan_f64(ms);
            uint32_t cb = cx - cs;
            double mb = mx - ms;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                PC[4 * lane + e] = cb;
                PM[4 * lane + e] = mb;
                cb += cq[e];
                mb += mq[e];
            }
            if (lane == kWave - 1) { PC[kCoarse] = cb; PM[kCoarse] = mb; }
        }
        wave_lds_sync();
        const uint32_t Nv = PC[kCoarse];
        const double S = PM[kCoarse];
        // first q in [0, 256) with pred(q) (monotone), or 256
        auto coarse_find = [&](auto pred) -> int {
            uint32_t m4 = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) m4 |= pred(4 * lane + e) ? (1u << e) : 0u;
            const uint64_t b = ballot(m4 != 0u);
            if (!b) return kCoarse;
            const int l = __builtin_ctzll(b);
            const uint32_t ml = uint32_t(__builtin_amdgcn_readlane(int(m4), l));
            return 4 * l + __builtin_ctz(ml);
        };
        int win_q = -1;
        // window of coarse position q: slot j <-> key (255 - q) * 256 + 255 - j
        auto load_window = [&](int q) {
            if (q == win_q) return;
            win_q = q;
            const int c = kCoarse - 1 - q;
#pragma unroll
            for (int e = 0; e < 4; ++e) { WC[4 * lane + e] = 0u; WC[kCoarse + 4 * lane + e] = 0u; }
            wave_lds_sync();
            // both halves' entries of the bin (<= 256 each): all loads in flight at once
            uint32_t ent[8];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t* gl = a.lists + (size_t(row) * 2 + h) * kListMax;
                const uint32_t f0 = DF[2 * kCoarse * h + c], f1 = DF[2 * kCoarse * h + kCoarse + c];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t i = f0 + uint32_t(lane + k * kWave);
                    ent[h * 4 + k] = i < f1 ? get_agent(&gl[i]) : 0u;
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (ent[u]) WC[(u >> 2) * kCoarse + (255u - ((ent[u] >> 16) & 255u))] = ent[u] & 0xffffu;
            wave_lds_sync();
            uint32_t cq[4];
            double mq[4];
            uint32_t cs = 0;
            double ms = 0.0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = 4 * lane + e;
                const uint32_t key = uint32_t(c * 256 + 255 - j);
                const float z = key_z<DT>(key, inv_t);
                const bool ok = isfinite(z);
                cq[e] = ok ? WC[j] + WC[kCoarse + j] : 0u;
                if (!ok) { WC[j] = 0u; WC[kCoarse + j] = 0u; }
                const double w = ok ? exp(double(z) - z0) : 0.0;
                WW[j] = w;
                mq[e] = double(cq[e]) * w;
                cs += cq[e];
                ms += mq[e];
            }
            const uint32_t cx = wave_incl_scan_u32(cs);
            const double mx = wave_incl_scan_f64(ms);
            uint32_t cb = cx - cs;
            double mb = mx - ms;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                WN[4 * lane + e] = cb;
                WM[4 * lane + e] = mb;
                cb += cq[e];
                mb += mq[e];
            }
            if (lane == kWave - 1) { WN[kCoarse] = cb; WM[kCoarse] = mb; }
            wave_lds_sync();
        };
        auto slot_cnt = [&](int j) -> uint32_t { return WN[j + 1] - WN[j]; };
        // position of the n-th element (1-based) in sorted order: coarse q, slot j, count before the slot
        struct Pos { int q, j; uint32_t before; double mass_before; };
        auto locate = [&](uint32_t nth) -> Pos {
            const int q = coarse_find([&](int qq) { return PC[qq + 1] >= nth; });
            load_window(q);
            const int j = coarse_find([&](int jj) { return PC[q] + WN[jj + 1] >= nth; });
            return Pos{q, j, PC[q] + WN[j], PM[q] + WM[j]};
        };
        const uint32_t cap = (p.top_k > 0 && uint32_t(p.top_k) < Nv) ? uint32_t(p.top_k) : Nv;
        double s_cap = S;
        if (cap < Nv) {
            const Pos ps = locate(cap);
            s_cap = ps.mass_before + double(cap - ps.before) * WW[ps.j];
        }
        uint32_t n_sup = cap;
        if (p.min_p > 0.0f) {
            // smallest key with w(key) >= min_p (w grows with the key); elements
            // below it are cut (the reference cuts at the first w < min_p)
            const double mp = double(p.min_p);
            auto ok = [&](int key) {
                const float z = key_z<DT>(uint32_t(key), inv_t);
                return isfinite(z) && exp(double(z) - z0) >= mp;
            };
            const int km = wave_search(0, int(tkmax) + 1, [&](int key) { return ok(key); });
            uint32_t n_minp = 0;
            if (km <= int(tkmax)) {
                const int q = kCoarse - 1 - (km >> 8);
                load_window(q);
                n_minp = PC[q] + WN[255 - (km & 255) + 1];
            }
            n_sup = min(n_sup, n_minp);
        }
        if (p.top_p < 1.0f) {
            const double target = double(p.top_p) * s_cap;
            const int q = coarse_find([&](int qq) { return PM[qq + 1] >= target || PC[qq + 1] >= cap; });
            if (q < kCoarse) {
                load_window(q);
                const int j = coarse_find([&](int jj) { return PM[q] + WM[jj + 1] >= target || PC[q] + WN[jj + 1] >= cap; });
                const uint32_t c = PC[q] + WN[j];
                if (j < kCoarse && c < cap) {
                    const double wc = PM[q] + WM[j], w = WW[j];
                    const uint32_t ce = min(slot_cnt(j), cap - c);
                    if (wc + double(ce) * w >= target) {
                        // smallest i with wc + (i + 1) w >= target
                        const double qq = (target - wc) / w;
                        int i = qq > 0.0 ? int(fmin(ceil(qq), double(ce))) - 1 : 0;
                        i = max(0, min(i, int(ce) - 1));
                        while (i > 0 && wc + double(i) * w >= target) --i;
                        while (i < int(ce) - 1 && wc + double(i + 1) * w < target) ++i;
                        n_sup = min(n_sup, c + uint32_t(i) + 1u);
                    }
                }
            }
        }
        if (n_sup < 1u) n_sup = 1u;
        const Pos pn = locate(n_sup);
        const uint32_t pn_take = n_sup - pn.before;
        const double s_n = pn.mass_before + double(pn_take) * WW[pn.j];
        const uint32_t pn_key = uint32_t((kCoarse - 1 - pn.q) * 256 + 255 - pn.j);
        const uint32_t pn_c0 = WC[pn.j];
        const double u = philox_uniform(p.seed, p.lane, p.position, 0u);
        const double t = u * s_n;
        // draw: first position (among the first n_sup) whose cumulative mass exceeds t
        int rq = coarse_find([&](int qq) { return PM[qq + 1] > t || PC[qq + 1] >= n_sup; });
        if (rq > pn.q) rq = pn.q;
        load_window(rq);
        int rj = coarse_find([&](int jj) { return PM[rq] + WM[jj + 1] > t || PC[rq] + WN[jj + 1] >= n_sup; });
        uint32_t rank;
        {
            const bool at_pn = rq == pn.q && rj >= pn.j;
            if (at_pn) rj = pn.j;
            const double wc = PM[rq] + WM[rj], w = WW[rj];
            const uint32_t ce = at_pn ? pn_take : slot_cnt(rj);
            if (wc + double(ce) * w > t) {
                // smallest i with wc + (i + 1) w > t
                const double qq = (t - wc) / w;
                int i = qq > 0.0 ? int(fmin(floor(qq), double(ce - 1))) : 0;
                i = max(0, min(i, int(ce) - 1));
                while (i > 0 && wc + double(i) * w > t) --i;
                while (i < int(ce) - 1 && wc + double(i + 1) * w <= t) ++i;
                rank = uint32_t(i);
            } else {   // rounding left t beyond the support: its last element
                rank = ce - 1u;
            }
        }
        const uint32_t r_c0 = WC[rj];
        if (lane == 0) {
            sh.r_key = int((kCoarse - 1 - rq) * 256 + 255 - rj);
            sh.r_half = rank < r_c0 ? 0 : 1;
            sh.rank = rank < r_c0 ? rank : rank - r_c0;
            sh.pn_key = int(pn_key);
            sh.pn_half = pn_take <= pn_c0 ? 0 : 1;
            sh.pn_take = pn_take <= pn_c0 ? pn_take : pn_take - pn_c0;
            sh.n_sup = n_sup;
            sh.s_n = s_n;
            sh.draw_u = u;
            sh.ctot = Nv;
            sh.slot = 0xffffffffu;
        }
    }
    if (tid < kFV + 2) sh.slot_tot[tid] = 0u;
    if (tid == 0) sh.n_match = 0u;
    __syncthreads();
    const uint16_t* P = reinterpret_cast<const uint16_t*>(lds + kOffP);   // dense path: filled above
    const int r_half = sh.r_half;
    const uint32_t r_key = uint32_t(sh.r_key);

    // ---- D. the owning half finds the rank-th logit of key r_key (id order:
    // head slot, vector slots 0..15 (thread-major inside a slot), tail slot)
    if (half == r_half) {
        uint32_t* fmask = lds32;   // [kFT] history-token candidates per owning thread
        fmask[tid] = 0u;
        const KeyPattern rkp = key_pattern<DT>(r_key);
        const uint32_t c_head = (tid < head && !fl_head && has_key<DT>(hbits, rkp));
        const uint32_t c_tail = (tid < tail && !fl_tail && has_key<DT>(tbits, rkp));
        // per-slot counts summed over the wave with shuffles: one LDS atomic
        // per wave and slot instead of one per thread
        auto wave_add = [&](int s2, uint32_t c) {
            c = wave_sum_u32(c);
            if (lane == 0 && c) atomicAdd(&sh.slot_tot[s2], c);
        };
        wave_add(0, c_head);
        uint32_t vm[kFV / 4] = {0u, 0u, 0u, 0u};   // candidate masks of the 16 vector slots
#pragma unroll
        for (int i0 = 0; i0 < kFV; i0 += kFV) {   // all 16 vectors in flight
            uint4 rv[kFV];
#pragma unroll
            for (int u = 0; u < kFV; ++u) rv[u] = row_vec(i0 + u);
#pragma unroll
            for (int u = 0; u < kFV; ++u) {
                const int i = i0 + u;
                const uint32_t m = i * kFT + tid < nvec ? match_mask8<DT>(rv[u], rkp) & ~vflags(i) : 0u;
                vm[i >> 2] |= m << (8 * (i & 3));
                wave_add(1 + i, __builtin_popcount(m));
            }
        }
        wave_add(kFV + 1, c_tail);
        // slot, owning thread and element index of the half's token h0 + off
        auto place = [&](int off, int* owner, int* j) -> int {
            if (off < head) { *owner = off; *j = 0; return 0; }
            const int rel = off - head;
            if (rel >= nvec * 8) { *owner = rel - nvec * 8; *j = 0; return kFV + 1; }
            const int v = rel >> 3;
            *owner = v & (kFT - 1);
            *j = rel & 7;
            return 1 + v / kFT;
        };
        // history tokens with key r_key: a scan of the rank-ordered penalized
        // logits (their token offsets found by rank only for the rare matches),
        // kept in a short list for the second step
        uint32_t* ML = reinterpret_cast<uint32_t*>(lds + kOffML);
        if constexpr (kDense) {
            if (pen) {
                const uint32_t* bmap = reinterpret_cast<const uint32_t*>(lds + kOffBmap);
                const uint16_t* pref = reinterpret_cast<const uint16_t*>(lds + kOffPref);
                for (uint32_t r = tid; r < n_flag; r += kFT) {
                    const uint32_t pb = P[r];
                    if (!has_key<DT>(pb, rkp)) continue;
                    int lo = 0, hi = kBmapWords;             // last word with pref <= r
                    while (lo < hi) {
                        const int mid = (lo + hi) >> 1;
                        if (uint32_t(pref[mid]) <= r) lo = mid + 1; else hi = mid;
                    }
                    const int w = lo - 1;
                    uint32_t bits = bmap[w];
                    for (uint32_t k = r - pref[w]; k > 0; --k) bits &= bits - 1u;
                    const int off = w * 32 + __builtin_ctz(bits);
                    int o, j;
                    atomicAdd(&sh.slot_tot[place(off, &o, &j)], 1u);
                    const uint32_t at = atomicAdd(&sh.n_match, 1u);
                    if (at < uint32_t(kMatchMax)) ML[at] = uint32_t(off);
                }
            }
        }
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
        if (sh.n_match <= uint32_t(kMatchMax)) {
            for (uint32_t m = tid; m < sh.n_match; m += kFT) {
                int o, j;
                if (place(int(ML[m]), &o, &j) == s) atomicOr(&fmask[o], 1u << j);
            }
        } else {   // (a list overflow: walk the bitmap)
            walk_words([&](uint32_t rank, int off) {
                const uint32_t pb = P[rank];
                int o, j;
                if (has_key<DT>(pb, rkp) && place(off, &o, &j) == s) atomicOr(&fmask[o], 1u << j);
            });
        }
        __syncthreads();
        uint32_t cm = fmask[tid];   // candidate bits (element j of this thread's group in slot s)
        if (s == 0) cm |= c_head;
        else if (s == kFV + 1) cm |= c_tail;
        else {
#pragma unroll
            for (int i = 0; i < kFV; ++i)
                if (s == 1 + i) cm |= (vm[i >> 2] >> (8 * (i & 3))) & 0xffu;
        }
        const uint32_t mine = __builtin_popcount(cm);
        uint32_t tot;
        const uint32_t ex = block_exclusive_scan_u32<kFT>(mine, sh.u, &tot);
        const uint32_t want = sh.slot_rank;
        if (s < 0 || s > kFV + 1) {
            if (tid == 0) {   // counts disagree with the histogram: cannot happen for consistent inputs
                a.tokens[row] = -1;
                if (a.uniforms) a.uniforms[row] = sh.draw_u;
                if (a.stats) {
                    vi_sample_stats st{};
                    st.flags = out_flags | VI_FLAG_ERROR;
                    a.stats[row] = st;
                }
            }
        } else if (mine && want >= ex && want < ex + mine) {
            uint32_t m = cm;
            for (uint32_t k = want - ex; k > 0; --k) m &= m - 1u;
            const int j = __builtin_ctz(m);
            int32_t token;
            if (s == 0) token = h0 + tid;
            else if (s == kFV + 1) token = vid0 + nvec * 8 + tid;
            else token = vid0 + ((s - 1) * kFT + tid) * 8 + j;
            a.tokens[row] = token;
            if (a.record) {   // both halves have read the state (they passed the pair barrier)
                const LaneState ls = lane_state(a.pstate + size_t(row) * a.pl.lane_bytes, a.pl);
                state_publish(ls, state_apply(ls, a.pl, V, token, 1));
            }
            if (a.uniforms) a.uniforms[row] = sh.draw_u;
            if (a.stats) {
                vi_sample_stats st{};
                st.flags = out_flags; st.support = sh.n_sup; st.finite = sh.ctot; st.support_mass = sh.s_n;
                st.uniform = sh.draw_u;
                a.stats[row] = st;
            }
        }
    }

    // ---- optional: hand the penalized bits and the support boundary to the
    // probs kernel (probs row = scratch for the bits until it overwrites them)
    if (a.probs) {
        uint32_t* pr = reinterpret_cast<uint32_t*>(a.probs + size_t(row) * size_t(a.probs_stride));
        if (tid < head && !fl_head) pr[h0 + tid] = hbits;
        if (tid < tail && !fl_tail) pr[vid0 + nvec * 8 + tid] = tbits;
#pragma unroll
        for (int i = 0; i < kFV; ++i) {
            const int v = i * kFT + tid;
            if (v < nvec) {
                const uint32_t fl = vflags(i);
                const uint4 dv = row_vec(i);
                const uint32_t w4[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (!((fl >> j) & 1u)) pr[vid0 + v * 8 + j] = (j & 1) ? (w4[j >> 1] >> 16) : (w4[j >> 1] & 0xffffu);
            }
        }
        walk_words([&](uint32_t rank, int off) { pr[h0 + off] = P[rank]; });
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

template <int DT>
void launch_full_dt(const FullArgs& a, bool dense, dim3 grid, hipStream_t stream) {
    if (dense) hipLaunchKernelGGL((full_kernel<DT, true>), grid, dim3(kFT), 0, stream, a);
    else hipLaunchKernelGGL((full_kernel<DT, false>), grid, dim3(kFT), 0, stream, a);
}

}  // namespace

bool full_supported(int dtype, int vocabulary, int64_t stride) {
    if (dtype != VI_BF16 && dtype != VI_F16) return false;
    const int H = (((vocabulary + 1) / 2) + 63) / 64 * 64;
    return H <= kVecMax * 8 && stride >= vocabulary;
}

size_t full_workspace(int rows) {
    return align_up(size_t(rows) * sizeof(PairBarrier), 256) + align_up(size_t(rows) * 2 * sizeof(HalfSummary), 256) +
           align_up(size_t(rows) * 2 * kListMax * 4, 256) + align_up(size_t(rows) * sizeof(RowBoundary), 256) +
           align_up(size_t(rows) * 2 * kHistMax * 2, 256) + 256;
}

vi_status launch_full(const SampleArgs& s, unsigned char* ws, size_t ws_bytes, hipStream_t stream) {
    if (reinterpret_cast<uintptr_t>(s.logits) % 16) return VI_ERR_UNSUPPORTED;
    Carver c(ws, ws_bytes);
    FullArgs a{};
    a.barriers = c.take<PairBarrier>(size_t(s.rows));
    a.summaries = c.take<HalfSummary>(size_t(s.rows) * 2);
    a.lists = c.take<uint32_t>(size_t(s.rows) * 2 * kListMax);
    a.bounds = c.take<RowBoundary>(size_t(s.rows));
    a.dense = c.take<uint16_t>(size_t(s.rows) * 2 * kHistMax);
    if (!c.ok) return VI_ERR_WORKSPACE;
    a.logits = s.logits; a.rows = s.rows; a.vocabulary = s.vocabulary;
    a.half_len = (((s.vocabulary + 1) / 2) + 63) / 64 * 64;
    a.stride = s.stride; a.params = s.params; a.histories = s.histories; a.offsets = s.offsets;
    if (s.pstate) {
        a.pstate = s.pstate; a.pl = s.playout; a.record = s.record;
    }
    a.tokens = s.tokens; a.uniforms = s.uniforms; a.probs = s.probs; a.probs_stride = s.probs_stride;
    a.stats = s.stats;
    const int groups = (s.rows + 7) / 8;
    const dim3 grid(groups * 16);
    // histories up to kHistMax tokens: dense penalty path; longer: general path
    const bool dense = s.pstate || s.max_history <= kHistMax;
    if (s.dtype == VI_BF16) launch_full_dt<VI_BF16>(a, dense, grid, stream);
    else launch_full_dt<VI_F16>(a, dense, grid, stream);
    vi_status st = launch_status();
    if (st != VI_OK || !s.probs) return st;
    const dim3 pgrid(2, s.rows), block(kFT);
    if (s.dtype == VI_BF16)
        hipLaunchKernelGGL(full_probs_kernel<VI_BF16>, pgrid, block, 0, stream, s.params, s.rows, s.vocabulary,
                           a.half_len, s.probs, s.probs_stride, a.bounds);
    else
        hipLaunchKernelGGL(full_probs_kernel<VI_F16>, pgrid, block, 0, stream, s.params, s.rows, s.vocabulary,
                           a.half_len, s.probs, s.probs_stride, a.bounds);
    return launch_status();
}

}  // namespace vi
