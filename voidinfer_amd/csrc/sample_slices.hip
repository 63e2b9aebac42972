// sample_slices.hip — full-vocabulary rows of the batched sampler (temperature
// > 0 and top_k = 0 or > 64): penalties, temperature, top-k / min-p / top-p over
// the whole vocabulary and the Philox inverse-CDF draw.  The row is read from
// HBM once; one slice of it is read again (from cache) to name the token.
//
// Key fact: bf16 / fp16 logits, and penalized logits stored back in the same
// dtype, take one of 65,536 bit patterns, and z = x' * (1/T) is a strictly
// monotone function of the pattern's order key (for T <= 65,536: distinct
// patterns give distinct fp32 products; +0 and -0 share z = 0).  The multiset
// of z over a row is therefore exactly a count histogram over patterns, and
// every truncation (top-k count, min-p ratio, top-p mass) and the draw reduce to
// prefix sums over the occupied patterns in z order; the float work (one fp64
// exp) is per occupied pattern, not per token.
//
// Shape.  A row is cut into slices of 32,768 tokens.  Persistent workgroups of
// 1024 threads (one per CU; the slices of a row on one XCD when there are at
// least 8 rows) take slices in turn.  A workgroup holds its slice in registers
// (4 x 16 bytes per thread) and has already requested the next slice's logits
// when it starts on the current one, so the HBM stream overlaps the LDS work.
// Per slice:
//   1. penalties: a bitmap of the slice's history tokens and an LDS hash of the
//      repeated ones' counts, from the lane's penalty state or its history;
//   2. a u16 count histogram indexed by raw pattern (word = pattern & 0x7fff,
//      half = sign bit), every logit counted as it arrives;
//   3. history tokens, gathered again from cache, are penalized and moved from
//      their raw pattern's count to the penalized pattern's;
//   4. one pass over the histogram: each coarse bin of 128 keys (bin = key >>
//      7) gets its (key << 16 | count) entries in key order, its valid count,
//      its largest valid key and the mass sum of count * exp(z(key) -
//      z(largest key)); entries and bin records go to HBM.
// A second launch merges, one workgroup per row: it sums the coarse tables,
// locates the bins holding the top-k, min-p and top-p cuts and the draw,
// resolves each inside its bin from the slices' list entries of that bin
// (exact key and rank), and reads the slice that holds the drawn rank again to
// name the token (id order among equal keys).
//
// Roofline: HBM; V x 2 bytes of logits per row, plus the penalty state's
// bitmap (V / 8 bytes) and repeat list, or the history.
#include <math.h>

#include "keys16.h"
#include "penalty_state.h"
#include "vi_device.h"
#include "vi_internal.h"

namespace vi {
namespace {

constexpr int kT = 1024;                  // threads per workgroup (one per CU: the LDS is the limit)
constexpr int kW = kT / kWave;            // waves per workgroup
constexpr int kSL = 32768;                // tokens per slice (counts fit 16 bits, whole bitmap words)
constexpr int kHW = 32768;                // histogram words (pattern & 0x7fff)
constexpr int kNV = (kSL + 8 * kT - 1) / (8 * kT);   // 16-byte vectors per thread and slice
constexpr int kWPT = (kSL / 32 + kT - 1) / kT;   // history bitmap words per thread (consecutive words)
constexpr int kBW = kWPT * kT;            // history bitmap words (a slice uses kSL / 32)
constexpr int kBins = 512;                // coarse bins of 128 keys, bin(key) = key >> 7
constexpr int kBinKeys = 128;
constexpr int kHeadWords = 32;            // slice head: n_list, n_valid, flags, top_key, bin mask [16], history tokens
constexpr int kHash = 2048;               // LDS repeat-count hash slots
constexpr uint32_t kHashFill = kHash * 3 / 4;
constexpr int kStage = 7168;              // history offsets staged per penalty round (u16): a lane with a
                                          // 32,768-token history puts ~4,050 tokens in a slice, one round
                                          // (the LDS beside the histogram sets the limit)
constexpr int kMaxSlices = 16;
constexpr int kPL = 2;                    // repeat-list entries prefetched per thread
constexpr int kPHist = 4;                 // history tokens prefetched per thread
constexpr uint32_t kTakeAll = 0xffffffffu;

// LDS map (bytes).  H: histogram, u16 counts in pairs (word p & 0x7fff: low half
// the pattern with sign 0, high half with sign 1); the merge reuses it.  B:
// history bitmap of the slice.  X: repeat hash (counts of the tokens seen more
// than once).  F: staged history offsets.  R: bitmap of the repeated tokens.
constexpr int kOffH = 0;
constexpr int kOffB = kOffH + 4 * kHW;
constexpr int kOffX = kOffB + 4 * kBW;
constexpr int kOffF = kOffX + 4 * kHash;
constexpr int kOffR = kOffF + 2 * kStage;     // R: the slice's tokens seen more than once (bitmap)
constexpr int kLds = kOffR + 4 * kBW;
constexpr int kQ = kHW / 2 / kT;          // 2-word histogram groups per thread (compaction)
constexpr int kSeg = kNV + 2;             // id-order segments: head, vectors, tail
static_assert(kWPT * kT == kBW && kSL % 32 == 0 && kSL < 65536 && kNV * 8 * kT >= kSL, "slice geometry");
static_assert(kQ * kW == 256 && kQ * 2 * kT == kHW, "compaction blocks of 128 patterns");
static_assert(kStage % kT == 0, "whole staging rounds per thread");

// Merge map inside H (bytes): per-slice bin (first | entries << 16), the
// slices' bin masks, bin counts and masses summed over slices, five gather
// slots (entries per slice and per-key counts).
constexpr int kOffMFE = 0;
constexpr int kOffMM = kOffMFE + 4 * kMaxSlices * kBins;
constexpr int kOffMC = kOffMM + 4 * kMaxSlices * (kBins / 32);
constexpr int kOffMR = kOffMC + 4 * kBins;
constexpr int kGatherSlots = 5;   // cap, min-p, top-p, support end, draw
constexpr int kGatherBytes = 4 * kMaxSlices * kBinKeys + 4 * kBinKeys + 4 * kMaxSlices;
constexpr int kOffGather = kOffMR + 8 * kBins;
static_assert(kOffGather + kGatherSlots * kGatherBytes <= 4 * kHW, "merge map");

using RowBound = FullBound;   // what the probs kernel and verification need to rebuild the support
static_assert(kSL == kFullSlice16 && kMaxSlices <= kFullBaseSlots, "full-route bases");

struct SliceArgs {
    const void* logits;
    int rows, vocabulary, slices, grid, xcd_aware;
    int64_t stride;
    const vi_row_params* params;
    const int32_t* histories;
    const int64_t* offsets;
    unsigned char* pstate;     // per-lane penalty states instead of histories (or null)
    PenaltyLayout pl;
    int record;
    int32_t* tokens;
    double* uniforms;
    float* probs;
    int64_t probs_stride;
    vi_sample_stats* stats;
    // workspace
    uint32_t* heads;           // [rows][slices][kHeadWords]: n_list, n_valid, flags, top_key, occupied-bin mask
    uint4* brec;               // [rows][slices][kBins], occupied bins only: first | entries << 16,
                               // valid logits | largest valid key << 16, mass relative to that key (double)
    uint32_t* lists;           // [rows][slices][kSL]; a slice's dense repeat counts before its list
    uint16_t* ptab;            // [rows][slices][kSL]: penalized patterns of the history tokens, in id order
    uint32_t* hbits;           // [rows][slices][kBW]: history bitmaps (history route; the state holds its own)
    int want_bounds;           // bounds and bases wanted (probs, or verification)
    RowBound* bounds;          // [rows]
    uint32_t* bases;           // [rows][kFullBaseSlots]: end-key logits in the slices before
};

struct Shared {
    uint32_t scan[kW + 1];
    uint32_t segs[kW][kSeg];
    // slice
    uint32_t flags, n_hash, overflow;
    uint32_t pflags[2];           // state-route penalty flags of items k (k & 1): built an item ahead
    uint32_t kmin, kmax, top_key, n_valid, n_list;
    uint32_t krange[kW];          // valid key range (kmin | kmax << 16) of items k .. k + kW - 1
    uint32_t bmask[kBins / 32];
    // merge
    uint32_t row_flags, row_valid, row_top;
    int32_t slot_bin[kGatherSlots];
    int32_t cap_bin, minp_bin, topp_bin, draw_bin, end_bin;
    int32_t cap_slot, minp_slot, topp_slot, draw_slot, end_slot;
    uint32_t cap_key, cap_take, minp_key, topp_key, topp_take, end_key, end_take, end_all;
    uint32_t n_support, draw_key, draw_rank, owner_slice, owner_rank, ok, hmask, tmask;
    uint32_t slice_hist[kMaxSlices];   // history tokens per slice
    int32_t token;
    double s_all, cap_mass, topp_target, s_n, u, draw_target;
};

// threadIdx.x behind an empty asm: arithmetic on it stays where it is written
// (the persistent loop's address computations would otherwise be hoisted out
// of the loop and held, or spilled, across it)
__device__ __forceinline__ int opaque_tid() {
    int t = int(threadIdx.x);
    asm volatile("" : "+v"(t));
    return t;
}

__device__ __forceinline__ int bin_of(uint32_t key) { return int(key >> 7); }
__device__ __forceinline__ uint32_t bin_first_key(int b) { return uint32_t(b) * uint32_t(kBinKeys); }

// value of lane `src` (per-lane source) for a 64-bit double
__device__ __forceinline__ double bperm_f64(double v, int src) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = uint32_t(__builtin_amdgcn_ds_bpermute(src << 2, int(uint32_t(b))));
    const uint32_t hi = uint32_t(__builtin_amdgcn_ds_bpermute(src << 2, int(uint32_t(b >> 32))));
    return __builtin_bit_cast(double, (uint64_t(hi) << 32) | lo);
}

// Adds each lane's value into dst[bin], where the lanes' bins are
// non-decreasing across the wave (bin < 0: nothing); one LDS atomic per run of
// equal bins.
__device__ __forceinline__ void wave_run_add(int bin, double v, double* dst) {
    const int lane = lane_id();
    const double incl = wave_incl_scan_f64(v);
    const int prev = __builtin_amdgcn_ds_bpermute(max(lane - 1, 0) << 2, bin);
    const int next = __builtin_amdgcn_ds_bpermute(min(lane + 1, kWave - 1) << 2, bin);
    const uint64_t heads = ballot(lane == 0 || prev != bin);
    const int start = 63 - __builtin_clzll(heads & ((2ull << lane) - 1ull));
    const double before = bperm_f64(incl, max(start - 1, 0));
    const double run = start == 0 ? incl : incl - before;
    if (bin >= 0 && (lane == kWave - 1 || next != bin)) atomicAdd(&dst[bin], run);
}

// A workgroup barrier that orders LDS only.  __syncthreads() also waits for
// every outstanding global load of the calling wave (its release fence covers
// global memory), so a barrier issued while the next slice's logits are in
// flight would wait for them; the slice pass synchronizes through LDS alone
// and orders its global stores explicitly.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// block_exclusive_scan_u32 with LDS-only barriers.
__device__ __forceinline__ uint32_t block_scan_lds(uint32_t v, uint32_t* tmp, uint32_t* total) {
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    const uint32_t x = wave_incl_scan_u32(v);
    if (lane == kWave - 1) tmp[wave] = x;
    lds_barrier();
    if (wave == 0) {
        const uint32_t t = lane < kW ? tmp[lane] : 0u;
        const uint32_t it = wave_incl_scan_u32(t);
        if (lane < kW) tmp[lane] = it - t;
        if (lane == kW - 1) tmp[kW] = it;
    }
    lds_barrier();
    const uint32_t r = tmp[wave] + x - v;
    *total = tmp[kW];
    lds_barrier();
    return r;
}

// Slice geometry inside the row.
struct Geo {
    int s0, n, head, nvec, tail;
    const uint16_t* base16;        // element s0 of the row
    const unsigned char* vbase;    // first 16-byte aligned element
};
__device__ __forceinline__ Geo geo_of(const SliceArgs& a, int row, int s) {
    Geo g;
    g.s0 = s * kSL;
    g.n = min(kSL, a.vocabulary - g.s0);
    const int64_t e0 = int64_t(row) * a.stride + g.s0;
    g.head = min(g.n, int((8 - (e0 & 7)) & 7));
    g.nvec = (g.n - g.head) / 8;
    g.tail = g.n - g.head - 8 * g.nvec;
    g.base16 = static_cast<const uint16_t*>(a.logits) + e0;
    g.vbase = reinterpret_cast<const unsigned char*>(g.base16 + g.head);
    return g;
}

struct SliceRegs {
    uint4 v[kNV];
    uint32_t hb, tb;
};
// Every load is issued, at a clamped in-bounds address (a slice holds at least one
// logit): users test v < nvec / tid < head / tid < tail themselves.  (A load under
// a branch is waited for where the branch joins, and a selected result is copied,
// which waits too: either would drain the prefetch as soon as it is issued.)
__device__ __forceinline__ void load_slice(const Geo& g, SliceRegs& r) {
    const int tid = opaque_tid();
    const int vl = max(g.nvec - 1, 0);
    const unsigned char* vb = g.nvec > 0 ? g.vbase : reinterpret_cast<const unsigned char*>(g.base16);
#pragma unroll
    for (int i = 0; i < kNV; ++i) r.v[i] = load16_cached(vb + size_t(min(i * kT + tid, vl)) * 16);
    r.hb = uint32_t(g.base16[tid < g.head ? tid : 0]);
    r.tb = uint32_t(g.base16[tid < g.tail ? g.head + 8 * g.nvec + tid : 0]);
}

// Item k of workgroup w: (row, slice), or false past the end.
__device__ __forceinline__ bool item_of(const SliceArgs& a, int w, int k, int* row, int* s) {
    if (a.xcd_aware) {
        const int x = w & 7, j = w >> 3;
        const int nx = (a.grid - x + 7) >> 3;      // workgroups on XCD x
        const int rx = (a.rows - x + 7) >> 3;      // rows on XCD x
        const int q = j + k * nx;
        if (q >= rx * a.slices) return false;
        *row = x + 8 * (q / a.slices);
        *s = q % a.slices;
        return true;
    }
    const int q = w + k * a.grid;
    if (q >= a.rows * a.slices) return false;
    *row = q / a.slices;
    *s = q % a.slices;
    return true;
}

__device__ __forceinline__ bool full_route_row(const vi_row_params& p) { return !topk_route(p); }

// ----------------------------------------------------------------- penalties
// Prefetched penalty inputs of one slice: its bitmap word (state route), the
// lane's header fields and the first repeat-list entries / history tokens.
struct PenPrefetch {
    uint32_t bword[kWPT], hflags, nrep;
    uint2 le[kPL];
    int32_t ht[kPHist];
};

struct PenCtx {
    bool pen, state;
    const unsigned char* lstate;
    const int32_t* hist;
    int64_t hn;
};
__device__ __forceinline__ PenCtx pen_ctx(const SliceArgs& a, int row, const vi_row_params& p) {
    PenCtx c{};
    c.state = a.pstate != nullptr;
    if (c.state) {
        c.lstate = a.pstate + size_t(row) * a.pl.lane_bytes;
        c.pen = penalties_active(p);
    } else {
        const int64_t b = a.offsets ? a.offsets[row] : 0;
        c.hn = (a.offsets && a.histories) ? a.offsets[row + 1] - b : 0;
        c.hist = a.histories ? a.histories + b : nullptr;
        c.pen = penalties_active(p) && c.hn > 0;
    }
    return c;
}

// A slice's penalty inputs (header, bitmap word and the repeat list's first
// kPL kT slots, read whatever the list's length: one round trip; or the
// history's head); issued a slice ahead.
__device__ __forceinline__ void pen_prefetch_head(const SliceArgs& a, const PenCtx& c, const Geo& g, PenPrefetch& f) {
    const int tid = opaque_tid();
#pragma unroll
    for (int q = 0; q < kWPT; ++q) f.bword[q] = 0u;
    f.hflags = 0u; f.nrep = 0u;
    if (!c.pen) return;
    if (c.state) {
        const PenaltyHeader* h = reinterpret_cast<const PenaltyHeader*>(c.lstate);
        f.hflags = h->flags;
        f.nrep = h->nrep;
        const uint32_t* b1 = reinterpret_cast<const uint32_t*>(c.lstate + a.pl.off_b1);
        const int nw = (g.n + 31) >> 5;
#pragma unroll
        for (int q = 0; q < kWPT; ++q)
            if (tid * kWPT + q < nw) f.bword[q] = b1[(g.s0 >> 5) + tid * kWPT + q];
        const uint2* list = reinterpret_cast<const uint2*>(c.lstate + a.pl.off_list);
#pragma unroll
        for (int j = 0; j < kPL; ++j) {
            const uint32_t i = uint32_t(j) * kT + uint32_t(tid);
            f.le[j] = i < uint32_t(a.pl.slots) ? list[i] : make_uint2(0u, 0u);
        }
    } else {
#pragma unroll
        for (int j = 0; j < kPHist; ++j) {
            const int64_t i = int64_t(j) * kT + tid;
            f.ht[j] = i < c.hn ? c.hist[i] : -1;
        }
    }
}

__device__ __forceinline__ uint32_t hash_slot(uint32_t off) { return (off * 0x9E3779B1u) >> 21; }

// Full counts of the slice's tokens in its dense table (when the repeat hash
// overflows).  All threads; uniform.
__device__ __forceinline__ void pen_dense_fill(const SliceArgs& a, const PenCtx& c, const Geo& g, const PenPrefetch& f,
                                               uint32_t* dense) {
    const int tid = opaque_tid();
    const int s1 = g.s0 + g.n;
    for (int i = tid; i < g.n; i += kT) put_agent(&dense[i], 0u);
    handoff_stores_done();
    __syncthreads();
    if (c.state) {
        const uint2* list = reinterpret_cast<const uint2*>(c.lstate + a.pl.off_list);
        const uint32_t nrep = min(uint32_t(__builtin_amdgcn_readfirstlane(int(f.nrep))), uint32_t(a.pl.slots));
        for (uint32_t i = tid; i < nrep; i += kT) {
            const uint2 e = list[i];
            const int t = int(e.x);
            if (e.y >= 2u && t >= g.s0 && t < s1) put_agent(&dense[t - g.s0], e.y);
        }
    } else {
        for (int64_t i = tid; i < c.hn; i += kT) {
            const int32_t t = c.hist[i];
            if (t >= g.s0 && t < s1) atomicAdd(&dense[t - g.s0], 1u);
        }
    }
    handoff_stores_done();
    __syncthreads();
}

// Records slice token `off` as seen 1 + extra times (add: one more occurrence of
// a token already recorded) in the repeat hash X and bitmap R; sets
// sh.overflow when the hash cannot hold it.
__device__ __forceinline__ void repeat_put(unsigned char* lds, Shared& sh, uint32_t off, uint32_t extra, bool add) {
    uint32_t* X = reinterpret_cast<uint32_t*>(lds + kOffX);
    uint32_t* R = reinterpret_cast<uint32_t*>(lds + kOffR);
        atomicOr(&R[off >> 5], 1u << (off & 31));
        if (extra > 0xffffu) { sh.overflow = 1u; return; }
        uint32_t h = hash_slot(off);
        const uint32_t key = (off + 1u) << 16;
        for (int probe = 0; probe < 64; ++probe) {
            uint32_t e = X[h];
            if (e == 0u) {
                e = atomicCAS(&X[h], 0u, key | extra);
                if (e == 0u) {
                    if (atomicAdd(&sh.n_hash, 1u) >= kHashFill) sh.overflow = 1u;
                    return;
                }
            }
            if ((e & 0xffff0000u) == key) {
                if (add) {
                    const uint32_t old = atomicAdd(&X[h], 1u);
                    if ((old & 0xffffu) == 0xffffu) sh.overflow = 1u;
                } else {
                    sh.overflow = 1u;   // a token twice in the repeat list: not a state's list
                }
                return;
            }
            h = (h + 1u) & uint32_t(kHash - 1);
        }
        sh.overflow = 1u;
    }

// Builds the slice's history bitmap in B and the repeat counts in X (or, when X
// overflows, full counts in the slice's dense table).  Sets sh.flags bits
// (BAD_HISTORY, ERROR) and sh.overflow.  All threads.
template <int DT>
__device__ __forceinline__ void pen_build(const SliceArgs& a, const PenCtx& c, const Geo& g, const PenPrefetch& f,
                          unsigned char* lds, Shared& sh, uint32_t* dense) {
    const int tid = opaque_tid();
    uint32_t* B = reinterpret_cast<uint32_t*>(lds + kOffB);
    uint32_t* X = reinterpret_cast<uint32_t*>(lds + kOffX);
    uint32_t* R = reinterpret_cast<uint32_t*>(lds + kOffR);
    const int nw = (g.n + 31) >> 5;
    for (int i = tid; i < kHash; i += kT) X[i] = 0u;
#pragma unroll
    for (int q = 0; q < kWPT; ++q) R[q * kT + tid] = 0u;
    if (tid == 0) { sh.n_hash = 0u; sh.overflow = 0u; }
    if (c.state) {
        const uint32_t lastm = (g.n & 31) ? (1u << (g.n & 31)) - 1u : ~0u;
#pragma unroll
        for (int q = 0; q < kWPT; ++q) {
            const int wd = tid * kWPT + q;
            B[wd] = wd < nw ? (f.bword[q] & (wd == nw - 1 ? lastm : ~0u)) : 0u;
        }
        const uint32_t hflags = uint32_t(__builtin_amdgcn_readfirstlane(int(f.hflags)));
        if (tid == 0 && hflags) atomicOr(&sh.flags, hflags & (VI_FLAG_BAD_HISTORY | VI_FLAG_ERROR));
    } else {
#pragma unroll
        for (int q = 0; q < kWPT; ++q) B[q * kT + tid] = 0u;
    }
    lds_barrier();
    auto hash_put = [&](uint32_t off, uint32_t extra, bool add) { repeat_put(lds, sh, off, extra, add); };
    const int s1 = g.s0 + g.n;
    if (c.state) {
        const uint2* list = reinterpret_cast<const uint2*>(c.lstate + a.pl.off_list);
        const uint32_t nrep = min(uint32_t(__builtin_amdgcn_readfirstlane(int(f.nrep))), uint32_t(a.pl.slots));
        auto put = [&](uint2 e) {
            const int t = int(e.x);
            if (e.y < 2u || t < g.s0 || t >= s1) return;
            hash_put(uint32_t(t - g.s0), e.y - 1u, false);
        };
#pragma unroll
        for (int j = 0; j < kPL; ++j)
            if (uint32_t(j) * kT + tid < nrep) put(f.le[j]);
        for (uint32_t i = uint32_t(kPL) * kT + tid; i < nrep; i += kT) put(list[i]);
    } else {
        auto rec = [&](int32_t t) {
            if (t < 0 || t >= a.vocabulary) { atomicOr(&sh.flags, uint32_t(VI_FLAG_BAD_HISTORY)); return; }
            if (t < g.s0 || t >= s1) return;
            const uint32_t off = uint32_t(t - g.s0), bit = 1u << (off & 31);
            const uint32_t old = atomicOr(&B[off >> 5], bit);
            if (old & bit) hash_put(off, 1u, true);
        };
#pragma unroll
        for (int j = 0; j < kPHist; ++j)
            if (int64_t(j) * kT + tid < c.hn) rec(f.ht[j]);
        // the rest in rounds of kHB tokens per thread, all requested before any is used
        constexpr int kHB = 8;
        for (int64_t i0 = int64_t(kPHist) * kT; i0 < c.hn; i0 += int64_t(kHB) * kT) {
            int32_t t8[kHB];
#pragma unroll
            for (int u = 0; u < kHB; ++u) {
                const int64_t i = i0 + int64_t(u) * kT + tid;
                t8[u] = i < c.hn ? c.hist[i] : 0;
            }
#pragma unroll
            for (int u = 0; u < kHB; ++u)
                if (i0 + int64_t(u) * kT + tid < c.hn) rec(t8[u]);
        }
    }
    lds_barrier();
    if (sh.overflow) pen_dense_fill(a, c, g, f, dense);   // (uniform)
}

// Occurrences of slice token `off` (its bitmap bit is set).
__device__ __forceinline__ uint32_t pen_count(const unsigned char* lds, const Shared& sh, const uint32_t* dense,
                                              uint32_t off) {
    if (sh.overflow) {
        const uint32_t c = get_agent(&dense[off]);
        return c ? c : 1u;
    }
    const uint32_t* R = reinterpret_cast<const uint32_t*>(lds + kOffR);
    if (!((R[off >> 5] >> (off & 31)) & 1u)) return 1u;   // seen once
    const uint32_t* X = reinterpret_cast<const uint32_t*>(lds + kOffX);
    uint32_t h = hash_slot(off);
    const uint32_t key = (off + 1u) << 16;
    for (int probe = 0; probe < kHash; ++probe) {
        const uint32_t e = X[h];
        if (e == 0u) return 1u;
        if ((e & 0xffff0000u) == key) return 1u + (e & 0xffffu);
        h = (h + 1u) & uint32_t(kHash - 1);
    }
    return 1u;
}

// Penalized bits of slice element `off` with raw bits `b` (b when not a history
// token or not finite).  `unrecord`: the slice offset of a token recorded into
// the state after the counts were to be taken (one occurrence is discounted), or
// ~0u.
template <int DT>
__device__ __forceinline__ uint32_t pen_bits(const unsigned char* lds, const Shared& sh, const uint32_t* dense,
                                             const vi_row_params& p, uint32_t off, uint32_t b,
                                             uint32_t unrecord = ~0u) {
    const uint32_t* B = reinterpret_cast<const uint32_t*>(lds + kOffB);
    if (!((B[off >> 5] >> (off & 31)) & 1u) || !Elem<DT>::finite_bits(b)) return b;
    uint32_t c = pen_count(lds, sh, dense, off);
    if (off == unrecord && --c == 0u) return b;
    return penalize_bits<DT>(b, c, p) & 0xffffu;
}

// Element j (0..7, possibly lane-varying) of a 16-byte vector of 16-bit values.
__device__ __forceinline__ uint32_t vec_elem(const uint4& v, int j) {
    const int q = j >> 1;
    const uint32_t w = q == 0 ? v.x : q == 1 ? v.y : q == 2 ? v.z : v.w;
    return (j & 1) ? (w >> 16) : (w & 0xffffu);
}

// Order key of slice element `off` after penalties, 0 when not finite (no
// finite pattern has key 0).
template <int DT>
__device__ __forceinline__ uint32_t elem_key(const unsigned char* lds, const Shared& sh, const uint32_t* dense,
                                             const vi_row_params& p, bool pen, uint32_t off, uint32_t b,
                                             uint32_t unrecord = ~0u) {
    const uint32_t pb = pen ? pen_bits<DT>(lds, sh, dense, p, off, b, unrecord) : b;
    return Elem<DT>::finite_bits(pb) ? key16(pb) : 0u;
}

// ------------------------------------------------------------ id-order ranks
// Positions of a per-element predicate over a slice held in registers, in id
// order: segment 0 the head elements (one per thread), segments 1..kNV the
// vectors i * kT + tid, segment kNV + 1 the tail elements.  cnt[x]: this
// thread's matches in segment x; excl[x] receives the matches before them in
// id order.  Returns the total.
__device__ __forceinline__ uint32_t id_order_prefix(const uint32_t cnt[kSeg], uint32_t excl[kSeg], Shared& sh) {
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    uint32_t incl[kSeg];
#pragma unroll
    for (int g = 0; g < kSeg; ++g) {
        incl[g] = wave_incl_scan_u32(cnt[g]);
        if (lane == kWave - 1) sh.segs[wave][g] = incl[g];
    }
    __syncthreads();
    // per segment: lane w holds wave w's count, one wave scan gives every
    // wave its offset (two values per segment in registers, not kW)
    uint32_t total = 0u;
#pragma unroll
    for (int g = 0; g < kSeg; ++g) {
        const uint32_t t = lane < kW ? sh.segs[lane][g] : 0u;
        const uint32_t iw = wave_incl_scan_u32(t);
        const uint32_t waves_before = uint32_t(__builtin_amdgcn_readlane(int(iw - t), wave));
        const uint32_t seg_total = uint32_t(__builtin_amdgcn_readlane(int(iw), kW - 1));
        excl[g] = total + waves_before + incl[g] - cnt[g];
        total += seg_total;
    }
    __syncthreads();
    return total;
}

// ------------------------------------------------------------------ merge
constexpr int kSlotsAll = kGatherSlots;
constexpr int kOffPC = kOffGather + kSlotsAll * kGatherBytes;   // [kMaxSlices] per-slice counts
constexpr int kOffTab = (kOffPC + 4 * 2 * kMaxSlices + 15) / 16 * 16;   // the owner slice's penalized patterns
constexpr int kTabCap = (4 * kHW - kOffTab) / 2 / 8 * 8;              // (u16 entries staged; more are read from HBM)
static_assert(kTabCap >= 8192, "merge map");

struct Slot {
    uint32_t* E;    // [kMaxSlices][kBinKeys] list entries of the bin, per slice
    uint32_t* FK;   // [kBinKeys] logits per key of the bin (all slices)
    uint32_t* NE;   // [kMaxSlices] entries per slice
};
__device__ __forceinline__ Slot slot_at(unsigned char* lds, int i) {
    unsigned char* b = lds + kOffGather + i * kGatherBytes;
    Slot s;
    s.E = reinterpret_cast<uint32_t*>(b);
    s.FK = s.E + kMaxSlices * kBinKeys;
    s.NE = s.FK + kBinKeys;
    return s;
}

// All threads: the list entries of bin b of every slice of `row`.
__device__ __forceinline__ void gather_bin(const SliceArgs& a, int row, int b, const Slot& sl, const uint32_t* MFE) {
    const int tid = threadIdx.x, S = a.slices;
    if (tid < kBinKeys) sl.FK[tid] = 0u;
    __syncthreads();
    const uint32_t k0 = bin_first_key(b);
    for (int idx = tid; idx < S * kBinKeys; idx += kT) {
        const int s = idx / kBinKeys, j = idx % kBinKeys;
        const uint32_t fe = MFE[s * kBins + b], ne = fe >> 16, f0 = fe & 0xffffu;
        if (j == 0) sl.NE[s] = ne;
        if (uint32_t(j) < ne) {
            const uint32_t e = a.lists[(size_t(row) * S + s) * kSL + f0 + j];
            sl.E[s * kBinKeys + j] = e;
            const uint32_t kj = (e >> 16) - k0;   // (< kBinKeys for every entry of bin b)
            if (kj < uint32_t(kBinKeys)) atomicAdd(&sl.FK[kj], e & 0xffffu);
        }
    }
    __syncthreads();
}

__device__ __forceinline__ double readlane_d(double v, int l) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint64_t r = uint64_t(uint32_t(__builtin_amdgcn_readlane(int(uint32_t(b)), l))) |
                       (uint64_t(uint32_t(__builtin_amdgcn_readlane(int(uint32_t(b >> 32)), l))) << 32);
    return __builtin_bit_cast(double, r);
}

// Wave 0 helpers over the coarse bins, in descending order: lane l holds bins
// kBins - 1 - kCPL l - i (i < kCPL).
constexpr int kCPL = kBins / kWave;
struct CoarseHit {
    int bin;
    double mass_before;
    uint32_t cnt_before;
};
// First non-empty bin b >= lo (descending) at which the cumulative count
// (mode 0: >= target) or mass (mode 1: >= target, mode 2: > target) is reached;
// bin -1 when none is.
__device__ __forceinline__ CoarseHit coarse_find(const double* MR, const uint32_t* MC, int lo, int mode, double target) {
    const int lane = lane_id();
    double vm[kCPL], tm = 0.0;
    uint32_t vc[kCPL], tc = 0u;
#pragma unroll
    for (int i = 0; i < kCPL; ++i) {
        const int b = kBins - 1 - kCPL * lane - i;
        const bool ok = b >= lo;
        vm[i] = ok ? MR[b] : 0.0;
        vc[i] = ok ? MC[b] : 0u;
        tm += vm[i];
        tc += vc[i];
    }
    double cm = wave_incl_scan_f64(tm) - tm;
    uint32_t cc = wave_incl_scan_u32(tc) - tc;
    int fi = -1;
    double fm = 0.0;
    uint32_t fc = 0u;
#pragma unroll
    for (int i = 0; i < kCPL; ++i) {
        const double nm = cm + vm[i];
        const uint32_t nc = cc + vc[i];
        const bool hit = mode == 0 ? double(nc) >= target : (mode == 1 ? nm >= target : nm > target);
        if (fi < 0 && hit && vc[i] > 0u) { fi = i; fm = cm; fc = cc; }
        cm = nm;
        cc = nc;
    }
    const uint64_t m = ballot(fi >= 0);
    if (!m) return CoarseHit{-1, 0.0, 0u};
    const int L = __builtin_ctzll(m);
    return CoarseHit{kBins - 1 - kCPL * L - readlane_i(fi, L), readlane_d(fm, L), uint32_t(readlane_i(int(fc), L))};
}
// Mass and count of the bins above bin b.
__device__ __forceinline__ void coarse_above(const double* MR, const uint32_t* MC, int b, double* m, uint32_t* c) {
    const int lane = lane_id();
    double tm = 0.0;
    uint32_t tc = 0u;
    for (int x = b + 1 + lane; x < kBins; x += kWave) { tm += MR[x]; tc += MC[x]; }
    *m = wave_sum_f64(tm);
    *c = wave_sum_u32(tc);
}

constexpr int kKPL = kBinKeys / kWave;   // keys per lane in fine_find
struct FineHit {
    bool found;
    uint32_t key, rank;
    double mass_before;     // mass of the bin's keys above `key`
    uint32_t cnt_before;
    double total_mass;      // of the (limited) bin
    uint32_t total_cnt;
    uint32_t last_key, last_cnt;   // the lowest key with logits (limited)
};
// Wave 0.  The keys of bin b in descending order (lane l: kBinKeys - 1 - kKPL l - i), with
// counts limited to the position (lim_key, lim_take): keys below lim_key count
// none, lim_key at most lim_take.  Finds the first element (key, rank) at which
// the cumulative count (mode 0: >= target) or mass (mode 1: >= target, mode 2:
// > target) is reached; mode 3 only totals.  Masses are exp(z - zmax) per logit.
template <int DT>
__device__ __forceinline__ FineHit fine_find(const uint32_t* FK, int b, int mode, double target, uint32_t lim_key, uint32_t lim_take,
                             double zmax, float inv_t) {
    const int lane = lane_id();
    const int k0 = int(bin_first_key(b));
    uint32_t c[kKPL];
    double w[kKPL], tm = 0.0;
    uint32_t tc = 0u;
#pragma unroll
    for (int i = 0; i < kKPL; ++i) {
        const int j = kBinKeys - 1 - kKPL * lane - i, key = k0 + j;
        uint32_t cc = FK[j];
        if (uint32_t(key) < lim_key) cc = 0u;
        else if (uint32_t(key) == lim_key) cc = min(cc, lim_take);
        c[i] = cc;
        w[i] = cc ? exp(double(key_z<DT>(uint32_t(key), inv_t)) - zmax) : 0.0;
        tm += double(cc) * w[i];
        tc += cc;
    }
    const double im = wave_incl_scan_f64(tm);
    const uint32_t ic = wave_incl_scan_u32(tc);
    double cm = im - tm;
    uint32_t cc = ic - tc;
    int fi = -1, li = -1;
    uint32_t fr = 0u;
    double fm = 0.0;
    uint32_t fc = 0u;
#pragma unroll
    for (int i = 0; i < kKPL; ++i) {
        const double nm = cm + double(c[i]) * w[i];
        const uint32_t nc = cc + c[i];
        if (c[i]) li = i;
        if (fi < 0 && c[i] && mode != 3) {
            bool hit;
            if (mode == 0) hit = double(nc) >= target;
            else if (mode == 1) hit = nm >= target;
            else hit = nm > target;
            if (hit) {
                uint32_t r;
                if (mode == 0) {
                    r = uint32_t(max(0.0, target - double(cc) - 1.0));
                } else {
                    const double x = (target - cm) / w[i];
                    double rr = mode == 1 ? ceil(x) - 1.0 : floor(x);
                    rr = fmin(fmax(rr, 0.0), double(c[i] - 1u));
                    r = uint32_t(rr);
                    for (int it = 0; it < 4; ++it) {   // settle the rounding of the estimate
                        if (r > 0u && (mode == 1 ? cm + double(r) * w[i] >= target : cm + double(r) * w[i] > target)) --r;
                        else if (r + 1u < c[i] && (mode == 1 ? cm + double(r + 1u) * w[i] < target
                                                              : cm + double(r + 1u) * w[i] <= target)) ++r;
                        else break;
                    }
                }
                fi = i; fr = min(r, c[i] - 1u); fm = cm; fc = cc;
            }
        }
        cm = nm;
        cc = nc;
    }
    FineHit h{};
    h.total_mass = readlane_d(im, kWave - 1);
    h.total_cnt = uint32_t(readlane_i(int(ic), kWave - 1));
    const uint64_t lm = ballot(li >= 0);
    if (lm) {
        const int L = 63 - __builtin_clzll(lm);
        const int i = readlane_i(li, L);
        h.last_key = uint32_t(k0 + kBinKeys - 1 - kKPL * L - i);
        // (c[] indexed by a lane-uniform i: pick it per lane first)
        uint32_t mine = 0u;
#pragma unroll
        for (int q = 0; q < kKPL; ++q) if (q == li) mine = c[q];
        h.last_cnt = uint32_t(readlane_i(int(mine), L));
    }
    const uint64_t m = ballot(fi >= 0);
    if (m) {
        const int L = __builtin_ctzll(m);
        const int i = readlane_i(fi, L);
        h.found = true;
        h.key = uint32_t(k0 + kBinKeys - 1 - kKPL * L - i);
        h.rank = uint32_t(readlane_i(int(fr), L));
        h.mass_before = readlane_d(fm, L);
        h.cnt_before = uint32_t(readlane_i(int(fc), L));
    }
    return h;
}

__device__ __forceinline__ void write_row(const SliceArgs& a, int row, int32_t token, double u, uint32_t flags,
                                          uint32_t support, uint32_t finite, double s_n) {
    a.tokens[row] = token;
    if (a.uniforms) a.uniforms[row] = u;
    if (a.stats) {
        vi_sample_stats st{};
        st.flags = flags;
        st.support = support;
        st.finite = finite;
        st.support_mass = s_n;
        st.uniform = u;
        a.stats[row] = st;
    }
}

// The row's decisions and its token (sh.kmin set).
template <int DT>
__device__ __forceinline__ void merge_row(const SliceArgs& a, int row, const vi_row_params& p, float inv_t, unsigned char* lds,
                          Shared& sh) {
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave, S = a.slices, V = a.vocabulary;
    uint32_t* MFE = reinterpret_cast<uint32_t*>(lds + kOffMFE);
    uint32_t* MC = reinterpret_cast<uint32_t*>(lds + kOffMC);
    double* MR = reinterpret_cast<double*>(lds + kOffMR);
    uint32_t* PC = reinterpret_cast<uint32_t*>(lds + kOffPC);   // [kMaxSlices] drawn key, [kMaxSlices] end key
    const size_t rs = size_t(row) * S;

    // ---- 0. slice heads (totals and occupied-bin masks), then the occupied bins'
    // records; each bin summed over the slices in slice order (deterministic)
    uint32_t* MM = reinterpret_cast<uint32_t*>(lds + kOffMM);   // [S][kBins / 32] occupied-bin masks
    constexpr int kMW = kBins / 32;
    if (tid < S * kMW) MM[tid] = a.heads[(rs + tid / kMW) * kHeadWords + 4 + tid % kMW];
    uint32_t h3[3] = {0u, 0u, 0u};
    if (tid < S) {
#pragma unroll
        for (int q = 0; q < 3; ++q) h3[q] = a.heads[(rs + tid) * kHeadWords + 1 + q];
        sh.slice_hist[tid] = a.heads[(rs + tid) * kHeadWords + 4 + kBins / 32];
    }
    if (tid < kGatherSlots) sh.slot_bin[tid] = -1;
    if (tid == 0) { sh.row_flags = 0u; sh.row_valid = 0u; sh.row_top = 0u; sh.token = -1; sh.ok = 1u; }
    __syncthreads();
    if (tid < S) { atomicAdd(&sh.row_valid, h3[0]); atomicOr(&sh.row_flags, h3[1]); atomicMax(&sh.row_top, h3[2]); }
    __syncthreads();
    const uint32_t top = sh.row_top, N = sh.row_valid;
    const double zmax = double(key_z<DT>(top, inv_t));
    // the occupied (slice, bin) pairs in slice-major order, one record load each;
    // the rescaled masses are summed as 2^-44 fixed point (u64 atomics: exact
    // in any order, so the sums do not depend on the order of arrival)
    uint32_t* OCC = reinterpret_cast<uint32_t*>(lds + kOffGather);   // (slice << 16 | bin) pairs (then gathers)
    uint64_t* MRI = reinterpret_cast<uint64_t*>(MR);
    for (int i = tid; i < S * kBins; i += kT) MFE[i] = 0u;
    if (tid < kBins) { MC[tid] = 0u; MRI[tid] = 0ull; }
    uint32_t mw = tid < S * kMW ? MM[tid] : 0u, npairs = 0u;
    const uint32_t pbase = block_scan_lds(uint32_t(__builtin_popcount(mw)), sh.scan, &npairs);
    {
        uint32_t o = pbase;
        const uint32_t s_ = uint32_t(tid / kMW), b0 = uint32_t(tid % kMW) * 32u;
        while (mw) {
            const int j = __builtin_ctz(mw);
            mw &= mw - 1u;
            OCC[o++] = (s_ << 16) | (b0 + uint32_t(j));
        }
    }
    __syncthreads();
    constexpr double kRowScale = 0x1p44;   // row masses <= V <= 2^19: sums stay below 2^63
    for (uint32_t i = tid; i < npairs; i += kT) {
        const uint32_t sb = OCC[i], q = sb >> 16, b = sb & 0xffffu;
        const uint4 r = a.brec[(rs + q) * kBins + b];
        MFE[q * kBins + b] = r.x;
        const uint32_t cnt = r.y & 0xffffu;
        atomicAdd(&MC[b], cnt);
        const double ms = __builtin_bit_cast(double, (uint64_t(r.w) << 32) | r.z);
        const double m = ms * exp(double(key_z<DT>(r.y >> 16, inv_t)) - zmax);
        atomicAdd(reinterpret_cast<unsigned long long*>(&MRI[b]), (unsigned long long)(rint(m * kRowScale)));
    }
    __syncthreads();
    if (tid < kBins) MR[tid] = double(MRI[tid]) * (1.0 / kRowScale);
    __syncthreads();
    const uint32_t out_flags = sh.row_flags & (VI_FLAG_NONFINITE | VI_FLAG_BAD_HISTORY);
    const bool fail = (sh.row_flags & VI_FLAG_ERROR) != 0u || !(p.temperature <= kMaxTemperature);
    if (fail || N == 0u) {
        if (tid == 0) {
            write_row(a, row, fail ? -1 : V, 0.0, out_flags | (fail ? VI_FLAG_ERROR : VI_FLAG_EMPTY), 0u, 0u, 0.0);
            if (a.want_bounds) a.bounds[row] = RowBound{0.0, 0.0, 0.0f, 0u, 0u, 0u};
        }
        __syncthreads();
        return;
    }
    // All threads: slot holding bin b (gathered into `slot` if absent).
    auto gather_into = [&](int b, int slot) -> int {
        for (int i = 0; i < kSlotsAll; ++i)
            if (sh.slot_bin[i] == b) return i;
        gather_bin(a, row, b, slot_at(lds, slot), MFE);
        if (tid == 0) sh.slot_bin[slot] = b;
        __syncthreads();
        return slot;
    };

    // ---- 1. totals; bins of the top-k cap and of the min-p cut
    if (wave == 0) {
        double tm = 0.0;
        for (int b = lane; b < kBins; b += kWave) tm += MR[b];
        const double s_all = wave_sum_f64(tm);
        int cap_bin = -1;
        if (p.top_k > 0 && uint32_t(p.top_k) < N) cap_bin = coarse_find(MR, MC, 0, 0, double(p.top_k)).bin;
        int minp_bin = -1;
        uint32_t kf = 0u;
        if (p.min_p > 0.0f) {
            const double mp = double(p.min_p);
            kf = uint32_t(wave_search(int(sh.kmin), int(top) + 1, [&](int key) {
                return exp(double(key_z<DT>(uint32_t(key), inv_t)) - zmax) >= mp;
            }));
            minp_bin = kf <= top ? bin_of(kf) : -1;
        }
        if (lane == 0) { sh.s_all = s_all; sh.cap_bin = cap_bin; sh.minp_bin = minp_bin; sh.minp_key = kf; }
    }
    __syncthreads();
    const int cap_slot = sh.cap_bin >= 0 ? gather_into(sh.cap_bin, 0) : -1;
    if (sh.minp_bin >= 0) (void)gather_into(sh.minp_bin, 1);

    // ---- 2. the cap's position and mass; the bin of the top-p cut
    if (wave == 0) {
        uint32_t ck = 0u, ct = kTakeAll;
        double cap_mass = sh.s_all;
        if (cap_slot >= 0) {
            double am;
            uint32_t ac;
            coarse_above(MR, MC, sh.cap_bin, &am, &ac);
            const FineHit f = fine_find<DT>(slot_at(lds, cap_slot).FK, sh.cap_bin, 0, double(p.top_k) - double(ac),
                                            0u, kTakeAll, zmax, inv_t);
            ck = f.found ? f.key : f.last_key;
            ct = f.found ? f.rank + 1u : max(f.last_cnt, 1u);
            const double mb = f.found ? f.mass_before : f.total_mass - double(f.last_cnt) *
                                                                       exp(double(key_z<DT>(ck, inv_t)) - zmax);
            cap_mass = am + mb + double(ct) * exp(double(key_z<DT>(ck, inv_t)) - zmax);
        }
        int topp_bin = -1;
        double target = 0.0;
        if (p.top_p < 1.0f) {
            target = double(p.top_p) * cap_mass;
            const CoarseHit h = coarse_find(MR, MC, cap_slot >= 0 ? sh.cap_bin + 1 : 0, 1, target);
            topp_bin = h.bin >= 0 ? h.bin : (cap_slot >= 0 ? sh.cap_bin : -1);
        }
        if (lane == 0) {
            sh.cap_key = ck; sh.cap_take = ct; sh.cap_mass = cap_mass;
            sh.topp_bin = topp_bin; sh.topp_target = target;
        }
    }
    __syncthreads();
    const int topp_slot = sh.topp_bin >= 0 ? gather_into(sh.topp_bin, 2) : -1;

    // ---- 3. the top-p position; the support's end: the earliest of the cap,
    // the min-p cut and the top-p cut, at least one logit
    if (wave == 0) {
        bool has_topp = false;
        uint32_t tk = 0u, tt = kTakeAll;
        if (topp_slot >= 0) {
            double am;
            uint32_t ac;
            coarse_above(MR, MC, sh.topp_bin, &am, &ac);
            const bool in_cap = cap_slot >= 0 && sh.topp_bin == sh.cap_bin;
            const FineHit f = fine_find<DT>(slot_at(lds, topp_slot).FK, sh.topp_bin, 1, sh.topp_target - am,
                                            in_cap ? sh.cap_key : 0u, in_cap ? sh.cap_take : kTakeAll, zmax, inv_t);
            if (f.found) { tk = f.key; tt = f.rank + 1u; has_topp = true; }
        }
        bool all = true;
        uint32_t ek = 0u, et = kTakeAll;
        auto consider = [&](uint32_t k, uint32_t t) {
            if (all || k > ek || (k == ek && t < et)) { ek = k; et = t; all = false; }
        };
        if (cap_slot >= 0) consider(sh.cap_key, sh.cap_take);
        if (p.min_p > 0.0f) consider(sh.minp_key, kTakeAll);
        if (has_topp) consider(tk, tt);
        if (!all && ek > top) { ek = top; et = 1u; }   // no logit passes (min_p > 1): the best one
        if (lane == 0) { sh.end_all = all ? 1u : 0u; sh.end_key = ek; sh.end_take = et; sh.end_bin = all ? -1 : bin_of(ek); }
    }
    __syncthreads();
    const int end_slot = sh.end_all ? -1 : gather_into(sh.end_bin, 3);

    // ---- 4. support mass, the draw's target and bin
    if (wave == 0) {
        double sn;
        uint32_t n;
        if (sh.end_all) {
            sn = sh.s_all;
            n = N;
        } else {
            double am;
            uint32_t ac;
            coarse_above(MR, MC, sh.end_bin, &am, &ac);
            const FineHit f = fine_find<DT>(slot_at(lds, end_slot).FK, sh.end_bin, 3, 0.0, sh.end_key, sh.end_take,
                                            zmax, inv_t);
            sn = am + f.total_mass;
            n = ac + f.total_cnt;
        }
        const double u = philox_uniform(p.seed, p.lane, p.position, 0u);
        const double t = u * sn;
        const CoarseHit h = coarse_find(MR, MC, sh.end_all ? 0 : sh.end_bin + 1, 2, t);
        int db = h.bin;
        if (db < 0 && !sh.end_all) db = sh.end_bin;
        if (db < 0) {   // (rounding past the last logit) the lowest bin holding one
            int lo = kBins;
            for (int b = lane; b < kBins; b += kWave) if (MC[b]) lo = min(lo, b);
#pragma unroll
            for (int o = 32; o; o >>= 1) lo = min(lo, __shfl_xor(lo, o, kWave));
            db = lo;
        }
        if (lane == 0) { sh.s_n = sn; sh.n_support = n; sh.u = u; sh.draw_target = t; sh.draw_bin = db; }
    }
    __syncthreads();
    const int draw_slot = gather_into(sh.draw_bin, 4);

    // ---- 5. the drawn (key, rank), then the slice holding it
    if (wave == 0) {
        double am;
        uint32_t ac;
        coarse_above(MR, MC, sh.draw_bin, &am, &ac);
        const bool in_end = !sh.end_all && sh.draw_bin == sh.end_bin;
        const FineHit f = fine_find<DT>(slot_at(lds, draw_slot).FK, sh.draw_bin, 2, sh.draw_target - am,
                                        in_end ? sh.end_key : 0u, in_end ? sh.end_take : kTakeAll, zmax, inv_t);
        if (lane == 0) {
            if (f.found) { sh.draw_key = f.key; sh.draw_rank = f.rank; }
            else if (f.last_cnt) { sh.draw_key = f.last_key; sh.draw_rank = f.last_cnt - 1u; }
            else sh.ok = 0u;
        }
    }
    if (tid < 2 * kMaxSlices) PC[tid] = 0u;
    __syncthreads();
    {
        const Slot ds = slot_at(lds, draw_slot);
        const uint32_t dk = sh.draw_key;
        for (int idx = tid; idx < S * kBinKeys; idx += kT) {
            const int s = idx / kBinKeys, j = idx % kBinKeys;
            if (uint32_t(j) < ds.NE[s]) {
                const uint32_t e = ds.E[s * kBinKeys + j];
                if ((e >> 16) == dk) PC[s] = e & 0xffffu;
            }
        }
        if (a.want_bounds && end_slot >= 0) {
            const Slot es = slot_at(lds, end_slot);
            const uint32_t ek = sh.end_key;
            for (int idx = tid; idx < S * kBinKeys; idx += kT) {
                const int s = idx / kBinKeys, j = idx % kBinKeys;
                if (uint32_t(j) < es.NE[s]) {
                    const uint32_t e = es.E[s * kBinKeys + j];
                    if ((e >> 16) == ek) PC[kMaxSlices + s] = e & 0xffffu;
                }
            }
        }
    }
    __syncthreads();
    if (wave == 0) {
        const uint32_t c = lane < S ? PC[lane] : 0u;
        const uint32_t incl = wave_incl_scan_u32(c);
        const uint32_t want = sh.draw_rank;
        const uint64_t m = ballot(lane < S && incl > want);
        if (m) {
            const int L = __builtin_ctzll(m);
            if (lane == L) { sh.owner_slice = uint32_t(L); sh.owner_rank = want - (incl - c); }
        } else if (lane == 0) {
            sh.ok = 0u;
        }
        if (a.want_bounds) {   // end-key logits in the slices before each slice (id order)
            const uint32_t ce = lane < S ? PC[kMaxSlices + lane] : 0u;
            const uint32_t ie = wave_incl_scan_u32(ce);
            if (lane < kFullBaseSlots) a.bases[size_t(row) * kFullBaseSlots + lane] = ie - ce;
        }
    }
    __syncthreads();

    // ---- 6. the owner slice read again: the owner_rank-th logit of the drawn
    // key in id order.  Thread t takes body vectors kNV t .. kNV t + kNV - 1, so
    // thread order is id order: the head logits (offsets < head, threads <
    // head), the body, the tail.  History tokens take their penalized patterns
    // from the slice pass's table (rank = their order among the slice's history
    // tokens); the history bitmap comes from the lane's state, or as the slice
    // pass published it.
    if (sh.ok) {
        const int os = int(sh.owner_slice);
        const Geo g = geo_of(a, row, os);
        uint4 v[kNV];
#pragma unroll
        for (int i = 0; i < kNV; ++i) {
            const int vi = kNV * tid + i;
            v[i] = vi < g.nvec ? load16_cached(g.vbase + size_t(vi) * 16) : make_uint4(0u, 0u, 0u, 0u);
        }
        const uint32_t hb = tid < g.head ? uint32_t(g.base16[tid]) : 0u;
        const uint32_t tb = tid < g.tail ? uint32_t(g.base16[g.head + 8 * g.nvec + tid]) : 0u;
        const PenCtx pc = pen_ctx(a, row, p);
        // the slice pass's table of penalized patterns, staged in LDS (loads issued
        // with the logits')
        const uint16_t* tab = a.ptab + (rs + os) * kSL;
        uint16_t* T = reinterpret_cast<uint16_t*>(lds + kOffTab);
        const uint32_t ntab = pc.pen ? min(sh.slice_hist[os], uint32_t(kTabCap)) : 0u;
        for (uint32_t i = tid; i < (ntab + 7u) / 8u; i += kT)
            reinterpret_cast<uint4*>(T)[i] = reinterpret_cast<const uint4*>(tab)[i];
        auto tab_at = [&](uint32_t rank) { return rank < ntab ? uint32_t(T[rank]) : uint32_t(tab[rank]); };
        // history flags: bit e of hmask for body element e of this thread; head / tail
        static_assert(kNV * 8 == 32, "a thread's body elements fill one 32-bit mask");
        const int nbv = max(0, min(kNV, g.nvec - kNV * tid));   // this thread's body vectors
        const uint32_t bodym = nbv >= kNV ? ~0u : (1u << (8 * nbv)) - 1u;
        uint32_t hmask = 0u;
        bool hh = false, th = false;
        if (pc.pen) {
            const uint32_t* bm = pc.state ? reinterpret_cast<const uint32_t*>(pc.lstate + a.pl.off_b1) + (g.s0 >> 5)
                                          : a.hbits + (rs + os) * kBW;
            const int nw = (g.n + 31) >> 5;
            const uint32_t lastm = (g.n & 31) ? (1u << (g.n & 31)) - 1u : ~0u;
            auto word = [&](int wd) { return wd < nw ? (bm[wd] & (wd == nw - 1 ? lastm : ~0u)) : 0u; };
            const uint32_t off0 = uint32_t(g.head + 8 * kNV * tid), wd0 = off0 >> 5, sft = off0 & 31u;
            const uint64_t two = uint64_t(word(int(wd0))) | (uint64_t(word(int(wd0) + 1)) << 32);
            hmask = nbv > 0 ? uint32_t(two >> sft) & bodym : 0u;
            if (tid < g.head) hh = (word(0) >> tid) & 1u;
            const uint32_t to = uint32_t(g.head + 8 * g.nvec + tid);
            if (tid < g.tail) th = (word(int(to >> 5)) >> (to & 31u)) & 1u;
        }
        // ranks of the history tokens: the head's (wave 0), the body's in thread
        // order, the tail's
        uint32_t hrank = 0u, trank = 0u, nhist = 0u, hexcl = 0u, h0 = 0u;
        if (pc.pen) {   // (uniform)
            if (wave == 0) {
                const uint64_t hb_ = ballot(hh), tb_ = ballot(th);
                const uint64_t below = (1ull << lane) - 1ull;
                hrank = uint32_t(__builtin_popcountll(hb_ & below));
                trank = uint32_t(__builtin_popcountll(tb_ & below));
                if (lane == 0) sh.n_hash = uint32_t(__builtin_popcountll(hb_));   // (history tokens among the head)
            }
            hexcl = block_scan_lds(uint32_t(__builtin_popcount(hmask)), sh.scan, &nhist);
            h0 = sh.n_hash;
        }
        const uint32_t dk = sh.draw_key;
        // patterns of the drawn key (+0 and -0 for key 0x8000): a logit matches when
        // its (penalized) pattern is one of them (the key map is one to one but
        // for the zeros, and the drawn key is finite)
        const uint32_t P1 = unkey16(dk), P2 = dk == 0x8000u ? 0x8000u : P1;
        auto match = [&](uint32_t b) { return b == P1 || b == P2; };
        uint32_t bits = 0u;
        uint32_t r = h0 + hexcl;
        if (!pc.pen || sh.slice_hist[os] <= uint32_t(kTabCap)) {   // (uniform) the table is staged whole
#pragma unroll
            for (int i = 0; i < kNV; ++i) {
                const uint32_t w4[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int e = 8 * i + j;
                    const uint32_t b = (j & 1) ? (w4[j >> 1] >> 16) : (w4[j >> 1] & 0xffffu);
                    const bool hist = (hmask >> e) & 1u;
                    const uint32_t pb = hist ? uint32_t(T[min(r, uint32_t(kTabCap - 1))]) : b;
                    r += hist ? 1u : 0u;
                    bits |= match(pb) ? 1u << e : 0u;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < kNV; ++i) {
                const uint32_t w4[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int e = 8 * i + j;
                    const uint32_t b = (j & 1) ? (w4[j >> 1] >> 16) : (w4[j >> 1] & 0xffffu);
                    const bool hist = (hmask >> e) & 1u;
                    const uint32_t pb = hist ? tab_at(r) : b;
                    r += hist ? 1u : 0u;
                    bits |= match(pb) ? 1u << e : 0u;
                }
            }
        }
        bits &= bodym;
        const bool hm = tid < g.head && match(hh ? tab_at(hrank) : hb);
        const bool tm = tid < g.tail && match(th ? tab_at(h0 + nhist + trank) : tb);
        if (wave == 0) {   // (head and tail logits belong to threads < 8)
            const uint64_t hmk = ballot(hm), tmk = ballot(tm);
            if (lane == 0) { sh.hmask = uint32_t(hmk); sh.tmask = uint32_t(tmk); }
        }
        const uint32_t nb = uint32_t(__builtin_popcount(bits));
        uint32_t nbody = 0u;
        const uint32_t bexcl = block_scan_lds(nb, sh.scan, &nbody);
        auto nth_bit = [](uint32_t m, uint32_t n) {   // index of the n-th set bit (n < popcount)
            for (; n > 0u; --n) m &= m - 1u;
            return __builtin_ctz(m);
        };
        const uint32_t hmk = sh.hmask, tmk = sh.tmask, nh = uint32_t(__builtin_popcount(hmk));
        const uint32_t want = sh.owner_rank;
        if (want < nh) {
            if (tid == nth_bit(hmk, want)) sh.token = g.s0 + tid;
        } else if (want - nh < nbody) {
            const uint32_t rr = want - nh;
            if (rr >= bexcl && rr < bexcl + nb) {
                const int j = nth_bit(bits, rr - bexcl);
                sh.token = g.s0 + g.head + 8 * (kNV * tid + j / 8) + j % 8;
            }
        } else if (want - nh - nbody < uint32_t(__builtin_popcount(tmk))) {
            if (tid == nth_bit(tmk, want - nh - nbody)) sh.token = g.s0 + g.head + 8 * g.nvec + tid;
        }
        __syncthreads();
    }
    if (tid == 0) {
        const int32_t tok = sh.token;
        if (tok < 0) {   // the tables disagree with the slice: cannot happen for consistent inputs
            write_row(a, row, -1, sh.u, out_flags | VI_FLAG_ERROR, 0u, 0u, 0.0);
        } else {
            write_row(a, row, tok, sh.u, out_flags, sh.n_support, N, sh.s_n);
            if (a.record && tok < V) {   // (the slice pass, an earlier launch, has read the state)
                const LaneState ls = lane_state(a.pstate + size_t(row) * a.pl.lane_bytes, a.pl);
                state_record_one(ls, a.pl, V, tok);
            }
        }
        if (a.want_bounds)
            a.bounds[row] = RowBound{zmax, sh.s_n, inv_t, sh.end_all ? 0u : sh.end_key,
                                     sh.end_all ? kTakeAll : sh.end_take, tok >= 0 ? 1u : 0u};
    }
    __syncthreads();
}

// ------------------------------------------------------------------ kernels
template <int DT>
__global__ __launch_bounds__(kT) void slice_kernel(SliceArgs a) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[kLds];
    __shared__ Shared sh;
    uint32_t* H = reinterpret_cast<uint32_t*>(lds + kOffH);
    uint4* H4 = reinterpret_cast<uint4*>(lds + kOffH);
    uint2* H2 = reinterpret_cast<uint2*>(lds + kOffH);
    uint32_t* B = reinterpret_cast<uint32_t*>(lds + kOffB);
    const int w = blockIdx.x;
    const int S = a.slices;

    int row = 0, s = 0;
    if (!item_of(a, w, 0, &row, &s)) return;
    // the histogram and the slice head's counters start empty (every slice leaves
    // them so)
#pragma unroll
    for (int q = 0; q < kHW / 4 / kT; ++q) H4[q * kT + threadIdx.x] = make_uint4(0u, 0u, 0u, 0u);
    if (threadIdx.x < kBins / 32) sh.bmask[threadIdx.x] = 0u;
    if (threadIdx.x == 0) { sh.n_list = 0u; sh.n_valid = 0u; sh.top_key = 0u; sh.pflags[0] = 0u; sh.pflags[1] = 0u; }
    SliceRegs cur{};
    PenPrefetch pf{};
    const bool state_route = a.pstate != nullptr;   // (launch-uniform)
    uint32_t bw[kWPT], rank0 = 0u, nf = 0u;          // the item's history bitmap word(s), rank base, total
#pragma unroll
    for (int q = 0; q < kWPT; ++q) bw[q] = 0u;
    uint16_t* F = reinterpret_cast<uint16_t*>(lds + kOffF);
    // State route: an item's penalty inputs (history bitmap B, repeat hash X and
    // bitmap R, history tokens staged in F at their id-order ranks) are built from
    // `pf` while the previous item compacts and publishes, in two halves around a
    // barrier.  First half: X and R emptied, B and this thread's bitmap word(s),
    // the words' population scan within the wave.
    uint32_t pen_incl = 0u, pen_pc = 0u;
    auto state_pen_a = [&](int r1, int s1, int par) {
        const int tid = opaque_tid(), lane = tid & (kWave - 1), wave = tid / kWave;
        const Geo g1 = geo_of(a, r1, s1);
        uint32_t* X = reinterpret_cast<uint32_t*>(lds + kOffX);
        uint32_t* R = reinterpret_cast<uint32_t*>(lds + kOffR);
        for (int i = tid; i < kHash; i += kT) X[i] = 0u;
        if (tid == 0) { sh.n_hash = 0u; sh.overflow = 0u; }
        const int nw = (g1.n + 31) >> 5;
        const uint32_t lastm = (g1.n & 31) ? (1u << (g1.n & 31)) - 1u : ~0u;
        uint32_t pc_ = 0u;
#pragma unroll
        for (int q = 0; q < kWPT; ++q) {
            const int wd = tid * kWPT + q;
            bw[q] = wd < nw ? (pf.bword[q] & (wd == nw - 1 ? lastm : ~0u)) : 0u;
            B[wd] = bw[q];
            R[wd] = 0u;
            pc_ += uint32_t(__builtin_popcount(bw[q]));
        }
        const uint32_t hflags = uint32_t(__builtin_amdgcn_readfirstlane(int(pf.hflags)));
        if (tid == 0 && hflags) atomicOr(&sh.pflags[par], hflags & (VI_FLAG_BAD_HISTORY | VI_FLAG_ERROR));
        pen_pc = pc_;
        pen_incl = wave_incl_scan_u32(pc_);
        if (lane == kWave - 1) sh.scan[wave] = pen_incl;
    };
    // Second half: the ranks, the repeat counts of the item's tokens from the
    // state's repeat list, the staging (then a barrier before F is read).
    auto state_pen_b = [&](int r1, int s1) {
        const int tid = opaque_tid(), lane = tid & (kWave - 1), wave = tid / kWave;
        const Geo g1 = geo_of(a, r1, s1);
        const PenCtx c1 = pen_ctx(a, r1, a.params[r1]);
        const uint32_t st = lane < kW ? sh.scan[lane] : 0u;
        const uint32_t si = wave_incl_scan_u32(st);
        nf = uint32_t(readlane_i(int(si), kW - 1));
        rank0 = (wave > 0 ? uint32_t(readlane_i(int(si), wave - 1)) : 0u) + pen_incl - pen_pc;
        const uint2* list = reinterpret_cast<const uint2*>(c1.lstate + a.pl.off_list);
        const uint32_t nrep = min(uint32_t(__builtin_amdgcn_readfirstlane(int(pf.nrep))), uint32_t(a.pl.slots));
        const int e1 = g1.s0 + g1.n;
        auto put = [&](uint2 e) {
            const int t = int(e.x);
            if (e.y < 2u || t < g1.s0 || t >= e1) return;
            repeat_put(lds, sh, uint32_t(t - g1.s0), e.y - 1u, false);
        };
#pragma unroll
        for (int j = 0; j < kPL; ++j)
            if (uint32_t(j) * kT + tid < nrep) put(pf.le[j]);
        for (uint32_t i = uint32_t(kPL) * kT + tid; i < nrep; i += kT) put(list[i]);
        uint32_t r = rank0;
#pragma unroll
        for (int q = 0; q < kWPT; ++q) {
            uint32_t bits = bw[q];
            while (bits && r < uint32_t(kStage)) {
                const int j = __builtin_ctz(bits);
                bits &= bits - 1u;
                F[r++] = uint16_t((tid * kWPT + q) * 32 + j);
            }
        }
    };
    // (after the barrier that follows state_pen_b) the dense counts when X overflowed
    auto state_pen_dense = [&](int r1, int s1) {
        if (sh.overflow)   // (uniform)
            pen_dense_fill(a, pen_ctx(a, r1, a.params[r1]), geo_of(a, r1, s1), pf,
                           a.lists + (size_t(r1) * S + s1) * kSL);
    };
    bool cur_pen = false;   // the item's penalty inputs were built ahead (state route)
    {
        const vi_row_params p0 = a.params[row];
        if (full_route_row(p0)) {
            const Geo g0 = geo_of(a, row, s);
            const PenCtx pc0 = pen_ctx(a, row, p0);
            load_slice(g0, cur);
            pen_prefetch_head(a, pc0, g0, pf);
            cur_pen = state_route && pc0.pen;
        }
    }
    lds_barrier();
    if (cur_pen) {   // (uniform) item 0's penalty inputs
        state_pen_a(row, s, 0);
        lds_barrier();
        state_pen_b(row, s);
        lds_barrier();
        state_pen_dense(row, s);
    }

    // One slice per iteration.  `cur` / `pf` hold its logits and penalty inputs,
    // requested during the previous iteration: the next slice's logits are loaded
    // into `cur` as soon as this slice's histogram has consumed it, and land
    // while the penalties, the compaction and the publication run.  Barriers
    // order LDS only, so nothing but the loop's first wait waits for them.
    // (Only the item indices are carried between iterations: parameters and
    // geometry are reloaded from the constant cache where they are used.)
    for (int k = 0;; ++k) {
        // this slice's loads have landed (and the previous slice's stores)
        __builtin_amdgcn_s_waitcnt(0x0f70);
        const int tid = opaque_tid();
        if (k % kW == 0) {   // the valid key ranges of this item and the next kW - 1, a wave each
            int r2 = 0, s2 = 0;
            if (item_of(a, w, k + tid / kWave, &r2, &s2)) {
                const uint32_t km = valid_key_range<DT>(a.params[r2].temperature);
                if ((tid & (kWave - 1)) == 0) sh.krange[tid / kWave] = km;
            }
        }
        const int lane = tid & (kWave - 1), wave = tid / kWave;
        int nrow = 0, ns = 0;
        const bool has_next = item_of(a, w, k + 1, &nrow, &ns);
        const vi_row_params p = a.params[row];
        const Geo g = geo_of(a, row, s);
        const PenCtx pc = pen_ctx(a, row, p);
        const bool full = full_route_row(p);
        const float inv_t = 1.0f / p.temperature;
        // the next slice's penalty inputs, then its logits (into the registers this
        // slice's logits occupied)
        auto prefetch_next = [&]() {
            if (!has_next) return;
            const vi_row_params np = a.params[nrow];
            if (!full_route_row(np)) return;
            const Geo ng = geo_of(a, nrow, ns);
            pen_prefetch_head(a, pen_ctx(a, nrow, np), ng, pf);
            load_slice(ng, cur);
        };
        uint32_t* dense = a.lists + (size_t(row) * S + s) * kSL;
        constexpr int kG = kStage / kT;   // history tokens gathered per thread and round
        uint32_t graw[kG], goff[kG];
#pragma unroll
        for (int u = 0; u < kG; ++u) { graw[u] = 0u; goff[u] = 0xffffffffu; }
        // the next item's penalty inputs are built during this one (state route)
        bool next_pen = false;
        if (state_route && has_next) {
            const vi_row_params np = a.params[nrow];
            next_pen = full_route_row(np) && penalties_active(np);
        }

        if (full) {
            if (tid == 0) sh.flags = 0u;
            // ---- 1. penalties: the slice's history bitmap B, the repeat hash X / bitmap
            // R, and the first round of history tokens staged in id order with their
            // raw logits requested (before the next slice's loads).  State route:
            // built during the previous item (or before the loop), F staged.
            if (pc.pen) {
                if (!pc.state) {
                    pen_build<DT>(a, pc, g, pf, lds, sh, dense);
                    uint32_t pc_ = 0u;
                    uint32_t* hb = a.hbits + (size_t(row) * S + s) * kBW;   // (for the merge's owner scan)
#pragma unroll
                    for (int q = 0; q < kWPT; ++q) {
                        bw[q] = B[tid * kWPT + q];
                        hb[tid * kWPT + q] = bw[q];
                        pc_ += __builtin_popcount(bw[q]);
                    }
                    rank0 = block_scan_lds(pc_, sh.scan, &nf);
                    // this thread's history tokens, staged at their ranks
                    uint32_t r = rank0;
#pragma unroll
                    for (int q = 0; q < kWPT; ++q) {
                        uint32_t bits = bw[q];
                        while (bits && r < uint32_t(kStage)) {
                            const int j = __builtin_ctz(bits);
                            bits &= bits - 1u;
                            F[r++] = uint16_t((tid * kWPT + q) * 32 + j);
                        }
                    }
                    lds_barrier();
                }
                const uint32_t m = min(uint32_t(kStage), nf);
#pragma unroll
                for (int u = 0; u < kG; ++u) {
                    const uint32_t e = uint32_t(u) * kT + tid;
                    goff[u] = e < m ? uint32_t(F[e]) : 0xffffffffu;
                    graw[u] = e < m ? uint32_t(g.base16[goff[u]]) : 0u;
                }
            }
        }
        if (full) {
            // ---- 2. raw-pattern histogram of the slice (no returned values: the
            // adds stream through the LDS).  Vectors past the slice's end are skipped
            // by a branch that is uniform in all waves but one (masked adds of 0
            // would all hit one word and serialize).
            auto hist_add = [&](uint32_t b) { atomicAdd(&H[b & 0x7fffu], (b & 0x8000u) ? 0x10000u : 1u); };
            if (pc.pen) {   // history tokens are left out here: the moves add their penalized patterns
                auto hist8 = [&](uint32_t off) {   // B bits off .. off + 7
                    const uint32_t wd = off >> 5, sft = off & 31u;
                    const uint64_t two = uint64_t(B[wd]) | (sft > 24u && wd + 1u < uint32_t(kBW) ? uint64_t(B[wd + 1u]) << 32 : 0ull);
                    return uint32_t(two >> sft) & 0xffu;
                };
                const unsigned char* B8 = reinterpret_cast<const unsigned char*>(B);
#pragma unroll
                for (int i = 0; i < kNV; ++i) {
                    const int vi = i * kT + tid;
                    if (vi < g.nvec) {
                        // (a history token adds 0 to its raw pattern's word: no per-element branch)
                        const uint32_t h8 = g.head == 0 ? uint32_t(B8[vi]) : hist8(uint32_t(g.head + 8 * vi));
                        const uint32_t w4[4] = {cur.v[i].x, cur.v[i].y, cur.v[i].z, cur.v[i].w};
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const uint32_t b = (j & 1) ? (w4[j >> 1] >> 16) : (w4[j >> 1] & 0xffffu);
                            atomicAdd(&H[b & 0x7fffu], ((h8 >> j) & 1u) ? 0u : ((b & 0x8000u) ? 0x10000u : 1u));
                        }
                    }
                }
                if (tid < g.head && !((B[tid >> 5] >> (tid & 31)) & 1u)) hist_add(cur.hb);
                const uint32_t to = uint32_t(g.head + 8 * g.nvec + tid);
                if (tid < g.tail && !((B[to >> 5] >> (to & 31)) & 1u)) hist_add(cur.tb);
            } else {
#pragma unroll
                for (int i = 0; i < kNV; ++i) {
                    if (i * kT + tid < g.nvec) {
                        const uint32_t w4[4] = {cur.v[i].x, cur.v[i].y, cur.v[i].z, cur.v[i].w};
#pragma unroll
                        for (int j = 0; j < 8; ++j) hist_add((j & 1) ? (w4[j >> 1] >> 16) : (w4[j >> 1] & 0xffffu));
                    }
                }
                if (tid < g.head) hist_add(cur.hb);
                if (tid < g.tail) hist_add(cur.tb);
            }
            prefetch_next();

            // ---- 3. the history tokens' penalized patterns (non-finite logits keep
            // their own)
            if (pc.pen) {
                // (all the patterns first, then the adds: the count lookups do not
                // wait behind earlier atomics)
                // (the patterns also go to the slice's table, by rank: the merge's
                // owner scan reads them instead of penalizing again)
                uint16_t* tab = a.ptab + (size_t(row) * S + s) * kSL;
                auto moves = [&](const uint32_t* off, const uint32_t* b, uint32_t c0) {
                    uint32_t pb[kG];
#pragma unroll
                    for (int u = 0; u < kG; ++u)
                        pb[u] = (off[u] != 0xffffffffu && Elem<DT>::finite_bits(b[u]))
                                    ? penalize_bits<DT>(b[u], pen_count(lds, sh, dense, off[u]), p) & 0xffffu
                                    : b[u];
#pragma unroll
                    for (int u = 0; u < kG; ++u) {
                        if (off[u] != 0xffffffffu) {
                            hist_add(pb[u]);
                            tab[c0 + uint32_t(u) * kT + tid] = uint16_t(pb[u]);
                        }
                    }
                };
                moves(goff, graw, 0u);
                for (uint32_t c0 = kStage; c0 < nf; c0 += kStage) {   // (long histories) further rounds
                    lds_barrier();   // (every thread has read the staged offsets)
                    uint32_t r = rank0;
#pragma unroll
                    for (int q = 0; q < kWPT; ++q) {
                        uint32_t bits = bw[q];
                        while (bits) {
                            const int j = __builtin_ctz(bits);
                            bits &= bits - 1u;
                            if (r >= c0 && r < c0 + kStage) F[r - c0] = uint16_t((tid * kWPT + q) * 32 + j);
                            ++r;
                        }
                    }
                    lds_barrier();
                    const uint32_t m = min(uint32_t(kStage), nf - c0);
                    uint32_t rr[kG], oo[kG];
#pragma unroll
                    for (int u = 0; u < kG; ++u) {
                        const uint32_t e = uint32_t(u) * kT + tid;
                        oo[u] = e < m ? uint32_t(F[e]) : 0xffffffffu;
                        rr[u] = e < m ? uint32_t(g.base16[oo[u]]) : 0u;
                    }
                    moves(oo, rr, c0);
                }
            }
            lds_barrier();

            // ---- 4. compaction, one pass over the histogram.  Thread t takes the
            // words of patterns d = 2 (q kT + t) + j (q < kQ, j < 2): a wave's 128
            // patterns of round q are the block m = q kW + wave, which fills exactly
            // one coarse bin of each sign (bins of 128 keys, bin = key >> 7):
            // positive keys 0x8000 | d in bin 256 + m, negative keys 0x7fff - d in
            // bin 255 - m.  A block's entries take one region of the slice's list,
            // [positive][negative], each bin's entries in ascending key order.  Bin
            // masses are sums of count * exp(z - z(bin's largest key)), one wave's
            // reduction in a fixed order; the weights only locate bins (the merge
            // resolves inside a bin in double precision): single precision,
            // |error| <= 1e-7 of the bin's largest weight.
            const uint32_t km = sh.krange[k % kW], kmin = km & 0xffffu, kmax = km >> 16;
            // the two words of round q, -0 merged into +0 (both z = 0)
            auto words = [&](int q) {
                uint2 v = H2[q * kT + tid];
                if (q == 0 && tid == 0) v.x = (v.x & 0xffffu) + (v.x >> 16);
                return v;
            };
            // weight of `cnt` logits of `key` in a bin whose largest logit is xr
            auto weight = [&](uint32_t key, float xr, uint32_t cnt) {
                // (x - x_ref) / T: the difference of two logits is exact when within a
                // factor 2 (Sterbenz) and within half an ulp otherwise; (finite inv_t:
                // the product is finite or -inf, never NaN)
                const float x = Elem<DT>::decode(unkey16(key));
                return float(cnt) * __builtin_amdgcn_exp2f(((x - xr) * inv_t) * 1.44269504088896340736f);
            };
            uint32_t* list = a.lists + (size_t(row) * S + s) * kSL;
            uint4* rec = a.brec + (size_t(row) * S + s) * kBins;
            bool invalid = false;
            // the wave's non-empty rounds (wave-uniform bits), from reads issued back to
            // back; then one iteration per non-empty round
            uint32_t rounds = 0u;
#pragma unroll
            for (int q = 0; q < kQ; ++q) {
                const uint2 v = H2[q * kT + tid];
                rounds |= ballot((v.x | v.y) != 0u) ? 1u << q : 0u;
            }
            rounds = uint32_t(__builtin_amdgcn_readfirstlane(int(rounds)));
#pragma unroll 1
            while (rounds) {
                const int q = __builtin_ctz(rounds);
                rounds &= rounds - 1u;
                const uint2 v = words(q);
                if ((v.x | v.y) != 0u) H2[q * kT + tid] = make_uint2(0u, 0u);   // empty again for the next slice
                const int m = q * kW + wave;
                const uint32_t d0 = uint32_t(2 * (q * kT + tid));
                // valid entries: bit j of pm / nm for the positive / negative pattern of
                // d0 + j; a block whose keys all lie in [kmin, kmax] (wave-uniform test)
                // needs no per-word key test
                const uint32_t w2[2] = {v.x, v.y};
                uint32_t pm = 0u, nm = 0u;
                const uint32_t dl = uint32_t(m) * 128u + 127u;   // the block's largest d
                if ((0x8000u | dl) <= kmax && 0x7fffu - dl >= kmin) {
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        pm |= (w2[j] & 0xffffu) ? 1u << j : 0u;
                        nm |= (w2[j] >> 16) ? 1u << j : 0u;
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const uint32_t d = d0 + uint32_t(j), cp = w2[j] & 0xffffu, cn = w2[j] >> 16;
                        const uint32_t kp = 0x8000u | d, kn = 0x7fffu - d;
                        const bool vp = kp >= kmin && kp <= kmax, vn = kn >= kmin && kn <= kmax;
                        pm |= (cp && vp) ? 1u << j : 0u;
                        nm |= (cn && vn) ? 1u << j : 0u;
                        invalid |= (cp && !vp) || (cn && !vn);
                    }
                }
                const uint32_t ne = uint32_t(__builtin_popcount(pm)) | (uint32_t(__builtin_popcount(nm)) << 16);
                const uint32_t ie = wave_incl_scan_u32(ne);
                const uint32_t e63 = uint32_t(readlane_i(int(ie), kWave - 1));
                if (e63 == 0u) continue;   // (wave-uniform) nothing valid in the block
                const uint32_t NP = e63 & 0xffffu, NB = e63 >> 16;
                uint32_t base = 0u;
                if (lane == 0) base = atomicAdd(&sh.n_list, NP + NB);
                // valid logits per sign (packed halves add without carry: a slice has at
                // most 32,768 logits) and the bins' largest valid keys
                const uint32_t vc = ((pm & 1u) ? (v.x & 0xffffu) : 0u) + ((pm & 2u) ? (v.y & 0xffffu) : 0u) +
                                    ((nm & 1u) ? (v.x & 0xffff0000u) : 0u) + ((nm & 2u) ? (v.y & 0xffff0000u) : 0u);
                const uint32_t c63 = wave_sum_u32(vc);
                const uint32_t pk = pm ? 0x8000u | (d0 + ((pm & 2u) ? 1u : 0u)) : 0u;   // largest: the last j
                const uint32_t nk = nm ? 0x7fffu - (d0 + ((nm & 1u) ? 0u : 1u)) : 0u;   // largest: the first j
                const uint64_t bp = ballot(pk != 0u), bn = ballot(nk != 0u);
                const uint32_t pkm = bp ? uint32_t(readlane_i(int(pk), 63 - __builtin_clzll(bp))) : 0u;
                const uint32_t nkm = bn ? uint32_t(readlane_i(int(nk), __builtin_ctzll(bn))) : 0u;
                base = uint32_t(__builtin_amdgcn_readfirstlane(int(base)));
                // entries in key order, and masses
                const uint32_t ex = ie - ne;
                uint32_t ip = base + (ex & 0xffffu);
                uint32_t in_ = base + NP + NB - 1u - (ex >> 16);
                const float xp = Elem<DT>::decode(unkey16(max(pkm, 1u)));
                const float xn = Elem<DT>::decode(unkey16(max(nkm, 1u)));
                float mp = 0.0f, mn = 0.0f;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const uint32_t d = d0 + uint32_t(j);
                    if ((pm >> j) & 1u) {
                        const uint32_t kp = 0x8000u | d, cp = w2[j] & 0xffffu;
                        list[ip++] = (kp << 16) | cp;
                        mp += weight(kp, xp, cp);
                    }
                    if ((nm >> j) & 1u) {
                        const uint32_t kn = 0x7fffu - d, cn = w2[j] >> 16;
                        list[in_--] = (kn << 16) | cn;
                        mn += weight(kn, xn, cn);
                    }
                }
                const float sp = wave_sum_f32(mp), sn = wave_sum_f32(mn);
                if (lane == 0) {
                    auto put = [&](int b, uint32_t first, uint32_t n, uint32_t cnt, uint32_t ref, float ms) {
                        const uint64_t mb = __builtin_bit_cast(uint64_t, double(ms));
                        rec[b] = make_uint4(first | (n << 16), cnt | (ref << 16), uint32_t(mb), uint32_t(mb >> 32));
                    };
                    const int bp_ = 256 + m, bn_ = 255 - m;
                    if (NP) { put(bp_, base, NP, c63 & 0xffffu, pkm, sp); atomicOr(&sh.bmask[bp_ >> 5], 1u << (bp_ & 31)); }
                    if (NB) { put(bn_, base + NP, NB, c63 >> 16, nkm, sn); atomicOr(&sh.bmask[bn_ >> 5], 1u << (bn_ & 31)); }
                    atomicAdd(&sh.n_valid, (c63 & 0xffffu) + (c63 >> 16));
                    atomicMax(&sh.top_key, max(pkm, nkm));
                }
            }
            // the next item's penalty inputs, first half (B, X, R and F are free: this
            // item's moves are done)
            if (next_pen) state_pen_a(nrow, ns, (k + 1) & 1);
            if (ballot(invalid) && lane == 0) atomicOr(&sh.flags, uint32_t(VI_FLAG_NONFINITE));
            lds_barrier();
            // ---- publish the slice's head (the merge is a later launch: plain
            // stores); each word is emptied by the thread that read it
            uint32_t* hd = a.heads + (size_t(row) * S + s) * kHeadWords;
            if (tid == 0) {
                hd[0] = sh.n_list;
                hd[1] = sh.n_valid;
                hd[2] = sh.flags | sh.pflags[k & 1];
                sh.pflags[k & 1] = 0u;
                hd[3] = sh.top_key;
                hd[4 + kBins / 32] = nf;
                sh.n_list = 0u; sh.n_valid = 0u; sh.top_key = 0u;
            }
            if (tid < kBins / 32) {
                hd[4 + tid] = sh.bmask[tid];
                sh.bmask[tid] = 0u;
            }
            if (next_pen) state_pen_b(nrow, ns);
            lds_barrier();
            if (next_pen) state_pen_dense(nrow, ns);
        } else {
            prefetch_next();
            if (next_pen) {
                state_pen_a(nrow, ns, (k + 1) & 1);
                lds_barrier();
                state_pen_b(nrow, ns);
                lds_barrier();
                state_pen_dense(nrow, ns);
            }
        }
        if (!has_next) break;
        row = nrow; s = ns;
    }
}

// One workgroup per full-route row: the decisions and the token.
template <int DT>
__global__ __launch_bounds__(kT) void merge_kernel(SliceArgs a) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[kLds];
    __shared__ Shared sh;
    const int row = blockIdx.x;
    const vi_row_params p = a.params[row];
    if (!full_route_row(p)) return;
    const float inv_t = 1.0f / p.temperature;
    if (threadIdx.x / kWave == 0) {
        const uint32_t km = valid_key_range<DT>(p.temperature);
        if (lane_id() == 0) { sh.kmin = km & 0xffffu; sh.kmax = km >> 16; }
    }
    __syncthreads();
    merge_row<DT>(a, row, p, inv_t, lds, sh);
}

// Filtered distribution of the full-route rows (test / diagnostics path): per
// slice, the penalized logits' keys decide support membership (keys above the
// support's end key; of the end key, the first end_take in id order over the
// row), and the support gets exp(z - z0) / S_n.
template <int DT>
__global__ __launch_bounds__(kT) void slice_probs_kernel(SliceArgs a) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[kLds];
    __shared__ Shared sh;
    const int w = blockIdx.x, S = a.slices;
    int row = 0, s = 0;
    for (int k = 0; item_of(a, w, k, &row, &s); ++k) {
        // (the thread index laundered per item: values derived from it stay
        // in the loop instead of being hoisted out of it and spilled)
        const int tid = opaque_tid();
        const vi_row_params p = a.params[row];
        if (!full_route_row(p)) continue;
        const RowBound bd = a.bounds[row];
        const Geo g = geo_of(a, row, s);
        float* pr = a.probs + size_t(row) * size_t(a.probs_stride) + g.s0;
        if (!bd.valid) {
            for (int i = tid; i < g.n; i += kT) pr[i] = 0.0f;
            continue;
        }
        SliceRegs r;
        load_slice(g, r);
        const PenCtx pc = pen_ctx(a, row, p);
        uint32_t* dense = a.lists + (size_t(row) * S + s) * kSL;
        if (pc.pen) {
            if (tid == 0) sh.flags = 0u;
            PenPrefetch f{};
            pen_prefetch_head(a, pc, g, f);
            pen_build<DT>(a, pc, g, f, lds, sh, dense);
        }
        // pass 1: logits of the support's end key, in id order
        uint32_t mask[kSeg], cnt[kSeg], excl[kSeg];
        const uint32_t ek = bd.end_key;
        // with record = 1 the sampler has already recorded the row's token into the
        // lane's state: the distribution is the one before that occurrence
        uint32_t unrec = ~0u;
        if (a.record && pc.pen) {
            const int32_t t = a.tokens[row];
            if (t >= g.s0 && t < g.s0 + g.n) unrec = uint32_t(t - g.s0);
        }
        auto keyof = [&](uint32_t off, uint32_t b) { return elem_key<DT>(lds, sh, dense, p, pc.pen, off, b, unrec); };
        mask[0] = (tid < g.head && keyof(uint32_t(tid), r.hb) == ek) ? 1u : 0u;
        mask[kSeg - 1] = (tid < g.tail && keyof(uint32_t(g.head + 8 * g.nvec + tid), r.tb) == ek) ? 1u : 0u;
#pragma unroll
        for (int i = 0; i < kNV; ++i) {
            const int v = i * kT + tid;
            uint32_t mm = 0u;
            if (v < g.nvec) {
#pragma unroll 1
                for (int j = 0; j < 8; ++j)
                    if (keyof(uint32_t(g.head + 8 * v + j), vec_elem(r.v[i], j)) == ek) mm |= 1u << j;
            }
            mask[1 + i] = mm;
        }
#pragma unroll
        for (int x = 0; x < kSeg; ++x) cnt[x] = __builtin_popcount(mask[x]);
        (void)id_order_prefix(cnt, excl, sh);
        const uint32_t base = bd.end_take == kTakeAll ? 0u : a.bases[size_t(row) * kFullBaseSlots + s];
        auto prob = [&](uint32_t key, uint32_t rank) -> float {
            if (!key || key < ek) return 0.0f;
            if (key == ek && bd.end_take != kTakeAll && base + rank >= bd.end_take) return 0.0f;
            const float z = key_z<DT>(key, bd.inv_t);
            return isfinite(z) ? float(exp(double(z) - bd.z0) / bd.s_n) : 0.0f;
        };
        // pass 2: probabilities
        if (tid < g.head) pr[tid] = prob(keyof(uint32_t(tid), r.hb), excl[0]);
        if (tid < g.tail)
            pr[g.head + 8 * g.nvec + tid] = prob(keyof(uint32_t(g.head + 8 * g.nvec + tid), r.tb), excl[kSeg - 1]);
#pragma unroll
        for (int i = 0; i < kNV; ++i) {
            const int v = i * kT + tid;
            if (v >= g.nvec) continue;
            uint32_t rk = excl[1 + i];
            float* out = pr + g.head + 8 * v;
#pragma unroll 1
            for (int j = 0; j < 8; ++j) {
                out[j] = prob(keyof(uint32_t(g.head + 8 * v + j), vec_elem(r.v[i], j)), rk);
                rk += (mask[1 + i] >> j) & 1u;
            }
        }
        __syncthreads();
    }
}


inline int slices_of(int vocabulary) { return (vocabulary + kSL - 1) / kSL; }

}  // namespace

SideStream* side_stream() {
    // (one per host thread and device: concurrent callers never share events)
    thread_local SideStream side[64];
    thread_local bool tried[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    SideStream& x = side[dev];
    if (!tried[dev]) {
        tried[dev] = true;
        if (hipStreamCreateWithFlags(&x.stream, hipStreamNonBlocking) != hipSuccess ||
            hipEventCreateWithFlags(&x.fork, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&x.join, hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            x.stream = nullptr;
        }
    }
    return x.stream ? &x : nullptr;
}

int device_cus() {
    static int cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

bool full_supported(int dtype, int vocabulary, int64_t stride) {
    return (dtype == VI_BF16 || dtype == VI_F16) && vocabulary > 0 && vocabulary <= kMaxSlices * kSL &&
           stride >= vocabulary;
}

size_t full_workspace(int rows, int vocabulary) {
    if (rows <= 0 || vocabulary <= 0) return 0;
    const size_t rs = size_t(rows) * size_t(slices_of(vocabulary));
    return align_up(rs * kHeadWords * 4, 256) + align_up(rs * kBins * 16, 256) + align_up(rs * kSL * 4, 256) +
           align_up(rs * kSL * 2, 256) + align_up(rs * kBW * 4, 256) +
           align_up(size_t(rows) * sizeof(RowBound), 256) +
           align_up(size_t(rows) * kFullBaseSlots * 4, 256) + 256;
}

vi_status launch_full(const SampleArgs& s, unsigned char* ws, size_t ws_bytes, hipStream_t stream) {
    if (reinterpret_cast<uintptr_t>(s.logits) % 16) return VI_ERR_UNSUPPORTED;
    if (!full_supported(s.dtype, s.vocabulary, s.stride)) return VI_ERR_UNSUPPORTED;
    SliceArgs a{};
    a.slices = slices_of(s.vocabulary);
    const size_t rs = size_t(s.rows) * size_t(a.slices);
    Carver c(ws, ws_bytes);
    a.heads = c.take<uint32_t>(rs * kHeadWords);
    a.brec = c.take<uint4>(rs * kBins);
    a.lists = c.take<uint32_t>(rs * kSL);
    a.ptab = c.take<uint16_t>(rs * kSL);
    a.hbits = c.take<uint32_t>(rs * kBW);
    a.bounds = c.take<RowBound>(size_t(s.rows));
    a.bases = c.take<uint32_t>(size_t(s.rows) * kFullBaseSlots);
    if (!c.ok) return VI_ERR_WORKSPACE;
    a.logits = s.logits; a.rows = s.rows; a.vocabulary = s.vocabulary; a.stride = s.stride;
    a.params = s.params; a.histories = s.histories; a.offsets = s.offsets;
    if (s.pstate) { a.pstate = s.pstate; a.pl = s.playout; a.record = s.record; }
    a.tokens = s.tokens; a.uniforms = s.uniforms; a.probs = s.probs; a.probs_stride = s.probs_stride;
    a.stats = s.stats;
    if (s.full_out) { a.bounds = s.full_out->bounds; a.bases = s.full_out->bases; }
    a.want_bounds = (s.probs || s.full_out) ? 1 : 0;
    const int items = s.rows * a.slices;
    a.grid = std::min(device_cus(), items);
    a.xcd_aware = (s.rows >= 8 && a.grid % 8 == 0) ? 1 : 0;
    if (s.dtype == VI_BF16) {
        hipLaunchKernelGGL(slice_kernel<VI_BF16>, dim3(a.grid), dim3(kT), 0, stream, a);
        hipLaunchKernelGGL(merge_kernel<VI_BF16>, dim3(s.rows), dim3(kT), 0, stream, a);
    } else {
        hipLaunchKernelGGL(slice_kernel<VI_F16>, dim3(a.grid), dim3(kT), 0, stream, a);
        hipLaunchKernelGGL(merge_kernel<VI_F16>, dim3(s.rows), dim3(kT), 0, stream, a);
    }
    vi_status st = launch_status();
    if (st != VI_OK || !s.probs) return st;
    if (s.dtype == VI_BF16) hipLaunchKernelGGL(slice_probs_kernel<VI_BF16>, dim3(a.grid), dim3(kT), 0, stream, a);
    else hipLaunchKernelGGL(slice_probs_kernel<VI_F16>, dim3(a.grid), dim3(kT), 0, stream, a);
    return launch_status();
}

}  // namespace vi
