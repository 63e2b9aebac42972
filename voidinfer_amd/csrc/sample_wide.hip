// sample_wide.hip — full-vocabulary rows of the batched sampler for fp32
// logits (temperature > 0 and top_k = 0 or > 64): penalties, temperature,
// top-k / min-p / top-p over the whole vocabulary and the Philox inverse-CDF
// draw.  Semantics as the 16-bit route's: order (z desc, id asc), weights
// exp(z - z_max), the cap, the min-p and top-p cuts, the draw.
//
// A 16-bit logit takes one of 65,536 patterns, so a count per pattern
// describes its row exactly; a 32-bit one does not.  Here a row is described
// in two levels, both keyed by z = x' * (1/T) itself:
//   * bins of z: bin j holds floor(64 z) = anchor - j, counted down from the
//     largest z (anchor = floor(64 z_max)).  4,096 bins of width 1/64 cover the
//     64 below the top; one deep bin holds the rest, whose weights (below
//     e^-63 of the largest) are counted but carry no mass.  A logit's weight
//     inside its bin, exp(z - bin floor) in [1, e^(1/64)), is kept as 2^-31
//     fixed point: bin masses are integer sums, exact in any order, and every
//     later sum over the same logits gives the same integers;
//   * the logits of the one bin a decision lands in, narrowed by 8-bit digits
//     of the 32-bit order key until one key remains; the rank among equal keys
//     follows from their common weight, the owner from their ids.
//
// Launches: (history route with penalties) the rows' presence bitmaps and
// count hashes; one workgroup per (row, slice of 16,384 logits) counts and
// weighs its bins (written over the occupied bins only) and writes the (key,
// id) pairs of its first 4,096 list positions grouped by bin; one workgroup per
// row adds the slices' bins, places the cap, the cuts and the draw, and names
// the token, recomputing from the slice's logits the pairs of a bin that lies
// past the written positions; optionally the filtered distribution.
//
// Roofline: HBM; V x 4 bytes of logits per row read once; per slice the
// occupied bins' counts and masses and at most 4,096 pairs written, a few bins
// of them read back.
#include <math.h>

#include "penalty_state.h"
#include "vi_device.h"
#include "vi_internal.h"

namespace vi {
namespace {

constexpr int kT = 1024;
constexpr int kW = kT / kWave;
constexpr int kSL = 16384;                 // logits per slice (slice offsets fit 16 bits)
constexpr int kVPT = kSL / (4 * kT);       // 16-byte vectors per thread and slice
constexpr int kMaxSlices = 32;
constexpr int kNB = 4096;                  // bins of width 1/64 below the top
constexpr int kDeep = kNB;                 // everything further down
constexpr int kStarts = kNB + 2;           // per slice: first list position of bins 0..kNB, then n_valid
constexpr double kPerUnit = 64.0;
constexpr float kFixUnit = 2147483648.0f;  // 2^31
constexpr double kFixScale = 1.0 / 2147483648.0;
constexpr int kCap = 8192;                 // logits of one bin staged in LDS (more are read from HBM)
constexpr int kPairs = 4096;               // list positions whose pairs the slice pass writes
constexpr int kDig = 256;
constexpr uint32_t kTakeAll = 0xffffffffu;
static_assert(kVPT * 4 * kT == kSL && kNB == 4 * kT, "slice and bin geometry");

struct WideHead {
    double anchor;                 // floor(64 z_top) of the slice
    uint32_t top_key, n_valid, flags;
    uint32_t nbins;                // bins 0 .. nbins - 1 may hold logits (the rest only the deep bin)
    uint32_t npairs;               // list positions 0 .. npairs - 1 written
    uint32_t pad;
};
static_assert(sizeof(WideHead) == 32, "slice head");

using WideBound = FullBound;   // what the probs kernel and verification need to rebuild the support
static_assert(kSL == kFullSlice32 && kMaxSlices == kFullBaseSlots, "full-route bases");

struct WideArgs {
    const void* logits;
    int rows, vocabulary, slices;
    int64_t stride;
    const vi_row_params* params;
    unsigned char* pstate;         // per-lane penalty states (or null: histories)
    PenaltyLayout pl;
    const int32_t* histories;
    const int64_t* offsets;
    int64_t max_history;
    uint32_t* hbits;               // [rows][words] presence bitmaps (history route)
    int words;
    uint2* hash;                   // [rows][hash_slots] (token + 1, count) (history route)
    int hash_shift, hash_slots;
    uint32_t* row_flags;           // [rows] history flags (history route)
    int record;
    int32_t* tokens;
    double* uniforms;
    float* probs;
    int64_t probs_stride;
    vi_sample_stats* stats;
    // workspace
    WideHead* heads;               // [rows][slices]
    uint32_t* starts;              // [rows][slices][kStarts]: bins 0 .. nbins, kNB, kNB + 1 written
    unsigned long long* mass;      // [rows][slices][kNB]: fixed-point bin masses, bins 0 .. nbins - 1
    uint32_t* keys;                // [rows][slices][kSL]: order keys, grouped by bin (first npairs
    uint16_t* ids;                 // [rows][slices][kSL]: slice offsets, same order   written, the rest on demand)
    int want_bounds;               // bounds and bases wanted (probs, or verification)
    WideBound* bounds;             // [rows]
    uint32_t* bases;               // [rows][kMaxSlices]: end-key logits in the slices before
};

__device__ __forceinline__ bool full_row(const vi_row_params& p) { return !topk_route(p); }

// Order key of a finite z (+0 and -0 share +0's), and back.  Finite z have
// keys in [0x00800000, 0xff7fffff]; key 0 marks "no valid logit".
__device__ __forceinline__ uint32_t key32(float z) {
    uint32_t u = __builtin_bit_cast(uint32_t, z);
    if (z == 0.0f) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float unkey32(uint32_t k) {
    return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Bin of key k below `anchor` (kDeep past the 4,096th) and its weight
// exp(z - bin floor) in 2^-31 units (0 in the deep bin).  64 z is exact in
// double and its floor and fraction too; the weight is one hardware exp2.
struct BinW {
    int bin;
    uint32_t fix;
};
__device__ __forceinline__ BinW bin_weight(uint32_t k, double anchor) {
    const double zz = double(unkey32(k)) * kPerUnit;
    const double f = floor(zz);
    const double j = anchor - f;
    if (!(j < double(kNB))) return {kDeep, 0u};
    const float d = float(zz - f);
    const float w = __builtin_amdgcn_exp2f(d * (1.44269504088896340736f / 64.0f));
    return {int(j), uint32_t(rintf(w * kFixUnit))};
}
__device__ __forceinline__ uint32_t weight_fix(uint32_t k) { return bin_weight(k, floor(double(unkey32(k)) * kPerUnit)).fix; }

// ------------------------------------------------------------------ penalties
struct WPen {
    bool on;
    const uint32_t* bits;   // presence bitmap (token t: bit t & 31 of word t >> 5)
    const uint2* table;     // (token + 1, count), linear probing
    int shift, slots;
};
__device__ __forceinline__ WPen wpen(const WideArgs& a, int row, const vi_row_params& p) {
    WPen w{};
    if (!penalties_active(p)) return w;
    if (a.pstate) {
        const unsigned char* st = a.pstate + size_t(row) * a.pl.lane_bytes;
        w.on = true;
        w.bits = reinterpret_cast<const uint32_t*>(st + a.pl.off_b1);
        w.table = reinterpret_cast<const uint2*>(st + a.pl.off_hash);
        w.shift = a.pl.shift;
        w.slots = a.pl.slots;
    } else if (a.histories && a.offsets && a.hash && a.offsets[row + 1] > a.offsets[row]) {
        w.on = true;
        w.bits = a.hbits + size_t(row) * size_t(a.words);
        w.table = a.hash + size_t(row) * size_t(a.hash_slots);
        w.shift = a.hash_shift;
        w.slots = a.hash_slots;
    }
    return w;
}

// Order key of logit t (raw bits b, presence word `word` holding t's bit);
// 0 when x, the penalized x' or z is not finite (*bad set).  `unrecord`: a
// token whose count is one too high (the sampler recorded it already).
__device__ __forceinline__ uint32_t logit_key(const WPen& w, const vi_row_params& p, float inv_t, int t, uint32_t b,
                                              uint32_t word, bool* bad, int unrecord = -1) {
    float x = __builtin_bit_cast(float, b);
    if (!isfinite(x)) { *bad = true; return 0u; }
    if (w.on && ((word >> (t & 31)) & 1u)) {
        uint32_t c = hash_count(w.table, w.shift, w.slots, t);
        if (t == unrecord && c) --c;
        if (c) x = __builtin_bit_cast(float, penalize_bits<VI_F32>(b, c, p));
        if (!isfinite(x)) { *bad = true; return 0u; }
    }
    if (x == 0.0f) x = 0.0f;
    const float z = x * inv_t;
    if (!isfinite(z)) { *bad = true; return 0u; }
    return key32(z);
}

// The history route's presence bitmap and count hash of each full-route row
// with penalties (the top-k route builds its own rows' hashes).
__global__ __launch_bounds__(256) void wide_history_kernel(WideArgs a) {
    const int r = blockIdx.x;
    const vi_row_params p = a.params[r];
    if (!full_row(p) || !penalties_active(p)) return;
    const int64_t b = a.offsets[r], n = a.offsets[r + 1] - b;
    if (n <= 0) return;
    __shared__ uint32_t s_flags;
    if (threadIdx.x == 0) s_flags = 0u;
    uint32_t* bits = a.hbits + size_t(r) * size_t(a.words);
    uint2* table = a.hash + size_t(r) * size_t(a.hash_slots);
    for (int i = threadIdx.x; i < a.words; i += blockDim.x) bits[i] = 0u;
    for (int i = threadIdx.x; i < a.hash_slots; i += blockDim.x) table[i] = make_uint2(0u, 0u);
    __syncthreads();
    if (n > a.max_history) {
        if (threadIdx.x == 0) s_flags = VI_FLAG_ERROR;
    } else {
        for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
            const int32_t t = a.histories[b + i];
            if (t < 0 || t >= a.vocabulary) { atomicOr(&s_flags, uint32_t(VI_FLAG_BAD_HISTORY)); continue; }
            uint32_t s = (uint32_t(t) * 0x9E3779B1u) >> a.hash_shift;
            for (int probe = 0; probe < a.hash_slots; ++probe) {
                const uint32_t old = atomicCAS(&table[s].x, 0u, uint32_t(t) + 1u);
                if (old == 0u || old == uint32_t(t) + 1u) { atomicAdd(&table[s].y, 1u); break; }
                s = (s + 1u) & uint32_t(a.hash_slots - 1);
            }
            atomicOr(&bits[t >> 5], 1u << (t & 31));
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) a.row_flags[r] = s_flags;
}

// Slice geometry: head logits before the first 16-byte boundary, vectors, tail.
struct WGeo {
    int s0, n, head, nvec, tail;
    const uint32_t* base;
};
__device__ __forceinline__ WGeo wgeo(const WideArgs& a, int row, int s) {
    WGeo g;
    g.s0 = s * kSL;
    g.n = min(kSL, a.vocabulary - g.s0);
    g.base = static_cast<const uint32_t*>(a.logits) + int64_t(row) * a.stride + g.s0;
    const uint32_t mis = uint32_t(reinterpret_cast<uintptr_t>(g.base) & 15u);   // (a multiple of 4)
    g.head = min(g.n, int(((16u - mis) & 15u) >> 2));
    g.nvec = (g.n - g.head) / 4;
    g.tail = g.n - g.head - 4 * g.nvec;
    return g;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o; o >>= 1) v = max(v, uint32_t(__shfl_xor(int(v), o, kWave)));
    return v;
}

// ------------------------------------------------------------------ slice pass
// One workgroup per (slice, row).  Thread t holds vectors i kT + t (i < kVPT)
// and one head and one tail logit.
__global__ __launch_bounds__(kT) void wide_slice_kernel(WideArgs a) {
    __shared__ uint32_t CNT[kNB + 1];
    __shared__ unsigned long long MASS[kNB];   // (then the staged pairs' offsets)
    __shared__ __attribute__((aligned(16))) uint32_t SKEY[kPairs];   // the staged pairs' keys
    static_assert(sizeof(MASS) >= kPairs * sizeof(uint16_t), "offset staging");
    __shared__ uint32_t s_top, s_flags, s_nb, s_plim, s_scan[kW + 1];
    const int s = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const vi_row_params p = a.params[row];
    if (!full_row(p)) return;
    const WGeo g = wgeo(a, row, s);
    const uint4* vb = reinterpret_cast<const uint4*>(g.base + g.head);
    uint4 v[kVPT];
#pragma unroll
    for (int i = 0; i < kVPT; ++i) {
        const int x = i * kT + tid;
        v[i] = x < g.nvec ? load16(vb + x) : make_uint4(0u, 0u, 0u, 0u);
    }
    const uint32_t hb = tid < g.head ? g.base[tid] : 0u;
    const uint32_t tb = tid < g.tail ? g.base[g.head + 4 * g.nvec + tid] : 0u;
    for (int i = tid; i <= kNB; i += kT) CNT[i] = 0u;
    for (int i = tid; i < kNB; i += kT) MASS[i] = 0ull;
    if (tid == 0) { s_top = 0u; s_flags = 0u; s_nb = 0u; s_plim = kNB + 1; }

    const WPen w = wpen(a, row, p);
    const float inv_t = 1.0f / p.temperature;
    bool bad = false;
    auto word_of = [&](int t) { return w.on ? w.bits[t >> 5] : 0u; };
    uint32_t k[kVPT][4];
#pragma unroll
    for (int i = 0; i < kVPT; ++i) {
        const int x = i * kT + tid;
        const int t0 = g.s0 + g.head + 4 * x;
        uint32_t w0 = 0u, w1 = 0u;
        if (x < g.nvec && w.on) { w0 = word_of(t0); w1 = word_of(t0 + 3); }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = t0 + e;
            k[i][e] = x < g.nvec ? logit_key(w, p, inv_t, t, vec_bits<VI_F32>(v[i], e), (t >> 5) == (t0 >> 5) ? w0 : w1, &bad)
                                 : 0u;
        }
    }
    const uint32_t hk = tid < g.head ? logit_key(w, p, inv_t, g.s0 + tid, hb, word_of(g.s0 + tid), &bad) : 0u;
    const int tt = g.s0 + g.head + 4 * g.nvec + tid;
    const uint32_t tk = tid < g.tail ? logit_key(w, p, inv_t, tt, tb, word_of(tt), &bad) : 0u;
    uint32_t mk = max(hk, tk);
#pragma unroll
    for (int i = 0; i < kVPT; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) mk = max(mk, k[i][e]);
    mk = wave_max_u32(mk);
    __syncthreads();   // (LDS cleared)
    if (lane_id() == 0 && mk) atomicMax(&s_top, mk);
    if (bad) atomicOr(&s_flags, uint32_t(VI_FLAG_NONFINITE));
    __syncthreads();
    const uint32_t top = s_top;
    WideHead* hd = a.heads + size_t(row) * a.slices + s;
    if (top == 0u) {
        if (tid == 0) *hd = WideHead{0.0, 0u, 0u, s_flags, 0u, 0u, 0u};
        return;
    }
    const double anchor = floor(double(unkey32(top)) * kPerUnit);

    // counts and fixed-point masses per bin
    uint16_t bin[kVPT][4];
    uint32_t nbl = 0u;   // one past the last non-deep bin holding logits
    auto count = [&](uint32_t key) -> uint16_t {
        if (!key) return uint16_t(0xffffu);
        const BinW b = bin_weight(key, anchor);
        atomicAdd(&CNT[b.bin], 1u);
        if (b.bin < kNB) {
            atomicAdd(&MASS[b.bin], (unsigned long long)b.fix);
            nbl = max(nbl, uint32_t(b.bin) + 1u);
        }
        return uint16_t(b.bin);
    };
#pragma unroll
    for (int i = 0; i < kVPT; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) bin[i][e] = count(k[i][e]);
    const uint16_t hbin = count(hk), tbin = count(tk);
    nbl = wave_max_u32(nbl);
    if (lane_id() == 0 && nbl) atomicMax(&s_nb, nbl);
    __syncthreads();
    const uint32_t nb = s_nb;

    // list positions: bins in order (thread t: bins 4t .. 4t + 3), the deep bin last
    const size_t rs = size_t(row) * a.slices + s;
    uint32_t c4[4], sum = 0u;
#pragma unroll
    for (int q = 0; q < 4; ++q) { c4[q] = CNT[4 * tid + q]; sum += c4[q]; }
    const uint32_t deep = CNT[kNB];
    uint32_t total = 0u;
    const uint32_t excl = block_exclusive_scan_u32<kT>(sum, s_scan, &total);
    // (bins past nb hold nothing: their starts, all `total`, and masses are
    // not written; the merge reads them as empty)
    uint32_t* st = a.starts + rs * kStarts;
    uint32_t o = excl;
    uint32_t plim = kNB + 1;   // first bin starting at or past kPairs
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t j = 4 * tid + q;
        if (j <= nb) st[j] = o;
        if (o >= uint32_t(kPairs)) plim = min(plim, j);
        CNT[j] = o;
        o += c4[q];
    }
    if (plim <= kNB) atomicMin(&s_plim, plim);
    unsigned long long* ms = a.mass + rs * kNB;
    for (int i = tid; i < int(nb); i += kT) ms[i] = MASS[i];
    const uint32_t npairs = min(total + deep, uint32_t(kPairs));
    if (tid == 0) {
        st[kNB] = total;
        st[kNB + 1] = total + deep;
        CNT[kNB] = total;
        if (total >= uint32_t(kPairs)) atomicMin(&s_plim, uint32_t(kNB));
        *hd = WideHead{anchor, top, total + deep, s_flags, nb, npairs, 0u};
    }
    __syncthreads();

    // the (key, offset) pairs of list positions below kPairs, grouped by bin:
    // placed in LDS, then written out whole (coalesced 16-byte stores)
    uint16_t* SOFF = reinterpret_cast<uint16_t*>(MASS);
    const uint32_t pl = s_plim;
    auto put = [&](uint32_t key, uint16_t b, int off) {
        if (!key || b >= pl) return;
        const uint32_t pos = atomicAdd(&CNT[b], 1u);
        if (pos < uint32_t(kPairs)) { SKEY[pos] = key; SOFF[pos] = uint16_t(off); }
    };
#pragma unroll
    for (int i = 0; i < kVPT; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) put(k[i][e], bin[i][e], g.head + 4 * (i * kT + tid) + e);
    put(hk, hbin, tid);
    put(tk, tbin, g.head + 4 * g.nvec + tid);
    __syncthreads();
    const int n = int(npairs);
    uint4* ko = reinterpret_cast<uint4*>(a.keys + rs * kSL);
    uint4* io = reinterpret_cast<uint4*>(a.ids + rs * kSL);
    for (int c = tid; c < (n + 3) / 4; c += kT) ko[c] = reinterpret_cast<const uint4*>(SKEY)[c];
    for (int c = tid; c < (n + 7) / 8; c += kT) io[c] = reinterpret_cast<const uint4*>(SOFF)[c];
}

// ------------------------------------------------------------------ merge
// One workgroup per row.  LDS: exclusive prefix counts and masses of the row's
// bins, one bin's logits staged for the narrowing, digit buckets.
struct MergeLds {
    uint32_t EXC[kNB + 2];          // logits in the bins before J; [kNB] all but deep, [kNB + 1] N
    double EXM[kNB + 1];            // mass of the bins before J; [kNB] the row's mass
    uint32_t CK[kCap];              // staged keys of one bin
    uint32_t CI[kCap];              // their slice << 16 | offset
    uint32_t BC[kDig];
    unsigned long long BF[kDig];
    uint32_t OB[kSL / 32];          // owner bitmap
    double dscan[kW + 1];
    uint32_t uscan[kW + 1];
    // slices
    int delta[kMaxSlices];          // A - anchor_s (kNB + 1: wholly deep; -1: no valid logit)
    uint32_t lo[kMaxSlices], pre[kMaxSlices + 1], pcnt[kMaxSlices];
    uint32_t nbin[kMaxSlices], npairs[kMaxSlices];   // the slice heads' nbins and npairs
    double sanc[kMaxSlices];        // the slices' anchors
    // pairs recomputed from the logits: per slice the row bin last done, and
    // the slice bins and list end of the current one
    int matJ[kMaxSlices], mjlo[kMaxSlices], mjhi[kMaxSlices];
    uint32_t mhi[kMaxSlices], mmask, mcnt;
    // scratch for block decisions
    uint32_t u0, u1, u2, u3, kmin, kmax;
    unsigned long long f0;
    double d0;
    uint32_t staged, n;
};

static_assert(offsetof(MergeLds, CI) % 8 == 0, "CI also holds 64-bit partial sums");

// Result of narrowing one bin: the key the target falls on, the rank there,
// and what the bin's higher keys hold.
struct RHit {
    bool found;
    uint32_t key, rank, cnt_key, cnt_before;
    unsigned long long fix_before, fix_key;
};

struct RowCtx {
    const WideArgs* a;
    int row, S;
    size_t rs0;       // row * slices
    double A, z0;
    const vi_row_params* p;
    WPen w;           // the row's penalties, as the slice pass applied them
    float inv_t;
};

__device__ __forceinline__ double unit_of(const RowCtx& c, int J) {   // 2^-31 x exp(bin floor - z0)
    return kFixScale * exp((c.A - double(J)) / kPerUnit - c.z0);
}

// Pairs of the slices in `mask` at their list ranges [lo, mhi), for bins past
// the positions the slice pass wrote: each slice's logits are read again and
// keyed and binned as the slice pass did (same penalties, temperature and
// anchor), so the range receives exactly its pairs (in another order within
// the range, which no reader depends on).  All threads.
__device__ void materialize(const RowCtx& c, MergeLds& L, uint32_t mask) {
    const WideArgs& a = *c.a;
    const int tid = threadIdx.x;
    while (mask) {
        const int s = __builtin_ctz(mask);
        mask &= mask - 1u;
        if (tid == 0) L.mcnt = 0u;
        __syncthreads();
        const WGeo g = wgeo(a, c.row, s);
        const double anchor = L.sanc[s];
        const int jlo = L.mjlo[s], jhi = L.mjhi[s];
        const uint32_t lo = L.lo[s], cnt = L.mhi[s] - lo;
        uint32_t* ko = a.keys + (c.rs0 + s) * kSL + lo;
        uint16_t* io = a.ids + (c.rs0 + s) * kSL + lo;
        bool bad = false;
        for (int x = tid; x < g.n; x += kT) {
            const int t = g.s0 + x;
            const uint32_t k = logit_key(c.w, *c.p, c.inv_t, t, g.base[x], c.w.on ? c.w.bits[t >> 5] : 0u, &bad);
            if (!k) continue;
            const int b = bin_weight(k, anchor).bin;
            if (b < jlo || b > jhi) continue;
            const uint32_t pos = atomicAdd(&L.mcnt, 1u);
            if (pos < cnt) { ko[pos] = k; io[pos] = uint16_t(x); }
        }
        __syncthreads();
    }
    __threadfence();   // (the stores, then the reads of this workgroup)
    __syncthreads();
}

// Candidates of row bin J: per slice the list range [lo, hi); staged in LDS
// when they fit.  All threads.
__device__ void gather_bin(const RowCtx& c, MergeLds& L, int J) {
    const WideArgs& a = *c.a;
    const int tid = threadIdx.x;
    if (tid < kWave) {
        uint32_t lo = 0u, hi = 0u;
        int jlo = 0, jhi = -1;
        if (tid < c.S && L.delta[tid] >= 0) {
            const uint32_t* st = a.starts + (c.rs0 + tid) * kStarts;
            const int d = L.delta[tid], nb = int(L.nbin[tid]);
            if (J < kNB) {
                if (d <= J && J - d < nb) { lo = st[J - d]; hi = st[J - d + 1]; jlo = jhi = J - d; }
            } else {   // the slice's bins from kNB - d on and its deep bin
                jlo = max(0, kNB - d);
                jhi = kDeep;
                lo = st[min(jlo, nb)];
                hi = st[kNB + 1];
            }
        }
        bool mat = false;
        if (tid < c.S && hi > lo && hi > L.npairs[tid] && L.matJ[tid] != J) {
            mat = true;
            L.matJ[tid] = J;
            L.mjlo[tid] = jlo;
            L.mjhi[tid] = jhi;
            L.mhi[tid] = hi;
        }
        const uint64_t mm = ballot(mat);
        const uint32_t cnt = hi - lo;
        const uint32_t incl = wave_incl_scan_u32(cnt);
        if (tid < kMaxSlices) { L.lo[tid] = lo; L.pre[tid] = incl - cnt; }
        if (tid == kWave - 1) { L.n = incl; L.pre[kMaxSlices] = incl; L.staged = incl <= uint32_t(kCap) ? 1u : 0u; }
        if (tid == 0) { L.kmin = 0xffffffffu; L.kmax = 0u; L.mmask = uint32_t(mm); }
    }
    __syncthreads();
    if (L.mmask) materialize(c, L, L.mmask);
    const uint32_t n = L.n;
    uint32_t mn = 0xffffffffu, mx = 0u;
    for (uint32_t i = tid; i < n; i += kT) {
        int s = 0;
        while (s + 1 < c.S && L.pre[s + 1] <= i) ++s;
        const size_t at = (c.rs0 + s) * kSL + L.lo[s] + (i - L.pre[s]);
        const uint32_t k = a.keys[at];
        if (L.staged) { L.CK[i] = k; L.CI[i] = (uint32_t(s) << 16) | a.ids[at]; }
        mn = min(mn, k);
        mx = max(mx, k);
    }
    mn = ~wave_max_u32(~mn);
    mx = wave_max_u32(mx);
    if (lane_id() == 0) { atomicMin(&L.kmin, mn); atomicMax(&L.kmax, mx); }
    __syncthreads();
}

// Candidate i of the gathered bin: key, and slice << 16 | offset.
__device__ __forceinline__ uint32_t cand_key(const RowCtx& c, const MergeLds& L, uint32_t i) {
    if (L.staged) return L.CK[i];
    int s = 0;
    while (s + 1 < c.S && L.pre[s + 1] <= i) ++s;
    return c.a->keys[(c.rs0 + s) * kSL + L.lo[s] + (i - L.pre[s])];
}
__device__ __forceinline__ uint32_t cand_id(const RowCtx& c, const MergeLds& L, uint32_t i) {
    if (L.staged) return L.CI[i];
    int s = 0;
    while (s + 1 < c.S && L.pre[s + 1] <= i) ++s;
    return (uint32_t(s) << 16) | c.a->ids[(c.rs0 + s) * kSL + L.lo[s] + (i - L.pre[s])];
}

// Narrows the gathered bin J to the logit at which the cumulative count
// (mode 0: >= target) or mass (mode 1: >= target, mode 2: > target) over the
// bin's logits in order is reached; target counts from the bin's start.  All
// threads; the result in every thread.
__device__ RHit narrow(const RowCtx& c, MergeLds& L, int J, int mode, double target) {
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const bool massy = J < kNB;   // (the deep bin's logits carry no mass)
    const double unit = massy ? unit_of(c, J) : 0.0;
    const uint32_t n = L.n;
    uint32_t klo = L.kmin, khi = L.kmax;
    RHit h{};
    if (n == 0u) return h;
    h.cnt_key = n;
    double tgt = target;
    while (klo < khi) {
        const uint32_t span = khi - klo;
        const int shift = max(0, 32 - __builtin_clz(span) - 8);
        if (tid < kDig) { L.BC[tid] = 0u; L.BF[tid] = 0ull; }
        __syncthreads();
        for (uint32_t i = tid; i < n; i += kT) {
            const uint32_t k = cand_key(c, L, i);
            if (k < klo || k > khi) continue;
            const uint32_t d = (k - klo) >> shift;
            atomicAdd(&L.BC[d], 1u);
            if (massy) atomicAdd(&L.BF[d], (unsigned long long)weight_fix(k));
        }
        __syncthreads();
        if (wave == 0) {
            // lane l: buckets 255 - 4l - q, highest keys first
            uint32_t bc[4];
            double bf[4];
            uint32_t tc = 0u;
            double tf = 0.0;   // (integers below 2^53: exact)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int b = kDig - 1 - 4 * lane - q;
                bc[q] = L.BC[b];
                bf[q] = double(L.BF[b]);
                tc += bc[q];
                tf += bf[q];
            }
            uint32_t cc = wave_incl_scan_u32(tc) - tc;
            double cf = wave_incl_scan_f64(tf) - tf;
            int fq = -1;
            uint32_t fc = 0u;
            double ff = 0.0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t nc = cc + bc[q];
                const double nf = cf + bf[q];
                bool hit;
                if (mode == 0) hit = double(nc) >= tgt;
                else if (mode == 1) hit = nf * unit >= tgt;
                else hit = nf * unit > tgt;
                if (fq < 0 && bc[q] && hit) { fq = q; fc = cc; ff = cf; }
                cc = nc;
                cf = nf;
            }
            const uint64_t m = ballot(fq >= 0);
            if (lane == 0) L.u0 = m ? 1u : 0u;
            if (m && lane == __builtin_ctzll(m)) {
                const uint32_t b = uint32_t(kDig - 1 - 4 * lane - fq);
                L.u1 = b;
                L.u2 = fc;
                L.u3 = bc[0] * (fq == 0) + bc[1] * (fq == 1) + bc[2] * (fq == 2) + bc[3] * (fq == 3);
                L.d0 = ff;
            }
        }
        __syncthreads();
        if (!L.u0) { h.found = false; __syncthreads(); return h; }
        const uint32_t b = L.u1;
        h.cnt_before += L.u2;
        h.fix_before += (unsigned long long)(L.d0);
        h.cnt_key = L.u3;
        tgt -= mode == 0 ? double(L.u2) : L.d0 * unit;
        const uint32_t nlo = klo + (b << shift);
        const uint32_t nhi = uint32_t(min(uint64_t(khi), uint64_t(nlo) + ((1ull << shift) - 1ull)));
        klo = nlo;
        khi = nhi;
        __syncthreads();
    }
    h.key = klo;
    h.found = true;
    if (massy) h.fix_key = weight_fix(klo);
    if (mode == 0) {
        h.rank = uint32_t(max(0.0, tgt - 1.0));
    } else {
        const double wk = double(h.fix_key) * unit;
        const uint32_t cnt = max(h.cnt_key, 1u);
        const double x = tgt / wk;
        double rr = mode == 1 ? ceil(x) - 1.0 : floor(x);
        rr = fmin(fmax(rr, 0.0), double(cnt - 1u));
        uint32_t r = uint32_t(rr);
        for (int it = 0; it < 4; ++it) {   // settle the rounding of the estimate
            const double at = double(r) * wk, up = double(r + 1u) * wk;
            if (r > 0u && (mode == 1 ? at >= tgt : at > tgt)) --r;
            else if (r + 1u < cnt && (mode == 1 ? up < tgt : up <= tgt)) ++r;
            else break;
        }
        h.rank = r;
    }
    return h;
}

// Count and fixed mass of the gathered bin's logits with key >= kmin.
__device__ void bin_above(const RowCtx& c, MergeLds& L, uint32_t kmin, uint32_t* cnt, unsigned long long* fix,
                          bool with_mass) {
    const int tid = threadIdx.x;
    if (tid == 0) { L.u0 = 0u; L.f0 = 0ull; }
    __syncthreads();
    uint32_t cn = 0u;
    unsigned long long fx = 0ull;
    for (uint32_t i = tid; i < L.n; i += kT) {
        const uint32_t k = cand_key(c, L, i);
        if (k >= kmin) { ++cn; if (with_mass) fx += weight_fix(k); }
    }
    if (cn) { atomicAdd(&L.u0, cn); atomicAdd(&L.f0, fx); }
    __syncthreads();
    *cnt = L.u0;
    *fix = L.f0;
    __syncthreads();
}

// Logits of key k per slice in the gathered bin (L.pcnt).
__device__ void key_per_slice(const RowCtx& c, MergeLds& L, uint32_t key) {
    const int tid = threadIdx.x;
    if (tid < kMaxSlices) L.pcnt[tid] = 0u;
    __syncthreads();
    for (uint32_t i = tid; i < L.n; i += kT)
        if (cand_key(c, L, i) == key) atomicAdd(&L.pcnt[cand_id(c, L, i) >> 16], 1u);
    __syncthreads();
}

// The rank-th logit of key `key` in id order, in the gathered bin: its token.
__device__ int32_t owner(const RowCtx& c, MergeLds& L, uint32_t key, uint32_t rank) {
    const int tid = threadIdx.x;
    key_per_slice(c, L, key);
    if (tid < kWave) {
        const uint32_t cnt = tid < kMaxSlices ? L.pcnt[tid] : 0u;
        const uint32_t incl = wave_incl_scan_u32(cnt);
        const uint64_t m = ballot(tid < c.S && incl > rank);
        if (tid == 0) L.u0 = m ? uint32_t(__builtin_ctzll(m)) : 0xffffffffu;
        if (m && tid == __builtin_ctzll(m)) L.u1 = rank - (incl - cnt);
    }
    if (tid < kSL / 32) L.OB[tid] = 0u;
    __syncthreads();
    const uint32_t os = L.u0;
    if (os == 0xffffffffu) { __syncthreads(); return -1; }
    for (uint32_t i = tid; i < L.n; i += kT)
        if (cand_key(c, L, i) == key) {
            const uint32_t id = cand_id(c, L, i);
            if ((id >> 16) == os) atomicOr(&L.OB[(id & 0xffffu) >> 5], 1u << (id & 31u));
        }
    __syncthreads();
    const uint32_t word = tid < kSL / 32 ? L.OB[tid] : 0u;
    uint32_t tot = 0u;
    const uint32_t before = block_exclusive_scan_u32<kT>(uint32_t(__builtin_popcount(word)), L.uscan, &tot);
    const uint32_t want = L.u1;
    if (tid == 0) L.u2 = 0xffffffffu;
    __syncthreads();
    if (want >= before && want < before + uint32_t(__builtin_popcount(word))) {
        uint32_t m = word;
        for (uint32_t r = want - before; r > 0u; --r) m &= m - 1u;
        L.u2 = uint32_t(tid) * 32u + uint32_t(__builtin_ctz(m));
    }
    __syncthreads();
    const uint32_t off = L.u2;
    __syncthreads();
    return off == 0xffffffffu ? -1 : int32_t(os * kSL + off);
}

// First bin J (in [0, kNB] for counts, [0, kNB) for masses) whose inclusive
// cumulative count (mode 0: >= target) or mass (1: >=, 2: >) reaches the
// target, among bins holding logits; -1 when none.
__device__ int find_bin(MergeLds& L, int mode, double target) {
    const int tid = threadIdx.x;
    if (tid == 0) L.u0 = 0xffffffffu;
    __syncthreads();
    int f = -1;
    const int last = mode == 0 ? kNB : kNB - 1;
    for (int q = 0; q < 4 + (tid == kT - 1 ? 1 : 0) && f < 0; ++q) {
        const int J = 4 * tid + q;
        if (J > last) break;
        const uint32_t cnt = L.EXC[J + 1] - L.EXC[J];
        if (!cnt) continue;
        bool hit;
        if (mode == 0) hit = double(L.EXC[J + 1]) >= target;
        else if (mode == 1) hit = L.EXM[J + 1] >= target;
        else hit = L.EXM[J + 1] > target;
        if (hit) f = J;
    }
    if (f >= 0) atomicMin(&L.u0, uint32_t(f));
    __syncthreads();
    const uint32_t r = L.u0;
    __syncthreads();
    return r == 0xffffffffu ? -1 : int(r);
}

// The n-th logit (1-based) of the row in order: (bin, key, rank).
struct Pos {
    int bin;
    uint32_t key, rank;
};
__device__ Pos nth_logit(const RowCtx& c, MergeLds& L, uint32_t n) {
    const int J = find_bin(L, 0, double(n));
    if (J < 0) return Pos{-1, 0u, 0u};
    gather_bin(c, L, J);
    const RHit h = narrow(c, L, J, 0, double(n) - double(L.EXC[J]));
    return Pos{J, h.key, h.rank};
}

// Smallest key in [lo, hi) with pred(key) (monotone false -> true), or hi;
// one wave, 64 probes per round.
template <class P>
__device__ __forceinline__ uint32_t wave_search_u32(uint32_t lo, uint32_t hi, P pred) {
    const int lane = lane_id();
    uint64_t l = lo, h = hi;
    while (h > l) {
        const uint64_t n = h - l;
        if (n <= uint64_t(kWave)) {
            const uint64_t m = ballot(uint64_t(lane) < n && pred(uint32_t(l + lane)));
            return m ? uint32_t(l + __builtin_ctzll(m)) : uint32_t(h);
        }
        const uint64_t step = (n + kWave - 1) / kWave;
        const uint64_t p = l + uint64_t(lane) * step;
        const uint64_t valid = ballot(p < h);
        const uint64_t m = ballot(p < h && pred(uint32_t(p)));
        if (!m) {
            l = l + uint64_t(63 - __builtin_clzll(valid)) * step + 1;
            continue;
        }
        const int f = __builtin_ctzll(m);
        if (f == 0) return uint32_t(l);
        const uint64_t nl = l + uint64_t(f - 1) * step + 1;
        h = l + uint64_t(f) * step;
        l = nl;
    }
    return uint32_t(l);
}

__device__ __forceinline__ void write_row(const WideArgs& a, int row, int32_t token, double u, uint32_t flags,
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

// Position order: (key desc, rank asc).  True when (k1, r1) comes after (k2, r2).
__device__ __forceinline__ bool after(uint32_t k1, uint32_t r1, uint32_t k2, uint32_t r2) {
    return k1 < k2 || (k1 == k2 && r1 > r2);
}

__global__ __launch_bounds__(kT) void wide_merge_kernel(WideArgs a) {
    __shared__ MergeLds L;
    const int row = blockIdx.x, tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const vi_row_params p = a.params[row];
    if (!full_row(p)) return;
    const int S = a.slices, V = a.vocabulary;
    const size_t rs0 = size_t(row) * S;

    // ---- 0. slice heads: the row's anchor, top key, valid logits and flags
    __shared__ double s_anchor;
    __shared__ uint32_t s_top, s_valid, s_flags, s_rb;
    if (tid == 0) { s_top = 0u; s_valid = 0u; s_flags = 0u; s_anchor = 0.0; s_rb = 0u; }
    __syncthreads();
    WideHead hd{};
    if (tid < S) {
        hd = a.heads[rs0 + tid];
        atomicAdd(&s_valid, hd.n_valid);
        atomicOr(&s_flags, hd.flags);
        if (hd.n_valid) atomicMax(&s_top, hd.top_key);
    }
    if (tid == 0) {
        uint32_t pf = 0u;
        if (a.pstate) {
            if (penalties_active(p))
                pf = reinterpret_cast<const PenaltyHeader*>(a.pstate + size_t(row) * a.pl.lane_bytes)->flags;
        } else if (a.row_flags && a.histories && a.offsets && a.hash && penalties_active(p) &&
                   a.offsets[row + 1] > a.offsets[row]) {
            pf = a.row_flags[row];
        }
        atomicOr(&s_flags, pf & uint32_t(VI_FLAG_BAD_HISTORY | VI_FLAG_ERROR));
    }
    __syncthreads();
    const uint32_t top = s_top, N = s_valid;
    if (tid < S && hd.n_valid && hd.top_key == top) s_anchor = hd.anchor;   // (equal tops: equal anchors)
    __syncthreads();
    const double A = s_anchor;
    const double z0 = double(unkey32(top));
    const uint32_t out_flags = s_flags & uint32_t(VI_FLAG_NONFINITE | VI_FLAG_BAD_HISTORY);
    const bool fail = (s_flags & VI_FLAG_ERROR) != 0u;
    if (fail || N == 0u) {
        if (tid == 0) {
            write_row(a, row, fail ? -1 : V, 0.0, out_flags | (fail ? VI_FLAG_ERROR : VI_FLAG_EMPTY), 0u, 0u, 0.0);
            if (a.want_bounds) a.bounds[row] = WideBound{0.0, 0.0, 0.0f, 0u, 0u, 0u};
        }
        return;
    }
    if (tid < kMaxSlices) {
        int d = -1;
        if (tid < S && hd.n_valid) {
            const double dd = A - hd.anchor;
            d = dd < double(kNB + 1) ? int(dd) : kNB + 1;
        }
        L.delta[tid] = d;
        if (d >= 0 && d < kNB) atomicMax(&s_rb, uint32_t(min(kNB, d + int(hd.nbins))));   // (row bins in use)
        L.nbin[tid] = hd.nbins;
        L.npairs[tid] = hd.npairs;
        L.sanc[tid] = hd.anchor;
        L.matJ[tid] = -1;
    }
    __syncthreads();
    RowCtx c{&a, row, S, rs0, A, z0, &p, wpen(a, row, p), 1.0f / p.temperature};

    // ---- 1. the row's bins: counts and masses summed over the slices (thread t:
    // bins 4t .. 4t + 3), then their exclusive prefixes in bin order
    // (four slices' loads issued together, unconditional at clamped places
    // and dropped afterwards: a load under a branch waits for the ones before).
    // When the row's bins in use fit in a half or a quarter of the 4,096, the
    // slices are shared out between two or four groups of threads (fewer
    // dependent load rounds each), whose sums meet in LDS.
    const int rb = int(s_rb);
    const int ways = rb <= kNB / 4 ? 4 : rb <= kNB / 2 ? 2 : 1;
    const int per = kT / ways, way = tid / per, quad = tid - way * per;
    const int sp = (S + ways - 1) / ways, sb = min(S, way * sp), se = min(S, sb + sp);
    uint32_t bc[4] = {0u, 0u, 0u, 0u};
    unsigned long long bf[4] = {0ull, 0ull, 0ull, 0ull};
    for (int s0 = sb; s0 < se; s0 += 4) {
        uint32_t lo[4][4], hi[4][4];
        unsigned long long mv[4][4];
        bool on[4][4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int sc = min(s0 + u, se - 1), d = L.delta[sc], nb = int(L.nbin[sc]);
            const bool live = s0 + u < se && d >= 0 && d < kNB;
            const uint32_t* st = a.starts + (rs0 + sc) * kStarts;
            const unsigned long long* ms = a.mass + (rs0 + sc) * kNB;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int j = 4 * quad + q - d;
                on[u][q] = live && j >= 0 && j < nb;
                const int jc = on[u][q] ? j : 0;
                lo[u][q] = st[jc];
                hi[u][q] = st[jc + 1];
                mv[u][q] = ms[jc];
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (on[u][q]) { bc[q] += hi[u][q] - lo[u][q]; bf[q] += mv[u][q]; }
    }
    if (ways > 1) {   // (the staging arrays are free until the first gather)
        unsigned long long* pm = reinterpret_cast<unsigned long long*>(L.CI);
        static_assert(3 * (kT / 4) * 4 <= kCap && 3 * (kT / 4) * 4 * 2 <= kCap, "partial sums staging");
        if (way > 0) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                L.CK[((way - 1) * per + quad) * 4 + q] = bc[q];
                pm[((way - 1) * per + quad) * 4 + q] = bf[q];
            }
        }
        __syncthreads();
        if (way == 0) {
            for (int w = 1; w < ways; ++w)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    bc[q] += L.CK[((w - 1) * per + quad) * 4 + q];
                    bf[q] += pm[((w - 1) * per + quad) * 4 + q];
                }
        } else {   // (their bins 4 tid .. 4 tid + 3 lie past the bins in use)
#pragma unroll
            for (int q = 0; q < 4; ++q) { bc[q] = 0u; bf[q] = 0ull; }
        }
    }
    double bm[4];
    uint32_t csum = 0u;
    double msum = 0.0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        bm[q] = bc[q] ? double(bf[q]) * unit_of(c, 4 * tid + q) : 0.0;
        csum += bc[q];
        msum += bm[q];
    }
    uint32_t ctot = 0u;
    const uint32_t cex = block_exclusive_scan_u32<kT>(csum, L.uscan, &ctot);
    {   // exclusive prefix of the per-thread masses, wave by wave in a fixed order
        const double incl = wave_incl_scan_f64(msum);
        const int src = max(lane - 1, 0);
        const uint64_t bits = __builtin_bit_cast(uint64_t, incl);
        const uint32_t lo = uint32_t(__builtin_amdgcn_ds_bpermute(src << 2, int(uint32_t(bits))));
        const uint32_t hi = uint32_t(__builtin_amdgcn_ds_bpermute(src << 2, int(uint32_t(bits >> 32))));
        const double wex = lane ? __builtin_bit_cast(double, (uint64_t(hi) << 32) | lo) : 0.0;
        if (lane == kWave - 1) L.dscan[wave] = incl;
        __syncthreads();
        if (wave == 0) {
            const double t = lane < kW ? L.dscan[lane] : 0.0;
            const double it = wave_incl_scan_f64(t);
            if (lane < kW) L.dscan[lane] = it - t;
        }
        __syncthreads();
        double m = L.dscan[wave] + wex;
        uint32_t cc = cex;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            L.EXC[4 * tid + q] = cc;
            L.EXM[4 * tid + q] = m;
            cc += bc[q];
            m += bm[q];
        }
        if (tid == kT - 1) {
            L.EXC[kNB] = cc;
            L.EXC[kNB + 1] = N;
            L.EXM[kNB] = m;
        }
    }
    __syncthreads();
    const double s_all = L.EXM[kNB];

    // ---- 2. the top-k cap
    bool cap_on = false;
    uint32_t cap_key = 0u, cap_take = kTakeAll;
    double cap_mass = s_all;
    if (p.top_k > 0 && uint32_t(p.top_k) < N) {
        const int J = find_bin(L, 0, double(p.top_k));
        gather_bin(c, L, J);
        const RHit h = narrow(c, L, J, 0, double(p.top_k) - double(L.EXC[J]));
        cap_on = true;
        cap_key = h.key;
        cap_take = h.rank + 1u;
        cap_mass = J < kNB ? L.EXM[J] + double(h.fix_before + (unsigned long long)cap_take * h.fix_key) * unit_of(c, J)
                           : s_all;
    }

    // ---- 3. the min-p cut: the smallest key whose weight reaches min_p
    uint32_t minp_key = 0u;
    const bool minp_on = p.min_p > 0.0f;
    if (minp_on) {
        __shared__ uint32_t s_kf;
        if (wave == 0) {
            const double mp = double(p.min_p);
            const uint32_t kf = wave_search_u32(0x00800000u, top + 1u, [&](uint32_t key) {
                return exp(double(unkey32(key)) - z0) >= mp;
            });
            if (lane == 0) s_kf = kf;
        }
        __syncthreads();
        minp_key = s_kf;
    }

    // ---- 4. the top-p cut over the cap's mass
    bool topp_on = false;
    uint32_t topp_key = 0u, topp_take = kTakeAll;
    int topp_bin = -1;
    RHit topp_h{};
    if (p.top_p < 1.0f) {
        const double target = double(p.top_p) * cap_mass;
        const int J = find_bin(L, 1, target);
        if (J >= 0) {
            gather_bin(c, L, J);
            topp_h = narrow(c, L, J, 1, target - L.EXM[J]);
            if (topp_h.found) { topp_on = true; topp_key = topp_h.key; topp_take = topp_h.rank + 1u; topp_bin = J; }
        }
    }

    // ---- 5. the support's end: the earliest of the cap, the min-p cut and the
    // top-p cut (at least the first logit); its size and mass
    bool all = true;
    int src = 0;   // 1 cap, 2 min-p, 3 top-p, 4 forced first logit
    uint32_t ek = 0u, et = kTakeAll;
    auto consider = [&](uint32_t k, uint32_t t, int from) {
        if (all || k > ek || (k == ek && t < et)) { ek = k; et = t; all = false; src = from; }
    };
    if (cap_on) consider(cap_key, cap_take, 1);
    if (minp_on) consider(minp_key, kTakeAll, 2);
    if (topp_on) consider(topp_key, topp_take, 3);
    if (!all && ek > top) { ek = top; et = 1u; src = 4; }   // no logit passes min-p: the first one
    uint32_t n_sup = N;
    double s_n = s_all;
    if (src == 1) {
        n_sup = uint32_t(p.top_k);
        s_n = cap_mass;
    } else if (src == 3) {
        n_sup = L.EXC[topp_bin] + topp_h.cnt_before + topp_take;
        s_n = L.EXM[topp_bin] +
              double(topp_h.fix_before + (unsigned long long)topp_take * topp_h.fix_key) * unit_of(c, topp_bin);
    } else if (src == 2) {
        const BinW b = bin_weight(ek, A);
        gather_bin(c, L, b.bin);
        uint32_t cn = 0u;
        unsigned long long fx = 0ull;
        bin_above(c, L, ek, &cn, &fx, b.bin < kNB);
        n_sup = L.EXC[b.bin] + cn;
        s_n = L.EXM[b.bin] + (b.bin < kNB ? double(fx) * unit_of(c, b.bin) : 0.0);
    } else if (src == 4) {
        n_sup = 1u;
        s_n = 1.0;
    }

    // ---- 6. the draw: the first support logit whose inclusive cumulative mass
    // exceeds u x S_n (the last support logit when rounding passes them all)
    const double u = philox_uniform(p.seed, p.lane, p.position, 0u);
    const double target = u * s_n;
    int dbin = find_bin(L, 2, target);
    uint32_t dkey = 0u, drank = 0u;
    bool dfound = false;
    if (dbin >= 0) {
        gather_bin(c, L, dbin);
        const RHit h = narrow(c, L, dbin, 2, target - L.EXM[dbin]);
        if (h.found && (all || !after(h.key, h.rank, ek, et == kTakeAll ? 0xffffffffu : et - 1u))) {
            dfound = true;
            dkey = h.key;
            drank = h.rank;
        }
    }
    if (!dfound) {   // (nth_logit leaves its bin gathered, as the draw above does)
        const Pos q = nth_logit(c, L, n_sup);
        dbin = q.bin;
        dkey = q.key;
        drank = q.rank;
    }
    const int32_t tok = dbin >= 0 ? owner(c, L, dkey, drank) : -1;

    // ---- 7. results; the bases of the end key for the probs kernel
    if (a.want_bounds && !all && et != kTakeAll) {
        const BinW b = bin_weight(ek, A);
        gather_bin(c, L, b.bin);
        key_per_slice(c, L, ek);
        if (tid < kMaxSlices) {
            uint32_t before = 0u;
            for (int s = 0; s < tid; ++s) before += L.pcnt[s];
            a.bases[size_t(row) * kMaxSlices + tid] = before;
        }
    }
    if (tid == 0) {
        if (tok < 0) {   // the bins disagree with the lists: cannot happen for consistent inputs
            write_row(a, row, -1, u, out_flags | VI_FLAG_ERROR, 0u, 0u, 0.0);
        } else {
            write_row(a, row, tok, u, out_flags, n_sup, N, s_n);
            if (a.record && a.pstate && tok < V) {   // (the slice pass, an earlier launch, has read the state)
                const LaneState ls = lane_state(a.pstate + size_t(row) * a.pl.lane_bytes, a.pl);
                state_record_one(ls, a.pl, V, tok);
            }
        }
        if (a.want_bounds)
            a.bounds[row] = WideBound{z0, s_n, 1.0f / p.temperature, all ? 0u : ek, all ? kTakeAll : et,
                                      tok >= 0 ? 1u : 0u};
    }
}

// Filtered distribution of the full-route rows (test / diagnostics path): one
// workgroup per (slice, row); thread t takes logits 16 t .. 16 t + 15, so that
// thread order is id order for the end key's ranks.
__global__ __launch_bounds__(kT) void wide_probs_kernel(WideArgs a) {
    __shared__ uint32_t s_scan[kW + 1];
    const int s = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const vi_row_params p = a.params[row];
    if (!full_row(p)) return;
    const WideBound bd = a.bounds[row];
    const WGeo g = wgeo(a, row, s);
    float* pr = a.probs + size_t(row) * size_t(a.probs_stride) + g.s0;
    constexpr int kE = kSL / kT;
    const int e0 = kE * tid;
    if (!bd.valid) {
        for (int e = 0; e < kE; ++e)
            if (e0 + e < g.n) pr[e0 + e] = 0.0f;
        return;
    }
    const WPen w = wpen(a, row, p);
    int unrec = -1;
    if (a.record && a.pstate) unrec = a.tokens[row];
    uint32_t key[kE];
    uint32_t cnt = 0u;
    bool bad = false;
#pragma unroll
    for (int e = 0; e < kE; ++e) {
        const int off = e0 + e;
        key[e] = 0u;
        if (off < g.n) {
            const int t = g.s0 + off;
            key[e] = logit_key(w, p, bd.inv_t, t, g.base[off], w.on ? w.bits[t >> 5] : 0u, &bad, unrec);
            cnt += (bd.end_take != kTakeAll && key[e] == bd.end_key && key[e]) ? 1u : 0u;
        }
    }
    uint32_t tot = 0u;
    uint32_t rank = block_exclusive_scan_u32<kT>(cnt, s_scan, &tot);
    if (bd.end_take != kTakeAll) rank += a.bases[size_t(row) * kMaxSlices + s];
#pragma unroll
    for (int e = 0; e < kE; ++e) {
        const int off = e0 + e;
        if (off >= g.n) continue;
        const uint32_t k = key[e];
        float pv = 0.0f;
        bool in = k != 0u && k >= bd.end_key;
        if (in && k == bd.end_key && bd.end_take != kTakeAll) in = rank++ < bd.end_take;
        if (in) pv = float(exp(double(unkey32(k)) - bd.z0) / bd.s_n);
        pr[off] = pv;
    }
}

inline int wide_slices(int vocabulary) { return (vocabulary + kSL - 1) / kSL; }
inline int bitmap_words(int vocabulary) { return int(align_up((size_t(vocabulary) + 31) / 32, 4)); }

}  // namespace

bool wide_supported(int vocabulary, int64_t stride) {
    return vocabulary > 0 && vocabulary <= kMaxSlices * kSL && stride >= vocabulary;
}

size_t wide_workspace(int rows, int vocabulary) {
    if (rows <= 0 || vocabulary <= 0) return 0;
    const size_t rs = size_t(rows) * size_t(wide_slices(vocabulary));
    return align_up(rs * sizeof(WideHead), 256) + align_up(rs * kStarts * 4, 256) + align_up(rs * kNB * 8, 256) +
           align_up(rs * kSL * 4, 256) + align_up(rs * kSL * 2, 256) +
           align_up(size_t(rows) * size_t(bitmap_words(vocabulary)) * 4, 256) +
           align_up(size_t(rows) * sizeof(WideBound), 256) + align_up(size_t(rows) * kMaxSlices * 4, 256) + 256;
}

vi_status launch_wide(const SampleArgs& s, unsigned char* ws, size_t ws_bytes, uint2* hash, int hash_shift,
                      int hash_slots, uint32_t* row_flags, hipStream_t stream) {
    if (!wide_supported(s.vocabulary, s.stride) || reinterpret_cast<uintptr_t>(s.logits) % 4) return VI_ERR_UNSUPPORTED;
    WideArgs a{};
    a.slices = wide_slices(s.vocabulary);
    const size_t rs = size_t(s.rows) * size_t(a.slices);
    Carver c(ws, ws_bytes);
    a.heads = c.take<WideHead>(rs);
    a.starts = c.take<uint32_t>(rs * kStarts);
    a.mass = c.take<unsigned long long>(rs * kNB);
    a.keys = c.take<uint32_t>(rs * kSL);
    a.ids = c.take<uint16_t>(rs * kSL);
    a.words = bitmap_words(s.vocabulary);
    a.hbits = c.take<uint32_t>(size_t(s.rows) * size_t(a.words));
    a.bounds = c.take<WideBound>(size_t(s.rows));
    a.bases = c.take<uint32_t>(size_t(s.rows) * kMaxSlices);
    if (!c.ok) return VI_ERR_WORKSPACE;
    a.logits = s.logits; a.rows = s.rows; a.vocabulary = s.vocabulary; a.stride = s.stride;
    a.params = s.params;
    if (s.pstate) {
        a.pstate = s.pstate; a.pl = s.playout; a.record = s.record;
    } else if (hash && s.histories && s.offsets) {
        a.histories = s.histories; a.offsets = s.offsets; a.max_history = s.max_history;
        a.hash = hash; a.hash_shift = hash_shift; a.hash_slots = hash_slots; a.row_flags = row_flags;
    }
    a.tokens = s.tokens; a.uniforms = s.uniforms; a.probs = s.probs; a.probs_stride = s.probs_stride;
    a.stats = s.stats;
    if (s.full_out) { a.bounds = s.full_out->bounds; a.bases = s.full_out->bases; }
    a.want_bounds = (s.probs || s.full_out) ? 1 : 0;
    if (a.hash) hipLaunchKernelGGL(wide_history_kernel, dim3(s.rows), dim3(256), 0, stream, a);
    hipLaunchKernelGGL(wide_slice_kernel, dim3(a.slices, s.rows), dim3(kT), 0, stream, a);
    hipLaunchKernelGGL(wide_merge_kernel, dim3(s.rows), dim3(kT), 0, stream, a);
    vi_status st = launch_status();
    if (st != VI_OK || !s.probs) return st;
    hipLaunchKernelGGL(wide_probs_kernel, dim3(a.slices, s.rows), dim3(kT), 0, stream, a);
    return launch_status();
}

}  // namespace vi
