// sample_parts.hip — full-vocabulary rows of the batched sampler (temperature
// > 0 and top_k = 0 or > 64) for bf16 / fp16 logits, in one launch: penalties
// from the lanes' penalty states applied in the pass that reads the logits,
// temperature, top-k / min-p / top-p over the whole vocabulary, and the Philox
// inverse-CDF draw.
//
// Key fact (as in sample_slices.hip): a penalized 16-bit logit takes one of
// 65,536 patterns and z = x' * (1/T) is a strictly monotone function of the
// pattern's order key, so the row's multiset of z is a count histogram over
// patterns and every cut and the draw are prefix sums over occupied keys.
//
// Shape.  A row is cut into P parts of at most 65,504 tokens (a key's count
// fits 16 bits; parts start on whole presence-bitmap words).  Persistent
// workgroups of 1024 threads (one per CU: the histogram is 128 KB of LDS) take
// parts, part-major (the parts of a row land on one XCD when the grid is a
// multiple of 8 rows).  Per part:
//   1. the part's logits, 8 x 16 bytes per thread, and the presence-bitmap
//      bytes of the same tokens are requested at once;
//   2. the repeated tokens of the part (count >= 2, from the lane's repeat
//      list) go to an LDS hash;
//   3. every token is counted at its final pattern: absent tokens at their raw
//      pattern, present ones penalized in registers (count 1 unless the hash
//      holds it) — u16 counts in pairs (word = key & 0x7fff, half = key >> 15);
//   4. one pass over the histogram writes the part's (key << 16 | count)
//      entries in key order (valid keys only) and zeroes it; the head (entries,
//      flags, largest valid key, valid count) follows;
// A second launch merges, one workgroup per row: every entry of the row's parts
// is weighted once (fp64 exp of z - z_max as 2^-44 fixed point) into 512
// coarse bins of 128 keys (exact u64 sums, so the order of arrival does not
// matter); suffix scans over the bins from the top key locate the top-k cap,
// the min-p and top-p cuts and the draw, each resolved inside its bin from the
// parts' entries of that bin (at most 128 per part); the part holding the
// drawn (key, rank) is read again to name the token (id order among equal
// keys), and the token is recorded in the lane's state when asked.
//
// Roofline: HBM; V x 2 bytes of logits per row, plus V / 8 bytes of presence
// bitmap and the lane's repeat list when penalties are active.
#include <math.h>

#include "keys16.h"
#include "penalty_state.h"
#include "vi_device.h"
#include "vi_internal.h"

namespace vi {
namespace {

constexpr int kT = 1024;                  // threads per workgroup
constexpr int kW = kT / kWave;            // waves per workgroup
constexpr int kNV = 8;                    // 16-byte vectors per thread and part
constexpr int kPartMax = 65504;           // tokens per part (< 65,536, a multiple of 32)
constexpr int kHW = 32768;                // histogram words
constexpr int kHS = 1024;                 // LDS repeat-hash slots
constexpr int kHSBits = 10;
constexpr uint32_t kHSFill = kHS * 3 / 4;
constexpr uint32_t kEmpty = 0xffffffffu;
constexpr int kBins = 512, kBinKeys = 128;
constexpr int kHead = 5;                  // entries, flags, largest valid key + 1, valid tokens, present tokens
constexpr double kScale = 0x1p44;         // fixed point of the weights (row masses < 2^63)
static_assert(kNV * 8 * kT >= kPartMax && kPartMax % 32 == 0, "part geometry");
static_assert(kHS == 1 << kHSBits, "hash size");

// LDS (bytes): H, the histogram (the merge's tables reuse it); X, the repeat
// hash; R, the part's repeat bitmap (count >= 2).
constexpr int kRW = 2048;                 // repeat-bitmap words (kPartMax bits)
constexpr int kOffH = 0;
constexpr int kOffX = kOffH + 4 * kHW;
constexpr int kOffR = kOffX + 4 * kHS;
constexpr int kStage = 9216;              // present-token offsets staged per round (u16)
constexpr int kOffF = kOffR + 4 * kRW;    // F: staged offsets of the part's present tokens
constexpr int kLds = kOffF + 2 * kStage;
static_assert(kStage % kT == 0, "whole staging rounds per thread");
static_assert(kRW * 32 >= kPartMax, "repeat bitmap");
// merge tables inside H
constexpr int kOffFirst = 0;                                 // u32 [parts][kBins]: first entry of a bin
constexpr int kOffNE = kOffFirst + 4 * kMaxParts16 * kBins;  // u32 [parts][kBins]: entries of a bin
constexpr int kOffBC = kOffNE + 4 * kMaxParts16 * kBins;     // u32 [kBins] tokens per bin
constexpr int kOffBM = kOffBC + 4 * kBins;                   // u64 [kBins] mass per bin
constexpr int kOffCC = kOffBM + 8 * kBins;                   // u32 [kBins] tokens from the top bin, inclusive
constexpr int kOffCM = kOffCC + 4 * kBins;                   // u64 [kBins] mass from the top bin, inclusive
constexpr int kOffFC = kOffCM + 8 * kBins;                   // u32 [parts][kBinKeys] a bin's counts per part
constexpr int kOffKN = kOffFC + 4 * kMaxParts16 * kBinKeys;  // u32 [kBinKeys] per key (descending), tokens
constexpr int kOffKC = kOffKN + 4 * kBinKeys;                // u32 [kBinKeys] tokens from the top, inclusive
constexpr int kOffKW = kOffKC + 4 * kBinKeys;                // u64 [kBinKeys] weight
constexpr int kOffKM = kOffKW + 8 * kBinKeys;                // u64 [kBinKeys] mass from the top, inclusive
constexpr int kMergeEnd = kOffKM + 8 * kBinKeys;
constexpr int kOffMatch = 65536;                             // u32 [kRW]: present tokens of the drawn key
static_assert(kMergeEnd <= kOffMatch && kOffMatch + 4 * kRW <= 4 * kHW, "merge tables");

struct PartArgs {
    const void* logits;
    int rows, vocabulary, parts, part_len, grid;
    int64_t stride;
    const vi_row_params* params;
    unsigned char* pstate;     // per-lane penalty states (or null: no penalties)
    PenaltyLayout pl;
    int record;
    int32_t* tokens;
    double* uniforms;
    vi_sample_stats* stats;
    uint32_t* heads;           // [rows][parts][kHead]
    uint32_t* lists;           // [rows][parts][part_len]: (key << 16 | count), key order
    uint32_t* plists;          // [rows][parts][part_len]: present tokens, (offset << 16 | final bits)
};

struct Shared {
    uint32_t scan[kW + 1];
    uint32_t flags, n_hash, overflow, kmin, kmax, top, nvalid, npres;
    // merge
    uint32_t m_flags, m_top, m_valid, m_base[kMaxParts16 + 1];
    uint32_t wc[kBins / kWave];
    uint64_t wm[kBins / kWave];
    int32_t res;
    uint32_t rnd[kNV], ri, rr;
    int32_t token;
    // decisions: ends are (tokens, mass) prefixes in (z desc, id asc) order
    uint32_t key, take, cnt_before;
    uint64_t mass_before, wfx;
};

// threadIdx.x and the lane behind an empty asm: arithmetic on them stays where
// it is written (the persistent loop's per-thread addresses would otherwise be
// hoisted out of the loop and held, or spilled, across it).
__device__ __forceinline__ int opaque_tid() {
    int t = int(threadIdx.x);
    asm volatile("" : "+v"(t));
    return t;
}

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Exclusive prefix of a per-thread u32 over the workgroup with LDS-only
// barriers (global loads in flight are not waited for); *total gets the sum.
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

template <int C, int R, bool B>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
    return uint64_t(dpp_u32<C, R, B>(uint32_t(v))) | (uint64_t(dpp_u32<C, R, B>(uint32_t(v >> 32))) << 32);
}
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t x) {
    x += dpp_u64<0x111, 0xf, true>(x);
    x += dpp_u64<0x112, 0xf, true>(x);
    x += dpp_u64<0x114, 0xf, true>(x);
    x += dpp_u64<0x118, 0xf, true>(x);
    x += dpp_u64<0x142, 0xa, false>(x);
    x += dpp_u64<0x143, 0xc, false>(x);
    return x;
}
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
    return uint64_t(uint32_t(__builtin_amdgcn_readlane(int(uint32_t(v)), l))) |
           (uint64_t(uint32_t(__builtin_amdgcn_readlane(int(uint32_t(v >> 32)), l))) << 32);
}

// Index k (0-based) of the k-th set bit of m.
__device__ __forceinline__ int nth_set_bit(uint32_t m, uint32_t k) {
    for (uint32_t i = 0; i < k; ++i) m &= m - 1u;
    return __builtin_ctz(m);
}

template <int DT>
__device__ __forceinline__ uint64_t weight_fx(uint32_t key, float inv_t, double z0) {
    const double w = exp(double(key_z<DT>(key, inv_t)) - z0);
    return uint64_t(rint(w * kScale));
}

__device__ __forceinline__ bool full_route_row(const vi_row_params& p) { return !topk_route(p); }

// Item k of workgroup w: (row, part), part-major, or false past the end.
__device__ __forceinline__ bool item_of(const PartArgs& a, int k, int* row, int* q) {
    const int idx = int(blockIdx.x) + k * a.grid;
    if (idx >= a.rows * a.parts) return false;
    *q = idx / a.rows;
    *row = idx % a.rows;
    return true;
}

// ------------------------------------------------------------ penalty inputs
struct PenIn {
    bool pen;
    const unsigned char* st;   // the lane's state
    uint32_t hflags;
};
__device__ __forceinline__ PenIn pen_in(const PartArgs& a, int row, const vi_row_params& p) {
    PenIn c{};
    c.pen = a.pstate != nullptr && penalties_active(p);
    if (c.pen) {
        c.st = a.pstate + size_t(row) * a.pl.lane_bytes;
        c.hflags = reinterpret_cast<const PenaltyHeader*>(c.st)->flags;
    }
    return c;
}

__device__ __forceinline__ uint32_t rh_slot(uint32_t off) { return (off * 0x9E3779B1u) >> (32 - kHSBits); }

// The part's repeated tokens (count >= 2 in the lane's repeat list): their bits
// in R and (offset << 16 | min(count, 0xffff)) in X.  Past the fill limit the
// hash stops taking entries and lookups that miss read the lane's own table.
__device__ __forceinline__ void build_repeat_hash(const PartArgs& a, const PenIn& c, int s0, int n, uint32_t* X,
                                                  uint32_t* R, Shared& sh) {
    const int tid = opaque_tid();
#pragma unroll
    for (int i = 0; i < kHS / kT; ++i) X[i * kT + tid] = kEmpty;
#pragma unroll
    for (int i = 0; i < kRW / kT; ++i) R[i * kT + tid] = 0u;
    if (tid == 0) { sh.n_hash = 0u; sh.overflow = 0u; }
    lds_barrier();
    const PenaltyHeader* hdr = reinterpret_cast<const PenaltyHeader*>(c.st);
    const uint32_t nrep = min(hdr->nrep, uint32_t(a.pl.slots));
    const uint2* list = reinterpret_cast<const uint2*>(c.st + a.pl.off_list);
    for (uint32_t e = uint32_t(tid); e < nrep; e += kT) {
        const uint2 ent = list[e];
        const int t = int(ent.x);
        if (ent.y < 2u || t < s0 || t >= s0 + n) continue;
        const uint32_t off = uint32_t(t - s0), v = (off << 16) | min(ent.y, 0xffffu);
        atomicOr(&R[off >> 5], 1u << (off & 31u));
        if (atomicAdd(&sh.n_hash, 1u) >= kHSFill) {
            sh.overflow = 1u;
            continue;
        }
        uint32_t s = rh_slot(off);
        for (int probe = 0; probe < kHS; ++probe) {   // a free slot exists: fill <= 3/4
            if (atomicCAS(&X[s], kEmpty, v) == kEmpty) break;
            s = (s + 1u) & uint32_t(kHS - 1);
        }
    }
    lds_barrier();
}

// Count of a repeated token (its R bit set) at offset `off` of the part
// starting at s0: from X, or from the lane's table when X does not hold it
// (hash full) or holds a saturated count.
__device__ __forceinline__ uint32_t repeat_count(const PartArgs& a, const PenIn& c, const uint32_t* X, int s0,
                                                 uint32_t off) {
    uint32_t s = rh_slot(off);
    for (int probe = 0; probe < kHS; ++probe) {
        const uint32_t v = X[s];
        if (v == kEmpty) break;
        if ((v >> 16) == off) {
            if ((v & 0xffffu) != 0xffffu) return v & 0xffffu;
            break;   // a count of 65,535 or more: the table has it
        }
        s = (s + 1u) & uint32_t(kHS - 1);
    }
    const uint2* table = reinterpret_cast<const uint2*>(c.st + a.pl.off_hash);
    return max(hash_count(table, a.pl.shift, a.pl.slots, s0 + int(off)), 2u);
}

// The part's logits and presence bytes (loads at clamped in-bounds addresses:
// users test the vector index against nvec).
template <int DT>
__device__ __forceinline__ void load_part(const PartArgs& a, const PenIn& c, int row, int s0, int nvec,
                                          uint4 (&v)[kNV], uint32_t (&pb)[kNV]) {
    const int tid = opaque_tid();
    const unsigned char* base =
        static_cast<const unsigned char*>(a.logits) + 2 * (size_t(row) * size_t(a.stride) + size_t(s0));
#pragma unroll
    for (int i = 0; i < kNV; ++i) v[i] = load16(base + 16 * size_t(min(i * kT + tid, nvec - 1)));
    if (c.pen) {
        const unsigned char* b1 = c.st + a.pl.off_b1 + (s0 >> 3);
#pragma unroll
        for (int i = 0; i < kNV; ++i) pb[i] = b1[min(i * kT + tid, nvec - 1)];
    } else {
#pragma unroll
        for (int i = 0; i < kNV; ++i) pb[i] = 0u;
    }
}

// Penalty of a history token (the arithmetic of penalize_bits, vi_device.h)
// with the division x / r done as Markstein's correction of x * (1/r): with
// inv = 1/r correctly rounded, q0 = RN(x * inv), the residual r0 = x - r * q0
// exact by an FMA, and RN(q0 + r0 * inv) is the correctly rounded quotient
// when nothing underflows or overflows (P. Markstein, "IA-64 and Elementary
// Functions", 2000, theorem 8.10) — so for |x| in [2^-100, 2^100] and r in
// [2^-20, 2^20]; other values take the IEEE division.  Three instructions in
// place of the division sequence, and no branch on the common path.
template <int DT>
__device__ __forceinline__ uint32_t penalize_fast(uint32_t bits, uint32_t count, const vi_row_params& p, float inv,
                                                  bool rep_fast) {
#pragma clang fp contract(off)
    const float x = Elem<DT>::decode(bits);
    float y = x;
    if (p.repetition_penalty != 1.0f) {
        const float q0 = x * inv;
        const float r0 = fmaf(-q0, p.repetition_penalty, x);
        float q = fmaf(r0, inv, q0);
        const float ax = fabsf(x);
        if (x > 0.0f && !(rep_fast && ax >= 0x1p-100f && ax <= 0x1p100f)) q = x / p.repetition_penalty;
        y = x > 0.0f ? q : x * p.repetition_penalty;
    }
    if (p.frequency_penalty != 0.0f) {
        const float t = p.frequency_penalty * float(count);
        y = y - t;
    }
    if (p.presence_penalty != 0.0f) y = y - p.presence_penalty;
    return Elem<DT>::round(y);
}

// Final (penalized) bits of a present token at offset off: count 1, or the
// repeat count when its R bit is set; a non-finite raw value stays as it is.
template <int DT>
__device__ __forceinline__ uint32_t present_final(const PartArgs& a, const PenIn& c, const vi_row_params& p,
                                                  const uint32_t* X, const unsigned char* R8, int s0, float inv,
                                                  bool rep_fast, uint32_t raw, uint32_t off) {
    if (!Elem<DT>::finite_bits(raw)) return raw;
    uint32_t cnt = 1u;
    if ((R8[off >> 3] >> (off & 7u)) & 1u) cnt = repeat_count(a, c, X, s0, off);
    return penalize_fast<DT>(raw, cnt, p, inv, rep_fast);
}

// Histogram slot of a 16-bit pattern: word = pattern & 0x7fff, the low half
// for sign 0 and the high half for sign 1 (the compaction puts the halves in
// key order and counts -0 with +0).
__device__ __forceinline__ uint32_t hist_inc(uint32_t b) { return 1u << ((b >> 15) << 4); }

// ------------------------------------------------------------------ part pass
// Histogram of the part's final patterns into H (zero on entry), then the
// compaction into the part's list and head (H zero again on exit).
template <int DT>
__device__ __forceinline__ void part_pass(const PartArgs& a, int row, int q, const vi_row_params& p, const PenIn& c,
                                          const uint4 (&v)[kNV], const uint32_t (&pb)[kNV], unsigned char* lds,
                                          Shared& sh) {
    const int tid = opaque_tid(), lane = tid & (kWave - 1), wave = tid / kWave;
    const int L = a.part_len, s0 = q * L, n = min(L, a.vocabulary - s0), nvec = n >> 3;
    uint32_t* H = reinterpret_cast<uint32_t*>(lds + kOffH);
    uint32_t* X = reinterpret_cast<uint32_t*>(lds + kOffX);
    uint32_t* R = reinterpret_cast<uint32_t*>(lds + kOffR);
    const unsigned char* R8 = reinterpret_cast<const unsigned char*>(R);
    uint16_t* F = reinterpret_cast<uint16_t*>(lds + kOffF);
    uint32_t* plist = a.plists + (size_t(row) * a.parts + q) * size_t(L);
    constexpr uint32_t kExp = DT == VI_BF16 ? 0x7f80u : 0x7c00u, kExpLsb = DT == VI_BF16 ? 0x80u : 0x400u;
    uint32_t bad = 0u;

    // ---- present tokens: their offsets, from the lane's presence-bitmap words
    // (thread t holds tokens [64 t, 64 t + 64) of the part), staged in id order
    // in F; every thread then takes every kT-th staged token, gathers its raw
    // logit again (from cache: the part was just read), penalizes it, counts it
    // and records (offset, final bits) in the part's present list.
    if (c.pen) {
        build_repeat_hash(a, c, s0, n, X, R, sh);
        const float inv = 1.0f / p.repetition_penalty;   // (IEEE division: correctly rounded)
        const bool rep_fast = p.repetition_penalty >= 0x1p-20f && p.repetition_penalty <= 0x1p20f;
        const uint32_t* b1w = reinterpret_cast<const uint32_t*>(c.st + a.pl.off_b1) + (s0 >> 5);
        const int nw = (n + 31) >> 5;
        uint32_t bw[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int wd = 2 * tid + u;
            const int nb = min(32, n - 32 * wd);
            bw[u] = wd < nw ? b1w[wd] & (nb >= 32 ? 0xffffffffu : (1u << nb) - 1u) : 0u;
        }
        uint32_t npres = 0u;
        const uint32_t rank0 = block_scan_lds(uint32_t(__builtin_popcount(bw[0]) + __builtin_popcount(bw[1])),
                                              sh.scan, &npres);
        const uint16_t* row16 = static_cast<const uint16_t*>(a.logits) + size_t(row) * size_t(a.stride) + size_t(s0);
        for (uint32_t r0 = 0; r0 < npres; r0 += kStage) {   // (uniform; one round up to 9,216 tokens)
            uint32_t r = rank0;
#pragma unroll
            for (int u = 0; u < 2; ++u)
                for (uint32_t bits = bw[u]; bits; bits &= bits - 1u, ++r)
                    if (r >= r0 && r < r0 + kStage) F[r - r0] = uint16_t(64 * tid + 32 * u + __builtin_ctz(bits));
            lds_barrier();
            const uint32_t m = min(npres - r0, uint32_t(kStage));
            uint32_t offs[kStage / kT], raws[kStage / kT];
#pragma unroll
            for (int k = 0; k < kStage / kT; ++k) {   // the gathers, all in flight
                const uint32_t idx = uint32_t(k * kT + tid);
                offs[k] = idx < m ? uint32_t(F[idx]) : 0u;
                raws[k] = idx < m ? uint32_t(row16[offs[k]]) : 0u;
            }
#pragma unroll
            for (int k = 0; k < kStage / kT; ++k) {
                const uint32_t idx = uint32_t(k * kT + tid);
                if (idx >= m) break;
                const uint32_t raw = raws[k], off = offs[k];
                const uint32_t bits = present_final<DT>(a, c, p, X, R8, s0, inv, rep_fast, raw, off);
                const uint32_t nf = ((bits & kExp) + kExpLsb) >> 15;
                bad |= nf;
                atomicAdd(&H[bits & 0x7fffu], (nf ^ 1u) * hist_inc(bits));
                plist[r0 + idx] = (off << 16) | bits;   // (the merge's owner scan reads it)
            }
            lds_barrier();
        }
        if (tid == 0) sh.npres = npres;
    }

    // ---- absent tokens at their raw pattern, branch-free (a present,
    // non-finite or out-of-range one adds 0)
#pragma unroll
    for (int i = 0; i < kNV; ++i) {
        const int vi = i * kT + tid;
        const uint32_t inb = uint32_t(vi < nvec);
        const uint32_t absent = inb ? ~pb[i] : 0u;
#pragma unroll
        for (int e = 0; e < 8; ++e) {   // (integer forms: no lane masks to hold)
            const uint32_t b = vec_bits<DT>(v[i], e);
            const uint32_t nf = ((b & kExp) + kExpLsb) >> 15;   // 1: exponent all ones
            bad |= inb & nf;
            atomicAdd(&H[b & 0x7fffu], ((absent >> e) & (nf ^ 1u) & 1u) << ((b >> 15) << 4));
        }
    }
    if (ballot(bad != 0u) && lane == 0) atomicOr(&sh.flags, uint32_t(VI_FLAG_NONFINITE));
    lds_barrier();

    // ---- compaction.  Word w holds pattern w (sign 0, key w | 0x8000) in its
    // low half and pattern w | 0x8000 (sign 1, key 0x7fff - w) in its high
    // half; -0 (the high half of word 0) is counted with +0.  The list is in
    // key order: the sign-1 entries by descending word, then the sign-0 ones by
    // ascending word.  Wave w takes words [2048 w, 2048 w + 2048) in 8 steps of
    // 4 words per lane; pass 1 counts (packed sign-0 | sign-1 << 16), pass 2
    // writes and zeroes.  A step whose keys all lie in [kmin, kmax] skips the
    // per-key range tests.
    const uint32_t kmin = sh.kmin, kmax = sh.kmax;
    constexpr int kWPW = kHW / kW;   // words per wave
    const int wbase = wave * kWPW;
    auto halves = [&](uint32_t wi, uint32_t h, uint32_t& lo, uint32_t& hi) {
        lo = h & 0xffffu;
        hi = h >> 16;
        if (wi == 0u) { lo += hi; hi = 0u; }   // -0 counts as +0
    };
    uint32_t xl = 0u;
    bool over = false;
#pragma unroll 1
    for (int st = 0; st < 8; ++st) {
        const uint32_t w0 = uint32_t(wbase + 256 * st);
        const uint4 h4 = *reinterpret_cast<const uint4*>(H + w0 + 4 * lane);
        if (!ballot((h4.x | h4.y | h4.z | h4.w) != 0u)) continue;   // (uniform) an empty step
        const bool inside = (w0 | 0x8000u) >= kmin && ((w0 + 255u) | 0x8000u) <= kmax &&
                            0x7fffu - (w0 + 255u) >= kmin && 0x7fffu - w0 <= kmax;
        const uint32_t w4[4] = {h4.x, h4.y, h4.z, h4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t wi = w0 + uint32_t(4 * lane + j);
            uint32_t lo, hi;
            halves(wi, w4[j], lo, hi);
            bool vlo = lo != 0u, vhi = hi != 0u;
            if (!inside) {
                const uint32_t klo = wi | 0x8000u, khi = 0x7fffu - wi;
                const bool ilo = klo >= kmin && klo <= kmax, ihi = khi >= kmin && khi <= kmax;
                over |= (vlo && !ilo) || (vhi && !ihi);
                vlo = vlo && ilo;
                vhi = vhi && ihi;
            }
            xl += uint32_t(vlo) | (uint32_t(vhi) << 16);
        }
    }
    const uint32_t wtot = wave_sum_u32(xl);
    if (lane == 0) sh.scan[wave] = wtot;
    if (ballot(over) && lane == 0) atomicOr(&sh.flags, uint32_t(VI_FLAG_NONFINITE));
    lds_barrier();
    uint32_t wb = 0u, tot = 0u;
#pragma unroll
    for (int w = 0; w < kW; ++w) {
        const uint32_t t = sh.scan[w];
        wb += w < wave ? t : 0u;
        tot += t;
    }
    const uint32_t n_pos = tot & 0xffffu, n_neg = tot >> 16, n_all = n_pos + n_neg;
    uint32_t* list = a.lists + (size_t(row) * a.parts + q) * size_t(L);
    uint32_t before = wb, nval = 0u;   // packed positions of the step's first entries
#pragma unroll 1
    for (int st = 0; st < 8; ++st) {
        const uint32_t w0 = uint32_t(wbase + 256 * st);
        uint4* src = reinterpret_cast<uint4*>(H + w0 + 4 * lane);
        const uint4 h4 = *src;
        if (!ballot((h4.x | h4.y | h4.z | h4.w) != 0u)) continue;   // (uniform) an empty step
        *src = make_uint4(0u, 0u, 0u, 0u);
        const bool inside = (w0 | 0x8000u) >= kmin && ((w0 + 255u) | 0x8000u) <= kmax &&
                            0x7fffu - (w0 + 255u) >= kmin && 0x7fffu - w0 <= kmax;
        const uint32_t w4[4] = {h4.x, h4.y, h4.z, h4.w};
        uint32_t lo4[4], hi4[4], xs = 0u;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t wi = w0 + uint32_t(4 * lane + j);
            halves(wi, w4[j], lo4[j], hi4[j]);
            if (!inside) {
                const uint32_t klo = wi | 0x8000u, khi = 0x7fffu - wi;
                if (!(klo >= kmin && klo <= kmax)) lo4[j] = 0u;
                if (!(khi >= kmin && khi <= kmax)) hi4[j] = 0u;
            }
            xs += uint32_t(lo4[j] != 0u) | (uint32_t(hi4[j] != 0u) << 16);
        }
        const uint32_t incl = wave_incl_scan_u32(xs);
        const uint32_t ex = before + incl - xs;
        before += uint32_t(readlane_i(int(incl), kWave - 1));
        uint32_t ppos = n_neg + (ex & 0xffffu), pneg = n_neg - 1u - (ex >> 16);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t wi = w0 + uint32_t(4 * lane + j);
            if (lo4[j]) {
                const uint32_t key = wi | 0x8000u;
                if (ppos == n_all - 1u) sh.top = key + 1u;
                list[ppos++] = (key << 16) | lo4[j];
            }
            if (hi4[j]) {
                const uint32_t key = 0x7fffu - wi;
                if (pneg == n_all - 1u) sh.top = key + 1u;
                list[pneg--] = (key << 16) | hi4[j];
            }
            nval += lo4[j] + hi4[j];
        }
    }
    const uint32_t wv = wave_sum_u32(nval);
    if (lane == 0) atomicAdd(&sh.nvalid, wv);
    lds_barrier();
    if (tid == 0) {
        uint32_t* hd = a.heads + (size_t(row) * a.parts + q) * kHead;
        hd[0] = n_all;
        hd[1] = sh.flags | (c.pen ? (c.hflags & (VI_FLAG_BAD_HISTORY | VI_FLAG_ERROR)) : 0u);
        hd[2] = n_all ? sh.top : 0u;
        hd[3] = sh.nvalid;
        hd[4] = sh.npres;
        sh.flags = 0u; sh.top = 0u; sh.nvalid = 0u; sh.npres = 0u;
    }
    lds_barrier();
}

// ------------------------------------------------------------------ merge
__device__ __forceinline__ void write_row(const PartArgs& a, int row, int32_t token, double u, uint32_t flags,
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

// First i in [0, n) with pred(i) (monotone false -> true over i), or n; every
// thread calls it; thread i < n evaluates pred(i) and pred(i - 1).
template <class F>
__device__ __forceinline__ int first_true(int n, F pred, Shared& sh) {
    const int tid = threadIdx.x;
    if (tid == 0) sh.res = n;
    __syncthreads();
    if (tid < n && pred(tid) && (tid == 0 || !pred(tid - 1))) sh.res = tid;
    __syncthreads();
    const int r = sh.res;
    __syncthreads();
    return r;
}

template <int DT>
__device__ __forceinline__ void merge_row(const PartArgs& a, int row, const vi_row_params& p, const PenIn& c,
                                          unsigned char* lds, Shared& sh) {
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const int P = a.parts, L = a.part_len, V = a.vocabulary;
    uint32_t* FIRST = reinterpret_cast<uint32_t*>(lds + kOffFirst);
    uint32_t* NE = reinterpret_cast<uint32_t*>(lds + kOffNE);
    uint32_t* BC = reinterpret_cast<uint32_t*>(lds + kOffBC);
    uint64_t* BM = reinterpret_cast<uint64_t*>(lds + kOffBM);
    uint32_t* CC = reinterpret_cast<uint32_t*>(lds + kOffCC);
    uint64_t* CM = reinterpret_cast<uint64_t*>(lds + kOffCM);
    uint32_t* FC = reinterpret_cast<uint32_t*>(lds + kOffFC);
    uint32_t* KN = reinterpret_cast<uint32_t*>(lds + kOffKN);
    uint32_t* KC = reinterpret_cast<uint32_t*>(lds + kOffKC);
    uint64_t* KW = reinterpret_cast<uint64_t*>(lds + kOffKW);
    uint64_t* KM = reinterpret_cast<uint64_t*>(lds + kOffKM);
    const size_t rp = size_t(row) * P;
    auto list_of = [&](int q) { return a.lists + (rp + q) * size_t(L); };

    // ---- heads
    uint32_t hn = 0u, hf = 0u, ht = 0u, hv = 0u;
    if (tid < P) {
        const uint32_t* hd = a.heads + (rp + tid) * kHead;
        hn = hd[0]; hf = hd[1]; ht = hd[2]; hv = hd[3];
    }
    if (tid == 0) { sh.m_flags = 0u; sh.m_top = 0u; sh.m_valid = 0u; }
    for (int i = tid; i < P * kBins; i += kT) { FIRST[i] = 0xffffffffu; NE[i] = 0u; }
    if (tid < kBins) { BC[tid] = 0u; BM[tid] = 0ull; }
    __syncthreads();
    if (tid < P) {
        atomicOr(&sh.m_flags, hf);
        atomicMax(&sh.m_top, ht);
        atomicAdd(&sh.m_valid, hv);
    }
    if (wave == 0) {   // entry bases of the parts
        const uint32_t nn = lane < P ? hn : 0u;
        const uint32_t in = wave_incl_scan_u32(nn);
        if (lane < P) sh.m_base[lane + 1] = in;
        if (lane == 0) sh.m_base[0] = 0u;
    }
    __syncthreads();
    const uint32_t flags = sh.m_flags, top1 = sh.m_top, N = sh.m_valid;
    const uint32_t out_flags = flags & (VI_FLAG_NONFINITE | VI_FLAG_BAD_HISTORY);
    const bool fail = (flags & VI_FLAG_ERROR) != 0u || !(p.temperature <= kMaxTemperature);
    if (fail || N == 0u || top1 == 0u) {
        if (tid == 0) write_row(a, row, fail ? -1 : V, 0.0, out_flags | (fail ? VI_FLAG_ERROR : VI_FLAG_EMPTY), 0u, 0u, 0.0);
        __syncthreads();
        return;
    }
    const float inv_t = 1.0f / p.temperature;
    const double z0 = double(key_z<DT>(top1 - 1u, inv_t));

    // ---- every entry into the coarse bins.  Thread t takes a contiguous run of
    // the concatenated lists (a part's list is in key order, so equal
    // (part, bin) tags are adjacent) and adds each tag's sums once (LDS atomics
    // per run, exact u64 mass sums).  Entries are loaded 8 at a time.
    const uint32_t E = sh.m_base[P];
    {
        const uint32_t per = (E + kT - 1) / kT, e0 = min(uint32_t(tid) * per, E), e1 = min(e0 + per, E);
        uint32_t tag = 0xffffffffu, rc = 0u, rn = 0u, rj = 0u;
        uint64_t rm = 0ull;
        auto flush = [&]() {
            if (tag == 0xffffffffu) return;
            const uint32_t q = tag >> 9, b = tag & uint32_t(kBins - 1);
            atomicAdd(&BC[b], rc);
            atomicAdd(reinterpret_cast<unsigned long long*>(&BM[b]), (unsigned long long)rm);
            atomicMin(&FIRST[q * kBins + b], rj);
            atomicAdd(&NE[q * kBins + b], rn);
        };
        int q = 0;
        while (q + 1 < P && e0 >= sh.m_base[q + 1]) ++q;
        constexpr int kEB = 8;
        for (uint32_t g = e0; g < e1; g += kEB) {
            uint32_t ents[kEB], js[kEB], qs[kEB];
#pragma unroll
            for (int u = 0; u < kEB; ++u) {
                const uint32_t e = g + uint32_t(u);
                while (e < e1 && q + 1 < P && e >= sh.m_base[q + 1]) ++q;
                qs[u] = uint32_t(q);
                js[u] = e - sh.m_base[q];
                ents[u] = e < e1 ? list_of(q)[js[u]] : 0u;
            }
            uint64_t ms[kEB];
#pragma unroll
            for (int u = 0; u < kEB; ++u)   // (count 0 past the end)
                ms[u] = uint64_t(ents[u] & 0xffffu) * weight_fx<DT>(ents[u] >> 16, inv_t, z0);
#pragma unroll
            for (int u = 0; u < kEB; ++u) {
                if (g + uint32_t(u) >= e1) break;
                const uint32_t t = (qs[u] << 9) | (ents[u] >> 23);   // (part, bin = key >> 7)
                if (t != tag) {
                    flush();
                    tag = t; rc = 0u; rn = 0u; rm = 0ull; rj = js[u];
                }
                rc += ents[u] & 0xffffu;
                rm += ms[u];
                ++rn;
            }
        }
        flush();
    }
    __syncthreads();

    // ---- prefix sums from the top bin: CC / CM [i] cover bins 511 .. 511 - i
    uint32_t ci = 0u;
    uint64_t mi = 0ull;
    if (tid < kBins) {
        const int b = kBins - 1 - tid;
        const uint32_t cb = BC[b];
        const uint64_t mb = BM[b];
        ci = wave_incl_scan_u32(cb);
        mi = wave_incl_scan_u64(mb);
        if (lane == kWave - 1) { sh.wc[wave] = ci; sh.wm[wave] = mi; }
    }
    __syncthreads();
    if (tid < kBins) {
        for (int w = 0; w < wave; ++w) { ci += sh.wc[w]; mi += sh.wm[w]; }
        CC[tid] = ci;
        CM[tid] = mi;
    }
    __syncthreads();
    const uint64_t s_all = CM[kBins - 1];

    // ---- fine tables of bin b: per key in descending order, tokens, weight,
    // and inclusive prefixes from the top of the row; FC keeps the per-part counts
    auto gather = [&](int b) {
        const int ib = kBins - 1 - b;
        const uint32_t c0 = ib ? CC[ib - 1] : 0u;
        const uint64_t m0 = ib ? CM[ib - 1] : 0ull;
        for (int i = tid; i < P * kBinKeys; i += kT) FC[i] = 0u;
        __syncthreads();
        {
            const int q = tid / kBinKeys, j = tid % kBinKeys;
            if (q < P && uint32_t(j) < NE[q * kBins + b]) {
                const uint32_t ent = list_of(q)[FIRST[q * kBins + b] + uint32_t(j)];
                FC[q * kBinKeys + ((ent >> 16) & uint32_t(kBinKeys - 1))] = ent & 0xffffu;
            }
        }
        __syncthreads();
        uint32_t kc = 0u;
        uint64_t km = 0ull;
        if (tid < kBinKeys) {
            const int kk = kBinKeys - 1 - tid;
            uint32_t cnt = 0u;
            for (int q = 0; q < P; ++q) cnt += FC[q * kBinKeys + kk];
            const uint64_t w = cnt ? weight_fx<DT>(uint32_t(b * kBinKeys + kk), inv_t, z0) : 0ull;
            KN[tid] = cnt;
            KW[tid] = w;
            kc = wave_incl_scan_u32(cnt);
            km = wave_incl_scan_u64(uint64_t(cnt) * w);
            if (lane == kWave - 1 && wave == 0) { sh.wc[0] = kc; sh.wm[0] = km; }
        }
        __syncthreads();
        if (tid < kBinKeys) {
            if (wave == 1) { kc += sh.wc[0]; km += sh.wm[0]; }
            KC[tid] = c0 + kc;
            KM[tid] = m0 + km;
        }
        __syncthreads();
    };
    // The key of fine index t in bin b, its tokens before it, its mass before it.
    auto key_at = [&](int b, int t) {
        t = min(t, kBinKeys - 1);
        if (tid == 0) {
            sh.key = uint32_t(b * kBinKeys + kBinKeys - 1 - t);
            sh.cnt_before = KC[t] - KN[t];
            sh.mass_before = KM[t] - uint64_t(KN[t]) * KW[t];
            sh.wfx = KW[t];
            sh.take = KN[t];
        }
        __syncthreads();
    };

    // ---- top-k cap: (tokens, mass) of the cap set
    uint32_t cap_cnt = N;
    uint64_t cap_mass = s_all;
    if (p.top_k > 0 && uint32_t(p.top_k) < N) {
        const uint32_t k = uint32_t(p.top_k);
        const int ib = first_true(kBins, [&](int i) { return CC[i] >= k; }, sh);
        const int b = kBins - 1 - ib;
        gather(b);
        const int t = first_true(kBinKeys, [&](int i) { return KC[i] >= k; }, sh);
        key_at(b, t);
        cap_cnt = k;
        cap_mass = sh.mass_before + uint64_t(k - sh.cnt_before) * sh.wfx;
        __syncthreads();
    }
    // ---- min-p: keys with w < min_p are cut (w of the top key is 1)
    uint32_t lim_cnt = cap_cnt;
    uint64_t lim_mass = cap_mass;
    if (p.min_p > 0.0f) {
        if (wave == 0) {
            const double mp = double(p.min_p);
            const int km = wave_search(int(sh.kmin), int(top1), [&](int key) {
                return exp(double(key_z<DT>(uint32_t(key), inv_t)) - z0) >= mp;
            });
            if (lane == 0) sh.res = km;
        }
        __syncthreads();
        const int km = sh.res;
        __syncthreads();
        if (km >= int(top1)) {   // min_p > 1: no token passes (the support keeps the first)
            lim_cnt = 0u;
            lim_mass = 0ull;
        } else {
            const int b = km >> 7;
            gather(b);
            const int tm = b * kBinKeys + kBinKeys - 1 - km;   // fine index of key km
            if (KC[tm] < lim_cnt) { lim_cnt = KC[tm]; lim_mass = KM[tm]; }
            __syncthreads();
        }
    }
    // ---- top-p: the first token whose cumulative mass reaches top_p * cap mass
    uint32_t n_sup = lim_cnt;
    uint64_t s_sup = lim_mass;
    if (p.top_p < 1.0f) {
        const double tgt = ceil(double(p.top_p) * double(cap_mass));
        const uint64_t tp = tgt <= 0.0 ? 0ull : uint64_t(tgt);
        const int ib = first_true(kBins, [&](int i) { return CM[i] >= tp; }, sh);
        if (ib < kBins) {
            const int b = kBins - 1 - ib;
            gather(b);
            const int t = first_true(kBinKeys, [&](int i) { return KM[i] >= tp; }, sh);
            key_at(b, t);
            const uint64_t rem = tp > sh.mass_before ? tp - sh.mass_before : 0ull;
            uint64_t take = sh.wfx ? (rem + sh.wfx - 1ull) / sh.wfx : 1ull;
            take = max(take, 1ull);
            const uint32_t pc = sh.cnt_before + uint32_t(take);
            if (pc < n_sup) { n_sup = pc; s_sup = sh.mass_before + take * sh.wfx; }
            __syncthreads();
        }
    }
    if (n_sup < 1u) {   // the first token alone
        n_sup = 1u;
        const int b = int(top1 - 1u) >> 7;
        gather(b);
        key_at(b, first_true(kBinKeys, [&](int i) { return KC[i] >= 1u; }, sh));
        s_sup = sh.wfx;
    }
    // ---- the draw: first token whose cumulative mass exceeds u * S_n
    const double u = philox_uniform(p.seed, p.lane, p.position, 0u);
    const double td_ = floor(u * double(s_sup));
    uint64_t td = td_ <= 0.0 ? 0ull : uint64_t(td_);
    if (td >= s_sup && s_sup) td = s_sup - 1ull;
    uint32_t pos = n_sup;   // 1-based position of the drawn token in (z desc, id asc) order
    bool found = false;
    {
        const int ib = first_true(kBins, [&](int i) { return CM[i] > td; }, sh);
        if (ib < kBins) {
            const int b = kBins - 1 - ib;
            gather(b);
            const int t = first_true(kBinKeys, [&](int i) { return KM[i] > td; }, sh);
            key_at(b, t);
            const uint64_t take = sh.wfx ? (td - sh.mass_before) / sh.wfx + 1ull : 1ull;
            pos = sh.cnt_before + uint32_t(take);
            found = pos <= n_sup;
        }
    }
    if (!found) {   // (rounding only) the support's last token: its key by count
        pos = n_sup;
        const int ib = first_true(kBins, [&](int i) { return CC[i] >= pos; }, sh);
        const int b = kBins - 1 - ib;
        gather(b);
        const int t = first_true(kBinKeys, [&](int i) { return KC[i] >= pos; }, sh);
        key_at(b, t);
    }
    const uint32_t K = sh.key, kk = K & uint32_t(kBinKeys - 1);
    uint32_t r = pos - sh.cnt_before;   // 1-based rank among the key's tokens in id order
    int qo = 0;
    for (; qo < P - 1; ++qo) {
        const uint32_t cq = FC[qo * kBinKeys + kk];
        if (r <= cq) break;
        r -= cq;
    }
    __syncthreads();

    // ---- the part holding it, read again: the r-th token of key K in id order
    const int s0 = qo * L, n = min(L, V - s0), nvec = n >> 3;
    uint4 v[kNV];
    uint32_t pb[kNV];
    load_part<DT>(a, c, row, s0, nvec, v, pb);
    uint32_t* M = reinterpret_cast<uint32_t*>(lds + kOffMatch);   // present tokens of key K
    const unsigned char* M8 = reinterpret_cast<const unsigned char*>(M);
    if (tid < kNV) sh.rnd[tid] = 0u;
    if (tid == 0) sh.token = -1;
#pragma unroll
    for (int i = 0; i < kRW / kT; ++i) M[i * kT + tid] = 0u;
    __syncthreads();
    if (c.pen) {   // present tokens of key K, from the part pass's present list
        const uint32_t np = a.heads[(rp + qo) * kHead + 4];
        const uint32_t* pl = a.plists + (rp + qo) * size_t(L);
        for (uint32_t k = uint32_t(tid); k < np; k += kT) {
            const uint32_t ent = pl[k], bits = ent & 0xffffu, off = ent >> 16;
            if (Elem<DT>::finite_bits(bits) && key16(bits) == K) atomicOr(&M[off >> 5], 1u << (off & 31u));
        }
    }
    __syncthreads();
    uint32_t mk[kNV];
#pragma unroll
    for (int i = 0; i < kNV; ++i) {   // absent tokens at their raw pattern, present ones from M
        const int vi = i * kT + tid;
        const bool inb = vi < nvec;
        const uint32_t absent = inb ? ~pb[i] : 0u;
        uint32_t m = 0u;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t bits = vec_bits<DT>(v[i], e);
            m |= uint32_t(((absent >> e) & 1u) && Elem<DT>::finite_bits(bits) && key16(bits) == K) << e;
        }
        m |= inb ? uint32_t(M8[vi]) : 0u;
        mk[i] = m;
        const uint32_t ws = wave_sum_u32(uint32_t(__builtin_popcount(m)));
        if (lane == 0 && ws) atomicAdd(&sh.rnd[i], ws);
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t rr = r;
        int ri = 0;
        for (; ri < kNV - 1; ++ri) {
            if (rr <= sh.rnd[ri]) break;
            rr -= sh.rnd[ri];
        }
        sh.ri = uint32_t(ri);
        sh.rr = rr;
    }
    __syncthreads();
    const int ri = int(sh.ri);
    const uint32_t rr = sh.rr;
    uint32_t m = 0u;
#pragma unroll
    for (int i = 0; i < kNV; ++i) m = i == ri ? mk[i] : m;
    const uint32_t cnt = uint32_t(__builtin_popcount(m));
    uint32_t total = 0u;
    const uint32_t excl = block_exclusive_scan_u32<kT>(cnt, sh.scan, &total);
    if (cnt && rr > excl && rr <= excl + cnt)
        sh.token = s0 + 8 * (ri * kT + tid) + nth_set_bit(m, rr - excl - 1u);
    __syncthreads();
    if (tid == 0) {
        const int32_t tok = sh.token;
        const double s_n = double(s_sup) * (1.0 / kScale);
        if (tok < 0) {   // the entries disagree with the part: cannot happen for consistent inputs
            write_row(a, row, -1, u, out_flags | VI_FLAG_ERROR, 0u, 0u, 0.0);
        } else {
            write_row(a, row, tok, u, out_flags, n_sup, N, s_n);
            if (a.record && a.pstate && tok < V) {
                const LaneState ls = lane_state(a.pstate + size_t(row) * a.pl.lane_bytes, a.pl);
                state_publish(ls, state_apply(ls, a.pl, V, tok, 1));
            }
        }
    }
    __syncthreads();
}

// ------------------------------------------------------------------ kernels
template <int DT>
__global__ __launch_bounds__(kT) void part_kernel(PartArgs a) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[kLds];
    __shared__ Shared sh;
    const int tid = threadIdx.x;
    uint32_t* H = reinterpret_cast<uint32_t*>(lds + kOffH);
#pragma unroll
    for (int i = 0; i < kHW / 4 / kT; ++i) reinterpret_cast<uint4*>(H)[i * kT + tid] = make_uint4(0u, 0u, 0u, 0u);
    if (tid == 0) { sh.flags = 0u; sh.top = 0u; sh.nvalid = 0u; sh.npres = 0u; }
    for (int k = 0;; ++k) {
        int row, q;
        if (!item_of(a, k, &row, &q)) break;
        const vi_row_params p = a.params[row];
        if (!full_route_row(p)) continue;
        const PenIn c = pen_in(a, row, p);
        const int L = a.part_len, s0 = q * L, nvec = min(L, a.vocabulary - s0) >> 3;
        uint4 v[kNV];
        uint32_t pb[kNV];
        load_part<DT>(a, c, row, s0, nvec, v, pb);
        if (tid < kWave) {
            const uint32_t kr = valid_key_range<DT>(p.temperature);
            if (tid == 0) { sh.kmin = kr & 0xffffu; sh.kmax = kr >> 16; }
        }
        lds_barrier();
        part_pass<DT>(a, row, q, p, c, v, pb, lds, sh);
    }
}

template <int DT>
__global__ __launch_bounds__(kT) void part_merge_kernel(PartArgs a) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[kLds];
    __shared__ Shared sh;
    const int row = int(blockIdx.x);
    const vi_row_params p = a.params[row];
    if (!full_route_row(p)) return;
    if (threadIdx.x < kWave) {
        const uint32_t kr = valid_key_range<DT>(p.temperature);
        if (threadIdx.x == 0) { sh.kmin = kr & 0xffffu; sh.kmax = kr >> 16; }
    }
    merge_row<DT>(a, row, p, pen_in(a, row, p), lds, sh);
}

}  // namespace

// Geometry of the parts route for a vocabulary: parts and tokens per part.
static void part_geometry(int vocabulary, int* parts, int* part_len) {
    const int P = (vocabulary + kPartMax - 1) / kPartMax;
    const int L = ((vocabulary + P - 1) / P + 31) / 32 * 32;
    *parts = P;
    *part_len = L;
}

bool parts_supported(int dtype, int vocabulary, int64_t stride, const void* logits) {
    if (dtype != VI_BF16 && dtype != VI_F16) return false;
    if (vocabulary < 8 || vocabulary % 8 || stride % 8 || reinterpret_cast<uintptr_t>(logits) % 16) return false;
    return vocabulary <= kMaxParts16 * kPartMax;
}

size_t parts_workspace(int rows, int vocabulary) {
    if (vocabulary <= 0 || vocabulary > kMaxParts16 * kPartMax) return 0;
    int P = 0, L = 0;
    part_geometry(vocabulary, &P, &L);
    const size_t rp = size_t(rows) * size_t(P);
    return align_up(rp * kHead * 4, 256) + 2 * align_up(rp * size_t(L) * 4, 256) + 768;
}

vi_status launch_parts(const SampleArgs& s, unsigned char* ws, size_t ws_bytes, hipStream_t stream) {
    if (!parts_supported(s.dtype, s.vocabulary, s.stride, s.logits)) return VI_ERR_UNSUPPORTED;
    PartArgs a{};
    part_geometry(s.vocabulary, &a.parts, &a.part_len);
    const size_t rp = size_t(s.rows) * size_t(a.parts);
    Carver c(ws, ws_bytes);
    a.heads = c.take<uint32_t>(rp * kHead);
    a.lists = c.take<uint32_t>(rp * size_t(a.part_len));
    a.plists = c.take<uint32_t>(rp * size_t(a.part_len));
    if (!c.ok) return VI_ERR_WORKSPACE;
    a.logits = s.logits; a.rows = s.rows; a.vocabulary = s.vocabulary; a.stride = s.stride;
    a.params = s.params;
    if (s.pstate) { a.pstate = s.pstate; a.pl = s.playout; a.record = s.record; }
    a.tokens = s.tokens; a.uniforms = s.uniforms; a.stats = s.stats;
    const int items = s.rows * a.parts;
    a.grid = std::min(device_cus(), items);
    if (s.dtype == VI_BF16) {
        hipLaunchKernelGGL(part_kernel<VI_BF16>, dim3(a.grid), dim3(kT), 0, stream, a);
        hipLaunchKernelGGL(part_merge_kernel<VI_BF16>, dim3(s.rows), dim3(kT), 0, stream, a);
    } else {
        hipLaunchKernelGGL(part_kernel<VI_F16>, dim3(a.grid), dim3(kT), 0, stream, a);
        hipLaunchKernelGGL(part_merge_kernel<VI_F16>, dim3(s.rows), dim3(kT), 0, stream, a);
    }
    return launch_status();
}

}  // namespace vi
