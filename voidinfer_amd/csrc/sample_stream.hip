// sample_stream.hip — full-vocabulary rows of the batched sampler, 16-bit
// logits (temperature > 0, top_k = 0 or > 64): penalties, temperature, top-k /
// min-p / top-p over the whole vocabulary and the Philox inverse-CDF draw.
// Serves rows whose logits are 16-byte aligned, whose vocabulary is a multiple
// of 8, and whose caller wants tokens (uniforms, stats, recording into penalty
// states) but no probabilities or bounds; the slice / merge kernels
// (sample_slices.hip) serve every other 16-bit row.
//
// Key fact: bf16 / fp16 logits, and penalized logits stored back in the same
// dtype, take one of 65,536 bit patterns, and z = x' * (1/T) is a strictly
// monotone function of the pattern's order key (for T <= 65,536; +0 and -0
// share z = 0).  The multiset of z over a row is a count histogram over
// patterns; every truncation and the draw are prefix sums over the occupied
// patterns in key order, with one exp per occupied pattern, not per token.
//
// Stream launch (stream_kernel).  A row is cut into P parts of at most 65,528
// tokens, so a part's count of one pattern fits 16 bits.  Persistent
// workgroups of 1024 threads (one per CU: the histogram takes 128 KB of LDS)
// take the parts of their XCD's rows in a fixed order, with the next part's
// first logits in flight while the current part finishes.  Each wave owns one
// 16-byte vector per lane and round (512 consecutive tokens), four rounds in
// flight per thread; no workgroup barrier runs inside the stream.  Every token
// adds one to its raw pattern's u16 count (histogram word = pattern & 0x7fff,
// half = sign).  Where the row has penalties, the wave stages its vectors in
// LDS, lists its history tokens (the presence bitmap's byte of each vector)
// and handles them 64 at a time, one per lane: the count moves from the raw
// pattern to the penalized one (occurrence count 1).  Tokens seen more than
// once (the repeat list) are corrected at the end of the part: one count moves
// from the count-1 pattern to the count-c one.  Each thread then owns 32
// histogram words (a group: 32 positive and 32 negative keys); the non-empty
// groups are stored at their place in the part's table, with an occupancy
// bitmap and the part's highest valid key, and the words are cleared.
//
// Merge launch (merge_kernel, one workgroup per row, on the XCD whose L2 holds
// the row's tables).  The row's occupied groups are summed over its parts per
// key; each occupied key is weighed exp(z - z0) once; prefix sums over 32-key
// blocks in descending key order (2^-40 fixed point: exact, independent of
// order) locate the top-k cap, the min-p and top-p cuts and the draw, each
// resolved inside its block; the part holding the drawn key's rank is read
// again to name the token (id order among equal keys), a history token's
// penalized key recognised from its raw key through the preimage of the drawn
// key under the (monotone) penalty.
//
// Roofline: HBM; V x 2 bytes of logits per row, plus the presence bitmap
// (V / 8 bytes) and the repeat list where the row has penalties.
#include <math.h>

#include <algorithm>

#include "keys16.h"
#include "penalty_state.h"
#include "vi_device.h"
#include "vi_internal.h"

namespace vi {
namespace {

constexpr int kT = 1024;                 // threads per workgroup
constexpr int kW = kT / kWave;           // waves per workgroup
constexpr int kHW = 32768;               // histogram words
constexpr int kGroups = 1024;            // 32-word groups (one per thread when published)
constexpr int kGW = 32;
constexpr int kDepth = 4;                // rounds of logits in flight per thread
constexpr int kXcds = 8;
constexpr int kRepPF = 2;                // repeat-list entries prefetched per thread
constexpr int kMaxParts = 16;            // parts per row
constexpr int kMaxPartLen = 65504;       // tokens per part (a multiple of 32 below 65,536)
constexpr int kPub = 32;                 // words per part header: the occupancy bitmap
constexpr uint32_t kTakeAll = 0xffffffffu;
constexpr double kFix = 0x1p40;          // fixed-point scale of the masses (w <= 1, counts <= 2^20)

// Stream LDS (bytes): H, the histogram (u16 counts in pairs: word p & 0x7fff,
// low half sign 0, high half sign 1); the waves' staged vectors; their lists
// of history tokens (u8 offsets inside the wave's 512 tokens; the lists of
// lanes 32..63 continue those of lanes 0..31, their offsets 256 higher).
constexpr int kOffH = 0;
constexpr int kOffStage = kOffH + 4 * kHW;
constexpr int kOffList = kOffStage + 16 * kT;
constexpr int kLds = kOffList + 8 * kT;
static_assert(kLds == 155648, "LDS map");

// Merge LDS (bytes).  The per-key counts of the row's occupied groups take
// what the fixed arrays leave (more groups than that are summed again from the
// parts' tables when needed).
constexpr int kOffMBits = 0;                          // u32[kMaxParts][32]: each part's occupied groups
constexpr int kOffMOcc = kOffMBits + 4 * 32 * kMaxParts;   // u32[32]: occupied in any part
constexpr int kOffMSlot = kOffMOcc + 128;             // u16[1024]: slot of group g
constexpr int kOffMGroupOf = kOffMSlot + 2048;        // u16[1024]: group of slot s
constexpr int kOffMBcnt = kOffMGroupOf + 2048;        // u32[2048]: logits per 32-key block
constexpr int kOffMBmass = kOffMBcnt + 8192;          // u64[2048]: block masses, fixed point
constexpr int kOffMCab = kOffMBmass + 16384;          // u32[2048]: logits in the blocks above
constexpr int kOffMMab = kOffMCab + 8192;             // u64[2048]: mass of the blocks above
constexpr int kOffMFlip = kOffMMab + 16384;           // u32[2048]: rescan flips (65,536 bits)
constexpr int kOffMKeys = kOffMFlip + 8192;           // uint4[slot][16]: (lo, hi) counts of word pairs
constexpr int kMLds = 155648;
constexpr uint32_t kSlotCap = (kMLds - kOffMKeys) / (16 * 16);
static_assert(kOffMKeys % 16 == 0 && kSlotCap >= 256, "merge map");

struct StreamArgs {
    const void* logits;
    int rows, vocabulary, parts, part_len, grid, xcd;
    int64_t stride;
    const vi_row_params* params;
    // penalty views: lane states, or the history prepass's bitmaps and lists
    const unsigned char* pstate;
    PenaltyLayout pl;
    const uint32_t* hb1;       // [rows][hwords] presence bitmaps (history route)
    const uint2* hlist;        // [rows][hcap] (token, count >= 2)
    const uint32_t* hhead;     // [rows][2]: repeat entries, flags
    int hwords, hcap;
    int record;
    int32_t* tokens;
    double* uniforms;
    vi_sample_stats* stats;
    // the parts' tables: header (occupied-group bitmap, highest valid key) and
    // the occupied groups' 32 words at their place
    uint32_t* ppub;            // [rows * parts][kPub]
    uint4* pwords;             // [rows * parts][kGroups][8]
};

// threadIdx.x behind an empty asm: address arithmetic on it stays in the loop
// that uses it instead of being hoisted and held across the persistent loop
__device__ __forceinline__ int opaque_tid() {
    int t = int(threadIdx.x);
    asm volatile("" : "+v"(t));
    return t;
}

// A workgroup barrier that orders LDS only (the stream's loads stay in flight).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// Exclusive prefix sum of v over the workgroup (total in *total), its barriers
// LDS-only: loads in flight stay in flight.
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
// s_waitcnt vmcnt(0): every vector memory access of the wave complete.
__device__ __forceinline__ void vm_drain() { __builtin_amdgcn_s_waitcnt(0x0f70); }
__device__ __forceinline__ void wave_lds_fence() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront", "local"); }

__device__ __forceinline__ void lds_add(uint32_t* p, uint32_t v) {
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// +1 / -1 at a 16-bit pattern's histogram half
__device__ __forceinline__ void hist_inc(uint32_t* H, uint32_t pat) {
    lds_add(&H[pat & 0x7fffu], (pat & 0x8000u) ? 0x10000u : 1u);
}
__device__ __forceinline__ void hist_dec(uint32_t* H, uint32_t pat) {
    lds_add(&H[pat & 0x7fffu], (pat & 0x8000u) ? 0xffff0000u : 0xffffffffu);
}

__device__ __forceinline__ uint32_t readlane_u(uint32_t v, int l) { return uint32_t(__builtin_amdgcn_readlane(int(v), l)); }
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
    return uint64_t(readlane_u(uint32_t(v), l)) | (uint64_t(readlane_u(uint32_t(v >> 32), l)) << 32);
}
// Inclusive prefix sums of u64 values over the wave (DPP, carries by hand).
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t x) {
    auto step = [](uint64_t v, auto dpp) {
        const uint64_t o = uint64_t(dpp(uint32_t(v))) | (uint64_t(dpp(uint32_t(v >> 32))) << 32);
        return v + o;
    };
    x = step(x, [](uint32_t u) { return dpp_u32<0x111, 0xf, true>(u); });
    x = step(x, [](uint32_t u) { return dpp_u32<0x112, 0xf, true>(u); });
    x = step(x, [](uint32_t u) { return dpp_u32<0x114, 0xf, true>(u); });
    x = step(x, [](uint32_t u) { return dpp_u32<0x118, 0xf, true>(u); });
    x = step(x, [](uint32_t u) { return dpp_u32<0x142, 0xa, false>(u); });
    x = step(x, [](uint32_t u) { return dpp_u32<0x143, 0xc, false>(u); });
    return x;
}

// ------------------------------------------------------------------ items
struct Item {
    int row, part, s0, n, nvec, rounds;
};
__device__ __forceinline__ Item part_geo(const StreamArgs& a, int row, int part) {
    Item it;
    it.row = row;
    it.part = part;
    it.s0 = part * a.part_len;
    it.n = min(a.part_len, a.vocabulary - it.s0);
    it.nvec = it.n >> 3;
    it.rounds = (it.nvec + kT - 1) / kT;
    return it;
}
// Parts of XCD x (the rows x, x + 8, ... when the launch is XCD-aware, else
// every row), in row-major order; the workgroups of the XCD take every nx-th.
__device__ __forceinline__ int xcd_rows(const StreamArgs& a, int x) { return a.xcd ? (a.rows - x + kXcds - 1) / kXcds : a.rows; }
__device__ __forceinline__ int xcd_wgs(const StreamArgs& a, int x) { return a.xcd ? (a.grid - x + kXcds - 1) / kXcds : a.grid; }
__device__ __forceinline__ Item item_at(const StreamArgs& a, int x, int q) {
    const int r = q / a.parts;
    return part_geo(a, a.xcd ? x + kXcds * r : r, q % a.parts);
}
__device__ __forceinline__ bool stream_row(const vi_row_params& p) { return !topk_route(p); }

struct PenView {
    const unsigned char* b1;
    const uint2* list;
    uint32_t nrep, flags;
    bool pen;
};
__device__ __forceinline__ PenView pen_view(const StreamArgs& a, int row, const vi_row_params& p) {
    PenView v{};
    if (a.pstate) {
        const unsigned char* st = a.pstate + size_t(row) * a.pl.lane_bytes;
        const PenaltyHeader* h = reinterpret_cast<const PenaltyHeader*>(st);
        v.b1 = st + a.pl.off_b1;
        v.list = reinterpret_cast<const uint2*>(st + a.pl.off_list);
        v.nrep = min(h->nrep, uint32_t(a.pl.slots));
        v.flags = h->flags & (VI_FLAG_BAD_HISTORY | VI_FLAG_ERROR);
        v.pen = penalties_active(p);
    } else if (a.hb1) {
        v.b1 = reinterpret_cast<const unsigned char*>(a.hb1 + size_t(row) * a.hwords);
        v.list = a.hlist + size_t(row) * a.hcap;
        v.nrep = a.hhead[2 * row];
        v.flags = a.hhead[2 * row + 1];
        v.pen = penalties_active(p);
    }
    return v;
}

// Penalized pattern of a 16-bit pattern seen `count` times; non-finite
// patterns stay as they are (they never reach the distribution).
template <int DT>
__device__ __forceinline__ uint32_t pen_pattern(uint32_t raw, uint32_t count, const vi_row_params& p, float inv_r,
                                                bool rep_fast) {
    if (!Elem<DT>::finite_bits(raw)) return raw;
    return penalize_fast<DT>(raw, count, p, inv_r, rep_fast) & 0xffffu;
}

// ------------------------------------------------------------------ weights
// exp(z(key) - z0): z in fp32 as the oracle forms it, the difference in fp64
// (exact), then 2^(d log2 e) as the hardware exp2 of the exponent rounded to
// fp32, corrected to first order by the rounding's remainder (relative error
// about one fp32 ulp).
template <int DT>
__device__ __forceinline__ double key_weight(uint32_t key, float inv_t, double z0) {
    const double d = double(key_z<DT>(key, inv_t)) - z0;
    const double a = d * 1.4426950408889634;
    const float ah = float(a);
    const float al = float(a - double(ah));
    const float e = __builtin_amdgcn_exp2f(ah);
    return ah < -125.0f ? 0.0 : double(e) * (1.0 + double(al) * 0.6931471805599453);
}
__device__ __forceinline__ uint64_t fixed_mass(uint32_t count, double w) {
    return uint64_t(llrint(double(count) * w * kFix));
}

// Keys of histogram word w: low half (sign 0) -> 0x8000 + w, high half (sign 1)
// -> 0x7fff - w.  Valid: a finite pattern whose z is finite (kmin..kmax).
template <int DT>
__device__ __forceinline__ bool key_valid(uint32_t key, uint32_t kmin, uint32_t kmax) {
    return key >= kmin && key <= kmax;
}

// ------------------------------------------------------------------ stream
constexpr int kMaxItems = 1024;          // parts one workgroup can take

struct StreamShared {
    int items[kMaxItems];                // the workgroup's parts (indices among its XCD's), in order
    uint32_t scan[kW + 1];
    // the part's occupied groups: byte q * 16 + wave, bit i -> group q * 128 + wave * 8 + i
    unsigned char occb[kGroups / 8];
};

// The presence bytes (one per vector) of a row from token s0: the lane
// state's or the history prepass's bitmap; without either, any readable byte
// per vector (the logits; the byte is then ignored).
__device__ __forceinline__ const unsigned char* presence_at(const StreamArgs& a, int row, int s0,
                                                            const unsigned char* vb) {
    if (a.pstate) return a.pstate + size_t(row) * a.pl.lane_bytes + a.pl.off_b1 + (s0 >> 3);
    if (a.hb1) return reinterpret_cast<const unsigned char*>(a.hb1 + size_t(row) * a.hwords) + (s0 >> 3);
    return vb;
}

// One part as the stream sees it: geometry, logits, presence bytes, repeat
// list, penalty parameters.
struct PartView {
    Item it;
    const unsigned char* vb;
    const unsigned char* pb;
    const uint2* list;
    uint32_t nrep;
    bool pen;
    float rep, pres, freq;
};

// PB: the call has presence bytes (lane states or the history prepass).
template <int DT, bool PB>
__global__ __launch_bounds__(kT) void stream_kernel(StreamArgs a) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[kLds];
    __shared__ StreamShared sh;
    uint32_t* H = reinterpret_cast<uint32_t*>(lds + kOffH);
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const int w = blockIdx.x;
    const int x = a.xcd ? w % kXcds : 0;
    const int wx = a.xcd ? w / kXcds : w;   // index among the XCD's workgroups
    const int nx = xcd_wgs(a, x), items = xcd_rows(a, x) * a.parts;

    // the histogram starts empty (every part leaves it so)
#pragma unroll
    for (int q = 0; q < kHW / 4 / kT; ++q)
        reinterpret_cast<uint4*>(H)[q * kT + tid] = make_uint4(0u, 0u, 0u, 0u);
    // the workgroup's parts: wx, wx + nx, ... of its XCD's (at most kMaxItems:
    // the launch checks), rows the kernel does not serve passed over
    int nitems;
    {
        const int ncand = wx < items ? (items - 1 - wx) / nx + 1 : 0;
        const int q = wx + tid * nx;
        const uint32_t ok = (tid < ncand && stream_row(a.params[item_at(a, x, q).row])) ? 1u : 0u;
        uint32_t tot;
        const uint32_t pos = block_scan_lds(ok, sh.scan, &tot);
        if (ok) sh.items[pos] = q;
        nitems = int(tot);
        lds_barrier();
    }
    if (nitems == 0) return;

    // A part's description.  The penalty parameters, the repeat list's length
    // and (a part ahead) its first entries come in through vector loads (the
    // address laundered into a VGPR): an outstanding scalar load would hold up
    // every LDS wait of the stream in between.
    auto view = [&](int k) -> PartView {
        PartView c;
        const int q = __builtin_amdgcn_readfirstlane(sh.items[k]);
        c.it = item_at(a, x, q);
        c.vb = static_cast<const unsigned char*>(a.logits) + 2 * (size_t(c.it.row) * size_t(a.stride) + size_t(c.it.s0));
        c.pb = presence_at(a, c.it.row, c.it.s0, c.vb);
        int z = 0;
        asm volatile("" : "+v"(z));
        const vi_row_params* pp = a.params + c.it.row + z;
        c.rep = pp->repetition_penalty;
        c.pres = pp->presence_penalty;
        c.freq = pp->frequency_penalty;
        c.pen = false;   // (settle)
        const uint32_t* nr;
        if (a.pstate) {
            const unsigned char* st = a.pstate + size_t(c.it.row) * a.pl.lane_bytes;
            c.list = reinterpret_cast<const uint2*>(st + a.pl.off_list);
            nr = &reinterpret_cast<const PenaltyHeader*>(st)->nrep;
        } else if (a.hb1) {
            c.list = a.hlist + size_t(c.it.row) * a.hcap;
            nr = a.hhead + 2 * c.it.row;
        } else {
            c.list = nullptr;
            nr = reinterpret_cast<const uint32_t*>(a.params);
        }
        c.nrep = nr[z];
        return c;
    };
    // the loaded fields made uniform (after their loads have landed)
    auto settle = [&](PartView& c) {
        auto rf = [](float f) { return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, f))); };
        c.rep = rf(c.rep);
        c.pres = rf(c.pres);
        c.freq = rf(c.freq);
        c.pen = PB && (c.rep != 1.0f || c.pres != 0.0f || c.freq != 0.0f);
        c.nrep = uint32_t(__builtin_amdgcn_readfirstlane(int(c.nrep)));
        if (a.pstate) c.nrep = min(c.nrep, uint32_t(a.pl.slots));
    };
    // The lane's repeat-list entries of a part (kRepPF of them), requested a
    // part ahead, whatever the list's length (read within the list's
    // capacity; entries past the length are dropped when used).
    const uint32_t list_cap = a.pstate ? uint32_t(a.pl.slots) : uint32_t(max(a.hcap, 1));
    auto load_re = [&](const PartView& c, uint2* e) {
#pragma unroll
        for (int j = 0; j < kRepPF; ++j) {
            e[j] = make_uint2(0u, 0u);
            if (PB) e[j] = c.list[min(uint32_t(j * kT + tid), list_cap - 1u)];
        }
    };

    PartView cur = view(0);
    bool has_next = nitems > 1;
    PartView nxt = has_next ? view(1) : cur;
    uint2 re[kRepPF];   // the current part's entries (those of the next once its corrections are made)
    load_re(cur, re);

    // Rounds in flight: a part's rounds are padded to whole turns of the ring
    // (the padding rounds count nothing), so round rho of every part sits in
    // slot rho % kDepth.  The round kDepth ahead is requested once the current
    // one is used: the current part's, the next part's, or (past the last
    // part) the last vector again, never used.  Every round issues exactly one
    // vector load (and one presence load), straight-line, so the waits count
    // on the loads' order.
    uint4 rv[kDepth];
    uint32_t rb[kDepth] = {};
    auto padded = [](int r) { return (r + kDepth - 1) & ~(kDepth - 1); };
    auto issue = [&](uint4& dv, uint32_t& db, int rel) {   // rel: rounds after the current part's first
        const int Rp = padded(cur.it.rounds);
        const bool in_nxt = rel >= Rp && has_next;
        const unsigned char* vb = in_nxt ? nxt.vb : cur.vb;
        const unsigned char* pb = in_nxt ? nxt.pb : cur.pb;
        const int nv = in_nxt ? nxt.it.nvec : cur.it.nvec;
        const int rr = in_nxt ? rel - Rp : rel;
        const int v = min(rr * kT + opaque_tid(), nv - 1);
        dv = load16(vb + size_t(v) * 16);
        // the dword holding the vector's presence byte (a 32-bit load result
        // stays in its register across the loop; a byte would be re-extended)
        if (PB) db = *reinterpret_cast<const uint32_t*>(pb + (v & ~3));
    };
#pragma unroll
    for (int s = 0; s < kDepth; ++s) issue(rv[s], rb[s], s);
    settle(cur);

    for (int k = 0;;) {
        vi_row_params p{};   // the fields the penalties read
        p.repetition_penalty = cur.rep;
        p.presence_penalty = cur.pres;
        p.frequency_penalty = cur.freq;
        const float inv_r = rep_inverse(p);
        const bool rep_fast = rep_fast_ok(p);
        const bool pen = cur.pen;
        const Item it = cur.it;
        const uint16_t* row16 = reinterpret_cast<const uint16_t*>(static_cast<const unsigned char*>(a.logits) +
                                                                  2 * size_t(it.row) * size_t(a.stride));
        auto in_part = [&](uint2 e) { return e.y >= 2u && int(e.x) >= it.s0 && int(e.x) < it.s0 + it.n; };
        // one count of a repeated token from its count-1 pattern to its count-c one
        auto correct = [&](uint2 e, uint32_t raw) {
            const uint32_t p1 = pen_pattern<DT>(raw, 1u, p, inv_r, rep_fast);
            const uint32_t pc = pen_pattern<DT>(raw, e.y, p, inv_r, rep_fast);
            if (p1 != pc) { hist_dec(H, p1); hist_inc(H, pc); }
        };
        uint32_t rraw[kRepPF] = {};

        // ---- the stream.  The repeat entries' logits are gathered at the
        // start of the last turn but one and their corrections made at the
        // start of the last turn (counts are added and taken in any order: the
        // 32-bit word holds their sum).
        const int Rp = padded(it.rounds);
        const int gather_turn = max(0, Rp - 2 * kDepth), corr_turn = Rp - kDepth;
        uint4* stage = reinterpret_cast<uint4*>(lds + kOffStage) + wave * kWave;
        const uint16_t* stage16 = reinterpret_cast<const uint16_t*>(stage);
        unsigned char* list = lds + kOffList + wave * 512;
        for (int gb = 0; gb < Rp; gb += kDepth) {
            if (pen && gb == gather_turn) {
#pragma unroll
                for (int j = 0; j < kRepPF; ++j) {
                    if (uint32_t(j * kT + tid) >= cur.nrep) re[j].y = 0u;
                    rraw[j] = in_part(re[j]) ? uint32_t(row16[re[j].x]) : 0u;
                }
            }
            if (pen && gb == corr_turn) {
#pragma unroll
                for (int j = 0; j < kRepPF; ++j)
                    if (in_part(re[j])) correct(re[j], rraw[j]);
            }
            if (gb == corr_turn && has_next) load_re(nxt, re);   // (in place: no copy waits for it)
#pragma unroll
            for (int s = 0; s < kDepth; ++s) {
                const int rho = gb + s;
                const uint4 v = rv[s];
                const bool valid = rho * kT + tid < it.nvec;   // (none on a padding round)
                const uint32_t b = (PB && valid) ? (rb[s] >> (8 * (tid & 3))) & 0xffu : 0u;
                if (valid) {
                    hist_inc(H, v.x & 0xffffu); hist_inc(H, v.x >> 16);
                    hist_inc(H, v.y & 0xffffu); hist_inc(H, v.y >> 16);
                    hist_inc(H, v.z & 0xffffu); hist_inc(H, v.z >> 16);
                    hist_inc(H, v.w & 0xffffu); hist_inc(H, v.w >> 16);
                }
                if (pen) {   // (uniform) the history tokens of the wave's 512 tokens
                    stage[lane] = v;
                    const uint32_t n = uint32_t(__builtin_popcount(b));
                    const uint32_t incl = wave_incl_scan_u32(n);
                    const uint32_t N = readlane_u(incl, kWave - 1), NA = readlane_u(incl, 31);
                    if (N) {
                        uint32_t pos = incl - n;
                        const uint32_t base = uint32_t(lane) * 8u;
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            if ((b >> j) & 1u) {
                                list[pos] = uint8_t(base + uint32_t(j));
                                ++pos;
                            }
                        }
                        wave_lds_fence();
                        for (uint32_t q0 = 0; q0 < N; q0 += kWave) {
                            const uint32_t q = q0 + uint32_t(lane);
                            if (q < N) {
                                const uint32_t off = uint32_t(list[q]) + (q >= NA ? 256u : 0u);
                                const uint32_t raw = stage16[off];
                                const uint32_t pb = pen_pattern<DT>(raw, 1u, p, inv_r, rep_fast);
                                if (pb != raw) { hist_dec(H, raw); hist_inc(H, pb); }
                            }
                        }
                        wave_lds_fence();
                    }
                }
                issue(rv[s], rb[s], rho + kDepth);
            }
        }

        lds_barrier();
        if (pen && cur.nrep > uint32_t(kRepPF * kT)) {   // (long repeat lists: the rest of the entries)
            for (uint32_t i = uint32_t(kRepPF * kT + tid); i < cur.nrep; i += kT) {
                const uint2 e = cur.list[i];
                if (in_part(e)) correct(e, row16[e.x]);
            }
            lds_barrier();
        }

        // ---- publication: the non-empty groups at their place in the part's
        // table and the occupancy bitmap; the histogram cleared.  Eight lanes
        // hold a group (lane 8i + j: its words 4j .. 4j + 3), so the LDS reads
        // are conflict-free and the stores coalesce.  Plain stores: the merge
        // launch reads them.
        {
            const size_t pi = size_t(it.row) * a.parts + it.part;
            uint4* dst = a.pwords + pi * (kGroups * kGW / 4);
            const int t = opaque_tid();
            uint4* H4 = reinterpret_cast<uint4*>(H);
#pragma unroll
            for (int q = 0; q < kHW / 4 / kT; ++q) {
                const int c = q * kT + t;            // 16-byte chunk c: words 4c .. 4c + 3 of group c / 8
                const uint4 d = H4[c];
                H4[c] = make_uint4(0u, 0u, 0u, 0u);
                const uint64_t bm = ballot((d.x | d.y | d.z | d.w) != 0u);
                // bit 8i of sm: group i of the wave's eight is occupied
                uint64_t sm = bm | (bm >> 4);
                sm |= sm >> 2;
                sm |= sm >> 1;
                sm &= 0x0101010101010101ull;
                const uint64_t lanes = (sm << 8) - sm;   // the occupied groups' lanes
                const uint32_t half = lane < 32 ? uint32_t(lanes) : uint32_t(lanes >> 32);
                if ((half >> (lane & 31)) & 1u) dst[c] = d;
                if (lane == 0) {
                    const uint32_t lo = uint32_t(sm), hi = uint32_t(sm >> 32);
                    sh.occb[q * kW + wave] = uint8_t((((lo * 0x00204081u) >> 21) & 0xfu) | ((((hi * 0x00204081u) >> 21) & 0xfu) << 4));
                }
            }
            lds_barrier();
            if (tid < 32) a.ppub[pi * kPub + tid] = reinterpret_cast<const uint32_t*>(sh.occb)[tid];
            // Stores and loads share one counter and may complete out of order:
            // with a store outstanding every wait on a load would have to drain
            // the counter.  Drain it once here instead.
            vm_drain();
        }

        // ---- the next part (its first turn already in flight)
        if (++k >= nitems) break;
        cur = nxt;
        settle(cur);
        has_next = k + 1 < nitems;
        if (has_next) nxt = view(k + 1);
    }
}

// ------------------------------------------------------------------ merge
struct MergeShared {
    uint32_t scan[kW + 1];
    uint32_t wtot[8][kW];
    uint64_t wmass[kW];
    uint32_t nslots, total_cnt, z0key, owner, orank, flags, kmin, kmax;
    uint64_t total_mass;
    uint32_t draw_key, draw_rank;
    uint32_t n_support, ok, lo1, hi1, nflip;
    int32_t token;
    double s_n, u;
};

// Key k's histogram location: group, word inside the group, half (0: low).
struct KeyLoc {
    uint32_t group, word, hi;
};
__device__ __forceinline__ KeyLoc key_loc(uint32_t k) {
    const uint32_t wd = k >= 0x8000u ? k - 0x8000u : 0x7fffu - k;
    return KeyLoc{wd >> 5, wd & 31u, k >= 0x8000u ? 0u : 1u};
}
// Order key of each 16-bit half of a word, -0 kept apart just below +0
// (0x7fff): the key is pattern ^ 0x8000 for a clear sign bit, ~pattern for a
// set one.
__device__ __forceinline__ uint32_t halves_key(uint32_t d) {
    typedef short s2 __attribute__((ext_vector_type(2)));
    const s2 sg = __builtin_bit_cast(s2, d) >> 15;   // 0 or -1 per half
    return d ^ (__builtin_bit_cast(uint32_t, sg) | 0x80008000u);
}
// Per 16-bit half: a - b (wrapping), max(a - b, 0), and min(a, 1).  The last
// two are written as the packed instructions (the compiler otherwise turns the
// pair into a compare and a select per half).
__device__ __forceinline__ uint32_t pk_sub_u16(uint32_t a, uint32_t b) {
    typedef unsigned short u2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u2, a) - __builtin_bit_cast(u2, b));
}
__device__ __forceinline__ uint32_t pk_sub_sat_u16(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_pk_sub_u16 %0, %1, %2 clamp" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ uint32_t pk_nonzero_u16(uint32_t a) {
    uint32_t r;
    asm("v_pk_min_u16 %0, %1, %2" : "=v"(r) : "v"(a), "s"(0x00010001u));
    return r;
}

template <int DT>
__global__ __launch_bounds__(kT) void merge_kernel(StreamArgs a) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[kMLds];
    __shared__ MergeShared sh;
    const int row = blockIdx.x;
    const vi_row_params p = a.params[row];
    if (!stream_row(p)) return;
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const int P = a.parts, V = a.vocabulary;
    uint32_t* pbits = reinterpret_cast<uint32_t*>(lds + kOffMBits);
    uint32_t* occ = reinterpret_cast<uint32_t*>(lds + kOffMOcc);
    uint16_t* slot_of = reinterpret_cast<uint16_t*>(lds + kOffMSlot);
    uint16_t* group_of = reinterpret_cast<uint16_t*>(lds + kOffMGroupOf);
    uint32_t* bcnt = reinterpret_cast<uint32_t*>(lds + kOffMBcnt);
    uint64_t* bmass = reinterpret_cast<uint64_t*>(lds + kOffMBmass);
    uint32_t* cab = reinterpret_cast<uint32_t*>(lds + kOffMCab);
    uint64_t* mab = reinterpret_cast<uint64_t*>(lds + kOffMMab);
    uint32_t* flip = reinterpret_cast<uint32_t*>(lds + kOffMFlip);
    uint4* keys = reinterpret_cast<uint4*>(lds + kOffMKeys);
    const size_t pi0 = size_t(row) * P;
    const PenView pv = pen_view(a, row, p);
    const float inv_t = 1.0f / p.temperature;

    // ---- 0. the parts' occupancy bitmaps; the valid key range
    for (int i = tid; i < P * 32; i += kT) pbits[i] = a.ppub[(pi0 + i / 32) * kPub + i % 32];
    // The first repeat entries (two per thread), requested now (reads within
    // the list whatever it holds); their logits are gathered once the owner
    // part is known, for the entries inside it only.
    const uint16_t* row16 = reinterpret_cast<const uint16_t*>(static_cast<const unsigned char*>(a.logits) +
                                                              2 * size_t(row) * size_t(a.stride));
    uint2 rep[2];
    {
        const uint2* rl = pv.pen ? pv.list : reinterpret_cast<const uint2*>(a.params);
        const uint32_t rn = pv.pen ? max(pv.nrep, 1u) : 1u;
#pragma unroll
        for (int j = 0; j < 2; ++j) rep[j] = rl[min(uint32_t(j * kT + tid), rn - 1u)];
    }
    if (wave == 1) {
        const uint32_t km = valid_key_range<DT>(p.temperature);
        if (lane == 0) { sh.kmin = km & 0xffffu; sh.kmax = km >> 16; }
    }
    for (int i = tid; i < 2048; i += kT) { bcnt[i] = 0u; bmass[i] = 0ull; }
    if (tid == 0) { sh.flags = pv.flags; sh.token = -1; sh.ok = 1u; sh.z0key = 0u; }
    lds_barrier();
    if (tid < 32) {
        uint32_t o = 0u;
        for (int pp = 0; pp < P; ++pp) o |= pbits[pp * 32 + tid];
        occ[tid] = o;
    }
    lds_barrier();
    // a slot per occupied group
    {
        const uint32_t o = (occ[tid >> 5] >> (tid & 31)) & 1u;
        uint32_t n = 0u;
        const uint32_t e = block_scan_lds(o, sh.scan, &n);
        if (o) { slot_of[tid] = uint16_t(e); group_of[e] = uint16_t(tid); }
        if (tid == 0) sh.nslots = n;
    }
    lds_barrier();
    const uint32_t nslots = sh.nslots;
    const bool store_keys = nslots <= kSlotCap;
    const uint32_t kmin = sh.kmin, kmax = sh.kmax;
    const bool fail = (sh.flags & VI_FLAG_ERROR) != 0u || !(p.temperature <= kMaxTemperature);

    // Counts of words 2q, 2q + 1 of group g summed over the parts: (lo0, hi0,
    // lo1, hi1); the parts' loads four at a time.
    auto sum_pair = [&](uint32_t g, uint32_t q) -> uint4 {
        uint4 c = make_uint4(0u, 0u, 0u, 0u);
        const uint64_t* src = reinterpret_cast<const uint64_t*>(a.pwords);
        for (int p0 = 0; p0 < P; p0 += 4) {
            uint64_t w2[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int pp = p0 + k;
                w2[k] = 0ull;
                if (pp < P && ((pbits[pp * 32 + (g >> 5)] >> (g & 31u)) & 1u))
                    w2[k] = src[((pi0 + pp) * kGroups + g) * 16 + q];
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t w0 = uint32_t(w2[k]), w1 = uint32_t(w2[k] >> 32);
                c.x += w0 & 0xffffu; c.y += w0 >> 16; c.z += w1 & 0xffffu; c.w += w1 >> 16;
            }
        }
        if (g == 0u && q == 0u) { c.x += c.y; c.y = 0u; }   // -0 is +0
        return c;
    };
    // ---- 1. per-key counts summed over the parts (a task: two words of a
    // group; two tasks per thread, their loads issued together) and the
    // highest valid key present, z0's.  Past kSlotCap occupied groups the
    // counts are not kept: a second pass adds them to the block sums.
    const uint32_t ntask = nslots * 16u;
    auto task_keys = [&](uint32_t t) { return uint32_t(group_of[t >> 4]) * kGW + 2u * (t & 15u); };
    auto top_of = [&](uint32_t t, uint4 c) -> uint32_t {
        const uint32_t w0 = task_keys(t);
        uint32_t m = 0u;
        auto consider = [&](uint32_t k, uint32_t n) {
            if (n && key_valid<DT>(k, kmin, kmax)) m = max(m, k);
        };
        consider(0x8000u + w0, c.x); consider(0x7fffu - w0, c.y); consider(0x8001u + w0, c.z); consider(0x7ffeu - w0, c.w);
        return m;
    };
    {
        uint32_t top = 0u;
        for (uint32_t t0 = 0; t0 < ntask; t0 += 2 * kT) {
            const uint32_t ta = t0 + uint32_t(tid), tb = ta + kT;
            const bool va = ta < ntask, vb = tb < ntask;
            const uint4 ca = va ? sum_pair(group_of[ta >> 4], ta & 15u) : make_uint4(0u, 0u, 0u, 0u);
            const uint4 cb = vb ? sum_pair(group_of[tb >> 4], tb & 15u) : make_uint4(0u, 0u, 0u, 0u);
            if (store_keys) {
                if (va) keys[ta] = ca;
                if (vb) keys[tb] = cb;
            }
            if (va) top = max(top, top_of(ta, ca));
            if (vb) top = max(top, top_of(tb, cb));
        }
#pragma unroll
        for (int o = 32; o; o >>= 1) top = max(top, uint32_t(__shfl_xor(int(top), o, kWave)));
        if (lane == 0 && top) atomicMax(&sh.z0key, top);
    }
    lds_barrier();
    const uint32_t z0key = sh.z0key;
    const double z0 = double(key_z<DT>(z0key, inv_t));
    if (!store_keys) {   // (block sums straight from the counts)
        auto add = [&](uint32_t k, uint32_t c) {
            if (!c) return;
            if (!key_valid<DT>(k, kmin, kmax)) { atomicOr(&sh.flags, uint32_t(VI_FLAG_NONFINITE)); return; }
            atomicAdd(&bcnt[k >> 5], c);
            atomicAdd(reinterpret_cast<unsigned long long*>(&bmass[k >> 5]),
                      (unsigned long long)fixed_mass(c, key_weight<DT>(k, inv_t, z0)));
        };
        auto add4 = [&](uint32_t t, uint4 c) {
            const uint32_t w0 = task_keys(t);
            add(0x8000u + w0, c.x); add(0x7fffu - w0, c.y); add(0x8001u + w0, c.z); add(0x7ffeu - w0, c.w);
        };
        for (uint32_t t0 = 0; t0 < ntask; t0 += 2 * kT) {
            const uint32_t ta = t0 + uint32_t(tid), tb = ta + kT;
            const bool va = ta < ntask, vb = tb < ntask;
            const uint4 ca = va ? sum_pair(group_of[ta >> 4], ta & 15u) : make_uint4(0u, 0u, 0u, 0u);
            const uint4 cb = vb ? sum_pair(group_of[tb >> 4], tb & 15u) : make_uint4(0u, 0u, 0u, 0u);
            if (va) add4(ta, ca);
            if (vb) add4(tb, cb);
        }
        lds_barrier();
    }
    // ---- 2. block sums: four threads per 32-key block, eight keys each
    if (store_keys) {
        const uint32_t nunits = nslots * 8u;
        for (uint32_t u0 = 0; u0 < nunits; u0 += kT) {
            const uint32_t u = u0 + uint32_t(tid);
            uint32_t c8 = 0u, blk = 0u;
            uint64_t m8 = 0ull;
            bool bad = false;
            if (u < nunits) {
                const uint32_t s = u >> 3, neg = (u >> 2) & 1u, qq = u & 3u, g = group_of[s];
#pragma unroll
                for (int i = 0; i < 8; i += 2) {
                    const uint4 c2 = keys[s * 16u + 4u * qq + uint32_t(i) / 2u];
                    const uint32_t wd = g * kGW + 8u * qq + uint32_t(i);
                    const uint32_t ca = neg ? c2.y : c2.x, cb = neg ? c2.w : c2.z;
                    const uint32_t ka = neg ? 0x7fffu - wd : 0x8000u + wd, kb = neg ? 0x7ffeu - wd : 0x8001u + wd;
                    if (ca) {
                        if (key_valid<DT>(ka, kmin, kmax)) { c8 += ca; m8 += fixed_mass(ca, key_weight<DT>(ka, inv_t, z0)); }
                        else bad = true;
                    }
                    if (cb) {
                        if (key_valid<DT>(kb, kmin, kmax)) { c8 += cb; m8 += fixed_mass(cb, key_weight<DT>(kb, inv_t, z0)); }
                        else bad = true;
                    }
                }
                blk = neg ? 1023u - g : 1024u + g;
            }
            // the four quarters of a block are lanes 4i .. 4i + 3
            c8 += dpp_u32<0xb1, 0xf, false>(c8);   // quad_perm [1,0,3,2]
            c8 += dpp_u32<0x4e, 0xf, false>(c8);   // quad_perm [2,3,0,1]
            {
                const uint64_t o1 = uint64_t(dpp_u32<0xb1, 0xf, false>(uint32_t(m8))) |
                                    (uint64_t(dpp_u32<0xb1, 0xf, false>(uint32_t(m8 >> 32))) << 32);
                m8 += o1;
                const uint64_t o2 = uint64_t(dpp_u32<0x4e, 0xf, false>(uint32_t(m8))) |
                                    (uint64_t(dpp_u32<0x4e, 0xf, false>(uint32_t(m8 >> 32))) << 32);
                m8 += o2;
            }
            if (u < nunits && (u & 3u) == 0u) { bcnt[blk] = c8; bmass[blk] = m8; }
            if (ballot(bad) && lane == 0) atomicOr(&sh.flags, uint32_t(VI_FLAG_NONFINITE));
        }
        lds_barrier();
    }
    // ---- 3. descending prefix sums over the 2048 blocks (thread t: blocks
    // 2047 - 2t and 2046 - 2t)
    {
        const int b0 = 2047 - 2 * tid, b1 = b0 - 1;
        const uint32_t c0 = bcnt[b0], c1 = bcnt[b1];
        const uint64_t m0 = bmass[b0], m1 = bmass[b1];
        const uint32_t ci = wave_incl_scan_u32(c0 + c1);
        const uint64_t mi = wave_incl_scan_u64(m0 + m1);
        if (lane == kWave - 1) { sh.scan[wave] = ci; sh.wmass[wave] = mi; }
        lds_barrier();
        uint32_t cb = 0u;
        uint64_t mb = 0ull;
        {   // the earlier waves' totals, one per lane, summed across the wave (exact integers)
            const bool e = lane < wave;
            cb = readlane_u(wave_incl_scan_u32(e ? sh.scan[lane] : 0u), kWave - 1);
            mb = readlane_u64(wave_incl_scan_u64(e ? sh.wmass[lane] : 0ull), kWave - 1);
        }
        if (tid == kT - 1) { sh.total_cnt = cb + ci; sh.total_mass = mb + mi; }
        const uint32_t ce = cb + ci - (c0 + c1);
        const uint64_t me = mb + mi - (m0 + m1);
        cab[b0] = ce; mab[b0] = me;
        cab[b1] = ce + c0; mab[b1] = me + m0;
    }
    lds_barrier();
    const uint32_t N = sh.total_cnt;
    const uint64_t Mtot = sh.total_mass;
    const uint32_t out_flags = sh.flags & (VI_FLAG_NONFINITE | VI_FLAG_BAD_HISTORY);
    if (fail || N == 0u) {
        if (tid == 0) {
            a.tokens[row] = fail ? -1 : V;
            if (a.uniforms) a.uniforms[row] = 0.0;
            if (a.stats) {
                vi_sample_stats st{};
                st.flags = out_flags | (fail ? VI_FLAG_ERROR : VI_FLAG_EMPTY);
                a.stats[row] = st;
            }
        }
        return;
    }

    // Count of key 32 b + 31 - lane (lanes < 32: the block's keys in descending
    // order; 0 for lanes >= 32 and invalid keys).  Wave-uniform b.
    auto block_key_count = [&](uint32_t b) -> uint32_t {
        const uint32_t k = 32u * b + 31u - uint32_t(lane & 31);
        if (lane >= 32 || !key_valid<DT>(k, kmin, kmax)) return 0u;
        const KeyLoc kl = key_loc(k);
        if (!((occ[kl.group >> 5] >> (kl.group & 31u)) & 1u)) return 0u;
        const uint4 c = store_keys ? keys[uint32_t(slot_of[kl.group]) * 16u + (kl.word >> 1)]
                                   : sum_pair(kl.group, kl.word >> 1);
        const uint32_t lo = (kl.word & 1u) ? c.z : c.x, hi = (kl.word & 1u) ? c.w : c.y;
        return kl.hi ? hi : lo;
    };
    // Wave 0: the first block (descending) at which the cumulative count
    // (mode 0: >= target) or fixed-point mass (mode 1: >= target, mode 2: >
    // target) is reached, searched over the blocks' running sums; -1 if none.
    auto block_search = [&](int mode, uint64_t target) -> int {
        if (mode == 1 && target == 0u) return -1;
        const int i = wave_search(0, 2048, [&](int i) {
            const int b = 2047 - i;
            if (mode == 0) return uint64_t(cab[b]) + bcnt[b] >= target;
            const uint64_t inc = mab[b] + bmass[b];
            return mode == 1 ? inc >= target : inc > target;
        });
        return i < 2048 ? 2047 - i : -1;
    };
    struct Fine {
        bool found;
        uint32_t key, take;   // position: the first `take` logits of `key` in id order
    };
    // Wave 0, inside block b: the first key at which the cumulative count
    // (mode 0: >= target) or mass (1: >= target, 2: > target) is reached, with
    // the counts limited to the position (lim_key, lim_take); target relative
    // to the block's start.
    auto fine_find = [&](uint32_t b, int mode, uint64_t target, uint32_t lim_key, uint32_t lim_take) -> Fine {
        const uint32_t k = 32u * b + 31u - uint32_t(lane & 31);
        uint32_t c = block_key_count(b);
        if (k < lim_key) c = 0u;
        else if (k == lim_key) c = min(c, lim_take);
        const uint64_t m = c ? fixed_mass(c, key_weight<DT>(k, inv_t, z0)) : 0ull;
        const uint64_t mi = wave_incl_scan_u64(m);
        const uint32_t ci = wave_incl_scan_u32(c);
        const uint64_t me = mi - m;
        const uint32_t cexcl = ci - c;
        bool hit = false;
        uint32_t take = 0u;
        if (c) {
            if (mode == 0) {
                hit = uint64_t(ci) >= target;
                if (hit) take = uint32_t(target - cexcl);
            } else {
                const double unit = double(m) / double(c);   // one logit's mass
                if (mode == 1) {
                    hit = mi >= target;
                    if (hit) take = uint32_t(ceil(double(target - me) / unit));
                } else {
                    hit = mi > target;
                    if (hit) take = uint32_t(floor(double(target - me) / unit)) + 1u;
                }
            }
            take = min(max(take, 1u), c);
        }
        const uint64_t hm = ballot(hit);
        Fine f{};
        if (hm) {
            const int L = __builtin_ctzll(hm);
            f.found = true;
            f.key = 32u * b + 31u - uint32_t(L);
            f.take = readlane_u(take, L);
        }
        return f;
    };
    // Wave 0: mass and count of the support through position (key, take).
    auto mass_through = [&](uint32_t key, uint32_t take, uint64_t* mass, uint32_t* cnt) {
        const uint32_t b = key >> 5;
        const uint32_t k = 32u * b + 31u - uint32_t(lane & 31);
        uint32_t c = block_key_count(b);
        if (k < key) c = 0u;
        else if (k == key) c = min(c, take);
        const uint64_t m = c ? fixed_mass(c, key_weight<DT>(k, inv_t, z0)) : 0ull;
        *mass = mab[b] + readlane_u64(wave_incl_scan_u64(m), kWave - 1);
        *cnt = cab[b] + readlane_u(wave_incl_scan_u32(c), kWave - 1);
    };

    // ---- 4. the decisions, in wave 0: the top-k cap, the min-p cut, the top-p
    // cut, the support's end (the earliest of them) and the draw
    if (wave == 0) {
        const bool has_cap = p.top_k > 0 && uint32_t(p.top_k) < N;
        uint32_t cap_key = 0u, cap_take = kTakeAll;
        double s_cap = double(Mtot);
        if (has_cap) {
            const int b = block_search(0, uint64_t(p.top_k));
            const Fine f = fine_find(uint32_t(b), 0, uint64_t(p.top_k) - cab[b], 0u, kTakeAll);
            uint64_t m;
            uint32_t c;
            mass_through(f.key, f.take, &m, &c);
            cap_key = f.key;
            cap_take = f.take;
            s_cap = double(m);
        }
        // min-p: the lowest key whose weight reaches min_p
        uint32_t minp_key = 0u;
        if (p.min_p > 0.0f) {
            const double mp = double(p.min_p);
            minp_key = uint32_t(wave_search(int(kmin), int(z0key) + 1, [&](int k) {
                return key_weight<DT>(uint32_t(k), inv_t, z0) >= mp;
            }));
        }
        // top-p: the first position whose cumulative mass reaches top_p of the cap's
        bool has_topp = false;
        uint32_t topp_key = 0u, topp_take = kTakeAll;
        if (p.top_p < 1.0f) {
            const uint64_t target = uint64_t(llrint(double(p.top_p) * s_cap));
            const int b = block_search(1, target);
            const int lowest = has_cap ? int(cap_key >> 5) : 0;
            if (b >= lowest) {
                const bool in_cap = has_cap && uint32_t(b) == (cap_key >> 5);
                const Fine f = fine_find(uint32_t(b), 1, target - mab[b], in_cap ? cap_key : 0u,
                                         in_cap ? cap_take : kTakeAll);
                has_topp = f.found;
                topp_key = f.key;
                topp_take = f.take;
            }
        }
        // the support's end, its mass, the uniform and the draw's target
        bool all = true;
        uint32_t ek = 0u, et = kTakeAll;
        auto consider = [&](uint32_t k, uint32_t t) {
            if (all || k > ek || (k == ek && t < et)) { ek = k; et = t; all = false; }
        };
        if (has_cap) consider(cap_key, cap_take);
        if (p.min_p > 0.0f) consider(minp_key, kTakeAll);
        if (has_topp) consider(topp_key, topp_take);
        if (!all && ek > z0key) { ek = z0key; et = 1u; }   // no logit passes min-p: the best one
        uint64_t sm = Mtot;
        uint32_t sc = N;
        if (!all) mass_through(ek, et, &sm, &sc);
        const double u = philox_uniform(p.seed, p.lane, p.position, 0u);
        const double target_d = u * double(sm);
        // the draw: the first support logit whose inclusive mass exceeds u * S_n
        const uint64_t t = uint64_t(target_d);
        int b = block_search(2, t);
        const int lowest = all ? 0 : int(ek >> 5);
        if (b < lowest) b = -1;
        uint32_t dk = 0u, dr = 0u;
        bool ok = false;
        if (b >= 0) {
            const bool in_end = !all && uint32_t(b) == (ek >> 5);
            const Fine f = fine_find(uint32_t(b), 2, t - mab[b], in_end ? ek : 0u, in_end ? et : kTakeAll);
            if (f.found) { dk = f.key; dr = f.take - 1u; ok = true; }
        }
        if (!ok) {   // rounding past the support's last logit: that logit
            for (int bb = lowest; bb < 2048 && !ok; ++bb) {
                if (!bcnt[bb]) continue;
                const uint32_t k = 32u * uint32_t(bb) + 31u - uint32_t(lane & 31);
                uint32_t c = block_key_count(uint32_t(bb));
                if (!all) {
                    if (k < ek) c = 0u;
                    else if (k == ek) c = min(c, et);
                }
                const uint64_t hm = ballot(c > 0u);
                if (hm) {
                    const int L = 63 - __builtin_clzll(hm);
                    dk = 32u * uint32_t(bb) + 31u - uint32_t(L);
                    dr = readlane_u(c, L) - 1u;
                    ok = true;
                }
            }
        }
        if (lane == 0) {
            sh.s_n = double(sm);
            sh.n_support = sc;
            sh.u = u;
            sh.draw_key = dk;
            sh.draw_rank = dr;
            sh.ok = ok ? 1u : 0u;
        }
    }
    lds_barrier();

    // ---- 5. the part holding the drawn rank (parts in id order) and, for the
    // rescan, the drawn key's preimage under the count-1 penalty: a history
    // token counted once has the drawn key exactly when its raw key lies in
    // [lo1, hi1) (the penalty is monotone in the logit)
    const float inv_r = rep_inverse(p);
    const bool rep_fast = rep_fast_ok(p);
    if (wave == 0 && sh.ok) {
        const uint32_t dk = sh.draw_key;
        const KeyLoc kl = key_loc(dk);
        uint32_t c = 0u;
        if (lane < P && ((pbits[lane * 32 + (kl.group >> 5)] >> (kl.group & 31u)) & 1u)) {
            const uint64_t* src = reinterpret_cast<const uint64_t*>(a.pwords) + ((pi0 + lane) * kGroups + kl.group) * 16;
            const uint64_t w2 = src[kl.word >> 1];
            const uint32_t wd = (kl.word & 1u) ? uint32_t(w2 >> 32) : uint32_t(w2);
            c = kl.hi ? (wd >> 16) : (wd & 0xffffu);
            if (dk == 0x8000u) c = (wd & 0xffffu) + (wd >> 16);   // +0 and -0
        }
        const uint32_t incl = wave_incl_scan_u32(c);
        const uint64_t hm = ballot(lane < P && incl > sh.draw_rank);
        if (hm) {
            const int L = __builtin_ctzll(hm);
            if (lane == L) { sh.owner = uint32_t(L); sh.orank = sh.draw_rank - (incl - c); }
        } else if (lane == 0) {
            sh.ok = 0u;
        }
    }
    if (wave == 1 && pv.pen && sh.ok) {
        constexpr int kNegMin = DT == VI_BF16 ? 0x0080 : 0x0400;
        constexpr int kPosMax = DT == VI_BF16 ? 0xff7f : 0xfbff;
        const uint32_t dk = sh.draw_key;
        auto fk = [&](int k) { return key16(pen_pattern<DT>(unkey16(uint32_t(k)), 1u, p, inv_r, rep_fast)); };
        const uint32_t lo = uint32_t(wave_search(kNegMin, kPosMax + 1, [&](int k) { return fk(k) >= dk; }));
        const uint32_t hi = uint32_t(wave_search(kNegMin, kPosMax + 1, [&](int k) { return fk(k) > dk; }));
        if (lane == 0) { sh.lo1 = lo; sh.hi1 = hi; }
    }
    for (int i = tid; i < 2048; i += kT) flip[i] = 0u;
    if (tid == 0) sh.nflip = 0u;
    // presence masks by byte for the rescan, in the decisions' running-sum
    // table (free now): entry b, word q: the halves of tokens 2q and 2q + 1 all
    // ones where that token is in the history
    {
        const uint32_t b = uint32_t(tid) >> 2, q = uint32_t(tid) & 3u;
        reinterpret_cast<uint32_t*>(lds + kOffMCab)[tid] = (((b >> (2u * q)) & 1u) ? 0x0000ffffu : 0u) |
                                                          (((b >> (2u * q + 1u)) & 1u) ? 0xffff0000u : 0u);
    }
    static_assert(256 * 16 <= kOffMMab - kOffMCab && kT == 1024, "presence masks");
    lds_barrier();

    // ---- 6. the owner part read again: its orank-th logit (id order) whose
    // penalized key is the drawn key.  Repeated tokens whose count changes the
    // answer are flipped.
    if (sh.ok) {
        const Item it = part_geo(a, row, int(sh.owner));
        const uint32_t dk = sh.draw_key;
        const bool pen = pv.pen;
        const unsigned char* vb = static_cast<const unsigned char*>(a.logits) +
                                  2 * (size_t(row) * size_t(a.stride) + size_t(it.s0));
        const unsigned char* pb = pen ? pv.b1 + (it.s0 >> 3) : nullptr;
        static_assert(kMaxPartLen / 8 <= 8 * kT, "a part is at most 8 rounds");
        // the part's logits and presence bytes, eight rounds of 1024 vectors,
        // all requested before the flips are worked out
        auto load_vec = [&](int v, uint4* d, uint32_t* b) {
            const int vc = min(v, it.nvec - 1);
            *d = load16_cached(vb + size_t(vc) * 16);
            *b = pb ? uint32_t(pb[vc]) : 0u;
        };
        uint4 vv[8];
        uint32_t bb[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) load_vec(k * kT + tid, &vv[k], &bb[k]);
        // the owner part's repeat entries' logits, requested behind the part
        // (their flips are worked out after the count, which they correct)
        auto in_owner = [&](uint2 e) { return e.y >= 2u && int(e.x) >= it.s0 && int(e.x) < it.s0 + it.n; };
        uint32_t raw[2] = {0u, 0u};
        if (pen) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (uint32_t(j * kT + tid) >= pv.nrep) rep[j].y = 0u;
                if (in_owner(rep[j])) raw[j] = uint32_t(row16[rep[j].x]);
            }
        }
        const uint4* pmask = reinterpret_cast<const uint4*>(lds + kOffMCab);
        // In the halves' key space (-0 just below +0): an absent token matches
        // when its key lies in [a0, a0 + w0] (the drawn key, with -0 for +0), a
        // history token when it lies in [a1, a1 + w1] (the preimage; none when
        // empty).
        const uint32_t a0 = dk == 0x8000u ? 0x7fffu : dk, w0 = dk == 0x8000u ? 1u : 0u;
        uint32_t a1 = 0u, w1 = 0u;
        bool empty1 = true;
        if (pen && sh.hi1 > sh.lo1) {
            uint32_t lo = sh.lo1, hi = sh.hi1 - 1u;
            if (lo <= 0x8000u && hi >= 0x8000u) lo = min(lo, 0x7fffu);
            a1 = lo; w1 = hi - lo; empty1 = false;
        }
        const uint32_t A0 = a0 | (a0 << 16), W0 = w0 | (w0 << 16), A1 = a1 | (a1 << 16), W1 = w1 | (w1 << 16);
        const uint32_t force = empty1 ? 0xffffffffu : 0u;   // history halves never match
        // Matches per round before the flips, three rounds to a word in 10-bit
        // fields (a wave's sums stay below 1024): per half, the range of the
        // token's kind is selected by the presence mask and tested as
        // max(key - base - width, 0) == 0.
        uint32_t pc[3] = {0u, 0u, 0u};
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int v = r * kT + tid;
            uint32_t c = 0u;
            if (v < it.nvec) {
                const uint4 M = pmask[bb[r]];
                const uint32_t w4[4] = {vv[r].x, vv[r].y, vv[r].z, vv[r].w};
                const uint32_t m4[4] = {M.x, M.y, M.z, M.w};
                uint32_t miss = 0u;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t base = (m4[q] & A1) | (~m4[q] & A0), width = (m4[q] & W1) | (~m4[q] & W0);
                    const uint32_t t = pk_sub_u16(halves_key(w4[q]), base);
                    miss += pk_nonzero_u16(pk_sub_sat_u16(t, width) | (m4[q] & force));
                }
                c = 8u - (miss & 0xffffu) - (miss >> 16);
            }
            pc[r / 3] += c << (10 * (r % 3));
        }
        auto field = [](uint32_t w, int r) { return (w >> (10 * (r % 3))) & 0x3ffu; };
        // Repeated tokens whose count changes the answer are flipped
        if (pen) {
            auto flip_if = [&](uint2 e, uint32_t rw) {
                if (!in_owner(e) || !Elem<DT>::finite_bits(rw)) return;
                const bool m1 = key16(pen_pattern<DT>(rw, 1u, p, inv_r, rep_fast)) == dk;
                const bool mc = key16(pen_pattern<DT>(rw, e.y, p, inv_r, rep_fast)) == dk;
                if (m1 != mc) {
                    const uint32_t off = e.x - uint32_t(it.s0);
                    atomicOr(&flip[off >> 5], 1u << (off & 31u));
                    atomicAdd(&sh.nflip, 1u);
                }
            };
#pragma unroll
            for (int j = 0; j < 2; ++j) flip_if(rep[j], raw[j]);
            for (uint32_t i = uint32_t(2 * kT + tid); i < pv.nrep; i += kT) {   // (long repeat lists)
                const uint2 e = pv.list[i];
                if (in_owner(e)) flip_if(e, uint32_t(row16[e.x]));
            }
        }
        lds_barrier();
        const bool flips = sh.nflip != 0u;
        // exact match bits of one vector (the scalar form of the count, flips applied)
        auto match_bits = [&](uint4 d, uint32_t b, int v) -> uint32_t {
            const uint32_t w4[4] = {d.x, d.y, d.z, d.w};
            uint32_t m = 0u;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t pat = (j & 1) ? (w4[j >> 1] >> 16) : (w4[j >> 1] & 0xffffu);
                const uint32_t k = (pat & 0x8000u) ? (~pat & 0xffffu) : (pat | 0x8000u);
                const bool present = (b >> j) & 1u;
                const bool hit = present ? (!empty1 && k - a1 <= w1) : (k - a0 <= w0);
                m |= hit ? (1u << j) : 0u;
            }
            if (flips) m ^= (flip[v >> 2] >> ((v & 3) * 8)) & 0xffu;
            return m;
        };
        if (flips) {   // (uniform) the flipped vectors counted again
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const int v = r * kT + tid;
                if (v < it.nvec && ((flip[v >> 2] >> ((v & 3) * 8)) & 0xffu)) {
                    const uint32_t c = uint32_t(__builtin_popcount(match_bits(vv[r], bb[r], v)));
                    pc[r / 3] += (c - field(pc[r / 3], r)) << (10 * (r % 3));
                }
            }
        }
        uint32_t pin[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) pin[i] = wave_incl_scan_u32(pc[i]);
        if (lane == kWave - 1) {
#pragma unroll
            for (int r = 0; r < 8; ++r) sh.wtot[r][wave] = field(pin[r / 3], r);
        }
        lds_barrier();
        // exclusive offsets of the (round, wave) blocks in id order (wave 0:
        // lane l holds blocks 2l and 2l + 1 of the 128)
        if (wave == 0) {
            const uint32_t b0 = sh.wtot[(2 * lane) >> 4][(2 * lane) & 15], b1 = sh.wtot[(2 * lane + 1) >> 4][(2 * lane + 1) & 15];
            const uint32_t incl = wave_incl_scan_u32(b0 + b1);
            sh.wtot[(2 * lane) >> 4][(2 * lane) & 15] = incl - b0 - b1;
            sh.wtot[(2 * lane + 1) >> 4][(2 * lane + 1) & 15] = incl - b1;
        }
        lds_barrier();
        const uint32_t want = sh.orank;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const uint32_t c = field(pc[r / 3], r);
            const uint32_t e = sh.wtot[r][wave] + field(pin[r / 3], r) - c;
            if (c && want >= e && want < e + c) {
                const int v = r * kT + tid;
                uint32_t m = match_bits(vv[r], bb[r], v);
                for (uint32_t k = want - e; k > 0u; --k) m &= m - 1u;
                sh.token = it.s0 + 8 * v + __builtin_ctz(m);
            }
        }
        lds_barrier();
    }

    // ---- 7. outputs
    if (tid == 0) {
        const int32_t tok = sh.token;
        if (tok < 0) {   // the tables disagree with the logits: cannot happen for consistent inputs
            a.tokens[row] = -1;
            if (a.uniforms) a.uniforms[row] = sh.u;
            if (a.stats) {
                vi_sample_stats st{};
                st.flags = out_flags | VI_FLAG_ERROR;
                a.stats[row] = st;
            }
        } else {
            a.tokens[row] = tok;
            if (a.uniforms) a.uniforms[row] = sh.u;
            if (a.stats) {
                vi_sample_stats st{};
                st.flags = out_flags;
                st.support = sh.n_support;
                st.finite = N;
                st.support_mass = sh.s_n / kFix;
                st.uniform = sh.u;
                a.stats[row] = st;
            }
            if (a.record && a.pstate && tok < V) {
                const LaneState ls = lane_state(const_cast<unsigned char*>(a.pstate) + size_t(row) * a.pl.lane_bytes,
                                                a.pl);
                state_record_one(ls, a.pl, V, tok);
            }
        }
    }
}

// ------------------------------------------------------------ history view
// Presence bitmap and repeat list of each row's history, in the layout the
// stream reads from a penalty state: one workgroup per row; bitmaps of the
// tokens seen once (B1) and more than once (B2) built with LDS atomics, then
// each B2 token's rank (population count of B2 before it) indexes its count.
struct HistArgs {
    const int32_t* histories;
    const int64_t* offsets;
    const vi_row_params* params;
    int vocabulary, words, cap;
    uint32_t* hb1;     // [rows][words]
    uint2* hlist;      // [rows][cap]
    uint32_t* hhead;   // [rows][2]
};
constexpr int kHistBatch = 32;   // history tokens per thread held in registers

constexpr int kHistLdsWords = 40896;   // B1 + B2 + counts (160 KB less the scalars)

__global__ __launch_bounds__(kT) void history_view_kernel(HistArgs h) {
    __shared__ __attribute__((aligned(16))) uint32_t hl[kHistLdsWords];
    const int row = blockIdx.x, tid = threadIdx.x;
    const int W = h.words;
    uint32_t* B1 = hl;              // then the prefix of B2 per word
    uint32_t* B2 = hl + W;
    uint32_t* cnt = hl + 2 * W;     // [cap]
    __shared__ uint32_t flags, nrep, scan[kW + 1];
    const int64_t b = h.offsets[row], e = h.offsets[row + 1];
    for (int i = tid; i < 2 * W; i += kT) hl[i] = 0u;
    if (tid == 0) flags = 0u;
    __syncthreads();
    const int V = h.vocabulary;
    // The history in batches of kHistBatch tokens per thread (one batch for
    // up to 32,768 tokens, kept in registers for the second pass).  Each pass
    // issues a batch's LDS operations back to back and uses their results
    // after, so their latencies overlap.
    const bool one_batch = e - b <= int64_t(kHistBatch) * kT;
    int32_t t[kHistBatch];
    auto load = [&](int64_t base) {
#pragma unroll
        for (int j = 0; j < kHistBatch; ++j) {
            const int64_t i = base + int64_t(j) * kT + tid;
            t[j] = i < e ? h.histories[i] : -2;   // (-2: past the end)
        }
    };
    for (int64_t base = b; base < e; base += int64_t(kHistBatch) * kT) {
        load(base);
#pragma unroll
        for (int j0 = 0; j0 < kHistBatch; j0 += kHistBatch / 2) {
            uint32_t old[kHistBatch / 2];
#pragma unroll
            for (int j = 0; j < kHistBatch / 2; ++j) {
                const int32_t tj = t[j0 + j];
                old[j] = 0u;
                if (tj >= 0 && tj < V) old[j] = atomicOr(&B1[tj >> 5], 1u << (tj & 31));
                else if (tj != -2) flags = VI_FLAG_BAD_HISTORY;
            }
#pragma unroll
            for (int j = 0; j < kHistBatch / 2; ++j) {
                const int32_t tj = t[j0 + j];
                const uint32_t bit = 1u << (tj & 31);
                if (tj >= 0 && tj < V && (old[j] & bit)) atomicOr(&B2[tj >> 5], bit);
            }
        }
    }
    __syncthreads();
    // B1 out; its LDS then holds the B2 rank of each word's first bit
    uint32_t* out = h.hb1 + size_t(row) * W;
    for (int i = tid; i < W; i += kT) out[i] = B1[i];
    const int per = (W + kT - 1) / kT, w0 = tid * per, w1 = min(W, w0 + per);
    uint32_t own = 0u;
    for (int i = w0; i < w1; ++i) own += uint32_t(__builtin_popcount(B2[i]));
    uint32_t total = 0u;
    const uint32_t ex = block_exclusive_scan_u32<kT>(own, scan, &total);   // (barriers: B1 read before)
    if (total > uint32_t(h.cap)) {   // cannot happen: the launcher sizes cap for the longest history
        if (tid == 0) { h.hhead[2 * row] = 0u; h.hhead[2 * row + 1] = flags | VI_FLAG_ERROR; }
        return;
    }
    {
        uint32_t r = ex;
        for (int i = w0; i < w1; ++i) { B1[i] = r; r += uint32_t(__builtin_popcount(B2[i])); }
    }
    for (uint32_t i = tid; i < total; i += kT) cnt[i] = 0u;
    __syncthreads();
    for (int64_t base = b; base < e; base += int64_t(kHistBatch) * kT) {
        if (!one_batch) load(base);
#pragma unroll
        for (int j0 = 0; j0 < kHistBatch; j0 += kHistBatch / 2) {   // (half a batch at a time: registers)
            uint32_t wd[kHistBatch / 2], r0[kHistBatch / 2];
#pragma unroll
            for (int j = 0; j < kHistBatch / 2; ++j) {
                const int32_t tj = t[j0 + j];
                const bool ok = tj >= 0 && tj < V;
                wd[j] = ok ? B2[tj >> 5] : 0u;
                r0[j] = ok ? B1[tj >> 5] : 0u;
            }
#pragma unroll
            for (int j = 0; j < kHistBatch / 2; ++j) {
                const uint32_t bit = 1u << (t[j0 + j] & 31);
                if (wd[j] & bit) atomicAdd(&cnt[r0[j] + uint32_t(__builtin_popcount(wd[j] & (bit - 1u)))], 1u);
            }
        }
    }
    __syncthreads();
    uint2* lst = h.hlist + size_t(row) * h.cap;
    for (int i = w0; i < w1; ++i) {
        uint32_t wd = B2[i], r = B1[i];
        while (wd) {
            const int j = __builtin_ctz(wd);
            wd &= wd - 1u;
            lst[r] = make_uint2(uint32_t(32 * i + j), cnt[r]);
            ++r;
        }
    }
    if (tid == 0) { h.hhead[2 * row] = total; h.hhead[2 * row + 1] = flags; }
}

}  // namespace

// ------------------------------------------------------------------ host
struct StreamPlan {
    int parts, part_len;
};
static StreamPlan stream_plan(int rows, int vocabulary) {
    const int cus = device_cus();
    int parts = (vocabulary + kMaxPartLen - 1) / kMaxPartLen;
    const int fill = (cus + std::max(rows, 1) - 1) / std::max(rows, 1);   // parts that give every CU one
    parts = std::max(parts, std::min(kMaxParts, fill));
    // a multiple of 32 tokens: every part's presence bytes start 4-byte aligned
    const int len = ((vocabulary + parts - 1) / parts + 31) / 32 * 32;
    return {(vocabulary + len - 1) / len, len};
}
static int hist_words(int vocabulary) { return (vocabulary + 31) / 32; }
static int hist_cap(int64_t max_history) { return int(std::max<int64_t>(max_history / 2, 1)); }
static bool hist_fits(int vocabulary, int64_t max_history) {
    return max_history <= (int64_t(1) << 30) &&
           2 * int64_t(hist_words(vocabulary)) + hist_cap(max_history) <= kHistLdsWords;
}

// The stream launch: workgroups, XCD-aware mapping, and the most parts one
// workgroup takes (its XCD's parts shared out in turn).
struct StreamGrid {
    int grid, xcd, per_wg;
};
static StreamGrid stream_grid(int rows, int parts) {
    StreamGrid g;
    const int items = rows * parts;
    g.grid = std::min(device_cus(), items);
    g.xcd = (rows >= kXcds && g.grid % kXcds == 0) ? 1 : 0;
    const int xr = g.xcd ? (rows + kXcds - 1) / kXcds : rows, xw = g.xcd ? g.grid / kXcds : g.grid;
    g.per_wg = (xr * parts + xw - 1) / xw;
    return g;
}

bool stream_supported(const SampleArgs& s) {
    if (s.dtype != VI_BF16 && s.dtype != VI_F16) return false;
    if (s.probs || s.full_out || s.rows <= 0) return false;
    if (s.vocabulary <= 0 || s.vocabulary % 8 || s.vocabulary > kMaxParts * kMaxPartLen) return false;
    if (s.stride < s.vocabulary || s.stride % 8 || reinterpret_cast<uintptr_t>(s.logits) % 16) return false;
    if (int64_t(s.rows) * kMaxParts > (int64_t(1) << 30)) return false;
    if (stream_grid(s.rows, stream_plan(s.rows, s.vocabulary).parts).per_wg > kMaxItems) return false;
    const bool hist = !s.pstate && s.histories && s.offsets && s.max_history > 0;
    if (hist && !hist_fits(s.vocabulary, s.max_history)) return false;
    return true;
}

size_t stream_workspace(int rows, int vocabulary, int64_t max_history) {
    if (rows <= 0 || vocabulary <= 0 || vocabulary % 8 || vocabulary > kMaxParts * kMaxPartLen) return 0;
    const StreamPlan pl = stream_plan(rows, vocabulary);
    const size_t np = size_t(rows) * pl.parts;
    size_t b = align_up(np * kPub * 4, 256) + align_up(np * kGroups * kGW * 4, 256);
    if (max_history > 0 && hist_fits(vocabulary, max_history))
        b += align_up(size_t(rows) * hist_words(vocabulary) * 4, 256) +
             align_up(size_t(rows) * hist_cap(max_history) * 8, 256) + align_up(size_t(rows) * 8, 256);
    return b + 256;
}

vi_status launch_stream(const SampleArgs& s, unsigned char* ws, size_t ws_bytes, hipStream_t stream) {
    if (!stream_supported(s)) return VI_ERR_UNSUPPORTED;
    const StreamPlan pl = stream_plan(s.rows, s.vocabulary);
    StreamArgs a{};
    a.logits = s.logits; a.rows = s.rows; a.vocabulary = s.vocabulary; a.stride = s.stride;
    a.parts = pl.parts; a.part_len = pl.part_len;
    a.params = s.params;
    a.record = s.pstate ? s.record : 0;
    a.tokens = s.tokens; a.uniforms = s.uniforms; a.stats = s.stats;
    const size_t np = size_t(s.rows) * pl.parts;
    Carver c(ws, ws_bytes);
    a.ppub = c.take<uint32_t>(np * kPub);
    a.pwords = c.take<uint4>(np * kGroups * (kGW / 4));
    const bool hist = !s.pstate && s.histories && s.offsets && s.max_history > 0;
    HistArgs h{};
    if (s.pstate) {
        a.pstate = s.pstate;
        a.pl = s.playout;
    } else if (hist) {
        h.histories = s.histories; h.offsets = s.offsets; h.params = s.params; h.vocabulary = s.vocabulary;
        h.words = hist_words(s.vocabulary);
        h.cap = hist_cap(s.max_history);
        h.hb1 = c.take<uint32_t>(size_t(s.rows) * h.words);
        h.hlist = c.take<uint2>(size_t(s.rows) * h.cap);
        h.hhead = c.take<uint32_t>(size_t(s.rows) * 2);
        a.hb1 = h.hb1; a.hlist = h.hlist; a.hhead = h.hhead; a.hwords = h.words; a.hcap = h.cap;
    }
    if (!c.ok) return VI_ERR_WORKSPACE;
    const StreamGrid sg = stream_grid(s.rows, pl.parts);
    a.grid = sg.grid;
    a.xcd = sg.xcd;
    if (hist) {
        hipLaunchKernelGGL(history_view_kernel, dim3(s.rows), dim3(kT), 0, stream, h);
        if (launch_status() != VI_OK) return VI_ERR_LAUNCH;
    }
    // the merge's workgroup of row r runs on the XCD whose workgroups streamed
    // the row (workgroup r goes to XCD r % 8, as the stream's rows do)
    const bool pb = a.pstate || a.hb1;
    if (s.dtype == VI_BF16) {
        if (pb) hipLaunchKernelGGL((stream_kernel<VI_BF16, true>), dim3(a.grid), dim3(kT), 0, stream, a);
        else hipLaunchKernelGGL((stream_kernel<VI_BF16, false>), dim3(a.grid), dim3(kT), 0, stream, a);
        hipLaunchKernelGGL(merge_kernel<VI_BF16>, dim3(s.rows), dim3(kT), 0, stream, a);
    } else {
        if (pb) hipLaunchKernelGGL((stream_kernel<VI_F16, true>), dim3(a.grid), dim3(kT), 0, stream, a);
        else hipLaunchKernelGGL((stream_kernel<VI_F16, false>), dim3(a.grid), dim3(kT), 0, stream, a);
        hipLaunchKernelGGL(merge_kernel<VI_F16>, dim3(s.rows), dim3(kT), 0, stream, a);
    }
    return launch_status();
}

}  // namespace vi
