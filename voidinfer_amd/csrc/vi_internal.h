// vi_internal.h — host-side launch interface between the C ABI (capi.hip) and the
// kernel translation units.  Not installed; not part of the ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/voidinfer_sampling.h"

namespace vi {

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }
inline int elem_size(int dtype) { return dtype == VI_F32 ? 4 : 2; }

// Bump allocator over a caller workspace; every region 256-byte aligned.
struct Carver {
    unsigned char* base;
    size_t size, used = 0;
    bool ok = true;
    Carver(void* b, size_t s) : base(static_cast<unsigned char*>(b)), size(s) {}
    template <class T> T* take(size_t count) {
        const size_t at = align_up(used, 256), bytes = align_up(count * sizeof(T), 256);
        used = at + bytes;
        if (!base || used > size) { ok = false; return nullptr; }
        return reinterpret_cast<T*>(base + at);
    }
};

// ---- greedy -----------------------------------------------------------------
struct GreedyPlan {
    int slices, slice_len;
};
GreedyPlan greedy_plan(int rows, int vocabulary);
size_t greedy_workspace(int rows, int vocabulary);
// arrival_rows: the rows the workspace was carved for (its arrival counters
// come first, that many; 0: rows).
vi_status launch_greedy(const void* logits, int dtype, int rows, int vocabulary, int64_t stride,
                        uint64_t serial, vi_greedy_row* out, void* ws, size_t ws_bytes,
                        hipStream_t stream, int arrival_rows = 0);
// Allocation-free greedy: the workspace is a 64 KiB device array of the library
// (every shape's greedy workspace fits it), its per-device address looked up by
// greedy_scratch_setup (vi_init, or the first call on a device).
constexpr size_t kGreedyScratchBytes = 65536;
vi_status greedy_scratch_setup(void** ptr);
vi_status launch_greedy_noalloc(const void* logits, int dtype, int rows, int vocabulary, int64_t stride,
                                uint64_t serial, vi_greedy_row* out, hipStream_t stream);
// VeriCache exact row scores (argmax + gap of next[r]); workspace as greedy.
vi_status launch_row_scores(const void* logits, int dtype, int rows, int vocabulary, int64_t stride,
                            const int64_t* next, int64_t* greedy, float* gap, void* ws, size_t ws_bytes,
                            hipStream_t stream);

// ---- top-k family -------------------------------------------------------------
enum TopkMode { kModeTopk = 0, kModePacket = 1, kModeSample = 2, kModeVerify = 3 };

struct PacketKeys {   // Exl3SampledKeys (sampled_select.cuh:38)
    int first;
    int depth[16];
    int inputs;
    int input[16];
};

struct TopkPlan {
    int slices, slice_len;
};
TopkPlan topk_plan(int rows, int vocabulary);
// Partial-list + counter bytes of one launch over `rows` rows.
size_t topk_partials_bytes(int rows, int vocabulary);

vi_status launch_topk_rows(const void* logits, int dtype, int rows, int vocabulary, int64_t stride,
                           int k, int64_t* ids, float* values, float* logprobs,
                           uint32_t* nonfinite_flag, void* ws, size_t ws_bytes, hipStream_t stream);

vi_status launch_packet(const void* scores, int dtype, int rows, int vocabulary, int64_t stride,
                        const vi_device_sampling& cfg, const PacketKeys& keys, uint64_t serial,
                        vi_greedy_row* out, void* ws, size_t ws_bytes, hipStream_t stream);
// VeriCache sampled row scores: the coupled draw of row r at key first_key + r
// (no drafted path) and the gap of next[r].
vi_status launch_sampled_scores(const void* scores, int dtype, int rows, int vocabulary, int64_t stride,
                                const vi_device_sampling& cfg, int first_key, float tolerance,
                                const int64_t* next, int64_t* chosen, float* gap, void* ws, size_t ws_bytes,
                                hipStream_t stream);

// Sorted, filtered top-k lists (z values, ids) of verification rows.  With
// `decide` (every lane listed) the rows' last workgroups also take decisions:
// decide_mode 2 over the target rows draws the bonus rows' tokens; decide_mode
// 1 over the draft rows (the target rows' lists complete before the launch)
// takes each position's accept decision, and each lane's last position walks
// the lane's chain.
struct PosDecision;
struct VerifyDecideArgs {
    int drafts, target_rows;
    const float* tlval;
    const int* tlidx;
    const uint32_t* tlvalid;
    const uint32_t* tlflags;
    const float* dlval;      // (the paired launch: the draft rows' lists, and the
    const int* dlidx;        //  positions' arrival counters [lanes][drafts + 1],
    const uint32_t* dlvalid; //  zero between calls)
    const uint32_t* dlflags;
    uint32_t* parr;
    const int32_t* drafted;
    PosDecision* dec;
    uint32_t* larr;
    const int64_t* terminal;
    int n_terminal;
    int32_t* accepted;
    int32_t* committed;
    int32_t* committed_count;
    uint32_t* lane_flags;
};
vi_status launch_verify_lists(const void* logits, int dtype, int rows, int layout_rows, int layout_slices,
                              int vocabulary, int64_t stride, const vi_row_params* params, int params_div,
                              float* lval, int* lidx, uint32_t* lvalid, uint32_t* lflags, int skip_unlisted,
                              void* ws, size_t ws_bytes, hipStream_t stream, const VerifyDecideArgs* decide = nullptr,
                              int decide_mode = 0);
// Target and draft rows of sampled verification in one launch (both row sets
// 16-byte aligned 16-bit logits, every lane listed): each position's decision
// is taken by the later of its two rows to finish (a bonus row decides alone),
// and each lane's last decided position walks the chain.
vi_status launch_verify_pair(const void* target, int target_dtype, int64_t target_stride, const void* draft,
                             int draft_dtype, int64_t draft_stride, int lanes, int vocabulary,
                             const vi_row_params* params, int layout_rows, int layout_slices, float* tval, int* tidx,
                             uint32_t* tvalid, uint32_t* tflags, float* dval, int* didx, uint32_t* dvalid,
                             uint32_t* dflags, const VerifyDecideArgs& decide, void* ws, size_t ws_bytes,
                             hipStream_t stream, int skip_unlisted);
bool verify_pair_supported(const void* target, int target_dtype, int64_t target_stride, const void* draft,
                           int draft_dtype, int64_t draft_stride);
size_t topk_partials_bytes_slices(int rows, int slices);

// History hash (token -> count) per row for the top-k sampler route.
size_t history_hash_slots(int64_t max_history);

// ---- per-lane penalty state --------------------------------------------------
// One lane's state, at lane * lane_bytes: a 64-byte header (flags as VI_FLAG_*
// bits, sticky until reset; keys = hash slots holding a token; total = tokens
// recorded minus tokens removed; nrep = repeat-list entries), a presence
// bitmap of ceil(V / 32) words (rounded up to 16 bytes), an open-addressing
// hash of (token + 1, count) pairs with linear probing from
// (token * 0x9E3779B1) >> (32 - log2 slots), per slot the 1-based index of the
// slot's token in the repeat list (0: none), and the repeat list: one
// (token, count) entry per token that has reached count 2 since the reset, in
// the order they did, holding the token's current count (an entry whose count
// fell below 2 is kept and ignored).  A removed token keeps its slot (count 0),
// so probe chains stay intact.
struct PenaltyHeader {
    uint32_t flags, keys;
    uint64_t total;
    uint32_t nrep;
    uint32_t pad[11];
};
static_assert(sizeof(PenaltyHeader) == 64, "penalty header");
struct PenaltyLayout {
    size_t lane_bytes, off_b1, off_hash, off_ridx, off_list;
    int words, slots, shift;
};
inline bool penalty_slots_ok(int slots) {
    return slots >= 64 && slots <= (1 << 26) && (slots & (slots - 1)) == 0;
}
inline PenaltyLayout penalty_layout(int vocabulary, int slots) {
    PenaltyLayout l{};
    l.words = int(align_up((size_t(vocabulary) + 31) / 32, 4));
    l.slots = slots;
    l.shift = 32 - __builtin_ctz(unsigned(slots));
    l.off_b1 = sizeof(PenaltyHeader);
    l.off_hash = align_up(l.off_b1 + 4 * size_t(l.words), 64);
    l.off_ridx = l.off_hash + 8 * size_t(slots);
    l.off_list = l.off_ridx + 4 * size_t(slots);
    l.lane_bytes = align_up(l.off_list + 8 * size_t(slots), 256);
    return l;
}
vi_status launch_penalty_reset(void* states, int lanes, const PenaltyLayout& l, hipStream_t stream);
vi_status launch_penalty_update(void* states, int lanes, int vocabulary, const PenaltyLayout& l,
                                const int32_t* tokens, const int64_t* offsets, int sign, hipStream_t stream);

// Filtered distribution of one full-route row, as the merges leave it for the
// probabilities and for verification: the support is every valid logit whose
// order key lies above end_key, plus the first end_take logits of end_key in id
// order (end_take ~0u: all of them; end_key 0: every valid logit); there
// p = exp(z - z0) / s_n.  valid = 0: no distribution (empty or failed row).
// Order keys: key16 of the (penalized) 16-bit pattern, or the 32-bit order key
// of z for fp32 rows.
struct FullBound {
    double z0, s_n;
    float inv_t;
    uint32_t end_key, end_take, valid;
};
constexpr int kFullBaseSlots = 32;   // bases per row: end-key logits in the slices before each slice
// Optional outputs of a full-route launch (verification reads them back).
struct FullOut {
    FullBound* bounds;   // [rows]
    uint32_t* bases;     // [rows][kFullBaseSlots]
};
// Logits per slice of the full routes (granularity of FullOut::bases).
constexpr int kFullSlice16 = 32768, kFullSlice32 = 16384;

struct SampleArgs {
    const void* logits;
    int dtype, rows, vocabulary;
    int64_t stride;
    const vi_row_params* params;
    const int32_t* histories;
    const int64_t* offsets;
    int64_t max_history;
    unsigned char* pstate;   // per-lane penalty states instead of histories (or null)
    PenaltyLayout playout;
    int record;              // append each row's sampled token to its lane's state
    int32_t* tokens;
    double* uniforms;
    float* probs;
    int64_t probs_stride;
    vi_sample_stats* stats;
    uint32_t route_mask;
    const FullOut* full_out;   // (optional) full-route rows' distributions
};
size_t sample_workspace(int rows, int vocabulary, int64_t max_history);
vi_status launch_sample(const SampleArgs& a, void* ws, size_t ws_bytes, hipStream_t stream);

// ---- full-vocabulary pair kernel --------------------------------------------
int device_cus();
// A second stream of the calling host thread on the current device, with a
// fork and a join event (created on first use; nullptr when unavailable): a
// call whose rows take both kernel routes runs the full-vocabulary route on it,
// joined back into the caller's stream before the call returns.
struct SideStream {
    hipStream_t stream;
    hipEvent_t fork, join;
};
SideStream* side_stream();
// ---- full-vocabulary rows, stream and merge launches (sample_stream.hip): 16-bit logits,
// aligned rows, vocabulary a multiple of 8, no probabilities or bounds wanted.
bool stream_supported(const SampleArgs& s);
size_t stream_workspace(int rows, int vocabulary, int64_t max_history);
vi_status launch_stream(const SampleArgs& s, unsigned char* ws, size_t ws_bytes, hipStream_t stream);
size_t full_workspace(int rows, int vocabulary);
vi_status launch_full(const SampleArgs& a, unsigned char* ws, size_t ws_bytes, hipStream_t stream);
bool full_supported(int dtype, int vocabulary, int64_t stride);
// fp32 rows of the full route (sample_wide.hip); the history route's hash and
// flags are the top-k route's buffers (rows of the two routes are disjoint).
size_t wide_workspace(int rows, int vocabulary);
bool wide_supported(int vocabulary, int64_t stride);
vi_status launch_wide(const SampleArgs& a, unsigned char* ws, size_t ws_bytes, uint2* hash, int hash_shift,
                      int hash_slots, uint32_t* row_flags, hipStream_t stream);

// ---- verification ----------------------------------------------------------------
struct VerifyArgs {
    int mode;
    const void* target;
    int target_dtype;
    int64_t target_stride;
    int target_rows;
    const void* draft;
    int draft_dtype;
    int64_t draft_stride;
    int lanes, drafts, vocabulary;
    const int32_t* drafted;
    const vi_row_params* params;
    const int64_t* terminal;
    int n_terminal;
    int32_t* accepted;
    int32_t* committed;
    int32_t* committed_count;
    uint32_t* lane_flags;
};
size_t verify_workspace(int lanes, int drafts, int vocabulary);
vi_status launch_verify(const VerifyArgs& a, void* ws, size_t ws_bytes, hipStream_t stream);

// ---- probes -----------------------------------------------------------------------
vi_status launch_probe_read(const void* src, size_t bytes, uint32_t* sink, hipStream_t stream);
vi_status launch_probe_copy(void* dst, const void* src, size_t bytes, hipStream_t stream);
vi_status launch_draft_choice(int lanes, int positions, int vocabulary, const float* scores,
                              const int64_t* candidates, const int64_t* seed_tokens,
                              const vi_draft_sampling* sampling, int64_t* proposals, hipStream_t stream);
vi_status launch_selector_chain(int lanes, int positions, int vocabulary, const int64_t* anchors,
                                const int64_t* candidates, const float* unary, const void* hidden,
                                const void* pred_codebook, const void* succ_codebook,
                                const vi_draft_sampling* sampling, int64_t* proposals, hipStream_t stream);
vi_status launch_presence_reset(int32_t* table, int vocabulary, hipStream_t stream);
vi_status launch_presence_truncate(int32_t* table, int vocabulary, int from, hipStream_t stream);
vi_status launch_presence_record(int32_t* table, int vocabulary, int first, const int64_t* tokens,
                                 size_t count, hipStream_t stream);

inline vi_status launch_status() {
    return hipGetLastError() == hipSuccess ? VI_OK : VI_ERR_LAUNCH;
}

}  // namespace vi
