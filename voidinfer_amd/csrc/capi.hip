// capi.hip — the extern "C" boundary (include/voidinfer_sampling.h): argument
// validation, workspace sizing and dispatch to the kernel translation units.
// No exceptions cross it, and nothing here allocates device memory or
// synchronizes.
#include <string.h>

#include <mutex>

#include "vi_internal.h"
#include "../../include/voidinfer_sampling.hpp"

using namespace vi;

namespace {

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }
inline bool dtype_ok(int d) { return d == VI_BF16 || d == VI_F16 || d == VI_F32; }

}  // namespace

extern "C" {

uint32_t vi_abi_version(void) { return 1u; }

vi_status vi_init(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return VI_ERR_DEVICE;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return VI_ERR_DEVICE;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return VI_ERR_DEVICE;
    // per-device address of the allocation-free greedy's scratch array
    return greedy_scratch_setup(nullptr);
}

const char* vi_status_string(vi_status status) {
    switch (status) {
        case VI_OK: return "ok";
        case VI_ERR_INVALID: return "invalid argument";
        case VI_ERR_UNSUPPORTED: return "unsupported request";
        case VI_ERR_WORKSPACE: return "workspace missing or too small";
        case VI_ERR_LAUNCH: return "HIP launch failed";
        case VI_ERR_DEVICE: return "device is not gfx950";
        default: return "unknown status";
    }
}

size_t vi_greedy_workspace_bytes(int rows, int vocabulary) {
    if (rows <= 0 || vocabulary <= 0) return 0;
    return greedy_workspace(rows, vocabulary);
}

vi_status vi_greedy_rows(const void* logits, int dtype, int rows, int vocabulary, int64_t row_stride,
                         uint64_t serial, vi_greedy_row* out, void* workspace, size_t workspace_bytes,
                         void* stream) {
    if (rows == 0) return VI_OK;
    if (rows < 0 || vocabulary <= 0 || row_stride < vocabulary || !dtype_ok(dtype) || !logits || !out)
        return VI_ERR_INVALID;
    return launch_greedy(logits, dtype, rows, vocabulary, row_stride, serial, out, workspace, workspace_bytes,
                         as_stream(stream));
}

vi_status vi_greedy_rows_noalloc(const void* logits, int dtype, int rows, int vocabulary, int64_t row_stride,
                                 uint64_t serial, vi_greedy_row* out, void* stream) {
    if (rows == 0) return VI_OK;
    if (rows < 0 || vocabulary <= 0 || row_stride < vocabulary || !dtype_ok(dtype) || !logits || !out)
        return VI_ERR_INVALID;
    return launch_greedy_noalloc(logits, dtype, rows, vocabulary, row_stride, serial, out, as_stream(stream));
}

size_t vi_topk_workspace_bytes(int rows, int vocabulary, int k) {
    if (rows <= 0 || vocabulary <= 0 || k <= 0) return 0;
    return topk_partials_bytes(rows, vocabulary);
}

vi_status vi_topk_rows(const void* logits, int dtype, int rows, int vocabulary, int64_t row_stride, int k,
                       int64_t* ids, float* values, float* logprobs, uint32_t* nonfinite_flag, void* workspace,
                       size_t workspace_bytes, void* stream) {
    if (rows == 0) return VI_OK;
    if (rows < 0 || vocabulary <= 0 || row_stride < vocabulary || k < 1 || k > 64 || k > vocabulary ||
        !dtype_ok(dtype) || !logits || !ids || !values)
        return VI_ERR_INVALID;
    return launch_topk_rows(logits, dtype, rows, vocabulary, row_stride, k, ids, values, logprobs, nonfinite_flag,
                            workspace, workspace_bytes, as_stream(stream));
}

vi_status vi_topk16_for_test(const uint16_t* logits, int rows, int vocab, int64_t* ids, float* values,
                             uint32_t* nonfinite_flag, void* stream) {
    if (rows == 0) return VI_OK;
    if (rows < 0 || vocab < 16 || !logits || !ids || !values) return VI_ERR_INVALID;
    // the library's scratch per device, grown to the largest shape seen
    struct Owned {
        void* ptr = nullptr;
        size_t bytes = 0;
    };
    static Owned owned[64];
    static std::mutex guard;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return VI_ERR_DEVICE;
    const size_t need = topk_partials_bytes(rows, vocab);
    // held until the launch is queued: another thread cannot grow (free) the
    // buffer between this call's choice of it and its launch
    std::lock_guard<std::mutex> lock(guard);
    Owned& o = owned[dev];
    if (o.bytes < need) {
        if (o.ptr && hipFree(o.ptr) != hipSuccess) return VI_ERR_LAUNCH;   // (waits for the device)
        o.ptr = nullptr;
        o.bytes = 0;
        if (hipMalloc(&o.ptr, need) != hipSuccess) return VI_ERR_LAUNCH;
        if (hipMemset(o.ptr, 0, need) != hipSuccess) return VI_ERR_LAUNCH;
        o.bytes = need;
    }
    return launch_topk_rows(logits, VI_F16, rows, vocab, vocab, 16, ids, values, nullptr, nonfinite_flag, o.ptr, need,
                            as_stream(stream));
}

size_t vi_sampled_packet_workspace_bytes(int rows, int vocabulary) {
    if (rows <= 0 || vocabulary <= 0) return 0;
    return topk_partials_bytes(rows, vocabulary);
}

vi_status vi_sampled_packet(const void* scores, int dtype, int rows, int vocabulary, int64_t row_stride,
                            const vi_device_sampling* cfg, int first_key, const int32_t* depths, int n_depths,
                            const int32_t* inputs, int n_inputs, uint64_t serial, vi_greedy_row* out,
                            void* workspace, size_t workspace_bytes, void* stream) {
    if (rows <= 0 || rows > 16 || vocabulary <= 0 || row_stride < vocabulary || !dtype_ok(dtype) || !scores ||
        !cfg || !out)
        return VI_ERR_INVALID;
    PacketKeys keys{};
    keys.first = first_key;
    const bool tree = n_depths == rows && depths;
    for (int r = 0; r < rows; ++r) keys.depth[r] = tree ? depths[r] : r;
    if (n_inputs == rows && inputs) {
        keys.inputs = rows;
        for (int r = 0; r < rows; ++r) keys.input[r] = inputs[r];
    }
    return launch_packet(scores, dtype, rows, vocabulary, row_stride, *cfg, keys, serial, out, workspace,
                         workspace_bytes, as_stream(stream));
}

size_t vi_row_scores_workspace_bytes(int rows, int vocabulary) {
    if (rows <= 0 || vocabulary <= 0) return 0;
    return greedy_workspace(rows, vocabulary);
}

vi_status vi_row_scores(const void* logits, int dtype, int rows, int vocabulary, int64_t row_stride,
                        const int64_t* next, int64_t* greedy, float* gap, void* workspace, size_t workspace_bytes,
                        void* stream) {
    if (rows == 0) return VI_OK;
    if (rows < 0 || vocabulary <= 0 || row_stride < vocabulary || !dtype_ok(dtype) || !logits || !next || !greedy ||
        !gap)
        return VI_ERR_INVALID;
    return launch_row_scores(logits, dtype, rows, vocabulary, row_stride, next, greedy, gap, workspace,
                             workspace_bytes, as_stream(stream));
}

size_t vi_sampled_scores_workspace_bytes(int rows, int vocabulary) {
    if (rows <= 0 || vocabulary <= 0) return 0;
    return topk_partials_bytes(rows, vocabulary);
}

vi_status vi_sampled_scores(const void* scores, int dtype, int rows, int vocabulary, int64_t row_stride,
                            const vi_device_sampling* cfg, int first_key, float tolerance, const int64_t* next,
                            int64_t* chosen, float* gap, void* workspace, size_t workspace_bytes, void* stream) {
    if (rows == 0) return VI_OK;
    if (rows < 0 || vocabulary <= 0 || row_stride < vocabulary || !dtype_ok(dtype) || !scores || !cfg || !next ||
        !chosen || !gap || !(tolerance >= 0.0f))
        return VI_ERR_INVALID;
    return launch_sampled_scores(scores, dtype, rows, vocabulary, row_stride, *cfg, first_key, tolerance, next, chosen,
                                 gap, workspace, workspace_bytes, as_stream(stream));
}

vi_status vi_draft_choice(int lanes, int positions, int vocabulary, const float* scores, const int64_t* candidates,
                          const int64_t* seed_tokens, const vi_draft_sampling* sampling, int64_t* proposals,
                          void* stream) {
    if (lanes == 0 || positions == 0) return VI_OK;
    if (lanes < 0 || positions < 0 || vocabulary <= 0 || !scores || !candidates || !sampling || !proposals)
        return VI_ERR_INVALID;
    return launch_draft_choice(lanes, positions, vocabulary, scores, candidates, seed_tokens, sampling, proposals,
                               as_stream(stream));
}

vi_status vi_selector_chain(int lanes, int positions, int vocabulary, const int64_t* anchors,
                            const int64_t* candidates, const float* unary, const void* hidden,
                            const void* pred_codebook, const void* succ_codebook,
                            const vi_draft_sampling* sampling, int64_t* proposals, void* stream) {
    if (lanes == 0 || positions == 0) return VI_OK;
    if (lanes < 0 || positions < 0 || vocabulary <= 0 || !anchors || !candidates || !unary || !hidden ||
        !pred_codebook || !succ_codebook || !proposals)
        return VI_ERR_INVALID;
    return launch_selector_chain(lanes, positions, vocabulary, anchors, candidates, unary, hidden, pred_codebook,
                                 succ_codebook, sampling, proposals, as_stream(stream));
}

vi_status vi_build_verification_tree(const int64_t* drafts, int depth, const int64_t* candidate_ids,
                                     const float* candidate_unary, int budget, int max_siblings, float row_cost,
                                     int32_t* chain_drafts, int64_t* sibling_tokens, int32_t* sibling_offsets,
                                     int32_t* sibling_count) {
    if (depth < 0 || budget < 0 || !chain_drafts || !sibling_count || (depth > 0 && (!drafts || !candidate_ids ||
        !candidate_unary)) || (budget > 0 && (!sibling_tokens || !sibling_offsets)) || !std::isfinite(row_cost))
        return VI_ERR_INVALID;
    try {   // (the host layer's implementation; nothing throws across the ABI)
        const std::size_t n = std::size_t(depth);
        const voidinfer_amd::Exl3VerificationTree t = voidinfer_amd::exl3_build_verification_tree(
            std::span<const int64_t>(drafts, n), std::span<const int64_t>(candidate_ids, n * 16),
            std::span<const float>(candidate_unary, n * 16), budget, max_siblings, row_cost);
        *chain_drafts = t.chain_drafts;
        *sibling_count = int32_t(t.sibling_tokens.size());
        for (std::size_t i = 0; i < t.sibling_tokens.size(); ++i) {
            sibling_tokens[i] = t.sibling_tokens[i];
            sibling_offsets[i] = t.sibling_offsets[i];
        }
        return VI_OK;
    } catch (const std::invalid_argument&) {
        return VI_ERR_INVALID;
    } catch (...) {
        return VI_ERR_UNSUPPORTED;
    }
}

vi_status vi_presence_reset(int32_t* table, int vocabulary, void* stream) {
    if (!table || vocabulary <= 0) return VI_ERR_INVALID;
    return launch_presence_reset(table, vocabulary, as_stream(stream));
}
vi_status vi_presence_truncate(int32_t* table, int vocabulary, int from, void* stream) {
    if (!table || vocabulary <= 0) return VI_ERR_INVALID;
    return launch_presence_truncate(table, vocabulary, from, as_stream(stream));
}
vi_status vi_presence_record(int32_t* table, int vocabulary, int first, const int64_t* tokens, size_t count,
                             void* stream) {
    if (!table || vocabulary <= 0 || (count && !tokens)) return VI_ERR_INVALID;
    return launch_presence_record(table, vocabulary, first, tokens, count, as_stream(stream));
}

size_t vi_sample_workspace_bytes(int rows, int vocabulary, int64_t max_history) {
    if (rows <= 0 || vocabulary <= 0 || max_history < 0) return 0;
    return sample_workspace(rows, vocabulary, max_history);
}

vi_status vi_sample_rows(const void* logits, int dtype, int rows, int vocabulary, int64_t row_stride,
                         const vi_row_params* params, const int32_t* histories, const int64_t* history_offsets,
                         int64_t max_history, int32_t* tokens, double* uniforms, float* probs,
                         int64_t probs_stride, vi_sample_stats* stats, uint32_t route_mask, void* workspace,
                         size_t workspace_bytes, void* stream) {
    if (rows == 0) return VI_OK;
    if (rows < 0 || vocabulary <= 0 || row_stride < vocabulary || !dtype_ok(dtype) || !logits || !params ||
        !tokens || max_history < 0 || (probs && probs_stride < vocabulary) || (histories && !history_offsets))
        return VI_ERR_INVALID;
    SampleArgs a{};
    a.logits = logits; a.dtype = dtype; a.rows = rows; a.vocabulary = vocabulary; a.stride = row_stride;
    a.params = params; a.histories = histories; a.offsets = history_offsets; a.max_history = max_history;
    a.tokens = tokens; a.uniforms = uniforms; a.probs = probs; a.probs_stride = probs_stride; a.stats = stats;
    a.route_mask = route_mask == 0 ? uint32_t(VI_ROUTE_ALL) : route_mask;
    return launch_sample(a, workspace, workspace_bytes, as_stream(stream));
}

size_t vi_penalty_state_bytes(int vocabulary, int slots) {
    if (vocabulary <= 0 || !penalty_slots_ok(slots)) return 0;
    return penalty_layout(vocabulary, slots).lane_bytes;
}

vi_status vi_penalty_state_reset(void* states, int lanes, int vocabulary, int slots, void* stream) {
    if (lanes == 0) return VI_OK;
    if (lanes < 0 || !states || vocabulary <= 0 || !penalty_slots_ok(slots)) return VI_ERR_INVALID;
    return launch_penalty_reset(states, lanes, penalty_layout(vocabulary, slots), as_stream(stream));
}

vi_status vi_penalty_state_update(void* states, int lanes, int vocabulary, int slots, const int32_t* tokens,
                                  const int64_t* offsets, int sign, void* stream) {
    if (lanes == 0) return VI_OK;
    if (lanes < 0 || !states || !tokens || vocabulary <= 0 || !penalty_slots_ok(slots) || (sign != 1 && sign != -1))
        return VI_ERR_INVALID;
    return launch_penalty_update(states, lanes, vocabulary, penalty_layout(vocabulary, slots), tokens, offsets, sign,
                                 as_stream(stream));
}

vi_status vi_sample_rows_state(const void* logits, int dtype, int rows, int vocabulary, int64_t row_stride,
                               const vi_row_params* params, void* states, int slots, int record, int32_t* tokens,
                               double* uniforms, float* probs, int64_t probs_stride, vi_sample_stats* stats,
                               uint32_t route_mask, void* workspace, size_t workspace_bytes, void* stream) {
    if (rows == 0) return VI_OK;
    if (rows < 0 || vocabulary <= 0 || row_stride < vocabulary || !dtype_ok(dtype) || !logits || !params ||
        !tokens || !states || !penalty_slots_ok(slots) || (probs && probs_stride < vocabulary) ||
        (record != 0 && record != 1))
        return VI_ERR_INVALID;
    SampleArgs a{};
    a.logits = logits; a.dtype = dtype; a.rows = rows; a.vocabulary = vocabulary; a.stride = row_stride;
    a.params = params; a.pstate = static_cast<unsigned char*>(states);
    a.playout = penalty_layout(vocabulary, slots); a.record = record;
    a.tokens = tokens; a.uniforms = uniforms; a.probs = probs; a.probs_stride = probs_stride; a.stats = stats;
    a.route_mask = route_mask == 0 ? uint32_t(VI_ROUTE_ALL) : route_mask;
    return launch_sample(a, workspace, workspace_bytes, as_stream(stream));
}

size_t vi_verify_workspace_bytes(int lanes, int drafts, int vocabulary) {
    if (lanes <= 0 || drafts <= 0 || vocabulary <= 0) return 0;
    return verify_workspace(lanes, drafts, vocabulary);
}

vi_status vi_verify_rows(int mode, const void* target, int target_dtype, int64_t target_stride, int target_rows,
                         const void* draft, int draft_dtype, int64_t draft_stride, int lanes, int drafts,
                         int vocabulary, const int32_t* drafted, const vi_row_params* params,
                         const int64_t* terminal, int n_terminal, int32_t* accepted, int32_t* committed,
                         int32_t* committed_count, uint32_t* lane_flags, void* workspace, size_t workspace_bytes,
                         void* stream) {
    if (lanes == 0) return VI_OK;
    if (lanes < 0 || drafts <= 0 || vocabulary <= 0 || (target_rows != drafts && target_rows != drafts + 1) ||
        !target || !dtype_ok(target_dtype) || target_stride < vocabulary || !drafted || !accepted || !committed ||
        !committed_count || n_terminal < 0 || (n_terminal && !terminal))
        return VI_ERR_INVALID;
    if (mode != VI_VERIFY_GREEDY && mode != VI_VERIFY_SAMPLED && mode != VI_VERIFY_SAMPLED_TOPK)
        return VI_ERR_INVALID;
    if (mode != VI_VERIFY_GREEDY &&
        (!draft || !dtype_ok(draft_dtype) || draft_stride < vocabulary || !params))
        return VI_ERR_INVALID;
    VerifyArgs a{};
    a.mode = mode; a.target = target; a.target_dtype = target_dtype; a.target_stride = target_stride;
    a.target_rows = target_rows; a.draft = draft; a.draft_dtype = draft_dtype; a.draft_stride = draft_stride;
    a.lanes = lanes; a.drafts = drafts; a.vocabulary = vocabulary; a.drafted = drafted; a.params = params;
    a.terminal = terminal; a.n_terminal = n_terminal; a.accepted = accepted; a.committed = committed;
    a.committed_count = committed_count; a.lane_flags = lane_flags;
    return launch_verify(a, workspace, workspace_bytes, as_stream(stream));
}

vi_status vi_probe_read(const void* src, size_t bytes, uint32_t* sink, void* stream) {
    if (!src || !sink || bytes % 16) return VI_ERR_INVALID;
    return launch_probe_read(src, bytes, sink, as_stream(stream));
}
vi_status vi_probe_copy(void* dst, const void* src, size_t bytes, void* stream) {
    if (!src || !dst || bytes % 16) return VI_ERR_INVALID;
    return launch_probe_copy(dst, src, bytes, as_stream(stream));
}

}  // extern "C"
