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
vi_status launch_greedy(const void* logits, int dtype, int rows, int vocabulary, int64_t stride,
                        uint64_t serial, vi_greedy_row* out, void* ws, size_t ws_bytes,
                        hipStream_t stream);
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

// Sorted, filtered top-k lists (z values, ids) of verification rows.
vi_status launch_verify_lists(const void* logits, int dtype, int rows, int layout_rows, int layout_slices,
                              int vocabulary, int64_t stride, const vi_row_params* params, int params_div,
                              float* lval, int* lidx, uint32_t* lvalid, uint32_t* lflags, void* ws,
                              size_t ws_bytes, hipStream_t stream);
size_t topk_partials_bytes_slices(int rows, int slices);

// History hash (token -> count) per row for the top-k sampler route.
size_t history_hash_slots(int64_t max_history);

struct SampleArgs {
    const void* logits;
    int dtype, rows, vocabulary;
    int64_t stride;
    const vi_row_params* params;
    const int32_t* histories;
    const int64_t* offsets;
    int64_t max_history;
    int32_t* tokens;
    double* uniforms;
    float* probs;
    int64_t probs_stride;
    vi_sample_stats* stats;
    uint32_t route_mask;
};
size_t sample_workspace(int rows, int vocabulary, int64_t max_history);
vi_status launch_sample(const SampleArgs& a, void* ws, size_t ws_bytes, hipStream_t stream);

// ---- full-vocabulary pair kernel --------------------------------------------
size_t full_workspace(int rows);
vi_status launch_full(const SampleArgs& a, unsigned char* ws, size_t ws_bytes, hipStream_t stream);
bool full_supported(int dtype, int vocabulary, int64_t stride);

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
vi_status launch_presence_reset(int32_t* table, int vocabulary, hipStream_t stream);
vi_status launch_presence_truncate(int32_t* table, int vocabulary, int from, hipStream_t stream);
vi_status launch_presence_record(int32_t* table, int vocabulary, int first, const int64_t* tokens,
                                 size_t count, hipStream_t stream);

inline vi_status launch_status() {
    return hipGetLastError() == hipSuccess ? VI_OK : VI_ERR_LAUNCH;
}

}  // namespace vi
