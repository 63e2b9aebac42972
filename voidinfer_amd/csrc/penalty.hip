// penalty.hip — per-lane penalty state: a presence bitmap, a token -> count
// hash and a repeat list of the tokens seen at least twice, kept current as
// tokens are recorded (sampled, drafted) or removed (rolled back).  The
// sampler reads it in place of the lane's history: the same penalties, without
// a scan of the history at every step.  It generalizes the reference's
// incremental first-occurrence table (exl3_presence_reset / truncate / record,
// src/exl3/text_model.cu:12139-12173, kept current by PresenceTrack::sync,
// src/exl3/exl3_engine_core.cpp:106-133) from presence to occurrence counts,
// which repetition and frequency penalties need.
//
// One workgroup per lane, two phases.  Phase 1 is lock-free: a token's slot is
// claimed with a CAS on its key, its count moves with atomics, the thread that
// takes a count from 0 to 1 sets the presence bit (1 -> 0 clears it), and the
// thread that takes a count from 1 to 2 for the first time since the reset
// appends the token to the repeat list.  After a workgroup barrier, phase 2
// copies each touched token's final count into its repeat-list entry (every
// writer of an entry writes the same value).  One call either records or
// removes, so the two never race.  A removed token keeps its slot (count 0):
// probe chains stay intact and a later record reuses it.
#include <algorithm>

#include "penalty_state.h"

namespace vi {
namespace {

constexpr int kUpdThreads = 256;

constexpr int kPerThread = 8;   // tokens a thread keeps slots for between the phases

__global__ __launch_bounds__(kUpdThreads) void state_update_kernel(unsigned char* states, PenaltyLayout l, int vocabulary,
                                                                    const int32_t* tokens, const int64_t* offsets,
                                                                    int sign) {
    const int lane = blockIdx.x;
    const LaneState s = lane_state(states + size_t(lane) * l.lane_bytes, l);
    if (!offsets) {   // one token per lane; a negative token (a row that failed) records nothing
        if (threadIdx.x == 0 && tokens[lane] >= 0) state_publish(s, state_apply(s, l, vocabulary, tokens[lane], sign));
        return;
    }
    const int64_t b = offsets[lane], e = offsets[lane + 1];
    // rounds of kPerThread tokens per thread: apply, barrier, publish
    for (int64_t base = b; base < e; base += int64_t(kUpdThreads) * kPerThread) {
        int slot[kPerThread];
#pragma unroll
        for (int j = 0; j < kPerThread; ++j) {
            const int64_t i = base + int64_t(j) * kUpdThreads + threadIdx.x;
            slot[j] = i < e ? state_apply(s, l, vocabulary, tokens[i], sign) : -1;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kPerThread; ++j) state_publish(s, slot[j]);
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void state_fill_kernel(uint4* dst, size_t n16) {
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = make_uint4(0, 0, 0, 0);
}

}  // namespace

vi_status launch_penalty_reset(void* states, int lanes, const PenaltyLayout& l, hipStream_t stream) {
    const size_t n16 = size_t(lanes) * l.lane_bytes / 16;
    const unsigned blocks = unsigned(std::min<size_t>((n16 + 255) / 256, 4096));
    hipLaunchKernelGGL(state_fill_kernel, dim3(blocks), dim3(256), 0, stream, static_cast<uint4*>(states), n16);
    return launch_status();
}

vi_status launch_penalty_update(void* states, int lanes, int vocabulary, const PenaltyLayout& l, const int32_t* tokens,
                                const int64_t* offsets, int sign, hipStream_t stream) {
    hipLaunchKernelGGL(state_update_kernel, dim3(lanes), dim3(kUpdThreads), 0, stream,
                       static_cast<unsigned char*>(states), l, vocabulary, tokens, offsets, sign);
    return launch_status();
}

}  // namespace vi
