// greedy.hip — greedy argmax rows (the gfx950 replacement of
// exl3_greedy_packet_{,wide_,split_}kernel, src/exl3/greedy_packet.cuh:15-246).
//
// Semantics (greedy_packet.cuh:12-14): per row, the largest finite value with
// the lowest index on ties; non-finite values are skipped and flagged; index =
// vocabulary when no value is finite.  Only comparisons, so the partition of the
// row into slices cannot change the answer.
//
// Shape: grid (slices, rows), 256 threads.  Each workgroup reduces one slice of
// one row (16-byte loads, wave64 xor-shuffle reduction, 4-wave LDS reduction);
// with more than one slice the last workgroup of a row to arrive (self-resetting
// arrival counter, as greedy_packet.cuh:139-246) reduces the slice partials in
// slice order.  Roofline: HBM, V x sizeof(logit) bytes per row.
//
// Row-score variant (SCORE = true; exact_row_score_kernel,
// src/exl3/text_model.cu:11393-11420, the VeriCache exact route): candidates
// are the values that compare greater than -Inf (NaN and -Inf never win, +Inf
// can), nothing is flagged, and the row's writer also emits the gap
// max - logit(next[r]) for a next in [0, V) other than the argmax (else 0).
#include <algorithm>
#include <mutex>

#include "row_scan.h"

#include "vi_internal.h"

namespace vi {
namespace {

constexpr int kGreedyThreads = 256;

struct GreedyPartial {
    float best;
    int index;
    uint32_t bad;
    uint32_t pad;
};

__device__ __forceinline__ void greedy_combine(float& best, int& index, float ob, int oi) {
    if (ob > best || (ob == best && oi < index)) { best = ob; index = oi; }
}

// Writes row r's result (one thread).
template <int DT, bool SCORE>
__device__ __forceinline__ void greedy_write(const void* row, int r, int vocabulary, float best, int index, bool bad,
                                             uint64_t serial, vi_greedy_row* out, const int64_t* next,
                                             int64_t* greedy, float* gap) {
    if constexpr (SCORE) {
        greedy[r] = index;
        const int64_t t = next[r];
        float g = 0.0f;
        if (t >= 0 && t < vocabulary && t != index)
            g = best - Elem<DT>::decode(static_cast<const typename Elem<DT>::Bits*>(row)[t]);
        gap[r] = g;
    } else {
        out[r].serial = serial; out[r].token = index; out[r].nonfinite = bad ? 1u : 0u;
    }
}

template <int DT, bool VEC, bool SCORE>
__global__ __launch_bounds__(kGreedyThreads) void greedy_kernel(
    const void* logits, int vocabulary, int64_t stride, int slice_len, uint64_t serial,
    vi_greedy_row* out, GreedyPartial* partials, uint32_t* arrivals, const int64_t* next, int64_t* greedy,
    float* gap) {
    const int slice = blockIdx.x, slices = gridDim.x, r = blockIdx.y;
    const void* row = static_cast<const unsigned char*>(logits) + size_t(r) * size_t(stride) * sizeof(typename Elem<DT>::Bits);
    const int begin = slice * slice_len, end = min(vocabulary, begin + slice_len);
    float best = -kInfF;
    int index = vocabulary;
    bool bad = false;
    auto elem = [&](uint32_t bits, int id, bool ok) {
        if (!ok) return;
        const float x = Elem<DT>::decode(bits);
        if constexpr (SCORE) {
            if (!(x > -kInfF)) return;
        } else {
            if (!Elem<DT>::finite_bits(bits)) { bad = true; return; }
        }
        if (x > best || (x == best && id < index)) { best = x; index = id; }
    };
    // Whole vectors: a thread visits its elements in increasing id order, so
    // within a vector free of non-finite values the first maximum is taken only
    // if it beats the running best strictly; a vector holding one goes element
    // by element.
    scan_slice_vec<DT, VEC, kGreedyThreads>(
        row, begin, end, [](const auto&, const auto&) {},
        [&](const uint4& dv, int id0, bool ok) {
            constexpr int P = Elem<DT>::kPerVec;
            if (!ok) return;
            if (any_nonfinite<DT>(dv)) {
#pragma unroll
                for (int j = 0; j < P; ++j) elem(vec_bits<DT>(dv, j), id0 + j, true);
                return;
            }
            float xs[P];
            float vmax = -kInfF;
#pragma unroll
            for (int j = 0; j < P; ++j) {
                xs[j] = Elem<DT>::decode(vec_bits<DT>(dv, j));
                vmax = fmaxf(vmax, xs[j]);
            }
            if (vmax > best) {
                int jj = P - 1;
#pragma unroll
                for (int j = P - 2; j >= 0; --j) jj = xs[j] == vmax ? j : jj;
                best = xs[jj];   // (the element's own value: +0 and -0 compare equal)
                index = id0 + jj;
            }
        },
        elem);
#pragma unroll
    for (int o = 32; o; o >>= 1) greedy_combine(best, index, shfl_xor_f(best, o), shfl_xor_i(index, o));
    const bool wave_bad = ballot(bad) != 0;
    __shared__ float s_best[kGreedyThreads / kWave];
    __shared__ int s_index[kGreedyThreads / kWave];
    __shared__ uint32_t s_bad[kGreedyThreads / kWave];
    __shared__ bool s_last;
    const int wave = threadIdx.x / kWave, lane = lane_id();
    if (lane == 0) { s_best[wave] = best; s_index[wave] = index; s_bad[wave] = wave_bad; }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t b = 0;
        for (int w = 0; w < kGreedyThreads / kWave; ++w) { greedy_combine(best, index, s_best[w], s_index[w]); b |= s_bad[w]; }
        if (slices == 1) {
            greedy_write<DT, SCORE>(row, r, vocabulary, best, index, b != 0, serial, out, next, greedy, gap);
            return;
        }
        GreedyPartial& p = partials[size_t(r) * slices + slice];
        put_agent(&p.best, best); put_agent(&p.index, index); put_agent(&p.bad, b);
        handoff_stores_done();
        s_last = atomicAdd(&arrivals[r], 1u) == uint32_t(slices - 1);
    }
    if (slices == 1) return;
    __syncthreads();
    if (!s_last || wave != 0) return;
    handoff_acquire();
    best = -kInfF; index = vocabulary;
    uint32_t b = 0;
    for (int s = lane; s < slices; s += kWave) {
        const GreedyPartial& p = partials[size_t(r) * slices + s];
        greedy_combine(best, index, get_agent(&p.best), get_agent(&p.index));
        b |= get_agent(&p.bad);
    }
#pragma unroll
    for (int o = 32; o; o >>= 1) greedy_combine(best, index, shfl_xor_f(best, o), shfl_xor_i(index, o));
    const bool any_bad = ballot(b != 0) != 0;
    if (lane == 0) {
        arrivals[r] = 0u;
        greedy_write<DT, SCORE>(row, r, vocabulary, best, index, any_bad, serial, out, next, greedy, gap);
    }
}

}  // namespace

GreedyPlan greedy_plan(int rows, int vocabulary) {
    // Aim for >= 1024 workgroups (4 per CU) with slices of >= 4096 logits.
    int slices = rows >= 1024 ? 1 : (1024 + rows - 1) / rows;
    slices = std::min(slices, std::max(1, vocabulary / 4096));
    slices = std::max(1, std::min(slices, 128));
    const int len = slice_len_for(vocabulary, slices);
    slices = (vocabulary + len - 1) / len;
    return {slices, len};
}

size_t greedy_workspace(int rows, int vocabulary) {
    const GreedyPlan p = greedy_plan(rows, vocabulary);
    if (p.slices == 1) return 0;
    return align_up(size_t(rows) * 4, 256) + align_up(size_t(rows) * p.slices * sizeof(GreedyPartial), 256);
}

namespace {

template <bool SCORE>
vi_status launch_greedy_kind(const void* logits, int dtype, int rows, int vocabulary, int64_t stride,
                             uint64_t serial, vi_greedy_row* out, const int64_t* next, int64_t* greedy, float* gap,
                             void* ws, size_t ws_bytes, int arrival_rows, hipStream_t stream) {
    const GreedyPlan p = greedy_plan(rows, vocabulary);
    GreedyPartial* partials = nullptr;
    uint32_t* arrivals = nullptr;
    if (p.slices > 1) {
        // The arrival counters come first, as many as the workspace was carved
        // for (arrival_rows >= rows): a launch over fewer rows of a workspace
        // carved for more (verification without its bonus row) finds them where
        // the kernels left them, at zero, and no partials of a smaller launch
        // lie under them.
        Carver c(ws, ws_bytes);
        arrivals = c.take<uint32_t>(size_t(std::max(rows, arrival_rows)));
        partials = c.take<GreedyPartial>(size_t(rows) * p.slices);
        if (!c.ok) return VI_ERR_WORKSPACE;
    }
    const bool vec = (reinterpret_cast<uintptr_t>(logits) % 16 == 0) && ((stride * elem_size(dtype)) % 16 == 0);
    const dim3 grid(p.slices, rows), block(kGreedyThreads);
#define VI_GREEDY_LAUNCH(DT, V)                                                                          \
    hipLaunchKernelGGL((greedy_kernel<DT, V, SCORE>), grid, block, 0, stream, logits, vocabulary, stride, \
                       p.slice_len, serial, out, partials, arrivals, next, greedy, gap)
    switch (dtype) {
        case VI_BF16: if (vec) VI_GREEDY_LAUNCH(VI_BF16, true); else VI_GREEDY_LAUNCH(VI_BF16, false); break;
        case VI_F16: if (vec) VI_GREEDY_LAUNCH(VI_F16, true); else VI_GREEDY_LAUNCH(VI_F16, false); break;
        default: if (vec) VI_GREEDY_LAUNCH(VI_F32, true); else VI_GREEDY_LAUNCH(VI_F32, false); break;
    }
#undef VI_GREEDY_LAUNCH
    return launch_status();
}

}  // namespace

vi_status launch_greedy(const void* logits, int dtype, int rows, int vocabulary, int64_t stride,
                        uint64_t serial, vi_greedy_row* out, void* ws, size_t ws_bytes,
                        hipStream_t stream, int arrival_rows) {
    return launch_greedy_kind<false>(logits, dtype, rows, vocabulary, stride, serial, out, nullptr, nullptr, nullptr,
                                     ws, ws_bytes, arrival_rows, stream);
}

// ---- allocation-free greedy (vi_greedy_rows_noalloc) ---------------------------
// The slice partials and arrival counters live in a file-scope device array
// instead of a caller workspace.  Every GPU the library runs on holds its own
// copy until the process ends; host code never passes `scratch` itself to a
// kernel (its host-side name is not a device address) but the per-device address
// that hipGetSymbolAddress returned, looked up once per device.
static __device__ __align__(256) unsigned char scratch[kGreedyScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

__global__ void zero_words_kernel(uint32_t* words, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) words[i] = 0u;
}

}  // namespace

vi_status greedy_scratch_setup(void** ptr) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return VI_ERR_DEVICE;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return VI_ERR_DEVICE;
        g_scratch_ptr[dev] = p;
    }
    if (ptr) *ptr = g_scratch_ptr[dev];
    return VI_OK;
}

vi_status launch_greedy_noalloc(const void* logits, int dtype, int rows, int vocabulary, int64_t stride,
                                uint64_t serial, vi_greedy_row* out, hipStream_t stream) {
    const size_t need = greedy_workspace(rows, vocabulary);
    if (need > kGreedyScratchBytes) return VI_ERR_WORKSPACE;
    void* ws = nullptr;
    const vi_status st = greedy_scratch_setup(&ws);
    if (st != VI_OK) return st;
    if (need > 0) {
        // The arrival counters (the first rows words) must start at zero; an
        // earlier call of more rows left its own partials past them.
        uint32_t* arrivals = static_cast<uint32_t*>(ws);
        hipLaunchKernelGGL(zero_words_kernel, dim3((rows + 255) / 256), dim3(256), 0, stream, arrivals, rows);
        if (launch_status() != VI_OK) return VI_ERR_LAUNCH;
    }
    return launch_greedy_kind<false>(logits, dtype, rows, vocabulary, stride, serial, out, nullptr, nullptr, nullptr,
                                     ws, kGreedyScratchBytes, rows, stream);
}

vi_status launch_row_scores(const void* logits, int dtype, int rows, int vocabulary, int64_t stride,
                            const int64_t* next, int64_t* greedy, float* gap, void* ws, size_t ws_bytes,
                            hipStream_t stream) {
    return launch_greedy_kind<true>(logits, dtype, rows, vocabulary, stride, 0, nullptr, next, greedy, gap, ws,
                                    ws_bytes, rows, stream);
}

}  // namespace vi
