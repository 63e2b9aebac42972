// misc.hip — presence-table maintenance and the bandwidth probes.
//
// Presence table (src/exl3/sampled_select.h:29-35, text_model.cu:12139-12173):
// first_occurrence[token] is the first output position of each generated
// token, VI_ABSENT_OCCURRENCE otherwise.  reset marks every token absent;
// truncate drops occurrences at positions >= from; record enters tokens[i] at
// position first + i, keeping earlier occurrences (atomicMin).
//
// Probes: a stream-read kernel (16-byte loads, one word written per workgroup)
// and a plain copy, used to calibrate FETCH_SIZE / WRITE_SIZE and to report the
// sampler's bandwidth against a measured read rate.
#include "vi_device.h"
#include "vi_internal.h"

namespace vi {
namespace {

__global__ void presence_fill_kernel(int32_t* table, int vocabulary) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < vocabulary) table[i] = VI_ABSENT_OCCURRENCE;
}
__global__ void presence_truncate_kernel(int32_t* table, int vocabulary, int from) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < vocabulary && table[i] >= from) table[i] = VI_ABSENT_OCCURRENCE;
}
__global__ void presence_record_kernel(int32_t* table, int vocabulary, int first, const int64_t* tokens,
                                       size_t count) {
    for (size_t i = threadIdx.x; i < count; i += blockDim.x) {
        const int64_t t = tokens[i];
        if (t >= 0 && t < vocabulary) atomicMin(&table[t], first + int(i));
    }
}

__global__ __launch_bounds__(256) void probe_read_kernel(const uint4* src, size_t n16, uint32_t* sink) {
    uint32_t acc = 0;
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const uint4 a = load16(src + i), b = load16(src + i + stride);
        const uint4 c = load16(src + i + 2 * stride), d = load16(src + i + 3 * stride);
        acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
    }
    for (; i < n16; i += stride) { const uint4 a = load16(src + i); acc ^= a.x ^ a.y ^ a.z ^ a.w; }
    for (int o = 32; o; o >>= 1) acc ^= __shfl_xor(acc, o, kWave);
    if (threadIdx.x == 0) sink[blockIdx.x] = acc;
}

__global__ __launch_bounds__(256) void probe_copy_kernel(uint4* dst, const uint4* src, size_t n16) {
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride)
        dst[i] = load16(src + i);
}

}  // namespace

vi_status launch_presence_reset(int32_t* table, int vocabulary, hipStream_t stream) {
    hipLaunchKernelGGL(presence_fill_kernel, dim3((vocabulary + 255) / 256), dim3(256), 0, stream, table, vocabulary);
    return launch_status();
}
vi_status launch_presence_truncate(int32_t* table, int vocabulary, int from, hipStream_t stream) {
    hipLaunchKernelGGL(presence_truncate_kernel, dim3((vocabulary + 255) / 256), dim3(256), 0, stream, table,
                       vocabulary, from);
    return launch_status();
}
vi_status launch_presence_record(int32_t* table, int vocabulary, int first, const int64_t* tokens, size_t count,
                                 hipStream_t stream) {
    if (count == 0) return VI_OK;
    hipLaunchKernelGGL(presence_record_kernel, dim3(1), dim3(256), 0, stream, table, vocabulary, first, tokens, count);
    return launch_status();
}

vi_status launch_probe_read(const void* src, size_t bytes, uint32_t* sink, hipStream_t stream) {
    hipLaunchKernelGGL(probe_read_kernel, dim3(2048), dim3(256), 0, stream, static_cast<const uint4*>(src),
                       bytes / 16, sink);
    return launch_status();
}
vi_status launch_probe_copy(void* dst, const void* src, size_t bytes, hipStream_t stream) {
    hipLaunchKernelGGL(probe_copy_kernel, dim3(2048), dim3(256), 0, stream, static_cast<uint4*>(dst),
                       static_cast<const uint4*>(src), bytes / 16);
    return launch_status();
}

}  // namespace vi
