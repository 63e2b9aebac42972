// row_scan.h — the streaming loop shared by the slice kernels: each workgroup
// walks [begin, end) of one logit row with 16-byte loads (four in flight per
// thread) or, for rows whose stride breaks 16-byte alignment, with coalesced
// element loads.  `fn(bits, id, valid)` sees every element once; loop trip
// counts are wave-uniform (lanes past the end get valid = false), so callers may
// use cross-lane operations inside `fn`.  The visiting order is irrelevant to
// the callers (all of them reduce with order-free comparisons).
#pragma once

#include "vi_device.h"

namespace vi {

template <int DT, bool VEC, int NT, class F>
__device__ __forceinline__ void scan_slice(const void* row, int begin, int end, F&& fn) {
    constexpr int P = Elem<DT>::kPerVec;
    const int tid = threadIdx.x;
    if constexpr (VEC) {
        // begin is a multiple of 64 elements; full vectors first, then the tail.
        const int nvec = (end - begin) / P;
        const unsigned char* base = static_cast<const unsigned char*>(row) + size_t(begin) * (16 / P);
        constexpr int U = 4;
        for (int vb = 0; vb < nvec; vb += U * NT) {
            uint4 d[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int v = vb + u * NT + tid;
                d[u] = v < nvec ? load16(base + size_t(v) * 16) : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int v = vb + u * NT + tid;
                const bool ok = v < nvec;
#pragma unroll
                for (int j = 0; j < P; ++j) fn(vec_bits<DT>(d[u], j), begin + v * P + j, ok);
            }
        }
        for (int ib = begin + nvec * P; ib < end; ib += NT) {
            const int i = ib + tid;
            const bool ok = i < end;
            fn(ok ? load_bits<DT>(row, i) : 0u, i, ok);
        }
    } else {
        for (int ib = begin; ib < end; ib += NT) {
            const int i = ib + tid;
            const bool ok = i < end;
            fn(ok ? load_bits<DT>(row, i) : 0u, i, ok);
        }
    }
}

// As scan_slice, with each full 16-byte vector handed over whole:
// vfn(vector, id of its element 0, valid) for the vectors, fn(bits, id, valid)
// for the elements past the last full vector (and for every element of a row
// whose stride breaks 16-byte alignment).  first(vectors[4], valid[4]) sees the
// first batch once, after its loads and before vfn (the batch is peeled off the
// loop); it is not called when the slice has no full vector.  Same trip-count
// guarantees.
template <int DT, bool VEC, int NT, class FB, class FV, class F>
__device__ __forceinline__ void scan_slice_vec(const void* row, int begin, int end, FB&& first, FV&& vfn, F&& fn) {
    constexpr int P = Elem<DT>::kPerVec;
    const int tid = threadIdx.x;
    if constexpr (VEC) {
        const int nvec = (end - begin) / P;
        const unsigned char* base = static_cast<const unsigned char*>(row) + size_t(begin) * (16 / P);
        constexpr int U = 4;
        if (nvec > 0) {   // (uniform) the first batch
            uint4 d[U];
            bool okv[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int v = u * NT + tid;
                okv[u] = v < nvec;
                d[u] = okv[u] ? load16(base + size_t(v) * 16) : make_uint4(0, 0, 0, 0);
            }
            first(d, okv);
#pragma unroll
            for (int u = 0; u < U; ++u) vfn(d[u], begin + (u * NT + tid) * P, okv[u]);
        }
        for (int vb = U * NT; vb < nvec; vb += U * NT) {
            uint4 d[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int v = vb + u * NT + tid;
                d[u] = v < nvec ? load16(base + size_t(v) * 16) : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int v = vb + u * NT + tid;
                vfn(d[u], begin + v * P, v < nvec);
            }
        }
        for (int ib = begin + nvec * P; ib < end; ib += NT) {
            const int i = ib + tid;
            const bool ok = i < end;
            fn(ok ? load_bits<DT>(row, i) : 0u, i, ok);
        }
    } else {
        for (int ib = begin; ib < end; ib += NT) {
            const int i = ib + tid;
            const bool ok = i < end;
            fn(ok ? load_bits<DT>(row, i) : 0u, i, ok);
        }
    }
}

// As scan_slice_vec, with the U vectors of a thread's batch handed over
// together, bfn(vectors[U], first vector index of the batch, valid[U]) (vector
// u of the batch is number vb + u * NT + threadIdx.x of the slice), and the
// next batch's loads issued before the current batch is handed over (two
// register buffers), so the HBM stream keeps going while a batch is worked on.
// scan_slice_batches_from: the first batch's vectors already requested by the
// caller (pre, as loaded here: zeros past the slice's vectors) when use_pre.
template <int DT, bool VEC, int NT, class FB, class FBatch, class F>
__device__ __forceinline__ void scan_slice_batches_from(const void* row, int begin, int end, const uint4 (&pre)[4],
                                                        bool use_pre, FB&& first, FBatch&& bfn, F&& fn) {
    constexpr int P = Elem<DT>::kPerVec;
    constexpr int U = 4;
    const int tid = threadIdx.x;
    if constexpr (VEC) {
        const int nvec = (end - begin) / P;
        const unsigned char* base = static_cast<const unsigned char*>(row) + size_t(begin) * (16 / P);
        auto load = [&](int vb, uint4 (&d)[U], bool (&ok)[U]) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int v = vb + u * NT + tid;
                ok[u] = v < nvec;
                d[u] = ok[u] ? load16(base + size_t(v) * 16) : make_uint4(0, 0, 0, 0);
            }
        };
        if (nvec > 0) {   // (uniform)
            uint4 d[U];
            bool ok[U];
            if (use_pre) {
#pragma unroll
                for (int u = 0; u < U; ++u) { d[u] = pre[u]; ok[u] = u * NT + tid < nvec; }
            } else {
                load(0, d, ok);
            }
            first(d, ok);
            for (int vb = 0;; vb += U * NT) {
                const bool more = vb + U * NT < nvec;   // (uniform)
                uint4 nd[U];
                bool nok[U];
                if (more) {
                    load(vb + U * NT, nd, nok);
                } else {
#pragma unroll
                    for (int u = 0; u < U; ++u) { nd[u] = make_uint4(0, 0, 0, 0); nok[u] = false; }
                }
                bfn(d, vb, ok);
                if (!more) break;
#pragma unroll
                for (int u = 0; u < U; ++u) { d[u] = nd[u]; ok[u] = nok[u]; }
            }
        }
        for (int ib = begin + nvec * P; ib < end; ib += NT) {
            const int i = ib + tid;
            const bool ok = i < end;
            fn(ok ? load_bits<DT>(row, i) : 0u, i, ok);
        }
    } else {
        for (int ib = begin; ib < end; ib += NT) {
            const int i = ib + tid;
            const bool ok = i < end;
            fn(ok ? load_bits<DT>(row, i) : 0u, i, ok);
        }
    }
}

template <int DT, bool VEC, int NT, class FB, class FBatch, class F>
__device__ __forceinline__ void scan_slice_batches(const void* row, int begin, int end, FB&& first, FBatch&& bfn,
                                                   F&& fn) {
    const uint4 none[4] = {};
    scan_slice_batches_from<DT, VEC, NT>(row, begin, end, none, false, first, bfn, fn);
}

// Slice boundaries: slice s of `slices` covers [s*len, min(V,(s+1)*len)), len a
// multiple of 64 elements.
__host__ __device__ inline int slice_len_for(int vocabulary, int slices) {
    const int len = (vocabulary + slices - 1) / slices;
    return (len + 63) / 64 * 64;
}

}  // namespace vi
