// transport.hip — greedy-packet readback: a pool of pinned host slots, each a
// buffer of packet rows with a completion event.  It stands in for the
// engine's per-context transfer pool (Exl3GreedyPacketTransfer,
// src/exl3/text_model.cu:779-900, used by submit_greedy_packet /
// finish_greedy_packet, :12225-12355) and for its cross-context batch
// (Exl3EngineGreedyPacketBatch, src/exl3/engine_greedy_packet_batch.h:17-60):
// because one vi_greedy_rows / vi_sampled_packet launch can write the rows of
// many lanes end to end, a batch is simply one submit of all of them — one
// device-to-host copy and one event for the whole decode step.
//
// Host code only.  Slot bookkeeping is under a mutex, so several engine threads
// may share a transport; a slot belongs to whoever submitted it until finish.
// A copy or wait that fails poisons its slot for the rest of the transport's
// life (the reference quarantines such a transfer).
#include <mutex>
#include <new>
#include <vector>

#include "vi_internal.h"

struct vi_packet_transport {
    struct Slot {
        vi_greedy_row* host = nullptr;   // pinned, max_rows rows
        hipEvent_t done = nullptr;
        int rows = 0;
        bool busy = false, poisoned = false;
    };
    std::mutex mu;
    std::vector<Slot> slots;
    int max_rows = 0;
};

namespace {

void release(vi_packet_transport* t) {
    for (auto& s : t->slots) {
        if (s.busy && s.done) (void)hipEventSynchronize(s.done);   // no copy may outlive its buffer
        if (s.done) (void)hipEventDestroy(s.done);
        if (s.host) (void)hipHostFree(s.host);
    }
    delete t;
}

}  // namespace

extern "C" {

vi_status vi_packet_transport_create(int slots, int max_rows, vi_packet_transport** out) {
    if (!out || slots <= 0 || slots > 1024 || max_rows <= 0 || max_rows > (1 << 20)) return VI_ERR_INVALID;
    *out = nullptr;
    auto* t = new (std::nothrow) vi_packet_transport;
    if (!t) return VI_ERR_UNSUPPORTED;
    t->max_rows = max_rows;
    t->slots.resize(size_t(slots));
    for (auto& s : t->slots) {
        if (hipHostMalloc(reinterpret_cast<void**>(&s.host), size_t(max_rows) * sizeof(vi_greedy_row),
                          hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&s.done, hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            release(t);
            return VI_ERR_DEVICE;
        }
    }
    *out = t;
    return VI_OK;
}

vi_status vi_packet_transport_destroy(vi_packet_transport* t) {
    if (!t) return VI_ERR_INVALID;
    release(t);
    return VI_OK;
}

vi_status vi_packet_submit(vi_packet_transport* t, const vi_greedy_row* device_rows, int rows, void* stream,
                           int* slot) {
    if (!t || !device_rows || !slot || rows <= 0 || rows > t->max_rows) return VI_ERR_INVALID;
    std::lock_guard<std::mutex> lock(t->mu);
    int k = -1;
    for (int i = 0; i < int(t->slots.size()); ++i)
        if (!t->slots[size_t(i)].busy && !t->slots[size_t(i)].poisoned) { k = i; break; }
    if (k < 0) return VI_ERR_WORKSPACE;   // every slot in flight (or poisoned)
    auto& s = t->slots[size_t(k)];
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (hipMemcpyAsync(s.host, device_rows, size_t(rows) * sizeof(vi_greedy_row), hipMemcpyDeviceToHost, st) !=
            hipSuccess ||
        hipEventRecord(s.done, st) != hipSuccess) {
        (void)hipGetLastError();
        s.poisoned = true;
        return VI_ERR_LAUNCH;
    }
    s.busy = true;
    s.rows = rows;
    *slot = k;
    return VI_OK;
}

vi_status vi_packet_query(vi_packet_transport* t, int slot, int* ready) {
    if (!t || !ready) return VI_ERR_INVALID;
    std::lock_guard<std::mutex> lock(t->mu);
    if (slot < 0 || slot >= int(t->slots.size()) || !t->slots[size_t(slot)].busy) return VI_ERR_INVALID;
    const hipError_t e = hipEventQuery(t->slots[size_t(slot)].done);
    if (e == hipSuccess) { *ready = 1; return VI_OK; }
    if (e == hipErrorNotReady) { (void)hipGetLastError(); *ready = 0; return VI_OK; }
    (void)hipGetLastError();
    t->slots[size_t(slot)].poisoned = true;
    return VI_ERR_LAUNCH;
}

vi_status vi_packet_finish(vi_packet_transport* t, int slot, vi_greedy_row* out, int rows) {
    if (!t || !out) return VI_ERR_INVALID;
    hipEvent_t done;
    const vi_greedy_row* host;
    {
        std::lock_guard<std::mutex> lock(t->mu);
        if (slot < 0 || slot >= int(t->slots.size())) return VI_ERR_INVALID;
        auto& s = t->slots[size_t(slot)];
        if (!s.busy || rows != s.rows) return VI_ERR_INVALID;
        done = s.done;
        host = s.host;
    }
    const bool ok = hipEventSynchronize(done) == hipSuccess;   // outside the lock: other slots stay usable
    std::lock_guard<std::mutex> lock(t->mu);
    auto& s = t->slots[size_t(slot)];
    s.busy = false;
    if (!ok) {
        (void)hipGetLastError();
        s.poisoned = true;
        return VI_ERR_LAUNCH;
    }
    for (int i = 0; i < rows; ++i) out[i] = host[i];
    return VI_OK;
}

}  // extern "C"
