// penalty_state.h — device-side updates of a lane's penalty state (layout in
// vi_internal.h): shared by the update kernel and by the samplers, which can
// record each row's sampled token in its lane's state as they write it.
#pragma once

#include "vi_device.h"
#include "vi_internal.h"

namespace vi {

struct LaneState {
    PenaltyHeader* hdr;
    uint32_t* b1;
    uint2* table;
    uint32_t* ridx;
    uint2* list;
};

__device__ __forceinline__ LaneState lane_state(unsigned char* st, const PenaltyLayout& l) {
    return LaneState{reinterpret_cast<PenaltyHeader*>(st), reinterpret_cast<uint32_t*>(st + l.off_b1),
                     reinterpret_cast<uint2*>(st + l.off_hash), reinterpret_cast<uint32_t*>(st + l.off_ridx),
                     reinterpret_cast<uint2*>(st + l.off_list)};
}

__device__ __forceinline__ uint32_t load_agent(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Phase 1 for token t; returns its slot, or -1 (ignored token / failure, flagged).
__device__ inline int state_apply(const LaneState& s, const PenaltyLayout& l, int vocabulary, int32_t t, int sign) {
    if (t < 0 || t >= vocabulary) {
        atomicOr(&s.hdr->flags, uint32_t(VI_FLAG_BAD_HISTORY));
        return -1;
    }
    const uint32_t key = uint32_t(t) + 1u, bit = 1u << (t & 31);
    uint32_t slot = (uint32_t(t) * 0x9E3779B1u) >> l.shift;
    for (int probe = 0; probe < l.slots; ++probe) {
        uint32_t k = load_agent(&s.table[slot].x);
        if (k == 0u) {
            if (sign < 0) break;   // not recorded
            k = atomicCAS(&s.table[slot].x, 0u, key);
            if (k == 0u) {
                atomicAdd(&s.hdr->keys, 1u);
                k = key;
            }
        }
        if (k == key) {
            if (sign > 0) {
                const uint32_t old = atomicAdd(&s.table[slot].y, 1u);
                if (old == 0u) atomicOr(&s.b1[t >> 5], bit);
                if (old == 1u && load_agent(&s.ridx[slot]) == 0u) {   // first repeat since the reset
                    const uint32_t idx = atomicAdd(&s.hdr->nrep, 1u);
                    s.list[idx] = make_uint2(uint32_t(t), 2u);   // (idx < slots: one entry per slot)
                    __hip_atomic_store(&s.ridx[slot], idx + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                atomicAdd(reinterpret_cast<unsigned long long*>(&s.hdr->total), 1ull);
            } else {
                uint32_t c = load_agent(&s.table[slot].y);
                for (;;) {
                    if (c == 0u) {   // removed more often than recorded
                        atomicOr(&s.hdr->flags, uint32_t(VI_FLAG_ERROR));
                        return -1;
                    }
                    const uint32_t prev = atomicCAS(&s.table[slot].y, c, c - 1u);
                    if (prev == c) break;
                    c = prev;
                }
                if (c == 1u) atomicAnd(&s.b1[t >> 5], ~bit);
                atomicAdd(reinterpret_cast<unsigned long long*>(&s.hdr->total), ~0ull);
            }
            return int(slot);
        }
        slot = (slot + 1u) & uint32_t(l.slots - 1);
    }
    // recording into a full table, or removing a token never recorded: the
    // state no longer describes a history, and every row sampled from it fails
    atomicOr(&s.hdr->flags, uint32_t(VI_FLAG_ERROR));
    return -1;
}

// Phase 2: the slot's final count into its repeat-list entry, if it has one.
__device__ __forceinline__ void state_publish(const LaneState& s, int slot) {
    if (slot < 0) return;
    const uint32_t r = load_agent(&s.ridx[slot]);
    if (r) __hip_atomic_store(&s.list[r - 1u].y, load_agent(&s.table[slot].y), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
}

// A sampler recording its row's token: the one writer of the lane's state in
// its launch, after every read of it.  Plain loads, issued together (the
// first probe's entry and repeat index, the presence word, the header), then
// plain stores: the state_apply(+1) / state_publish result without their
// chain of returning atomics.
__device__ inline void state_record_one(const LaneState& s, const PenaltyLayout& l, int vocabulary, int32_t t) {
    if (t < 0 || t >= vocabulary) {
        s.hdr->flags |= uint32_t(VI_FLAG_BAD_HISTORY);
        return;
    }
    const uint32_t key = uint32_t(t) + 1u, bit = 1u << (t & 31);
    uint32_t slot = (uint32_t(t) * 0x9E3779B1u) >> l.shift;
    uint2 e = s.table[slot];
    uint32_t ridx = s.ridx[slot];
    const uint32_t word = s.b1[t >> 5];
    uint32_t keys = s.hdr->keys, nrep = s.hdr->nrep;
    const uint64_t total = s.hdr->total;
    for (int probe = 1; e.x != 0u && e.x != key; ++probe) {   // (collisions: rare)
        if (probe >= l.slots) {
            s.hdr->flags |= uint32_t(VI_FLAG_ERROR);
            return;
        }
        slot = (slot + 1u) & uint32_t(l.slots - 1);
        e = s.table[slot];
        ridx = s.ridx[slot];
    }
    if (e.x == 0u) {
        s.table[slot].x = key;
        s.hdr->keys = keys + 1u;
    }
    const uint32_t old = e.y;
    s.table[slot].y = old + 1u;
    if (old == 0u) s.b1[t >> 5] = word | bit;
    if (old == 1u && ridx == 0u) {   // first repeat since the reset
        s.list[nrep] = make_uint2(uint32_t(t), 2u);
        s.ridx[slot] = nrep + 1u;
        s.hdr->nrep = nrep + 1u;
    } else if (ridx) {
        s.list[ridx - 1u].y = old + 1u;
    }
    s.hdr->total = total + 1u;
}

}  // namespace vi
