// keys16.h — the 16-bit logit keys of the full-vocabulary routes: z of a key at
// a temperature, the valid key range, and a wave-parallel search over keys.
#pragma once

#include "vi_device.h"

namespace vi {

// Temperatures above this are refused by the 16-bit full routes: the pattern
// argument needs distinct fp32 products x * (1/T) for distinct patterns.
constexpr float kMaxTemperature = 65536.0f;

template <int DT>
__device__ __forceinline__ float key_z(uint32_t key, float inv_t) {
    return Elem<DT>::decode(unkey16(key)) * inv_t;
}

// Smallest i in [lo, hi) with pred(i) (pred monotone false -> true), or hi.
// Wave-uniform call; 64 probes per round.
template <class P>
__device__ __forceinline__ int wave_search(int lo, int hi, P pred) {
    const int lane = lane_id();
    while (hi > lo) {
        const int n = hi - lo;
        if (n <= kWave) {
            const uint64_t m = ballot(lane < n && pred(lo + lane));
            return m ? lo + __builtin_ctzll(m) : hi;
        }
        const int step = (n + kWave - 1) / kWave;
        const int p = lo + lane * step;
        const uint64_t valid = ballot(p < hi);
        const uint64_t m = ballot(p < hi && pred(p));
        if (!m) {
            const int last = 63 - __builtin_clzll(valid);
            lo = lo + last * step + 1;
            continue;
        }
        const int f = __builtin_ctzll(m);
        if (f == 0) return lo;
        const int nlo = lo + (f - 1) * step + 1;
        hi = lo + f * step;
        lo = nlo;
        if (lo == hi) return lo;
    }
    return lo;
}

// Smallest and largest valid keys (finite pattern, finite z) at a temperature,
// kmin | kmax << 16 (1 | 0 << 16: none); one wave.
template <int DT>
__device__ __forceinline__ uint32_t valid_key_range(float temperature) {
    constexpr int kPosMax = DT == VI_BF16 ? 0xff7f : 0xfbff;   // largest finite key
    constexpr int kNegMin = DT == VI_BF16 ? 0x0080 : 0x0400;   // smallest finite key
    const float inv_t = 1.0f / temperature;
    if (!(temperature <= kMaxTemperature) || !isfinite(inv_t)) return 1u;
    const int kbad = wave_search(0x8000, kPosMax + 1, [&](int key) { return !isfinite(key_z<DT>(uint32_t(key), inv_t)); });
    const int kgood = wave_search(kNegMin, 0x8000, [&](int key) { return isfinite(key_z<DT>(uint32_t(key), inv_t)); });
    return uint32_t(kgood) | (uint32_t(kbad - 1) << 16);
}

}  // namespace vi
