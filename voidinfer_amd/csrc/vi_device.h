// vi_device.h — device helpers shared by the gfx950 sampling kernels.
//
// Wave64 primitives (ballot / readlane / ds_bpermute / DPP), 16-byte row loads, the
// 16-bit order-preserving logit keys, Philox4x32-10, the SplitMix64/Gumbel
// noise of the coupled route, and the penalty arithmetic of the batched sampler.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/voidinfer_sampling.h"

#include <type_traits>

namespace vi {

constexpr int kWave = 64;
constexpr float kInfF = __builtin_huge_valf();

// ------------------------------------------------------------------ wave ops
__device__ __forceinline__ int lane_id() { return __lane_id(); }
__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ int readlane_i(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
// Value of lane (lane - 1); lane 0 gets its own value.  DPP wave_shr:1 (a VALU
// move across the whole wave; lane 0 keeps the `old` operand, its own value).
__device__ __forceinline__ int shift_up_i(int v) {
    return __builtin_amdgcn_update_dpp(v, v, 0x138, 0xf, 0xf, false);
}
__device__ __forceinline__ float shift_up_f(float v) {
    return __builtin_bit_cast(float, shift_up_i(__builtin_bit_cast(int, v)));
}

// (value desc, id asc): exl3_sampled_better (sampled_select.cuh:55-57).
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    // bitwise, not short-circuit: straight-line compares instead of exec-mask branches
    return (v > bv) | ((v == bv) & (i < bi));
}

// ------------------------------------------- hand-off between workgroups
// gfx950 has one L2 per XCD and the L2s are not coherent with one another, so an
// agent-scope release / acquire fence writes back and invalidates the whole L2
// of the XCD (buffer_wbl2 / buffer_inv), microseconds per workgroup.  Values one
// workgroup hands to another within a launch therefore travel as agent-scope
// atomic stores and loads (the compiler lowers those to accesses the L2 writes
// through and never serves from a stale line): the writer stores with put_agent,
// drains with handoff_stores_done (its stores acknowledged before the arrival
// read-modify-write that follows), and the reader, once that RMW has told it
// every writer arrived, reads with get_agent.
template <class T> __device__ __forceinline__ void put_agent(T* p, T v) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit values");
    using U = std::conditional_t<sizeof(T) == 4, uint32_t, uint64_t>;
    __hip_atomic_store(reinterpret_cast<U*>(p), __builtin_bit_cast(U, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T> __device__ __forceinline__ T get_agent(const T* p) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit values");
    using U = std::conditional_t<sizeof(T) == 4, uint32_t, uint64_t>;
    return __builtin_bit_cast(T, __hip_atomic_load(reinterpret_cast<const U*>(p), __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ void handoff_stores_done() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");   // no store is moved below (compiler)
    __builtin_amdgcn_s_waitcnt(0x0f70);                      // vmcnt(0): every store acknowledged
}
__device__ __forceinline__ void handoff_acquire() {
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");   // no load is moved above (compiler)
}

// --------------------------------------------------------------- element decode
template <int DT> struct Elem;
template <> struct Elem<VI_BF16> {
    using Bits = uint16_t;
    static constexpr int kPerVec = 8;
    __device__ static float decode(uint32_t b) { return __builtin_bit_cast(float, b << 16); }
    __device__ static bool finite_bits(uint32_t b) { return (b & 0x7f80u) != 0x7f80u; }
    __device__ static bool nan_bits(uint32_t b) { return (b & 0x7fffu) > 0x7f80u; }
    // order keys (key16) of the non-finite patterns: the 128 lowest and highest
    __device__ static bool nonfinite_key(uint32_t k) { return k < 0x80u || k >= 0xff80u; }
    // Round to nearest even (the hardware conversion v_cvt_pk_bf16_f32).
    __device__ static uint32_t round(float f) {
        return uint32_t(__builtin_bit_cast(uint16_t, static_cast<__bf16>(f)));
    }
};
template <> struct Elem<VI_F16> {
    using Bits = uint16_t;
    static constexpr int kPerVec = 8;
    __device__ static float decode(uint32_t b) {
        return float(__builtin_bit_cast(_Float16, uint16_t(b)));
    }
    __device__ static bool finite_bits(uint32_t b) { return (b & 0x7c00u) != 0x7c00u; }
    __device__ static bool nan_bits(uint32_t b) { return (b & 0x7fffu) > 0x7c00u; }
    // order keys (key16) of the non-finite patterns: the 1024 lowest and highest
    __device__ static bool nonfinite_key(uint32_t k) { return k < 0x400u || k >= 0xfc00u; }
    __device__ static uint32_t round(float f) {
        return uint32_t(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f)));
    }
};
template <> struct Elem<VI_F32> {
    using Bits = uint32_t;
    static constexpr int kPerVec = 4;
    __device__ static float decode(uint32_t b) { return __builtin_bit_cast(float, b); }
    __device__ static bool finite_bits(uint32_t b) { return (b & 0x7f800000u) != 0x7f800000u; }
    __device__ static bool nan_bits(uint32_t b) { return (b & 0x7fffffffu) > 0x7f800000u; }
    __device__ static uint32_t round(float f) { return __builtin_bit_cast(uint32_t, f); }
};

// Bits of element j (0..kPerVec-1) of a 16-byte vector.
template <int DT>
__device__ __forceinline__ uint32_t vec_bits(const uint4& v, int j) {
    if constexpr (DT == VI_F32) {
        return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
    } else {
        const uint32_t w = (j >> 1) == 0 ? v.x : (j >> 1) == 1 ? v.y : (j >> 1) == 2 ? v.z : v.w;
        return (j & 1) ? (w >> 16) : (w & 0xffffu);
    }
}

template <int DT>
__device__ __forceinline__ uint32_t load_bits(const void* row, int64_t i) {
    if constexpr (DT == VI_F32) return static_cast<const uint32_t*>(row)[i];
    else return static_cast<const uint16_t*>(row)[i];
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
// Streaming 16-byte load (non-temporal hint: logits are read once).
__device__ __forceinline__ uint4 load16(const void* p) {
    const u32x4_t v = __builtin_nontemporal_load(static_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
// Ordinary (cached) 16-byte load.
__device__ __forceinline__ uint4 load16_cached(const void* p) {
    const u32x4_t v = *static_cast<const u32x4_t*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 16-bit order-preserving key of a sign-magnitude bf16 / fp16 pattern; -0 and
// +0 share the key of +0.
__device__ __forceinline__ uint32_t key16(uint32_t b) {
    if (b == 0x8000u) b = 0;
    return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
}
__device__ __forceinline__ uint32_t unkey16(uint32_t k) {
    return (k & 0x8000u) ? (k & 0x7fffu) : (~k & 0xffffu);
}

// Any non-finite element in a 16-byte vector, from the raw words: adding the
// lowest exponent step to the magnitude carries into the sign position exactly
// when the exponent field is all ones (no carry crosses into the next element).
template <int DT>
__device__ __forceinline__ bool any_nonfinite(const uint4& v) {
    constexpr uint32_t M = DT == VI_F32 ? 0x7fffffffu : 0x7fff7fffu;
    constexpr uint32_t A = DT == VI_F32 ? 0x00800000u : (DT == VI_F16 ? 0x04000400u : 0x00800080u);
    constexpr uint32_t S = DT == VI_F32 ? 0x80000000u : 0x80008000u;
    const uint32_t t = ((v.x & M) + A) | ((v.y & M) + A) | ((v.z & M) + A) | ((v.w & M) + A);
    return (t & S) != 0u;
}

// ------------------------------------------------------------------ RNG
// SplitMix64 finalizer (sampled_select.cuh:41-46).
__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}
// Gumbel(0,1) of (seed, key, token) (sampled_select.cuh:47-54).
__device__ __forceinline__ float gumbel(uint64_t seed, int key, int token) {
    uint64_t h = splitmix64(seed ^ (uint64_t(uint32_t(key)) * 0xD1B54A32D192ED03ull));
    h = splitmix64(h ^ (uint64_t(uint32_t(token)) * 0x2545F4914F6CDD1Dull));
    const float u = (float(uint32_t(h >> 40)) + 0.5f) * (1.0f / 16777216.0f);
    return -logf(-logf(u));
}

// Philox4x32-10 (Salmon et al., SC'11); word order as rocRAND's engine.
__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        if (r) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        const uint32_t lo0 = 0xD2511F53u * c.x, hi0 = __umulhi(0xD2511F53u, c.x);
        const uint32_t lo1 = 0xCD9E8D57u * c.z, hi1 = __umulhi(0xCD9E8D57u, c.z);
        c = make_uint4(hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0);
    }
    return c;
}
// 53-bit uniform in [0,1) of (seed, lane, position, purpose); counter
// (position, 0, lane, purpose), key = seed.
__device__ __forceinline__ double philox_uniform(uint64_t seed, uint32_t lane, int32_t position,
                                                 uint32_t purpose) {
    const uint4 o = philox4x32_10(make_uint4(uint32_t(position), 0u, lane, purpose), uint32_t(seed),
                                  uint32_t(seed >> 32));
    const uint64_t m = (uint64_t(o.x) << 21) | uint64_t(o.y >> 11);
    return double(m) * 0x1p-53;
}

// ------------------------------------------------------------------ penalties
// Penalty of a history token with `count` occurrences (HF repetition, then
// OpenAI frequency and presence), fp32 without contraction, stored back in the
// logits' dtype (round to nearest even).  Returns the penalized bits.
template <int DT>
__device__ __forceinline__ uint32_t penalize_bits(uint32_t bits, uint32_t count, const vi_row_params& p) {
    // Separate roundings, as in the reference's CPU path: the library is built
    // with -ffp-contract=off, and the product and the difference stay apart.
#pragma clang fp contract(off)
    float y = Elem<DT>::decode(bits);
    if (p.repetition_penalty != 1.0f) y = (y > 0.0f) ? y / p.repetition_penalty : y * p.repetition_penalty;
    if (p.frequency_penalty != 0.0f) {
        const float t = p.frequency_penalty * float(count);
        y = y - t;
    }
    if (p.presence_penalty != 0.0f) y = y - p.presence_penalty;
    return Elem<DT>::round(y);
}
// penalize_bits with the division x / r done as Markstein's correction of
// x * (1/r): with inv = 1/r correctly rounded, q0 = RN(x * inv), the residual
// r0 = x - r * q0 exact by an FMA, and RN(q0 + r0 * inv) is the correctly
// rounded quotient when nothing underflows or overflows (P. Markstein, "IA-64
// and Elementary Functions", 2000, theorem 8.10) — so for |x| in [2^-100,
// 2^100] and r in [2^-20, 2^20] (rep_fast); other values take the IEEE
// division.  Three instructions in place of the division sequence on the
// common path; bit-exact against penalize_bits (tests/cpp/test_markstein.cpp).
template <int DT>
__device__ __forceinline__ uint32_t penalize_fast(uint32_t bits, uint32_t count, const vi_row_params& p, float inv,
                                                  bool rep_fast) {
#pragma clang fp contract(off)
    const float x = Elem<DT>::decode(bits);
    float y = x;
    if (p.repetition_penalty != 1.0f) {
        const float q0 = x * inv;
        const float r0 = fmaf(-q0, p.repetition_penalty, x);
        float q = fmaf(r0, inv, q0);
        const float ax = fabsf(x);
        if (x > 0.0f && !(rep_fast && ax >= 0x1p-100f && ax <= 0x1p100f)) q = x / p.repetition_penalty;
        y = x > 0.0f ? q : x * p.repetition_penalty;
    }
    if (p.frequency_penalty != 0.0f) {
        const float t = p.frequency_penalty * float(count);
        y = y - t;
    }
    if (p.presence_penalty != 0.0f) y = y - p.presence_penalty;
    return Elem<DT>::round(y);
}
// The reciprocal and the range condition penalize_fast takes, per row.
__device__ __forceinline__ float rep_inverse(const vi_row_params& p) { return 1.0f / p.repetition_penalty; }
__device__ __forceinline__ bool rep_fast_ok(const vi_row_params& p) {
    return p.repetition_penalty >= 0x1p-20f && p.repetition_penalty <= 0x1p20f;
}
__device__ __forceinline__ bool penalties_active(const vi_row_params& p) {
    return p.repetition_penalty != 1.0f || p.presence_penalty != 0.0f || p.frequency_penalty != 0.0f;
}
// Penalties can only lower a logit (so a raw value bounds the penalized one).
__device__ __forceinline__ bool penalties_lower_only(const vi_row_params& p) {
    return p.repetition_penalty >= 1.0f && p.presence_penalty >= 0.0f && p.frequency_penalty >= 0.0f;
}
// Count of `token` in a (token + 1, count) open-addressing hash with linear
// probing from (token * 0x9E3779B1) >> shift (0 if absent).
__device__ __forceinline__ uint32_t hash_count(const uint2* table, int shift, int slots, int token) {
    uint32_t s = (uint32_t(token) * 0x9E3779B1u) >> shift;
    for (int probe = 0; probe < slots; ++probe) {
        const uint2 e = table[s];
        if (e.x == uint32_t(token) + 1u) return e.y;
        if (e.x == 0u) return 0u;
        s = (s + 1u) & uint32_t(slots - 1);
    }
    return 0u;
}
// Rows served by the top-k kernel family: argmax rows and 1 <= top_k <= 64.
// Sampled verification from top-k lists needs 1 <= top_k <= 64 on a lane with
// temperature > 0; any other sampled lane is refused (VI_FLAG_ERROR).
__device__ __forceinline__ bool verify_list_refused(const vi_row_params& p) {
    return p.temperature > 0.0f && (p.top_k < 1 || p.top_k > 64);
}
// The list length the verification scan keeps for such a lane (1 when refused).
__device__ __forceinline__ int verify_list_k(const vi_row_params& p) {
    return verify_list_refused(p) ? 1 : p.top_k;
}
__device__ __forceinline__ bool topk_route(const vi_row_params& p) {
    return !(p.temperature > 0.0f) || (p.top_k >= 1 && p.top_k <= 64);
}

// ------------------------------------------------------------ DPP wave scans
// Inclusive prefix sums over the 64 lanes of a wave with DPP moves: row shifts
// 1, 2, 4, 8 inside each 16-lane row, then the row_bcast:15 / row_bcast:31
// carries between rows.  VALU-latency data movement, no LDS crossbar.
template <int kCtrl, int kRowMask, bool kBound>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), kCtrl, kRowMask, 0xf, kBound));
}
template <int kCtrl, int kRowMask, bool kBound>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint64_t r = uint64_t(dpp_u32<kCtrl, kRowMask, kBound>(uint32_t(b))) |
                       (uint64_t(dpp_u32<kCtrl, kRowMask, kBound>(uint32_t(b >> 32))) << 32);
    return __builtin_bit_cast(double, r);
}
// Lane exchanges through ds_bpermute: the LDS crossbar, off the VALU's issue
// slots (the kernels that use these are VALU-bound, so DPP or permlane forms of
// xor distances 4..32, which take several VALU instructions each, cost more).
__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, kWave); }
__device__ __forceinline__ int shfl_xor_i(int v, int m) { return __shfl_xor(v, m, kWave); }
__device__ __forceinline__ unsigned shfl_xor_u(unsigned v, int m) { return __shfl_xor(v, m, kWave); }
__device__ __forceinline__ double shfl_xor_d(double v, int m) { return __shfl_xor(v, m, kWave); }
// Value of lane 63 - lane.
__device__ __forceinline__ uint32_t lanes_reverse(uint32_t v) {
    return uint32_t(__builtin_amdgcn_ds_bpermute((kWave - 1 - lane_id()) << 2, int(v)));
}
// The same exchanges as VALU moves, for latency-bound chains of a single wave
// (no LDS round trip per stage): DPP quad and row patterns for xor distances
// up to 8 (row_half_mirror then a quad reversal gives lane ^ 4, row_ror:8
// gives lane ^ 8), gfx950's permlane swaps for 16 and 32 (with both operands
// the same register, the swap leaves lane ^ 16 (^ 32) in the first result on
// odd rows (the upper half) and in the second elsewhere).
template <int M> __device__ __forceinline__ uint32_t lanes_xor_dpp(uint32_t v) {
    static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "xor distance");
    if constexpr (M == 1) {
        return dpp_u32<0xb1, 0xf, false>(v);                              // quad_perm [1,0,3,2]
    } else if constexpr (M == 2) {
        return dpp_u32<0x4e, 0xf, false>(v);                              // quad_perm [2,3,0,1]
    } else if constexpr (M == 4) {
        return dpp_u32<0x1b, 0xf, false>(dpp_u32<0x141, 0xf, false>(v));  // lane ^ 7, then ^ 3
    } else if constexpr (M == 8) {
        return dpp_u32<0x128, 0xf, false>(v);                             // row_ror:8
    } else if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane_id() & 16) ? r[0] : r[1];
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (lane_id() & 32) ? r[0] : r[1];
    }
}
__device__ __forceinline__ uint32_t lanes_xor_dpp(uint32_t v, int m) {   // (folded when m is known)
    switch (m) {
        case 1: return lanes_xor_dpp<1>(v);
        case 2: return lanes_xor_dpp<2>(v);
        case 4: return lanes_xor_dpp<4>(v);
        case 8: return lanes_xor_dpp<8>(v);
        case 16: return lanes_xor_dpp<16>(v);
        case 32: return lanes_xor_dpp<32>(v);
        default: return uint32_t(__shfl_xor(int(v), m, kWave));
    }
}
__device__ __forceinline__ uint32_t lanes_reverse_dpp(uint32_t v) {   // row_mirror (^ 15), then ^ 16, ^ 32
    return lanes_xor_dpp<32>(lanes_xor_dpp<16>(dpp_u32<0x140, 0xf, false>(v)));
}
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t x) {
    x += dpp_u32<0x111, 0xf, true>(x);    // row_shr:1
    x += dpp_u32<0x112, 0xf, true>(x);    // row_shr:2
    x += dpp_u32<0x114, 0xf, true>(x);    // row_shr:4
    x += dpp_u32<0x118, 0xf, true>(x);    // row_shr:8
    x += dpp_u32<0x142, 0xa, false>(x);   // row_bcast:15 -> rows 1, 3
    x += dpp_u32<0x143, 0xc, false>(x);   // row_bcast:31 -> rows 2, 3
    return x;
}
__device__ __forceinline__ double wave_incl_scan_f64(double x) {
    x += dpp_f64<0x111, 0xf, true>(x);
    x += dpp_f64<0x112, 0xf, true>(x);
    x += dpp_f64<0x114, 0xf, true>(x);
    x += dpp_f64<0x118, 0xf, true>(x);
    x += dpp_f64<0x142, 0xa, false>(x);
    x += dpp_f64<0x143, 0xc, false>(x);
    return x;
}
// Sum over the wave in a fixed order (the scan's), returned in every lane.
__device__ __forceinline__ float wave_sum_f32(float x) {
    auto step = [](float v, auto dpp) { return v + __builtin_bit_cast(float, dpp(__builtin_bit_cast(uint32_t, v))); };
    x = step(x, [](uint32_t u) { return dpp_u32<0x111, 0xf, true>(u); });
    x = step(x, [](uint32_t u) { return dpp_u32<0x112, 0xf, true>(u); });
    x = step(x, [](uint32_t u) { return dpp_u32<0x114, 0xf, true>(u); });
    x = step(x, [](uint32_t u) { return dpp_u32<0x118, 0xf, true>(u); });
    x = step(x, [](uint32_t u) { return dpp_u32<0x142, 0xa, false>(u); });
    x = step(x, [](uint32_t u) { return dpp_u32<0x143, 0xc, false>(u); });
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), kWave - 1));
}
// Sum over the wave, returned in every lane.
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t x) {
    return uint32_t(__builtin_amdgcn_readlane(int(wave_incl_scan_u32(x)), kWave - 1));
}
__device__ __forceinline__ double wave_sum_f64(double x) {
    const uint64_t b = __builtin_bit_cast(uint64_t, wave_incl_scan_f64(x));
    const uint64_t r = uint64_t(uint32_t(__builtin_amdgcn_readlane(int(uint32_t(b)), kWave - 1))) |
                       (uint64_t(uint32_t(__builtin_amdgcn_readlane(int(uint32_t(b >> 32)), kWave - 1))) << 32);
    return __builtin_bit_cast(double, r);
}

// ------------------------------------------------------------------ block scan
// Exclusive prefix of a per-thread u32 over the block (blockDim.x = NT); `tmp`
// holds NT/64 + 1 words.  Returns the exclusive prefix; *total gets the sum.
template <int NT>
__device__ __forceinline__ uint32_t block_exclusive_scan_u32(uint32_t v, uint32_t* tmp, uint32_t* total) {
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    const uint32_t x = wave_incl_scan_u32(v);
    if (lane == kWave - 1) tmp[wave] = x;
    __syncthreads();
    if (wave == 0) {   // scan of the wave totals in wave 0
        const uint32_t t = lane < NT / kWave ? tmp[lane] : 0u;
        const uint32_t it = wave_incl_scan_u32(t);
        if (lane < NT / kWave) tmp[lane] = it - t;
        if (lane == NT / kWave - 1) tmp[NT / kWave] = it;
    }
    __syncthreads();
    const uint32_t r = tmp[wave] + x - v;
    *total = tmp[NT / kWave];
    __syncthreads();
    return r;
}

}  // namespace vi
