// The samplers' division x / r (penalize_fast, voidinfer_amd/csrc/vi_device.h):
// q0 = RN(x * inv), r0 = RN(x - r * q0) by an FMA, q = RN(q0 + r0 * inv), with
// inv = RN(1 / r), taken for |x| in [2^-100, 2^100] and r in [2^-20, 2^20].
// Checked bit for bit against the IEEE division: every positive finite bf16 x
// in the range for 256 repetition penalties in [1, 1.5] and for 320 penalties
// spread over [2^-20, 2^20] (every fifth binade and its all-ones mantissa among
// them, the range's ends included), sampled x for 20,000 more penalties, and
// the fp32 x at and next to 2^-100 and 2^100 for all of them.  Built with
// -ffp-contract=off, as the library is.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

static float f_of(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

int main() {
    std::mt19937 rng(12345);
    long checked = 0, bad = 0;
    auto check = [&](float x, float rep, float inv) {
        if (!(std::fabs(x) >= 0x1p-100f && std::fabs(x) <= 0x1p100f)) return;
        volatile float xv = x, rv = rep;
        const float q_ieee = xv / rv;
        const float q0 = x * inv;
        const float r0 = std::fma(-q0, rep, x);
        const float q = std::fma(r0, inv, q0);
        ++checked;
        if (u_of(q) != u_of(q_ieee)) {
            if (bad < 5) std::printf("mismatch x=%a r=%a ieee=%a markstein=%a\n", x, rep, q_ieee, q);
            ++bad;
        }
    };
    // the penalties: [1, 1.5] densely, then the range's edges and structure
    // (2^-20 and 2^20 exactly, all-ones mantissas, every fifth binade), then
    // random ones over [2^-20, 2^20]
    std::vector<float> reps;
    for (int k = 0; k < 256; ++k)
        reps.push_back(1.0f + float(k) / 512.0f + std::uniform_real_distribution<float>(0.0f, 1.0f / 512.0f)(rng));
    const int n_full_a = int(reps.size());
    reps.push_back(0x1p-20f);
    reps.push_back(0x1p20f);
    for (int e = -20; e < 20; e += 5) {
        reps.push_back(std::ldexp(1.0f, e));
        reps.push_back(f_of(u_of(std::ldexp(1.0f, e)) | 0x7fffffu));   // just below the next power of two
        reps.push_back(f_of(u_of(std::ldexp(1.0f, e)) | 1u));          // just above this one
    }
    while (reps.size() < size_t(n_full_a + 320)) {
        const uint32_t m = rng() & 0x7fffffu, e = 127u - 20u + uint32_t(rng() % 40u);
        reps.push_back(f_of((e << 23) | m));
    }
    const int n_full = int(reps.size());
    for (int k = 0; k < 20000; ++k) {
        const uint32_t m = rng() & 0x7fffffu, e = 127u - 20u + uint32_t(rng() % 40u);
        reps.push_back(f_of((e << 23) | m));
    }
    // x at and next to the range's ends (fp32: the samplers' inputs are decoded
    // 16-bit patterns, but the condition is on the fp32 value)
    const float edges[] = {0x1p-100f, std::nextafter(0x1p-100f, 1.0f), 0x1p100f, std::nextafter(0x1p100f, 0.0f),
                           -0x1p-100f, -0x1p100f};
    for (size_t k = 0; k < reps.size(); ++k) {
        const float rep = reps[k];
        volatile float one = 1.0f, rv = rep;
        const float inv = one / rv;
        const uint32_t step = int(k) < n_full ? 1u : 97u;
        for (uint32_t b = 1; b < 0x7f80u; b += step) check(f_of(b << 16), rep, inv);
        for (const float x : edges) check(x, rep, inv);
    }
    std::printf("checked %ld quotients, %ld mismatches\n", checked, bad);
    return bad != 0;
}
