// The samplers' division x / r (penalize_fast, voidinfer_amd/csrc/vi_device.h):
// q0 = RN(x * inv), r0 = RN(x - r * q0) by an FMA, q = RN(q0 + r0 * inv), with
// inv = RN(1 / r), taken for |x| in [2^-100, 2^100] and r in [2^-20, 2^20].
// Checked bit for bit against the IEEE division: every positive finite bf16 x
// for 256 repetition penalties in [1, 1.5], and sampled x for 20,000 penalties
// spread over [2^-20, 2^20].  Built with -ffp-contract=off, as the library is.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>

static float f_of(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

int main() {
    std::mt19937 rng(12345);
    long checked = 0, bad = 0;
    for (int k = 0; k < 20256; ++k) {
        float rep;
        if (k < 256) {
            rep = 1.0f + float(k) / 512.0f + std::uniform_real_distribution<float>(0.0f, 1.0f / 512.0f)(rng);
        } else {
            const uint32_t m = rng() & 0x7fffffu, e = 127u - 20u + uint32_t(rng() % 41u);
            rep = f_of((e << 23) | m);
        }
        volatile float one = 1.0f, rv = rep;
        const float inv = one / rv;
        const uint32_t step = k < 256 ? 1u : 97u;
        for (uint32_t b = 1; b < 0x7f80u; b += step) {
            const float x = f_of(b << 16);
            if (!(std::fabs(x) >= 0x1p-100f && std::fabs(x) <= 0x1p100f)) continue;
            volatile float xv = x;
            const float q_ieee = xv / rv;
            const float q0 = x * inv;
            const float r0 = std::fma(-q0, rep, x);
            const float q = std::fma(r0, inv, q0);
            ++checked;
            if (u_of(q) != u_of(q_ieee)) {
                if (bad < 5) std::printf("mismatch x=%a r=%a ieee=%a markstein=%a\n", x, rep, q_ieee, q);
                ++bad;
            }
        }
    }
    std::printf("checked %ld quotients, %ld mismatches\n", checked, bad);
    return bad != 0;
}
