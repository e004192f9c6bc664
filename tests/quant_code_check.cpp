// Host check of wq::quant_code and wq::quant_word (four codes packed) in
// webyiq_amd/csrc/quant_code.hpp, the division-free int8 code of the
// activation quantisers, against its
// definition rint(v / d) with an IEEE float32 quotient.  Built with g++ by
// tests/test_quant_code.py.  Inputs are shaped as the quantisers produce
// them: d = amax / 127 over scales from subnormal to 2^100, |v| <= amax;
// random v plus v within 16 ulps of every half-integer boundary (k + 0.5) d,
// where the fast path must hand over to the exact quotient.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <random>

#include "quant_code.hpp"

int main() {
    std::mt19937_64 gen(20261201);
    std::uniform_real_distribution<float> unit(-1.0f, 1.0f), mant(1.0f, 2.0f);
    std::uniform_int_distribution<int> expo(-140, 100);
    long n = 0, bad = 0, near = 0;
    float ring[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto check = [&](float v, float d, float rd) {
        const int want = (int)rintf(v / d);
        const int got = wq::quant_code(v, d, rd);
        ++n;
        if (got != want) {
            if (bad < 10) std::printf("mismatch v=%a d=%a got=%d want=%d\n", v, d, got, want);
            ++bad;
        }
        // quant_word over this value and the three before it (same d)
        ring[n & 3] = v;
        const uint32_t w = wq::quant_word(ring[0], ring[1], ring[2], ring[3], d, rd);
        for (int b = 0; b < 4; ++b) {
            const int8_t code = (int8_t)((w >> (8 * b)) & 0xFFu);
            if (code != (int8_t)(int)rintf(ring[b] / d)) {
                if (bad < 10) std::printf("word mismatch v=%a d=%a byte %d\n", ring[b], d, b);
                ++bad;
            }
        }
    };
    for (int i = 0; i < 3000; ++i) {
        const float amax = std::ldexp(mant(gen), expo(gen));
        const float d = amax / 127.0f;
        if (!(d > 0.0f)) continue;
        const float rd = 1.0f / d;
        for (float& r : ring) r = 0.0f;
        check(amax, d, rd);
        check(-amax, d, rd);
        for (int j = 0; j < 400; ++j) check(unit(gen) * amax, d, rd);
        for (int k = -128; k <= 127; ++k) {
            float h = ((float)k + 0.5f) * d;
            for (int s = 0; s < 16; ++s) h = std::nextafter(h, -INFINITY);
            for (int s = 0; s < 33; ++s, h = std::nextafter(h, INFINITY)) {
                if (std::fabs(h) > amax) continue;
                ++near;
                check(h, d, rd);
            }
        }
    }
    std::printf("checked %ld (%ld near a half-integer) mismatches %ld\n", n, near, bad);
    return bad != 0;
}
