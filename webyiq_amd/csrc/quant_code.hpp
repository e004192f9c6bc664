// int8 code of the activation quantiser, shared by the device kernels and a
// host-compiled exhaustive check (tests/test_quant_code.py builds it with g++).
#pragma once
#include <cmath>
#include <cstdint>

#ifndef WQ_HD
#define WQ_HD __host__ __device__
#endif

namespace wq {

// rint(v / d) with v / d the IEEE quotient, without a division on the common
// path; rd = 1 / d (IEEE), d > 0, |v| <= 127 d (|v / d| < 128).
// a = v * rd is within 2^-23 relative (<= 1.6e-5 absolute) of v / d and the
// IEEE quotient within 0.5 ulp (<= 3.9e-6), so both round to the same integer
// unless v * rd (exact, by the fma) lies within 2^-13 of a half-integer; only
// then (or when rd overflowed: NaN compares false) is the quotient computed.
WQ_HD inline bool quant_code_ok(float v, float rd, float r) {
    return 0.5f - fabsf(fmaf(v, rd, -r)) >= 0x1p-13f;
}

WQ_HD inline int quant_code(float v, float d, float rd) {
    const float r = rintf(v * rd);
    if (!quant_code_ok(v, rd, r)) return (int)rintf(v / d);
    return (int)r;
}

// Four codes, quant_code's each, packed low byte first; one branch for the
// rare exact quotients of the four.
WQ_HD inline uint32_t quant_word(float v0, float v1, float v2, float v3, float d, float rd) {
    float r0 = rintf(v0 * rd), r1 = rintf(v1 * rd), r2 = rintf(v2 * rd), r3 = rintf(v3 * rd);
    const bool k0 = quant_code_ok(v0, rd, r0), k1 = quant_code_ok(v1, rd, r1);
    const bool k2 = quant_code_ok(v2, rd, r2), k3 = quant_code_ok(v3, rd, r3);
    if (!(k0 && k1 && k2 && k3)) {
        if (!k0) r0 = rintf(v0 / d);
        if (!k1) r1 = rintf(v1 / d);
        if (!k2) r2 = rintf(v2 / d);
        if (!k3) r3 = rintf(v3 / d);
    }
    return ((uint32_t)(int)r0 & 0xFFu) | (((uint32_t)(int)r1 & 0xFFu) << 8) |
           (((uint32_t)(int)r2 & 0xFFu) << 16) | (((uint32_t)(int)r3 & 0xFFu) << 24);
}

}  // namespace wq
