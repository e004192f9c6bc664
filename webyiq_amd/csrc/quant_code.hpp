// int8 code of the activation quantiser, shared by the device kernels and a
// host-compiled exhaustive check (tests/test_quant_code.py builds it with g++).
#pragma once
#include <cmath>

#ifndef WQ_HD
#define WQ_HD __host__ __device__
#endif

namespace wq {

// rint(v / d) with v / d the IEEE quotient, without a division on the common
// path; rd = 1 / d (IEEE), d > 0, |v| <= 127 d (|v / d| < 128).
// a = v * rd is within 2^-23 relative (<= 1.6e-5 absolute) of v / d and the
// IEEE quotient within 0.5 ulp (<= 3.9e-6), so both round to the same integer
// unless a lies within 2^-13 of a half-integer; only then (or when rd
// overflowed: NaN compares false) is the quotient computed exactly.
WQ_HD inline int quant_code(float v, float d, float rd) {
    const float a = v * rd;
    const float r = rintf(a);
    if (!(0.5f - fabsf(a - r) >= 0x1p-13f)) return (int)rintf(v / d);
    return (int)r;
}

}  // namespace wq
