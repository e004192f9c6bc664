// Shared device helpers for the gfx950 int4 x int8 kernels.
//
// Data layout (webyIQ's packed-int4 format, tools/convert.py:8-12):
//   wq  u32 [N, K/8]   word i of row n holds codes 8i..8i+7:
//                      byte b = q[8i+b] | q[8i+4+b] << 4, so
//                      w & 0x0F0F0F0F        -> int8 codes 8i+0..3
//                      (w >> 4) & 0x0F0F0F0F -> int8 codes 8i+4..7
//   ws  u32 [N, K/G]   low half f16 scale s, high half f16 min m; w = q*s + m
//   xq  i8  [M, K]     activations, x ~= xq * dx
//   dx  f32 [M, K/GA]  GA = K (per token) or 32
//   xs  i32 [M, K/Ge]  sum of xq per accumulation group, Ge = min(G, GA)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "quant_code.hpp"

namespace wq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr uint32_t kNibbleMask = 0x0F0F0F0Fu;

__device__ __forceinline__ float f16lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(w & 0xFFFFu));
}
__device__ __forceinline__ float f16hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(w >> 16));
}

// Signed 4 x int8 dot product with int32 accumulate (v_dot4_i32_i8); the
// reference's dot4I8Packed (crates/engine/src/gpu.rs:70-75 defines it as the
// sign-extended byte dot).  Nibble codes 0..15 are non-negative int8.
__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// 32 codes (one 16-byte load of a packed row) against 32 int8 activations.
__device__ __forceinline__ int dot32(const uint4& w, const uint4& xa, const uint4& xb) {
    int acc = 0;
    acc = dot4(w.x & kNibbleMask, xa.x, acc);
    acc = dot4((w.x >> 4) & kNibbleMask, xa.y, acc);
    acc = dot4(w.y & kNibbleMask, xa.z, acc);
    acc = dot4((w.y >> 4) & kNibbleMask, xa.w, acc);
    acc = dot4(w.z & kNibbleMask, xb.x, acc);
    acc = dot4((w.z >> 4) & kNibbleMask, xb.y, acc);
    acc = dot4(w.w & kNibbleMask, xb.z, acc);
    acc = dot4((w.w >> 4) & kNibbleMask, xb.w, acc);
    return acc;
}

// Sum over the 4 lanes of a quad (exact int32, order-free) via DPP.
__device__ __forceinline__ int quad_sum(int v) {
    v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);  // quad_perm [1,0,3,2]
    v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);  // quad_perm [2,3,0,1]
    return v;
}

// DPP lane moves (gfx9 encodings).  Within a row of 16 lanes: quad_perm
// [1,0,3,2] / [2,3,0,1] pair lanes i ^ 1 / i ^ 2; row_half_mirror pairs
// i with 7 - i in each half-row, row_mirror i with 15 - i.  row_bcast15 /
// row_bcast31 hand lane 15 (31) to the next row (rows 2 and 3).
constexpr int kDppXor1 = 0xB1;
constexpr int kDppXor2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;
constexpr int kDppBcast15 = 0x142;
constexpr int kDppBcast31 = 0x143;
constexpr int kDppRowShr4 = 0x114;  // lane i of a row reads lane i - 4 (0 for i < 4)
constexpr int kDppRowShr8 = 0x118;  // lane i of a row reads lane i - 8 (0 for i < 8)

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xF, false);
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

// Sum of the 64 lanes in the order of the xor butterfly (p[i] + p[i ^ o] for
// o = 1, 2, ..., 32: a pairwise tree in lane order), returned to every lane.
// After each level the partners' values are equal, so the mirror moves pair
// the same values as the xor partners and each addition is one of the
// tree's (IEEE addition commutes).  Rows 1 and 3 form R0 + R1 and R2 + R3;
// row 3 then adds R0 + R1.
__device__ __forceinline__ float wave_sum_tree(float v) {
    v = v + dpp_f<kDppXor1>(v);
    v = v + dpp_f<kDppXor2>(v);
    v = v + dpp_f<kDppHalfMirror>(v);
    v = v + dpp_f<kDppMirror>(v);
    v = v + dpp_f<kDppBcast15, 0xA>(v);  // rows 0, 2 add +0 (unused)
    v = v + dpp_f<kDppBcast31, 0xC>(v);  // row 3: (R2 + R3) + (R0 + R1)
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// One pass (16 groups of 128 codes, quad k of 16-lane row r = group 4r + k,
// every lane of a quad holding its group's s, A, m, X) folded in the
// canonical per-token order: each pair of groups (2i, 2i + 1) that exists
// runs the chain c = fma(s, A, c); c = fma(m, X, c) from c = 0 (row_shr:4
// hands quad 2k's value to quad 2k + 1, which completes the pair); the 8
// pair values then meet as a pairwise tree, ((p0 + p1) + (p2 + p3)) +
// ((p4 + p5) + (p6 + p7)) (row_shr:8 pairs a row's two pairs, row_bcast15/31
// the rows).  Returned to every lane.  c never becomes -0 (each step rounds
// an exact sum with +0 or a non-zero term to nearest), so a skipped
// group's pass-through and an empty pair's +0 are the oracle's.
__device__ __forceinline__ float pass_pairs8(bool act, float s, float A, float m, float X) {
    float c = act ? fmaf(m, X, fmaf(s, A, 0.0f)) : 0.0f;
    const float ci = dpp_f<kDppRowShr4>(c);  // quads 1, 3: the pair's first group
    c = act ? fmaf(m, X, fmaf(s, A, ci)) : ci;
    c = c + dpp_f<kDppRowShr8>(c);           // lanes 12..15: p(2r + 1) + p(2r)
    c = c + dpp_f<kDppBcast15, 0xA>(c);      // rows 1, 3: row r + row r - 1
    c = c + dpp_f<kDppBcast31, 0xC>(c);      // row 3: rows 2, 3 + rows 0, 1
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(c), 63));
}

// Sum of squares of one float4 chunk: an fmaf chain in index order.
__device__ __forceinline__ float chunk_ss(float4 v) {
    float c = fmaf(v.x, v.x, 0.0f);
    c = fmaf(v.y, v.y, c);
    c = fmaf(v.z, v.z, c);
    return fmaf(v.w, v.w, c);
}

// Maximum of the 64 lanes (exact, order-free), returned to every lane.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_f<kDppMirror>(v));
    v = fmaxf(v, dpp_f<kDppBcast15, 0xA>(v));
    v = fmaxf(v, dpp_f<kDppBcast31, 0xC>(v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Maximum over aligned groups of 8 lanes, in every lane of the group
// (|values| >= 0, so the 0 that a masked move never produces is harmless).
__device__ __forceinline__ float max8(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    return fmaxf(v, dpp_f<kDppHalfMirror>(v));
}

// Exact int32 sums over aligned groups of 8 lanes (every lane of the group)
// and of 32 lanes (in rows 1 and 3: lanes 16..31 hold lanes 0..31's sum,
// lanes 48..63 that of lanes 32..63).
__device__ __forceinline__ int sum8(int v) {
    v += dpp_i<kDppXor1>(v);
    v += dpp_i<kDppXor2>(v);
    return v + dpp_i<kDppHalfMirror>(v);
}
__device__ __forceinline__ int sum32_rows13(int v) {
    v = sum8(v);
    v += dpp_i<kDppMirror>(v);
    return v + dpp_i<kDppBcast15, 0xA>(v);
}

// Non-temporal 16-byte load for weights that are streamed exactly once.
__device__ __forceinline__ uint4 load_stream16(const void* p) {
    v4i v = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
    return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}

__device__ __forceinline__ uint4 load16(const void* p) {
    return *reinterpret_cast<const uint4*>(p);
}

// Force a kernel argument into registers at this point.  Scalar loads of
// kernel arguments are otherwise sunk next to their first use, and one issued
// after the main memory wait adds a whole memory round trip to the critical
// path of a latency-bound kernel.
template <typename T>
__device__ __forceinline__ void pin_arg(const T& v) {
    asm volatile("" ::"s"(v));
}

// SiLU(a) * u in the reference's form a / (1 + exp(-a)) * u
// (crates/engine/src/shaders/gemv_q4q8.wgsl:128).
__device__ __forceinline__ float silu_mul(float a, float u) {
    return a / (1.0f + expf(-a)) * u;
}

// Order-preserving key for argmax over floats: larger value -> larger key,
// equal values -> the lower index wins (its complement is larger).  -0.0 is
// folded onto +0.0 so that the two compare equal, as `>` does.
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
    uint32_t u = __float_as_uint(v + 0.0f);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}

// Correctly rounded single-precision square root: the hardware estimate is
// within one ulp, and the candidate with the smallest |x - c^2| (exact in
// double: c^2 has 48 significant bits) is the rounded root (a square root is
// never exactly halfway between two floats).
// total / K (IEEE).  For K a power of two it is the product with 2^-n,
// rounded once like the quotient, so the same value without a division.
__device__ __forceinline__ float mean_of(float total, int K) {
    if ((K & (K - 1)) == 0) return total * __int_as_float((127 - __builtin_ctz(K)) << 23);
    return total / (float)K;
}

__device__ float sqrt_rn(float x) {
    float y = __builtin_amdgcn_sqrtf(x);
    if (!(x > 0.0f) || isinf(x) || !(y > 0.0f)) return y;
    float lo = __uint_as_float(__float_as_uint(y) - 1u);
    float hi = __uint_as_float(__float_as_uint(y) + 1u);
    double xd = (double)x;
    double ey = fabs(xd - (double)y * (double)y);
    double el = fabs(xd - (double)lo * (double)lo);
    double eh = fabs(xd - (double)hi * (double)hi);
    float r = y;
    if (el < ey) { r = lo; ey = el; }
    if (eh < ey) r = hi;
    return r;
}

}  // namespace wq
