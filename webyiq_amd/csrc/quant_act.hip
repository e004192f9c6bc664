// Activation quantiser (webyIQ crates/engine/src/shaders/quant.wgsl:19-62 and
// the torch fake-quant hook tools/reference.py:43-48), one workgroup per token.
//
//   optional RMSNorm: v = (x * r) * nw, r = 1 / sqrt(mean(x^2) + eps)
//   per activation group (GA = K or 32): dx = amax / 127,
//   xq = dx > 0 ? round_half_even(v / dx) : 0   (IEEE division, as torch)
//   xs[e] = sum of xq over accumulation group e (Ge = min(G, GA) elements)
//
// Thread i of the 256 owns float4 chunks i, i+256, ...; every reduction that
// feeds a rounding (the RMSNorm sum of squares) runs in a fixed order that the
// CPU oracle restates, so int8 codes are reproducible bit for bit.
#include "common.hpp"
#include "launch.hpp"

#pragma clang fp contract(off)

namespace wq {
namespace {

constexpr int kQuantThreads = 256;

// Correctly rounded single-precision square root: the hardware estimate is
// within one ulp, and the candidate with the smallest |x - c^2| (exact in
// double: c^2 has 48 significant bits) is the rounded root (a square root is
// never exactly halfway between two floats).
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

// Up to kCacheChunks float4 per thread stay in registers (K <= 8192): the row
// is read from memory once; longer rows are re-read (L2 hits) per pass.
constexpr int kCacheChunks = 8;

template <bool NORM, bool PER_TOKEN, int GE, bool CACHED>
__global__ __launch_bounds__(kQuantThreads) void quant_act_kernel(QuantArgs a) {
    pin_arg(a.x); pin_arg(a.norm_w); pin_arg(a.eps); pin_arg(a.K);
    pin_arg(a.xq); pin_arg(a.dx); pin_arg(a.xs);
    const int tid = threadIdx.x;
    const int64_t t = blockIdx.x;
    const int K = (int)a.K;
    const int nchunk = K / 4;
    const int jmax = (nchunk + kQuantThreads - 1) / kQuantThreads;
    const int JL = CACHED ? kCacheChunks : jmax;  // constant trip count when cached
    const float4* xr = reinterpret_cast<const float4*>(a.x + t * a.K);
    const float4* nw = reinterpret_cast<const float4*>(a.norm_w);
    __shared__ float red[kQuantThreads];
    const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);

    // one round of loads: the whole row (and norm weight) for this thread
    float4 xc[CACHED ? kCacheChunks : 1], wc[CACHED && NORM ? kCacheChunks : 1];
    if (CACHED) {
#pragma unroll
        for (int j = 0; j < kCacheChunks; ++j) {
            int c = tid + kQuantThreads * j;
            bool ok = j < jmax && c < nchunk;
            xc[j] = ok ? xr[c] : zero4;
            if (NORM) wc[j] = ok ? nw[c] : zero4;
        }
    }
    auto raw = [&](int j, int c) -> float4 { return CACHED ? xc[CACHED ? j : 0] : xr[c]; };

    float r = 1.0f;
    if (NORM) {
        float p = 0.0f;
#pragma unroll
        for (int j = 0; j < JL; ++j) {
            int c = tid + kQuantThreads * j;
            if (j < jmax && c < nchunk) {
                float4 v = raw(j, c);
                p = fmaf(v.x, v.x, p);
                p = fmaf(v.y, v.y, p);
                p = fmaf(v.z, v.z, p);
                p = fmaf(v.w, v.w, p);
            }
        }
        red[tid] = p;
        __syncthreads();
        for (int s = kQuantThreads / 2; s > 0; s >>= 1) {
            if (tid < s) red[tid] = red[tid] + red[tid + s];
            __syncthreads();
        }
        r = 1.0f / sqrt_rn(red[0] / (float)K + a.eps);
        __syncthreads();
    }

    auto load = [&](int j, int c) -> float4 {
        float4 v = raw(j, c);
        if (NORM) {
            float4 w = CACHED ? wc[CACHED && NORM ? j : 0] : nw[c];
            v.x = (v.x * r) * w.x;
            v.y = (v.y * r) * w.y;
            v.z = (v.z * r) * w.z;
            v.w = (v.w * r) * w.w;
        }
        return v;
    };

    // Per-token scale: block-wide absolute maximum (exact, order-free).
    float dtok = 0.0f;
    if (PER_TOKEN) {
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < JL; ++j) {
            int c = tid + kQuantThreads * j;
            if (j < jmax && c < nchunk) {
                float4 v = load(j, c);
                m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            }
        }
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        if ((tid & 63) == 0) red[tid >> 6] = m;
        __syncthreads();
        float amax = red[0];
        for (int w = 1; w < kQuantThreads / 64; ++w) amax = fmaxf(amax, red[w]);
        dtok = amax / 127.0f;
        if (tid == 0) a.dx[t] = dtok;
    }

    uint32_t* xq = reinterpret_cast<uint32_t*>(a.xq + t * a.K);
    constexpr int kLanesPerGe = GE / 4;  // lanes (float4 chunks) per xs group
#pragma unroll
    for (int j = 0; j < JL; ++j) {
        if (j >= jmax) break;
        int c = tid + kQuantThreads * j;
        bool valid = c < nchunk;
        float4 v = valid ? load(j, c) : zero4;
        float d = dtok;
        if (!PER_TOKEN) {
            // 32-element activation group = 8 consecutive lanes
            float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
            for (int o = 1; o < 8; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
            d = m / 127.0f;
            if (valid && (tid & 7) == 0) a.dx[t * (a.K / 32) + c / 8] = d;
        }
        int q0 = 0, q1 = 0, q2 = 0, q3 = 0;
        if (d > 0.0f) {
            q0 = (int)rintf(v.x / d);
            q1 = (int)rintf(v.y / d);
            q2 = (int)rintf(v.z / d);
            q3 = (int)rintf(v.w / d);
        }
        if (valid)
            xq[c] = (uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8) |
                    ((uint32_t)(q2 & 0xFF) << 16) | ((uint32_t)(q3 & 0xFF) << 24);
        int s = q0 + q1 + q2 + q3;
        for (int o = 1; o < kLanesPerGe; o <<= 1) s += __shfl_xor(s, o);
        if (valid && (tid % kLanesPerGe) == 0) a.xs[t * (a.K / GE) + c / kLanesPerGe] = s;
    }
}

template <bool NORM, bool CACHED>
hipError_t dispatch_quant(const QuantArgs& a, hipStream_t s) {
    dim3 grid((unsigned)a.M), block(kQuantThreads);
    bool pt = a.GA == a.K;
    int ge = a.GA < a.G ? a.GA : a.G;
    if (pt && ge == 128)
        hipLaunchKernelGGL((quant_act_kernel<NORM, true, 128, CACHED>), grid, block, 0, s, a);
    else if (pt && ge == 32)
        hipLaunchKernelGGL((quant_act_kernel<NORM, true, 32, CACHED>), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((quant_act_kernel<NORM, false, 32, CACHED>), grid, block, 0, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_quant_act(const QuantArgs& a, hipStream_t s) {
    const bool cached = a.K <= 4 * kQuantThreads * kCacheChunks;
    if (a.norm_w) return cached ? dispatch_quant<true, true>(a, s) : dispatch_quant<true, false>(a, s);
    return cached ? dispatch_quant<false, true>(a, s) : dispatch_quant<false, false>(a, s);
}

}  // namespace wq
