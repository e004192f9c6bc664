// Lane l of wave w owns the 32-element slices 2048 j + 32 l of the passes
// j = w, w + 4, ... of its token's row -- the slice a decode GEMV lane owns --
// and every reduction that feeds a rounding (the RMSNorm sum of squares) runs
// in a fixed order the CPU oracle restates: an fmaf chain per slice, a
// wavefront xor butterfly per pass, pass sums added in pass order.  So int8
// codes are reproducible bit for bit, here and in the fused GEMV quantiser.
#include "common.hpp"
#include "launch.hpp"

#pragma clang fp contract(off)

namespace wq {
namespace {

constexpr int kQuantThreads = 256;
constexpr int kQuantWaves = kQuantThreads / 64;
constexpr int kPass = 2048;  // codes per wavefront pass (64 lanes x 32)

// CACHED (K <= 4 passes): one slice per lane, loaded once and kept in
// registers.  Longer rows are re-read (L2 hits) in each phase.
template <bool NORM, bool PER_TOKEN, int GE, bool CACHED>
__global__ __launch_bounds__(kQuantThreads) void quant_act_kernel(QuantArgs a) {
    pin_arg(a.x); pin_arg(a.norm_w); pin_arg(a.eps); pin_arg(a.K);
    pin_arg(a.xq); pin_arg(a.dx); pin_arg(a.xs);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t t = blockIdx.x;
    const int K = (int)a.K;
    const int J = (K + kPass - 1) / kPass;
    const int NL = CACHED ? 1 : (J - wave + kQuantWaves - 1) / kQuantWaves;  // this wave's passes
    const float* xr = a.x + t * a.K;
    __shared__ float red[kQuantWaves];

    // slice i of this lane: pass j = wave + 4 i, codes [base, base + 32)
    auto base_of = [&](int i) { return kPass * (wave + kQuantWaves * i) + 32 * lane; };
    auto load_slice = [&](int b, float4* v) {
        const float4* p = reinterpret_cast<const float4*>(xr + b);
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = p[u];
    };
    float4 xc[8], wc[8];
    const bool act0 = base_of(0) < K && wave < J;
    if (CACHED) {
        load_slice(act0 ? base_of(0) : 0, xc);
        if (NORM) {
            const float4* p = reinterpret_cast<const float4*>(a.norm_w + (act0 ? base_of(0) : 0));
#pragma unroll
            for (int u = 0; u < 8; ++u) wc[u] = p[u];
        }
    }
    // this lane's slice i as (optionally normalised) values
    float r = 1.0f;
    auto slice = [&](int i, float4* v) {
        const int b = base_of(i);
        if (CACHED) {
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = xc[u];
        } else {
            load_slice(b, v);
        }
        if (NORM) {
            const float4* p = reinterpret_cast<const float4*>(a.norm_w + b);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float4 w = CACHED ? wc[u] : p[u];
                v[u].x = (v[u].x * r) * w.x;
                v[u].y = (v[u].y * r) * w.y;
                v[u].z = (v[u].z * r) * w.z;
                v[u].w = (v[u].w * r) * w.w;
            }
        }
    };

    if (NORM) {
        // rounds of 4 passes: wave w adds pass 4 q + w; every thread then adds
        // the round's pass sums in pass order
        float total = 0.0f;
        const int rounds = (J + kQuantWaves - 1) / kQuantWaves;
        for (int q = 0; q < rounds; ++q) {
            const int b = kPass * (wave + kQuantWaves * q) + 32 * lane;
            float pp = 0.0f;
            if (wave + kQuantWaves * q < J && b < K) {
                float4 v[8];
                if (CACHED) {
#pragma unroll
                    for (int u = 0; u < 8; ++u) v[u] = xc[u];
                } else {
                    load_slice(b, v);
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    pp = fmaf(v[u].x, v[u].x, pp);
                    pp = fmaf(v[u].y, v[u].y, pp);
                    pp = fmaf(v[u].z, v[u].z, pp);
                    pp = fmaf(v[u].w, v[u].w, pp);
                }
            }
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) pp = pp + __shfl_xor(pp, o);
            if (lane == 0) red[wave] = pp;
            __syncthreads();
            const int np = min(kQuantWaves, J - kQuantWaves * q);
            for (int w = 0; w < np; ++w) total = total + red[w];
            __syncthreads();
        }
        r = 1.0f / sqrt_rn(total / (float)K + a.eps);
    }

    // Per-token scale: block-wide absolute maximum (exact, order-free).
    float dtok = 0.0f;
    if (PER_TOKEN) {
        float m = 0.0f;
        for (int i = 0; i < NL; ++i) {
            if (base_of(i) >= K || (CACHED && !act0)) continue;
            float4 v[8];
            slice(i, v);
#pragma unroll
            for (int u = 0; u < 8; ++u)
                m = fmaxf(m, fmaxf(fmaxf(fabsf(v[u].x), fabsf(v[u].y)), fmaxf(fabsf(v[u].z), fabsf(v[u].w))));
        }
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        if (lane == 0) red[wave] = m;
        __syncthreads();
        float amax = red[0];
        for (int w = 1; w < kQuantWaves; ++w) amax = fmaxf(amax, red[w]);
        dtok = amax / 127.0f;
        if (tid == 0) a.dx[t] = dtok;
    }

    for (int i = 0; i < NL; ++i) {
        const int b = base_of(i);
        const bool valid = b < K && (!CACHED || act0);
        float4 v[8];
        if (valid) {
            slice(i, v);
        } else {
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        float d = dtok;
        if (!PER_TOKEN) {
            // the slice is one 32-element activation group
            float m = 0.0f;
#pragma unroll
            for (int u = 0; u < 8; ++u)
                m = fmaxf(m, fmaxf(fmaxf(fabsf(v[u].x), fabsf(v[u].y)), fmaxf(fabsf(v[u].z), fabsf(v[u].w))));
            d = m / 127.0f;
            if (valid) a.dx[t * (a.K / 32) + b / 32] = d;
        }
        uint32_t wds[8];
        int cs = 0;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            int q0 = 0, q1 = 0, q2 = 0, q3 = 0;
            if (d > 0.0f) {
                q0 = (int)rintf(v[u].x / d);
                q1 = (int)rintf(v[u].y / d);
                q2 = (int)rintf(v[u].z / d);
                q3 = (int)rintf(v[u].w / d);
            }
            wds[u] = (uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8) | ((uint32_t)(q2 & 0xFF) << 16) |
                     ((uint32_t)(q3 & 0xFF) << 24);
            cs += q0 + q1 + q2 + q3;
        }
        if (GE == 128) cs = quad_sum(cs);  // 4 consecutive lanes = one 128-group
        if (valid) {
            uint4* xo = reinterpret_cast<uint4*>(a.xq + t * a.K + b);
            xo[0] = make_uint4(wds[0], wds[1], wds[2], wds[3]);
            xo[1] = make_uint4(wds[4], wds[5], wds[6], wds[7]);
            if ((lane % (GE / 32)) == 0) a.xs[t * (a.K / GE) + b / GE] = cs;
        }
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
    const bool cached = a.K <= kQuantWaves * kPass;
    if (a.norm_w) return cached ? dispatch_quant<true, true>(a, s) : dispatch_quant<true, false>(a, s);
    return cached ? dispatch_quant<false, true>(a, s) : dispatch_quant<false, false>(a, s);
}

}  // namespace wq
