// Flash-decoding merge with the int8 epilogue of the o projection's input
// (webyIQ crates/engine/src/shaders/attn_combine.wgsl:1-83, dispatched per
// (token, head) by graph.rs:289-291).
//
// Chunk c of head h for token m holds, at part[((m H + h) nch + c) (D + 2)]:
// the D output sums of the chunk (weights exp(s - m_c)), its maximum score
// m_c and its weight sum l_c (attn.wgsl:78-113).  Token m covers positions
// 0 ..= pos + m, i.e. chunks 0 .. n-1 with n = (pos + m + 32) / 32.
//
//   mx = max_c m_c;  w_c = exp(m_c - mx);  l = sum_c w_c l_c
//   o  = (sum_c w_c part_c) / l;  gated: o /= 1 + exp(-g)
//   per 32 dims: dx = amax / 127, xq = rint(o / dx) (IEEE quotient, as the
//   activation quantiser), xs = sum of xq.
//
// One workgroup of four wavefronts per (token, head); lane l owns dims
// DPL l .. DPL l + DPL - 1 (DPL = D / 64).  Order of the sums, which the CPU
// oracle restates: l -- lane l accumulates fmaf(w_c, l_c, .) over chunks
// c = l, l + 64, ... in order, then the lanes' pairwise tree
// (wave_sum_tree); o -- wave w runs one fmaf chain per dim over the chunks
// c = w, w + 4, w + 8, ... in order, and the four chains are added as
// (o_0 + o_1) + (o_2 + o_3).  The chunk weights go through LDS.
#include "common.hpp"
#include "launch.hpp"

#pragma clang fp contract(off)

namespace wq {
namespace {

constexpr int kCombineWaves = 4;
constexpr int kChunk = 32;  // positions per chunk (attn.wgsl CH)

// max / sum over aligned groups of L lanes (L = 8, 16 or 32), every lane of
// the group; exact (max, int32 sums)
template <int L>
__device__ __forceinline__ float group_max(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
    if (L >= 16) v = fmaxf(v, dpp_f<kDppMirror>(v));
    if (L >= 32) v = fmaxf(v, __shfl_xor(v, 16));
    return v;
}
template <int L>
__device__ __forceinline__ int group_sum(int v) {
    v += dpp_i<kDppXor1>(v);
    v += dpp_i<kDppXor2>(v);
    v += dpp_i<kDppHalfMirror>(v);
    if (L >= 16) v += dpp_i<kDppMirror>(v);
    if (L >= 32) v += __shfl_xor(v, 16);
    return v;
}

template <int DPL>
__global__ __launch_bounds__(64 * kCombineWaves) void attn_combine_kernel(AttnCombineArgs a) {
    pin_arg(a.part); pin_arg(a.M); pin_arg(a.H); pin_arg(a.nch); pin_arg(a.pos); pin_arg(a.params);
    pin_arg(a.gate); pin_arg(a.gate_stride); pin_arg(a.xq); pin_arg(a.dx); pin_arg(a.xs);
    constexpr int D = 64 * DPL;
    constexpr int LPG = 32 / DPL;  // lanes per 32-dim group
    constexpr int UNROLL = 8;      // chunks in flight per wavefront
    extern __shared__ float sh[];  // chunk weights [nch] | chains of waves 1..3 [3][D]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t item = blockIdx.x;  // m * H + h
    const int64_t m = item / a.H, h = item - m * a.H;
    const int nch = (int)a.nch;
    // the step's position: the host's, or the device Params' (clamped to the
    // host bound, so that n <= nch whatever the buffer holds)
    int64_t pos = a.pos;
    if (a.params) {
        const int64_t p = (int64_t)a.params[kParamPos];
        pos = p < a.pos ? p : a.pos;
    }
    const int n = (int)((pos + m + kChunk) / kChunk);  // <= nch (checked on the host)
    const float* hb = a.part + item * (int64_t)nch * (D + 2);
    float* w = sh;
    float* chains = sh + nch;

    // The partials of this wave's first UNROLL chunks and (wave 0) the first
    // weight sums do not depend on the maximum: their loads are issued with
    // the maxima's, one memory round trip instead of two.
    const float* pl = hb + DPL * lane;
    float pf[UNROLL][DPL];
#pragma unroll
    for (int q = 0; q < UNROLL; ++q) {
        const int cq = wave + kCombineWaves * q;
#pragma unroll
        for (int k = 0; k < DPL; ++k) pf[q][k] = cq < n ? pl[(int64_t)cq * (D + 2) + k] : 0.0f;
    }
    const float lf = wave == 0 && lane < n ? hb[(int64_t)lane * (D + 2) + D + 1] : 0.0f;

    // chunk maxima (attn_combine.wgsl:39-42), in every wavefront
    float ml = -3.0e38f;
    for (int c = lane; c < n; c += 64) ml = fmaxf(ml, hb[(int64_t)c * (D + 2) + D]);
    const float mx = wave_max(ml);
    // chunk weights (:46), once per workgroup
    for (int c = tid; c < n; c += 64 * kCombineWaves) w[c] = expf(hb[(int64_t)c * (D + 2) + D] - mx);
    __syncthreads();

    // wave w's chains over chunks w, w + 4, ... (:48)
    float acc[DPL];
#pragma unroll
    for (int k = 0; k < DPL; ++k) acc[k] = 0.0f;
#pragma unroll
    for (int q = 0; q < UNROLL; ++q) {  // the prefetched chunks, in order
        const int cq = wave + kCombineWaves * q;
        if (cq < n) {
            const float wc = w[cq];
#pragma unroll
            for (int k = 0; k < DPL; ++k) acc[k] = fmaf(wc, pf[q][k], acc[k]);
        }
    }
    int c = wave + kCombineWaves * UNROLL;
    for (; c + kCombineWaves * (UNROLL - 1) < n; c += kCombineWaves * UNROLL) {
        float p[UNROLL][DPL], wc[UNROLL];
#pragma unroll
        for (int q = 0; q < UNROLL; ++q) {
            const int cq = c + kCombineWaves * q;
            wc[q] = w[cq];
#pragma unroll
            for (int k = 0; k < DPL; ++k) p[q][k] = pl[(int64_t)cq * (D + 2) + k];
        }
#pragma unroll
        for (int q = 0; q < UNROLL; ++q)
#pragma unroll
            for (int k = 0; k < DPL; ++k) acc[k] = fmaf(wc[q], p[q][k], acc[k]);
    }
    for (; c < n; c += kCombineWaves) {
        const float wc = w[c];
#pragma unroll
        for (int k = 0; k < DPL; ++k) acc[k] = fmaf(wc, pl[(int64_t)c * (D + 2) + k], acc[k]);
    }
    if (wave > 0) {
#pragma unroll
        for (int k = 0; k < DPL; ++k) chains[(wave - 1) * D + DPL * lane + k] = acc[k];
    }
    // weight sum (:47), lane-parallel then the lane tree
    float ll = 0.0f;
    if (wave == 0) {
        if (lane < n) ll = fmaf(w[lane], lf, ll);
        for (int cc = lane + 64; cc < n; cc += 64) ll = fmaf(w[cc], hb[(int64_t)cc * (D + 2) + D + 1], ll);
    }
    __syncthreads();
    if (wave > 0) return;  // no barrier follows
    const float l = wave_sum_tree(ll);

    float o[DPL];
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
        const int i = DPL * lane + k;
        const float s = (acc[k] + chains[i]) + (chains[D + i] + chains[2 * D + i]);
        o[k] = s / l;  // :50
    }
    if (a.gate) {  // :51-54, gate rows [head: q (D) | gate (D)]
        const float* g = a.gate + m * a.gate_stride + h * 2 * D + D + DPL * lane;
#pragma unroll
        for (int k = 0; k < DPL; ++k) o[k] = o[k] / (1.0f + expf(-g[k]));
    }

    // per-32 int8 groups (:59-82)
    float am = 0.0f;
#pragma unroll
    for (int k = 0; k < DPL; ++k) am = fmaxf(am, fabsf(o[k]));
    const float d = group_max<LPG>(am) / 127.0f;
    const float rd = 1.0f / d;
    uint32_t word = 0;
    int sum = 0;
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
        const int q = d > 0.0f ? quant_code(o[k], d, rd) : 0;
        sum += q;
        word |= ((uint32_t)q & 0xFFu) << (8 * k);
    }
    sum = group_sum<LPG>(sum);
    const int64_t K = a.H * D;
    int8_t* xr = a.xq + m * K + h * D + DPL * lane;
    if (DPL == 4) *reinterpret_cast<uint32_t*>(xr) = word;
    else if (DPL == 2) *reinterpret_cast<uint16_t*>(xr) = (uint16_t)word;
    else *xr = (int8_t)word;
    if ((lane % LPG) == 0) {
        const int64_t gi = m * (K / 32) + (h * D + DPL * lane) / 32;
        a.dx[gi] = d;
        a.xs[gi] = sum;
    }
}

}  // namespace

hipError_t launch_attn_combine(const AttnCombineArgs& a, hipStream_t s) {
    dim3 grid((unsigned)(a.M * a.H)), block(64 * kCombineWaves);
    const size_t lds = ((size_t)a.nch + 3 * (size_t)a.D) * sizeof(float);
    switch (a.D) {
        case 64: hipLaunchKernelGGL((attn_combine_kernel<1>), grid, block, lds, s, a); break;
        case 128: hipLaunchKernelGGL((attn_combine_kernel<2>), grid, block, lds, s, a); break;
        default: hipLaunchKernelGGL((attn_combine_kernel<4>), grid, block, lds, s, a); break;
    }
    return hipGetLastError();
}

}  // namespace wq
