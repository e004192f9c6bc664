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

// The leading arguments are what the first loads need (the partials, the
// Params pointer, H, nch and the host's position bound); this translation
// unit preloads them into SGPRs (-amdgpu-kernarg-preload-count=5), so no
// scalar load of the argument segment precedes the first loads.
template <int DPL>
__global__ __launch_bounds__(64 * kCombineWaves) void attn_combine_kernel(const float* kpart, const uint32_t* kparams,
                                                                          int kH, int knch, int kpos,
                                                                          AttnCombineArgs a) {
    a.part = kpart; a.params = kparams; a.H = kH; a.nch = knch; a.pos = kpos;
    constexpr int D = 64 * DPL;
    constexpr int LPG = 32 / DPL;  // lanes per 32-dim group
    constexpr int UNROLL = 8;      // chunks in flight per wavefront
    extern __shared__ float sh[];  // chunk weights [nch] | chains of waves 1..3 [3][D]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int item = (int)blockIdx.x;  // m * H + h (M <= 64, H <= 1024: checked on the host)
    const int m = item / kH, h = item - m * kH;
    const int nch = (int)a.nch;
    // n_hi: the chunk count at the host's bound, n: at the step's position
    const int n_hi = (kpos + m + kChunk) / kChunk;  // <= nch (checked on the host)
    const float* hb = a.part + (int64_t)item * nch * (D + 2);
    float* w = sh;
    float* chains = sh + nch;

    // The partials of this wave's first UNROLL chunks, the weight sum and
    // maximum of chunk `lane` and the maximum of chunk `tid` depend neither
    // on the maximum nor on the Params load: they are loaded up to the host's
    // bound before the position is read, one memory round trip instead of
    // three, and masked to the step's chunks where they are used.
    const float* pl = hb + DPL * lane;
    float pf[UNROLL][DPL];
#pragma unroll
    for (int q = 0; q < UNROLL; ++q) {
        const int cq = wave + kCombineWaves * q;
        const int cc = cq < n_hi ? cq : 0;  // loads from a valid chunk, no branch
#pragma unroll
        for (int k = 0; k < DPL; ++k) {
            const float v = pl[(int64_t)cc * (D + 2) + k];
            pf[q][k] = cq < n_hi ? v : 0.0f;
        }
    }
    const int lc = lane < n_hi ? lane : 0;
    const float lv = hb[(int64_t)lc * (D + 2) + D + 1], mv = hb[(int64_t)lc * (D + 2) + D];
    const float m0 = lane < n_hi ? mv : -3.0e38f;
    const int tcc = tid < n_hi ? tid : 0;
    const float mt = hb[(int64_t)tcc * (D + 2) + D];  // chunk tid's maximum (tid < n <= n_hi where used)
    asm volatile("" ::: "memory");  // the Params read below stays behind these loads
    const uint32_t p_dev = a.params ? a.params[kParamPos] : 0xFFFFFFFFu;
    // the rest of the arguments, in SGPRs once the loads are in flight
    pin_arg(a.M); pin_arg(a.gate); pin_arg(a.gate_stride); pin_arg(a.xq); pin_arg(a.dx); pin_arg(a.xs);

    // the step's position: the host's, or the device Params' (clamped to the
    // host bound, so that n <= n_hi <= nch whatever the buffer holds)
    const int64_t pos = (int64_t)p_dev < a.pos ? (int64_t)p_dev : a.pos;
    const int n = (int)((pos + m + kChunk) / kChunk);

    // chunk maxima (attn_combine.wgsl:39-42), in every wavefront
    float ml = lane < n ? m0 : -3.0e38f;
    for (int c = lane + 64; c < n; c += 64) ml = fmaxf(ml, hb[(int64_t)c * (D + 2) + D]);
    const float mx = wave_max(ml);
    // chunk weights (:46), once per workgroup; chunk tid's maximum was loaded up front
    if (tid < n) w[tid] = expf(mt - mx);
    for (int c = tid + 64 * kCombineWaves; c < n; c += 64 * kCombineWaves)
        w[c] = expf(hb[(int64_t)c * (D + 2) + D] - mx);
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
        if (lane < n) ll = fmaf(w[lane], lv, ll);  // lane < n <= n_hi: lv is chunk lane's
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
        case 64: hipLaunchKernelGGL((attn_combine_kernel<1>), grid, block, lds, s, a.part, a.params, (int)a.H, (int)a.nch, (int)a.pos, a); break;
        case 128: hipLaunchKernelGGL((attn_combine_kernel<2>), grid, block, lds, s, a.part, a.params, (int)a.H, (int)a.nch, (int)a.pos, a); break;
        default: hipLaunchKernelGGL((attn_combine_kernel<4>), grid, block, lds, s, a.part, a.params, (int)a.H, (int)a.nch, (int)a.pos, a); break;
    }
    return hipGetLastError();
}

}  // namespace wq
