// Activation quantiser (webyIQ crates/engine/src/shaders/quant.wgsl:19-62 and
// the torch fake-quant hook tools/reference.py:43-48).
//
//   optional RMSNorm: v = (x * r) * nw, r = 1 / sqrt(mean(x^2) + eps)
//   per activation group (GA = K or 32): dx = amax / 127,
//   xq = dx > 0 ? round_half_even(v / dx) : 0   (IEEE division, as torch)
//   xs[e] = sum of xq over accumulation group e (Ge = min(G, GA) elements)
//
// The row is read in passes of 2048 elements (512 float4 chunks): load u
// (0..7) of pass j gives lane l the chunk 512 j + 64 u + l, so every load
// instruction reads 1 KiB of consecutive memory and every code store writes
// 256 consecutive bytes.  The RMSNorm sum of squares, the one reduction that
// feeds a rounding, runs in a fixed order the CPU oracle restates: an fmaf
// chain per chunk, a pairwise tree over a lane's 8 chunks, a pairwise tree
// over the 64 lanes (wave_sum_tree), pass sums added in pass order.  The tree
// over a lane's chunks lets waves that hold 2, 4 or 8 of its loads form the
// same value, so codes are bit-identical across the kernels below and the
// fused GEMV quantiser.
//
// Two layouts: few tokens -- one workgroup of eight waves per token, wave w
// taking load w of every pass (latency: 1.0 us less than four waves with
// the RMSNorm, 0.5 us without); many tokens -- one wavefront per token,
// four tokens per workgroup, no barriers (throughput).
#include "common.hpp"
#include "launch.hpp"

#pragma clang fp contract(off)

namespace wq {
namespace {

constexpr int kQuantThreads = 256;
constexpr int kQuantWaves = kQuantThreads / 64;
constexpr int kPassChunks = 512;   // float4 chunks per 2048-element pass
constexpr int kSplitMaxPasses = 8; // split layout: K <= 16384
constexpr int kSplitMaxTokens = 16;

__device__ __forceinline__ float4 normed(float4 v, float r, float4 w) {
    v.x = (v.x * r) * w.x;
    v.y = (v.y * r) * w.y;
    v.z = (v.z * r) * w.z;
    v.w = (v.w * r) * w.w;
    return v;
}

__device__ __forceinline__ float absmax4(float4 v) {
    return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}

__device__ __forceinline__ uint32_t pack_codes(float4 v, float d, float rd, int& sum) {
    const uint32_t w = d > 0.0f ? quant_word(v.x, v.y, v.z, v.w, d, rd) : 0u;
    sum = dot4(w, 0x01010101u, 0);
    return w;
}

// Codes, per-32 scales and group sums of one load (64 consecutive chunks
// starting at chunk c - lane) of token t.
template <bool PER_TOKEN, int GE>
__device__ __forceinline__ void emit(const QuantArgs& a, int64_t t, int c, bool valid, float4 v, float dtok,
                                     float rtok, int lane) {
    float d = dtok, rd = rtok;
    if (!PER_TOKEN) {
        // the 32-element activation group = 8 consecutive lanes
        d = max8(absmax4(v)) / 127.0f;
        rd = 1.0f / d;
        if (valid && (lane & 7) == 0) a.dx[t * (a.K / 32) + c / 8] = d;
    }
    int sum;
    const uint32_t wd = pack_codes(valid ? v : make_float4(0.f, 0.f, 0.f, 0.f), d, rd, sum);
    if (valid) reinterpret_cast<uint32_t*>(a.xq + t * a.K)[c] = wd;
    if (GE == 32) {
        const int s8 = sum8(sum);
        if (valid && (lane & 7) == 0) a.xs[t * (a.K / 32) + c / 8] = s8;
    } else {
        const int s32 = sum32_rows13(sum);
        if (valid && (lane & 31) == 16) a.xs[t * (a.K / 128) + c / 32] = s32;
    }
}

// One workgroup of QW = 4 or 8 waves per token; wave w holds loads
// LPW w .. LPW w + LPW - 1 of every pass (LPW = 8 / QW).  The per-wave
// RMSNorm subtotals meet in the lane tree's own order: with four waves each
// holds a pair (c0 + c1, ...) and they meet as (s0 + s1) + (s2 + s3); with
// eight each holds one chunk and they meet as ((s0 + s1) + (s2 + s3)) +
// ((s4 + s5) + (s6 + s7)).
template <bool NORM, bool PER_TOKEN, int GE, int QW>
__global__ __launch_bounds__(64 * QW) void quant_split_kernel(const float* kx, const float* knw, int kK, int kM,
                                                              QuantArgs a) {
    static_assert(QW == 4 || QW == 8, "waves per token");
    constexpr int LPW = 8 / QW;  // loads per wave and pass
    a.x = kx; a.norm_w = knw; a.K = kK; a.M = kM;  // preloaded (leading arguments)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t t = blockIdx.x;
    const int K = (int)a.K;
    const int nchunk = K / 4;
    const int J = (nchunk + kPassChunks - 1) / kPassChunks;
    const float4* xr = reinterpret_cast<const float4*>(a.x + t * a.K);
    const float4* nw = reinterpret_cast<const float4*>(a.norm_w);
    __shared__ float sub[kSplitMaxPasses][QW][64];  // per-wave lane subtotals
    __shared__ float red[kSplitMaxPasses];
    __shared__ float wred[QW];
    const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
    auto chunk = [&](int j, int i) { return kPassChunks * j + 64 * (LPW * wave + i) + lane; };

    float4 xc[kSplitMaxPasses][LPW], wc[kSplitMaxPasses][LPW];
#pragma unroll
    for (int j = 0; j < kSplitMaxPasses; ++j)
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int c = chunk(j, i);
            const bool ok = j < J && c < nchunk;
            const int cc = ok ? c : 0;  // loads from a valid chunk, no branch
            const float4 xv = xr[cc];
            xc[j][i] = ok ? xv : zero4;
            if (NORM) {
                const float4 wv = nw[cc];
                wc[j][i] = ok ? wv : zero4;
            }
        }
    // the outputs and epsilon, in SGPRs once the loads are in flight
    pin_arg(a.eps); pin_arg(a.xq); pin_arg(a.dx); pin_arg(a.xs);

    float r = 1.0f;
    if (NORM) {
#pragma unroll
        for (int j = 0; j < kSplitMaxPasses; ++j)
            if (j < J) sub[j][wave][lane] = LPW == 2 ? chunk_ss(xc[j][0]) + chunk_ss(xc[j][LPW - 1]) : chunk_ss(xc[j][0]);
        __syncthreads();
        // wave w completes passes w, w + QW, ...: the lane tree, then the lane tree
#pragma unroll
        for (int q = 0; q < (kSplitMaxPasses + QW - 1) / QW; ++q) {
            const int j = wave + QW * q;
            if (j < J) {
                const float* sj = &sub[j][0][lane];
                float p;
                if (QW == 4) p = (sj[0] + sj[64]) + (sj[128] + sj[192]);
                else p = ((sj[0] + sj[64]) + (sj[128] + sj[192])) + ((sj[256] + sj[320]) + (sj[384] + sj[448]));
                const float s = wave_sum_tree(p);
                if (lane == 0) red[j] = s;
            }
        }
        __syncthreads();
        float total = 0.0f;
        for (int j = 0; j < J; ++j) total = total + red[j];
        r = 1.0f / sqrt_rn(mean_of(total, K) + a.eps);
    }

    float dtok = 0.0f;
    if (PER_TOKEN) {
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < kSplitMaxPasses; ++j)
#pragma unroll
            for (int i = 0; i < LPW; ++i) {
                const int c = chunk(j, i);
                if (j < J && c < nchunk) m = fmaxf(m, absmax4(NORM ? normed(xc[j][i], r, wc[j][i]) : xc[j][i]));
            }
        m = wave_max(m);
        if (lane == 0) wred[wave] = m;
        __syncthreads();
        float amax = wred[0];
#pragma unroll
        for (int w = 1; w < QW; ++w) amax = fmaxf(amax, wred[w]);
        dtok = amax / 127.0f;
        if (tid == 0) a.dx[t] = dtok;
    }
    const float rtok = 1.0f / dtok;
#pragma unroll
    for (int j = 0; j < kSplitMaxPasses; ++j) {
        if (j >= J) break;
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int c = chunk(j, i);
            const float4 v = NORM ? normed(xc[j][i], r, wc[j][i]) : xc[j][i];
            emit<PER_TOKEN, GE>(a, t, c, c < nchunk, v, dtok, rtok, lane);
        }
    }
}

// One wavefront per token, 4 tokens per workgroup, no barriers.  JC > 0:
// rows of at most JC passes stay in registers; JC == 0: longer rows are
// re-read (L2 hits) in each phase.
template <bool NORM, bool PER_TOKEN, int GE, int JC>
__global__ __launch_bounds__(kQuantThreads) void quant_wave_kernel(const float* kx, const float* knw, int kK, int kM,
                                                                   QuantArgs a) {
    a.x = kx; a.norm_w = knw; a.K = kK; a.M = kM;  // preloaded (leading arguments)
    const int lane = threadIdx.x & 63;
    const int64_t t = (int64_t)blockIdx.x * kQuantWaves + (threadIdx.x >> 6);
    if (t >= a.M) return;  // whole wavefronts; the kernel has no barrier
    const int K = (int)a.K;
    const int nchunk = K / 4;
    const int J = (nchunk + kPassChunks - 1) / kPassChunks;
    const float4* xr = reinterpret_cast<const float4*>(a.x + t * a.K);
    const float4* nw = reinterpret_cast<const float4*>(a.norm_w);
    const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
    auto chunk = [&](int j, int u) { return kPassChunks * j + 64 * u + lane; };

    constexpr int NC = JC > 0 ? JC : 1;
    float4 xc[NC][8], wc[NC][8];
    if (JC > 0) {
#pragma unroll
        for (int j = 0; j < NC; ++j)
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int c = chunk(j, u);
                const bool ok = j < J && c < nchunk;
                const int cc = ok ? c : 0;  // loads from a valid chunk, no branch
                const float4 xv = xr[cc];
                xc[j][u] = ok ? xv : zero4;
                if (NORM) {
                    const float4 wv = nw[cc];
                    wc[j][u] = ok ? wv : zero4;
                }
            }
    }
    // the outputs and epsilon, in SGPRs once the loads are in flight
    pin_arg(a.eps); pin_arg(a.xq); pin_arg(a.dx); pin_arg(a.xs);
    auto raw = [&](int j, int u) -> float4 {
        if (JC > 0) return xc[JC > 0 ? j : 0][u];
        const int c = chunk(j, u);
        return c < nchunk ? xr[c] : zero4;
    };
    auto nwt = [&](int j, int u) -> float4 {
        if (JC > 0) return wc[JC > 0 ? j : 0][u];
        const int c = chunk(j, u);
        return c < nchunk ? nw[c] : zero4;
    };
    // f(j) for every pass; constant j (registers) when the row is cached
    auto for_passes = [&](auto&& f) {
        if constexpr (JC > 0) {
#pragma unroll
            for (int j = 0; j < NC; ++j)
                if (j < J) f(j);
        } else {
            for (int j = 0; j < J; ++j) f(j);
        }
    };

    float r = 1.0f;
    if (NORM) {
        float total = 0.0f;
        for_passes([&](int j) {
            float c[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) c[u] = chunk_ss(raw(j, u));
            const float p = ((c[0] + c[1]) + (c[2] + c[3])) + ((c[4] + c[5]) + (c[6] + c[7]));
            total = total + wave_sum_tree(p);
        });
        r = 1.0f / sqrt_rn(mean_of(total, K) + a.eps);
    }
    auto load = [&](int j, int u) -> float4 { return NORM ? normed(raw(j, u), r, nwt(j, u)) : raw(j, u); };

    float dtok = 0.0f;
    if (PER_TOKEN) {
        float m = 0.0f;
        for_passes([&](int j) {
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (chunk(j, u) < nchunk) m = fmaxf(m, absmax4(load(j, u)));
        });
        dtok = wave_max(m) / 127.0f;
        if (lane == 0) a.dx[t] = dtok;
    }
    const float rtok = 1.0f / dtok;
    for_passes([&](int j) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = chunk(j, u);
            emit<PER_TOKEN, GE>(a, t, c, c < nchunk, load(j, u), dtok, rtok, lane);
        }
    });
}

// MTP input stage (mtp_in.wgsl:45-89), one wavefront per (token, half), four
// per workgroup, no barriers.  The norms scale as the reference does,
// v * (r * w); their sums of squares run in this file's order (above), each
// over the values it normalises.  Output row 2m + half of the [2M, K] view.
template <int JC>
__global__ __launch_bounds__(kQuantThreads) void mtp_in_kernel(MtpInArgs a) {
    pin_arg(a.emb); pin_arg(a.x); pin_arg(a.norm_f); pin_arg(a.norm_e); pin_arg(a.norm_h);
    pin_arg(a.eps); pin_arg(a.K); pin_arg(a.M); pin_arg(a.xq); pin_arg(a.dx); pin_arg(a.xs);
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kQuantWaves + (threadIdx.x >> 6);
    if (row >= 2 * a.M) return;  // whole wavefronts; the kernel has no barrier
    const int64_t m = row >> 1;
    const bool hidden = (row & 1) != 0;  // half 1: the hidden state
    const int K = (int)a.K;
    const int nchunk = K / 4;
    const int J = (nchunk + kPassChunks - 1) / kPassChunks;
    const float4* src = reinterpret_cast<const float4*>((hidden ? a.x : a.emb) + m * a.K);
    const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
    auto chunk = [&](int j, int u) { return kPassChunks * j + 64 * u + lane; };

    // rows of one pass: the input and both norm weights in registers, all
    // loaded up front; longer rows: the input cached for up to 3 passes, the
    // weights read (L2 hits) where they are used
    constexpr int NC = JC > 0 ? JC : 1;
    constexpr bool WREG = JC == 1;
    const float* w0 = hidden ? a.norm_f : a.norm_e;
    float4 xc[NC][8], wc0[8], wc1[8];
    if (JC > 0) {
#pragma unroll
        for (int j = 0; j < NC; ++j)
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int c = chunk(j, u);
                const bool ok = j < J && c < nchunk;
                xc[j][u] = ok ? src[c] : zero4;
                if (WREG && j == 0) {
                    wc0[u] = ok ? reinterpret_cast<const float4*>(w0)[c] : zero4;
                    wc1[u] = ok && hidden ? reinterpret_cast<const float4*>(a.norm_h)[c] : zero4;
                }
            }
    }
    auto raw = [&](int j, int u) -> float4 {
        if (JC > 0) return xc[JC > 0 ? j : 0][u];
        const int c = chunk(j, u);
        return c < nchunk ? src[c] : zero4;
    };
    // norm weight 0 (norm_e or norm_f) or 1 (norm_h) of chunk (j, u)
    auto weight = [&](int which, int j, int u) -> float4 {
        if (WREG) return which ? wc1[u] : wc0[u];
        const int c = chunk(j, u);
        return c < nchunk ? reinterpret_cast<const float4*>(which ? a.norm_h : w0)[c] : zero4;
    };
    auto scale = [](float4 v, float r, float4 w) {  // mtp_in.wgsl:56,65,70: v *= r * w
        v.x = v.x * (r * w.x);
        v.y = v.y * (r * w.y);
        v.z = v.z * (r * w.z);
        v.w = v.w * (r * w.w);
        return v;
    };
    auto for_passes = [&](auto&& f) {
        if constexpr (JC > 0) {
#pragma unroll
            for (int j = 0; j < NC; ++j)
                if (j < J) f(j);
        } else {
            for (int j = 0; j < J; ++j) f(j);
        }
    };
    // 1 / rms of the values vals(j, u) (mtp_in.wgsl:26-42)
    auto inv_rms = [&](auto&& vals) {
        float total = 0.0f;
        for_passes([&](int j) {
            float c[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) c[u] = chunk_ss(vals(j, u));
            const float p = ((c[0] + c[1]) + (c[2] + c[3])) + ((c[4] + c[5]) + (c[6] + c[7]));
            total = total + wave_sum_tree(p);
        });
        return 1.0f / sqrt_rn(mean_of(total, K) + a.eps);
    };

    const float r0 = inv_rms(raw);
    auto v0 = [&](int j, int u) { return scale(raw(j, u), r0, weight(0, j, u)); };
    float r1 = 0.0f;
    if (hidden) r1 = inv_rms(v0);
    auto out = [&](int j, int u) { return hidden ? scale(v0(j, u), r1, weight(1, j, u)) : v0(j, u); };

    QuantArgs q{};
    q.K = a.K;
    q.xq = a.xq;
    q.dx = a.dx;
    q.xs = a.xs;
    for_passes([&](int j) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = chunk(j, u);
            emit<false, 32>(q, row, c, c < nchunk, out(j, u), 0.0f, 0.0f, lane);
        }
    });
}

// MTP input stage for rows of at most kSplitMaxPasses passes: one workgroup
// of eight waves per (token, half), wave w holding load w of every pass (the
// few-token quantiser's split).  The sums of squares meet in the lane tree's
// order through LDS, as in quant_split_kernel, so the codes are
// bit-identical to mtp_in_kernel's.
__global__ __launch_bounds__(512) void mtp_in_split_kernel(MtpInArgs a) {
    constexpr int QW = 8;
    pin_arg(a.emb); pin_arg(a.x); pin_arg(a.norm_f); pin_arg(a.norm_e); pin_arg(a.norm_h);
    pin_arg(a.eps); pin_arg(a.K); pin_arg(a.M); pin_arg(a.xq); pin_arg(a.dx); pin_arg(a.xs);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t row = blockIdx.x;  // output row 2m + half
    const int64_t m = row >> 1;
    const bool hidden = (row & 1) != 0;
    const int K = (int)a.K;
    const int nchunk = K / 4;
    const int J = (nchunk + kPassChunks - 1) / kPassChunks;
    const float4* src = reinterpret_cast<const float4*>((hidden ? a.x : a.emb) + m * a.K);
    const float4* w0 = reinterpret_cast<const float4*>(hidden ? a.norm_f : a.norm_e);
    const float4* w1 = reinterpret_cast<const float4*>(a.norm_h);
    __shared__ float sub[kSplitMaxPasses][QW][64];
    __shared__ float red[kSplitMaxPasses];
    const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
    auto chunk = [&](int j) { return kPassChunks * j + 64 * wave + lane; };

    float4 xc[kSplitMaxPasses], wc0[kSplitMaxPasses], wc1[kSplitMaxPasses];
#pragma unroll
    for (int j = 0; j < kSplitMaxPasses; ++j) {
        const int c = chunk(j);
        const bool ok = j < J && c < nchunk;
        xc[j] = ok ? src[c] : zero4;
        wc0[j] = ok ? w0[c] : zero4;
        wc1[j] = ok && hidden ? w1[c] : zero4;
    }
    auto scale = [](float4 v, float r, float4 w) {  // mtp_in.wgsl:56,65,70: v *= r * w
        v.x = v.x * (r * w.x);
        v.y = v.y * (r * w.y);
        v.z = v.z * (r * w.z);
        v.w = v.w * (r * w.w);
        return v;
    };
    // 1 / rms of the values vals(j) (mtp_in.wgsl:26-42), the lane tree's order
    auto inv_rms = [&](auto&& vals) {
#pragma unroll
        for (int j = 0; j < kSplitMaxPasses; ++j)
            if (j < J) sub[j][wave][lane] = chunk_ss(vals(j));
        __syncthreads();
        // wave w completes pass w: the tree over the waves, then over the lanes
        if (wave < J) {
            const float* sj = &sub[wave][0][lane];
            const float p = ((sj[0] + sj[64]) + (sj[128] + sj[192])) + ((sj[256] + sj[320]) + (sj[384] + sj[448]));
            const float ps = wave_sum_tree(p);
            if (lane == 0) red[wave] = ps;
        }
        __syncthreads();
        float total = 0.0f;
        for (int j = 0; j < J; ++j) total = total + red[j];
        return 1.0f / sqrt_rn(mean_of(total, K) + a.eps);
    };
    const float r0 = inv_rms([&](int j) { return xc[j]; });
    float r1 = 0.0f;
    if (hidden) r1 = inv_rms([&](int j) { return scale(xc[j], r0, wc0[j]); });  // uniform per workgroup

    QuantArgs q{};
    q.K = a.K;
    q.xq = a.xq;
    q.dx = a.dx;
    q.xs = a.xs;
#pragma unroll
    for (int j = 0; j < kSplitMaxPasses; ++j) {
        if (j >= J) break;
        const int c = chunk(j);
        const float4 v0 = scale(xc[j], r0, wc0[j]);
        emit<false, 32>(q, row, c, c < nchunk, hidden ? scale(v0, r1, wc1[j]) : v0, 0.0f, 0.0f, lane);
    }
}

template <bool NORM, bool PT, int GE>
hipError_t dispatch_rows(const QuantArgs& a, hipStream_t s) {
    const int64_t passes = (a.K + 4 * kPassChunks - 1) / (4 * kPassChunks);
    if (a.M <= kSplitMaxTokens && passes <= kSplitMaxPasses) {
#ifndef WQ_QUANT_SPLIT_WAVES
#define WQ_QUANT_SPLIT_WAVES 8
#endif
        hipLaunchKernelGGL((quant_split_kernel<NORM, PT, GE, WQ_QUANT_SPLIT_WAVES>), dim3((unsigned)a.M),
                           dim3(64 * WQ_QUANT_SPLIT_WAVES), 0, s, a.x, a.norm_w, (int)a.K, (int)a.M, a);
        return hipGetLastError();
    }
    dim3 grid((unsigned)((a.M + kQuantWaves - 1) / kQuantWaves)), block(kQuantThreads);
    if (passes <= 1)
        hipLaunchKernelGGL((quant_wave_kernel<NORM, PT, GE, 1>), grid, block, 0, s, a.x, a.norm_w, (int)a.K,
                           (int)a.M, a);
    else if (passes <= 3)
        hipLaunchKernelGGL((quant_wave_kernel<NORM, PT, GE, 3>), grid, block, 0, s, a.x, a.norm_w, (int)a.K,
                           (int)a.M, a);
    else
        hipLaunchKernelGGL((quant_wave_kernel<NORM, PT, GE, 0>), grid, block, 0, s, a.x, a.norm_w, (int)a.K,
                           (int)a.M, a);
    return hipGetLastError();
}

template <bool NORM>
hipError_t dispatch_format(const QuantArgs& a, hipStream_t s) {
    const bool pt = a.GA == a.K;
    const int ge = a.GA < a.G ? a.GA : a.G;
    if (pt && ge == 128) return dispatch_rows<NORM, true, 128>(a, s);
    if (pt && ge == 32) return dispatch_rows<NORM, true, 32>(a, s);
    return dispatch_rows<NORM, false, 32>(a, s);
}

}  // namespace

hipError_t launch_quant_act(const QuantArgs& a, hipStream_t s) {
    return a.norm_w ? dispatch_format<true>(a, s) : dispatch_format<false>(a, s);
}

hipError_t launch_mtp_in(const MtpInArgs& a, hipStream_t s) {
    const int64_t passes = (a.K + 4 * kPassChunks - 1) / (4 * kPassChunks);
    if (passes <= kSplitMaxPasses && 2 * a.M <= 65535) {
        hipLaunchKernelGGL(mtp_in_split_kernel, dim3((unsigned)(2 * a.M)), dim3(512), 0, s, a);
        return hipGetLastError();
    }
    dim3 grid((unsigned)((2 * a.M + kQuantWaves - 1) / kQuantWaves)), block(kQuantThreads);
    if (passes <= 1)
        hipLaunchKernelGGL((mtp_in_kernel<1>), grid, block, 0, s, a);
    else if (passes <= 3)
        hipLaunchKernelGGL((mtp_in_kernel<3>), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((mtp_in_kernel<0>), grid, block, 0, s, a);
    return hipGetLastError();
}

}  // namespace wq
