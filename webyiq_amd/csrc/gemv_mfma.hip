// Decode GEMV for 3..8 tokens and long outputs (N >= 16384: the lm_head) on
// int8 MFMA, per-token activations and weight group 128 (the BASELINE format) -- the operator of gemv_q4q8.hip (webyIQ
// crates/engine/src/shaders/gemv_q4q8.wgsl:36-131, Builder::gemv
// graph.rs:190-198; the lm_head + greedy argmax of graph.rs:476-486 with
// ARGMAX), for the token counts where the dot4 kernel's per-token VALU work
// (8 dot4 + a DPP quad sum + an LDS write per token, row and lane) bounds it.
//
// A workgroup of 4 waves owns RB = 16 * RBW weight rows: RBW blocks of 16
// rows, each block's K split between 4 / RBW waves (at most 16 groups per
// wave).  Per 128-group a wave runs two v_mfma_i32_16x16x64_i8, tokens x
// rows: lane l supplies token l % 16 of the activations and row l % 16 of
// the weights, both for codes 32 q .. 32 q + 31 of the group (q = l / 16;
// 16 codes per MFMA), the same code subset for both operands, so each
// result is an exact int32 group sum.  Weight chunks (16 bytes per lane and
// group) are all issued before the first is used; the int8 activations are
// staged in LDS once per workgroup.  The fp32 epilogue is the dot4 kernel's
// order -- per (token, row) and pass of 16 groups, eight chains
// c = fma(s, A, c); c = fma(m, X, c) over the pairs of groups (2i, 2i + 1),
// the pairwise tree over the 8 pair values, the pass sums in order, times
// dx -- so outputs are bit-identical to it and to the oracle.  For K <= 2048 (gemv_mfma_rows_kernel)
// a wave owns every group of its rows and the chains run in the MFMA result
// registers; for longer rows the K split meets through LDS.
#include "argmax_combine.hpp"
#include "common.hpp"
#include "launch.hpp"

#pragma clang fp contract(off)

namespace wq {
namespace {

constexpr int kWaves = 4;
constexpr int kMaxGpw = 16;  // groups per wave
static_assert(kMaxGpw == 16, "the fold's eight pair chains span the 16 groups of a 2048-code pass");

// The pairwise tree over a pass's 8 pair values.
__device__ __forceinline__ float tree8(const float (&p)[8]) {
    return ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
}
// waves per workgroup of the K <= 2048 register-chain kernel
#ifndef WQ_MFMA_ROWS_WAVES
#define WQ_MFMA_ROWS_WAVES 4
#endif
constexpr int kRowsWaves = WQ_MFMA_ROWS_WAVES;

typedef __attribute__((address_space(3))) void lds_void;

// Direct global -> LDS loads of 16 (4) bytes per lane: lane l's bytes land at
// LDS address lds + 16 l (4 l); base and lds are wave-uniform.  Inline
// assembly, so that the compiler's wait-count pass leaves them to the
// explicit wait below.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)p);
}
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* base, uint32_t off, const void* lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 ::"v"(off), "s"(uniform_ptr(base)), "s"(lds_addr(lds)) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t off, const void* lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
                 ::"v"(off), "s"(uniform_ptr(base)), "s"(lds_addr(lds)) : "memory", "m0");
}
#pragma clang diagnostic pop

struct MfmaGemvParams {
    LinearArgs a;
    ArgmaxArgs am;
    int NG;       // groups per row = K / 128
    int NGP;      // LDS row stride of the group sums / scale pairs (16-byte rows)
    int gpw;      // groups per wave = ceil(NG / KSPLIT)
    int nblocks;  // gridDim.x
};

template <int MT, int MODE, int RBW, bool ARGMAX>
__global__ __launch_bounds__(256) void gemv_mfma_kernel(MfmaGemvParams p) {
    constexpr int NH = MODE == 2 ? 2 : 1;  // gate (+ up) row halves
    constexpr int RB = 16 * RBW;           // rows per workgroup
    extern __shared__ __align__(16) unsigned char smem[];
    const LinearArgs& a = p.a;
    pin_arg(a.wq); pin_arg(a.ws); pin_arg(a.xq); pin_arg(a.dx); pin_arg(a.xs); pin_arg(a.y);
    pin_arg(a.acc_dump); pin_arg(a.N); pin_arg(a.K); pin_arg(a.M);
    pin_arg(p.NG); pin_arg(p.NGP); pin_arg(p.gpw);
    if (ARGMAX) {
        pin_arg(p.am.ids); pin_arg(p.am.tok_out); pin_arg(p.am.keys); pin_arg(p.am.ticket);
        pin_arg(p.nblocks);
    }
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int K = (int)a.K;
    const int NG = p.NG, NGP = p.NGP, gpw = p.gpw;
    const int64_t N = a.N;
    const int blk = wave % RBW;       // this wave's row block
    const int g0 = (wave / RBW) * gpw;  // its first group
    const int ng = NG - g0 < gpw ? NG - g0 : gpw;  // its groups (>= 1: see the launcher)
    const int64_t r0 = (int64_t)blockIdx.x * RB;
    const int c = lane & 15, q = lane >> 4;

    // LDS: group sums [MT][NH][RB][NGP] i32 | (s, m) [NH][RB][NGP] f32x2 |
    //      activation group sums [MT * NG, 64-rounded] i32 | scales [64] f32 |
    //      int8 activations [MT][K]
    int32_t* acc_lds = reinterpret_cast<int32_t*>(smem);
    float2* sm_lds = reinterpret_cast<float2*>(acc_lds + (size_t)MT * NH * RB * NGP);
    int32_t* xs_lds = reinterpret_cast<int32_t*>(sm_lds + (size_t)NH * RB * NGP);
    float* dx_lds = reinterpret_cast<float*>(xs_lds + ((MT * NG + 63) & ~63));
    unsigned char* xq_lds = reinterpret_cast<unsigned char*>(dx_lds + 64);

    // 1. the activations, their group sums and scales go global -> LDS
    //    directly (no registers), issued first; then every weight chunk and
    //    scale word of this lane, a fixed number of loads (groups past this
    //    wave's last re-read it) so that one wait below covers exactly the
    //    direct-to-LDS loads
    const int xchunks = (int)(a.M * K / 16);  // 16-byte chunks of the real tokens
    for (int base = 64 * wave; base < xchunks; base += 256)
        dma16(a.xq, 16u * (uint32_t)(base + lane < xchunks ? base + lane : 0), xq_lds + 16 * base);
    const int nxs = (int)a.M * NG;
    for (int base = 64 * wave; base < nxs; base += 256)
        dma4(a.xs, 4u * (uint32_t)(base + lane < nxs ? base + lane : 0), xs_lds + base);
    if (wave == 0) dma4(a.dx, 4u * (uint32_t)(lane < a.M ? lane : 0), dx_lds);
    int64_t row = r0 + 16 * blk + c;
    row = row < N ? row : N - 1;
    uint4 wv[NH][kMaxGpw];
    uint32_t sv[NH][kMaxGpw / 4];
    // plain (cached) loads: each 128-byte line holds two consecutive groups
    // of a row, read by two loads of the same lane; the streamed form
    // measured 4-5 % slower here (the dot4 kernel, one load per line, keeps it)
#pragma unroll
    for (int i = 0; i < kMaxGpw; ++i) {
        const int gi = g0 + (i < ng ? i : ng - 1);
#pragma unroll
        for (int h = 0; h < NH; ++h)
            wv[h][i] = load16(reinterpret_cast<const unsigned char*>(a.wq) + (row + h * N) * (K / 2) + 64 * gi +
                              16 * q);
    }
#pragma unroll
    for (int i = 0; i < kMaxGpw / 4; ++i) {  // group g0 + 4 i + q
        const int gi = g0 + (4 * i + q < ng ? 4 * i + q : ng - 1);
#pragma unroll
        for (int h = 0; h < NH; ++h) sv[h][i] = a.ws[(row + h * N) * NG + gi];
    }
    // the direct-to-LDS loads (issued first) have landed: at most the weight
    // loads remain in flight
    constexpr int kWeightLoads = NH * (kMaxGpw + kMaxGpw / 4);
    static_assert(kWeightLoads < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((kWeightLoads & 15) | ((kWeightLoads >> 4) << 14) | (7 << 4));
    asm volatile("s_barrier" ::: "memory");

    // 3. per group: two MFMAs (codes 32 q .. +15, then +16 .. +31 of the group)
    const int m = c < MT ? c : MT - 1;  // token of this lane's activation operand
    const unsigned char* xr = xq_lds + m * K + 16 * 2 * q;
#pragma unroll
    for (int i = 0; i < kMaxGpw; ++i) {
        if (i >= ng) continue;
        const int g = g0 + i;
        const v4i a0 = *reinterpret_cast<const v4i*>(xr + 128 * g);
        const v4i a1 = *reinterpret_cast<const v4i*>(xr + 128 * g + 16);
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            const v4i b0{(int)(wv[h][i].x & kNibbleMask), (int)((wv[h][i].x >> 4) & kNibbleMask),
                         (int)(wv[h][i].y & kNibbleMask), (int)((wv[h][i].y >> 4) & kNibbleMask)};
            const v4i b1{(int)(wv[h][i].z & kNibbleMask), (int)((wv[h][i].z >> 4) & kNibbleMask),
                         (int)(wv[h][i].w & kNibbleMask), (int)((wv[h][i].w >> 4) & kNibbleMask)};
            v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, v4i{0, 0, 0, 0}, 0, 0, 0);
            d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, d, 0, 0, 0);
            // lane (row c, quarter q) holds tokens 4 q .. 4 q + 3
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int t = 4 * q + j;
                if (t < MT) acc_lds[((t * NH + h) * RB + 16 * blk + c) * NGP + g] = d[j];
            }
        }
    }
#pragma unroll
    for (int i = 0; i < kMaxGpw / 4; ++i) {
        const int gi = 4 * i + q;
        if (gi < ng) {
#pragma unroll
            for (int h = 0; h < NH; ++h)
                sm_lds[(h * RB + 16 * blk + c) * NGP + g0 + gi] = make_float2(f16lo(sv[h][i]), f16hi(sv[h][i]));
        }
    }
    __syncthreads();

    if (a.acc_dump) {  // test hook: the group sums exactly as the epilogue reads them
        const int rows_total = NH * (int)N;
        for (int i = tid; i < MT * NH * RB * NG; i += 256) {
            const int ee = i % NG, rl = (i / NG) % RB, h = (i / (NG * RB)) % NH, t = i / (NG * RB * NH);
            const int64_t rr = r0 + rl;
            if (t < a.M && rr < N)
                a.acc_dump[((int64_t)t * rows_total + h * N + rr) * NG + ee] = acc_lds[((t * NH + h) * RB + rl) * NGP + ee];
        }
    }

    // 4. fp32 epilogue per (token, row), in the dot4 kernel's group-128 order
    auto chain = [&](int t, int h, int rl) -> float {
        const int32_t* ar = acc_lds + ((t * NH + h) * RB + rl) * NGP;
        const float2* sr = sm_lds + (h * RB + rl) * NGP;
        const int32_t* xsr = xs_lds + t * NG;
        // per pass of 16 groups a chain per pair of groups (those that
        // exist), the pairwise tree over the 8 pairs, the pass sums added
        // in order
        float total = 0.0f;
        for (int e0 = 0; e0 < NG; e0 += 16) {
            float c[8];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int ee = e0 + 4 * q;
                float c0 = 0.0f, c1 = 0.0f;
                if (ee + 3 < NG && (NG & 3) == 0) {
                    const int4 a4 = *reinterpret_cast<const int4*>(ar + ee);
                    const int4 xi = *reinterpret_cast<const int4*>(xsr + ee);
                    const float4 w01 = *reinterpret_cast<const float4*>(sr + ee);
                    const float4 w23 = *reinterpret_cast<const float4*>(sr + ee + 2);
                    c0 = fmaf(w01.y, (float)xi.x, fmaf(w01.x, (float)a4.x, c0));
                    c0 = fmaf(w01.w, (float)xi.y, fmaf(w01.z, (float)a4.y, c0));
                    c1 = fmaf(w23.y, (float)xi.z, fmaf(w23.x, (float)a4.z, c1));
                    c1 = fmaf(w23.w, (float)xi.w, fmaf(w23.z, (float)a4.w, c1));
                } else {
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int ek = ee + k;
                        if (ek < NG) {
                            const float2 w = sr[ek];
                            float& cc = k < 2 ? c0 : c1;
                            cc = fmaf(w.y, (float)xsr[ek], fmaf(w.x, (float)ar[ek], cc));
                        }
                    }
                }
                c[2 * q] = c0;
                c[2 * q + 1] = c1;
            }
            const float tp = tree8(c);
            total = e0 == 0 ? tp : total + tp;
        }
        return total * dx_lds[t];
    };
    if (!ARGMAX) {
        for (int o = tid; o < MT * RB; o += 256) {
            const int t = o / RB, rl = o - t * RB;
            const int64_t rr = r0 + rl;
            if (t >= a.M || rr >= N) continue;
            const float v = chain(t, 0, rl);
            float* yo = a.y + (int64_t)t * N + rr;
            if (MODE == 0) {
                *yo = v;
            } else if (MODE == 1) {
                *yo = *yo + v;
            } else {
                *yo = silu_mul(v, chain(t, 1, rl));
            }
        }
        return;
    }

    // fused greedy argmax, one key per (token, row), then the cross-workgroup combine
    unsigned long long* keys = reinterpret_cast<unsigned long long*>(acc_lds);  // reused after a barrier
    float vals[(MT * RB + 255) / 256];
#pragma unroll
    for (int k = 0; k < (MT * RB + 255) / 256; ++k) {
        const int o = tid + 256 * k;
        const int t = o / RB, rl = o - t * RB;
        vals[k] = (o < MT * RB && t < a.M && r0 + rl < N) ? chain(t, 0, rl) : -3.4e38f;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < (MT * RB + 255) / 256; ++k) {
        const int o = tid + 256 * k;
        if (o >= MT * RB) break;
        const int t = o / RB, rl = o - t * RB;
        const int64_t rr = r0 + rl;
        unsigned long long key = 0;
        if (t < a.M && rr < N) {
            if (a.y) a.y[(int64_t)t * N + rr] = vals[k];
            if (vals[k] > -3.0e38f) key = argmax_key(vals[k], (uint32_t)rr);
        }
        keys[o] = key;
    }
    __syncthreads();
    const unsigned long long best = block_best<MT>(keys, RB, (int)a.M);
    argmax_combine<MT>(p.am, (int)a.M, p.nblocks, best);
}

// K <= 2048 (at most 16 groups): every wave owns all groups of a 16-row
// block and each lane runs the fp32 chains of its row and four tokens in
// registers, in the LDS chain's order (no group-sum buffer: ~27 KB of LDS,
// five workgroups per CU).  The scale words are loaded before the weights,
// so their exchange through LDS is done when the first weight group lands;
// each group's two MFMAs and its fold step then run as soon as that group
// lands (folding after the last group's MFMAs was 1-1.5 us slower on the
// lm_head shapes).  Measured against 2 and 8 waves per workgroup, 4 is
// fastest.  The MFMA's token rows 8..15 are padding; the results of tokens
// 4 q + 2, 4 q + 3 move into those lanes (two lane swaps per group), so
// each lane folds two tokens, not four.  An earlier split of the fold
// between the wave's halves (MFMA rows 8..15 repeating tokens 0..7, odd
// pairs in the upper lanes, a lane exchange before the tree) was measured
// much slower (38.9 -> 63.3 us at 8 tokens x 151,936 rows).
// Store and argmax instances are held to 96 VGPRs: five workgroups per CU
// (the LDS allows five) overlap one another's loads and compute (38.65
// against 39.86 us at 8 tokens x 151,936 rows; six spill).
// The leading arguments are what the first loads need (operand pointers,
// N, K, M and the group counts packed as NG | NGP << 16); this translation
// unit preloads them into SGPRs (-amdgpu-kernarg-preload-count=8), so no
// scalar load of the argument segment precedes the first loads.  The rest is
// read from the parameter struct once the loads are in flight.
template <int MT, int MODE, bool ARGMAX>
__global__ __launch_bounds__(64 * kRowsWaves, (MODE == 0 ? 5 : 1)) void gemv_mfma_rows_kernel(
    const uint32_t* kwq, const uint32_t* kws, const int8_t* kxq, const int32_t* kxs, const float* kdx, int kN, int kK,
    uint32_t kmg, MfmaGemvParams pk) {
    static_assert(MT == 8, "the fold's lane map spreads tokens 0..7 over both halves of the wave");
    constexpr int NH = MODE == 2 ? 2 : 1;
    constexpr int RB = 16 * kRowsWaves;  // rows per workgroup: one 16-row block per wave
    constexpr int NT = 64 * kRowsWaves;  // threads
    extern __shared__ __align__(16) unsigned char smem[];
    MfmaGemvParams p = pk;
    p.a.wq = kwq; p.a.ws = kws; p.a.xq = kxq; p.a.xs = kxs; p.a.dx = kdx;
    p.a.N = kN; p.a.K = kK; p.a.M = kmg & 255;
    p.NG = (kmg >> 8) & 255; p.NGP = kmg >> 16;
    const LinearArgs& a = p.a;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = (int)a.K;
    const int NG = p.NG, NGP = p.NGP;  // NG <= kMaxGpw
    const int64_t N = a.N;
    const int c = lane & 15, q = lane >> 4;

    // LDS: (s, m) [NH][RB][NGP] f32x2 | activation group sums [MT * NG, 64-rounded] i32 |
    //      scales [64] f32 | int8 activations [MT][K] | per-wave best keys [waves][MT]
    float2* sm_lds = reinterpret_cast<float2*>(smem);
    int32_t* xs_lds = reinterpret_cast<int32_t*>(sm_lds + (size_t)NH * RB * NGP);
    float* dx_lds = reinterpret_cast<float*>(xs_lds + ((MT * NG + 63) & ~63));
    unsigned char* xq_lds = reinterpret_cast<unsigned char*>(dx_lds + 64);
    unsigned long long* wbest = reinterpret_cast<unsigned long long*>(xq_lds + (size_t)MT * K);

    // the activations, once per workgroup (direct to LDS)
    const int xchunks = (int)(a.M * K / 16);
    for (int base = 64 * wave; base < xchunks; base += NT)
        dma16(a.xq, 16u * (uint32_t)(base + lane < xchunks ? base + lane : 0), xq_lds + 16 * base);
    const int nxs = (int)a.M * NG;
    for (int base = 64 * wave; base < nxs; base += NT)
        dma4(a.xs, 4u * (uint32_t)(base + lane < nxs ? base + lane : 0), xs_lds + base);
    if (wave == 0) dma4(a.dx, 4u * (uint32_t)(lane < a.M ? lane : 0), dx_lds);

    const int m = c < MT ? c : MT - 1;  // token of this lane's activation operand
    const unsigned char* xr = xq_lds + m * K + 16 * 2 * q;
    // The MFMA result gives lane (q, c) tokens 4 q .. 4 q + 3 of row c; for
    // q >= 2 those are padding rows (MT = 8).  Tokens 4 q + 2, 4 q + 3 of the
    // lower half are swapped into the upper half (v_permlane32_swap: lane
    // 32 + l takes lane l's value), so every lane folds two tokens: tp[j].
    const int tp0 = lane < 32 ? 4 * q : 4 * q - 6;
    const int tp[2] = {tp0, tp0 + 1};
    unsigned long long best[2] = {0, 0};  // keys of tokens tp[j] (this lane's row)

    {
        const int64_t rr = (int64_t)blockIdx.x * RB + 16 * wave + c;  // this lane's row
        const int64_t row = rr < N ? rr : N - 1;
        // the scale words first (a few bytes; they land with the activations),
        // then the weights in group order, so that each group's products and
        // fold start as soon as its own weights land
        uint32_t sv[NH][kMaxGpw / 4];
#pragma unroll
        for (int i = 0; i < kMaxGpw / 4; ++i) {  // group 4 i + q
            const int gi = 4 * i + q < NG ? 4 * i + q : NG - 1;
#pragma unroll
            for (int h = 0; h < NH; ++h) sv[h][i] = a.ws[(row + h * N) * NG + gi];
        }
        uint4 wv[NH][kMaxGpw];
#pragma unroll
        for (int i = 0; i < kMaxGpw; ++i) {
            const int gi = i < NG ? i : NG - 1;
#pragma unroll
            for (int h = 0; h < NH; ++h)  // plain loads, as in gemv_mfma_kernel
                wv[h][i] = load16(reinterpret_cast<const unsigned char*>(a.wq) + (row + h * N) * (K / 2) +
                                  64 * gi + 16 * q);
        }
        // the rest of the arguments, in SGPRs now that the loads are in flight
        pin_arg(a.y); pin_arg(a.acc_dump);
        if (ARGMAX) {
            pin_arg(p.am.ids); pin_arg(p.am.tok_out); pin_arg(p.am.keys); pin_arg(p.am.ticket);
            pin_arg(p.nblocks);
        }
        // the direct-to-LDS loads and the scale words (issued first) have
        // landed: at most the weight loads remain in flight
        constexpr int kLoads = NH * kMaxGpw;
        static_assert(kLoads < 64, "vmcnt range");
        __builtin_amdgcn_s_waitcnt((kLoads & 15) | ((kLoads >> 4) << 14) | (7 << 4));
        // every lane needs the (s, m) of all groups of its row: through LDS
#pragma unroll
        for (int i = 0; i < kMaxGpw / 4; ++i) {
            const int gi = 4 * i + q;
            if (gi < NG) {
#pragma unroll
                for (int h = 0; h < NH; ++h)
                    sm_lds[(h * RB + 16 * wave + c) * NGP + gi] = make_float2(f16lo(sv[h][i]), f16hi(sv[h][i]));
            }
        }
        __syncthreads();  // the activations (every wave's loads) and the (s, m) pairs
        // per group, in order: two MFMAs (codes 32 q .. +15, then +16 .. +31)
        // and at once the fp32 fold of (token 4 q + j, row) -- a chain per
        // pair of groups (those that exist); the pairwise tree over the 8
        // pairs follows
        const int rows_total = NH * (int)N;
        // this lane's two tokens' activation group sums
        const int32_t* xsp[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) xsp[j] = xs_lds + (tp[j] < MT ? tp[j] : MT - 1) * NG;
        float cc[NH][2][8];
#pragma unroll
        for (int h = 0; h < NH; ++h)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int k = 0; k < 8; ++k) cc[h][j][k] = 0.0f;
#pragma unroll
        for (int i = 0; i < kMaxGpw; ++i) {
            if (i >= NG) continue;  // uniform
            const v4i a0 = *reinterpret_cast<const v4i*>(xr + 128 * i);
            const v4i a1 = *reinterpret_cast<const v4i*>(xr + 128 * i + 16);
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const v4i b0{(int)(wv[h][i].x & kNibbleMask), (int)((wv[h][i].x >> 4) & kNibbleMask),
                             (int)(wv[h][i].y & kNibbleMask), (int)((wv[h][i].y >> 4) & kNibbleMask)};
                const v4i b1{(int)(wv[h][i].z & kNibbleMask), (int)((wv[h][i].z >> 4) & kNibbleMask),
                             (int)(wv[h][i].w & kNibbleMask), (int)((wv[h][i].w >> 4) & kNibbleMask)};
                v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, v4i{0, 0, 0, 0}, 0, 0, 0);
                d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, d, 0, 0, 0);
                if (a.acc_dump) {  // test hook: the group sums the chains fold
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int t = 4 * q + j;
                        if (t < a.M && rr < N) a.acc_dump[((int64_t)t * rows_total + h * N + rr) * NG + i] = d[j];
                    }
                }
                const float2 w = sm_lds[(h * RB + 16 * wave + c) * NGP + i];
                const auto s02 = __builtin_amdgcn_permlane32_swap((uint32_t)d[0], (uint32_t)d[2], false, false);
                const auto s13 = __builtin_amdgcn_permlane32_swap((uint32_t)d[1], (uint32_t)d[3], false, false);
                const int e[2] = {(int)s02[0], (int)s13[0]};
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    cc[h][j][i / 2] = fmaf(w.y, (float)xsp[j][i], fmaf(w.x, (float)e[j], cc[h][j][i / 2]));
            }
        }
        float v[NH][2];
#pragma unroll
        for (int h = 0; h < NH; ++h)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int t = tp[j] < MT ? tp[j] : MT - 1;
                v[h][j] = tree8(cc[h][j]) * dx_lds[t];
            }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int t = tp[j];
            if (t >= a.M || rr >= N) continue;
            if (ARGMAX) {
                if (a.y) a.y[(int64_t)t * N + rr] = v[0][j];
                if (v[0][j] > -3.0e38f) {
                    const unsigned long long key = argmax_key(v[0][j], (uint32_t)rr);
                    best[j] = key > best[j] ? key : best[j];
                }
            } else {
                float* yo = a.y + (int64_t)t * N + rr;
                if (MODE == 0) {
                    *yo = v[0][j];
                } else if (MODE == 1) {
                    *yo = *yo + v[0][j];
                } else {
                    *yo = silu_mul(v[0][j], v[NH - 1][j]);
                }
            }
        }
    }
    if (!ARGMAX) return;

    // the workgroup's best key per token: over the wave's 16 rows by
    // shuffles, over the 4 waves through LDS; then the cross-workgroup combine
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        unsigned long long key = best[j];
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) {
            const unsigned long long u = __shfl_xor(key, o, 16);
            key = u > key ? u : key;
        }
        if (c == 0 && tp[j] < MT) wbest[wave * MT + tp[j]] = key;
    }
    __syncthreads();
    unsigned long long wb = 0;
    if (tid < MT && tid < a.M)
#pragma unroll
        for (int w = 0; w < kRowsWaves; ++w) wb = wbest[w * MT + tid] > wb ? wbest[w * MT + tid] : wb;
    argmax_combine<MT>(p.am, (int)a.M, p.nblocks, wb);
}

template <int MT, int MODE, bool ARGMAX>
hipError_t launch_rbw(const MfmaGemvParams& gp, int rbw, size_t lds, unsigned grid, hipStream_t s) {
    dim3 g(grid), b(64 * kWaves);
    switch (rbw) {
        case 2: hipLaunchKernelGGL((gemv_mfma_kernel<MT, MODE, 2, ARGMAX>), g, b, lds, s, gp); break;
        default: hipLaunchKernelGGL((gemv_mfma_kernel<MT, MODE, 1, ARGMAX>), g, b, lds, s, gp); break;
    }
    return hipGetLastError();
}

}  // namespace

// Measured (8 tokens, K = 2048): 12.1 us against 18.9 us for the dot4 kernel
// at N = 32768, but slower below ~16K rows, where staging the activations
// per workgroup and the extra barrier are not amortised.
bool gemv_mfma_fits(const LinearArgs& a) {
    return a.GA == a.K && a.G == 128 && a.M >= 3 && a.M <= 8 && a.K <= 8192 && a.N >= 16384;
}

hipError_t launch_gemv_mfma(const LinearArgs& a, const ArgmaxArgs* am, hipStream_t s) {
    MfmaGemvParams gp{};
    gp.a = a;
    if (am) gp.am = *am;
    const int NG = (int)(a.K / 128);
    // row blocks per workgroup (the rest of the 4 waves split K, <= 16 groups
    // each): as many as K allows while the grid still covers the 256 CUs
    int rbw = NG <= kMaxGpw ? 4 : NG <= 2 * kMaxGpw ? 2 : 1;
    while (rbw > 1 && (a.N + 16 * rbw - 1) / (16 * rbw) < 256) rbw /= 2;
    const int ksplit = kWaves / rbw;
    gp.NG = NG;
    gp.NGP = (NG + 4) & ~3;
    gp.gpw = (NG + ksplit - 1) / ksplit;
    const int rb = 16 * rbw, nh = a.mode == 2 ? 2 : 1, mt = 8;
    const unsigned grid = (unsigned)((a.N + rb - 1) / rb);
    gp.nblocks = (int)grid;
    const size_t lds = (size_t)mt * nh * rb * gp.NGP * 4 + (size_t)nh * rb * gp.NGP * 8 +
                       (size_t)((mt * NG + 63) & ~63) * 4 + 64 * 4 + (size_t)mt * a.K;
    if (rbw == kWaves) {  // K <= 2048: the register-chain kernel, 128 rows per workgroup
        const int rbr = 16 * kRowsWaves;
        const size_t lds_rows = (size_t)nh * rbr * gp.NGP * 8 + (size_t)((mt * NG + 63) & ~63) * 4 + 64 * 4 +
                                (size_t)mt * a.K + (size_t)kRowsWaves * mt * 8;
        const unsigned rgrid = (unsigned)((a.N + rbr - 1) / rbr);
        gp.nblocks = (int)rgrid;
        dim3 g(rgrid), b(64 * kRowsWaves);
        // the preloaded arguments: M, NG and NGP packed in one word
        const uint32_t mg = (uint32_t)a.M | ((uint32_t)gp.NG << 8) | ((uint32_t)gp.NGP << 16);
#define WQ_ROWS_LAUNCH(MODE_, ARGMAX_)                                                                          \
    hipLaunchKernelGGL((gemv_mfma_rows_kernel<8, MODE_, ARGMAX_>), g, b, lds_rows, s, a.wq, a.ws, a.xq, a.xs, \
                       a.dx, (int)a.N, (int)a.K, mg, gp)
        if (am) {
            WQ_ROWS_LAUNCH(0, true);
        } else {
            switch (a.mode) {
                case 0: WQ_ROWS_LAUNCH(0, false); break;
                case 1: WQ_ROWS_LAUNCH(1, false); break;
                default: WQ_ROWS_LAUNCH(2, false); break;
            }
        }
#undef WQ_ROWS_LAUNCH
        return hipGetLastError();
    }
    if (am) return launch_rbw<8, 0, true>(gp, rbw, lds, grid, s);
    switch (a.mode) {
        case 0: return launch_rbw<8, 0, false>(gp, rbw, lds, grid, s);
        case 1: return launch_rbw<8, 1, false>(gp, rbw, lds, grid, s);
        default: return launch_rbw<8, 2, false>(gp, rbw, lds, grid, s);
    }
}

}  // namespace wq
