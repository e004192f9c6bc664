// Prefill GEMM Y[M, N] = X W^T on int8 MFMA (webyIQ
// crates/engine/src/shaders/gemm_q4q8.wgsl, host side Builder::gemm in
// crates/engine/src/graph.rs:200-205; the reference runs it on ALU
// dot4I8Packed in 32x32 tiles).
//
// MI355X design.  A workgroup of 4 waves (2 x 2) owns a BM-token x BN-row
// output tile.  Per K step of 128 codes the packed int4 weight tile (BN x 64 B)
// and the int8 activation tile (BM x 128 B) are staged in LDS (the next step's
// tiles are already in flight in registers).  Each wave expands its weight
// fragments nibble -> int8 in registers and feeds v_mfma_i32_16x16x64_i8
// (16x16x32 for 32-code groups).  The int32 accumulator of a group is exact;
// at each group boundary it is folded into the fp32 accumulator with the same
// fma chain as the GEMV and the CPU oracle:
//   acc = fma(s, A, acc); acc = fma(m, X, acc)      (per-token activations)
// so GEMM and GEMV outputs agree bit for bit.  Tiles are mapped XCD by XCD so
// that the workgroups sharing a weight tile share one L2.
#include "common.hpp"
#include "launch.hpp"

#pragma clang fp contract(off)

namespace wq {
namespace {

constexpr int kBK = 128;         // codes per K step
constexpr int kThreads = 256;    // 4 waves
constexpr int kXcds = 8;         // MI355X: 8 XCDs, workgroups dispatched round robin

struct GemmParams {
    LinearArgs a;
    int tilesM, tilesN;
    int NE, NG;
};

template <int BM, int BN, int G, bool PT, int MODE>
__global__ __launch_bounds__(kThreads) void gemm_kernel(GemmParams p) {
    constexpr int GE = PT ? G : 32;         // accumulation group
    constexpr int KS = GE >= 64 ? 64 : 32;  // codes per MFMA
    constexpr int MPG = GE / KS;            // MFMAs per group
    constexpr int NES = kBK / GE;           // accumulation groups per K step
    constexpr int NGS = kBK / G;            // weight groups per K step
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TM = WM / 16, TN = WN / 16;
    constexpr int ASTR = kBK + 16;          // LDS row strides (bank spread)
    constexpr int BSTR = kBK / 2 + 8;
    constexpr int A_PER_T = BM * (kBK / 16) / kThreads;
    constexpr int B_PER_T = BN * (kBK / 32) / kThreads;
    static_assert(A_PER_T * kThreads == BM * (kBK / 16), "A tile split");
    static_assert(B_PER_T * kThreads == BN * (kBK / 32), "B tile split");
    static_assert(MODE != 2 || TN % 2 == 0, "mode 2 pairs gate/up subtiles");
    constexpr int S_PER_T = (BN * NGS + kThreads - 1) / kThreads;  // scale words per thread
    constexpr int X_PER_T = (BM * NES + kThreads - 1) / kThreads;  // group sums per thread

    __shared__ __align__(16) unsigned char As[BM * ASTR];
    __shared__ __align__(16) unsigned char Bs[BN * BSTR];
    __shared__ uint32_t Ss[BN * NGS];
    __shared__ __align__(16) float Xs[BM * NES];
    __shared__ __align__(16) float Ds[PT ? 1 : BM * NES];

    const LinearArgs& a = p.a;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t M = a.M, N = a.N;
    const int K = (int)a.K;

    // XCD-aware tile order: consecutive tiles (same weight columns) on one XCD
    const int T = p.tilesM * p.tilesN;
    const int bid = blockIdx.x;
    const int xcd = bid % kXcds, li = bid / kXcds;
    const int per = T / kXcds, rem = T % kXcds;
    const int lt = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + li;
    const int tile_n = lt / p.tilesM, tile_m = lt % p.tilesM;
    const int64_t m0 = (int64_t)tile_m * BM;
    constexpr int OUTW = MODE == 2 ? BN / 2 : BN;  // output columns per tile
    const int64_t n0 = (int64_t)tile_n * OUTW;

    // weight row of tile row r (mode 2: first half gate rows, second half up rows)
    auto wrow = [&](int r) -> int64_t {
        if (MODE == 2) {
            int64_t n = n0 + (r < BN / 2 ? r : r - BN / 2);
            n = n < N ? n : N - 1;
            return r < BN / 2 ? n : n + N;
        }
        int64_t n = n0 + r;
        return n < N ? n : N - 1;
    };
    auto trow = [&](int r) -> int64_t {
        int64_t t = m0 + r;
        return t < M ? t : M - 1;
    };

    const unsigned char* wbytes = reinterpret_cast<const unsigned char*>(a.wq);
    const size_t row_bytes = (size_t)K / 2;

    uint4 ra[A_PER_T], rb[B_PER_T];
    uint32_t rs[S_PER_T] = {};
    int32_t rx[X_PER_T] = {};
    float rd[X_PER_T] = {};
    auto prefetch = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_PER_T; ++i) {
            int c = tid + kThreads * i;
            int r = c / (kBK / 16), c16 = c % (kBK / 16);
            ra[i] = load16(a.xq + trow(r) * K + k0 + 16 * c16);
        }
#pragma unroll
        for (int i = 0; i < B_PER_T; ++i) {
            int c = tid + kThreads * i;
            int r = c / (kBK / 32), c16 = c % (kBK / 32);
            rb[i] = load16(wbytes + (size_t)wrow(r) * row_bytes + k0 / 2 + 16 * c16);
        }
#pragma unroll
        for (int i = 0; i < S_PER_T; ++i) {
            int c = tid + kThreads * i;
            if (c < BN * NGS) rs[i] = a.ws[wrow(c / NGS) * p.NG + k0 / G + c % NGS];
        }
#pragma unroll
        for (int i = 0; i < X_PER_T; ++i) {
            int c = tid + kThreads * i;
            if (c < BM * NES) {
                rx[i] = a.xs[trow(c / NES) * p.NE + k0 / GE + c % NES];
                if (!PT) rd[i] = a.dx[trow(c / NES) * (K / 32) + k0 / 32 + c % NES];
            }
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < A_PER_T; ++i) {
            int c = tid + kThreads * i;
            int r = c / (kBK / 16), c16 = c % (kBK / 16);
            *reinterpret_cast<uint4*>(As + r * ASTR + 16 * c16) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_PER_T; ++i) {
            int c = tid + kThreads * i;
            int r = c / (kBK / 32), c16 = c % (kBK / 32);
            uint2* dst = reinterpret_cast<uint2*>(Bs + r * BSTR + 16 * c16);
            dst[0] = make_uint2(rb[i].x, rb[i].y);
            dst[1] = make_uint2(rb[i].z, rb[i].w);
        }
#pragma unroll
        for (int i = 0; i < S_PER_T; ++i) {
            int c = tid + kThreads * i;
            if (c < BN * NGS) Ss[c] = rs[i];
        }
#pragma unroll
        for (int i = 0; i < X_PER_T; ++i) {
            int c = tid + kThreads * i;
            if (c < BM * NES) {
                Xs[c] = (float)rx[i];
                if (!PT) Ds[c] = rd[i];
            }
        }
    };

    // output-space subtile bases (tile rows of W) for this wave
    auto bbase = [&](int jj) -> int {
        if (MODE == 2) {
            constexpr int H = TN / 2;
            return jj < H ? wn * (BN / 4) + 16 * jj : BN / 2 + wn * (BN / 4) + 16 * (jj - H);
        }
        return wn * WN + 16 * jj;
    };

    v4f facc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int jj = 0; jj < TN; ++jj) facc[i][jj] = v4f{0.f, 0.f, 0.f, 0.f};

    const int rows_total = MODE == 2 ? 2 * (int)N : (int)N;
    const int nsteps = K / kBK;
    prefetch(0);
    for (int step = 0; step < nsteps; ++step) {
        stage();
        __syncthreads();
        if (step + 1 < nsteps) prefetch((step + 1) * kBK);

#pragma unroll 1
        for (int ge = 0; ge < NES; ++ge) {
            v4i iacc[TM][TN];
#pragma unroll
            for (int kk = 0; kk < MPG; ++kk) {
                const int koff = ge * GE + kk * KS;
                if (KS == 64) {
                    v4i af[TM], bf[TN];
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        const int r = wm * WM + 16 * i + (lane & 15);
                        af[i] = *reinterpret_cast<const v4i*>(As + r * ASTR + koff + 16 * (lane >> 4));
                    }
#pragma unroll
                    for (int jj = 0; jj < TN; ++jj) {
                        const int r = bbase(jj) + (lane & 15);
                        uint2 w = *reinterpret_cast<const uint2*>(Bs + r * BSTR + (koff + 16 * (lane >> 4)) / 2);
                        bf[jj] = v4i{(int)(w.x & kNibbleMask), (int)((w.x >> 4) & kNibbleMask),
                                     (int)(w.y & kNibbleMask), (int)((w.y >> 4) & kNibbleMask)};
                    }
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int jj = 0; jj < TN; ++jj)
                            iacc[i][jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                                af[i], bf[jj], kk == 0 ? v4i{0, 0, 0, 0} : iacc[i][jj], 0, 0, 0);
                } else {
                    long af[TM], bf[TN];
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        const int r = wm * WM + 16 * i + (lane & 15);
                        af[i] = *reinterpret_cast<const long*>(As + r * ASTR + koff + 8 * (lane >> 4));
                    }
#pragma unroll
                    for (int jj = 0; jj < TN; ++jj) {
                        const int r = bbase(jj) + (lane & 15);
                        uint32_t w = *reinterpret_cast<const uint32_t*>(Bs + r * BSTR + (koff + 8 * (lane >> 4)) / 2);
                        uint64_t lo = w & kNibbleMask, hi = (w >> 4) & kNibbleMask;
                        bf[jj] = (long)(lo | (hi << 32));
                    }
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int jj = 0; jj < TN; ++jj)
                            iacc[i][jj] = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                                af[i], bf[jj], kk == 0 ? v4i{0, 0, 0, 0} : iacc[i][jj], 0, 0, 0);
                }
            }

            if (a.acc_dump) {  // test hook: the exact group sums this tile produced
                const int64_t e = (int64_t)step * NES + ge;
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int jj = 0; jj < TN; ++jj)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            int64_t t = m0 + wm * WM + 16 * i + 4 * (lane >> 4) + r;
                            int br = bbase(jj) + (lane & 15);
                            int64_t nn = n0 + (MODE == 2 ? (br < BN / 2 ? br : br - BN / 2) : br);
                            if (t < M && nn < N) {
                                int64_t wr = MODE == 2 && br >= BN / 2 ? nn + N : nn;
                                a.acc_dump[(t * rows_total + wr) * p.NE + e] = iacc[i][jj][r];
                            }
                        }
            }

            // fold the exact group sums into the fp32 accumulators
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int tr = wm * WM + 16 * i + 4 * (lane >> 4);
                float xg[4], dg[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    xg[r] = Xs[(tr + r) * NES + ge];
                    dg[r] = PT ? 0.0f : Ds[(tr + r) * NES + ge];
                }
#pragma unroll
                for (int jj = 0; jj < TN; ++jj) {
                    const uint32_t sw = Ss[(bbase(jj) + (lane & 15)) * NGS + (ge * GE) / G];
                    const float s = f16lo(sw), m = f16hi(sw);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if (PT) {
                            facc[i][jj][r] = fmaf(s, (float)iacc[i][jj][r], facc[i][jj][r]);
                            facc[i][jj][r] = fmaf(m, xg[r], facc[i][jj][r]);
                        } else {
                            facc[i][jj][r] = fmaf(s * dg[r], (float)iacc[i][jj][r], facc[i][jj][r]);
                            facc[i][jj][r] = fmaf(m * dg[r], xg[r], facc[i][jj][r]);
                        }
                    }
                }
            }
        }
        __syncthreads();
    }

    // epilogue: per-token scale, output mode, store
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t t = m0 + wm * WM + 16 * i + 4 * (lane >> 4) + r;
            if (t >= M) continue;
            const float d = PT ? a.dx[t] : 1.0f;
            constexpr int JO = MODE == 2 ? TN / 2 : TN;
#pragma unroll
            for (int jj = 0; jj < JO; ++jj) {
                const int br = bbase(jj) + (lane & 15);
                const int64_t n = n0 + br;
                if (n >= N) continue;
                float v = PT ? facc[i][jj][r] * d : facc[i][jj][r];
                float* yo = a.y + t * N + n;
                if (MODE == 0) {
                    *yo = v;
                } else if (MODE == 1) {
                    *yo = *yo + v;
                } else {
                    float u = PT ? facc[i][jj + TN / 2][r] * d : facc[i][jj + TN / 2][r];
                    *yo = silu_mul(v, u);
                }
            }
        }
    }
}

template <int BM, int BN, int G, bool PT>
hipError_t launch_mode(const GemmParams& gp, hipStream_t s) {
    dim3 grid((unsigned)(gp.tilesM * gp.tilesN)), block(kThreads);
    switch (gp.a.mode) {
        case 0: hipLaunchKernelGGL((gemm_kernel<BM, BN, G, PT, 0>), grid, block, 0, s, gp); break;
        case 1: hipLaunchKernelGGL((gemm_kernel<BM, BN, G, PT, 1>), grid, block, 0, s, gp); break;
        default: hipLaunchKernelGGL((gemm_kernel<BM, BN, G, PT, 2>), grid, block, 0, s, gp); break;
    }
    return hipGetLastError();
}

template <int BM, int BN>
hipError_t launch_tile(const LinearArgs& a, hipStream_t s) {
    GemmParams gp{};
    gp.a = a;
    const bool pt = a.GA == a.K;
    const int ge = pt ? a.G : 32;
    const int outw = a.mode == 2 ? BN / 2 : BN;
    gp.tilesM = (int)((a.M + BM - 1) / BM);
    gp.tilesN = (int)((a.N + outw - 1) / outw);
    gp.NE = (int)(a.K / ge);
    gp.NG = (int)(a.K / a.G);
    if (a.G == 128)
        return pt ? launch_mode<BM, BN, 128, true>(gp, s) : launch_mode<BM, BN, 128, false>(gp, s);
    return pt ? launch_mode<BM, BN, 32, true>(gp, s) : launch_mode<BM, BN, 32, false>(gp, s);
}

}  // namespace

hipError_t launch_gemm(const LinearArgs& a, hipStream_t s) {
    return launch_tile<128, 128>(a, s);
}

}  // namespace wq
