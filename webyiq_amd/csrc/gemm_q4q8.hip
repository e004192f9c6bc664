// Prefill GEMM Y[M, N] = X W^T on int8 MFMA (webyIQ
// crates/engine/src/shaders/gemm_q4q8.wgsl, host side Builder::gemm in
// crates/engine/src/graph.rs:200-205; the reference runs it on ALU
// dot4I8Packed in 32x32 tiles).
//
// y[t,n] = dx[t] * sum_g (s[n,g] * A[t,n,g] + m[n,g] * X[t,g]),
// A = exact int32 sum of q * xq over group g, X = sum of xq over g.
//
// MI355X design.  A workgroup of 8 waves (2 along M x 4 along N, two waves per
// SIMD so one wave's VALU fold overlaps the other's MFMAs) owns a 128-token x
// BN-row tile; BN is chosen by the host so that the grid covers the 256 CUs.
// Per K step of 128 codes the int8 activation tile (128 x 128 B) and the
// packed int4 weight tile (BN x 64 B) go global -> registers -> LDS into one of
// two buffers while the other buffer feeds the MFMAs: one barrier per step.
// Each wave reads its weight fragments packed (8 B = 16 codes per lane),
// expands nibbles to int8 in registers and issues v_mfma_i32_16x16x64_i8
// (16x16x32 for 32-code groups).  The int32 group sums are exact.
//
// Folding the group sums into fp32 is VALU work per output element per group
// (it costs as much as the MFMAs), so the per-token group-128 format keeps it
// at two instructions, acc = fma(s, float(A), acc), and moves the min term
// sum_g m * X onto an f16 MFMA at the start: X = 64 * X_hi + X_lo with
// X_hi, X_lo exact in f16 (|X| <= 128 * 127) and m, 64 * m exact f16, so one
// v_mfma_f32_16x16x32_f16 per 16 groups computes it with exact products.
// Other formats (group 32, per-32 activation scales) fold both terms on the
// VALU in the GEMV's order.  Tiles are assigned XCD by XCD so that the
// workgroups sharing a weight tile share one L2.
#include "common.hpp"
#include "launch.hpp"

#pragma clang fp contract(off)

namespace wq {
namespace {

constexpr int kBK = 128;       // codes per K step
constexpr int kBM = 128;       // tokens per tile
constexpr int kConsumers = 8;  // waves running MFMAs (2 along M x 4 along N)
constexpr int kProducers = 4;  // waves staging tiles global -> LDS
constexpr int kThreads = 64 * (kConsumers + kProducers);
constexpr int kProdThreads = 64 * kProducers;
constexpr int kXcds = 8;       // MI355X: 8 XCDs, workgroups dispatched round robin
#ifndef WQ_GEMM_PREFETCH
#define WQ_GEMM_PREFETCH 4
#endif
// K steps of tiles in flight in the producers' registers (even, so that the
// LDS buffer of an unrolled step is a constant)
constexpr int kPrefetchSteps = WQ_GEMM_PREFETCH;

typedef _Float16 v8h __attribute__((ext_vector_type(8)));

struct GemmParams {
    LinearArgs a;
    int tilesM, tilesN;
    int NE, NG;
};

template <int BN, int G, bool PT, int MODE, bool DUMP>
__global__ __launch_bounds__(kThreads) void gemm_kernel(GemmParams p) {
    constexpr int PF = kPrefetchSteps;
    constexpr int BM = kBM;
    constexpr int GE = PT ? G : 32;         // accumulation group
    constexpr int KS = GE >= 64 ? 64 : 32;  // codes per MFMA
    constexpr int MPG = GE / KS;            // MFMAs per group and subtile
    constexpr int NES = kBK / GE;           // accumulation groups per K step
    constexpr int NGS = kBK / G;            // weight groups per K step
    constexpr bool FAST = PT && G == 128;   // min term on the f16 MFMA
    constexpr int WM = BM / 2, WN = BN / 4;
    constexpr int TM = WM / 16, TN = WN / 16;
    constexpr int ASTR = kBK + 16;          // LDS row strides (bank spread)
    constexpr int BSTR = kBK / 2 + 8;
    constexpr int A_CH = BM * (kBK / 16), B_CH = BN * (kBK / 32);  // 16-byte chunks per tile
    constexpr int A_PER_T = (A_CH + kProdThreads - 1) / kProdThreads;
    constexpr int B_PER_T = (B_CH + kProdThreads - 1) / kProdThreads;
    constexpr int S_PER_T = (BN * NGS + kProdThreads - 1) / kProdThreads;
    constexpr int X_PER_T = FAST ? 0 : (BM * NES + kProdThreads - 1) / kProdThreads;
    constexpr int XR = X_PER_T > 0 ? X_PER_T : 1;
    static_assert(TN >= 1 && BN % 64 == 0, "tile width");
    static_assert(MODE != 2 || TN % 2 == 0, "mode 2 pairs gate/up subtiles");
    static_assert(PF % 2 == 0, "even ring: the LDS buffer of an unrolled step is static");

    __shared__ __align__(16) unsigned char As[2][BM * ASTR];
    __shared__ __align__(16) unsigned char Bs[2][BN * BSTR];
    __shared__ uint32_t Ss[2][BN * NGS];
    __shared__ __align__(16) float Xs[2][FAST ? 1 : BM * NES];
    __shared__ __align__(16) float Ds[2][PT ? 1 : BM * NES];

    const LinearArgs& a = p.a;
    pin_arg(a.wq); pin_arg(a.ws); pin_arg(a.xq); pin_arg(a.dx); pin_arg(a.xs); pin_arg(a.y);
    pin_arg(a.N); pin_arg(a.K); pin_arg(a.M);
    pin_arg(p.tilesM); pin_arg(p.tilesN); pin_arg(p.NE); pin_arg(p.NG);
    if (DUMP) pin_arg(a.acc_dump);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t M = a.M, N = a.N;
    const int K = (int)a.K;
    const int NG = p.NG, NE = p.NE;
    const int nsteps = K / kBK;

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

    if (wave >= kConsumers) {
        // ---------------- producer waves: global -> register ring -> LDS ----
        const int pt = tid - 64 * kConsumers;
        const unsigned char* xq_b = reinterpret_cast<const unsigned char*>(a.xq);
        const unsigned char* wq_b = reinterpret_cast<const unsigned char*>(a.wq);
        uint32_t a_off[A_PER_T], b_off[B_PER_T], s_off[S_PER_T], x_off[XR], d_off[XR];
        int a_dst[A_PER_T], b_dst[B_PER_T];
#pragma unroll
        for (int i = 0; i < A_PER_T; ++i) {
            int c = pt + kProdThreads * i;
            c = c < A_CH ? c : A_CH - 1;
            int r = c / (kBK / 16), c16 = c % (kBK / 16);
            a_off[i] = (uint32_t)(trow(r) * K + 16 * c16);
            a_dst[i] = r * ASTR + 16 * c16;
        }
#pragma unroll
        for (int i = 0; i < B_PER_T; ++i) {
            int c = pt + kProdThreads * i;
            c = c < B_CH ? c : B_CH - 1;
            int r = c / (kBK / 32), c16 = c % (kBK / 32);
            b_off[i] = (uint32_t)(wrow(r) * (K / 2) + 16 * c16);
            b_dst[i] = r * BSTR + 16 * c16;
        }
#pragma unroll
        for (int i = 0; i < S_PER_T; ++i) {
            int c = pt + kProdThreads * i;
            c = c < BN * NGS ? c : 0;
            s_off[i] = (uint32_t)(wrow(c / NGS) * NG + c % NGS);
        }
#pragma unroll
        for (int i = 0; i < X_PER_T; ++i) {
            int c = pt + kProdThreads * i;
            c = c < BM * NES ? c : 0;
            x_off[i] = (uint32_t)(trow(c / NES) * NE + c % NES);
            d_off[i] = (uint32_t)(trow(c / NES) * (K / 32) + c % NES);
        }
        // ring of PF steps in flight; every load is unconditional (steps past
        // the end re-read the last one) so the wait before a stage covers only
        // the oldest slot
        uint4 ra[PF][A_PER_T], rb[PF][B_PER_T];
        uint32_t rs[PF][S_PER_T];
        int32_t rx[PF][XR];
        float rd[PF][XR];
        auto prefetch = [&](int step, const int q) {
            step = step < nsteps ? step : nsteps - 1;
            const int k0 = step * kBK;
#pragma unroll
            for (int i = 0; i < A_PER_T; ++i) ra[q][i] = load16(xq_b + a_off[i] + k0);
#pragma unroll
            for (int i = 0; i < B_PER_T; ++i) rb[q][i] = load_stream16(wq_b + b_off[i] + k0 / 2);
#pragma unroll
            for (int i = 0; i < S_PER_T; ++i) rs[q][i] = a.ws[s_off[i] + step * NGS];
#pragma unroll
            for (int i = 0; i < X_PER_T; ++i) {
                rx[q][i] = a.xs[x_off[i] + step * NES];
                if (!PT) rd[q][i] = a.dx[d_off[i] + step * NES];
            }
        };
        auto stage = [&](const int buf, const int q) {
#pragma unroll
            for (int i = 0; i < A_PER_T; ++i)
                if (A_CH % kProdThreads == 0 || pt + kProdThreads * i < A_CH)
                    *reinterpret_cast<uint4*>(&As[buf][a_dst[i]]) = ra[q][i];
#pragma unroll
            for (int i = 0; i < B_PER_T; ++i) {
                if (B_CH % kProdThreads == 0 || pt + kProdThreads * i < B_CH) {
                    uint2* dst = reinterpret_cast<uint2*>(&Bs[buf][b_dst[i]]);
                    dst[0] = make_uint2(rb[q][i].x, rb[q][i].y);
                    dst[1] = make_uint2(rb[q][i].z, rb[q][i].w);
                }
            }
#pragma unroll
            for (int i = 0; i < S_PER_T; ++i) {
                int c = pt + kProdThreads * i;
                if (c < BN * NGS) Ss[buf][c] = rs[q][i];
            }
#pragma unroll
            for (int i = 0; i < X_PER_T; ++i) {
                int c = pt + kProdThreads * i;
                if (c < BM * NES) {
                    Xs[buf][c] = (float)rx[q][i];
                    if (!PT) Ds[buf][c] = rd[q][i];
                }
            }
        };
#pragma unroll
        for (int q = 0; q < PF; ++q) prefetch(q, q);
        stage(0, 0);
        prefetch(PF, 0);  // slot s % PF holds step s: slot 0 moves on to step PF
        __syncthreads();
        // iteration i: stage step i + 1 (slot (i+1) % PF) into the buffer the
        // consumers are not reading, refill that slot with step i + 1 + PF
        for (int s0 = 0; s0 < nsteps; s0 += PF) {
#pragma unroll
            for (int u = 0; u < PF; ++u) {
                stage((u + 1) & 1, (u + 1) % PF);
                prefetch(s0 + u + 1 + PF, (u + 1) % PF);
                if (s0 + u < nsteps) __syncthreads();
            }
        }
        return;
    }

    // ---------------- consumer waves (2 along M x 4 along N) ----------------
    const int wm = wave >> 2, wn = wave & 3;
    const int l16 = lane & 15, lq = lane >> 4;
    // tile row (of W) of this lane's column in subtile jj
    auto bcol = [&](int jj) -> int {
        if (MODE == 2) {
            constexpr int H = TN / 2;
            return (jj < H ? wn * (BN / 8) + 16 * jj : BN / 2 + wn * (BN / 8) + 16 * (jj - H)) + l16;
        }
        return wn * WN + 16 * jj + l16;
    };

    v4f facc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int jj = 0; jj < TN; ++jj) facc[i][jj] = v4f{0.f, 0.f, 0.f, 0.f};

    if (FAST) {
        // min term: facc = sum_g m[n,g] * X[t,g] on v_mfma_f32_16x16x32_f16.
        // Lane quarter lq holds k = 8 lq .. 8 lq + 7 of both operands:
        // lq 0/1 -> (X_hi, 64 m) of groups 0-7 / 8-15, lq 2/3 -> (X_lo, m).
        // All loads of a block are issued before any is used (indices past
        // the last group are clamped, their values zeroed afterwards).
        const int gq = 8 * (lq & 1);
        const bool hi_half = lq < 2;
        for (int b = 0; b < NG; b += 16) {
            int32_t xv[TM][8];
            uint32_t wv[TN][8];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int32_t* xr = a.xs + trow(wm * WM + 16 * i + l16) * NE;
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int g = b + gq + u;
                    xv[i][u] = xr[g < NG ? g : NG - 1];
                }
            }
#pragma unroll
            for (int jj = 0; jj < TN; ++jj) {
                const uint32_t* sr = a.ws + wrow(bcol(jj)) * NG;
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int g = b + gq + u;
                    wv[jj][u] = sr[g < NG ? g : NG - 1];
                }
            }
            v8h xa[TM], mb[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int32_t v = b + gq + u < NG ? xv[i][u] : 0;
                    xa[i][u] = (_Float16)(hi_half ? (v >> 6) : (v & 63));
                }
#pragma unroll
            for (int jj = 0; jj < TN; ++jj)
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const float m = b + gq + u < NG ? f16hi(wv[jj][u]) : 0.0f;
                    mb[jj][u] = (_Float16)(hi_half ? 64.0f * m : m);
                }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int jj = 0; jj < TN; ++jj)
                    facc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[i], mb[jj], facc[i][jj], 0, 0, 0);
        }
    }
    // per-token scales of this lane's 16 output rows, fetched early
    float dtok[TM][4];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) dtok[i][r] = PT ? a.dx[trow(wm * WM + 16 * i + 4 * lq + r)] : 1.0f;
    const int rows_total = MODE == 2 ? 2 * (int)N : (int)N;
    __syncthreads();  // step 0 is staged

    auto compute = [&](const int step, const int buf) {
        const unsigned char* Ab = As[buf];
        const unsigned char* Bb = Bs[buf];
#pragma unroll 1
        for (int ge = 0; ge < NES; ++ge) {
            // activation sums / scales of this lane's 4 tokens per subtile row
            float xg[TM][4], dg[TM][4];
            if (!FAST) {
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int tr = wm * WM + 16 * i + 4 * lq + r;
                        xg[i][r] = Xs[buf][tr * NES + ge];
                        dg[i][r] = PT ? 0.0f : Ds[buf][tr * NES + ge];
                    }
            }
            // A fragments of the whole group (MPG k-slices)
            v4i af4[MPG][TM];
            long af2[MPG][TM];
#pragma unroll
            for (int kk = 0; kk < MPG; ++kk) {
                const int koff = ge * GE + kk * KS;
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const int r = wm * WM + 16 * i + l16;
                    if (KS == 64)
                        af4[kk][i] = *reinterpret_cast<const v4i*>(Ab + r * ASTR + koff + 16 * lq);
                    else
                        af2[kk][i] = *reinterpret_cast<const long*>(Ab + r * ASTR + koff + 8 * lq);
                }
            }
#pragma unroll
            for (int jj = 0; jj < TN; ++jj) {
                const int br = bcol(jj);
                v4i iacc[TM];
#pragma unroll
                for (int kk = 0; kk < MPG; ++kk) {
                    const int koff = ge * GE + kk * KS;
                    if (KS == 64) {
                        uint2 w = *reinterpret_cast<const uint2*>(Bb + br * BSTR + koff / 2 + 8 * lq);
                        v4i bf = v4i{(int)(w.x & kNibbleMask), (int)((w.x >> 4) & kNibbleMask),
                                     (int)(w.y & kNibbleMask), (int)((w.y >> 4) & kNibbleMask)};
#pragma unroll
                        for (int i = 0; i < TM; ++i)
                            iacc[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                                af4[kk][i], bf, kk == 0 ? v4i{0, 0, 0, 0} : iacc[i], 0, 0, 0);
                    } else {
                        uint32_t w = *reinterpret_cast<const uint32_t*>(Bb + br * BSTR + koff / 2 + 4 * lq);
                        long bf = (long)((uint64_t)(w & kNibbleMask) | ((uint64_t)((w >> 4) & kNibbleMask) << 32));
#pragma unroll
                        for (int i = 0; i < TM; ++i)
                            iacc[i] = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                                af2[kk][i], bf, kk == 0 ? v4i{0, 0, 0, 0} : iacc[i], 0, 0, 0);
                    }
                }
                if (DUMP) {  // test hook: the exact group sums this tile produced
                    const int64_t e = (int64_t)step * NES + ge;
                    const int64_t nn = n0 + (MODE == 2 ? (br < BN / 2 ? br : br - BN / 2) : br);
                    const int64_t wr = MODE == 2 && br >= BN / 2 ? nn + N : nn;
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int64_t t = m0 + wm * WM + 16 * i + 4 * lq + r;
                            if (t < M && nn < N) a.acc_dump[(t * rows_total + wr) * NE + e] = iacc[i][r];
                        }
                }
                // fold the exact group sums into the fp32 accumulators
                const uint32_t sw = Ss[buf][br * NGS + (ge * GE) / G];
                const float s = f16lo(sw), m = f16hi(sw);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float v = facc[i][jj][r];
                        if (FAST) {
                            v = fmaf(s, (float)iacc[i][r], v);
                        } else if (PT) {
                            v = fmaf(s, (float)iacc[i][r], v);
                            v = fmaf(m, xg[i][r], v);
                        } else {
                            v = fmaf(s * dg[i][r], (float)iacc[i][r], v);
                            v = fmaf(m * dg[i][r], xg[i][r], v);
                        }
                        facc[i][jj][r] = v;
                    }
            }
        }
    };
    for (int s0 = 0; s0 < nsteps; s0 += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            if (s0 + u < nsteps) {
                compute(s0 + u, u & 1);
                __syncthreads();
            }
        }
    }

    // epilogue: per-token scale, output mode, store (mode 1 reads every old
    // value of its outputs in one batch first)
    constexpr int JO = MODE == 2 ? TN / 2 : TN;
    float yold[MODE == 1 ? TM : 1][4][MODE == 1 ? JO : 1];
    if (MODE == 1) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int jj = 0; jj < JO; ++jj) {
                    const int64_t t = trow(wm * WM + 16 * i + 4 * lq + r);
                    int64_t n = n0 + bcol(jj);
                    n = n < N ? n : N - 1;
                    yold[i][r][jj] = a.y[t * N + n];
                }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t t = m0 + wm * WM + 16 * i + 4 * lq + r;
            if (t >= M) continue;
            const float d = dtok[i][r];
#pragma unroll
            for (int jj = 0; jj < JO; ++jj) {
                const int64_t n = n0 + bcol(jj);
                if (n >= N) continue;
                float v = PT ? facc[i][jj][r] * d : facc[i][jj][r];
                float* yo = a.y + t * N + n;
                if (MODE == 0) {
                    *yo = v;
                } else if (MODE == 1) {
                    *yo = yold[i][r][jj] + v;
                } else {
                    float u = PT ? facc[i][jj + TN / 2][r] * d : facc[i][jj + TN / 2][r];
                    *yo = silu_mul(v, u);
                }
            }
        }
    }
}

template <int BN, int G, bool PT, bool DUMP>
hipError_t launch_mode(const GemmParams& gp, hipStream_t s) {
    dim3 grid((unsigned)(gp.tilesM * gp.tilesN)), block(kThreads);
    switch (gp.a.mode) {
        case 0: hipLaunchKernelGGL((gemm_kernel<BN, G, PT, 0, DUMP>), grid, block, 0, s, gp); break;
        case 1: hipLaunchKernelGGL((gemm_kernel<BN, G, PT, 1, DUMP>), grid, block, 0, s, gp); break;
        default:
            if constexpr ((BN / 64) % 2 == 0)
                hipLaunchKernelGGL((gemm_kernel<BN, G, PT, 2, DUMP>), grid, block, 0, s, gp);
            else
                return hipErrorInvalidConfiguration;  // the host never pairs mode 2 with this width
            break;
    }
    return hipGetLastError();
}

template <int BN, bool DUMP>
hipError_t launch_tile(const LinearArgs& a, hipStream_t s) {
    GemmParams gp{};
    gp.a = a;
    const bool pt = a.GA == a.K;
    const int ge = pt ? a.G : 32;
    const int outw = a.mode == 2 ? BN / 2 : BN;
    gp.tilesM = (int)((a.M + kBM - 1) / kBM);
    gp.tilesN = (int)((a.N + outw - 1) / outw);
    gp.NE = (int)(a.K / ge);
    gp.NG = (int)(a.K / a.G);
    if (a.G == 128)
        return pt ? launch_mode<BN, 128, true, DUMP>(gp, s) : launch_mode<BN, 128, false, DUMP>(gp, s);
    return pt ? launch_mode<BN, 32, true, DUMP>(gp, s) : launch_mode<BN, 32, false, DUMP>(gp, s);
}

// Widest weight tile that still gives every CU a tile (MI355X: 256 CUs), the
// narrowest when even that leaves CUs idle.  Mode 2 needs gate/up subtile
// pairs per wave: widths 256 or 128.
int pick_bn(const LinearArgs& a) {
    const int64_t tm = (a.M + kBM - 1) / kBM;
    if (a.mode == 2) return tm * ((a.N + 127) / 128) >= 256 ? 256 : 128;
    static const int choices[] = {192, 128, 64};
    for (int bn : choices)
        if (tm * ((a.N + bn - 1) / bn) >= 256) return bn;
    return 64;
}

template <bool DUMP>
hipError_t launch_bn(const LinearArgs& a, hipStream_t s) {
    switch (pick_bn(a)) {
        case 256: return launch_tile<256, DUMP>(a, s);
        case 192: return launch_tile<192, DUMP>(a, s);
        case 128: return launch_tile<128, DUMP>(a, s);
        default: return launch_tile<64, DUMP>(a, s);
    }
}

}  // namespace

hipError_t launch_gemm(const LinearArgs& a, hipStream_t s) {
    return a.acc_dump ? launch_bn<true>(a, s) : launch_bn<false>(a, s);
}

}  // namespace wq
