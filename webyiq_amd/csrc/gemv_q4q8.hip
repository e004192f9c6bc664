// Decode GEMV, M <= 8 tokens (webyIQ crates/engine/src/shaders/gemv_q4q8.wgsl,
// host side Builder::gemv in crates/engine/src/graph.rs:190-198), and the
// lm_head GEMV with fused greedy argmax (graph.rs:476-486 + argmax.wgsl).
//
// y[t,n] = sum_g dx * (s[n,g] * A[t,n,g] + m[n,g] * X[t,g]),
// A = sum over group g of q * xq (int32, exact), X = sum of xq over g.
//
// MI355X mapping.  The packed weight matrix is one HBM stream.  A wavefront
// pass reads 1 KiB of one row (64 lanes x 16 B: one fully coalesced
// global_load_dwordx4), i.e. 2048 codes; a row of K codes takes J = K/2048
// passes.  Wave w of a workgroup serves pass j = w / nslots for rows
// slot, slot + nslots, ... (slot = w % nslots; nslots is 1, 2 or 4), so each
// lane keeps the 32 activations of its pass in registers for every token.  All weight loads of
// a workgroup are issued before the first one is consumed (IPW rows per wave),
// so the whole matrix is in flight at once across the chip.
//
// Each lane computes its 32-code dot product with 8 v_dot4_i32_i8, a quad of
// lanes (DPP) completes a 128-group; the exact int32 group sums stay in
// registers (one token, per-token group 128) or go to LDS.
// The fp32 epilogue folds each (token, row) in a fixed order the CPU oracle
// restates, so outputs are bit-reproducible (modes 0 and 1) and the fused
// argmax sees the same logits.  Per-token group-128 (the BASELINE format):
// per 2048-code pass of 16 groups, eight chains c = fma(s, A, c);
// c = fma(m, X, c) over the pairs of groups (2i, 2i + 1), the pairwise tree
// over the 8 pair values, the pass sums added in order -- for one token in
// registers (DPP moves across the wave's quads, no LDS round trip when a
// row is one pass), for more through LDS, four lanes per (token, row).
// Per-32 activation scales: per pass of 64 groups of 32, sixteen chains over
// four consecutive groups and the pairwise tree over them, four lanes per
// (token, row).  Per-token group 32: the same chains and tree with the
// token's scale applied to the total.
#include "argmax_combine.hpp"
#include "common.hpp"
#include "launch.hpp"

#pragma clang fp contract(off)

namespace wq {

#ifdef WQ_TIMELINE
// Timing build only (-DWQ_TIMELINE: libwebyiq_q4q8_timeline.so, which
// bench.py --timeline loads; the product library has none of this).  Thread
// 0 of each of the first kTimelineWgs workgroups of the one-token plain GEMV
// writes s_memrealtime (a 100 MHz clock) at five points: entry, its
// activations landed, its first weight row landed, its rows' products done,
// its outputs stored.  Each stamp adds a test of the value it marks, so it is
// taken only once that value's load has returned.
constexpr int kTimelineWgs = 4096;
__device__ unsigned long long wq_timeline[kTimelineWgs * 8];
#define WQ_STAMP(k, dep)                                                                              \
    do {                                                                                              \
        if (!QIN && !ARGMAX && MT == 1 && threadIdx.x == 0 && blockIdx.x < kTimelineWgs)              \
            wq_timeline[blockIdx.x * 8 + (k)] = __builtin_amdgcn_s_memrealtime() + ((dep) == 0x7654321u); \
    } while (0)
// the same stamps from gemv_one_kernel (one token by construction)
#define WQ_STAMP_ONE(k, dep)                                                                          \
    do {                                                                                              \
        if (threadIdx.x == 0 && blockIdx.x < kTimelineWgs)                                            \
            wq_timeline[blockIdx.x * 8 + (k)] = __builtin_amdgcn_s_memrealtime() + ((dep) == 0x7654321u); \
    } while (0)
#else
#define WQ_STAMP(k, dep) ((void)0)
#define WQ_STAMP_ONE(k, dep) ((void)0)
#endif

namespace {

struct GemvParams {
    LinearArgs a;
    ArgmaxArgs am;
    QuantInArgs qin;  // QIN kernels: the f32 input and optional RMSNorm
    int J;       // passes per row = ceil(K / 2048)
    int nslots;  // row slots per workgroup = waves / J
    int RB;      // rows per workgroup = nslots * IPW
    int NE;      // accumulation groups per row = K / Ge
    int NEP;     // padded LDS row stride of the group sums
    int NG;      // weight groups per row = K / G
    int nblocks; // gridDim.x
};

// LDS pointer p rounded up to a multiple of A bytes, as an offset from the LDS
// base: rounding the pointer as an integer loses its address space, and its
// accesses become flat ones, which count (and wait) with the global loads.
template <int A, typename T>
__device__ __forceinline__ T* lds_align(unsigned char* base, const void* p) {
    const size_t off = static_cast<size_t>(reinterpret_cast<const unsigned char*>(p) - base);
    return reinterpret_cast<T*>(base + ((off + A - 1) & ~size_t(A - 1)));
}

template <int MT, int MODE, int G, bool PT, int IPW, bool ARGMAX, bool QIN>
// Everything the first global loads need leads the argument list as separate
// arguments: the weight, activation, weight-scale and activation-scale
// pointers (with the fused quantiser: its f32 input and norm weight in the
// activation and activation-scale slots), N, K, two words packing the plan
// (RB | nslots << 8 | J << 12 | M << 16, and NG | NE << 16) and the
// activation sums.  This translation unit
// is built with -amdgpu-kernarg-preload-count=9, so these 14 SGPRs (the user
// SGPRs left beside the argument segment's address) arrive with the wave
// instead of through a scalar load of the argument segment that every wave
// would wait for before its first load (probe kernels of the headline GEMV's
// shape: 0.2-0.33 us per launch).  The output pointer follows them; the
// parameter struct carries the same values and the rest, read after the loads
// are issued.
__global__ __launch_bounds__(512) void gemv_kernel(const uint32_t* kwq, const int8_t* kxq, const uint32_t* kws,
                                                   const float* kdx, int kN, int kK, uint32_t kplan, uint32_t kgroups,
                                                   const int32_t* kxs, float* ky, GemvParams pk) {
    constexpr int GE = PT ? G : 32;        // accumulation group
    constexpr int LPG = GE / 32;           // lanes per accumulation group (1 or 4)
    constexpr int LPW = G / 32;            // lanes per weight group (1 or 4)
    constexpr int NH = MODE == 2 ? 2 : 1;  // gate (+ up) row halves
    extern __shared__ __align__(16) unsigned char smem[];

    GemvParams p = pk;
    p.a.wq = kwq;
    p.a.ws = kws;
    if (QIN) {  // the fused quantiser's f32 input and norm weight take the activation slots
        p.qin.x = reinterpret_cast<const float*>(kxq);
        p.qin.norm_w = kdx;
    } else {
        p.a.xq = kxq;
        p.a.dx = kdx;
    }
    p.a.xs = kxs;
    p.a.y = ky;
    p.a.N = kN;
    p.a.K = kK;
    p.a.M = (kplan >> 16) & 255;
    p.RB = kplan & 255;
    p.nslots = (kplan >> 8) & 15;
    p.J = (kplan >> 12) & 15;
    p.NG = kgroups & 0xFFFF;
    p.NE = kgroups >> 16;
    const LinearArgs& a = p.a;
    const int tid = threadIdx.x;
    WQ_STAMP(0, 0u);
    const int lane = tid & 63;
    // The wave index and what derives from it are wave-uniform values in
    // SGPRs: row addresses are then scalar bases plus a 32-bit lane offset,
    // and the few dozen instructions before the last load is issued are
    // mostly scalar (with three waves a SIMD, each vector instruction there
    // delays the loads of all three).
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int NW = p.J * p.nslots;  // waves (blockDim.x / 64, without its late scalar load)
    const int nthreads = 64 * NW;
    // wave = j * nslots + slot; nslots is 1, 2 or 4 (a power of two)
    const int slot = wave & (p.nslots - 1);
    const int j = wave >> (p.nslots >> 1);
    const int64_t N = a.N;
    const int K = (int)a.K;
    const int RB = p.RB;
    const int NE = p.NE, NG = p.NG;
    const int NEP = (NE + 4) & ~3;  // the plan's padded stride (make_plan), from a preloaded value
    const int NGS = NG + 2;  // LDS row stride of the (s, m) pairs: rows on distinct banks
    const int NDX = PT ? 1 : K / 32;
    const int64_t r0 = (int64_t)blockIdx.x * RB;

    // LDS: group sums [MT][NH][RB][NEP] i32 | weight (s, m) [NH][RB][NG] f32x2 |
    //      activation sums [MT][NE] f32 | activation scales [MT][NDX] f32,
    //      each part 16-byte aligned (the epilogue reads them 16 bytes at a time)
    int32_t* acc_lds = reinterpret_cast<int32_t*>(smem);
    float2* sm_lds = reinterpret_cast<float2*>(acc_lds + (size_t)MT * NH * RB * NEP);
    float* xs_lds = lds_align<16, float>(smem, sm_lds + (size_t)NH * RB * NGS);
    float* dx_lds = lds_align<16, float>(smem, xs_lds + (size_t)MT * NE);
    // fused quantiser scratch (QIN kernels have no argmax keys)
    static_assert(!(QIN && ARGMAX), "no fused quantiser in the lm_head kernel");
    float* qin_lds = lds_align<16, float>(smem, dx_lds + (size_t)MT * NDX);

    // Lanes past the end of a partial pass (K % 2048 != 0) load from position 0
    // and never write their results: every load below is unconditional, so no
    // branch can hold a wait that would serialise a second memory round trip.
    const int kraw = kGemvPassK * j + 32 * lane;  // first code of this lane's slice
    const bool kact = kraw < K;
    const int kpos = kact ? kraw : 0;
    const int e = kpos / GE;  // this lane's accumulation group
    const int g = kpos / G;   // this lane's weight group
    const size_t row_bytes = (size_t)K / 2;
    const uint32_t woff = (uint32_t)kpos / 2;  // this lane's byte offset in a packed row

    // 0. fused quantiser input first, coalesced and split between the
    //    nslots waves of a pass: the wave of pass j and slot s reads loads
    //    u0 + i (u0 = s * us, i < us = 8 / nslots), i.e. chunks
    //    512 j + 64 u + lane, of each token and of the norm weight.  Issued
    //    before the weight stream, so waiting for them does not wait for it.
    constexpr int QT = QIN ? MT : 1;
    float4 qx[QT][8], qw[8];
    const int qus = 8 >> (p.nslots >> 1), qu0 = slot * qus;  // 8 / nslots: nslots is 1, 2 or 4
    // f(i) for this wave's loads i < qus; the skipped ones are branched over
    // (uniformly), not computed and discarded
    auto for_chunks = [&](auto&& f) {
#pragma unroll
        for (int i = 0; i < 2; ++i) f(i);
        if (qus >= 4) {
            asm volatile("");
#pragma unroll
            for (int i = 2; i < 4; ++i) f(i);
        }
        if (qus == 8) {
            asm volatile("");
#pragma unroll
            for (int i = 4; i < 8; ++i) f(i);
        }
    };
    if constexpr (QIN) {
        const int nchunk = K / 4;
        const float* nsrc = p.qin.norm_w ? p.qin.norm_w : p.qin.x;  // unconditional loads
        for_chunks([&](int i) {
            const int c = 512 * j + 64 * (qu0 + i) + lane;
            const uint32_t cb = (uint32_t)(c < nchunk ? c : 0) * 16u;  // the chunk's byte offset in a row
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const int tt = (t == 0 || t < (int)a.M) ? t : (int)a.M - 1;  // M >= 1
                const unsigned char* xt = reinterpret_cast<const unsigned char*>(p.qin.x + (size_t)tt * K);
                qx[t][i] = *reinterpret_cast<const float4*>(xt + cb);
            }
            qw[i] = *reinterpret_cast<const float4*>(reinterpret_cast<const unsigned char*>(nsrc) + cb);
        });
        // keep these loads ahead of the weight stream (no sinking into their
        // use, which would wait for every weight load)
        asm volatile("" ::: "memory");
    }

    uint4 xa[MT], xb[MT];
    int32_t xsv[MT];
    float dxv[MT];
    if constexpr (!QIN) {
        // the activations first (a few KiB, L2-resident): row s's products
        // can then start as soon as its weights land
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int tt = (t == 0 || t < (int)a.M) ? t : (int)a.M - 1;  // M >= 1
            const unsigned char* xt = reinterpret_cast<const unsigned char*>(a.xq) + (size_t)tt * K;  // uniform
            xa[t] = load16(xt + (uint32_t)kpos);
            xb[t] = load16(xt + (uint32_t)kpos + 16);
            xsv[t] = (a.xs + (size_t)tt * NE)[e];
            dxv[t] = (a.dx + (size_t)tt * NDX)[PT ? 0 : e];
        }
        asm volatile("" ::: "memory");  // keep them ahead of the weight stream
    }

    // 1. issue every global load of this lane before the first one is consumed
    //    (one memory round trip; rows past N re-read row N-1)
    uint4 wv[NH][IPW];
    uint32_t sv[NH][IPW];
#pragma unroll
    for (int s = 0; s < IPW; ++s) {
        // 32-bit row indices (rows * K / 2 < 4 GiB: checked on the host)
        int row = (int)r0 + slot + p.nslots * s;
        row = row < (int)N ? row : (int)N - 1;
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            const uint32_t rh = (uint32_t)(row + h * (int)N);
            const unsigned char* rp = reinterpret_cast<const unsigned char*>(a.wq) + (size_t)rh * row_bytes;
            wv[h][s] = load_stream16(rp + woff);
            sv[h][s] = (a.ws + (size_t)rh * NG)[g];
        }
        asm volatile("" ::: "memory");  // loads stay in row order: row s lands before row s + 1
    }
    // the arguments read later, in SGPRs now that the loads are in flight
    // (a scalar load sunk next to a late use would add a round trip there)
    pin_arg(a.acc_dump);
    if (QIN) { pin_arg(p.qin.eps); pin_arg(p.qin.xq); pin_arg(p.qin.dx); pin_arg(p.qin.xs); }
    if (ARGMAX) {
        pin_arg(p.am.ids); pin_arg(p.am.tok_out); pin_arg(p.am.keys); pin_arg(p.am.ticket);
        pin_arg(p.nblocks);
    }
    if constexpr (!QIN) {
        WQ_STAMP(1, xa[0].x ^ xb[0].w ^ (uint32_t)xsv[0] ^ __float_as_uint(dxv[0]));
        WQ_STAMP(2, wv[0][0].x ^ sv[0][0]);
    }
    if constexpr (QIN) {
        // Fused per-token quantiser, while the weight loads are in flight:
        // the quant_act kernels' arithmetic and reduction order (per-chunk
        // fmaf chains, a pairwise tree over a lane's 8 chunks -- here split
        // over the waves of the pass and completed through LDS -- a pairwise
        // tree over the lanes, pass sums in pass order), so codes, scales and
        // sums are bit-identical to wq_quant_act's.  Every wave completes
        // every pass's tree itself (no second exchange).  Each wave quantises
        // its own chunks into LDS; every wave then reads its lane's 32 codes.
        static_assert(!QIN || (PT && MT <= 2), "the fused quantiser is per token, M <= 2");
        float* wmax = qin_lds + MT * 8;       // [MT][8] absmax per wave
        float* sub = qin_lds + MT * 16;       // [MT][8 waves][64] lane subtrees
        uint32_t* codes = lds_align<16, uint32_t>(smem, sub + MT * 8 * 64);  // [MT][K/4]
        const int nchunk = K / 4;
        const int nsl = p.nslots;
        auto valid = [&](int i) { return 512 * j + 64 * (qu0 + i) + lane < nchunk; };  // partial pass
        if (p.qin.norm_w) {
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                float c[8];
                for_chunks([&](int i) { c[i] = valid(i) ? chunk_ss(qx[t][i]) : 0.0f; });
                // this wave's subtree: 2, 4 or 8 of the lane's chunks
                float st = c[0] + c[1];
                if (qus >= 4) st = st + (c[2] + c[3]);
                if (qus == 8) st = st + ((c[4] + c[5]) + (c[6] + c[7]));
                sub[(t * 8 + slot * p.J + j) * 64 + lane] = st;
            }
            __syncthreads();
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                // pass jj's lane partials: slot s's subtree sits at index s * J + jj;
                // the pass sums are added in pass order (J <= 8)
                float total = 0.0f;
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    if (jj < p.J) {
                        const float* sp = sub + (t * 8 + jj) * 64 + lane;
                        float pl = sp[0];
                        if (nsl == 2) pl = pl + sp[p.J * 64];
                        if (nsl == 4) pl = (pl + sp[64]) + (sp[128] + sp[192]);  // J == 1
                        total = total + wave_sum_tree(pl);
                    }
                }
                const float r = 1.0f / sqrt_rn(mean_of(total, K) + p.qin.eps);
                for_chunks([&](int i) {
                    qx[t][i].x = (qx[t][i].x * r) * qw[i].x;
                    qx[t][i].y = (qx[t][i].y * r) * qw[i].y;
                    qx[t][i].z = (qx[t][i].z * r) * qw[i].z;
                    qx[t][i].w = (qx[t][i].w * r) * qw[i].w;
                });
            }
        }
        // per-token absmax (order-free), dx = amax / 127
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            float mx = 0.0f;
            for_chunks([&](int i) {
                if (valid(i))
                    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(qx[t][i].x), fabsf(qx[t][i].y)),
                                         fmaxf(fabsf(qx[t][i].z), fabsf(qx[t][i].w))));
            });
            mx = wave_max(mx);
            if (lane == 0) wmax[t * 8 + wave] = mx;
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            // NW <= 8 waves; all 8 read at once
            const float4 ma = reinterpret_cast<const float4*>(wmax + t * 8)[0];
            const float4 mb = reinterpret_cast<const float4*>(wmax + t * 8)[1];
            const float mm[8] = {ma.x, ma.y, ma.z, ma.w, mb.x, mb.y, mb.z, mb.w};
            float amax = mm[0];
#pragma unroll
            for (int w = 1; w < 8; ++w) amax = w < NW ? fmaxf(amax, mm[w]) : amax;
            dxv[t] = amax / 127.0f;
        }
        // codes of this wave's chunks -> LDS (and, from workgroup 0, to memory)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const float d = dxv[t], rd = 1.0f / d;
            const int64_t tt = t < a.M ? t : a.M - 1;
            for_chunks([&](int i) {
                if (!valid(i)) return;
                const int c = 512 * j + 64 * (qu0 + i) + lane;
                const uint32_t wd =
                    d > 0.0f ? quant_word(qx[t][i].x, qx[t][i].y, qx[t][i].z, qx[t][i].w, d, rd) : 0u;
                codes[t * nchunk + c] = wd;
                if (blockIdx.x == 0 && t < a.M) reinterpret_cast<uint32_t*>(p.qin.xq + tt * a.K)[c] = wd;
            });
        }
        __syncthreads();
        // this lane's 32 codes and its group's code sum
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const uint4* cp = reinterpret_cast<const uint4*>(codes + t * nchunk + kpos / 4);
            xa[t] = cp[0];
            xb[t] = cp[1];
            int cs = 0;
            cs = dot4(xa[t].x, 0x01010101u, cs);
            cs = dot4(xa[t].y, 0x01010101u, cs);
            cs = dot4(xa[t].z, 0x01010101u, cs);
            cs = dot4(xa[t].w, 0x01010101u, cs);
            cs = dot4(xb[t].x, 0x01010101u, cs);
            cs = dot4(xb[t].y, 0x01010101u, cs);
            cs = dot4(xb[t].z, 0x01010101u, cs);
            cs = dot4(xb[t].w, 0x01010101u, cs);
            xsv[t] = LPG == 4 ? quad_sum(cs) : cs;
            if (blockIdx.x == 0 && slot == 0 && kact && t < a.M) {
                if ((lane % LPG) == 0) p.qin.xs[(int64_t)t * NE + e] = xsv[t];
                if (tid == 0) p.qin.dx[t] = dxv[t];
            }
        }
    }

    if constexpr (PT && G == 128 && MT == 1) {
        // Per-token group-128 epilogue in registers (one token: few outputs
        // per workgroup, so latency matters more than lane occupancy).
        // After quad_sum every lane of a quad holds its group's exact sum A,
        // and pass_pairs8 folds the pass's 16 groups in the canonical order
        // (a chain per pair of groups, the pairwise tree over the pairs).
        // A row of one pass (K <= 2048) is complete in its wave; with several
        // passes the wave sums meet through LDS and are added in pass order.
        const bool lead = kact && (lane & 3) == 0;
        const int rows_total = NH * (int)N;
        float vals[NH][IPW][MT];
        // y of token 0, local row rl (the plain GEMV's one-token emit)
        auto emit_row = [&](int rl, float v0, float v1, float d) {
            const int row = (int)r0 + rl;
            if (row < (int)N) {
                float* yo = a.y + row;
                const float v = v0 * d;
                if (MODE == 0) *yo = v;
                else if (MODE == 1) *yo = *yo + v;
                else *yo = silu_mul(v, v1 * d);
            }
        };
#pragma unroll
        for (int s = 0; s < IPW; ++s) {
            const int row = (int)r0 + slot + p.nslots * s;  // 32-bit: compared on the scalar unit
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const float ws_s = f16lo(sv[h][s]), ws_m = f16hi(sv[h][s]);
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    const int d = quad_sum(dot32(wv[h][s], xa[t], xb[t]));
                    if (a.acc_dump) {  // test hook (uniform branch): the exact group sums
                        if (lead && t < (int)a.M && row < (int)N)
                            a.acc_dump[((int64_t)t * rows_total + h * N + row) * NE + e] = d;
                    }
                    vals[h][s][t] = pass_pairs8(kact, ws_s, (float)d, ws_m, (float)xsv[t]);
                }
            }
            // one pass: the row is complete; one lane stores it now, so that
            // only the last row's fold and store follow the last load
            if (!ARGMAX && MT == 1 && p.J == 1 && lane == 0)
                emit_row(slot + p.nslots * s, vals[0][s][0], vals[NH - 1][s][0], dxv[0]);
        }
#ifdef WQ_TIMELINE
        {
            float all = 0.0f;
#pragma unroll
            for (int s = 0; s < IPW; ++s) all += vals[0][s][0];
            WQ_STAMP(3, __float_as_uint(all));
        }
#endif
        unsigned long long* keys = lds_align<8, unsigned long long>(smem, dx_lds + (size_t)MT * NDX);
        // y (or the argmax key) of (token t, local row rl) from the row sums
        auto emit = [&](int t, int rl, float v0, float v1, float d) {
            const int64_t row = r0 + rl;
            const bool ok = t < a.M && row < N;
            if constexpr (ARGMAX) {
                unsigned long long key = 0;
                if (ok) {
                    const float v = v0 * d;
                    if (a.y) a.y[(int64_t)t * N + row] = v;
                    if (v > -3.0e38f) key = argmax_key(v, (uint32_t)row);
                }
                keys[t * RB + rl] = key;
            } else if (ok) {
                float* yo = a.y + (int64_t)t * N + row;
                const float v = v0 * d;
                if (MODE == 0) {
                    *yo = v;
                } else if (MODE == 1) {
                    *yo = *yo + v;
                } else {
                    *yo = silu_mul(v, v1 * d);
                }
            }
        };
        static_assert(IPW * MT <= 64, "one lane per (row, token)");
        if (p.J == 1 && !ARGMAX && MT == 1) {
            WQ_STAMP(4, 0u);  // every row was stored as it completed
        } else if (p.J == 1) {
            // lane s * MT + t of the wave emits (token t, its row s)
            float v0 = 0.0f, v1 = 0.0f, dsel = 0.0f;
            int tsel = -1, rsel = 0;
#pragma unroll
            for (int s = 0; s < IPW; ++s)
#pragma unroll
                for (int t = 0; t < MT; ++t)
                    if (lane == s * MT + t) {
                        v0 = vals[0][s][t];
                        v1 = vals[NH - 1][s][t];
                        dsel = dxv[t];
                        tsel = t;
                        rsel = slot + p.nslots * s;
                    }
            if (tsel >= 0) emit(tsel, rsel, v0, v1, dsel);
            WQ_STAMP(4, 0u);
        } else {
            // pass sums [t][h][rl][pass] -> LDS, then each (token, row) adds
            // its passes left to right
            float* part = reinterpret_cast<float*>(acc_lds);
            const int J = p.J;
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                float v = 0.0f;
                int idx = -1;
#pragma unroll
                for (int s = 0; s < IPW; ++s)
#pragma unroll
                    for (int t = 0; t < MT; ++t)
                        if (lane == s * MT + t) {
                            v = vals[h][s][t];
                            idx = ((t * NH + h) * RB + slot + p.nslots * s) * J + j;
                        }
                if (idx >= 0) part[idx] = v;
            }
            if (tid == 0) {
#pragma unroll
                for (int t = 0; t < MT; ++t) dx_lds[t] = dxv[t];
            }
            __syncthreads();
            for (int o = tid; o < MT * RB; o += nthreads) {
                const int t = o / RB, rl = o - t * RB;
                float v[NH];
#pragma unroll
                for (int h = 0; h < NH; ++h) {
                    const float* pp = part + ((t * NH + h) * RB + rl) * J;
                    float tot = pp[0];
                    for (int jj = 1; jj < J; ++jj) tot = tot + pp[jj];
                    v[h] = tot;
                }
                emit(t, rl, v[0], v[NH - 1], dx_lds[t]);
            }
        }
        if constexpr (ARGMAX) {
            __syncthreads();
            const unsigned long long best = block_best<MT>(keys, RB, (int)a.M);
            argmax_combine<MT>(p.am, (int)a.M, p.nblocks, best);
        }
        return;
    }

    // 2. activation sums / scales and weight (s, m) -> LDS
    if (slot == 0 && kact && (lane % LPG) == 0) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            xs_lds[t * NE + e] = (float)xsv[t];
            if (!PT) dx_lds[t * NDX + e] = dxv[t];
        }
    }
    if (PT && tid == 0) {
#pragma unroll
        for (int t = 0; t < MT; ++t) dx_lds[t] = dxv[t];
    }

    // 3. per row, in load order (each row as soon as its loads land): the
    //    weight (s, m) pairs and the exact int32 group sums -> LDS
#pragma unroll
    for (int s = 0; s < IPW; ++s) {
        const int rl = slot + p.nslots * s;
#pragma unroll
        for (int h = 0; h < NH; ++h) {
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                int d = dot32(wv[h][s], xa[t], xb[t]);
                if (LPG == 4) d = quad_sum(d);
                if (kact && (lane % LPG) == 0) acc_lds[((t * NH + h) * RB + rl) * NEP + e] = d;
            }
            if (kact && (lane % LPW) == 0)
                sm_lds[(h * RB + rl) * NGS + g] = make_float2(f16lo(sv[h][s]), f16hi(sv[h][s]));
        }
    }
    __syncthreads();

    if (a.acc_dump) {  // test hook: the group sums exactly as the epilogue reads them
        const int rows_total = NH * (int)N;
        for (int i = tid; i < MT * NH * RB * NE; i += nthreads) {
            int ee = i % NE;
            int rl = (i / NE) % RB;
            int h = (i / (NE * RB)) % NH;
            int t = i / (NE * RB * NH);
            int64_t row = r0 + rl;
            if (t < a.M && row < N)
                a.acc_dump[((int64_t)t * rows_total + h * N + row) * NE + ee] =
                    acc_lds[((t * NH + h) * RB + rl) * NEP + ee];
        }
    }

    if constexpr (PT && G == 128) {
        // Per-token group-128, several tokens: four lanes per (token, row).
        // Per pass, lane q runs the pair chains c = fma(s, A, c);
        // c = fma(m, X, c) from 0 over groups (4q, 4q + 1) and (4q + 2,
        // 4q + 3) (those that exist) and adds the two; two quad moves
        // complete the pairwise tree over the 8 pairs; the pass sums are
        // added in order.  The register epilogue's order.
        unsigned long long* keys = lds_align<8, unsigned long long>(smem, dx_lds + (size_t)MT * NDX);
        const bool vec = (NE & 3) == 0;
        for (int o = tid; o < 4 * MT * RB; o += nthreads) {
            const int q = o & 3, oo = o >> 2;
            const int t = oo / RB, rl = oo - t * RB;
            const float* xsr = xs_lds + t * NE;
            float tot[NH];
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const int32_t* ar = acc_lds + ((t * NH + h) * RB + rl) * NEP;
                const float2* sr = sm_lds + (h * RB + rl) * NGS;
                float total = 0.0f;
                for (int e0 = 0; e0 < NE; e0 += 16) {
                    const int eb = e0 + 4 * q;
                    float c0 = 0.0f, c1 = 0.0f;
                    if (vec && eb < NE) {
                        const int4 a4 = *reinterpret_cast<const int4*>(ar + eb);
                        const float4 x4 = *reinterpret_cast<const float4*>(xsr + eb);
                        const float4 w01 = *reinterpret_cast<const float4*>(sr + eb);
                        const float4 w23 = *reinterpret_cast<const float4*>(sr + eb + 2);
                        c0 = fmaf(w01.y, x4.x, fmaf(w01.x, (float)a4.x, c0));
                        c0 = fmaf(w01.w, x4.y, fmaf(w01.z, (float)a4.y, c0));
                        c1 = fmaf(w23.y, x4.z, fmaf(w23.x, (float)a4.z, c1));
                        c1 = fmaf(w23.w, x4.w, fmaf(w23.z, (float)a4.w, c1));
                    } else if (!vec) {
#pragma unroll
                        for (int k = 0; k < 4; ++k)
                            if (eb + k < NE) {
                                const float2 w = sr[eb + k];
                                float& c = k < 2 ? c0 : c1;
                                c = fmaf(w.y, xsr[eb + k], fmaf(w.x, (float)ar[eb + k], c));
                            }
                    }
                    float v = c0 + c1;
                    v = v + dpp_f<kDppXor1>(v);
                    v = v + dpp_f<kDppXor2>(v);
                    total = e0 == 0 ? v : total + v;
                }
                tot[h] = total;
            }
            if (q != 0) continue;
            const int64_t row = r0 + rl;
            const bool ok = t < a.M && row < N;
            const float d = dx_lds[t];
            if constexpr (ARGMAX) {
                unsigned long long key = 0;
                if (ok) {
                    const float v = tot[0] * d;
                    if (a.y) a.y[(int64_t)t * N + row] = v;
                    if (v > -3.0e38f) key = argmax_key(v, (uint32_t)row);
                }
                keys[t * RB + rl] = key;
            } else if (ok) {
                float* yo = a.y + (int64_t)t * N + row;
                const float v = tot[0] * d;
                if (MODE == 0) {
                    *yo = v;
                } else if (MODE == 1) {
                    *yo = *yo + v;
                } else {
                    *yo = silu_mul(v, tot[NH - 1] * d);
                }
            }
        }
        if constexpr (ARGMAX) {
            __syncthreads();
            const unsigned long long best = block_best<MT>(keys, RB, (int)a.M);
            argmax_combine<MT>(p.am, (int)a.M, p.nblocks, best);
        }
        return;
    }

    if constexpr (!PT || G == 32) {
        // Per-32 activation scales: four lanes per (token, row).  Per pass of
        // 64 groups of 32, lane q runs the chains c = fma(s dx, A, c);
        // c = fma(m dx, X, c) from 0 over groups 16q + 4i .. 16q + 4i + 3
        // (i = 0..3) and forms (c0 + c1) + (c2 + c3); two quad moves complete
        // the pairwise tree over the pass's 16 chains; the pass sums are
        // added in order.  Per-token group 32: the same with the token's dx
        // outside, c = fma(s, A, c); c = fma(m, X, c) and total * dx.  The
        // oracle's order.
        unsigned long long* keys = lds_align<8, unsigned long long>(smem, dx_lds + (size_t)MT * NDX);
        for (int o = tid; o < 4 * MT * RB; o += nthreads) {
            const int q = o & 3, oo = o >> 2;
            const int t = oo / RB, rl = oo - t * RB;
            const float* xsr = xs_lds + t * NE;
            const float* dr = dx_lds + t * NDX;
            float tot[NH];
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const int32_t* ar = acc_lds + ((t * NH + h) * RB + rl) * NEP;
                const float2* sr = sm_lds + (h * RB + rl) * NGS;
                float total = 0.0f;
                for (int e0 = 0; e0 < NE; e0 += 64) {
                    float c[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int eb = e0 + 16 * q + 4 * i;  // NE is a multiple of 4
                        float v = 0.0f;
                        if (eb < NE) {
                            const int4 a4 = *reinterpret_cast<const int4*>(ar + eb);
                            const float4 x4 = *reinterpret_cast<const float4*>(xsr + eb);
                            // (per token: dx is applied to the total)
                            const float4 d4 = PT ? make_float4(1.f, 1.f, 1.f, 1.f)
                                                 : *reinterpret_cast<const float4*>(dr + eb);
                            float2 w0, w1, w2, w3;
                            if constexpr (G == 128) {  // the four groups share one weight group
                                w0 = w1 = w2 = w3 = sr[eb / 4];
                            } else {
                                const float4 w01 = *reinterpret_cast<const float4*>(sr + eb);
                                const float4 w23 = *reinterpret_cast<const float4*>(sr + eb + 2);
                                w0 = make_float2(w01.x, w01.y);
                                w1 = make_float2(w01.z, w01.w);
                                w2 = make_float2(w23.x, w23.y);
                                w3 = make_float2(w23.z, w23.w);
                            }
                            if constexpr (PT) {
                                v = fmaf(w0.x, (float)a4.x, v);
                                v = fmaf(w0.y, x4.x, v);
                                v = fmaf(w1.x, (float)a4.y, v);
                                v = fmaf(w1.y, x4.y, v);
                                v = fmaf(w2.x, (float)a4.z, v);
                                v = fmaf(w2.y, x4.z, v);
                                v = fmaf(w3.x, (float)a4.w, v);
                                v = fmaf(w3.y, x4.w, v);
                            } else {
                                v = fmaf(w0.x * d4.x, (float)a4.x, v);
                                v = fmaf(w0.y * d4.x, x4.x, v);
                                v = fmaf(w1.x * d4.y, (float)a4.y, v);
                                v = fmaf(w1.y * d4.y, x4.y, v);
                                v = fmaf(w2.x * d4.z, (float)a4.z, v);
                                v = fmaf(w2.y * d4.z, x4.z, v);
                                v = fmaf(w3.x * d4.w, (float)a4.w, v);
                                v = fmaf(w3.y * d4.w, x4.w, v);
                            }
                        }
                        c[i] = v;
                    }
                    float v = (c[0] + c[1]) + (c[2] + c[3]);
                    v = v + dpp_f<kDppXor1>(v);
                    v = v + dpp_f<kDppXor2>(v);
                    total = e0 == 0 ? v : total + v;
                }
                tot[h] = PT ? total * dr[0] : total;
            }
            if (q != 0) continue;
            const int64_t row = r0 + rl;
            const bool ok = t < a.M && row < N;
            if constexpr (ARGMAX) {
                unsigned long long key = 0;
                if (ok) {
                    const float v = tot[0];
                    if (a.y) a.y[(int64_t)t * N + row] = v;
                    if (v > -3.0e38f) key = argmax_key(v, (uint32_t)row);
                }
                keys[t * RB + rl] = key;
            } else if (ok) {
                float* yo = a.y + (int64_t)t * N + row;
                const float v = tot[0];
                if (MODE == 0) {
                    *yo = v;
                } else if (MODE == 1) {
                    *yo = *yo + v;
                } else {
                    *yo = silu_mul(v, tot[NH - 1]);
                }
            }
        }
        if constexpr (ARGMAX) {
            __syncthreads();
            const unsigned long long best = block_best<MT>(keys, RB, (int)a.M);
            argmax_combine<MT>(p.am, (int)a.M, p.nblocks, best);
        }
        return;
    }
}

// Up to eight tokens (MT = 1, 2, 4, 8 slots; M of them real), one
// 2048-code pass per row (K = 2048), per-token activations at group 128:
// the decode GEMV's most common instances (the headline shape, the qkv and
// gate_up projections of a hidden size of 2048, and their verify launches),
// in a kernel of their own.  The arithmetic and its order are gemv_kernel's
// register epilogue exactly (dot32, quad_sum, pass_pairs8, times dx, per
// token), which its LDS epilogue for several tokens reproduces, so outputs
// are bit-identical to either; what this kernel drops is the generality
// around them (plan fields decoded at run time, partial passes, the
// pass-count and debug-dump branches, and for several tokens the group
// sums' LDS round trip and barrier).  Each (token, row) value is folded by
// the whole wave, so the dispatch takes this kernel only while a wave folds
// at most eight of them (one_fits).  Four waves per workgroup, one row slot
// each, IPW rows per wave; rows past N re-read row N - 1 and store nothing;
// token slots past M re-read token M - 1 and store nothing.  The eight
// arguments are preloaded into SGPRs (14 of them).  (The grid has its own
// rows-per-wave rule, at the dispatch.)
constexpr int kOneSlots = 4;

template <int MODE, int IPW, int MT>
__global__ __launch_bounds__(64 * kOneSlots) void gemv_one_kernel(const uint32_t* wq, const int8_t* xq,
                                                                   const uint32_t* ws, const int32_t* xs,
                                                                   const float* dx, float* y, int N, int M) {
    static_assert(MT == 1 || MT == 2 || MT == 4 || MT == 8, "up to eight tokens");
    constexpr int NH = MODE == 2 ? 2 : 1;  // gate (+ up) row halves
    constexpr uint32_t kRowBytes = kGemvPassK / 2, kGroups = kGemvPassK / 128;
    WQ_STAMP_ONE(0, 0u);
    const int lane = threadIdx.x & 63;
    const int slot = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r0 = (int)blockIdx.x * (kOneSlots * IPW);
    const uint32_t kpos = 32u * lane;  // this lane's 32 codes
    const uint32_t g = (uint32_t)lane >> 2;  // its group of 128
    // the activations first (L2-resident), then every row's weights and scale word
    uint4 xa[MT], xb[MT];
    int32_t xsv[MT];
    float dxv[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int tt = (t == 0 || t < M) ? t : M - 1;  // padding tokens re-read the last one
        xa[t] = load16(xq + tt * kGemvPassK + kpos);
        xb[t] = load16(xq + tt * kGemvPassK + kpos + 16);
        xsv[t] = xs[tt * (int)kGroups + g];
        dxv[t] = dx[tt];
    }
    asm volatile("" ::: "memory");
    uint4 wv[NH][IPW];
    uint32_t sv[NH][IPW];
#pragma unroll
    for (int s = 0; s < IPW; ++s) {
        const int row = min(r0 + slot + kOneSlots * s, N - 1);
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            const size_t rh = (size_t)(row + h * N);
            wv[h][s] = load_stream16(reinterpret_cast<const unsigned char*>(wq) + rh * kRowBytes + kpos / 2);
            sv[h][s] = ws[rh * kGroups + g];
        }
        asm volatile("" ::: "memory");  // loads stay in row order: row s lands before row s + 1
    }
    WQ_STAMP_ONE(1, xa[0].x ^ xb[0].w ^ (uint32_t)xsv[0] ^ __float_as_uint(dxv[0]));
    WQ_STAMP_ONE(2, wv[0][0].x ^ sv[0][0]);
#pragma unroll
    for (int s = 0; s < IPW; ++s) {
        float v[MT][NH];
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const int d = quad_sum(dot32(wv[h][s], xa[t], xb[t]));
                v[t][h] = pass_pairs8(true, f16lo(sv[h][s]), (float)d, f16hi(sv[h][s]), (float)xsv[t]);
            }
        const int row = r0 + slot + kOneSlots * s;
        // the row is complete: stored now, token t by lane t (its read,
        // SiLU and store in parallel with the other tokens')
        float v0 = v[0][0], v1 = v[0][NH - 1], dd = dxv[0];
#pragma unroll
        for (int t = 1; t < MT; ++t)
            if (lane == t) {
                v0 = v[t][0];
                v1 = v[t][NH - 1];
                dd = dxv[t];
            }
        if (lane < MT && lane < M && row < N) {
            float* yo = y + (size_t)lane * N + row;
            const float o = v0 * dd;
            if (MODE == 0) *yo = o;
            else if (MODE == 1) *yo = *yo + o;
            else *yo = silu_mul(o, v1 * dd);
        }
        if (s == IPW - 1) WQ_STAMP_ONE(3, __float_as_uint(v0));
    }
    WQ_STAMP_ONE(4, 0u);
}

// ------------------------------------------------------------ dispatch ----

struct Plan {
    int MT, IPW, J, nslots, waves, RB, NE, NEP, NG;
    size_t lds;
    unsigned grid;
};

// Grid target: 3 workgroups per CU (256 CUs), i.e. three waves per SIMD,
// whose loads and register epilogues overlap one another.
#ifndef WQ_GEMV_TARGET_WGS
#define WQ_GEMV_TARGET_WGS 768
#endif
constexpr int64_t kGemvTargetWgs = WQ_GEMV_TARGET_WGS;
constexpr int64_t kGemvCus = 256;

int round_tokens(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }

Plan make_plan(const LinearArgs& a, bool argmax, bool qin = false) {
    Plan p{};
    p.MT = round_tokens(a.M);
    const bool pt = a.GA == a.K;
    const int ge = pt ? a.G : 32;
    p.J = (int)((a.K + kGemvPassK - 1) / kGemvPassK);
    p.nslots = p.J >= 4 ? 1 : (4 + p.J - 1) / p.J;
    p.waves = p.J * p.nslots;
    p.NE = (int)(a.K / ge);
    p.NEP = (p.NE + 4) & ~3;  // 16-byte rows, spread over LDS banks
    p.NG = (int)(a.K / a.G);
    const int nh = a.mode == 2 ? 2 : 1;
    // rows per wave: the fewest loads per lane that still keep the grid within
    // the target (all loads issued up front).  With the fused quantiser every
    // workgroup re-quantises the whole input (MT x K floats from L2), so it
    // keeps one workgroup per CU per weight half (measured best for the
    // decode layer's four fused shapes at 1 and 2 tokens).  One row per wave
    // only where two would leave CUs idle: a wave's second row hides the
    // first one's arithmetic.
    int ipw = 8;
    static const int choices[] = {1, 2, 3, 4, 6, 8};
    const int64_t target = qin ? kGemvCus * nh : kGemvTargetWgs;
    auto grid_of = [&](int c) { return (a.N + (int64_t)p.nslots * c - 1) / ((int64_t)p.nslots * c); };
    for (int c : choices) {
        if (grid_of(c) <= target) { ipw = c; break; }
    }
    if (ipw == 1 && grid_of(2) >= kGemvCus) ipw = 2;
    // The fused lm_head argmax: three rows per wave while that keeps the grid
    // within 8,192 workgroups (one token: 10.65 against 11.24 us at 32,768
    // rows, where the target rule gave eight; at 151,936 rows three and eight
    // are alike and the rule's eight keeps the grid at 4,748).
    if (argmax && grid_of(3) <= 8192) ipw = 3;
    // LDS budget: 64 KiB per workgroup
    auto lds_of = [&](int ipw_) {
        size_t rb = (size_t)p.nslots * ipw_;
        size_t b = (size_t)p.MT * nh * rb * p.NEP * 4 + (size_t)nh * rb * (p.NG + 2) * 8 +
                   (size_t)p.MT * p.NE * 4 + (size_t)p.MT * (pt ? 1 : a.K / 32) * 4;
        if (argmax) b += 16 + (size_t)p.MT * rb * 8;
        if (qin) b += (size_t)p.MT * (16 * 4 + 8 * 64 * 4 + a.K) + 32;
        b += 32;  // 16-byte alignment of the activation sums and scales
        return b;
    };
    // registers: weights in flight (4 per row half) + activations (8 per token)
    // (the fused quantiser also holds its f32 input and norm weight: 4 per load)
    auto regs_of = [&](int ipw_) {
        return nh * ipw_ * 4 + 8 * p.MT + (qin ? 4 * (8 / p.nslots) * (p.MT + 1) : 0);
    };
    while (ipw > 1 && (lds_of(ipw) > 65536 || regs_of(ipw) > 96))
        ipw = ipw == 8 ? 6 : ipw == 6 ? 4 : ipw - 1;
    p.IPW = ipw;
    p.RB = p.nslots * ipw;
    p.lds = lds_of(ipw);
    p.grid = (unsigned)((a.N + p.RB - 1) / p.RB);
    return p;
}

template <int MT, int MODE, int G, bool PT, bool ARGMAX, bool QIN>
hipError_t launch_ipw(const Plan& pl, const GemvParams& gp, hipStream_t s) {
    dim3 grid(pl.grid), block(64 * pl.waves);
    const LinearArgs& a = gp.a;
    // the preloaded arguments (gemv_kernel): plan fields packed in two words
    const uint32_t plan = (uint32_t)gp.RB | ((uint32_t)gp.nslots << 8) | ((uint32_t)gp.J << 12) | ((uint32_t)a.M << 16);
    const uint32_t groups = (uint32_t)gp.NG | ((uint32_t)gp.NE << 16);
    const int8_t* xq_slot = QIN ? reinterpret_cast<const int8_t*>(gp.qin.x) : a.xq;
    const float* dx_slot = QIN ? gp.qin.norm_w : a.dx;
#define WQ_GEMV_LAUNCH(IPW)                                                                                 \
    hipLaunchKernelGGL((gemv_kernel<MT, MODE, G, PT, IPW, ARGMAX, QIN>), grid, block, pl.lds, s, a.wq, xq_slot, \
                       a.ws, dx_slot, (int)a.N, (int)a.K, plan, groups, a.xs, a.y, gp)
    switch (pl.IPW) {
        case 1: WQ_GEMV_LAUNCH(1); break;
        case 2: WQ_GEMV_LAUNCH(2); break;
        case 3: WQ_GEMV_LAUNCH(3); break;
        case 4: WQ_GEMV_LAUNCH(4); break;
        case 6: WQ_GEMV_LAUNCH(6); break;
        default: WQ_GEMV_LAUNCH(8); break;
    }
#undef WQ_GEMV_LAUNCH
    return hipGetLastError();
}

template <int MT, int MODE, bool ARGMAX, bool QIN>
hipError_t launch_gpt(const Plan& pl, const GemvParams& gp, hipStream_t s) {
    const bool pt = gp.a.GA == gp.a.K;
    if constexpr (QIN) {  // per token only (checked on the host)
        return gp.a.G == 128 ? launch_ipw<MT, MODE, 128, true, ARGMAX, true>(pl, gp, s)
                             : launch_ipw<MT, MODE, 32, true, ARGMAX, true>(pl, gp, s);
    } else {
        if (gp.a.G == 128) {
            return pt ? launch_ipw<MT, MODE, 128, true, ARGMAX, false>(pl, gp, s)
                      : launch_ipw<MT, MODE, 128, false, ARGMAX, false>(pl, gp, s);
        }
        return pt ? launch_ipw<MT, MODE, 32, true, ARGMAX, false>(pl, gp, s)
                  : launch_ipw<MT, MODE, 32, false, ARGMAX, false>(pl, gp, s);
    }
}

template <int MODE, bool ARGMAX, bool QIN>
hipError_t launch_mt(const Plan& pl, const GemvParams& gp, hipStream_t s) {
    if constexpr (QIN) {  // M <= 2 (checked on the host)
        return pl.MT == 1 ? launch_gpt<1, MODE, ARGMAX, true>(pl, gp, s)
                          : launch_gpt<2, MODE, ARGMAX, true>(pl, gp, s);
    } else {
        switch (pl.MT) {
            case 1: return launch_gpt<1, MODE, ARGMAX, false>(pl, gp, s);
            case 2: return launch_gpt<2, MODE, ARGMAX, false>(pl, gp, s);
            case 4: return launch_gpt<4, MODE, ARGMAX, false>(pl, gp, s);
            default: return launch_gpt<8, MODE, ARGMAX, false>(pl, gp, s);
        }
    }
}

GemvParams params_of(const LinearArgs& a, const Plan& pl) {
    GemvParams gp{};
    gp.a = a;
    gp.J = pl.J;
    gp.nslots = pl.nslots;
    gp.RB = pl.RB;
    gp.NE = pl.NE;
    gp.NEP = pl.NEP;
    gp.NG = pl.NG;
    gp.nblocks = (int)pl.grid;
    return gp;
}

}  // namespace

template <int MODE, int MT>
hipError_t launch_one(const LinearArgs& a, int ipw, unsigned grid, hipStream_t s) {
    dim3 g(grid), b(64 * kOneSlots);
#define WQ_ONE_LAUNCH(IPW) \
    hipLaunchKernelGGL((gemv_one_kernel<MODE, IPW, MT>), g, b, 0, s, a.wq, a.xq, a.ws, a.xs, a.dx, a.y, (int)a.N, \
                       (int)a.M)
    switch (ipw) {
        case 1: WQ_ONE_LAUNCH(1); break;
        case 2: WQ_ONE_LAUNCH(2); break;
        case 3: WQ_ONE_LAUNCH(3); break;
        case 4: WQ_ONE_LAUNCH(4); break;
        case 6: WQ_ONE_LAUNCH(6); break;
        default: WQ_ONE_LAUNCH(8); break;
    }
#undef WQ_ONE_LAUNCH
    return hipGetLastError();
}

// rows per wave of the specialised kernel: the fewest that keep the grid
// within the target, one included
int one_ipw(const LinearArgs& a) {
    for (int c : {1, 2, 3, 4, 6, 8})
        if ((a.N + kOneSlots * c - 1) / (kOneSlots * c) <= kGemvTargetWgs) return c;
    return 8;
}
// one or two tokens always; 3..8 while each wave folds at most eight
// (token, row) values (tokens x row halves x rows per wave), beyond which
// the LDS epilogue, which spreads the folds over lanes, is faster
bool one_fits(const LinearArgs& a) {
    if (a.M <= 2) return true;
    const int mt = a.M <= 4 ? 4 : 8, nh = a.mode == 2 ? 2 : 1;
    return mt * nh * one_ipw(a) <= 8;
}

hipError_t launch_gemv(const LinearArgs& a, hipStream_t s) {
    if (gemv_mfma_fits(a)) return launch_gemv_mfma(a, nullptr, s);
    // up to eight tokens (one_fits), one full pass, per-token group 128, no
    // debug dump: the specialised kernel (bit-identical outputs; the rows
    // per wave do not change any output, only which wave computes a row)
    if (a.M <= 8 && a.GA == a.K && a.G == 128 && a.K == kGemvPassK && !a.acc_dump && one_fits(a)) {
        // the fewest rows per wave that keep the grid within the target, one
        // included (measured: one row per wave at N = 2048 and 3072, 2.19
        // and 2.33 us against 2.24 and 2.42 with two; two at N = 6144)
        const int ipw = one_ipw(a);
        const unsigned grid = (unsigned)((a.N + kOneSlots * ipw - 1) / (kOneSlots * ipw));
        if (a.M > 4) {
            switch (a.mode) {
                case 0: return launch_one<0, 8>(a, ipw, grid, s);
                case 1: return launch_one<1, 8>(a, ipw, grid, s);
                default: return launch_one<2, 8>(a, ipw, grid, s);
            }
        }
        if (a.M > 2) {
            switch (a.mode) {
                case 0: return launch_one<0, 4>(a, ipw, grid, s);
                case 1: return launch_one<1, 4>(a, ipw, grid, s);
                default: return launch_one<2, 4>(a, ipw, grid, s);
            }
        }
        if (a.M == 2) {
            switch (a.mode) {
                case 0: return launch_one<0, 2>(a, ipw, grid, s);
                case 1: return launch_one<1, 2>(a, ipw, grid, s);
                default: return launch_one<2, 2>(a, ipw, grid, s);
            }
        }
        switch (a.mode) {
            case 0: return launch_one<0, 1>(a, ipw, grid, s);
            case 1: return launch_one<1, 1>(a, ipw, grid, s);
            default: return launch_one<2, 1>(a, ipw, grid, s);
        }
    }
    Plan pl = make_plan(a, false);
    GemvParams gp = params_of(a, pl);
    switch (a.mode) {
        case 0: return launch_mt<0, false, false>(pl, gp, s);
        case 1: return launch_mt<1, false, false>(pl, gp, s);
        default: return launch_mt<2, false, false>(pl, gp, s);
    }
}

hipError_t launch_lm_head_argmax(const LinearArgs& a, const ArgmaxArgs& am, hipStream_t s) {
    if (gemv_mfma_fits(a)) return launch_gemv_mfma(a, &am, s);
    Plan pl = make_plan(a, true);
    GemvParams gp = params_of(a, pl);
    gp.am = am;
    return launch_mt<0, true, false>(pl, gp, s);
}

hipError_t launch_gemv_quant_in(const LinearArgs& a, const QuantInArgs& q, hipStream_t s) {
    Plan pl = make_plan(a, false, true);
    GemvParams gp = params_of(a, pl);
    gp.qin = q;
    switch (a.mode) {
        case 0: return launch_mt<0, false, true>(pl, gp, s);
        case 1: return launch_mt<1, false, true>(pl, gp, s);
        default: return launch_mt<2, false, true>(pl, gp, s);
    }
}

}  // namespace wq

#ifdef WQ_TIMELINE
// The stamps of the last launch (kTimelineWgs x 8 words) into host memory.
extern "C" int wq_timeline_read(void* host, size_t bytes) {
    const size_t n = sizeof(unsigned long long) * wq::kTimelineWgs * 8;
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(wq::wq_timeline), bytes < n ? bytes : n);
}
#endif
