// Prefill GEMM Y[M, N] = X W^T on int8 MFMA (webyIQ
// crates/engine/src/shaders/gemm_q4q8.wgsl, host side Builder::gemm in
// crates/engine/src/graph.rs:200-205; the reference runs it on ALU
// dot4I8Packed in 32x32 tiles).
//
// y[t,n] = dx[t] * sum_g (s[n,g] * A[t,n,g] + m[n,g] * X[t,g]),
// A = exact int32 sum of q * xq over group g, X = sum of xq over g.
//
// MI355X design.  A workgroup of 4 waves (2 along M x 2 along N, one per SIMD)
// owns a 128-token x BN-row tile, and each wave a 64 x BN/2 block of 32 x 32
// subtiles computed with v_mfma_i32_32x32x32_i8 (the full-rate int8 MFMA on
// gfx950; the 16x16x64 form runs at half rate).  Every tile of a K step (128
// codes) travels global -> LDS directly (global_load_lds, no registers): the
// int8 activations, the packed int4 weights, the scale words.  A ring of 4
// LDS stages keeps 3 steps in flight; each step ends with one barrier,
// preceded by a wait for exactly the loads of the next step.  Each wave
// expands its weight fragments from nibbles to int8 in registers.  Tiles
// are stored in rows whose 16-byte chunks are XOR-swizzled by the row index,
// so that the 16-byte fragment reads of consecutive rows hit distinct banks.
//
// Folding the exact group sums into fp32 is VALU work per output element per
// group, as much issue time as the MFMAs themselves.  The per-token formats
// (group 128, and group 32 with one MFMA pair and one fold per group) keep it
// at two instructions, acc = fma(s, float(A), acc), and compute the min term
// sum_g m * X up front on the f16 MFMA: X = 64 * X_hi + X_lo with 64 * X_hi
// and X_lo exact in f16 (|X| <= 128 * 127), so each product with the f16 m
// is exact.  Per-32 activation scales fold both terms on the VALU.  Tiles
// are assigned XCD by XCD so that the workgroups sharing a weight tile share
// one L2.
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

#pragma clang fp contract(off)

namespace wq {
namespace {

constexpr int kBK = 128;          // codes per K step (= bytes per int8 tile row)
constexpr int kBM = 128;          // tokens per tile
constexpr int kWaveGroup = 256;   // 4 waves: 2 along M x 2 along N
constexpr int kXcds = 8;          // MI355X: 8 XCDs, workgroups dispatched round robin
constexpr int kLdsBytes = 160 * 1024;  // LDS per workgroup (gfx950)

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

// Spin limit of a split-K partner's wait for the first half's partial sums
// (each poll one device-coherent load plus a short sleep; ~0.5 s, far beyond
// any launch).
constexpr unsigned kSplitSpinLimit = 1u << 22;
// s_getreg operand of HW_REG_XCC_ID (hardware register 20 on gfx940 and
// later), bits 3:0: the XCD the wave runs on
constexpr int kHwRegXccId = 20 | (0 << 6) | ((4 - 1) << 11);

struct GemmParams {
    LinearArgs a;
    int tilesM, tilesN;
    int NE, NG;
    // split K across workgroup pairs (FAST formats): workspace of per-tile
    // ready flags (one 64-byte line each) and partial sums
    int split;
    unsigned int* flags;  // [T] lines
    float* part;          // [T][128 * BN] partial sums of the first half
};

// Chunk swizzles: activation rows are 128 bytes (8 chunks), packed weight
// rows 64 bytes (4 chunks); chunk c of row r sits at position c ^ f(r).
__device__ __forceinline__ int swz_a(int r) { return (r ^ (r >> 3)) & 7; }
__device__ __forceinline__ int swz_b(int r) { return (r >> 1) & 3; }
// Packed weight rows of two K steps (128 bytes, 8 chunks: the even step's 4,
// then the odd step's): chunk c of row r at position c ^ swz_p(r), so that 16
// consecutive rows' 16-byte reads of one chunk cover 256 distinct bytes of
// banks.
__device__ __forceinline__ int swz_p(int r) { return (r >> 1) & 7; }

// f(std::integral_constant<int, I>) for I = B .. E-1, in order
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// 16 codes (8 packed bytes) -> 16 int8 in code order: the low nibbles of a
// word are codes 8i..8i+3, the high nibbles 8i+4..8i+7.
__device__ __forceinline__ v4i expand8(uint32_t w0, uint32_t w1) {
    return v4i{(int)(w0 & kNibbleMask), (int)((w0 >> 4) & kNibbleMask),
               (int)(w1 & kNibbleMask), (int)((w1 >> 4) & kNibbleMask)};
}

// End of a pipeline step: wait until at most n vector-memory operations of
// this wave are in flight and all its LDS operations are done, then barrier.
// The barrier carries no memory fence, so loads issued for later steps stay
// in flight across it.
template <int n>
__device__ __forceinline__ void step_barrier() {
    static_assert(n >= 0 && n < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4));
    asm volatile("s_barrier" ::: "memory");
}

// Direct global -> LDS loads of 16 (4) bytes per lane: lane l's bytes land at
// LDS address lds + 16 l (4 l); base and lds are wave-uniform, off per lane.
// Written as inline assembly so that the compiler's wait-count pass does not
// track them: it cannot tell the stages of the ring apart and would wait for
// every load in flight before the first LDS read of a step.  The waits these
// loads need are explicit (step_barrier); for loads the compiler does track,
// untracked loads issued in between only make its waits stricter.
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
__device__ __forceinline__ void dma4(const void* base, uint32_t off, const void* lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
                 ::"v"(off), "s"(uniform_ptr(base)), "s"(lds_addr(lds)) : "memory", "m0");
}
// The same with the LDS destination given as a wave-uniform 32-bit LDS byte
// address (kept in scalar registers by the caller: no per-load conversion of
// a generic pointer).
__device__ __forceinline__ void dma16_at(const void* base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 ::"v"(off), "s"(uniform_ptr(base)), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma4_at(const void* base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
                 ::"v"(off), "s"(uniform_ptr(base)), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

// Threads of a workgroup: the per-token group-128 format runs two groups of
// 4 waves on alternate K steps (two waves per SIMD, so that one wave's fold
// overlaps the other's MFMAs), the other formats one group (their fp32 fold
// order is fixed).
constexpr int gemm_threads(int G, bool PT) { return PT && (G == 128 || G == 32) ? 2 * kWaveGroup : kWaveGroup; }

template <int BN, int G, bool PT, int MODE, bool DUMP>
__global__ __launch_bounds__(gemm_threads(G, PT)) void gemm_kernel(GemmParams p) {
    constexpr int BM = kBM;
    constexpr int GE = PT ? G : 32;          // accumulation group
    constexpr bool FAST = PT && (G == 128 || G == 32);  // min term on the f16 MFMA
    constexpr bool G32 = FAST && G == 32;    // one MFMA and one fold per group
    constexpr int KS = FAST ? 2 : 1;         // wave groups splitting the K steps
    constexpr int NES = kBK / GE;            // accumulation groups per step
    constexpr int NGS = kBK / G;             // weight groups per step
    constexpr int TM = 2;                    // 32-token subtiles per wave
    constexpr int TN = BN / 64;              // 32-row subtiles per wave
    constexpr int NST = FAST ? 4 : 3;        // LDS stages (steps in flight + 1)
    // direct-to-LDS instructions per wave and step (4 waves share each tile)
    constexpr int A_PW = BM * kBK / 1024 / 4;          // 1 KiB activation blocks
    constexpr int B_PW = BN * (kBK / 2) / 1024 / 4;    // 1 KiB packed weight blocks
    constexpr int S_W = BN * NGS;                      // scale words per step
    constexpr int S_PW = (S_W + 255) / 256;            // 64-word blocks
    constexpr int X_PW = FAST ? 0 : NES * BM / 256;    // group sums (non-fast)
    constexpr int D_PW = PT ? 0 : NES * BM / 256;      // per-32 scales
    constexpr int VM = A_PW + B_PW + S_PW + X_PW + D_PW;
    static_assert(BN % 64 == 0 && B_PW == TN, "tile width");
    static_assert(MODE != 2 || TN % 2 == 0, "mode 2 pairs gate/up subtiles");
    static_assert((NST - 2) * VM < 64, "vmcnt range");

    // LDS: NST stages of (activations, packed weights, scale words, group
    // sums, per-32 scales); the partial sums of the second wave group reuse
    // it at the end.  With two wave groups (PAIRB) the packed weights of a
    // round's two steps share one buffer of BN rows x 128 bytes, NST / 2 of
    // them after the stages: a row's two 64-byte halves are one cache line,
    // fetched by one load, half of the rows by each group.
    constexpr bool PAIRB = KS == 2;
    constexpr int A_SZ = BM * kBK, B_SZ = BN * kBK / 2, S_SZ = S_PW * 1024;
    constexpr int X_SZ = FAST ? 16 : NES * BM * 4, D_SZ = PT ? 16 : NES * BM * 4;
    constexpr int OFF_S = A_SZ + (PAIRB ? 0 : B_SZ), OFF_X = OFF_S + S_SZ, OFF_D = OFF_X + X_SZ;
    constexpr int ST_SZ = OFF_D + D_SZ;
    constexpr int PB_BASE = NST * ST_SZ;  // pair buffers (PAIRB)
    constexpr int RING_SZ = PB_BASE + (PAIRB ? NST * B_SZ : 0);
    constexpr int RED_SZ = KS > 1 ? kWaveGroup * TM * TN * 16 * 4 : 0;
    constexpr int NWAVES = gemm_threads(G, PT) / 64;
    constexpr int TR_STRIDE = 36;  // floats per row of a wave's 32 x 32 output transpose (16-byte rows)
    constexpr int TR_SZ = NWAVES * 32 * TR_STRIDE * 4;
    constexpr int BODY_SZ = RING_SZ > RED_SZ ? RING_SZ : RED_SZ;
    // + the tile's per-token scales; then (per-token group-128 format) the
    // tile's scale words for the whole K range, loaded once: BN rows of NGP
    // words (NGP = NG rounded up to odd, so that 32 consecutive rows read
    // distinct banks), in what is left of the 160 KiB
    constexpr int SP_BASE = (BODY_SZ > TR_SZ ? BODY_SZ : TR_SZ) + BM * 4;
    constexpr int SP_NGP = FAST ? (kLdsBytes - SP_BASE) / (BN * 4) : 0;  // row words that fit
    constexpr int LDS_SZ = SP_BASE + BN * SP_NGP * 4;
    static_assert(LDS_SZ <= kLdsBytes, "LDS");
    __shared__ __align__(1024) unsigned char lds[LDS_SZ];
    float* dx_tile = reinterpret_cast<float*>(lds + SP_BASE - BM * 4);
    auto As = [&](int st) -> int8_t* { return reinterpret_cast<int8_t*>(lds + st * ST_SZ); };
    // packed weights of stage st: its own region, or (PAIRB) the pair buffer
    // of its round, the step's half selected when reading
    auto Bs = [&](int st) -> uint32_t* {
        return reinterpret_cast<uint32_t*>(PAIRB ? lds + PB_BASE + (st >> 1) * 2 * B_SZ : lds + st * ST_SZ + A_SZ);
    };
    auto Ss = [&](int st) -> uint32_t* { return reinterpret_cast<uint32_t*>(lds + st * ST_SZ + OFF_S); };
    auto Xs = [&](int st) -> int32_t* {  // [group][token]
        return reinterpret_cast<int32_t*>(lds + st * ST_SZ + OFF_X);
    };
    auto Ds = [&](int st) -> float* { return reinterpret_cast<float*>(lds + st * ST_SZ + OFF_D); };

    const LinearArgs& a = p.a;
    pin_arg(a.wq); pin_arg(a.ws); pin_arg(a.xq); pin_arg(a.dx); pin_arg(a.xs); pin_arg(a.y);
    pin_arg(a.N); pin_arg(a.K); pin_arg(a.M); pin_arg(a.params);
    pin_arg(p.tilesM); pin_arg(p.tilesN); pin_arg(p.NE); pin_arg(p.NG);
    if (DUMP) pin_arg(a.acc_dump);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // wave group (K steps s with s % KS == wk) and wave within its group;
    // wave-uniform, so that every step and stage index derived from them
    // stays scalar
    const int wk = __builtin_amdgcn_readfirstlane(tid / kWaveGroup);
    const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) & 3);
    // tokens of this call: M, or (device Params) min(p.m, M) read when the
    // kernel runs; the grid is sized for M
    int64_t M = a.M;
    if (a.params) {
        const int64_t pm = (int64_t)a.params[kParamM];
        M = pm < M ? pm : M;
    }
    const int64_t N = a.N;
    const int K = (int)a.K;
    const int NG = p.NG, NE = p.NE;

    // XCD-aware tile order: consecutive tiles (same weight rows) on one XCD
    const int T = p.tilesM * p.tilesN;
    int bid = blockIdx.x;
    // Split K (FAST formats): workgroups T.. 2T-1 take the second half of the
    // K steps of tile bid - T; with T a multiple of 8 the pair shares an XCD.
    // (Widths up to 128 only: the exchange's registers do not fit beside the
    // wider tiles' accumulators.)
    constexpr bool SPLITOK = FAST && BN <= 128;
    const bool split = SPLITOK && p.split;
    const int half = split && bid >= T ? 1 : 0;
    bid -= half * T;
    const int nsteps = split ? K / kBK / 2 : K / kBK;  // this workgroup's K steps
    const int s_begin = half * nsteps;
    const int NGL = split ? NG / 2 : NG;               // its weight groups
    const int g_begin = half * NGL;
    const int xcd = bid % kXcds, li = bid / kXcds;
    const int per = T / kXcds, rem = T % kXcds;
    const int lt = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + li;
    // tiles in groups of GM token tiles: the run of consecutive tiles one
    // XCD takes spans GM token tiles x (run / GM) row tiles, so that for long
    // rows (K >= 4096, 128 tokens x K bytes per token tile) its L2 holds the
    // activations of 4 token tiles rather than of all of them; shorter rows
    // keep every token tile of a row tile together (GM = tilesM)
    const int GM = K >= 4096 ? 4 : p.tilesM;
    const int grp = lt / (GM * p.tilesN);
    const int gm = p.tilesM - grp * GM < GM ? p.tilesM - grp * GM : GM;
    const int off = lt - grp * GM * p.tilesN;
    const int tile_m = grp * GM + off % gm, tile_n = off / gm;
    const int64_t m0 = (int64_t)tile_m * BM;
    if (m0 >= M) return;  // a token tile past this step's tokens (uniform: nothing issued yet)
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

    // ---------------- staging: per-lane source offsets ----------------
    // A direct-to-LDS instruction writes 64 consecutive 16-byte (or 4-byte)
    // slots, lane l the l-th; each lane fetches whatever belongs in its slot.
    uint32_t a_off[A_PW], b_off[B_PW], s_off[S_PW], x_off[X_PW > 0 ? X_PW : 1], d_off[D_PW > 0 ? D_PW : 1];
#pragma unroll
    for (int i = 0; i < A_PW; ++i) {  // block = 8 rows of 128 B
        const int r = 8 * (A_PW * wave + i) + lane / 8;
        a_off[i] = (uint32_t)(trow(r) * K + 16 * ((lane % 8) ^ swz_a(r)));
    }
#pragma unroll
    for (int i = 0; i < B_PW; ++i) {
        if constexpr (PAIRB) {  // block = 8 rows of 128 B; the 8 waves cover BN rows
            const int r = 8 * ((4 * wk + wave) * B_PW + i) + lane / 8;
            b_off[i] = (uint32_t)(wrow(r) * (K / 2) + 16 * ((lane % 8) ^ swz_p(r)));
        } else {  // block = 16 rows of 64 B
            const int r = 16 * (B_PW * wave + i) + lane / 4;
            b_off[i] = (uint32_t)(wrow(r) * (K / 2) + 16 * ((lane % 4) ^ swz_b(r)));
        }
    }
#pragma unroll
    for (int i = 0; i < S_PW; ++i) {  // block = 64 scale words, [row][group]
        int w = 64 * (S_PW * wave + i) + lane;
        w = w < S_W ? w : 0;  // padding slots re-read word 0
        s_off[i] = (uint32_t)(wrow(w / NGS) * NG + w % NGS);
    }
#pragma unroll
    for (int i = 0; i < X_PW; ++i) {  // block = 64 tokens of one group, [group][token]
        const int w = 64 * (X_PW * wave + i) + lane;
        x_off[i] = (uint32_t)(trow(w % BM) * NE + w / BM);
    }
#pragma unroll
    for (int i = 0; i < D_PW; ++i) {
        const int w = 64 * (D_PW * wave + i) + lane;
        d_off[i] = (uint32_t)(trow(w % BM) * (K / 32) + w / BM);
    }
    // The scale words of every K step at once when they fit (the per-token
    // group-128 format) and the row has 32 steps or more: each step
    // otherwise fetches BN scattered 4-byte words, one cache-line request
    // each.  Measured: K = 6144, N = 2048 27.08 -> 25.49 us; at K = 2048 (16
    // steps) the preload's start-up cost outweighs it, 22.31 -> 22.65 us.
    const int NGPs = NGL + 1 - (NGL & 1);  // odd row stride
    // (the last 64-word instruction may run up to 63 words past BN rows)
    const bool spre = FAST && !G32 && nsteps >= 32 && BN * NGPs + 64 <= BN * SP_NGP;  // uniform
    const uint32_t* sp_lds = reinterpret_cast<const uint32_t*>(lds + SP_BASE);
    // Every load is unconditional (steps past the end re-read the last one),
    // so each call issues the same vector-memory instructions per wave.
    // LDS byte address of the ring (scalar); stage st, part at byte b of it
    const uint32_t lds0 = lds_addr(lds);
    auto stage_at = [&](int st, int b) -> uint32_t { return lds0 + (uint32_t)(st * ST_SZ + b); };
    auto dma = [&](int step, const int st) {
        step = step < nsteps ? step : nsteps - 1;
        const int8_t* xq = a.xq + (s_begin + step) * kBK;
        const uint32_t* ws = a.ws + (s_begin + step) * NGS;
#pragma unroll
        for (int i = 0; i < A_PW; ++i) dma16_at(xq, a_off[i], stage_at(st, 1024 * (A_PW * wave + i)));
        if constexpr (PAIRB) {
            // steps s0 and s0 + 1 into the pair buffer of stage st; with an
            // odd step count the last round has no second step, and the lanes
            // of the second halves re-read the first (a row's end is not
            // passed): the half of a lane's chunk is bit 2 of
            // (lane % 8) ^ swz_p(r), = ((lane >> 2) ^ block) & 1
            const int s0 = step & ~1;
            const uint8_t* wq = reinterpret_cast<const uint8_t*>(a.wq) + (s_begin + s0) * (kBK / 2);
            const bool tail = s0 + 1 >= nsteps;  // uniform
#pragma unroll
            for (int i = 0; i < B_PW; ++i) {
                const int blk = (4 * wk + wave) * B_PW + i;
                const uint32_t off = tail ? b_off[i] - 64u * (uint32_t)(((lane >> 2) ^ blk) & 1) : b_off[i];
                dma16_at(wq, off, lds0 + (uint32_t)(PB_BASE + (st >> 1) * 2 * B_SZ + 1024 * blk));
            }
        } else {
            const uint8_t* wq = reinterpret_cast<const uint8_t*>(a.wq) + (s_begin + step) * (kBK / 2);
#pragma unroll
            for (int i = 0; i < B_PW; ++i) dma16_at(wq, b_off[i], stage_at(st, A_SZ + 1024 * (B_PW * wave + i)));
        }
        if (!spre) {
#pragma unroll
            for (int i = 0; i < S_PW; ++i)
                dma4_at(ws, 4 * s_off[i], stage_at(st, OFF_S + 256 * (S_PW * wave + i)));
        }
        if constexpr (!FAST) {
            const int32_t* xs = a.xs + step * NES;
#pragma unroll
            for (int i = 0; i < X_PW; ++i)
                dma4_at(xs, 4 * x_off[i], stage_at(st, OFF_X + 256 * (X_PW * wave + i)));
        }
        if constexpr (!PT) {
            const float* dxp = a.dx + step * NES;
#pragma unroll
            for (int i = 0; i < D_PW; ++i)
                dma4_at(dxp, 4 * d_off[i], stage_at(st, OFF_D + 256 * (D_PW * wave + i)));
        }
    };

    // ---------------- compute layout ----------------
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, h = lane >> 5;
    // tile row (of W) of this lane's column in subtile j
    auto bcol = [&](int j) -> int {
        if (MODE == 2) {
            constexpr int H = TN / 2;
            return (j < H ? wn * (BN / 4) + 32 * j : BN / 2 + wn * (BN / 4) + 32 * (j - H)) + l32;
        }
        return wn * (BN / 2) + 32 * j + l32;
    };
    // token row (within the tile) of accumulator element r of subtile i
    auto arow = [&](int i, int r) -> int { return wm * 64 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3); };

    // min term operands: blocks of 8 groups, wave group wk taking blocks
    // wk, wk + KS, ... (the groups' partial sums are added at the end like
    // their K steps'), with NSL blocks in flight per wave in registers: two
    // up to 2 columns per wave, one at 3.  The first NSL are requested
    // before any tile load: loads return in issue order, so operands
    // requested after the tiles would land after them.  With 4 columns the
    // registers are short: wave group 0 loads each block after the tiles,
    // when it is used.
    constexpr int NSL = TN <= 2 ? 2 : TN == 3 ? 1 : 0;
    constexpr int NSA = NSL > 0 ? NSL : 1;  // register slots
    // (with split K, this workgroup's groups g_begin .. g_begin + NGL - 1)
    const int nfull = NGL % 8 == 0 ? NGL / 8 : 0;  // full blocks (32-byte aligned rows: K a multiple of 1024)
    const int nblk = (NGL + 7) / 8;
    const int32_t* xr[TM];
    const uint32_t* sr[TN];
    int32_t xv[NSA][TM][8];
    uint32_t wv[NSA][TN][8];
    auto mt_full = [&](int32_t (&x)[TM][8], uint32_t (&w)[TN][8], int blk) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int4 lo = *reinterpret_cast<const int4*>(xr[i] + 8 * blk);
            const int4 hi = *reinterpret_cast<const int4*>(xr[i] + 8 * blk + 4);
            x[i][0] = lo.x; x[i][1] = lo.y; x[i][2] = lo.z; x[i][3] = lo.w;
            x[i][4] = hi.x; x[i][5] = hi.y; x[i][6] = hi.z; x[i][7] = hi.w;
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint4 lo = *reinterpret_cast<const uint4*>(sr[j] + 8 * blk);
            const uint4 hi = *reinterpret_cast<const uint4*>(sr[j] + 8 * blk + 4);
            w[j][0] = lo.x; w[j][1] = lo.y; w[j][2] = lo.z; w[j][3] = lo.w;
            w[j][4] = hi.x; w[j][5] = hi.y; w[j][6] = hi.z; w[j][7] = hi.w;
        }
    };
    // word by word, indices past the last group clamped (their values are zeroed)
    auto mt_words = [&](int32_t (&x)[TM][8], uint32_t (&w)[TN][8], int blk) {
        const int b = 8 * blk;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int u = 0; u < 8; ++u) x[i][u] = xr[i][b + u < NGL ? b + u : NGL - 1];
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int u = 0; u < 8; ++u) w[j][u] = sr[j][b + u < NGL ? b + u : NGL - 1];
    };
    auto mt_load = [&](auto slot, int blk) {
        constexpr int S = decltype(slot)::value;
        if (blk < nfull) mt_full(xv[S], wv[S], blk);
        else mt_words(xv[S], wv[S], blk);
    };
    using ic0 = std::integral_constant<int, 0>;
    using ic1 = std::integral_constant<int, NSA - 1>;
    auto mt_rows = [&]() {
#pragma unroll
        for (int i = 0; i < TM; ++i) xr[i] = a.xs + trow(wm * 64 + 32 * i + l32) * NE + g_begin;
#pragma unroll
        for (int j = 0; j < TN; ++j) sr[j] = a.ws + wrow(bcol(j)) * NG + g_begin;
    };
    if constexpr (FAST && NSL >= 1) {
        mt_rows();
        if (wk < nblk) mt_load(ic0{}, wk);
        if constexpr (NSL == 2)
            if (wk + KS < nblk) mt_load(ic1{}, wk + KS);
    }

    if (spre) {  // 64 words per instruction, the workgroup's waves in turn
        const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int nins = (BN * NGPs + 63) / 64;
        for (int i = wid; i < nins; i += NWAVES) {
            const int pw = 64 * i + lane;
            const int r = pw / NGPs, gg = pw - r * NGPs;
            const uint32_t src = r < BN && gg < NGL ? (uint32_t)(wrow(r) * NG + g_begin + gg) : 0u;  // padding: word 0
            dma4_at(a.ws, 4 * src, lds0 + (uint32_t)(SP_BASE + 256 * i));
        }
    }
    // the tile's per-token scales for the epilogue, ahead of the ring loads
    // (every wait below also covers them)
    if (PT && wave < BM / 64 && (KS == 1 || wk == 0))
        dma4(a.dx, 4 * (uint32_t)trow(64 * wave + lane), dx_tile + 64 * wave);

    // prologue loads: one group loads steps 0 .. NST-2; two groups load
    // their first step each
    if (KS == 1) {
#pragma unroll
        for (int q = 0; q < NST - 1; ++q) dma(q, q);
    } else {
        dma(wk, wk);
    }

    v16f facc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) facc[i][j] = v16f{};

    // min term: facc += sum_g m[n,g] * X[t,g] (per-token group-128 format
    // only) on v_mfma_f32_32x32x16_f16.  One MFMA covers 8 groups: lane half
    // h = 0 holds (64 X_hi, m), h = 1 (X_lo, m) of groups b .. b+7, both
    // halves of a row reading the same 32 bytes.
    auto min_term_block = [&](const int32_t (&xv)[TM][8], const uint32_t (&wv)[TN][8], int b) {
        v8h xa[TM], mb[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int32_t v = b + u < NGL ? xv[i][u] : 0;
                xa[i][u] = (_Float16)(h == 0 ? (float)((v >> 6) * 64) : (float)(v & 63));
            }
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int u = 0; u < 8; ++u)
                mb[j][u] = b + u < NGL ? __builtin_bit_cast(_Float16, (unsigned short)(wv[j][u] >> 16))
                                      : (_Float16)0.0f;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                facc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa[i], mb[j], facc[i][j], 0, 0, 0);
    };
    // this wave group's min term blocks, the two register slots in turn
    if constexpr (FAST && NSL == 0) {  // wave group 0 alone, block by block
        if (wk == 0) {
            mt_rows();
            for (int blk = 0; blk < nfull; ++blk) {
                int32_t x[TM][8];
                uint32_t w[TN][8];
                mt_full(x, w, blk);
                min_term_block(x, w, 8 * blk);
            }
            for (int blk = nfull; blk < nblk; ++blk) {
                int32_t x[TM][8];
                uint32_t w[TN][8];
                mt_words(x, w, blk);
                min_term_block(x, w, 8 * blk);
            }
        }
    } else if constexpr (FAST && NSL == 1) {
        for (int blk = wk; blk < nblk; blk += KS) {
            min_term_block(xv[0], wv[0], 8 * blk);
            if (blk + KS < nblk) mt_load(ic0{}, blk + KS);
        }
    } else if constexpr (FAST) {
        for (int blk = wk; blk < nblk; blk += 2 * KS) {
            min_term_block(xv[0], wv[0], 8 * blk);
            if (blk + 2 * KS < nblk) mt_load(ic0{}, blk + 2 * KS);
            if (blk + KS >= nblk) break;
            min_term_block(xv[NSA - 1], wv[NSA - 1], 8 * (blk + KS));
            if (blk + 3 * KS < nblk) mt_load(ic1{}, blk + 3 * KS);
        }
    }

    // the first step of each group has landed
    step_barrier<KS == 1 ? (NST - 2) * VM : 0>();

    const int rows_total = MODE == 2 ? 2 * (int)N : (int)N;
    auto dump = [&](int step, int e_local, int i, int br, const v16i& acc) {
        const int64_t e = (int64_t)(s_begin + step) * NES + e_local;
        const int64_t nn = n0 + (MODE == 2 ? (br < BN / 2 ? br : br - BN / 2) : br);
        const int64_t wr = MODE == 2 && br >= BN / 2 ? nn + N : nn;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t t = m0 + arow(i, r);
            if (t < M && nn < N) a.acc_dump[(t * rows_total + wr) * NE + e] = acc[r];
        }
    };

    auto compute = [&](const int step, const int st) __attribute__((always_inline)) {
        const int8_t* Ab = As(st);
        const uint8_t* Bb = reinterpret_cast<const uint8_t*>(Bs(st));
        // 16-byte chunk c (of 4) of this step's packed weights in tile row br
        auto bfrag = [&](int br, int c) -> uint4 {
            if constexpr (PAIRB)
                return *reinterpret_cast<const uint4*>(Bb + br * 128 + 16 * ((4 * (st & 1) + c) ^ swz_p(br)));
            else
                return *reinterpret_cast<const uint4*>(Bb + br * 64 + 16 * (c ^ swz_b(br)));
        };
        const uint32_t* Sb = Ss(st);
        // (FAST) scale word of tile row br for this step: Sx[br * sst]
        const uint32_t* Sx = spre ? sp_lds + step : Sb;
        const int sst = spre ? NGPs : 1;
        if (FAST) {
            // k-slice ks of lane half h = codes 64 h + 16 ks .. +15 of the
            // group (any assignment shared by both operands gives the same
            // sums): 32 contiguous packed bytes per lane and weight row.
            // Group 32: k-slice ks = group ks, lane half h its codes
            // 32 ks + 16 h .. +15, so that each MFMA sums one group.
            v4i af[4][TM];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int ra = wm * 64 + 32 * i + l32;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks)
                    af[ks][i] = *reinterpret_cast<const v4i*>(
                        Ab + ra * kBK + 16 * ((G32 ? 2 * ks + h : 4 * h + ks) ^ swz_a(ra)));
            }
            // (group 32) the 8 packed bytes of group c, lane half h, in tile row br
            auto bhalf = [&](int br, int c) -> uint2 {
                return *reinterpret_cast<const uint2*>(Bb + br * 128 + 16 * ((4 * (st & 1) + c) ^ swz_p(br)) + 8 * h);
            };
            auto bload = [&](int br, uint4& p0, uint4& p1) {
                if constexpr (G32) {
                    const uint2 q0 = bhalf(br, 0), q1 = bhalf(br, 1), q2 = bhalf(br, 2), q3 = bhalf(br, 3);
                    p0 = uint4{q0.x, q0.y, q1.x, q1.y};
                    p1 = uint4{q2.x, q2.y, q3.x, q3.y};
                } else {
                    p0 = bfrag(br, 2 * h);
                    p1 = bfrag(br, 2 * h + 1);
                }
            };
            // with up to 3 columns per wave, every column's packed weight
            // fragment and scale are read up front (one LDS latency per step
            // instead of one per column); wider tiles have no registers to spare
            constexpr bool PRE = TN <= 3;
            uint4 pb[PRE ? TN : 1][2];
            float sv[PRE ? TN : 1];
            if constexpr (PRE) {
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const int br = bcol(j);
                    bload(br, pb[j][0], pb[j][1]);
                    if constexpr (!G32) sv[j] = f16lo(Sx[br * sst]);
                }
            }
            // the columns with compile-time indices (a run-time column index
            // into facc or pb would put those arrays in scratch memory)
            static_for<0, TN>([&](auto jc) __attribute__((always_inline)) {
                constexpr int j = decltype(jc)::value;
                const int br = bcol(j);
                uint4 p0, p1;
                if constexpr (PRE) {
                    p0 = pb[j][0];
                    p1 = pb[j][1];
                } else {
                    bload(br, p0, p1);
                }
                v16i acc[TM];
                if constexpr (G32) {
                    // the row's four scale words of this step (16 bytes), then
                    // per group its two MFMAs and its fold (groups as
                    // compile-time indices: no array is indexed at run time)
                    const uint4 sw4 = *reinterpret_cast<const uint4*>(Sb + br * NGS);
                    auto group = [&](auto gc, uint32_t swg, uint32_t w0, uint32_t w1) __attribute__((always_inline)) {
                        constexpr int g = decltype(gc)::value;
                        const v4i b = expand8(w0, w1);
#pragma unroll
                        for (int i = 0; i < TM; ++i)
                            acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[g][i], b, v16i{}, 0, 0, 0);
                        const float s = f16lo(swg);
#pragma unroll
                        for (int i = 0; i < TM; ++i) {
                            if (DUMP) dump(step, g, i, br, acc[i]);
#pragma unroll
                            for (int r = 0; r < 16; ++r) facc[i][j][r] = fmaf(s, (float)acc[i][r], facc[i][j][r]);
                        }
                    };
                    group(std::integral_constant<int, 0>{}, sw4.x, p0.x, p0.y);
                    group(std::integral_constant<int, 1>{}, sw4.y, p0.z, p0.w);
                    group(std::integral_constant<int, 2>{}, sw4.z, p1.x, p1.y);
                    group(std::integral_constant<int, 3>{}, sw4.w, p1.z, p1.w);
                } else {
                    const v4i bf[4] = {expand8(p0.x, p0.y), expand8(p0.z, p0.w), expand8(p1.x, p1.y),
                                       expand8(p1.z, p1.w)};
#pragma unroll
                    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                        for (int i = 0; i < TM; ++i)
                            acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[ks][i], bf[ks],
                                                                           ks == 0 ? v16i{} : acc[i], 0, 0, 0);
                    const float s = PRE ? sv[PRE ? j : 0] : f16lo(Sx[br * sst]);
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        if (DUMP) dump(step, 0, i, br, acc[i]);
#pragma unroll
                        for (int r = 0; r < 16; ++r) facc[i][j][r] = fmaf(s, (float)acc[i][r], facc[i][j][r]);
                    }
                }
            });
        } else {
            // one MFMA per accumulation group of 32 codes, groups in order;
            // lane half h takes codes 32 ks + 16 h .. +15
#pragma unroll 1
            for (int ks = 0; ks < 4; ++ks) {
                v4i af[TM];
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const int ra = wm * 64 + 32 * i + l32;
                    af[i] = *reinterpret_cast<const v4i*>(Ab + ra * kBK + 16 * ((2 * ks + h) ^ swz_a(ra)));
                }
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const int br = bcol(j);
                    const uint2 pw = *reinterpret_cast<const uint2*>(Bb + br * 64 + 16 * (ks ^ swz_b(br)) + 8 * h);
                    const v4i bf = expand8(pw.x, pw.y);
                    const uint32_t sw = Sb[br * NGS + (32 * ks) / G];
                    const float s = f16lo(sw), m = f16hi(sw);
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        const v16i acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf, v16i{}, 0, 0, 0);
                        if (DUMP) dump(step, ks, i, br, acc);
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const int tr = wm * 64 + 32 * i + 8 * q + 4 * h;
                            const int4 xg = *reinterpret_cast<const int4*>(&Xs(st)[ks * BM + tr]);
                            float4 dg = make_float4(0.f, 0.f, 0.f, 0.f);
                            if (!PT) dg = *reinterpret_cast<const float4*>(&Ds(st)[ks * BM + tr]);
                            const float xr[4] = {(float)xg.x, (float)xg.y, (float)xg.z, (float)xg.w};
                            const float dr[4] = {dg.x, dg.y, dg.z, dg.w};
#pragma unroll
                            for (int u = 0; u < 4; ++u) {
                                const int r = 4 * q + u;
                                float v = facc[i][j][r];
                                if (PT) {
                                    v = fmaf(s, (float)acc[r], v);
                                    v = fmaf(m, xr[u], v);
                                } else {
                                    v = fmaf(s * dr[u], (float)acc[r], v);
                                    v = fmaf(m * dr[u], xr[u], v);
                                }
                                facc[i][j][r] = v;
                            }
                        }
                    }
                }
            }
        }
    };

    if constexpr (KS == 1) {
        // step s: load step s + NST - 1 into stage (s - 1) % NST, which step
        // s - 1 left before the last barrier; compute step s from stage
        // s % NST; wait for the loads of step s + 1 and barrier.
        for (int s = 0; s < nsteps; ++s) {
            dma(s + NST - 1, (s + NST - 1) % NST);
            compute(s, s % NST);
            step_barrier<(NST - 2) * VM>();
        }
    } else {
        // round r: group wk loads step 2r + 2 + wk into the stage that its
        // step 2r - 2 + wk left and computes step 2r + wk; both steps of the
        // next round land before the barrier.  A group only ever uses stages
        // wk and wk + 2, so (up to 3 columns per wave) rounds run in pairs
        // with the stage parity fixed at compile time: each fragment address
        // is then a loop-invariant lane address plus a constant (the
        // instruction's offset field), not a per-step addition.
        static_assert(KS == 2 && NST == 4, "two groups on a ring of four stages");
        if constexpr (TN <= 3) {
            auto round = [&](auto parity, int r) __attribute__((always_inline)) {
                constexpr int P = decltype(parity)::value;
                const int sl = 2 * r + 2 + wk, sc = 2 * r + wk;
                dma(sl, wk + 2 * (1 - P));
                if (sc < nsteps) compute(sc, wk + 2 * P);
                step_barrier<0>();
            };
            for (int r = 0; 2 * r < nsteps; r += 2) {
                round(std::integral_constant<int, 0>{}, r);
                if (2 * (r + 1) >= nsteps) break;
                round(std::integral_constant<int, 1>{}, r + 1);
            }
        } else {  // wider tiles: no registers for the extra lane addresses
            for (int r = 0; KS * r < nsteps; ++r) {
                const int sl = KS * r + KS + wk, sc = KS * r + wk;
                dma(sl, sl % NST);
                if (sc < nsteps) compute(sc, sc % NST);
                step_barrier<0>();
            }
        }
    }
    // no direct-to-LDS load may outlive the workgroup
    step_barrier<0>();

    // subtiles this wave stores: all of them with one wave group; with two,
    // group g stores subtile row i = g after adding the other group's partial
    // sums (exchanged through LDS, 16 bytes per lane and instruction,
    // lane-major; the fp32 addition of two partials is the same in either
    // order)
    constexpr int I0 = 0, I1 = KS > 1 ? 1 : TM;
    int ilo = I0, ihi = I1;
    if constexpr (KS > 1) {
        static_assert(TM == 2, "one subtile row per wave group");
        v4f* red = reinterpret_cast<v4f*>(lds);
        const int give = 1 - wk;  // the subtile row the other group stores
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                v4f v;
#pragma unroll
                for (int u = 0; u < 4; ++u) v[u] = wk == 0 ? facc[1][j][4 * q + u] : facc[0][j][4 * q + u];
                red[(((give * 4 + wave) * TN + j) * 4 + q) * 64 + lane] = v;
            }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const v4f o = red[(((wk * 4 + wave) * TN + j) * 4 + q) * 64 + lane];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int r = 4 * q + u;
                    if (wk == 0) facc[0][j][r] = facc[0][j][r] + o[u];
                    else facc[1][j][r] = o[u] + facc[1][j][r];
                }
            }
        ilo = wk;
        ihi = wk + 1;
    }

    // Split K: the first half's workgroup hands its partial sums (this
    // thread's subtile row ilo, every column) to its partner through the
    // workspace and ends; the partner adds them to its own, first half
    // first (one fixed order), and runs the epilogue.  The partial stores
    // and loads are agent-scope atomics (sc1: performed at the device's
    // coherence point, past a non-coherent L2), so the same argument as the
    // lm_head argmax combine orders them without a release fence: the
    // stores are complete (vmcnt 0) in every wave before the barrier, the
    // flag is set after it, and the partner's loads are issued after its
    // poll has seen the flag.  The partner waits only for a workgroup of
    // lower index (dispatched before it, waiting for nothing), and the wait
    // is bounded: if it ran out, the tile's outputs are written as NaN.
    if constexpr (SPLITOK) {
        if (split) {
            // this thread's values, subtile row wk, as 4 x TN 16-byte chunks
            // (compile-time indices only: a run-time index would put facc in
            // scratch memory); chunk c of this thread at slot[c * 64]
            static_assert(TN <= 2, "the exchange holds 8 chunks in flight");
            v4f* slot = reinterpret_cast<v4f*>(p.part) + (size_t)lt * (BM * BN / 4) +
                        (size_t)(tid >> 6) * (TN * 4 * 64) + lane;
            unsigned int* flag = p.flags + (size_t)lt * 16;
            // the XCD this workgroup runs on (gfx950 XCC_ID, bits 3:0)
            const unsigned xcc = __builtin_amdgcn_s_getreg(kHwRegXccId) & 15u;
            if (half == 0) {
                // written through to the device's coherence point (sc1, the
                // agent-scope store), each 64 lanes' chunks 1 KiB contiguous
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        v4f v;
#pragma unroll
                        for (int u = 0; u < 4; ++u) v[u] = wk == 0 ? facc[0][j][4 * q + u] : facc[1][j][4 * q + u];
                        asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(slot + (j * 4 + q) * 64), "v"(v)
                                     : "memory");
                    }
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // every partial store of this wave has completed
                __syncthreads();
                // the flag tells the partner where the sums were written from
                if (tid == 0)
                    __hip_atomic_store(flag, 1u + xcc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return;
            }
            __shared__ unsigned int ready;
            if (tid == 0) {
                unsigned spins = 0;
                unsigned v = 0;
                while ((v = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == 0 &&
                       ++spins < kSplitSpinLimit)
                    __builtin_amdgcn_s_sleep(1);
                ready = v;
                if (v) __hip_atomic_store(flag, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __syncthreads();
            const unsigned rv = ready;
            // All 4 TN chunks in flight at once.  From the partner's own XCD
            // the sums are in this L2 (a write-through store updates it):
            // loads that skip only the CU's cache (sc0); from another XCD,
            // loads at the coherence point (sc1, the agent-scope load).
            // (One statement issues the loads and waits for them, so that no
            // destination register is read or moved before its data landed.)
            v4f buf[8];
            const v4f* s0 = slot;
            const v4f* s1 = slot + 4 * 64;  // chunks 4..7: 4 KiB on (immediate offsets stop at 4095)
#define WQ_LOAD4(CP, O0, O1, O2, O3, B)                               \
    "global_load_dwordx4 %" #O0 ", %" #B ", off " CP "\n\t"           \
    "global_load_dwordx4 %" #O1 ", %" #B ", off offset:1024 " CP "\n\t" \
    "global_load_dwordx4 %" #O2 ", %" #B ", off offset:2048 " CP "\n\t" \
    "global_load_dwordx4 %" #O3 ", %" #B ", off offset:3072 " CP "\n\t"
            if constexpr (TN == 1) {
                if (rv == 1u + xcc)
                    asm volatile(WQ_LOAD4("sc0", 0, 1, 2, 3, 4) "s_waitcnt vmcnt(0)"
                                 : "=&v"(buf[0]), "=&v"(buf[1]), "=&v"(buf[2]), "=&v"(buf[3])
                                 : "v"(s0)
                                 : "memory");
                else
                    asm volatile(WQ_LOAD4("sc1", 0, 1, 2, 3, 4) "s_waitcnt vmcnt(0)"
                                 : "=&v"(buf[0]), "=&v"(buf[1]), "=&v"(buf[2]), "=&v"(buf[3])
                                 : "v"(s0)
                                 : "memory");
            } else {
                if (rv == 1u + xcc)
                    asm volatile(WQ_LOAD4("sc0", 0, 1, 2, 3, 8) WQ_LOAD4("sc0", 4, 5, 6, 7, 9) "s_waitcnt vmcnt(0)"
                                 : "=&v"(buf[0]), "=&v"(buf[1]), "=&v"(buf[2]), "=&v"(buf[3]), "=&v"(buf[4]),
                                   "=&v"(buf[5]), "=&v"(buf[6]), "=&v"(buf[7])
                                 : "v"(s0), "v"(s1)
                                 : "memory");
                else
                    asm volatile(WQ_LOAD4("sc1", 0, 1, 2, 3, 8) WQ_LOAD4("sc1", 4, 5, 6, 7, 9) "s_waitcnt vmcnt(0)"
                                 : "=&v"(buf[0]), "=&v"(buf[1]), "=&v"(buf[2]), "=&v"(buf[3]), "=&v"(buf[4]),
                                   "=&v"(buf[5]), "=&v"(buf[6]), "=&v"(buf[7])
                                 : "v"(s0), "v"(s1)
                                 : "memory");
            }
#undef WQ_LOAD4
            const bool timed_out = rv == 0;
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int r = 4 * q + u;
                        const float v = timed_out ? __builtin_nanf("") : buf[j * 4 + q][u];
                        if (wk == 0) facc[0][j][r] = v + facc[0][j][r];
                        else facc[1][j][r] = v + facc[1][j][r];
                    }
        }
    }

    // epilogue: per-token scale and output mode in registers, then each
    // 32 x 32 subtile goes through a per-wave LDS transpose so that every lane
    // stores 16 consecutive bytes of a row (8 lanes cover a 128-byte row
    // segment) instead of single words down a column
    __syncthreads();  // the ring and the exchange area are free again
    constexpr int JO = MODE == 2 ? TN / 2 : TN;
    float* tr = reinterpret_cast<float*>(lds) + (tid >> 6) * (32 * TR_STRIDE);
    const bool vec_ok = (reinterpret_cast<uintptr_t>(a.y) & 15) == 0 && (N & 3) == 0;  // 16-byte rows chunks
    float dtok[16];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        if (i < ilo || i >= ihi) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) dtok[r] = PT ? dx_tile[arow(i, r)] : 1.0f;
#pragma unroll
        for (int j = 0; j < JO; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float v = PT ? facc[i][j][r] * dtok[r] : facc[i][j][r];
                if (MODE == 2) v = silu_mul(v, PT ? facc[i][j + TN / 2][r] * dtok[r] : facc[i][j + TN / 2][r]);
                tr[(8 * (r >> 2) + 4 * h + (r & 3)) * TR_STRIDE + l32] = v;
            }
            __builtin_amdgcn_wave_barrier();  // LDS operations of a wave complete in order
            const int64_t c0 = n0 + bcol(j) - l32 + 4 * (lane & 7);  // first output column of this lane
            float4 o[4], yo4[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int row = 8 * q + (lane >> 3);
                o[q] = *reinterpret_cast<const float4*>(tr + row * TR_STRIDE + 4 * (lane & 7));
            }
            if (MODE == 1) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int64_t t = m0 + wm * 64 + 32 * i + 8 * q + (lane >> 3);
                    yo4[q] = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (t < M && vec_ok && c0 + 3 < N) yo4[q] = *reinterpret_cast<const float4*>(a.y + t * N + c0);
                }
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t t = m0 + wm * 64 + 32 * i + 8 * q + (lane >> 3);
                if (t >= M) continue;
                float* yp = a.y + t * N + c0;
                if (vec_ok && c0 + 3 < N) {
                    float4 v = o[q];
                    if (MODE == 1) {
                        v.x = yo4[q].x + v.x;
                        v.y = yo4[q].y + v.y;
                        v.z = yo4[q].z + v.z;
                        v.w = yo4[q].w + v.w;
                    }
                    // streamed: the output is not re-read here, and lines left
                    // dirty in L2 would be written back at the end of the kernel
                    __builtin_nontemporal_store(v4f{v.x, v.y, v.z, v.w}, reinterpret_cast<v4f*>(yp));
                } else {
                    const float vv[4] = {o[q].x, o[q].y, o[q].z, o[q].w};
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (c0 + u < N) yp[u] = MODE == 1 ? yp[u] + vv[u] : vv[u];
                }
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
}

template <int BN, int G, bool PT, bool DUMP>
hipError_t launch_mode(const GemmParams& gp, hipStream_t s) {
    dim3 grid((unsigned)(gp.tilesM * gp.tilesN * (gp.split ? 2 : 1))), block(gemm_threads(G, PT));
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

int64_t tiles_of(const LinearArgs& a, int bn) {
    const int64_t outw = a.mode == 2 ? bn / 2 : bn;
    return ((a.M + kBM - 1) / kBM) * ((a.N + outw - 1) / outw);
}

// Workspace of a split launch: one 64-byte flag line per tile, then (256-byte
// aligned) each tile's 128 x bn partial sums.
size_t split_flag_bytes(int64_t tiles) { return (((size_t)tiles * 64) + 255) / 256 * 256; }
size_t split_bytes(const LinearArgs& a, int bn) {
    const int64_t t = tiles_of(a, bn);
    return split_flag_bytes(t) + (size_t)t * kBM * bn * 4;
}

template <int BN, bool DUMP>
hipError_t launch_tile(const LinearArgs& a, hipStream_t s, bool split = false) {
    GemmParams gp{};
    gp.a = a;
    const bool pt = a.GA == a.K;
    const int ge = pt ? a.G : 32;
    const int outw = a.mode == 2 ? BN / 2 : BN;
    gp.tilesM = (int)((a.M + kBM - 1) / kBM);
    gp.tilesN = (int)((a.N + outw - 1) / outw);
    gp.NE = (int)(a.K / ge);
    gp.NG = (int)(a.K / a.G);
    if (split) {
        gp.split = 1;
        gp.flags = static_cast<unsigned int*>(a.workspace);
        gp.part = reinterpret_cast<float*>(static_cast<unsigned char*>(a.workspace) +
                                           split_flag_bytes((int64_t)gp.tilesM * gp.tilesN));
    }
    if (a.G == 128 && pt) return launch_mode<BN, 128, true, DUMP>(gp, s);
    if (a.G == 32 && pt) return launch_mode<BN, 32, true, DUMP>(gp, s);
    // the group-sum dump of the other formats runs widths up to 128 only
    // (launch_gemm); wider dump instances are not built
    if constexpr (DUMP && BN > 128) {
        return hipErrorInvalidConfiguration;
    } else {
        if (a.G == 128) return launch_mode<BN, 128, false, DUMP>(gp, s);
        return launch_mode<BN, 32, false, DUMP>(gp, s);
    }
}

// Tile width: the fewest (rounds of 256 workgroups, one per CU) x (cost of
// one tile), a tile's cost modelled as c0 + BN with c0 = 63 columns' worth of
// fixed work (prologue, epilogue).  The model is a fit of two measured
// launches at K = 2048, N = 6144: 256 workgroups of BN = 192 in 21.4 us and
// 192 of BN = 64 in 10.65 us.  Against the earlier rule (the widest width
// that still fills every CU, else the narrowest) it picks 128 at M = 512
// (19.3 -> 15.1 us) and 192 at M = 2048 (52.0 -> 43.1 us) and the same
// width elsewhere.  Mode 2 needs gate/up subtile pairs per wave: widths 256
// or 128.
//
// With K split across a workgroup pair (per-token formats, widths up to 128,
// K a multiple of 512 with 32 steps or more, a workspace), the same model
// extended by the K steps: a workgroup's time is c0 + steps x (ca + cb x BN)
// (c0 3.2 us of prologue and epilogue, ca 0.131 us per step of activation
// staging, cb 0.00525 us per step and column: a fit of the launches above and
// of K = 6144, N = 2048 at width 64, 25.6 us), a split workgroup running half
// the steps plus ~3 us for the exchange (measured: M = 512 and 256, K = 6144,
// N = 2048 at width 64 split: 18.3 and 17.3 us against 24.5 and 24.1 us
// unsplit; M = 1024 at width 128 split: 25.9 against 26.2 us at width 64).  It splits where the unsplit grid
// leaves CUs idle: M = 1024, K = 6144, N = 2048 (width 128 in 256 pairs of
// halves instead of 256 tiles of width 64), and the M = 256 / 512 prefills.
struct Plan {
    int bn;
    bool split;
};

Plan pick_plan(const LinearArgs& a, bool allow_split) {
    constexpr int64_t kCu = 256;
    constexpr double kC0 = 3.2, kCa = 0.131, kCb = 0.00525, kExchange = 3.0;
    const double steps = (double)(a.K / kBK);
    static const int widths[] = {256, 192, 128, 64};
    Plan best{64, false};
    double best_cost = -1.0;
    for (int bn : widths) {
        if (a.mode == 2 && bn != 256 && bn != 128) continue;
        const int64_t tiles = tiles_of(a, bn);
        for (int sp = 0; sp < (allow_split && bn <= 128 ? 2 : 1); ++sp) {
            const int64_t wgs = tiles * (sp ? 2 : 1);
            const double rounds = (double)((wgs + kCu - 1) / kCu);
            const double cost = rounds * (kC0 + (sp ? kExchange : 0.0) + steps / (sp ? 2 : 1) * (kCa + kCb * bn));
            if (best_cost < 0 || cost < best_cost) {
                best = Plan{bn, sp != 0};
                best_cost = cost;
            }
        }
    }
    return best;
}

// the shapes whose K the pair can split: per-token activations at group 128
// or 32 (the formats with two wave groups), an even number of steps per half
bool split_shape(const LinearArgs& a) {
    return a.GA == a.K && (a.G == 128 || a.G == 32) && a.K % 512 == 0 && a.K / kBK >= 32;
}

template <bool DUMP>
hipError_t launch_bn(const LinearArgs& a, hipStream_t s) {
    Plan pl{64, false};
    if (!DUMP && split_shape(a)) {
        pl = pick_plan(a, true);
        if (pl.split && !(a.workspace && a.workspace_bytes >= split_bytes(a, pl.bn))) pl = pick_plan(a, false);
    } else {
        pl = pick_plan(a, false);
    }
    switch (pl.bn) {
        case 256: return launch_tile<256, DUMP>(a, s);
        case 192: return launch_tile<192, DUMP>(a, s);
        case 128: return launch_tile<128, DUMP>(a, s, pl.split);
        default: return launch_tile<64, DUMP>(a, s, pl.split);
    }
}

}  // namespace

size_t gemm_workspace_bytes(const LinearArgs& a) {
    if (!split_shape(a)) return 0;
    const Plan pl = pick_plan(a, true);
    return pl.split ? split_bytes(a, pl.bn) : 0;
}

// The group-sum dump (a test hook) of the per-token group-128 format runs the
// tile width the production launch picks for the same shape, so the sums it
// stores are those of the kernel instance that serves the call.  The other
// formats dump from the narrow widths (64, or 128 for gate/up pairs): their
// wide dump instances exceed the register file.
hipError_t launch_gemm(const LinearArgs& a, hipStream_t s) {
    if (!a.acc_dump) return launch_bn<false>(a, s);
    if (a.GA == a.K) return launch_bn<true>(a, s);
    return a.mode == 2 ? launch_tile<128, true>(a, s) : launch_tile<64, true>(a, s);
}

}  // namespace wq
