// int4 embedding lookup and packed-row gather (webyIQ
// crates/engine/src/shaders/embed.wgsl and gather_rows.wgsl; host side
// crates/engine/src/graph.rs:439-443 (embedding of the step's tokens) and
// graph.rs:511-516 (one-time gather of the reduced draft lm_head rows)).
//
// Both are pure HBM streams.  One thread owns one 16-byte chunk of a packed
// row (32 codes, one global_load_dwordx4): the lookup writes its 32
// dequantised values as 8 float4 stores, the gather copies the chunk.  Rows
// are flattened across the grid so that every launch covers all CUs.
#include "common.hpp"
#include "launch.hpp"

#pragma clang fp contract(off)

namespace wq {
namespace {

constexpr int kThreads = 256;

// x[m, k] = q * s + m for the row tok[m] of the packed matrix (the
// reference's f32(q) * s.x + s.y: a product, then a sum).  Token ids outside
// [0, V) produce a zero row.
template <int G>
__global__ __launch_bounds__(kThreads) void embed_kernel(EmbedArgs a) {
    pin_arg(a.q); pin_arg(a.s); pin_arg(a.ids); pin_arg(a.x); pin_arg(a.V); pin_arg(a.K); pin_arg(a.M);
    const int64_t chunks = a.K / 32;
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (idx >= a.M * chunks) return;
    const int64_t m = idx / chunks, c = idx - m * chunks;
    const uint32_t t = a.ids[m];
    float4* out = reinterpret_cast<float4*>(a.x + m * a.K + 32 * c);
    if ((int64_t)t >= a.V) {
#pragma unroll
        for (int i = 0; i < 8; ++i) out[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        return;
    }
    const uint4 w = load_stream16(reinterpret_cast<const unsigned char*>(a.q) + (int64_t)t * (a.K / 2) + 16 * c);
    const uint32_t* srow = a.s + (int64_t)t * (a.K / G);
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
        const int64_t k0 = 32 * c + 8 * wi;  // first code of this word
        const uint32_t sw = srow[k0 / G];
        const float s = f16lo(sw), mn = f16hi(sw);
        float v[8];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            v[b] = (float)((words[wi] >> (8 * b)) & 15u) * s + mn;
            v[4 + b] = (float)((words[wi] >> (8 * b + 4)) & 15u) * s + mn;
        }
        out[2 * wi] = make_float4(v[0], v[1], v[2], v[3]);
        out[2 * wi + 1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

// dst row r of (q, s) = src row ids[r]; ids outside [0, V) give zero rows.
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(GatherArgs a) {
    pin_arg(a.q); pin_arg(a.s); pin_arg(a.ids); pin_arg(a.dq); pin_arg(a.ds); pin_arg(a.V); pin_arg(a.K);
    pin_arg(a.G); pin_arg(a.R);
    const int64_t qchunks = a.K / 32;  // 16-byte chunks per packed row
    const int64_t swords = a.K / a.G;  // scale words per row
    const int64_t per_row = qchunks + swords;
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (idx >= a.R * per_row) return;
    const int64_t r = idx / per_row, c = idx - r * per_row;
    const uint32_t src = a.ids[r];
    const bool ok = (int64_t)src < a.V;
    if (c < qchunks) {
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (ok) v = load_stream16(reinterpret_cast<const unsigned char*>(a.q) + (int64_t)src * (a.K / 2) + 16 * c);
        *reinterpret_cast<uint4*>(reinterpret_cast<unsigned char*>(a.dq) + r * (a.K / 2) + 16 * c) = v;
    } else {
        const int64_t wdx = c - qchunks;
        a.ds[r * swords + wdx] = ok ? a.s[(int64_t)src * swords + wdx] : 0u;
    }
}

}  // namespace

hipError_t launch_embed(const EmbedArgs& a, hipStream_t s) {
    const int64_t n = a.M * (a.K / 32);
    dim3 grid((unsigned)((n + kThreads - 1) / kThreads)), block(kThreads);
    if (a.G == 128)
        hipLaunchKernelGGL(embed_kernel<128>, grid, block, 0, s, a);
    else
        hipLaunchKernelGGL(embed_kernel<32>, grid, block, 0, s, a);
    return hipGetLastError();
}

hipError_t launch_gather_rows(const GatherArgs& a, hipStream_t s) {
    const int64_t n = a.R * (a.K / 32 + a.K / a.G);
    dim3 grid((unsigned)((n + kThreads - 1) / kThreads)), block(kThreads);
    hipLaunchKernelGGL(gather_rows_kernel, grid, block, 0, s, a);
    return hipGetLastError();
}

}  // namespace wq
