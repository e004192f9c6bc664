// Standalone greedy argmax (webyIQ crates/engine/src/shaders/argmax.wgsl:14-43)
// and the graph-capture-safe zero fill used for workspaces.
//
// One workgroup per row of logits.  Each (value, index) pair is turned into an
// order-preserving 64-bit key (value in the high word, complemented index in
// the low word), so the maximum key is the reference's winner: the largest
// value > -3e38, ties to the lowest index, NaN never selected.
#include "common.hpp"
#include "launch.hpp"

namespace wq {
namespace {

constexpr int kArgmaxThreads = 1024;

__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float* logits, int64_t V,
                                                                const uint32_t* ids,
                                                                uint32_t* tok_out) {
    const int64_t t = blockIdx.x;
    const float* row = logits + t * V;
    unsigned long long best = 0;
    for (int64_t i = threadIdx.x; i < V; i += kArgmaxThreads) {
        float v = row[i];
        if (v > -3.0e38f) {
            unsigned long long k = argmax_key(v, (uint32_t)i);
            best = k > best ? k : best;
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        unsigned long long other = __shfl_xor(best, o);
        best = other > best ? other : best;
    }
    __shared__ unsigned long long wbest[kArgmaxThreads / 64];
    if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kArgmaxThreads / 64; ++w) best = wbest[w] > best ? wbest[w] : best;
        best = wbest[0] > best ? wbest[0] : best;
        uint32_t idx = best ? 0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull) : 0u;
        tok_out[t] = ids ? ids[idx] : idx;
    }
}

__global__ void fill_zero_kernel(unsigned char* p, size_t bytes) {
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < bytes; i += stride) p[i] = 0;
}

}  // namespace

hipError_t launch_argmax(const float* logits, int64_t M, int64_t V, const uint32_t* ids,
                         uint32_t* tok_out, hipStream_t s) {
    hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)M), dim3(kArgmaxThreads), 0, s, logits, V, ids,
                       tok_out);
    return hipGetLastError();
}

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t s) {
    size_t blocks = (bytes + 255) / 256;
    if (blocks > 1024) blocks = 1024;
    if (blocks == 0) blocks = 1;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                       static_cast<unsigned char*>(p), bytes);
    return hipGetLastError();
}

}  // namespace wq
