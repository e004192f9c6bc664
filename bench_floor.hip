// Per-launch floors for the decode GEMV's launch shape (bench.py --floor):
// kernels on the GEMV's grid for M = 1, K = 2048, N = 6144 (768 workgroups
// of 4 waves, 2 rows per wave) that do none of its arithmetic.
//   empty      -- no loads, no stores: the launch and drain cost alone;
//   read       -- every weight row (1 KiB, one 16-byte streamed load per
//                 lane) and its scale words (each lane its group's word),
//                 all issued before the first is used, folded by XOR per
//                 lane, no store (a store guarded by the folded value keeps
//                 the loads live);
//   read_store -- the same loads, and one 4-byte result per row (y);
//   kind 3     -- the empty kernel on a given number of workgroups (the
//                 dispatch cost against grid size).
// They bound from below what any kernel that streams the same bytes in
// one launch can reach; bench.py times them as the GEMV is timed (graph
// replays rotating over the weight copies).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kIpw = 2;      // rows per wave
constexpr int kSlots = 4;    // waves per workgroup
constexpr int kRowU4 = 64;   // 16-byte chunks per 1 KiB row
constexpr int kRowWs = 16;   // scale words per row (K / 128)

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void floor_empty(int* out, int n) {
    if (threadIdx.x == 0 && (int)blockIdx.x == n) out[0] = 1;  // never true: n = grid size
}

template <bool STORE_ROWS>
__global__ __launch_bounds__(256) void floor_read(const v4u* __restrict__ w, const uint32_t* __restrict__ ws,
                                                  uint32_t* __restrict__ out, int n) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r0 = blockIdx.x * kSlots * kIpw;
    v4u v[kIpw];
    uint32_t s[kIpw];
#pragma unroll
    for (int i = 0; i < kIpw; ++i) {
        int row = r0 + wave + kSlots * i;
        row = row < n ? row : n - 1;
        v[i] = __builtin_nontemporal_load(w + (size_t)row * kRowU4 + lane);
        s[i] = ws[(size_t)row * kRowWs + (lane >> 2)];
    }
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < kIpw; ++i) {
        const uint32_t r = v[i].x ^ v[i].y ^ v[i].z ^ v[i].w ^ s[i];
        if (STORE_ROWS) {
            // one word per row, lane 0's fold (no cross-lane work)
            const int row = r0 + wave + kSlots * i;
            if (lane == 0 && row < n) out[row] = r;
        } else {
            acc ^= r;
        }
    }
    // no store in practice: one only where a lane's fold equals the row
    // count (keeps the loads live; out holds n words, grid < n)
    if (!STORE_ROWS && acc == (uint32_t)n) out[blockIdx.x] = acc;
}

int grid_of(int n) { return (n + kSlots * kIpw - 1) / (kSlots * kIpw); }

}  // namespace

// out: at least n words.  n: weight rows (K = 2048).  Returns a hipError_t.
extern "C" int floor_launch(void* stream, int kind, const void* w, const void* ws, void* out, int n) {
    hipStream_t s = (hipStream_t)stream;
    const int grid = grid_of(n);
    if (kind == 0)
        hipLaunchKernelGGL(floor_empty, dim3(grid), dim3(256), 0, s, (int*)out, grid);
    else if (kind == 3)  // the empty kernel on n workgroups of 256 threads (dispatch cost against grid size)
        hipLaunchKernelGGL(floor_empty, dim3(n), dim3(256), 0, s, (int*)out, n);
    else if (kind == 1)
        hipLaunchKernelGGL(floor_read<false>, dim3(grid), dim3(256), 0, s, (const v4u*)w, (const uint32_t*)ws,
                           (uint32_t*)out, n);
    else
        hipLaunchKernelGGL(floor_read<true>, dim3(grid), dim3(256), 0, s, (const v4u*)w, (const uint32_t*)ws,
                           (uint32_t*)out, n);
    return (int)hipGetLastError();
}
