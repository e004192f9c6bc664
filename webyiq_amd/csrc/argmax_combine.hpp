// Cross-workgroup greedy argmax combine of the fused lm_head kernels
// (argmax.wgsl:19-43 semantics: the maximum key wins; a key holds the
// order-preserving value bits above the complemented index, so ties go to
// the lowest index; 0 means no value qualified).
#pragma once

#include "common.hpp"
#include "launch.hpp"

namespace wq {

// The workgroup's best key per token from its keys [MT][RB] in LDS, for
// thread t < min(MT, M) (0 elsewhere).  32 lanes per token each fold every
// 32nd key, then an xor-shuffle maximum over the 32 (the workgroup has at
// least 256 threads, so MT <= 8 tokens fit); the results meet in LDS.
template <int MT>
__device__ __forceinline__ unsigned long long block_best(const unsigned long long* keys, int RB, int M) {
    static_assert(MT * 32 <= 256, "32 lanes per token");
    __shared__ unsigned long long tok_best[MT];
    const int tid = threadIdx.x;
    const int t = tid >> 5, j = tid & 31;
    if (t < MT) {
        unsigned long long v = 0;
        for (int rl = j; rl < RB; rl += 32) v = keys[t * RB + rl] > v ? keys[t * RB + rl] : v;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) {
            const unsigned long long u = __shfl_xor(v, o, 32);
            v = u > v ? u : v;
        }
        if (j == 0) tok_best[t] = v;
    }
    __syncthreads();
    return tid < MT && tid < M ? tok_best[tid] : 0ull;
}

// Every workgroup calls this once with its best key for token tid in
// threads tid < M (0 elsewhere).  Keys and tickets live in kArgmaxSlots
// cache lines; the last workgroup of each slot takes a top ticket; the last
// of those reduces the slots, writes the token (mapped through ids when set)
// and clears the workspace for the next call.
//
// Ordering without release fences.  A release fence at agent scope writes
// back the whole L2 of the workgroup's XCD (the 8 XCDs' L2s are not coherent
// with one another); one per workgroup cost 225 us on the 151,936-row head.
// The combine instead orders its accesses by completion:
//  1. Every access to the workspace is an agent-scope atomic (atomicMax and
//     atomicAdd on device memory, and __hip_atomic_load/store with
//     __HIP_MEMORY_SCOPE_AGENT).  gfx950 performs these at the device's
//     coherence point, past the XCD-local L2, not in a per-XCD copy.
//  2. A returning atomic delivers its value only after it has been performed
//     there.  The keys' atomicMax results are consumed (the empty asm below)
//     before the barrier, so thread 0's ticket atomicAdd is issued only after
//     every key update of its workgroup has been performed.
//  3. The ticket counts are a total order on each counter.  The workgroup
//     that reads in_slot - 1 from its slot's counter issued its top-counter
//     atomicAdd after every other workgroup of the slot had performed its
//     ticket, hence (by 2) its keys; the same holds one level up for the
//     workgroup that reads used - 1 from the top counter.
//  4. That last workgroup then reads the keys with agent-scope atomic loads,
//     issued after its own top ticket returned, so each load is performed
//     after every key update, at the same coherence point.
// The HIP memory model guarantees visibility only through release/acquire
// pairs, so points 1, 2 and 4 rest on this hardware's completion order rather
// than on the language model.  The last workgroup adds an agent-scope
// acquire fence before its loads (one L2 invalidate on one XCD, not
// measurable at these sizes), so no stale line of its XCD's L2 can be read
// even if a key load were served from the L2.
template <int MT>
__device__ __forceinline__ void argmax_combine(const ArgmaxArgs& am, int M, int nblocks, unsigned long long best) {
    __shared__ unsigned int last_block;
    __shared__ unsigned long long slot_keys[kArgmaxSlots * MT];
    const int tid = threadIdx.x, nthreads = blockDim.x;
    const int kslot = (int)(blockIdx.x % kArgmaxSlots);
    if (tid < MT && tid < M) {
        const unsigned long long old = atomicMax(am.keys + kslot * kArgmaxSlotWords + tid, best);
        asm volatile("" ::"v"(old));  // the returned value: this atomic has been performed
    }
    __syncthreads();
    const int used = nblocks < kArgmaxSlots ? nblocks : kArgmaxSlots;
    if (tid == 0) {
        const unsigned in_slot = (unsigned)((nblocks - kslot + kArgmaxSlots - 1) / kArgmaxSlots);
        unsigned int done = atomicAdd(am.ticket + kslot * kArgmaxSlotWords * 2, 1u);
        bool last = false;
        if (done == in_slot - 1) {
            unsigned int top = atomicAdd(am.ticket + kArgmaxSlots * kArgmaxSlotWords * 2, 1u);
            last = top == (unsigned)used - 1;
        }
        last_block = last;
    }
    __syncthreads();
    if (last_block) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        // every slot key read at once (independent device-coherent loads),
        // then reduced in LDS
        for (int o = tid; o < used * MT; o += nthreads)
            slot_keys[o] = __hip_atomic_load(am.keys + (o / MT) * kArgmaxSlotWords + (o % MT), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (tid < M) {
            unsigned long long k = 0;
            for (int sl = 0; sl < used; ++sl) k = slot_keys[sl * MT + tid] > k ? slot_keys[sl * MT + tid] : k;
            uint32_t idx = k ? 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull) : 0u;
            am.tok_out[tid] = am.ids ? am.ids[idx] : idx;
        }
        __syncthreads();
        for (int o = tid; o < used * MT; o += nthreads)
            __hip_atomic_store(am.keys + (o / MT) * kArgmaxSlotWords + (o % MT), 0ull, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        for (int o = tid; o <= used; o += nthreads)
            __hip_atomic_store(am.ticket + (o < used ? o * kArgmaxSlotWords * 2 : kArgmaxSlots * kArgmaxSlotWords * 2),
                               0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace wq
