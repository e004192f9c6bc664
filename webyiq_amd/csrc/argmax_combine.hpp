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

// Spin limit of the final workgroup's wait for the others' tickets (each poll
// is one device-coherent load plus a short sleep; the limit is ~0.5 s, far
// beyond any launch, so the wait ends even if a ticket never came).
constexpr unsigned kArgmaxSpinLimit = 1u << 22;

// Every workgroup calls this once, as its last action, with its best key for
// token tid in threads tid < M (0 elsewhere).  Keys live in kArgmaxSlots
// cache lines (workgroup b updates slot b % kArgmaxSlots) and so do the
// tickets.  Every workgroup but the last one (the highest index, dispatched
// last) merges its keys, takes a ticket in its slot and ends: its waves
// past the first leave at once, the first waits for one atomic.  The last
// workgroup merges its own keys, waits until every slot counts all of its
// other workgroups, then reduces the slots (one wave per token, a lane per
// slot), writes the token (mapped through ids when set) and clears the
// workspace for the next call.
//
// A variant without tickets (a key line per workgroup, published with one
// store and polled by the last workgroup until non-zero) was measured slower
// on the large heads (31.3 -> 37.3 us at 151,936 rows, one token; 40.4 ->
// 64.6 us at 8 tokens): the last workgroup's scans of every line, repeated
// while the stream still runs, load the device's coherence point.
//
// Ordering without release fences.  A release fence at agent scope writes
// back the whole L2 of the workgroup's XCD (the 8 XCDs' L2s are not coherent
// with one another); one per workgroup cost 225 us on the 151,936-row head.
// The combine instead orders its accesses by completion:
//  1. Every access to the workspace is an agent-scope atomic (atomicMax and
//     fetch-add on device memory, and __hip_atomic_load/store with
//     __HIP_MEMORY_SCOPE_AGENT).  gfx950 performs these at the device's
//     coherence point, past the XCD-local L2, not in a per-XCD copy.
//  2. A returning atomic delivers its value only after it has been performed
//     there.  A workgroup's key atomicMax results are consumed (the empty asm
//     below; the wave waits for all of its lanes) before its first lane
//     issues the ticket, so each ticket is performed after its workgroup's
//     key updates have been performed.
//  3. The last workgroup reads each slot's ticket count with agent-scope
//     loads until it equals the number of other workgroups of that slot:
//     every ticket, hence (by 2) every key update, has then been performed.
//  4. It then reads the keys with agent-scope atomic loads issued after
//     those polls returned, so each load is performed after every key update,
//     at the same coherence point.
// The HIP memory model guarantees visibility only through release/acquire
// pairs, so points 1, 2 and 4 rest on this hardware's completion order rather
// than on the language model.  No acquire fence precedes the key loads: they
// are agent-scope atomic loads (`global_load ... sc1`, performed at the
// coherence point, never served from a stale line of the XCD's L2) of words
// that only agent-scope atomics write, which is what the gfx950 memory model
// makes coherent without a fence; a fence would only add one L2 invalidate
// (0.3-0.4 us per call, measured) for the non-atomic loads that follow none.
//
// Cost: the combine adds 2.5-4 us per call on the lm_head shapes, almost all
// of it after the last stream ends (the last tickets landing, the final
// workgroup's loads and stores: device-coherent round trips of ~0.3 us idle,
// longer while the stream drains).
//
// Progress: the last workgroup waits only for workgroups of lower index.
// Workgroups are dispatched in index order, so each of those has been
// dispatched to some CU when the last one runs; none waits for anything, so
// each finishes.  The wait is bounded all the same (kArgmaxSpinLimit); if it
// ran out, the tokens are written as 0xFFFFFFFF (no index has that value:
// V <= 0xFFFFFFFE), and keys and tickets landing after the clear leave the
// workspace non-zero.  The host then clears it before the next call
// (wq_workspace_clear, or wq_lm_head_noalloc_reset for the library's own
// array): once the launch has completed, every late key and ticket has
// landed, so a stream-ordered clear leaves it zero.
template <int MT>
__device__ __forceinline__ void argmax_combine(const ArgmaxArgs& am, int M, int nblocks, unsigned long long best) {
    const int tid = threadIdx.x, nthreads = blockDim.x;
    const int kslot = (int)(blockIdx.x % kArgmaxSlots);
    const bool final_block = (int)blockIdx.x == nblocks - 1;
    if (!final_block && tid >= 64) return;  // only the first wave takes part
    if (tid < MT && tid < M) {
        const unsigned long long old = atomicMax(am.keys + kslot * kArgmaxSlotWords + tid, best);
        // The ordering point of step 2: the returned value is consumed here
        // (the compiler waits for the atomic's return before this statement),
        // and the "memory" clobber keeps the ticket below, an access to
        // another address, from being moved above it.
        asm volatile("" ::"v"(old) : "memory");
    }
    if (!final_block) {
        if (tid == 0)
            __hip_atomic_fetch_add(am.ticket + kslot * kArgmaxSlotWords * 2, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        return;
    }

    __shared__ unsigned int timed_out;
    const int used = nblocks < kArgmaxSlots ? nblocks : kArgmaxSlots;
    if (tid < 64) {
        // lane l polls slot l: it expects the other workgroups of that slot
        const int sl = tid;
        unsigned want = 0;
        if (sl < used) {
            want = (unsigned)((nblocks - sl + kArgmaxSlots - 1) / kArgmaxSlots);
            if (sl == kslot) want -= 1;  // this workgroup takes no ticket
        }
        unsigned spins = 0;
        bool done = false;
        while (true) {
            const unsigned have = sl < used ? __hip_atomic_load(am.ticket + sl * kArgmaxSlotWords * 2,
                                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                            : 0u;
            done = __all(have >= want);
            if (done || ++spins >= kArgmaxSpinLimit) break;
            __builtin_amdgcn_s_sleep(1);
        }
        if (tid == 0) timed_out = done ? 0u : 1u;
    }
    __syncthreads();
    // Wave w reduces tokens w, w + nwaves, ...: lane l reads slot l's key
    // (independent device-coherent loads), a 64-lane maximum (exact,
    // order-free), and each lane then clears the key it read.
    const int wave = tid >> 6, lane = tid & 63, nwaves = nthreads >> 6;
    for (int t = wave; t < M && t < MT; t += nwaves) {
        unsigned long long* kp = am.keys + lane * kArgmaxSlotWords + t;
        unsigned long long k = lane < used ? __hip_atomic_load(kp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const unsigned long long u = __shfl_xor(k, o, 64);
            k = u > k ? u : k;
        }
        if (lane == 0) {
            const uint32_t idx = k ? 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull) : 0u;
            am.tok_out[t] = timed_out ? 0xFFFFFFFFu : am.ids ? am.ids[idx] : idx;
        }
        if (lane < used) __hip_atomic_store(kp, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (tid < used)
        __hip_atomic_store(am.ticket + tid * kArgmaxSlotWords * 2, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace wq
