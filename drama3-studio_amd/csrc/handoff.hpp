// Hand-off words of the single-launch decodes: the workspace head's two
// buffers of kHandoffWords 32-bit words (layout.hpp).  A call publishes its
// intermediate values into buffer (epoch & 1) with agent-scope stores, one
// word per value and never 0, so a reader takes a non-zero word as ready
// with no counter or fence; each call zero-fills the other buffer for the
// next one.  The epoch comes from the head's call counters.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "common.hpp"
#include "layout.hpp"

namespace dmoe {

typedef unsigned int v4u __attribute__((ext_vector_type(4)));
constexpr int kBufferWord3 = 0x00020000;  // raw buffer resource, gfx9 family
constexpr int kCpolSc1 = 16;              // the cache policy of an agent-scope atomic access

__device__ __forceinline__ __amdgpu_buffer_rsrc_t handoff_buffer(uint32_t* base) {
    return __builtin_amdgcn_make_buffer_rsrc(base, 0, kHandoffWords * 4, kBufferWord3);
}

// 16 bytes of hand-off words with the agent-scope load's cache policy (no
// stale copy from a non-coherent cache); each 4-byte word is read whole.
__device__ __forceinline__ v4i load_handoff16(__amdgpu_buffer_rsrc_t r, int byte_offset) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, byte_offset, 0, kCpolSc1));
}

// The call counter of workgroup B (slot B % kEpochSlots, 64-bit counters
// kEpochStride bytes apart): every workgroup of a call adds 1 to its slot,
// so with G workgroups per call (always the CU count) the workgroups of
// call c on a slot read c n .. c n + n - 1 and agree on epoch c + 1.
__device__ __forceinline__ uint64_t take_call_ticket(int* sync, int B) {
    return __hip_atomic_fetch_add((unsigned long long*)(sync + (B % kEpochSlots) * (kEpochStride / 4)), 1ull,
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t call_epoch(uint64_t ticket, int B, int G) {
    const int slot = B % kEpochSlots, n_slot = (G - slot + kEpochSlots - 1) / kEpochSlots;
    return (uint32_t)(ticket / (uint64_t)n_slot) + 1u;
}

// Workgroup B's share of the buffer the next call polls (all kHandoffWords
// words over the G workgroups, 16 bytes per thread and store).
__device__ __forceinline__ void clear_next_handoff(uint32_t* ht, uint32_t epoch, int B, int G, int tid, int nthreads) {
    const __amdgpu_buffer_rsrc_t next = handoff_buffer(ht + (int64_t)((epoch + 1) & 1) * kHandoffWords);
    const int share = (kHandoffWords / 4 + G - 1) / G * 4;  // words per workgroup, a multiple of 4
    for (int i = tid * 4; i < share; i += nthreads * 4) {
        const int word = B * share + i;
        if (word < kHandoffWords)
            __builtin_amdgcn_raw_buffer_store_b128(v4u{0u, 0u, 0u, 0u}, next, word * 4, 0, kCpolSc1);
    }
}

}  // namespace dmoe
