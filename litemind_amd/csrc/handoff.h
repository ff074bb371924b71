// handoff.h -- values one workgroup hands to another inside a launch.
//
// Device-scope accesses (`sc1`): stores write through the XCD's L2 to memory
// and loads bypass it, so a value written by a workgroup on one XCD is seen by
// a workgroup on another within the same launch without an L2 writeback or
// invalidate.
#pragma once

#include "lm_internal.h"

namespace lm {

__device__ inline void store_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void store_coherent(int32_t* p, int32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float load_coherent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline int32_t load_coherent(const int32_t* p) {
    return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Tagged hand-off words: the value in the low 32 bits, the launch's sequence
// number in the high 32, written with one 64-bit device-scope store.  A reader
// knows a word is this launch's from the word itself, so the writer neither
// waits for its store nor counts it anywhere.
__device__ inline void publish(uint64_t* p, uint32_t seq, uint32_t bits) {
    __hip_atomic_store(p, (static_cast<uint64_t>(seq) << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One wave polls words [0, n) (n <= 64) until all carry `seq`; lane i < n then
// holds the low 32 bits of word i.  Bounded: after `limit` polls it sets
// *error and returns what it read.
__device__ inline uint32_t wait_tagged(const uint64_t* p, int n, uint32_t seq, uint32_t* error, uint32_t limit) {
    const int lane = threadIdx.x & 63;
    uint32_t spins = 0;
    for (;;) {
        const uint64_t v = lane < n ? __hip_atomic_load(const_cast<uint64_t*>(p) + lane, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT)
                                    : static_cast<uint64_t>(seq) << 32;
        if (__ballot(static_cast<uint32_t>(v >> 32) != seq) == 0) {
            return static_cast<uint32_t>(v);
        }
        if (++spins > limit) {
            if (lane == 0) {
                __hip_atomic_store(error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            return static_cast<uint32_t>(v);
        }
        __builtin_amdgcn_s_sleep(2);
    }
}

}  // namespace lm
