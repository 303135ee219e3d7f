// Workgroup bitonic sort of 64-bit keys held in LDS.
//
// Element i lives in keys[i] and is handled by thread i % NT (slot i / NT), so the low six
// bits of i are the lane. Compare-exchange stages with stride < 64 pair lanes of one wave and
// run in registers through cross-lane shuffles; only strides >= 64 go through LDS with a
// workgroup barrier. For P = 1024 that is 15 barriers instead of the 55 of an all-LDS network.
#pragma once

#include "dt_common.h"

namespace tdt {

__device__ inline unsigned long long shfl_xor_u64(unsigned long long v, int m) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m, 64);
    return ((unsigned long long)hi << 32) | lo;
}

// One register stage: element i and its partner i ^ s (s < 64) of the bitonic merge of blocks
// of `size` (ascending where (i & size) == 0). The lower element keeps the minimum of an
// ascending pair, the upper the maximum; descending pairs swap roles.
__device__ inline unsigned long long bitonic_lane_stage(unsigned long long x, uint32_t i,
                                                        uint32_t size, uint32_t s) {
    const unsigned long long y = shfl_xor_u64(x, (int)s);
    const bool up = (i & size) == 0u;
    const bool lower = (i & s) == 0u;
    const unsigned long long mn = x < y ? x : y, mx = x < y ? y : x;
    return (lower == up) ? mn : mx;
}

// Sorts keys[0, P) ascending. P is a power of two >= 2; every thread of the workgroup (NT of
// them, a multiple of 64) must call it. Ends with a barrier.
template <uint32_t NT>
__device__ void block_sort_u64(unsigned long long* keys, uint32_t P) {
    const uint32_t tid = threadIdx.x;
    const uint32_t slots = (P + NT - 1u) / NT;
    // All merges of blocks up to 64 elements are wave-local. For P < 64 the lanes past P hold
    // a dummy: a partner i ^ s of a valid i (s < P, P a power of two) is valid too.
    const uint32_t small = P < 64u ? P : 64u;
    for (uint32_t k = 0; k < slots; ++k) {
        const uint32_t i = k * NT + tid;
        unsigned long long x = i < P ? keys[i] : ~0ull;
        for (uint32_t size = 2; size <= small; size <<= 1)
            for (uint32_t s = size >> 1; s > 0u; s >>= 1) x = bitonic_lane_stage(x, i, size, s);
        if (i < P) keys[i] = x;
    }
    __syncthreads();
    for (uint32_t size = 128; size <= P; size <<= 1) {
        for (uint32_t stride = size >> 1; stride >= 64u; stride >>= 1) {
            for (uint32_t i = tid; i < P / 2u; i += NT) {
                const uint32_t lo = 2u * i - (i & (stride - 1u));
                const uint32_t hi = lo + stride;
                const bool up = (lo & size) == 0u;
                const unsigned long long x = keys[lo], y = keys[hi];
                if ((x > y) == up) { keys[lo] = y; keys[hi] = x; }
            }
            __syncthreads();
        }
        for (uint32_t k = 0; k < slots; ++k) {
            const uint32_t i = k * NT + tid;
            unsigned long long x = i < P ? keys[i] : ~0ull;
            for (uint32_t s = 32; s > 0u; s >>= 1) x = bitonic_lane_stage(x, i, size, s);
            if (i < P) keys[i] = x;
        }
        __syncthreads();
    }
}

}  // namespace tdt
