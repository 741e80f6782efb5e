// Wavefront-level helpers shared by the HIP sources (device code only).
#pragma once

#include "common.h"

namespace mnx {

// Sum of v over this lane's run of equal keys, from this lane to the run's end
// (the lanes of a run are contiguous; a run ends where the key changes).  After
// the call the first lane of every run holds that run's total; returns whether
// this lane is the first of its run.  All 64 lanes of the wavefront must take part.
template <typename T, int K>
__device__ __forceinline__ bool run_reduce(int key, T (&v)[K]) {
    const int lane = threadIdx.x & (kWave - 1);
    const int prev = __shfl_up(key, 1);
    const bool head = lane == 0 || prev != key;
    const unsigned long long heads = __ballot(head);
    const unsigned long long above = lane == kWave - 1 ? 0ull : heads & (~0ull << (lane + 1));
    const int end = above ? __builtin_ctzll(above) : kWave;
    for (int off = 1; off < kWave; off <<= 1) {
        const bool take = lane + off < end;
        for (int k = 0; k < K; ++k) {
            const T o = __shfl_down(v[k], off);
            if (take) v[k] += o;
        }
    }
    return head;
}

}  // namespace mnx
