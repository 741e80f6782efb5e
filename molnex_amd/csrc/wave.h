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

// Cross-lane exchanges without LDS.  Stride 32 / 16: gfx950's permlane swaps
// exchange the upper half of `x` with the lower half of `z` (per 64- or
// 32-lane half), so x' + z' is, on every lane, the pair sum of the value that
// lane keeps (x on the lower lanes, z on the upper).  Stride 8 / 4 / 2 / 1: DPP
// row_mirror, row_half_mirror and quad_perm pair lane L with L^15, L^7, L^3,
// L^1, which flip bit 3, 2, 1, 0 of the lane id respectively.
__device__ __forceinline__ void pair_sum_swap32(float& x, float& z) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(z), false, false);
    x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ void pair_sum_swap16(float& x, float& z) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(z), false, false);
    x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int OFF>
__device__ __forceinline__ float dpp_partner(float v) {
    static_assert(OFF == 8 || OFF == 4 || OFF == 2 || OFF == 1, "row-local stride");
    return OFF == 8 ? dpp<0x140>(v) : OFF == 4 ? dpp<0x141>(v) : OFF == 2 ? dpp<0x1b>(v) : dpp<0xb1>(v);
}

template <int OFF, int CNT, int V>
__device__ __forceinline__ void rs_step(float (&a)[V], int lane) {
    if constexpr (CNT > 1) {
        constexpr int h = CNT / 2;
        if constexpr (OFF == 32 || OFF == 16) {
#pragma unroll
            for (int i = 0; i < h; ++i) {
                if constexpr (OFF == 32) pair_sum_swap32(a[i], a[h + i]);
                else pair_sum_swap16(a[i], a[h + i]);
            }
        } else {
            const bool hi = (lane & OFF) != 0;
#pragma unroll
            for (int i = 0; i < h; ++i) {
                const float keep = hi ? a[h + i] : a[i];
                const float send = hi ? a[i] : a[h + i];
                a[i] = keep + dpp_partner<OFF>(send);
            }
        }
        rs_step<OFF / 2, h, V>(a, lane);
    } else if constexpr (OFF >= 1) {
        if constexpr (OFF == 32 || OFF == 16) {
            float z = a[0];
            if constexpr (OFF == 32) pair_sum_swap32(a[0], z);
            else pair_sum_swap16(a[0], z);
        } else {
            a[0] += dpp_partner<OFF>(a[0]);
        }
        rs_step<OFF / 2, 1, V>(a, lane);
    }
}

// Sum V per-lane values over the 64 lanes; returns one of the V sums, which one
// given by reduce_scatter_index (lanes sharing an index hold the same sum).
template <int V>
__device__ __forceinline__ float wave_reduce_scatter(float (&a)[V], int lane) {
    rs_step<32, V, V>(a, lane);
    return a[0];
}

template <int V>
__device__ __forceinline__ int reduce_scatter_index(int lane) {
    int idx = 0, off = 32;
#pragma unroll
    for (int cnt = V; cnt > 1; cnt >>= 1) {
        if (lane & off) idx += cnt >> 1;
        off >>= 1;
    }
    return idx;
}

}  // namespace mnx
