// Device-wide exclusive prefix sum used by the cell list and the CSR builder.
// Three launches: per-tile sums, one-block scan of the tile sums, per-tile
// rescan with the tile's offset.  Deterministic (integer adds, fixed order).
#pragma once

#include "common.h"

namespace mnx {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanThreads * kScanItems;  // 2048 elements per tile
constexpr int kScanMaxTiles = 1024 * 16;              // top-level capacity

template <typename TOut>
__device__ inline TOut block_exclusive_scan(TOut v, TOut* sh, TOut* total) {
    // sh: kScanThreads entries of LDS
    const int t = threadIdx.x;
    sh[t] = v;
    __syncthreads();
    for (int off = 1; off < kScanThreads; off <<= 1) {
        TOut add = t >= off ? sh[t - off] : TOut(0);
        __syncthreads();
        sh[t] += add;
        __syncthreads();
    }
    TOut incl = sh[t];
    if (total) *total = sh[kScanThreads - 1];
    __syncthreads();
    return incl - v;
}

template <typename TIn, typename TOut>
__global__ void __launch_bounds__(kScanThreads) k_scan_tile_sums(const TIn* __restrict__ in, int64_t n,
                                                                  TOut* __restrict__ tile_sums) {
    __shared__ TOut sh[kScanThreads];
    const int64_t base = int64_t(blockIdx.x) * kScanTile + int64_t(threadIdx.x) * kScanItems;
    TOut s = 0;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k)
        if (base + k < n) s += TOut(in[base + k]);
    TOut tot;
    block_exclusive_scan<TOut>(s, sh, &tot);
    if (threadIdx.x == 0) tile_sums[blockIdx.x] = tot;
}

template <typename TOut>
__global__ void __launch_bounds__(1024) k_scan_top(TOut* __restrict__ tile_sums, int64_t ntiles,
                                                   TOut* __restrict__ grand_total) {
    __shared__ TOut sh[1024];
    constexpr int kPer = kScanMaxTiles / 1024;
    const int t = threadIdx.x;
    TOut loc[kPer];
    TOut s = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        int64_t idx = int64_t(t) * kPer + k;
        loc[k] = idx < ntiles ? tile_sums[idx] : TOut(0);
        s += loc[k];
    }
    sh[t] = s;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
        TOut add = t >= off ? sh[t - off] : TOut(0);
        __syncthreads();
        sh[t] += add;
        __syncthreads();
    }
    TOut run = sh[t] - s;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        int64_t idx = int64_t(t) * kPer + k;
        if (idx < ntiles) tile_sums[idx] = run;
        run += loc[k];
    }
    if (t == 1023 && grand_total) *grand_total = sh[1023];
}

template <typename TIn, typename TOut>
__global__ void __launch_bounds__(kScanThreads) k_scan_apply(const TIn* __restrict__ in, int64_t n,
                                                              const TOut* __restrict__ tile_offsets,
                                                              TOut* __restrict__ out) {
    __shared__ TOut sh[kScanThreads];
    const int64_t base = int64_t(blockIdx.x) * kScanTile + int64_t(threadIdx.x) * kScanItems;
    TOut vals[kScanItems];
    TOut s = 0;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        vals[k] = base + k < n ? TOut(in[base + k]) : TOut(0);
        s += vals[k];
    }
    TOut run = block_exclusive_scan<TOut>(s, sh, nullptr) + tile_offsets[blockIdx.x];
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        if (base + k < n) out[base + k] = run;
        run += vals[k];
    }
}

inline size_t scan_workspace_elems(int64_t n) { return size_t(ceil_div(n > 0 ? n : 1, kScanTile)); }

// out[k] = sum_{q<k} in[q] for k < n; *grand_total (device, may be null) = sum of all.
template <typename TIn, typename TOut>
int exclusive_scan(const TIn* in, int64_t n, TOut* out, TOut* tile_ws, TOut* grand_total,
                   hipStream_t stream) {
    const int64_t ntiles = ceil_div(n > 0 ? n : 1, kScanTile);
    if (ntiles > kScanMaxTiles) return set_error(MNX_ERR_INVALID, "scan length %lld too large", (long long)n);
    hipLaunchKernelGGL((k_scan_tile_sums<TIn, TOut>), dim3(ntiles), dim3(kScanThreads), 0, stream, in, n, tile_ws);
    MNX_CHECK_LAUNCH();
    hipLaunchKernelGGL((k_scan_top<TOut>), dim3(1), dim3(1024), 0, stream, tile_ws, ntiles, grand_total);
    MNX_CHECK_LAUNCH();
    hipLaunchKernelGGL((k_scan_apply<TIn, TOut>), dim3(ntiles), dim3(kScanThreads), 0, stream, in, n, tile_ws, out);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

}  // namespace mnx
