// Segment sums over a CSR: the scatter primitives scatter_sum / batch_add
// (src/molix/F/scatter.py:13-51) and the neighbour sum of MessageAggregation
// (src/molrep/interaction/aggregation.py:93-117), which the reference runs as
// torch scatter_add_ (one atomic per element).
//
//   out[n][:] = sum_{k = row_ptr[n] .. row_ptr[n+1]-1} w[perm[k]] * values[perm[k]][:]
//
// One wavefront per (segment, block of columns): lanes own columns (four
// contiguous floats per lane when the row length allows 16-byte loads), the
// segment's rows are walked in CSR order (ascending row id within a segment)
// with four rows' loads in flight, and each output row is written once: no
// atomics, a fixed summation order (bitwise reproducible).  Few long segments
// (per-graph sums over large systems) take a workgroup each instead, whose
// threads split the rows and combine them by a fixed tree (k_segment_sum_wg).
//
// Backward: grad_values[r][:] = w[r] * grad_out[index[r]][:] (a gather) and
// grad_w[r] = <values[r], grad_out[index[r]]> (a dot product per row), one
// wavefront per row.

#include "common.h"

namespace mnx {
namespace {

constexpr int kSegThreads = 256;
constexpr int kWavesPerBlock = kSegThreads / kWave;

template <bool VEC>
__global__ void __launch_bounds__(kSegThreads) k_segment_sum(const float* __restrict__ values, int64_t dim,
                                                             const int32_t* __restrict__ row_ptr,
                                                             const int32_t* __restrict__ perm,
                                                             const float* __restrict__ w, int64_t num_segments,
                                                             int64_t col_blocks, float* __restrict__ out) {
    constexpr int kPer = VEC ? 4 : 1;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t item = int64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
    if (item >= num_segments * col_blocks) return;
    const int64_t seg = item / col_blocks;
    const int64_t col = (item % col_blocks) * (kWave * kPer) + int64_t(lane) * kPer;
    const bool active = col < dim;
    const int b = row_ptr[seg], e = row_ptr[seg + 1];
    float acc[kPer] = {};
    int k = b;
    for (; k + 4 <= e; k += 4) {
        int rows[4];
        float ws[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            rows[u] = __builtin_amdgcn_readfirstlane(perm[k + u]);
            ws[u] = w ? w[rows[u]] : 1.f;
        }
        float v[4][kPer];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (!active) {
#pragma unroll
                for (int q = 0; q < kPer; ++q) v[u][q] = 0.f;
            } else if (VEC) {
                const float4 t = *reinterpret_cast<const float4*>(values + int64_t(rows[u]) * dim + col);
                v[u][0] = t.x;
                v[u][kPer > 1 ? 1 : 0] = t.y;
                v[u][kPer > 2 ? 2 : 0] = t.z;
                v[u][kPer > 3 ? 3 : 0] = t.w;
            } else {
                v[u][0] = values[int64_t(rows[u]) * dim + col];
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int q = 0; q < kPer; ++q) acc[q] = fmaf(ws[u], v[u][q], acc[q]);
    }
    for (; k < e; ++k) {
        const int row = __builtin_amdgcn_readfirstlane(perm[k]);
        const float ws = w ? w[row] : 1.f;
        if (!active) continue;
        if (VEC) {
            const float4 t = *reinterpret_cast<const float4*>(values + int64_t(row) * dim + col);
            const float tv[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int q = 0; q < kPer; ++q) acc[q] = fmaf(ws, tv[q], acc[q]);
        } else {
            acc[0] = fmaf(ws, values[int64_t(row) * dim + col], acc[0]);
        }
    }
    if (!active) return;
    if (VEC) {
        *reinterpret_cast<float4*>(out + seg * dim + col) = make_float4(acc[0], acc[kPer > 1 ? 1 : 0],
                                                                        acc[kPer > 2 ? 2 : 0], acc[kPer > 3 ? 3 : 0]);
    } else {
        out[seg * dim + col] = acc[0];
    }
}

// Few long segments (per-graph sums of a batch of large systems): one workgroup of 1024 threads per
// (segment, block of DP columns).  Thread t owns column t % DP of the block and row slot t / DP; the
// slots walk the segment's rows strided by their count, each adding its rows in ascending CSR
// order (four loads in flight), and the slots are then combined by a fixed binary tree in LDS:
// no atomics, a fixed summation order.
constexpr int kWgThreads = 1024;

template <int DP>
__global__ void __launch_bounds__(kWgThreads) k_segment_sum_wg(const float* __restrict__ values, int64_t dim,
                                                               const int32_t* __restrict__ row_ptr,
                                                               const int32_t* __restrict__ perm,
                                                               const float* __restrict__ w, int64_t col_blocks,
                                                               float* __restrict__ out) {
    constexpr int kSlots = kWgThreads / DP;
    __shared__ float red[kWgThreads];
    const int64_t seg = blockIdx.x / col_blocks;
    const int64_t col = (blockIdx.x % col_blocks) * DP + threadIdx.x % DP;
    const int slot = threadIdx.x / DP;
    const bool active = col < dim;
    const int b = row_ptr[seg], e = row_ptr[seg + 1];
    float acc = 0.f;
    int k = b + slot;
    for (; k + 3 * kSlots < e; k += 4 * kSlots) {
        float v[4], ws[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int row = perm[k + u * kSlots];
            ws[u] = w ? w[row] : 1.f;
            v[u] = active ? values[int64_t(row) * dim + col] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) acc = fmaf(ws[u], v[u], acc);
    }
    for (; k < e; k += kSlots) {
        const int row = perm[k];
        acc = fmaf(w ? w[row] : 1.f, active ? values[int64_t(row) * dim + col] : 0.f, acc);
    }
    red[threadIdx.x] = acc;
    __syncthreads();
#pragma unroll
    for (int half = kSlots / 2; half > 0; half >>= 1) {
        if (slot < half) red[threadIdx.x] += red[threadIdx.x + half * DP];
        __syncthreads();
    }
    if (slot == 0 && active) out[seg * dim + col] = red[threadIdx.x];
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

__global__ void __launch_bounds__(kSegThreads) k_segment_sum_bwd(const float* __restrict__ g,
                                                                 const int64_t* __restrict__ index,
                                                                 const float* __restrict__ w,
                                                                 const float* __restrict__ values, int64_t rows,
                                                                 int64_t dim, int64_t num_segments,
                                                                 float* __restrict__ gv, float* __restrict__ gw) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t r = int64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int64_t n = index[r];
    const bool ok = n >= 0 && n < num_segments;
    const float wr = w ? w[r] : 1.f;
    float dot = 0.f;
    for (int64_t c = lane; c < dim; c += kWave) {
        const float gc = ok ? g[n * dim + c] : 0.f;
        if (gv) gv[r * dim + c] = wr * gc;
        if (gw) dot = fmaf(values[r * dim + c], gc, dot);
    }
    if (gw) {
        dot = wave_sum(dot);
        if (lane == 0) gw[r] = dot;
    }
}

// ---------------------------------------------------------------------------
// Class grouping: a stable counting sort of node ids by a small class id (the
// element of each node; classes outside [0, S) form class S), giving the node
// order and class boundaries that the element-indexed linear and the symmetric
// contraction's weight gradient walk.  One wavefront per segment of
// kGroupSeg consecutive nodes, 64 nodes per step in ascending order; within a
// step each distinct class present is handled by one ballot (rank = number of
// lower lanes of the same class), so the order within a class is ascending
// node id.  Three launches: per-segment class counts, an exclusive scan of
// the (class, segment) counts in class-major order, and the placement.  Every
// workspace entry is written before it is read: no clearing is needed.
// ---------------------------------------------------------------------------

constexpr int kGroupSeg = 1024;
constexpr int kGroupScanThreads = 1024;

__device__ __forceinline__ int node_class(const int64_t* __restrict__ cls, int64_t i, int S) {
    const int64_t c = cls[i];
    return c >= 0 && c < S ? int(c) : S;
}

// fn(class, lanes of that class in this step, rank of this lane among them) for each distinct class
// present among the active lanes of one 64-node step
template <typename Fn>
__device__ __forceinline__ void for_each_class(bool active, int c, Fn fn) {
    const int lane = threadIdx.x & (kWave - 1);
    const uint64_t below = (uint64_t(1) << lane) - 1;
    uint64_t todo = __ballot(active);  // wave-uniform: the loop and the barriers inside fn are uniform
    while (todo) {
        const int first = __ffsll((unsigned long long)todo) - 1;
        const int lc = __shfl(c, first);
        const bool mine = active && c == lc;
        const uint64_t mask = __ballot(mine);
        fn(lc, __popcll(mask), mine, __popcll(mask & below));
        todo &= ~mask;
    }
}

__global__ void __launch_bounds__(kWave) k_group_count(const int64_t* __restrict__ cls, int64_t n, int S,
                                                       int64_t nseg, int32_t* __restrict__ counts) {
    extern __shared__ int32_t cnt[];
    const int64_t seg = blockIdx.x;
    for (int s = threadIdx.x; s <= S; s += kWave) cnt[s] = 0;
    __syncthreads();
    const int64_t b = seg * kGroupSeg, e = min(b + kGroupSeg, n);
    for (int64_t i0 = b; i0 < e; i0 += kWave) {
        const int64_t i = i0 + threadIdx.x;
        const bool active = i < e;
        const int c = active ? node_class(cls, i, S) : 0;
        for_each_class(active, c, [&](int lc, int num, bool, int) {
            if (threadIdx.x == 0) cnt[lc] += num;
            __syncthreads();
        });
    }
    __syncthreads();
    for (int s = threadIdx.x; s <= S; s += kWave) counts[int64_t(s) * nseg + seg] = cnt[s];
}

// exclusive scan of counts[(S+1) * nseg] in place (one workgroup); class_start[s] = counts[s * nseg]
// after the scan, class_start[S + 1] = n
__global__ void __launch_bounds__(kGroupScanThreads) k_group_scan(int32_t* __restrict__ counts, int64_t len,
                                                                  int64_t nseg, int S, int64_t n,
                                                                  int32_t* __restrict__ class_start) {
    __shared__ int32_t part[kGroupScanThreads];
    const int t = threadIdx.x;
    const int64_t per = (len + kGroupScanThreads - 1) / kGroupScanThreads;
    const int64_t b = min(int64_t(t) * per, len), e = min(b + per, len);
    int32_t sum = 0;
    for (int64_t i = b; i < e; ++i) sum += counts[i];
    part[t] = sum;
    __syncthreads();
    for (int off = 1; off < kGroupScanThreads; off <<= 1) {  // Hillis-Steele inclusive scan of the partials
        const int32_t v = t >= off ? part[t - off] : 0;
        __syncthreads();
        part[t] += v;
        __syncthreads();
    }
    int32_t run = part[t] - sum;
    for (int64_t i = b; i < e; ++i) {
        const int32_t v = counts[i];
        counts[i] = run;
        run += v;
    }
    __syncthreads();
    if (nseg == 0) {
        for (int s = t; s <= S + 1; s += kGroupScanThreads) class_start[s] = 0;
        return;
    }
    for (int s = t; s <= S; s += kGroupScanThreads) class_start[s] = counts[int64_t(s) * nseg];
    if (t == 0) class_start[S + 1] = int32_t(n);
}

__global__ void __launch_bounds__(kWave) k_group_place(const int64_t* __restrict__ cls, int64_t n, int S,
                                                       int64_t nseg, const int32_t* __restrict__ offsets,
                                                       int32_t* __restrict__ order) {
    extern __shared__ int32_t base[];
    const int64_t seg = blockIdx.x;
    for (int s = threadIdx.x; s <= S; s += kWave) base[s] = offsets[int64_t(s) * nseg + seg];
    __syncthreads();
    const int64_t b = seg * kGroupSeg, e = min(b + kGroupSeg, n);
    for (int64_t i0 = b; i0 < e; i0 += kWave) {
        const int64_t i = i0 + threadIdx.x;
        const bool active = i < e;
        const int c = active ? node_class(cls, i, S) : 0;
        for_each_class(active, c, [&](int lc, int num, bool mine, int rank) {
            const int32_t at = base[lc];
            if (mine) order[at + rank] = int32_t(i);
            __syncthreads();
            if (threadIdx.x == 0) base[lc] = at + num;
            __syncthreads();
        });
    }
}

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

int mnx_segment_sum_f32(const float* values, int64_t num_rows, int32_t dim, const int32_t* row_ptr,
                        const int32_t* perm, const float* weights, int64_t num_segments, float* out,
                        mnx_stream_t stream_) {
    clear_error();
    hipStream_t stream = (hipStream_t)stream_;
    MNX_REQUIRE(num_rows >= 0 && num_segments >= 0 && dim >= 0, "sizes out of range");
    if (num_segments == 0 || dim == 0) return MNX_OK;
    MNX_REQUIRE(row_ptr && out && (num_rows == 0 || (values && perm)), "null pointer argument");
    // few segments averaging 64 rows or more (e.g. one graph of a large system): a workgroup per
    // segment and column block, since one wavefront per segment would leave the GPU nearly idle
    int dp = 1;
    while (dp < dim && dp < kWgThreads) dp *= 2;
    const int64_t wg_blocks = num_segments * ceil_div(int64_t(dim), int64_t(dp));
    if (wg_blocks <= 4096 && num_rows >= 64 * num_segments) {
        const int64_t cb = ceil_div(int64_t(dim), int64_t(dp));
        const dim3 g = dim3(unsigned(wg_blocks));
#define MNX_SEG_WG(D)                                                                                      \
    case D:                                                                                                \
        hipLaunchKernelGGL(k_segment_sum_wg<D>, g, dim3(kWgThreads), 0, stream, values, int64_t(dim), row_ptr, \
                           perm, weights, cb, out);                                                       \
        break;
        switch (dp) {
            MNX_SEG_WG(1) MNX_SEG_WG(2) MNX_SEG_WG(4) MNX_SEG_WG(8) MNX_SEG_WG(16) MNX_SEG_WG(32) MNX_SEG_WG(64)
            MNX_SEG_WG(128) MNX_SEG_WG(256) MNX_SEG_WG(512) MNX_SEG_WG(1024)
        }
#undef MNX_SEG_WG
        MNX_CHECK_LAUNCH();
        return MNX_OK;
    }
    const bool vec = dim % 4 == 0 && reinterpret_cast<uintptr_t>(values) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(out) % 16 == 0;
    const int64_t per_block = vec ? kWave * 4 : kWave;
    const int64_t col_blocks = ceil_div(dim, per_block);
    const int64_t items = num_segments * col_blocks;
    const dim3 grid(unsigned(ceil_div(items, kWavesPerBlock)));
    if (vec)
        hipLaunchKernelGGL(k_segment_sum<true>, grid, dim3(kSegThreads), 0, stream, values, int64_t(dim), row_ptr, perm,
                           weights, num_segments, col_blocks, out);
    else
        hipLaunchKernelGGL(k_segment_sum<false>, grid, dim3(kSegThreads), 0, stream, values, int64_t(dim), row_ptr,
                           perm, weights, num_segments, col_blocks, out);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_segment_sum_bwd_f32(const float* grad_out, const int64_t* index, const float* weights, const float* values,
                            int64_t num_rows, int32_t dim, int64_t num_segments, float* grad_values,
                            float* grad_weights, mnx_stream_t stream_) {
    clear_error();
    hipStream_t stream = (hipStream_t)stream_;
    MNX_REQUIRE(num_rows >= 0 && num_segments >= 0 && dim >= 0, "sizes out of range");
    if (num_rows == 0 || (!grad_values && !grad_weights)) return MNX_OK;
    MNX_REQUIRE(index && (grad_out || num_segments == 0), "null pointer argument");
    MNX_REQUIRE(!grad_weights || values, "grad_weights needs values");
    hipLaunchKernelGGL(k_segment_sum_bwd, dim3(unsigned(ceil_div(num_rows, kWavesPerBlock))), dim3(kSegThreads), 0,
                       stream, grad_out, index, weights, values, num_rows, int64_t(dim), num_segments, grad_values,
                       grad_weights);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

size_t mnx_class_groups_workspace_bytes(int64_t num_nodes, int32_t num_classes) {
    if (num_nodes < 0 || num_classes < 0) return 0;
    return size_t(ceil_div(num_nodes, int64_t(kGroupSeg))) * size_t(num_classes + 1) * sizeof(int32_t) + 256;
}

int mnx_class_groups(const int64_t* classes, int64_t num_nodes, int32_t num_classes, int32_t* order,
                     int32_t* class_start, void* workspace, size_t workspace_bytes, mnx_stream_t stream_) {
    clear_error();
    hipStream_t stream = (hipStream_t)stream_;
    MNX_REQUIRE(num_nodes >= 0 && num_nodes < (int64_t(1) << 31), "num_nodes out of range");
    MNX_REQUIRE(num_classes >= 0 && num_classes <= MNX_CLASS_GROUPS_MAX_CLASSES, "num_classes %d not in [0, %d]",
                num_classes, MNX_CLASS_GROUPS_MAX_CLASSES);
    MNX_REQUIRE(class_start && (num_nodes == 0 || (classes && order)), "null pointer argument");
    const size_t need = mnx_class_groups_workspace_bytes(num_nodes, num_classes);
    MNX_REQUIRE(workspace && workspace_bytes >= need, "workspace %zu < %zu bytes", workspace_bytes, need);
    const int64_t nseg = ceil_div(num_nodes, int64_t(kGroupSeg));
    const size_t lds = size_t(num_classes + 1) * sizeof(int32_t);
    int32_t* counts = static_cast<int32_t*>(workspace);
    if (nseg > 0) {
        hipLaunchKernelGGL(k_group_count, dim3(unsigned(nseg)), dim3(kWave), lds, stream, classes, num_nodes,
                           int(num_classes), nseg, counts);
        MNX_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL(k_group_scan, dim3(1), dim3(kGroupScanThreads), 0, stream, counts,
                       nseg * (num_classes + 1), nseg, int(num_classes), num_nodes, class_start);
    MNX_CHECK_LAUNCH();
    if (nseg > 0) {
        hipLaunchKernelGGL(k_group_place, dim3(unsigned(nseg)), dim3(kWave), lds, stream, classes, num_nodes,
                           int(num_classes), nseg, counts, order);
        MNX_CHECK_LAUNCH();
    }
    return MNX_OK;
}

}  // extern "C"
