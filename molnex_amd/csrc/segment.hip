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
// atomics, a fixed summation order (bitwise reproducible).
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

}  // extern "C"
