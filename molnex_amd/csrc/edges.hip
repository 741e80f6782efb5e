// Bond vectors of an edge list and their gradient with respect to positions:
//   diff[e] = pos[receiver(e)] - pos[sender(e)] - shift[e]
// for edge_index rows [sender, receiver] -- the reference's convention
// bond_diff = pos[target] - pos[source] (src/molix/data/tasks/neighbor_list.py:86-95),
// through which forces are differentiated (src/molpot/derivation/force_derivation.py:28-45).
//
// Backward: grad_pos[a] = sum_{e: receiver a} g[e] - sum_{e: sender a} g[e].
// Edge lists from the neighbor list come grouped by receiver, so each
// wavefront first sums the receiver terms over its runs of equal receivers and
// adds one atomic per run; sender terms are added per edge.

#include "common.h"
#include "wave.h"

namespace mnx {
namespace {

constexpr int kEdgeThreads = 256;

__global__ void __launch_bounds__(kEdgeThreads) k_bond_fwd(const float* __restrict__ pos,
                                                           const int64_t* __restrict__ ei, const float* __restrict__ sh,
                                                           int64_t E, int64_t N, float* __restrict__ diff) {
    const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const int64_t s = ei[2 * e], r = ei[2 * e + 1];
    const bool ok = s >= 0 && s < N && r >= 0 && r < N;
    for (int k = 0; k < 3; ++k) {
        float v = ok ? pos[3 * r + k] - pos[3 * s + k] : __builtin_nanf("");
        if (sh) v -= sh[3 * e + k];
        diff[3 * e + k] = v;
    }
}

__global__ void __launch_bounds__(kEdgeThreads) k_bond_bwd(const int64_t* __restrict__ ei,
                                                           const float* __restrict__ g, int64_t E, int64_t N,
                                                           float* __restrict__ gpos) {
    const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    int recv = -1;
    float v[3] = {0.f, 0.f, 0.f};
    if (e < E) {
        const int64_t s = ei[2 * e], r = ei[2 * e + 1];
        if (s >= 0 && s < N && r >= 0 && r < N) {
            recv = int(r);
            for (int k = 0; k < 3; ++k) {
                v[k] = g[3 * e + k];
                atomicAdd(gpos + 3 * s + k, -v[k]);
            }
        }
    }
    if (run_reduce<float, 3>(recv, v) && recv >= 0)
        for (int k = 0; k < 3; ++k) atomicAdd(gpos + 3 * int64_t(recv) + k, v[k]);
}

__global__ void k_zero_f32(float* __restrict__ p, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.f;
}

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

int mnx_bond_vectors_f32(const float* pos, int64_t num_atoms, const int64_t* edge_index, const float* shifts,
                         int64_t num_edges, float* diff, mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(num_atoms >= 0 && num_edges >= 0 && num_atoms < (int64_t(1) << 31), "sizes out of range");
    if (num_edges == 0) return MNX_OK;
    MNX_REQUIRE(pos && edge_index && diff, "null pointer argument");
    hipLaunchKernelGGL(k_bond_fwd, dim3(ceil_div(num_edges, kEdgeThreads)), dim3(kEdgeThreads), 0,
                       (hipStream_t)stream, pos, edge_index, shifts, num_edges, num_atoms, diff);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_bond_vectors_bwd_f32(const int64_t* edge_index, const float* grad_diff, int64_t num_edges,
                             int64_t num_atoms, float* grad_pos, mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(num_atoms >= 0 && num_edges >= 0 && num_atoms < (int64_t(1) << 31), "sizes out of range");
    MNX_REQUIRE(grad_pos || num_atoms == 0, "null pointer argument");
    if (num_atoms > 0) {
        hipLaunchKernelGGL(k_zero_f32, dim3(ceil_div(3 * num_atoms, 256)), dim3(256), 0, (hipStream_t)stream,
                           grad_pos, 3 * num_atoms);
        MNX_CHECK_LAUNCH();
    }
    if (num_edges == 0) return MNX_OK;
    MNX_REQUIRE(edge_index && grad_diff, "null pointer argument");
    hipLaunchKernelGGL(k_bond_bwd, dim3(ceil_div(num_edges, kEdgeThreads)), dim3(kEdgeThreads), 0,
                       (hipStream_t)stream, edge_index, grad_diff, num_edges, num_atoms, grad_pos);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

}  // extern "C"
