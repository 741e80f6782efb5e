// Undirected pairs of a directed edge list.  The radial MLP's per-edge weights
// (src/molrep/interaction/radial_mlp.py:76-82, fed to ConvTP,
// src/molrep/interaction/tensor_product.py:72-79,101-111) depend on the edge
// only through its radial features, and an edge s -> r and its reverse r -> s
// have the same distance: a neighbor list emits bond vectors that are exact
// negations of each other, so their features agree bit for bit.  Pairing the
// two lets the MLP and its output run once per undirected pair.
//
// rev[e] = the one edge e2 != e with sender(e2) = receiver(e),
// receiver(e2) = sender(e) and feats[e2] equal to feats[e] bit for bit (F
// floats per edge); -1 when there is none or more than one (periodic images
// of one pair at equal distances), and then *d_bad counts the edge.  The
// candidates are the receiver-CSR segment of sender(e) (mnx_csr_build), one
// thread per edge.  When every segment lists its senders in ascending order
// (edge lists sorted by receiver and sender, as a neighbor list emits them;
// checked by a first pass) the thread binary-searches its segment for the run
// of sender receiver(e), else it scans the whole segment.

#include "common.h"
#include "scan.h"

namespace mnx {
namespace {

// unsorted[0] = 1 if some receiver segment of the CSR lists a larger sender before a smaller one
// (positions t, t + 1 of one segment: the same receiver).
__global__ void k_segments_unsorted(const int64_t* __restrict__ ei, int64_t E, const int32_t* __restrict__ perm,
                                    const int32_t* __restrict__ snd, int32_t* __restrict__ unsorted) {
    const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t + 1 >= E) return;
    if (snd[t] > snd[t + 1] && ei[2 * int64_t(perm[t]) + 1] == ei[2 * int64_t(perm[t + 1]) + 1]) unsorted[0] = 1;
}

__global__ void k_edge_reverse(const int64_t* __restrict__ ei, int64_t E, int64_t N,
                               const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ perm,
                               const int32_t* __restrict__ snd, const uint32_t* __restrict__ feats, int F,
                               const int32_t* __restrict__ unsorted, int32_t* __restrict__ rev,
                               int32_t* __restrict__ bad) {
    const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const int64_t s = ei[2 * e], r = ei[2 * e + 1];
    int found = -1, count = 0;
    if (s >= 0 && s < N && r >= 0 && r < N) {
        const uint32_t* fe = feats + e * F;
        int beg = row_ptr[s], end = row_ptr[s + 1];
        if (!unsorted[0]) {  // first position with sender >= r
            int lo = beg, hi = end;
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (snd[mid] < r) lo = mid + 1;
                else hi = mid;
            }
            beg = lo;
        }
        for (int t = beg; t < end; ++t) {
            if (snd[t] != r) {
                if (!unsorted[0] && snd[t] > r) break;
                continue;
            }
            const int e2 = perm[t];
            if (e2 == e) continue;
            const uint32_t* f2 = feats + int64_t(e2) * F;
            bool same = true;
            for (int k = 0; k < F; ++k) same = same && (f2[k] == fe[k]);
            if (same) {
                found = e2;
                ++count;
            }
        }
    }
    rev[e] = count == 1 ? found : -1;
    const uint64_t m = __ballot(count != 1);  // one atomic per wavefront
    if (m && int(threadIdx.x & 63) == __ffsll((unsigned long long)m) - 1) atomicAdd(bad, int(__popcll(m)));
}

// Numbering of the pairs once rev is known: flag[e] = 1 for the lead (lower id) of each pair, and
// bad[0] counts edges whose partner does not point back.
__global__ void k_pair_flags(const int32_t* __restrict__ rev, int64_t E, int32_t* __restrict__ flag,
                             int32_t* __restrict__ bad) {
    const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const int r = rev[e];
    const bool ok = r >= 0 && r < E && rev[r] == int32_t(e);
    flag[e] = ok && r > e ? 1 : 0;
    const uint64_t m = __ballot(!ok);
    if (m && int(threadIdx.x & 63) == __ffsll((unsigned long long)m) - 1) atomicAdd(bad, int(__popcll(m)));
}

// rank[e] = number of leads before e.  Pair rank[e] of lead e: lead[P] = e, pairs[P] = (e, rev[e]);
// every edge's weight row is its lead's rank.  Writes stay inside the E/2 pair slots whatever rev
// holds (bad[0] > 0 then tells the caller to discard them).
__global__ void k_pair_place(const int32_t* __restrict__ rev, const int32_t* __restrict__ flag,
                             const int32_t* __restrict__ rank, int64_t E, int32_t* __restrict__ wrow,
                             int64_t* __restrict__ lead, int32_t* __restrict__ pairs) {
    const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const int64_t half = E / 2;
    const int r = rev[e];
    if (flag[e]) {
        const int64_t P = rank[e];
        if (P < half) {
            lead[P] = e;
            pairs[2 * P] = int32_t(e);
            pairs[2 * P + 1] = r;
        }
    }
    const int64_t m = (r >= 0 && r < e) ? r : e;
    wrow[e] = rank[m] < half ? rank[m] : 0;
}

// bad[0] += number of pairs whose two edges' feature rows differ in any bit.
__global__ void k_pairs_verify(const int32_t* __restrict__ pairs, int64_t P, const uint32_t* __restrict__ feats,
                               int F, int32_t* __restrict__ bad) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= P) return;
    const uint32_t* a = feats + int64_t(pairs[2 * i]) * F;
    const uint32_t* b = feats + int64_t(pairs[2 * i + 1]) * F;
    bool same = true;
    for (int k = 0; k < F; ++k) same = same && a[k] == b[k];
    const uint64_t m = __ballot(!same);
    if (m && int(threadIdx.x & 63) == __ffsll((unsigned long long)m) - 1) atomicAdd(bad, int(__popcll(m)));
}

// dst[i][:] = src[idx[i]][:] (F floats per row), and its adjoint dst[idx[i]][:] = src[i][:]: one
// thread per element (the rows of radial features are 32 bytes, too short for row-wise loops).
__global__ void k_gather_rows(const float* __restrict__ src, const int64_t* __restrict__ idx, int64_t n, int F,
                              float* __restrict__ dst) {
    const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= n * F) return;
    const int64_t i = t / F;
    dst[t] = src[idx[i] * F + (t - i * F)];
}

__global__ void k_scatter_rows(const float* __restrict__ src, const int64_t* __restrict__ idx, int64_t n, int F,
                               float* __restrict__ dst) {
    const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= n * F) return;
    const int64_t i = t / F;
    dst[idx[i] * F + (t - i * F)] = src[t];
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// dst[i] = src[pairs[i][0]] + src[pairs[i][1]], one thread per 4 floats (F a multiple of 4).
__global__ void k_pair_sum_rows(const float* __restrict__ src, const int32_t* __restrict__ pairs, int64_t n, int F4,
                                float* __restrict__ dst) {
    const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= n * F4) return;
    const int64_t i = t / F4;
    const int f = int(t - i * F4);
    const f32x4 a = reinterpret_cast<const f32x4*>(src)[int64_t(pairs[2 * i]) * F4 + f];
    const f32x4 b = reinterpret_cast<const f32x4*>(src)[int64_t(pairs[2 * i + 1]) * F4 + f];
    reinterpret_cast<f32x4*>(dst)[t] = a + b;
}

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

int mnx_edge_reverse(const int64_t* edge_index, int64_t num_edges, int64_t num_nodes, const int32_t* row_ptr,
                     const int32_t* perm, const int32_t* senders_sorted, const float* feats, int32_t num_feats,
                     int32_t* rev, int32_t* d_bad, mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(num_edges >= 0 && num_edges < (int64_t(1) << 31) && num_nodes >= 0 &&
                    num_nodes < (int64_t(1) << 31), "sizes out of range");
    MNX_REQUIRE(num_feats >= 0 && num_feats <= 1024, "feature width %d out of range", num_feats);
    if (num_edges == 0) return MNX_OK;
    MNX_REQUIRE(edge_index && row_ptr && perm && senders_sorted && rev && d_bad && (feats || num_feats == 0),
                "null pointer argument");
    const dim3 grid(unsigned(ceil_div(num_edges, 256)));
    // d_bad[1] holds the segment-order flag (the caller clears both words)
    hipLaunchKernelGGL(k_segments_unsorted, grid, dim3(256), 0, (hipStream_t)stream, edge_index, num_edges, perm,
                       senders_sorted, d_bad + 1);
    MNX_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_edge_reverse, grid, dim3(256), 0, (hipStream_t)stream, edge_index, num_edges, num_nodes,
                       row_ptr, perm, senders_sorted, reinterpret_cast<const uint32_t*>(feats), num_feats,
                       d_bad + 1, rev, d_bad);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_gather_rows_f32(const float* src, const int64_t* idx, int64_t n, int32_t F, float* dst,
                        mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(n >= 0 && F >= 1 && F <= 4096, "sizes out of range");
    if (n == 0) return MNX_OK;
    MNX_REQUIRE(src && idx && dst, "null pointer argument");
    hipLaunchKernelGGL(k_gather_rows, dim3(unsigned(ceil_div(n * F, 256))), dim3(256), 0, (hipStream_t)stream, src, idx,
                       n, F, dst);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_scatter_rows_f32(const float* src, const int64_t* idx, int64_t n, int32_t F, float* dst,
                         mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(n >= 0 && F >= 1 && F <= 4096, "sizes out of range");
    if (n == 0) return MNX_OK;
    MNX_REQUIRE(src && idx && dst, "null pointer argument");
    hipLaunchKernelGGL(k_scatter_rows, dim3(unsigned(ceil_div(n * F, 256))), dim3(256), 0, (hipStream_t)stream, src,
                       idx, n, F, dst);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_edge_pairs_verify(const int32_t* pairs, int64_t num_pairs, const float* feats, int32_t num_feats,
                          int32_t* d_bad, mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(num_pairs >= 0 && num_feats >= 0 && num_feats <= 1024, "sizes out of range");
    if (num_pairs == 0) return MNX_OK;
    MNX_REQUIRE(pairs && d_bad && (feats || num_feats == 0), "null pointer argument");
    hipLaunchKernelGGL(k_pairs_verify, dim3(unsigned(ceil_div(num_pairs, 256))), dim3(256), 0, (hipStream_t)stream,
                       pairs, num_pairs, reinterpret_cast<const uint32_t*>(feats), num_feats, d_bad);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

size_t mnx_edge_pairs_workspace_bytes(int64_t num_edges) {
    if (num_edges < 0) return 0;
    const size_t e = size_t(num_edges > 0 ? num_edges : 1);
    return 3 * (e * sizeof(int32_t) + 256) + scan_workspace_elems(num_edges) * sizeof(int32_t) + 2 * 256;
}

int mnx_edge_pairs(const int64_t* edge_index, int64_t num_edges, int64_t num_nodes, const int32_t* row_ptr,
                   const int32_t* perm, const int32_t* senders_sorted, const float* feats, int32_t num_feats,
                   int32_t* wrow, int64_t* lead, int32_t* pairs, int32_t* d_bad, void* workspace,
                   size_t workspace_bytes, mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(num_edges >= 0 && num_edges % 2 == 0, "edge count %lld must be even", (long long)num_edges);
    if (num_edges == 0) return MNX_OK;
    MNX_REQUIRE(wrow && lead && pairs && d_bad && workspace, "null pointer argument");
    const size_t need = mnx_edge_pairs_workspace_bytes(num_edges);
    if (workspace_bytes < need)
        return set_error(MNX_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes, need);
    Workspace ws{static_cast<char*>(workspace), workspace_bytes};
    int32_t* rev = ws.take<int32_t>(size_t(num_edges));
    int32_t* flag = ws.take<int32_t>(size_t(num_edges));
    int32_t* rank = ws.take<int32_t>(size_t(num_edges));
    int32_t* tiles = ws.take<int32_t>(scan_workspace_elems(num_edges));
    int rc = mnx_edge_reverse(edge_index, num_edges, num_nodes, row_ptr, perm, senders_sorted, feats, num_feats, rev,
                              d_bad, stream);
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid(unsigned(ceil_div(num_edges, 256)));
    hipLaunchKernelGGL(k_pair_flags, grid, dim3(256), 0, s, rev, num_edges, flag, d_bad);
    MNX_CHECK_LAUNCH();
    rc = exclusive_scan<int32_t, int32_t>(flag, num_edges, rank, tiles, nullptr, s);
    if (rc) return rc;
    hipLaunchKernelGGL(k_pair_place, grid, dim3(256), 0, s, rev, flag, rank, num_edges, wrow, lead, pairs);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_pair_sum_rows_f32(const float* src, const int32_t* pairs, int64_t num_pairs, int32_t F, float* dst,
                          mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(num_pairs >= 0 && F >= 0 && F % 4 == 0, "pair sum: F must be a multiple of 4");
    if (num_pairs == 0 || F == 0) return MNX_OK;
    MNX_REQUIRE(src && pairs && dst && (uintptr_t)src % 16 == 0 && (uintptr_t)dst % 16 == 0,
                "pair sum: null or unaligned pointer");
    hipLaunchKernelGGL(k_pair_sum_rows, dim3(unsigned(ceil_div(num_pairs * (F / 4), 256))), dim3(256), 0,
                       (hipStream_t)stream, src, pairs, num_pairs, F / 4, dst);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

}  // extern "C"
