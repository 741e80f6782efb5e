// Receiver CSR of an (E, 2) int64 edge list [sender, receiver] -- the index
// structure behind ConvTP's gather (indices_1) and scatter-sum (indices_out),
// src/molrep/interaction/tensor_product.py:101-111.  Counting sort by receiver
// (atomic slot claims), then each receiver's segment is sorted by edge id so
// the result is deterministic.  Edges whose sender or receiver lies outside
// [0, N) are left out and counted in *d_invalid.
//
// Edge lists that already come grouped by receiver in ascending order (the
// neighbor list's output, and the reference's NeighborList task before it
// appends the reversed edges) are detected on the device while counting: then
// the CSR is the identity permutation and the placement and segment sort are
// skipped, with no host synchronisation.

#include <mutex>

#include "common.h"
#include "scan.h"

namespace mnx {
namespace {

struct CsrWs {
    int32_t* counts;
    int32_t* fill;
    int32_t* tiles;
    int32_t* invalid;
    int32_t* unsorted;  // 0: all edges valid and grouped by receiver in ascending order
};

CsrWs carve_csr(void* base, size_t bytes, int64_t N, size_t* used) {
    Workspace ws{static_cast<char*>(base), bytes};
    CsrWs w;
    w.counts = ws.take<int32_t>(N + 1);
    w.fill = ws.take<int32_t>(N + 1);
    w.tiles = ws.take<int32_t>(scan_workspace_elems(N + 1));
    w.invalid = ws.take<int32_t>(2);  // [0] invalid count, [1] unsorted flag (cleared together)
    w.unsorted = w.invalid + 1;
    *used = ws.used;
    return w;
}

__device__ __forceinline__ bool edge_ok(const int64_t* ei, int64_t e, int64_t N) {
    const int64_t s = ei[2 * e], r = ei[2 * e + 1];
    return s >= 0 && s < N && r >= 0 && r < N;
}

__global__ void k_fill_i32(int32_t* __restrict__ p, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

// Per-receiver edge counts, aggregated per wavefront: each run of equal receivers among a
// wavefront's 64 consecutive edges adds its length with one atomic (receiver-grouped lists,
// the common case, put ~52 consecutive edges on one counter, which per-edge atomics
// serialise on), and the invalid-count / unsorted flags are set once per wavefront.
__global__ void k_count_recv(const int64_t* __restrict__ ei, int64_t E, int64_t N, int32_t* __restrict__ counts,
                             int32_t* __restrict__ invalid, int32_t* __restrict__ unsorted) {
    const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int lane = threadIdx.x & (kWave - 1);
    const bool in = e < E;
    const bool ok = in && edge_ok(ei, e, N);
    const int32_t key = ok ? int32_t(ei[2 * e + 1]) : -1;  // N < 2^31
    const bool desc = ok && e > 0 && ei[2 * e + 1] < ei[2 * e - 1];
    const uint64_t bad = __ballot(in && !ok), dsc = __ballot(desc), okm = __ballot(ok);
    if (lane == 0) {
        if (bad) atomicAdd(invalid, int32_t(__popcll(bad)));
        if (bad || dsc) atomicOr(unsorted, 1);
    }
    const int32_t prev = __shfl_up(key, 1);
    const bool head = ok && (lane == 0 || key != prev);
    const uint64_t stop = __ballot(head) | ~okm;  // a run ends before the next head or invalid lane
    if (head) {
        const uint64_t after = stop & ~((uint64_t(2) << lane) - 1);  // positions above this lane
        const int end = after ? __ffsll((unsigned long long)after) - 1 : kWave;
        atomicAdd(&counts[key], end - lane);
    }
}

__global__ void k_place_edges(const int64_t* __restrict__ ei, int64_t E, int64_t N, const int32_t* __restrict__ row_ptr,
                              int32_t* __restrict__ fill, int32_t* __restrict__ perm, int32_t* __restrict__ snd,
                              const int32_t* __restrict__ unsorted) {
    const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E) return;
    if (*unsorted == 0) {  // grouped by receiver, all valid: CSR slot e holds edge e
        perm[e] = int32_t(e);
        if (snd) snd[e] = int32_t(ei[2 * e]);
        return;
    }
    if (!edge_ok(ei, e, N)) return;
    const int64_t r = ei[2 * e + 1];
    perm[row_ptr[r] + atomicAdd(&fill[r], 1)] = int32_t(e);
}

__global__ void k_sort_segments(const int64_t* __restrict__ ei, int64_t N, const int32_t* __restrict__ row_ptr,
                                int32_t* __restrict__ perm, int32_t* __restrict__ snd,
                                const int32_t* __restrict__ unsorted) {
    const int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r >= N || *unsorted == 0) return;
    const int b = row_ptr[r], e = row_ptr[r + 1];
    for (int k = b + 1; k < e; ++k) {
        const int v = perm[k];
        int q = k - 1;
        while (q >= b && perm[q] > v) {
            perm[q + 1] = perm[q];
            --q;
        }
        perm[q + 1] = v;
    }
    if (snd)
        for (int k = b; k < e; ++k) snd[k] = int32_t(ei[2 * int64_t(perm[k])]);
}

__global__ void k_copy_invalid(const int32_t* __restrict__ src, int32_t* __restrict__ dst) { *dst = *src; }

// Allocation-free variant: the scratch (per-receiver counters, scan tiles,
// flags) lives in one file-scope device array instead of a caller workspace.
// Each device holds its own copy at its own address, found once per device
// with hipGetSymbolAddress; host code uses that address, never the array's
// name (which is only a host-side stand-in).  Every call on a device shares
// the array, so calls that overlap on one device race.
constexpr int64_t kNoallocMaxNodes = MNX_CSR_NOALLOC_MAX_NODES;
constexpr size_t kAlign = 256;
constexpr size_t align_up(size_t v) { return (v + kAlign - 1) & ~(kAlign - 1); }
// counts, fill (N + 1 each), scan tiles, the two flags; the same carve as carve_csr
constexpr size_t kNoallocScratchBytes =
    align_up(sizeof(int32_t) * (kNoallocMaxNodes + 1)) * 2 +
    align_up(sizeof(int32_t) * size_t((kNoallocMaxNodes + 1 + kScanTile - 1) / kScanTile)) + align_up(2 * sizeof(int32_t)) + kAlign;

static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int csr_scratch(void** out) {
    int dev = -1;
    MNX_HIP_TRY(hipGetDevice(&dev));
    MNX_REQUIRE(dev >= 0 && dev < kMaxDevices, "device ordinal %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        MNX_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        MNX_REQUIRE(p != nullptr, "hipGetSymbolAddress returned a null address");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return MNX_OK;
}

int csr_build(const int64_t* edge_index, int64_t E, int64_t N, int32_t* row_ptr, int32_t* perm,
              int32_t* senders_sorted, int32_t* d_invalid, void* workspace, size_t ws_bytes,
              hipStream_t stream) {
    MNX_REQUIRE(N >= 0 && N < (int64_t(1) << 31) && E >= 0 && E < (int64_t(1) << 31), "sizes out of range");
    MNX_REQUIRE(row_ptr && (E == 0 || (edge_index && perm)), "null pointer argument");
    size_t need = 0;
    CsrWs w = carve_csr(workspace, ws_bytes, N, &need);
    if (!workspace || ws_bytes < need) return set_error(MNX_ERR_WORKSPACE, "workspace %zu < %zu bytes", ws_bytes, need);
    const int tb = 256;
    // clear counters with fill kernels (no memset nodes if a caller captures this into a graph)
    for (int32_t* p : {w.counts, w.fill}) {
        hipLaunchKernelGGL(k_fill_i32, dim3(ceil_div(N + 1, tb)), dim3(tb), 0, stream, p, N + 1);
        MNX_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL(k_fill_i32, dim3(1), dim3(2), 0, stream, w.invalid, int64_t(2));  // invalid, unsorted
    MNX_CHECK_LAUNCH();
    if (E > 0) {
        hipLaunchKernelGGL(k_count_recv, dim3(ceil_div(E, tb)), dim3(tb), 0, stream, edge_index, E, N, w.counts,
                           w.invalid, w.unsorted);
        MNX_CHECK_LAUNCH();
    }
    // row_ptr[0..N] = exclusive scan of counts[0..N] (counts[N] == 0, so row_ptr[N] = valid edges)
    int rc = exclusive_scan<int32_t, int32_t>(w.counts, N + 1, row_ptr, w.tiles, (int32_t*)nullptr, stream);
    if (rc) return rc;
    if (E > 0 && N > 0) {
        hipLaunchKernelGGL(k_place_edges, dim3(ceil_div(E, tb)), dim3(tb), 0, stream, edge_index, E, N, row_ptr,
                           w.fill, perm, senders_sorted, w.unsorted);
        MNX_CHECK_LAUNCH();
        hipLaunchKernelGGL(k_sort_segments, dim3(ceil_div(N, tb)), dim3(tb), 0, stream, edge_index, N, row_ptr,
                           perm, senders_sorted, w.unsorted);
        MNX_CHECK_LAUNCH();
    }
    if (d_invalid) {
        hipLaunchKernelGGL(k_copy_invalid, dim3(1), dim3(1), 0, stream, w.invalid, d_invalid);
        MNX_CHECK_LAUNCH();
    }
    return MNX_OK;
}

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

size_t mnx_csr_workspace_bytes(int64_t N, int64_t E) {
    (void)E;
    size_t used = 0;
    carve_csr(nullptr, 0, N < 0 ? 0 : N, &used);
    return used + 256;
}

int mnx_csr_build(const int64_t* edge_index, int64_t E, int64_t N, int32_t* row_ptr, int32_t* perm,
                  int32_t* senders_sorted, int32_t* d_invalid, void* workspace, size_t ws_bytes,
                  mnx_stream_t stream) {
    clear_error();
    return csr_build(edge_index, E, N, row_ptr, perm, senders_sorted, d_invalid, workspace, ws_bytes,
                     (hipStream_t)stream);
}

int mnx_csr_build_noalloc(const int64_t* edge_index, int64_t E, int64_t N, int32_t* row_ptr, int32_t* perm,
                          int32_t* senders_sorted, int32_t* d_invalid, mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(N >= 0 && N <= kNoallocMaxNodes, "num_nodes %lld exceeds the allocation-free limit of %lld",
                (long long)N, (long long)kNoallocMaxNodes);
    void* base = nullptr;
    int rc = csr_scratch(&base);
    if (rc) return rc;
    return csr_build(edge_index, E, N, row_ptr, perm, senders_sorted, d_invalid, base, kNoallocScratchBytes,
                     (hipStream_t)stream);
}

}  // extern "C"
