// Receiver CSR of an (E, 2) int64 edge list [sender, receiver] -- the index
// structure behind ConvTP's gather (indices_1) and scatter-sum (indices_out),
// src/molrep/interaction/tensor_product.py:101-111.  Counting sort by receiver
// (atomic slot claims), then each receiver's segment is sorted by edge id so
// the result is deterministic (a wavefront per segment: bitonic in registers up
// to 64 edges, merge passes beyond).  Edges whose sender or receiver lies outside
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
    int32_t* nlong;     // segments longer than one wavefront, listed for k_sort_long
};

CsrWs carve_csr(void* base, size_t bytes, int64_t N, size_t* used) {
    Workspace ws{static_cast<char*>(base), bytes};
    CsrWs w;
    w.counts = ws.take<int32_t>(N + 1);
    w.fill = ws.take<int32_t>(N + 1);
    w.tiles = ws.take<int32_t>(scan_workspace_elems(N + 1));
    w.invalid = ws.take<int32_t>(3);  // [0] invalid count, [1] unsorted flag, [2] long segments (cleared together)
    w.unsorted = w.invalid + 1;
    w.nlong = w.invalid + 2;
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

// Sorting each receiver's segment by edge id (the placement claims slots with atomics, in
// arbitrary order).  k_sort_short: one wavefront per receiver; segments of up to 64 edges are
// sorted in registers (bitonic network over the lanes) and written with their senders; longer
// ones are appended to a list (in the `fill` array, free after the placement) for k_sort_long:
// one wavefront per listed segment, grid-strided, which sorts runs of 64 in registers and merges
// them pairwise (each element's output position = its rank in its run + the number of smaller
// elements in the partner run, by binary search: edge ids are distinct) -- in LDS for segments
// of up to kSortLds edges, else in global memory with the senders array as the second buffer.
// O(n log^2 n) per segment instead of an insertion sort's O(n^2) on one thread.
constexpr int kSortLds = 4096;

__device__ __forceinline__ int bitonic64(int v, int lane) {
#pragma unroll
    for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const int other = __shfl_xor(v, stride, kWave);
            const bool up = (lane & size) == 0 || size == kWave;
            const bool low = (lane & stride) == 0;
            v = (low == up) ? min(v, other) : max(v, other);
        }
    }
    return v;
}

// number of entries of the sorted a[0..n) smaller than v
__device__ __forceinline__ int count_below(const int32_t* a, int n, int v) {
    int lo = 0, hi = n;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (a[mid] < v) lo = mid + 1; else hi = mid;
    }
    return lo;
}

// one merge pass over a segment of len entries: runs of `run` from src merged pairwise into dst
__device__ __forceinline__ void merge_pass(const int32_t* src, int32_t* dst, int len, int run, int lane) {
    for (int k = lane; k < len; k += kWave) {
        const int a0 = k / (2 * run) * (2 * run);
        const int a1 = min(a0 + run, len), b1 = min(a0 + 2 * run, len);
        const int v = src[k];
        const int pos = k < a1 ? (k - a0) + count_below(src + a1, b1 - a1, v)
                               : (k - a1) + count_below(src + a0, a1 - a0, v);
        dst[a0 + pos] = v;
    }
}

__global__ void __launch_bounds__(256) k_sort_short(const int64_t* __restrict__ ei, int64_t N,
                                                    const int32_t* __restrict__ row_ptr, int32_t* __restrict__ perm,
                                                    int32_t* __restrict__ snd, const int32_t* __restrict__ unsorted,
                                                    int32_t* __restrict__ long_list, int32_t* __restrict__ nlong) {
    const int64_t r = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & (kWave - 1);
    if (r >= N || *unsorted == 0) return;
    const int b = row_ptr[r], len = row_ptr[r + 1] - b;
    if (len > kWave) {
        if (lane == 0) long_list[atomicAdd(nlong, 1)] = int32_t(r);
        return;
    }
    if (len == 0) return;
    const int v = bitonic64(lane < len ? perm[b + lane] : INT32_MAX, lane);
    if (lane < len) {
        perm[b + lane] = v;
        if (snd) snd[b + lane] = int32_t(ei[2 * int64_t(v)]);
    }
}

__global__ void __launch_bounds__(kWave) k_sort_long(const int64_t* __restrict__ ei, const int32_t* __restrict__ row_ptr,
                                                     int32_t* __restrict__ perm, int32_t* __restrict__ snd,
                                                     const int32_t* __restrict__ long_list,
                                                     const int32_t* __restrict__ nlong) {
    __shared__ int32_t buf[2][kSortLds];
    const int lane = threadIdx.x;
    const int count = *nlong;
    for (int li = blockIdx.x; li < count; li += gridDim.x) {
        const int r = long_list[li];
        const int b = row_ptr[r], len = row_ptr[r + 1] - b;
        int32_t* seg = perm + b;
        // runs of 64 in registers
        for (int c0 = 0; c0 < len; c0 += kWave) {
            const int v = bitonic64(c0 + lane < len ? seg[c0 + lane] : INT32_MAX, lane);
            if (c0 + lane < len) {
                if (len <= kSortLds) buf[0][c0 + lane] = v; else seg[c0 + lane] = v;
            }
        }
        __syncthreads();
        if (len <= kSortLds) {
            int cur = 0;
            for (int run = kWave; run < len; run *= 2) {
                merge_pass(buf[cur], buf[cur ^ 1], len, run, lane);
                cur ^= 1;
                __syncthreads();
            }
            for (int k = lane; k < len; k += kWave) seg[k] = buf[cur][k];
        } else if (snd) {
            // merge passes in global memory, the senders array as the second buffer
            int32_t* src = seg;
            int32_t* dst = snd + b;
            for (int run = kWave; run < len; run *= 2) {
                merge_pass(src, dst, len, run, lane);
                int32_t* t = src;
                src = dst;
                dst = t;
                __syncthreads();
            }
            if (src != seg)
                for (int k = lane; k < len; k += kWave) seg[k] = src[k];
        } else if (lane == 0) {
            // no second buffer: one lane merges the runs by insertion (runs are sorted already)
            for (int k = kWave; k < len; ++k) {
                const int v = seg[k];
                int q = k - 1;
                while (q >= 0 && seg[q] > v) {
                    seg[q + 1] = seg[q];
                    --q;
                }
                seg[q + 1] = v;
            }
        }
        __syncthreads();
        if (snd)
            for (int k = lane; k < len; k += kWave) snd[b + k] = int32_t(ei[2 * int64_t(seg[k])]);
        __syncthreads();
    }
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
    align_up(sizeof(int32_t) * size_t((kNoallocMaxNodes + 1 + kScanTile - 1) / kScanTile)) + align_up(3 * sizeof(int32_t)) + kAlign;

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
    hipLaunchKernelGGL(k_fill_i32, dim3(1), dim3(3), 0, stream, w.invalid, int64_t(3));  // invalid, unsorted, nlong
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
        // the fill counters are done with after the placement: they hold the list of long segments
        hipLaunchKernelGGL(k_sort_short, dim3(ceil_div(N, 4)), dim3(256), 0, stream, edge_index, N, row_ptr, perm,
                           senders_sorted, w.unsorted, w.fill, w.nlong);
        MNX_CHECK_LAUNCH();
        hipLaunchKernelGGL(k_sort_long, dim3(unsigned(std::min<int64_t>(N, 2048))), dim3(kWave), 0, stream,
                           edge_index, row_ptr, perm, senders_sorted, w.fill, w.nlong);
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
