// Channelwise tensor product fused with gather (senders) and scatter-sum
// (receivers), forward and backward, for gfx950.
//
// Replaces cuet.ChannelWiseTensorProduct as called by ConvTP
// (src/molrep/interaction/tensor_product.py:72-79,104-111): per-edge weights,
// ir_mul layout, indices_1 = senders, indices_out = receivers.
//
// Work decomposition: one wavefront per (receiver, channel block, path group);
// lanes are channels, the receiver's edges are walked in CSR order so the
// receiver's output row stays in registers and is written once (no atomics in
// the forward).  Per-edge data that is uniform across channels (harmonics,
// edge and sender ids) lives in scalar registers; the per-edge weights are
// streamed with non-temporal loads; sender rows are gathered (L2/MALL reuse).
// The backward keeps the receiver's output gradient folded with the coupling
// coefficients in registers and accumulates grad_x with fp32 atomics; grad_Y
// partial sums per (edge, group, channel block) are reduced by a second kernel.

#include "common.h"
#include "wave.h"

namespace mnx {
namespace {

// blockIdx -> receiver, so that each XCD (blocks are dealt round-robin over the
// 8 XCDs) walks one contiguous range of receivers and keeps its gathers in its L2.
__device__ __forceinline__ int64_t xcd_node(int64_t b, int64_t nblocks) {
    const int64_t per = nblocks >> 3;
    return (b & 7) * per + (b >> 3);
}

struct TPConfigInfo {
    int in_mask, sh_mask, out_mask, num_paths, nx, ny, no, ngroups;
};

typedef void (*TPFwdFn)(const float*, const float*, const float*, const int32_t*, const int32_t*, const int32_t*,
                        const int32_t*, int64_t, int, float*);
typedef void (*TPBwdFn)(const float*, const float*, const float*, const float*, const int32_t*, const int32_t*,
                        const int32_t*, const int32_t*, int64_t, int, float*, float*, float*, int, int);

#include "tp_gen.inc"

__global__ void k_reduce_partials(const float* __restrict__ part, int64_t E, int npart, int ny,
                                  float* __restrict__ gY) {
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= E * ny) return;
    const int64_t e = idx / ny;
    const int m = int(idx - e * ny);
    const float* p = part + e * npart * ny + m;
    float s = 0.f;
    for (int q = 0; q < npart; ++q) s += p[int64_t(q) * ny];
    gY[idx] = s;
}

__global__ void k_zero(float* __restrict__ p, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.f;
}

int check_common(int config, int channels, int64_t N, int64_t E) {
    MNX_REQUIRE(config >= 0 && config < kNumTPConfigs, "invalid tp config %d", config);
    MNX_REQUIRE(channels > 0 && channels <= 4096, "channels out of range: %d", channels);
    MNX_REQUIRE(N >= 0 && N < (int64_t(1) << 31) && E >= 0 && E < (int64_t(1) << 31), "sizes out of range");
    return MNX_OK;
}

dim3 node_grid(int64_t N, int cblocks) { return dim3(unsigned(8 * ceil_div(N > 0 ? N : 1, 8)), unsigned(cblocks)); }

// grad_Y partial rows per edge: one per (backward group, channel block)
int64_t bwd_partials(int config, int C) {
    int64_t np = 0;
    for (int g = 0; g < kTPConfigs[config].ngroups; ++g) np += ceil_div(C, 64 * kTPBwdCPL[config][g]);
    return np;
}

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

int mnx_tp_config(int32_t in_mask, int32_t sh_mask, int32_t out_mask) {
    for (int i = 0; i < kNumTPConfigs; ++i)
        if (kTPConfigs[i].in_mask == in_mask && kTPConfigs[i].sh_mask == sh_mask && kTPConfigs[i].out_mask == out_mask)
            return i;
    return -1;
}

int mnx_tp_config_info(int32_t config, int32_t* info) {
    clear_error();
    MNX_REQUIRE(config >= 0 && config < kNumTPConfigs && info, "invalid tp config %d", config);
    const TPConfigInfo& c = kTPConfigs[config];
    info[0] = c.num_paths;
    info[1] = c.nx;
    info[2] = c.ny;
    info[3] = c.no;
    return MNX_OK;
}

int mnx_tp_fwd_f32(int32_t config, int32_t C, const float* x, const float* Y, const float* w,
                   const int32_t* row_ptr, const int32_t* perm, const int32_t* snd, int64_t N, int64_t E,
                   float* out, mnx_stream_t stream) {
    return mnx_tp_fwd_rows_f32(config, C, x, Y, w, nullptr, row_ptr, perm, snd, N, E, out, stream);
}

int mnx_tp_fwd_rows_f32(int32_t config, int32_t C, const float* x, const float* Y, const float* w,
                        const int32_t* wrow, const int32_t* row_ptr, const int32_t* perm, const int32_t* snd,
                        int64_t N, int64_t E, float* out, mnx_stream_t stream) {
    clear_error();
    int rc = check_common(config, C, N, E);
    if (rc) return rc;
    if (N == 0) return MNX_OK;
    MNX_REQUIRE(out && row_ptr && (E == 0 || (x && Y && w && perm && snd)), "null pointer argument");
    const TPConfigInfo& cfg = kTPConfigs[config];
    const int cpl = C > 64 ? 2 : 1;
    const int cblocks = int(ceil_div(C, 64 * cpl));
    const dim3 grid = node_grid(N, cblocks);
    for (int g = 0; g < cfg.ngroups; ++g) {
        const bool full = C % (64 * cpl) == 0;
        TPFwdFn fn = cpl == 2 ? (full ? kTPFwdF2 : kTPFwd2)[config][g] : (full ? kTPFwdF1 : kTPFwd1)[config][g];
        hipLaunchKernelGGL(fn, grid, dim3(64), 0, (hipStream_t)stream, x, Y, w, row_ptr, perm, snd, wrow, N, C, out);
        MNX_CHECK_LAUNCH();
    }
    return MNX_OK;
}

size_t mnx_tp_bwd_workspace_bytes(int32_t config, int32_t C, int64_t E) {
    if (config < 0 || config >= kNumTPConfigs || C <= 0 || E < 0) return 0;
    const TPConfigInfo& cfg = kTPConfigs[config];
    return size_t(E > 0 ? E : 1) * size_t(bwd_partials(config, C)) * size_t(cfg.ny) * sizeof(float) + 256;
}

int mnx_tp_bwd_f32(int32_t config, int32_t C, const float* x, const float* Y, const float* w, const float* gout,
                   const int32_t* row_ptr, const int32_t* perm, const int32_t* snd, int64_t N, int64_t E,
                   float* gx, float* gY, float* gw, void* ws, size_t ws_bytes, mnx_stream_t stream) {
    return mnx_tp_bwd_rows_f32(config, C, x, Y, w, nullptr, gout, row_ptr, perm, snd, N, E, gx, gY, gw, ws,
                               ws_bytes, stream);
}

int mnx_tp_bwd_rows_f32(int32_t config, int32_t C, const float* x, const float* Y, const float* w,
                        const int32_t* wrow, const float* gout, const int32_t* row_ptr, const int32_t* perm,
                        const int32_t* snd, int64_t N, int64_t E, float* gx, float* gY, float* gw, void* ws,
                        size_t ws_bytes, mnx_stream_t stream) {
    clear_error();
    int rc = check_common(config, C, N, E);
    if (rc) return rc;
    if (N == 0 || E == 0) return MNX_OK;
    MNX_REQUIRE(x && Y && w && gout && row_ptr && perm && snd, "null pointer argument");
    const TPConfigInfo& cfg = kTPConfigs[config];
    const int npart = int(bwd_partials(config, C));
    float* part = nullptr;
    if (gY) {
        const size_t need = mnx_tp_bwd_workspace_bytes(config, C, E);
        if (!ws || ws_bytes < need) return set_error(MNX_ERR_WORKSPACE, "workspace %zu < %zu bytes", ws_bytes, need);
        // every (edge, partial) row is written by exactly one wavefront, since
        // every edge of the CSR belongs to one receiver (mnx_csr_build rejects
        // out-of-range indices), so the buffer needs no clearing.
        part = static_cast<float*>(ws);
    }
    int pbase = 0;
    for (int g = 0; g < cfg.ngroups; ++g) {
        const int cblocks = int(ceil_div(C, 64 * kTPBwdCPL[config][g]));
        const bool full = C % (64 * kTPBwdCPL[config][g]) == 0;
        hipLaunchKernelGGL((full ? kTPBwdF : kTPBwd)[config][g], node_grid(N, cblocks), dim3(64), 0,
                           (hipStream_t)stream, x, Y, w, gout,
                           row_ptr, perm, snd, wrow, N, C, gx, gw, part, npart, pbase);
        MNX_CHECK_LAUNCH();
        pbase += cblocks;
    }
    if (gY) {
        const int64_t tot = E * cfg.ny;
        hipLaunchKernelGGL(k_reduce_partials, dim3(unsigned(ceil_div(tot, 256))), dim3(256), 0, (hipStream_t)stream,
                           part, E, npart, cfg.ny, gY);
        MNX_CHECK_LAUNCH();
    }
    return MNX_OK;
}

int mnx_tp_group_paths(int32_t config, int32_t* bounds) {
    clear_error();
    MNX_REQUIRE(config >= 0 && config < kNumTPConfigs && bounds, "invalid tp config %d", config);
    const int ng = kTPConfigs[config].ngroups;
    for (int g = 0; g <= ng; ++g) bounds[g] = kTPGroupPaths[config][g];
    return ng;
}

int mnx_tp_bwd_group_rows_f32(int32_t config, int32_t C, int32_t group, const float* x, const float* Y,
                              const float* w, const int32_t* wrow, const float* gout, const int32_t* row_ptr,
                              const int32_t* perm, const int32_t* snd, int64_t N, int64_t E, float* gx, float* gw,
                              void* ws, size_t ws_bytes, mnx_stream_t stream) {
    clear_error();
    int rc = check_common(config, C, N, E);
    if (rc) return rc;
    const TPConfigInfo& cfg = kTPConfigs[config];
    MNX_REQUIRE(group >= 0 && group < cfg.ngroups, "group %d not in [0, %d)", group, cfg.ngroups);
    if (N == 0 || E == 0) return MNX_OK;
    MNX_REQUIRE(x && Y && w && gout && row_ptr && perm && snd, "null pointer argument");
    float* part = nullptr;
    if (ws) {
        const size_t need = mnx_tp_bwd_workspace_bytes(config, C, E);
        if (ws_bytes < need) return set_error(MNX_ERR_WORKSPACE, "workspace %zu < %zu bytes", ws_bytes, need);
        part = static_cast<float*>(ws);
    }
    int pbase = 0;
    for (int g = 0; g < group; ++g) pbase += int(ceil_div(C, 64 * kTPBwdCPL[config][g]));
    const int npart = int(bwd_partials(config, C));
    const int cblocks = int(ceil_div(C, 64 * kTPBwdCPL[config][group]));
    const bool full = C % (64 * kTPBwdCPL[config][group]) == 0;
    hipLaunchKernelGGL((full ? kTPBwdF : kTPBwd)[config][group], node_grid(N, cblocks), dim3(64), 0,
                       (hipStream_t)stream, x, Y, w, gout, row_ptr, perm, snd, wrow, N, C, gx, gw, part, npart, pbase);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_tp_bwd_reduce_gy_f32(int32_t config, int32_t C, int64_t E, const void* ws, size_t ws_bytes, float* gY,
                             mnx_stream_t stream) {
    clear_error();
    int rc = check_common(config, C, 0, E);
    if (rc) return rc;
    if (E == 0) return MNX_OK;
    MNX_REQUIRE(ws && gY, "null pointer argument");
    const size_t need = mnx_tp_bwd_workspace_bytes(config, C, E);
    if (ws_bytes < need) return set_error(MNX_ERR_WORKSPACE, "workspace %zu < %zu bytes", ws_bytes, need);
    const TPConfigInfo& cfg = kTPConfigs[config];
    const int64_t tot = E * cfg.ny;
    hipLaunchKernelGGL(k_reduce_partials, dim3(unsigned(ceil_div(tot, 256))), dim3(256), 0, (hipStream_t)stream,
                       static_cast<const float*>(ws), E, int(bwd_partials(config, C)), cfg.ny, gY);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_tp_bwd_sender_f32(int32_t config, int32_t C, const float* x, const float* Y, const float* w,
                          const float* gout, const int32_t* s_row_ptr, const int32_t* s_perm,
                          const int32_t* s_receivers, int64_t N, int64_t E, float* gx, float* gY, float* gw,
                          mnx_stream_t stream) {
    return mnx_tp_bwd_sender_rows_f32(config, C, x, Y, w, nullptr, gout, s_row_ptr, s_perm, s_receivers, N, E, gx,
                                      gY, gw, stream);
}

int mnx_tp_bwd_sender_rows_f32(int32_t config, int32_t C, const float* x, const float* Y, const float* w,
                               const int32_t* wrow, const float* gout, const int32_t* s_row_ptr,
                               const int32_t* s_perm, const int32_t* s_receivers, int64_t N, int64_t E, float* gx,
                               float* gY, float* gw, mnx_stream_t stream) {
    clear_error();
    int rc = check_common(config, C, N, E);
    if (rc) return rc;
    if (N == 0) return MNX_OK;
    MNX_REQUIRE(s_row_ptr && (E == 0 || (x && Y && w && gout && s_perm && s_receivers)), "null pointer argument");
    const TPConfigInfo& cfg = kTPConfigs[config];
    if (gY && E > 0) {  // accumulated in place by the subgroup kernels (a fill kernel: no memset node)
        const int64_t n = E * cfg.ny;
        hipLaunchKernelGGL(k_zero, dim3(unsigned(ceil_div(n, 256))), dim3(256), 0, (hipStream_t)stream, gY, n);
        MNX_CHECK_LAUNCH();
    }
    // every (sender, component, channel) of grad_x is stored by the first subgroup of its
    // input l (senders without edges store zeros) and accumulated by the later ones; each
    // edge lies in one sender segment of the CSR (mnx_csr_build rejects out-of-range indices)
    for (int g = 0; g < kTPBwSNum[config]; ++g) {
        const int cblocks = int(ceil_div(C, 64 * kTPBwSCPL[config][g]));
        hipLaunchKernelGGL(kTPBwS[config][g], node_grid(N, cblocks), dim3(64), 0, (hipStream_t)stream, x, Y, w,
                           gout, s_row_ptr, s_perm, s_receivers, wrow, N, C, gx, gw, E > 0 ? gY : nullptr, 0, 0);
        MNX_CHECK_LAUNCH();
    }
    return MNX_OK;
}

}  // extern "C"
