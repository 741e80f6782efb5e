// Per-edge channelwise tensor product with shared weights (Allegro's layer
// product, src/molzoo/allegro.py:352-359,457-458): out[e] = TP(s[e] x[e], Y[e]; w),
// no scatter, with an optional per-edge, per-channel scale s of x (the env
// weights of allegro.py:447-450).  The kernels are generated per configuration by gen_edge_tp.py
// (edge_tp_gen.inc); configuration ids are those of mnx_tp_config.  Lanes hold
// (edge, channel) pairs, 64 / min(C, 64) edges per wavefront.
//
// HBM traffic per edge: forward 4 (NX + NO) C + 4 NY bytes; backward
// 4 (2 NX + NO) C + 8 NY bytes (plus one weight-gradient partial per
// wavefront).
//
// mnx_edge_tp_proj_*: the product fused with the projection that follows it in each Allegro layer
// (allegro.py:363-367, cuet.Linear(tp.irreps_out, irreps_in)) for 16 channels.  The product's NO
// rows never reach HBM.  Forward: a wavefront takes 16 edges at a time (lane = edge mod 16 and a
// quarter of the channels), each path's components are the A operands of fp32 16x16x4
// matrix-core products with the projection weights (staged once per workgroup in LDS, in operand
// order), and only the projected irreps (l = 0..l_max, 16 channels each) are written.  Backward:
// one edge per 16-lane row, channel c in lane c; the incoming gradient is taken back through the
// projection by rotating it through the row (DPP) against LDS-staged weights, then the product's
// backward.  Per edge: forward 4 (NX + NI) 16 + 4 NY bytes, backward 4 (2 NX + NI) 16 + 8 NY
// (NI = projected components).

#include "common.h"

namespace mnx {
namespace {

struct ETPInfo {
    int ok, np, nx, ny, no;
    int fwd_groups;  // edge groups per forward wavefront
};

typedef void (*ETPFwdFn)(const float*, const float*, const float*, const float*, int64_t, int, float*);
typedef void (*ETPBwdFn)(const float*, const float*, const float*, const float*, const float*, int64_t, int, float*,
                         float*, float*, float*);
// fused product + projection, 16 channels: (x, Y, w, xs, xs2, wp, E, out) and
// (grad_proj, x, Y, w, xs, xs2, wp, E, gx, gY, gw_part, gxs, gxs2)
typedef void (*ETPFwdPFn)(const float*, const float*, const float*, const float*, const float*, const float*,
                          int64_t, float*);
typedef void (*ETPBwdPFn)(const float*, const float*, const float*, const float*, const float*, const float*,
                          const float*, int64_t, float*, float*, float*, float*, float*);

typedef float f4 __attribute__((ext_vector_type(4)));  // one matrix-core accumulator / operand quad

// Lane i of each 16-lane row receives the value of lane (i - K) mod 16 of the same row
// (DPP row_ror:K; one edge per row in the fused kernels).
template <int K>
__device__ __forceinline__ float ror16(float v) {
    if constexpr (K == 0) {
        return v;
    } else {
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x120 + K, 0xF, 0xF, true));
    }
}

#include "edge_tp_gen.inc"

constexpr int kETPThreads = 256;   // four wavefronts
constexpr int kETPBwdWaves = 2048; // wavefronts of the backward grid (grid-stride over edges)

constexpr int kETPReduceThreads = 256;
constexpr int kETPProjChannels = 16;  // channel count of the fused product + projection kernels

// Sums the per-wavefront weight-gradient partials in a fixed order: one workgroup per output
// value, each thread a fixed strided subset of the partials, then a fixed tree in LDS.
__global__ void __launch_bounds__(kETPReduceThreads) k_etp_reduce(const float* __restrict__ part, int64_t nparts,
                                                                  int64_t n, float* __restrict__ gw) {
    __shared__ float red[kETPReduceThreads];
    const int64_t i = blockIdx.x;
    float s = 0.f;
    for (int64_t b = threadIdx.x; b < nparts; b += kETPReduceThreads) s += part[b * n + i];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = kETPReduceThreads / 2; w > 0; w >>= 1) {
        if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) gw[i] = red[0];
}

int etp_variant(int C) {
    for (int v = 0; v < kETPNumVariants; ++v)
        if (kETPVariantCW[v] * kETPVariantCPL[v] == C) return v;
    return -1;
}

int etp_check(int32_t config, int32_t C, int64_t E, int* variant) {
    MNX_REQUIRE(config >= 0 && config < kETPNumConfigs, "edge tensor product: config %d out of range", config);
    if (!kETPInfo[config].ok)
        return set_error(MNX_ERR_UNSUPPORTED,
                         "edge tensor product: no per-edge kernel for config %d (input, harmonics and output l "
                         "must all be 0..l_max)",
                         config);
    *variant = etp_variant(C);
    if (*variant < 0)
        return set_error(MNX_ERR_UNSUPPORTED, "edge tensor product: %d channels (8, 16, 32, 64 or 128 compiled)", C);
    MNX_REQUIRE(E >= 0 && E < (int64_t(1) << 33), "edge count out of range");  // forward grid < 2^31 blocks
    return MNX_OK;
}

// Wavefronts of the fused product + projection forward: groups of 16 edges, grid-stride, at most
// cap wavefronts (a multiple of 4: whole workgroups).
constexpr int64_t kETPProjFwdWaves = 8192;
// The fused backward (161 VGPRs at l_max 2: three wavefronts per SIMD) walks groups of 4 edges
// with 3072 wavefronts: 1.61 ms against 1.74 ms with the plain backward's 2048 at 2.6 M edges.
constexpr int64_t kETPProjBwdWaves = 3072;
int64_t etp_proj_bwd_waves(int64_t E) {
    const int64_t groups = (E + 3) / 4;
    const int64_t waves = groups < kETPProjBwdWaves ? groups : kETPProjBwdWaves;
    return ((waves + 3) / 4) * 4;
}
int64_t etp_proj_waves(int64_t E, int64_t cap) {
    const int64_t groups = (E + 15) / 16;
    const int64_t waves = groups < cap ? groups : cap;
    return ((waves + 3) / 4) * 4;
}

int64_t etp_bwd_waves(int64_t E, int C) {
    const int64_t G = 64 / (C < 64 ? C : 64);
    const int64_t groups = (E + G - 1) / G;
    int64_t waves = groups < kETPBwdWaves ? groups : kETPBwdWaves;
    return ((waves + 3) / 4) * 4;
}

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

int mnx_edge_tp_fwd_f32(int32_t config, int32_t channels, const float* x, const float* Y, const float* w,
                        const float* x_scale, int64_t num_edges, float* out, mnx_stream_t stream) {
    clear_error();
    int v = -1;
    int rc = etp_check(config, channels, num_edges, &v);
    if (rc) return rc;
    if (num_edges == 0) return MNX_OK;
    MNX_REQUIRE(x && Y && w && out, "null pointer argument");
    const int64_t G = 64 / kETPVariantCW[v];
    const int64_t blocks = ceil_div(ceil_div(num_edges, G * kETPInfo[config].fwd_groups), kETPThreads / 64);
    hipLaunchKernelGGL(kETPFwd[config][v], dim3(unsigned(blocks)), dim3(kETPThreads), 0, (hipStream_t)stream, x, Y,
                       w, x_scale, num_edges, channels, out);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

size_t mnx_edge_tp_bwd_workspace_bytes(int32_t config, int32_t channels, int64_t num_edges) {
    int v = -1;
    if (etp_check(config, channels, num_edges, &v)) return 0;
    return size_t(etp_bwd_waves(num_edges, channels)) * kETPInfo[config].np * channels * sizeof(float);
}

int mnx_edge_tp_bwd_f32(int32_t config, int32_t channels, const float* x, const float* Y, const float* w,
                        const float* x_scale, const float* grad_out, int64_t num_edges, float* grad_x,
                        float* grad_Y, float* grad_w, float* grad_x_scale, void* workspace, size_t workspace_bytes,
                        mnx_stream_t stream) {
    clear_error();
    int v = -1;
    int rc = etp_check(config, channels, num_edges, &v);
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    const int64_t nw = int64_t(kETPInfo[config].np) * channels;
    if (num_edges == 0) {
        if (grad_w) {
            // no edges: the weight gradient is zero (the reduction over no partials)
            hipLaunchKernelGGL(k_etp_reduce, dim3(unsigned(nw)), dim3(kETPReduceThreads), 0, s,
                               static_cast<const float*>(nullptr), int64_t(0), nw, grad_w);
            MNX_CHECK_LAUNCH();
        }
        return MNX_OK;
    }
    MNX_REQUIRE(x && Y && w && grad_out, "null pointer argument");
    const int64_t waves = etp_bwd_waves(num_edges, channels);
    const size_t need = size_t(waves) * nw * sizeof(float);
    MNX_REQUIRE(workspace && workspace_bytes >= need, "edge tensor product backward: workspace of %zu bytes needed",
                need);
    float* part = static_cast<float*>(workspace);
    hipLaunchKernelGGL(kETPBwd[config][v], dim3(unsigned(waves / 4)), dim3(kETPThreads), 0, s, grad_out, x, Y, w,
                       x_scale, num_edges, channels, grad_x, grad_Y, part, grad_x_scale);
    MNX_CHECK_LAUNCH();
    if (grad_w) {
        hipLaunchKernelGGL(k_etp_reduce, dim3(unsigned(nw)), dim3(kETPReduceThreads), 0, s, part, waves, nw, grad_w);
        MNX_CHECK_LAUNCH();
    }
    return MNX_OK;
}

int32_t mnx_edge_tp_proj_info(int32_t config, int32_t* blocks) {
    clear_error();
    if (config < 0 || config >= kETPNumConfigs) {
        set_error(MNX_ERR_INVALID, "edge tensor product: config %d out of range", config);
        return -1;
    }
    const int* b = kETPProjBlocks[config];
    if (!kETPInfo[config].ok || b[0] == 0) {
        set_error(MNX_ERR_UNSUPPORTED, "edge tensor product: no fused projection for config %d", config);
        return 0;
    }
    if (blocks)
        for (int i = 0; i < 4 * b[0]; ++i) blocks[i] = b[1 + i];
    return b[0];
}

size_t mnx_edge_tp_proj_bwd_workspace_bytes(int32_t config, int64_t num_edges) {
    int v = -1;
    if (etp_check(config, kETPProjChannels, num_edges, &v) || kETPProjBlocks[config][0] == 0) return 0;
    return size_t(etp_proj_bwd_waves(num_edges)) * kETPInfo[config].np * kETPProjChannels * sizeof(float);
}

int mnx_edge_tp_proj_fwd_f32(int32_t config, const float* x, int32_t x_shared, const float* Y, const float* w,
                             const float* x_scale, const float* x_scale2, const float* proj, int64_t num_edges,
                             float* out, mnx_stream_t stream) {
    clear_error();
    int v = -1;
    int rc = etp_check(config, kETPProjChannels, num_edges, &v);
    if (rc) return rc;
    if (num_edges == 0) return MNX_OK;
    MNX_REQUIRE(x && Y && w && proj && out, "null pointer argument");
    const int64_t waves = etp_proj_waves(num_edges, kETPProjFwdWaves);
    hipLaunchKernelGGL(kETPFwdP[config][x_shared ? 1 : 0], dim3(unsigned(waves / 4)), dim3(kETPThreads), 0,
                       (hipStream_t)stream, x, Y, w, x_scale, x_scale2, proj, num_edges, out);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_edge_tp_proj_bwd_f32(int32_t config, const float* x, int32_t x_shared, const float* Y, const float* w,
                             const float* x_scale, const float* x_scale2, const float* proj, const float* grad_out,
                             int64_t num_edges, float* grad_x, float* grad_Y, float* grad_w, float* grad_x_scale,
                             float* grad_x_scale2, void* workspace, size_t workspace_bytes, mnx_stream_t stream) {
    clear_error();
    int v = -1;
    int rc = etp_check(config, kETPProjChannels, num_edges, &v);
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    const int64_t nw = int64_t(kETPInfo[config].np) * kETPProjChannels;
    if (num_edges == 0) {
        if (grad_w) {
            hipLaunchKernelGGL(k_etp_reduce, dim3(unsigned(nw)), dim3(kETPReduceThreads), 0, s,
                               static_cast<const float*>(nullptr), int64_t(0), nw, grad_w);
            MNX_CHECK_LAUNCH();
        }
        return MNX_OK;
    }
    MNX_REQUIRE(x && Y && w && proj && grad_out, "null pointer argument");
    const int64_t waves = etp_proj_bwd_waves(num_edges);
    const size_t need = size_t(waves) * nw * sizeof(float);
    MNX_REQUIRE(workspace && workspace_bytes >= need,
                "edge tensor product + projection backward: workspace of %zu bytes needed", need);
    float* part = static_cast<float*>(workspace);
    hipLaunchKernelGGL(kETPBwdP[config][x_shared ? 1 : 0], dim3(unsigned(waves / 4)), dim3(kETPThreads), 0, s,
                       grad_out, x, Y, w, x_scale, x_scale2, proj, num_edges, grad_x, grad_Y, part, grad_x_scale,
                       grad_x_scale2);
    MNX_CHECK_LAUNCH();
    if (grad_w) {
        hipLaunchKernelGGL(k_etp_reduce, dim3(unsigned(nw)), dim3(kETPReduceThreads), 0, s, part, waves, nw, grad_w);
        MNX_CHECK_LAUNCH();
    }
    return MNX_OK;
}

}  // extern "C"
