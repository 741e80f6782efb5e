// Channelwise tensor-product backward fused with the input gradient of the radial
// MLP's output layer, for gfx950.
//
// The reference computes the per-edge weights w = h W^T + b with the last Linear
// of RadialWeightMLP (src/molrep/interaction/radial_mlp.py:76-82) and hands them to
// cuet.ChannelWiseTensorProduct (src/molrep/interaction/tensor_product.py:72-79,
// 101-111); autograd then writes the per-edge weight gradient gw (2.6 M x 2944
// floats, 30.8 GB at the config-3 size) and reads it back for grad_h = gw W.
// Here the tensor-product backward forms gw in registers (lanes = channels, one
// wavefront per channel block of 64) exactly as tp.hip's receiver walk does,
// stages each edge's gw row of the current path group in LDS, and every few edges
// multiplies the staged rows by the group's slice of W on the matrix cores:
//
//   hpart[group, block][t][k] = sum_{p in group, c in block} gw[e(t)][p][c] W[p C + c][k]
//
// for CSR slot t of edge e(t).  A small kernel then sums the partials of every
// (group, channel block) in a fixed order into grad_h[e] (no atomics).
//
// Work decomposition: persistent workgroups of NWAVE wavefronts, one per compute
// unit (the W slice, P paths x 64 channels x K hidden, as pre-split fp16
// fragments, stays in LDS for the whole kernel).  Each wavefront walks an equal
// share of the CSR slots, so every workgroup has the same number of phases;
// receivers change along a wavefront's range (it folds the new receiver's output
// gradient).  A phase is SW edges per wavefront; then a barrier, 16 x 16 output
// tiles on v_mfma_f32_16x16x32_f16 (lane l holds A[l%16][8(l/16)+j],
// B[8(l/16)+j][l%16], j < 8, and D[4(l/16)+r][l%16], r < 4), and a barrier before
// the staging is reused.  Products are near-fp32: the split-fp16 scheme of
// edge_weights.hip (rows of gw and columns of W scaled by powers of two from their
// largest magnitude, each split into two fp16 parts, three products accumulated
// smallest first in fp32, scales undone in the epilogue).
//
// grad_x is accumulated with fp32 atomics and grad_Y partials per (edge, group,
// channel block) are reduced by a second kernel, as in tp.hip.

#include "common.h"
#include "ew.h"
#include "wave.h"

namespace mnx {
namespace {

constexpr int kFusedMaxPaths = 8;

typedef void (*TPFusedFn)(const float*, const float*, const float*, const float*, const int32_t*, const int32_t*,
                          const int32_t*, const int32_t*, int64_t, int64_t, int, float*, float*, int, int,
                          const f16x8*, const float*, float*);

struct TPFusedKernel {
    TPFusedFn fn;
    int nwave, sw, lds;
};

struct TPFusedGroup {
    int paths;
    int pk[kFusedMaxPaths];  // weight-row index (path number) of each path of the group
    TPFusedKernel k[2];      // per hidden width kFusedKH[i]
};

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// One phase's matrix-core work: the (SLOTS x KH) block of partial grad_h rows from the
// staged gw rows and the resident W fragments, written at the rows' CSR slots.
template <int P, int NWAVE, int SW, int KH>
__device__ __forceinline__ void fused_gh_tiles(const f16x8* __restrict__ sW, const _Float16* __restrict__ sA,
                                               const int* __restrict__ sE, const int* __restrict__ sT,
                                               const float* __restrict__ kscale, float* __restrict__ hp, int lane,
                                               int wave) {
    constexpr int SLOTS = NWAVE * SW, AST = P * 64 + 8, KSTEPS = P * 2, CT = KH / 16;
    constexpr int RT = (SLOTS + 15) / 16;
    for (int tile = wave; tile < RT * CT; tile += NWAVE) {
        const int rt = tile % RT, ct = tile / RT;
        const int row = rt * 16 + (lane & 15);
        const bool valid = row < SLOTS && sT[row < SLOTS ? row : 0] >= 0;
        // the row's two fp16 planes (already scaled and split by the wavefront that staged it)
        const _Float16* __restrict__ arow = sA + (valid ? row : 0) * AST + 8 * (lane >> 4);
        const f16x8* __restrict__ wb = sW + ct * KSTEPS * 128 + lane;
        const f16x8 zero = {};
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
        for (int s = 0; s < KSTEPS; ++s) {
            const f16x8 a0 = valid ? *reinterpret_cast<const f16x8*>(arow + 32 * s) : zero;
            const f16x8 a1 = valid ? *reinterpret_cast<const f16x8*>(arow + SLOTS * AST + 32 * s) : zero;
            const f16x8 b0 = wb[s * 128], b1 = wb[s * 128 + 64];
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b0, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b1, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0, acc, 0, 0, 0);
        }
        const int col = ct * 16 + (lane & 15);
        const float ks = kscale[col];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int srow = rt * 16 + 4 * (lane >> 4) + r;
            if (srow < SLOTS) {
                const int t = sT[srow];
                if (t >= 0) hp[int64_t(t) * KH + col] = ldexpf(acc[r] * ks, sE[srow]);
            }
        }
    }
}

#include "tp_bwf_gen.inc"

// Column scales of W (N x K): scale[k] = 2^e with 2^e <= max_n |W[n][k]| < 2^(e+1)
// (1 for an all-zero column); one workgroup per column.
__global__ void __launch_bounds__(256) k_fused_scales(const float* __restrict__ W, int N, int K,
                                                      float* __restrict__ scale) {
    __shared__ float part[256];
    const int k = blockIdx.x;
    float m = 0.f;
    for (int n = threadIdx.x; n < N; n += 256) m = fmaxf(m, fabsf(W[int64_t(n) * K + k]));
    part[threadIdx.x] = m;
    __syncthreads();
    for (int h = 128; h > 0; h >>= 1) {
        if (threadIdx.x < h) part[threadIdx.x] = fmaxf(part[threadIdx.x], part[threadIdx.x + h]);
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const int e = ew_exp(part[0]);
        scale[k] = ldexpf(1.f, e == kEwNoExp ? 0 : e);
    }
}

struct FusedPackLayout {
    int ngroups, cblocks, C, K;
    int paths[4];
    int pk[4][kFusedMaxPaths];
    int64_t off[4];  // first f16x8 vector of each group's slices
};

// W fragments, one thread per fp16 element: per (group, channel block) slice
// [ct < K/16][s < 2P][plane][lane][j < 8] holds the plane of W[n][k] / scale[k] with
// contraction index q = 32 s + 8 (lane / 16) + j = 64 (path slot) + channel in block,
// n = pk[path slot] * C + 64 cb + channel, k = 16 ct + lane % 16.
__global__ void k_fused_pack(const float* __restrict__ W, const float* __restrict__ scale, FusedPackLayout L,
                             _Float16* __restrict__ frag, int64_t total) {
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    int g = 0;
    while (g + 1 < L.ngroups && idx >= L.off[g + 1] * 8) ++g;
    const int P = L.paths[g];
    int64_t r = idx - L.off[g] * 8;
    const int j = int(r % 8);
    r /= 8;
    const int lane = int(r % 64);
    r /= 64;
    const int plane = int(r % 2);
    r /= 2;
    const int s = int(r % (2 * P));
    r /= 2 * P;
    const int ct = int(r % (L.K / 16));
    const int cb = int(r / (L.K / 16));
    const int q = 32 * s + 8 * (lane / 16) + j;
    const int64_t n = int64_t(L.pk[g][q / 64]) * L.C + 64 * cb + q % 64;
    const int k = 16 * ct + lane % 16;
    const float v = ldexpf(W[n * L.K + k], -ilogbf(scale[k]));
    const _Float16 h0 = (_Float16)v;
    frag[idx] = plane == 0 ? h0 : (_Float16)(v - (float)h0);
}

// grad_h[perm[t]][k] = sum_q hpart[q][t][k], partials added in a fixed order; one thread
// per (slot, four columns).
__global__ void k_fused_sum(const float* __restrict__ hpart, int nparts, int64_t E, int K,
                            const int32_t* __restrict__ perm, float* __restrict__ gh) {
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int kq = K / 4;
    if (idx >= E * kq) return;
    const int64_t t = idx / kq;
    const int k4 = int(idx % kq) * 4;
    f32x4 acc = *reinterpret_cast<const f32x4*>(hpart + t * K + k4);
    for (int q = 1; q < nparts; ++q) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(hpart + (q * E + t) * K + k4);
        acc += v;
    }
    *reinterpret_cast<f32x4*>(gh + int64_t(perm[t]) * K + k4) = acc;
}

__global__ void k_fused_reduce_gy(const float* __restrict__ part, int64_t E, int npart, int ny, float* __restrict__ gY) {
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= E * ny) return;
    const int64_t e = idx / ny;
    const int m = int(idx - e * ny);
    const float* p = part + e * npart * ny + m;
    float s = 0.f;
    for (int q = 0; q < npart; ++q) s += p[int64_t(q) * ny];
    gY[idx] = s;
}

int fused_kh_index(int K) {
    for (int i = 0; i < kNumFusedKH; ++i)
        if (kFusedKH[i] == K) return i;
    return -1;
}

int num_configs() { return int(sizeof(kTPFused) / sizeof(kTPFused[0])); }

int num_groups(int config) {
    int g = 0;
    while (g < 4 && kTPFused[config][g].paths > 0) ++g;
    return g;
}

bool supported(int config, int C, int K) {
    if (config < 0 || config >= num_configs() || C <= 0 || C % 64 != 0 || C > 4096) return false;
    const int ki = fused_kh_index(K);
    if (ki < 0) return false;
    const int ng = num_groups(config);
    if (ng == 0) return false;
    for (int g = 0; g < ng; ++g)
        if (!kTPFused[config][g].k[ki].fn) return false;
    return true;
}

struct FusedSizes {
    int64_t frag_vecs, npart, ny, total_paths;
};

FusedSizes sizes(int config, int C, int K) {
    FusedSizes s{0, 0, 0, 0};
    const int cb = C / 64;
    for (int g = 0; g < num_groups(config); ++g) {
        s.frag_vecs += int64_t(cb) * kTPFused[config][g].paths * K * 16;
        s.npart += cb;
        s.total_paths += kTPFused[config][g].paths;
    }
    return s;
}

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

int mnx_tp_bwd_gh_supported(int32_t config, int32_t C, int32_t K) { return supported(config, C, K) ? 1 : 0; }

size_t mnx_tp_bwd_gh_workspace_bytes(int32_t config, int32_t C, int64_t E, int32_t K, int32_t ny) {
    if (!supported(config, C, K) || E < 0 || ny < 0) return 0;
    const FusedSizes s = sizes(config, C, K);
    const int64_t Ee = E > 0 ? E : 1;
    Workspace w{nullptr, 0};
    w.take<float>(size_t(Ee) * size_t(s.npart) * size_t(ny));  // grad_Y partials
    w.take<float>(size_t(K));                                 // column scales
    w.take<f16x8>(size_t(s.frag_vecs));                       // W fragments
    w.take<float>(size_t(s.npart) * size_t(Ee) * size_t(K));  // grad_h partials
    return w.used + 256;
}

int mnx_tp_bwd_gh_rows_f32(int32_t config, int32_t C, const float* x, const float* Y, const float* w,
                           const int32_t* wrow, const float* gout, const int32_t* row_ptr, const int32_t* perm,
                           const int32_t* snd, int64_t N, int64_t E, int32_t ny, const float* W, int32_t K,
                           float* gx, float* gY, float* gh, void* ws, size_t ws_bytes, mnx_stream_t stream_) {
    clear_error();
    hipStream_t stream = (hipStream_t)stream_;
    MNX_REQUIRE(supported(config, C, K), "tp_bwd_gh: no fused kernel for config %d, C = %d, K = %d", config, C, K);
    MNX_REQUIRE(N >= 0 && N < (int64_t(1) << 31) && E >= 0 && E < (int64_t(1) << 31), "sizes out of range");
    MNX_REQUIRE(ny > 0 && ny <= 64, "ny out of range");
    if (N == 0 || E == 0) return MNX_OK;
    MNX_REQUIRE(x && Y && w && gout && row_ptr && perm && snd && W && gh, "null pointer argument");
    MNX_REQUIRE(reinterpret_cast<uintptr_t>(gh) % 16 == 0, "grad_h must be 16-byte aligned");
    const size_t need = mnx_tp_bwd_gh_workspace_bytes(config, C, E, K, ny);
    MNX_REQUIRE(ws && ws_bytes >= need, "workspace %zu < %zu bytes", ws_bytes, need);
    const FusedSizes sz = sizes(config, C, K);
    const int cblocks = C / 64, ki = fused_kh_index(K), ng = num_groups(config);
    Workspace wsp{static_cast<char*>(ws), ws_bytes};
    float* gyp = wsp.take<float>(size_t(E) * size_t(sz.npart) * size_t(ny));
    float* kscale = wsp.take<float>(size_t(K));
    f16x8* frag = wsp.take<f16x8>(size_t(sz.frag_vecs));
    float* hpart = wsp.take<float>(size_t(sz.npart) * size_t(E) * size_t(K));

    // W column scales and fragments
    const int Nw = int(sz.total_paths) * C;
    hipLaunchKernelGGL(k_fused_scales, dim3(unsigned(K)), dim3(256), 0, stream, W, Nw, int(K), kscale);
    MNX_CHECK_LAUNCH();
    FusedPackLayout lay{};
    lay.ngroups = ng;
    lay.cblocks = cblocks;
    lay.C = C;
    lay.K = K;
    int64_t off = 0;
    for (int g = 0; g < ng; ++g) {
        lay.paths[g] = kTPFused[config][g].paths;
        for (int p = 0; p < kFusedMaxPaths; ++p) lay.pk[g][p] = kTPFused[config][g].pk[p];
        lay.off[g] = off;
        off += int64_t(cblocks) * lay.paths[g] * K * 16;
    }
    const int64_t total = sz.frag_vecs * 8;
    hipLaunchKernelGGL(k_fused_pack, dim3(unsigned(ceil_div(total, 256))), dim3(256), 0, stream, W, kscale, lay,
                       reinterpret_cast<_Float16*>(frag), total);
    MNX_CHECK_LAUNCH();

    // one persistent workgroup per compute unit and channel block, a multiple of 8 (XCDs)
    static int cus[64] = {};
    int dev = 0;
    MNX_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return set_error(MNX_ERR_INVALID, "device id %d out of range", dev);
    if (cus[dev] == 0) MNX_HIP_TRY(hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev));
    int64_t nwg = std::max<int64_t>(8, (cus[dev] / cblocks) / 8 * 8);
    int pbase = 0;
    for (int g = 0; g < ng; ++g) {
        const TPFusedKernel& kk = kTPFused[config][g].k[ki];
        {  // dynamic LDS beyond 64 KB: allowed once per kernel and device
            static std::mutex mu;
            static std::unordered_map<const void*, uint64_t> done;
            std::lock_guard<std::mutex> lock(mu);
            uint64_t& bits = done[reinterpret_cast<const void*>(kk.fn)];
            if (!(bits >> dev & 1)) {
                MNX_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(kk.fn),
                                                hipFuncAttributeMaxDynamicSharedMemorySize, kk.lds));
                bits |= uint64_t(1) << dev;
            }
        }
        hipLaunchKernelGGL(kk.fn, dim3(unsigned(nwg), unsigned(cblocks)), dim3(64 * kk.nwave), size_t(kk.lds), stream,
                           x, Y, w, gout, row_ptr, perm, snd, wrow, N, E, C, gx, gY ? gyp : nullptr,
                           int(sz.npart), pbase, frag + lay.off[g], kscale, hpart + int64_t(pbase) * E * K);
        MNX_CHECK_LAUNCH();
        pbase += cblocks;
    }
    hipLaunchKernelGGL(k_fused_sum, dim3(unsigned(ceil_div(E * (K / 4), 256))), dim3(256), 0, stream, hpart,
                       int(sz.npart), E, int(K), perm, gh);
    MNX_CHECK_LAUNCH();
    if (gY) {
        hipLaunchKernelGGL(k_fused_reduce_gy, dim3(unsigned(ceil_div(E * ny, 256))), dim3(256), 0, stream, gyp, E,
                           int(sz.npart), int(ny), gY);
        MNX_CHECK_LAUNCH();
    }
    return MNX_OK;
}

}  // extern "C"
