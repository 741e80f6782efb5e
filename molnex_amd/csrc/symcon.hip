// Symmetric contraction of scalar channels, the form the reference builds:
// cuet.SymmetricContraction("{D}x0e" -> "{D}x0e", contraction_degree = nu,
// num_elements = S, original_mace=True) (src/molrep/interaction/
// symmetric_contraction.py:90-109).  For 0e inputs the symmetric products of
// degree k have one coupling path each, so per node n of element z and channel c
//   out[n][c] = sum_{k=1..nu} W[z][k-1][c] * x[n][c]^k.
// Forward: one thread per (node, channel), coalesced along channels.
// Backward: grad_x in the same layout; grad_W reduced per (element, degree,
// channel) in registers over a chunk of nodes, then one atomic per chunk.
//
// The general (equivariant) contraction -- irreps 0e+1o+..+l_in in, 0e (+1o)
// out, correlation <= 3 -- runs the generated kernels of sc_gen.inc: one thread
// per (node, channel) in the forward; the backward walks a chunk of nodes in a
// caller-given order (nodes grouped by element) per channel, keeping the weight
// gradient of the current element in registers and flushing it with one atomic
// per path when the element changes.

#include "common.h"

namespace mnx {
namespace {

constexpr int kMaxDeg = 4;
constexpr int kMaxElem = 16;

__global__ void k_sc_fwd(const float* __restrict__ x, const int64_t* __restrict__ z, const float* __restrict__ W,
                         int64_t N, int D, int S, int nu, float* __restrict__ out) {
    const int c = blockIdx.y * blockDim.x + threadIdx.x;
    const int64_t n = blockIdx.x;
    if (c >= D) return;
    const int64_t e = z[n];
    float acc = 0.f;
    if (e >= 0 && e < S) {
        const float xv = x[n * D + c];
        float p = 1.f;
        for (int k = 0; k < nu; ++k) {
            p *= xv;
            acc = fmaf(W[(e * nu + k) * D + c], p, acc);
        }
    }
    out[n * D + c] = acc;
}

// grid.x: node chunks, grid.y: channel blocks
__global__ void k_sc_bwd(const float* __restrict__ x, const int64_t* __restrict__ z, const float* __restrict__ W,
                         const float* __restrict__ g, int64_t N, int D, int S, int nu, int64_t chunk,
                         float* __restrict__ gx, float* __restrict__ gW) {
    const int c = blockIdx.y * blockDim.x + threadIdx.x;
    if (c >= D) return;
    float acc[kMaxElem][kMaxDeg];
#pragma unroll
    for (int s = 0; s < kMaxElem; ++s)
#pragma unroll
        for (int k = 0; k < kMaxDeg; ++k) acc[s][k] = 0.f;
    const int64_t n0 = int64_t(blockIdx.x) * chunk;
    const int64_t n1 = n0 + chunk < N ? n0 + chunk : N;
    for (int64_t n = n0; n < n1; ++n) {
        const int64_t e = z[n];
        const float gv = g[n * D + c];
        const float xv = x[n * D + c];
        float dx = 0.f;
        if (e >= 0 && e < S) {
            float p = 1.f;  // x^k
            float pm = 1.f; // x^(k-1)
#pragma unroll
            for (int k = 0; k < kMaxDeg; ++k) {
                if (k >= nu) break;
                p *= xv;
                dx = fmaf(float(k + 1) * W[(e * nu + k) * D + c], pm, dx);
                pm = p;
#pragma unroll
                for (int s = 0; s < kMaxElem; ++s)
                    if (s == e) acc[s][k] = fmaf(gv, p, acc[s][k]);
            }
        }
        if (gx) gx[n * D + c] = gv * dx;
    }
    if (gW) {
        for (int s = 0; s < S; ++s)
            for (int k = 0; k < nu; ++k) {
                float v = 0.f;
#pragma unroll
                for (int q = 0; q < kMaxElem; ++q)
#pragma unroll
                    for (int r = 0; r < kMaxDeg; ++r)
                        if (q == s && r == k) v = acc[q][r];
                if (v != 0.f) atomicAdd(gW + (int64_t(s) * nu + k) * D + c, v);
            }
    }
}

#include "sc_gen.inc"

constexpr int kSCChunk = 16;

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

int mnx_sc_scalar_fwd_f32(const float* x, const int64_t* types, const float* W, int64_t N, int32_t D, int32_t S,
                          int32_t nu, float* out, mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(N >= 0 && N < (int64_t(1) << 31) && D > 0 && S > 0 && S <= kMaxElem && nu >= 1 && nu <= kMaxDeg,
                "unsupported sizes (S <= %d, 1 <= degree <= %d)", kMaxElem, kMaxDeg);
    if (N == 0) return MNX_OK;
    MNX_REQUIRE(x && types && W && out, "null pointer argument");
    const int tb = 64;
    hipLaunchKernelGGL(k_sc_fwd, dim3(unsigned(N), unsigned(ceil_div(D, tb))), dim3(tb), 0, (hipStream_t)stream, x,
                       types, W, N, D, S, nu, out);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_sc_scalar_bwd_f32(const float* x, const int64_t* types, const float* W, const float* grad_out, int64_t N,
                          int32_t D, int32_t S, int32_t nu, float* grad_x, float* grad_W, mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(N >= 0 && N < (int64_t(1) << 31) && D > 0 && S > 0 && S <= kMaxElem && nu >= 1 && nu <= kMaxDeg,
                "unsupported sizes (S <= %d, 1 <= degree <= %d)", kMaxElem, kMaxDeg);
    if (N == 0) return MNX_OK;
    MNX_REQUIRE(x && types && W && grad_out, "null pointer argument");
    const int tb = 64;
    const int64_t chunk = 256;
    hipLaunchKernelGGL(k_sc_bwd, dim3(unsigned(ceil_div(N, chunk)), unsigned(ceil_div(D, tb))), dim3(tb), 0,
                       (hipStream_t)stream, x, types, W, grad_out, N, D, S, nu, chunk, grad_x, grad_W);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_sc_config(int32_t l_in, int32_t l_out, int32_t correlation) {
    clear_error();
    for (int i = 0; i < kNumSCConfigs; ++i) {
        const SCConfig& c = kSCConfigs[i];
        if (c.l_in == l_in && c.l_out == l_out && c.nu == correlation) return i;
    }
    set_error(MNX_ERR_UNSUPPORTED, "no symmetric-contraction kernel for l_in %d, L_out %d, correlation %d (l_in 1..3, L_out 0..1, "
              "correlation 1..3)", l_in, l_out, correlation);
    return -1;
}

int mnx_sc_config_info(int32_t config, int32_t* info) {
    clear_error();
    MNX_REQUIRE(config >= 0 && config < kNumSCConfigs && info, "bad symmetric-contraction config %d", config);
    const SCConfig& c = kSCConfigs[config];
    info[0] = c.ni;
    info[1] = c.no;
    info[2] = c.paths;
    info[3] = c.nnz;
    return MNX_OK;
}

int mnx_sc_fwd_f32(int32_t config, const float* A, const int64_t* types, const float* W, int64_t N, int32_t C,
                   int32_t S, float* out, mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(config >= 0 && config < kNumSCConfigs, "bad symmetric-contraction config %d", config);
    MNX_REQUIRE(N >= 0 && C > 0 && S > 0 && N * int64_t(C) < (int64_t(1) << 40), "bad sizes");
    if (N == 0) return MNX_OK;
    MNX_REQUIRE(A && types && W && out, "null pointer argument");
    const int64_t threads = N * C;
    hipLaunchKernelGGL(kSCFwd[config], dim3(unsigned(ceil_div(threads, int64_t(256)))), dim3(256), 0,
                       (hipStream_t)stream, A, types, W, N, int(C), int(S), out);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_sc_bwd_f32(int32_t config, const float* A, const int64_t* types, const float* W, const float* grad_out,
                   const int32_t* order, int64_t N, int32_t C, int32_t S, float* grad_A, float* grad_W,
                   mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(config >= 0 && config < kNumSCConfigs, "bad symmetric-contraction config %d", config);
    MNX_REQUIRE(N >= 0 && N < (int64_t(1) << 31) && C > 0 && S > 0 && N * int64_t(C) < (int64_t(1) << 40),
                "bad sizes");
    if (N == 0 || (!grad_A && !grad_W)) return MNX_OK;
    MNX_REQUIRE(A && types && W && grad_out, "null pointer argument");
    const SCBwdFn fn = grad_A && grad_W ? kSCBwdAW[config] : grad_A ? kSCBwdA[config] : kSCBwdW[config];
    const int64_t threads = ceil_div(N, int64_t(kSCChunk)) * C;
    hipLaunchKernelGGL(fn, dim3(unsigned(ceil_div(threads, int64_t(256)))), dim3(256), 0, (hipStream_t)stream, A,
                       types, W, grad_out, order, N, int(C), int(S), kSCChunk, grad_A, grad_W);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_sc_bwd2_f32(int32_t config, const float* A, const int64_t* types, const float* W, const float* grad_out,
                    const float* seed_A, const float* seed_W, const int32_t* order, int64_t N, int32_t C,
                    int32_t S, float* d_grad_out, float* d_A, float* d_W, mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(config >= 0 && config < kNumSCConfigs, "bad symmetric-contraction config %d", config);
    MNX_REQUIRE(N >= 0 && N < (int64_t(1) << 31) && C > 0 && S > 0 && N * int64_t(C) < (int64_t(1) << 40),
                "bad sizes");
    if (N == 0 || (!d_grad_out && !d_A && !d_W)) return MNX_OK;
    MNX_REQUIRE(A && types && W && grad_out, "null pointer argument");
    const int64_t threads = ceil_div(N, int64_t(kSCChunk)) * C;
    hipLaunchKernelGGL(kSCBwd2[config], dim3(unsigned(ceil_div(threads, int64_t(256)))), dim3(256), 0,
                       (hipStream_t)stream, A, types, W, grad_out, seed_A, seed_W, order, N, int(C), int(S), kSCChunk,
                       d_grad_out, d_A, d_W);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

}  // extern "C"
