// Per-channel products of Allegro's ir_mul edge tensors (D components x F channels per edge,
// channel innermost), forward and backward in one pass each:
//
// channel scale, the output env scaling (src/molzoo/allegro.py:95-128, _scale_by_channel):
//   out[e][d][c] = t[e][d][c] s[e][c]
//   grad_t[e][d][c] = g[e][d][c] s[e][c],       grad_s[e][c] = sum_d g[e][d][c] t[e][d][c]
//
// channel outer product, the env-weighted harmonics of the pair embedding
// (src/molzoo/allegro.py:55-92, Y_lm(e) env(e, c)):
//   out[e][d][c] = y[e][d] s[e][c]
//   grad_y[e][d] = sum_c g[e][d][c] s[e][c],    grad_s[e][c] = sum_d g[e][d][c] y[e][d]
//
// channel outer product over a stack, the cutoff envelope on the per-layer features of Allegro's
// encoder (src/molzoo/allegro.py:628-641), L inputs s_l (E, F) stacked into one (E, L, F) output:
//   out[e][l][c] = y[e] s_l[e][c]
//   grad_s_l[e][c] = g[e][l][c] y[e],           grad_y[e] = sum_l sum_c g[e][l][c] s_l[e][c]
// (the stack is never formed on its own: one pass reads the L inputs and writes the output).
//
// (torch's broadcasting backward makes separate passes and reduces over the middle dimension at
// ~1 TB/s).  One thread per (edge, four channels): the D component rows are loaded before any
// arithmetic (D a template constant for l_max = 0..3, i.e. D = 1, 4, 9, 16), sums over d in a
// fixed order; the sum over channels of grad_y is a float4 sum and an xor reduction over the
// F/4 adjacent lanes of an edge.

#include "common.h"

namespace mnx {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kCsThreads = 256;

__device__ __forceinline__ float hsum(const f32x4& v) { return (v[0] + v[1]) + (v[2] + v[3]); }

template <int D>
__global__ void __launch_bounds__(kCsThreads) k_chscale_fwd(const f32x4* __restrict__ t, const f32x4* __restrict__ s,
                                                            int64_t n4, int F4, f32x4* __restrict__ out) {
    for (int64_t i = int64_t(blockIdx.x) * kCsThreads + threadIdx.x; i < n4; i += int64_t(gridDim.x) * kCsThreads) {
        const int64_t e = i / F4;
        const int64_t base = e * D * F4 + (i - e * F4);
        const f32x4 sc = s[i];
        f32x4 v[D];
#pragma unroll
        for (int d = 0; d < D; ++d) v[d] = t[base + d * F4];
#pragma unroll
        for (int d = 0; d < D; ++d) out[base + d * F4] = v[d] * sc;
    }
}

template <int D>
__global__ void __launch_bounds__(kCsThreads) k_chscale_bwd(const f32x4* __restrict__ g, const f32x4* __restrict__ t,
                                                            const f32x4* __restrict__ s, int64_t n4, int F4,
                                                            f32x4* __restrict__ gt, f32x4* __restrict__ gs) {
    for (int64_t i = int64_t(blockIdx.x) * kCsThreads + threadIdx.x; i < n4; i += int64_t(gridDim.x) * kCsThreads) {
        const int64_t e = i / F4;
        const int64_t base = e * D * F4 + (i - e * F4);
        f32x4 gv[D];
#pragma unroll
        for (int d = 0; d < D; ++d) gv[d] = g[base + d * F4];
        if (gs) {
            f32x4 tv[D];
#pragma unroll
            for (int d = 0; d < D; ++d) tv[d] = t[base + d * F4];
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int d = 0; d < D; ++d) acc += gv[d] * tv[d];
            gs[i] = acc;
        }
        if (gt) {
            const f32x4 sc = s[i];
#pragma unroll
            for (int d = 0; d < D; ++d) gt[base + d * F4] = gv[d] * sc;
        }
    }
}

template <int D>
__global__ void __launch_bounds__(kCsThreads) k_chouter_fwd(const float* __restrict__ y, const f32x4* __restrict__ s,
                                                            int64_t n4, int F4, f32x4* __restrict__ out) {
    for (int64_t i = int64_t(blockIdx.x) * kCsThreads + threadIdx.x; i < n4; i += int64_t(gridDim.x) * kCsThreads) {
        const int64_t e = i / F4;
        const int64_t base = e * D * F4 + (i - e * F4);
        const f32x4 sc = s[i];
        float yv[D];
#pragma unroll
        for (int d = 0; d < D; ++d) yv[d] = y[e * D + d];
#pragma unroll
        for (int d = 0; d < D; ++d) out[base + d * F4] = yv[d] * sc;
    }
}

// the F4 lanes of an edge are adjacent and aligned (i = e F4 + c, F4 a power of two dividing 64,
// and the grid stride a multiple of 64), so all of them are active together
template <int D>
__global__ void __launch_bounds__(kCsThreads) k_chouter_bwd(const f32x4* __restrict__ g, const float* __restrict__ y,
                                                            const f32x4* __restrict__ s, int64_t n4, int F4,
                                                            float* __restrict__ gy, f32x4* __restrict__ gs) {
    for (int64_t i = int64_t(blockIdx.x) * kCsThreads + threadIdx.x; i < n4; i += int64_t(gridDim.x) * kCsThreads) {
        const int64_t e = i / F4;
        const int c = int(i - e * F4);
        const int64_t base = e * D * F4 + c;
        f32x4 gv[D];
#pragma unroll
        for (int d = 0; d < D; ++d) gv[d] = g[base + d * F4];
        if (gs) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int d = 0; d < D; ++d) acc += gv[d] * y[e * D + d];
            gs[i] = acc;
        }
        if (gy) {
            const f32x4 sc = s[i];
            float p[D];
#pragma unroll
            for (int d = 0; d < D; ++d) p[d] = hsum(gv[d] * sc);
            for (int m = 1; m < F4; m <<= 1)
#pragma unroll
                for (int d = 0; d < D; ++d) p[d] += __shfl_xor(p[d], m, 64);
            if (c == 0) {
#pragma unroll
                for (int d = 0; d < D; ++d) gy[e * D + d] = p[d];
            }
        }
    }
}

constexpr int kStackMax = 8;
struct StackIn {
    const f32x4* p[kStackMax];
};
struct StackOut {
    f32x4* p[kStackMax];
};

// one thread per (edge, four channels) for all L layers; the layer loop is unrolled (L a template
// constant), so each input's pointer is a kernel argument read with a constant offset
template <int L>
__global__ void __launch_bounds__(kCsThreads) k_chouter_stack_fwd(const float* __restrict__ y, StackIn s, int64_t n4,
                                                                  int F4, f32x4* __restrict__ out) {
    for (int64_t i = int64_t(blockIdx.x) * kCsThreads + threadIdx.x; i < n4; i += int64_t(gridDim.x) * kCsThreads) {
        const int64_t e = i / F4;
        const float ye = y[e];
        f32x4 v[L];
#pragma unroll
        for (int l = 0; l < L; ++l) v[l] = s.p[l][i];
        f32x4* o = out + e * (L - 1) * F4 + i;  // (e L + l) F4 + c with i = e F4 + c
#pragma unroll
        for (int l = 0; l < L; ++l) o[l * F4] = v[l] * ye;
    }
}

// grad_y's sum over channels: a float4 sum per layer, added over the layers in order, then an xor
// reduction over the F/4 adjacent lanes of an edge (all active together, as in k_chouter_bwd)
template <int L>
__global__ void __launch_bounds__(kCsThreads) k_chouter_stack_bwd(const f32x4* __restrict__ g,
                                                                  const float* __restrict__ y, StackIn s, int64_t n4,
                                                                  int F4, float* __restrict__ gy, StackOut gs,
                                                                  bool need_s) {
    for (int64_t i = int64_t(blockIdx.x) * kCsThreads + threadIdx.x; i < n4; i += int64_t(gridDim.x) * kCsThreads) {
        const int64_t e = i / F4;
        const f32x4* gr = g + e * (L - 1) * F4 + i;
        f32x4 gv[L];
#pragma unroll
        for (int l = 0; l < L; ++l) gv[l] = gr[l * F4];
        if (need_s) {
            const float ye = y[e];
#pragma unroll
            for (int l = 0; l < L; ++l) gs.p[l][i] = gv[l] * ye;
        }
        if (gy) {
            float p = 0.f;
#pragma unroll
            for (int l = 0; l < L; ++l) p += hsum(gv[l] * s.p[l][i]);
            for (int m = 1; m < F4; m <<= 1) p += __shfl_xor(p, m, 64);
            if (i - e * F4 == 0) gy[e] = p;
        }
    }
}

int check_cs(int64_t E, int32_t D, int32_t F) {
    MNX_REQUIRE(E >= 0 && F >= 4 && F % 4 == 0 && E * D * int64_t(F) < (int64_t(1) << 40),
                "channel product: sizes out of range (F must be a positive multiple of 4)");
    MNX_REQUIRE(D == 1 || D == 4 || D == 9 || D == 16, "channel product: %d components (1, 4, 9 or 16: l_max 0..3)", D);
    return MNX_OK;
}

unsigned cs_grid(int64_t n4) { return unsigned(std::min<int64_t>(ceil_div(n4, kCsThreads), 65536)); }

#define MNX_CS_SWITCH(KERNEL, ...)                                                                             \
    switch (D) {                                                                                              \
        case 1: hipLaunchKernelGGL(KERNEL<1>, dim3(cs_grid(n4)), dim3(kCsThreads), 0, st, __VA_ARGS__); break;   \
        case 4: hipLaunchKernelGGL(KERNEL<4>, dim3(cs_grid(n4)), dim3(kCsThreads), 0, st, __VA_ARGS__); break;   \
        case 9: hipLaunchKernelGGL(KERNEL<9>, dim3(cs_grid(n4)), dim3(kCsThreads), 0, st, __VA_ARGS__); break;   \
        default: hipLaunchKernelGGL(KERNEL<16>, dim3(cs_grid(n4)), dim3(kCsThreads), 0, st, __VA_ARGS__); break; \
    }

bool aligned16(const void* p) { return (uintptr_t)p % 16 == 0; }

int check_stack(int64_t E, int32_t L, int32_t F) {
    MNX_REQUIRE(L >= 1 && L <= kStackMax, "channel outer stack: %d inputs (1 to %d)", L, kStackMax);
    MNX_REQUIRE(E >= 0 && F >= 4 && F % 4 == 0 && F / 4 <= 64 && ((F / 4) & (F / 4 - 1)) == 0 &&
                    E * L * int64_t(F) < (int64_t(1) << 40),
                "channel outer stack: sizes out of range (F / 4 must be a power of two <= 64)");
    return MNX_OK;
}

#define MNX_STACK_SWITCH(KERNEL, ...)                                                                      \
    switch (L) {                                                                                          \
        case 1: hipLaunchKernelGGL(KERNEL<1>, dim3(cs_grid(n4)), dim3(kCsThreads), 0, st, __VA_ARGS__); break; \
        case 2: hipLaunchKernelGGL(KERNEL<2>, dim3(cs_grid(n4)), dim3(kCsThreads), 0, st, __VA_ARGS__); break; \
        case 3: hipLaunchKernelGGL(KERNEL<3>, dim3(cs_grid(n4)), dim3(kCsThreads), 0, st, __VA_ARGS__); break; \
        case 4: hipLaunchKernelGGL(KERNEL<4>, dim3(cs_grid(n4)), dim3(kCsThreads), 0, st, __VA_ARGS__); break; \
        case 5: hipLaunchKernelGGL(KERNEL<5>, dim3(cs_grid(n4)), dim3(kCsThreads), 0, st, __VA_ARGS__); break; \
        case 6: hipLaunchKernelGGL(KERNEL<6>, dim3(cs_grid(n4)), dim3(kCsThreads), 0, st, __VA_ARGS__); break; \
        case 7: hipLaunchKernelGGL(KERNEL<7>, dim3(cs_grid(n4)), dim3(kCsThreads), 0, st, __VA_ARGS__); break; \
        default: hipLaunchKernelGGL(KERNEL<8>, dim3(cs_grid(n4)), dim3(kCsThreads), 0, st, __VA_ARGS__); break; \
    }

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

int mnx_channel_scale_f32(const float* t, const float* s, int64_t E, int32_t D, int32_t F, float* out,
                          mnx_stream_t stream) {
    clear_error();
    int rc = check_cs(E, D, F);
    if (rc) return rc;
    if (E == 0) return MNX_OK;
    MNX_REQUIRE(t && s && out, "null pointer argument");
    MNX_REQUIRE(aligned16(t) && aligned16(s) && aligned16(out), "channel scale: pointers must be 16-byte aligned");
    const int64_t n4 = E * (F / 4);
    hipStream_t st = (hipStream_t)stream;
    MNX_CS_SWITCH(k_chscale_fwd, reinterpret_cast<const f32x4*>(t), reinterpret_cast<const f32x4*>(s), n4, F / 4,
                  reinterpret_cast<f32x4*>(out));
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_channel_scale_bwd_f32(const float* grad, const float* t, const float* s, int64_t E, int32_t D, int32_t F,
                              float* grad_t, float* grad_s, mnx_stream_t stream) {
    clear_error();
    int rc = check_cs(E, D, F);
    if (rc) return rc;
    if (E == 0 || (!grad_t && !grad_s)) return MNX_OK;
    MNX_REQUIRE(grad && (!grad_t || s) && (!grad_s || t), "null pointer argument");
    MNX_REQUIRE(aligned16(grad) && aligned16(t) && aligned16(s) && aligned16(grad_t) && aligned16(grad_s),
                "channel scale: pointers must be 16-byte aligned");
    const int64_t n4 = E * (F / 4);
    hipStream_t st = (hipStream_t)stream;
    MNX_CS_SWITCH(k_chscale_bwd, reinterpret_cast<const f32x4*>(grad), reinterpret_cast<const f32x4*>(t),
                  reinterpret_cast<const f32x4*>(s), n4, F / 4, reinterpret_cast<f32x4*>(grad_t),
                  reinterpret_cast<f32x4*>(grad_s));
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_channel_outer_f32(const float* y, const float* s, int64_t E, int32_t D, int32_t F, float* out,
                          mnx_stream_t stream) {
    clear_error();
    int rc = check_cs(E, D, F);
    if (rc) return rc;
    if (E == 0) return MNX_OK;
    MNX_REQUIRE(y && s && out, "null pointer argument");
    MNX_REQUIRE(aligned16(s) && aligned16(out), "channel outer product: s and out must be 16-byte aligned");
    const int64_t n4 = E * (F / 4);
    hipStream_t st = (hipStream_t)stream;
    MNX_CS_SWITCH(k_chouter_fwd, y, reinterpret_cast<const f32x4*>(s), n4, F / 4, reinterpret_cast<f32x4*>(out));
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_channel_outer_bwd_f32(const float* grad, const float* y, const float* s, int64_t E, int32_t D, int32_t F,
                              float* grad_y, float* grad_s, mnx_stream_t stream) {
    clear_error();
    int rc = check_cs(E, D, F);
    if (rc) return rc;
    if (E == 0 || (!grad_y && !grad_s)) return MNX_OK;
    const int F4 = F / 4;
    MNX_REQUIRE(F4 <= 64 && (F4 & (F4 - 1)) == 0, "channel outer product: F / 4 must be a power of two <= 64");
    MNX_REQUIRE(grad && (!grad_y || s) && (!grad_s || y), "null pointer argument");
    MNX_REQUIRE(aligned16(grad) && aligned16(s) && aligned16(grad_s),
                "channel outer product: grad, s and grad_s must be 16-byte aligned");
    const int64_t n4 = E * F4;
    hipStream_t st = (hipStream_t)stream;
    MNX_CS_SWITCH(k_chouter_bwd, reinterpret_cast<const f32x4*>(grad), y, reinterpret_cast<const f32x4*>(s), n4, F4,
                  grad_y, reinterpret_cast<f32x4*>(grad_s));
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_channel_outer_stack_f32(const float* y, const float* const* s, int32_t L, int64_t E, int32_t F, float* out,
                                mnx_stream_t stream) {
    clear_error();
    int rc = check_stack(E, L, F);
    if (rc) return rc;
    if (E == 0) return MNX_OK;
    MNX_REQUIRE(y && s && out, "null pointer argument");
    MNX_REQUIRE(aligned16(out), "channel outer stack: out must be 16-byte aligned");
    StackIn in{};
    for (int l = 0; l < L; ++l) {
        MNX_REQUIRE(s[l] && aligned16(s[l]), "channel outer stack: input %d null or not 16-byte aligned", l);
        in.p[l] = reinterpret_cast<const f32x4*>(s[l]);
    }
    const int64_t n4 = E * (F / 4);
    hipStream_t st = (hipStream_t)stream;
    MNX_STACK_SWITCH(k_chouter_stack_fwd, y, in, n4, F / 4, reinterpret_cast<f32x4*>(out));
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_channel_outer_stack_bwd_f32(const float* grad, const float* y, const float* const* s, int32_t L, int64_t E,
                                    int32_t F, float* grad_y, float* const* grad_s, mnx_stream_t stream) {
    clear_error();
    int rc = check_stack(E, L, F);
    if (rc) return rc;
    if (E == 0 || (!grad_y && !grad_s)) return MNX_OK;
    MNX_REQUIRE(grad && aligned16(grad), "channel outer stack: grad null or not 16-byte aligned");
    MNX_REQUIRE(!grad_s || y, "null pointer argument");
    MNX_REQUIRE(!grad_y || s, "null pointer argument");
    StackIn in{};
    StackOut out{};
    for (int l = 0; l < L; ++l) {
        if (grad_y) {
            MNX_REQUIRE(s[l] && aligned16(s[l]), "channel outer stack: input %d null or not 16-byte aligned", l);
            in.p[l] = reinterpret_cast<const f32x4*>(s[l]);
        }
        if (grad_s) {
            MNX_REQUIRE(grad_s[l] && aligned16(grad_s[l]), "channel outer stack: grad_s %d null or not 16-byte aligned",
                        l);
            out.p[l] = reinterpret_cast<f32x4*>(grad_s[l]);
        }
    }
    const int64_t n4 = E * (F / 4);
    hipStream_t st = (hipStream_t)stream;
    MNX_STACK_SWITCH(k_chouter_stack_bwd, reinterpret_cast<const f32x4*>(grad), y, in, n4, F / 4, grad_y, out,
                     grad_s != nullptr);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

}  // extern "C"
