// Shared pieces of the split-fp16 matrix-core products of the radial MLP's
// output layer (edge_weights.hip) and of the fused tensor-product weight
// gradient (tp_gh.hip): vector types, the LDS stage size, the per-row /
// per-column power-of-two scaling and the two-part fp16 split, and the shape of
// the pre-split weight fragments.
#pragma once

#include "common.h"

namespace mnx {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kEwFwdThreads = 512;                   // eight wavefronts
constexpr int kEwFwdRows = (kEwFwdThreads / 64) * 32;  // edges per forward workgroup
constexpr int kEwBwdThreads = 256;                   // four wavefronts
constexpr int kEwBwdRows = (kEwBwdThreads / 64) * 32;  // edges per backward workgroup
constexpr int kEwStageVec = 1024;                    // f16x8 vectors per LDS stage (16 KB)
constexpr int kEwNoExp = -127;                       // scale exponent of an all-zero row

// Weight fragment layouts (fp16 elements, 8 per lane-vector), of W scaled by the
// reciprocal of its column scale (forward: per output n; backward: per output k):
//  forward, B = W^T (K x N): [stage][plane][q < KS][t < SC][lane][8] holds
//    W[n][k], k = 16q + 8(lane/32) + j, n = 32(SC*stage + t) + lane%32;
//  backward, A = W^T (K x N): [stage][plane][q < NQ][t < T][lane][8] holds
//    W[n][c], n = 16(NQ*stage + q) + 8(lane/32) + j, c = 32t + lane%32;
// zero outside the matrix.  KS * SC = NQ * T = 8, so every stage is 2 * 8 * 64
// vectors.  The planes are followed by the column scales as fp32 (N of them
// forward, K backward), each a power of two.
struct EwShape {
    int K, N;
    __host__ __device__ int ks() const { return K / 16; }
    __host__ __device__ int sc() const { return 8 / ks(); }
    __host__ __device__ int tiles_b() const { return (K + 31) / 32; }
    __host__ __device__ int nq() const { return 8 / tiles_b(); }
    __host__ __device__ int stages_f() const { return (N + 32 * sc() - 1) / (32 * sc()); }
    __host__ __device__ int stages_b() const { return (N + 16 * nq() - 1) / (16 * nq()); }
    __host__ __device__ int64_t planes(bool bwd) const {
        return int64_t(bwd ? stages_b() : stages_f()) * kEwStageVec * 8;
    }
    // fp16 elements in all: the planes, then the scales (two fp16 slots per fp32)
    __host__ __device__ int64_t elems(bool bwd) const { return planes(bwd) + 2 * int64_t(bwd ? K : N); }
};

// Exponent e with 2^e <= m < 2^(e+1), clamped so that 2^e and 2^-e are normal;
// kEwNoExp for m == 0, 0 for inf/NaN (left to propagate).
__device__ __forceinline__ int ew_exp(float m) {
    if (m == 0.f) return kEwNoExp;
    if (!(m <= 3.402823466e38f)) return 0;
    return min(max(ilogbf(m), -126), 126);
}

// a0 = f16(x s), a1 = f16(x s - a0) for the 8 values: each part is one mixed-precision fma
// (v_fma_mix, f32 operands and f16 result; a0 enters the second as an f16 operand), so the scaling
// and conversions cost two vector instructions per value.  s is a power of two, so x s is exact
// and the parts equal those of the plain product.
__device__ __forceinline__ void split8(const f32x4& lo, const f32x4& hi, float s, f16x8& a0, f16x8& a1) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float x = j < 4 ? lo[j] : hi[j - 4];
        const _Float16 h0 = (_Float16)__builtin_fmaf(x, s, 0.0f);
        a0[j] = h0;
        a1[j] = (_Float16)__builtin_fmaf(x, s, -(float)h0);
    }
}

// max(m, |values|): one v_max3_f32 with absolute-value source modifiers per two values.  fmaxf
// compiles to ~1.8 instructions per value here (each |x| is first canonicalised, an IEEE-mode
// quieting of signalling NaNs that no arithmetic produces); quiet NaNs are ignored either way.
__device__ __forceinline__ float absmax8(const f32x4& lo, const f32x4& hi, float m) {
#pragma unroll
    for (int j = 0; j < 4; ++j) asm("v_max3_f32 %0, |%1|, |%2|, %0" : "+v"(m) : "v"(lo[j]), "v"(hi[j]));
    return m;
}

__device__ __forceinline__ f32x16 mfma(const f16x8& a, const f16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

}  // namespace mnx
