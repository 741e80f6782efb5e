// Real spherical harmonics l <= 3 (component normalisation) of normalised
// vectors, forward and backward; replaces cuet.SphericalHarmonics(ls,
// normalize=True) behind molrep.embedding.SphericalHarmonics
// (src/molrep/embedding/angular.py:89,104).  One thread per vector.
//
// Basis (u = v / |v|, zero vector -> u = 0):
//   l=0: 1
//   l=1: sqrt3 (x, y, z)
//   l=2: sqrt15 xy, sqrt15 yz, sqrt5/2 (2z^2-x^2-y^2), sqrt15 xz, sqrt15/2 (x^2-y^2)
//   l=3: a y(3x^2-y^2), b xyz, c y(4z^2-x^2-y^2), sqrt7/2 z(2z^2-3x^2-3y^2),
//        c x(4z^2-x^2-y^2), b/2 z(x^2-y^2), a x(x^2-3y^2)
//   with a = sqrt(35/8), b = sqrt(105), c = sqrt(21/8).

#include "common.h"

namespace mnx {
namespace {

constexpr float S3 = 1.7320508075688772f;
constexpr float S5 = 2.23606797749979f;
constexpr float S7 = 2.6457513110645907f;
constexpr float S15 = 3.872983346207417f;
constexpr float A3 = 2.091650066335189f;   // sqrt(35/8)
constexpr float B3 = 10.246950765959598f;  // sqrt(105)
constexpr float C3 = 1.620185174601965f;   // sqrt(21/8)

__device__ __forceinline__ void unit(float vx, float vy, float vz, float& x, float& y, float& z, float& inv_r) {
    const float r = sqrtf(vx * vx + vy * vy + vz * vz);
    inv_r = r > 0.f ? 1.f / r : 0.f;
    x = vx * inv_r;
    y = vy * inv_r;
    z = vz * inv_r;
}

template <int LMAX>
__global__ void k_sh_fwd(const float* __restrict__ v, int64_t n, float* __restrict__ out) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float x, y, z, ir;
    unit(v[3 * i], v[3 * i + 1], v[3 * i + 2], x, y, z, ir);
    constexpr int D = (LMAX + 1) * (LMAX + 1);
    float Y[D];
    Y[0] = 1.f;
    if (LMAX >= 1) {
        Y[1] = S3 * x;
        Y[2] = S3 * y;
        Y[3] = S3 * z;
    }
    if (LMAX >= 2) {
        Y[4] = S15 * x * y;
        Y[5] = S15 * y * z;
        Y[6] = 0.5f * S5 * (2.f * z * z - x * x - y * y);
        Y[7] = S15 * x * z;
        Y[8] = 0.5f * S15 * (x * x - y * y);
    }
    if (LMAX >= 3) {
        const float x2 = x * x, y2 = y * y, z2 = z * z;
        Y[9] = A3 * y * (3.f * x2 - y2);
        Y[10] = B3 * x * y * z;
        Y[11] = C3 * y * (4.f * z2 - x2 - y2);
        Y[12] = 0.5f * S7 * z * (2.f * z2 - 3.f * x2 - 3.f * y2);
        Y[13] = C3 * x * (4.f * z2 - x2 - y2);
        Y[14] = 0.5f * B3 * z * (x2 - y2);
        Y[15] = A3 * x * (x2 - 3.f * y2);
    }
    float* o = out + i * D;
#pragma unroll
    for (int k = 0; k < D; ++k) o[k] = Y[k];
}

template <int LMAX>
__global__ void k_sh_bwd(const float* __restrict__ v, const float* __restrict__ go, int64_t n,
                         float* __restrict__ gv) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float x, y, z, ir;
    unit(v[3 * i], v[3 * i + 1], v[3 * i + 2], x, y, z, ir);
    constexpr int D = (LMAX + 1) * (LMAX + 1);
    const float* g = go + i * D;
    // gradient of sum_k g_k Y_k(u) with respect to u (Y as homogeneous polynomials)
    float gx = 0.f, gy = 0.f, gz = 0.f;
    if (LMAX >= 1) {
        gx += S3 * g[1];
        gy += S3 * g[2];
        gz += S3 * g[3];
    }
    if (LMAX >= 2) {
        const float g4 = g[4], g5 = g[5], g6 = g[6], g7 = g[7], g8 = g[8];
        gx += S15 * (y * g4 + z * g7 + x * g8) - S5 * x * g6;
        gy += S15 * (x * g4 + z * g5 - y * g8) - S5 * y * g6;
        gz += S15 * (y * g5 + x * g7) + 2.f * S5 * z * g6;
    }
    if (LMAX >= 3) {
        const float x2 = x * x, y2 = y * y, z2 = z * z;
        const float g9 = g[9], g10 = g[10], g11 = g[11], g12 = g[12], g13 = g[13], g14 = g[14], g15 = g[15];
        gx += A3 * 6.f * x * y * g9 + B3 * y * z * g10 - 2.f * C3 * x * y * g11 - 3.f * S7 * x * z * g12 +
              C3 * (4.f * z2 - 3.f * x2 - y2) * g13 + B3 * x * z * g14 + A3 * 3.f * (x2 - y2) * g15;
        gy += A3 * 3.f * (x2 - y2) * g9 + B3 * x * z * g10 + C3 * (4.f * z2 - x2 - 3.f * y2) * g11 -
              3.f * S7 * y * z * g12 - 2.f * C3 * x * y * g13 - B3 * y * z * g14 - A3 * 6.f * x * y * g15;
        gz += B3 * x * y * g10 + 8.f * C3 * y * z * g11 + 0.5f * S7 * (6.f * z2 - 3.f * x2 - 3.f * y2) * g12 +
              8.f * C3 * x * z * g13 + 0.5f * B3 * (x2 - y2) * g14;
    }
    // chain rule through u = v/|v|: dv = (g_u - u (u . g_u)) / |v|
    const float ug = x * gx + y * gy + z * gz;
    gv[3 * i + 0] = (gx - x * ug) * ir;
    gv[3 * i + 1] = (gy - y * ug) * ir;
    gv[3 * i + 2] = (gz - z * ug) * ir;
}

template <template <int> class K, typename... A>
int launch_l(int lmax, int64_t n, hipStream_t s, A... args) {
    const int tb = 256;
    const dim3 grid(unsigned(ceil_div(n, tb)));
    switch (lmax) {
        case 0: hipLaunchKernelGGL(K<0>::fn, grid, dim3(tb), 0, s, args...); break;
        case 1: hipLaunchKernelGGL(K<1>::fn, grid, dim3(tb), 0, s, args...); break;
        case 2: hipLaunchKernelGGL(K<2>::fn, grid, dim3(tb), 0, s, args...); break;
        case 3: hipLaunchKernelGGL(K<3>::fn, grid, dim3(tb), 0, s, args...); break;
        default: return set_error(MNX_ERR_UNSUPPORTED, "l_max=%d not supported (<= 3)", lmax);
    }
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

template <int L>
struct Fwd {
    static constexpr auto fn = k_sh_fwd<L>;
};
template <int L>
struct Bwd {
    static constexpr auto fn = k_sh_bwd<L>;
};

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

int mnx_sh_fwd_f32(const float* vec, int64_t n, int32_t l_max, float* out, mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(n >= 0, "n must be >= 0");
    if (n == 0) return MNX_OK;
    MNX_REQUIRE(vec && out, "null pointer argument");
    return launch_l<Fwd>(l_max, n, (hipStream_t)stream, vec, n, out);
}

int mnx_sh_bwd_f32(const float* vec, const float* grad_out, int64_t n, int32_t l_max, float* grad_vec,
                   mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(n >= 0, "n must be >= 0");
    if (n == 0) return MNX_OK;
    MNX_REQUIRE(vec && grad_out && grad_vec, "null pointer argument");
    return launch_l<Bwd>(l_max, n, (hipStream_t)stream, vec, grad_out, n, grad_vec);
}

}  // extern "C"
