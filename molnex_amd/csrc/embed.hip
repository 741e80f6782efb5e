// Radial edge embedding: the Bessel basis times the cutoff envelope,
//   f[e][k] = c(r_e) * (phi_k(r_e) - mu_k) / sigma_k,
//   phi_k(r) = sqrt(2 / r_cut) sin(k pi r / r_cut) / (r + eps),   k = 1 .. n,
// with c the cosine envelope 0.5 (cos(pi r / r_cut) + 1) or the polynomial one
// u(x) = (1 - x)^3 sum_{j<p} C(j+2, 2) x^j, x = r / r_cut (both 0 for r >= r_cut),
// as MACE combines them (src/molrep/embedding/radial.py:36-148,
// src/molrep/embedding/cutoff.py:23-161, src/molzoo/mace.py:180-182).  One
// thread per edge: r is read once, the n values are written as one row; the
// backward reads the row's gradient and writes dL/dr (basis terms in fp64).  The torch composition
// this replaces makes ~20 passes over the (E, n) values forward and backward.

#include "common.h"

namespace mnx {
namespace {

constexpr int kEmbThreads = 256;
constexpr int kEmbMaxRadial = 32;

struct EmbArgs {
    int n;
    float r_cut, eps, pref, w;  // pref = sqrt(2 / r_cut), w = pi / r_cut (rounded once, as the reference's buffers)
    int cutoff;    // 0 none, 1 cosine, 2 polynomial
    int exponent;  // polynomial envelope
    const float* mu;     // [n] or null (no shift / scale)
    const float* sigma;  // [n] or null
};

// envelope and its derivative with respect to r
__device__ __forceinline__ void envelope(float r, const EmbArgs& a, float& c, float& dc) {
    if (a.cutoff == 0) {
        c = 1.f;
        dc = 0.f;
        return;
    }
    if (!(r < a.r_cut)) {
        c = 0.f;
        dc = 0.f;
        return;
    }
    if (a.cutoff == 1) {
        float s, co;
        sincosf(float(M_PI) * (r / a.r_cut), &s, &co);
        c = 0.5f * (co + 1.f);
        dc = -0.5f * float(M_PI) / a.r_cut * s;
        return;
    }
    const float x = r / a.r_cut;
    const int p = a.exponent;
    // g(x) = sum_{j<p} C(j+2, 2) x^j and g'(x), Horner, highest coefficient first
    float g = float((p + 1) * p / 2), gp = 0.f;
    for (int j = p - 2; j >= 0; --j) {
        gp = fmaf(gp, x, g);
        g = fmaf(g, x, float((j + 2) * (j + 1) / 2));
    }
    const float om = 1.f - x;
    const float om2 = om * om;
    c = om2 * om * g;
    dc = (om2 * om * gp - 3.f * om2 * g) / a.r_cut;
}

__global__ void __launch_bounds__(kEmbThreads) k_bessel_cutoff(const float* __restrict__ r, int64_t E, EmbArgs a,
                                                               float* __restrict__ out) {
    const int64_t e = int64_t(blockIdx.x) * kEmbThreads + threadIdx.x;
    if (e >= E) return;
    const float re = r[e];
    float c, dc;
    envelope(re, a, c, dc);
    const float inv = 1.f / (re + a.eps);
    float* o = out + e * a.n;
    for (int k = 0; k < a.n; ++k) {
        float phi = a.pref * sinf(re * (float(k + 1) * a.w)) * inv;
        if (a.mu) phi = (phi - a.mu[k]) / a.sigma[k];
        o[k] = phi * c;
    }
}

__global__ void __launch_bounds__(kEmbThreads) k_bessel_cutoff_bwd(const float* __restrict__ r, int64_t E, EmbArgs a,
                                                                   const float* __restrict__ grad,
                                                                   float* __restrict__ grad_r) {
    const int64_t e = int64_t(blockIdx.x) * kEmbThreads + threadIdx.x;
    if (e >= E) return;
    const float re = r[e];
    float c, dc;
    envelope(re, a, c, dc);
    // d/dr [pref sin(f r) / (r + eps)] = pref (f cos(f r) - sin(f r) / (r + eps)) / (r + eps): the two
    // terms cancel to ~(f r)^2 / 3 of their size for small f r (about 1e-5 at r = 1e-3 A), so the
    // basis and its derivative are evaluated in fp64 here (one thread per edge, n terms)
    const double rd = double(re), inv = 1.0 / (rd + double(a.eps));
    const float* g = grad + e * a.n;
    double acc = 0.0;
    for (int k = 0; k < a.n; ++k) {
        const double f = double(float(k + 1) * a.w);
        double s, co;
        sincos(rd * f, &s, &co);
        double phi = double(a.pref) * s * inv;
        double dphi = double(a.pref) * (f * co - s * inv) * inv;
        if (a.mu) {
            phi = (phi - double(a.mu[k])) / double(a.sigma[k]);
            dphi = dphi / double(a.sigma[k]);
        }
        acc += double(g[k]) * (dphi * double(c) + phi * double(dc));
    }
    grad_r[e] = float(acc);
}

int check_args(int64_t E, int n, double r_cut, double eps, int cutoff, int exponent, const float* mu,
               const float* sigma) {
    MNX_REQUIRE(E >= 0 && E < (int64_t(1) << 40), "edge count out of range");
    MNX_REQUIRE(n >= 1 && n <= kEmbMaxRadial, "num_radial %d not in [1, %d]", n, kEmbMaxRadial);
    MNX_REQUIRE(r_cut > 0.0 && eps >= 0.0, "r_cut must be positive and eps non-negative");
    MNX_REQUIRE(cutoff >= 0 && cutoff <= 2, "cutoff kind %d not in {0 none, 1 cosine, 2 polynomial}", cutoff);
    MNX_REQUIRE(cutoff != 2 || (exponent >= 1 && exponent <= 64), "polynomial exponent %d not in [1, 64]", exponent);
    MNX_REQUIRE((mu == nullptr) == (sigma == nullptr), "mu and sigma must both be given or both be null");
    return MNX_OK;
}

EmbArgs make_args(int n, double r_cut, double eps, int cutoff, int exponent, const float* mu, const float* sigma) {
    return EmbArgs{n, float(r_cut), float(eps), float(sqrt(2.0 / r_cut)), float(M_PI / r_cut), cutoff, exponent, mu,
                   sigma};
}

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

int mnx_bessel_cutoff_f32(const float* r, int64_t num_edges, int32_t num_radial, double r_cut, double eps,
                          const float* mu, const float* sigma, int32_t cutoff, int32_t exponent, float* out,
                          mnx_stream_t stream) {
    clear_error();
    int rc = check_args(num_edges, num_radial, r_cut, eps, cutoff, exponent, mu, sigma);
    if (rc) return rc;
    if (num_edges == 0) return MNX_OK;
    MNX_REQUIRE(r && out, "null pointer argument");
    hipLaunchKernelGGL(k_bessel_cutoff, dim3(unsigned(ceil_div(num_edges, kEmbThreads))), dim3(kEmbThreads), 0,
                       (hipStream_t)stream, r, num_edges,
                       make_args(num_radial, r_cut, eps, cutoff, exponent, mu, sigma), out);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_bessel_cutoff_bwd_f32(const float* r, int64_t num_edges, int32_t num_radial, double r_cut, double eps,
                              const float* mu, const float* sigma, int32_t cutoff, int32_t exponent,
                              const float* grad, float* grad_r, mnx_stream_t stream) {
    clear_error();
    int rc = check_args(num_edges, num_radial, r_cut, eps, cutoff, exponent, mu, sigma);
    if (rc) return rc;
    if (num_edges == 0) return MNX_OK;
    MNX_REQUIRE(r && grad && grad_r, "null pointer argument");
    hipLaunchKernelGGL(k_bessel_cutoff_bwd, dim3(unsigned(ceil_div(num_edges, kEmbThreads))), dim3(kEmbThreads), 0,
                       (hipStream_t)stream, r, num_edges,
                       make_args(num_radial, r_cut, eps, cutoff, exponent, mu, sigma), grad, grad_r);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

}  // extern "C"
