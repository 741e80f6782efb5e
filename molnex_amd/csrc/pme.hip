// Particle-mesh Ewald on gfx950: B-spline charge spreading, reciprocal-space
// convolution with the energy sum, force / charge-derivative gathering, and the
// real-space pair sum.  The 3-D FFTs between spread and convolve (forward) and
// between convolve and gather (backward) are rocFFT transforms issued by the
// caller on the same stream (torch.fft on ROCm).
//
// Follows the reference's CPU op (src/molix/op/src/pme/pme_cpu.cpp) term by
// term: box inversion (:22-35), grid index and B-spline recursion (:37-91),
// spreading (:240-256), influence function and energy (:263-294), gather
// (:311-343), direct sum with exclusions (:95-164).  The reference's CUDA path
// (pme_cuda.cu:394,460) supports spline orders 4 and 5; these kernels take any
// order 3..8.  Accumulations into the grid and per-atom derivatives use fp32 /
// fp64 atomics; energies are reduced deterministically in fp64.

#include <math.h>

#include "common.h"

namespace mnx {
namespace {

constexpr int kMaxOrder = 8;

template <typename T>
struct Recip {
    T r[3][3];
};

template <typename T>
__device__ __forceinline__ Recip<T> invert_box(const T* __restrict__ b) {
    Recip<T> R;
    const T s = T(1) / (b[0] * b[4] * b[8]);
    R.r[0][0] = b[4] * b[8] * s;
    R.r[0][1] = 0;
    R.r[0][2] = 0;
    R.r[1][0] = -b[3] * b[8] * s;
    R.r[1][1] = b[0] * b[8] * s;
    R.r[1][2] = 0;
    R.r[2][0] = (b[3] * b[7] - b[4] * b[6]) * s;
    R.r[2][1] = -b[0] * b[7] * s;
    R.r[2][2] = b[0] * b[4] * s;
    return R;
}

// Grid origin and B-spline weights (and derivatives when dd != nullptr) of one atom.
template <typename T>
__device__ __forceinline__ void spline(const T* __restrict__ pos, int64_t atom, const T* __restrict__ box,
                                       const Recip<T>& R, const int grid[3], int order, int gidx[3],
                                       T (&d)[kMaxOrder][3], T (*dd)[3]) {
    T p[3] = {pos[3 * atom], pos[3 * atom + 1], pos[3 * atom + 2]};
    for (int i = 2; i >= 0; --i) {
        const T sc = floor(p[i] * R.r[i][i]);
        for (int j = 0; j < 3; ++j) p[j] -= sc * box[3 * i + j];
    }
    for (int i = 0; i < 3; ++i) {
        T t = p[0] * R.r[0][i] + p[1] * R.r[1][i] + p[2] * R.r[2][i];
        t = (t - floor(t)) * grid[i];
        const int ti = int(t);
        const T dr = t - ti;
        gidx[i] = ti % grid[i];
        d[order - 1][i] = 0;
        d[1][i] = dr;
        d[0][i] = 1 - dr;
        for (int j = 3; j < order; ++j) {
            const T div = T(1) / (j - 1);
            d[j - 1][i] = div * dr * d[j - 2][i];
            for (int k = 1; k < j - 1; ++k)
                d[j - k - 1][i] = div * ((dr + k) * d[j - k - 2][i] + (j - k - dr) * d[j - k - 1][i]);
            d[0][i] = div * (1 - dr) * d[0][i];
        }
        if (dd) {
            dd[0][i] = -d[0][i];
            for (int j = 1; j < order; ++j) dd[j][i] = d[j - 1][i] - d[j][i];
        }
        const T sc = T(1) / (order - 1);
        d[order - 1][i] = sc * dr * d[order - 2][i];
        for (int j = 1; j < order - 1; ++j)
            d[order - j - 1][i] = sc * ((dr + j) * d[order - j - 2][i] + (order - j - dr) * d[order - j - 1][i]);
        d[0][i] = sc * (1 - dr) * d[0][i];
    }
}

// One wavefront lane per (atom, ix); each lane spreads its order^2 (iy, iz) points.
template <typename T>
__global__ void k_spread(const T* __restrict__ pos, const T* __restrict__ q, const T* __restrict__ box, int64_t n,
                         int gx, int gy, int gz, int order, T sqrt_k, T* __restrict__ grid) {
    const int64_t tid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t atom = tid / order;
    const int ix = int(tid - atom * order);
    if (atom >= n) return;
    const int G[3] = {gx, gy, gz};
    const Recip<T> R = invert_box<T>(box);
    int gi[3];
    T d[kMaxOrder][3];
    spline<T>(pos, atom, box, R, G, order, gi, d, nullptr);
    const int x = (gi[0] + ix) % gx;
    const T wx = q[atom] * sqrt_k * d[ix][0];
    T* __restrict__ plane = grid + int64_t(x) * gy * gz;
    for (int iy = 0; iy < order; ++iy) {
        const int y = (gi[1] + iy) % gy;
        const T wxy = wx * d[iy][1];
        T* __restrict__ row = plane + int64_t(y) * gz;
        for (int iz = 0; iz < order; ++iz) atomicAdd(row + (gi[2] + iz) % gz, wxy * d[iz][2]);
    }
}

constexpr int kConvThreads = 256;

// In-place multiply of the half-spectrum grid by the influence function and the
// per-block energy partial sums (pme_cpu.cpp:263-294).
template <typename T>
__global__ void __launch_bounds__(kConvThreads) k_convolve(T* __restrict__ cgrid, const T* __restrict__ box, int gx,
                                                           int gy, int gz, T alpha, const T* __restrict__ xm,
                                                           const T* __restrict__ ym, const T* __restrict__ zm,
                                                           double* __restrict__ partials) {
    __shared__ double red[kConvThreads];
    const int zs = gz / 2 + 1;
    const int64_t total = int64_t(gx) * gy * zs;
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    double e = 0.0;
    if (idx < total) {
        const Recip<T> R = invert_box<T>(box);
        const int kx = int(idx / (int64_t(gy) * zs));
        const int rem = int(idx - int64_t(kx) * gy * zs);
        const int ky = rem / zs;
        const int kz = rem - ky * zs;
        const int mx = kx < (gx + 1) / 2 ? kx : kx - gx;
        const int my = ky < (gy + 1) / 2 ? ky : ky - gy;
        const int mz = kz < (gz + 1) / 2 ? kz : kz - gz;
        const T mhx = mx * R.r[0][0];
        const T mhy = mx * R.r[1][0] + my * R.r[1][1];
        const T mhz = mx * R.r[2][0] + my * R.r[2][1] + mz * R.r[2][2];
        const T m2 = mhx * mhx + mhy * mhy + mhz * mhz;
        const T scale_f = T(M_PI) * box[0] * box[4] * box[8];
        const T denom = m2 * (scale_f * xm[kx] * ym[ky]) * zm[kz];
        const T rexp = T(M_PI * M_PI) / (alpha * alpha);
        const T eterm = idx == 0 ? T(0) : exp(-rexp * m2) / denom;
        const T s = (kz > 0 && kz <= (gz - 1) / 2) ? T(2) : T(1);
        T* c = cgrid + 2 * idx;
        const T re = c[0], im = c[1];
        e = double(s * eterm * (re * re + im * im));
        c[0] = re * eterm;
        c[1] = im * eterm;
    }
    red[threadIdx.x] = e;
    __syncthreads();
    for (int off = kConvThreads / 2; off > 0; off >>= 1) {
        if (threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
        __syncthreads();
    }
    if (threadIdx.x == 0) partials[blockIdx.x] = red[0];
}

// energy = scale * sum(partials), summed by one block in a fixed order.
template <typename T>
__global__ void __launch_bounds__(1024) k_sum_partials(const double* __restrict__ partials, int64_t n, double scale,
                                                       T* __restrict__ energy) {
    __shared__ double red[1024];
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += 1024) s += partials[i];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int off = 512; off > 0; off >>= 1) {
        if (threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
        __syncthreads();
    }
    if (threadIdx.x == 0) *energy = T(scale * red[0]);
}

// d/dpos and d/dq of the reciprocal energy from the back-transformed grid (pme_cpu.cpp:311-343).
template <typename T>
__global__ void k_gather(const T* __restrict__ pos, const T* __restrict__ q, const T* __restrict__ box, int64_t n,
                         const T* __restrict__ grid, int gx, int gy, int gz, int order, T sqrt_k,
                         T* __restrict__ dpos, T* __restrict__ dq) {
    const int64_t atom = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (atom >= n) return;
    const int G[3] = {gx, gy, gz};
    const Recip<T> R = invert_box<T>(box);
    int gi[3];
    T d[kMaxOrder][3], dd[kMaxOrder][3];
    spline<T>(pos, atom, box, R, G, order, gi, d, dd);
    T p0 = 0, p1 = 0, p2 = 0, s = 0;
    for (int ix = 0; ix < order; ++ix) {
        const int x = (gi[0] + ix) % gx;
        for (int iy = 0; iy < order; ++iy) {
            const int y = (gi[1] + iy) % gy;
            const T* row = grid + (int64_t(x) * gy + y) * gz;
            const T dxy = d[ix][0] * d[iy][1], dxdy = dd[ix][0] * d[iy][1], xdy = d[ix][0] * dd[iy][1];
            for (int iz = 0; iz < order; ++iz) {
                const T g = row[(gi[2] + iz) % gz];
                p0 += dxdy * d[iz][2] * g;
                p1 += xdy * d[iz][2] * g;
                p2 += dxy * dd[iz][2] * g;
                s += dxy * d[iz][2] * g;
            }
        }
    }
    const T sc = q[atom] * sqrt_k;
    dpos[3 * atom + 0] = sc * (p0 * gx * R.r[0][0]);
    dpos[3 * atom + 1] = sc * (p0 * gx * R.r[1][0] + p1 * gy * R.r[1][1]);
    dpos[3 * atom + 2] = sc * (p0 * gx * R.r[2][0] + p1 * gy * R.r[2][1] + p2 * gz * R.r[2][2]);
    dq[atom] = s * sqrt_k;
}

// Real-space pair sum over the given pair list minus excluded pairs (pme_cpu.cpp:110-135).
template <typename T>
__global__ void __launch_bounds__(kConvThreads) k_direct_pairs(const T* __restrict__ q, int64_t n,
                                                               const int32_t* __restrict__ nb, int64_t P, const T* __restrict__ dl,
                                                               const T* __restrict__ r, const int32_t* __restrict__ excl,
                                                               int max_excl, T alpha, T coulomb,
                                                               T* __restrict__ dpos, T* __restrict__ dq,
                                                               double* __restrict__ partials) {
    __shared__ double red[kConvThreads];
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    double e = 0.0;
    if (i < P) {
        const int a1 = nb[i], a2 = nb[P + i];
        // -1 marks padding (reference); any other out-of-range index is skipped too
        bool include = a1 > -1 && a1 < n && a2 >= 0 && a2 < n;
        for (int j = 0; include && j < max_excl && excl[int64_t(a1) * max_excl + j] >= a2; ++j)
            if (excl[int64_t(a1) * max_excl + j] == a2) include = false;
        if (include) {
            const T rr = r[i];
            const T inv = T(1) / rr;
            const T ar = alpha * rr;
            const T ex = exp(-ar * ar);
            const T ec = erfc(ar);
            const T pref = coulomb * inv;
            const T c1 = q[a1], c2 = q[a2];
            e = double(pref * ec * c1 * c2);
            atomicAdd(dq + a1, pref * ec * c2);
            atomicAdd(dq + a2, pref * ec * c1);
            const T dedr = pref * c1 * c2 * (ec + ar * ex * T(M_2_SQRTPI)) * inv * inv;
            for (int k = 0; k < 3; ++k) {
                atomicAdd(dpos + 3 * a1 + k, -dedr * dl[3 * i + k]);
                atomicAdd(dpos + 3 * a2 + k, dedr * dl[3 * i + k]);
            }
        }
    }
    red[threadIdx.x] = e;
    __syncthreads();
    for (int off = kConvThreads / 2; off > 0; off >>= 1) {
        if (threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
        __syncthreads();
    }
    if (threadIdx.x == 0) partials[blockIdx.x] = red[0];
}

// Excluded pairs' erf term, removed from the reciprocal-space sum (pme_cpu.cpp:137-162).
template <typename T>
__global__ void __launch_bounds__(kConvThreads) k_direct_excl(const T* __restrict__ pos, const T* __restrict__ q,
                                                              int64_t n, const int32_t* __restrict__ excl,
                                                              int max_excl, T alpha, T coulomb,
                                                              T* __restrict__ dpos, T* __restrict__ dq,
                                                              double* __restrict__ partials) {
    __shared__ double red[kConvThreads];
    const int64_t a = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    double e = 0.0;
    if (a < n) {
        for (int j = 0; j < max_excl; ++j) {
            const int b = excl[a * max_excl + j];
            if (!(b > a)) break;
            if (b >= n) continue;
            T dr[3];
            for (int k = 0; k < 3; ++k) dr[k] = pos[3 * a + k] - pos[3 * int64_t(b) + k];
            const T rr = sqrt(dr[0] * dr[0] + dr[1] * dr[1] + dr[2] * dr[2]);
            const T inv = T(1) / rr;
            const T ar = alpha * rr;
            const T ex = exp(-ar * ar);
            const T ef = erf(ar);
            const T pref = coulomb * inv;
            const T c1 = q[a], c2 = q[b];
            e -= double(pref * ef * c1 * c2);
            atomicAdd(dq + a, -pref * ef * c2);
            atomicAdd(dq + b, -pref * ef * c1);
            const T dedr = pref * c1 * c2 * (ef - ar * ex * T(M_2_SQRTPI)) * inv * inv;
            for (int k = 0; k < 3; ++k) {
                atomicAdd(dpos + 3 * a + k, dedr * dr[k]);
                atomicAdd(dpos + 3 * int64_t(b) + k, -dedr * dr[k]);
            }
        }
    }
    red[threadIdx.x] = e;
    __syncthreads();
    for (int off = kConvThreads / 2; off > 0; off >>= 1) {
        if (threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
        __syncthreads();
    }
    if (threadIdx.x == 0) partials[blockIdx.x] = red[0];
}

int check_grid(int gx, int gy, int gz, int order) {
    MNX_REQUIRE(gx > 0 && gy > 0 && gz > 0 && int64_t(gx) * gy * gz < (int64_t(1) << 31), "bad grid size");
    MNX_REQUIRE(order >= 3 && order <= kMaxOrder, "spline order %d not in [3, %d]", order, kMaxOrder);
    MNX_REQUIRE(gx >= order && gy >= order && gz >= order, "grid smaller than the spline order");
    return MNX_OK;
}

template <typename T>
int spread(const T* pos, const T* q, const T* box, int64_t n, int gx, int gy, int gz, int order, double coulomb,
           T* grid, hipStream_t s) {
    clear_error();
    int rc = check_grid(gx, gy, gz, order);
    if (rc) return rc;
    MNX_REQUIRE(grid && box && (n == 0 || (pos && q)), "null pointer argument");
    MNX_HIP_TRY(hipMemsetAsync(grid, 0, sizeof(T) * size_t(gx) * gy * gz, s));
    if (n == 0) return MNX_OK;
    const int64_t threads = n * order;
    hipLaunchKernelGGL((k_spread<T>), dim3(ceil_div(threads, 256)), dim3(256), 0, s, pos, q, box, n, gx, gy, gz,
                       order, T(sqrt(coulomb)), grid);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int64_t conv_blocks(int gx, int gy, int gz) { return ceil_div(int64_t(gx) * gy * (gz / 2 + 1), kConvThreads); }

template <typename T>
int convolve(T* cgrid, const T* box, int gx, int gy, int gz, double alpha, const T* xm, const T* ym, const T* zm,
             T* energy, void* ws, size_t ws_bytes, hipStream_t s) {
    clear_error();
    int rc = check_grid(gx, gy, gz, 3);
    if (rc) return rc;
    MNX_REQUIRE(cgrid && box && xm && ym && zm && energy, "null pointer argument");
    const int64_t nb = conv_blocks(gx, gy, gz);
    if (!ws || ws_bytes < size_t(nb) * sizeof(double))
        return set_error(MNX_ERR_WORKSPACE, "workspace %zu < %zu bytes", ws_bytes, size_t(nb) * sizeof(double));
    double* part = static_cast<double*>(ws);
    hipLaunchKernelGGL((k_convolve<T>), dim3(nb), dim3(kConvThreads), 0, s, cgrid, box, gx, gy, gz, T(alpha), xm, ym,
                       zm, part);
    MNX_CHECK_LAUNCH();
    hipLaunchKernelGGL((k_sum_partials<T>), dim3(1), dim3(1024), 0, s, part, nb, 0.5, energy);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

template <typename T>
int gather(const T* pos, const T* q, const T* box, int64_t n, const T* grid, int gx, int gy, int gz, int order,
           double coulomb, T* dpos, T* dq, hipStream_t s) {
    clear_error();
    int rc = check_grid(gx, gy, gz, order);
    if (rc) return rc;
    if (n == 0) return MNX_OK;
    MNX_REQUIRE(pos && q && box && grid && dpos && dq, "null pointer argument");
    hipLaunchKernelGGL((k_gather<T>), dim3(ceil_div(n, 128)), dim3(128), 0, s, pos, q, box, n, grid, gx, gy, gz, order,
                       T(sqrt(coulomb)), dpos, dq);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

size_t direct_ws(int64_t n, int64_t P) { return size_t(ceil_div(P > 0 ? P : 1, kConvThreads) + ceil_div(n > 0 ? n : 1, kConvThreads)) * sizeof(double); }

template <typename T>
int direct(const T* pos, const T* q, int64_t n, const int32_t* nb, int64_t P, const T* deltas, const T* dist,
           const int32_t* excl, int max_excl, double alpha, double coulomb, T* energy, T* dpos, T* dq, void* ws,
           size_t ws_bytes, hipStream_t s) {
    clear_error();
    MNX_REQUIRE(n >= 0 && P >= 0 && max_excl >= 0, "sizes out of range");
    MNX_REQUIRE(energy && (n == 0 || (pos && q && dpos && dq)), "null pointer argument");
    MNX_REQUIRE(max_excl == 0 || excl, "exclusions pointer is null");
    if (!ws || ws_bytes < direct_ws(n, P)) return set_error(MNX_ERR_WORKSPACE, "workspace too small");
    double* part = static_cast<double*>(ws);
    const int64_t b1 = ceil_div(P > 0 ? P : 1, kConvThreads), b2 = ceil_div(n > 0 ? n : 1, kConvThreads);
    MNX_HIP_TRY(hipMemsetAsync(part, 0, sizeof(double) * (b1 + b2), s));
    if (n > 0) {
        MNX_HIP_TRY(hipMemsetAsync(dpos, 0, sizeof(T) * 3 * n, s));
        MNX_HIP_TRY(hipMemsetAsync(dq, 0, sizeof(T) * n, s));
    }
    if (P > 0) {
        hipLaunchKernelGGL((k_direct_pairs<T>), dim3(b1), dim3(kConvThreads), 0, s, q, n, nb, P, deltas, dist, excl,
                           max_excl, T(alpha), T(coulomb), dpos, dq, part);
        MNX_CHECK_LAUNCH();
    }
    if (n > 0 && max_excl > 0) {
        hipLaunchKernelGGL((k_direct_excl<T>), dim3(b2), dim3(kConvThreads), 0, s, pos, q, n, excl, max_excl,
                           T(alpha), T(coulomb), dpos, dq, part + b1);
        MNX_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL((k_sum_partials<T>), dim3(1), dim3(1024), 0, s, part, b1 + b2, 1.0, energy);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

int mnx_pme_spread_f32(const float* pos, const float* q, const float* box, int64_t n, int32_t gx, int32_t gy,
                       int32_t gz, int32_t order, double coulomb, float* grid, mnx_stream_t s) {
    return spread<float>(pos, q, box, n, gx, gy, gz, order, coulomb, grid, (hipStream_t)s);
}
int mnx_pme_spread_f64(const double* pos, const double* q, const double* box, int64_t n, int32_t gx, int32_t gy,
                       int32_t gz, int32_t order, double coulomb, double* grid, mnx_stream_t s) {
    return spread<double>(pos, q, box, n, gx, gy, gz, order, coulomb, grid, (hipStream_t)s);
}
size_t mnx_pme_convolve_workspace_bytes(int32_t gx, int32_t gy, int32_t gz) {
    return size_t(conv_blocks(gx, gy, gz)) * sizeof(double) + 256;
}
int mnx_pme_convolve_f32(float* cgrid, const float* box, int32_t gx, int32_t gy, int32_t gz, double alpha,
                         const float* xm, const float* ym, const float* zm, float* energy, void* ws, size_t ws_bytes,
                         mnx_stream_t s) {
    return convolve<float>(cgrid, box, gx, gy, gz, alpha, xm, ym, zm, energy, ws, ws_bytes, (hipStream_t)s);
}
int mnx_pme_convolve_f64(double* cgrid, const double* box, int32_t gx, int32_t gy, int32_t gz, double alpha,
                         const double* xm, const double* ym, const double* zm, double* energy, void* ws,
                         size_t ws_bytes, mnx_stream_t s) {
    return convolve<double>(cgrid, box, gx, gy, gz, alpha, xm, ym, zm, energy, ws, ws_bytes, (hipStream_t)s);
}
int mnx_pme_gather_f32(const float* pos, const float* q, const float* box, int64_t n, const float* grid, int32_t gx,
                       int32_t gy, int32_t gz, int32_t order, double coulomb, float* dpos, float* dq, mnx_stream_t s) {
    return gather<float>(pos, q, box, n, grid, gx, gy, gz, order, coulomb, dpos, dq, (hipStream_t)s);
}
int mnx_pme_gather_f64(const double* pos, const double* q, const double* box, int64_t n, const double* grid,
                       int32_t gx, int32_t gy, int32_t gz, int32_t order, double coulomb, double* dpos, double* dq,
                       mnx_stream_t s) {
    return gather<double>(pos, q, box, n, grid, gx, gy, gz, order, coulomb, dpos, dq, (hipStream_t)s);
}
size_t mnx_pme_direct_workspace_bytes(int64_t n, int64_t num_pairs) { return direct_ws(n, num_pairs) + 256; }
int mnx_pme_direct_f32(const float* pos, const float* q, int64_t n, const int32_t* neighbors, int64_t num_pairs,
                       const float* deltas, const float* distances, const int32_t* exclusions, int32_t max_excl,
                       double alpha, double coulomb, float* energy, float* dpos, float* dq, void* ws,
                       size_t ws_bytes, mnx_stream_t s) {
    return direct<float>(pos, q, n, neighbors, num_pairs, deltas, distances, exclusions, max_excl, alpha, coulomb,
                         energy, dpos, dq, ws, ws_bytes, (hipStream_t)s);
}
int mnx_pme_direct_f64(const double* pos, const double* q, int64_t n, const int32_t* neighbors, int64_t num_pairs,
                       const double* deltas, const double* distances, const int32_t* exclusions, int32_t max_excl,
                       double alpha, double coulomb, double* energy, double* dpos, double* dq, void* ws,
                       size_t ws_bytes, mnx_stream_t s) {
    return direct<double>(pos, q, n, neighbors, num_pairs, deltas, distances, exclusions, max_excl, alpha, coulomb,
                          energy, dpos, dq, ws, ws_bytes, (hipStream_t)s);
}

}  // extern "C"
