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
// order 3..8.  The spread is a gather over mesh bricks (no atomics, fixed
// summation order); the direct-space derivatives use fp32 / fp64 atomics, and
// energies are reduced deterministically in fp64.

#include <math.h>

#include "common.h"
#include "scan.h"
#include "wave.h"

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

// Grid origin index and fractional offset of one atom along each axis (pme_cpu.cpp:37-60).
// The index is clamped into [0, grid) so that a non-finite position cannot address
// memory outside the mesh (its weights are then non-finite, as in the reference).
template <typename T>
__device__ __forceinline__ void grid_coord(const T* __restrict__ pos, int64_t atom, const T* __restrict__ box,
                                           const Recip<T>& R, const int grid[3], int gidx[3], T frac[3]) {
    T p[3] = {pos[3 * atom], pos[3 * atom + 1], pos[3 * atom + 2]};
    for (int i = 2; i >= 0; --i) {
        const T sc = floor(p[i] * R.r[i][i]);
        for (int j = 0; j < 3; ++j) p[j] -= sc * box[3 * i + j];
    }
    for (int i = 0; i < 3; ++i) {
        T t = p[0] * R.r[0][i] + p[1] * R.r[1][i] + p[2] * R.r[2][i];
        t = (t - floor(t)) * grid[i];
        const int ti = int(t);
        frac[i] = t - ti;
        const int g = ti % grid[i];
        gidx[i] = g < 0 ? 0 : (g < grid[i] ? g : grid[i] - 1);
    }
}

// Grid origin and B-spline weights (and derivatives when dd != nullptr) of one atom.
template <typename T>
__device__ __forceinline__ void spline(const T* __restrict__ pos, int64_t atom, const T* __restrict__ box,
                                       const Recip<T>& R, const int grid[3], int order, int gidx[3],
                                       T (&d)[kMaxOrder][3], T (*dd)[3]) {
    T frac[3];
    grid_coord<T>(pos, atom, box, R, grid, gidx, frac);
    for (int i = 0; i < 3; ++i) {
        const T dr = frac[i];
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

// ---------------------------------------------------------------------------
// Spreading as a gather over mesh bricks.  The mesh is cut into bricks of
// kBrick^3 points (the last brick along an axis may be partial).  Atoms are
// binned by the brick holding their spline origin, in ascending atom order
// inside each brick.  One workgroup owns one brick: it stages the splines of
// every atom whose origin lies in the brick or in the bricks that precede it
// within order-1 points (cyclically).  Each lane owns one (y, z) column of the
// brick, each of the four wavefronts sums a quarter of the staged atoms into
// its lanes' columns, and the four partial sums are added in wave order and
// stored once.  No atomics, every mesh point written exactly once (no
// clearing pass), and a fixed summation order.
// ---------------------------------------------------------------------------
constexpr int kBrick = 8;          // mesh points per brick edge (>= kMaxOrder - 1)
constexpr int kBrickThreads = 256; // two mesh points per thread
constexpr int kBrickStage = 256;   // atom splines staged in LDS per pass
constexpr int kAxisSrc = 3;        // source bricks per axis (see axis_sources)
static_assert(kBrick * kBrick == kWave, "one lane per (y, z) column of a brick");
static_assert(kBrickStage * 3 * kMaxOrder >= kBrickThreads * kBrick, "reduction fits the staging area");

__device__ __forceinline__ int brick_of(const int gi[3], int nby, int nbz) {
    return ((gi[0] / kBrick) * nby + gi[1] / kBrick) * nbz + gi[2] / kBrick;
}

template <typename T>
__global__ void k_bin_count(const T* __restrict__ pos, const T* __restrict__ box, int64_t n, int gx, int gy, int gz,
                            int nby, int nbz, int32_t* __restrict__ brick, int32_t* __restrict__ counts) {
    const int64_t a = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (a >= n) return;
    const int G[3] = {gx, gy, gz};
    const Recip<T> R = invert_box<T>(box);
    int gi[3];
    T frac[3];
    grid_coord<T>(pos, a, box, R, G, gi, frac);
    const int b = brick_of(gi, nby, nbz);
    brick[a] = b;
    atomicAdd(counts + b, 1);
}

__global__ void k_bin_place(const int32_t* __restrict__ brick, int64_t n, const int32_t* __restrict__ ptr,
                            int32_t* __restrict__ fill, int32_t* __restrict__ slots) {
    const int64_t a = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (a >= n) return;
    const int b = brick[a];
    slots[ptr[b] + atomicAdd(fill + b, 1)] = int32_t(a);
}

// Ascending atom order inside each brick: slot j moves to its rank within its brick.
__global__ void k_bin_rank(const int32_t* __restrict__ brick, const int32_t* __restrict__ ptr,
                           const int32_t* __restrict__ slots, int64_t n, int32_t* __restrict__ perm) {
    const int64_t j = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (j >= n) return;
    const int a = slots[j];
    const int b = brick[a];
    const int lo = ptr[b], hi = ptr[b + 1];
    int r = 0;
    for (int k = lo; k < hi; ++k) r += slots[k] < a;
    perm[lo + r] = a;
}

// Bricks along one axis whose atoms reach destination brick b: b itself and the
// bricks before it (cyclically) covering the order-1 points ahead of b's first
// point.  Only the last brick of an axis can be partial, so three suffice.
__device__ __forceinline__ int axis_sources(int b, int nb, int G, int order, int out[kAxisSrc]) {
    int k = 0;
    out[k++] = b;
    int need = order - 1, cur = b;
    while (need > 0 && k < kAxisSrc) {
        cur = cur == 0 ? nb - 1 : cur - 1;
        if (cur == b) break;
        out[k++] = cur;
        need -= min(kBrick, G - cur * kBrick);
    }
    return k;
}

template <typename T>
__global__ void __launch_bounds__(kBrickThreads)
    k_spread_bricks(const T* __restrict__ pos, const T* __restrict__ q, const T* __restrict__ box, int gx, int gy,
                    int gz, int nbx, int nby, int nbz, int order, T sqrt_k, const int32_t* __restrict__ ptr,
                    const int32_t* __restrict__ perm, T* __restrict__ grid) {
    constexpr int kSrc = kAxisSrc * kAxisSrc * kAxisSrc;
    __shared__ int s_src[kSrc];
    __shared__ int s_off[kSrc + 1];
    __shared__ int s_nsrc;
    __shared__ int s_rel[kBrickStage];             // packed brick-relative origin, -1: misses the brick
    __shared__ T s_w[kBrickStage][3 * kMaxOrder];  // [x weights * q sqrt(k) | y weights | z weights]
    const int bid = blockIdx.x;
    const int bz = bid % nbz, by = (bid / nbz) % nby, bx = bid / (nbz * nby);
    if (threadIdx.x == 0) {
        int sx[kAxisSrc], sy[kAxisSrc], sz[kAxisSrc];
        const int nx = axis_sources(bx, nbx, gx, order, sx);
        const int ny = axis_sources(by, nby, gy, order, sy);
        const int nz = axis_sources(bz, nbz, gz, order, sz);
        int k = 0, off = 0;
        for (int i = 0; i < nx; ++i)
            for (int j = 0; j < ny; ++j)
                for (int l = 0; l < nz; ++l) {
                    const int s = (sx[i] * nby + sy[j]) * nbz + sz[l];
                    s_src[k] = s;
                    s_off[k] = off;
                    off += ptr[s + 1] - ptr[s];
                    ++k;
                }
        s_off[k] = off;
        s_nsrc = k;
    }
    __syncthreads();
    const int total = s_off[s_nsrc];
    const int G[3] = {gx, gy, gz};
    const int S[3] = {bx * kBrick, by * kBrick, bz * kBrick};
    const Recip<T> R = invert_box<T>(box);
    const int t = threadIdx.x, lane = t & (kWave - 1), wave = t / kWave;
    // lane -> (y, z) column of the brick; acc[x] for its 8 points along x
    const int ly = lane >> 3, lz = lane & 7;
    T acc[kBrick];
    for (int x = 0; x < kBrick; ++x) acc[x] = 0;
    for (int base = 0; base < total; base += kBrickStage) {
        const int cnt = min(kBrickStage, total - base);
        for (int c = t; c < cnt; c += kBrickThreads) {
            const int g = base + c;
            int s = 0;
            while (s_off[s + 1] <= g) ++s;
            const int atom = perm[ptr[s_src[s]] + (g - s_off[s])];
            int gi[3];
            T d[kMaxOrder][3];
            spline<T>(pos, atom, box, R, G, order, gi, d, nullptr);
            // origin relative to the brick start, cyclically in (-G, brick size); the atom
            // reaches the brick along an axis iff that offset is > -order
            int rel[3];
            bool reach = true;
            for (int a = 0; a < 3; ++a) {
                int r = gi[a] - S[a];
                r += r < 0 ? G[a] : 0;
                if (r >= min(kBrick, G[a] - S[a])) r -= G[a];
                reach = reach && r > -order;
                rel[a] = r;
            }
            s_rel[c] = reach ? (rel[0] + 8) | ((rel[1] + 8) << 4) | ((rel[2] + 8) << 8) : -1;
            if (reach) {
                const T qs = q[atom] * sqrt_k;
                for (int k = 0; k < order; ++k) {
                    s_w[c][k] = qs * d[k][0];
                    s_w[c][kMaxOrder + k] = d[k][1];
                    s_w[c][2 * kMaxOrder + k] = d[k][2];
                }
            }
        }
        __syncthreads();
        // wave w sums candidates w, w + 4, ... in order (wave-uniform skip of non-reaching ones)
        for (int c = wave; c < cnt; c += kBrickThreads / kWave) {
            const int pk = s_rel[c];
            if (pk < 0) continue;
            const int rx = (pk & 15) - 8, ry = ((pk >> 4) & 15) - 8, rz = (pk >> 8) - 8;
            int dy = ly - ry;
            dy += dy < 0 ? gy : 0;
            int dz = lz - rz;
            dz += dz < 0 ? gz : 0;
            const bool in = dy < order && dz < order;
            const T wyz = in ? s_w[c][kMaxOrder + dy] * s_w[c][2 * kMaxOrder + dz] : T(0);
#pragma unroll
            for (int x = 0; x < kBrick; ++x) {
                int dx = x - rx;
                dx += dx < 0 ? gx : 0;
                if (dx < order) acc[x] += s_w[c][dx] * wyz;
            }
        }
        __syncthreads();
    }
    // the four waves' partial sums, added in wave order (reuses the staging area)
    T* red = &s_w[0][0];
    for (int x = 0; x < kBrick; ++x) red[(wave * kBrick + x) * kWave + lane] = acc[x];
    __syncthreads();
    for (int i = t; i < kBrick * kWave; i += kBrickThreads) {
        const int x = i / kWave, l = i % kWave;
        T v = red[x * kWave + l];
        for (int w = 1; w < kBrickThreads / kWave; ++w) v += red[(w * kBrick + x) * kWave + l];
        const int px = S[0] + x, py = S[1] + (l >> 3), pz = S[2] + (l & 7);
        if (px < gx && py < gy && pz < gz) grid[(int64_t(px) * gy + py) * gz + pz] = v;
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

// Block-wide fp64 sum of one value per thread into partials[blockIdx.x].
__device__ __forceinline__ void block_partial(double e, double* __restrict__ partials) {
    __shared__ double red[kConvThreads];
    red[threadIdx.x] = e;
    __syncthreads();
    for (int off = kConvThreads / 2; off > 0; off >>= 1) {
        if (threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
        __syncthreads();
    }
    if (threadIdx.x == 0) partials[blockIdx.x] = red[0];
}

// Real-space pair sum over the given pair list minus excluded pairs (pme_cpu.cpp:110-135).
// GRAD: also dE/dq and dE/dpos (pme_cpu.cpp:195-215).  Pair lists come grouped by
// their first atom (the neighbor list's row order), so the first atom's four
// derivative terms are summed over each run of equal rows in the wavefront and
// added once per run; the second atom's terms are added per pair.  Each pair's
// terms are evaluated in fp64 whatever the storage type (erfc/exp/division in
// double cost nothing next to the pair list's memory latency), so the fp32 path
// differs from an fp64 evaluation only by its rounded inputs and the fp32
// accumulation of the derivatives.
template <typename T, bool GRAD>
__global__ void __launch_bounds__(kConvThreads) k_direct_pairs(const T* __restrict__ q, int64_t n,
                                                               const int32_t* __restrict__ nb, int64_t P, const T* __restrict__ dl,
                                                               const T* __restrict__ r, const int32_t* __restrict__ excl,
                                                               int max_excl, double alpha, double coulomb,
                                                               T* __restrict__ dpos, T* __restrict__ dq,
                                                               double* __restrict__ partials) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    double e = 0.0;
    int row = -1;
    double g1[4] = {0, 0, 0, 0};  // d/dq and d/dpos of the pair's first atom
    if (i < P) {
        const int a1 = nb[i], a2 = nb[P + i];
        // -1 marks padding (reference); any other out-of-range index is skipped too
        bool include = a1 > -1 && a1 < n && a2 >= 0 && a2 < n;
        if (include) row = a1;
        for (int j = 0; include && j < max_excl && excl[int64_t(a1) * max_excl + j] >= a2; ++j)
            if (excl[int64_t(a1) * max_excl + j] == a2) include = false;
        if (include) {
            const double rr = double(r[i]);
            const double inv = 1.0 / rr;
            const double ar = alpha * rr;
            const double ec = erfc(ar);
            const double pref = coulomb * inv;
            const double c1 = double(q[a1]), c2 = double(q[a2]);
            e = pref * ec * c1 * c2;
            if (GRAD) {
                const double ex = exp(-ar * ar);
                const double dedr = pref * c1 * c2 * (ec + ar * ex * M_2_SQRTPI) * inv * inv;
                g1[0] = pref * ec * c2;
                atomicAdd(dq + a2, T(pref * ec * c1));
                for (int k = 0; k < 3; ++k) {
                    const double f = dedr * double(dl[3 * i + k]);
                    g1[1 + k] = -f;
                    atomicAdd(dpos + 3 * a2 + k, T(f));
                }
            }
        }
    }
    if (GRAD) {
        if (run_reduce<double, 4>(row, g1) && row >= 0) {
            atomicAdd(dq + row, T(g1[0]));
            for (int k = 0; k < 3; ++k) atomicAdd(dpos + 3 * row + k, T(g1[1 + k]));
        }
    }
    block_partial(e, partials);
}

// Excluded pairs' erf term, removed from the reciprocal-space sum (pme_cpu.cpp:137-162).
// One thread per atom a; a's own derivative terms are summed over its exclusions
// and added once.  Pair terms in fp64 as above.
template <typename T, bool GRAD>
__global__ void __launch_bounds__(kConvThreads) k_direct_excl(const T* __restrict__ pos, const T* __restrict__ q,
                                                              int64_t n, const int32_t* __restrict__ excl,
                                                              int max_excl, double alpha, double coulomb,
                                                              T* __restrict__ dpos, T* __restrict__ dq,
                                                              double* __restrict__ partials) {
    const int64_t a = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    double e = 0.0;
    if (a < n) {
        double ga[4] = {0, 0, 0, 0};
        for (int j = 0; j < max_excl; ++j) {
            const int b = excl[a * max_excl + j];
            if (!(b > a)) break;
            if (b >= n) continue;
            double dr[3];
            for (int k = 0; k < 3; ++k) dr[k] = double(pos[3 * a + k]) - double(pos[3 * int64_t(b) + k]);
            const double rr = sqrt(dr[0] * dr[0] + dr[1] * dr[1] + dr[2] * dr[2]);
            const double inv = 1.0 / rr;
            const double ar = alpha * rr;
            const double ef = erf(ar);
            const double pref = coulomb * inv;
            const double c1 = double(q[a]), c2 = double(q[b]);
            e -= pref * ef * c1 * c2;
            if (GRAD) {
                const double ex = exp(-ar * ar);
                const double dedr = pref * c1 * c2 * (ef - ar * ex * M_2_SQRTPI) * inv * inv;
                ga[0] -= pref * ef * c2;
                atomicAdd(dq + b, T(-pref * ef * c1));
                for (int k = 0; k < 3; ++k) {
                    ga[1 + k] += dedr * dr[k];
                    atomicAdd(dpos + 3 * int64_t(b) + k, T(-dedr * dr[k]));
                }
            }
        }
        if (GRAD && max_excl > 0) {
            atomicAdd(dq + a, T(ga[0]));
            for (int k = 0; k < 3; ++k) atomicAdd(dpos + 3 * a + k, T(ga[1 + k]));
        }
    }
    block_partial(e, partials);
}

template <typename T>
__global__ void k_fill(T* __restrict__ p, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = T(0);
}

int check_grid(int gx, int gy, int gz, int order) {
    MNX_REQUIRE(gx > 0 && gy > 0 && gz > 0 && int64_t(gx) * gy * gz < (int64_t(1) << 31), "bad grid size");
    MNX_REQUIRE(order >= 3 && order <= kMaxOrder, "spline order %d not in [3, %d]", order, kMaxOrder);
    MNX_REQUIRE(gx >= order && gy >= order && gz >= order, "grid smaller than the spline order");
    return MNX_OK;
}

struct BrickWs {
    int32_t *counts, *fill, *ptr, *tiles, *brick, *slots, *perm;
};

BrickWs carve_bricks(void* base, int64_t n, int64_t nbricks, size_t* used) {
    Workspace ws{static_cast<char*>(base), 0};
    BrickWs w;
    w.counts = ws.take<int32_t>(nbricks + 1);
    w.fill = ws.take<int32_t>(nbricks + 1);
    w.ptr = ws.take<int32_t>(nbricks + 1);
    w.tiles = ws.take<int32_t>(scan_workspace_elems(nbricks + 1));
    w.brick = ws.take<int32_t>(n);
    w.slots = ws.take<int32_t>(n);
    w.perm = ws.take<int32_t>(n);
    *used = ws.used;
    return w;
}

int64_t brick_count(int g) { return ceil_div(g, kBrick); }

size_t spread_ws(int64_t n, int gx, int gy, int gz) {
    size_t used = 0;
    carve_bricks(nullptr, n > 0 ? n : 0, brick_count(gx) * brick_count(gy) * brick_count(gz), &used);
    return used + 256;
}

template <typename T>
int spread(const T* pos, const T* q, const T* box, int64_t n, int gx, int gy, int gz, int order, double coulomb,
           T* grid, void* ws, size_t ws_bytes, hipStream_t s) {
    clear_error();
    int rc = check_grid(gx, gy, gz, order);
    if (rc) return rc;
    MNX_REQUIRE(n >= 0 && n < (int64_t(1) << 31), "atom count out of range");
    MNX_REQUIRE(grid && box && (n == 0 || (pos && q)), "null pointer argument");
    const int nbx = int(brick_count(gx)), nby = int(brick_count(gy)), nbz = int(brick_count(gz));
    const int64_t nbricks = int64_t(nbx) * nby * nbz;
    size_t need = 0;
    BrickWs w = carve_bricks(ws, n, nbricks, &need);
    if (!ws || ws_bytes < need) return set_error(MNX_ERR_WORKSPACE, "workspace %zu < %zu bytes", ws_bytes, need);
    const int tb = 256;
    for (int32_t* p : {w.counts, w.fill}) {
        hipLaunchKernelGGL((k_fill<int32_t>), dim3(ceil_div(nbricks + 1, tb)), dim3(tb), 0, s, p, nbricks + 1);
        MNX_CHECK_LAUNCH();
    }
    if (n > 0) {
        hipLaunchKernelGGL((k_bin_count<T>), dim3(ceil_div(n, tb)), dim3(tb), 0, s, pos, box, n, gx, gy, gz, nby, nbz,
                           w.brick, w.counts);
        MNX_CHECK_LAUNCH();
    }
    rc = exclusive_scan<int32_t, int32_t>(w.counts, nbricks + 1, w.ptr, w.tiles, (int32_t*)nullptr, s);
    if (rc) return rc;
    if (n > 0) {
        hipLaunchKernelGGL(k_bin_place, dim3(ceil_div(n, tb)), dim3(tb), 0, s, w.brick, n, w.ptr, w.fill, w.slots);
        MNX_CHECK_LAUNCH();
        hipLaunchKernelGGL(k_bin_rank, dim3(ceil_div(n, tb)), dim3(tb), 0, s, w.brick, w.ptr, w.slots, n, w.perm);
        MNX_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL((k_spread_bricks<T>), dim3(nbricks), dim3(kBrickThreads), 0, s, pos, q, box, gx, gy, gz, nbx,
                       nby, nbz, order, T(sqrt(coulomb)), w.ptr, w.perm, grid);
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

template <typename T, bool GRAD>
void launch_direct(const T* pos, const T* q, int64_t n, const int32_t* nb, int64_t P, const T* deltas, const T* dist,
                   const int32_t* excl, int max_excl, double alpha, double coulomb, T* dpos, T* dq, double* part,
                   int64_t b1, int64_t b2, hipStream_t s) {
    if (b1 > 0)
        hipLaunchKernelGGL((k_direct_pairs<T, GRAD>), dim3(b1), dim3(kConvThreads), 0, s, q, n, nb, P, deltas, dist,
                           excl, max_excl, alpha, coulomb, dpos, dq, part);
    if (b2 > 0)
        hipLaunchKernelGGL((k_direct_excl<T, GRAD>), dim3(b2), dim3(kConvThreads), 0, s, pos, q, n, excl, max_excl,
                           alpha, coulomb, dpos, dq, part + b1);
}

template <typename T>
int direct(const T* pos, const T* q, int64_t n, const int32_t* nb, int64_t P, const T* deltas, const T* dist,
           const int32_t* excl, int max_excl, double alpha, double coulomb, T* energy, T* dpos, T* dq, void* ws,
           size_t ws_bytes, hipStream_t s) {
    clear_error();
    MNX_REQUIRE(n >= 0 && P >= 0 && max_excl >= 0, "sizes out of range");
    MNX_REQUIRE(energy && (n == 0 || (pos && q)), "null pointer argument");
    MNX_REQUIRE((dpos == nullptr) == (dq == nullptr), "dpos and dq must both be given or both be null");
    MNX_REQUIRE(max_excl == 0 || excl, "exclusions pointer is null");
    MNX_REQUIRE(P == 0 || (nb && deltas && dist), "null pair-list pointer");
    if (!ws || ws_bytes < direct_ws(n, P)) return set_error(MNX_ERR_WORKSPACE, "workspace too small");
    double* part = static_cast<double*>(ws);
    const int64_t b1 = P > 0 ? ceil_div(P, kConvThreads) : 0;
    const int64_t b2 = (n > 0 && max_excl > 0) ? ceil_div(n, kConvThreads) : 0;
    const bool grad = dpos != nullptr;
    if (grad && n > 0) {
        hipLaunchKernelGGL((k_fill<T>), dim3(ceil_div(3 * n, 256)), dim3(256), 0, s, dpos, 3 * n);
        MNX_CHECK_LAUNCH();
        hipLaunchKernelGGL((k_fill<T>), dim3(ceil_div(n, 256)), dim3(256), 0, s, dq, n);
        MNX_CHECK_LAUNCH();
    }
    if (grad)
        launch_direct<T, true>(pos, q, n, nb, P, deltas, dist, excl, max_excl, alpha, coulomb, dpos, dq, part, b1, b2,
                               s);
    else
        launch_direct<T, false>(pos, q, n, nb, P, deltas, dist, excl, max_excl, alpha, coulomb, dpos, dq, part, b1,
                                b2, s);
    MNX_CHECK_LAUNCH();
    // every launched block wrote its partial; with no blocks the energy is 0
    hipLaunchKernelGGL((k_sum_partials<T>), dim3(1), dim3(1024), 0, s, part, b1 + b2, 1.0, energy);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

size_t mnx_pme_spread_workspace_bytes(int64_t n, int32_t gx, int32_t gy, int32_t gz) {
    return spread_ws(n, gx > 0 ? gx : 1, gy > 0 ? gy : 1, gz > 0 ? gz : 1);
}
int mnx_pme_spread_f32(const float* pos, const float* q, const float* box, int64_t n, int32_t gx, int32_t gy,
                       int32_t gz, int32_t order, double coulomb, float* grid, void* ws, size_t ws_bytes,
                       mnx_stream_t s) {
    return spread<float>(pos, q, box, n, gx, gy, gz, order, coulomb, grid, ws, ws_bytes, (hipStream_t)s);
}
int mnx_pme_spread_f64(const double* pos, const double* q, const double* box, int64_t n, int32_t gx, int32_t gy,
                       int32_t gz, int32_t order, double coulomb, double* grid, void* ws, size_t ws_bytes,
                       mnx_stream_t s) {
    return spread<double>(pos, q, box, n, gx, gy, gz, order, coulomb, grid, ws, ws_bytes, (hipStream_t)s);
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
