// Cell-list neighbor list for gfx950.
//
// Replaces the O(N^2) pair enumeration of torch.ops.molix.get_neighbor_pairs
// (reference CPU src/molix/op/src/neighbors/get_neighbor_pairs.cpp:28-77, CUDA
// get_neighbor_pairs.cu:29-79) with a cell list, while keeping the reference
// CPU path's pair predicate and geometry bit for bit:
//   d = pos[i] - pos[j]                                      (.cpp:44)
//   for k = 2, 1, 0: d -= rint(d[k] / box[k][k]) * box[k]   (.cpp:45-49; torch::round is
//                                                             round-half-even)
//   dist = sqrt(fma(d2, d2, fma(d1, d1, d0 * d0)))            (linalg_vector_norm, .cpp:50)
//   keep iff dist <= cutoff && dist > 0                       (.cpp:52)
// Output is sorted by (i, j) like the CPU enumeration order (.cpp:38-43), which
// the CUDA reference does not guarantee (atomicAdd slots, .cu:69).
//
// Layout of the work: atoms are binned into cells whose slab widths exceed the
// cutoff (fractional coordinates for periodic cells), each cell's atoms sorted by
// id.  Four wavefronts share a cell (each takes every fourth atom of it as a
// centre): they fetch the 27 neighbour cells' ranges in one round trip, load each
// candidate once and test it against all of their centres (count pass: a screening
// distance on positions moved into the primary cell, the reference arithmetic near
// the cutoff; the accept ballots are kept), then the emit pass compacts the accepted
// j of each centre from the ballots into LDS, sorts them in registers (bitonic,
// <= 64) or by rank, and writes each centre's segment with coalesced stores.  Grids with
// fewer than 3 cells along a periodic axis use one wavefront per atom over all
// atoms (brute mode).  This translation unit is compiled with -ffp-contract=off.

#include <math.h>

#include <algorithm>

#include "common.h"
#include "scan.h"

namespace mnx {
namespace {

constexpr int kNlCap = 4096;  // max neighbours of one atom (LDS list of the per-atom emit)
constexpr int kEmitBuf = 1024; // LDS list per wavefront of the cell emit; atoms with more
                               // neighbours are written by the per-atom emit
constexpr int64_t kNlBlocks = 16384;  // grid-stride launches of the count / emit kernels
constexpr int kCellParts = 4;          // wavefronts per cell (each takes every 4th atom of it)
constexpr int kMaskChunks = 16;        // acceptance masks kept per centre: 16 x 64 candidates; cells
                                       // with more candidates are tested again by the emit
constexpr int kPreChunks = 8;          // candidate chunks a cell unit loads into registers at once
constexpr float kCellMargin = 1.0001f;

struct NlGrid {
    int32_t brute;  // 1: all-pairs scan (periodic axis with < 3 cells)
    int32_t periodic;
    int32_t n[3];
    int32_t ncells;
    int32_t overflow;  // set when an atom has more than kNlCap neighbours
    int32_t nbig;      // atoms with more than kEmitBuf neighbours (listed in NlWs::big)
    double lo[3];
    double inv_w[3];
    double rinv[6];  // inverse of the lower-triangular cell: f_c = z*r5, ...
};

// Position moved into the primary cell, in cell order (screening test of the count pass).
template <typename T>
struct alignas(4 * sizeof(T)) PosW {
    T x, y, z, w;
};

struct NlWs {
    NlGrid* grid;
    int32_t* cell_of;
    int32_t* cell_count;
    int32_t* cell_start;
    int32_t* cell_fill;
    int32_t* atoms_sorted;
    int32_t* counts;
    int32_t* big;
    uint64_t* masks;  // per centre: the count pass's accept ballot of each 64-candidate chunk
    void* posw;       // PosW<T> per cell-ordered slot
    int64_t* offsets;
    int64_t* total;
    int64_t* tiles64;
    int32_t* tiles32;
    int64_t max_cells;
};

int64_t max_cells_for(int64_t n) { return 2 * n + 64; }

NlWs carve(void* base, size_t bytes, int64_t n, size_t* used) {
    Workspace ws{static_cast<char*>(base), bytes};
    NlWs w;
    w.max_cells = max_cells_for(n);
    w.grid = ws.take<NlGrid>(1);
    w.cell_of = ws.take<int32_t>(n > 0 ? n : 1);
    w.cell_count = ws.take<int32_t>(w.max_cells);
    w.cell_start = ws.take<int32_t>(w.max_cells + 1);
    w.cell_fill = ws.take<int32_t>(w.max_cells);
    w.atoms_sorted = ws.take<int32_t>(n > 0 ? n : 1);
    w.counts = ws.take<int32_t>(n > 0 ? n : 1);
    w.big = ws.take<int32_t>(n > 0 ? n : 1);
    w.masks = ws.take<uint64_t>(size_t(n > 0 ? n : 1) * kMaskChunks);
    w.posw = ws.take<PosW<double>>(n > 0 ? n : 1);
    w.offsets = ws.take<int64_t>(n + 1);
    w.total = ws.take<int64_t>(1);
    w.tiles64 = ws.take<int64_t>(scan_workspace_elems(n));
    w.tiles32 = ws.take<int32_t>(scan_workspace_elems(w.max_cells));
    *used = ws.used;
    return w;
}

// ---------------------------------------------------------------------------
// Exact reference geometry
// ---------------------------------------------------------------------------

template <typename T>
struct Geo {
    T d[3];
    T dist;
    T shift[3];
};

__device__ __forceinline__ float fma_(float a, float b, float c) { return fmaf(a, b, c); }
__device__ __forceinline__ double fma_(double a, double b, double c) { return fma(a, b, c); }
__device__ __forceinline__ float rint_(float a) { return rintf(a); }
__device__ __forceinline__ double rint_(double a) { return rint(a); }
__device__ __forceinline__ float sqrt_(float a) { return sqrtf(a); }
__device__ __forceinline__ double sqrt_(double a) { return sqrt(a); }

// Minimum image and distance of the difference vector d, the reference's arithmetic.
template <typename T>
__device__ __forceinline__ void geo_from_d(const T* __restrict__ box, T d0, T d1, T d2, bool periodic, bool want_shift,
                                           Geo<T>& g) {
    T s0 = 0, s1 = 0, s2 = 0;
    if (periodic) {
#pragma unroll
        for (int k = 2; k >= 0; --k) {
            const T dk = k == 2 ? d2 : (k == 1 ? d1 : d0);
            const T s = rint_(dk / box[4 * k]);
            const T b0 = s * box[3 * k + 0], b1 = s * box[3 * k + 1], b2 = s * box[3 * k + 2];
            d0 = d0 - b0;
            d1 = d1 - b1;
            d2 = d2 - b2;
            if (want_shift) {
                s0 = s0 + b0;
                s1 = s1 + b1;
                s2 = s2 + b2;
            }
        }
    }
    g.d[0] = d0;
    g.d[1] = d1;
    g.d[2] = d2;
    g.dist = sqrt_(fma_(d2, d2, fma_(d1, d1, d0 * d0)));
    g.shift[0] = s0;
    g.shift[1] = s1;
    g.shift[2] = s2;
}

// Geometry of the pair (hi, lo) with hi > lo, in the reference's orientation.
template <typename T>
__device__ __forceinline__ void pair_geo(const T* __restrict__ pos, const T* __restrict__ box, int hi, int lo,
                                         bool periodic, bool want_shift, Geo<T>& g) {
    geo_from_d<T>(box, pos[3 * hi + 0] - pos[3 * lo + 0], pos[3 * hi + 1] - pos[3 * lo + 1],
                  pos[3 * hi + 2] - pos[3 * lo + 2], periodic, want_shift, g);
}

// Acceptance of a candidate pair, decided as the reference decides it.  A cheap test
// (minimum image through the reciprocal box diagonal, squared distance without the fma
// chain) settles every candidate whose squared distance is clear of cutoff^2 by a relative
// 1e-4 -- far more than the rounding difference between the two evaluations -- and the
// exact reference arithmetic decides the rest (the band around the cutoff and zero
// distance).  The two image choices can differ only where a fractional coordinate is
// within rounding of 1/2, i.e. at about half a cell height of the box, which the cell list
// keeps above the cutoff (>= 3 cells of width >= cutoff along every periodic axis).
template <typename T>
struct AcceptTest {
    T inv[3];
    T c2lo, c2hi, c2tiny;
    T b[9];  // the box, held in registers for the cheap test
};

// The all-pairs fallback (a periodic axis with < 3 cells) gets no cheap test: there the
// half-box distance can be within the cutoff.
template <typename T>
__device__ __forceinline__ AcceptTest<T> accept_test(const T* box, bool periodic, bool brute, T cutoff) {
    AcceptTest<T> a;
    for (int k = 0; k < 3; ++k) a.inv[k] = periodic ? T(1) / box[4 * k] : T(0);
    const T c2 = cutoff * cutoff;
    a.c2lo = brute ? T(0) : c2 * T(0.9999);
    a.c2hi = brute ? T(INFINITY) : c2 * T(1.0001);
    a.c2tiny = c2 * T(1e-20);
    for (int k = 0; k < 9; ++k) a.b[k] = periodic ? box[k] : T(0);
    return a;
}

// Value of lane q (wave-uniform q) broadcast to the wavefront through v_readlane.
__device__ __forceinline__ int lane_value(int v, int q) { return __builtin_amdgcn_readlane(v, q); }
__device__ __forceinline__ float lane_value(float v, int q) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), q));
}
__device__ __forceinline__ uint64_t lane_value(uint64_t v, int q) {
    const uint32_t lo = __builtin_amdgcn_readlane(int(v & 0xffffffffu), q),
                   hi = __builtin_amdgcn_readlane(int(v >> 32), q);
    return (uint64_t(hi) << 32) | lo;
}
__device__ __forceinline__ double lane_value(double v, int q) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane(int(b & 0xffffffff), q), hi = __builtin_amdgcn_readlane(int(b >> 32), q);
    return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned int>(lo));
}

// Value of lane (lane ^ s) for a power of two s < 64: DPP for 1, 2 (quad permutes) and 8
// (rotation by 8 within a row of 16), the LDS crossbar without memory (ds_swizzle, xor
// within 32 lanes) for 4 and 16, ds_bpermute for 32.
__device__ __forceinline__ int lane_xor(int v, int s) {
    switch (s) {
        case 1: return __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
        case 2: return __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
        case 8: return __builtin_amdgcn_update_dpp(v, v, 0x128, 0xF, 0xF, false);  // row_ror:8
        case 4: return __builtin_amdgcn_ds_swizzle(v, 0x101F);                     // and 31, xor 4
        case 16: return __builtin_amdgcn_ds_swizzle(v, 0x401F);                    // and 31, xor 16
        default: return __shfl_xor(v, s, kWave);
    }
}

// Decision for the pair at positions a, b.  It does not depend on the order: a - b is the
// exact negation of b - a, and the minimum image and the norm are symmetric in sign.
template <typename T>
__device__ __forceinline__ bool accept_xyz(const T* box, T ax, T ay, T az, T bx, T by, T bz, bool periodic, T cutoff,
                                           const AcceptTest<T>& at) {
    T d0 = ax - bx, d1 = ay - by, d2 = az - bz;
    const T e0 = d0, e1 = d1, e2 = d2;
    if (periodic) {
#pragma unroll
        for (int k = 2; k >= 0; --k) {
            const T dk = k == 2 ? d2 : (k == 1 ? d1 : d0);
            const T s = rint_(dk * at.inv[k]);
            d0 = d0 - s * at.b[3 * k + 0];
            d1 = d1 - s * at.b[3 * k + 1];
            d2 = d2 - s * at.b[3 * k + 2];
        }
    }
    const T r2 = d0 * d0 + d1 * d1 + d2 * d2;
    if (r2 > at.c2hi) return false;
    if (r2 < at.c2lo && r2 > at.c2tiny) return true;
    Geo<T> g;
    geo_from_d<T>(box, e0, e1, e2, periodic, false, g);
    return g.dist <= cutoff && g.dist > T(0);
}

template <typename T>
__device__ __forceinline__ bool accept(const T* pos, const T* box, int i, int j, bool periodic, T cutoff,
                                       const AcceptTest<T>& at) {
    return accept_xyz<T>(box, pos[3 * i], pos[3 * i + 1], pos[3 * i + 2], pos[3 * j], pos[3 * j + 1], pos[3 * j + 2],
                         periodic, cutoff, at);
}

// ---------------------------------------------------------------------------
// Grid set-up and binning
// ---------------------------------------------------------------------------

template <typename T>
__global__ void __launch_bounds__(1024) k_grid_setup(const T* __restrict__ pos, int64_t n, const T* __restrict__ box,
                                                     double cutoff, int64_t max_cells, NlGrid* __restrict__ grid) {
    __shared__ double smin[3][1024], smax[3][1024];
    const int t = threadIdx.x;
    double mn[3] = {1e300, 1e300, 1e300}, mx[3] = {-1e300, -1e300, -1e300};
    if (!box) {
        for (int64_t i = t; i < n; i += 1024)
            for (int k = 0; k < 3; ++k) {
                double v = double(pos[3 * i + k]);
                mn[k] = fmin(mn[k], v);
                mx[k] = fmax(mx[k], v);
            }
    }
    for (int k = 0; k < 3; ++k) {
        smin[k][t] = mn[k];
        smax[k][t] = mx[k];
    }
    __syncthreads();
    for (int off = 512; off > 0; off >>= 1) {
        if (t < off)
            for (int k = 0; k < 3; ++k) {
                smin[k][t] = fmin(smin[k][t], smin[k][t + off]);
                smax[k][t] = fmax(smax[k][t], smax[k][t + off]);
            }
        __syncthreads();
    }
    if (t != 0) return;
    NlGrid g{};
    const double cw = cutoff * double(kCellMargin) + 1e-12;
    if (box) {
        const double ax = box[0], bx = box[3], by = box[4], cx = box[6], cy = box[7], cz = box[8];
        // perpendicular slab widths of the lower-triangular cell
        const double vol = fabs(ax * by * cz);
        const double bxc = sqrt((by * cz) * (by * cz) + (bx * cz) * (bx * cz) + (bx * cy - by * cx) * (bx * cy - by * cx));
        const double axc = sqrt((ax * cz) * (ax * cz) + (ax * cy) * (ax * cy));
        const double h[3] = {vol / bxc, vol / axc, fabs(cz)};
        g.periodic = 1;
        for (int k = 0; k < 3; ++k) {
            double m = floor(h[k] / cw);
            g.n[k] = m < 1 ? 1 : (m > 1024 ? 1024 : int(m));
        }
        g.rinv[0] = 1.0 / ax;
        g.rinv[1] = bx;
        g.rinv[2] = 1.0 / by;
        g.rinv[3] = cx;
        g.rinv[4] = cy;
        g.rinv[5] = 1.0 / cz;
        while (int64_t(g.n[0]) * g.n[1] * g.n[2] > max_cells) {
            int kmax = g.n[0] >= g.n[1] ? (g.n[0] >= g.n[2] ? 0 : 2) : (g.n[1] >= g.n[2] ? 1 : 2);
            g.n[kmax] = (g.n[kmax] + 1) / 2;
        }
        g.brute = (g.n[0] < 3 || g.n[1] < 3 || g.n[2] < 3) ? 1 : 0;
    } else {
        g.periodic = 0;
        for (int k = 0; k < 3; ++k) {
            double lo = n > 0 ? smin[k][0] : 0.0, hi = n > 0 ? smax[k][0] : 0.0;
            double ext = hi - lo;
            double m = floor(ext / cw);
            g.n[k] = m < 1 ? 1 : (m > 1024 ? 1024 : int(m));
            g.lo[k] = lo;
        }
        while (int64_t(g.n[0]) * g.n[1] * g.n[2] > max_cells) {
            int kmax = g.n[0] >= g.n[1] ? (g.n[0] >= g.n[2] ? 0 : 2) : (g.n[1] >= g.n[2] ? 1 : 2);
            g.n[kmax] = (g.n[kmax] + 1) / 2;
        }
        for (int k = 0; k < 3; ++k) {
            double ext = (n > 0 ? smax[k][0] : 0.0) - g.lo[k];
            g.inv_w[k] = ext > 0 ? double(g.n[k]) / ext : 0.0;
        }
        g.brute = 0;
    }
    g.ncells = g.brute ? 1 : g.n[0] * g.n[1] * g.n[2];
    *grid = g;
}

template <typename T>
__device__ __forceinline__ void cell_coords(const T* pos, int64_t i, const NlGrid& g, int c[3]) {
    const double x = pos[3 * i], y = pos[3 * i + 1], z = pos[3 * i + 2];
    if (g.periodic) {
        double f[3];
        f[2] = z * g.rinv[5];
        f[1] = (y - f[2] * g.rinv[4]) * g.rinv[2];
        f[0] = (x - f[1] * g.rinv[1] - f[2] * g.rinv[3]) * g.rinv[0];
        for (int k = 0; k < 3; ++k) {
            double fk = f[k] - floor(f[k]);
            int ck = int(fk * g.n[k]);
            c[k] = ck < 0 ? 0 : (ck >= g.n[k] ? g.n[k] - 1 : ck);
        }
    } else {
        const double v[3] = {x, y, z};
        for (int k = 0; k < 3; ++k) {
            int ck = int((v[k] - g.lo[k]) * g.inv_w[k]);
            c[k] = ck < 0 ? 0 : (ck >= g.n[k] ? g.n[k] - 1 : ck);
        }
    }
}

template <typename T>
__global__ void k_bin(const T* __restrict__ pos, int64_t n, const NlGrid* __restrict__ gp, int32_t* __restrict__ cell_of,
                      int32_t* __restrict__ cell_count) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const NlGrid g = *gp;
    int cid = 0;
    if (!g.brute) {
        int c[3];
        cell_coords<T>(pos, i, g, c);
        cid = (c[2] * g.n[1] + c[1]) * g.n[0] + c[0];
    }
    cell_of[i] = cid;
    atomicAdd(&cell_count[cid], 1);
}

__global__ void k_place(int64_t n, const int32_t* __restrict__ cell_of, const int32_t* __restrict__ cell_start,
                        int32_t* __restrict__ cell_fill, int32_t* __restrict__ atoms_sorted) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int cid = cell_of[i];
    const int slot = cell_start[cid] + atomicAdd(&cell_fill[cid], 1);
    atoms_sorted[slot] = int32_t(i);
}

// Each cell's atom list in ascending order (deterministic after the atomic placement into
// `slots`): the atom in slot k moves to its rank within its cell.  The same slot of `posw`
// receives the atom's position moved into the primary cell (by whole box vectors, from the
// fractional coordinates that binned it), which the count pass's screening test reads.
template <typename T>
__global__ void k_rank_cells(int64_t n, const T* __restrict__ pos, const T* __restrict__ box,
                             const NlGrid* __restrict__ gp, const int32_t* __restrict__ cell_of,
                             const int32_t* __restrict__ cell_start, const int32_t* __restrict__ slots,
                             int32_t* __restrict__ atoms_sorted, PosW<T>* __restrict__ posw) {
    const int64_t k = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (k >= n) return;
    const int a = slots[k];
    const int c = cell_of[a];
    const int b = cell_start[c], e = cell_start[c + 1];
    int r = 0;
    for (int t = b; t < e; ++t) r += slots[t] < a;
    atoms_sorted[b + r] = a;
    const double x = pos[3 * a], y = pos[3 * a + 1], z = pos[3 * a + 2];
    PosW<T> p;
    if (gp->periodic) {
        // the fractional coordinates of cell_coords; box rows (ax,0,0), (bx,by,0), (cx,cy,cz)
        const NlGrid& g = *gp;
        const double f2 = z * g.rinv[5];
        const double f1 = (y - f2 * g.rinv[4]) * g.rinv[2];
        const double f0 = (x - f1 * g.rinv[1] - f2 * g.rinv[3]) * g.rinv[0];
        const double n0 = floor(f0), n1 = floor(f1), n2 = floor(f2);
        p.x = T(x - n0 * double(box[0]) - n1 * double(box[3]) - n2 * double(box[6]));
        p.y = T(y - n1 * double(box[4]) - n2 * double(box[7]));
        p.z = T(z - n2 * double(box[8]));
    } else {
        p.x = T(x);
        p.y = T(y);
        p.z = T(z);
    }
    p.w = T(0);
    posw[b + r] = p;
}

// ---------------------------------------------------------------------------
// Candidate scan: one wavefront per atom
// ---------------------------------------------------------------------------

// Atom ranges of the 27 neighbour cells of cell (cx, cy, cz), flattened: lanes 0..26 hold
// (begin, length) of neighbour cell (dz, dy, dx) = lane in base 3, fetched in one round trip,
// and `incl` is the inclusive prefix sum of the lengths over lanes; `total` candidates in all.
struct CellRanges {
    int rb, rlen, incl, total;
};

__device__ __forceinline__ CellRanges cell_ranges(const NlGrid& g, int cx, int cy, int cz,
                                                  const int32_t* __restrict__ cell_start, int lane) {
    CellRanges cr{0, 0, 0, 0};
    if (lane < 27) {
        int z = cz + lane / 9 - 1, y = cy + (lane / 3) % 3 - 1, x = cx + lane % 3 - 1;
        bool in = true;
        if (g.periodic) {
            z = (z + g.n[2]) % g.n[2];
            y = (y + g.n[1]) % g.n[1];
            x = (x + g.n[0]) % g.n[0];
        } else {
            in = z >= 0 && z < g.n[2] && y >= 0 && y < g.n[1] && x >= 0 && x < g.n[0];
        }
        if (in) {
            const int cid = (z * g.n[1] + y) * g.n[0] + x;
            cr.rb = cell_start[cid];
            cr.rlen = cell_start[cid + 1] - cr.rb;
        }
    }
    int incl = cr.rlen;  // lanes >= 27 add 0
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) {
        const int v = __shfl_up(incl, o, kWave);
        if (lane >= o) incl += v;
    }
    cr.incl = incl;
    cr.total = __shfl(incl, 26, kWave);
    return cr;
}

// Candidate number k of the flattened ranges (-1 past the end); every lane must call it.
__device__ __forceinline__ int cell_candidate(const CellRanges& cr, int k, const int32_t* __restrict__ atoms_sorted) {
    int r = 0;  // number of ranges that end at or before k (branch-free search over 27 entries)
#pragma unroll
    for (int step = 16; step > 0; step >>= 1) {
        const int probe = __shfl(cr.incl, r + step - 1, kWave);
        if (r + step <= 26 && probe <= k) r += step;
    }
    const int start = __shfl(cr.rb, r, kWave);
    const int first = __shfl(cr.incl - cr.rlen, r, kWave);
    return k < cr.total ? atoms_sorted[start + (k - first)] : -1;
}

// Calls f(j) for every candidate j of atom i (each j at most once), lanes in parallel.
template <typename T, typename F>
__device__ __forceinline__ void for_candidates(const T* pos, int i, int64_t n, const NlGrid& g,
                                               const int32_t* __restrict__ cell_start,
                                               const int32_t* __restrict__ atoms_sorted, int mode, F&& f) {
    const int lane = threadIdx.x & (kWave - 1);
    if (g.brute) {
        const int64_t end = mode == MNX_NLIST_HALF ? i : n;
        for (int64_t base = 0; base < end; base += kWave) {
            const int64_t j = base + lane;
            f(j < end && j != i ? int(j) : -1);
        }
        return;
    }
    int c[3];
    cell_coords<T>(pos, i, g, c);
    const CellRanges cr = cell_ranges(g, c[0], c[1], c[2], cell_start, lane);
    for (int base = 0; base < cr.total; base += kWave) {
        int j = cell_candidate(cr, base + lane, atoms_sorted);
        if (mode == MNX_NLIST_HALF ? j >= i : j == i) j = -1;
        f(j);
    }
}

// All-pairs fallback (a periodic axis with fewer than 3 cells): one wavefront per atom,
// grid-stride; cell grids are handled by k_count_cells / k_emit_cells.
template <typename T>
__global__ void __launch_bounds__(kWave) k_count(const T* __restrict__ pos, int64_t n, const T* __restrict__ box,
                                                 T cutoff, int mode, NlGrid* __restrict__ gp,
                                                 const int32_t* __restrict__ cell_start,
                                                 const int32_t* __restrict__ atoms_sorted,
                                                 int32_t* __restrict__ counts) {
    const NlGrid g = *gp;
    if (!g.brute) return;
    const bool periodic = g.periodic;
    const AcceptTest<T> at = accept_test<T>(box, periodic, true, cutoff);
    for (int i = blockIdx.x; i < n; i += gridDim.x) {
        int count = 0;
        for_candidates<T>(pos, i, n, g, cell_start, atoms_sorted, mode, [&](int j) {
            const bool ok = j >= 0 && accept<T>(pos, box, i, j, periodic, cutoff, at);
            count += __popcll(__ballot(ok));
        });
        if (threadIdx.x == 0) {
            counts[i] = count;
            if (count > kNlCap) atomicExch(&gp->overflow, 1);
        }
    }
}

// Bitonic sort of `len` ints in LDS (len <= kNlCap), ascending; pads with INT_MAX.
__device__ void lds_sort(int32_t* buf, int len) {
    int m = 1;
    while (m < len) m <<= 1;
    const int lane = threadIdx.x;
    for (int k = len + lane; k < m; k += kWave) buf[k] = 0x7fffffff;
    __syncthreads();
    for (int size = 2; size <= m; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int t = lane; t < (m >> 1); t += kWave) {
                const int lo = 2 * t - (t & (stride - 1));
                const int hi = lo + stride;
                const bool up = (lo & size) == 0;
                const int a = buf[lo], b = buf[hi];
                if ((a > b) == up) {
                    buf[lo] = b;
                    buf[hi] = a;
                }
            }
            __syncthreads();
        }
    }
}

// Writes pair (i, j) at `slot` with the reference geometry (row = the larger index).
template <typename T>
__device__ __forceinline__ void write_pair(const T* __restrict__ pos, const T* __restrict__ box, bool periodic, int i,
                                           int j, int64_t slot, int32_t* __restrict__ idx_i,
                                           int32_t* __restrict__ idx_j, T* __restrict__ deltas,
                                           T* __restrict__ dist, T* __restrict__ shifts) {
    Geo<T> gg;
    const bool flip = i < j;
    pair_geo<T>(pos, box, flip ? j : i, flip ? i : j, periodic, shifts != nullptr, gg);
    if (idx_i) idx_i[slot] = i;
    if (idx_j) idx_j[slot] = j;
    if (deltas) {
        deltas[3 * slot + 0] = flip ? -gg.d[0] : gg.d[0];
        deltas[3 * slot + 1] = flip ? -gg.d[1] : gg.d[1];
        deltas[3 * slot + 2] = flip ? -gg.d[2] : gg.d[2];
    }
    if (dist) dist[slot] = gg.dist;
    if (shifts) {
        shifts[3 * slot + 0] = flip ? -gg.shift[0] : gg.shift[0];
        shifts[3 * slot + 1] = flip ? -gg.shift[1] : gg.shift[1];
        shifts[3 * slot + 2] = flip ? -gg.shift[2] : gg.shift[2];
    }
}

template <typename T>
__global__ void __launch_bounds__(kWave) k_emit(const T* __restrict__ pos, int64_t n, const T* __restrict__ box,
                                                T cutoff, int mode, int layout, const NlGrid* __restrict__ gp,
                                                const int32_t* __restrict__ cell_start,
                                                const int32_t* __restrict__ atoms_sorted,
                                                const int32_t* __restrict__ big,
                                                const int64_t* __restrict__ offsets, int64_t capacity,
                                                int32_t* __restrict__ idx_i, int32_t* __restrict__ idx_j,
                                                T* __restrict__ deltas, T* __restrict__ dist,
                                                T* __restrict__ shifts) {
    __shared__ int32_t buf[kNlCap];
    const NlGrid g = *gp;
    // brute grids: every atom; cell grids: the atoms the cell emit leaves (> kEmitBuf
    // neighbours, listed by the count pass)
    const bool only_big = !g.brute;
    const int64_t items = only_big ? g.nbig : n;
    const bool periodic = g.periodic;
    const int lane = threadIdx.x;
    const AcceptTest<T> at = accept_test<T>(box, periodic, true, cutoff);
    for (int64_t t = blockIdx.x; t < items; t += gridDim.x) {
        const int i = only_big ? big[t] : int(t);
        int count = 0;
        __syncthreads();  // buf is reused across atoms
        for_candidates<T>(pos, i, n, g, cell_start, atoms_sorted, mode, [&](int j) {
            const bool ok = j >= 0 && accept<T>(pos, box, i, j, periodic, cutoff, at);
            const uint64_t m = __ballot(ok);
            const int before = __popcll(m & ((uint64_t(1) << lane) - 1));
            if (ok && count + before < kNlCap) buf[count + before] = j;
            count += __popcll(m);
        });
        if (count > kNlCap) count = kNlCap;  // flagged by k_count; host reports the error
        __syncthreads();
        lds_sort(buf, count);
        const int64_t base = layout == MNX_NLIST_TRIANGULAR ? 0 : offsets[i];
        for (int k = lane; k < count; k += kWave) {
            const int j = buf[k];
            const int64_t slot = layout == MNX_NLIST_TRIANGULAR ? int64_t(i) * (i - 1) / 2 + j : base + k;
            if (slot < capacity) write_pair<T>(pos, box, periodic, i, j, slot, idx_i, idx_j, deltas, dist, shifts);
        }
    }
}

// ---------------------------------------------------------------------------
// Cell grids: kCellParts wavefronts per cell, each taking every kCellParts-th atom of
// the cell as a "centre".  All centres share the 27 neighbour cells, so each
// candidate position is loaded once per wavefront and tested against all of its
// centres (whose coordinates are wave-uniform).  Grid-stride over (cell, part); the
// all-pairs fallback (k_count / k_emit) handles brute-force grids.
// ---------------------------------------------------------------------------

__device__ __forceinline__ int64_t cell_of_block(int64_t c, const NlGrid& g, int* cx, int* cy, int* cz) {
    *cx = int(c % g.n[0]);
    *cy = int((c / g.n[0]) % g.n[1]);
    *cz = int(c / (int64_t(g.n[0]) * g.n[1]));
    return c;
}

// Slot (index into the cell-ordered arrays) of candidate number k of the flattened ranges,
// -1 past the end, and in *cell the neighbour-cell lane (0..26) it comes from; every lane must
// call it.
__device__ __forceinline__ int cell_candidate_slot(const CellRanges& cr, int k, int* cell) {
    int r = 0;
#pragma unroll
    for (int step = 16; step > 0; step >>= 1) {
        const int probe = __shfl(cr.incl, r + step - 1, kWave);
        if (r + step <= 26 && probe <= k) r += step;
    }
    const int start = __shfl(cr.rb, r, kWave);
    const int first = __shfl(cr.incl - cr.rlen, r, kWave);
    *cell = r;
    return k < cr.total ? start + (k - first) : -1;
}

// The count pass screens each (centre, candidate) pair by the squared distance between the
// centre's position in the primary cell and the candidate's, moved by the box vectors that
// wrap its neighbour cell next to the centre's cell.  With >= 3 cells of width >= the cutoff
// along every periodic axis this is the minimum image for every pair within the cutoff (any
// other image is more than twice the cutoff away).  Pairs clear of cutoff^2 by a relative
// 1e-3 are settled by it -- the rounding of the wrapped positions is orders of magnitude
// smaller -- and the reference arithmetic on the original positions decides the band and
// zero distances, so the accepted set is the reference's.
template <typename T, bool HALF>
__global__ void __launch_bounds__(kWave) k_count_cells(const T* __restrict__ pos, const T* __restrict__ box, T cutoff,
                                                       NlGrid* __restrict__ gp, const int32_t* __restrict__ cell_start,
                                                       const int32_t* __restrict__ atoms_sorted,
                                                       const PosW<T>* __restrict__ posw,
                                                       int32_t* __restrict__ counts, int32_t* __restrict__ big,
                                                       uint64_t* __restrict__ masks) {
    const NlGrid g = *gp;
    if (g.brute) return;
    const int lane = threadIdx.x;
    const bool periodic = g.periodic;
    const T c2 = cutoff * cutoff;
    const T c2lo = c2 * T(0.999), c2hi = c2 * T(1.001), c2tiny = c2 * T(1e-20);
    for (int64_t v = blockIdx.x; v < g.ncells * kCellParts; v += gridDim.x) {
        const int64_t c = v / kCellParts;
        const int part = int(v - c * kCellParts);
        const int cb = cell_start[c], ce = cell_start[c + 1];
        const int ncent = (ce - cb - part + kCellParts - 1) / kCellParts;  // centres part, part + P, ...
        if (ncent <= 0) continue;
        int cx, cy, cz;
        cell_of_block(c, g, &cx, &cy, &cz);
        const CellRanges cr = cell_ranges(g, cx, cy, cz, cell_start, lane);
        // lanes 0..26: the box vectors that bring neighbour cell `lane` next to this cell
        T shx = T(0), shy = T(0), shz = T(0);
        if (periodic && lane < 27) {
            const int z = cz + lane / 9 - 1, y = cy + (lane / 3) % 3 - 1, x = cx + lane % 3 - 1;
            const int wz = z < 0 ? -1 : (z >= g.n[2] ? 1 : 0), wy = y < 0 ? -1 : (y >= g.n[1] ? 1 : 0),
                      wx = x < 0 ? -1 : (x >= g.n[0] ? 1 : 0);
            shx = T(wx) * box[0] + T(wy) * box[3] + T(wz) * box[6];
            shy = T(wy) * box[4] + T(wz) * box[7];
            shz = T(wz) * box[8];
        }
        for (int q0 = 0; q0 < ncent; q0 += kWave) {
            const int nq = ncent - q0 < kWave ? ncent - q0 : kWave;
            const int my_slot = lane < nq ? cb + part + (q0 + lane) * kCellParts : -1;
            const int my_i = my_slot >= 0 ? atoms_sorted[my_slot] : -1;
            PosW<T> mp{T(0), T(0), T(0), T(0)};
            if (my_slot >= 0) mp = posw[my_slot];
            int my_count = 0;
            const bool keep_masks = cr.total <= kWave * kMaskChunks;  // wave-uniform
            for (int base = 0; base < cr.total; base += kWave) {
                int r;
                const int slot = cell_candidate_slot(cr, base + lane, &r);
                const T sx = __shfl(shx, r, kWave), sy = __shfl(shy, r, kWave), sz = __shfl(shz, r, kWave);
                const int j = slot >= 0 ? atoms_sorted[slot] : -1;
                PosW<T> jp{T(0), T(0), T(0), T(0)};
                if (slot >= 0) jp = posw[slot];
                const T jx = jp.x + sx, jy = jp.y + sy, jz = jp.z + sz;
                for (int q = 0; q < nq; ++q) {
                    const int i = lane_value(my_i, q);
                    const T dx = lane_value(mp.x, q) - jx, dy = lane_value(mp.y, q) - jy,
                            dz = lane_value(mp.z, q) - jz;
                    const T r2 = dx * dx + dy * dy + dz * dz;
                    bool ok = j >= 0 && (HALF ? j < i : j != i) && !(r2 > c2hi);
                    if (ok && !(r2 < c2lo && r2 > c2tiny)) {
                        // the band around the cutoff and (near-)zero distances: reference arithmetic
                        Geo<T> gg;
                        pair_geo<T>(pos, box, i, j, periodic, false, gg);
                        ok = gg.dist <= cutoff && gg.dist > T(0);
                    }
                    const uint64_t m = __ballot(ok);
                    if (lane == q) {
                        my_count += __popcll(m);
                        if (keep_masks) masks[int64_t(my_i) * kMaskChunks + base / kWave] = m;
                    }
                }
            }
            if (lane < nq) {
                counts[my_i] = my_count;
                if (my_count > kNlCap) atomicExch(&gp->overflow, 1);
                if (my_count > kEmitBuf) big[atomicAdd(&gp->nbig, 1)] = my_i;
            }
        }
    }
}

template <typename T>
__global__ void __launch_bounds__(kWave) k_emit_cells(const T* __restrict__ pos, const T* __restrict__ box, T cutoff,
                                                      int mode, int layout, const NlGrid* __restrict__ gp,
                                                      const int32_t* __restrict__ cell_start,
                                                      const int32_t* __restrict__ atoms_sorted,
                                                      const int32_t* __restrict__ counts,
                                                      const uint64_t* __restrict__ masks,
                                                      const int64_t* __restrict__ offsets, int64_t capacity,
                                                      int32_t* __restrict__ idx_i, int32_t* __restrict__ idx_j,
                                                      T* __restrict__ deltas, T* __restrict__ dist,
                                                      T* __restrict__ shifts) {
    __shared__ int32_t buf[kEmitBuf];  // accepted j of a batch of centres, one segment per centre
    const NlGrid g = *gp;
    if (g.brute) return;
    const int lane = threadIdx.x;
    const bool periodic = g.periodic;
    const AcceptTest<T> at = accept_test<T>(box, periodic, false, cutoff);
    for (int64_t v = blockIdx.x; v < g.ncells * kCellParts; v += gridDim.x) {
        const int64_t c = v / kCellParts;
        const int part = int(v - c * kCellParts);
        const int cb = cell_start[c], ce = cell_start[c + 1];
        const int ncent = (ce - cb - part + kCellParts - 1) / kCellParts;  // centres part, part + P, ...
        if (ncent <= 0) continue;
        int cx, cy, cz;
        cell_of_block(c, g, &cx, &cy, &cz);
        const CellRanges cr = cell_ranges(g, cx, cy, cz, cell_start, lane);
        // as in the count pass: the candidate ids of up to kPreChunks chunks loaded at once
        const int nchunks = (cr.total + kWave - 1) / kWave;  // wave-uniform
        const bool pre = nchunks <= kPreChunks;               // implies the count pass kept the masks
        int jr[kPreChunks];
        if (pre) {
#pragma unroll
            for (int b = 0; b < kPreChunks; ++b) jr[b] = b < nchunks ? cell_candidate(cr, b * kWave + lane, atoms_sorted) : -1;
        }
        for (int q0 = 0; q0 < ncent;) {
            // a batch of centres whose segments fit the buffer (kEmitBuf entries)
            const int avail = ncent - q0 < kWave ? ncent - q0 : kWave;
            const int my_i = lane < avail ? atoms_sorted[cb + part + (q0 + lane) * kCellParts] : -1;
            // centres with more than kEmitBuf neighbours take no buffer space here (per-atom emit)
            const int cnt_i = lane < avail ? counts[my_i] : 0;
            const int my_cnt = cnt_i > kEmitBuf ? 0 : cnt_i;
            const T mx = my_i >= 0 ? pos[3 * my_i] : T(0), my = my_i >= 0 ? pos[3 * my_i + 1] : T(0),
                    mz = my_i >= 0 ? pos[3 * my_i + 2] : T(0);
            int incl = my_cnt;
#pragma unroll
            for (int o = 1; o < kWave; o <<= 1) {
                const int v = __shfl_up(incl, o, kWave);
                if (lane >= o) incl += v;
            }
            int nq = __popcll(__ballot(lane < avail && incl <= kEmitBuf));  // incl is non-decreasing
            if (nq == 0) nq = 1;
            const int my_off = incl - my_cnt;
            int my_fill = 0;
            __syncthreads();  // previous batch's segments fully read
            // the count pass left each centre's accept ballots (the same candidates in the same
            // order): reuse them instead of testing again, unless the cell had too many candidates
            const bool use_masks = cr.total <= kWave * kMaskChunks;  // wave-uniform
            // appends candidate j (accepted or not by this lane's `ok`) to centre q's segment
            auto place = [&](int q, int j, bool ok) {
                const int seg = lane_value(my_off, q);
                const int cap = lane_value(my_cnt, q);
                const int fill = lane_value(my_fill, q);
                const uint64_t m = __ballot(ok);
                const int before = __popcll(m & ((uint64_t(1) << lane) - 1));
                if (ok && fill + before < cap) buf[seg + fill + before] = j;
                if (lane == q) my_fill += __popcll(m);
            };
            if (pre) {
                // each lane holds its own centre's ballots of every chunk; centre q's are read
                // from lane q, and its segment is filled chunk after chunk with a uniform count
                uint64_t mk[kPreChunks];
#pragma unroll
                for (int b = 0; b < kPreChunks; ++b)
                    mk[b] = (b < nchunks && my_i >= 0) ? masks[int64_t(my_i) * kMaskChunks + b] : 0;
                const uint64_t below = (uint64_t(1) << lane) - 1;
                for (int q = 0; q < nq; ++q) {
                    const int seg = lane_value(my_off, q);
                    const int cap = lane_value(my_cnt, q);
                    int fill = 0;
#pragma unroll
                    for (int b = 0; b < kPreChunks; ++b) {
                        if (b < nchunks) {
                            const uint64_t m = lane_value(mk[b], q);
                            const int at = fill + __popcll(m & below);
                            if (((m >> lane) & 1) && at < cap) buf[seg + at] = jr[b];
                            fill += __popcll(m);
                        }
                    }
                    if (lane == q) my_fill = fill;
                }
            } else {
                for (int base = 0; base < cr.total; base += kWave) {
                    const int j = cell_candidate(cr, base + lane, atoms_sorted);
                    T jx = T(0), jy = T(0), jz = T(0);
                    if (!use_masks && j >= 0) {
                        jx = pos[3 * j];
                        jy = pos[3 * j + 1];
                        jz = pos[3 * j + 2];
                    }
                    for (int q = 0; q < nq; ++q) {
                        const int i = lane_value(my_i, q);
                        bool ok;
                        if (use_masks) {
                            const uint64_t cm =
                                masks[int64_t(__builtin_amdgcn_readfirstlane(i)) * kMaskChunks + base / kWave];
                            ok = (cm >> lane) & 1;
                        } else {
                            const bool keep = j >= 0 && (mode == MNX_NLIST_HALF ? j < i : j != i);
                            ok = keep && accept_xyz<T>(box, lane_value(mx, q), lane_value(my, q), lane_value(mz, q),
                                                       jx, jy, jz, periodic, cutoff, at);
                        }
                        place(q, j, ok);
                    }
                }
            }
            __syncthreads();
            // each centre's segment, ranked by j (the j are distinct), written at its offset
            for (int q = 0; q < nq; ++q) {
                const int i = lane_value(my_i, q);
                const int seg = lane_value(my_off, q);
                // entries actually written (equal to the count pass's unless it overflowed)
                const int cap = lane_value(my_cnt, q);
                const int got = lane_value(my_fill, q);
                const int len = got < cap ? got : cap;
                const int64_t obase = layout == MNX_NLIST_TRIANGULAR ? 0 : offsets[i];
                if (len <= kWave) {
                    // one element per lane, bitonic-sorted across the wavefront, written in order
                    int v = lane < len ? buf[seg + lane] : INT32_MAX;
#pragma unroll
                    for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
                        for (int stride = size >> 1; stride > 0; stride >>= 1) {
                            const int other = lane_xor(v, stride);
                            const bool up = (lane & size) == 0 || size == kWave;
                            const bool low = (lane & stride) == 0;
                            v = (low == up) ? min(v, other) : max(v, other);
                        }
                    }
                    if (lane < len) {
                        const int64_t slot =
                            layout == MNX_NLIST_TRIANGULAR ? int64_t(i) * (i - 1) / 2 + v : obase + lane;
                        if (slot < capacity) write_pair<T>(pos, box, periodic, i, v, slot, idx_i, idx_j, deltas, dist,
                                                           shifts);
                    }
                } else {
                    for (int k = lane; k < len; k += kWave) {
                        const int v = buf[seg + k];
                        int rank = 0;
                        for (int t = 0; t < len; ++t) rank += buf[seg + t] < v ? 1 : 0;
                        const int64_t slot =
                            layout == MNX_NLIST_TRIANGULAR ? int64_t(i) * (i - 1) / 2 + v : obase + rank;
                        if (slot < capacity) write_pair<T>(pos, box, periodic, i, v, slot, idx_i, idx_j, deltas, dist,
                                                           shifts);
                    }
                }
            }
            q0 += nq;
        }
    }
}

// Reference padding (-1 / NaN) for slots [from, capacity); `from` read from device when from_dev != null.
template <typename T>
__global__ void k_pad(int64_t from_host, const int64_t* __restrict__ from_dev, int64_t capacity,
                      int32_t* __restrict__ idx_i, int32_t* __restrict__ idx_j, T* __restrict__ deltas,
                      T* __restrict__ dist, T* __restrict__ shifts) {
    const int64_t from = from_dev ? *from_dev : from_host;
    const T nan = T(NAN);
    for (int64_t s = from + int64_t(blockIdx.x) * blockDim.x + threadIdx.x; s < capacity;
         s += int64_t(gridDim.x) * blockDim.x) {
        if (s < 0) continue;
        if (idx_i) idx_i[s] = -1;
        if (idx_j) idx_j[s] = -1;
        if (deltas) deltas[3 * s] = deltas[3 * s + 1] = deltas[3 * s + 2] = nan;
        if (dist) dist[s] = nan;
        if (shifts) shifts[3 * s] = shifts[3 * s + 1] = shifts[3 * s + 2] = nan;
    }
}

// Zeroes the per-cell counters and the grid header.
__global__ void k_nl_clear(int32_t* __restrict__ cell_count, int32_t* __restrict__ cell_fill, int64_t ncells,
                           int32_t* __restrict__ grid_words, int64_t ngrid) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < ncells) {
        cell_count[i] = 0;
        cell_fill[i] = 0;
    }
    if (i < ngrid) grid_words[i] = 0;
}

// *d_total = pair count, or -1 when some atom exceeded kNlCap neighbours.
__global__ void k_report_total(const NlGrid* __restrict__ gp, const int64_t* __restrict__ total,
                               int64_t* __restrict__ d_total) {
    *d_total = gp->overflow ? int64_t(-1) : *total;
}

template <typename T>
int nlist_count(const T* pos, int64_t n, double cutoff, const T* box, int mode, void* ws, size_t ws_bytes,
                int64_t* d_total, hipStream_t stream) {
    clear_error();
    MNX_REQUIRE(n >= 0 && n < (int64_t(1) << 31), "num_atoms out of range: %lld", (long long)n);
    MNX_REQUIRE(mode == MNX_NLIST_HALF || mode == MNX_NLIST_FULL, "bad mode %d", mode);
    MNX_REQUIRE(n == 0 || pos, "positions is null");
    MNX_REQUIRE(cutoff > 0, "cutoff must be positive");
    size_t need = 0;
    NlWs w = carve(ws, ws_bytes, n, &need);
    if (ws_bytes < need || !ws) return set_error(MNX_ERR_WORKSPACE, "workspace %zu < %zu bytes", ws_bytes, need);
    {
        // cleared by a kernel rather than hipMemsetAsync, so the sequence can sit in a captured HIP graph
        const int64_t ng = int64_t(sizeof(NlGrid) / sizeof(int32_t));
        const int64_t m = w.max_cells > ng ? w.max_cells : ng;
        hipLaunchKernelGGL(k_nl_clear, dim3(ceil_div(m, 256)), dim3(256), 0, stream, w.cell_count, w.cell_fill,
                           int64_t(w.max_cells), reinterpret_cast<int32_t*>(w.grid), ng);
        MNX_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL((k_grid_setup<T>), dim3(1), dim3(1024), 0, stream, pos, n, box, cutoff, w.max_cells, w.grid);
    MNX_CHECK_LAUNCH();
    if (n > 0) {
        const int tb = 256;
        hipLaunchKernelGGL((k_bin<T>), dim3(ceil_div(n, tb)), dim3(tb), 0, stream, pos, n, w.grid, w.cell_of, w.cell_count);
        MNX_CHECK_LAUNCH();
    }
    int rc = exclusive_scan<int32_t, int32_t>(w.cell_count, w.max_cells, w.cell_start, w.tiles32,
                                              w.cell_start + w.max_cells, stream);
    if (rc) return rc;
    if (n > 0) {
        const int tb = 256;
        // place into `counts` (free until the count pass), then rank within each cell
        hipLaunchKernelGGL(k_place, dim3(ceil_div(n, tb)), dim3(tb), 0, stream, n, w.cell_of, w.cell_start,
                           w.cell_fill, w.counts);
        MNX_CHECK_LAUNCH();
        PosW<T>* posw = static_cast<PosW<T>*>(w.posw);
        hipLaunchKernelGGL((k_rank_cells<T>), dim3(ceil_div(n, tb)), dim3(tb), 0, stream, n, pos, box, w.grid,
                           w.cell_of, w.cell_start, w.counts, w.atoms_sorted, posw);
        MNX_CHECK_LAUNCH();
        const unsigned blocks = unsigned(std::min<int64_t>(std::max<int64_t>(n, w.max_cells * kCellParts), kNlBlocks));
        if (mode == MNX_NLIST_HALF)
            hipLaunchKernelGGL((k_count_cells<T, true>), dim3(blocks), dim3(kWave), 0, stream, pos, box, T(cutoff),
                               w.grid, w.cell_start, w.atoms_sorted, posw, w.counts, w.big, w.masks);
        else
            hipLaunchKernelGGL((k_count_cells<T, false>), dim3(blocks), dim3(kWave), 0, stream, pos, box, T(cutoff),
                               w.grid, w.cell_start, w.atoms_sorted, posw, w.counts, w.big, w.masks);
        MNX_CHECK_LAUNCH();
        hipLaunchKernelGGL((k_count<T>), dim3(blocks), dim3(kWave), 0, stream, pos, n, box, T(cutoff), mode, w.grid,
                           w.cell_start, w.atoms_sorted, w.counts);
        MNX_CHECK_LAUNCH();
    }
    rc = exclusive_scan<int32_t, int64_t>(w.counts, n, w.offsets, w.tiles64, w.total, stream);
    if (rc) return rc;
    if (d_total) {
        hipLaunchKernelGGL(k_report_total, dim3(1), dim3(1), 0, stream, w.grid, w.total, d_total);
        MNX_CHECK_LAUNCH();
    }
    return MNX_OK;
}

template <typename T>
int nlist_emit(const T* pos, int64_t n, double cutoff, const T* box, int mode, int layout, const void* ws,
               size_t ws_bytes, int64_t capacity, int32_t* idx_i, int32_t* idx_j, T* deltas, T* dist, T* shifts,
               hipStream_t stream) {
    clear_error();
    MNX_REQUIRE(capacity >= 0, "capacity must be >= 0");
    MNX_REQUIRE(layout == MNX_NLIST_COMPACT || (layout == MNX_NLIST_TRIANGULAR && mode == MNX_NLIST_HALF),
                "triangular layout needs the half list");
    size_t need = 0;
    NlWs w = carve(const_cast<void*>(ws), ws_bytes, n, &need);
    if (ws_bytes < need || !ws) return set_error(MNX_ERR_WORKSPACE, "workspace %zu < %zu bytes", ws_bytes, need);
    if (capacity == 0) return MNX_OK;
    const int tb = 256;
    const int64_t pad_blocks = std::min<int64_t>(ceil_div(capacity, tb), 65536);
    if (layout == MNX_NLIST_TRIANGULAR) {
        hipLaunchKernelGGL((k_pad<T>), dim3(pad_blocks), dim3(tb), 0, stream, int64_t(0), (const int64_t*)nullptr,
                           capacity, idx_i, idx_j, deltas, dist, shifts);
        MNX_CHECK_LAUNCH();
    } else {
        hipLaunchKernelGGL((k_pad<T>), dim3(pad_blocks), dim3(tb), 0, stream, int64_t(0), (const int64_t*)w.total,
                           capacity, idx_i, idx_j, deltas, dist, shifts);
        MNX_CHECK_LAUNCH();
    }
    if (n > 0) {
        const unsigned blocks = unsigned(std::min<int64_t>(std::max<int64_t>(n, w.max_cells * kCellParts), kNlBlocks));
        hipLaunchKernelGGL((k_emit_cells<T>), dim3(blocks), dim3(kWave), 0, stream, pos, box, T(cutoff), mode, layout,
                           w.grid, w.cell_start, w.atoms_sorted, w.counts, w.masks, w.offsets, capacity, idx_i, idx_j,
                           deltas, dist, shifts);
        MNX_CHECK_LAUNCH();
        hipLaunchKernelGGL((k_emit<T>), dim3(blocks), dim3(kWave), 0, stream, pos, n, box, T(cutoff), mode, layout,
                           w.grid, w.cell_start, w.atoms_sorted, w.big, w.offsets, capacity, idx_i, idx_j, deltas,
                           dist, shifts);
        MNX_CHECK_LAUNCH();
    }
    return MNX_OK;
}

template <typename T>
__global__ void k_nl_backward(const int32_t* __restrict__ ii, const int32_t* __restrict__ jj,
                              const T* __restrict__ d, const T* __restrict__ dist, const T* __restrict__ gd,
                              const T* __restrict__ gdist, int64_t slots, T* __restrict__ gpos) {
    const int64_t s = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (s >= slots) return;
    const int i = ii[s], j = jj[s];
    if (i < 0 || j < 0) return;
    const T inv = T(1) / dist[s];
    const T gds = gdist ? gdist[s] : T(0);
    for (int k = 0; k < 3; ++k) {
        T g = (gd ? gd[3 * s + k] : T(0)) + d[3 * s + k] * inv * gds;
        atomicAdd(&gpos[3 * i + k], g);
        atomicAdd(&gpos[3 * j + k], -g);
    }
}

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

size_t mnx_nlist_workspace_bytes(int64_t num_atoms) {
    size_t used = 0;
    carve(nullptr, 0, num_atoms < 0 ? 0 : num_atoms, &used);
    return used + 256;
}

int mnx_nlist_count_f32(const float* pos, int64_t n, double cutoff, const float* box, int32_t mode, void* ws,
                        size_t ws_bytes, int64_t* d_total, mnx_stream_t stream) {
    return nlist_count<float>(pos, n, cutoff, box, mode, ws, ws_bytes, d_total, (hipStream_t)stream);
}
int mnx_nlist_count_f64(const double* pos, int64_t n, double cutoff, const double* box, int32_t mode, void* ws,
                        size_t ws_bytes, int64_t* d_total, mnx_stream_t stream) {
    return nlist_count<double>(pos, n, cutoff, box, mode, ws, ws_bytes, d_total, (hipStream_t)stream);
}
int mnx_nlist_emit_f32(const float* pos, int64_t n, double cutoff, const float* box, int32_t mode, int32_t layout,
                       const void* ws, size_t ws_bytes, int64_t capacity, int32_t* idx_i, int32_t* idx_j,
                       float* deltas, float* distances, float* shifts, mnx_stream_t stream) {
    return nlist_emit<float>(pos, n, cutoff, box, mode, layout, ws, ws_bytes, capacity, idx_i, idx_j, deltas,
                             distances, shifts, (hipStream_t)stream);
}
int mnx_nlist_emit_f64(const double* pos, int64_t n, double cutoff, const double* box, int32_t mode,
                       int32_t layout, const void* ws, size_t ws_bytes, int64_t capacity, int32_t* idx_i,
                       int32_t* idx_j, double* deltas, double* distances, double* shifts, mnx_stream_t stream) {
    return nlist_emit<double>(pos, n, cutoff, box, mode, layout, ws, ws_bytes, capacity, idx_i, idx_j, deltas,
                              distances, shifts, (hipStream_t)stream);
}

int mnx_nlist_backward_f32(const int32_t* idx_i, const int32_t* idx_j, const float* deltas, const float* distances,
                           const float* grad_deltas, const float* grad_distances, int64_t num_slots,
                           int64_t num_atoms, float* grad_pos, mnx_stream_t stream) {
    clear_error();
    (void)num_atoms;
    if (num_slots <= 0) return MNX_OK;
    const int tb = 256;
    hipLaunchKernelGGL((k_nl_backward<float>), dim3(ceil_div(num_slots, tb)), dim3(tb), 0, (hipStream_t)stream,
                       idx_i, idx_j, deltas, distances, grad_deltas, grad_distances, num_slots, grad_pos);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_nlist_backward_f64(const int32_t* idx_i, const int32_t* idx_j, const double* deltas, const double* distances,
                           const double* grad_deltas, const double* grad_distances, int64_t num_slots,
                           int64_t num_atoms, double* grad_pos, mnx_stream_t stream) {
    clear_error();
    (void)num_atoms;
    if (num_slots <= 0) return MNX_OK;
    const int tb = 256;
    hipLaunchKernelGGL((k_nl_backward<double>), dim3(ceil_div(num_slots, tb)), dim3(tb), 0, (hipStream_t)stream,
                       idx_i, idx_j, deltas, distances, grad_deltas, grad_distances, num_slots, grad_pos);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

}  // extern "C"
