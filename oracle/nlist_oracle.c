/*
 * TEST INFRASTRUCTURE ONLY -- the parity oracle for the neighbor list.  Never
 * linked into or called by the product path.
 *
 * Plain-C restatement of the reference CPU op molix::get_neighbor_pairs
 * (/root/reference/src/molix/op/src/neighbors/get_neighbor_pairs.cpp:28-77),
 * rounding every operation the way that tensorised code does:
 *   rows/cols enumerated as row > col, row-major            (.cpp:38-43)
 *   d = pos[row] - pos[col]                                  (.cpp:44)
 *   for k = 2, 1, 0: s = nearbyint(d[k] / box[k][k]);        (.cpp:46-48; torch::round
 *                    d[c] -= s * box[k][c] for c = 0..2       rounds half to even)
 *   dist = sqrt(fma(d2, d2, fma(d1, d1, d0 * d0)))           (.cpp:50; ATen's fp norm
 *                                                              kernel accumulates with fma)
 *   keep iff dist <= cutoff && dist > 0                      (.cpp:52)
 * The fma-chain form of the norm was established against the compiled
 * reference (tests/golden/make_nlist_golden.py records it in the fixtures).
 *
 * oracle_nlist_half_*: O(N^2) brute force in the reference's order.
 * oracle_nlist_cells_*: same predicate over a cell list (for large N), pairs
 *                       emitted in the same (row, col) order.
 * Compiled with -ffp-contract=off (oracle/Makefile).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define GEO(T, FMA, RINT, SQRT)                                                                   \
    static void geo_##T(const T* pos, const T* box, int64_t r, int64_t c, T* d, T* dist) {        \
        d[0] = pos[3 * r + 0] - pos[3 * c + 0];                                                   \
        d[1] = pos[3 * r + 1] - pos[3 * c + 1];                                                   \
        d[2] = pos[3 * r + 2] - pos[3 * c + 2];                                                   \
        if (box) {                                                                                \
            for (int k = 2; k >= 0; --k) {                                                        \
                T s = RINT(d[k] / box[4 * k]);                                                    \
                T b0 = s * box[3 * k + 0], b1 = s * box[3 * k + 1], b2 = s * box[3 * k + 2];      \
                d[0] = d[0] - b0;                                                                 \
                d[1] = d[1] - b1;                                                                 \
                d[2] = d[2] - b2;                                                                 \
            }                                                                                     \
        }                                                                                         \
        *dist = SQRT(FMA(d[2], d[2], FMA(d[1], d[1], d[0] * d[0])));                              \
    }

GEO(float, fmaf, nearbyintf, sqrtf)
GEO(double, fma, nearbyint, sqrt)

#define HALF(T)                                                                                   \
    int64_t oracle_nlist_half_##T(const T* pos, int64_t n, double cutoff, const T* box,           \
                                  int64_t cap, int32_t* rows, int32_t* cols, T* deltas, T* dist) { \
        const T cut = (T)cutoff;                                                                  \
        int64_t found = 0;                                                                        \
        for (int64_t r = 1; r < n; ++r)                                                           \
            for (int64_t c = 0; c < r; ++c) {                                                     \
                T d[3], ds;                                                                       \
                geo_##T(pos, box, r, c, d, &ds);                                                  \
                if (!(ds <= cut && ds > 0)) continue;                                             \
                if (found < cap) {                                                                \
                    rows[found] = (int32_t)r;                                                     \
                    cols[found] = (int32_t)c;                                                     \
                    memcpy(deltas + 3 * found, d, sizeof d);                                      \
                    dist[found] = ds;                                                             \
                }                                                                                 \
                ++found;                                                                          \
            }                                                                                     \
        return found;                                                                             \
    }

HALF(float)
HALF(double)

/* ---- cell-accelerated variant (cubic/orthorhombic or open boxes) ---- */

static int cmp_i32(const void* a, const void* b) {
    int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
    return (x > y) - (x < y);
}

#define CELLS(T)                                                                                  \
    int64_t oracle_nlist_cells_##T(const T* pos, int64_t n, double cutoff, const T* box,          \
                                   int64_t cap, int32_t* rows, int32_t* cols, T* deltas, T* dist) { \
        const T cut = (T)cutoff;                                                                  \
        double lo[3], ext[3];                                                                     \
        int nc[3];                                                                                \
        for (int k = 0; k < 3; ++k) {                                                             \
            if (box) {                                                                            \
                lo[k] = 0;                                                                        \
                ext[k] = box[4 * k];                                                              \
            } else {                                                                              \
                double mn = 1e300, mx = -1e300;                                                   \
                for (int64_t i = 0; i < n; ++i) {                                                 \
                    mn = fmin(mn, pos[3 * i + k]);                                                \
                    mx = fmax(mx, pos[3 * i + k]);                                                \
                }                                                                                 \
                lo[k] = n ? mn : 0;                                                               \
                ext[k] = n ? mx - mn : 0;                                                         \
            }                                                                                     \
            nc[k] = (int)floor(ext[k] / (cutoff * 1.001));                                       \
            if (nc[k] < 1) nc[k] = 1;                                                             \
            if (nc[k] > 256) nc[k] = 256;                                                         \
        }                                                                                         \
        if (box && (nc[0] < 3 || nc[1] < 3 || nc[2] < 3 || box[1] != 0 || box[2] != 0 ||        \
                    box[3] != 0 || box[5] != 0 || box[6] != 0 || box[7] != 0))                    \
            return oracle_nlist_half_##T(pos, n, cutoff, box, cap, rows, cols, deltas, dist);     \
        const int64_t ncell = (int64_t)nc[0] * nc[1] * nc[2];                                     \
        int32_t* cell = malloc(sizeof(int32_t) * (n ? n : 1));                                    \
        int32_t* start = calloc(ncell + 1, sizeof(int32_t));                                      \
        int32_t* order = malloc(sizeof(int32_t) * (n ? n : 1));                                   \
        int32_t* buf = malloc(sizeof(int32_t) * (n ? n : 1));                                     \
        int cc[3];                                                                                \
        for (int64_t i = 0; i < n; ++i) {                                                         \
            for (int k = 0; k < 3; ++k) {                                                         \
                double f = ext[k] > 0 ? (pos[3 * i + k] - lo[k]) / ext[k] : 0.0;                  \
                if (box) f -= floor(f);                                                           \
                int c = (int)(f * nc[k]);                                                         \
                cc[k] = c < 0 ? 0 : (c >= nc[k] ? nc[k] - 1 : c);                                \
            }                                                                                     \
            cell[i] = (cc[2] * nc[1] + cc[1]) * nc[0] + cc[0];                                   \
            start[cell[i] + 1]++;                                                                 \
        }                                                                                         \
        for (int64_t c = 0; c < ncell; ++c) start[c + 1] += start[c];                             \
        {                                                                                         \
            int32_t* fill = calloc(ncell, sizeof(int32_t));                                       \
            for (int64_t i = 0; i < n; ++i) order[start[cell[i]] + fill[cell[i]]++] = (int32_t)i; \
            free(fill);                                                                           \
        }                                                                                         \
        int64_t found = 0;                                                                        \
        for (int64_t r = 0; r < n; ++r) {                                                         \
            int m = 0;                                                                            \
            const int c0 = cell[r] % nc[0], c1 = (cell[r] / nc[0]) % nc[1], c2 = cell[r] / (nc[0] * nc[1]); \
            for (int dz = -1; dz <= 1; ++dz)                                                      \
                for (int dy = -1; dy <= 1; ++dy)                                                  \
                    for (int dx = -1; dx <= 1; ++dx) {                                            \
                        int x = c0 + dx, y = c1 + dy, z = c2 + dz;                                \
                        if (box) {                                                                \
                            x = (x + nc[0]) % nc[0];                                              \
                            y = (y + nc[1]) % nc[1];                                              \
                            z = (z + nc[2]) % nc[2];                                              \
                        } else if (x < 0 || y < 0 || z < 0 || x >= nc[0] || y >= nc[1] || z >= nc[2]) \
                            continue;                                                             \
                        const int64_t cid = ((int64_t)z * nc[1] + y) * nc[0] + x;                 \
                        for (int32_t q = start[cid]; q < start[cid + 1]; ++q)                     \
                            if (order[q] < r) buf[m++] = order[q];                                \
                    }                                                                             \
            qsort(buf, m, sizeof(int32_t), cmp_i32);                                              \
            for (int q = 0; q < m; ++q) {                                                         \
                if (q > 0 && buf[q] == buf[q - 1]) continue;                                      \
                T d[3], ds;                                                                       \
                geo_##T(pos, box, r, buf[q], d, &ds);                                             \
                if (!(ds <= cut && ds > 0)) continue;                                             \
                if (found < cap) {                                                                \
                    rows[found] = (int32_t)r;                                                     \
                    cols[found] = buf[q];                                                         \
                    memcpy(deltas + 3 * found, d, sizeof d);                                      \
                    dist[found] = ds;                                                             \
                }                                                                                 \
                ++found;                                                                          \
            }                                                                                     \
        }                                                                                         \
        free(cell);                                                                               \
        free(start);                                                                              \
        free(order);                                                                              \
        free(buf);                                                                                \
        return found;                                                                             \
    }

CELLS(float)
CELLS(double)
