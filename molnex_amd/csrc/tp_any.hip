// Table-driven channelwise tensor product + scatter for irreps that no compiled
// configuration covers (cuet.ChannelWiseTensorProduct over any irreps,
// src/molrep/interaction/tensor_product.py:72-79,101-111): a multiplicity per
// block of the input, any parities (odd couplings such as 1o x 1o -> 1e),
// several blocks of one l, l <= 3.
//
// A path table (passed by value in the kernel arguments) gives per path its
// coupling triple and the offsets of its x block, Y block, output block and
// weight segment, and its multiplicity u:
//
//   out[r][oo + m3*u + c] = sum_{e -> r} w[e][wo + c] sum_{m1,m2} cf[m1][m2][m3]
//                                        x[s][xo + m1*u + c] Y[e][yo + m2]
//
// The per-triple arithmetic (coefficients baked in) comes from gen_tp_any.py;
// the kernels dispatch on the triple once per path.  Lanes are channels.
//
// Forward: one wavefront per (receiver, path, 64-channel chunk), walking the
// receiver's CSR segment with the chunk's output rows in registers; every
// output element is written once (the paths' output blocks tile the row).
// Backward: one wavefront per (receiver, group of consecutive paths reading
// one x block, 64-channel chunk): per edge the block's rows are loaded once,
// every path of the group adds M^T g into registers and grad_x takes one fp32
// atomic per component and channel; grad_w is written per (edge, path,
// channel); grad_Y per (edge, path, chunk) is summed over the lanes by a
// reduce-scatter and added with fp32 atomics (the caller clears grad_x and
// grad_Y).

#include "common.h"
#include "tp_any_gen.inc"
#include "wave.h"

namespace mnx {
namespace {

constexpr int kAnyThreads = 256;
constexpr int kAnyWaves = kAnyThreads / kWave;
constexpr int kAnyMaxPaths = MNX_TP_ANY_MAX_PATHS;
constexpr int kAnyHeader = 5;
constexpr int kAnyFields = 6;

struct TPAnyTable {
    int num_paths, nx, ny, no, nw;
    int type[kAnyMaxPaths], xoff[kAnyMaxPaths], yoff[kAnyMaxPaths], ooff[kAnyMaxPaths], woff[kAnyMaxPaths],
        mul[kAnyMaxPaths];
};

__device__ __forceinline__ int64_t uniform64(int v) { return int64_t(__builtin_amdgcn_readfirstlane(v)); }

template <int T>
__device__ __forceinline__ void any_fwd_walk(int xo, int yo, int oo, int wo, int mul, int c0, int nx, int ny,
                                             int no, int nw, int64_t r, int lane, const float* __restrict__ x,
                                             const float* __restrict__ Y, const float* __restrict__ w,
                                             const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ perm,
                                             const int32_t* __restrict__ senders, float* __restrict__ out) {
    using P = TPAny<T>;
    const int c = c0 + lane;
    const bool ok = c < mul;
    float acc[P::D3] = {};
    const int b = row_ptr[r], end = row_ptr[r + 1];
    for (int k = b; k < end; ++k) {
        const int64_t e = uniform64(perm[k]);
        const int64_t s = uniform64(senders[k]);
        float y[P::D2], xv[P::D1];
#pragma unroll
        for (int m = 0; m < P::D2; ++m) y[m] = Y[e * ny + yo + m];
#pragma unroll
        for (int m = 0; m < P::D1; ++m) xv[m] = ok ? x[s * nx + xo + m * mul + c] : 0.f;
        const float wv = ok ? w[e * nw + wo + c] : 0.f;
        P::fwd(y, xv, wv, acc);
    }
    if (!ok) return;
#pragma unroll
    for (int m = 0; m < P::D3; ++m) out[r * no + oo + m * mul + c] = acc[m];
}

__global__ void __launch_bounds__(kAnyThreads) k_tp_any_fwd(const TPAnyTable tb, const float* __restrict__ x,
                                                            const float* __restrict__ Y,
                                                            const float* __restrict__ w,
                                                            const int32_t* __restrict__ row_ptr,
                                                            const int32_t* __restrict__ perm,
                                                            const int32_t* __restrict__ senders, int64_t N,
                                                            float* __restrict__ out) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t r = int64_t(blockIdx.x) * kAnyWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (r >= N) return;
    // work item blockIdx.y -> (path, channel chunk)
    int rem = blockIdx.y, p = 0;
    for (; p < tb.num_paths; ++p) {
        const int nch = (tb.mul[p] + kWave - 1) / kWave;
        if (rem < nch) break;
        rem -= nch;
    }
    if (p >= tb.num_paths) return;
    const int xo = tb.xoff[p], yo = tb.yoff[p], oo = tb.ooff[p], wo = tb.woff[p], mul = tb.mul[p];
#define MNX_ANY_FWD(T)                                                                                     \
    any_fwd_walk<T>(xo, yo, oo, wo, mul, rem * kWave, tb.nx, tb.ny, tb.no, tb.nw, r, lane, x, Y, w, row_ptr, \
                    perm, senders, out)
    MNX_TP_ANY_SWITCH(tb.type[p], MNX_ANY_FWD)
#undef MNX_ANY_FWD
}

// One path of the backward for edge e, the x block's values xv already loaded: v = M^T g folded
// into the group's grad_x accumulator, the weight gradient written, this path's share of
// grad_Y[e] summed over the lanes (reduce-scatter without LDS) and added by the lanes holding a sum.
// Paths whose input l differs from the group's compile to nothing (never selected).
template <int T, int L1>
__device__ __forceinline__ void any_bwd_step(int yo, int oo, int wo, int mul, int c, bool ok, int ny, int no, int nw,
                                             int64_t r, int64_t e, int lane, const float* xv,
                                             const float* __restrict__ Y, const float* __restrict__ w,
                                             const float* __restrict__ go, float* __restrict__ gY,
                                             float* __restrict__ gw, float* gacc) {
    if constexpr (TPAny<T>::L1 == L1) {
        using P = TPAny<T>;
        float y[P::D2], g[P::D3], v[P::D1], q[P::D2];
#pragma unroll
        for (int m = 0; m < P::D2; ++m) y[m] = Y[e * ny + yo + m];
#pragma unroll
        for (int m = 0; m < P::D3; ++m) g[m] = ok ? go[r * no + oo + m * mul + c] : 0.f;
        const float wv = ok ? w[e * nw + wo + c] : 0.f;
        P::bwd(y, xv, g, v, q);
#pragma unroll
        for (int m = 0; m < P::D1; ++m) gacc[m] = fmaf(wv, v[m], gacc[m]);
        if (ok && gw) {
            float t = 0.f;
#pragma unroll
            for (int m = 0; m < P::D1; ++m) t = fmaf(xv[m], v[m], t);
            gw[e * nw + wo + c] = t;
        }
        if (gY) {
            float a[8];
#pragma unroll
            for (int m = 0; m < 8; ++m) a[m] = m < P::D2 ? wv * q[m < P::D2 ? m : 0] : 0.f;
            const float t = wave_reduce_scatter<8>(a, lane);
            const int qi = reduce_scatter_index<8>(lane);
            if ((lane & 7) == 0 && qi < P::D2) atomicAdd(gY + e * ny + yo + qi, t);
        }
    }
}

// The paths [p0, p1) that read one x block (same offset and multiplicity, input l = L1), one
// 64-channel chunk: per edge the block's rows are loaded once and the paths' grad_x
// contributions summed in registers before the atomics (one per component and channel).
template <int L1>
__device__ __forceinline__ void any_bwd_group(const TPAnyTable& tb, int p0, int p1, int c0, int64_t r, int lane,
                                              const float* __restrict__ x, const float* __restrict__ Y,
                                              const float* __restrict__ w, const float* __restrict__ go,
                                              const int32_t* __restrict__ row_ptr,
                                              const int32_t* __restrict__ perm,
                                              const int32_t* __restrict__ senders, float* __restrict__ gx,
                                              float* __restrict__ gY, float* __restrict__ gw) {
    constexpr int D1 = 2 * L1 + 1;
    const int xo = tb.xoff[p0], mul = tb.mul[p0];
    const int c = c0 + lane;
    const bool ok = c < mul;
    const int b = row_ptr[r], end = row_ptr[r + 1];
    for (int k = b; k < end; ++k) {
        const int64_t e = uniform64(perm[k]);
        const int64_t s = uniform64(senders[k]);
        float xv[D1], gacc[D1] = {};
#pragma unroll
        for (int m = 0; m < D1; ++m) xv[m] = ok ? x[s * tb.nx + xo + m * mul + c] : 0.f;
        for (int p = p0; p < p1; ++p) {
            const int yo = tb.yoff[p], oo = tb.ooff[p], wo = tb.woff[p];
#define MNX_ANY_BWD(T)                                                                                       \
    any_bwd_step<T, L1>(yo, oo, wo, mul, c, ok, tb.ny, tb.no, tb.nw, r, e, lane, xv, Y, w, go, gY, gw, gacc)
            MNX_TP_ANY_SWITCH(tb.type[p], MNX_ANY_BWD)
#undef MNX_ANY_BWD
        }
        if (ok && gx) {
#pragma unroll
            for (int m = 0; m < D1; ++m) atomicAdd(gx + s * tb.nx + xo + m * mul + c, gacc[m]);
        }
    }
}

// Paths p and p + 1 belong to one group when they read the same x block.
__device__ __forceinline__ bool same_block(const TPAnyTable& tb, int p, int q) {
    return tb.xoff[p] == tb.xoff[q] && tb.mul[p] == tb.mul[q] && kTPAnyL1(tb.type[p]) == kTPAnyL1(tb.type[q]);
}

__global__ void __launch_bounds__(kAnyThreads) k_tp_any_bwd(const TPAnyTable tb, const float* __restrict__ x,
                                                            const float* __restrict__ Y,
                                                            const float* __restrict__ w,
                                                            const float* __restrict__ go,
                                                            const int32_t* __restrict__ row_ptr,
                                                            const int32_t* __restrict__ perm,
                                                            const int32_t* __restrict__ senders, int64_t N,
                                                            float* __restrict__ gx, float* __restrict__ gY,
                                                            float* __restrict__ gw) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t r = int64_t(blockIdx.x) * kAnyWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (r >= N) return;
    // work item blockIdx.y -> (group of paths on one x block, channel chunk)
    int rem = blockIdx.y, p0 = 0, p1 = 0;
    while (p0 < tb.num_paths) {
        p1 = p0 + 1;
        while (p1 < tb.num_paths && same_block(tb, p0, p1)) ++p1;
        const int nch = (tb.mul[p0] + kWave - 1) / kWave;
        if (rem < nch) break;
        rem -= nch;
        p0 = p1;
    }
    if (p0 >= tb.num_paths) return;
    switch (kTPAnyL1(tb.type[p0])) {
        case 0: any_bwd_group<0>(tb, p0, p1, rem * kWave, r, lane, x, Y, w, go, row_ptr, perm, senders, gx, gY, gw); break;
        case 1: any_bwd_group<1>(tb, p0, p1, rem * kWave, r, lane, x, Y, w, go, row_ptr, perm, senders, gx, gY, gw); break;
        case 2: any_bwd_group<2>(tb, p0, p1, rem * kWave, r, lane, x, Y, w, go, row_ptr, perm, senders, gx, gY, gw); break;
        case 3: any_bwd_group<3>(tb, p0, p1, rem * kWave, r, lane, x, Y, w, go, row_ptr, perm, senders, gx, gY, gw); break;
        default: break;
    }
}

// Work items of the backward: channel chunks of the groups of consecutive paths on one x block.
int64_t bwd_items(const TPAnyTable& tb) {
    int64_t items = 0;
    for (int p0 = 0, p1; p0 < tb.num_paths; p0 = p1) {
        p1 = p0 + 1;
        while (p1 < tb.num_paths && tb.xoff[p1] == tb.xoff[p0] && tb.mul[p1] == tb.mul[p0] &&
               kTPAnyL[tb.type[p1]][0] == kTPAnyL[tb.type[p0]][0])
            ++p1;
        items += ceil_div(tb.mul[p0], kWave);
    }
    return items;
}

// Parses and checks a host table: [num_paths, nx, ny, no, nw, then per path (triple, xoff, yoff,
// ooff, woff, mul)].  Every block must lie inside its row and the output blocks must tile the
// output row exactly (each output element written once by the forward).
int parse_table(const int32_t* t, int32_t len, TPAnyTable& tb) {
    MNX_REQUIRE(t && len >= kAnyHeader, "tp_any: table too short");
    const int P = t[0];
    MNX_REQUIRE(P >= 0 && P <= kAnyMaxPaths, "tp_any: %d paths (at most %d)", P, kAnyMaxPaths);
    MNX_REQUIRE(len == kAnyHeader + kAnyFields * P, "tp_any: table length %d does not match %d paths", len, P);
    tb.num_paths = P;
    tb.nx = t[1];
    tb.ny = t[2];
    tb.no = t[3];
    tb.nw = t[4];
    MNX_REQUIRE(tb.nx >= 0 && tb.no >= 0 && tb.nw >= 0 && tb.ny >= 0, "tp_any: negative row width");
    int64_t out_total = 0, w_total = 0;
    for (int p = 0; p < P; ++p) {
        const int32_t* f = t + kAnyHeader + kAnyFields * p;
        const int T = f[0];
        MNX_REQUIRE(T >= 0 && T < kTPAnyTriples, "tp_any: path %d has an unknown coupling triple %d", p, T);
        const int d1 = 2 * kTPAnyL[T][0] + 1, d2 = 2 * kTPAnyL[T][1] + 1, d3 = 2 * kTPAnyL[T][2] + 1;
        const int mul = f[5];
        MNX_REQUIRE(mul > 0, "tp_any: path %d has multiplicity %d", p, mul);
        MNX_REQUIRE(f[1] >= 0 && int64_t(f[1]) + int64_t(d1) * mul <= tb.nx, "tp_any: path %d x block outside the row", p);
        MNX_REQUIRE(f[2] >= 0 && f[2] + d2 <= tb.ny, "tp_any: path %d Y block outside the row", p);
        MNX_REQUIRE(f[3] >= 0 && int64_t(f[3]) + int64_t(d3) * mul <= tb.no, "tp_any: path %d output block outside the row", p);
        MNX_REQUIRE(f[4] >= 0 && int64_t(f[4]) + mul <= tb.nw, "tp_any: path %d weight segment outside the row", p);
        tb.type[p] = T;
        tb.xoff[p] = f[1];
        tb.yoff[p] = f[2];
        tb.ooff[p] = f[3];
        tb.woff[p] = f[4];
        tb.mul[p] = mul;
        out_total += int64_t(d3) * mul;
        w_total += mul;
    }
    MNX_REQUIRE(out_total == tb.no, "tp_any: output blocks (%lld values) do not tile the row of %d",
                (long long)out_total, tb.no);
    MNX_REQUIRE(w_total == tb.nw, "tp_any: weight segments (%lld) do not tile the row of %d", (long long)w_total,
                tb.nw);
    // output blocks must not overlap: with the total equal to the row, disjoint <=> tiling
    for (int p = 0; p < P; ++p)
        for (int q = p + 1; q < P; ++q) {
            const int64_t a0 = tb.ooff[p], a1 = a0 + int64_t(2 * kTPAnyL[tb.type[p]][2] + 1) * tb.mul[p];
            const int64_t b0 = tb.ooff[q], b1 = b0 + int64_t(2 * kTPAnyL[tb.type[q]][2] + 1) * tb.mul[q];
            MNX_REQUIRE(a1 <= b0 || b1 <= a0, "tp_any: output blocks of paths %d and %d overlap", p, q);
            MNX_REQUIRE(tb.woff[p] + tb.mul[p] <= tb.woff[q] || tb.woff[q] + tb.mul[q] <= tb.woff[p],
                        "tp_any: weight segments of paths %d and %d overlap", p, q);
        }
    return MNX_OK;
}

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

int mnx_tp_any_triple(int32_t l1, int32_t l2, int32_t l3) {
    for (int t = 0; t < kTPAnyTriples; ++t)
        if (kTPAnyL[t][0] == l1 && kTPAnyL[t][1] == l2 && kTPAnyL[t][2] == l3) return t;
    return -1;
}

int mnx_tp_any_fwd_f32(const int32_t* table, int32_t table_len, const float* x, const float* Y, const float* w,
                       const int32_t* row_ptr, const int32_t* perm, const int32_t* senders_sorted,
                       int64_t num_nodes, int64_t num_edges, float* out, mnx_stream_t stream_) {
    clear_error();
    hipStream_t stream = (hipStream_t)stream_;
    TPAnyTable tb;
    const int rc = parse_table(table, table_len, tb);
    if (rc != MNX_OK) return rc;
    MNX_REQUIRE(num_nodes >= 0 && num_edges >= 0, "sizes out of range");
    if (num_nodes == 0 || tb.no == 0) return MNX_OK;
    MNX_REQUIRE(x && out && row_ptr && (num_edges == 0 || (Y && w && perm && senders_sorted)), "null pointer argument");
    int64_t items = 0;
    for (int p = 0; p < tb.num_paths; ++p) items += ceil_div(tb.mul[p], kWave);
    MNX_REQUIRE(items <= 65535, "tp_any: %lld channel chunks (at most 65535)", (long long)items);
    MNX_REQUIRE(ceil_div(num_nodes, kAnyWaves) < (int64_t(1) << 31), "tp_any: too many nodes");
    const dim3 grid{unsigned(ceil_div(num_nodes, kAnyWaves)), unsigned(items)};
    k_tp_any_fwd<<<grid, kAnyThreads, 0, stream>>>(tb, x, Y, w, row_ptr, perm, senders_sorted, num_nodes, out);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_tp_any_bwd_f32(const int32_t* table, int32_t table_len, const float* x, const float* Y, const float* w,
                       const float* grad_out, const int32_t* row_ptr, const int32_t* perm,
                       const int32_t* senders_sorted, int64_t num_nodes, int64_t num_edges, float* grad_x,
                       float* grad_Y, float* grad_w, mnx_stream_t stream_) {
    clear_error();
    hipStream_t stream = (hipStream_t)stream_;
    TPAnyTable tb;
    const int rc = parse_table(table, table_len, tb);
    if (rc != MNX_OK) return rc;
    MNX_REQUIRE(num_nodes >= 0 && num_edges >= 0, "sizes out of range");
    if (num_nodes == 0 || num_edges == 0 || (!grad_x && !grad_Y && !grad_w)) return MNX_OK;
    MNX_REQUIRE(x && Y && w && grad_out && row_ptr && perm && senders_sorted, "null pointer argument");
    const int64_t items = bwd_items(tb);
    MNX_REQUIRE(items <= 65535, "tp_any: %lld channel chunks (at most 65535)", (long long)items);
    MNX_REQUIRE(ceil_div(num_nodes, kAnyWaves) < (int64_t(1) << 31), "tp_any: too many nodes");
    const dim3 grid{unsigned(ceil_div(num_nodes, kAnyWaves)), unsigned(items)};
    k_tp_any_bwd<<<grid, kAnyThreads, 0, stream>>>(tb, x, Y, w, grad_out, row_ptr, perm, senders_sorted, num_nodes,
                                                    grad_x, grad_Y, grad_w);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

}  // extern "C"
