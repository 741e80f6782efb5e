// Output layer of the radial weight MLP: the per-edge tensor-product weights
//   w[e][n] = sum_k h[e][k] W[n][k] + b[n]        (E x N, N = weight_numel)
// and the gradient with respect to its input
//   gh[e][k] = sum_n gw[e][n] W[n][k]
// (the last Linear of src/molrep/interaction/radial_mlp.py:38-93; at 2.6 M edges
// and N = 2944 the forward's result alone is 30.8 GB).
//
// Arithmetic: near-fp32 products on the fp16 matrix cores.  Operands are first
// brought to a common power-of-two scale (each row of h and of the gradient
// multiplied by 2^-e with 2^e <= its largest magnitude < 2^(e+1); each output
// column of W likewise), then each scaled value a is split into two fp16 parts,
// a0 = f16(a), a1 = f16(a - a0) (round to nearest even; the difference is exact
// in fp32), so that a = a0 + a1 + r with |r| <= 2^-22 |a| (absolute 2^-25 of the
// row's largest magnitude where a1 falls below the fp16 normal range).  A
// product a*b is taken as a1 b0 + a0 b1 + a0 b0, smallest first, each exact in
// the fp32 accumulator of v_mfma_f32_32x32x16_f16; the dropped a1 b1 and the
// residuals are below 3 * 2^-22 |a b| per product, a few fp32 rounding units and
// under the rounding of a K-term fp32 sum.  The scales are powers of two and
// are undone exactly in the epilogue.  Three fp16 MFMAs per K = 16 take 3/16 of
// the matrix-core cycles of the eight fp32 MFMAs (v_mfma_f32_32x32x2f32) over
// the same K and half those of a three-way bf16 split (six products), which
// matters where the layer is matrix-core bound (K = 128, and the clock held
// down by matrix-core power).
//
// MFMA 32x32x16 operand layout: lane l holds A[l%32][8(l/32) + j] and
// B[8(l/32) + j][l%32], j < 8; the accumulator's register r of lane l is
// D[8(r/4) + 4(l/32) + r%4][l%32].
//
// Forward: a workgroup of eight wavefronts owns 256 edges (32 per wavefront,
// their scaled, split rows of h held in registers for the whole kernel) and
// walks the N columns in LDS stages of 16 KB of pre-split weights,
// double-buffered: a stage's fragments are loaded into registers while the
// previous stage is multiplied, so one barrier per stage suffices.  Results
// leave as non-temporal stores, 128 contiguous bytes per row and
// half-wavefront (the store pattern that reaches the HBM write rate; 32-byte
// pieces per row made non-temporal stores five times slower on MI355X).
//
// Backward: a wavefront owns 32 edges and all K output columns (in registers),
// computed transposed, D = W^T grad^T, so that each lane's accumulator column
// is one edge; the E x N gradient streams in once (the next stage's rows loaded
// while the current one is multiplied; ordinary cached loads, since each
// 128-byte line is read by four 16-byte pieces and non-temporal loads of such
// pieces ran at 2/3 of the rate) and is scaled and split on the fly.  A row's
// scale is the running maximum over the stages seen so far: when it grows,
// the accumulator is rescaled by the (exact) power of two.  The transposed
// weights come through the same LDS stages.

#include "common.h"
#include "ew.h"

namespace mnx {
namespace {

// Column scales: forward one thread per output n (max over its K weights); backward
// one workgroup per output k (max over the N weights of column k).
__global__ void k_ew_scales(const float* __restrict__ W, int K, int N, int bwd, float* __restrict__ scale) {
    if (!bwd) {
        const int n = blockIdx.x * blockDim.x + threadIdx.x;
        if (n >= N) return;
        float m = 0.f;
        for (int k = 0; k < K; ++k) m = fmaxf(m, fabsf(W[int64_t(n) * K + k]));
        const int e = ew_exp(m);
        scale[n] = ldexpf(1.f, e == kEwNoExp ? 0 : e);
        return;
    }
    __shared__ float part[256];
    const int k = blockIdx.x;
    float m = 0.f;
    for (int n = threadIdx.x; n < N; n += blockDim.x) m = fmaxf(m, fabsf(W[int64_t(n) * K + k]));
    part[threadIdx.x] = m;
    __syncthreads();
    for (int w = blockDim.x / 2; w > 0; w /= 2) {
        if (threadIdx.x < w) part[threadIdx.x] = fmaxf(part[threadIdx.x], part[threadIdx.x + w]);
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const int e = ew_exp(part[0]);
        scale[k] = ldexpf(1.f, e == kEwNoExp ? 0 : e);
    }
}

// One thread per fragment element (both layouts); the scales are already in place.
__global__ void k_ew_pack(const float* __restrict__ W, EwShape sh, bool bwd, const float* __restrict__ scale,
                          _Float16* __restrict__ frag) {
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= sh.planes(bwd)) return;
    const int j = int(idx % 8), lane = int((idx / 8) % 64);
    int64_t rest = idx / 512;
    int n, k, p;
    if (!bwd) {
        const int sc = sh.sc(), ks = sh.ks();
        const int t = int(rest % sc);
        rest /= sc;
        const int q = int(rest % ks);
        rest /= ks;
        p = int(rest % 2);
        const int s = int(rest / 2);
        k = 16 * q + 8 * (lane / 32) + j;
        n = 32 * (sc * s + t) + lane % 32;
    } else {
        const int T = sh.tiles_b(), nq = sh.nq();
        const int t = int(rest % T);
        rest /= T;
        const int q = int(rest % nq);
        rest /= nq;
        p = int(rest % 2);
        const int s = int(rest / 2);
        n = 16 * (nq * s + q) + 8 * (lane / 32) + j;
        k = 32 * t + lane % 32;
    }
    _Float16 part = (_Float16)0.f;
    if (n < sh.N && k < sh.K) {
        const float v = ldexpf(W[int64_t(n) * sh.K + k], -ilogbf(scale[bwd ? k : n]));
        const _Float16 h0 = (_Float16)v;
        part = p == 0 ? h0 : (_Float16)(v - (float)h0);
    }
    frag[idx] = part;
}

template <int KS>
__global__ __launch_bounds__(kEwFwdThreads) void k_ew_fwd(const float* __restrict__ h,
                                                          const int32_t* __restrict__ hrows, int64_t E,
                                                          const f16x8* __restrict__ frag,
                                                          const float* __restrict__ colscale,
                                                          const float* __restrict__ bias, int N, int nstages,
                                                          float* __restrict__ out) {
    constexpr int K = 16 * KS, SC = 8 / KS;
    constexpr int PER = kEwStageVec / kEwFwdThreads;
    // Column tiles multiplied together: two independent accumulator chains keep the matrix
    // core busy between dependent MFMAs.
    constexpr int TP = SC >= 2 ? 2 : 1;
    __shared__ f16x8 sB[2][kEwStageVec];
    __shared__ float sBias[2][SC * 32], sCol[2][SC * 32];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t row0 = int64_t(blockIdx.x) * kEwFwdRows + wave * 32;

    f16x8 a0[KS], a1[KS];
    float rs[16];  // scales of the accumulator rows this lane holds
    {
        const int64_t row = row0 + (lane & 31);
        const bool ok = row < E;
        const int64_t hrow = ok ? (hrows ? int64_t(hrows[row]) : row) : 0;  // output row -> row of h
        const float* src = h + hrow * K + 8 * (lane >> 5);
        f32x4 v[KS][2];
        float m = 0.f;
#pragma unroll
        for (int q = 0; q < KS; ++q) {
            v[q][0] = v[q][1] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (ok) {
                v[q][0] = *reinterpret_cast<const f32x4*>(src + 16 * q);
                v[q][1] = *reinterpret_cast<const f32x4*>(src + 16 * q + 4);
            }
            m = absmax8(v[q][0], v[q][1], m);
        }
        m = fmaxf(m, __shfl_xor(m, 32));
        int e = ew_exp(m);
        if (e == kEwNoExp) e = 0;
        const float si = ldexpf(1.f, -e), so = ldexpf(1.f, e);
#pragma unroll
        for (int q = 0; q < KS; ++q) split8(v[q][0], v[q][1], si, a0[q], a1[q]);
#pragma unroll
        for (int r = 0; r < 16; ++r) rs[r] = __shfl(so, 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3));
    }

    f16x8 pre[PER];
    float pbias = 0.f, pcol = 1.f;
    auto fetch = [&](int s) {
        const f16x8* src = frag + int64_t(s) * kEwStageVec + threadIdx.x;
#pragma unroll
        for (int i = 0; i < PER; ++i) pre[i] = src[i * kEwFwdThreads];
        if (threadIdx.x < SC * 32) {
            const int n = s * SC * 32 + threadIdx.x;
            pbias = (bias && n < N) ? bias[n] : 0.f;
            pcol = n < N ? colscale[n] : 1.f;
        }
    };
    fetch(0);
    for (int s = 0; s < nstages; ++s) {
        const int buf = s & 1;
#pragma unroll
        for (int i = 0; i < PER; ++i) sB[buf][threadIdx.x + i * kEwFwdThreads] = pre[i];
        if (threadIdx.x < SC * 32) {
            sBias[buf][threadIdx.x] = pbias;
            sCol[buf][threadIdx.x] = pcol;
        }
        __syncthreads();
        if (s + 1 < nstages) fetch(s + 1);
        const f16x8* B = &sB[buf][lane];
        auto bq = [&](int p, int q, int t) -> const f16x8& { return B[((p * KS + q) * SC + t) * 64]; };
#pragma unroll
        for (int t0 = 0; t0 < SC; t0 += TP) {
            if ((s * SC + t0) * 32 >= N) break;
            f32x16 acc[2] = {f32x16{}, f32x16{}};
            auto ti = [&](int u) { return TP == 2 ? t0 + u : t0; };
#pragma unroll
            for (int q = 0; q < KS; ++q)
#pragma unroll
                for (int u = 0; u < TP; ++u) {
                    acc[u] = mfma(a1[q], bq(0, q, ti(u)), acc[u]);
                    acc[u] = mfma(a0[q], bq(1, q, ti(u)), acc[u]);
                }
#pragma unroll
            for (int q = 0; q < KS; ++q)
#pragma unroll
                for (int u = 0; u < TP; ++u) acc[u] = mfma(a0[q], bq(0, q, ti(u)), acc[u]);
#pragma unroll
            for (int u = 0; u < TP; ++u) {
                const int n = (s * SC + t0 + u) * 32 + (lane & 31);
                if (n >= N) continue;
                const float b = sBias[buf][(t0 + u) * 32 + (lane & 31)];
                const float cs = sCol[buf][(t0 + u) * 32 + (lane & 31)];
                float* o = out + (row0 + 4 * (lane >> 5)) * N + n;
                if (row0 + 32 <= E) {  // whole row block valid: no per-row branches
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        __builtin_nontemporal_store(fmaf(acc[u][r] * rs[r], cs, b),
                                                    o + int64_t(8 * (r >> 2) + (r & 3)) * N);
                } else {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int64_t row = row0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                        if (row < E)
                            __builtin_nontemporal_store(fmaf(acc[u][r] * rs[r], cs, b),
                                                        o + int64_t(8 * (r >> 2) + (r & 3)) * N);
                    }
                }
            }
        }
    }
}

// PAIR: row i of the product is the sum of gradient rows pairs[i][0] and pairs[i][1] (the two
// directed edges that share one row of weights), E the number of pairs.
// ld: the row stride of gw (N for a whole row; wider for a column slice); ldh: the row stride of gh
// (K, or wider when gh is a column block of a wider tensor); accumulate: gh += instead of gh = (the
// partial products over column slices, added in launch order).
// RAGGED: N is not a multiple of the stage width 16 NQ, so the last stage's loads are guarded;
// otherwise every load is unconditional (rows past E read row 0, their results are not stored),
// which keeps the loaded values in the registers the products read (a guarded load has to be
// merged with the zero default: ~190 register moves per stage and wavefront).
template <int T, bool PAIR, bool RAGGED>
__global__ __launch_bounds__(kEwBwdThreads, T >= 2 ? 3 : 2) void k_ew_bwd(const float* __restrict__ gw, int64_t E, int N,
                                                       const f16x8* __restrict__ frag,
                                                       const float* __restrict__ colscale, int K, int nstages,
                                                       const int32_t* __restrict__ pairs,
                                                       float* __restrict__ gh, int64_t ld, int64_t ldh,
                                                       bool accumulate) {
    constexpr int NQ = 8 / T;
    constexpr int PER = kEwStageVec / kEwBwdThreads;
    __shared__ f16x8 sB[2][kEwStageVec];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t row0 = int64_t(blockIdx.x) * kEwBwdRows + wave * 32;
    const int64_t arow = row0 + (lane & 31);
    const bool aok = arow < E;
    const int64_t src0 = PAIR ? (aok ? int64_t(pairs[2 * arow]) : 0) : (aok ? arow : 0);
    const int64_t src1 = PAIR ? (aok ? int64_t(pairs[2 * arow + 1]) : 0) : 0;
    const float* asrc = gw + src0 * ld + 8 * (lane >> 5);
    const float* bsrc = gw + src1 * ld + 8 * (lane >> 5);

    // the gradient rows of two stages alternate between two register sets (the loop is unrolled
    // by two, so that neither set is copied into the other at the loop's back edge)
    using Rows = f32x4[NQ][2];
    Rows ra, rb;
    auto fetch_a = [&](Rows& r, int s) {
        if (!RAGGED) {
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                f32x4 lo = *reinterpret_cast<const f32x4*>(asrc + 16 * (NQ * s + q));
                f32x4 hi = *reinterpret_cast<const f32x4*>(asrc + 16 * (NQ * s + q) + 4);
                if (PAIR) {
                    lo += *reinterpret_cast<const f32x4*>(bsrc + 16 * (NQ * s + q));
                    hi += *reinterpret_cast<const f32x4*>(bsrc + 16 * (NQ * s + q) + 4);
                }
                r[q][0] = lo;
                r[q][1] = hi;
            }
            return;
        }
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int n = 16 * (NQ * s + q) + 8 * (lane >> 5);
            f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = lo;
            if (aok && n < N) {
                lo = *reinterpret_cast<const f32x4*>(asrc + 16 * (NQ * s + q));
                hi = *reinterpret_cast<const f32x4*>(asrc + 16 * (NQ * s + q) + 4);
                if (PAIR) {
                    lo += *reinterpret_cast<const f32x4*>(bsrc + 16 * (NQ * s + q));
                    hi += *reinterpret_cast<const f32x4*>(bsrc + 16 * (NQ * s + q) + 4);
                }
            }
            r[q][0] = lo;
            r[q][1] = hi;
        }
    };
    f16x8 pre[PER];
    auto fetch_b = [&](int s) {
        const f16x8* src = frag + int64_t(s) * kEwStageVec + threadIdx.x;
#pragma unroll
        for (int i = 0; i < PER; ++i) pre[i] = src[i * kEwBwdThreads];
    };

    // acc[t]: D = W^T grad^T, register r of lane l = gh[row0 + l%32][32t + 8(r/4) + 4(l/32) + r%4],
    // in units of 2^ecur (this lane's row scale so far)
    f32x16 acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = f32x16{};
    int ecur = kEwNoExp;
    // stage s: its rows in cur, W's fragments in pre (staged into LDS buffer buf); loads stage
    // s + 1 into nxt and pre.  With two gradient rows per product row (PAIR) those loads are issued
    // first, so that they have the whole stage to arrive (measured: K = 128, 1.44 -> 1.41 ms at
    // 512 columns, 3.39 -> 3.31 ms at 1280); with one row per product row they wait until after the
    // barrier (K = 64, 2944 columns: 6.80 ms, 7.12 ms when issued first)
    auto stage = [&](int s, int buf, Rows& cur, Rows& nxt) {
#pragma unroll
        for (int i = 0; i < PER; ++i) sB[buf][threadIdx.x + i * kEwBwdThreads] = pre[i];
        if (PAIR && s + 1 < nstages) {
            fetch_b(s + 1);
            fetch_a(nxt, s + 1);
        }
        float m = 0.f;
#pragma unroll
        for (int q = 0; q < NQ; ++q) m = absmax8(cur[q][0], cur[q][1], m);
        m = fmaxf(m, __shfl_xor(m, 32));
        const int enew = max(ecur, ew_exp(m));
        if (__ballot(enew != ecur)) {
            const float f = ldexpf(1.f, ecur - enew);
#pragma unroll
            for (int t = 0; t < T; ++t) acc[t] *= f;
        }
        ecur = enew;
        f16x8 g0[NQ], g1[NQ];
        const float si = ldexpf(1.f, -ecur);
#pragma unroll
        for (int q = 0; q < NQ; ++q) split8(cur[q][0], cur[q][1], si, g0[q], g1[q]);
        __syncthreads();
        if (!PAIR && s + 1 < nstages) {
            fetch_a(nxt, s + 1);
            fetch_b(s + 1);
        }
        const f16x8* B = &sB[buf][lane];
        auto wq = [&](int p, int q, int t) -> const f16x8& { return B[((p * NQ + q) * T + t) * 64]; };
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
                acc[t] = mfma(wq(0, q, t), g1[q], acc[t]);
                acc[t] = mfma(wq(1, q, t), g0[q], acc[t]);
                acc[t] = mfma(wq(0, q, t), g0[q], acc[t]);
            }
        }
    };
    fetch_a(ra, 0);
    fetch_b(0);
    for (int s = 0; s < nstages; s += 2) {
        stage(s, 0, ra, rb);
        if (s + 1 < nstages) stage(s + 1, 1, rb, ra);
    }
    if (!aok) return;
    const float so = ldexpf(1.f, ecur == kEwNoExp ? 0 : ecur);
    float* dst = gh + arow * ldh;
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const int c = 32 * t + 8 * r4 + 4 * (lane >> 5);
            if (c >= K) continue;
            const f32x4 cs = *reinterpret_cast<const f32x4*>(colscale + c);
            f32x4 v;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = acc[t][4 * r4 + i] * so * cs[i];
            if (accumulate) v += *reinterpret_cast<const f32x4*>(dst + c);
            *reinterpret_cast<f32x4*>(dst + c) = v;
        }
}

int check_ew(int32_t K, int32_t N) {
    if (K != 16 && K != 32 && K != 64 && K != 128)
        return set_error(MNX_ERR_UNSUPPORTED, "edge weights: input width %d not 16, 32, 64 or 128", K);
    MNX_REQUIRE(N >= 1 && N < (1 << 24), "edge weights: output width %d out of range", N);
    return MNX_OK;
}

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

int64_t mnx_edge_weights_frag_elems(int32_t K, int32_t N, int32_t backward) {
    if (check_ew(K, N)) return -1;
    const EwShape sh{K, N};
    return sh.elems(backward != 0);
}

int mnx_edge_weights_pack_f32(const float* weight, int32_t K, int32_t N, int32_t backward, uint16_t* frag,
                              mnx_stream_t stream) {
    clear_error();
    int rc = check_ew(K, N);
    if (rc) return rc;
    MNX_REQUIRE(weight && frag, "null pointer argument");
    MNX_REQUIRE((uintptr_t)frag % 16 == 0, "frag must be 16-byte aligned");
    const EwShape sh{K, N};
    const bool bwd = backward != 0;
    const int64_t total = sh.planes(bwd);
    hipStream_t s = (hipStream_t)stream;
    float* scale = reinterpret_cast<float*>(frag + total);
    if (bwd)
        hipLaunchKernelGGL(k_ew_scales, dim3(K), dim3(256), 0, s, weight, K, N, 1, scale);
    else
        hipLaunchKernelGGL(k_ew_scales, dim3(unsigned(ceil_div(N, 256))), dim3(256), 0, s, weight, K, N, 0, scale);
    MNX_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_ew_pack, dim3(unsigned(ceil_div(total, 256))), dim3(256), 0, s, weight, sh, bwd, scale,
                       reinterpret_cast<_Float16*>(frag));
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_edge_weights_f32(const float* h, int64_t num_edges, int32_t K, const uint16_t* frag, const float* bias,
                         int32_t N, float* out, mnx_stream_t stream) {
    return mnx_edge_weights_rows_f32(h, nullptr, num_edges, K, frag, bias, N, out, stream);
}

int mnx_edge_weights_rows_f32(const float* h, const int32_t* rows, int64_t num_edges, int32_t K,
                              const uint16_t* frag, const float* bias, int32_t N, float* out, mnx_stream_t stream) {
    clear_error();
    int rc = check_ew(K, N);
    if (rc) return rc;
    MNX_REQUIRE(num_edges >= 0 && num_edges < (int64_t(1) << 36), "edge count out of range");
    if (num_edges == 0) return MNX_OK;
    MNX_REQUIRE(h && frag && out, "null pointer argument");
    MNX_REQUIRE(((uintptr_t)h | (uintptr_t)frag) % 16 == 0, "h and frag must be 16-byte aligned");
    const EwShape sh{K, N};
    const dim3 grid(unsigned(ceil_div(num_edges, kEwFwdRows))), block(kEwFwdThreads);
    const f16x8* f = reinterpret_cast<const f16x8*>(frag);
    const float* cs = reinterpret_cast<const float*>(frag + sh.planes(false));
    hipStream_t s = (hipStream_t)stream;
    switch (K) {
        case 16: hipLaunchKernelGGL(k_ew_fwd<1>, grid, block, 0, s, h, rows, num_edges, f, cs, bias, N, sh.stages_f(), out); break;
        case 32: hipLaunchKernelGGL(k_ew_fwd<2>, grid, block, 0, s, h, rows, num_edges, f, cs, bias, N, sh.stages_f(), out); break;
        case 64: hipLaunchKernelGGL(k_ew_fwd<4>, grid, block, 0, s, h, rows, num_edges, f, cs, bias, N, sh.stages_f(), out); break;
        default: hipLaunchKernelGGL(k_ew_fwd<8>, grid, block, 0, s, h, rows, num_edges, f, cs, bias, N, sh.stages_f(), out); break;
    }
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_edge_weights_bwd_f32(const float* grad_w, int64_t num_edges, int32_t N, const uint16_t* frag, int32_t K,
                             float* grad_h, mnx_stream_t stream) {
    return mnx_edge_weights_bwd_pairs_f32(grad_w, nullptr, num_edges, N, frag, K, grad_h, stream);
}

int mnx_edge_weights_bwd_pairs_f32(const float* grad_w, const int32_t* pairs, int64_t num_edges, int32_t N,
                                   const uint16_t* frag, int32_t K, float* grad_h, mnx_stream_t stream) {
    return mnx_edge_weights_bwd_cols_f32(grad_w, N, pairs, num_edges, N, frag, K, grad_h, 0, stream);
}

int mnx_edge_weights_bwd_cols_f32(const float* grad_w, int64_t ld, const int32_t* pairs, int64_t num_edges,
                                  int32_t N, const uint16_t* frag, int32_t K, float* grad_h, int32_t accumulate,
                                  mnx_stream_t stream) {
    return mnx_edge_weights_bwd_into_f32(grad_w, ld, pairs, num_edges, N, frag, K, grad_h, K, accumulate, stream);
}

int mnx_edge_weights_bwd_into_f32(const float* grad_w, int64_t ld, const int32_t* pairs, int64_t num_edges,
                                  int32_t N, const uint16_t* frag, int32_t K, float* grad_h, int64_t ldh,
                                  int32_t accumulate, mnx_stream_t stream) {
    clear_error();
    int rc = check_ew(K, N);
    if (rc) return rc;
    MNX_REQUIRE(ld >= N && ld % 4 == 0, "edge weights backward: row stride %lld below the width %d or not a "
                "multiple of 4", (long long)ld, N);
    MNX_REQUIRE(ldh >= K && ldh % 4 == 0, "edge weights backward: output row stride %lld below the width %d or "
                "not a multiple of 4", (long long)ldh, K);
    MNX_REQUIRE(N % 8 == 0, "edge weights backward: output width %d not a multiple of 8", N);
    MNX_REQUIRE(num_edges >= 0 && num_edges < (int64_t(1) << 36), "edge count out of range");
    if (num_edges == 0) return MNX_OK;
    MNX_REQUIRE(grad_w && frag && grad_h, "null pointer argument");
    MNX_REQUIRE(((uintptr_t)grad_w | (uintptr_t)frag | (uintptr_t)grad_h) % 16 == 0,
                "grad_w, frag and grad_h must be 16-byte aligned");
    const EwShape sh{K, N};
    const dim3 grid(unsigned(ceil_div(num_edges, kEwBwdRows))), block(kEwBwdThreads);
    const f16x8* f = reinterpret_cast<const f16x8*>(frag);
    const float* cs = reinterpret_cast<const float*>(frag + sh.planes(true));
    hipStream_t s = (hipStream_t)stream;
    const int tiles = sh.tiles_b();
    // stage width 16 NQ = 128 / tiles columns
    const bool ragged = N % (128 / tiles) != 0;
    decltype(&k_ew_bwd<1, true, true>) fn;
    if (ragged)
        fn = pairs ? (tiles == 1 ? k_ew_bwd<1, true, true> : tiles == 2 ? k_ew_bwd<2, true, true> : k_ew_bwd<4, true, true>)
                   : (tiles == 1 ? k_ew_bwd<1, false, true> : tiles == 2 ? k_ew_bwd<2, false, true> : k_ew_bwd<4, false, true>);
    else
        fn = pairs ? (tiles == 1 ? k_ew_bwd<1, true, false> : tiles == 2 ? k_ew_bwd<2, true, false> : k_ew_bwd<4, true, false>)
                   : (tiles == 1 ? k_ew_bwd<1, false, false> : tiles == 2 ? k_ew_bwd<2, false, false> : k_ew_bwd<4, false, false>);
    hipLaunchKernelGGL(fn, grid, block, 0, s, grad_w, num_edges, N, f, cs, K, sh.stages_b(), pairs, grad_h, ld, ldh,
                       accumulate != 0);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

}  // extern "C"
