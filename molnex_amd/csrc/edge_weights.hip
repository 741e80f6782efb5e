// Output layer of the radial weight MLP: the per-edge tensor-product weights
//   w[e][n] = sum_k h[e][k] W[n][k] + b[n]        (E x N, N = weight_numel)
// and the gradient with respect to its input
//   gh[e][k] = sum_n gw[e][n] W[n][k]
// (the last Linear of src/molrep/interaction/radial_mlp.py:38-93; at 2.6 M edges
// and N = 2944 the forward's result alone is 30.8 GB).
//
// Arithmetic: fp32-accurate products on the bf16 matrix cores.  Each fp32
// operand a is split into three bf16 parts, a0 = bf16(a), a1 = bf16(a - a0),
// a2 = bf16(a - a0 - a1) (round to nearest even; the differences are exact in
// fp32), so that a = a0 + a1 + a2 + r with |r| <= 2^-27 |a|.  A product a*b is
// taken as the six partial products a_i b_j with i + j <= 2; the dropped terms
// are below 2^-25 |a b|, under the fp32 rounding of the sum itself.  Each
// partial product is exact in the fp32 accumulator of v_mfma_f32_32x32x16_bf16,
// and the six of them are accumulated smallest first.  Six bf16 MFMAs over
// K = 16 take 3/8 of the matrix-core cycles of the eight fp32 MFMAs
// (v_mfma_f32_32x32x2f32) over the same K, which takes the forward from the
// fp32 matrix-core rate to the HBM store rate of its output.
//
// MFMA 32x32x16 bf16 operand layout: lane l holds A[l%32][8(l/32) + j] and
// B[8(l/32) + j][l%32], j < 8; the accumulator's register r of lane l is
// D[8(r/4) + 4(l/32) + r%4][l%32].
//
// Forward: a workgroup of eight wavefronts owns 256 edges (32 per wavefront,
// their split rows of h held in registers for the whole kernel) and walks the N
// columns in LDS stages of 24 KB of pre-split weights, double-buffered: a
// stage's fragments are loaded into registers while the previous stage is
// multiplied, so one barrier per stage suffices.  Results leave as
// non-temporal stores, 128 contiguous bytes per row and half-wavefront (the
// store pattern that reaches the HBM write rate; 32-byte pieces per row made
// non-temporal stores five times slower on MI355X).
//
// Backward: a wavefront owns 32 edges and all K output columns (in registers);
// the E x N gradient streams in once (the next stage's rows loaded while the
// current one is multiplied; ordinary cached loads, since each 128-byte line is
// read by four 16-byte pieces and non-temporal loads of such pieces ran at 2/3
// of the rate) and is split on the fly, the transposed weights come through the
// same LDS stages.

#include "common.h"

namespace mnx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kEwFwdThreads = 512;                   // eight wavefronts
constexpr int kEwFwdRows = (kEwFwdThreads / 64) * 32;  // edges per forward workgroup
constexpr int kEwBwdThreads = 256;                   // four wavefronts
constexpr int kEwBwdRows = (kEwBwdThreads / 64) * 32;  // edges per backward workgroup
constexpr int kEwStageVec = 1536;                    // bf16x8 vectors per LDS stage (24 KB)

// Weight fragment layouts (bf16 elements, 8 per lane-vector).
//  forward, B = W^T (K x N): [stage][plane][q < KS][t < SC][lane][8] holds
//    W[n][k], k = 16q + 8(lane/32) + j, n = 32(SC*stage + t) + lane%32;
//  backward, B = W (N x K): [stage][plane][q < NQ][t < T][lane][8] holds
//    W[n][c], n = 16(NQ*stage + q) + 8(lane/32) + j, c = 32t + lane%32;
// zero outside the matrix.  KS * SC = NQ * T = 8, so every stage is 3 * 8 * 64
// vectors.
struct EwShape {
    int K, N;
    __host__ __device__ int ks() const { return K / 16; }
    __host__ __device__ int sc() const { return 8 / ks(); }
    __host__ __device__ int tiles_b() const { return (K + 31) / 32; }
    __host__ __device__ int nq() const { return 8 / tiles_b(); }
    __host__ __device__ int stages_f() const { return (N + 32 * sc() - 1) / (32 * sc()); }
    __host__ __device__ int stages_b() const { return (N + 16 * nq() - 1) / (16 * nq()); }
    __host__ __device__ int64_t elems_f() const { return int64_t(stages_f()) * kEwStageVec * 8; }
    __host__ __device__ int64_t elems_b() const { return int64_t(stages_b()) * kEwStageVec * 8; }
};

__device__ __forceinline__ void split3(float v, __bf16& b0, __bf16& b1, __bf16& b2) {
    b0 = (__bf16)v;
    float r = v - (float)b0;
    b1 = (__bf16)r;
    r -= (float)b1;
    b2 = (__bf16)r;
}

__device__ __forceinline__ void split8(const f32x4& lo, const f32x4& hi, bf16x8& a0, bf16x8& a1, bf16x8& a2) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        __bf16 b0, b1, b2;
        split3(j < 4 ? lo[j] : hi[j - 4], b0, b1, b2);
        a0[j] = b0;
        a1[j] = b1;
        a2[j] = b2;
    }
}

__device__ __forceinline__ f32x16 mfma(const bf16x8& a, const bf16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// One thread per fragment element (both layouts).
__global__ void k_ew_pack(const float* __restrict__ W, EwShape sh, bool bwd, __bf16* __restrict__ frag) {
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t total = bwd ? sh.elems_b() : sh.elems_f();
    if (idx >= total) return;
    const int j = int(idx % 8), lane = int((idx / 8) % 64);
    int64_t rest = idx / 512;
    int n, k, p;
    if (!bwd) {
        const int sc = sh.sc(), ks = sh.ks();
        const int t = int(rest % sc);
        rest /= sc;
        const int q = int(rest % ks);
        rest /= ks;
        p = int(rest % 3);
        const int s = int(rest / 3);
        k = 16 * q + 8 * (lane / 32) + j;
        n = 32 * (sc * s + t) + lane % 32;
    } else {
        const int T = sh.tiles_b(), nq = sh.nq();
        const int t = int(rest % T);
        rest /= T;
        const int q = int(rest % nq);
        rest /= nq;
        p = int(rest % 3);
        const int s = int(rest / 3);
        n = 16 * (nq * s + q) + 8 * (lane / 32) + j;
        k = 32 * t + lane % 32;
    }
    __bf16 part = (__bf16)0.f;
    if (n < sh.N && k < sh.K) {
        __bf16 b0, b1, b2;
        split3(W[int64_t(n) * sh.K + k], b0, b1, b2);
        part = p == 0 ? b0 : (p == 1 ? b1 : b2);
    }
    frag[idx] = part;
}

template <int KS>
__global__ __launch_bounds__(kEwFwdThreads) void k_ew_fwd(const float* __restrict__ h, int64_t E,
                                                          const bf16x8* __restrict__ frag,
                                                          const float* __restrict__ bias, int N, int nstages,
                                                          float* __restrict__ out) {
    constexpr int K = 16 * KS, SC = 8 / KS;
    constexpr int PER = kEwStageVec / kEwFwdThreads;
    // Column tiles multiplied together: two independent accumulator chains keep the matrix
    // core busy between dependent MFMAs (with one tile per stage, K = 128, a second chain
    // costs more in registers than it gains).
    constexpr int TP = SC >= 2 ? 2 : 1;
    __shared__ bf16x8 sB[2][kEwStageVec];
    __shared__ float sBias[2][SC * 32];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t row0 = int64_t(blockIdx.x) * kEwFwdRows + wave * 32;

    bf16x8 a0[KS], a1[KS], a2[KS];
    {
        const int64_t row = row0 + (lane & 31);
        const bool ok = row < E;
        const float* src = h + (ok ? row : 0) * K + 8 * (lane >> 5);
#pragma unroll
        for (int q = 0; q < KS; ++q) {
            f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = lo;
            if (ok) {
                lo = *reinterpret_cast<const f32x4*>(src + 16 * q);
                hi = *reinterpret_cast<const f32x4*>(src + 16 * q + 4);
            }
            split8(lo, hi, a0[q], a1[q], a2[q]);
        }
    }

    bf16x8 pre[PER];
    float pbias = 0.f;
    auto fetch = [&](int s) {
        const bf16x8* src = frag + int64_t(s) * kEwStageVec + threadIdx.x;
#pragma unroll
        for (int i = 0; i < PER; ++i) pre[i] = src[i * kEwFwdThreads];
        if (threadIdx.x < SC * 32) {
            const int n = s * SC * 32 + threadIdx.x;
            pbias = (bias && n < N) ? bias[n] : 0.f;
        }
    };
    fetch(0);
    for (int s = 0; s < nstages; ++s) {
        const int buf = s & 1;
#pragma unroll
        for (int i = 0; i < PER; ++i) sB[buf][threadIdx.x + i * kEwFwdThreads] = pre[i];
        if (threadIdx.x < SC * 32) sBias[buf][threadIdx.x] = pbias;
        __syncthreads();
        if (s + 1 < nstages) fetch(s + 1);
        const bf16x8* B = &sB[buf][lane];
        auto bq = [&](int p, int q, int t) -> const bf16x8& { return B[((p * KS + q) * SC + t) * 64]; };
#pragma unroll
        for (int t0 = 0; t0 < SC; t0 += TP) {
            if ((s * SC + t0) * 32 >= N) break;
            f32x16 acc[2] = {f32x16{}, f32x16{}};
            // accumulator and column tile of chain u
            auto ai = [&](int, int u) { return u; };
            auto ti = [&](int u) { return TP == 2 ? t0 + u : t0; };
#pragma unroll
            for (int q = 0; q < KS; ++q)
#pragma unroll
                for (int u = 0; u < TP; ++u) {
                    f32x16& c = acc[ai(q, u)];
                    c = mfma(a2[q], bq(0, q, ti(u)), c);
                    c = mfma(a1[q], bq(1, q, ti(u)), c);
                    c = mfma(a0[q], bq(2, q, ti(u)), c);
                }
#pragma unroll
            for (int q = 0; q < KS; ++q)
#pragma unroll
                for (int u = 0; u < TP; ++u) {
                    f32x16& c = acc[ai(q, u)];
                    c = mfma(a1[q], bq(0, q, ti(u)), c);
                    c = mfma(a0[q], bq(1, q, ti(u)), c);
                }
#pragma unroll
            for (int q = 0; q < KS; ++q)
#pragma unroll
                for (int u = 0; u < TP; ++u) acc[ai(q, u)] = mfma(a0[q], bq(0, q, ti(u)), acc[ai(q, u)]);
#pragma unroll
            for (int u = 0; u < TP; ++u) {
                const int n = (s * SC + t0 + u) * 32 + (lane & 31);
                if (n >= N) continue;
                const float b = sBias[buf][(t0 + u) * 32 + (lane & 31)];
                float* o = out + (row0 + 4 * (lane >> 5)) * N + n;
                if (row0 + 32 <= E) {  // whole row block valid: no per-row branches
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        __builtin_nontemporal_store(acc[u][r] + b, o + int64_t(8 * (r >> 2) + (r & 3)) * N);
                } else {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int64_t row = row0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                        if (row < E) __builtin_nontemporal_store(acc[u][r] + b, o + int64_t(8 * (r >> 2) + (r & 3)) * N);
                    }
                }
            }
        }
    }
}

template <int T>
__global__ __launch_bounds__(kEwBwdThreads) void k_ew_bwd(const float* __restrict__ gw, int64_t E, int N,
                                                       const bf16x8* __restrict__ frag, int K, int nstages,
                                                       float* __restrict__ gh) {
    constexpr int NQ = 8 / T;
    constexpr int PER = kEwStageVec / kEwBwdThreads;
    __shared__ bf16x8 sB[2][kEwStageVec];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t row0 = int64_t(blockIdx.x) * kEwBwdRows + wave * 32;
    const int64_t arow = row0 + (lane & 31);
    const bool aok = arow < E;
    const float* asrc = gw + (aok ? arow : 0) * N + 8 * (lane >> 5);

    f32x4 ra[NQ][2];
    auto fetch_a = [&](int s) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int n = 16 * (NQ * s + q) + 8 * (lane >> 5);
            f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = lo;
            if (aok && n < N) {
                lo = *reinterpret_cast<const f32x4*>(asrc + 16 * (NQ * s + q));
                hi = *reinterpret_cast<const f32x4*>(asrc + 16 * (NQ * s + q) + 4);
            }
            ra[q][0] = lo;
            ra[q][1] = hi;
        }
    };
    bf16x8 pre[PER];
    auto fetch_b = [&](int s) {
        const bf16x8* src = frag + int64_t(s) * kEwStageVec + threadIdx.x;
#pragma unroll
        for (int i = 0; i < PER; ++i) pre[i] = src[i * kEwBwdThreads];
    };

    f32x16 acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = f32x16{};
    fetch_a(0);
    fetch_b(0);
    for (int s = 0; s < nstages; ++s) {
        const int buf = s & 1;
#pragma unroll
        for (int i = 0; i < PER; ++i) sB[buf][threadIdx.x + i * kEwBwdThreads] = pre[i];
        bf16x8 a0[NQ], a1[NQ], a2[NQ];
#pragma unroll
        for (int q = 0; q < NQ; ++q) split8(ra[q][0], ra[q][1], a0[q], a1[q], a2[q]);
        __syncthreads();
        if (s + 1 < nstages) {
            fetch_a(s + 1);
            fetch_b(s + 1);
        }
        const bf16x8* B = &sB[buf][lane];
        auto bq = [&](int p, int q, int t) -> const bf16x8& { return B[((p * NQ + q) * T + t) * 64]; };
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
                acc[t] = mfma(a2[q], bq(0, q, t), acc[t]);
                acc[t] = mfma(a1[q], bq(1, q, t), acc[t]);
                acc[t] = mfma(a0[q], bq(2, q, t), acc[t]);
                acc[t] = mfma(a1[q], bq(0, q, t), acc[t]);
                acc[t] = mfma(a0[q], bq(1, q, t), acc[t]);
                acc[t] = mfma(a0[q], bq(0, q, t), acc[t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int c = 32 * t + (lane & 31);
        if (c >= K) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t row = row0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (row < E) gh[row * K + c] = acc[t][r];
        }
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
    return backward ? sh.elems_b() : sh.elems_f();
}

int mnx_edge_weights_pack_f32(const float* weight, int32_t K, int32_t N, int32_t backward, uint16_t* frag,
                              mnx_stream_t stream) {
    clear_error();
    int rc = check_ew(K, N);
    if (rc) return rc;
    MNX_REQUIRE(weight && frag, "null pointer argument");
    const EwShape sh{K, N};
    const int64_t total = backward ? sh.elems_b() : sh.elems_f();
    hipLaunchKernelGGL(k_ew_pack, dim3(ceil_div(total, 256)), dim3(256), 0, (hipStream_t)stream, weight, sh,
                       backward != 0, reinterpret_cast<__bf16*>(frag));
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_edge_weights_f32(const float* h, int64_t num_edges, int32_t K, const uint16_t* frag, const float* bias,
                         int32_t N, float* out, mnx_stream_t stream) {
    clear_error();
    int rc = check_ew(K, N);
    if (rc) return rc;
    MNX_REQUIRE(num_edges >= 0 && num_edges < (int64_t(1) << 36), "edge count out of range");
    if (num_edges == 0) return MNX_OK;
    MNX_REQUIRE(h && frag && out, "null pointer argument");
    MNX_REQUIRE(((uintptr_t)h | (uintptr_t)frag) % 16 == 0, "h and frag must be 16-byte aligned");
    const EwShape sh{K, N};
    const dim3 grid(unsigned(ceil_div(num_edges, kEwFwdRows))), block(kEwFwdThreads);
    const bf16x8* f = reinterpret_cast<const bf16x8*>(frag);
    hipStream_t s = (hipStream_t)stream;
    switch (K) {
        case 16: hipLaunchKernelGGL(k_ew_fwd<1>, grid, block, 0, s, h, num_edges, f, bias, N, sh.stages_f(), out); break;
        case 32: hipLaunchKernelGGL(k_ew_fwd<2>, grid, block, 0, s, h, num_edges, f, bias, N, sh.stages_f(), out); break;
        case 64: hipLaunchKernelGGL(k_ew_fwd<4>, grid, block, 0, s, h, num_edges, f, bias, N, sh.stages_f(), out); break;
        default: hipLaunchKernelGGL(k_ew_fwd<8>, grid, block, 0, s, h, num_edges, f, bias, N, sh.stages_f(), out); break;
    }
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_edge_weights_bwd_f32(const float* grad_w, int64_t num_edges, int32_t N, const uint16_t* frag, int32_t K,
                             float* grad_h, mnx_stream_t stream) {
    clear_error();
    int rc = check_ew(K, N);
    if (rc) return rc;
    MNX_REQUIRE(N % 8 == 0, "edge weights backward: output width %d not a multiple of 8", N);
    MNX_REQUIRE(num_edges >= 0 && num_edges < (int64_t(1) << 36), "edge count out of range");
    if (num_edges == 0) return MNX_OK;
    MNX_REQUIRE(grad_w && frag && grad_h, "null pointer argument");
    MNX_REQUIRE(((uintptr_t)grad_w | (uintptr_t)frag) % 16 == 0, "grad_w and frag must be 16-byte aligned");
    const EwShape sh{K, N};
    const dim3 grid(unsigned(ceil_div(num_edges, kEwBwdRows))), block(kEwBwdThreads);
    const bf16x8* f = reinterpret_cast<const bf16x8*>(frag);
    hipStream_t s = (hipStream_t)stream;
    switch (sh.tiles_b()) {
        case 1: hipLaunchKernelGGL(k_ew_bwd<1>, grid, block, 0, s, grad_w, num_edges, N, f, K, sh.stages_b(), grad_h); break;
        case 2: hipLaunchKernelGGL(k_ew_bwd<2>, grid, block, 0, s, grad_w, num_edges, N, f, K, sh.stages_b(), grad_h); break;
        default: hipLaunchKernelGGL(k_ew_bwd<4>, grid, block, 0, s, grad_w, num_edges, N, f, K, sh.stages_b(), grad_h); break;
    }
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

}  // extern "C"
