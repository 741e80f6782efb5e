// Fused weight gradient of the channelwise tensor product and the radial MLP's
// output layer: for the per-edge weights w[e] = W h[e] + b (the last Linear of
// src/molrep/interaction/radial_mlp.py:76-82, applied in ConvTP,
// src/molrep/interaction/tensor_product.py:72-79,101-111),
//
//   grad_h[e][k] = sum_n gw[e][n] W[n][k],
//   gw[e][p*C + c] = sum_m3 g[r][o3+m3][c] sum_m1 M_p(Y[e])[m3][m1] x[s][o1+m1][c]
//
// with s / r the edge's sender / receiver and g the gradient of the scattered
// output.  gw is the tensor product's weight gradient; here it never leaves the
// registers: each wavefront owns 32 edges (lanes = edges, two lanes per edge),
// produces gw for 8 consecutive channels of one path per lane and k-step, in
// the operand layout of v_mfma_f32_32x32x16_f16, and multiplies it straight
// into grad_h with the pre-split output-layer weights streamed through LDS --
// the matrix-core part of edge_weights.hip's backward, whose gradient rows are
// otherwise read from the (E x num_paths*C) tensor the tensor-product backward
// writes.  Products are near-fp32: gw rows are brought to a power-of-two scale
// (the running maximum over the stages seen so far) and split into two fp16
// parts, W columns likewise at pack time; three fp16 products per pair are
// accumulated in fp32 (see edge_weights.hip).

#include <utility>

#include "common.h"
#include "ew.h"

namespace mnx {
namespace {

template <int CFG>
struct TPGH;
template <int CFG>
struct TPGH2;

#include "tp_gh_gen.inc"

template <int CFG, int T>
__global__ __launch_bounds__(kEwBwdThreads) void k_tp_gh(const float* __restrict__ x, const float* __restrict__ Y,
                                                         const float* __restrict__ g,
                                                         const int64_t* __restrict__ ei, int64_t E, int64_t Nn,
                                                         int C, const f16x8* __restrict__ frag,
                                                         const float* __restrict__ colscale, int K, int nstages,
                                                         float* __restrict__ gh) {
    using P = TPGH<CFG>;
    constexpr int NQ = 8 / T;
    __shared__ f16x8 sB[2][kEwStageVec];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5;
    const int64_t row0 = int64_t(blockIdx.x) * kEwBwdRows + wave * 32;
    const int64_t arow = row0 + (lane & 31);
    const bool aok = arow < E;
    int64_t snd = 0, rcv = 0;
    bool eok = false;
    if (aok) {
        snd = ei[2 * arow];
        rcv = ei[2 * arow + 1];
        eok = snd >= 0 && snd < Nn && rcv >= 0 && rcv < Nn;
    }
    float y[P::NY];
#pragma unroll
    for (int i = 0; i < P::NY; ++i) y[i] = eok ? Y[arow * P::NY + i] : 0.f;
    const float* xr = x + (eok ? snd : 0) * int64_t(P::NX) * C + 8 * half;
    const float* gr = g + (eok ? rcv : 0) * int64_t(P::NO) * C + 8 * half;
    const int N = P::NP * C;

    // gw of stage s: NQ k-steps of 16 columns n = p*C + c (this lane: 8 of them)
    f32x4 ra[NQ][2];
    auto make_a = [&](int s) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int n0 = 16 * (NQ * s + q);
            float v[8];
            if (eok && n0 < N) {
                const int p = n0 / C, c = n0 - p * C;
                P::gw(p, xr + c, gr + c, C, y, v);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = 0.f;
            }
            ra[q][0] = f32x4{v[0], v[1], v[2], v[3]};
            ra[q][1] = f32x4{v[4], v[5], v[6], v[7]};
        }
    };
    constexpr int PER = kEwStageVec / kEwBwdThreads;
    f16x8 pre[PER];
    auto fetch_b = [&](int s) {
        const f16x8* src = frag + int64_t(s) * kEwStageVec + threadIdx.x;
#pragma unroll
        for (int i = 0; i < PER; ++i) pre[i] = src[i * kEwBwdThreads];
    };

    // acc[t]: D = W^T gw^T, register r of lane l = gh[row0 + l%32][32t + 8(r/4) + 4(l/32) + r%4],
    // in units of 2^ecur (this lane's row scale so far)
    f32x16 acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = f32x16{};
    int ecur = kEwNoExp;
    fetch_b(0);
    make_a(0);
    for (int s = 0; s < nstages; ++s) {
        const int buf = s & 1;
#pragma unroll
        for (int i = 0; i < PER; ++i) sB[buf][threadIdx.x + i * kEwBwdThreads] = pre[i];
        float m = 0.f;
#pragma unroll
        for (int q = 0; q < NQ; ++q) m = absmax8(ra[q][0], ra[q][1], m);
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
        for (int q = 0; q < NQ; ++q) split8(ra[q][0], ra[q][1], si, g0[q], g1[q]);
        __syncthreads();
        if (s + 1 < nstages) fetch_b(s + 1);
        const f16x8* B = &sB[buf][lane];
        auto wq = [&](int pl, int q, int t) -> const f16x8& { return B[((pl * NQ + q) * T + t) * 64]; };
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
                acc[t] = mfma(wq(0, q, t), g1[q], acc[t]);
                acc[t] = mfma(wq(1, q, t), g0[q], acc[t]);
                acc[t] = mfma(wq(0, q, t), g0[q], acc[t]);
            }
        }
        // the next stage's gradient rows while the matrix cores work on this one
        if (s + 1 < nstages) make_a(s + 1);
    }
    if (!aok) return;
    const float so = ldexpf(1.f, ecur == kEwNoExp ? 0 : ecur);
    float* dst = gh + arow * K;
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const int c = 32 * t + 8 * r4 + 4 * half;
            if (c >= K) continue;
            const f32x4 cs = *reinterpret_cast<const f32x4*>(colscale + c);
            f32x4 v;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = acc[t][4 * r4 + i] * so * cs[i];
            *reinterpret_cast<f32x4*>(dst + c) = v;
        }
}

// Receiver-batched form.  Wavefront w of the workgroup takes batch b = 4 blockIdx + w:
// up to 32 consecutive edges of one receiver's CSR segment (batches = (receiver, first
// slot) pairs), lanes l and l + 32 sharing edge l % 32 as in k_tp_gh.  The contraction
// over n = p*C + c runs in the order of TPGH2<CFG>::run (group, 16-channel chunk, path):
// the lane's sender rows of a group and its share of the receiver's output-gradient rows
// are loaded one chunk ahead, the gradient rows staged in the wavefront's LDS area, so each
// k-step forms gw from registers and LDS.  The weights come pre-arranged in that order
// (the backward fragment of W with its rows permuted); each k-step's slice of them is
// staged through LDS for the four wavefronts, double-buffered, one barrier per k-step.
template <int T>
struct GH2Sink {
    static constexpr int NQ = 8 / T;            // k-steps per fragment stage
    static constexpr int kVec = 2 * T * 64;      // f16x8 per k-step (both planes)
    static constexpr int PER = (kVec + kEwBwdThreads - 1) / kEwBwdThreads;
    f16x8 (*sB)[kVec];
    const f16x8* frag;
    f32x16 acc[T];
    f16x8 pre[PER];
    int ecur, ks, nks, lane;

    // this thread's share of k-step k's weights: plane p, tile t of k-step q of stage k / NQ
    __device__ __forceinline__ void fetch(int k) {
        const int st = k / NQ, q = k - st * NQ;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = threadIdx.x + i * kEwBwdThreads;
            if (idx < kVec) {
                const int pl = idx / (T * 64), rest = idx - pl * (T * 64);
                pre[i] = frag[int64_t(st) * kEwStageVec + (pl * NQ + q) * (T * 64) + rest];
            }
        }
    }

    __device__ __forceinline__ void step(f32x4 o0, f32x4 o1) {
        float m = absmax8(o0, o1, 0.f);
        m = fmaxf(m, __shfl_xor(m, 32));
        const int enew = max(ecur, ew_exp(m));
        if (__ballot(enew != ecur)) {
            const float f = ldexpf(1.f, ecur - enew);
#pragma unroll
            for (int i = 0; i < T; ++i) acc[i] *= f;
        }
        ecur = enew;
        f16x8 g0, g1;
        split8(o0, o1, ldexpf(1.f, -ecur), g0, g1);
        f16x8* B = sB[ks & 1];
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = threadIdx.x + i * kEwBwdThreads;
            if (idx < kVec) B[idx] = pre[i];
        }
        __syncthreads();
        if (ks + 1 < nks) fetch(ks + 1);
#pragma unroll
        for (int i = 0; i < T; ++i) acc[i] = mfma(B[(0 * T + i) * 64 + lane], g1, acc[i]);
#pragma unroll
        for (int i = 0; i < T; ++i) acc[i] = mfma(B[(1 * T + i) * 64 + lane], g0, acc[i]);
#pragma unroll
        for (int i = 0; i < T; ++i) acc[i] = mfma(B[(0 * T + i) * 64 + lane], g0, acc[i]);
        ++ks;
    }
};

template <int CFG, int T>
__global__ __launch_bounds__(kEwBwdThreads, 2) void k_tp_gh2(const float* __restrict__ x,
                                                             const float* __restrict__ Y,
                                                             const float* __restrict__ g,
                                                             const int32_t* __restrict__ row_ptr,
                                                             const int32_t* __restrict__ perm,
                                                             const int32_t* __restrict__ snd,
                                                             const int32_t* __restrict__ batches, int64_t nbatch,
                                                             int C, const f16x8* __restrict__ frag,
                                                             const float* __restrict__ colscale, int K,
                                                             float* __restrict__ gh) {
    using P = TPGH2<CFG>;
    using Sink = GH2Sink<T>;
    constexpr int kWaves = kEwBwdThreads / 64;
    __shared__ f16x8 sB[2][Sink::kVec];
    __shared__ f32x4 sG[kWaves][2 * P::GROWS * 4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5;
    const int64_t b = int64_t(blockIdx.x) * kWaves + wave;
    const bool bok = b < nbatch;  // wave-uniform
    int r = 0, t0 = 0, t1 = 0;
    if (bok) {
        r = batches[2 * b];
        t0 = batches[2 * b + 1];
        t1 = min(t0 + 32, row_ptr[r + 1]);
    }
    const int t = t0 + (lane & 31);
    const bool eok = bok && t < t1;
    const int e = eok ? perm[t] : 0, sn = eok ? snd[t] : 0;
    float y[P::NY];
#pragma unroll
    for (int i = 0; i < P::NY; ++i) y[i] = eok ? Y[int64_t(e) * P::NY + i] : 0.f;
    const float* xr = x + int64_t(sn) * (int64_t(P::NX) * C) + 8 * half;
    const float* grow = g + int64_t(r) * (int64_t(P::NO) * C);

    Sink st;
    st.sB = sB;
    st.frag = frag;
#pragma unroll
    for (int i = 0; i < T; ++i) st.acc[i] = f32x16{};
    st.ecur = kEwNoExp;
    st.ks = 0;
    st.nks = (C / 16) * P::NP;
    st.lane = lane;
    st.fetch(0);
    P::run(st, xr, grow, C, reinterpret_cast<float*>(&sG[wave][0]), lane, eok, bok, y);

    if (!eok) return;
    const float so = ldexpf(1.f, st.ecur == kEwNoExp ? 0 : st.ecur);
    float* dst = gh + int64_t(e) * K;
#pragma unroll
    for (int i = 0; i < T; ++i)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const int c = 32 * i + 8 * r4 + 4 * half;
            if (c >= K) continue;
            const f32x4 cs = *reinterpret_cast<const f32x4*>(colscale + c);
            f32x4 v;
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] = st.acc[i][4 * r4 + k] * so * cs[k];
            *reinterpret_cast<f32x4*>(dst + c) = v;
        }
}

typedef void (*TPGH2Fn)(const float*, const float*, const float*, const int32_t*, const int32_t*, const int32_t*,
                        const int32_t*, int64_t, int, const f16x8*, const float*, int, float*);

template <int CFG>
TPGH2Fn pick2_tiles(int tiles) {
    switch (tiles) {
        case 1: return k_tp_gh2<CFG, 1>;
        case 2: return k_tp_gh2<CFG, 2>;
        default: return k_tp_gh2<CFG, 4>;
    }
}

template <int... I>
TPGH2Fn pick2(int cfg, int tiles, std::integer_sequence<int, I...>) {
    TPGH2Fn fn = nullptr;
    ((cfg == I ? (fn = pick2_tiles<I>(tiles), 0) : 0), ...);
    return fn;
}

typedef void (*TPGHFn)(const float*, const float*, const float*, const int64_t*, int64_t, int64_t, int,
                       const f16x8*, const float*, int, int, float*);

template <int CFG>
TPGHFn pick_tiles(int tiles) {
    switch (tiles) {
        case 1: return k_tp_gh<CFG, 1>;
        case 2: return k_tp_gh<CFG, 2>;
        default: return k_tp_gh<CFG, 4>;
    }
}

template <int... I>
TPGHFn pick(int cfg, int tiles, std::integer_sequence<int, I...>) {
    TPGHFn fn = nullptr;
    ((cfg == I ? (fn = pick_tiles<I>(tiles), 0) : 0), ...);
    return fn;
}

// W rows in k_tp_gh2's contraction order: group by group, 16-channel chunk, path.
template <int CFG>
void gh2_rows(int C, int32_t* rows) {
    using P = TPGH2<CFG>;
    int n = 0, base = 0;
    for (int G = 0; G < P::NG; ++G) {
        for (int cc = 0; cc < C / 16; ++cc)
            for (int j = 0; j < P::GP[G]; ++j) {
                const int p = P::ORDER[base + j];
                for (int i = 0; i < 16; ++i) rows[n++] = p * C + 16 * cc + i;
            }
        base += P::GP[G];
    }
}

template <int... I>
void pick_rows(int cfg, int C, int32_t* rows, std::integer_sequence<int, I...>) {
    ((cfg == I ? (gh2_rows<I>(C, rows), 0) : 0), ...);
}

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

int mnx_tp_weight_grad_f32(int32_t config, int32_t C, const float* x, const float* Y, const float* grad_out,
                           const int64_t* edge_index, int64_t num_nodes, int64_t num_edges, const uint16_t* frag,
                           int32_t K, float* grad_h, mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(config >= 0 && config < kNumTPGHConfigs, "invalid tp config %d", config);
    MNX_REQUIRE(C > 0 && C % 16 == 0 && C <= 4096, "channels must be a positive multiple of 16, got %d", C);
    MNX_REQUIRE(K == 16 || K == 32 || K == 64 || K == 128, "hidden width %d not 16, 32, 64 or 128", K);
    MNX_REQUIRE(num_nodes >= 0 && num_nodes < (int64_t(1) << 31) && num_edges >= 0 &&
                    num_edges < (int64_t(1) << 31), "sizes out of range");
    if (num_edges == 0) return MNX_OK;
    MNX_REQUIRE(x && Y && grad_out && edge_index && frag && grad_h, "null pointer argument");
    MNX_REQUIRE(((uintptr_t)x | (uintptr_t)grad_out | (uintptr_t)frag) % 16 == 0,
                "x, grad_out and frag must be 16-byte aligned");
    int np = 0;
    {
        int32_t info[4];
        if (mnx_tp_config_info(config, info)) return MNX_ERR_INVALID;
        np = info[0];
    }
    const EwShape sh{K, np * C};
    const f16x8* f = reinterpret_cast<const f16x8*>(frag);
    const float* cs = reinterpret_cast<const float*>(frag + sh.planes(true));
    TPGHFn fn = pick(config, sh.tiles_b(), std::make_integer_sequence<int, kNumTPGHConfigs>{});
    MNX_REQUIRE(fn, "no fused weight-gradient kernel for config %d", config);
    hipLaunchKernelGGL(fn, dim3(unsigned(ceil_div(num_edges, kEwBwdRows))), dim3(kEwBwdThreads), 0,
                       (hipStream_t)stream, x, Y, grad_out, edge_index, num_edges, num_nodes, C, f, cs, K,
                       sh.stages_b(), grad_h);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_tp_weight_grad_batched_f32(int32_t config, int32_t C, const float* x, const float* Y, const float* grad_out,
                                   const int32_t* row_ptr, const int32_t* perm, const int32_t* senders,
                                   const int32_t* batches, int64_t num_batches, int64_t num_nodes,
                                   int64_t num_edges, const uint16_t* frag, int32_t K, float* grad_h,
                                   mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(config >= 0 && config < kNumTPGHConfigs, "invalid tp config %d", config);
    MNX_REQUIRE(C > 0 && C % 16 == 0 && C <= 4096, "channels must be a positive multiple of 16, got %d", C);
    MNX_REQUIRE(K == 16 || K == 32 || K == 64 || K == 128, "hidden width %d not 16, 32, 64 or 128", K);
    MNX_REQUIRE(num_nodes >= 0 && num_nodes < (int64_t(1) << 31) && num_edges >= 0 &&
                    num_edges < (int64_t(1) << 31) && num_batches >= 0 && num_batches < (int64_t(1) << 31),
                "sizes out of range");
    if (num_edges == 0 || num_batches == 0) return MNX_OK;
    MNX_REQUIRE(x && Y && grad_out && row_ptr && perm && senders && batches && frag && grad_h,
                "null pointer argument");
    MNX_REQUIRE(((uintptr_t)x | (uintptr_t)grad_out | (uintptr_t)frag) % 16 == 0,
                "x, grad_out and frag must be 16-byte aligned");
    int np = 0;
    {
        int32_t info[4];
        if (mnx_tp_config_info(config, info)) return MNX_ERR_INVALID;
        np = info[0];
    }
    const EwShape sh{K, np * C};
    const f16x8* f = reinterpret_cast<const f16x8*>(frag);
    const float* cs = reinterpret_cast<const float*>(frag + sh.planes(true));
    TPGH2Fn fn = pick2(config, sh.tiles_b(), std::make_integer_sequence<int, kNumTPGHConfigs>{});
    MNX_REQUIRE(fn, "no fused weight-gradient kernel for config %d", config);
    hipLaunchKernelGGL(fn, dim3(unsigned(ceil_div(num_batches, kEwBwdThreads / 64))), dim3(kEwBwdThreads), 0,
                       (hipStream_t)stream, x, Y, grad_out, row_ptr, perm, senders, batches, num_batches, C, f, cs,
                       K, grad_h);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_tp_weight_grad_rows(int32_t config, int32_t C, int32_t* rows) {
    clear_error();
    MNX_REQUIRE(config >= 0 && config < kNumTPGHConfigs, "invalid tp config %d", config);
    MNX_REQUIRE(C > 0 && C % 16 == 0 && C <= 4096, "channels must be a positive multiple of 16, got %d", C);
    MNX_REQUIRE(rows, "null pointer argument");
    pick_rows(config, C, rows, std::make_integer_sequence<int, kNumTPGHConfigs>{});
    return MNX_OK;
}

}  // extern "C"
