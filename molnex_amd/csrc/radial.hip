// Hidden stack of the radial weight MLP, fused into one kernel per direction:
//   h = silu(W_L ... silu(W_2 silu(W_1 f + b_1) + b_2) ... + b_L)
// with f the (E, K) radial edge features and h (E, H) the input of the MLP's
// last Linear (src/molrep/interaction/radial_mlp.py:38-93: [Linear(in, hidden) ->
// SiLU] x num_layers, then Linear(hidden, out)).  The backward maps dL/dh to
// dL/df, recomputing the forward in registers.
//
// One wavefront owns 32 edges.  Every layer is a v_mfma_f32_32x32x2f32 product
// with the features on the M side and the 32 edges on the N side:
//   out^T (H x 32) = W (H x K) . in^T (K x 32).
// The D layout of an MFMA tile (lane l holds column l%32, i.e. one edge, and
// rows 8*(r/4) + 4*(l/32) + r%4 in register r) is taken directly as the B
// operand of the next layer by ordering the contraction index so that k-step s
// of lane half h reads feature 8*(s/4) + 4*h + s%4 -- the feature that register
// s%16 of tile s/16 holds.  Activations therefore stay in registers across
// layers.  The weights are pre-arranged (k_radial_pack) in that k order,
// "fragment" layout [tile][s/4][lane][s%4], staged through LDS, so every
// A-operand read is one conflict-free 16-byte LDS read per lane.
//
// Layers with K = hidden inputs (every layer but the first, forward and
// backward) run on the fp16 matrix cores with near-fp32 products: each edge's
// activation column and each weight row are brought to a power-of-two scale
// (largest magnitude in [1, 2)), every scaled value v is split into two fp16
// parts, v0 = f16(v), v1 = f16(v - v0) (|v - v0 - v1| <= 2^-22 |v|), and the
// three partial products w1 v0 + w0 v1 + w0 v0 are accumulated in fp32 by
// v_mfma_f32_32x32x16_f16 (the dropped terms are below 3 * 2^-22 |w v|); the
// scales are undone exactly on the accumulator.  The D layout feeds these
// layers too: fp16 k-step q of lane half h, element j, is feature
// 16q + 8(j/4) + 4h + j%4, i.e. registers 8(q%2) .. +7 of tile q/2.  The weights
// of these layers are pre-scaled and pre-split into two fp16 planes, layout
// [q][tile][plane][lane][8], with one scale per output row.  The first layer
// (K = the few radial features) stays on fp32 MFMAs.

#include "common.h"

namespace mnx {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kRadThreads = 256;  // four wavefronts, 32 edges each
constexpr int kRadEdgesPerBlock = (kRadThreads / 64) * 32;
constexpr int kRadMaxIn = 64;

// Fragment buffer layout (floats): forward fragments of layers 0..L-1, backward
// (transposed) fragments of layers 0..L-1, the L x H biases, then the row scales
// of the split blocks (forward layers 1..L-1: H each; backward layers 0..L-1:
// 32 * tiles_bwd(j) each; powers of two).  Forward layer 0 is fp32
// ([tile][kp/8][lane][4]); every other block holds two fp16 planes,
// [H/16][tiles][2][lane][8] (512 floats per k-step and tile).
constexpr int kX2Block = 512;  // floats per (k-step, tile) of split-fp16 fragments

struct RadLayout {
    int kin, kp, H, L;
    __host__ __device__ int tiles_bwd(int j) const { return ((j == 0 ? kp : H) + 31) / 32; }
    __host__ __device__ int64_t fwd_size(int j) const {
        return j == 0 ? int64_t(H / 32) * (kp / 8) * 256 : int64_t(H / 32) * (H / 16) * kX2Block;
    }
    __host__ __device__ int64_t bwd_size(int j) const { return int64_t(tiles_bwd(j)) * (H / 16) * kX2Block; }
    __host__ __device__ int64_t fwd_off(int j) const {
        int64_t o = 0;
        for (int i = 0; i < j; ++i) o += fwd_size(i);
        return o;
    }
    __host__ __device__ int64_t bwd_off(int j) const {
        int64_t o = fwd_off(L);
        for (int i = 0; i < j; ++i) o += bwd_size(i);
        return o;
    }
    __host__ __device__ int64_t bias_off() const { return bwd_off(L); }
    // row scales: forward layer j >= 1, backward layer j
    __host__ __device__ int64_t fscale_off(int j) const { return bias_off() + int64_t(L) * H + int64_t(j - 1) * H; }
    __host__ __device__ int64_t bscale_off(int j) const {
        int64_t o = bias_off() + int64_t(L) * H + int64_t(L - 1) * H;
        for (int i = 0; i < j; ++i) o += 32 * tiles_bwd(i);
        return o;
    }
    __host__ __device__ int64_t scales_total() const { return int64_t(L - 1) * H + (bscale_off(L) - bscale_off(0)); }
    __host__ __device__ int64_t total() const { return bscale_off(L); }
    // raw parameters: per layer W_j (H x K_j, row-major as torch.nn.Linear) then b_j (H)
    __host__ __device__ int64_t raw_w(int j) const { return j == 0 ? 0 : int64_t(H) * kin + H + int64_t(j - 1) * (H * H + H); }
    __host__ __device__ int64_t raw_b(int j) const { return raw_w(j) + int64_t(H) * (j == 0 ? kin : H); }
    __host__ __device__ int64_t raw_total() const { return raw_w(L); }
};

// Exponent e with 2^e <= m < 2^(e+1), clamped so that 2^e and 2^-e are normal; 0 for
// m == 0 and for inf/NaN (left to propagate).
__device__ __forceinline__ int rad_exp(float m) {
    if (!(m > 0.f) || !(m <= 3.402823466e38f)) return 0;
    return min(max(ilogbf(m), -126), 126);
}

// Row scales of the split blocks, one wavefront per row: forward layer j >= 1 row m
// is W_j[m][:], backward layer j row m is column m of W_j (W_j^T[m][:]); rows past
// the layer (padding of the last tile) get 1.
__global__ void k_radial_scales(const float* __restrict__ raw, RadLayout lay, float* __restrict__ frag) {
    const int lane = threadIdx.x & 63;
    const int64_t i = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
    const int64_t n = lay.scales_total();
    if (i >= n) return;
    const int64_t o = lay.fscale_off(1) + i;
    float m = 0.f;
    if (o < lay.bscale_off(0)) {  // forward layer j >= 1
        const int j = 1 + int(i / lay.H), row = int(i % lay.H);
        const float* W = raw + lay.raw_w(j);
        for (int f = lane; f < lay.H; f += 64) m = fmaxf(m, fabsf(W[int64_t(row) * lay.H + f]));
    } else {
        int j = 0;
        while (o >= lay.bscale_off(j + 1)) ++j;
        const int row = int(o - lay.bscale_off(j));
        const int kraw = j == 0 ? lay.kin : lay.H;
        const float* W = raw + lay.raw_w(j);
        if (row < kraw)
            for (int f = lane; f < lay.H; f += 64) m = fmaxf(m, fabsf(W[int64_t(f) * kraw + row]));
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if (lane == 0) frag[o] = ldexpf(1.f, rad_exp(m));
}

// Builds the fragment buffer from the raw parameters and the row scales (already in
// place); one thread per float (two fp16 values in the split blocks).
__global__ void k_radial_pack(const float* __restrict__ raw, RadLayout lay, float* __restrict__ frag) {
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= lay.fscale_off(1)) return;
    float v = 0.f;
    if (idx >= lay.bias_off()) {
        const int64_t b = idx - lay.bias_off();
        const int j = int(b / lay.H), m = int(b % lay.H);
        v = raw[lay.raw_b(j) + m];
    } else if (idx < lay.fwd_off(1)) {
        // forward layer 0, fp32 fragments [tile][q][lane][4]: k-step 4q+i of lane half h = feature 8q+4h+i
        const int i = int(idx % 4), lane = int((idx / 4) % 64);
        const int64_t rest = idx / 256;
        const int nq = lay.kp / 8;
        const int q = int(rest % nq), t = int(rest / nq);
        const int k = 8 * q + 4 * (lane / 32) + i;
        const int row = 32 * t + lane % 32;
        if (k < lay.kin) v = raw[lay.raw_w(0) + int64_t(row) * lay.kin + k];
    } else {
        const bool bwd = idx >= lay.bwd_off(0);
        int j = bwd ? 0 : 1;
        while (idx >= (bwd ? lay.bwd_off(j + 1) : lay.fwd_off(j + 1))) ++j;
        const int64_t r = idx - (bwd ? lay.bwd_off(j) : lay.fwd_off(j));
        const int kraw = j == 0 ? lay.kin : lay.H;  // layer j's input width
        const int tiles = bwd ? lay.tiles_bwd(j) : lay.H / 32;
        const float* W = raw + lay.raw_w(j);
        const float* scale = frag + (bwd ? lay.bscale_off(j) : lay.fscale_off(j));
        f16x2 pair;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t e = 2 * r + u;  // fp16 element within the block
            const int j8 = int(e % 8), lane = int((e / 8) % 64), p = int((e / 512) % 2);
            const int t = int((e / 1024) % tiles), q = int(e / (1024 * int64_t(tiles)));
            const int row = 32 * t + lane % 32;                                // A row
            const int f = 16 * q + 8 * (j8 / 4) + 4 * (lane / 32) + j8 % 4;  // contraction feature
            float w = 0.f;
            if (!bwd) {
                if (row < lay.H && f < lay.H) w = W[int64_t(row) * kraw + f];  // W_j[out][in]
            } else {
                if (row < kraw && f < lay.H) w = W[int64_t(f) * kraw + row];   // W_j^T
            }
            w = ldexpf(w, -ilogbf(scale[row]));
            const _Float16 h0 = (_Float16)w;
            pair[u] = p == 0 ? h0 : (_Float16)(w - (float)h0);
        }
        v = __builtin_bit_cast(float, pair);
    }
    frag[idx] = v;
}

// sigmoid(z) = 1 / (1 + 2^(-z log2 e)) from the hardware exp2 and reciprocal (a few
// ulp; the IEEE-exact expf and division would cost ~28 VALU instructions per
// element, as much issue time as the MFMAs of a layer).  Saturates correctly:
// z -> -inf gives 1/inf = 0, z -> +inf gives 1.
__device__ __forceinline__ float sigmoid(float z) {
    return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(z * -1.4426950408889634f));
}

__device__ __forceinline__ float silu(float z) { return z * sigmoid(z); }

__device__ __forceinline__ float silu_grad(float z) {
    const float s = sigmoid(z);
    return s * (1.f + z * (1.f - s));
}

// Fragments reach the MFMAs through LDS: a workgroup stages up to kRadChunk
// floats of one layer's fragments (whole output tiles) at a time and its four
// wavefronts share them.
constexpr int kRadChunk = 8192;       // floats (32 KB)
constexpr int kRadChunkWide = 16384;  // floats (64 KB): a whole 128-wide layer, for the backward

template <int CH>
struct RadSharedT {
    static constexpr int kChunk = CH;
    f32x4 frag[CH / 4];
    float bias[4 * 128];
};

// Copies n floats (a multiple of 4, 16-byte aligned) of fragments into LDS; the
// caller brackets it with barriers.
__device__ __forceinline__ void stage(const float* __restrict__ src, int n, f32x4* __restrict__ dst) {
    const f32x4* s4 = reinterpret_cast<const f32x4*>(src);
    for (int i = threadIdx.x; i < n / 4; i += kRadThreads) dst[i] = s4[i];
}

// Exponent of the lane's activation column (largest magnitude over both lane
// halves, i.e. the whole edge) for the split of a layer's B operand.
template <int NQ>
__device__ __forceinline__ int column_exp(const float (&in)[NQ / 2][16]) {
    float m = 0.f;
#pragma unroll
    for (int t = 0; t < NQ / 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) m = fmaxf(m, fabsf(in[t][r]));
    m = fmaxf(m, __shfl_xor(m, 32));
    return rad_exp(m);
}

// k-steps q0 .. q0 + QN - 1 (those below NQ) of a split-fp16 layer: fragments fr
// (LDS, k-step q0 first, [QN][T][2][64 lanes] f32x4 of 8 fp16), activations in
// the D layout scaled by sinv before the split.
template <int T, int NQ, int QN>
__device__ __forceinline__ void mfma_steps(const f32x4* __restrict__ fr, int q0, const float (&in)[NQ / 2][16],
                                           float sinv, f32x16 (&acc)[T], int lane) {
#pragma unroll
    for (int qq = 0; qq < QN; ++qq) {
        const int q = q0 + qq;
        if (q >= NQ) break;
        f16x8 b0, b1;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float v = in[q / 2][8 * (q % 2) + j] * sinv;
            const _Float16 h0 = (_Float16)v;
            b0[j] = h0;
            b1[j] = (_Float16)(v - (float)h0);
        }
        auto a = [&](int t, int p) { return __builtin_bit_cast(f16x8, fr[((qq * T + t) * 2 + p) * 64 + lane]); };
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a(t, 1), b0, acc[t], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a(t, 0), b1, acc[t], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a(t, 0), b0, acc[t], 0, 0, 0);
    }
}

// Undoes the column scale 2^-ex and the weight row scales rscale on the accumulator.
template <int T>
__device__ __forceinline__ void unscale(const float* __restrict__ rscale, int ex, f32x16 (&acc)[T], int lane) {
    const float so = ldexpf(1.f, ex);
    const int half = lane >> 5;
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 rs = *reinterpret_cast<const f32x4*>(rscale + 32 * t + 8 * g + 4 * half);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t][4 * g + i] = acc[t][4 * g + i] * so * rs[i];
        }
}

// acc[t] = W(tile t) . in over K = 16 * NQ features held in the D layout as
// in[q/2][8(q%2) + j] for k-step q (split-fp16 products, see the top of the file),
// acc zero on entry.  The layer's fragments f ([NQ][T][2][64 lanes][8 fp16]) are
// staged in chunks of whole k-steps; rscale holds the layer's row scales.  The
// lane's activations are scaled by their edge's power of two (largest magnitude
// of the column in [1, 2)) before the split and the result by its inverse and the
// row scales.  Every wavefront of the workgroup must call it (barriers inside).
template <int T, int NQ, class Sh>
__device__ __forceinline__ void mfma_layer(const float* __restrict__ f, const float* __restrict__ rscale,
                                           const float (&in)[NQ / 2][16], f32x16 (&acc)[T], Sh& sh, int lane) {
    constexpr int kRadChunk = Sh::kChunk;
    constexpr int kStep = T * kX2Block;  // floats per k-step
    constexpr int kQPC = kRadChunk / kStep < NQ ? kRadChunk / kStep : NQ;  // k-steps per chunk
    static_assert(kQPC >= 1, "one k-step of fragments must fit the staging area");
    const int ex = column_exp<NQ>(in);
    const float sinv = ldexpf(1.f, -ex);
#pragma unroll
    for (int q0 = 0; q0 < NQ; q0 += kQPC) {
        __syncthreads();
        stage(f + q0 * kStep, (NQ - q0 < kQPC ? NQ - q0 : kQPC) * kStep, sh.frag);
        __syncthreads();
        mfma_steps<T, NQ, kQPC>(sh.frag, q0, in, sinv, acc, lane);
    }
    unscale<T>(rscale, ex, acc, lane);
}

// The same product with the whole layer's fragments resident in LDS (no barriers).
// Software-pipelined one k-step ahead: the fragments of k-step q + 1 are read and
// its activations split while the matrix cores work on k-step q (two register
// buffers each).  At four row tiles a scheduling barrier per k-step keeps the
// compiler from hoisting every k-step's reads to the top (which costs ~256
// registers at one wavefront per SIMD); narrower layers leave it free.
template <int T, int NQ>
__device__ __forceinline__ void mfma_layer_res(const f32x4* __restrict__ fr, const float* __restrict__ rscale,
                                               const float (&in)[NQ / 2][16], f32x16 (&acc)[T], int lane) {
    const int ex = column_exp<NQ>(in);
    const float sinv = ldexpf(1.f, -ex);
    f32x4 buf[2][T][2];
    f16x8 b0[2], b1[2];
    auto fetch = [&](int q) {
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int p = 0; p < 2; ++p) buf[q & 1][t][p] = fr[((q * T + t) * 2 + p) * 64 + lane];
    };
    auto split = [&](int q) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float v = in[q / 2][8 * (q % 2) + j] * sinv;
            const _Float16 h0 = (_Float16)v;
            b0[q & 1][j] = h0;
            b1[q & 1][j] = (_Float16)(v - (float)h0);
        }
    };
    fetch(0);
    split(0);
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        if (q + 1 < NQ) {
            fetch(q + 1);
            split(q + 1);
        }
        auto a = [&](int t, int p) { return __builtin_bit_cast(f16x8, buf[q & 1][t][p]); };
#pragma unroll
        for (int t = 0; t < T; ++t)
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a(t, 1), b0[q & 1], acc[t], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < T; ++t)
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a(t, 0), b1[q & 1], acc[t], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < T; ++t)
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a(t, 0), b0[q & 1], acc[t], 0, 0, 0);
        if constexpr (T >= 4) __builtin_amdgcn_sched_barrier(0);
    }
    unscale<T>(rscale, ex, acc, lane);
}

// Layer 0: B operand read straight from the (E, kin) features; k-step 4q+i of lane
// half h = feature 8q+4h+i.  Its fragments (T x kp/8 blocks) fit one chunk.
template <int T, class Sh>
__device__ __forceinline__ void first_layer(const float* __restrict__ f, const float* __restrict__ feats, int64_t e,
                                            bool valid, int kin, int kp, f32x16 (&acc)[T], Sh& sh, int lane) {
    const int nq = kp / 8, half = lane >> 5;
    __syncthreads();
    stage(f, T * nq * 256, sh.frag);
    __syncthreads();
    for (int q = 0; q < nq; ++q) {
        float b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int k = 8 * q + 4 * half + i;
            b[i] = (valid && k < kin) ? feats[e * kin + k] : 0.f;
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const f32x4 a = sh.frag[(t * nq + q) * 64 + lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[i], acc[t], 0, 0, 0);
        }
    }
}

// Layer 0 with its fragments resident in LDS at fr.
template <int T>
__device__ __forceinline__ void first_layer_res(const f32x4* __restrict__ fr, const float* __restrict__ feats,
                                                int64_t e, bool valid, int kin, int kp, f32x16 (&acc)[T], int lane) {
    const int nq = kp / 8, half = lane >> 5;
    for (int q = 0; q < nq; ++q) {
        float b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int k = 8 * q + 4 * half + i;
            b[i] = (valid && k < kin) ? feats[e * kin + k] : 0.f;
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const f32x4 a = fr[(t * nq + q) * 64 + lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[i], acc[t], 0, 0, 0);
        }
    }
}

template <int T>
__device__ __forceinline__ void zero(f32x16 (&acc)[T]) {
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
}

// feature index of register r of tile t in lane half h
__device__ __forceinline__ int dfeat(int t, int r, int half) { return 32 * t + 8 * (r / 4) + 4 * half + r % 4; }

// Biases into LDS (read once per workgroup); visible after the next barrier.
template <class Sh>
__device__ __forceinline__ void stage_bias(const float* __restrict__ b, int n, Sh& sh) {
    for (int i = threadIdx.x; i < n; i += kRadThreads) sh.bias[i] = b[i];
}

// Wavefronts past the last edge still run (all lanes invalid) because the
// workgroup shares barriers; they store nothing.
template <int H, int L>
__global__ void __launch_bounds__(kRadThreads) k_radial_fwd(const float* __restrict__ feats, int64_t E, int kin,
                                                            const float* __restrict__ frag, RadLayout lay,
                                                            float* __restrict__ out) {
    constexpr int T = H / 32;
    __shared__ RadSharedT<kRadChunk> sh;
    const int lane = threadIdx.x & 63, half = lane >> 5;
    const int64_t e = (int64_t(blockIdx.x) * (kRadThreads / 64) + threadIdx.x / 64) * 32 + (lane & 31);
    const bool valid = e < E;
    stage_bias(frag + lay.bias_off(), L * H, sh);
    f32x16 acc[T];
    float act[T][16];
    zero(acc);
    first_layer<T>(frag + lay.fwd_off(0), feats, e, valid, kin, lay.kp, acc, sh, lane);
#pragma unroll
    for (int j = 0; j < L; ++j) {
        if (j > 0) {
            zero(acc);
            mfma_layer<T, H / 16>(frag + lay.fwd_off(j), frag + lay.fscale_off(j), act, acc, sh, lane);
        }
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) act[t][r] = silu(acc[t][r] + sh.bias[j * H + dfeat(t, r, half)]);
    }
    if (valid) {
        float* o = out + e * H;
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 v = {act[t][4 * g], act[t][4 * g + 1], act[t][4 * g + 2], act[t][4 * g + 3]};
                *reinterpret_cast<f32x4*>(o + 32 * t + 8 * g + 4 * half) = v;
            }
    }
}

template <int T0>
__device__ __forceinline__ void store_grad_feats(const f32x16 (&a0)[T0], float* __restrict__ grad_feats, int64_t e,
                                                 bool valid, int kin, int half) {
    if (!valid) return;
#pragma unroll
    for (int t = 0; t < T0; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int k = dfeat(t, r, half);
            if (k < kin) grad_feats[e * kin + k] = a0[t][r];
        }
}

template <int H, int L>
__global__ void __launch_bounds__(kRadThreads) k_radial_bwd(const float* __restrict__ feats, int64_t E, int kin,
                                                            const float* __restrict__ frag, RadLayout lay,
                                                            const float* __restrict__ grad_h,
                                                            float* __restrict__ grad_feats) {
    constexpr int T = H / 32;
    __shared__ RadSharedT<H == 128 ? kRadChunkWide : kRadChunk> sh;
    const int lane = threadIdx.x & 63, half = lane >> 5;
    const int64_t e = (int64_t(blockIdx.x) * (kRadThreads / 64) + threadIdx.x / 64) * 32 + (lane & 31);
    const bool valid = e < E;
    stage_bias(frag + lay.bias_off(), L * H, sh);
    // forward recompute, keeping the pre-activations z_0 .. z_{L-2}; the last
    // layer's pre-activation stays in acc (its activation is not needed)
    float z[L > 1 ? L - 1 : 1][T][16];
    float g[T][16];
    f32x16 acc[T];
    zero(acc);
    first_layer<T>(frag + lay.fwd_off(0), feats, e, valid, kin, lay.kp, acc, sh, lane);
#pragma unroll
    for (int j = 0; j < L; ++j) {
        if (j > 0) {
            zero(acc);
            mfma_layer<T, H / 16>(frag + lay.fwd_off(j), frag + lay.fscale_off(j), g, acc, sh, lane);  // g holds silu(z_{j-1})
        }
        if (j < L - 1) {
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    z[j][t][r] = acc[t][r] + sh.bias[j * H + dfeat(t, r, half)];
                    g[t][r] = silu(z[j][t][r]);
                }
        }
    }
    // g = dL/dh * silu'(z_{L-1}), dL/dh read in the D layout
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (valid) v = *reinterpret_cast<const f32x4*>(grad_h + e * H + 32 * t + 8 * q + 4 * half);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 4 * q + i;
                g[t][r] = v[i] * silu_grad(acc[t][r] + sh.bias[(L - 1) * H + dfeat(t, r, half)]);
            }
        }
    // back through layers L-1 .. 1: g <- (W_j^T g) * silu'(z_{j-1})
#pragma unroll
    for (int j = L - 1; j >= 1; --j) {
        zero(acc);
        mfma_layer<T, H / 16>(frag + lay.bwd_off(j), frag + lay.bscale_off(j), g, acc, sh, lane);
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) g[t][r] = acc[t][r] * silu_grad(z[j - 1][t][r]);
    }
    // layer 0: dL/df^T (kp x 32) = W_0^T g, in ceil(kp / 32) <= 2 row tiles
    if (lay.tiles_bwd(0) == 1) {
        f32x16 a0[1];
        zero(a0);
        mfma_layer<1, H / 16>(frag + lay.bwd_off(0), frag + lay.bscale_off(0), g, a0, sh, lane);
        store_grad_feats(a0, grad_feats, e, valid, kin, half);
    } else {
        f32x16 a0[2];
        zero(a0);
        mfma_layer<2, H / 16>(frag + lay.bwd_off(0), frag + lay.bscale_off(0), g, a0, sh, lane);
        store_grad_feats(a0, grad_feats, e, valid, kin, half);
    }
}

// ---------------------------------------------------------------------------
// Resident variants, used when the padded input width is at most kRadResKp:
// the fragments and biases one direction needs (at most ~153 KB, H = 128 with
// two layers backward) are staged into LDS once per workgroup, and each
// wavefront then walks groups of 32 edges, grid-strided, with no further
// barriers -- the per-layer staging of the kernels above (a barrier and up to
// 64 KB copied per layer and 128 edges) dominated at one wavefront per SIMD.
// The grid is as many workgroups as fit the device at once.
// ---------------------------------------------------------------------------

constexpr int kRadResKp = 16;

// A zero the compiler cannot see through, recomputed per edge group: offsetting the
// bias and row-scale pointers by it keeps their loads at their uses (hoisted out of
// the group loop they would hold ~270 registers for the whole kernel).
__device__ __forceinline__ int opaque_zero() {
    int z;
    asm volatile("s_mov_b32 %0, 0" : "=s"(z));
    return z;
}

// KP: the padded input width the LDS copy is sized for (kRadResKp, or 64 for the backward of
// stacks up to 64 wide: the pair embedding's 40 inputs); the input gradient is ceil(KP / 32) row
// tiles.
template <int H, int L, bool BWD, int KP = kRadResKp>
constexpr int rad_res_floats() {
    constexpr int T = H / 32;
    int n = T * (KP / 8) * 256 + (L - 1) * T * (H / 16) * kX2Block + L * H;  // forward layers, biases
    if (BWD) n += ((KP + 31) / 32) * (H / 16) * kX2Block + (L - 1) * T * (H / 16) * kX2Block;  // backward 0, 1..L-1
    return n;
}

template <int H, int L>
__global__ void __launch_bounds__(kRadThreads) k_radial_fwd_res(const float* __restrict__ feats, int64_t E, int kin,
                                                                const float* __restrict__ frag, RadLayout lay,
                                                                float* __restrict__ out) {
    constexpr int T = H / 32;
    __shared__ f32x4 res[rad_res_floats<H, L, false>() / 4];
    const int nf = int(lay.fwd_off(L));  // forward fragments, then the biases
    stage(frag, nf, res);
    stage(frag + lay.bias_off(), L * H, res + nf / 4);
    __syncthreads();
    const float* bias = reinterpret_cast<const float*>(res) + nf;
    const int lane = threadIdx.x & 63, half = lane >> 5;
    const int64_t groups = (E + 31) / 32, stride = int64_t(gridDim.x) * (kRadThreads / 64);
    for (int64_t grp = int64_t(blockIdx.x) * (kRadThreads / 64) + (threadIdx.x >> 6); grp < groups; grp += stride) {
        const int64_t e = grp * 32 + (lane & 31);
        const bool valid = e < E;
        const int z0 = opaque_zero();
        const float* bs = bias + z0;
        const float* fs = frag + z0;
        f32x16 acc[T];
        float act[T][16];
        zero(acc);
        first_layer_res<T>(res, feats, e, valid, kin, lay.kp, acc, lane);
#pragma unroll
        for (int j = 0; j < L; ++j) {
            if (j > 0) {
                zero(acc);
                mfma_layer_res<T, H / 16>(res + lay.fwd_off(j) / 4, fs + lay.fscale_off(j), act, acc, lane);
            }
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) act[t][r] = silu(acc[t][r] + bs[j * H + dfeat(t, r, half)]);
        }
        if (valid) {
            float* o = out + e * H;
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const f32x4 v = {act[t][4 * g], act[t][4 * g + 1], act[t][4 * g + 2], act[t][4 * g + 3]};
                    *reinterpret_cast<f32x4*>(o + 32 * t + 8 * g + 4 * half) = v;
                }
        }
    }
}

template <int H, int L, int KP>
__global__ void __launch_bounds__(kRadThreads) k_radial_bwd_res(const float* __restrict__ feats, int64_t E, int kin,
                                                                const float* __restrict__ frag, RadLayout lay,
                                                                const float* __restrict__ grad_h,
                                                                float* __restrict__ grad_feats) {
    constexpr int T = H / 32;
    __shared__ f32x4 res[rad_res_floats<H, L, true, KP>() / 4];
    stage(frag, int(lay.fscale_off(1)), res);  // both directions' fragments and the biases, as laid out in frag
    __syncthreads();
    const float* bias = reinterpret_cast<const float*>(res) + lay.bias_off();
    const int lane = threadIdx.x & 63, half = lane >> 5;
    const int64_t groups = (E + 31) / 32, stride = int64_t(gridDim.x) * (kRadThreads / 64);
    for (int64_t grp = int64_t(blockIdx.x) * (kRadThreads / 64) + (threadIdx.x >> 6); grp < groups; grp += stride) {
        const int64_t e = grp * 32 + (lane & 31);
        const bool valid = e < E;
        const int z0 = opaque_zero();
        const float* bs = bias + z0;
        const float* fs = frag + z0;
        float z[L > 1 ? L - 1 : 1][T][16];
        float g[T][16];
        f32x16 acc[T];
        zero(acc);
        first_layer_res<T>(res, feats, e, valid, kin, lay.kp, acc, lane);
#pragma unroll
        for (int j = 0; j < L; ++j) {
            if (j > 0) {
                zero(acc);
                mfma_layer_res<T, H / 16>(res + lay.fwd_off(j) / 4, fs + lay.fscale_off(j), g, acc, lane);
            }
            if (j < L - 1) {
#pragma unroll
                for (int t = 0; t < T; ++t)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        z[j][t][r] = acc[t][r] + bs[j * H + dfeat(t, r, half)];
                        g[t][r] = silu(z[j][t][r]);
                    }
            }
        }
        // g = dL/dh * silu'(z_{L-1}), dL/dh read in the D layout
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f32x4 v = valid ? *reinterpret_cast<const f32x4*>(grad_h + e * H + 32 * t + 8 * q + 4 * half)
                                      : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = 4 * q + i;
                    g[t][r] = v[i] * silu_grad(acc[t][r] + bs[(L - 1) * H + dfeat(t, r, half)]);
                }
            }
#pragma unroll
        for (int j = L - 1; j >= 1; --j) {
            zero(acc);
            mfma_layer_res<T, H / 16>(res + lay.bwd_off(j) / 4, fs + lay.bscale_off(j), g, acc, lane);
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) g[t][r] = acc[t][r] * silu_grad(z[j - 1][t][r]);
        }
        constexpr int T0 = (KP + 31) / 32;  // dL/df^T row tiles (the launch matches them to kp)
        f32x16 a0[T0];
        zero(a0);
        mfma_layer_res<T0, H / 16>(res + lay.bwd_off(0) / 4, fs + lay.bscale_off(0), g, a0, lane);
        store_grad_feats(a0, grad_feats, e, valid, kin, half);
    }
}

// Workgroups of a resident kernel: as many as fit the device at once.
template <class K>
int resident_grid(K kernel, int64_t E) {
    const int64_t need = ceil_div(ceil_div(E, 32), kRadThreads / 64);
    return int(device_fill_grid(reinterpret_cast<const void*>(kernel), kRadThreads, need));
}

RadLayout make_layout(int kin, int H, int L) { return RadLayout{kin, (kin + 7) & ~7, H, L}; }

int check_shape(int kin, int H, int L) {
    MNX_REQUIRE(kin > 0 && kin <= kRadMaxIn, "radial MLP input width %d not in [1, %d]", kin, kRadMaxIn);
    const bool ok = ((H == 32 || H == 64) && L >= 1 && L <= 4) || (H == 128 && L >= 1 && L <= 2);
    if (!ok)
        return set_error(MNX_ERR_UNSUPPORTED,
                         "radial MLP hidden stack %d x %d not compiled (32 or 64 wide up to 4 layers, 128 up to 2)", H,
                         L);
    return MNX_OK;
}

template <int H, int L>
void launch_fwd(const float* feats, int64_t E, int kin, const float* frag, RadLayout lay, float* out, hipStream_t s) {
    // resident only at 128 wide: narrower forwards are VALU-bound (SiLU) and run slightly
    // faster per-layer staged, with more workgroups in flight
    const int grid = H == 128 && lay.kp <= kRadResKp ? resident_grid(k_radial_fwd_res<H, L>, E) : 0;
    if (grid > 0)
        hipLaunchKernelGGL((k_radial_fwd_res<H, L>), dim3(grid), dim3(kRadThreads), 0, s, feats, E, kin, frag, lay,
                           out);
    else
        hipLaunchKernelGGL((k_radial_fwd<H, L>), dim3(ceil_div(E, kRadEdgesPerBlock)), dim3(kRadThreads), 0, s, feats,
                           E, kin, frag, lay, out);
}

template <int H, int L>
void launch_bwd(const float* feats, int64_t E, int kin, const float* frag, RadLayout lay, const float* gh, float* gf,
                hipStream_t s) {
    // resident up to 16 inputs (one input-gradient tile), and for stacks up to 64 wide from 40 to 64
    // inputs (two tiles: the LDS copy stays within ~130 KB)
    const bool wide = H <= 64 && lay.kp > 32 && lay.kp <= 64;
    const int grid = lay.kp <= kRadResKp ? resident_grid(k_radial_bwd_res<H, L, kRadResKp>, E)
                     : wide             ? resident_grid(k_radial_bwd_res<H, L, (H <= 64 ? 64 : kRadResKp)>, E)
                                        : 0;
    if (grid > 0 && !wide)
        hipLaunchKernelGGL((k_radial_bwd_res<H, L, kRadResKp>), dim3(grid), dim3(kRadThreads), 0, s, feats, E, kin,
                           frag, lay, gh, gf);
    else if (grid > 0)
        hipLaunchKernelGGL((k_radial_bwd_res<H, L, (H <= 64 ? 64 : kRadResKp)>), dim3(grid), dim3(kRadThreads), 0, s,
                           feats, E, kin, frag, lay, gh, gf);
    else
        hipLaunchKernelGGL((k_radial_bwd<H, L>), dim3(ceil_div(E, kRadEdgesPerBlock)), dim3(kRadThreads), 0, s, feats,
                           E, kin, frag, lay, gh, gf);
}

#define MNX_RAD_DISPATCH(FN, ...)                                     \
    switch (H * 8 + L) {                                              \
        case 32 * 8 + 1: FN<32, 1>(__VA_ARGS__); break;               \
        case 32 * 8 + 2: FN<32, 2>(__VA_ARGS__); break;               \
        case 32 * 8 + 3: FN<32, 3>(__VA_ARGS__); break;               \
        case 32 * 8 + 4: FN<32, 4>(__VA_ARGS__); break;               \
        case 64 * 8 + 1: FN<64, 1>(__VA_ARGS__); break;               \
        case 64 * 8 + 2: FN<64, 2>(__VA_ARGS__); break;               \
        case 64 * 8 + 3: FN<64, 3>(__VA_ARGS__); break;               \
        case 64 * 8 + 4: FN<64, 4>(__VA_ARGS__); break;               \
        case 128 * 8 + 1: FN<128, 1>(__VA_ARGS__); break;             \
        default: FN<128, 2>(__VA_ARGS__); break;                      \
    }

// Second derivative of the hidden layers' SiLU (training with a force loss): with
// s(x) = x sigma(x), s' = sigma (1 + x (1 - sigma)), s'' = sigma (1 - sigma) (2 + x (1 - 2 sigma)),
// the first-order product gx = g s'(x) has the adjoints dx = gg g s''(x) and dg = gg s'(x): one pass
// over x, g, gg (four values per lane when the sizes allow 16-byte access).
// 1 - sigma(x) is evaluated as sigma(-x), not by subtraction, which would cancel for x >> 0.
__device__ __forceinline__ void silu_bwd2_one(float x, float g, float gg, float& dx, float& dg) {
    const float sg = 1.f / (1.f + expf(-x));
    const float om = 1.f / (1.f + expf(x));
    dg = gg * (sg * fmaf(x, om, 1.f));
    dx = gg * g * (sg * om * fmaf(x, om - sg, 2.f));
}

// VEC: 16-byte loads and stores (every pointer 16-byte aligned); otherwise four scalar elements
// per thread (views at an offset that is not a multiple of four floats)
template <bool VEC>
__global__ void __launch_bounds__(256) k_silu_bwd2(const float* __restrict__ x, const float* __restrict__ g,
                                                   const float* __restrict__ gg, int64_t n, float* __restrict__ dx,
                                                   float* __restrict__ dg) {
    const int64_t i4 = (int64_t(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (VEC && i4 + 4 <= n) {
        const float4 a = *reinterpret_cast<const float4*>(x + i4);
        const float4 b = *reinterpret_cast<const float4*>(g + i4);
        const float4 c = *reinterpret_cast<const float4*>(gg + i4);
        float4 ox, og;
        silu_bwd2_one(a.x, b.x, c.x, ox.x, og.x);
        silu_bwd2_one(a.y, b.y, c.y, ox.y, og.y);
        silu_bwd2_one(a.z, b.z, c.z, ox.z, og.z);
        silu_bwd2_one(a.w, b.w, c.w, ox.w, og.w);
        *reinterpret_cast<float4*>(dx + i4) = ox;
        *reinterpret_cast<float4*>(dg + i4) = og;
    } else {
        const int64_t end = i4 + 4 < n ? i4 + 4 : n;
        for (int64_t i = i4; i < end; ++i) silu_bwd2_one(x[i], g[i], gg[i], dx[i], dg[i]);
    }
}

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

int64_t mnx_radial_raw_floats(int32_t kin, int32_t hidden, int32_t layers) {
    if (check_shape(kin, hidden, layers)) return -1;
    return make_layout(kin, hidden, layers).raw_total();
}

int64_t mnx_radial_frag_floats(int32_t kin, int32_t hidden, int32_t layers) {
    if (check_shape(kin, hidden, layers)) return -1;
    return make_layout(kin, hidden, layers).total();
}

int mnx_radial_pack_f32(const float* raw, int32_t kin, int32_t hidden, int32_t layers, float* frag,
                        mnx_stream_t stream) {
    clear_error();
    int rc = check_shape(kin, hidden, layers);
    if (rc) return rc;
    MNX_REQUIRE(raw && frag, "null pointer argument");
    MNX_REQUIRE((uintptr_t)frag % 16 == 0, "frag must be 16-byte aligned");
    const RadLayout lay = make_layout(kin, hidden, layers);
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(k_radial_scales, dim3(ceil_div(lay.scales_total(), 4)), dim3(256), 0, s, raw, lay, frag);
    MNX_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_radial_pack, dim3(ceil_div(lay.fscale_off(1), 256)), dim3(256), 0, s, raw, lay, frag);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_radial_fwd_f32(const float* feats, int64_t num_edges, int32_t kin, int32_t hidden, int32_t layers,
                       const float* frag, float* out, mnx_stream_t stream) {
    clear_error();
    int rc = check_shape(kin, hidden, layers);
    if (rc) return rc;
    MNX_REQUIRE(num_edges >= 0 && num_edges < (int64_t(1) << 36), "edge count out of range");
    if (num_edges == 0) return MNX_OK;
    MNX_REQUIRE(feats && frag && out, "null pointer argument");
    MNX_REQUIRE(((uintptr_t)frag | (uintptr_t)out) % 16 == 0, "frag and out must be 16-byte aligned");
    const int H = hidden, L = layers;
    const RadLayout lay = make_layout(kin, H, L);
    MNX_RAD_DISPATCH(launch_fwd, feats, num_edges, kin, frag, lay, out, (hipStream_t)stream);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_radial_bwd_f32(const float* feats, int64_t num_edges, int32_t kin, int32_t hidden, int32_t layers,
                       const float* frag, const float* grad_h, float* grad_feats, mnx_stream_t stream) {
    clear_error();
    int rc = check_shape(kin, hidden, layers);
    if (rc) return rc;
    MNX_REQUIRE(num_edges >= 0 && num_edges < (int64_t(1) << 36), "edge count out of range");
    if (num_edges == 0) return MNX_OK;
    MNX_REQUIRE(feats && frag && grad_h && grad_feats, "null pointer argument");
    MNX_REQUIRE(((uintptr_t)frag | (uintptr_t)grad_h) % 16 == 0, "frag and grad_h must be 16-byte aligned");
    const int H = hidden, L = layers;
    const RadLayout lay = make_layout(kin, H, L);
    MNX_RAD_DISPATCH(launch_bwd, feats, num_edges, kin, frag, lay, grad_h, grad_feats, (hipStream_t)stream);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

int mnx_silu_bwd2_f32(const float* x, const float* grad, const float* grad_grad, int64_t n, float* grad_x,
                      float* grad_grad_out, mnx_stream_t stream_) {
    clear_error();
    hipStream_t stream = (hipStream_t)stream_;
    MNX_REQUIRE(n >= 0, "silu_bwd2: n out of range");
    if (n == 0) return MNX_OK;
    MNX_REQUIRE(x && grad && grad_grad && grad_x && grad_grad_out, "null pointer argument");
    bool aligned = true;
    for (const void* p : {(const void*)x, (const void*)grad, (const void*)grad_grad, (const void*)grad_x,
                          (const void*)grad_grad_out})
        aligned = aligned && reinterpret_cast<uintptr_t>(p) % 16 == 0;
    const unsigned blocks = unsigned(ceil_div(ceil_div(n, 4), 256));
    if (aligned)
        k_silu_bwd2<true><<<blocks, 256, 0, stream>>>(x, grad, grad_grad, n, grad_x, grad_grad_out);
    else
        k_silu_bwd2<false><<<blocks, 256, 0, stream>>>(x, grad, grad_grad, n, grad_x, grad_grad_out);
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

}  // extern "C"
