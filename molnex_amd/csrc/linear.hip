// Equivariant (ir_mul) block linear on MFMA: one output irrep block
//   out[n][off + i*N + p] = sum_k A[(n, i)][k] * W[k][p]
// where row (n, i) of A (node n, irrep component i < d) concatenates
// segments of the input rows: segment s contributes len_s values starting at
// a[n*stride + col_s + i*comp_s].  This is cuet.Linear / e3nn Linear in ir_mul
// layout (src/molrep/interaction/linear.py:43-105): for an output block
// mul_o x ir the segments are the input blocks of the same irrep and W their
// stacked (mul_in x mul_o) weights, scaled by 1/sqrt(fan_in).  The gradient
// with respect to an input block is the same product with the output-gradient
// blocks as segments and the transposed weights.
//
// Each wavefront owns 32 rows (M side of v_mfma_f32_32x32x16_bf16) and up to 128
// output columns (N side, NT tiles); A is read straight from the strided input
// (32 bytes per lane and k-step, no gather copy).  W arrives pre-arranged by the
// caller in MFMA fragment order, [column group][64-row chunk][k/16][tile][lane][8]
// (lane l holds W[16q + 8(l/32) + j][32t + l%32]) with zero padding
// (mnx_block_linear_frag_floats gives its size); each chunk is staged into LDS
// by the workgroup's eight wavefronts, split there into three bf16 planes.
//
// Arithmetic: fp32-accurate products on the bf16 matrix cores.  Each fp32
// operand x is split exactly into x0 = bf16(x), x1 = bf16(x - x0),
// x2 = bf16(x - x0 - x1); the six partial products x_i y_j with i + j <= 2 are
// accumulated in fp32, smallest first (the dropped terms are below 2^-25 |x y|),
// at 3/8 of the matrix-core cycles of fp32 MFMAs.  The D tiles are stored 128
// contiguous bytes per row.
//
// Indexed mode (cuet.Linear(weight_classes=S, method="indexed_linear"),
// src/molrep/interaction/element_update.py:101-109,147-158): every node has a
// class (element) and its own weight set.  The caller groups the nodes by class
// (`order`, ascending class, rows of an out-of-range class last) and passes the
// class boundaries; workgroup b finds its class from those boundaries (each
// class owns ceil(count * d / 256) consecutive workgroups), reads its rows
// through `order` and uses the weights of its class.  The out-of-range class
// writes zeros.  No host synchronisation: the grid is sized for the worst case
// (one partial workgroup per class) and surplus workgroups exit at once.

#include <algorithm>
#include <cstdlib>

#include "common.h"

namespace mnx {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void split3(float v, __bf16& b0, __bf16& b1, __bf16& b2) {
    b0 = (__bf16)v;
    float r = v - (float)b0;
    b1 = (__bf16)r;
    r -= (float)b1;
    b2 = (__bf16)r;
}

__device__ __forceinline__ f32x16 mfma_bf16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

constexpr int kLinThreads = 512;  // eight wavefronts x 32 rows
constexpr int kLinKC = 64;        // rows of W staged per pass
constexpr int kLinMaxSeg = 8;

struct LinSeg {
    int64_t col;  // column of component 0
    int32_t comp; // column step between components
    int32_t len;  // values contributed (multiple of 8)
    int32_t k0;   // first contraction index of the segment
};

struct LinArgs {
    const float* a;
    int64_t a_stride;
    int32_t nseg, K;
    LinSeg seg[kLinMaxSeg];
    const float* w;  // fragment-ordered weights
    int32_t N, d;
    int64_t R;
    float* out;
    int64_t out_stride, out_off;
    int32_t out_comp;
    // indexed mode
    const int32_t* order;        // [R] node ids grouped by class
    const int32_t* class_start;  // [S + 2] first position in order of classes 0..S (S = out of range)
    int32_t S;
    int64_t w_class_stride;      // floats between the weight sets of consecutive classes
};

constexpr int kLinRowsPerBlock = (kLinThreads / kWave) * 32;

// NT: output tiles of 32 columns per wavefront; D: components per row group when it
// is 1, 3, 5 or 7 (divisions by it become multiplies), 0 = read p.d.
template <int NT, int D, bool IDX>
__global__ void __launch_bounds__(kLinThreads) k_block_linear(LinArgs p) {
    constexpr int KQ = kLinKC / 16;  // bf16 k-steps per staged chunk
    const int d = D ? D : p.d;
    __shared__ bf16x8 sw[3][KQ][NT][kWave];
    const int lane = threadIdx.x & 63, half = lane >> 5, wave = threadIdx.x >> 6;
    int64_t row0, rows;
    int K = p.K;
    const float* wcls = p.w;
    if (IDX) {
        // this workgroup's class: classes 0..S (S = out of range, zeros) own consecutive runs of
        // ceil(count * d / rows per block) workgroups
        const int64_t b = blockIdx.x;
        int64_t first = 0;
        int cls = 0;
        for (; cls <= p.S; ++cls) {
            const int64_t cnt = int64_t(p.class_start[cls + 1] - p.class_start[cls]) * d;
            const int64_t nb = (cnt + kLinRowsPerBlock - 1) / kLinRowsPerBlock;
            if (b < first + nb) break;
            first += nb;
        }
        if (cls > p.S) return;  // surplus workgroup (the grid is sized for the worst case)
        row0 = int64_t(p.class_start[cls]) * d + (b - first) * kLinRowsPerBlock + wave * 32;
        rows = int64_t(p.class_start[cls + 1]) * d;
        if (cls == p.S) K = 0;  // out-of-range class: zero output
        else wcls = p.w + int64_t(cls) * p.w_class_stride;
    } else {
        row0 = (int64_t(blockIdx.x) * (kLinThreads / kWave) + wave) * 32;
        rows = p.R * d;
    }
    const int64_t row = row0 + (lane & 31);
    const bool valid = row < rows;
    // (node, component) of row0 once; rows within the tile follow in 32-bit arithmetic
    const int64_t n0 = row0 / d;
    const int c0 = int(row0 - n0 * d);
    const int64_t n = n0 + (c0 + (lane & 31)) / d;
    const int ci = (c0 + (lane & 31)) % d;
    const int64_t node = IDX ? (valid ? int64_t(p.order[n]) : 0) : n;
    const float* arow = p.a + node * p.a_stride;
    const int col0 = blockIdx.y * NT * 32;
    f32x16 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
    constexpr int kChunk4 = KQ * NT * kWave * 2;  // fp32 float4s per staged chunk
    const int nchunks = (p.K + kLinKC - 1) / kLinKC;
    const f32x4* wsrc = reinterpret_cast<const f32x4*>(wcls) + int64_t(blockIdx.y) * nchunks * kChunk4;
    bf16x4* sw4 = reinterpret_cast<bf16x4*>(&sw[0][0][0][0]);
    // per segment, this lane's offset of contraction index k is base[s] + k (row-relative)
    int32_t base[kLinMaxSeg];
#pragma unroll
    for (int sg = 0; sg < kLinMaxSeg; ++sg)
        base[sg] = sg < p.nseg ? int32_t(p.seg[sg].col + int64_t(ci) * p.seg[sg].comp - p.seg[sg].k0) : 0;
    for (int k0 = 0; k0 < K; k0 += kLinKC) {
        // this chunk's A operands first (8 consecutive values per lane and k-step): their
        // latency overlaps the weight staging below
        f32x4 av[KQ][2];
#pragma unroll
        for (int q = 0; q < KQ; ++q) {
            const int k = k0 + 16 * q + 8 * half;
            int32_t off = 0;
#pragma unroll
            for (int sg = 0; sg < kLinMaxSeg; ++sg)
                if (sg < p.nseg && k >= p.seg[sg].k0) off = base[sg];
            av[q][0] = av[q][1] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (valid && k < p.K) {
                av[q][0] = *reinterpret_cast<const f32x4*>(arow + off + k);
                av[q][1] = *reinterpret_cast<const f32x4*>(arow + off + k + 4);
            }
        }
        __syncthreads();
        // stage and split the chunk: fp32 float4 idx = ((q * NT + t) * 64 + lane) * 2 + h holds
        // elements 4h..4h+3 of lane `lane`'s fragment; plane p goes to sw[p][q][t][lane]
        for (int idx = threadIdx.x; idx < kChunk4; idx += kLinThreads) {
            const f32x4 v = wsrc[idx];
            bf16x4 b0, b1, b2;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                __bf16 x0, x1, x2;
                split3(v[i], x0, x1, x2);
                b0[i] = x0;
                b1[i] = x1;
                b2[i] = x2;
            }
            sw4[idx] = b0;
            sw4[kChunk4 + idx] = b1;
            sw4[2 * kChunk4 + idx] = b2;
        }
        wsrc += kChunk4;
        __syncthreads();
        const int nq = (min(kLinKC, p.K - k0) + 15) / 16;
#pragma unroll
        for (int q = 0; q < KQ; ++q) {
            if (q < nq) {
                bf16x8 a0, a1, a2;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    __bf16 x0, x1, x2;
                    split3(j < 4 ? av[q][0][j] : av[q][1][j - 4], x0, x1, x2);
                    a0[j] = x0;
                    a1[j] = x1;
                    a2[j] = x2;
                }
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = mfma_bf16(a2, sw[0][q][t][lane], acc[t]);
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = mfma_bf16(a1, sw[1][q][t][lane], acc[t]);
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = mfma_bf16(a0, sw[2][q][t][lane], acc[t]);
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = mfma_bf16(a1, sw[0][q][t][lane], acc[t]);
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = mfma_bf16(a0, sw[1][q][t][lane], acc[t]);
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = mfma_bf16(a0, sw[0][q][t][lane], acc[t]);
            }
        }
    }
    // output row offsets of this lane's 16 accumulator registers
    int64_t obase[16];
    bool oval[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int o = 8 * (r / 4) + 4 * half + r % 4;
        const int64_t nn = n0 + (c0 + o) / d;
        const int ii = (c0 + o) % d;
        oval[r] = row0 + o < rows;
        const int64_t on = IDX ? (oval[r] ? int64_t(p.order[nn]) : 0) : nn;
        obase[r] = on * p.out_stride + p.out_off + int64_t(ii) * p.out_comp;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int c = col0 + 32 * t + (lane & 31);
        if (c >= p.N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (oval[r]) p.out[obase[r] + c] = acc[t][r];
    }
}

// Resident form for K <= 128 (plain mode): a workgroup stages its column group's whole weight
// block once, split into the three bf16 planes (at most 96 KB of LDS), then each wavefront walks
// row tiles (tile = blockIdx.x * 8 + wave, stepping by the grid) without further barriers.  The
// next tile's A operands are loaded k-step by k-step as soon as the current tile's k-step has been
// split, so their latency runs under the current tile's matrix-core products.
constexpr int kLinResMaxK = 128;

template <int NT, int D>
__global__ void __launch_bounds__(kLinThreads) k_block_linear_res(LinArgs p) {
    constexpr int KQ = kLinResMaxK / 16;
    const int d = D ? D : p.d;
    __shared__ bf16x8 sw[3][KQ][NT][kWave];
    const int lane = threadIdx.x & 63, half = lane >> 5, wave = threadIdx.x >> 6;
    const int nq = (p.K + 15) / 16;
    const int col0 = blockIdx.y * NT * 32;
    {
        // fp32 float4 idx = ((q * NT + t) * 64 + lane) * 2 + h of the column group's fragment
        const int nchunks = (p.K + kLinKC - 1) / kLinKC;
        const int n4 = nq * NT * kWave * 2;
        const f32x4* wsrc = reinterpret_cast<const f32x4*>(p.w) + int64_t(blockIdx.y) * nchunks * (kLinKC / 16) * NT * kWave * 2;
        bf16x4* sw4 = reinterpret_cast<bf16x4*>(&sw[0][0][0][0]);
        constexpr int kPlane4 = KQ * NT * kWave * 2;  // bf16x4 per plane
        for (int idx = threadIdx.x; idx < n4; idx += kLinThreads) {
            const f32x4 v = wsrc[idx];
            bf16x4 b0, b1, b2;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                __bf16 x0, x1, x2;
                split3(v[i], x0, x1, x2);
                b0[i] = x0;
                b1[i] = x1;
                b2[i] = x2;
            }
            sw4[idx] = b0;
            sw4[kPlane4 + idx] = b1;
            sw4[2 * kPlane4 + idx] = b2;
        }
        __syncthreads();
    }
    const int64_t rows = p.R * d;
    const int64_t ntiles = (rows + 31) / 32;
    const int64_t tstep = int64_t(gridDim.x) * (kLinThreads / kWave);
    int32_t base[kLinMaxSeg];
    // A operands of row tile `tile`: row pointer and per-segment offsets of this lane's row
    auto locate = [&](int64_t tile, const float*& arow, bool& valid) {
        const int64_t row0 = tile * 32;
        const int64_t n0 = row0 / d;
        const int c0 = int(row0 - n0 * d);
        const int64_t n = n0 + (c0 + (lane & 31)) / d;
        const int ci = (c0 + (lane & 31)) % d;
        valid = row0 + (lane & 31) < rows;
        arow = p.a + n * p.a_stride;
#pragma unroll
        for (int sg = 0; sg < kLinMaxSeg; ++sg)
            base[sg] = sg < p.nseg ? int32_t(p.seg[sg].col + int64_t(ci) * p.seg[sg].comp - p.seg[sg].k0) : 0;
    };
    auto load_q = [&](const float* arow, bool valid, int q, f32x4 (&dst)[2]) {
        const int k = 16 * q + 8 * half;
        int32_t off = 0;
#pragma unroll
        for (int sg = 0; sg < kLinMaxSeg; ++sg)
            if (sg < p.nseg && k >= p.seg[sg].k0) off = base[sg];
        dst[0] = dst[1] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (valid && k < p.K) {
            dst[0] = *reinterpret_cast<const f32x4*>(arow + off + k);
            dst[1] = *reinterpret_cast<const f32x4*>(arow + off + k + 4);
        }
    };
    int64_t tile = int64_t(blockIdx.x) * (kLinThreads / kWave) + wave;
    if (tile >= ntiles) return;  // no barrier after this point
    f32x4 av[KQ][2];
    const float* arow;
    bool valid;
    locate(tile, arow, valid);
#pragma unroll
    for (int q = 0; q < KQ; ++q)
        if (q < nq) load_q(arow, valid, q, av[q]);
    for (; tile < ntiles; tile += tstep) {
        const int64_t row0 = tile * 32;
        const int64_t n0 = row0 / d;
        const int c0 = int(row0 - n0 * d);
        const int64_t next = tile + tstep;
        const bool more = next < ntiles;
        const float* arow_n = arow;
        bool valid_n = false;
        if (more) locate(next, arow_n, valid_n);
        f32x16 acc[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
#pragma unroll
        for (int q = 0; q < KQ; ++q) {
            if (q < nq) {
                bf16x8 a0, a1, a2;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    __bf16 x0, x1, x2;
                    split3(j < 4 ? av[q][0][j] : av[q][1][j - 4], x0, x1, x2);
                    a0[j] = x0;
                    a1[j] = x1;
                    a2[j] = x2;
                }
                if (more) load_q(arow_n, valid_n, q, av[q]);
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = mfma_bf16(a2, sw[0][q][t][lane], acc[t]);
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = mfma_bf16(a1, sw[1][q][t][lane], acc[t]);
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = mfma_bf16(a0, sw[2][q][t][lane], acc[t]);
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = mfma_bf16(a1, sw[0][q][t][lane], acc[t]);
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = mfma_bf16(a0, sw[1][q][t][lane], acc[t]);
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = mfma_bf16(a0, sw[0][q][t][lane], acc[t]);
            }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int o = 8 * (r / 4) + 4 * half + r % 4;
            if (row0 + o >= rows) continue;
            const int64_t nn = n0 + (c0 + o) / d;
            const int ii = (c0 + o) % d;
            float* ob = p.out + nn * p.out_stride + p.out_off + int64_t(ii) * p.out_comp;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int c = col0 + 32 * t + (lane & 31);
                if (c < p.N) ob[c] = acc[t][r];
            }
        }
        arow = arow_n;
        valid = valid_n;
    }
}

template <int NT>
void launch_res(int d, dim3 grid, hipStream_t s, const LinArgs& p) {
    switch (d) {
        case 1: hipLaunchKernelGGL((k_block_linear_res<NT, 1>), grid, dim3(kLinThreads), 0, s, p); break;
        case 3: hipLaunchKernelGGL((k_block_linear_res<NT, 3>), grid, dim3(kLinThreads), 0, s, p); break;
        case 5: hipLaunchKernelGGL((k_block_linear_res<NT, 5>), grid, dim3(kLinThreads), 0, s, p); break;
        case 7: hipLaunchKernelGGL((k_block_linear_res<NT, 7>), grid, dim3(kLinThreads), 0, s, p); break;
        default: hipLaunchKernelGGL((k_block_linear_res<NT, 0>), grid, dim3(kLinThreads), 0, s, p); break;
    }
}

// output tiles of 32 columns per wavefront for N columns (the column-group width is 32 * this)
int lin_tiles(int N) { return N >= 128 ? 4 : int(ceil_div(N, 32)); }

template <int NT, bool IDX>
void launch_nt(int d, dim3 grid, hipStream_t s, const LinArgs& p) {
    switch (d) {
        case 1: hipLaunchKernelGGL((k_block_linear<NT, 1, IDX>), grid, dim3(kLinThreads), 0, s, p); break;
        case 3: hipLaunchKernelGGL((k_block_linear<NT, 3, IDX>), grid, dim3(kLinThreads), 0, s, p); break;
        case 5: hipLaunchKernelGGL((k_block_linear<NT, 5, IDX>), grid, dim3(kLinThreads), 0, s, p); break;
        case 7: hipLaunchKernelGGL((k_block_linear<NT, 7, IDX>), grid, dim3(kLinThreads), 0, s, p); break;
        default: hipLaunchKernelGGL((k_block_linear<NT, 0, IDX>), grid, dim3(kLinThreads), 0, s, p); break;
    }
}

// the resident form unless the environment sets MNX_LIN_RESIDENT=0 (to compare with the chunked
// kernel; both give bit-identical results)
bool lin_resident() {
    static const bool on = [] {
        const char* e = std::getenv("MNX_LIN_RESIDENT");
        return !(e && e[0] == '0');
    }();
    return on;
}

// shared argument checks and launch of both entry points
int block_linear(const float* a, int64_t a_stride, int32_t nseg, const int64_t* seg_col, const int32_t* seg_comp,
                 const int32_t* seg_len, const float* w, int32_t N, int64_t R, int32_t d, float* out,
                 int64_t out_stride, int64_t out_off, int32_t out_comp, const int32_t* order,
                 const int32_t* class_start, int32_t S, int64_t w_class_stride, hipStream_t stream) {
    MNX_REQUIRE(nseg >= 0 && nseg <= kLinMaxSeg, "segment count %d not in [0, %d]", nseg, kLinMaxSeg);
    MNX_REQUIRE(R >= 0 && d >= 1 && N >= 1 && R * d < (int64_t(1) << 40), "sizes out of range");
    if (R == 0) return MNX_OK;
    MNX_REQUIRE(out && (nseg == 0 || (a && w && seg_col && seg_comp && seg_len)), "null pointer argument");
    const bool idx = order != nullptr;
    MNX_REQUIRE(!idx || (class_start && S >= 1 && S <= 4096 && w_class_stride >= 0 && w_class_stride % 4 == 0),
                "indexed linear: bad class arguments");
    LinArgs p{};
    p.a = a;
    p.a_stride = a_stride;
    p.nseg = nseg;
    p.K = 0;
    for (int s = 0; s < nseg; ++s) {
        MNX_REQUIRE(seg_len[s] > 0 && seg_len[s] % 8 == 0 && seg_comp[s] % 4 == 0 && seg_col[s] % 4 == 0,
                    "segment %d: length must be a positive multiple of 8, offsets multiples of 4", s);
        p.seg[s] = LinSeg{seg_col[s], seg_comp[s], seg_len[s], p.K};
        p.K += seg_len[s];
    }
    MNX_REQUIRE(nseg == 0 || (a_stride % 4 == 0 && (uintptr_t)a % 16 == 0), "input rows must be 16-byte aligned");
    for (int s = 0; s < nseg; ++s)
        MNX_REQUIRE(seg_col[s] + int64_t(d - 1) * seg_comp[s] + seg_len[s] < (int64_t(1) << 31),
                    "segment %d exceeds 2^31 columns", s);
    MNX_REQUIRE(nseg == 0 || (uintptr_t)w % 16 == 0, "weights must be 16-byte aligned");
    p.w = w;
    p.N = N;
    p.d = d;
    p.R = R;
    p.out = out;
    p.out_stride = out_stride;
    p.out_off = out_off;
    p.out_comp = out_comp;
    p.order = order;
    p.class_start = class_start;
    p.S = S;
    p.w_class_stride = w_class_stride;
    // indexed: every class (and the out-of-range one) may end in a partial workgroup
    const int64_t blocks = ceil_div(R * d, kLinRowsPerBlock) + (idx ? S + 1 : 0);
    MNX_REQUIRE(blocks < (int64_t(1) << 31), "too many rows");
    const int nt = lin_tiles(N);
    const dim3 grid(unsigned(blocks), unsigned(ceil_div(N, nt * 32)));
    if (!idx && p.K > 0 && p.K <= kLinResMaxK && nt >= 2 && lin_resident()) {
        // weights resident in LDS: one workgroup per CU walks row tiles.  Not for one column tile
        // (N <= 32): there each wavefront's single accumulator chain is latency-bound at the
        // resident grid's occupancy, and the chunked kernel's full grid is faster (Allegro's
        // 16-channel projection over 2.6 M edges x 5 components: 576 vs 690 us)
        const dim3 rgrid(unsigned(std::min<int64_t>(blocks, 256)), grid.y);
        switch (nt) {
            case 1: launch_res<1>(d, rgrid, stream, p); break;
            case 2: launch_res<2>(d, rgrid, stream, p); break;
            case 3: launch_res<3>(d, rgrid, stream, p); break;
            default: launch_res<4>(d, rgrid, stream, p); break;
        }
        MNX_CHECK_LAUNCH();
        return MNX_OK;
    }
    if (idx) {
        switch (nt) {
            case 1: launch_nt<1, true>(d, grid, stream, p); break;
            case 2: launch_nt<2, true>(d, grid, stream, p); break;
            case 3: launch_nt<3, true>(d, grid, stream, p); break;
            default: launch_nt<4, true>(d, grid, stream, p); break;
        }
    } else {
        switch (nt) {
            case 1: launch_nt<1, false>(d, grid, stream, p); break;
            case 2: launch_nt<2, false>(d, grid, stream, p); break;
            case 3: launch_nt<3, false>(d, grid, stream, p); break;
            default: launch_nt<4, false>(d, grid, stream, p); break;
        }
    }
    MNX_CHECK_LAUNCH();
    return MNX_OK;
}

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

int64_t mnx_block_linear_frag_floats(int32_t K, int32_t N) {
    if (K < 0 || N < 1) return -1;
    const int nt = lin_tiles(N);
    return ceil_div(N, nt * 32) * ceil_div(K, kLinKC) * int64_t(kLinKC / 16) * nt * kWave * 8;
}

int mnx_block_linear_f32(const float* a, int64_t a_stride, int32_t nseg, const int64_t* seg_col,
                         const int32_t* seg_comp, const int32_t* seg_len, const float* w, int32_t N, int64_t R,
                         int32_t d, float* out, int64_t out_stride, int64_t out_off, int32_t out_comp,
                         mnx_stream_t stream) {
    clear_error();
    return block_linear(a, a_stride, nseg, seg_col, seg_comp, seg_len, w, N, R, d, out, out_stride, out_off,
                        out_comp, nullptr, nullptr, 0, 0, (hipStream_t)stream);
}

int mnx_indexed_block_linear_f32(const float* a, int64_t a_stride, int32_t nseg, const int64_t* seg_col,
                                 const int32_t* seg_comp, const int32_t* seg_len, const float* w,
                                 int64_t w_class_stride, int32_t num_classes, const int32_t* order,
                                 const int32_t* class_start, int32_t N, int64_t R, int32_t d, float* out,
                                 int64_t out_stride, int64_t out_off, int32_t out_comp, mnx_stream_t stream) {
    clear_error();
    MNX_REQUIRE(order && class_start, "indexed linear: order and class_start are required");
    return block_linear(a, a_stride, nseg, seg_col, seg_comp, seg_len, w, N, R, d, out, out_stride, out_off,
                        out_comp, order, class_start, num_classes, w_class_stride, (hipStream_t)stream);
}

}  // extern "C"
