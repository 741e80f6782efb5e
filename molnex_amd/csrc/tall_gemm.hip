// C = A^T B for tall operands: A [K][M] and B [K][N] with K (rows: edges or
// nodes) far larger than M and N.  These are the weight gradients of the
// per-edge layers when training, dW = grad^T h summed over every edge (the
// radial MLP's output layer, src/molrep/interaction/radial_mlp.py:76-82, and
// its second derivatives): 2.6 M rows of 1280 and 128 columns at config 5.
//
// Arithmetic: fp32-accurate products on the bf16 matrix cores, as in the block
// linear: each operand value v is split exactly into v0 = bf16(v),
// v1 = bf16(v - v0), v2 = bf16(v - v0 - v1) and the six partial products with
// i + j <= 2 are accumulated in fp32, smallest first
// (v_mfma_f32_32x32x16_bf16; the dropped terms are below 2^-25 |a b|).
//
// Tiling: a workgroup of eight wavefronts owns a 256 x 128 tile of C (wave
// tile 64 x 64, 2 x 2 MFMA tiles) over one slab of rows.  Per 16-row step each
// thread loads 8 rows of one A column (and, for half the threads, of one B
// column) through buffer descriptors (scalar row offsets: no per-load vector
// address arithmetic; 64 consecutive columns per wavefront instruction) two
// steps ahead, splits them once and stores the three planes to LDS in MFMA
// operand order (double-buffered, one barrier per step); the wavefronts read
// their operands from there, so each value is loaded and split once per
// workgroup.  Two workgroups fit a CU (at most 128 VGPRs and 72 KB of LDS
// each), so one's products run while the other waits at its barrier.  Each slab
// writes its partial tile to a workspace [slab][M][N]; a second kernel sums the
// slabs in a fixed order (deterministic, no atomics).  Optionally the loader
// threads also sum their A columns (compensated), giving A's column sums (a
// layer's bias gradient) from the same read.  Slabs are sized so that the grid
// holds about four workgroups per CU.

#include "common.h"

namespace mnx {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kTGThreads = 512;
constexpr int kTGBM = 256;
constexpr int kTGBN = 128;
constexpr int kTGTargetBlocks = 1024;

__device__ __forceinline__ void tg_split(const float (&v)[8], bf16x8& b0, bf16x8& b1, bf16x8& b2) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const __bf16 x0 = (__bf16)v[j];
        float r = v[j] - (float)x0;
        const __bf16 x1 = (__bf16)r;
        r -= (float)x1;
        b0[j] = x0;
        b1[j] = x1;
        b2[j] = (__bf16)r;
    }
}

__device__ __forceinline__ f32x16 tg_mfma(const bf16x8& a, const bf16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// One 16-byte LDS element per (plane, half step, column): the 8 bf16 values of rows
// 8 * half .. 8 * half + 7 of a 16-row step, i.e. one lane's MFMA operand.  Columns innermost, so
// that a wavefront's stores (64 consecutive columns) and loads (two runs of 32) are contiguous.
struct TGStage {
    bf16x8 a[3][2][kTGBM];
    bf16x8 b[3][2][kTGBN];
};

__global__ void __launch_bounds__(kTGThreads, 4) k_tall_tn(const float* __restrict__ A, int64_t lda,
                                                        const float* __restrict__ B, int64_t ldb, int64_t K,
                                                        int M, int N, int64_t kslab, int mtiles, int ntiles,
                                                        int64_t slabs, float* __restrict__ part,
                                                        float* __restrict__ cpart) {
    __shared__ TGStage stage[2];
    // XCD-aware order: workgroups are dealt round-robin over the 8 XCDs, so XCD x = b mod 8 takes
    // the contiguous item range starting at x * per, items ordered (slab, N tile, M tile): the M
    // tiles of one slab run together on one XCD and share that slab's B rows in its L2.
    const int64_t total = int64_t(mtiles) * ntiles * slabs;
    const int64_t per = (total + 7) / 8;
    const int64_t item = int64_t(blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (item >= total) return;
    const int tm = int(item % mtiles);
    const int tn = int((item / mtiles) % ntiles);
    const int64_t slab = item / (int64_t(mtiles) * ntiles);
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int half = lane >> 5, l32 = lane & 31;
    const int wm = wave & 3, wn = wave >> 2;
    const int64_t kb = slab * kslab;
    const int64_t ke = min(K, kb + kslab);

    // loader roles: every thread splits 8 rows of one A column, threads below 256 also 8 rows of
    // one B column (kh: which 8 rows of the step; wave-uniform)
    const int am = tid % kTGBM, akh = tid / kTGBM;
    const int bn = tid % kTGBN, bkh = (tid / kTGBN) & 1;
    const bool bload = tid < 2 * kTGBN;
    const int ga = tm * kTGBM + am, gb = tn * kTGBN + bn;
    const bool va = ga < M, vb = bload && gb < N;
    // full steps load through buffer descriptors: the step's base in the descriptor, the row
    // offset j * ld in a scalar register, the lane's offset (its 8-row half, its column; column 0
    // for columns outside the matrix, whose products are discarded) in one vector register.  Every
    // row read is below ke.  (The builtin returns the 32 bits as an integer: reinterpreted.)
    const int voa = int((8 * akh * lda + (va ? ga : 0)) * 4);
    const int vob = int((8 * bkh * ldb + (vb ? gb : 0)) * 4);
    auto load_full = [&](int64_t k, float (&av)[8], float (&bv)[8]) {
        const __amdgpu_buffer_rsrc_t ra =
            __builtin_amdgcn_make_buffer_rsrc((void*)(A + k * lda), (short)0, int(16 * lda * 4), 0x00020000);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            av[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ra, voa, int(j * lda * 4), 0));
        if (bload) {
            const __amdgpu_buffer_rsrc_t rb =
                __builtin_amdgcn_make_buffer_rsrc((void*)(B + k * ldb), (short)0, int(16 * ldb * 4), 0x00020000);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                bv[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, vob, int(j * ldb * 4), 0));
        }
    };
    // the last, partial step of a slab: rows at or beyond ke read as zero
    auto load_tail = [&](int64_t k, float (&av)[8], float (&bv)[8]) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int64_t ka = k + 8 * akh + j, kbb = k + 8 * bkh + j;
            av[j] = ka < ke && va ? A[ka * lda + ga] : 0.f;
            bv[j] = kbb < ke && vb ? B[kbb * ldb + gb] : 0.f;
        }
    };
    // column sums of A over this thread's rows (the bias gradient of the layer, when asked for):
    // compensated, so that the long per-thread chain keeps fp32 accuracy
    float csum = 0.f, ccomp = 0.f;
    auto put = [&](TGStage& st, const float (&av)[8], const float (&bv)[8]) {
        if (cpart && tn == 0) {
            const float t = ((av[0] + av[1]) + (av[2] + av[3])) + ((av[4] + av[5]) + (av[6] + av[7]));
            const float yk = t - ccomp;
            const float nk = csum + yk;
            ccomp = (nk - csum) - yk;
            csum = nk;
        }
        bf16x8 x0, x1, x2;
        tg_split(av, x0, x1, x2);
        st.a[0][akh][am] = x0;
        st.a[1][akh][am] = x1;
        st.a[2][akh][am] = x2;
        if (bload) {
            tg_split(bv, x0, x1, x2);
            st.b[0][bkh][bn] = x0;
            st.b[1][bkh][bn] = x1;
            st.b[2][bkh][bn] = x2;
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[t][u][r] = 0.f;
    // the six partial products, each issued for the four independent accumulator tiles in turn
    // (consecutive MFMAs never wait on each other's result); grouped by A plane so that one A plane
    // is live at a time: a2 b0, a1 b1, a1 b0, a0 b2, a0 b1, a0 b0 (the 2^-16-sized terms ahead of the
    // 2^-8-sized ones except a0 b2, which follows a1 b0)
    auto products = [&](const TGStage& st) {
        bf16x8 b[3][2];
#pragma unroll
        for (int q = 0; q < 3; ++q)
#pragma unroll
            for (int u = 0; u < 2; ++u) b[q][u] = st.b[q][half][wn * 64 + 32 * u + l32];
        constexpr int PLANE[3] = {2, 1, 0};
        constexpr int NB[3] = {1, 2, 3};  // partner B planes per A plane: b0 | b1, b0 | b2, b1, b0
        constexpr int BP[3][3] = {{0, 0, 0}, {1, 0, 0}, {2, 1, 0}};
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            bf16x8 a[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) a[t] = st.a[PLANE[i]][half][wm * 64 + 32 * t + l32];
#pragma unroll
            for (int j = 0; j < NB[i]; ++j)
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int u = 0; u < 2; ++u) acc[t][u] = tg_mfma(a[t], b[BP[i][j]][u], acc[t][u]);
        }
    };

    // Pipeline over the slab's full steps: step s is split into stage[s & 1] one iteration ahead
    // of its products and loaded one iteration before that; one barrier per step.  The partial
    // last step (if any) follows on its own.
    const int64_t nfull = ke > kb ? (ke - kb) / 16 : 0;
    float av[8], bv[8];
    if (nfull > 0) {
        load_full(kb, av, bv);
        put(stage[0], av, bv);
        if (nfull > 1) load_full(kb + 16, av, bv);
    }
    __syncthreads();
    for (int64_t st = 0; st < nfull; ++st) {
        if (st + 1 < nfull) {
            put(stage[(st + 1) & 1], av, bv);
            if (st + 2 < nfull) load_full(kb + 16 * (st + 2), av, bv);
        }
        products(stage[st & 1]);
        __syncthreads();
    }
    if (kb + 16 * nfull < ke) {
        load_tail(kb + 16 * nfull, av, bv);
        put(stage[0], av, bv);
        __syncthreads();
        products(stage[0]);
    }

    if (cpart && tn == 0 && va) cpart[(slab * 2 + akh) * M + ga] = csum;
    // D tile layout: lane holds rows 8 (r / 4) + 4 half + r % 4 of column l32
    const int m0 = tm * kTGBM + wm * 64, n0 = tn * kTGBN + wn * 64;
    float* dst = part + slab * M * N;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int n = n0 + 32 * u + l32;
            if (n >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + 32 * t + 8 * (r / 4) + 4 * half + r % 4;
                if (m < M) dst[int64_t(m) * N + n] = acc[t][u][r];
            }
        }
}

// C[i] = sum_s part[s][i] (zeros when there are no slabs): eight partial sums over the slabs
// s = j mod 8, so that eight loads are in flight, combined pairwise; a fixed order (deterministic).
__global__ void __launch_bounds__(256) k_sum_slabs(const float* __restrict__ part, int64_t slabs, int64_t mn,
                                                   float* __restrict__ C) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= mn) return;
    float s[8] = {};
    int64_t z = 0;
    for (; z + 8 <= slabs; z += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = part[(z + j) * mn + i];
#pragma unroll
        for (int j = 0; j < 8; ++j) s[j] += v[j];
    }
    for (int j = 0; z < slabs; ++z, ++j) s[j] += part[z * mn + i];
    C[i] = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
}

struct TallPlan {
    int64_t slabs, kslab;
};

TallPlan tall_plan(int64_t K, int M, int N) {
    const int64_t tiles = ceil_div(M, kTGBM) * ceil_div(N, kTGBN);
    int64_t slabs = std::max<int64_t>(1, kTGTargetBlocks / std::max<int64_t>(tiles, 1));
    slabs = std::min<int64_t>(slabs, std::max<int64_t>(1, ceil_div(K, 512)));
    int64_t kslab = ceil_div(ceil_div(K, slabs), 16) * 16;
    if (kslab == 0) kslab = 16;
    return {ceil_div(K, kslab), kslab};
}

}  // namespace
}  // namespace mnx

using namespace mnx;

extern "C" {

size_t mnx_tall_tn_workspace_bytes(int64_t K, int32_t M, int32_t N) {
    if (K <= 0 || M <= 0 || N <= 0) return 0;
    const TallPlan p = tall_plan(K, M, N);
    return size_t(p.slabs) * (size_t(M) * size_t(N) + 2 * size_t(M)) * sizeof(float);
}

int mnx_tall_tn_f32(const float* A, int64_t lda, const float* B, int64_t ldb, int64_t K, int32_t M, int32_t N,
                    float* C, float* colsum_a, void* workspace, size_t workspace_bytes, mnx_stream_t stream_) {
    clear_error();
    hipStream_t stream = (hipStream_t)stream_;
    MNX_REQUIRE(K >= 0 && M >= 0 && N >= 0, "tall_tn: sizes out of range");
    if (M == 0 || N == 0) return MNX_OK;
    MNX_REQUIRE(C, "tall_tn: null output");
    const int64_t mn = int64_t(M) * N;
    if (K == 0) {
        k_sum_slabs<<<unsigned(ceil_div(mn, 256)), 256, 0, stream>>>(nullptr, 0, mn, C);
        MNX_CHECK_LAUNCH();
        if (colsum_a) {
            k_sum_slabs<<<unsigned(ceil_div(M, 256)), 256, 0, stream>>>(nullptr, 0, M, colsum_a);
            MNX_CHECK_LAUNCH();
        }
        return MNX_OK;
    }
    MNX_REQUIRE(A && B, "tall_tn: null input");
    MNX_REQUIRE(lda >= M && ldb >= N, "tall_tn: row strides (%lld, %lld) below the widths (%d, %d)",
                (long long)lda, (long long)ldb, M, N);
    // byte offsets of a 16-row step stay in 32 bits (buffer descriptors)
    MNX_REQUIRE(lda < (int64_t(1) << 25) && ldb < (int64_t(1) << 25), "tall_tn: row strides of 2^25 or more");
    const TallPlan p = tall_plan(K, M, N);
    const size_t need = size_t(p.slabs) * (size_t(mn) + 2 * size_t(M)) * sizeof(float);
    MNX_REQUIRE(workspace && workspace_bytes >= need, "tall_tn: workspace of %zu bytes, %zu needed",
                workspace_bytes, need);
    float* part = static_cast<float*>(workspace);
    const int mt = int(ceil_div(M, kTGBM)), nt = int(ceil_div(N, kTGBN));
    const int64_t blocks = 8 * ceil_div(int64_t(mt) * nt * p.slabs, 8);
    MNX_REQUIRE(blocks < (int64_t(1) << 31), "tall_tn: %lld workgroups", (long long)blocks);
    float* cpart = colsum_a ? part + size_t(p.slabs) * size_t(mn) : nullptr;
    k_tall_tn<<<unsigned(blocks), kTGThreads, 0, stream>>>(A, lda, B, ldb, K, M, N, p.kslab, mt, nt, p.slabs,
                                                            part, cpart);
    MNX_CHECK_LAUNCH();
    k_sum_slabs<<<unsigned(ceil_div(mn, 256)), 256, 0, stream>>>(part, p.slabs, mn, C);
    MNX_CHECK_LAUNCH();
    if (colsum_a) {
        k_sum_slabs<<<unsigned(ceil_div(M, 256)), 256, 0, stream>>>(cpart, 2 * p.slabs, M, colsum_a);
        MNX_CHECK_LAUNCH();
    }
    return MNX_OK;
}

}  // extern "C"
