// Host side of the f32 GEMM core: tile-shape planning, split-K scratch and
// the C-ABI entry points nrs_gemm / nrs_gemm_nt_splitk / nrs_bmm. The kernels
// are in gemm_kernel.hpp.
#include <algorithm>

#include "gemm_kernel.hpp"

namespace nrs {

// ------------------------------------------------------------------ host side

namespace {

using KernelFn = void (*)(GemmArgs);

struct TileShape {
    int bm, bn, bk, threads;
};

template <int BM, int BN, int BK, int WM_, int WN_, int PF, bool AK, bool BKC>
KernelFn pick_vec(bool vec4) {
    return vec4 ? gemm_kernel<BM, BN, BK, WM_, WN_, AK, BKC, 4, 2, PF>
                : gemm_kernel<BM, BN, BK, WM_, WN_, AK, BKC, 1, 2, PF>;
}

template <int BM, int BN, int BK, int WM_, int WN_, int PF>
KernelFn pick_layout(int layout, bool vec4) {
    switch (layout) {
        case NRS_NN: return pick_vec<BM, BN, BK, WM_, WN_, PF, true, false>(vec4);
        case NRS_NT: return pick_vec<BM, BN, BK, WM_, WN_, PF, true, true>(vec4);
        default: return pick_vec<BM, BN, BK, WM_, WN_, PF, false, false>(vec4);
    }
}

// Tile configurations (chosen by a sweep over the workload shapes on MI355X).
// All run two waves per SIMD (register budget capped at 256 per lane,
// accumulators in VGPRs):
//  * 256x256x32, 8 waves of 128x64, ~140 KB LDS, prefetch depth 1: large
//    GEMMs (83-85% of FP32 MFMA peak at 4096^3 and 8192^3);
//  * 64x64x32, 4 waves of 32x32, prefetch depth 2: everything mid-sized
//    (bmm items, conv GEMMs, projections, split-K weight gradients);
//  * 32x256x32, 4 waves of 32x64: outputs with at most 32 rows.
enum TileId { T256x256 = 0, T64x64, T32x256, T_COUNT };
const TileShape kShapes[T_COUNT] = {
    {256, 256, 32, 512},
    {64, 64, 32, 256},
    {32, 256, 32, 256},
};

KernelFn kernel_for(int tile, int layout, bool vec4) {
    switch (tile) {
        case T256x256: return pick_layout<256, 256, 32, 2, 4, 1>(layout, vec4);
        case T64x64: return pick_layout<64, 64, 32, 2, 2, 2>(layout, vec4);
        default: return pick_layout<32, 256, 32, 1, 4, 1>(layout, vec4);
    }
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

struct Plan {
    int tile;
    int slices;
    int64_t k_per_slice;
};

// Chooses the tile shape and the number of K slices. The 256x256 tile is
// used only with 128-bit loads (its scalar-load variant spills).
Plan plan_gemm(int64_t M, int64_t N, int64_t K, int64_t batch, bool vec4, bool allow_split,
               int force_slices) {
    const int cus = num_cus();
    auto tiles_of = [&](int t) {
        return cdiv(M, kShapes[t].bm) * cdiv(N, kShapes[t].bn) * batch;
    };
    Plan pl{T64x64, 1, K};
    if (M <= 32 && N >= 256)
        pl.tile = T32x256;
    else if (vec4 && tiles_of(T256x256) >= cus)
        pl.tile = T256x256;
    const TileShape& s = kShapes[pl.tile];
    const int64_t tiles = tiles_of(pl.tile);
    int slices = 1;
    if (force_slices > 0) {
        slices = force_slices;
    } else if (allow_split && batch == 1 && tiles < cus && (2 * tiles <= cus || K >= 2048)) {
        // About three workgroups per CU, each slice at least two k-tiles.
        const int64_t want = cdiv(3 * (int64_t)cus, tiles);
        const int64_t max_by_k = std::max<int64_t>(1, K / (2 * s.bk));
        slices = (int)std::min<int64_t>(want, max_by_k);
    }
    if (slices < 1) slices = 1;
    int64_t kps = cdiv(cdiv(K, slices), s.bk) * s.bk;
    if (kps <= 0) kps = s.bk;
    slices = (int)std::max<int64_t>(1, cdiv(K, kps));
    pl.slices = slices;
    pl.k_per_slice = kps;
    return pl;
}

}  // namespace

// Shared launcher: C[b] = epi(op(A[b]) op(B[b])) + beta*C[b] for b < batch.
int gemm_launch(int layout, float* C, const float* A, const float* B, int64_t M, int64_t N,
                int64_t K, int64_t batch, int64_t sA, int64_t sB, int64_t sC, float beta,
                const float* bias, int epi, int64_t nchw_P, bool allow_split, int force_slices) {
    NRS_ARG_CHECK(layout >= NRS_NN && layout <= NRS_TN, "gemm: unknown layout %d", layout);
    NRS_ARG_CHECK(M >= 0 && N >= 0 && K >= 0 && batch >= 0, "gemm: negative size");
    if (M == 0 || N == 0 || batch == 0) return NRS_OK;
    NRS_ARG_CHECK(C != nullptr, "gemm: null C");
    NRS_ARG_CHECK(K == 0 || (A != nullptr && B != nullptr), "gemm: null operand");
    NRS_ARG_CHECK(!(epi & (NRS_EPI_BIAS_COL | NRS_EPI_BIAS_ROW)) || bias != nullptr,
                  "gemm: bias epilogue with null bias");
    NRS_ARG_CHECK(M <= INT32_MAX && N <= INT32_MAX, "gemm: dimension too large");

    const int64_t lda = (layout == NRS_TN) ? M : K;
    const int64_t ldb = (layout == NRS_NT) ? K : N;

    // 128-bit loads need 16-byte aligned rows of both operands (k-slices
    // are multiples of BK, hence of 4).
    bool vec4 = aligned16(A) && aligned16(B) && (lda % 4 == 0) && (ldb % 4 == 0) &&
                (sA % 4 == 0 || batch == 1) && (sB % 4 == 0 || batch == 1);
    // Bounds are checked per vector: the guarded dimension must be a multiple of 4.
    if (layout == NRS_NN) vec4 = vec4 && (K % 4 == 0) && (N % 4 == 0);
    if (layout == NRS_NT) vec4 = vec4 && (K % 4 == 0);
    if (layout == NRS_TN) vec4 = vec4 && (M % 4 == 0) && (N % 4 == 0);

    Plan pl = plan_gemm(M, N, K, batch, vec4, allow_split && nchw_P == 0, force_slices);
    const TileShape& s = kShapes[pl.tile];

    GemmArgs p{};
    p.A = A;
    p.B = B;
    p.C = C;
    p.bias = bias;
    p.M = M;
    p.N = N;
    p.K = K;
    p.lda = lda;
    p.ldb = ldb;
    p.ldc = N;
    p.sA = sA;
    p.sB = sB;
    p.sC = sC;
    p.tiles_m = (int)cdiv(M, s.bm);
    p.tiles_n = (int)cdiv(N, s.bn);
    p.group_m = 8;
    p.beta = beta;
    p.epi = epi;
    p.nchw_P = nchw_P;
    p.k_per_slice = pl.k_per_slice;
    NRS_ARG_CHECK((int64_t)p.tiles_m * p.tiles_n <= INT32_MAX && batch <= 65535,
                  "gemm: grid too large");

    KernelFn fn = kernel_for(pl.tile, layout, vec4);
    dim3 grid((unsigned)(p.tiles_m * p.tiles_n), (unsigned)pl.slices, (unsigned)batch);
    if (pl.slices > 1) {
        NRS_ARG_CHECK(batch == 1, "gemm: split-K with batch > 1 unsupported");
        float* ws = workspace(sizeof(float) * (size_t)pl.slices * (size_t)M * (size_t)N, 0);
        if (!ws) return NRS_ERR_ALLOC;
        p.partial = ws;
        hipLaunchKernelGGL(fn, grid, dim3(s.threads), 0, stream(), p);
        NRS_LAUNCH_CHECK("gemm (split-K partials)");
        const int64_t total = M * N;
        unsigned blocks = (unsigned)std::min<int64_t>(cdiv(total, 64), 4 * (int64_t)num_cus());
        hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(64 * kSplitGroups), 0,
                           stream(), p, pl.slices);
        NRS_LAUNCH_CHECK("gemm (split-K reduce)");
    } else {
        p.partial = nullptr;
        hipLaunchKernelGGL(fn, grid, dim3(s.threads), 0, stream(), p);
        NRS_LAUNCH_CHECK("gemm");
    }
    return NRS_OK;
}

}  // namespace nrs

extern "C" {

int nrs_gemm(int layout, float* C, const float* A, const float* B, int64_t rows, int64_t cols,
             int64_t inner, float beta, const float* bias, int epilogue) {
    NRS_REQUIRE_INIT();
    return nrs::gemm_launch(layout, C, A, B, rows, cols, inner, 1, 0, 0, 0, beta, bias, epilogue,
                            0, true, 0);
}

int nrs_gemm_nt_splitk(float* C, const float* A, const float* B, int64_t rows, int64_t cols,
                       int64_t inner, float beta) {
    NRS_REQUIRE_INIT();
    return nrs::gemm_launch(NRS_NT, C, A, B, rows, cols, inner, 1, 0, 0, 0, beta, nullptr,
                            NRS_EPI_NONE, 0, true, 0);
}

int nrs_bmm(int layout, float* C, const float* A, const float* B, int64_t batch, int64_t rows,
            int64_t cols, int64_t inner, float beta) {
    NRS_REQUIRE_INIT();
    return nrs::gemm_launch(layout, C, A, B, rows, cols, inner, batch, rows * inner,
                            cols * inner, rows * cols, beta, nullptr, NRS_EPI_NONE, 0, false, 0);
}

}  // extern "C"
