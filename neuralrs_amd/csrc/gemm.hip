// Host side of the f32 GEMM core: tile-shape planning, split-K scratch and
// the C-ABI entry points nrs_gemm / nrs_gemm_nt_splitk / nrs_bmm. The kernels
// are in gemm_kernel.hpp.
#include <algorithm>

#include "gemm_kernel.hpp"
#include "gemm_skinny.hpp"
#include "gemm_wsplit.hpp"

namespace nrs {

// ------------------------------------------------------------------ host side

namespace {

using KernelFn = void (*)(GemmArgs);

struct TileShape {
    int bm, bn, bk, threads;
};

template <int BM, int BN, int BK, int WM_, int WN_, int PF, bool AK, bool BKC, int AM = OP_DENSE,
          int BMD = OP_DENSE>
KernelFn pick_vec(bool vec4) {
    return vec4 ? gemm_kernel<BM, BN, BK, WM_, WN_, AK, BKC, 4, 2, PF, AM, BMD>
                : gemm_kernel<BM, BN, BK, WM_, WN_, AK, BKC, 1, 2, PF, AM, BMD>;
}

// One load width only (the other variant of some tiles spills).
template <int BM, int BN, int BK, int WM_, int WN_, int PF, int VEC>
KernelFn pick_fixed(int layout) {
    switch (layout) {
        case NRS_NN: return gemm_kernel<BM, BN, BK, WM_, WN_, true, false, VEC, 2, PF>;
        case NRS_NT: return gemm_kernel<BM, BN, BK, WM_, WN_, true, true, VEC, 2, PF>;
        default: return gemm_kernel<BM, BN, BK, WM_, WN_, false, false, VEC, 2, PF>;
    }
}

template <int BM, int BN, int BK, int WM_, int WN_, int PF>
KernelFn pick_layout(int layout, bool vec4) {
    switch (layout) {
        case NRS_NN: return pick_vec<BM, BN, BK, WM_, WN_, PF, true, false>(vec4);
        case NRS_NT: return pick_vec<BM, BN, BK, WM_, WN_, PF, true, true>(vec4);
        default: return pick_vec<BM, BN, BK, WM_, WN_, PF, false, false>(vec4);
    }
}

// The implicit-GEMM convolution variants exist for the two tiles the conv
// shapes use: NN with an OP_IM2COL B (forward, stride-1 input gradient) and
// NT with an OP_NCHW A (weight gradient).
template <int BM, int BN, int BK, int WM_, int WN_, int PF>
KernelFn pick_conv(int layout, int amode, int bmode, bool vec4) {
    if (layout == NRS_NN && amode == OP_DENSE && bmode == OP_IM2COL)
        return pick_vec<BM, BN, BK, WM_, WN_, PF, true, false, OP_DENSE, OP_IM2COL>(vec4);
    if (layout == NRS_NT && amode == OP_NCHW && bmode == OP_DENSE)
        return pick_vec<BM, BN, BK, WM_, WN_, PF, true, true, OP_NCHW, OP_DENSE>(vec4);
    return nullptr;
}

// Tile configurations (chosen by a sweep over the workload shapes on MI355X).
// All run two waves per SIMD (register budget capped at 256 per lane,
// accumulators in VGPRs):
//  * 256x256x32, 8 waves of 128x64, ~140 KB LDS, prefetch depth 1: large
//    GEMMs (83-85% of FP32 MFMA peak at 4096^3 and 8192^3);
//  * 64x64x32, 4 waves of 32x32, prefetch depth 2: everything mid-sized
//    (bmm items, conv GEMMs, projections, split-K weight gradients);
//  * 128x128x32, 8 waves of 64x32, prefetch depth 2: dense GEMMs with one
//    to three of its tiles per CU (2048^3: 132 vs 150 us on 64x128; the cfg4
//    FFN 4096x1024x256: 24.6 vs 24.9 us);
//  * 64x128x32, 4 waves of 32x64, prefetch depth 2: grids of at least two
//    of its tiles per CU and K >= 256 whose 128x128 grid would be mostly
//    padding (2048^3 ran 162 us on it against 175 us on 64x64);
//  * 32x256x32, 4 waves of 32x64, prefetch depth 2 (1 with scalar loads):
//    outputs with at most 32 rows;
//  * 32x128x32, 4 waves of 32x32, prefetch depth 2: convolutions whose GEMM
//    has at most 32 rows (a 64-row tile would double the MFMA work);
//  * 128x32x32, 4 waves of 32x32, prefetch depth 2: outputs with at most 32
//    columns, e.g. attention's P.V and its input gradients (d_head 32);
//  * 64x64x32 with k-split wave sets (KS = 2: 8 waves, two per 32x32
//    sub-block, each reducing half of every k-tile), prefetch depth 2: dense
//    GEMMs with at most two 64x64 tiles per CU and no K split, which would
//    otherwise run one wave per SIMD (cfg4 projections 4096x256x256:
//    9.3 -> 8.7 us NT; FFN 4096x256x1024: 29.0 -> 25.1 us NN).
enum TileId { T256x256 = 0, T64x64, T32x256, T32x128, T128x32, T64x128, T64x64S2, T128x128, T_COUNT };
const TileShape kShapes[T_COUNT] = {
    {256, 256, 32, 512},
    {64, 64, 32, 256},
    {32, 256, 32, 256},
    {32, 128, 32, 256},
    {128, 32, 32, 256},
    {64, 128, 32, 256},
    {64, 64, 32, 512},
    {128, 128, 32, 512},
};

// `pf` is the register prefetch depth the plan asks for; tiles that have no
// variant for it return nullptr.
KernelFn kernel_for(int tile, int pf, int layout, bool vec4, int amode, int bmode) {
    if (amode != OP_DENSE || bmode != OP_DENSE) {
        switch (tile) {
            case T64x64: return pick_conv<64, 64, 32, 2, 2, 2>(layout, amode, bmode, vec4);
            case T32x128: return pick_conv<32, 128, 32, 1, 4, 2>(layout, amode, bmode, vec4);
            default: return nullptr;
        }
    }
    switch (tile) {
        case T256x256: return pick_layout<256, 256, 32, 2, 4, 1>(layout, vec4);
        case T64x64:
            return pf == 1 ? pick_layout<64, 64, 32, 2, 2, 1>(layout, vec4)
                           : pick_layout<64, 64, 32, 2, 2, 2>(layout, vec4);
        case T32x256:  // depth 2 with 128-bit loads; its scalar-load variant needs depth 1
            return vec4 ? pick_fixed<32, 256, 32, 1, 4, 2, 4>(layout)
                        : pick_fixed<32, 256, 32, 1, 4, 1, 1>(layout);
        case T64x128:  // planned only with 128-bit loads (the scalar variant spills)
            return vec4 ? pick_fixed<64, 128, 32, 2, 2, 2, 4>(layout) : nullptr;
        case T128x32:
            return pf == 1 ? pick_layout<128, 32, 32, 4, 1, 1>(layout, vec4)
                           : pick_layout<128, 32, 32, 4, 1, 2>(layout, vec4);
        case T128x128:  // planned only with 128-bit loads
            return vec4 ? pick_fixed<128, 128, 32, 2, 4, 2, 4>(layout) : nullptr;
        case T64x64S2:  // planned only with 128-bit loads
            if (!vec4) return nullptr;
            switch (layout) {
                case NRS_NN: return gemm_kernel<64, 64, 32, 2, 2, true, false, 4, 2, 2, OP_DENSE, OP_DENSE, 2>;
                case NRS_NT: return gemm_kernel<64, 64, 32, 2, 2, true, true, 4, 2, 2, OP_DENSE, OP_DENSE, 2>;
                default: return gemm_kernel<64, 64, 32, 2, 2, false, false, 4, 2, 2, OP_DENSE, OP_DENSE, 2>;
            }
        default: return nullptr;
    }
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

struct Plan {
    int tile;
    int slices;
    int64_t k_per_slice;
    int pf;  // register prefetch depth (k-tiles in flight per thread)
};

// Chooses the tile shape and the number of K slices. The 256x256 tile is
// used only with 128-bit loads (its scalar-load variant spills) and when at
// least 85% of its tile grid is real output.
Plan plan_gemm(int64_t M, int64_t N, int64_t K, int64_t batch, bool vec4, bool dense,
               bool allow_split, int force_slices) {
    const int cus = num_cus();
    auto tiles_of = [&](int t) {
        return cdiv(M, kShapes[t].bm) * cdiv(N, kShapes[t].bn) * batch;
    };
    // fraction of a tile grid's area that is real output (the rest is padding)
    auto fill = [&](int t) {
        return (double)(M * N) / ((double)cdiv(M, kShapes[t].bm) * kShapes[t].bm *
                                  cdiv(N, kShapes[t].bn) * kShapes[t].bn);
    };
    Plan pl{T64x64, 1, K, 2};
    if (dense) {
        if (M <= 32 && N >= 256)
            pl.tile = T32x256;
        else if (N <= 32 && M >= 128 && vec4)  // its scalar-load variants spill
            pl.tile = T128x32;
        else if (vec4 && tiles_of(T256x256) >= cus && fill(T256x256) >= 0.85)
            pl.tile = T256x256;
        else if (vec4 && tiles_of(T128x128) >= cus && fill(T128x128) >= 0.85)
            pl.tile = T128x128;
        else if (vec4 && tiles_of(T64x128) >= 2 * cus && K >= 256 && fill(T64x128) >= 0.85)
            pl.tile = T64x128;
    } else if (M <= 32) {  // gathered (convolution) operands: 64x64 or 32x128
        pl.tile = T32x128;
    }
    const TileShape& s = kShapes[pl.tile];
    const int64_t tiles = tiles_of(pl.tile);
    int slices = 1;
    if (force_slices > 0) {
        slices = force_slices;
    } else if (allow_split && batch == 1 && tiles < cus && (2 * tiles <= cus || K >= 2048) &&
               K >= 8 * s.bk) {
        // (a K of fewer than 8 k-tiles is not split: the reduce launch
        // costs more than the shorter k loop saves, e.g. 256x784 over
        // K = 128: 12.7 us split in two, 6.1 us whole)
        // About three workgroups per CU (one for the 32x256 tile, whose
        // workgroups stream a whole K slice of B: 8 slices of the skinny
        // 32x8192x8192 GEMM measured 67.8 us against 72.4 us at 24), each
        // slice at least two k-tiles, at most 256 slices (the reduction reads
        // every slice of every output).
        // Grids of 16 or more tiles keep at least 8 k-tiles per slice: their
        // partials are big, and a 3-k-tile slice is all latency (the cfg4
        // weight gradient 256x256 over K = 4096: 43 slices 19.4 us, 16
        // slices 14.9 us).
        const int64_t per_cu = pl.tile == T32x256 ? 1 : 3;
        const int64_t want = std::min<int64_t>(256, cdiv(per_cu * (int64_t)cus, tiles));
        const int64_t max_by_k = std::max<int64_t>(1, K / ((tiles >= 16 ? 8 : 2) * s.bk));
        slices = (int)std::min<int64_t>(want, max_by_k);
    }
    if (slices < 1) slices = 1;
    // Unsplit dense 64x64 grids of at most two tiles per CU: k-split wave sets.
    if (dense && vec4 && slices == 1 && force_slices <= 0 && pl.tile == T64x64 &&
        tiles <= 2 * (int64_t)cus && cdiv(K, s.bk) >= 2)
        pl.tile = T64x64S2;
    int64_t kps = cdiv(cdiv(K, slices), s.bk) * s.bk;
    if (kps <= 0) kps = s.bk;
    slices = (int)std::max<int64_t>(1, cdiv(K, kps));
    pl.slices = slices;
    pl.k_per_slice = kps;
    // Prefetch depth of the mid-size dense tiles (the k loop is padded to a
    // multiple of it): a single k-tile runs unpadded at depth 1.
    if (dense && (pl.tile == T64x64 || pl.tile == T128x32) && cdiv(kps, s.bk) <= 1) pl.pf = 1;
    return pl;
}

}  // namespace

namespace {

// Argument checks shared by every GEMM entry; `empty` is set for a call with
// nothing to compute (a zero output dimension or batch).
int check_call(const GemmCall& c, bool& empty) {
    const int64_t M = c.M, N = c.N, K = c.K, batch = c.batch;
    empty = false;
    NRS_ARG_CHECK(c.layout >= NRS_NN && c.layout <= NRS_TN, "gemm: unknown layout %d", c.layout);
    NRS_ARG_CHECK(M >= 0 && N >= 0 && K >= 0 && batch >= 0, "gemm: negative size");
    if (M == 0 || N == 0 || batch == 0) {
        empty = true;
        return NRS_OK;
    }
    NRS_ARG_CHECK(c.C != nullptr, "gemm: null C");
    NRS_ARG_CHECK(K == 0 || (c.A != nullptr && c.B != nullptr), "gemm: null operand");
    NRS_ARG_CHECK(!(c.epi & (NRS_EPI_BIAS_COL | NRS_EPI_BIAS_ROW)) || c.bias != nullptr,
                  "gemm: bias epilogue with null bias");
    NRS_ARG_CHECK(M <= INT32_MAX && N <= INT32_MAX, "gemm: dimension too large");
    const bool dense = c.amode == OP_DENSE && c.bmode == OP_DENSE;
    NRS_ARG_CHECK(dense || (c.gather_bytes > 0 && c.gather_bytes <= 0x80000000ll),
                  "gemm: gathered operand must be 1 B .. 2 GiB");
    NRS_ARG_CHECK(!c.mask || (dense && batch == 1 && c.nchw_P == 0),
                  "gemm: a mask needs a dense, unbatched, row-major GEMM");
    NRS_ARG_CHECK(!c.sum_row || (dense && batch == 1 && c.nchw_P == 0 && c.epi == NRS_EPI_NONE &&
                                 M < INT32_MAX),
                  "gemm: a row of sums needs a dense, unbatched GEMM without epilogue");
    return NRS_OK;
}

// 128-bit loads need 16-byte aligned rows of both operands (k-slices are
// multiples of BK, hence of 4). Bounds are checked per vector, so the guarded
// dimension must be a multiple of 4.
bool vec4_loads(const GemmCall& c) {
    const int layout = c.layout;
    const int64_t M = c.M, N = c.N, K = c.K, batch = c.batch;
    const int64_t lda = (layout == NRS_TN) ? M : K;
    const int64_t ldb = (layout == NRS_NT) ? K : N;
    bool a_vec, b_vec;
    if (c.amode == OP_NCHW)  // four columns never straddle an image
        a_vec = aligned16(c.A) && c.cg.P % 4 == 0 && K % 4 == 0;
    else
        a_vec = aligned16(c.A) && lda % 4 == 0 && (c.sA % 4 == 0 || batch == 1) &&
                (layout == NRS_TN ? M % 4 == 0 : K % 4 == 0);
    if (c.bmode == OP_IM2COL)  // gathered element-wise; only the LDS store is vectorised
        b_vec = true;
    else
        b_vec = aligned16(c.B) && ldb % 4 == 0 && (c.sB % 4 == 0 || batch == 1) &&
                (layout == NRS_NT ? K % 4 == 0 : N % 4 == 0);
    return a_vec && b_vec;
}

// Kernel arguments of call c on tile shape s with plan pl (partial unset).
int make_args(GemmArgs& p, const GemmCall& c, const TileShape& s, const Plan& pl) {
    const int64_t M = c.M, N = c.N, K = c.K;
    p = GemmArgs{};
    p.A = c.A;
    p.B = c.B;
    p.C = c.C;
    p.bias = c.bias;
    p.M = M;
    p.N = N;
    p.K = K;
    p.lda = (c.layout == NRS_TN) ? M : K;
    p.ldb = (c.layout == NRS_NT) ? K : N;
    p.ldc = N;
    p.sA = c.sA;
    p.sB = c.sB;
    p.sC = c.sC;
    p.mrows = M + (c.sum_row ? 1 : 0);
    p.sum_row = c.sum_row;
    p.sum_beta = c.sum_beta;
    p.mask = c.mask;
    p.tiles_m = (int)cdiv(p.mrows, s.bm);
    p.tiles_n = (int)cdiv(N, s.bn);
    p.group_m = 8;
    p.beta = c.beta;
    p.epi = c.epi;
    p.nchw_P = c.nchw_P;
    p.k_per_slice = pl.k_per_slice;
    p.cg = c.cg;
    p.gather_bytes = c.gather_bytes;
    if (c.amode != OP_DENSE || c.bmode != OP_DENSE) {
        NRS_ARG_CHECK(c.cg.P >= 1 && c.cg.P <= INT32_MAX && c.cg.ow >= 1 && c.cg.ow <= INT32_MAX &&
                          K <= INT32_MAX,
                      "gemm: convolution geometry out of range");
        p.cg.div_P = make_fastdiv((uint32_t)c.cg.P);
        p.cg.div_ow = make_fastdiv((uint32_t)c.cg.ow);
    }
    if (c.nchw_P > 0) {
        NRS_ARG_CHECK(c.nchw_P <= INT32_MAX, "gemm: NCHW plane too large");
        p.div_nchw = make_fastdiv((uint32_t)c.nchw_P);
    }
    // (the kernel renumbers a split grid by its linear id, tiles * slices)
    NRS_ARG_CHECK((int64_t)p.tiles_m * p.tiles_n * pl.slices <= INT32_MAX && c.batch <= 65535,
                  "gemm: grid too large");
    return NRS_OK;
}

void launch_reduce(GemmArgs p, int slices);

}  // namespace

void launch_splitk_reduce(GemmArgs p, int slices) { launch_reduce(p, slices); }

namespace {

void launch_reduce(GemmArgs p, int slices) {
    const int64_t total = p.mrows * p.N;
    if (p.N % 4 == 0 && p.nchw_P == 0 && p.ldc == p.N && aligned16(p.C) && aligned16(p.partial)) {
        const unsigned blocks =
            (unsigned)std::max<int64_t>(1, std::min<int64_t>(cdiv(total / 4, 256), 8 * (int64_t)num_cus()));
        hipLaunchKernelGGL(splitk_reduce4_kernel, dim3(blocks), dim3(256), 0, stream(), p, slices);
        return;
    }
    unsigned blocks = (unsigned)std::min<int64_t>(cdiv(total, 64), 4 * (int64_t)num_cus());
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(64 * kSplitGroups), 0, stream(), p,
                       slices);
}

}  // namespace

int gemm_run(const GemmCall& c) {
    bool empty;
    const int rc = check_call(c, empty);
    if (rc != NRS_OK || empty) return rc;
    const int layout = c.layout;
    const int64_t M = c.M, N = c.N, K = c.K, batch = c.batch;
    // few output tiles over a reduction of at most a few rounds: one launch
    // of the short-GEMM kernel, no split-K partials or reduce launch
    if (wsplit_eligible(c, true)) return wsplit_run(&c, 1, nullptr);
    // at most 32 rows over a long B: B streamed into registers
    if (skinny_eligible(c)) return skinny_run(c);
    const bool dense = c.amode == OP_DENSE && c.bmode == OP_DENSE;
    const bool vec4 = vec4_loads(c);

    Plan pl = plan_gemm(M + (c.sum_row ? 1 : 0), N, K, batch, vec4, dense,
                        c.allow_split && c.nchw_P == 0, c.force_slices);
    const TileShape& s = kShapes[pl.tile];
    GemmArgs p;
    const int arc = make_args(p, c, s, pl);
    if (arc != NRS_OK) return arc;

    KernelFn fn = kernel_for(pl.tile, pl.pf, layout, vec4, c.amode, c.bmode);
    NRS_ARG_CHECK(fn != nullptr, "gemm: no kernel for layout %d with operand modes %d/%d", layout,
                  c.amode, c.bmode);
    dim3 grid((unsigned)(p.tiles_m * p.tiles_n), (unsigned)pl.slices, (unsigned)batch);
    if (pl.slices > 1) {
        NRS_ARG_CHECK(batch == 1, "gemm: split-K with batch > 1 unsupported");
        const size_t need = sizeof(float) * (size_t)pl.slices * (size_t)p.mrows * (size_t)N;
        float* ws;
        if (c.partial_buf) {
            NRS_ARG_CHECK(need <= c.partial_cap,
                          "gemm: split-K partials of %zu bytes (%d slices of %lld x %lld) exceed "
                          "the %zu-byte scratch of the no-allocation entry point",
                          need, pl.slices, (long long)M, (long long)N, c.partial_cap);
            ws = c.partial_buf;
        } else {
            ws = workspace(need, 0);
            if (!ws) return NRS_ERR_ALLOC;
        }
        p.partial = ws;
        hipLaunchKernelGGL(fn, grid, dim3(s.threads), 0, stream(), p);
        NRS_LAUNCH_CHECK("gemm (split-K partials)");
        launch_reduce(p, pl.slices);
        NRS_LAUNCH_CHECK("gemm (split-K reduce)");
    } else {
        p.partial = nullptr;
        hipLaunchKernelGGL(fn, grid, dim3(s.threads), 0, stream(), p);
        NRS_LAUNCH_CHECK("gemm");
    }
    return NRS_OK;
}

bool overlaps(const void* a, size_t abytes, const void* b, size_t bbytes) {
    const char* x = static_cast<const char*>(a);
    const char* y = static_cast<const char*>(b);
    return x < y + bbytes && y < x + abytes;
}

// True when no call's outputs (C, the row of sums) overlap another call's
// outputs or operands (A, B, bias, and extra[j] of call j when given), so the
// calls may run in any order or together.
bool outputs_independent(const GemmCall* calls, int count, const OperandRange* extra) {
    struct Range {
        const void* p;
        size_t bytes;
    };
    auto ranges = [&](int idx, bool outputs_only, Range (&r)[7]) {
        const GemmCall& c = calls[idx];
        int n = 0;
        r[n++] = {c.C, sizeof(float) * (size_t)(c.M * c.N)};
        if (c.sum_row) r[n++] = {c.sum_row, sizeof(float) * (size_t)c.N};
        if (outputs_only) return n;
        r[n++] = {c.A, sizeof(float) * (size_t)(c.M * c.K)};
        r[n++] = {c.B, sizeof(float) * (size_t)(c.K * c.N)};
        if (c.epi & (NRS_EPI_BIAS_COL | NRS_EPI_BIAS_ROW))
            r[n++] = {c.bias, sizeof(float) * (size_t)std::max<int64_t>(
                                  (c.epi & NRS_EPI_BIAS_COL) ? c.N : 0,
                                  (c.epi & NRS_EPI_BIAS_ROW) ? c.M : 0)};
        if (c.mask) r[n++] = {c.mask, sizeof(float) * (size_t)(c.M * c.N)};
        if (extra && extra[idx].p) r[n++] = {extra[idx].p, extra[idx].bytes};
        return n;
    };
    for (int i = 0; i < count; ++i) {
        if (calls[i].M == 0 || calls[i].N == 0) continue;
        Range out[7], other[7];
        const int no = ranges(i, true, out);
        for (int j = 0; j < count; ++j) {
            if (j == i || calls[j].M == 0 || calls[j].N == 0) continue;
            const int nj = ranges(j, false, other);
            for (int a = 0; a < no; ++a)
                for (int b = 0; b < nj; ++b)
                    if (overlaps(out[a].p, out[a].bytes, other[b].p, other[b].bytes)) return false;
        }
    }
    return true;
}

namespace {

// The group kernel's tile: 64x64x32, 2x2 waves of 32x32, prefetch depth 2,
// compiled for up to four waves per SIMD so that several problems'
// workgroups share a CU.
constexpr int kGroupBM = 64, kGroupBN = 64, kGroupBK = 32, kGroupThreads = 256;
static_assert(kGroupMax >= NRS_GEMM_GROUP_MAX, "group size of the kernel and the C ABI");
static_assert(sizeof(GemmGroupArgs) <= 4096, "group kernel arguments");

}  // namespace

namespace {

// The group kernel's plan: K slices per call, and the order the problems take
// in the grid.
struct GroupPlan {
    Plan plans[kGroupMax];
    int order[kGroupMax];
    int live_n = 0;
    size_t partial_floats = 0;  // split-K partials of every split call
};

// Plans each problem of a group: a problem of few tiles over a long K is
// split so that it brings about one workgroup per CU (at least 8 k-tiles per
// slice, 2 for a grid under 16 tiles), like a launch of its own would. The
// plan of a call does not depend on the other calls of its group.
void plan_group(const GemmCall* calls, int count, GroupPlan& gp) {
    const int cus = num_cus();
    const TileShape s{kGroupBM, kGroupBN, kGroupBK, kGroupThreads};
    for (int i = 0; i < count; ++i) {
        const GemmCall& c = calls[i];
        if (c.M == 0 || c.N == 0) continue;
        const int64_t tiles = cdiv(c.M + (c.sum_row ? 1 : 0), s.bm) * cdiv(c.N, s.bn);
        int64_t slices = 1;
        if (tiles * 2 <= cus && c.K >= 8 * s.bk) {
            const int64_t want = std::min<int64_t>(256, cdiv(cus, tiles));
            const int64_t max_by_k = std::max<int64_t>(1, c.K / ((tiles >= 16 ? 8 : 2) * s.bk));
            slices = std::max<int64_t>(1, std::min(want, max_by_k));
        }
        const int64_t kps = cdiv(cdiv(c.K, slices), s.bk) * s.bk;
        gp.plans[i] = Plan{T64x64, (int)std::max<int64_t>(1, cdiv(c.K, kps)), kps, 2};
        if (gp.plans[i].slices > 1)
            gp.partial_floats += (size_t)gp.plans[i].slices *
                                 (size_t)((c.M + (c.sum_row ? 1 : 0)) * c.N);
        // Workgroups are dispatched in grid order, so the problems whose
        // workgroups run longest (most k-tiles each) go first: started last
        // they would run on alone after the short ones drain (the FFN
        // backward pair, dW over 32 k-tiles per workgroup behind dX's 1024
        // tiles of 8, took 74 us that way against 60 us long-first).
        int j = gp.live_n++;
        for (; j > 0 && gp.plans[gp.order[j - 1]].k_per_slice < kps; --j)
            gp.order[j] = gp.order[j - 1];
        gp.order[j] = i;
    }
}

// Launches the group kernel on a plan; split calls write their partials to
// consecutive regions of `partials` (gp.partial_floats floats), in call
// order. g receives the launched arguments (the caller reduces the splits).
int launch_group(const GemmCall* calls, const GroupPlan& gp, float* partials, GemmGroupArgs& g,
                 float** part_of_call = nullptr) {
    const TileShape s{kGroupBM, kGroupBN, kGroupBK, kGroupThreads};
    float* part_of[kGroupMax] = {};
    float* ws = partials;
    for (int oi = 0; oi < gp.live_n; ++oi) {
        const int i = gp.order[oi];
        if (gp.plans[i].slices <= 1) continue;
        part_of[i] = ws;
        ws += (size_t)gp.plans[i].slices *
              (size_t)((calls[i].M + (calls[i].sum_row ? 1 : 0)) * calls[i].N);
    }
    int next = 0;
    int64_t total_wgs = 0;
    for (int oi = 0; oi < gp.live_n; ++oi) {
        const int i = gp.order[oi];
        const GemmCall& c = calls[i];
        const Plan& pl = gp.plans[i];
        const int64_t tiles = cdiv(c.M + (c.sum_row ? 1 : 0), s.bm) * cdiv(c.N, s.bn);
        GemmArgs& p = g.prob[next];
        const int rc = make_args(p, c, s, pl);
        if (rc != NRS_OK) return rc;
        total_wgs = (total_wgs + 7) / 8 * 8;
        g.first[next] = (int)total_wgs;
        g.layout[next] = c.layout;
        g.slices[next] = pl.slices;
        if (pl.slices > 1) p.partial = part_of[i];
        total_wgs += tiles * pl.slices;
        ++next;
    }
    g.count = next;
    if (part_of_call)
        for (int i = 0; i < kGroupMax; ++i) part_of_call[i] = part_of[i];
    NRS_ARG_CHECK(total_wgs <= INT32_MAX, "gemm group: grid too large");
    hipLaunchKernelGGL((gemm_group_kernel<kGroupBM, kGroupBN, kGroupBK, 2, 2, 4, 2>),
                       dim3((unsigned)total_wgs), dim3(kGroupThreads), 0, stream(), g);
    NRS_LAUNCH_CHECK("gemm group");
    return NRS_OK;
}

}  // namespace

int gemm_group_run(const GemmCall* calls, int count) {
    NRS_ARG_CHECK(count >= 0 && (count == 0 || calls != nullptr), "gemm group: bad count");
    // Checks first, so that an invalid call launches nothing.
    bool grouped = count >= 2 && count <= NRS_GEMM_GROUP_MAX;
    bool short_group = grouped;  // every live call fits the short-GEMM kernel
    bool is_live[kGroupMax] = {};
    int live = 0;
    for (int i = 0; i < count; ++i) {
        bool empty;
        const int rc = check_call(calls[i], empty);
        if (rc != NRS_OK) return rc;
        if (empty) continue;
        ++live;
        if (i < kGroupMax) is_live[i] = true;
        const GemmCall& c = calls[i];
        grouped = grouped && c.amode == OP_DENSE && c.bmode == OP_DENSE && c.batch == 1 &&
                  c.nchw_P == 0 && c.partial_buf == nullptr && c.force_slices == 0 &&
                  c.K > 0 && vec4_loads(c);
        short_group = short_group && wsplit_eligible(c, true);
    }
    // An output overlapping another call's operand, bias or output would make
    // the result depend on the order the problems run in: such groups run one
    // call after another, in the order given.
    if ((grouped || short_group) && !outputs_independent(calls, count, nullptr))
        grouped = short_group = false;
    if (short_group && live >= 2) {
        GemmCall live_calls[kGroupMax];
        int n = 0;
        for (int i = 0; i < count; ++i)
            if (is_live[i]) live_calls[n++] = calls[i];
        return wsplit_run(live_calls, n, nullptr);
    }
    if (!grouped || live < 2) {
        for (int i = 0; i < count; ++i) {
            const int rc = gemm_run(calls[i]);
            if (rc != NRS_OK) return rc;
        }
        return NRS_OK;
    }

    GroupPlan gp;
    plan_group(calls, count, gp);
    float* partials = nullptr;
    if (gp.partial_floats > 0) {
        partials = workspace(sizeof(float) * gp.partial_floats, 0);
        if (!partials) return NRS_ERR_ALLOC;
    }
    GemmGroupArgs g{};
    const int rc = launch_group(calls, gp, partials, g);
    if (rc != NRS_OK) return rc;
    for (int q = 0; q < g.count; ++q)
        if (g.slices[q] > 1) {
            launch_reduce(g.prob[q], g.slices[q]);
            NRS_LAUNCH_CHECK("gemm group (split-K reduce)");
        }
    return NRS_OK;
}

namespace {

// The sums that finish a shared-operand backward, in one launch. Problem q
// stores v = R_0 (+ beta * old) + R_1 + ... into dst, each part's R_j being
// its one product or the sum of its split-K slices in slice order from 0;
// with in_dst, dst already holds R_0 (+ beta * old) and every listed part is
// added to it. These are the operations, in the same order, of the products'
// epilogues and of splitk_reduce4_kernel when the products run one group
// after another. A problem's workgroups are a contiguous block range, so the
// problem index is uniform per workgroup.
constexpr int kSumMax = 4;
struct SumPart {
    const float* src;
    int slices;
};
struct SumProblem {
    float* dst;
    int64_t total4;  // float4s of dst (and of each slice)
    float beta;
    int nparts;
    int in_dst;
    SumPart part[3];
};
struct GroupSumArgs {
    SumProblem prob[kSumMax];
    int first[kSumMax];   // first workgroup of each problem, ascending
    int blocks[kSumMax];  // its workgroups
    int count;
};

__device__ __forceinline__ f32x4 sum_part(const SumPart& s, int64_t i, int64_t total4) {
    const f32x4* src = reinterpret_cast<const f32x4*>(s.src) + i;
    if (s.slices == 1) return *src;
    // eight slices' loads in flight, added in slice order
    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    int k = 0;
    for (; k + 8 <= s.slices; k += 8) {
        f32x4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = src[(int64_t)(k + j) * total4];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc = acc + v[j];
    }
    for (; k < s.slices; ++k) acc = acc + src[(int64_t)k * total4];
    return acc;
}

__global__ __launch_bounds__(256) void group_sum_kernel(GroupSumArgs a) {
    const int b = blockIdx.x;
    int q = 0;
#pragma unroll
    for (int j = 1; j < kSumMax; ++j)
        if (j < a.count && b >= a.first[j]) q = j;
    const SumProblem& p = a.prob[q];
    const int64_t step = (int64_t)a.blocks[q] * 256;
    for (int64_t i = (int64_t)(b - a.first[q]) * 256 + threadIdx.x; i < p.total4; i += step) {
        f32x4* dst = reinterpret_cast<f32x4*>(p.dst) + i;
        f32x4 v;
        int j = 0;
        if (p.in_dst) {
            v = *dst;
        } else {
            v = sum_part(p.part[0], i, p.total4);
            if (p.beta != 0.0f) v = v + p.beta * *dst;
            j = 1;
        }
        for (; j < p.nparts; ++j) v = sum_part(p.part[j], i, p.total4) + v;
        *dst = v;
    }
}

}  // namespace

int shared_lhs_backward(float* dx, float* const* dw, const float* const* g, const float* x,
                        const float* const* w, int count, int64_t rows, int64_t inner,
                        int64_t cols, float beta_x, const float* beta_w) {
    NRS_ARG_CHECK(count >= 1 && count <= 3, "shared-lhs backward: %d products (1 to 3)", count);
    NRS_ARG_CHECK(dw && g && w && beta_w, "shared-lhs backward: null array");
    NRS_ARG_CHECK(rows >= 0 && inner >= 0 && cols >= 0, "shared-lhs backward: negative size");
    // the pair of closure i: dx (+)= g_i . W_i^T, dW_i = x^T . g_i + beta_w[i] * dW_i
    GemmCall pair[3][2];
    for (int i = 0; i < count; ++i) {
        GemmCall& d = pair[i][0];
        d.layout = NRS_NT;
        d.C = dx;
        d.A = g[i];
        d.B = w[i];
        d.M = rows;
        d.N = inner;
        d.K = cols;
        d.beta = i == 0 ? beta_x : 1.0f;
        GemmCall& e = pair[i][1];
        e.layout = NRS_TN;
        e.C = dw[i];
        e.A = x;
        e.B = g[i];
        e.M = inner;
        e.N = cols;
        e.K = rows;
        e.beta = beta_w[i];
        for (const GemmCall& c : pair[i]) {
            bool empty;
            const int rc = check_call(c, empty);
            if (rc != NRS_OK) return rc;
        }
    }
    // One group for all products when every pair would run the group kernel
    // (not the short-GEMM kernel) and no output overlaps another output or an
    // operand; otherwise the closures' sequence.
    bool fused = count >= 2 && rows > 0 && inner > 0 && cols > 0 && (rows * inner) % 4 == 0 &&
                 (inner * cols) % 4 == 0 && aligned16(dx);
    for (int i = 0; i < count && fused; ++i)
        for (const GemmCall& c : pair[i])
            fused = fused && vec4_loads(c) && aligned16(c.C);
    for (int i = 0; i < count && fused; ++i)
        fused = !(wsplit_eligible(pair[i][0], true) && wsplit_eligible(pair[i][1], true));
    if (fused) {
        const OperandRange outs[4] = {{dx, sizeof(float) * (size_t)(rows * inner)},
                                      {dw[0], sizeof(float) * (size_t)(inner * cols)},
                                      {count > 1 ? dw[1] : nullptr, sizeof(float) * (size_t)(inner * cols)},
                                      {count > 2 ? dw[2] : nullptr, sizeof(float) * (size_t)(inner * cols)}};
        OperandRange ins[7] = {{x, sizeof(float) * (size_t)(rows * inner)}};
        for (int i = 0; i < count; ++i) {
            ins[1 + 2 * i] = {w[i], sizeof(float) * (size_t)(inner * cols)};
            ins[2 + 2 * i] = {g[i], sizeof(float) * (size_t)(rows * cols)};
        }
        for (int a = 0; a <= count && fused; ++a) {
            for (int b = 0; b < 1 + 2 * count; ++b)
                fused = fused && !overlaps(outs[a].p, outs[a].bytes, ins[b].p, ins[b].bytes);
            for (int b = a + 1; b <= count; ++b)
                fused = fused && !overlaps(outs[a].p, outs[a].bytes, outs[b].p, outs[b].bytes);
        }
    }
    if (!fused) {
        for (int i = 0; i < count; ++i) {
            const int rc = gemm_group_run(pair[i], 2);
            if (rc != NRS_OK) return rc;
        }
        return NRS_OK;
    }

    // calls 0..count-1: the input-gradient products (the first into dx with
    // beta_x when not split, the others with beta 0 into scratch when not
    // split); count..2*count-1: the weight gradients
    GemmCall calls[kGroupMax];
    for (int i = 0; i < count; ++i) {
        calls[i] = pair[i][0];
        calls[i].beta = 0.0f;
        calls[count + i] = pair[i][1];
    }
    GroupPlan gp;
    plan_group(calls, 2 * count, gp);
    const size_t dx_floats = (size_t)(rows * inner);
    const bool first_in_dx = gp.plans[0].slices == 1;
    if (first_in_dx) calls[0].beta = beta_x;
    size_t direct = 0;
    for (int i = first_in_dx ? 1 : 0; i < count; ++i)
        direct += gp.plans[i].slices == 1 ? dx_floats : 0;
    float* ws = workspace(sizeof(float) * (gp.partial_floats + direct), 0);
    if (!ws) return NRS_ERR_ALLOC;
    float* region = ws + gp.partial_floats;
    float* direct_of[3] = {};
    for (int i = first_in_dx ? 1 : 0; i < count; ++i)
        if (gp.plans[i].slices == 1) {
            direct_of[i] = region;
            calls[i].C = region;
            region += dx_floats;
        }
    GemmGroupArgs ga{};
    float* part_of[kGroupMax] = {};
    int rc = launch_group(calls, gp, ws, ga, part_of);
    if (rc != NRS_OK) return rc;

    GroupSumArgs sa{};
    const int64_t cap = 8 * (int64_t)num_cus();
    int blocks = 0;
    auto add = [&](SumProblem p) {
        const int q = sa.count++;
        sa.prob[q] = p;
        sa.first[q] = blocks;
        sa.blocks[q] = (int)std::max<int64_t>(1, std::min<int64_t>(cdiv(p.total4, 256), cap));
        blocks += sa.blocks[q];
    };
    SumProblem px{};
    px.dst = dx;
    px.total4 = (int64_t)dx_floats / 4;
    px.beta = beta_x;
    px.in_dst = first_in_dx ? 1 : 0;
    for (int i = first_in_dx ? 1 : 0; i < count; ++i)
        px.part[px.nparts++] =
            direct_of[i] ? SumPart{direct_of[i], 1} : SumPart{part_of[i], gp.plans[i].slices};
    add(px);
    for (int i = 0; i < count; ++i) {
        const int c = count + i;
        if (gp.plans[c].slices <= 1) continue;  // written with its beta by the group kernel
        SumProblem pw{};
        pw.dst = dw[i];
        pw.total4 = inner * cols / 4;
        pw.beta = beta_w[i];
        pw.nparts = 1;
        pw.part[0] = SumPart{part_of[c], gp.plans[c].slices};
        add(pw);
    }
    hipLaunchKernelGGL(group_sum_kernel, dim3((unsigned)blocks), dim3(256), 0, stream(), sa);
    NRS_LAUNCH_CHECK("shared-lhs backward (sums)");
    return NRS_OK;
}

}  // namespace nrs

namespace nrs {

// The GemmCall of one bmm product over contiguous items.
GemmCall bmm_call(int layout, float* C, const float* A, const float* B, int64_t batch,
                  int64_t rows, int64_t cols, int64_t inner, float beta) {
    GemmCall c;
    c.layout = layout;
    c.C = C;
    c.A = A;
    c.B = B;
    c.M = rows;
    c.N = cols;
    c.K = inner;
    c.batch = batch;
    c.sA = rows * inner;
    c.sB = cols * inner;
    c.sC = rows * cols;
    c.beta = beta;
    c.allow_split = false;
    return c;
}

}  // namespace nrs

namespace nrs {

// nrs_linear_backward, with the input gradient masked (v = 0 where
// mask <= 0) when mask is non-null.
int linear_backward(float* dx, float* dw, float* db, const float* grad, const float* x,
                    const float* w, const float* mask, int64_t batch, int64_t in_f, int64_t out_f,
                    float beta_x, float beta_w, float beta_b) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(batch >= 0 && in_f >= 0 && out_f >= 0, "linear backward: negative size");
    NRS_ARG_CHECK(dw != nullptr, "linear backward: null weight gradient");
    if (in_f == 0 && db) {  // no weight rows to carry the row of sums
        const int rc = nrs_sum_axis0(db, grad, batch, out_f, beta_b);
        if (rc != NRS_OK || !dx) return rc;
        db = nullptr;
    }
    // The row of sums rides the weight-gradient product when it costs no
    // extra tile row (in_f not a multiple of 64), the product is small, or
    // the extra 64-row tile row is cheaper than the column-sum launches
    // (two for more than 1024 rows, ~3 us each): at most 2^28 FLOP, e.g. the
    // cfg4 FFN's 1024 x 256 weight gradient (68 tiles in place of 64). The
    // 256 x 1024 one (80 tiles in place of 64, 2^29 FLOP more) sums after
    // the group in a launch of its own.
    float* db_after = nullptr;
    if (db && in_f % 64 == 0 && in_f * out_f > 65536 && 128 * out_f * batch > (int64_t)1 << 28) {
        db_after = db;
        db = nullptr;
    }
    nrs::GemmCall calls[2];
    int n = 0;
    nrs::GemmCall& cw = calls[n++];  // dW = x^T . grad, db = column sums of grad
    cw.layout = NRS_TN;
    cw.C = dw;
    cw.A = x;
    cw.B = grad;
    cw.M = in_f;
    cw.N = out_f;
    cw.K = batch;
    cw.beta = beta_w;
    cw.sum_row = db;
    cw.sum_beta = beta_b;
    if (dx) {  // dx = grad . W^T
        nrs::GemmCall& cx = calls[n++];
        cx.layout = NRS_NT;
        cx.C = dx;
        cx.A = grad;
        cx.B = w;
        cx.M = batch;
        cx.N = in_f;
        cx.K = out_f;
        cx.beta = beta_x;
        cx.mask = mask;
    }
    const int rc = nrs::gemm_group_run(calls, n);
    if (rc != NRS_OK || !db_after) return rc;
    return nrs_sum_axis0(db_after, grad, batch, out_f, beta_b);
}

}  // namespace nrs

extern "C" {

int nrs_gemm(int layout, float* C, const float* A, const float* B, int64_t rows, int64_t cols,
             int64_t inner, float beta, const float* bias, int epilogue) {
    NRS_REQUIRE_INIT();
    nrs::GemmCall c;
    c.layout = layout;
    c.C = C;
    c.A = A;
    c.B = B;
    c.M = rows;
    c.N = cols;
    c.K = inner;
    c.beta = beta;
    c.bias = bias;
    c.epi = epilogue;
    return nrs::gemm_run(c);
}

int nrs_gemm_group(const nrs_gemm_desc* descs, int count) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(count >= 0 && count <= NRS_GEMM_GROUP_MAX,
                  "gemm group: %d calls (at most %d)", count, NRS_GEMM_GROUP_MAX);
    NRS_ARG_CHECK(count == 0 || descs != nullptr, "gemm group: null descriptors");
    nrs::GemmCall calls[NRS_GEMM_GROUP_MAX];
    for (int i = 0; i < count; ++i) {
        const nrs_gemm_desc& d = descs[i];
        nrs::GemmCall& c = calls[i];
        c.layout = d.layout;
        c.C = d.C;
        c.A = d.A;
        c.B = d.B;
        c.M = d.rows;
        c.N = d.cols;
        c.K = d.inner;
        c.beta = d.beta;
        c.bias = d.bias;
        c.epi = d.epilogue;
    }
    return nrs::gemm_group_run(calls, count);
}

int nrs_matmul_shared_lhs_backward(float* dx, float* const* dw, const float* const* g,
                                   const float* x, const float* const* w, int count, int64_t rows,
                                   int64_t inner, int64_t cols, float beta_x,
                                   const float* beta_w) {
    NRS_REQUIRE_INIT();
    return nrs::shared_lhs_backward(dx, dw, g, x, w, count, rows, inner, cols, beta_x, beta_w);
}

int nrs_linear_backward(float* dx, float* dw, float* db, const float* grad, const float* x,
                        const float* w, int64_t batch, int64_t in_f, int64_t out_f, float beta_x,
                        float beta_w, float beta_b) {
    return nrs::linear_backward(dx, dw, db, grad, x, w, nullptr, batch, in_f, out_f, beta_x,
                                beta_w, beta_b);
}

int nrs_linear_backward_relu(float* dx, float* dw, float* db, const float* grad, const float* x,
                             const float* w, const float* mask, int64_t batch, int64_t in_f,
                             int64_t out_f, float beta_x, float beta_w, float beta_b) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(!dx || mask, "linear backward relu: null mask");
    return nrs::linear_backward(dx, dw, db, grad, x, w, dx ? mask : nullptr, batch, in_f, out_f,
                                beta_x, beta_w, beta_b);
}

int nrs_linear_cross_entropy(float* logits, float* grad, const float* x, const float* w,
                             const float* bias, const float* target, int64_t batch, int64_t in_f,
                             int64_t classes) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(batch >= 0 && in_f >= 0 && classes >= 1, "linear cross_entropy: bad shape");
    if (batch == 0) return NRS_OK;
    NRS_ARG_CHECK(logits && grad && target && (in_f == 0 || (x && w)),
                  "linear cross_entropy: null pointer");
    // Both outputs are written while other workgroups still read x, w, the
    // bias and the targets, so no output may share memory with an input or
    // with the other output.
    const size_t out_bytes = sizeof(float) * (size_t)(batch * classes);
    const size_t x_bytes = sizeof(float) * (size_t)(batch * in_f);
    const size_t w_bytes = sizeof(float) * (size_t)(in_f * classes);
    const size_t b_bytes = bias ? sizeof(float) * (size_t)classes : 0;
    for (float* dst : {logits, grad}) {
        NRS_ARG_CHECK(!nrs::overlaps(dst, out_bytes, x, x_bytes) &&
                          !nrs::overlaps(dst, out_bytes, w, w_bytes) &&
                          !nrs::overlaps(dst, out_bytes, bias, b_bytes) &&
                          !nrs::overlaps(dst, out_bytes, target, out_bytes),
                      "linear cross_entropy: logits and grad must not overlap x, w, bias or target");
    }
    NRS_ARG_CHECK(!nrs::overlaps(logits, out_bytes, grad, out_bytes),
                  "linear cross_entropy: logits and grad must not overlap");
    nrs::GemmCall c;
    c.layout = NRS_NN;
    c.C = logits;
    c.A = x;
    c.B = w;
    c.M = batch;
    c.N = classes;
    c.K = in_f;
    c.bias = bias;
    c.epi = bias ? NRS_EPI_BIAS_COL : NRS_EPI_NONE;
    bool empty;
    const int rc = nrs::check_call(c, empty);
    if (rc != NRS_OK) return rc;
    if (classes <= 16 && nrs::wsplit_eligible(c, false)) {
        nrs::WsExtra e;
        e.ce_grad = grad;
        e.ce_target = target;
        return nrs::wsplit_run(&c, 1, &e);
    }
    const int grc = nrs::gemm_run(c);
    if (grc != NRS_OK) return grc;
    return nrs_cross_entropy_backward(grad, logits, target, batch, classes);
}

int nrs_gemm_nt_splitk(float* C, const float* A, const float* B, int64_t rows, int64_t cols,
                       int64_t inner, float beta) {
    NRS_REQUIRE_INIT();
    nrs::GemmCall c;
    c.layout = NRS_NT;
    c.C = C;
    c.A = A;
    c.B = B;
    c.M = rows;
    c.N = cols;
    c.K = inner;
    c.beta = beta;
    return nrs::gemm_run(c);
}

int nrs_gemm_nt_splitk_noalloc(float* C, const float* A, const float* B, int64_t rows,
                               int64_t cols, int64_t inner, float beta) {
    NRS_REQUIRE_INIT();
    float* scratch = nrs::noalloc_scratch();
    NRS_ARG_CHECK(scratch != nullptr, "nrs_gemm_nt_splitk_noalloc: scratch of device %d not set up",
                  nrs::device());
    nrs::GemmCall c;
    c.layout = NRS_NT;
    c.C = C;
    c.A = A;
    c.B = B;
    c.M = rows;
    c.N = cols;
    c.K = inner;
    c.beta = beta;
    c.partial_buf = scratch;  // every partial is written before it is read: no clearing
    c.partial_cap = nrs::kNoAllocScratchBytes;
    return nrs::gemm_run(c);
}

int nrs_bmm(int layout, float* C, const float* A, const float* B, int64_t batch, int64_t rows,
            int64_t cols, int64_t inner, float beta) {
    NRS_REQUIRE_INIT();
    const nrs::GemmCall c = nrs::bmm_call(layout, C, A, B, batch, rows, cols, inner, beta);
    const int rc = nrs::bmm_small(c);
    return rc == nrs::kBmmUnsupported ? nrs::gemm_run(c) : rc;
}

int nrs_bmm_backward(int layout, float* dA, float* dB, const float* G, const float* A,
                     const float* B, int64_t batch, int64_t m, int64_t k, int64_t n, float beta) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(layout == NRS_NN || layout == NRS_NT,
                  "bmm backward: forward layout must be NN or NT, got %d", layout);
    // forward NN: C = A . B, B [k][n]: dA = G . B^T (NT), dB = A^T . G (TN);
    // forward NT: C = A . B^T, B [n][k]: dA = G . B (NN), dB = G^T . A (TN)
    const bool nn = layout == NRS_NN;
    const nrs::GemmCall ca =
        nrs::bmm_call(nn ? NRS_NT : NRS_NN, dA, G, B, batch, m, k, n, beta);
    const nrs::GemmCall cb = nn ? nrs::bmm_call(NRS_TN, dB, A, G, batch, k, n, m, beta)
                                : nrs::bmm_call(NRS_TN, dB, G, A, batch, n, k, m, beta);
    if (dA && dB) {
        // both gradients of small items: one launch
        const int rc = nrs::bmm_small_pair(ca, cb);
        if (rc != nrs::kBmmUnsupported) return rc;
    }
    if (dA) {
        const int rc = nrs_bmm(ca.layout, dA, ca.A, ca.B, batch, ca.M, ca.N, ca.K, beta);
        if (rc) return rc;
    }
    if (dB) {
        const int rc = nrs_bmm(cb.layout, dB, cb.A, cb.B, batch, cb.M, cb.N, cb.K, beta);
        if (rc) return rc;
    }
    return NRS_OK;
}

}  // extern "C"
