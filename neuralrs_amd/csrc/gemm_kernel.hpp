// Device side of the f32 GEMM core for gfx950: the replacement for
// matmul_nn / matmul_nt / matmul_tn / matmul_nt_splitk
// (src/cuda/graph/matmul.rs:44-261) and the bmm kernels
// (src/cuda/graph/bmm.rs:12-56).
//
// Design (CDNA4, wave64):
//  * v_mfma_f32_32x32x2_f32 does the contraction in full f32 (products and
//    sums rounded to f32, like the reference's FMA loop, only in another
//    order). A workgroup of WAVES_M x WAVES_N waves owns a BM x BN block of C;
//    each wave owns a (32*FM) x (32*FN) sub-block in FM*FN 16-float
//    accumulators. Kernels are compiled for two waves per SIMD (at most 256
//    registers per lane), so the accumulators live in VGPRs and nothing
//    spills.
//  * A and B tiles are staged through LDS, double-buffered, one barrier per
//    k-tile. Global loads are 128-bit where alignment allows and are issued
//    PF k-tiles ahead into a register ring, so their latency hides behind the
//    MFMAs of the tiles in between.
//  * An operand whose reduction dimension is contiguous in memory (A of NN/NT,
//    B of NT) keeps it contiguous in LDS ([mn][k], row stride BK+4 floats:
//    16-byte fragment reads are bank-conflict-free); the other kind is kept
//    [k][mn] (row stride BMN+8) and read 4 bytes per lane, conflict-free too.
//    Within a group of 8 k values, lane half h (lanes 32h..32h+31) takes
//    k = 8g + 4h + p for MFMA step p = 0..3 on both operands, so one 16-byte
//    LDS read feeds four MFMAs.
//  * Split-K (grid.y slices) writes raw partial tiles to scratch; a second
//    kernel sums the slices in slice order (deterministic) and applies the
//    epilogue. The reference accumulates slices with float atomicAdd.
//  * Workgroup ids are remapped so that each XCD (workgroups are dealt to the
//    8 XCDs round-robin) owns a compact, grouped block of output tiles, which
//    keeps the A rows and B columns those tiles share inside that XCD's L2.
#pragma once

#include "buffer_ops.hpp"
#include "gemm_args.hpp"
#include "gemm_call.hpp"

namespace nrs {

// Tile coordinates for workgroup `bid` of `tiles` total: XCD-compact, then
// grouped along M so neighbouring workgroups share A rows and B columns.
__device__ __forceinline__ void tile_coords(const GemmArgs& p, int bid, int& tm, int& tn) {
    const int tiles = p.tiles_m * p.tiles_n;
    int id = bid;
    if ((tiles & 7) == 0) id = (bid & 7) * (tiles >> 3) + (bid >> 3);
    const int per_group = p.group_m * p.tiles_n;
    const int group = id / per_group;
    const int first_m = group * p.group_m;
    const int gsize = min(p.tiles_m - first_m, p.group_m);
    const int in_group = id - group * per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, bool AK, bool BKC, int VEC, int KS = 1>
struct Cfg {
    static constexpr int NT = 64 * WAVES_M * WAVES_N * KS;
    static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    static constexpr int FM = WM / 32, FN = WN / 32;
    static constexpr int SA = AK ? (BK + 4) : (BM + 8);
    static constexpr int SB = BKC ? (BK + 4) : (BN + 8);
    static constexpr int A_ELEMS = AK ? BM * SA : BK * SA;
    static constexpr int B_ELEMS = BKC ? BN * SB : BK * SB;
    static constexpr int STAGE = A_ELEMS + B_ELEMS;
    static constexpr int A_LOADS = BM * BK / (VEC * NT);
    static constexpr int B_LOADS = BN * BK / (VEC * NT);
    static_assert(FM >= 1 && FN >= 1, "wave tile must be at least 32x32");
    static_assert(FM * 32 * WAVES_M == BM && FN * 32 * WAVES_N == BN, "wave grid");
    static_assert(BK % (8 * KS) == 0, "BK must split into groups of 8 per k-split wave set");
    static_assert(A_LOADS >= 1 && B_LOADS >= 1, "tile too small for the thread count");
    static_assert(A_LOADS * VEC * NT == BM * BK && B_LOADS * VEC * NT == BN * BK, "load split");
    static_assert(2 * STAGE * 4 <= 160 * 1024, "LDS budget");
};

// Position of load q of a k-tile of one operand (same mapping for the global
// load and the LDS store).
template <int BMN, int BK, bool KC, int VEC>
__device__ __forceinline__ void tile_pos(int q, int64_t mn0, int64_t k0, int64_t& mn, int64_t& k) {
    if (KC) {
        mn = mn0 + q / (BK / VEC);
        k = k0 + (q % (BK / VEC)) * VEC;
    } else {
        k = k0 + q / (BMN / VEC);
        mn = mn0 + (q % (BMN / VEC)) * VEC;
    }
}

// Loads the k-tile [k0, k0+BK) of one dense operand into registers.
// KC: reduction dim contiguous (X[mn*ld + k]); else X[k*ld + mn].
// With CHECK, out-of-range elements read the operand's first element
// instead, and store_tile replaces them by zero; without it (tiles known to
// lie inside the operand) the address is used as is. The loads stay
// unconditional and their values are not touched until the LDS store, so the
// compiler waits only for the oldest prefetch slot.
template <int BMN, int BK, bool KC, int VEC, int LOADS, int NT, bool CHECK = true>
__device__ __forceinline__ void load_tile(float (&r)[LOADS][VEC], const float* X, int64_t ld,
                                          int64_t mn0, int64_t MN, int64_t k0, int64_t kend,
                                          int tid) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        int64_t mn, k;
        tile_pos<BMN, BK, KC, VEC>(tid + i * NT, mn0, k0, mn, k);
        const float* src = KC ? X + mn * ld + k : X + k * ld + mn;
        if constexpr (CHECK) src = ((mn < MN) & (k < kend)) ? src : X;
        if constexpr (VEC == 4) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(src);
            r[i][0] = v[0];
            r[i][1] = v[1];
            r[i][2] = v[2];
            r[i][3] = v[3];
        } else {
            r[i][0] = *src;
        }
    }
}

// Bit i set: load i of this thread (see tile_pos) lies in the operand's
// [0, MN) rows/columns. Fixed for the whole k loop, so computed once.
template <int BMN, int BK, bool KC, int VEC, int LOADS, int NT>
__device__ __forceinline__ uint32_t tile_mn_bits(int64_t mn0, int64_t MN, int tid) {
    static_assert(LOADS <= 32, "mask bits");
    uint32_t bits = 0;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        int64_t mn, k;
        tile_pos<BMN, BK, KC, VEC>(tid + i * NT, mn0, 0, mn, k);
        bits |= (uint32_t)(mn < MN) << i;
    }
    return bits;
}

// Bit i set: load i of this thread starts at row (column) `one` of the
// operand: the row of ones of a row-of-sums product.
template <int BMN, int BK, bool KC, int VEC, int LOADS, int NT>
__device__ __forceinline__ uint32_t tile_one_bits(int64_t mn0, int64_t one, int tid) {
    uint32_t bits = 0;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        int64_t mn, k;
        tile_pos<BMN, BK, KC, VEC>(tid + i * NT, mn0, 0, mn, k);
        bits |= (uint32_t)(mn == one) << i;
    }
    return bits;
}

// Stores a k-tile to LDS. MASK: zero the elements load_tile read out of
// range (dense operands; gathered operands arrive already zero-filled):
// load i is in range iff bit i of mn_bits is set and its k offset inside the
// tile is below krem = kend - k0.
template <int BMN, int BK, bool KC, int VEC, int LOADS, int S, int NT, bool MASK>
__device__ __forceinline__ void store_tile(float* s, const float (&r)[LOADS][VEC], int tid,
                                           uint32_t mn_bits, int64_t krem, uint32_t one_bits = 0) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int q = tid + i * NT;
        int off, kofs;
        if (KC) {
            off = (q / (BK / VEC)) * S + (q % (BK / VEC)) * VEC;
            kofs = (q % (BK / VEC)) * VEC;
        } else {
            off = (q / (BMN / VEC)) * S + (q % (BMN / VEC)) * VEC;
            kofs = q / (BMN / VEC);
        }
        bool ok = true;
        float one = 0.0f;  // the row of ones (row of sums) in place of zeros
        if constexpr (MASK) {
            ok = ((mn_bits >> i) & 1u) & (kofs < krem);
            one = (((one_bits >> i) & 1u) & (kofs < krem)) ? 1.0f : 0.0f;
        }
        if constexpr (VEC == 4) {
            // a vector along mn starts at the ones row (M % 4 == 0); along k
            // it lies wholly in the row
            *reinterpret_cast<f32x4*>(s + off) =
                ok ? f32x4{r[i][0], r[i][1], r[i][2], r[i][3]}
                   : (KC ? f32x4{one, one, one, one} : f32x4{one, 0.f, 0.f, 0.f});
        } else {
            s[off] = ok ? r[i][0] : one;
        }
    }
}

// Fragment for MFMA steps p = 0..3 of k-group g: element p is the operand
// value at (mn = base + lane%32, k = 8g + 4*(lane/32) + p).
template <bool KC, int S>
__device__ __forceinline__ f32x4 read_frag(const float* s, int mn, int g, int h) {
    if (KC) {
        return *reinterpret_cast<const f32x4*>(s + mn * S + 8 * g + 4 * h);
    } else {
        const float* q = s + (8 * g + 4 * h) * S + mn;
        return f32x4{q[0], q[S], q[2 * S], q[3 * S]};
    }
}

// OP_IM2COL lane mapping: lane <-> column. A workgroup's BN columns are
// spread over consecutive lanes and each thread walks k-rows
// tid / BN + e * (NT / BN), e < BK * BN / NT, so one wave-wide load reads one
// k-row across BN consecutive output pixels (contiguous input for stride 1)
// and the k-row, hence its table entry, is the same for the whole wave. The
// values are kept in the operand's [LOADS][VEC] register slot in flat order
// e = i * VEC + v.
struct Im2colCol {
    int base;  // element offset of (img, channel 0, iy0, ix0) in the tensor
    int iy0, ix0;
};

template <int BN>
__device__ __forceinline__ void im2col_col(Im2colCol& ci, const GemmArgs& p, int64_t n0, int tid) {
    // 32-bit math: the host keeps N and the gathered tensor below 2^31 elements.
    const ConvGeom& g = p.cg;
    const int col = (int)(n0 + tid % BN);
    if (col < (int)p.N) {
        uint32_t img, pp, oy, ox;
        fast_divmod((uint32_t)col, g.div_P, img, pp);
        fast_divmod(pp, g.div_ow, oy, ox);
        ci.iy0 = oy * g.stride - g.pad_h;
        ci.ix0 = ox * g.stride - g.pad_w;
        ci.base = (int)img * (int)(g.C * g.H * g.W) + ci.iy0 * (int)g.W + ci.ix0;
    } else {  // out of range: fails every bounds test of load_im2col
        ci.iy0 = -(1 << 29);
        ci.ix0 = -(1 << 29);
        ci.base = 0;
    }
}

// Decomposition of reduction index k = (ic*kh + i)*kw + j of an OP_IM2COL
// operand: x = offset (ic*H + i)*W + j inside one image, y = i | j << 16.
// Built once per workgroup into LDS for the first kIm2colTable k values, so
// the k-loop does one LDS read per k-row instead of two integer divisions.
constexpr int kIm2colTable = 2048;

__device__ __forceinline__ int2 im2col_k_entry(const ConvGeom& g, int k) {
    const int khkw = g.kh * g.kw;
    const int ic = k / khkw;
    const int rem = k - ic * khkw;
    const int ii = rem / g.kw;
    const int jj = rem - ii * g.kw;
    return make_int2((int)(((int64_t)ic * g.H + ii) * g.W + jj), ii | (jj << 16));
}

// k-tile of an OP_IM2COL operand (k-major, BN columns): element (k, n) is
// image[img(n), ic(k), iy0(n) + i(k), ix0(n) + j(k)] or 0 outside the image.
// `ktab` holds im2col_k_entry for k < kIm2colTable (null: compute it).
template <int BN, int BK, int VEC, int LOADS, int NT>
__device__ __forceinline__ void load_im2col(float (&r)[LOADS][VEC], __amdgpu_buffer_rsrc_t X,
                                            const ConvGeom& g, const Im2colCol& ci,
                                            const int2* ktab, int64_t k0, int64_t kend, int tid) {
    constexpr int RSTEP = NT / BN;  // k-rows covered by one pass of the workgroup
    static_assert(NT % BN == 0 && LOADS * VEC * RSTEP == BK, "im2col lane mapping");
#pragma unroll
    for (int e = 0; e < LOADS * VEC; ++e) {
        const int64_t k = k0 + tid / BN + e * RSTEP;
        const bool kin = k < kend;
        const int2 t = ktab ? ktab[kin ? (int)k : 0] : im2col_k_entry(g, kin ? (int)k : 0);
        const int ii = t.y & 0xffff, jj = t.y >> 16;
        const bool ok = kin & ((unsigned)(ci.iy0 + ii) < (unsigned)g.H) &
                        ((unsigned)(ci.ix0 + jj) < (unsigned)g.W);
        r[e / VEC][e % VEC] = buffer_load1(X, ok ? (ci.base + t.x) * 4 : kOutOfRange);
    }
}

// LDS store of a k-tile loaded by load_im2col ([k][n] layout, row stride S).
template <int BN, int BK, int VEC, int LOADS, int S, int NT>
__device__ __forceinline__ void store_im2col(float* s, const float (&r)[LOADS][VEC], int tid) {
    constexpr int RSTEP = NT / BN;
#pragma unroll
    for (int e = 0; e < LOADS * VEC; ++e)
        s[(tid / BN + e * RSTEP) * S + tid % BN] = r[e / VEC][e % VEC];
}

// k-tile of an OP_NCHW operand (reduction-contiguous, BM channels): element
// (m, k) is T[img(k), m, p(k)] of an NCHW tensor with M channels. With VEC = 4
// the host guarantees P % 4 == 0, so four consecutive columns never straddle
// an image and the load is one aligned 128-bit access.
template <int BM, int BK, int VEC, int LOADS, int NT>
__device__ __forceinline__ void load_nchw(float (&r)[LOADS][VEC], __amdgpu_buffer_rsrc_t X,
                                          const FastDiv& divP, int64_t m0, int64_t M, int64_t k0,
                                          int64_t kend, int tid) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int q = tid + i * NT;
        const int64_t m = m0 + q / (BK / VEC);
        const int64_t k = k0 + (q % (BK / VEC)) * VEC;
        const bool ok = (m < M) & (k < kend);
        uint32_t img, pp;  // the host keeps K = N*P below 2^31
        fast_divmod((uint32_t)(ok ? k : 0), divP, img, pp);
        const int off = ok ? (int)((((int64_t)img * M + m) * divP.d + pp) * 4) : kOutOfRange;
        if constexpr (VEC == 4) {
            const f32x4 v = buffer_load4(X, off);
            r[i][0] = v[0];
            r[i][1] = v[1];
            r[i][2] = v[2];
            r[i][3] = v[3];
        } else {
            r[i][0] = buffer_load1(X, off);
        }
    }
}

// Template parameters of gemm_block / gemm_kernel:
// WPE (kernels): minimum waves per SIMD the register allocation must allow.
// PF: prefetch depth. Global loads for k-tile j go into register slot j % PF
// and are issued PF tiles before tile j is stored to LDS, so each load has
// PF tiles of MFMA work to land in (small tiles need PF > 1 to cover HBM
// latency; the 256x256 tile has enough work per k-tile with PF = 1).
// AMODE / BMODE: OperandMode of A and B (OP_NCHW needs AK, OP_IM2COL needs
// !BKC).
// KS: wave sets splitting each k-tile. KS = 2 runs two waves per output
// sub-block, each reducing half of every k-tile's groups of 8, and adds the
// second set's accumulators to the first's through LDS at the end (fixed
// order): twice the waves per SIMD for tiles that would leave one wave per
// SIMD waiting on its barrier and LDS reads.
// INTERIOR (gemm_tile): the whole output tile lies inside C and the K slice
// is a whole number of k-tiles, so dense operands load and store without
// per-element bounds selects.
//
// gemm_tile computes the output tile at (m0, n0) over K range [kbeg, kend)
// of batch item `batch` (partials: slice `slice`), staging through `smem`
// (2 * STAGE floats); gemm_block finds the tile of workgroup `bid` and picks
// the interior or the bounds-checked form; gemm_kernel runs one GEMM per
// launch, gemm_group_kernel several.
template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, bool AK, bool BKC, int VEC, int PF,
          int AMODE, int BMODE, int KS, bool INTERIOR>
__device__ __forceinline__ void gemm_tile(const GemmArgs& p, float* smem, int64_t m0, int64_t n0,
                                          int64_t kbeg, int64_t kend, int slice, int64_t batch) {
    using C_ = Cfg<BM, BN, BK, WAVES_M, WAVES_N, AK, BKC, VEC, KS>;
    static_assert(AMODE != OP_IM2COL && BMODE != OP_NCHW, "unsupported operand mode");
    static_assert(AMODE != OP_NCHW || AK, "OP_NCHW is a reduction-contiguous operand");
    static_assert(BMODE != OP_IM2COL || !BKC, "OP_IM2COL is a k-major operand");
    constexpr int FM = C_::FM, FN = C_::FN, NT = C_::NT;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int kset = wave / (WAVES_M * WAVES_N);  // k-split wave set
    const int wv = wave - kset * (WAVES_M * WAVES_N);
    const int h = lane >> 5;
    const int l32 = lane & 31;
    const int wm0 = (wv / WAVES_N) * C_::WM;
    const int wn0 = (wv % WAVES_N) * C_::WN;

    const float* A = p.A + batch * p.sA;
    const float* B = p.B + batch * p.sB;

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    float ra[PF][C_::A_LOADS][VEC];
    float rb[PF][C_::B_LOADS][VEC];

    Im2colCol icol;
    __shared__ int2 ktab_s[BMODE == OP_IM2COL ? kIm2colTable : 1];
    const int2* ktab = nullptr;
    if constexpr (BMODE == OP_IM2COL) {
        im2col_col<BN>(icol, p, n0, tid);
        if (p.K <= kIm2colTable) {
            for (int k = tid; k < (int)p.K; k += NT) ktab_s[k] = im2col_k_entry(p.cg, k);
            __syncthreads();
            ktab = ktab_s;
        }
    }
    const __amdgpu_buffer_rsrc_t gather = buffer_rsrc(AMODE == OP_NCHW ? A : B, p.gather_bytes);
    // Main loop: the body is straight-line (tile t is reduced from LDS, tile
    // t + 1 goes from its register slot to the other LDS buffer, tile
    // t + 1 + PF is loaded into the freed slot; loads past the end are
    // masked or skipped), so the compiler can count the loads in flight and
    // wait only for the slot it stores, PF tiles after issuing it. With kPeel it runs
    // while tile t + 1 is real and the last tiles go through the tail below,
    // which loads nothing, stores no padding tile and reduces no padding tile
    // (a single-tile GEMM would otherwise wait one more memory round trip for
    // a padding tile before its epilogue).
    // Wave tiles of at most two accumulators peel the tail; the large tiles
    // keep one straight-line loop over the k-tile count rounded up to PF
    // (padding tiles load as zeros): with 128 accumulator registers the
    // peeled tail costs them spills, and their k loops are long.
    constexpr bool kPeel = FM * FN <= 2;
    // Loads past the slice's end are skipped (not clamped) where no padding
    // tile is reduced: with kPeel, or with one tile in flight.
    constexpr bool kSkipPast = kPeel || PF == 1;
    static_assert(!INTERIOR || (kSkipPast && AMODE == OP_DENSE && BMODE == OP_DENSE),
                  "interior tiles skip the loads past the end");
    auto loadA = [&](float (&r)[C_::A_LOADS][VEC], int64_t k0) {
        if constexpr (AMODE == OP_NCHW)
            load_nchw<BM, BK, VEC, C_::A_LOADS, NT>(r, gather, p.cg.div_P, m0, p.M, k0, kend, tid);
        else if constexpr (INTERIOR)
            load_tile<BM, BK, AK, VEC, C_::A_LOADS, NT, false>(r, A, p.lda, m0, p.M, k0, kend, tid);
        else
            load_tile<BM, BK, AK, VEC, C_::A_LOADS, NT>(r, A, p.lda, m0, p.M, k0, kend, tid);
    };
    const uint32_t a_bits = tile_mn_bits<BM, BK, AK, VEC, C_::A_LOADS, NT>(m0, p.M, tid);
    const uint32_t a_ones =
        p.sum_row ? tile_one_bits<BM, BK, AK, VEC, C_::A_LOADS, NT>(m0, p.M, tid) : 0u;
    const uint32_t b_bits = tile_mn_bits<BN, BK, BKC, VEC, C_::B_LOADS, NT>(n0, p.N, tid);
    auto storeA = [&](float* dst, const float (&r)[C_::A_LOADS][VEC], int64_t k0) {
        if constexpr (INTERIOR)
            store_tile<BM, BK, AK, VEC, C_::A_LOADS, C_::SA, NT, false>(dst, r, tid, a_bits, BK);
        else
            store_tile<BM, BK, AK, VEC, C_::A_LOADS, C_::SA, NT, AMODE == OP_DENSE>(
                dst, r, tid, a_bits, kend - k0, a_ones);
    };
    auto storeB = [&](float* dst, const float (&r)[C_::B_LOADS][VEC], int64_t k0) {
        if constexpr (BMODE == OP_IM2COL)
            store_im2col<BN, BK, VEC, C_::B_LOADS, C_::SB, NT>(dst, r, tid);
        else if constexpr (INTERIOR)
            store_tile<BN, BK, BKC, VEC, C_::B_LOADS, C_::SB, NT, false>(dst, r, tid, b_bits, BK);
        else
            store_tile<BN, BK, BKC, VEC, C_::B_LOADS, C_::SB, NT, true>(dst, r, tid, b_bits,
                                                                         kend - k0);
    };
    auto loadB = [&](float (&r)[C_::B_LOADS][VEC], int64_t k0) {
        if constexpr (BMODE == OP_IM2COL)
            load_im2col<BN, BK, VEC, C_::B_LOADS, NT>(r, gather, p.cg, icol, ktab, k0, kend, tid);
        else if constexpr (INTERIOR)
            load_tile<BN, BK, BKC, VEC, C_::B_LOADS, NT, false>(r, B, p.ldb, n0, p.N, k0, kend, tid);
        else
            load_tile<BN, BK, BKC, VEC, C_::B_LOADS, NT>(r, B, p.ldb, n0, p.N, k0, kend, tid);
    };

    const int ntiles = kend > kbeg ? (int)((kend - kbeg + BK - 1) / BK) : 0;
    const int nloop = kPeel ? ntiles : (ntiles + PF - 1) / PF * PF;
    if (ntiles > 0) {
        loadA(ra[0], kbeg);
        loadB(rb[0], kbeg);
        storeA(smem, ra[0], kbeg);
        storeB(smem + C_::A_ELEMS, rb[0], kbeg);
#pragma unroll
        for (int j = 1; j <= PF; ++j) {
            if ((!kPeel && !kSkipPast) || j < ntiles) {  // uniform
                const int64_t kj = kbeg + (int64_t)j * BK;
                loadA(ra[j % PF], kj);
                loadB(rb[j % PF], kj);
            }
        }
        __syncthreads();
    }

    auto reduce_tile = [&](int t) {
        const float* sA = smem + (t & 1) * C_::STAGE;
        const float* sB = sA + C_::A_ELEMS;
#pragma unroll
        for (int gg = 0; gg < BK / 8 / KS; ++gg) {
            const int g = kset * (BK / 8 / KS) + gg;
            f32x4 af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = read_frag<AK, C_::SA>(sA, wm0 + 32 * i + l32, g, h);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                bf[j] = read_frag<BKC, C_::SB>(sB, wn0 + 32 * j + l32, g, h);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s], bf[j][s],
                                                                        acc[i][j], 0, 0, 0);
        }
    };

    // The loop is unrolled by PF so every register-slot index is a constant.
    int t0 = 0;
    for (; kPeel ? t0 + PF < ntiles : t0 < nloop; t0 += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const int t = t0 + u;
            reduce_tile(t);
            const int slot = (u + 1) % PF;
            float* dA = smem + ((t + 1) & 1) * C_::STAGE;
            const int64_t ks = kbeg + (int64_t)(t + 1) * BK;
            storeA(dA, ra[slot], ks);
            storeB(dA + C_::A_ELEMS, rb[slot], ks);
            const int64_t kn = kbeg + (int64_t)(t + 1 + PF) * BK;
            if (!kSkipPast || kn < kend) {  // uniform
                loadA(ra[slot], kn);
                loadB(rb[slot], kn);
            }
            __syncthreads();
        }
    }

    // Accumulator (i, j) element r of this lane is C[row, col] with
    // row = 32i + 8(r/4) + 4h + r%4, col = 32j + lane%32 inside the wave tile.
    // Every output column gets one base offset and a row stride, so element
    // (row, col) lands at base + row * stride: row-major C has base = col and
    // stride = ldc; NCHW C has base = img*M*P + (col - img*P) and stride = P;
    // split-K partials are row-major [M][N] per slice. The options (bias,
    // ReLU, beta) and the bounds tests are uniform per workgroup and hoisted
    // out of the element loop.
    const bool full = (m0 + BM <= p.M) && (n0 + BN <= p.N);
    const bool plain =
        p.partial != nullptr || (p.epi == NRS_EPI_NONE && p.beta == 0.0f && p.mask == nullptr);
    float* out;
    int64_t stride;
    if (p.partial) {
        out = p.partial + (int64_t)slice * p.mrows * p.N;
        stride = p.N;
    } else {
        out = p.C + batch * p.sC;
        stride = p.nchw_P > 0 ? p.nchw_P : p.ldc;
    }
    int64_t cbase[FN];
    bool colok[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int64_t col = n0 + wn0 + 32 * j + l32;
        colok[j] = col < p.N;
        if (p.partial == nullptr && p.nchw_P > 0) {
            uint32_t img, pc;  // N < 2^31 (checked on the host)
            fast_divmod((uint32_t)col, p.div_nchw, img, pc);
            cbase[j] = (int64_t)img * p.M * p.nchw_P + pc;
        } else {
            cbase[j] = col;
        }
    }
    const int64_t row0 = m0 + wm0 + 4 * h;  // row of element r = 0 of fragment i = 0
    const float beta = p.partial ? 0.0f : p.beta;
    // Small wave tiles load the values an accumulating epilogue adds to
    // before the last k-tiles are reduced, so that round trip overlaps the
    // MFMAs instead of following them (clamped, always-valid addresses;
    // values of lanes that store nothing are unused).
    constexpr bool kEarlyOld = FM * FN <= 2;
    float early[kEarlyOld ? FM : 1][kEarlyOld ? FN : 1][16];
    if constexpr (kEarlyOld) {
        if (beta != 0.0f && kset == 0) {  // uniform
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int64_t row = row0 + 32 * i + 8 * (r >> 2) + (r & 3);
                        const bool ok = colok[j] & (row < p.M);
                        early[i][j][r] = out[ok ? cbase[j] + row * stride : 0];
                    }
        }
    }

    // Tail: the last (at most PF) tiles; only real tiles are stored and reduced.
#pragma unroll
    for (int u = 0; u < PF; ++u) {
        const int t = t0 + u;
        if (kPeel && t < ntiles) {  // uniform
            reduce_tile(t);
            if (t + 1 < ntiles) {
                const int slot = (u + 1) % PF;
                float* dA = smem + ((t + 1) & 1) * C_::STAGE;
                const int64_t ks = kbeg + (int64_t)(t + 1) * BK;
                storeA(dA, ra[slot], ks);
                storeB(dA + C_::A_ELEMS, rb[slot], ks);
                __syncthreads();
            }
        }
    }

    if constexpr (KS > 1) {
        // the other wave sets' accumulators, added to set 0's in set order
        constexpr int WS = WAVES_M * WAVES_N;
        static_assert((KS - 1) * WS * FM * FN * 16 * 64 <= 2 * C_::STAGE, "k-split LDS space");
        __syncthreads();  // every wave is done with the staging buffers
        if (kset > 0) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        smem[((((kset - 1) * WS + wv) * FM + i) * FN + j) * 1024 + r * 64 + lane] =
                            acc[i][j][r];
        }
        __syncthreads();
        if (kset > 0) return;  // uniform; no barrier follows
#pragma unroll
        for (int s2 = 0; s2 < KS - 1; ++s2)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        acc[i][j][r] += smem[(((s2 * WS + wv) * FM + i) * FN + j) * 1024 + r * 64 + lane];
    }

    if (plain && full) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                float* dst = out + cbase[j] + (row0 + 32 * i) * stride;
#pragma unroll
                for (int r = 0; r < 16; ++r) dst[(8 * (r >> 2) + (r & 3)) * stride] = acc[i][j][r];
            }
    } else {
        const bool bias_col = !p.partial && (p.epi & NRS_EPI_BIAS_COL);
        const bool bias_row = !p.partial && (p.epi & NRS_EPI_BIAS_ROW);
        const bool relu = !p.partial && (p.epi & NRS_EPI_RELU);
        const float* mask = p.partial ? nullptr : p.mask;  // row-major C only
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const float bc = (bias_col && colok[j]) ? p.bias[n0 + wn0 + 32 * j + l32] : 0.0f;
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                // The fragment's 16 old values and row biases are loaded
                // before any store, unconditionally from a clamped (always
                // valid) address: a load inside the store's bounds branch
                // would be sunk there by the compiler and cost a round trip
                // per element. Values of lanes that store nothing are unused.
                float old[16], br[16];
                bool live[16];
                if (beta != 0.0f || bias_row || mask) {  // uniform
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int64_t row = row0 + 32 * i + 8 * (r >> 2) + (r & 3);
                        const bool ok = colok[j] & (row < p.M);
                        if constexpr (kEarlyOld)
                            old[r] = beta != 0.0f ? early[i][j][r] : 0.0f;
                        else
                            old[r] = beta != 0.0f ? out[ok ? cbase[j] + row * stride : 0] : 0.0f;
                        br[r] = bias_row ? p.bias[ok ? row : 0] : 0.0f;
                        live[r] = mask ? mask[ok ? cbase[j] + row * stride : 0] > 0.0f : true;
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                // All 16 results first, each in a register of its own
                // (pinned by the empty asm; they overwrite the old values):
                // computed inside each store's bounds branch they would share
                // one temporary, and a store's data register cannot be
                // overwritten before the store has read it, so every store
                // would wait for the one before it.
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float v = acc[i][j][r];
                    if (bias_col) v += bc;
                    if (bias_row) v += br[r];
                    if (relu) v = fmaxf(v, 0.0f);
                    if (mask && !live[r]) v = 0.0f;
                    if (beta != 0.0f) v = v + beta * old[r];
                    old[r] = v;
                    asm volatile("" : "+v"(old[r]));
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int64_t row = row0 + 32 * i + 8 * (r >> 2) + (r & 3);
                    if (colok[j] && row < p.M) out[cbase[j] + row * stride] = old[r];
                }
                if (p.sum_row) {  // uniform; the row of sums, raw
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int64_t row = row0 + 32 * i + 8 * (r >> 2) + (r & 3);
                        if (colok[j] && row == p.M) {
                            if (p.partial) {
                                out[cbase[j] + row * stride] = acc[i][j][r];
                            } else {
                                float* sr = p.sum_row + cbase[j];
                                float v = acc[i][j][r];
                                if (p.sum_beta != 0.0f) v = v + p.sum_beta * *sr;
                                *sr = v;
                            }
                        }
                    }
                }
            }
        }
    }
}

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, bool AK, bool BKC, int VEC, int PF,
          int AMODE, int BMODE, int KS>
__device__ __forceinline__ void gemm_block(const GemmArgs& p, float* smem, int bid, int slice,
                                           int64_t batch) {
    using C_ = Cfg<BM, BN, BK, WAVES_M, WAVES_N, AK, BKC, VEC, KS>;
    int tm, tn;
    tile_coords(p, bid, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int64_t kbeg = (int64_t)slice * p.k_per_slice;
    const int64_t kend = min(p.K, kbeg + p.k_per_slice);
    constexpr bool kInteriorForm =
        AMODE == OP_DENSE && BMODE == OP_DENSE && (C_::FM * C_::FN <= 2 || PF == 1);
    if constexpr (kInteriorForm) {
        if (m0 + BM <= p.M && n0 + BN <= p.N && (kend - kbeg) % BK == 0) {  // uniform
            gemm_tile<BM, BN, BK, WAVES_M, WAVES_N, AK, BKC, VEC, PF, AMODE, BMODE, KS, true>(
                p, smem, m0, n0, kbeg, kend, slice, batch);
            return;
        }
    }
    gemm_tile<BM, BN, BK, WAVES_M, WAVES_N, AK, BKC, VEC, PF, AMODE, BMODE, KS, false>(
        p, smem, m0, n0, kbeg, kend, slice, batch);
}

// Split K over a tile count that is not a multiple of 8: the workgroups are
// dealt to the 8 XCDs round-robin by linear id, so the tiles of one K slice
// would land on different XCDs, each fetching the slice's shared operand panel
// into its own L2 (the 64x576 weight gradient over K = 100352 read its A panel
// nine times). Renumber so that every XCD owns whole slices: logical id =
// (slice, tile), tile fastest, in contiguous runs per XCD (a bijection on the
// grid; each slice still writes its own partial). With a multiple of 8,
// tile_coords already gives each XCD a compact block of every slice's tiles,
// which measured faster on 256-wide weight gradients than whole slices per
// XCD. `lin` is the workgroup's linear id, its low three bits its XCD.
__device__ __forceinline__ void split_coords(int lin, int tiles, int slices, int& bid, int& slice) {
    if (slices > 1 && (tiles & 7) != 0) {
        const int total = tiles * slices;
        const int xcd = lin & 7, per = total >> 3, extra = total & 7;
        const int id = xcd * per + min(xcd, extra) + (lin >> 3);
        slice = id / tiles;
        bid = id - slice * tiles;
    } else {
        slice = lin / tiles;
        bid = lin - slice * tiles;
    }
}

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, bool AK, bool BKC, int VEC, int WPE,
          int PF = 1, int AMODE = OP_DENSE, int BMODE = OP_DENSE, int KS = 1>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N * KS) __attribute__((amdgpu_waves_per_eu(WPE)))
void gemm_kernel(GemmArgs p) {
    using C_ = Cfg<BM, BN, BK, WAVES_M, WAVES_N, AK, BKC, VEC, KS>;
    __shared__ __attribute__((aligned(16))) float smem[2 * C_::STAGE];
    int bid = blockIdx.x, slice = blockIdx.y;
    if (gridDim.y > 1 && (gridDim.x & 7) != 0)
        split_coords(blockIdx.x + blockIdx.y * gridDim.x, gridDim.x, gridDim.y, bid, slice);
    gemm_block<BM, BN, BK, WAVES_M, WAVES_N, AK, BKC, VEC, PF, AMODE, BMODE, KS>(p, smem, bid, slice,
                                                                                 blockIdx.z);
}

// Several independent dense GEMMs in one launch (the products of one
// backward step, or projections of one input): problem q owns workgroups
// [first[q], first[q] + tiles_q * slices[q]) of a 1-D grid, each range
// starting at a multiple of 8 so that a workgroup's XCD is its id within the
// problem modulo 8, as in a launch of its own (ids past a problem's range,
// the padding up to the next multiple of 8, exit at once). The problems'
// workgroups share the CUs, so one problem's load latency, barriers and
// epilogue overlap another's MFMAs; one launch per GEMM leaves each CU a
// single workgroup of small tiles whose waves all stall at the same points.
// Problems of one group launch: the C ABI's groups (NRS_GEMM_GROUP_MAX) and
// the backward of three products sharing their left operand (three input-
// gradient and three weight-gradient products).
constexpr int kGroupMax = 6;
struct GemmGroupArgs {
    GemmArgs prob[kGroupMax];
    int first[kGroupMax];   // first workgroup id of each problem, ascending
    int layout[kGroupMax];  // NRS_NN / NRS_NT / NRS_TN
    int slices[kGroupMax];  // K slices (partials to prob[q].partial when > 1)
    int count;
};

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int WPE, int PF>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) __attribute__((amdgpu_waves_per_eu(WPE)))
void gemm_group_kernel(GemmGroupArgs g) {
    constexpr int kNN = 2 * Cfg<BM, BN, BK, WAVES_M, WAVES_N, true, false, 4>::STAGE;
    constexpr int kNT = 2 * Cfg<BM, BN, BK, WAVES_M, WAVES_N, true, true, 4>::STAGE;
    constexpr int kTN = 2 * Cfg<BM, BN, BK, WAVES_M, WAVES_N, false, false, 4>::STAGE;
    constexpr int kMax = kNN > kNT ? (kNN > kTN ? kNN : kTN) : (kNT > kTN ? kNT : kTN);
    __shared__ __attribute__((aligned(16))) float smem[kMax];
    const int b = blockIdx.x;
    int q = 0;
#pragma unroll
    for (int i = 1; i < kGroupMax; ++i)
        if (i < g.count && b >= g.first[i]) q = i;
    const GemmArgs& p = g.prob[q];
    const int tiles = p.tiles_m * p.tiles_n, slices = g.slices[q];
    const int lin = b - g.first[q];
    if (lin >= tiles * slices) return;  // uniform: padding up to the next problem
    int bid, slice;
    split_coords(lin, tiles, slices, bid, slice);
    switch (g.layout[q]) {
        case NRS_NN:
            gemm_block<BM, BN, BK, WAVES_M, WAVES_N, true, false, 4, PF, OP_DENSE, OP_DENSE, 1>(
                p, smem, bid, slice, 0);
            break;
        case NRS_NT:
            gemm_block<BM, BN, BK, WAVES_M, WAVES_N, true, true, 4, PF, OP_DENSE, OP_DENSE, 1>(
                p, smem, bid, slice, 0);
            break;
        default:
            gemm_block<BM, BN, BK, WAVES_M, WAVES_N, false, false, 4, PF, OP_DENSE, OP_DENSE, 1>(
                p, smem, bid, slice, 0);
            break;
    }
}

// Sums split-K partials and applies the epilogue. A workgroup covers 64
// consecutive outputs with kSplitGroups slice groups: group y sums slices
// [y*per, (y+1)*per) in ascending order, then the group sums are added in
// group order. The order depends only on the slice count, so the result is
// deterministic; every partial read is a coalesced 64-float row segment.
constexpr int kSplitGroups = 16;

__global__ __launch_bounds__(64 * kSplitGroups) void splitk_reduce_kernel(GemmArgs p,
                                                                         int slices) {
    __shared__ float red[kSplitGroups][64];
    const int64_t total = p.mrows * p.N;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int per = (slices + kSplitGroups - 1) / kSplitGroups;
    const int s0 = min(slices, ty * per), s1 = min(slices, s0 + per);
    for (int64_t base = (int64_t)blockIdx.x * 64; base < total; base += (int64_t)gridDim.x * 64) {
        const int64_t e = base + tx;
        float v = 0.0f;
        if (e < total)
            for (int s = s0; s < s1; ++s) v += p.partial[(int64_t)s * total + e];
        red[ty][tx] = v;
        __syncthreads();
        if (ty == 0 && e < total) {
            float r = red[0][tx];
#pragma unroll
            for (int y = 1; y < kSplitGroups; ++y) r += red[y][tx];
            const int64_t row = e / p.N;
            if (row < p.M) {
                epilogue_store(p, p.C, row, e - row * p.N, r);
            } else {  // the row of sums
                float* sr = p.sum_row + (e - row * p.N);
                if (p.sum_beta != 0.0f) r = r + p.sum_beta * *sr;
                *sr = r;
            }
        }
        __syncthreads();
    }
}

// The same sum for row-major outputs of whole float4s (N % 4 == 0, C and the
// partials 16-byte aligned): a thread owns four consecutive outputs and adds
// the slices in slice order with 128-bit loads, eight (then four) slices'
// loads in flight at a time; no LDS, no barrier. Row-major epilogue only.
__global__ __launch_bounds__(256) void splitk_reduce4_kernel(GemmArgs p, int slices) {
    const int64_t total = p.mrows * p.N, total4 = total >> 2;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total4;
         i += (int64_t)gridDim.x * 256) {
        const f32x4* src = reinterpret_cast<const f32x4*>(p.partial) + i;
        const int64_t stride4 = total4;
        f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        int s = 0;
        for (; s + 8 <= slices; s += 8) {
            f32x4 v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = src[(int64_t)(s + j) * stride4];
#pragma unroll
            for (int j = 0; j < 8; ++j) acc = acc + v[j];
        }
        if (s + 4 <= slices) {
            f32x4 v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = src[(int64_t)(s + j) * stride4];
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = acc + v[j];
            s += 4;
        }
        for (; s < slices; ++s) acc = acc + src[(int64_t)s * stride4];
        const int64_t e = i << 2, row = e / p.N, col = e - row * p.N;
        if (row < p.M) {
            if (p.epi & NRS_EPI_BIAS_COL)
                acc = acc + f32x4{p.bias[col], p.bias[col + 1], p.bias[col + 2], p.bias[col + 3]};
            if (p.epi & NRS_EPI_BIAS_ROW) acc = acc + p.bias[row];
            if (p.epi & NRS_EPI_RELU) {
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[j] = fmaxf(acc[j], 0.0f);
            }
            if (p.mask) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (!(p.mask[row * p.ldc + col + j] > 0.0f)) acc[j] = 0.0f;
            }
            f32x4* dst = reinterpret_cast<f32x4*>(p.C + row * p.ldc + col);
            if (p.beta != 0.0f) acc = acc + p.beta * *dst;
            *dst = acc;
        } else {  // the row of sums
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float r = acc[j];
                float* sr = p.sum_row + col + j;
                if (p.sum_beta != 0.0f) r = r + p.sum_beta * *sr;
                *sr = r;
            }
        }
    }
}

}  // namespace nrs
