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

#include "nrs_internal.hpp"

namespace nrs {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct GemmArgs {
    const float* A;
    const float* B;
    float* C;
    const float* bias;
    float* partial;  // split-K partials [slices][M][N]; null = apply epilogue directly
    int64_t M, N, K;
    int64_t lda, ldb, ldc;
    int64_t sA, sB, sC;  // batch strides in elements
    int64_t k_per_slice; // multiple of BK
    int tiles_m, tiles_n;
    int group_m;         // tile-swizzle group height
    float beta;
    int epi;
    int64_t nchw_P;      // > 0: C is NCHW [N_img][M][P] with column = img*P + p
};

// v (+bias) (relu) (+ beta*C_old), stored at row-major or NCHW position.
__device__ __forceinline__ void epilogue_store(const GemmArgs& p, float* C, int64_t row,
                                               int64_t col, float v) {
    if (p.epi & NRS_EPI_BIAS_COL) v += p.bias[col];
    if (p.epi & NRS_EPI_BIAS_ROW) v += p.bias[row];
    if (p.epi & NRS_EPI_RELU) v = fmaxf(v, 0.0f);
    int64_t idx;
    if (p.nchw_P > 0) {
        int64_t img = col / p.nchw_P;
        idx = (img * p.M + row) * p.nchw_P + (col - img * p.nchw_P);
    } else {
        idx = row * p.ldc + col;
    }
    if (p.beta != 0.0f) v = v + p.beta * C[idx];
    C[idx] = v;
}

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

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, bool AK, bool BKC, int VEC>
struct Cfg {
    static constexpr int NT = 64 * WAVES_M * WAVES_N;
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
    static_assert(BK % 8 == 0, "BK must be a multiple of 8");
    static_assert(A_LOADS >= 1 && B_LOADS >= 1, "tile too small for the thread count");
    static_assert(A_LOADS * VEC * NT == BM * BK && B_LOADS * VEC * NT == BN * BK, "load split");
    static_assert(2 * STAGE * 4 <= 160 * 1024, "LDS budget");
};

// Loads the k-tile [k0, k0+BK) of one operand into registers.
// KC: reduction dim contiguous (X[mn*ld + k]); else X[k*ld + mn].
template <int BMN, int BK, bool KC, int VEC, int LOADS, int NT>
__device__ __forceinline__ void load_tile(float (&r)[LOADS][VEC], const float* X, int64_t ld,
                                          int64_t mn0, int64_t MN, int64_t k0, int64_t kend,
                                          int tid) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int q = tid + i * NT;
        int64_t mn, k;
        if (KC) {
            mn = mn0 + q / (BK / VEC);
            k = k0 + (q % (BK / VEC)) * VEC;
        } else {
            k = k0 + q / (BMN / VEC);
            mn = mn0 + (q % (BMN / VEC)) * VEC;
        }
        const bool ok = (mn < MN) && (k < kend);
        const float* src = KC ? X + mn * ld + k : X + k * ld + mn;
        if constexpr (VEC == 4) {
            const f32x4 v = ok ? *reinterpret_cast<const f32x4*>(src) : f32x4{0.f, 0.f, 0.f, 0.f};
            r[i][0] = v[0];
            r[i][1] = v[1];
            r[i][2] = v[2];
            r[i][3] = v[3];
        } else {
            r[i][0] = ok ? *src : 0.0f;
        }
    }
}

template <int BMN, int BK, bool KC, int VEC, int LOADS, int S, int NT>
__device__ __forceinline__ void store_tile(float* s, const float (&r)[LOADS][VEC], int tid) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int q = tid + i * NT;
        int off;
        if (KC)
            off = (q / (BK / VEC)) * S + (q % (BK / VEC)) * VEC;
        else
            off = (q / (BMN / VEC)) * S + (q % (BMN / VEC)) * VEC;
        if constexpr (VEC == 4) {
            *reinterpret_cast<f32x4*>(s + off) = f32x4{r[i][0], r[i][1], r[i][2], r[i][3]};
        } else {
            s[off] = r[i][0];
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

// WPE: minimum waves per SIMD the register allocation must allow.
// PF: prefetch depth. Global loads for k-tile j go into register slot j % PF
// and are issued PF tiles before tile j is stored to LDS, so each load has
// PF tiles of MFMA work to land in (small tiles need PF > 1 to cover HBM
// latency; the 256x256 tile has enough work per k-tile with PF = 1).
template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, bool AK, bool BKC, int VEC, int WPE,
          int PF = 1>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) __attribute__((amdgpu_waves_per_eu(WPE)))
void gemm_kernel(GemmArgs p) {
    using C_ = Cfg<BM, BN, BK, WAVES_M, WAVES_N, AK, BKC, VEC>;
    constexpr int FM = C_::FM, FN = C_::FN, NT = C_::NT;
    __shared__ __attribute__((aligned(16))) float smem[2 * C_::STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int h = lane >> 5;
    const int l32 = lane & 31;
    const int wm0 = (wave / WAVES_N) * C_::WM;
    const int wn0 = (wave % WAVES_N) * C_::WN;

    int tm, tn;
    tile_coords(p, blockIdx.x, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int slice = blockIdx.y;
    const int64_t batch = blockIdx.z;

    const float* A = p.A + batch * p.sA;
    const float* B = p.B + batch * p.sB;
    const int64_t kbeg = (int64_t)slice * p.k_per_slice;
    const int64_t kend = min(p.K, kbeg + p.k_per_slice);

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    float ra[PF][C_::A_LOADS][VEC];
    float rb[PF][C_::B_LOADS][VEC];

    const int ntiles = kend > kbeg ? (int)((kend - kbeg + BK - 1) / BK) : 0;
    if (ntiles > 0) {
        load_tile<BM, BK, AK, VEC, C_::A_LOADS, NT>(ra[0], A, p.lda, m0, p.M, kbeg, kend, tid);
        load_tile<BN, BK, BKC, VEC, C_::B_LOADS, NT>(rb[0], B, p.ldb, n0, p.N, kbeg, kend, tid);
        store_tile<BM, BK, AK, VEC, C_::A_LOADS, C_::SA, NT>(smem, ra[0], tid);
        store_tile<BN, BK, BKC, VEC, C_::B_LOADS, C_::SB, NT>(smem + C_::A_ELEMS, rb[0], tid);
#pragma unroll
        for (int j = 1; j <= PF; ++j) {
            if (j < ntiles) {
                const int64_t kj = kbeg + (int64_t)j * BK;
                load_tile<BM, BK, AK, VEC, C_::A_LOADS, NT>(ra[j % PF], A, p.lda, m0, p.M, kj, kend, tid);
                load_tile<BN, BK, BKC, VEC, C_::B_LOADS, NT>(rb[j % PF], B, p.ldb, n0, p.N, kj, kend, tid);
            }
        }
        __syncthreads();
    }

    // The loop is unrolled by PF so every register-slot index is a constant.
    for (int t0 = 0; t0 < ntiles; t0 += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const int t = t0 + u;
            if (t < ntiles) {
                const float* sA = smem + (t & 1) * C_::STAGE;
                const float* sB = sA + C_::A_ELEMS;
#pragma unroll
                for (int g = 0; g < BK / 8; ++g) {
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
                if (t + 1 < ntiles) {
                    const int slot = (u + 1) % PF;
                    float* dA = smem + ((t + 1) & 1) * C_::STAGE;
                    store_tile<BM, BK, AK, VEC, C_::A_LOADS, C_::SA, NT>(dA, ra[slot], tid);
                    store_tile<BN, BK, BKC, VEC, C_::B_LOADS, C_::SB, NT>(dA + C_::A_ELEMS, rb[slot], tid);
                    if (t + 1 + PF < ntiles) {
                        const int64_t kn = kbeg + (int64_t)(t + 1 + PF) * BK;
                        load_tile<BM, BK, AK, VEC, C_::A_LOADS, NT>(ra[slot], A, p.lda, m0, p.M, kn, kend, tid);
                        load_tile<BN, BK, BKC, VEC, C_::B_LOADS, NT>(rb[slot], B, p.ldb, n0, p.N, kn, kend, tid);
                    }
                }
                __syncthreads();
            }
        }
    }

    // Accumulator (i, j) element r of this lane is C[row, col] with
    // row = 32i + 8(r/4) + 4h + r%4, col = 32j + lane%32 inside the wave tile.
    if (p.partial) {
        float* P = p.partial + (int64_t)slice * p.M * p.N;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int64_t col = n0 + wn0 + 32 * j + l32;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int64_t row = m0 + wm0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (row < p.M && col < p.N) P[row * p.N + col] = acc[i][j][r];
                }
            }
    } else {
        float* C = p.C + batch * p.sC;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int64_t col = n0 + wn0 + 32 * j + l32;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int64_t row = m0 + wm0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (row < p.M && col < p.N) epilogue_store(p, C, row, col, acc[i][j][r]);
                }
            }
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
    const int64_t total = p.M * p.N;
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
            epilogue_store(p, p.C, row, e - row * p.N, r);
        }
        __syncthreads();
    }
}

}  // namespace nrs
