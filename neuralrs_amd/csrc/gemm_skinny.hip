// Skinny GEMMs, C[M, N] = op(A) . B with M <= 32 and B stored [K][N]: the
// matmul_nn / matmul_tn of src/cuda/graph/matmul.rs:44-94,148-198 when the
// output has at most 32 rows (e.g. the cfg5 sweep's 32 x 8192 x 8192). Such
// a product reads B once and little else, so it is bound by streaming B
// from HBM, not by the matrix cores.
//
// B goes straight from HBM into registers, no LDS: a wave owns a strip of
// 128 columns and one K range. Lane l (c = l % 32, h = l / 32) loads, for
// each group of 8 k values, the four rows k = 8g + 4h + p (p = 0..3) of B at
// columns n0 + 4c .. n0 + 4c + 3 as one 128-bit load each, and the 128-bit A
// fragment of row c at the same four k. Element e of the B vector is the
// lane's value of column block e, so one group feeds 4 steps x 4 blocks of
// v_mfma_f32_32x32x2f32, and block e's output column j is n0 + 4j + e. A
// ring of kSkinnyDepth groups of loads is kept in flight per wave.
// The 8 waves of a workgroup take consecutive K ranges of one strip; their
// partial 32 x 128 blocks meet in LDS and are added in wave order. With one
// K slice per strip the epilogue is applied there; else the blocks are
// split-K partials summed in slice order by the reduce kernel (a fixed
// order either way).
#include <algorithm>

#include "gemm_args.hpp"
#include "gemm_skinny.hpp"

namespace nrs {
namespace {

constexpr int kSkinnyWaves = 8;
constexpr int kSkinnyDepth = 2;     // groups of 8 k values in flight per wave (4, 6, 8 measured slower)
constexpr int kSkinnyCols = 128;    // columns per strip (4 blocks of 32)

struct SkinnyFrag {
    f32x4 b[4];  // rows 8g + 4h + p of B, columns n0 + 4c .. +3
    f32x4 a;     // A row c at k = 8g + 4h .. +3
};

template <bool AK>
__device__ __forceinline__ void skinny_load(SkinnyFrag& f, const GemmArgs& p,
                                            __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb,
                                            int k, int kend, int c, int col) {
    const bool col_ok = col < p.N;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int kk = k + q;
        f.b[q] = buffer_load4(rb, (col_ok & (kk < kend)) ? (int)(((int64_t)kk * p.ldb + col) * 4)
                                                          : kOutOfRange);
    }
    const bool m_ok = c < p.M;
    if constexpr (AK) {  // A [M][K]; kend is a multiple of 4 or K itself (K % 4 == 0)
        f.a = buffer_load4(ra, (m_ok & (k < kend)) ? (int)(((int64_t)c * p.lda + k) * 4)
                                                   : kOutOfRange);
    } else {  // A [K][M]
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int kk = k + q;
            f.a[q] = buffer_load1(ra, (m_ok & (kk < kend)) ? (int)(((int64_t)kk * p.lda + c) * 4)
                                                            : kOutOfRange);
        }
    }
}

template <bool AK>
__global__ __launch_bounds__(64 * kSkinnyWaves) __attribute__((amdgpu_waves_per_eu(2)))
void gemm_skinny_kernel(GemmArgs p, int strips, int slices, int kw) {
    __shared__ float red[kSkinnyWaves][64][64];  // [wave][accumulator float][lane]
    const int lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int strip = (int)blockIdx.x % strips, slice = (int)blockIdx.x / strips;
    const int n0 = strip * kSkinnyCols;
    const int col = n0 + 4 * c;
    const int64_t kb64 = ((int64_t)slice * kSkinnyWaves + w) * kw;
    const int kb = (int)std::min<int64_t>(kb64, p.K);
    const int kend = (int)std::min<int64_t>(kb64 + kw, p.K);
    const auto ra = buffer_rsrc(p.A, p.M * p.K * 4), rb = buffer_rsrc(p.B, p.K * p.N * 4);
    const int groups = (kend - kb + 7) / 8;
    const int padded = (groups + kSkinnyDepth - 1) / kSkinnyDepth * kSkinnyDepth;

    f32x16 acc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = f32x16{};
    SkinnyFrag fr[kSkinnyDepth];
#pragma unroll
    for (int d = 0; d < kSkinnyDepth; ++d)
        skinny_load<AK>(fr[d], p, ra, rb, kb + 8 * d + 4 * h, kend, c, col);
    for (int g = 0; g < padded; g += kSkinnyDepth) {
#pragma unroll
        for (int d = 0; d < kSkinnyDepth; ++d) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[e] = __builtin_amdgcn_mfma_f32_32x32x2f32(fr[d].a[q], fr[d].b[q][e], acc[e],
                                                                 0, 0, 0);
            // refill the slot with the group kDepth ahead (past the range the
            // loads return zero and are never reduced). The scheduling
            // barriers keep slot order: left alone, the compiler gathers all
            // refills and waits for every one before the next MFMAs.
            __builtin_amdgcn_sched_barrier(0);
            skinny_load<AK>(fr[d], p, ra, rb, kb + 8 * (g + d + kSkinnyDepth) + 4 * h, kend, c,
                            col);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[w][e * 16 + r][lane] = acc[e][r];
    __syncthreads();
    // thread t sums, in wave order, accumulator floats (t / 64 + 8 j) of lane t % 64
    const int tl = threadIdx.x & 63, t8 = threadIdx.x >> 6;
    float* out = slices > 1 ? p.partial + (int64_t)slice * p.M * p.N : nullptr;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int r = t8 + 8 * j;  // accumulator float: block r / 16, element r % 16
        float v = 0.0f;
#pragma unroll
        for (int ww = 0; ww < kSkinnyWaves; ++ww) v += red[ww][r][tl];
        const int e = r >> 4, el = r & 15;
        const int row = 8 * (el >> 2) + 4 * (tl >> 5) + (el & 3);
        const int cc = n0 + 4 * (tl & 31) + e;
        if (row < p.M && cc < p.N) {
            if (out)
                out[(int64_t)row * p.N + cc] = v;
            else
                epilogue_store(p, p.C, row, cc, v);
        }
    }
}

bool aligned16(const void* q) { return ((uintptr_t)q & 15) == 0; }

}  // namespace

bool skinny_eligible(const GemmCall& c) {
    if (c.amode != OP_DENSE || c.bmode != OP_DENSE || c.batch != 1 || c.nchw_P != 0 ||
        c.force_slices != 0 || c.sum_row != nullptr || c.layout == NRS_NT)
        return false;
    if (c.M < 1 || c.M > 32 || c.N < 1024 || c.K < 256 || c.N % 4 != 0 || !aligned16(c.B))
        return false;
    if (c.layout == NRS_NN && (c.K % 4 != 0 || !aligned16(c.A))) return false;
    const int64_t limit = int64_t(1) << 31;
    return c.K * c.N * 4 < limit && c.M * c.K * 4 < limit && c.M * c.N * 4 < limit;
}

int skinny_run(const GemmCall& c) {
    const int cus = num_cus();
    const int64_t strips = (c.N + kSkinnyCols - 1) / kSkinnyCols;
    // one workgroup of 8 waves per CU, each wave at least 8 groups of k
    int64_t slices = std::max<int64_t>(1, std::min<int64_t>(cus / std::max<int64_t>(1, strips),
                                                            c.K / (kSkinnyWaves * 64)));
    int64_t kw = (c.K + slices * kSkinnyWaves - 1) / (slices * kSkinnyWaves);
    kw = (kw + 7) / 8 * 8;
    slices = (c.K + kw * kSkinnyWaves - 1) / (kw * kSkinnyWaves);
    NRS_ARG_CHECK(strips * slices <= INT32_MAX && kw <= INT32_MAX, "skinny gemm: grid too large");
    GemmArgs p{};
    p.A = c.A;
    p.B = c.B;
    p.C = c.C;
    p.bias = c.bias;
    p.M = c.M;
    p.N = c.N;
    p.K = c.K;
    p.lda = c.layout == NRS_TN ? c.M : c.K;
    p.ldb = c.N;
    p.ldc = c.N;
    p.mrows = c.M;
    p.beta = c.beta;
    p.epi = c.epi;
    p.mask = c.mask;
    if (slices > 1) {
        const size_t need = sizeof(float) * (size_t)slices * (size_t)(c.M * c.N);
        float* ws;
        if (c.partial_buf) {
            NRS_ARG_CHECK(need <= c.partial_cap,
                          "gemm: split-K partials of %zu bytes exceed the %zu-byte scratch of the "
                          "no-allocation entry point",
                          need, c.partial_cap);
            ws = c.partial_buf;
        } else {
            ws = workspace(need, 0);
            if (!ws) return NRS_ERR_ALLOC;
        }
        p.partial = ws;
    }
    auto fn = c.layout == NRS_NN ? gemm_skinny_kernel<true> : gemm_skinny_kernel<false>;
    hipLaunchKernelGGL(fn, dim3((unsigned)(strips * slices)), dim3(64 * kSkinnyWaves), 0, stream(), p,
                       (int)strips, (int)slices, (int)kw);
    NRS_LAUNCH_CHECK("skinny gemm");
    if (slices > 1) {
        launch_splitk_reduce(p, (int)slices);
        NRS_LAUNCH_CHECK("skinny gemm (split-K reduce)");
    }
    return NRS_OK;
}

}  // namespace nrs
