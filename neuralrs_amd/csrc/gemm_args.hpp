// Kernel arguments of one GEMM problem and its element epilogue, shared by
// the tiled core (gemm_kernel.hpp), the skinny kernel and the split-K reduce.
#pragma once

#include "buffer_ops.hpp"
#include "gemm_call.hpp"

namespace nrs {

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
    ConvGeom cg;         // operand geometry for the implicit-GEMM operand modes
    int64_t gather_bytes;  // size of the gathered operand's tensor (<= 2 GiB)
    FastDiv div_nchw;      // divider for nchw_P
    // Row of sums: non-null adds output row M, whose A row is all ones, so it
    // holds sum_k op(B)[k][col]; it goes to sum_row[col] (+ sum_beta * old)
    // instead of C (split-K partials carry it as their row M).
    float* sum_row;
    float sum_beta;
    int64_t mrows;  // rows of the product: M, or M + 1 with a row of sums
    // non-null: row-major [M][ldc]; v = 0 where mask <= 0 (before beta)
    const float* mask;
};



// Sums `slices` split-K partial tiles of p (p.partial, [slices][mrows][N]) in
// slice order and applies p's epilogue (defined with the GEMM host code).
void launch_splitk_reduce(GemmArgs p, int slices);

// v (+bias) (relu) (+ beta*C_old), stored at row-major or NCHW position.
__device__ __forceinline__ void epilogue_store(const GemmArgs& p, float* C, int64_t row,
                                               int64_t col, float v) {
    if (p.epi & NRS_EPI_BIAS_COL) v += p.bias[col];
    if (p.epi & NRS_EPI_BIAS_ROW) v += p.bias[row];
    if (p.epi & NRS_EPI_RELU) v = fmaxf(v, 0.0f);
    int64_t idx;
    if (p.nchw_P > 0) {
        uint32_t img, pc;
        fast_divmod((uint32_t)col, p.div_nchw, img, pc);
        idx = ((int64_t)img * p.M + row) * p.nchw_P + pc;
    } else {
        idx = row * p.ldc + col;
        if (p.mask && !(p.mask[idx] > 0.0f)) v = 0.0f;
    }
    if (p.beta != 0.0f) v = v + p.beta * C[idx];
    C[idx] = v;
}

}  // namespace nrs
