// Host-facing description of one GEMM launch, shared by the GEMM entry
// points (gemm.hip) and the convolution lowering (conv.hip).
#pragma once

#include "fastdiv.hpp"
#include "nrs_internal.hpp"

namespace nrs {

// Geometry of an implicit-GEMM convolution operand: the NCHW image an
// operand is read from and the convolution that maps it to GEMM columns
// (column = img * P + oy * ow + ox, P = oh * ow).
struct ConvGeom {
    int64_t C, H, W;            // channels and spatial size of the image read
    int kh, kw, stride, pad_h, pad_w;
    int64_t oh, ow, P;          // output spatial size of the convolution
    FastDiv div_P, div_ow;      // dividers for P and ow (set by gemm_run)
};

// Operand modes of the GEMM kernel:
//   OP_DENSE   row-major matrix (leading dimension from the layout);
//   OP_IM2COL  B only, k-major [k = (ic*kh + i)*kw + j][n = column]: the
//              im2col matrix of the NCHW image `cg`, gathered on the fly with
//              zero padding (the column matrix of src/cuda/nn/conv.rs:27-58
//              without materialising it);
//   OP_NCHW    A only, reduction-contiguous [m = channel][k = column]: an NCHW
//              tensor with M channels and cg.P pixels per image, read in place
//              as the [M, N*P] operand (the out2mm reorder of
//              src/cuda/nn/conv.rs:94-108 without materialising it).
enum OperandMode { OP_DENSE = 0, OP_IM2COL = 1, OP_NCHW = 2 };

// C[b] = epi(op(A[b]) op(B[b])) + beta * C[b], b < batch.
struct GemmCall {
    int layout = NRS_NN;
    float* C = nullptr;
    const float* A = nullptr;
    const float* B = nullptr;
    int64_t M = 0, N = 0, K = 0, batch = 1;
    int64_t sA = 0, sB = 0, sC = 0;  // batch strides in elements
    float beta = 0.0f;
    const float* bias = nullptr;
    int epi = NRS_EPI_NONE;
    int64_t nchw_P = 0;       // > 0: C is stored NCHW [img][M][nchw_P]
    bool allow_split = true;  // split-K allowed (batch == 1, row-major C only)
    int force_slices = 0;
    int amode = OP_DENSE, bmode = OP_DENSE;
    ConvGeom cg{};
    int64_t gather_bytes = 0;  // bytes of the gathered (non-dense) operand's tensor
    // Caller-provided split-K partials buffer (no allocation): used instead of
    // the library's scratch slot when set; a plan whose partials exceed
    // partial_cap bytes is rejected.
    float* partial_buf = nullptr;
    size_t partial_cap = 0;
    // Row of sums (dense, batch 1, no epilogue): non-null also computes
    // sum_row[c] = sum_k op(B)[k][c] + sum_beta * sum_row[c] as an extra
    // output row whose A row is all ones (a Linear's bias gradient beside
    // its weight gradient).
    float* sum_row = nullptr;
    float sum_beta = 0.0f;
    // ReLU-backward mask (dense, unbatched, row-major C): output elements
    // whose mask[row][col] is not > 0 are 0 before beta * old is added.
    const float* mask = nullptr;
};

int gemm_run(const GemmCall& c);
// Up to NRS_GEMM_GROUP_MAX dense calls in one launch of the group kernel when they
// qualify (see nrs_gemm_group), else gemm_run on each in order.
int gemm_group_run(const GemmCall* calls, int count);

// nrs_matmul_shared_lhs_backward: the backward of count <= 3 products
// x . W_i, the input-gradient parts added in index order.
int shared_lhs_backward(float* dx, float* const* dw, const float* const* g, const float* x,
                        const float* const* w, int count, int64_t rows, int64_t inner,
                        int64_t cols, float beta_x, const float* beta_w);

// nrs_linear_backward (dx = grad . w^T masked where mask <= 0 when mask is
// given, dw = x^T . grad, db = column sums of grad; each + beta * old).
int linear_backward(float* dx, float* dw, float* db, const float* grad, const float* x,
                    const float* w, const float* mask, int64_t batch, int64_t in_f, int64_t out_f,
                    float beta_x, float beta_w, float beta_b);

// Whether byte ranges [a, a + abytes) and [b, b + bbytes) share memory (an
// empty range overlaps nothing).
bool overlaps(const void* a, size_t abytes, const void* b, size_t bbytes);

// A further operand of a call (e.g. an epilogue's mask) for the overlap check.
struct OperandRange {
    const void* p;
    size_t bytes;
};
// True when no call's outputs (C, row of sums) overlap another call's outputs
// or operands (A, B, bias, extra[j] of call j when extra is non-null).
bool outputs_independent(const GemmCall* calls, int count, const OperandRange* extra);

// Batched products of small dense items (M, N, K <= 128, 16-byte aligned
// items, K or the transposed operand's rows in whole float4s), without
// epilogue; returns kBmmUnsupported (launching nothing) for any other call.
constexpr int kBmmUnsupported = -1;
int bmm_small(const GemmCall& c);
// Two gradient products of one bmm (ga: NT or NN, gb: TN) in one launch when
// both qualify for bmm_small; kBmmUnsupported (launching nothing) otherwise.
int bmm_small_pair(const GemmCall& ga, const GemmCall& gb);

// The GemmCall of one bmm product over contiguous items (no split-K).
GemmCall bmm_call(int layout, float* C, const float* A, const float* B, int64_t batch,
                  int64_t rows, int64_t cols, int64_t inner, float beta);

}  // namespace nrs
