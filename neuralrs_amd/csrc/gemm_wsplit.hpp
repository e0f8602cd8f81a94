// Short GEMMs (gemm_wsplit.hip): products of few output tiles, each 16x16
// block of C reduced by the waves of one workgroup, in one launch.
#pragma once

#include "gemm_call.hpp"

namespace nrs {

constexpr int kWsMax = 4;                 // problems per launch
constexpr int64_t kWsMaxK = 1 << 24;      // longest reduction taken
constexpr int kWsAutoMaxK = 2048;         // longest reduction the planner sends here
constexpr int kWsMask = 1 << 8;           // epilogue: v = 0 where mask <= 0
constexpr int kWsCe = 1 << 9;             // epilogue: fused cross-entropy seed

struct WsProblem {
    const float* A;
    const float* B;
    float* C;
    const float* bias;
    const float* mask;    // kWsMask: [M][N] like C
    float* aux;           // kWsCe: the gradient of the logits [M][N]
    const float* target;  // kWsCe: one-hot target [M][N]
    float* sum_row;       // row of sums (see GemmCall::sum_row)
    int64_t lda, ldb, ldc, a_bytes, b_bytes;
    int M, N, K, layout, mode, epi, tiles_n, first;
    float beta, sum_beta, inv_batch;
};

struct WsArgs {
    WsProblem prob[kWsMax];
    int count;
};

// Epilogue operands beyond GemmCall's: the cross-entropy seed's output and
// target (N <= 16, no beta, no row of sums).
struct WsExtra {
    float* ce_grad = nullptr;
    const float* ce_target = nullptr;
};

// Whether the short-GEMM kernel can take c (automatic: and whether the
// planner should send it there rather than to the tiled core).
bool wsplit_eligible(const GemmCall& c, bool automatic);
// One launch of `count` problems (each eligible, outputs independent of the
// other problems' operands); extra may be null.
int wsplit_run(const GemmCall* calls, int count, const WsExtra* extra);

}  // namespace nrs
