// Slab-resident convolution: host-side interface (kernel in conv_slab.hip).
//
// out[n, m, oy, ox] = sum_{c,i,j} x[n, c, oy*s - pad_h + i, ox*s - pad_w + j] * Wt(m, c, i, j)
//                     (+ bias[m]) + beta * out
// with Wt(m, c, i, j) = w[m][c][i][j] (forward), or, with `flip`, the
// flipped, channel-transposed w[c][m][kh-1-i][kw-1-j] (the stride-1 input
// gradient of a convolution with weights w, read as a forward convolution of
// the output gradient).
#pragma once

#include "fastdiv.hpp"
#include "nrs_internal.hpp"

namespace nrs {

struct SlabConv {
    const float* x = nullptr;     // NCHW [N][C][H][W]
    const float* w = nullptr;     // [M][C][kh][kw], or [C][M][kh][kw] with flip
    const float* bias = nullptr;  // [M] or null
    float* out = nullptr;         // NCHW [N][M][OH][OW]
    int64_t N = 0;
    int C = 0, H = 0, W = 0, M = 0, kh = 0, kw = 0, stride = 1, pad_h = 0, pad_w = 0;
    int OH = 0, OW = 0;
    bool flip = false;
    float beta = 0.0f;
};

// Launches the convolution when its tiles fit the slab kernel's limits and
// returns NRS_OK; returns kSlabUnsupported (launching nothing) when they do
// not, so the caller can take another lowering. Other codes are errors.
constexpr int kSlabUnsupported = -1;
int slab_conv(const SlabConv& s);

// The same convolution for 3x3 stride-1 layers whose whole padded image
// (rows of at most 16 floats) and weight block fit LDS, with a channel count
// that is a multiple of 16 (conv_img.hip): one staging round per workgroup,
// weights in their natural order (no packing launch). kSlabUnsupported
// (launching nothing) for other shapes.
int img_conv(const SlabConv& s);

// The same convolution by Winograd F(2x2, 3x3) (conv_wino.hip), for "same"
// 3x3 stride-1 layers over images of at most 16x16 with an even width,
// C % 8 == 0 and M % 32 == 0; kSlabUnsupported (launching nothing) for
// other shapes.
int wino_conv(const SlabConv& s);

// The same convolution, chunk-pipelined (conv_pipe.hip), for "same" 3x3
// stride-1 layers over images of at most 14x14 (even width >= 4, whole pixel
// quads) with C % 16 == 0 and M % 32 == 0; kSlabUnsupported (launching
// nothing) for other shapes.
int pipe_conv(const SlabConv& s);

// Weight gradient dw[m][c][i][j] += sum g[n,m,oy,ox] * x[n,c,oy*s-pad+i,ox*s-pad+j]
// and, when db is given, bias gradient db[m] += sum g[n,m,oy,ox], with
// per-image partial sums added in a fixed order. dw is required; returns
// kSlabUnsupported (launching nothing) for shapes outside the kernel's limits.
struct SlabWgrad {
    const float* x = nullptr;  // NCHW [N][C][H][W]
    const float* g = nullptr;  // NCHW [N][M][OH][OW]
    float* dw = nullptr;       // [M][C][kh][kw]
    float* db = nullptr;       // [M] or null
    int64_t N = 0;
    int C = 0, H = 0, W = 0, M = 0, kh = 0, kw = 0, stride = 1, pad = 0, OH = 0, OW = 0;
    float beta = 1.0f;  // dw = gradient + beta * dw (likewise db); 0 reads nothing
};
int slab_wgrad(const SlabWgrad& s);

// The stride-1 input gradient d (a slab convolution with flip) and the
// weight gradient w of one backward call, in one launch of both kernels'
// workgroups (then the weight gradient's partial sum). Returns
// kSlabUnsupported (launching nothing) unless both fit their kernels.
int slab_backward_pair(const SlabConv& d, const SlabWgrad& w);

// The backward of a "same" 3x3 stride-1 layer in one chunk-pipelined launch
// (conv_pipe.hip): the weight and bias gradient w (dw required) and, when d
// is given, the input gradient d (a flipped convolution of w.g), then the
// weight gradient's partial sum. Needs pipe_conv's geometry, C % 32 == 0 and
// M % 64 == 0; returns kSlabUnsupported (launching nothing) otherwise.
// With `lo`, d's input is the 2x2 stride-2 max pool of relu(y), y a "same"
// 3x3 stride-1 layer with lo->c_lo (1 or 2) input channels, and the launch
// also gives that layer's weight and bias gradient (lo->dw required), from
// d's result as the pooled gradient; d->beta must be 0. Both partial sums
// then run in one launch.
struct PipeLower {
    const int32_t* am = nullptr;      // the pool's argmax [N][d->M][H][W]
    const float* pooled = nullptr;    // the pooled values (d's forward input)
    const float* x = nullptr;         // the lower layer's input [N][c_lo][2H][2W]
    float* dw = nullptr;              // [d->M][c_lo][3][3]
    float* db = nullptr;              // [d->M] or null
    int c_lo = 0;
    float beta = 1.0f;                // as SlabWgrad::beta
};
int pipe_backward(const SlabConv* d, const SlabWgrad& w, const PipeLower* lo = nullptr);

// Weight and bias gradient of a convolution with c_in*kh*kw <= 15 taps and at
// most 64 output channels, on the matrix cores (conv_few_taps.hip): dw += and
// db += (either may be null). Returns kSlabUnsupported (launching nothing)
// for shapes outside the kernel's limits.
struct FewTapsWgrad {
    const float* x = nullptr;  // NCHW [N][C][H][W]
    const float* g = nullptr;  // NCHW [N][M][OH][OW]
    float* dw = nullptr;       // [M][C][kh][kw] or null
    float* db = nullptr;       // [M] or null
    int64_t N = 0;
    int C = 0, H = 0, W = 0, M = 0, kh = 0, kw = 0, stride = 1, pad = 0, OH = 0, OW = 0;
    // g absent: the output gradient is the 2x2 (stride 2) max-pool backward of
    // gp [N][M][OH/2][OW/2] with argmax am (flat indices of the conv output),
    // expanded on the fly: g[e] = gp[w] where am[w] == e, else 0
    const float* gp = nullptr;
    const int32_t* am = nullptr;
    // with a ReLU between the conv and the pooling: the pooled values, whose
    // sign gates each window's gradient (null: no ReLU)
    const float* pv = nullptr;
    float beta = 1.0f;  // dw = gradient + beta * dw (likewise db); 0 reads nothing
};
int few_taps_wgrad(const FewTapsWgrad& s);

// dw[m][c][tap] = sum over slices of part_w[slice][m][tap][c] + beta * dw
// (when dw is given) and db[m] = sum over slices of part_b[slice][m] +
// beta * db (when db is given), the slices added in a fixed order; one
// launch. beta 0 reads neither.
int wgrad_partial_sum(float* dw, float* db, const float* part_w, const float* part_b, int slices,
                      int M, int C, int taps, float beta = 1.0f);
// The arguments of one such sum, and two of them in one launch.
struct WgradSumArgs {
    float* dw;
    float* db;
    const float* part_w;
    const float* part_b;
    int slices, M, C, taps;
    float beta;
};
int wgrad_partial_sum_pair(const WgradSumArgs& p0, const WgradSumArgs& p1);

}  // namespace nrs
