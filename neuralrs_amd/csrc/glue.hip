// Glue kernels around the GEMMs of the attention and Linear paths, so the
// resident ops that feed bmm/matmul stay on the device:
//   transpose2d      src/cuda/graph/transpose.rs:10-24   (batched 2-D transpose)
//   vscale           src/cuda/graph/scale.rs:10-20       (x * s)
//   softmax fwd/bwd  src/cuda/graph/softmax.rs:11-35     (last dim)
//   vrelu/relu_grad  src/cuda/graph/relu.rs:16-28
//   slice_fwd/bwd    src/cuda/graph/slice_cols.rs:12-29  (column slice)
//   concat_write/read src/cuda/graph/concat_cols.rs:12-29 (column concat)
//   and the per-head slice/concat loops of MultiHeadAttention
//   (src/cuda/nn/multihead.rs:43-52,72-81) as one launch each
// Every backward entry point takes beta: gin = local + beta * gin, so beta = 1
// fuses the accumulate_into() the reference launches after each of them
// (src/cuda/runtime.rs:67-83).
#include <algorithm>

#include "nrs_internal.hpp"

namespace nrs {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

inline unsigned grid_for(int64_t n) {
    int64_t b = (n + 255) / 256;
    int64_t cap = 16 * (int64_t)num_cus();
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(b, cap));
}

// out[b, j, i] = in[b, i, j] through a 32x33 LDS tile: reads and writes are
// both row-contiguous (coalesced), the odd stride keeps the column reads of
// the tile free of bank conflicts.
__global__ __launch_bounds__(256) void transpose_kernel(float* __restrict__ out,
                                                        const float* __restrict__ in, int64_t R,
                                                        int64_t C, int64_t tiles_r,
                                                        int64_t tiles_c) {
    __shared__ float t[32][33];
    const int64_t per_batch = tiles_r * tiles_c;
    const int64_t b = blockIdx.x / per_batch;
    const int64_t rem = blockIdx.x - b * per_batch;
    const int64_t r0 = (rem / tiles_c) * 32, c0 = (rem % tiles_c) * 32;
    const float* src = in + b * R * C;
    float* dst = out + b * R * C;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int i = ty; i < 32; i += 8) {
        const int64_t r = r0 + i, c = c0 + tx;
        if (r < R && c < C) t[i][tx] = src[r * C + c];
    }
    __syncthreads();
    for (int i = ty; i < 32; i += 8) {
        const int64_t c = c0 + i, r = r0 + tx;  // out row c, column r
        if (r < R && c < C) dst[c * R + r] = t[tx][i];
    }
}

__global__ __launch_bounds__(256) void scale_kernel(float* out, const float* x, float s,
                                                    int64_t n, float beta) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) {
        float v = x[i] * s;
        if (beta != 0.0f) v = v + beta * out[i];
        out[i] = v;
    }
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// One wave per row of softmax(scale * x): max, sum of exp(t - max), then
// exp(t - max) / sum, with t = x * scale rounded to f32 first, as vscale
// followed by softmax_forward computes it. Lane l takes elements l, l + 64,
// ... in that order. PER > 0: the row (width <= 64 * PER) stays in registers
// and is read once. PER = 0: any width, re-read per pass. Both orders of
// summation are the same, so every form gives the same bits.
template <int PER>
__global__ __launch_bounds__(256) void softmax_fwd_kernel(float* __restrict__ out,
                                                          const float* __restrict__ in,
                                                          int64_t rows, int64_t width,
                                                          float scale) {
    // x * scale is rounded before the max subtraction, as when vscale runs
    // first: no multiply-add contraction here
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t waves = (int64_t)gridDim.x * 4;
    for (int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); r < rows; r += waves) {
        const float* x = in + r * width;
        float* y = out + r * width;
        if constexpr (PER > 0) {
            float v[PER];
            float m = -INFINITY;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int f = lane + 64 * i;
                v[i] = f < width ? x[f] * scale : -INFINITY;
                m = fmaxf(m, v[i]);
            }
            m = wave_max(m);
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                v[i] = lane + 64 * i < width ? expf(v[i] - m) : 0.0f;
                s += v[i];
            }
            s = wave_sum(s);
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int f = lane + 64 * i;
                if (f < width) y[f] = v[i] / s;
            }
        } else {
            float m = -INFINITY;
            for (int64_t f = lane; f < width; f += 64) m = fmaxf(m, x[f] * scale);
            m = wave_max(m);
            float s = 0.0f;
            for (int64_t f = lane; f < width; f += 64) s += expf(x[f] * scale - m);
            s = wave_sum(s);
            for (int64_t f = lane; f < width; f += 64) y[f] = expf(x[f] * scale - m) / s;
        }
    }
}

// gin = (y * (g - sum(y * g))) * scale + beta * gin, with y the forward
// output: softmax_backward followed by scale_grad in one pass (scale 1 is
// softmax_backward alone). Same lane order and register forms as above.
template <int PER>
__global__ __launch_bounds__(256) void softmax_bwd_kernel(float* __restrict__ gin,
                                                          const float* __restrict__ y,
                                                          const float* __restrict__ g,
                                                          int64_t rows, int64_t width,
                                                          float scale, float beta) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t waves = (int64_t)gridDim.x * 4;
    for (int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); r < rows; r += waves) {
        const float* yr = y + r * width;
        const float* gr = g + r * width;
        float* o = gin + r * width;
        if constexpr (PER > 0) {
            float yv[PER], gv[PER], ov[PER];
            float d = 0.0f;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int f = lane + 64 * i;
                const bool in = f < width;
                yv[i] = in ? yr[f] : 0.0f;
                gv[i] = in ? gr[f] : 0.0f;
                ov[i] = (in && beta != 0.0f) ? o[f] : 0.0f;
                d += yv[i] * gv[i];
            }
            d = wave_sum(d);
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int f = lane + 64 * i;
                float v = yv[i] * (gv[i] - d);
                if (scale != 1.0f) v = v * scale;
                if (beta != 0.0f) v = v + beta * ov[i];
                if (f < width) o[f] = v;
            }
        } else {
            float d = 0.0f;
            for (int64_t f = lane; f < width; f += 64) d += yr[f] * gr[f];
            d = wave_sum(d);
            for (int64_t f = lane; f < width; f += 64) {
                float v = yr[f] * (gr[f] - d);
                if (scale != 1.0f) v = v * scale;
                if (beta != 0.0f) v = v + beta * o[f];
                o[f] = v;
            }
        }
    }
}

__global__ __launch_bounds__(256) void relu_fwd_kernel(float* out, const float* x, int64_t n) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step)
        out[i] = x[i] > 0.0f ? x[i] : 0.0f;
}

__global__ __launch_bounds__(256) void relu_bwd_kernel(float* gin, const float* grad,
                                                       const float* x, int64_t n, float beta) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) {
        float v = x[i] > 0.0f ? grad[i] : 0.0f;
        if (beta != 0.0f) v = v + beta * gin[i];
        gin[i] = v;
    }
}

// dst[h][r][c] = src[h][r][c] + beta * dst[h][r][c] over heads x rows x
// width, each operand addressed through its own head and row strides
// (floats). V = 4: 128-bit accesses (width, strides and both base addresses
// are multiples of 4 floats); V = 1 otherwise.
struct StridedCopy {
    float* dst;
    const float* src;
    int64_t heads, rows, width;
    int64_t d_h, d_r, s_h, s_r;
    float beta;
};

template <int V>
__global__ __launch_bounds__(256) void strided_copy_kernel(StridedCopy a) {
    const int64_t wv = a.width / V, total = a.heads * a.rows * wv;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += step) {
        const int64_t item = t / wv, c = (t - item * wv) * V;
        const int64_t h = item / a.rows, r = item - h * a.rows;
        const float* sp = a.src + h * a.s_h + r * a.s_r + c;
        float* dp = a.dst + h * a.d_h + r * a.d_r + c;
        if constexpr (V == 4) {
            f32x4 v = *reinterpret_cast<const f32x4*>(sp);
            if (a.beta != 0.0f) v = v + a.beta * *reinterpret_cast<const f32x4*>(dp);
            *reinterpret_cast<f32x4*>(dp) = v;
        } else {
            float v = *sp;
            if (a.beta != 0.0f) v = v + a.beta * *dp;
            *dp = v;
        }
    }
}

int strided_copy(const StridedCopy& a, const char* what) {
    const int64_t n = a.heads * a.rows * a.width;
    if (n == 0) return NRS_OK;
    const bool v4 = a.width % 4 == 0 && a.d_h % 4 == 0 && a.d_r % 4 == 0 && a.s_h % 4 == 0 &&
                    a.s_r % 4 == 0 && ((uintptr_t)a.dst & 15) == 0 && ((uintptr_t)a.src & 15) == 0;
    if (v4)
        hipLaunchKernelGGL(strided_copy_kernel<4>, dim3(grid_for(n / 4)), dim3(256), 0, stream(),
                           a);
    else
        hipLaunchKernelGGL(strided_copy_kernel<1>, dim3(grid_for(n)), dim3(256), 0, stream(), a);
    NRS_LAUNCH_CHECK(what);
    return NRS_OK;
}

inline unsigned rows_grid(int64_t rows) {
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>((rows + 3) / 4, 32 * (int64_t)num_cus()));
}

}  // namespace
}  // namespace nrs

namespace nrs {
namespace {

// One column block of a rows x total_cols matrix against a dense rows x width
// one. into_wide: the block receives (dst = wide + col, row stride
// total_cols); otherwise the dense matrix does.
int nrs_slice_cols_backward_impl(float* dst, const float* src, int64_t rows, int64_t total_cols,
                                 int64_t col, int64_t width, float beta, bool into_wide) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(rows >= 0 && width >= 0 && col >= 0 && total_cols >= 0 &&
                      col + width <= total_cols,
                  "column slice: columns [%lld, %lld) outside %lld", (long long)col,
                  (long long)(col + width), (long long)total_cols);
    if (rows == 0 || width == 0) return NRS_OK;
    NRS_ARG_CHECK(dst && src && (const float*)dst != src, "column slice: null or aliased pointer");
    StridedCopy a{};
    a.heads = 1;
    a.rows = rows;
    a.width = width;
    a.beta = beta;
    if (into_wide) {
        a.dst = dst + col;
        a.d_r = total_cols;
        a.src = src;
        a.s_r = width;
    } else {
        a.dst = dst;
        a.d_r = width;
        a.src = src + col;
        a.s_r = total_cols;
    }
    return strided_copy(a, into_wide ? "column slice (into the wide matrix)" : "column slice");
}

// [rows][heads * width] <-> [heads][rows][width]
int nrs_heads_impl(float* dst, const float* src, int64_t rows, int64_t heads, int64_t width,
                   float beta, bool split) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(rows >= 0 && heads >= 0 && width >= 0, "heads: negative size");
    if (rows == 0 || heads == 0 || width == 0) return NRS_OK;
    NRS_ARG_CHECK(dst && src && (const float*)dst != src, "heads: null or aliased pointer");
    StridedCopy a{};
    a.dst = dst;
    a.src = src;
    a.heads = heads;
    a.rows = rows;
    a.width = width;
    a.beta = beta;
    const int64_t dense_h = rows * width, dense_r = width, wide_h = width, wide_r = heads * width;
    a.d_h = split ? dense_h : wide_h;
    a.d_r = split ? dense_r : wide_r;
    a.s_h = split ? wide_h : dense_h;
    a.s_r = split ? wide_r : dense_r;
    return strided_copy(a, split ? "split heads" : "merge heads");
}

}  // namespace
}  // namespace nrs

using nrs::nrs_heads_impl;
using nrs::nrs_slice_cols_backward_impl;

extern "C" {

int nrs_transpose(float* out, const float* in, int64_t batch, int64_t rows, int64_t cols) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(batch >= 0 && rows >= 0 && cols >= 0, "transpose: negative size");
    if (batch == 0 || rows == 0 || cols == 0) return NRS_OK;
    NRS_ARG_CHECK(out && in && out != in, "transpose: null or aliased pointer");
    const int64_t tr = (rows + 31) / 32, tc = (cols + 31) / 32;
    const int64_t blocks = batch * tr * tc;
    NRS_ARG_CHECK(blocks <= INT32_MAX, "transpose: too many tiles");
    hipLaunchKernelGGL(nrs::transpose_kernel, dim3((unsigned)blocks), dim3(256), 0, nrs::stream(),
                       out, in, rows, cols, tr, tc);
    NRS_LAUNCH_CHECK("transpose");
    return NRS_OK;
}

int nrs_scale(float* out, const float* x, float s, int64_t n, float beta) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(n >= 0, "scale: negative size");
    if (n == 0) return NRS_OK;
    NRS_ARG_CHECK(out && x, "scale: null pointer");
    hipLaunchKernelGGL(nrs::scale_kernel, dim3(nrs::grid_for(n)), dim3(256), 0, nrs::stream(), out,
                       x, s, n, beta);
    NRS_LAUNCH_CHECK("scale");
    return NRS_OK;
}

int nrs_softmax_forward_scaled(float* out, const float* in, int64_t rows, int64_t width,
                               float scale) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(rows >= 0 && width > 0, "softmax: bad shape");
    if (rows == 0) return NRS_OK;
    NRS_ARG_CHECK(out && in, "softmax: null pointer");
    auto fn = width <= 64    ? nrs::softmax_fwd_kernel<1>
              : width <= 128 ? nrs::softmax_fwd_kernel<2>
              : width <= 256 ? nrs::softmax_fwd_kernel<4>
              : width <= 512 ? nrs::softmax_fwd_kernel<8>
                             : nrs::softmax_fwd_kernel<0>;
    hipLaunchKernelGGL(fn, dim3(nrs::rows_grid(rows)), dim3(256), 0, nrs::stream(), out, in, rows,
                       width, scale);
    NRS_LAUNCH_CHECK("softmax forward");
    return NRS_OK;
}

int nrs_softmax_forward(float* out, const float* in, int64_t rows, int64_t width) {
    return nrs_softmax_forward_scaled(out, in, rows, width, 1.0f);
}

int nrs_softmax_backward_scaled(float* gin, const float* y, const float* grad, int64_t rows,
                                int64_t width, float scale, float beta) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(rows >= 0 && width > 0, "softmax backward: bad shape");
    if (rows == 0) return NRS_OK;
    NRS_ARG_CHECK(gin && y && grad, "softmax backward: null pointer");
    auto fn = width <= 64    ? nrs::softmax_bwd_kernel<1>
              : width <= 128 ? nrs::softmax_bwd_kernel<2>
              : width <= 256 ? nrs::softmax_bwd_kernel<4>
              : width <= 512 ? nrs::softmax_bwd_kernel<8>
                             : nrs::softmax_bwd_kernel<0>;
    hipLaunchKernelGGL(fn, dim3(nrs::rows_grid(rows)), dim3(256), 0, nrs::stream(), gin, y, grad,
                       rows, width, scale, beta);
    NRS_LAUNCH_CHECK("softmax backward");
    return NRS_OK;
}

int nrs_softmax_backward(float* gin, const float* y, const float* grad, int64_t rows,
                         int64_t width, float beta) {
    return nrs_softmax_backward_scaled(gin, y, grad, rows, width, 1.0f, beta);
}

int nrs_slice_cols(float* out, const float* in, int64_t rows, int64_t total_cols,
                   int64_t col_start, int64_t width) {
    return nrs_slice_cols_backward_impl(out, in, rows, total_cols, col_start, width, 0.0f, false);
}

int nrs_slice_cols_backward(float* gin, const float* grad, int64_t rows, int64_t total_cols,
                            int64_t col_start, int64_t width, float beta) {
    return nrs_slice_cols_backward_impl(gin, grad, rows, total_cols, col_start, width, beta, true);
}

int nrs_concat_cols(float* out, const float* part, int64_t rows, int64_t total_cols,
                    int64_t col_offset, int64_t width) {
    return nrs_slice_cols_backward_impl(out, part, rows, total_cols, col_offset, width, 0.0f, true);
}

int nrs_concat_cols_backward(float* gpart, const float* grad, int64_t rows, int64_t total_cols,
                             int64_t col_offset, int64_t width, float beta) {
    return nrs_slice_cols_backward_impl(gpart, grad, rows, total_cols, col_offset, width, beta,
                                        false);
}

int nrs_split_heads(float* out, const float* in, int64_t rows, int64_t heads, int64_t width,
                    float beta) {
    return nrs_heads_impl(out, in, rows, heads, width, beta, true);
}

int nrs_merge_heads(float* out, const float* in, int64_t rows, int64_t heads, int64_t width,
                    float beta) {
    return nrs_heads_impl(out, in, rows, heads, width, beta, false);
}

int nrs_relu_forward(float* out, const float* x, int64_t n) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(n >= 0, "relu: negative size");
    if (n == 0) return NRS_OK;
    NRS_ARG_CHECK(out && x, "relu: null pointer");
    hipLaunchKernelGGL(nrs::relu_fwd_kernel, dim3(nrs::grid_for(n)), dim3(256), 0, nrs::stream(),
                       out, x, n);
    NRS_LAUNCH_CHECK("relu forward");
    return NRS_OK;
}

int nrs_relu_backward(float* gin, const float* grad, const float* x, int64_t n, float beta) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(n >= 0, "relu backward: negative size");
    if (n == 0) return NRS_OK;
    NRS_ARG_CHECK(gin && grad && x, "relu backward: null pointer");
    hipLaunchKernelGGL(nrs::relu_bwd_kernel, dim3(nrs::grid_for(n)), dim3(256), 0, nrs::stream(),
                       gin, grad, x, n, beta);
    NRS_LAUNCH_CHECK("relu backward");
    return NRS_OK;
}

}  // extern "C"
