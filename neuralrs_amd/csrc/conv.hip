// Conv2d lowering for gfx950: the five primitive kernels of
// src/cuda/nn/conv.rs:27-149 (same index semantics) and the whole-op
// forward/backward of nn::conv2d (src/cuda/nn/conv.rs:244-328) built on the
// MFMA GEMM core.
//
// Data layout: NCHW images; the column matrix is [c_in*kh*kw, N*out_h*out_w]
// with columns grouped by sample (col = ni*P + p, P = out_h*out_w) and rows
// following the weight layout (row = (ic*kh + i)*kw + j), so the weight
// [c_out, c_in*kh*kw] multiplies it directly.
//
// Differences from the reference's launch sequence, all numerically neutral:
//  * forward: the GEMM epilogue writes NCHW + bias itself (col2out fused);
//  * backward: the reference's second im2col (conv.rs:317) remains, but the
//    dcols/col2im, wgrad and bias-grad results are added straight into the
//    caller's gradients (beta = 1), replacing three accumulate passes;
//  * wgrad split-K combines slices deterministically, bias grad is a
//    two-level deterministic reduction instead of c_out serial threads.
#include <algorithm>

#include "nrs_internal.hpp"

namespace nrs {

int gemm_launch(int layout, float* C, const float* A, const float* B, int64_t M, int64_t N,
                int64_t K, int64_t batch, int64_t sA, int64_t sB, int64_t sC, float beta,
                const float* bias, int epi, int64_t nchw_P, bool allow_split, int force_slices);

namespace {

inline unsigned grid_for(int64_t n, int per_block = 256) {
    int64_t b = (n + per_block - 1) / per_block;
    int64_t cap = 32 * (int64_t)num_cus();
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(b, cap));
}

// cols[row, ni*P + p]: one thread per column-matrix element, consecutive
// threads along the row so the writes are coalesced.
__global__ __launch_bounds__(256) void im2col_kernel(float* __restrict__ cols,
                                                     const float* __restrict__ input, int64_t N,
                                                     int64_t c_in, int64_t in_h, int64_t in_w,
                                                     int kh, int kw, int stride, int pad,
                                                     int64_t out_h, int64_t out_w) {
    const int64_t P = out_h * out_w;
    const int64_t width = N * P;
    const int64_t total = c_in * kh * kw * width;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += step) {
        const int64_t row = idx / width;
        const int64_t rest = idx - row * width;
        const int64_t ni = rest / P;
        const int64_t p = rest - ni * P;
        const int64_t oy = p / out_w;
        const int64_t ox = p - oy * out_w;
        const int j = (int)(row % kw);
        const int i = (int)((row / kw) % kh);
        const int64_t ic = row / (kw * kh);
        const int64_t iy = oy * stride + i - pad;
        const int64_t ix = ox * stride + j - pad;
        float v = 0.0f;
        if (iy >= 0 && iy < in_h && ix >= 0 && ix < in_w)
            v = input[((ni * c_in + ic) * in_h + iy) * in_w + ix];
        cols[idx] = v;
    }
}

// out[ni, oc, p] = mm[oc, ni*P + p] + bias[oc]
__global__ __launch_bounds__(256) void col2out_kernel(float* __restrict__ out,
                                                      const float* __restrict__ mm,
                                                      const float* __restrict__ bias, int64_t N,
                                                      int64_t c_out, int64_t P) {
    const int64_t total = N * c_out * P;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += step) {
        const int64_t p = idx % P;
        const int64_t oc = (idx / P) % c_out;
        const int64_t ni = idx / (P * c_out);
        out[idx] = mm[oc * (N * P) + ni * P + p] + bias[oc];
    }
}

// mm[oc, ni*P + p] = grad[ni, oc, p]
__global__ __launch_bounds__(256) void out2mm_kernel(float* __restrict__ mm,
                                                     const float* __restrict__ grad, int64_t N,
                                                     int64_t c_out, int64_t P) {
    const int64_t total = N * c_out * P;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += step) {
        const int64_t p = idx % P;
        const int64_t oc = (idx / P) % c_out;
        const int64_t ni = idx / (P * c_out);
        mm[oc * (N * P) + ni * P + p] = grad[idx];
    }
}

// dinput[ni, ic, y, x] = sum over covering (i, j) of dcols[row, ni*P + oy*out_w + ox]
// (i, j ascending, as conv.rs:130-147), then + beta * dinput.
__global__ __launch_bounds__(256) void col2im_kernel(float* __restrict__ dinput,
                                                     const float* __restrict__ dcols, int64_t N,
                                                     int64_t c_in, int64_t in_h, int64_t in_w,
                                                     int kh, int kw, int stride, int pad,
                                                     int64_t out_h, int64_t out_w, float beta) {
    const int64_t total = N * c_in * in_h * in_w;
    const int64_t P = out_h * out_w;
    const int64_t width = N * P;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += step) {
        const int64_t x = idx % in_w;
        const int64_t y = (idx / in_w) % in_h;
        const int64_t ic = (idx / (in_w * in_h)) % c_in;
        const int64_t ni = idx / (in_w * in_h * c_in);
        float acc = 0.0f;
        for (int i = 0; i < kh; ++i) {
            const int64_t oyn = y + pad - i;
            if (oyn < 0 || oyn % stride != 0) continue;
            const int64_t oy = oyn / stride;
            if (oy >= out_h) continue;
            for (int j = 0; j < kw; ++j) {
                const int64_t oxn = x + pad - j;
                if (oxn < 0 || oxn % stride != 0) continue;
                const int64_t ox = oxn / stride;
                if (ox >= out_w) continue;
                const int64_t row = (ic * kh + i) * kw + j;
                acc += dcols[row * width + ni * P + oy * out_w + ox];
            }
        }
        if (beta != 0.0f) acc = acc + beta * dinput[idx];
        dinput[idx] = acc;
    }
}

constexpr int kRedThreads = 256;

// Block-wide deterministic sum (fixed tree over the 256 lanes).
__device__ __forceinline__ float block_sum(float v, float* red) {
    const int t = threadIdx.x;
    red[t] = v;
    __syncthreads();
#pragma unroll
    for (int s = kRedThreads / 2; s > 0; s >>= 1) {
        if (t < s) red[t] += red[t + s];
        __syncthreads();
    }
    return red[0];
}

// Stage 1 of the bias gradient: partial[oc, chunk] = sum of grad[ni, oc, p]
// over the chunk's slice of the flattened (ni, p) range.
__global__ __launch_bounds__(kRedThreads) void bias_grad_partial_kernel(
    float* __restrict__ partial, const float* __restrict__ grad, int64_t N, int64_t c_out,
    int64_t P, int64_t per_chunk) {
    __shared__ float red[kRedThreads];
    const int64_t oc = blockIdx.y;
    const int64_t chunk = blockIdx.x;
    const int64_t total = N * P;
    const int64_t e0 = chunk * per_chunk;
    const int64_t e1 = min(total, e0 + per_chunk);
    float acc = 0.0f;
    for (int64_t e = e0 + threadIdx.x; e < e1; e += kRedThreads) {
        const int64_t ni = e / P;
        const int64_t p = e - ni * P;
        acc += grad[(ni * c_out + oc) * P + p];
    }
    const float s = block_sum(acc, red);
    if (threadIdx.x == 0) partial[oc * gridDim.x + chunk] = s;
}

// Stage 2: out[c] = sum_k partial[c, k] (k ascending) + beta * out[c].
__global__ __launch_bounds__(kRedThreads) void rows_sum_kernel(float* __restrict__ out,
                                                               const float* __restrict__ partial,
                                                               int64_t n_out, int64_t n_part,
                                                               float beta) {
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= n_out) return;
    float v = 0.0f;
    for (int64_t k = 0; k < n_part; ++k) v += partial[c * n_part + k];
    if (beta != 0.0f) v = v + beta * out[c];
    out[c] = v;
}

}  // namespace

int bias_grad_launch(float* dbias, const float* grad, int64_t N, int64_t c_out, int64_t P,
                     float beta) {
    if (c_out == 0) return NRS_OK;
    const int64_t total = N * P;
    // Chunks so that ~4 workgroups per CU run in total, each >= 4096 elements.
    int64_t chunks = std::max<int64_t>(1, (4 * (int64_t)num_cus() + c_out - 1) / c_out);
    chunks = std::min<int64_t>(chunks, std::max<int64_t>(1, total / 4096));
    const int64_t per_chunk = std::max<int64_t>(1, (total + chunks - 1) / chunks);
    chunks = std::max<int64_t>(1, (total + per_chunk - 1) / per_chunk);
    NRS_ARG_CHECK(c_out <= 65535, "conv2d bias grad: c_out too large");
    float* part = workspace(sizeof(float) * (size_t)(c_out * chunks), 3);
    if (!part) return NRS_ERR_ALLOC;
    if (total == 0) {
        int zrc = zero_fill(part, sizeof(float) * (size_t)(c_out * chunks));
        if (zrc) return zrc;
    } else {
        hipLaunchKernelGGL(bias_grad_partial_kernel, dim3((unsigned)chunks, (unsigned)c_out),
                           dim3(kRedThreads), 0, stream(), part, grad, N, c_out, P, per_chunk);
        NRS_LAUNCH_CHECK("conv2d bias grad (partials)");
    }
    hipLaunchKernelGGL(rows_sum_kernel, dim3((unsigned)((c_out + 255) / 256)), dim3(kRedThreads),
                       0, stream(), dbias, part, c_out, chunks, beta);
    NRS_LAUNCH_CHECK("conv2d bias grad (combine)");
    return NRS_OK;
}

namespace {

struct ConvDims {
    int64_t N, c_in, in_h, in_w, c_out, kh, kw, stride, pad, out_h, out_w;
};

int conv_dims(ConvDims& d, int64_t N, int64_t c_in, int64_t in_h, int64_t in_w, int64_t c_out,
              int64_t kh, int64_t kw, int64_t stride, int64_t pad) {
    NRS_ARG_CHECK(N >= 0 && c_in >= 0 && in_h >= 0 && in_w >= 0 && c_out >= 0,
                  "conv2d: negative size");
    NRS_ARG_CHECK(kh > 0 && kw > 0 && stride > 0 && pad >= 0, "conv2d: bad kernel/stride/pad");
    NRS_ARG_CHECK(in_h + 2 * pad >= kh && in_w + 2 * pad >= kw,
                  "conv2d: kernel larger than padded input");
    d = ConvDims{N, c_in, in_h, in_w, c_out, kh, kw, stride, pad,
                 (in_h + 2 * pad - kh) / stride + 1, (in_w + 2 * pad - kw) / stride + 1};
    return NRS_OK;
}

int launch_im2col(float* cols, const float* input, const ConvDims& d) {
    const int64_t total = d.c_in * d.kh * d.kw * d.N * d.out_h * d.out_w;
    if (total == 0) return NRS_OK;
    hipLaunchKernelGGL(im2col_kernel, dim3(grid_for(total)), dim3(256), 0, stream(), cols, input,
                       d.N, d.c_in, d.in_h, d.in_w, (int)d.kh, (int)d.kw, (int)d.stride,
                       (int)d.pad, d.out_h, d.out_w);
    NRS_LAUNCH_CHECK("conv2d im2col");
    return NRS_OK;
}

int launch_col2im(float* dinput, const float* dcols, const ConvDims& d, float beta) {
    const int64_t total = d.N * d.c_in * d.in_h * d.in_w;
    if (total == 0) return NRS_OK;
    hipLaunchKernelGGL(col2im_kernel, dim3(grid_for(total)), dim3(256), 0, stream(), dinput, dcols,
                       d.N, d.c_in, d.in_h, d.in_w, (int)d.kh, (int)d.kw, (int)d.stride,
                       (int)d.pad, d.out_h, d.out_w, beta);
    NRS_LAUNCH_CHECK("conv2d col2im");
    return NRS_OK;
}

int launch_out2mm(float* mm, const float* grad, const ConvDims& d) {
    const int64_t P = d.out_h * d.out_w;
    const int64_t total = d.N * d.c_out * P;
    if (total == 0) return NRS_OK;
    hipLaunchKernelGGL(out2mm_kernel, dim3(grid_for(total)), dim3(256), 0, stream(), mm, grad,
                       d.N, d.c_out, P);
    NRS_LAUNCH_CHECK("conv2d out2mm");
    return NRS_OK;
}

}  // namespace
}  // namespace nrs

extern "C" {

int nrs_im2col(float* cols, const float* input, int64_t N, int64_t c_in, int64_t in_h,
               int64_t in_w, int64_t kh, int64_t kw, int64_t stride, int64_t pad) {
    NRS_REQUIRE_INIT();
    nrs::ConvDims d;
    int rc = nrs::conv_dims(d, N, c_in, in_h, in_w, 0, kh, kw, stride, pad);
    if (rc) return rc;
    return nrs::launch_im2col(cols, input, d);
}

int nrs_col2out(float* out, const float* mm_out, const float* bias, int64_t N, int64_t c_out,
                int64_t out_h, int64_t out_w) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(N >= 0 && c_out >= 0 && out_h >= 0 && out_w >= 0, "col2out: negative size");
    const int64_t P = out_h * out_w, total = N * c_out * P;
    if (total == 0) return NRS_OK;
    hipLaunchKernelGGL(nrs::col2out_kernel, dim3(nrs::grid_for(total)), dim3(256), 0,
                       nrs::stream(), out, mm_out, bias, N, c_out, P);
    NRS_LAUNCH_CHECK("conv2d col2out");
    return NRS_OK;
}

int nrs_out2mm(float* mm_grad, const float* grad, int64_t N, int64_t c_out, int64_t out_h,
               int64_t out_w) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(N >= 0 && c_out >= 0 && out_h >= 0 && out_w >= 0, "out2mm: negative size");
    nrs::ConvDims d{N, 0, 0, 0, c_out, 1, 1, 1, 0, out_h, out_w};
    return nrs::launch_out2mm(mm_grad, grad, d);
}

int nrs_col2im(float* dinput, const float* dcols, int64_t N, int64_t c_in, int64_t in_h,
               int64_t in_w, int64_t kh, int64_t kw, int64_t stride, int64_t pad, float beta) {
    NRS_REQUIRE_INIT();
    nrs::ConvDims d;
    int rc = nrs::conv_dims(d, N, c_in, in_h, in_w, 0, kh, kw, stride, pad);
    if (rc) return rc;
    return nrs::launch_col2im(dinput, dcols, d, beta);
}

int nrs_conv2d_bias_grad(float* dbias, const float* grad, int64_t N, int64_t c_out,
                         int64_t out_h, int64_t out_w, float beta) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(N >= 0 && c_out >= 0 && out_h >= 0 && out_w >= 0, "bias_grad: negative size");
    return nrs::bias_grad_launch(dbias, grad, N, c_out, out_h * out_w, beta);
}

int nrs_conv2d_forward(float* out, const float* input, const float* weight, const float* bias,
                       int64_t N, int64_t c_in, int64_t in_h, int64_t in_w, int64_t c_out,
                       int64_t kh, int64_t kw, int64_t stride, int64_t pad) {
    NRS_REQUIRE_INIT();
    nrs::ConvDims d;
    int rc = nrs::conv_dims(d, N, c_in, in_h, in_w, c_out, kh, kw, stride, pad);
    if (rc) return rc;
    const int64_t col_h = c_in * kh * kw, P = d.out_h * d.out_w, width = N * P;
    if (c_out == 0 || width == 0) return NRS_OK;
    float* cols = nrs::workspace(sizeof(float) * (size_t)std::max<int64_t>(1, col_h * width), 1);
    if (!cols) return NRS_ERR_ALLOC;
    rc = nrs::launch_im2col(cols, input, d);
    if (rc) return rc;
    // out(NCHW) = W[c_out, col_h] . cols[col_h, N*P] + bias[oc]
    return nrs::gemm_launch(NRS_NN, out, weight, cols, c_out, width, col_h, 1, 0, 0, 0, 0.0f, bias,
                            bias ? NRS_EPI_BIAS_ROW : NRS_EPI_NONE, P, false, 0);
}

int nrs_conv2d_backward(float* dinput, float* dweight, float* dbias, const float* grad,
                        const float* input, const float* weight, int64_t N, int64_t c_in,
                        int64_t in_h, int64_t in_w, int64_t c_out, int64_t kh, int64_t kw,
                        int64_t stride, int64_t pad) {
    NRS_REQUIRE_INIT();
    nrs::ConvDims d;
    int rc = nrs::conv_dims(d, N, c_in, in_h, in_w, c_out, kh, kw, stride, pad);
    if (rc) return rc;
    const int64_t col_h = c_in * kh * kw, P = d.out_h * d.out_w, width = N * P;
    if (c_out == 0) return NRS_OK;
    float* gmm = nrs::workspace(sizeof(float) * (size_t)std::max<int64_t>(1, c_out * width), 2);
    if (!gmm) return NRS_ERR_ALLOC;
    rc = nrs::launch_out2mm(gmm, grad, d);  // [c_out, N*P]
    if (rc) return rc;
    float* cols = nrs::workspace(sizeof(float) * (size_t)std::max<int64_t>(1, col_h * width), 1);
    if (!cols) return NRS_ERR_ALLOC;
    if (dinput) {
        // dcols[col_h, N*P] = W^T . G ; dinput += col2im(dcols)   (conv.rs:304-312)
        rc = nrs::gemm_launch(NRS_TN, cols, weight, gmm, col_h, width, c_out, 1, 0, 0, 0, 0.0f,
                              nullptr, NRS_EPI_NONE, 0, true, 0);
        if (rc) return rc;
        rc = nrs::launch_col2im(dinput, cols, d, 1.0f);
        if (rc) return rc;
    }
    if (dweight) {
        // dW[c_out, col_h] += G . cols^T   (conv.rs:314-320, split-K NT)
        rc = nrs::launch_im2col(cols, input, d);
        if (rc) return rc;
        rc = nrs::gemm_launch(NRS_NT, dweight, gmm, cols, c_out, col_h, width, 1, 0, 0, 0, 1.0f,
                              nullptr, NRS_EPI_NONE, 0, true, 0);
        if (rc) return rc;
    }
    if (dbias) {
        rc = nrs::bias_grad_launch(dbias, grad, N, c_out, P, 1.0f);  // conv.rs:322
        if (rc) return rc;
    }
    return NRS_OK;
}

}  // extern "C"
