// Gradient plumbing and glue kernels around the GEMMs:
//   accumulate   src/cuda/runtime.rs:13-19     acc += src (every backward edge)
//   vadd         src/cuda/graph/add.rs:19-23   out = a + b
//   bias_add     src/cuda/graph/add.rs:25-30   out = a + bias[col]
//   sum_axis0    src/cuda/reduce.rs:12-21      Linear bias grad
//   maxpool fwd/bwd src/cuda/nn/maxpool.rs:18-52 (CNN workload glue)
// All are HBM-bound streams: 128-bit accesses where the pointers allow,
// grid-stride loops capped at a few workgroups per CU.
#include <algorithm>

#include "fastdiv.hpp"
#include "nrs_internal.hpp"

namespace nrs {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

inline unsigned grid_for(int64_t n) {
    int64_t b = (n + 255) / 256;
    int64_t cap = 16 * (int64_t)num_cus();
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(b, cap));
}

inline bool a16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// out = a + b  (out may alias a: the accumulate case)
template <bool VEC>
__global__ __launch_bounds__(256) void add_kernel(float* out, const float* a, const float* b,
                                                  int64_t n) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (VEC) {
        const int64_t nv = n / 4;
        for (int64_t i = t0; i < nv; i += step) {
            const f32x4 x = reinterpret_cast<const f32x4*>(a)[i];
            const f32x4 y = reinterpret_cast<const f32x4*>(b)[i];
            reinterpret_cast<f32x4*>(out)[i] = x + y;
        }
        for (int64_t i = nv * 4 + t0; i < n; i += step) out[i] = a[i] + b[i];
    } else {
        for (int64_t i = t0; i < n; i += step) out[i] = a[i] + b[i];
    }
}

__global__ __launch_bounds__(256) void bias_add_kernel(float* out, const float* a,
                                                       const float* bias, int64_t rows,
                                                       int64_t cols) {
    const int64_t n = rows * cols;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step)
        out[i] = a[i] + bias[i % cols];
}

// out[chunk][c] = sum_{r in chunk} in[r, c] (+ beta * out[c] for a single
// chunk) for chunks of `chunk_rows` rows (blockIdx.y): a workgroup owns 64
// columns of one chunk and splits its rows into 16 contiguous groups, one
// wave each; a lane issues its group's loads 16 at a time, and the group
// sums are added in group order (deterministic).
constexpr int kColGroups = 16, kColBatch = 16, kColSingleRows = kColGroups * 4 * kColBatch;
constexpr int kColChunkRows = kColGroups * kColBatch;

__global__ __launch_bounds__(64 * kColGroups) void colsum_single_kernel(float* __restrict__ out,
                                                                       const float* __restrict__ in,
                                                                       int64_t rows, int64_t cols,
                                                                       int64_t chunk_rows, float beta) {
    __shared__ float red[kColGroups][64];
    const int x = threadIdx.x & 63, y = threadIdx.x >> 6;
    const int64_t c = (int64_t)blockIdx.x * 64 + x;
    const int64_t first = (int64_t)blockIdx.y * chunk_rows;
    in += first * cols;
    out += (int64_t)blockIdx.y * cols;
    rows = min(chunk_rows, rows - first);
    const int64_t per = (rows + kColGroups - 1) / kColGroups;
    const int64_t r0 = min(rows, y * per), r1 = min(rows, r0 + per);
    const int64_t cc = c < cols ? c : cols - 1;  // clamped: always a valid address
    float v = 0.0f;
    for (int64_t rb = r0; rb < r1; rb += kColBatch) {
        float t[kColBatch];
#pragma unroll
        for (int u = 0; u < kColBatch; ++u) t[u] = in[min(rb + u, r1 - 1) * cols + cc];
#pragma unroll
        for (int u = 0; u < kColBatch; ++u)
            if (rb + u < r1) v += t[u];
    }
    red[y][x] = v;
    __syncthreads();
    if (y != 0 || c >= cols) return;
    float r = red[0][x];
#pragma unroll
    for (int g = 1; g < kColGroups; ++g) r += red[g][x];
    if (beta != 0.0f) r = r + beta * out[c];
    out[c] = r;
}

// partial[chunk, c] = sum_{r in chunk} in[r, c], r ascending.
__global__ __launch_bounds__(256) void colsum_partial_kernel(float* __restrict__ partial,
                                                             const float* __restrict__ in,
                                                             int64_t rows, int64_t cols,
                                                             int64_t rows_per_chunk) {
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t chunk = blockIdx.y;
    if (c >= cols) return;
    const int64_t r0 = chunk * rows_per_chunk;
    const int64_t r1 = min(rows, r0 + rows_per_chunk);
    float acc = 0.0f;
    for (int64_t r = r0; r < r1; ++r) acc += in[r * cols + c];
    partial[chunk * cols + c] = acc;
}

// out[c] = sum_chunk partial[chunk, c] (chunk ascending) + beta * out[c].
__global__ __launch_bounds__(256) void colsum_combine_kernel(float* __restrict__ out,
                                                             const float* __restrict__ partial,
                                                             int64_t cols, int64_t chunks,
                                                             float beta) {
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= cols) return;
    float v = 0.0f;
    for (int64_t k = 0; k < chunks; ++k) v += partial[k * cols + c];
    if (beta != 0.0f) v = v + beta * out[c];
    out[c] = v;
}

__global__ __launch_bounds__(256) void maxpool_fwd_kernel(float* __restrict__ out,
                                                          int32_t* __restrict__ argmax,
                                                          const float* __restrict__ input,
                                                          int64_t N, int64_t C, int64_t in_h,
                                                          int64_t in_w, int k, int stride,
                                                          int64_t out_h, int64_t out_w) {
    const int64_t total = N * C * out_h * out_w;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += step) {
        const int64_t ox = idx % out_w;
        const int64_t oy = (idx / out_w) % out_h;
        const int64_t nc = idx / (out_w * out_h);
        const int64_t base = nc * in_h * in_w;
        int64_t best_i = base + (oy * stride) * in_w + ox * stride;
        float best = input[best_i];
        for (int i = 0; i < k; ++i)
            for (int j = 0; j < k; ++j) {
                const int64_t ii = base + (oy * stride + i) * in_w + ox * stride + j;
                const float v = input[ii];
                if (v > best) {
                    best = v;
                    best_i = ii;
                }
            }
        out[idx] = best;
        argmax[idx] = (int32_t)best_i;
    }
}

// dinput[e] += sum over windows (oy, ox ascending) whose argmax is e of grad.
__global__ __launch_bounds__(256) void maxpool_bwd_kernel(float* __restrict__ dinput,
                                                          const float* __restrict__ grad,
                                                          const int32_t* __restrict__ argmax,
                                                          int64_t N, int64_t C, int64_t in_h,
                                                          int64_t in_w, int k, int stride,
                                                          int64_t out_h, int64_t out_w) {
    const int64_t total = N * C * in_h * in_w;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += step) {
        const int64_t x = e % in_w;
        const int64_t y = (e / in_w) % in_h;
        const int64_t nc = e / (in_w * in_h);
        // windows with oy*stride <= y <= oy*stride + k - 1
        const int64_t oy_lo = y - k + 1 > 0 ? (y - k + 1 + stride - 1) / stride : 0;
        const int64_t oy_hi = min(out_h - 1, y / stride);
        const int64_t ox_lo = x - k + 1 > 0 ? (x - k + 1 + stride - 1) / stride : 0;
        const int64_t ox_hi = min(out_w - 1, x / stride);
        float acc = 0.0f;
        bool hit = false;
        for (int64_t oy = oy_lo; oy <= oy_hi; ++oy)
            for (int64_t ox = ox_lo; ox <= ox_hi; ++ox) {
                const int64_t o = (nc * out_h + oy) * out_w + ox;
                if (argmax[o] == (int32_t)e) {
                    acc = hit ? acc + grad[o] : grad[o];
                    hit = true;
                }
            }
        if (hit) dinput[e] = dinput[e] + acc;
    }
}

// Non-overlapping windows (k == stride), 32-bit indexing (the host checks
// the input fits): one output per thread, window scanned row by row with a
// strict > so the first maximum wins, as maxpool_forward does.
__global__ __launch_bounds__(256) void maxpool_fwd_tiled_kernel(float* __restrict__ out,
                                                                int32_t* __restrict__ argmax,
                                                                const float* __restrict__ input,
                                                                int total, int in_h, int in_w,
                                                                int k, FastDiv div_ow,
                                                                FastDiv div_oh) {
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += gridDim.x * blockDim.x) {
        uint32_t r, ox, nc, oy;
        fast_divmod((uint32_t)idx, div_ow, r, ox);
        fast_divmod(r, div_oh, nc, oy);
        const int base = nc * in_h * in_w + (oy * k) * in_w + ox * k;
        int best_i = base;
        float best = input[base];
        for (int i = 0; i < k; ++i)
            for (int j = 0; j < k; ++j) {
                const int ii = base + i * in_w + j;
                const float v = input[ii];
                if (v > best) {
                    best = v;
                    best_i = ii;
                }
            }
        out[idx] = best;
        argmax[idx] = best_i;
    }
}

// k == stride: every input element lies in at most one window, so
// dinput[e] += grad[w] exactly when argmax[w] == e; other elements are not
// touched.
__global__ __launch_bounds__(256) void maxpool_bwd_tiled_kernel(float* __restrict__ dinput,
                                                                const float* __restrict__ grad,
                                                                const int32_t* __restrict__ argmax,
                                                                int total, FastDiv div_inw,
                                                                FastDiv div_inh, FastDiv div_k,
                                                                int out_h, int out_w) {
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
        uint32_t r, x, nc, y;
        fast_divmod((uint32_t)e, div_inw, r, x);
        fast_divmod(r, div_inh, nc, y);
        const int oy = (int)fast_div(y, div_k), ox = (int)fast_div(x, div_k);
        if (oy < out_h && ox < out_w) {
            const int w = ((int)nc * out_h + oy) * out_w + ox;
            if (argmax[w] == e) dinput[e] = dinput[e] + grad[w];
        }
    }
}

}  // namespace
}  // namespace nrs

extern "C" {

int nrs_accumulate(float* acc, const float* src, int64_t n) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(n >= 0, "accumulate: negative size");
    if (n == 0) return NRS_OK;
    NRS_ARG_CHECK(acc && src, "accumulate: null pointer");
    if (nrs::a16(acc) && nrs::a16(src))
        hipLaunchKernelGGL(nrs::add_kernel<true>, dim3(nrs::grid_for(n / 4 + 1)), dim3(256), 0,
                           nrs::stream(), acc, acc, src, n);
    else
        hipLaunchKernelGGL(nrs::add_kernel<false>, dim3(nrs::grid_for(n)), dim3(256), 0,
                           nrs::stream(), acc, acc, src, n);
    NRS_LAUNCH_CHECK("accumulate");
    return NRS_OK;
}

int nrs_vadd(float* out, const float* a, const float* b, int64_t n) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(n >= 0, "vadd: negative size");
    if (n == 0) return NRS_OK;
    NRS_ARG_CHECK(out && a && b, "vadd: null pointer");
    if (nrs::a16(out) && nrs::a16(a) && nrs::a16(b))
        hipLaunchKernelGGL(nrs::add_kernel<true>, dim3(nrs::grid_for(n / 4 + 1)), dim3(256), 0,
                           nrs::stream(), out, a, b, n);
    else
        hipLaunchKernelGGL(nrs::add_kernel<false>, dim3(nrs::grid_for(n)), dim3(256), 0,
                           nrs::stream(), out, a, b, n);
    NRS_LAUNCH_CHECK("vadd");
    return NRS_OK;
}

int nrs_bias_add(float* out, const float* a, const float* bias, int64_t rows, int64_t cols) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(rows >= 0 && cols >= 0, "bias_add: negative size");
    if (rows == 0 || cols == 0) return NRS_OK;
    NRS_ARG_CHECK(out && a && bias, "bias_add: null pointer");
    hipLaunchKernelGGL(nrs::bias_add_kernel, dim3(nrs::grid_for(rows * cols)), dim3(256), 0,
                       nrs::stream(), out, a, bias, rows, cols);
    NRS_LAUNCH_CHECK("bias_add");
    return NRS_OK;
}

int nrs_sum_axis0(float* out, const float* in, int64_t rows, int64_t cols, float beta) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(rows >= 0 && cols >= 0, "sum_axis0: negative size");
    if (cols == 0) return NRS_OK;
    NRS_ARG_CHECK(out && (in || rows == 0), "sum_axis0: null pointer");
    const unsigned cb = (unsigned)((cols + 63) / 64);
    if (rows <= nrs::kColSingleRows) {
        // short columns (a Linear's bias gradient over a batch): one launch
        hipLaunchKernelGGL(nrs::colsum_single_kernel, dim3(cb), dim3(64 * nrs::kColGroups), 0,
                           nrs::stream(), out, in, rows, cols, std::max<int64_t>(rows, 1), beta);
        NRS_LAUNCH_CHECK("sum_axis0");
        return NRS_OK;
    }
    if (rows <= (int64_t)nrs::kColChunkRows * nrs::kColSingleRows && rows <= 65535ll * nrs::kColChunkRows) {
        // chunks of 256 rows summed side by side, then the chunk sums (at
        // most kColSingleRows of them) in chunk order
        const int64_t chunks = (rows + nrs::kColChunkRows - 1) / nrs::kColChunkRows;
        float* part = nrs::workspace(sizeof(float) * (size_t)(chunks * cols), 3);
        if (!part) return NRS_ERR_ALLOC;
        hipLaunchKernelGGL(nrs::colsum_single_kernel, dim3(cb, (unsigned)chunks),
                           dim3(64 * nrs::kColGroups), 0, nrs::stream(), part, in, rows, cols,
                           (int64_t)nrs::kColChunkRows, 0.0f);
        NRS_LAUNCH_CHECK("sum_axis0 (chunks)");
        hipLaunchKernelGGL(nrs::colsum_single_kernel, dim3(cb), dim3(64 * nrs::kColGroups), 0,
                           nrs::stream(), out, part, chunks, cols, chunks, beta);
        NRS_LAUNCH_CHECK("sum_axis0");
        return NRS_OK;
    }
    const int64_t col_blocks = (cols + 255) / 256;
    // Row chunks so that ~2 workgroups per CU run, each chunk >= 64 rows.
    int64_t chunks = std::max<int64_t>(1, (2 * (int64_t)nrs::num_cus()) / col_blocks);
    chunks = std::min<int64_t>(chunks, std::max<int64_t>(1, rows / 64));
    chunks = std::min<int64_t>(chunks, 65535);
    const int64_t per = rows > 0 ? (rows + chunks - 1) / chunks : 1;
    chunks = rows > 0 ? (rows + per - 1) / per : 1;
    float* part = nrs::workspace(sizeof(float) * (size_t)(chunks * cols), 3);
    if (!part) return NRS_ERR_ALLOC;
    hipLaunchKernelGGL(nrs::colsum_partial_kernel, dim3((unsigned)col_blocks, (unsigned)chunks),
                       dim3(256), 0, nrs::stream(), part, in, rows, cols, per);
    NRS_LAUNCH_CHECK("sum_axis0 (partials)");
    hipLaunchKernelGGL(nrs::colsum_combine_kernel, dim3((unsigned)col_blocks), dim3(256), 0,
                       nrs::stream(), out, part, cols, chunks, beta);
    NRS_LAUNCH_CHECK("sum_axis0 (combine)");
    return NRS_OK;
}

int nrs_maxpool_forward(float* out, int32_t* argmax, const float* input, int64_t N, int64_t C,
                        int64_t in_h, int64_t in_w, int64_t k, int64_t stride) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(k > 0 && stride > 0 && in_h >= k && in_w >= k, "maxpool: bad window");
    NRS_ARG_CHECK(N * C * in_h * in_w <= INT32_MAX, "maxpool: input too large for int32 argmax");
    const int64_t oh = (in_h - k) / stride + 1, ow = (in_w - k) / stride + 1;
    const int64_t total = N * C * oh * ow;
    if (total == 0) return NRS_OK;
    if (k == stride)
        hipLaunchKernelGGL(nrs::maxpool_fwd_tiled_kernel, dim3(nrs::grid_for(total)), dim3(256), 0,
                           nrs::stream(), out, argmax, input, (int)total, (int)in_h, (int)in_w,
                           (int)k, nrs::make_fastdiv((uint32_t)ow), nrs::make_fastdiv((uint32_t)oh));
    else
        hipLaunchKernelGGL(nrs::maxpool_fwd_kernel, dim3(nrs::grid_for(total)), dim3(256), 0,
                           nrs::stream(), out, argmax, input, N, C, in_h, in_w, (int)k,
                           (int)stride, oh, ow);
    NRS_LAUNCH_CHECK("maxpool forward");
    return NRS_OK;
}

int nrs_maxpool_backward(float* dinput, const float* grad, const int32_t* argmax, int64_t N,
                         int64_t C, int64_t in_h, int64_t in_w, int64_t k, int64_t stride) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(k > 0 && stride > 0 && in_h >= k && in_w >= k, "maxpool: bad window");
    NRS_ARG_CHECK(N * C * in_h * in_w <= INT32_MAX, "maxpool: input too large for int32 argmax");
    const int64_t oh = (in_h - k) / stride + 1, ow = (in_w - k) / stride + 1;
    const int64_t total = N * C * in_h * in_w;
    if (total == 0) return NRS_OK;
    if (k == stride)
        hipLaunchKernelGGL(nrs::maxpool_bwd_tiled_kernel, dim3(nrs::grid_for(total)), dim3(256), 0,
                           nrs::stream(), dinput, grad, argmax, (int)total,
                           nrs::make_fastdiv((uint32_t)in_w), nrs::make_fastdiv((uint32_t)in_h),
                           nrs::make_fastdiv((uint32_t)k), (int)oh, (int)ow);
    else
        hipLaunchKernelGGL(nrs::maxpool_bwd_kernel, dim3(nrs::grid_for(total)), dim3(256), 0,
                           nrs::stream(), dinput, grad, argmax, N, C, in_h, in_w, (int)k,
                           (int)stride, oh, ow);
    NRS_LAUNCH_CHECK("maxpool backward");
    return NRS_OK;
}

}  // extern "C"
