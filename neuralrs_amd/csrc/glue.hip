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
//   layernorm        src/cuda/nn/normalization.rs:14-85  (TransformerBlock)
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

// LayerNorm forward, one wave per row (src/cuda/nn/normalization.rs:14-40
// ln_forward, which runs one thread per row): mean, biased variance,
// inv_std = 1 / sqrt(var + eps), x_norm = (x - mean) * inv_std and
// out = gamma * x_norm + beta. PER > 0 keeps the row (features <= 64 * PER)
// in registers; PER = 0 re-reads it. A non-null `in2` normalises in + in2
// (the sum rounded to f32 as the residual add computes it) without writing
// the sum out.
template <int PER>
__global__ __launch_bounds__(256) void layernorm_fwd_kernel(
    float* __restrict__ out, float* __restrict__ xn_out, float* __restrict__ istd_out,
    const float* __restrict__ in, const float* __restrict__ in2, const float* __restrict__ gamma,
    const float* __restrict__ beta, int64_t rows, int64_t F, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t waves = (int64_t)gridDim.x * 4;
    const float nf = (float)F;
    for (int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); r < rows; r += waves) {
        const float* x = in + r * F;
        const float* x2 = in2 ? in2 + r * F : nullptr;
        auto at = [&](int64_t f) { return x2 ? x[f] + x2[f] : x[f]; };
        float* y = out + r * F;
        float* xn = xn_out + r * F;
        if constexpr (PER > 0) {
            float v[PER];
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int f = lane + 64 * i;
                v[i] = f < F ? at(f) : 0.0f;
                s += v[i];
            }
            const float mean = wave_sum(s) / nf;
            float q = 0.0f;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const float d = lane + 64 * i < F ? v[i] - mean : 0.0f;
                q += d * d;
            }
            const float istd = 1.0f / sqrtf(wave_sum(q) / nf + eps);
            if (lane == 0) istd_out[r] = istd;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int f = lane + 64 * i;
                if (f < F) {
                    const float t = (v[i] - mean) * istd;
                    xn[f] = t;
                    y[f] = gamma[f] * t + beta[f];
                }
            }
        } else {
            float s = 0.0f;
            for (int64_t f = lane; f < F; f += 64) s += at(f);
            const float mean = wave_sum(s) / nf;
            float q = 0.0f;
            for (int64_t f = lane; f < F; f += 64) {
                const float d = at(f) - mean;
                q += d * d;
            }
            const float istd = 1.0f / sqrtf(wave_sum(q) / nf + eps);
            if (lane == 0) istd_out[r] = istd;
            for (int64_t f = lane; f < F; f += 64) {
                const float t = (at(f) - mean) * istd;
                xn[f] = t;
                y[f] = gamma[f] * t + beta[f];
            }
        }
    }
}

// LayerNorm input gradient, one wave per row (normalization.rs:57-80 ln_dx):
// dxh = grad * gamma, dinput = inv_std * (dxh - sum(dxh)/F - x_norm *
// sum(dxh * x_norm)/F) + acc * dinput.
// dinput = dx + acc * dinput and, when dinput2 is set, dinput2 = dx + acc2 *
// dinput2 (the input gradient of norm(a + b) goes to both a and b).
__global__ __launch_bounds__(256) void layernorm_dx_kernel(
    float* __restrict__ dinput, float* __restrict__ dinput2, const float* __restrict__ grad,
    const float* __restrict__ gamma, const float* __restrict__ x_norm,
    const float* __restrict__ inv_std, int64_t rows, int64_t F, float acc, float acc2) {
    const int lane = threadIdx.x & 63;
    const int64_t waves = (int64_t)gridDim.x * 4;
    const float nf = (float)F;
    for (int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); r < rows; r += waves) {
        const float* g = grad + r * F;
        const float* xn = x_norm + r * F;
        float s1 = 0.0f, s2 = 0.0f;
        for (int64_t f = lane; f < F; f += 64) {
            const float d = g[f] * gamma[f];
            s1 += d;
            s2 += d * xn[f];
        }
        s1 = wave_sum(s1) / nf;
        s2 = wave_sum(s2) / nf;
        const float istd = inv_std[r];
        float* o = dinput + r * F;
        float* o2 = dinput2 ? dinput2 + r * F : nullptr;
        for (int64_t f = lane; f < F; f += 64) {
            const float dx = istd * (g[f] * gamma[f] - s1 - xn[f] * s2);
            o[f] = acc != 0.0f ? dx + acc * o[f] : dx;
            if (o2) o2[f] = acc2 != 0.0f ? dx + acc2 * o2[f] : dx;
        }
    }
}

// LayerNorm parameter gradients over rows (normalization.rs:41-56 ln_reduce
// runs one thread per feature over every row). Block (x, c) sums rows
// [c*rc, (c+1)*rc) of grad * x_norm and grad for 256 features into
// partial[c], issuing 8 rows' loads before adding any (rc: kLnRows, or a
// larger multiple of 8 when the rows would need more than 65535 chunks). The combine kernel
// splits the chunks into kLnGroups contiguous ranges summed in parallel
// (ascending inside a range) and adds the ranges in order, so the result is
// deterministic.
constexpr int kLnRows = 32, kLnGroups = 16;

__global__ __launch_bounds__(256) void layernorm_param_partial_kernel(
    float* __restrict__ part_g, float* __restrict__ part_b, const float* __restrict__ grad,
    const float* __restrict__ x_norm, int64_t rows, int64_t F, int64_t rc) {
    const int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (f >= F) return;
    const int64_t r0 = (int64_t)blockIdx.y * rc;
    float dg = 0.0f, db = 0.0f;
    for (int64_t b = 0; b < rc; b += 8) {
        float gv[8], xv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t r = r0 + b + u;
            const bool ok = r < rows;
            gv[u] = ok ? grad[r * F + f] : 0.0f;
            xv[u] = ok ? x_norm[r * F + f] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            dg += gv[u] * xv[u];
            db += gv[u];
        }
    }
    part_g[(int64_t)blockIdx.y * F + f] = dg;
    part_b[(int64_t)blockIdx.y * F + f] = db;
}

// Input gradient (when dinput is set) and parameter partials (when part_g
// is set) in one pass, F <= 64 * PER; every LayerNorm backward of such a
// width runs this kernel, so each gradient has the same bits whichever
// others a call asks for: block c
// owns rows [c*rc, (c+1)*rc); wave w takes row pairs r0 + 2w + 8k, +1 (both
// rows' loads issued before either is used), writes each row's input
// gradient exactly as layernorm_dx_kernel does, and sums grad * x_norm and
// grad over its rows in row order; the four waves' sums are added in wave
// order into partial[c] for layernorm_param_combine_kernel. grad and x_norm
// are read once for both gradients.
template <int PER>
__global__ __launch_bounds__(256) void layernorm_bwd_fused_kernel(
    float* __restrict__ dinput, float* __restrict__ dinput2, float* __restrict__ part_g,
    float* __restrict__ part_b, const float* __restrict__ grad, const float* __restrict__ gamma,
    const float* __restrict__ x_norm, const float* __restrict__ inv_std, int64_t rows, int64_t F,
    int64_t rc, float acc, float acc2) {
    __shared__ float red[2][4][64 * PER];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t r0 = (int64_t)blockIdx.x * rc, r1 = min(rows, r0 + rc);
    const float nf = (float)F;
    float gm[PER], pg[PER], pb[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int f = lane + 64 * i;
        // gamma is only needed (and may be null) without an input gradient
        gm[i] = (dinput != nullptr && f < F) ? gamma[f] : 0.0f;
        pg[i] = 0.0f;
        pb[i] = 0.0f;
    }
    for (int64_t rb = r0 + 2 * w; rb < r1; rb += 8) {
        const bool two = rb + 1 < r1;  // wave-uniform
        float g[2][PER], xn[2][PER];
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int f = lane + 64 * i;
                const bool ok = f < F && (q == 0 || two);
                const int64_t at = ok ? (rb + q) * F + f : 0;
                g[q][i] = ok ? grad[at] : 0.0f;
                xn[q][i] = ok ? x_norm[at] : 0.0f;
            }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            if (q == 1 && !two) break;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                pg[i] += g[q][i] * xn[q][i];
                pb[i] += g[q][i];
            }
            if (!dinput) continue;  // parameter gradients only
            const int64_t r = rb + q;
            float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const float d = g[q][i] * gm[i];
                s1 += d;
                s2 += d * xn[q][i];
            }
            s1 = wave_sum(s1) / nf;
            s2 = wave_sum(s2) / nf;
            const float istd = inv_std[r];
            float* o = dinput + r * F;
            float* o2 = dinput2 ? dinput2 + r * F : nullptr;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int f = lane + 64 * i;
                if (f < F) {
                    const float dx = istd * (g[q][i] * gm[i] - s1 - xn[q][i] * s2);
                    o[f] = acc != 0.0f ? dx + acc * o[f] : dx;
                    if (o2) o2[f] = acc2 != 0.0f ? dx + acc2 * o2[f] : dx;
                }
            }
        }
    }
    if (!part_g) return;  // input gradient only (uniform)
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        red[0][w][lane + 64 * i] = pg[i];
        red[1][w][lane + 64 * i] = pb[i];
    }
    __syncthreads();
    for (int f = threadIdx.x; f < F; f += 256) {
        float sg = red[0][0][f], sb = red[1][0][f];
#pragma unroll
        for (int y = 1; y < 4; ++y) {
            sg += red[0][y][f];
            sb += red[1][y][f];
        }
        part_g[(int64_t)blockIdx.x * F + f] = sg;
        part_b[(int64_t)blockIdx.x * F + f] = sb;
    }
}

__global__ __launch_bounds__(64 * kLnGroups) void layernorm_param_combine_kernel(
    float* __restrict__ dgamma, float* __restrict__ dbeta, const float* __restrict__ part_g,
    const float* __restrict__ part_b, int64_t chunks, int64_t F, float acc) {
    __shared__ float red[2][kLnGroups][64];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int64_t f = (int64_t)blockIdx.x * 64 + tx;
    const int64_t per = (chunks + kLnGroups - 1) / kLnGroups;
    const int64_t c0 = min(chunks, ty * per), c1 = min(chunks, c0 + per);
    float dg = 0.0f, db = 0.0f;
    if (f < F) {
        for (int64_t c = c0; c < c1; c += 8) {
            float gv[8], bv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const bool ok = c + u < c1;
                gv[u] = ok ? part_g[(c + u) * F + f] : 0.0f;
                bv[u] = ok ? part_b[(c + u) * F + f] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                dg += gv[u];
                db += bv[u];
            }
        }
    }
    red[0][ty][tx] = dg;
    red[1][ty][tx] = db;
    __syncthreads();
    if (ty == 0 && f < F) {
        float sg = red[0][0][tx], sb = red[1][0][tx];
#pragma unroll
        for (int y = 1; y < kLnGroups; ++y) {
            sg += red[0][y][tx];
            sb += red[1][y][tx];
        }
        if (dgamma) dgamma[f] = acc != 0.0f ? sg + acc * dgamma[f] : sg;
        if (dbeta) dbeta[f] = acc != 0.0f ? sb + acc * dbeta[f] : sb;
    }
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

// Cross-entropy of raw logits against a target (one-hot rows), one thread
// per row as the reference's kernels (src/cuda/loss/cross_entropy.rs:18-58):
// the row max folded from its first logit, the sum of expf(l - max) in class
// order; GRAD: out[row] = (softmax - target) * (1 / batch), the fused seed of
// cross_entropy_backward; else out[row] = sum_c -t_c * (l_c - log_sum_exp).
template <bool GRAD>
__global__ __launch_bounds__(256) void cross_entropy_kernel(float* __restrict__ out,
                                                            const float* __restrict__ logits,
                                                            const float* __restrict__ target,
                                                            int64_t batch, int64_t classes) {
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= batch) return;
    const float* l = logits + b * classes;
    const float* t = target + b * classes;
    float mx = l[0];
    for (int64_t c = 1; c < classes; ++c) mx = fmaxf(mx, l[c]);
    float sum = 0.0f;
    for (int64_t c = 0; c < classes; ++c) sum += expf(l[c] - mx);
    if constexpr (GRAD) {
        const float inv_batch = 1.0f / (float)batch;
        float* g = out + b * classes;
        for (int64_t c = 0; c < classes; ++c) g[c] = (expf(l[c] - mx) / sum - t[c]) * inv_batch;
    } else {
        const float lse = logf(sum) + mx;
        float loss = 0.0f;
        for (int64_t c = 0; c < classes; ++c) loss += -t[c] * (l[c] - lse);
        out[b] = loss;
    }
}

int cross_entropy_launch(bool grad, float* out, const float* logits, const float* target,
                         int64_t batch, int64_t classes) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(batch >= 0 && classes > 0, "cross_entropy: bad shape");
    if (batch == 0) return NRS_OK;
    NRS_ARG_CHECK(out && logits && target, "cross_entropy: null pointer");
    NRS_ARG_CHECK((batch + 255) / 256 <= INT32_MAX, "cross_entropy: batch too large");
    const dim3 grid((unsigned)((batch + 255) / 256));
    if (grad)
        hipLaunchKernelGGL(cross_entropy_kernel<true>, grid, dim3(256), 0, stream(), out, logits,
                           target, batch, classes);
    else
        hipLaunchKernelGGL(cross_entropy_kernel<false>, grid, dim3(256), 0, stream(), out, logits,
                           target, batch, classes);
    NRS_LAUNCH_CHECK(grad ? "cross_entropy backward" : "cross_entropy forward");
    return NRS_OK;
}

}  // namespace
}  // namespace nrs

using nrs::nrs_heads_impl;
using nrs::nrs_slice_cols_backward_impl;
using nrs::cross_entropy_launch;

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

int nrs_cross_entropy_forward(float* row_loss, const float* logits, const float* target,
                              int64_t batch, int64_t classes) {
    return cross_entropy_launch(false, row_loss, logits, target, batch, classes);
}

int nrs_cross_entropy_backward(float* grad, const float* logits, const float* target,
                               int64_t batch, int64_t classes) {
    return cross_entropy_launch(true, grad, logits, target, batch, classes);
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

int nrs_add_layernorm_forward(float* out, float* x_norm, float* inv_std, const float* in,
                              const float* in2, const float* gamma, const float* beta,
                              int64_t rows, int64_t features, float eps) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(rows >= 0 && features > 0, "layernorm: bad shape");
    if (rows == 0) return NRS_OK;
    NRS_ARG_CHECK(out && x_norm && inv_std && in && gamma && beta, "layernorm: null pointer");
    const int64_t F = features;
    auto fn = F <= 64    ? nrs::layernorm_fwd_kernel<1>
              : F <= 128 ? nrs::layernorm_fwd_kernel<2>
              : F <= 256 ? nrs::layernorm_fwd_kernel<4>
              : F <= 512 ? nrs::layernorm_fwd_kernel<8>
                         : nrs::layernorm_fwd_kernel<0>;
    hipLaunchKernelGGL(fn, dim3(nrs::rows_grid(rows)), dim3(256), 0, nrs::stream(), out, x_norm,
                       inv_std, in, in2, gamma, beta, rows, F, eps);
    NRS_LAUNCH_CHECK("layernorm forward");
    return NRS_OK;
}

int nrs_layernorm_forward(float* out, float* x_norm, float* inv_std, const float* in,
                          const float* gamma, const float* beta, int64_t rows, int64_t features,
                          float eps) {
    return nrs_add_layernorm_forward(out, x_norm, inv_std, in, nullptr, gamma, beta, rows,
                                     features, eps);
}

int nrs_layernorm_backward(float* dinput, float* dgamma, float* dbeta, const float* grad,
                           const float* gamma, const float* x_norm, const float* inv_std,
                           int64_t rows, int64_t features, float acc) {
    return nrs_add_layernorm_backward(dinput, nullptr, dgamma, dbeta, grad, gamma, x_norm, inv_std,
                                      rows, features, acc, 0.0f, acc);
}

int nrs_add_layernorm_backward(float* da, float* db, float* dgamma, float* dbeta, const float* grad,
                               const float* gamma, const float* x_norm, const float* inv_std,
                               int64_t rows, int64_t features, float beta_a, float beta_b,
                               float beta_params) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(db == nullptr || da != nullptr, "layernorm backward: second input gradient "
                                                  "without the first");
    float* dinput = da;
    const float acc = beta_params;
    NRS_ARG_CHECK(rows >= 0 && features > 0, "layernorm backward: bad shape");
    const int64_t F = features;
    if (rows == 0) {
        // no rows: the parameter gradients are the empty sums, 0 + acc * old
        if (dgamma || dbeta) {
            NRS_ARG_CHECK((F + 63) / 64 <= INT32_MAX, "layernorm backward: too large");
            hipLaunchKernelGGL(nrs::layernorm_param_combine_kernel, dim3((unsigned)((F + 63) / 64)),
                               dim3(64 * nrs::kLnGroups), 0, nrs::stream(), dgamma, dbeta,
                               nullptr, nullptr, int64_t(0), F, acc);
            NRS_LAUNCH_CHECK("layernorm backward (parameters)");
        }
        return NRS_OK;
    }
    NRS_ARG_CHECK(grad && x_norm, "layernorm backward: null pointer");
    if ((dinput || dgamma || dbeta) && F <= 512) {
        // the input gradient and the parameter partials from one pass over
        // grad and x_norm, then the chunk partials combined
        NRS_ARG_CHECK(!dinput || (gamma && inv_std), "layernorm backward: null gamma or inv_std");
        int64_t rc = 8;
        if ((rows + rc - 1) / rc > INT32_MAX / 2) rc = ((rows + INT32_MAX / 2 - 1) / (INT32_MAX / 2) + 7) / 8 * 8;
        const int64_t chunks = (rows + rc - 1) / rc;
        const bool params = dgamma || dbeta;
        float* part = nullptr;
        if (params) {
            part = nrs::workspace(sizeof(float) * 2 * (size_t)(chunks * F), 0);
            if (!part) return NRS_ERR_ALLOC;
        }
        auto fn = F <= 64    ? nrs::layernorm_bwd_fused_kernel<1>
                  : F <= 128 ? nrs::layernorm_bwd_fused_kernel<2>
                  : F <= 256 ? nrs::layernorm_bwd_fused_kernel<4>
                             : nrs::layernorm_bwd_fused_kernel<8>;
        hipLaunchKernelGGL(fn, dim3((unsigned)chunks), dim3(256), 0, nrs::stream(), dinput, db,
                           part, params ? part + chunks * F : nullptr, grad, gamma, x_norm,
                           inv_std, rows, F, rc, beta_a, beta_b);
        NRS_LAUNCH_CHECK("layernorm backward (input and parameter partials)");
        if (!params) return NRS_OK;
        hipLaunchKernelGGL(nrs::layernorm_param_combine_kernel, dim3((unsigned)((F + 63) / 64)),
                           dim3(64 * nrs::kLnGroups), 0, nrs::stream(), dgamma, dbeta, part,
                           part + chunks * F, chunks, F, acc);
        NRS_LAUNCH_CHECK("layernorm backward (parameters)");
        return NRS_OK;
    }
    if (dinput) {
        NRS_ARG_CHECK(gamma && inv_std, "layernorm backward: null gamma or inv_std");
        hipLaunchKernelGGL(nrs::layernorm_dx_kernel, dim3(nrs::rows_grid(rows)), dim3(256), 0,
                           nrs::stream(), dinput, db, grad, gamma, x_norm, inv_std, rows, F,
                           beta_a, beta_b);
        NRS_LAUNCH_CHECK("layernorm backward (input)");
    }
    if (dgamma || dbeta) {
        int64_t rc = nrs::kLnRows;
        if ((rows + rc - 1) / rc > 65535) rc = ((rows + 65534) / 65535 + 7) / 8 * 8;
        const int64_t chunks = (rows + rc - 1) / rc;
        const int64_t fb = (F + 255) / 256, fb64 = (F + 63) / 64;
        NRS_ARG_CHECK(fb64 <= INT32_MAX && chunks <= 65535, "layernorm backward: too large");
        float* part = nrs::workspace(sizeof(float) * 2 * (size_t)(chunks * F), 0);
        if (!part) return NRS_ERR_ALLOC;
        hipLaunchKernelGGL(nrs::layernorm_param_partial_kernel, dim3((unsigned)fb, (unsigned)chunks),
                           dim3(256), 0, nrs::stream(), part, part + chunks * F, grad, x_norm, rows,
                           F, rc);
        NRS_LAUNCH_CHECK("layernorm backward (parameter partials)");
        hipLaunchKernelGGL(nrs::layernorm_param_combine_kernel, dim3((unsigned)fb64),
                           dim3(64 * nrs::kLnGroups), 0, nrs::stream(), dgamma, dbeta, part,
                           part + chunks * F, chunks, F, acc);
        NRS_LAUNCH_CHECK("layernorm backward (parameters)");
    }
    return NRS_OK;
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
