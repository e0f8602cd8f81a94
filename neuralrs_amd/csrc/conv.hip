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
// How the whole-op entry points differ from the reference's launch sequence
// (the arithmetic is the same products and f32 sums, in another order):
//  * forward is ONE implicit-GEMM kernel: the GEMM's B operand gathers the
//    column matrix straight from the NCHW input (no cols buffer, no second
//    pass) and its epilogue adds the bias and stores NCHW (no col2out);
//  * the stride-1 input gradient is the implicit-GEMM convolution of the
//    output gradient with the flipped, channel-transposed weights and padding
//    k-1-pad, added into dinput (replaces out2mm + TN GEMM + dcols + col2im;
//    other strides keep that explicit sequence);
//  * the weight gradient reads the output gradient in place as an NCHW
//    operand (no out2mm) against the im2col matrix, split-K with a
//    deterministic slice reduction instead of float atomics;
//  * the bias gradient is a two-level deterministic reduction instead of
//    c_out serial threads;
//  * all three gradients are added into the caller's buffers (beta = 1),
//    replacing the reference's three accumulate passes.
#include <algorithm>

#include "buffer_ops.hpp"
#include "conv_slab.hpp"
#include "gemm_call.hpp"

namespace nrs {

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

// Same column matrix, four consecutive columns per thread written with one
// 128-bit store: blockIdx.y is the row (ic, i, j), so its decomposition is
// uniform across the workgroup, and all column index math is 32-bit. Needs
// P % 4 == 0 (four columns never straddle an image) and sizes < 2^31.
__global__ __launch_bounds__(256) void im2col_rows_kernel(float* __restrict__ cols,
                                                          const float* __restrict__ input,
                                                          int c_in, int in_h, int in_w, int kh,
                                                          int kw, int stride, int pad,
                                                          FastDiv div_P, FastDiv div_ow,
                                                          int width4) {
    const int row = blockIdx.y;
    const int j = row % kw;
    const int i = (row / kw) % kh;
    const int ic = row / (kw * kh);
    const float* src = input + (int64_t)ic * in_h * in_w;
    float4* dst = reinterpret_cast<float4*>(cols + (int64_t)row * width4 * 4);
    for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < width4; t += gridDim.x * blockDim.x) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            uint32_t ni, pp, oy, ox;
            fast_divmod((uint32_t)(4 * t + u), div_P, ni, pp);
            fast_divmod(pp, div_ow, oy, ox);
            const int iy = (int)oy * stride + i - pad, ix = (int)ox * stride + j - pad;
            const bool ok = ((unsigned)iy < (unsigned)in_h) & ((unsigned)ix < (unsigned)in_w);
            const float x = src[ok ? ((int64_t)ni * c_in * in_h + iy) * in_w + ix : 0];
            v[u] = ok ? x : 0.0f;
        }
        dst[t] = make_float4(v[0], v[1], v[2], v[3]);
    }
}

// wf[ic, oc, i, j] = w[oc, ic, kh-1-i, kw-1-j]: the weights of the
// convolution whose output is the stride-1 input gradient.
__global__ __launch_bounds__(256) void flip_weights_kernel(float* __restrict__ wf,
                                                           const float* __restrict__ w, int c_out,
                                                           int c_in, int kh, int kw) {
    const int total = c_out * c_in * kh * kw;
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
        const int j = e % kw;
        const int i = (e / kw) % kh;
        const int oc = (e / (kw * kh)) % c_out;
        const int ic = e / (kw * kh * c_out);
        wf[e] = w[((oc * c_in + ic) * kh + (kh - 1 - i)) * kw + (kw - 1 - j)];
    }
}

// Direct convolution for layers with very few input taps (c_in*kh*kw <=
// kDirectTaps), e.g. a first layer over grayscale images, where a GEMM tile
// would be mostly padding and the layer is bound by writing its output. One
// thread per output pixel: its taps are loaded once (branch-free: clamped
// index, then zeroed), then it produces a block of up to `ocb` (<=
// kDirectOcBlock) output channels (blockIdx.y) from wave-uniform weights, so
// consecutive lanes store consecutive pixels of each channel plane (with
// non-temporal stores: the output is not read again here and would evict the
// input from L2). The sum runs over the taps in (ic, i, j) order. 32-bit
// indexing (checked on the host).
constexpr int kDirectTaps = 32, kDirectOcBlock = 64;

template <int TAPS>
__global__ __launch_bounds__(256) void conv_fwd_direct_kernel(
    float* __restrict__ out, const float* __restrict__ input, const float* __restrict__ weight,
    const float* __restrict__ bias, int N, int c_in, int in_h, int in_w, int c_out, int kh, int kw,
    int stride, int pad, int ocb, FastDiv div_P, FastDiv div_ow) {
    // tap t = (ic*kh + i)*kw + j: offset inside one image and (i, j); the
    // block's weights (zero past the taps) and biases
    constexpr int WROW = (TAPS + 3) & ~3;  // whole float4s per weight row
    __shared__ int2 tab[TAPS];
    __shared__ __attribute__((aligned(16))) float wsh[kDirectOcBlock][WROW];
    __shared__ float bsh[kDirectOcBlock];
    const int taps = c_in * kh * kw;
    const int oc0 = blockIdx.y * ocb;
    const int oc1 = min(c_out, oc0 + ocb);
    if (threadIdx.x < TAPS) {
        const int t = threadIdx.x < taps ? threadIdx.x : 0;
        const int j = t % kw, i = (t / kw) % kh, ic = t / (kw * kh);
        tab[threadIdx.x] = make_int2((ic * in_h + i) * in_w + j, i | (j << 16));
    }
    // weights and biases: every load issued before any store (zero-returning
    // buffer loads need no select, which would make each load wait for the
    // previous one)
    constexpr int WN = kDirectOcBlock * WROW, WPT = (WN + 255) / 256;
    const auto rw = buffer_rsrc(weight, (int64_t)c_out * taps * 4);
    const auto rb = buffer_rsrc(bias ? bias : weight, bias ? (int64_t)c_out * 4 : 0);
    float wv[WPT];
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
        const int e = threadIdx.x + 256 * k, o = e / WROW, t = e - o * WROW;
        const bool ok = (e < WN) & (oc0 + o < oc1) & (t < taps);  // (rows past ocb stay 0)
        wv[k] = buffer_load1(rw, ok ? ((oc0 + o) * taps + t) * 4 : kOutOfRange);
    }
    const int bo = oc0 + (int)threadIdx.x;
    const bool bok = (threadIdx.x < kDirectOcBlock) & (bo < oc1);
    const float bv = buffer_load1(rb, bok ? bo * 4 : kOutOfRange);
#pragma unroll
    for (int k = 0; k < WPT; ++k)
        if (threadIdx.x + 256 * k < WN) (&wsh[0][0])[threadIdx.x + 256 * k] = wv[k];
    if (threadIdx.x < kDirectOcBlock) bsh[threadIdx.x] = bv;
    __syncthreads();
    const int P = (int)div_P.d, total = N * P;
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += gridDim.x * blockDim.x) {
        uint32_t n, pp, oy, ox;
        fast_divmod((uint32_t)idx, div_P, n, pp);
        fast_divmod(pp, div_ow, oy, ox);
        const int iy0 = (int)oy * stride - pad, ix0 = (int)ox * stride - pad;
        const float* img = input + (int64_t)n * c_in * in_h * in_w;
        const int base = iy0 * in_w + ix0;
        float x[TAPS];
#pragma unroll
        for (int t = 0; t < TAPS; ++t) {
            const int2 e = tab[t];
            const int i = e.y & 0xffff, j = e.y >> 16;
            const bool ok = (t < taps) & ((unsigned)(iy0 + i) < (unsigned)in_h) &
                            ((unsigned)(ix0 + j) < (unsigned)in_w);
            const float v = img[ok ? base + e.x : 0];
            x[t] = ok ? v : 0.0f;
        }
        float* o = out + (int64_t)n * c_out * P + pp;
        // weights past the taps are zero (and so are the taps): no guard, so
        // the weight reads are not serialised behind per-tap branches
#pragma unroll 2
        for (int oc = oc0; oc < oc1; ++oc) {
            const float* w = wsh[oc - oc0];
            float acc = 0.0f;
#pragma unroll
            for (int t = 0; t < TAPS; ++t) acc += w[t] * x[t];
            __builtin_nontemporal_store(acc + bsh[oc - oc0], o + (int64_t)oc * P);
        }
    }
}

// The same direct convolution for "same"-padded 3x3 stride-1 layers with
// CIN <= 3 input channels and rows of a multiple of 4 pixels: one thread per
// quad of 4 consecutive output pixels of one row and QOC output channels, so
// each channel leaves as one 128-bit store per lane (a wave writes 1 KiB of a
// channel plane per store). The quad's 3*CIN input row segments of 6 floats
// are read as an aligned 128-bit load plus its two neighbours, issued before
// the weights are staged, so the input and weight round trips overlap. Same
// sum order as conv_fwd_direct_kernel: taps in (ic, i, j) order from zero,
// then + bias.
// Output channels per thread: 8 for the plain forward, 4 for the pooled one
// (cfg3 conv1 + ReLU + pool: 5.9 -> 5.4 us, 2 channels 6.6 us; the plain
// forward: 4.7 us at 8, 4.8 at 4, 5.8 at 2).
constexpr int kQuadOcFwd = 8, kQuadOcPool = 4;
// Threads per workgroup of the pixel-quad forward: one wave, so the grid
// spreads evenly over the CUs (cfg3 conv1: 1568 workgroups, ~6 per CU; in
// workgroups of 256 threads, 392 of them left 136 CUs with twice the work).
constexpr int kQuadThreads = 64;

template <int CIN, int QOC>
__global__ __launch_bounds__(kQuadThreads) void conv_fwd_quad_kernel(
    float* __restrict__ out, const float* __restrict__ input, const float* __restrict__ weight,
    const float* __restrict__ bias, int N, int H, int W, int c_out, FastDiv div_qimg,
    FastDiv div_qrow) {
    constexpr int ROWS = 3 * CIN, TAPS = 9 * CIN;
    __shared__ __attribute__((aligned(16))) float wsh[QOC][TAPS];
    __shared__ float bsh[QOC];
    const int tid = threadIdx.x;
    const int P = H * W, oc0 = blockIdx.y * QOC;
    const int64_t quads = (int64_t)N * (P >> 2);
    const int g = blockIdx.x * kQuadThreads + tid;
    const bool valid = g < quads;
    uint32_t n, qq, oy, qx;
    fast_divmod((uint32_t)(valid ? g : 0), div_qimg, n, qq);
    fast_divmod(qq, div_qrow, oy, qx);
    const int ox = 4 * (int)qx;
    // input row segments: columns ox-1 .. ox+4 of rows oy-1 .. oy+1
    const auto rx = buffer_rsrc(input, (int64_t)N * CIN * P * 4);
    float seg[ROWS][6];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        const int ic = r / 3, iy = (int)oy + r % 3 - 1;
        const bool rok = valid & ((unsigned)iy < (unsigned)H);
        const int base = (((int)n * CIN + ic) * H + iy) * W + ox;
        const f32x4 mid = buffer_load4(rx, rok ? base * 4 : kOutOfRange);
        seg[r][0] = buffer_load1(rx, (rok & (ox > 0)) ? (base - 1) * 4 : kOutOfRange);
        seg[r][5] = buffer_load1(rx, (rok & (ox + 4 < W)) ? (base + 4) * 4 : kOutOfRange);
#pragma unroll
        for (int u = 0; u < 4; ++u) seg[r][1 + u] = mid[u];
    }
    // this block's weights (zero past c_out) and biases
    constexpr int WN = QOC * TAPS, WPT = (WN + kQuadThreads - 1) / kQuadThreads;
    const auto rw = buffer_rsrc(weight, (int64_t)c_out * TAPS * 4);
    const auto rb = buffer_rsrc(bias ? bias : weight, bias ? (int64_t)c_out * 4 : 0);
    float wv[WPT];
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
        const int e = tid + kQuadThreads * k;
        wv[k] = buffer_load1(rw, e < WN ? (oc0 * TAPS + e) * 4 : kOutOfRange);
    }
    const float bv = buffer_load1(rb, tid < QOC ? (oc0 + tid) * 4 : kOutOfRange);
#pragma unroll
    for (int k = 0; k < WPT; ++k)
        if (tid + kQuadThreads * k < WN) (&wsh[0][0])[tid + kQuadThreads * k] = wv[k];
    if (tid < QOC) bsh[tid] = bv;
    __syncthreads();
    if (!valid) return;
    float* o = out + ((int64_t)n * c_out + oc0) * P + (int)oy * W + ox;
    const int noc = min(QOC, c_out - oc0);
#pragma unroll
    for (int oc = 0; oc < QOC; ++oc) {
        if (oc >= noc) break;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                const float w = wsh[oc][r * 3 + j];
#pragma unroll
                for (int u = 0; u < 4; ++u) acc[u] += w * seg[r][u + j];
            }
        const float b = bsh[oc];
        __builtin_nontemporal_store(acc + b, reinterpret_cast<f32x4*>(o + (int64_t)oc * P));
    }
}

// Forward of a "same" 3x3 layer followed by 2x2 max pooling of stride 2: the
// conv2d then MaxPool2d of a CNN (src/cuda/nn/conv.rs:244-277,
// src/cuda/nn/maxpool.rs:18-46) in one pass. A thread owns a 4-wide, 2-tall
// block of the conv output, i.e. two pooled outputs, for QOC output channels;
// its input is 4 rows of 6 floats per input channel. Each conv value is
// computed as conv_fwd_quad_kernel computes it (same products in the same
// order, then + bias); each 2x2 window keeps the first maximum in scan order
// and records the conv output's flat element index, as maxpool_forward does.
// The conv output is written only when out is set; the pooled values and
// indices leave as 64-bit stores.
template <int CIN, int QOC>
__global__ __launch_bounds__(kQuadThreads) void conv_fwd_pool_quad_kernel(
    float* __restrict__ pooled, int32_t* __restrict__ argmax, float* __restrict__ out,
    const float* __restrict__ input, const float* __restrict__ weight,
    const float* __restrict__ bias, int N, int H, int W, int c_out, int relu, FastDiv div_bimg,
    FastDiv div_brow) {
    constexpr int ROWS = 4 * CIN, TAPS = 9 * CIN;
    __shared__ __attribute__((aligned(16))) float wsh[QOC][TAPS];
    __shared__ float bsh[QOC];
    const int tid = threadIdx.x;
    const int P = H * W, PW = W >> 1, PP = (H >> 1) * PW, oc0 = blockIdx.y * QOC;
    const int64_t blocks = (int64_t)N * (H >> 1) * (W >> 2);
    const int g = blockIdx.x * kQuadThreads + tid;
    const bool valid = g < blocks;
    uint32_t n, qq, py, qx;
    fast_divmod((uint32_t)(valid ? g : 0), div_bimg, n, qq);
    fast_divmod(qq, div_brow, py, qx);
    const int oy = 2 * (int)py, ox = 4 * (int)qx;
    // input row segments: columns ox-1 .. ox+4 of rows oy-1 .. oy+2
    const auto rx = buffer_rsrc(input, (int64_t)N * CIN * P * 4);
    float seg[ROWS][6];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        const int ic = r / 4, iy = oy + r % 4 - 1;
        const bool rok = valid & ((unsigned)iy < (unsigned)H);
        const int base = (((int)n * CIN + ic) * H + iy) * W + ox;
        const f32x4 mid = buffer_load4(rx, rok ? base * 4 : kOutOfRange);
        seg[r][0] = buffer_load1(rx, (rok & (ox > 0)) ? (base - 1) * 4 : kOutOfRange);
        seg[r][5] = buffer_load1(rx, (rok & (ox + 4 < W)) ? (base + 4) * 4 : kOutOfRange);
#pragma unroll
        for (int u = 0; u < 4; ++u) seg[r][1 + u] = mid[u];
    }
    constexpr int WN = QOC * TAPS, WPT = (WN + kQuadThreads - 1) / kQuadThreads;
    const auto rw = buffer_rsrc(weight, (int64_t)c_out * TAPS * 4);
    const auto rb = buffer_rsrc(bias ? bias : weight, bias ? (int64_t)c_out * 4 : 0);
    float wv[WPT];
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
        const int e = tid + kQuadThreads * k;
        wv[k] = buffer_load1(rw, e < WN ? (oc0 * TAPS + e) * 4 : kOutOfRange);
    }
    const float bv = buffer_load1(rb, tid < QOC ? (oc0 + tid) * 4 : kOutOfRange);
#pragma unroll
    for (int k = 0; k < WPT; ++k)
        if (tid + kQuadThreads * k < WN) (&wsh[0][0])[tid + kQuadThreads * k] = wv[k];
    if (tid < QOC) bsh[tid] = bv;
    __syncthreads();
    if (!valid) return;
    const int noc = min(QOC, c_out - oc0);
#pragma unroll
    for (int oc = 0; oc < QOC; ++oc) {
        if (oc >= noc) break;
        f32x4 a0 = {0.0f, 0.0f, 0.0f, 0.0f}, a1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ic = 0; ic < CIN; ++ic)
#pragma unroll
            for (int i = 0; i < 3; ++i)
#pragma unroll
                for (int j = 0; j < 3; ++j) {
                    const float w = wsh[oc][(ic * 3 + i) * 3 + j];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        a0[u] += w * seg[ic * 4 + i][u + j];
                        a1[u] += w * seg[ic * 4 + i + 1][u + j];
                    }
                }
        const float b = bsh[oc];
        const f32x4 v0 = a0 + b, v1 = a1 + b;
        const int plane = ((int)n * c_out + oc0 + oc) * P;
        const int e00 = plane + oy * W + ox;  // flat index of (oy, ox)
        // the pooled values: of relu(conv) when a ReLU sits between the two
        // (vrelu's x > 0 ? x : 0), else of the conv values
        f32x4 r0 = v0, r1 = v1;
        if (relu) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                r0[u] = v0[u] > 0.0f ? v0[u] : 0.0f;
                r1[u] = v1[u] > 0.0f ? v1[u] : 0.0f;
            }
        }
        f32x2 pv;
        int32_t pi[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {  // windows of columns 2h, 2h + 1
            float best = r0[2 * h];
            int bi = e00 + 2 * h;
            if (r0[2 * h + 1] > best) { best = r0[2 * h + 1]; bi = e00 + 2 * h + 1; }
            if (r1[2 * h] > best) { best = r1[2 * h]; bi = e00 + W + 2 * h; }
            if (r1[2 * h + 1] > best) { best = r1[2 * h + 1]; bi = e00 + W + 2 * h + 1; }
            pv[h] = best;
            pi[h] = bi;
        }
        const int64_t po = ((int64_t)n * c_out + oc0 + oc) * PP + (int)py * PW + 2 * (int)qx;
        *reinterpret_cast<f32x2*>(pooled + po) = pv;
        *reinterpret_cast<int2*>(argmax + po) = make_int2(pi[0], pi[1]);
        if (out) {
            __builtin_nontemporal_store(v0, reinterpret_cast<f32x4*>(out + e00));
            __builtin_nontemporal_store(v1, reinterpret_cast<f32x4*>(out + e00 + W));
        }
    }
}

// Direct input gradient for c_in <= kDirectCin (any stride): one thread per
// input pixel accumulates, for its c_in channels, every (oc, i, j) whose
// window covers it, with weights (c_out*c_in*kh*kw <= kDirectWeights) from
// LDS. The covering output positions are found once; the output channels
// are then taken kDirectBatch at a time with all their loads issued before
// any is used. dinput = that sum + beta * dinput.
constexpr int kDirectCin = 4, kDirectWeights = 8192, kDirectBatch = 8, kDirectWin = 9;

__global__ __launch_bounds__(256) void conv_dgrad_direct_kernel(
    float* __restrict__ dinput, const float* __restrict__ grad, const float* __restrict__ weight,
    int N, int c_in, int in_h, int in_w, int c_out, int kh, int kw, FastDiv div_stride, int pad,
    int out_h, int out_w, FastDiv div_HW, FastDiv div_inw, float beta) {
    __shared__ float wsh[kDirectWeights];
    const int wn = c_out * c_in * kh * kw;
    for (int e = threadIdx.x; e < wn; e += blockDim.x) wsh[e] = weight[e];
    __syncthreads();
    const int HW = in_h * in_w, total = N * HW, P = out_h * out_w;
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += gridDim.x * blockDim.x) {
        uint32_t n, pix, y, x;
        fast_divmod((uint32_t)idx, div_HW, n, pix);
        fast_divmod(pix, div_inw, y, x);
        // covering windows: output offset and tap index (i*kw + j), at most
        // kDirectWin of them (the host checks kh*kw <= kDirectWin)
        int off[kDirectWin], tap[kDirectWin];
        int nwin = 0;
        for (int i = 0; i < kh; ++i) {
            const int oyn = (int)y + pad - i;
            if (oyn < 0) continue;
            uint32_t oy, ry;
            fast_divmod((uint32_t)oyn, div_stride, oy, ry);
            if (ry != 0 || (int)oy >= out_h) continue;
            for (int j = 0; j < kw; ++j) {
                const int oxn = (int)x + pad - j;
                if (oxn < 0) continue;
                uint32_t ox, rx;
                fast_divmod((uint32_t)oxn, div_stride, ox, rx);
                if (rx != 0 || (int)ox >= out_w) continue;
                off[nwin] = (int)oy * out_w + (int)ox;
                tap[nwin] = i * kw + j;
                ++nwin;
            }
        }
        float acc[kDirectCin] = {0.0f, 0.0f, 0.0f, 0.0f};
        const float* gn = grad + n * c_out * P;
        for (int oc0 = 0; oc0 < c_out; oc0 += kDirectBatch) {
            float gv[kDirectBatch][kDirectWin];
#pragma unroll
            for (int b = 0; b < kDirectBatch; ++b)
#pragma unroll
                for (int w = 0; w < kDirectWin; ++w) {
                    const bool ok = (oc0 + b < c_out) & (w < nwin);
                    const float v = gn[ok ? (oc0 + b) * P + off[w] : 0];
                    gv[b][w] = ok ? v : 0.0f;
                }
#pragma unroll
            for (int b = 0; b < kDirectBatch; ++b)
#pragma unroll
                for (int w = 0; w < kDirectWin; ++w)
                    if ((oc0 + b < c_out) & (w < nwin))
#pragma unroll
                        for (int ic = 0; ic < kDirectCin; ++ic)
                            if (ic < c_in)
                                acc[ic] += wsh[((oc0 + b) * c_in + ic) * kh * kw + tap[w]] * gv[b][w];
        }
#pragma unroll
        for (int ic = 0; ic < kDirectCin; ++ic)
            if (ic < c_in) {
                float* dst = dinput + (n * c_in + ic) * HW + pix;
                float v = acc[ic];
                if (beta != 0.0f) v = v + beta * *dst;
                *dst = v;
            }
    }
}

// The stride-1 input gradient of a "same" 3x3 layer with CIN <= 4 input
// channels and rows of a multiple of 4 pixels (conv.rs:304-312 without the
// dcols matrix). A workgroup owns one image and a band of `band` input rows;
// a thread owns a quad of 4 pixels of one row in one of `groups` output-
// channel groups. Per chunk of kQuadDgradOc output channels the block stages
// the gradient rows the band's windows touch (band + 2 rows of `pitch`
// floats: the row at columns 4 .. 4+W-1 and zero around it, each row copied
// as 128-bit loads and stores) and the chunk's weights; a thread then reads,
// per (oc, i), its six gradient values as one 128-bit and two 32-bit LDS
// reads and forms
//   dinput[c, y, x] += grad[oc, y + 1 - i, x + 1 - j] * W[oc, c, i, j]
// for its 4 pixels, over (oc, i, j) in order. The groups' sums are added in
// group order, then to the old dinput.
constexpr int kQuadDgradOc = 32, kQuadDgradStage = 12;

template <int CIN>
__global__ __launch_bounds__(256) void conv_dgrad_quad_kernel(
    float* __restrict__ dinput, const float* __restrict__ grad, const float* __restrict__ weight,
    int c_in, int H, int W, int c_out, int band, int bands, int pitch, int groups, int qpg,
    int lq, FastDiv div_slots, FastDiv div_pq) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int tid = threadIdx.x;
    const int n = blockIdx.x / bands, y0 = (blockIdx.x - n * bands) * band;
    const int rows = min(band, H - y0);
    const int rrows = band + 2, tile = rrows * pitch, HW = H * W;
    float* gt = lds;                                       // [oc][rrows][pitch]
    float* wsh = lds + kQuadDgradOc * tile;                // [oc][CIN][9]
    float* red = wsh + kQuadDgradOc * CIN * 9;             // [groups][qpg][CIN][4]
    // this thread's quad and channel group: a row's quads sit in a run of
    // 2^lq lanes (a power of two >= W/4; the run's extra lanes idle), so no
    // row straddles two waves
    const int grp = tid / qpg, q = tid - grp * qpg, nq = W >> 2;
    const int yy = q >> lq, qx = q & ((1 << lq) - 1);
    const bool live = grp < groups && yy < rows && qx < nq;
    const int x0 = 4 * qx;
    const float* gimg = grad + (int64_t)n * c_out * HW;
    const auto rg = buffer_rsrc(gimg, (int64_t)c_out * HW * 4);
    const auto rw = buffer_rsrc(weight, (int64_t)c_out * c_in * 9 * 4);
    float acc[CIN][4] = {};
    const int slots = rrows * (pitch >> 2);  // float4 slots per channel tile
    for (int oc0 = 0; oc0 < c_out; oc0 += kQuadDgradOc) {
        const int nch = min(kQuadDgradOc, c_out - oc0);
        if (oc0) __syncthreads();
        // stage: float4 slot e of channel tile ch holds columns 4*k .. 4*k+3
        // of tile row r, i.e. gradient row y0 - 1 + r, columns 4*k - 4 ..;
        // a round issues all its loads (and, first, the chunk's weights
        // [o][c][tap], zero past c_in and c_out) before any LDS store
        constexpr int WPT = (kQuadDgradOc * CIN * 9 + 255) / 256;
        for (int e0 = 0; e0 < nch * slots; e0 += 256 * kQuadDgradStage) {
            float wv[WPT];
            if (e0 == 0) {
#pragma unroll
                for (int k = 0; k < WPT; ++k) {
                    const int e = tid + 256 * k;
                    const int o = e / (CIN * 9), rem = e - o * CIN * 9, c = rem / 9, t = rem - c * 9;
                    const bool ok = (o < nch) & (c < c_in) & (e < kQuadDgradOc * CIN * 9);
                    wv[k] = buffer_load1(rw, ok ? (((oc0 + o) * c_in + c) * 9 + t) * 4 : kOutOfRange);
                }
            }
            f32x4 v[kQuadDgradStage];
            int dst[kQuadDgradStage];
#pragma unroll
            for (int u = 0; u < kQuadDgradStage; ++u) {
                const int e = e0 + u * 256 + tid;
                uint32_t ch, sl, r, k;
                fast_divmod((uint32_t)e, div_slots, ch, sl);
                fast_divmod(sl, div_pq, r, k);
                const int gy = y0 - 1 + (int)r, gx = 4 * (int)k - 4;
                const bool ok = (e < nch * slots) & ((unsigned)gy < (unsigned)H) & (gx >= 0) & (gx < W);
                v[u] = buffer_load4(rg, ok ? (((oc0 + (int)ch) * H + gy) * W + gx) * 4 : kOutOfRange);
                dst[u] = e < nch * slots ? (int)ch * tile + (int)r * pitch + 4 * (int)k : -1;
            }
            if (e0 == 0) {
#pragma unroll
                for (int k = 0; k < WPT; ++k)
                    if (tid + 256 * k < kQuadDgradOc * CIN * 9) wsh[tid + 256 * k] = wv[k];
            }
#pragma unroll
            for (int u = 0; u < kQuadDgradStage; ++u)
                if (dst[u] >= 0) *reinterpret_cast<f32x4*>(gt + dst[u]) = v[u];
        }
        __syncthreads();
        if (live) {
            for (int o = grp; o < nch; o += groups) {
                const float* gr0 = gt + o * tile + x0 + 4;
                const float* wo = wsh + o * CIN * 9;
#pragma unroll
                for (int i = 0; i < 3; ++i) {
                    // gradient row y + 1 - i = tile row (yy + 2 - i)
                    const float* gr = gr0 + (yy + 2 - i) * pitch;
                    const f32x4 mid = *reinterpret_cast<const f32x4*>(gr);
                    // the outer neighbours are the adjacent quads' edge values
                    // (the next and previous lanes: consecutive lanes own
                    // consecutive quads of a row), zero at the row's ends
                    // where the tile's halo is zero; wave shifts by one lane
                    // in place of two 32-bit LDS reads whose 4-float lane
                    // stride hit each bank four times
                    // (each element into a scalar first: a bit_cast of the
                    // vector element expression read element 0 for both)
                    const float m3 = mid[3], m0 = mid[0];
                    const float left = __builtin_bit_cast(
                        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, m3), 0x138, 0xf,
                                                           0xf, false));
                    const float right = __builtin_bit_cast(
                        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, m0), 0x130, 0xf,
                                                           0xf, false));
                    const float gv[6] = {qx == 0 ? 0.0f : left, mid[0], mid[1], mid[2], mid[3],
                                         qx == nq - 1 ? 0.0f : right};
#pragma unroll
                    for (int j = 0; j < 3; ++j)
#pragma unroll
                        for (int c = 0; c < CIN; ++c) {
                            const float w = wo[c * 9 + i * 3 + j];
                            // pixel x0 + u reads column x0 + u + 1 - j
#pragma unroll
                            for (int u = 0; u < 4; ++u) acc[c][u] += gv[u + 2 - j] * w;
                        }
                }
            }
        }
    }
    // the groups' sums in group order, then + old dinput
    __syncthreads();
    if (live) {
#pragma unroll
        for (int c = 0; c < CIN; ++c)
            *reinterpret_cast<f32x4*>(red + ((grp * qpg + q) * CIN + c) * 4) =
                f32x4{acc[c][0], acc[c][1], acc[c][2], acc[c][3]};
    }
    __syncthreads();
    if (grp != 0 || !live) return;
    float* drow = dinput + (int64_t)n * c_in * HW + (y0 + yy) * W + x0;
#pragma unroll
    for (int c = 0; c < CIN; ++c) {
        if (c >= c_in) break;
        f32x4 r = *reinterpret_cast<const f32x4*>(red + (q * CIN + c) * 4);
        for (int g2 = 1; g2 < groups; ++g2) r += *reinterpret_cast<const f32x4*>(red + ((g2 * qpg + q) * CIN + c) * 4);
        f32x4* d = reinterpret_cast<f32x4*>(drow + (int64_t)c * HW);
        *d = r + *d;
    }
}

// Stride-1 input gradient for c_in <= kDirectCin, from LDS. A workgroup owns
// one image and a band of `band` input rows; each thread owns kDgradRun
// adjacent pixels of one row. Per chunk of `occ` output channels the block
// stages the output-gradient rows the band's windows touch (band + kh - 1
// rows of `pitch` floats, zero outside the gradient) and the chunk's weights
// flipped along the row, wf[o][i][jj][c] = W[oc0+o, c, i, KW-1-jj]. The
// workgroup's threads form `groups` channel groups over the same pixel runs
// (more waves busy when a band has few runs); for each (oc, i) of its
// channels a thread reads the kDgradRun + KW - 1 gradient values its pixels'
// windows share once and forms
//   dinput[c, y, x] += grad[oc, y + pad - i, x + pad - KW + 1 + jj] * wf[oc][i][jj][c]
// for all its pixels (the reference's sum over (oc, i, j), j = KW-1-jj);
// the groups' sums are added in group order. dinput = that sum + dinput. KW is the exact kernel width and CIN covers
// c_in (1, or 4 with zero weights past c_in).
constexpr int kDgradRun = 4, kDgradStage = 12, kDgradWStage = 2;

template <int KW, int CIN>
__global__ __launch_bounds__(256) void conv_dgrad_small_kernel(
    float* __restrict__ dinput, const float* __restrict__ grad, const float* __restrict__ weight,
    int c_in, int in_h, int in_w, int c_out, int kh, int pad, int out_h, int out_w, int band,
    int bands, int occ, int ngx, int pitch, int groups, int tpg, FastDiv div_ngx,
    FastDiv div_kh) {
    constexpr int NG = kDgradRun + KW - 1;  // gradient values per (oc, i)
    // [occ][gr][pitch] gradient tile, then the chunk's flipped weights
    extern __shared__ __attribute__((aligned(16))) float gt[];
    const int n = blockIdx.x / bands, y0 = (blockIdx.x - n * bands) * band;
    const int rows = min(band, in_h - y0);
    const int gr = band + kh - 1, tile = gr * pitch, gw = in_w + KW - 1;
    const int oy_base = y0 + pad - (kh - 1), ox_base = pad - (KW - 1);
    const int P = out_h * out_w, HW = in_h * in_w;
    const float* gimg = grad + (int64_t)n * c_out * P;
    // `groups` channel groups of tpg threads (whole waves) cover the same
    // pixel runs, each over its share of every chunk's output channels
    const int grp = __builtin_amdgcn_readfirstlane((int)threadIdx.x / tpg);
    const int tig = (int)threadIdx.x - grp * tpg;
    uint32_t yy, xg;
    fast_divmod((uint32_t)tig, div_ngx, yy, xg);
    const bool live = (int)yy < rows;
    const int x0 = (int)xg * kDgradRun;
    // this thread's tile row for kernel row i is yy + kh - 1 - i
    const int tbase = ((live ? (int)yy : 0) + kh - 1) * pitch + x0;
    float acc[kDgradRun][CIN] = {};
    float* wsh = gt + ((occ * tile + 3) & ~3);
    // the input-gradient values this thread adds to (group 0 writes them),
    // loaded now so the final stores do not wait on a memory round trip
    // (Zero-returning buffer loads here and below: a select after a load
    // would make the compiler wait for it before issuing the next.)
    const int dpix = (y0 + (live ? (int)yy : 0)) * in_w + x0;
    float* drow = dinput + (int64_t)n * c_in * HW + dpix;
    const auto rd = buffer_rsrc(dinput + (int64_t)n * c_in * HW, (int64_t)c_in * HW * 4);
    float old[kDgradRun][CIN];
#pragma unroll
    for (int c = 0; c < CIN; ++c)
#pragma unroll
        for (int r = 0; r < kDgradRun; ++r) {
            const bool ok = live & (grp == 0) & (c < c_in) & (x0 + r < in_w);
            old[r][c] = buffer_load1(rd, ok ? (c * HW + dpix + r) * 4 : kOutOfRange);
        }
    const auto rw = buffer_rsrc(weight, (int64_t)c_out * c_in * kh * KW * 4);
    const auto rg = buffer_rsrc(gimg, (int64_t)c_out * P * 4);
    // this thread's staging items e = tid + k*256 over (channel, tile row,
    // column quad): its first item's position, and the advance of 256 items
    // as whole channels, rows and quads, applied with carries (no division
    // per item: a wave64 VALU instruction costs four cycles, and a division
    // some forty of them)
    const int quads = pitch >> 2, slots = gr * quads;
    const int ch_step = 256 / slots, slot_step = 256 - ch_step * slots;
    const int r_step = slot_step / quads, c4_step = slot_step - r_step * quads;
    const int ch_t = (int)threadIdx.x / slots, slot_t = (int)threadIdx.x - ch_t * slots;
    const int r_t = slot_t / quads, c4_t = slot_t - r_t * quads;
    for (int oc0 = 0; oc0 < c_out; oc0 += occ) {
        const int nch = min(occ, c_out - oc0);
        if (oc0) __syncthreads();
        const int items = nch * slots;
        // the chunk's flipped weights wf[o][i][jj][c]: up to kDgradWStage
        // entries per thread, loaded alongside the gradient rows
        const int wn = nch * kh * KW;  // (o, i, jj)
        float wv[kDgradWStage][CIN];
#pragma unroll
        for (int k = 0; k < kDgradWStage; ++k) {
            const int e = (int)threadIdx.x + k * 256;
            const int ee = min(e, wn - 1);
            const int oi = ee / KW, jj = ee - oi * KW;  // KW is a constant
            const int o = (int)fast_div((uint32_t)oi, div_kh), i = oi - o * kh;
            const int woff = ((oc0 + o) * c_in * kh + i) * KW + (KW - 1 - jj);
#pragma unroll
            for (int c = 0; c < CIN; ++c) {
                const bool ok = (e < wn) & (c < c_in);
                wv[k][c] = buffer_load1(rw, ok ? (woff + c * kh * KW) * 4 : kOutOfRange);
            }
        }
        // the chunk's gradient rows: every load of a batch before its stores
        int ch = ch_t, r = r_t, c4 = c4_t;
        for (int b0 = 0; b0 < items; b0 += 256 * kDgradStage) {
            f32x4 v[kDgradStage];
            int dst[kDgradStage];
#pragma unroll
            for (int u = 0; u < kDgradStage; ++u) {
                dst[u] = -1;
                if (b0 + u * 256 < items) {  // uniform
                    const int oy = oy_base + r, ox = ox_base + 4 * c4;
                    const bool row_ok = (ch < nch) & ((unsigned)oy < (unsigned)out_h);
                    const int goff = (oc0 + min(ch, nch - 1)) * P + oy * out_w + ox;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const bool ok = row_ok & ((unsigned)(ox + e) < (unsigned)out_w) &
                                        (4 * c4 + e < gw);
                        v[u][e] = buffer_load1(rg, ok ? (goff + e) * 4 : kOutOfRange);
                    }
                    if (ch < nch) dst[u] = ch * tile + r * pitch + 4 * c4;
                }
                c4 += c4_step;
                int carry = c4 >= quads;
                c4 -= carry ? quads : 0;
                r += r_step + carry;
                carry = r >= gr;
                r -= carry ? gr : 0;
                ch += ch_step + carry;
            }
#pragma unroll
            for (int u = 0; u < kDgradStage; ++u)
                if (dst[u] >= 0) *reinterpret_cast<f32x4*>(gt + dst[u]) = v[u];
            // nothing outstanding at the loop edge: the compiler would
            // otherwise wait for the loads above before the first row load
            __builtin_amdgcn_s_waitcnt(0);
        }
#pragma unroll
        for (int k = 0; k < kDgradWStage; ++k) {
            const int e = (int)threadIdx.x + k * 256;
            if (e < wn)
#pragma unroll
                for (int c = 0; c < CIN; ++c) wsh[e * CIN + c] = wv[k][c];
        }
        for (int e = threadIdx.x + 256 * kDgradWStage; e < wn; e += blockDim.x) {
            const int oi = e / KW, jj = e - oi * KW;
            const int o = oi / kh, i = oi - o * kh;
            const float* w = weight + ((int64_t)(oc0 + o) * c_in * kh + i) * KW + (KW - 1 - jj);
#pragma unroll
            for (int c = 0; c < CIN; ++c) wsh[e * CIN + c] = c < c_in ? w[(int64_t)c * kh * KW] : 0.0f;
        }
        __syncthreads();
        const int per = (nch + groups - 1) / groups;
        const int o_lo = min(nch, grp * per), o_hi = min(nch, o_lo + per);
        if (live) {
            // (o, i) steps in order over this group's channels; the gradient
            // row pointer moves up one row per kernel row and to the next
            // channel's tile after kh rows, the weights are contiguous per step
            const float* g = gt + o_lo * tile + tbase;
            const float* w = wsh + o_lo * kh * KW * CIN;
            int i = 0;
#pragma unroll 4
            for (int oi = o_lo * kh; oi < o_hi * kh; ++oi) {
                float gv[NG];
#pragma unroll
                for (int q = 0; q < NG; ++q) gv[q] = g[q];
#pragma unroll
                for (int jj = 0; jj < KW; ++jj)
#pragma unroll
                    for (int c = 0; c < CIN; ++c) {
                        const float wv = w[jj * CIN + c];
#pragma unroll
                        for (int r = 0; r < kDgradRun; ++r) acc[r][c] += gv[r + jj] * wv;
                    }
                w += KW * CIN;
                if (++i == kh) {
                    i = 0;
                    g += tile + (kh - 1) * pitch;
                } else {
                    g -= pitch;
                }
            }
        }
    }
    if (groups > 1) {
        // the groups' partial sums, added in group order by group 0
        __syncthreads();  // every group is done reading the tiles
        float* red = gt;   // [groups][tpg][kDgradRun][CIN]
#pragma unroll
        for (int r = 0; r < kDgradRun; ++r)
#pragma unroll
            for (int c = 0; c < CIN; ++c) red[((grp * tpg + tig) * kDgradRun + r) * CIN + c] = acc[r][c];
        __syncthreads();
        if (grp != 0) return;
#pragma unroll
        for (int r = 0; r < kDgradRun; ++r)
#pragma unroll
            for (int c = 0; c < CIN; ++c) {
                float v = red[(tig * kDgradRun + r) * CIN + c];
                for (int g2 = 1; g2 < groups; ++g2) v += red[((g2 * tpg + tig) * kDgradRun + r) * CIN + c];
                acc[r][c] = v;
            }
    }
    if (!live) return;
#pragma unroll
    for (int c = 0; c < CIN; ++c)
        if (c < c_in)
#pragma unroll
            for (int r = 0; r < kDgradRun; ++r)
                if (x0 + r < in_w) drow[(int64_t)c * HW + r] = acc[r][c] + old[r][c];
}

// Weight and bias gradient for layers with few taps (c_in*kh*kw <= TAPS):
// one workgroup of kWgradWaves wavefronts per (image, block of OCW output
// channels). Thread q takes pixels p = q, q + 256, ... (kWgradPix per batch,
// all their loads issued together): it loads each pixel's taps once and, per
// channel, one coalesced gradient value, accumulating
//   dW[oc, t] += g[n, oc, p] * x_t(n, p),   db[oc] += g[n, oc, p]
// in ascending pixel order; the 64 lanes of a wave are then added in lane
// order and the waves in wave order. The per-image sums go to
// pw[n][oc*taps + t] and pb[n][oc] for a fixed-order sum over images.
constexpr int kWgradWaves = 4, kWgradPix = 4;

template <int TAPS, int OCW>
__global__ __launch_bounds__(64 * kWgradWaves) void conv_wgrad_small_kernel(
    float* __restrict__ pw, float* __restrict__ pb, const float* __restrict__ grad,
    const float* __restrict__ input, int c_in, int in_h, int in_w, int c_out, int kh, int kw,
    int stride, int pad, FastDiv div_ow, int P) {
    constexpr int NT = 64 * kWgradWaves, NV = OCW * (TAPS + 1);
    __shared__ int2 tab[TAPS];
    __shared__ float red[NT][NV + 1];
    __shared__ float wsum[kWgradWaves][NV];
    const int taps = c_in * kh * kw;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid < TAPS) {
        const int t = tid < taps ? tid : 0;
        const int j = t % kw, i = (t / kw) % kh, ic = t / (kw * kh);
        tab[tid] = make_int2((ic * in_h + i) * in_w + j, i | (j << 16));
    }
    __syncthreads();
    const int n = blockIdx.x, oc0 = blockIdx.y * OCW;
    const float* img = input + (int64_t)n * c_in * in_h * in_w;
    const float* gimg = grad + ((int64_t)n * c_out + oc0) * P;
    float aw[OCW][TAPS] = {}, ab[OCW] = {};
    for (int p0 = tid; p0 < P; p0 += NT * kWgradPix) {
        float x[kWgradPix][TAPS], g[kWgradPix][OCW];
#pragma unroll
        for (int k = 0; k < kWgradPix; ++k) {
            const int p = p0 + k * NT;
            const bool pl = p < P;
            uint32_t oy, ox;
            fast_divmod((uint32_t)(pl ? p : 0), div_ow, oy, ox);
            const int iy0 = (int)oy * stride - pad, ix0 = (int)ox * stride - pad;
            const int base = iy0 * in_w + ix0;
#pragma unroll
            for (int t = 0; t < TAPS; ++t) {
                const int2 e = tab[t];
                const int i = e.y & 0xffff, j = e.y >> 16;
                const bool ok = pl & (t < taps) & ((unsigned)(iy0 + i) < (unsigned)in_h) &
                                ((unsigned)(ix0 + j) < (unsigned)in_w);
                const float v = img[ok ? base + e.x : 0];
                x[k][t] = ok ? v : 0.0f;
            }
#pragma unroll
            for (int o = 0; o < OCW; ++o) {
                const bool live = pl & (oc0 + o < c_out);
                const float v = gimg[live ? (int64_t)o * P + p : 0];
                g[k][o] = live ? v : 0.0f;
            }
        }
#pragma unroll
        for (int k = 0; k < kWgradPix; ++k)
#pragma unroll
            for (int o = 0; o < OCW; ++o) {
#pragma unroll
                for (int t = 0; t < TAPS; ++t) aw[o][t] += g[k][o] * x[k][t];
                ab[o] += g[k][o];
            }
    }
    // every thread's NV sums go to LDS; value v of wave w is then summed
    // over that wave's 64 lanes in lane order by lane v of the wave, and the
    // wave sums are added in wave order
#pragma unroll
    for (int o = 0; o < OCW; ++o) {
#pragma unroll
        for (int t = 0; t < TAPS; ++t) red[tid][o * (TAPS + 1) + t] = aw[o][t];
        red[tid][o * (TAPS + 1) + TAPS] = ab[o];
    }
    __syncthreads();
    for (int v = lane; v < NV; v += 64) {
        float r = 0.0f;
#pragma unroll 16
        for (int l = 0; l < 64; ++l) r += red[wave * 64 + l][v];
        wsum[wave][v] = r;
    }
    __syncthreads();
    for (int v = tid; v < NV; v += NT) {
        const int o = v / (TAPS + 1), t = v - o * (TAPS + 1);
        if (oc0 + o >= c_out || (t < TAPS && t >= taps)) continue;
        float r = wsum[0][v];
#pragma unroll
        for (int w = 1; w < kWgradWaves; ++w) r += wsum[w][v];
        if (t == TAPS)
            pb[(int64_t)n * c_out + oc0 + o] = r;
        else
            pw[((int64_t)n * c_out + oc0 + o) * taps + t] = r;
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

constexpr int kBiasThreads = 1024;

// dbias[oc] = sum over (ni, p) of grad[ni, oc, p] (+ beta * dbias[oc]), one
// workgroup per channel. Each thread sums a fixed strided subset in
// ascending order, then the 1024 partial sums are combined by a fixed tree,
// so the result is deterministic. Reads are 128-bit when P % 4 == 0 and the
// tensor is 16-byte aligned.
__global__ __launch_bounds__(kBiasThreads) void bias_grad_kernel(float* __restrict__ dbias,
                                                                 const float* __restrict__ grad,
                                                                 int N, int c_out, FastDiv div_P,
                                                                 float beta, bool vec4) {
    __shared__ float red[kBiasThreads];
    const int oc = blockIdx.x;
    const int t = threadIdx.x;
    const int P = (int)div_P.d;
    float acc = 0.0f;
    if (vec4) {  // div_P divides by P / 4 here
        const int P4 = P, total4 = N * P4;
        for (int e = t; e < total4; e += kBiasThreads) {
            uint32_t ni, q;
            fast_divmod((uint32_t)e, div_P, ni, q);
            const float4 v = reinterpret_cast<const float4*>(
                grad + ((int64_t)ni * c_out + oc) * (4 * P4))[q];
            acc += (v.x + v.y) + (v.z + v.w);
        }
    } else {
        const int total = N * P;
        for (int e = t; e < total; e += kBiasThreads) {
            uint32_t ni, q;
            fast_divmod((uint32_t)e, div_P, ni, q);
            acc += grad[((int64_t)ni * c_out + oc) * P + q];
        }
    }
    red[t] = acc;
    __syncthreads();
#pragma unroll
    for (int s = kBiasThreads / 2; s > 0; s >>= 1) {
        if (t < s) red[t] += red[t + s];
        __syncthreads();
    }
    if (t == 0) {
        float v = red[0];
        if (beta != 0.0f) v = v + beta * dbias[oc];
        dbias[oc] = v;
    }
}

}  // namespace

// dst = beta * dst when there is nothing to sum (a gradient over an empty
// batch); beta 0 writes zeros whatever dst held.
int zero_or_scale(float* dst, int64_t n, float beta) {
    if (!dst || n == 0 || beta == 1.0f) return NRS_OK;
    if (beta == 0.0f) return zero_fill(dst, sizeof(float) * (size_t)n);
    return nrs_scale(dst, dst, beta, n, 0.0f);
}

int zero_or_scale_bias(float* dbias, int64_t c_out, float beta) {
    return zero_or_scale(dbias, c_out, beta);
}

int bias_grad_launch(float* dbias, const float* grad, int64_t N, int64_t c_out, int64_t P,
                     float beta) {
    if (c_out == 0) return NRS_OK;
    NRS_ARG_CHECK(c_out <= INT32_MAX && N * P <= INT32_MAX && N * c_out * P <= INT32_MAX * 4ll,
                  "conv2d bias grad: tensor too large");
    if (N * P == 0) return zero_or_scale_bias(dbias, c_out, beta);
    const bool vec4 = ((uintptr_t)grad & 15) == 0 && P % 4 == 0;
    hipLaunchKernelGGL(bias_grad_kernel, dim3((unsigned)c_out), dim3(kBiasThreads), 0, stream(),
                       dbias, grad, (int)N, (int)c_out,
                       make_fastdiv((uint32_t)(vec4 ? P / 4 : P)), beta, vec4);
    NRS_LAUNCH_CHECK("conv2d bias grad");
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
    const int64_t rows = d.c_in * d.kh * d.kw, P = d.out_h * d.out_w, width = d.N * P;
    const int64_t total = rows * width;
    if (total == 0) return NRS_OK;
    const bool fast = P % 4 == 0 && ((uintptr_t)cols & 15) == 0 && rows <= 65535 &&
                      d.N * d.c_in * d.in_h * d.in_w <= INT32_MAX && width <= INT32_MAX;
    if (fast) {
        const int64_t width4 = width / 4;
        const unsigned bx = (unsigned)std::max<int64_t>(
            1, std::min<int64_t>((width4 + 255) / 256, (8 * (int64_t)num_cus() + rows - 1) / rows));
        hipLaunchKernelGGL(im2col_rows_kernel, dim3(bx, (unsigned)rows), dim3(256), 0, stream(),
                           cols, input, (int)d.c_in, (int)d.in_h, (int)d.in_w, (int)d.kh,
                           (int)d.kw, (int)d.stride, (int)d.pad, make_fastdiv((uint32_t)P),
                           make_fastdiv((uint32_t)d.out_w), (int)width4);
    } else {
        hipLaunchKernelGGL(im2col_kernel, dim3(grid_for(total)), dim3(256), 0, stream(), cols,
                           input, d.N, d.c_in, d.in_h, d.in_w, (int)d.kh, (int)d.kw,
                           (int)d.stride, (int)d.pad, d.out_h, d.out_w);
    }
    NRS_LAUNCH_CHECK("conv2d im2col");
    return NRS_OK;
}

// The implicit-GEMM convolution out = conv(image, weight) (+ bias) + beta*out,
// NCHW in and out, for the stride and padding of g.
int implicit_conv(float* out, const float* image, const float* weight, const float* bias,
                  int64_t N, int64_t c_out, const ConvGeom& g, float beta) {
    GemmCall c;
    c.layout = NRS_NN;
    c.C = out;
    c.A = weight;
    c.B = image;
    c.M = c_out;
    c.N = N * g.P;
    c.K = g.C * g.kh * g.kw;
    c.beta = beta;
    c.bias = bias;
    c.epi = bias ? NRS_EPI_BIAS_ROW : NRS_EPI_NONE;
    c.nchw_P = g.P;
    c.allow_split = false;
    c.bmode = OP_IM2COL;
    c.cg = g;
    c.gather_bytes = N * g.C * g.H * g.W * (int64_t)sizeof(float);
    return gemm_run(c);
}

// Gathered operands are read through 32-bit buffer offsets.
constexpr int64_t kMaxGatherBytes = 0x80000000ll;

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

// dinput += the stride-1 input gradient of a layer with c_in <= kDirectCin
// and a kernel width the row kernel is built for, gathered from LDS;
// kSlabUnsupported when it does not apply or its tiles do not fit.
// dinput = beta * dinput ahead of a kernel that only accumulates (beta 0:
// a fill, nothing read).
int prescale_grad(float* dinput, int64_t n, float beta) {
    if (beta == 1.0f) return NRS_OK;
    if (beta == 0.0f) return zero_fill(dinput, sizeof(float) * (size_t)n);
    return nrs_scale(dinput, dinput, beta, n, 0.0f);
}

int quad_dgrad(float* dinput, const float* grad, const float* weight, const ConvDims& d,
               float beta) {
    if (d.stride != 1 || d.c_in > 4 || d.kh != 3 || d.kw != 3 || d.pad != 1 || d.in_w % 4 ||
        d.in_w > 64 || d.out_h != d.in_h || d.out_w != d.in_w || ((uintptr_t)dinput & 15) ||
        ((uintptr_t)grad & 15) || d.c_out * d.in_h * d.in_w > INT32_MAX / 4 ||
        d.c_in * d.in_h * d.in_w > INT32_MAX / 4)
        return kSlabUnsupported;
    // a row's W/4 quads take a run of 2^lq lanes (the kernel's neighbour
    // exchange shifts values between adjacent lanes of one wave)
    const int W4 = (int)d.in_w / 4;
    int lq = 0;
    while ((1 << lq) < W4) ++lq;
    // bands of rows so that about two workgroups per CU run, whose quads
    // fill at most 256 threads
    int64_t bands = std::max<int64_t>(1, std::min<int64_t>(d.in_h, (2 * num_cus() + d.N - 1) / d.N));
    int64_t band = (d.in_h + bands - 1) / bands;
    band = std::max<int64_t>(1, std::min<int64_t>(band, 256 >> lq));
    bands = (d.in_h + band - 1) / band;
    if (d.N * bands > INT32_MAX) return kSlabUnsupported;
    const int qpg = (int)(band << lq);  // quad slots per band
    int groups = 4;
    while (groups > 1 && groups * qpg > 256) groups /= 2;
    if (qpg > 256) return kSlabUnsupported;
    const int pitch = (int)d.in_w + 8;  // 4 zero columns either side
    const int rrows = (int)band + 2, CIN = d.c_in == 1 ? 1 : 4;
    const size_t lds = sizeof(float) * ((size_t)kQuadDgradOc * rrows * pitch +
                                        (size_t)kQuadDgradOc * CIN * 9 + (size_t)groups * qpg * CIN * 4);
    if (lds > 64 * 1024) return kSlabUnsupported;
    auto fn = CIN == 1 ? conv_dgrad_quad_kernel<1> : conv_dgrad_quad_kernel<4>;
    if (int rc = prescale_grad(dinput, d.N * d.c_in * d.in_h * d.in_w, beta)) return rc;
    hipLaunchKernelGGL(fn, dim3((unsigned)(d.N * bands)), dim3(256), lds, stream(), dinput, grad,
                       weight, (int)d.c_in, (int)d.in_h, (int)d.in_w, (int)d.c_out, (int)band,
                       (int)bands, pitch, groups, qpg, lq, make_fastdiv((uint32_t)(rrows * (pitch / 4))),
                       make_fastdiv((uint32_t)(pitch / 4)));
    NRS_LAUNCH_CHECK("conv2d input gradient (pixel quads)");
    return NRS_OK;
}

int small_dgrad(float* dinput, const float* grad, const float* weight, const ConvDims& d,
                float beta) {
    if (d.stride != 1 || d.c_in > kDirectCin) return kSlabUnsupported;
    const int rq = quad_dgrad(dinput, grad, weight, d, beta);
    if (rq != kSlabUnsupported) return rq;
    const int64_t ngx = (d.in_w + kDgradRun - 1) / kDgradRun;
    if (ngx > 256) return kSlabUnsupported;
    // row pitch: the runs' windows, whole float4s
    const int64_t pitch = (ngx * kDgradRun + d.kw - 1 + 3) / 4 * 4;
    // about two workgroups per CU, at most 256 threads' rows per band
    int64_t bands = std::max<int64_t>(1, std::min<int64_t>(d.in_h, (2 * num_cus() + d.N - 1) / d.N));
    int64_t band = std::min<int64_t>((d.in_h + bands - 1) / bands, 256 / ngx);
    bands = (d.in_h + band - 1) / band;
    const int64_t tile = (band + d.kh - 1) * pitch, limit = 64 * 1024 / 4;
    const int64_t per_ch = tile + 4 * d.kh * d.kw;  // gradient tile + weights
    // (byte offsets inside one image and the weights fit the buffer loads'
    // 31 bits)
    if (per_ch > limit - 3 || d.N * bands > INT32_MAX || d.c_out > INT32_MAX ||
        d.c_out * d.out_h * d.out_w > INT32_MAX / 4 || d.c_in * d.in_h * d.in_w > INT32_MAX / 4 ||
        d.c_out * d.c_in * d.kh * d.kw > INT32_MAX / 4)
        return kSlabUnsupported;
    const int64_t occ = std::min<int64_t>(d.c_out, (limit - 3) / per_ch);
    // channel groups: whole waves of threads per group, enough for the runs
    const int64_t runs = band * ngx;
    int groups = 4;
    while (groups > 1 && (256 / groups < runs || groups > d.c_out)) groups /= 2;
    const int tpg = 256 / groups;
    const int64_t red = (int64_t)groups * tpg * kDgradRun * 4;  // group partials, CIN <= 4
    const size_t lds = (size_t)std::max<int64_t>(((occ * tile + 3) & ~3ll) + occ * 4 * d.kh * d.kw,
                                                 groups > 1 ? red : 0) * 4;
    const bool c1 = d.c_in == 1;
    void (*fn)(float*, const float*, const float*, int, int, int, int, int, int, int, int, int,
               int, int, int, int, int, int, FastDiv, FastDiv) = nullptr;
    switch (d.kw) {
        case 1: fn = c1 ? conv_dgrad_small_kernel<1, 1> : conv_dgrad_small_kernel<1, 4>; break;
        case 2: fn = c1 ? conv_dgrad_small_kernel<2, 1> : conv_dgrad_small_kernel<2, 4>; break;
        case 3: fn = c1 ? conv_dgrad_small_kernel<3, 1> : conv_dgrad_small_kernel<3, 4>; break;
        case 5: fn = c1 ? conv_dgrad_small_kernel<5, 1> : conv_dgrad_small_kernel<5, 4>; break;
        case 7: fn = c1 ? conv_dgrad_small_kernel<7, 1> : conv_dgrad_small_kernel<7, 4>; break;
        default: return kSlabUnsupported;
    }
    if (int rc = prescale_grad(dinput, d.N * d.c_in * d.in_h * d.in_w, beta)) return rc;
    hipLaunchKernelGGL(fn, dim3((unsigned)(d.N * bands)), dim3(256), lds, stream(), dinput, grad,
                       weight, (int)d.c_in, (int)d.in_h, (int)d.in_w, (int)d.c_out, (int)d.kh,
                       (int)d.pad, (int)d.out_h, (int)d.out_w, (int)band, (int)bands, (int)occ,
                       (int)ngx, (int)pitch, groups, tpg, make_fastdiv((uint32_t)ngx),
                       make_fastdiv((uint32_t)d.kh));
    NRS_LAUNCH_CHECK("conv2d input gradient (small)");
    return NRS_OK;
}

// dweight += and dbias += (either may be null) for a layer with c_in*kh*kw <=
// kDirectTaps: per-image sums, then a fixed-order sum over the images.
int small_wgrad(float* dweight, float* dbias, const float* grad, const float* input,
                const ConvDims& d, float beta) {
    const int64_t taps = d.c_in * d.kh * d.kw, P = d.out_h * d.out_w;
    if (d.N * P == 0) return NRS_OK;
    const int ocw = taps <= 9 ? 4 : (taps <= 16 ? 2 : 1);
    const int64_t blocks_y = (d.c_out + ocw - 1) / ocw;
    NRS_ARG_CHECK(blocks_y <= 65535 && d.N <= INT32_MAX && P <= INT32_MAX &&
                      d.N * d.c_out * (taps + 1) <= INT32_MAX &&
                      d.c_in * d.in_h * d.in_w <= INT32_MAX,
                  "conv2d weight gradient: tensor too large");
    float* pw = workspace(sizeof(float) * (size_t)(d.N * d.c_out * (taps + 1)), 3);
    if (!pw) return NRS_ERR_ALLOC;
    float* pb = pw + d.N * d.c_out * taps;
    auto fn = taps <= 9 ? conv_wgrad_small_kernel<9, 4>
                        : (taps <= 16 ? conv_wgrad_small_kernel<16, 2>
                                      : conv_wgrad_small_kernel<32, 1>);
    hipLaunchKernelGGL(fn, dim3((unsigned)d.N, (unsigned)blocks_y), dim3(64 * kWgradWaves), 0,
                       stream(), pw, pb,
                       grad, input, (int)d.c_in, (int)d.in_h, (int)d.in_w, (int)d.c_out,
                       (int)d.kh, (int)d.kw, (int)d.stride, (int)d.pad,
                       make_fastdiv((uint32_t)d.out_w), (int)P);
    NRS_LAUNCH_CHECK("conv2d weight gradient (small)");
    // the per-image partials are [n][oc][taps]: the slab layout with one
    // channel of `taps` taps; weights and bias summed in one launch
    return wgrad_partial_sum(dweight, dbias, pw, pb, (int)d.N, (int)d.c_out, 1, (int)taps, beta);
}

// dinput += the stride-1 input gradient as a slab convolution of the output
// gradient with the flipped, channel-transposed weights (padding k-1-pad).
// With `wg`, the weight gradient it describes runs in the same launch when
// both fit their slab kernels (*wg_done is then set).
int slab_dgrad(float* dinput, const float* grad, const float* weight, int64_t N, int64_t c_in,
               int64_t in_h, int64_t in_w, int64_t c_out, int64_t kh, int64_t kw, int64_t pad,
               const ConvDims& d, const SlabWgrad* wg, bool* wg_done, float beta) {
    if (c_in > INT32_MAX || c_out > INT32_MAX || in_h > INT32_MAX || in_w > INT32_MAX)
        return kSlabUnsupported;
    SlabConv s;
    s.x = grad;
    s.w = weight;
    s.out = dinput;
    s.N = N;
    s.C = (int)c_out;
    s.H = (int)d.out_h;
    s.W = (int)d.out_w;
    s.M = (int)c_in;
    s.kh = (int)kh;
    s.kw = (int)kw;
    s.stride = 1;
    s.pad_h = (int)(kh - 1 - pad);
    s.pad_w = (int)(kw - 1 - pad);
    s.OH = (int)in_h;
    s.OW = (int)in_w;
    s.flip = true;
    s.beta = beta;
    if (wg) {
        // with the weight gradient: both in one launch
        int rc = pipe_backward(&s, *wg);
        if (rc != kSlabUnsupported) {
            *wg_done = rc == NRS_OK;
            return rc;
        }
        rc = slab_backward_pair(s, *wg);
        if (rc != kSlabUnsupported) {
            *wg_done = rc == NRS_OK;
            return rc;
        }
    } else {
        // small 3x3 images: Winograd F(2x2, 3x3) over the flipped weights,
        // else the gradient image resident in LDS, the weights flipped while
        // they are staged (no packing launch)
        int rc = wino_conv(s);
        if (rc != kSlabUnsupported) return rc;
        rc = pipe_conv(s);
        if (rc != kSlabUnsupported) return rc;
        rc = img_conv(s);
        if (rc != kSlabUnsupported) return rc;
    }
    return slab_conv(s);
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

}  // extern "C"

namespace nrs {
namespace {

// conv2d (+ ReLU when relu) + max pooling, the forward of both fused entry points.
int conv_pool_forward(float* pooled, int32_t* argmax, float* out, const float* input,
                      const float* weight, const float* bias, int64_t N, int64_t c_in, int64_t in_h,
                      int64_t in_w, int64_t c_out, int64_t kh, int64_t kw, int64_t stride,
                      int64_t pad, int64_t pool_k, int64_t pool_stride, bool relu) {
    NRS_REQUIRE_INIT();
    nrs::ConvDims d;
    int rc = nrs::conv_dims(d, N, c_in, in_h, in_w, c_out, kh, kw, stride, pad);
    if (rc) return rc;
    NRS_ARG_CHECK(pool_k > 0 && pool_stride > 0 && d.out_h >= pool_k && d.out_w >= pool_k,
                  "conv2d maxpool: bad window");
    NRS_ARG_CHECK(N * c_out * d.out_h * d.out_w <= INT32_MAX,
                  "conv2d maxpool: conv output too large for int32 argmax");
    if (c_out == 0 || N == 0) return NRS_OK;
    NRS_ARG_CHECK(pooled && argmax && input && weight, "conv2d maxpool: null pointer");
    auto a8 = [](const void* q) { return ((uintptr_t)q & 7) == 0; };
    if (kh == 3 && kw == 3 && stride == 1 && pad == 1 && c_in <= 3 && in_w % 4 == 0 &&
        in_h % 2 == 0 && pool_k == 2 && pool_stride == 2 && c_out <= 65535 &&
        ((uintptr_t)input & 15) == 0 && (!out || ((uintptr_t)out & 15) == 0) && a8(pooled) &&
        a8(argmax) && N * c_in * in_h * in_w <= INT32_MAX / 4 &&
        N * std::max(c_in, c_out) * in_h * in_w <= INT32_MAX) {
        const int64_t blocks = N * (in_h / 2) * (in_w / 4);
        constexpr int QOC = nrs::kQuadOcPool;
        auto fn = c_in == 1 ? nrs::conv_fwd_pool_quad_kernel<1, QOC>
                            : (c_in == 2 ? nrs::conv_fwd_pool_quad_kernel<2, QOC>
                                         : nrs::conv_fwd_pool_quad_kernel<3, QOC>);
        hipLaunchKernelGGL(fn, dim3((unsigned)((blocks + nrs::kQuadThreads - 1) / nrs::kQuadThreads),
                                    (unsigned)((c_out + QOC - 1) / QOC)),
                           dim3(nrs::kQuadThreads), 0, nrs::stream(), pooled, argmax, out, input,
                           weight, bias, (int)N, (int)in_h, (int)in_w, (int)c_out, relu ? 1 : 0,
                           nrs::make_fastdiv((uint32_t)((in_h / 2) * (in_w / 4))),
                           nrs::make_fastdiv((uint32_t)(in_w / 4)));
        NRS_LAUNCH_CHECK("conv2d + maxpool forward (pixel blocks)");
        return NRS_OK;
    }
    // any other shape: the conv output (the caller's, else library scratch),
    // its ReLU (in scratch), then the pooling
    const int64_t conv_elems = N * c_out * d.out_h * d.out_w;
    float* y = out;
    if (!y) {
        y = nrs::workspace(sizeof(float) * (size_t)conv_elems, 5);
        if (!y) return NRS_ERR_ALLOC;
    }
    rc = nrs_conv2d_forward(y, input, weight, bias, N, c_in, in_h, in_w, c_out, kh, kw, stride, pad);
    if (rc) return rc;
    const float* a = y;
    if (relu) {
        float* r = out ? nrs::workspace(sizeof(float) * (size_t)conv_elems, 5) : y;
        if (!r) return NRS_ERR_ALLOC;
        if ((rc = nrs_relu_forward(r, y, conv_elems))) return rc;
        a = r;
    }
    return nrs_maxpool_forward(pooled, argmax, a, N, c_out, d.out_h, d.out_w, pool_k, pool_stride);
}

// The backward of max pooling (over a ReLU of the conv output when pooled is
// given: its values gate each window's gradient) then the conv backward.
int pool_conv_backward(float* dinput, float* dweight, float* dbias, const float* grad_pooled,
                       const int32_t* argmax, const float* pooled, const float* input,
                       const float* weight, int64_t N, int64_t c_in, int64_t in_h, int64_t in_w,
                       int64_t c_out, int64_t kh, int64_t kw, int64_t stride, int64_t pad,
                       int64_t pool_k, int64_t pool_stride, float beta_params) {
    NRS_REQUIRE_INIT();
    nrs::ConvDims d;
    int rc = nrs::conv_dims(d, N, c_in, in_h, in_w, c_out, kh, kw, stride, pad);
    if (rc) return rc;
    NRS_ARG_CHECK(pool_k > 0 && pool_stride > 0 && d.out_h >= pool_k && d.out_w >= pool_k,
                  "maxpool conv2d backward: bad window");
    const int64_t conv_elems = N * c_out * d.out_h * d.out_w;
    NRS_ARG_CHECK(conv_elems <= INT32_MAX,
                  "maxpool conv2d backward: conv output too large for int32 argmax");
    if (c_out == 0 || (!dinput && !dweight && !dbias)) return NRS_OK;
    if (N == 0) {
        // no images: the parameter gradients keep beta_params of what they held
        if ((rc = nrs::zero_or_scale(dweight, c_out * c_in * kh * kw, beta_params))) return rc;
        return nrs::zero_or_scale(dbias, c_out, beta_params);
    }
    NRS_ARG_CHECK(grad_pooled && argmax && input && weight, "maxpool conv2d backward: null pointer");
    if (!dinput && pool_k == 2 && pool_stride == 2 && c_in * kh * kw <= nrs::kDirectTaps &&
        c_out <= INT32_MAX) {
        // weight and bias gradients with the pooled gradient expanded while
        // it is loaded
        nrs::FewTapsWgrad f;
        f.x = input;
        f.g = nullptr;
        f.gp = grad_pooled;
        f.am = argmax;
        f.pv = pooled;
        f.beta = beta_params;
        f.dw = dweight;
        f.db = dbias;
        f.N = N;
        f.C = (int)c_in;
        f.H = (int)in_h;
        f.W = (int)in_w;
        f.M = (int)c_out;
        f.kh = (int)kh;
        f.kw = (int)kw;
        f.stride = (int)stride;
        f.pad = (int)pad;
        f.OH = (int)d.out_h;
        f.OW = (int)d.out_w;
        if ((rc = nrs::few_taps_wgrad(f)) != nrs::kSlabUnsupported) return rc;
    }
    if (pooled) {
        // the ReLU's gate applied to the pooled gradient: a window passes its
        // gradient only when its pooled value is > 0
        const int64_t np = N * c_out * ((d.out_h - pool_k) / pool_stride + 1) *
                           ((d.out_w - pool_k) / pool_stride + 1);
        float* gm = nrs::workspace(sizeof(float) * (size_t)std::max<int64_t>(1, np), 6);
        if (!gm) return NRS_ERR_ALLOC;
        if ((rc = nrs_relu_backward(gm, grad_pooled, pooled, np, 0.0f))) return rc;
        grad_pooled = gm;
    }
    // any other case: the conv output's gradient in library scratch (the
    // pooling's backward into zeros), then the conv backward
    float* g = nrs::workspace(sizeof(float) * (size_t)conv_elems, 5);
    if (!g) return NRS_ERR_ALLOC;
    if ((rc = nrs::zero_fill(g, sizeof(float) * (size_t)conv_elems))) return rc;
    rc = nrs_maxpool_backward(g, grad_pooled, argmax, N, c_out, d.out_h, d.out_w, pool_k,
                              pool_stride);
    if (rc) return rc;
    return nrs_conv2d_backward_ex(dinput, dweight, dbias, g, input, weight, N, c_in, in_h, in_w,
                                  c_out, kh, kw, stride, pad, 1.0f, beta_params);
}

}  // namespace
}  // namespace nrs

extern "C" {

int nrs_conv2d_maxpool_forward(float* pooled, int32_t* argmax, float* out, const float* input,
                               const float* weight, const float* bias, int64_t N, int64_t c_in,
                               int64_t in_h, int64_t in_w, int64_t c_out, int64_t kh, int64_t kw,
                               int64_t stride, int64_t pad, int64_t pool_k, int64_t pool_stride) {
    return nrs::conv_pool_forward(pooled, argmax, out, input, weight, bias, N, c_in, in_h, in_w,
                                  c_out, kh, kw, stride, pad, pool_k, pool_stride, false);
}

int nrs_conv2d_relu_maxpool_forward(float* pooled, int32_t* argmax, float* out,
                                    const float* input, const float* weight, const float* bias,
                                    int64_t N, int64_t c_in, int64_t in_h, int64_t in_w,
                                    int64_t c_out, int64_t kh, int64_t kw, int64_t stride,
                                    int64_t pad, int64_t pool_k, int64_t pool_stride) {
    return nrs::conv_pool_forward(pooled, argmax, out, input, weight, bias, N, c_in, in_h, in_w,
                                  c_out, kh, kw, stride, pad, pool_k, pool_stride, true);
}

int nrs_maxpool_conv2d_backward(float* dinput, float* dweight, float* dbias,
                                const float* grad_pooled, const int32_t* argmax,
                                const float* input, const float* weight, int64_t N, int64_t c_in,
                                int64_t in_h, int64_t in_w, int64_t c_out, int64_t kh, int64_t kw,
                                int64_t stride, int64_t pad, int64_t pool_k,
                                int64_t pool_stride) {
    return nrs::pool_conv_backward(dinput, dweight, dbias, grad_pooled, argmax, nullptr, input,
                                   weight, N, c_in, in_h, in_w, c_out, kh, kw, stride, pad, pool_k,
                                   pool_stride, 1.0f);
}

int nrs_maxpool_relu_conv2d_backward(float* dinput, float* dweight, float* dbias,
                                     const float* grad_pooled, const int32_t* argmax,
                                     const float* pooled, const float* input, const float* weight,
                                     int64_t N, int64_t c_in, int64_t in_h, int64_t in_w,
                                     int64_t c_out, int64_t kh, int64_t kw, int64_t stride,
                                     int64_t pad, int64_t pool_k, int64_t pool_stride,
                                     float beta_params) {
    NRS_ARG_CHECK(pooled || N * c_out == 0, "maxpool relu conv2d backward: null pooled values");
    return nrs::pool_conv_backward(dinput, dweight, dbias, grad_pooled, argmax, pooled, input,
                                   weight, N, c_in, in_h, in_w, c_out, kh, kw, stride, pad, pool_k,
                                   pool_stride, beta_params);
}

int nrs_conv2d_maxpool_relu_conv2d_backward(
    float* dpooled, float* dweight, float* dbias, float* dweight_lo, float* dbias_lo,
    const float* grad, const float* pooled, const float* weight, const int32_t* argmax,
    const float* input_lo, const float* weight_lo, int64_t N, int64_t c_in_lo, int64_t in_h,
    int64_t in_w, int64_t c_mid, int64_t kh_lo, int64_t kw_lo, int64_t stride_lo,
    int64_t pad_lo, int64_t pool_k, int64_t pool_stride, int64_t c_out, int64_t kh, int64_t kw,
    int64_t stride, int64_t pad, float beta_params) {
    NRS_REQUIRE_INIT();
    // the lower pair's geometry: conv output, then the pooled image (the
    // upper layer's input)
    nrs::ConvDims lo;
    int rc = nrs::conv_dims(lo, N, c_in_lo, in_h, in_w, c_mid, kh_lo, kw_lo, stride_lo, pad_lo);
    if (rc) return rc;
    NRS_ARG_CHECK(pool_k >= 1 && pool_stride >= 1 && lo.out_h >= pool_k && lo.out_w >= pool_k,
                  "conv2d maxpool relu conv2d backward: bad pooling window");
    const int64_t ph = (lo.out_h - pool_k) / pool_stride + 1;
    const int64_t pw = (lo.out_w - pool_k) / pool_stride + 1;
    nrs::ConvDims up;
    if ((rc = nrs::conv_dims(up, N, c_mid, ph, pw, c_out, kh, kw, stride, pad))) return rc;
    NRS_ARG_CHECK(dpooled || N * c_mid * ph * pw == 0,
                  "conv2d maxpool relu conv2d backward: null pooled gradient");
    // one launch (and the two partial sums in one more): the upper layer on
    // the chunk-pipelined kernel, the lower a "same" 3x3 stride-1 layer of 1
    // or 2 input channels under 2x2 stride-2 pooling of an even image
    const bool fused =
        N >= 1 && dweight && dweight_lo && c_out >= 1 && c_mid >= 1 && kh_lo == 3 && kw_lo == 3 &&
        stride_lo == 1 && pad_lo == 1 && c_in_lo >= 1 && c_in_lo <= 2 && pool_k == 2 &&
        pool_stride == 2 && in_h % 2 == 0 && in_w % 2 == 0 && grad && pooled && weight && argmax &&
        input_lo && c_mid <= INT32_MAX && c_out <= INT32_MAX && ph <= 16 && pw <= 16;
    if (fused) {
        nrs::SlabConv s;
        s.x = grad;
        s.w = weight;
        s.out = dpooled;
        s.N = N;
        s.C = (int)c_out;
        s.H = (int)up.out_h;
        s.W = (int)up.out_w;
        s.M = (int)c_mid;
        s.kh = (int)kh;
        s.kw = (int)kw;
        s.stride = 1;
        s.pad_h = (int)(kh - 1 - pad);
        s.pad_w = (int)(kw - 1 - pad);
        s.OH = (int)ph;
        s.OW = (int)pw;
        s.flip = true;
        s.beta = 0.0f;
        nrs::SlabWgrad w;
        w.x = pooled;
        w.g = grad;
        w.dw = dweight;
        w.db = dbias;
        w.N = N;
        w.C = (int)c_mid;
        w.H = (int)ph;
        w.W = (int)pw;
        w.M = (int)c_out;
        w.kh = (int)kh;
        w.kw = (int)kw;
        w.stride = (int)stride;
        w.pad = (int)pad;
        w.OH = (int)up.out_h;
        w.OW = (int)up.out_w;
        w.beta = beta_params;
        nrs::PipeLower l;
        l.am = argmax;
        l.pooled = pooled;
        l.x = input_lo;
        l.dw = dweight_lo;
        l.db = dbias_lo;
        l.c_lo = (int)c_in_lo;
        l.beta = beta_params;
        if (stride == 1 && (rc = nrs::pipe_backward(&s, w, &l)) != nrs::kSlabUnsupported) return rc;
    }
    // any other shape: the two backward calls, the pooled gradient written
    // by the first and read by the second
    if ((rc = nrs_conv2d_backward_ex(dpooled, dweight, dbias, grad, pooled, weight, N, c_mid, ph,
                                     pw, c_out, kh, kw, stride, pad, 0.0f, beta_params)))
        return rc;
    return nrs_maxpool_relu_conv2d_backward(nullptr, dweight_lo, dbias_lo, dpooled, argmax, pooled,
                                            input_lo, weight_lo, N, c_in_lo, in_h, in_w, c_mid,
                                            kh_lo, kw_lo, stride_lo, pad_lo, pool_k, pool_stride,
                                            beta_params);
}

int nrs_conv2d_forward(float* out, const float* input, const float* weight, const float* bias,
                       int64_t N, int64_t c_in, int64_t in_h, int64_t in_w, int64_t c_out,
                       int64_t kh, int64_t kw, int64_t stride, int64_t pad) {
    NRS_REQUIRE_INIT();
    nrs::ConvDims d;
    int rc = nrs::conv_dims(d, N, c_in, in_h, in_w, c_out, kh, kw, stride, pad);
    if (rc) return rc;
    const int64_t P = d.out_h * d.out_w;
    if (c_out == 0 || N * P == 0) return NRS_OK;
    NRS_ARG_CHECK(kh < 32768 && kw < 32768 && c_in * in_h * in_w <= INT32_MAX &&
                      c_in * kh * kw <= INT32_MAX,
                  "conv2d: kernel or image too large");
    nrs::ConvGeom g{c_in, in_h, in_w, (int)kh, (int)kw, (int)stride, (int)pad, (int)pad,
                    d.out_h, d.out_w, P};
    if (c_in * kh * kw <= nrs::kDirectTaps && c_out <= 65535 &&
        N * std::max(c_in * in_h * in_w, c_out * P) <= INT32_MAX) {
        const int64_t taps = c_in * kh * kw;
        if (kh == 3 && kw == 3 && stride == 1 && pad == 1 && c_in <= 3 && in_w % 4 == 0 &&
            ((uintptr_t)out & 15) == 0 && ((uintptr_t)input & 15) == 0 &&
            N * c_in * in_h * in_w <= INT32_MAX / 4) {
            // "same" 3x3 over rows of whole quads: four pixels per thread
            const int64_t quads = N * P / 4;
            constexpr int QOC = nrs::kQuadOcFwd;
            auto fn = c_in == 1 ? nrs::conv_fwd_quad_kernel<1, QOC>
                                : (c_in == 2 ? nrs::conv_fwd_quad_kernel<2, QOC>
                                             : nrs::conv_fwd_quad_kernel<3, QOC>);
            hipLaunchKernelGGL(fn, dim3((unsigned)((quads + nrs::kQuadThreads - 1) / nrs::kQuadThreads),
                                        (unsigned)((c_out + QOC - 1) / QOC)),
                               dim3(nrs::kQuadThreads), 0, nrs::stream(), out, input, weight, bias, (int)N,
                               (int)in_h, (int)in_w, (int)c_out,
                               nrs::make_fastdiv((uint32_t)(P / 4)),
                               nrs::make_fastdiv((uint32_t)(in_w / 4)));
            NRS_LAUNCH_CHECK("conv2d forward (direct, pixel quads)");
            return NRS_OK;
        }
        // few taps per output: direct convolution, one thread per pixel
        auto fn = taps <= 9 ? nrs::conv_fwd_direct_kernel<9>
                            : (taps <= 16 ? nrs::conv_fwd_direct_kernel<16>
                                          : nrs::conv_fwd_direct_kernel<32>);
        const unsigned bx = (unsigned)std::min<int64_t>((N * P + 255) / 256, 65535);
        // output channels per workgroup: halved (down to 8) until there are
        // about three workgroups per CU, so the output's stores spread evenly
        // (cfg3 conv1: 392 workgroups of 32 channels left 136 CUs with twice
        // the work; 784 of 16 channels: 6.7 -> 5.7 us). A smaller block
        // re-reads the pixel's taps, which hit in L2.
        int64_t ocb = nrs::kDirectOcBlock;
        while (ocb > 8 && ocb / 2 >= c_out) ocb /= 2;  // no block wider than the layer
        auto blocks = [&](int64_t b) { return (int64_t)bx * ((c_out + b - 1) / b); };
        while (ocb > 8 && blocks(ocb) < 3 * (int64_t)nrs::num_cus() && blocks(ocb / 2) > blocks(ocb))
            ocb /= 2;
        const unsigned by = (unsigned)((c_out + ocb - 1) / ocb);
        hipLaunchKernelGGL(fn, dim3(bx, by), dim3(256), 0, nrs::stream(), out, input,
                           weight, bias, (int)N, (int)c_in, (int)in_h, (int)in_w, (int)c_out,
                           (int)kh, (int)kw, (int)stride, (int)pad, (int)ocb,
                           nrs::make_fastdiv((uint32_t)P), nrs::make_fastdiv((uint32_t)d.out_w));
        NRS_LAUNCH_CHECK("conv2d forward (direct)");
        return NRS_OK;
    }
    {
        // input slab and weights staged in LDS, reduction on the matrix cores
        nrs::SlabConv s;
        s.x = input;
        s.w = weight;
        s.bias = bias;
        s.out = out;
        s.N = N;
        s.C = (int)c_in;
        s.H = (int)in_h;
        s.W = (int)in_w;
        s.M = (int)c_out;
        s.kh = (int)kh;
        s.kw = (int)kw;
        s.stride = (int)stride;
        s.pad_h = s.pad_w = (int)pad;
        s.OH = (int)d.out_h;
        s.OW = (int)d.out_w;
        if (c_out <= INT32_MAX && d.out_h <= INT32_MAX && d.out_w <= INT32_MAX) {
            // small "same" 3x3 images: Winograd F(2x2, 3x3) on the matrix
            // cores, else the whole image resident in LDS
            rc = nrs::wino_conv(s);
            if (rc != nrs::kSlabUnsupported) return rc;
            rc = nrs::pipe_conv(s);
            if (rc != nrs::kSlabUnsupported) return rc;
            rc = nrs::img_conv(s);
            if (rc != nrs::kSlabUnsupported) return rc;
            rc = nrs::slab_conv(s);
            if (rc != nrs::kSlabUnsupported) return rc;
        }
    }
    if (N * c_in * in_h * in_w * (int64_t)sizeof(float) <= nrs::kMaxGatherBytes) {
        // out(NCHW) = W[c_out, c_in*kh*kw] . im2col(input) + bias[oc], the
        // column matrix gathered inside the GEMM (conv.rs:266-277 without the
        // cols buffer and col2out).
        return nrs::implicit_conv(out, input, weight, bias, N, c_out, g, 0.0f);
    }
    // Inputs over 2 GiB: materialised im2col, then the GEMM with the NCHW +
    // bias epilogue.
    const int64_t col_h = c_in * kh * kw, width = N * P;
    float* cols = nrs::workspace(sizeof(float) * (size_t)(col_h * width), 1);
    if (!cols) return NRS_ERR_ALLOC;
    rc = nrs::launch_im2col(cols, input, d);
    if (rc) return rc;
    nrs::GemmCall c;
    c.layout = NRS_NN;
    c.C = out;
    c.A = weight;
    c.B = cols;
    c.M = c_out;
    c.N = width;
    c.K = col_h;
    c.bias = bias;
    c.epi = bias ? NRS_EPI_BIAS_ROW : NRS_EPI_NONE;
    c.nchw_P = P;
    c.allow_split = false;
    return nrs::gemm_run(c);
}

int nrs_conv2d_backward(float* dinput, float* dweight, float* dbias, const float* grad,
                        const float* input, const float* weight, int64_t N, int64_t c_in,
                        int64_t in_h, int64_t in_w, int64_t c_out, int64_t kh, int64_t kw,
                        int64_t stride, int64_t pad) {
    return nrs_conv2d_backward_beta(dinput, dweight, dbias, grad, input, weight, N, c_in, in_h,
                                    in_w, c_out, kh, kw, stride, pad, 1.0f);
}

int nrs_conv2d_backward_beta(float* dinput, float* dweight, float* dbias, const float* grad,
                             const float* input, const float* weight, int64_t N, int64_t c_in,
                             int64_t in_h, int64_t in_w, int64_t c_out, int64_t kh, int64_t kw,
                             int64_t stride, int64_t pad, float beta_input) {
    return nrs_conv2d_backward_ex(dinput, dweight, dbias, grad, input, weight, N, c_in, in_h, in_w,
                                  c_out, kh, kw, stride, pad, beta_input, 1.0f);
}

int nrs_conv2d_backward_ex(float* dinput, float* dweight, float* dbias, const float* grad,
                           const float* input, const float* weight, int64_t N, int64_t c_in,
                           int64_t in_h, int64_t in_w, int64_t c_out, int64_t kh, int64_t kw,
                           int64_t stride, int64_t pad, float beta_input, float beta_params) {
    NRS_REQUIRE_INIT();
    nrs::ConvDims d;
    int rc = nrs::conv_dims(d, N, c_in, in_h, in_w, c_out, kh, kw, stride, pad);
    if (rc) return rc;
    const int64_t col_h = c_in * kh * kw, P = d.out_h * d.out_w, width = N * P;
    if (c_out == 0) return NRS_OK;
    if (N == 0) {
        // no images (the output always has a pixel): dinput is empty and the
        // parameter gradients keep beta_params of what they held
        if ((rc = nrs::zero_or_scale(dweight, c_out * col_h, beta_params))) return rc;
        return nrs::zero_or_scale(dbias, c_out, beta_params);
    }
    NRS_ARG_CHECK(kh < 32768 && kw < 32768 && c_in * in_h * in_w <= INT32_MAX &&
                      c_out * d.out_h * d.out_w <= INT32_MAX && c_out * kh * kw <= INT32_MAX,
                  "conv2d: kernel or image too large");
    // the slab weight gradient's arguments (it runs beside a slab input
    // gradient when both fit, else on its own below)
    nrs::SlabWgrad w;
    const bool slab_w = dweight && col_h > nrs::kDirectTaps && c_in <= INT32_MAX &&
                        c_out <= INT32_MAX && in_h <= INT32_MAX && in_w <= INT32_MAX;
    if (slab_w) {
        w.x = input;
        w.g = grad;
        w.dw = dweight;
        w.db = dbias;
        w.N = N;
        w.C = (int)c_in;
        w.H = (int)in_h;
        w.W = (int)in_w;
        w.M = (int)c_out;
        w.kh = (int)kh;
        w.kw = (int)kw;
        w.stride = (int)stride;
        w.pad = (int)pad;
        w.OH = (int)d.out_h;
        w.OW = (int)d.out_w;
        w.beta = beta_params;
    }
    bool wgrad_done = false;
    if (dinput) {
        const int64_t grad_bytes = N * c_out * P * (int64_t)sizeof(float);
        if ((rc = nrs::small_dgrad(dinput, grad, weight, d, beta_input)) != nrs::kSlabUnsupported) {
            // a handful of input channels, stride 1: gather from LDS
            if (rc) return rc;
        } else if (c_in <= nrs::kDirectCin && c_out * c_in * kh * kw <= nrs::kDirectWeights &&
                   kh * kw <= nrs::kDirectWin &&
                   N * std::max(c_in * in_h * in_w, c_out * P) <= INT32_MAX) {
            // a handful of input channels: direct gather per input pixel
            hipLaunchKernelGGL(nrs::conv_dgrad_direct_kernel, dim3(nrs::grid_for(N * in_h * in_w)),
                               dim3(256), 0, nrs::stream(), dinput, grad, weight, (int)N, (int)c_in,
                               (int)in_h, (int)in_w, (int)c_out, (int)kh, (int)kw,
                               nrs::make_fastdiv((uint32_t)stride), (int)pad, (int)d.out_h,
                               (int)d.out_w, nrs::make_fastdiv((uint32_t)(in_h * in_w)),
                               nrs::make_fastdiv((uint32_t)in_w), beta_input);
            NRS_LAUNCH_CHECK("conv2d input gradient (direct)");
        } else if (stride == 1 && pad <= kh - 1 && pad <= kw - 1 &&
                   (rc = slab_dgrad(dinput, grad, weight, N, c_in, in_h, in_w, c_out, kh, kw,
                                    pad, d, slab_w ? &w : nullptr, &wgrad_done, beta_input)) !=
                       nrs::kSlabUnsupported) {
            // dinput += conv(grad, flipped W) with padding k-1-pad, staged in LDS
            if (rc) return rc;
        } else if (stride == 1 && pad <= kh - 1 && pad <= kw - 1 &&
                   grad_bytes <= nrs::kMaxGatherBytes) {
            // dinput += conv(grad, flipped W) with padding k-1-pad: the
            // TN GEMM + col2im of conv.rs:304-312 as one implicit GEMM.
            const int64_t wn = c_out * c_in * kh * kw;
            float* wf = nrs::workspace(sizeof(float) * (size_t)std::max<int64_t>(1, wn), 2);
            if (!wf) return NRS_ERR_ALLOC;
            hipLaunchKernelGGL(nrs::flip_weights_kernel, dim3(nrs::grid_for(wn)), dim3(256), 0,
                               nrs::stream(), wf, weight, (int)c_out, (int)c_in, (int)kh, (int)kw);
            NRS_LAUNCH_CHECK("conv2d flip weights");
            nrs::ConvGeom g{c_out, d.out_h, d.out_w, (int)kh, (int)kw, 1, (int)(kh - 1 - pad),
                            (int)(kw - 1 - pad), in_h, in_w, in_h * in_w};
            rc = nrs::implicit_conv(dinput, grad, wf, nullptr, N, c_in, g, beta_input);
            if (rc) return rc;
        } else {
            // dcols[col_h, N*P] = W^T . G ; dinput += col2im(dcols)   (conv.rs:304-312)
            float* gmm = nrs::workspace(sizeof(float) * (size_t)std::max<int64_t>(1, c_out * width), 2);
            if (!gmm) return NRS_ERR_ALLOC;
            rc = nrs::launch_out2mm(gmm, grad, d);  // [c_out, N*P]
            if (rc) return rc;
            float* cols = nrs::workspace(sizeof(float) * (size_t)std::max<int64_t>(1, col_h * width), 1);
            if (!cols) return NRS_ERR_ALLOC;
            nrs::GemmCall c;
            c.layout = NRS_TN;
            c.C = cols;
            c.A = weight;
            c.B = gmm;
            c.M = col_h;
            c.N = width;
            c.K = c_out;
            rc = nrs::gemm_run(c);
            if (rc) return rc;
            rc = nrs::launch_col2im(dinput, cols, d, beta_input);
            if (rc) return rc;
        }
    }
    if (wgrad_done) return NRS_OK;
    if ((dweight || dbias) && col_h <= nrs::kDirectTaps) {
        // few taps: both gradients from one pass over the output gradient
        // (conv.rs:314-322 without the cols matrix), on the matrix cores
        // when the layer fits that kernel
        nrs::FewTapsWgrad f;
        f.x = input;
        f.g = grad;
        f.dw = dweight;
        f.db = dbias;
        f.N = N;
        f.C = (int)c_in;
        f.H = (int)in_h;
        f.W = (int)in_w;
        f.M = (int)std::min<int64_t>(c_out, INT32_MAX);
        f.kh = (int)kh;
        f.kw = (int)kw;
        f.stride = (int)stride;
        f.pad = (int)pad;
        f.OH = (int)d.out_h;
        f.OW = (int)d.out_w;
        f.beta = beta_params;
        if ((rc = nrs::few_taps_wgrad(f)) != nrs::kSlabUnsupported) return rc;
        return nrs::small_wgrad(dweight, dbias, grad, input, d, beta_params);
    }
    if (slab_w) {
        // input slab and gradient rows staged in LDS, reduction on the matrix
        // cores, per-slice partials summed in a fixed order
        rc = nrs::pipe_backward(nullptr, w);
        if (rc != nrs::kSlabUnsupported) return rc;
        rc = nrs::slab_wgrad(w);
        if (rc != nrs::kSlabUnsupported) return rc;
    }
    if (dweight) {
        // dW[c_out, col_h] += G . cols^T   (conv.rs:314-320, split-K NT), with
        // G read in place from NCHW when it fits a buffer (no out2mm).
        float* cols = nrs::workspace(sizeof(float) * (size_t)std::max<int64_t>(1, col_h * width), 1);
        if (!cols) return NRS_ERR_ALLOC;
        rc = nrs::launch_im2col(cols, input, d);
        if (rc) return rc;
        nrs::GemmCall c;
        c.layout = NRS_NT;
        c.C = dweight;
        c.B = cols;
        c.M = c_out;
        c.N = col_h;
        c.K = width;
        c.beta = beta_params;
        const int64_t grad_bytes = N * c_out * P * (int64_t)sizeof(float);
        if (grad_bytes <= nrs::kMaxGatherBytes) {
            c.A = grad;
            c.amode = nrs::OP_NCHW;
            c.cg.P = P;
            c.cg.ow = d.out_w;
            c.gather_bytes = grad_bytes;
        } else {
            float* gmm = nrs::workspace(sizeof(float) * (size_t)(c_out * width), 2);
            if (!gmm) return NRS_ERR_ALLOC;
            rc = nrs::launch_out2mm(gmm, grad, d);
            if (rc) return rc;
            c.A = gmm;
        }
        rc = nrs::gemm_run(c);
        if (rc) return rc;
    }
    if (dbias) {
        rc = nrs::bias_grad_launch(dbias, grad, N, c_out, P, beta_params);  // conv.rs:322
        if (rc) return rc;
    }
    return NRS_OK;
}

}  // extern "C"
