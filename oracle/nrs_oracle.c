/*
 * CPU oracle for the NeuralRs f32 matrix-multiply family.
 *
 * TEST INFRASTRUCTURE ONLY. This file restates, in plain C, the reference's
 * CPU algorithms for the GEMM / bmm / conv2d path so the HIP library can be
 * checked against them. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker (or the timed CPU
 * baseline). The product library never links or calls it.
 *
 * Build flags matter: -O2 -mavx2 -mfma -ffp-contract=off. Rust never fuses
 * a*b+c into an FMA unless the source asks for it (the AVX2 intrinsic in
 * dot_simd is the only FMA on the CPU path), so contraction must stay off for
 * the scalar loops to round exactly as the reference does.
 *
 * Every function cites the reference file:line it follows. Pinning of each
 * function (known answers, f64 ground truth, invariants, gradchecks) lives in
 * tests/test_oracle.py.
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* src/ops/simd.rs:8-37  dot_simd                                            */
/* 8-lane AVX2 FMA accumulator over the first 8*floor(n/8) elements, the     */
/* lanes summed left to right (tmp[0]+tmp[1]+...+tmp[7]), then the scalar    */
/* tail added one product at a time with separate multiply and add.          */
/* ------------------------------------------------------------------------ */
EXPORT float orc_dot_simd(const float *a, const float *b, int64_t n) {
    int64_t chunks = n / 8;
    int64_t rem = n % 8;
    __m256 acc = _mm256_setzero_ps();
    for (int64_t i = 0; i < chunks; ++i) {
        __m256 va = _mm256_loadu_ps(a + i * 8);
        __m256 vb = _mm256_loadu_ps(b + i * 8);
        acc = _mm256_fmadd_ps(va, vb, acc);
    }
    float tmp[8];
    _mm256_storeu_ps(tmp, acc);
    float sum = tmp[0] + tmp[1];
    sum = sum + tmp[2];
    sum = sum + tmp[3];
    sum = sum + tmp[4];
    sum = sum + tmp[5];
    sum = sum + tmp[6];
    sum = sum + tmp[7];
    int64_t tail = chunks * 8;
    for (int64_t i = 0; i < rem; ++i) {
        float p = a[tail + i] * b[tail + i];
        sum = sum + p;
    }
    return sum;
}

/* ------------------------------------------------------------------------ */
/* src/ops/simd.rs:42-77  matmul_simd (the default x86-64 ops::matmul,       */
/* src/ops/matmul.rs:47-56). Serial transpose of B into bt[n][k], then one   */
/* task per output row (Rayon par_chunks_mut(n)); each output element is an */
/* independent dot_simd, so the threading does not change any bits.          */
/* nthreads <= 0 uses the OpenMP default.                                    */
/* ------------------------------------------------------------------------ */
EXPORT void orc_matmul_simd(const float *A, const float *B, float *C,
                            int64_t m, int64_t k, int64_t n, int nthreads) {
    float *bt = (float *)malloc(sizeof(float) * (size_t)(n * k > 0 ? n * k : 1));
    for (int64_t row = 0; row < k; ++row)
        for (int64_t col = 0; col < n; ++col)
            bt[col * k + row] = B[row * n + col];
#ifdef _OPENMP
    int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#endif
    for (int64_t i = 0; i < m; ++i) {
        const float *arow = A + i * k;
        for (int64_t j = 0; j < n; ++j)
            C[i * n + j] = orc_dot_simd(arow, bt + j * k, k);
    }
    (void)nthreads;
    free(bt);
}

/* Rows [row0, row0+rows) of matmul_simd, for a bounded CPU-baseline sample. */
EXPORT void orc_matmul_simd_rows(const float *A, const float *B, float *C,
                                 int64_t m, int64_t k, int64_t n,
                                 int64_t row0, int64_t rows, int nthreads) {
    (void)m;
    orc_matmul_simd(A + row0 * k, B, C, rows, k, n, nthreads);
}

/* ------------------------------------------------------------------------ */
/* src/ops/matmul.rs:58-96  non-x86 fallback: sum over t ascending.          */
/* ------------------------------------------------------------------------ */
EXPORT void orc_matmul_naive(const float *A, const float *B, float *C,
                             int64_t m, int64_t k, int64_t n) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            float sum = 0.0f;
            for (int64_t t = 0; t < k; ++t) {
                float p = A[i * k + t] * B[t * n + j];
                sum = sum + p;
            }
            C[i * n + j] = sum;
        }
}

/* ------------------------------------------------------------------------ */
/* src/autograd/graph/matmul.rs:17-24  forward: data[i,j] += a[i,t]*b[t,j],  */
/* t ascending, starting from 0.0. Every output keeps exactly that sequence  */
/* of roundings; only the loop nest is reordered (a row of accumulators,     */
/* j innermost), so the bits equal the reference's i-j-t nest while the      */
/* loop runs at cache speed at the TransformerBlock sizes.                   */
/* ------------------------------------------------------------------------ */
EXPORT void orc_graph_matmul_forward(const float *A, const float *B, float *C,
                                     int64_t m, int64_t k, int64_t n) {
    for (int64_t i = 0; i < m; ++i) {
        float *acc = C + i * n;
        for (int64_t j = 0; j < n; ++j) acc[j] = 0.0f;
        for (int64_t t = 0; t < k; ++t) {
            const float a = A[i * k + t];
            const float *brow = B + t * n;
            for (int64_t j = 0; j < n; ++j) {
                float p = a * brow[j];
                acc[j] = acc[j] + p;
            }
        }
    }
}

/* src/autograd/graph/matmul.rs:37-63  backward, accumulating into dA, dB:   */
/*   dA[i,t] += sum_j g[i,j]*b[t,j]  (j ascending, partial sum from 0.0)     */
/*   dB[t,j] += sum_i a[i,t]*g[i,j]  (i ascending)                          */
/* Each partial sum sees the reference's terms in the reference's order; the */
/* nests are reordered so the independent sums advance together (dA over t  */
/* against a transposed copy of b, dB over whole rows), bits unchanged.     */
EXPORT void orc_graph_matmul_backward(const float *A, const float *B, const float *G,
                                      float *dA, float *dB,
                                      int64_t m, int64_t k, int64_t n) {
    float *bt = (float *)malloc(sizeof(float) * (size_t)(k * n > 0 ? k * n : 1));
    float *acc = (float *)malloc(sizeof(float) * (size_t)(k * n > k ? k * n : (k > 0 ? k : 1)));
    for (int64_t t = 0; t < k; ++t)
        for (int64_t j = 0; j < n; ++j) bt[j * k + t] = B[t * n + j];
    for (int64_t i = 0; i < m; ++i) {
        for (int64_t t = 0; t < k; ++t) acc[t] = 0.0f;
        for (int64_t j = 0; j < n; ++j) {
            const float g = G[i * n + j];
            const float *bcol = bt + j * k;
            for (int64_t t = 0; t < k; ++t) {
                float p = g * bcol[t];
                acc[t] = acc[t] + p;
            }
        }
        for (int64_t t = 0; t < k; ++t) dA[i * k + t] = dA[i * k + t] + acc[t];
    }
    for (int64_t e = 0; e < k * n; ++e) acc[e] = 0.0f;
    for (int64_t i = 0; i < m; ++i)
        for (int64_t t = 0; t < k; ++t) {
            const float a = A[i * k + t];
            const float *grow = G + i * n;
            float *arow = acc + t * n;
            for (int64_t j = 0; j < n; ++j) {
                float p = a * grow[j];
                arow[j] = arow[j] + p;
            }
        }
    for (int64_t e = 0; e < k * n; ++e) dB[e] = dB[e] + acc[e];
    free(acc);
    free(bt);
}

/* ------------------------------------------------------------------------ */
/* src/autograd/graph/bmm.rs:25-40  forward, per batch item, t ascending.    */
/* ------------------------------------------------------------------------ */
EXPORT void orc_graph_bmm_forward(const float *A, const float *B, float *C,
                                  int64_t batch, int64_t m, int64_t k, int64_t n) {
    for (int64_t bi = 0; bi < batch; ++bi)
        orc_matmul_naive(A + bi * m * k, B + bi * k * n, C + bi * m * n, m, k, n);
}

/* src/autograd/graph/bmm.rs:52-93  backward: per-item grads built in zeroed */
/* temporaries, then added into dA/dB element by element.                    */
EXPORT void orc_graph_bmm_backward(const float *A, const float *B, const float *G,
                                   float *dA, float *dB,
                                   int64_t batch, int64_t m, int64_t k, int64_t n) {
    size_t na = (size_t)(batch * m * k), nb = (size_t)(batch * k * n);
    float *ag = (float *)calloc(na ? na : 1, sizeof(float));
    float *bg = (float *)calloc(nb ? nb : 1, sizeof(float));
    for (int64_t bi = 0; bi < batch; ++bi) {
        int64_t ao = bi * m * k, bo = bi * k * n, oo = bi * m * n;
        for (int64_t i = 0; i < m; ++i)
            for (int64_t t = 0; t < k; ++t) {
                float g = 0.0f;
                for (int64_t j = 0; j < n; ++j) {
                    float p = G[oo + i * n + j] * B[bo + t * n + j];
                    g = g + p;
                }
                ag[ao + i * k + t] = ag[ao + i * k + t] + g;
            }
        for (int64_t t = 0; t < k; ++t)
            for (int64_t j = 0; j < n; ++j) {
                float g = 0.0f;
                for (int64_t i = 0; i < m; ++i) {
                    float p = A[ao + i * k + t] * G[oo + i * n + j];
                    g = g + p;
                }
                bg[bo + t * n + j] = bg[bo + t * n + j] + g;
            }
    }
    for (size_t i = 0; i < na; ++i) dA[i] = dA[i] + ag[i];
    for (size_t i = 0; i < nb; ++i) dB[i] = dB[i] + bg[i];
    free(ag);
    free(bg);
}

/* ------------------------------------------------------------------------ */
/* src/autograd/graph/add.rs:19-70  add with the 2-D + 1-D bias broadcast.   */
/* ------------------------------------------------------------------------ */
EXPORT void orc_graph_add_bias_forward(const float *a, const float *bias, float *out,
                                       int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c)
            out[r * cols + c] = a[r * cols + c] + bias[c];
}

/* add.rs:52-64: a.grad += g elementwise; bias.grad[f] += g[bi,f], bi ascending. */
EXPORT void orc_graph_add_bias_backward(const float *g, float *da, float *dbias,
                                        int64_t rows, int64_t cols) {
    for (int64_t i = 0; i < rows * cols; ++i) da[i] = da[i] + g[i];
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c)
            dbias[c] = dbias[c] + g[r * cols + c];
}

/* ------------------------------------------------------------------------ */
/* src/ops/im2col.rs:6-56  im2col, CPU layout [n][col_h][col_w] with         */
/* row = (ic*kh+i)*kw+j and column oy*out_w+ox; zero outside the input.      */
/* ------------------------------------------------------------------------ */
EXPORT void orc_im2col(const float *data, float *col,
                       int64_t n, int64_t c, int64_t in_h, int64_t in_w,
                       int64_t kh, int64_t kw, int64_t stride, int64_t pad) {
    int64_t out_h = (in_h + 2 * pad - kh) / stride + 1;
    int64_t out_w = (in_w + 2 * pad - kw) / stride + 1;
    int64_t col_h = c * kh * kw, col_w = out_h * out_w;
    for (int64_t ni = 0; ni < n; ++ni)
        for (int64_t ic = 0; ic < c; ++ic)
            for (int64_t i = 0; i < kh; ++i)
                for (int64_t j = 0; j < kw; ++j) {
                    int64_t row = (ic * kh + i) * kw + j;
                    for (int64_t oy = 0; oy < out_h; ++oy)
                        for (int64_t ox = 0; ox < out_w; ++ox) {
                            int64_t iy = oy * stride + i, ix = ox * stride + j;
                            float v = 0.0f;
                            if (!(iy < pad || ix < pad || iy >= pad + in_h || ix >= pad + in_w))
                                v = data[((ni * c + ic) * in_h + (iy - pad)) * in_w + (ix - pad)];
                            col[(ni * col_h + row) * col_w + oy * out_w + ox] = v;
                        }
                }
}

/* src/ops/im2col.rs:59-98  conv2d_im2col: per sample, matmul_simd(W, cols)  */
/* then + bias[oc].                                                          */
EXPORT void orc_conv2d_im2col(const float *data, const float *weight, const float *bias,
                              float *out, int64_t n, int64_t c_in, int64_t c_out,
                              int64_t in_h, int64_t in_w, int64_t kh, int64_t kw,
                              int64_t stride, int64_t pad, int nthreads) {
    int64_t out_h = (in_h + 2 * pad - kh) / stride + 1;
    int64_t out_w = (in_w + 2 * pad - kw) / stride + 1;
    int64_t col_h = c_in * kh * kw, col_w = out_h * out_w;
    float *col = (float *)malloc(sizeof(float) * (size_t)(n * col_h * col_w + 1));
    float *res = (float *)malloc(sizeof(float) * (size_t)(c_out * col_w + 1));
    orc_im2col(data, col, n, c_in, in_h, in_w, kh, kw, stride, pad);
    for (int64_t ni = 0; ni < n; ++ni) {
        orc_matmul_simd(weight, col + ni * col_h * col_w, res, c_out, col_h, col_w, nthreads);
        for (int64_t oc = 0; oc < c_out; ++oc)
            for (int64_t p = 0; p < col_w; ++p)
                out[(ni * c_out + oc) * col_w + p] = res[oc * col_w + p] + bias[oc];
    }
    free(col);
    free(res);
}

/* ------------------------------------------------------------------------ */
/* src/nn/conv.rs:33-97  Conv2d forward: direct convolution on a zero-padded */
/* copy; per output sum over (ic, i, j) ascending from 0.0, then + bias.     */
/* ------------------------------------------------------------------------ */
static float *pad_input(const float *raw, int64_t n, int64_t c, int64_t in_h, int64_t in_w,
                        int64_t pad) {
    int64_t ph = in_h + 2 * pad, pw = in_w + 2 * pad;
    float *d = (float *)calloc((size_t)(n * c * ph * pw + 1), sizeof(float));
    for (int64_t ni = 0; ni < n; ++ni)
        for (int64_t ic = 0; ic < c; ++ic)
            for (int64_t y = 0; y < in_h; ++y)
                for (int64_t x = 0; x < in_w; ++x)
                    d[((ni * c + ic) * ph + y + pad) * pw + x + pad] =
                        raw[((ni * c + ic) * in_h + y) * in_w + x];
    return d;
}

EXPORT void orc_conv2d_forward(const float *input, const float *weight, const float *bias,
                               float *out, int64_t n, int64_t c_in, int64_t c_out,
                               int64_t in_h, int64_t in_w, int64_t kh, int64_t kw,
                               int64_t stride, int64_t pad) {
    int64_t ph = in_h + 2 * pad, pw = in_w + 2 * pad;
    int64_t out_h = (ph - kh) / stride + 1, out_w = (pw - kw) / stride + 1;
    float *d = pad_input(input, n, c_in, in_h, in_w, pad);
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t map = 0; map < n * c_out; ++map) {
        int64_t ni = map / c_out, oc = map % c_out;
        for (int64_t oy = 0; oy < out_h; ++oy)
            for (int64_t ox = 0; ox < out_w; ++ox) {
                float sum = 0.0f;
                for (int64_t ic = 0; ic < c_in; ++ic)
                    for (int64_t i = 0; i < kh; ++i)
                        for (int64_t j = 0; j < kw; ++j) {
                            float p = d[((ni * c_in + ic) * ph + oy * stride + i) * pw + ox * stride + j] *
                                      weight[((oc * c_in + ic) * kh + i) * kw + j];
                            sum = sum + p;
                        }
                sum = sum + bias[oc];
                out[(map * out_h + oy) * out_w + ox] = sum;
            }
    }
    free(d);
}

/* ------------------------------------------------------------------------ */
/* src/nn/conv.rs:110-200  Conv2d backward, accumulating into dinput,        */
/* dweight, dbias.                                                           */
/* wgrad/bgrad (:114-150): the reference folds over units u = ni*c_out+oc    */
/* with Rayon fold/reduce, whose partitioning is chosen at run time, so its  */
/* bits are not reproducible; this restatement uses one partition (units in */
/* ascending order, a single fold) and is pinned by tolerance only.          */
/* dgrad (:152-179): per sample, loops oc, oy, ox, ic, i, j ascending into a */
/* zeroed padded buffer, then un-padded and added (:181-194).                */
/* ------------------------------------------------------------------------ */
EXPORT void orc_conv2d_backward(const float *input, const float *weight, const float *grad,
                                float *dinput, float *dweight, float *dbias,
                                int64_t n, int64_t c_in, int64_t c_out,
                                int64_t in_h, int64_t in_w, int64_t kh, int64_t kw,
                                int64_t stride, int64_t pad) {
    int64_t ph = in_h + 2 * pad, pw = in_w + 2 * pad;
    int64_t out_h = (ph - kh) / stride + 1, out_w = (pw - kw) / stride + 1;
    int64_t w_len = c_out * c_in * kh * kw;
    float *d = pad_input(input, n, c_in, in_h, in_w, pad);

    float *wg = (float *)calloc((size_t)(w_len + 1), sizeof(float));
    float *bg = (float *)calloc((size_t)(c_out + 1), sizeof(float));
    for (int64_t unit = 0; unit < n * c_out; ++unit) {
        int64_t ni = unit / c_out, oc = unit % c_out;
        for (int64_t oy = 0; oy < out_h; ++oy)
            for (int64_t ox = 0; ox < out_w; ++ox) {
                float g = grad[((ni * c_out + oc) * out_h + oy) * out_w + ox];
                bg[oc] = bg[oc] + g;
                for (int64_t ic = 0; ic < c_in; ++ic)
                    for (int64_t i = 0; i < kh; ++i)
                        for (int64_t j = 0; j < kw; ++j) {
                            int64_t w_idx = ((oc * c_in + ic) * kh + i) * kw + j;
                            float p = g * d[((ni * c_in + ic) * ph + oy * stride + i) * pw + ox * stride + j];
                            wg[w_idx] = wg[w_idx] + p;
                        }
            }
    }

    int64_t in_block = c_in * ph * pw;
    float *pg = (float *)calloc((size_t)(n * in_block + 1), sizeof(float));
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t ni = 0; ni < n; ++ni) {
        float *chunk = pg + ni * in_block;
        for (int64_t oc = 0; oc < c_out; ++oc)
            for (int64_t oy = 0; oy < out_h; ++oy)
                for (int64_t ox = 0; ox < out_w; ++ox) {
                    float g = grad[((ni * c_out + oc) * out_h + oy) * out_w + ox];
                    for (int64_t ic = 0; ic < c_in; ++ic)
                        for (int64_t i = 0; i < kh; ++i)
                            for (int64_t j = 0; j < kw; ++j) {
                                int64_t loc = (ic * ph + oy * stride + i) * pw + ox * stride + j;
                                float p = g * weight[((oc * c_in + ic) * kh + i) * kw + j];
                                chunk[loc] = chunk[loc] + p;
                            }
                }
    }
    for (int64_t ni = 0; ni < n; ++ni)
        for (int64_t ic = 0; ic < c_in; ++ic)
            for (int64_t y = 0; y < in_h; ++y)
                for (int64_t x = 0; x < in_w; ++x) {
                    int64_t dst = ((ni * c_in + ic) * in_h + y) * in_w + x;
                    dinput[dst] = dinput[dst] + pg[((ni * c_in + ic) * ph + y + pad) * pw + x + pad];
                }
    for (int64_t k = 0; k < w_len; ++k) dweight[k] = dweight[k] + wg[k];
    for (int64_t k = 0; k < c_out; ++k) dbias[k] = dbias[k] + bg[k];
    free(pg);
    free(wg);
    free(bg);
    free(d);
}

/* ------------------------------------------------------------------------ */
/* Restatements of the reference GPU primitives' index semantics, which the  */
/* C-ABI primitives keep (src/cuda/nn/conv.rs:27-149, src/cuda/reduce.rs,    */
/* src/cuda/runtime.rs, src/cuda/graph/add.rs). Integer/index work: the HIP  */
/* versions must match these bit for bit.                                    */
/* ------------------------------------------------------------------------ */

/* cuda/nn/conv.rs:27-58: cols[row, ni*P + p], shape [c_in*kh*kw, N*P]. */
EXPORT void orc_gpu_im2col(const float *input, float *cols, int64_t N, int64_t c_in,
                           int64_t in_h, int64_t in_w, int64_t kh, int64_t kw,
                           int64_t stride, int64_t pad) {
    int64_t out_h = (in_h + 2 * pad - kh) / stride + 1;
    int64_t out_w = (in_w + 2 * pad - kw) / stride + 1;
    int64_t P = out_h * out_w, width = N * P, col_h = c_in * kh * kw;
    for (int64_t row = 0; row < col_h; ++row) {
        int64_t j = row % kw, i = (row / kw) % kh, ic = row / (kw * kh);
        for (int64_t rest = 0; rest < width; ++rest) {
            int64_t ni = rest / P, p = rest % P, oy = p / out_w, ox = p % out_w;
            int64_t iy = oy * stride + i - pad, ix = ox * stride + j - pad;
            float v = 0.0f;
            if (iy >= 0 && iy < in_h && ix >= 0 && ix < in_w)
                v = input[((ni * c_in + ic) * in_h + iy) * in_w + ix];
            cols[row * width + rest] = v;
        }
    }
}

/* cuda/nn/conv.rs:62-76: NCHW out = mm_out[oc, ni*P+p] + bias[oc]. */
EXPORT void orc_gpu_col2out(const float *mm, const float *bias, float *out,
                            int64_t N, int64_t c_out, int64_t P) {
    for (int64_t idx = 0; idx < N * c_out * P; ++idx) {
        int64_t p = idx % P, oc = (idx / P) % c_out, ni = idx / (P * c_out);
        out[idx] = mm[oc * (N * P) + ni * P + p] + bias[oc];
    }
}

/* cuda/nn/conv.rs:94-108: [c_out, N*P] <- NCHW grad. */
EXPORT void orc_gpu_out2mm(const float *grad, float *mm, int64_t N, int64_t c_out, int64_t P) {
    for (int64_t idx = 0; idx < N * c_out * P; ++idx) {
        int64_t p = idx % P, oc = (idx / P) % c_out, ni = idx / (P * c_out);
        mm[oc * (N * P) + ni * P + p] = grad[idx];
    }
}

/* cuda/nn/conv.rs:113-149: gather dcols onto input pixels, (i, j) ascending. */
EXPORT void orc_gpu_col2im(const float *dcols, float *dinput, int64_t N, int64_t c_in,
                           int64_t in_h, int64_t in_w, int64_t kh, int64_t kw,
                           int64_t stride, int64_t pad) {
    int64_t out_h = (in_h + 2 * pad - kh) / stride + 1;
    int64_t out_w = (in_w + 2 * pad - kw) / stride + 1;
    int64_t P = out_h * out_w, width = N * P;
    for (int64_t idx = 0; idx < N * c_in * in_h * in_w; ++idx) {
        int64_t x = idx % in_w, y = (idx / in_w) % in_h;
        int64_t ic = (idx / (in_w * in_h)) % c_in, ni = idx / (in_w * in_h * c_in);
        float acc = 0.0f;
        for (int64_t i = 0; i < kh; ++i) {
            int64_t oyn = y + pad - i;
            if (oyn < 0 || oyn % stride != 0) continue;
            int64_t oy = oyn / stride;
            if (oy >= out_h) continue;
            for (int64_t j = 0; j < kw; ++j) {
                int64_t oxn = x + pad - j;
                if (oxn < 0 || oxn % stride != 0) continue;
                int64_t ox = oxn / stride;
                if (ox >= out_w) continue;
                int64_t row = (ic * kh + i) * kw + j;
                acc = acc + dcols[row * width + ni * P + oy * out_w + ox];
            }
        }
        dinput[idx] = acc;
    }
}

/* cuda/nn/conv.rs:78-90: db[oc] = sum over (ni, oy, ox) ascending. */
EXPORT void orc_gpu_bias_grad(const float *grad, float *dbias, int64_t N, int64_t c_out,
                              int64_t P) {
    for (int64_t oc = 0; oc < c_out; ++oc) {
        float acc = 0.0f;
        for (int64_t ni = 0; ni < N; ++ni)
            for (int64_t p = 0; p < P; ++p) acc = acc + grad[(ni * c_out + oc) * P + p];
        dbias[oc] = acc;
    }
}

/* cuda/reduce.rs:12-21: out[c] = sum_r in[r, c], r ascending. */
EXPORT void orc_sum_axis0(const float *in, float *out, int64_t rows, int64_t cols) {
    for (int64_t c = 0; c < cols; ++c) {
        float acc = 0.0f;
        for (int64_t r = 0; r < rows; ++r) acc = acc + in[r * cols + c];
        out[c] = acc;
    }
}

/* cuda/nn/maxpool.rs:18-52: first-max wins (strict >), argmax is the flat   */
/* input index; backward scatters grad to argmax with +=.                    */
EXPORT void orc_maxpool_forward(const float *input, float *out, int32_t *argmax,
                                int64_t N, int64_t C, int64_t in_h, int64_t in_w,
                                int64_t k, int64_t stride) {
    int64_t out_h = (in_h - k) / stride + 1, out_w = (in_w - k) / stride + 1;
    for (int64_t idx = 0; idx < N * C * out_h * out_w; ++idx) {
        int64_t ox = idx % out_w, oy = (idx / out_w) % out_h;
        int64_t ch = (idx / (out_w * out_h)) % C, ni = idx / (out_w * out_h * C);
        int64_t first = ((ni * C + ch) * in_h + oy * stride) * in_w + ox * stride;
        float best = input[first];
        int64_t bi = first;
        for (int64_t i = 0; i < k; ++i)
            for (int64_t j = 0; j < k; ++j) {
                int64_t ii = ((ni * C + ch) * in_h + oy * stride + i) * in_w + ox * stride + j;
                if (input[ii] > best) { best = input[ii]; bi = ii; }
            }
        out[idx] = best;
        argmax[idx] = (int32_t)bi;
    }
}

EXPORT void orc_maxpool_backward(const float *grad, const int32_t *argmax, float *dinput,
                                 int64_t total) {
    for (int64_t idx = 0; idx < total; ++idx) dinput[argmax[idx]] = dinput[argmax[idx]] + grad[idx];
}

/* ------------------------------------------------------------------------ */
/* f64 ground truth for the three GEMM layouts of the reference              */
/* (src/cuda/graph/matmul.rs:44-198):                                        */
/*   layout 0 NN: C[r,c] = sum_t A[r*inner+t] * B[t*cols+c]                  */
/*   layout 1 NT: C[r,c] = sum_t A[r*inner+t] * B[c*inner+t]                 */
/*   layout 2 TN: C[r,c] = sum_t A[t*rows+r]  * B[t*cols+c]                  */
/* Also returns absprod[r,c] = sum_t |a||b|, the scale that bounds any f32   */
/* summation order's rounding error. The rowset form computes only the rows */
/* listed in rowidx (output row s holds row rowidx[s]).                      */
/* ------------------------------------------------------------------------ */
EXPORT void orc_gemm_f64_rowset(int layout, const float *A, const float *B, double *C,
                                double *absprod, int64_t rows, int64_t cols, int64_t inner,
                                const int64_t *rowidx, int64_t nsel) {
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1)
#endif
    for (int64_t s = 0; s < nsel; ++s) {
        int64_t r = rowidx ? rowidx[s] : s;
        double *acc = (double *)calloc((size_t)cols + 1, sizeof(double));
        double *aab = (double *)calloc((size_t)cols + 1, sizeof(double));
        for (int64_t t = 0; t < inner; ++t) {
            double a = layout == 2 ? (double)A[t * rows + r] : (double)A[r * inner + t];
            if (layout == 1) {
                for (int64_t c = 0; c < cols; ++c) {
                    double b = (double)B[c * inner + t];
                    acc[c] += a * b;
                    aab[c] += fabs(a * b);
                }
            } else {
                const float *brow = B + t * cols;
                for (int64_t c = 0; c < cols; ++c) {
                    double b = (double)brow[c];
                    acc[c] += a * b;
                    aab[c] += fabs(a * b);
                }
            }
        }
        for (int64_t c = 0; c < cols; ++c) {
            C[s * cols + c] = acc[c];
            if (absprod) absprod[s * cols + c] = aab[c];
        }
        free(acc);
        free(aab);
    }
}

EXPORT void orc_gemm_f64(int layout, const float *A, const float *B, double *C, double *absprod,
                         int64_t rows, int64_t cols, int64_t inner) {
    orc_gemm_f64_rowset(layout, A, B, C, absprod, rows, cols, inner, NULL, rows);
}

/* ------------------------------------------------------------------------ */
/* Attention / MLP glue twins (CPU autograd ops), used by the composed-op    */
/* parity tests.                                                              */
/* src/autograd/graph/transpose.rs:4-25 forward: out[b, j, i] = in[b, i, j]. */
/* ------------------------------------------------------------------------ */
EXPORT void orc_transpose(const float *in, float *out, int64_t batch, int64_t rows,
                          int64_t cols) {
    for (int64_t b = 0; b < batch; ++b) {
        int64_t off = b * rows * cols;
        for (int64_t i = 0; i < rows; ++i)
            for (int64_t j = 0; j < cols; ++j) out[off + j * rows + i] = in[off + i * cols + j];
    }
}

/* src/autograd/graph/transpose.rs:35-45 backward: ga[b,i,j] += g[b,j,i].    */
EXPORT void orc_transpose_backward(const float *g, float *ga, int64_t batch, int64_t rows,
                                   int64_t cols) {
    for (int64_t b = 0; b < batch; ++b) {
        int64_t off = b * rows * cols;
        for (int64_t i = 0; i < rows; ++i)
            for (int64_t j = 0; j < cols; ++j)
                ga[off + i * cols + j] = ga[off + i * cols + j] + g[off + j * rows + i];
    }
}

/* src/autograd/graph/slice_cols.rs:12-31 forward: out[r, c] = a[r, col_start */
/* + c] for c < col_end - col_start (rows = len / total_cols).                */
EXPORT void orc_slice_cols(const float *a, float *out, int64_t rows, int64_t total_cols,
                           int64_t col_start, int64_t col_end) {
    const int64_t w = col_end - col_start;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < w; ++c) out[r * w + c] = a[r * total_cols + (col_start + c)];
}

/* src/autograd/graph/slice_cols.rs:36-44 backward:                           */
/* ga[r, col_start + c] += grad[r, c].                                        */
EXPORT void orc_slice_cols_backward(const float *grad, float *ga, int64_t rows,
                                    int64_t total_cols, int64_t col_start, int64_t col_end) {
    const int64_t w = col_end - col_start;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < w; ++c)
            ga[r * total_cols + (col_start + c)] = ga[r * total_cols + (col_start + c)] +
                                                   grad[r * w + c];
}

/* src/autograd/graph/concat_cols.rs:22-30 forward, one part at col_offset:   */
/* out[r, col_offset + c] = part[r, c].                                       */
EXPORT void orc_concat_part(const float *part, float *out, int64_t rows, int64_t total_cols,
                            int64_t col_offset, int64_t pw) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < pw; ++c) out[r * total_cols + (col_offset + c)] = part[r * pw + c];
}

/* src/autograd/graph/concat_cols.rs:44-55 backward, one part:                */
/* gpart[r, c] += grad[r, col_offset + c].                                    */
EXPORT void orc_concat_part_backward(const float *grad, float *gpart, int64_t rows,
                                     int64_t total_cols, int64_t col_offset, int64_t pw) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < pw; ++c)
            gpart[r * pw + c] = gpart[r * pw + c] + grad[r * total_cols + (col_offset + c)];
}

/* nn::normalization::LayerNorm (src/nn/normalization.rs:24-56) forward:     */
/* per row, mean = sum/F and var = sum((x-mean)^2)/F summed left to right,    */
/* istd = 1/sqrt(var + eps), x_norm = (x - mean)*istd, out = gamma*x_norm +   */
/* beta. x_norm and inv_std are kept for the backward.                        */
EXPORT void orc_layernorm_forward(const float *in, const float *gamma, const float *beta,
                                  float *out, float *x_norm, float *inv_std, int64_t rows,
                                  int64_t F, float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *x = in + r * F;
        float s = 0.0f;
        for (int64_t f = 0; f < F; ++f) s = s + x[f];
        const float mean = s / (float)F;
        float q = 0.0f;
        for (int64_t f = 0; f < F; ++f) {
            const float d = x[f] - mean;
            q = q + d * d;
        }
        const float var = q / (float)F;
        const float istd = 1.0f / sqrtf(var + eps);
        inv_std[r] = istd;
        for (int64_t f = 0; f < F; ++f) {
            const float xn = (x[f] - mean) * istd;
            x_norm[r * F + f] = xn;
            out[r * F + f] = gamma[f] * xn + beta[f];
        }
    }
}

/* src/nn/normalization.rs:58-97 backward: per row sum1 = sum(dxh), sum2 =    */
/* sum(dxh*x_norm) with dxh = grad*gamma; din += istd*(dxh - sum1/F -         */
/* x_norm*sum2/F); dgamma += grad*x_norm and dbeta += grad over rows (the     */
/* per-call sums are added to the running grads at the end).                  */
EXPORT void orc_layernorm_backward(const float *grad, const float *gamma, const float *x_norm,
                                   const float *inv_std, float *din, float *dgamma,
                                   float *dbeta, int64_t rows, int64_t F) {
    float *dg = (float *)calloc((size_t)F, sizeof(float));
    float *db = (float *)calloc((size_t)F, sizeof(float));
    const float nf = (float)F;
    for (int64_t r = 0; r < rows; ++r) {
        const float istd = inv_std[r];
        float s1 = 0.0f, s2 = 0.0f;
        for (int64_t f = 0; f < F; ++f) {
            const float d = grad[r * F + f] * gamma[f];
            s1 = s1 + d;
            s2 = s2 + d * x_norm[r * F + f];
        }
        for (int64_t f = 0; f < F; ++f) {
            const int64_t i = r * F + f;
            const float d = grad[i] * gamma[f];
            din[i] = din[i] + istd * (d - s1 / nf - x_norm[i] * s2 / nf);
            dg[f] = dg[f] + grad[i] * x_norm[i];
            db[f] = db[f] + grad[i];
        }
    }
    for (int64_t f = 0; f < F; ++f) {
        dgamma[f] = dgamma[f] + dg[f];
        dbeta[f] = dbeta[f] + db[f];
    }
    free(dg);
    free(db);
}

/* src/autograd/graph/scale.rs:7-33: out = x*s; backward ga += g*s.          */
EXPORT void orc_scale(const float *x, float *out, float s, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = x[i] * s;
}
EXPORT void orc_scale_backward(const float *g, float *ga, float s, int64_t n) {
    for (int64_t i = 0; i < n; ++i) ga[i] = ga[i] + g[i] * s;
}

/* src/autograd/graph/softmax.rs:14-35 forward: per row, max folded from     */
/* -inf, exps = exp(x - max), sum of exps left to right, out = exp / sum.   */
EXPORT void orc_softmax_forward(const float *in, float *out, int64_t rows, int64_t width) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *x = in + r * width;
        float mx = -INFINITY;
        for (int64_t f = 0; f < width; ++f) mx = fmaxf(mx, x[f]);
        float sum = 0.0f;
        for (int64_t f = 0; f < width; ++f) {
            out[r * width + f] = expf(x[f] - mx);
            sum = sum + out[r * width + f];
        }
        for (int64_t f = 0; f < width; ++f) out[r * width + f] = out[r * width + f] / sum;
    }
}

/* src/autograd/graph/softmax.rs:43-57 backward from the forward output y:  */
/* dot = sum_f y*g (left to right); ga += y*(g - dot).                       */
EXPORT void orc_softmax_backward(const float *y, const float *g, float *ga, int64_t rows,
                                 int64_t width) {
    for (int64_t r = 0; r < rows; ++r) {
        float dot = 0.0f;
        for (int64_t f = 0; f < width; ++f) dot = dot + y[r * width + f] * g[r * width + f];
        for (int64_t f = 0; f < width; ++f) {
            int64_t i = r * width + f;
            ga[i] = ga[i] + y[i] * (g[i] - dot);
        }
    }
}

/* src/nn/loss.rs:49-75 (CrossEntropyLoss::forward): per row, max folded    */
/* from -inf with f32::max, sum_exp = sum of exp(x - max) in class order,    */
/* log_sum_exp = ln(sum_exp) + max; total += -t * (x - log_sum_exp) over     */
/* rows then classes; returns total / batch.                                 */
EXPORT float orc_cross_entropy_loss(const float *logits, const float *target, int64_t batch,
                                    int64_t classes) {
    float total = 0.0f;
    for (int64_t b = 0; b < batch; ++b) {
        const float *row = logits + b * classes;
        float mx = -INFINITY;
        for (int64_t c = 0; c < classes; ++c) mx = fmaxf(mx, row[c]);
        float sum_exp = 0.0f;
        for (int64_t c = 0; c < classes; ++c) sum_exp = sum_exp + expf(row[c] - mx);
        const float lse = logf(sum_exp) + mx;
        for (int64_t c = 0; c < classes; ++c) {
            const float log_softmax = row[c] - lse;
            total = total + (-target[b * classes + c]) * log_softmax;
        }
    }
    return total / (float)batch;
}

/* src/nn/loss.rs:77-106 (CrossEntropyLoss::backward): exps = exp(x - max),  */
/* sum in class order, grad = (exps / sum - t) / batch (assigned).           */
EXPORT void orc_cross_entropy_grad(const float *logits, const float *target, float *grad,
                                   int64_t batch, int64_t classes) {
    for (int64_t b = 0; b < batch; ++b) {
        const float *row = logits + b * classes;
        float mx = -INFINITY;
        for (int64_t c = 0; c < classes; ++c) mx = fmaxf(mx, row[c]);
        float sum = 0.0f;
        for (int64_t c = 0; c < classes; ++c) sum = sum + expf(row[c] - mx);
        for (int64_t c = 0; c < classes; ++c) {
            const float softmax_c = expf(row[c] - mx) / sum;
            grad[b * classes + c] = (softmax_c - target[b * classes + c]) / (float)batch;
        }
    }
}

/* src/autograd/graph/relu.rs:10-45: out = x > 0 ? x : 0; ga += x > 0 ? g : 0. */
EXPORT void orc_relu_forward(const float *x, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = x[i] > 0.0f ? x[i] : 0.0f;
}
EXPORT void orc_relu_backward(const float *x, const float *g, float *ga, int64_t n) {
    for (int64_t i = 0; i < n; ++i) ga[i] = ga[i] + (x[i] > 0.0f ? g[i] : 0.0f);
}

/* Threads of the OpenMP loops above (the CPU baseline's 1-thread figures). */
EXPORT void orc_set_threads(int n) {
#ifdef _OPENMP
    omp_set_num_threads(n > 0 ? n : 1);
#else
    (void)n;
#endif
}

EXPORT int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
