/*
 * nrs_hip.h -- C ABI of the MI355X (gfx950) backend for NeuralRs's f32
 * matrix-multiply family.
 *
 * This is the drop-in boundary: the entry points are the kernel-level seams
 * that the reference's resident GPU ops call today through cudarc, so a `hip`
 * cargo feature beside `cuda` (Cargo.toml:23-26) can bind them with
 * `extern "C"` declarations and keep the operator API (`runtime::to_cuda`,
 * `graph::matmul`, `graph::bmm`, `nn::conv2d`, `nn::Linear`) unchanged.
 *
 * Conventions (all entry points):
 *   - f32 only, row-major matrices, NCHW images, sizes as int64_t.
 *   - Device pointers are allocated by the caller (nrs_malloc or any HIP
 *     allocation on the same device); the library owns only its internal
 *     scratch (split-K partials, im2col columns), grown lazily and released
 *     by nrs_shutdown().
 *   - Every call is asynchronous on the library stream (nrs_set_stream;
 *     default: the null stream) except the D->H copies and nrs_sync, exactly
 *     like the reference's single default stream (src/cuda/backend.rs:30-32).
 *   - Return 0 (NRS_OK) on success, else an NRS_ERR_* code; the message is in
 *     nrs_last_error(). The reference panics on the same conditions
 *     (e.g. "cuda matmul: inner dims mismatch", src/cuda/graph/matmul.rs:398);
 *     the host wrapper turns a non-zero code into that panic/exception.
 *   - Not thread-safe (the reference's host side is Rc<RefCell>, !Send).
 */
#ifndef NRS_HIP_H
#define NRS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum nrs_status {
    NRS_OK = 0,
    NRS_ERR_HIP = 1,   /* a HIP runtime call or kernel launch failed      */
    NRS_ERR_ARG = 2,   /* bad shape, null pointer or unsupported argument */
    NRS_ERR_ALLOC = 3, /* device allocation failed                        */
};

/* GEMM operand layouts: the three kernels of src/cuda/graph/matmul.rs. */
enum nrs_layout {
    NRS_NN = 0, /* C[r,c] = sum_t A[r,t] B[t,c]; A [rows,inner], B [inner,cols] (matmul_nn :44-94)  */
    NRS_NT = 1, /* C[r,c] = sum_t A[r,t] B[c,t]; A [rows,inner], B [cols,inner] (matmul_nt :96-146) */
    NRS_TN = 2, /* C[r,c] = sum_t A[t,r] B[t,c]; A [inner,rows], B [inner,cols] (matmul_tn :148-198)*/
};

/* Epilogue flags for nrs_gemm (bit-or). Applied after the product:
 *   v = acc (+ bias) (relu) ; C = v + beta * C_old                           */
enum nrs_epilogue {
    NRS_EPI_NONE = 0,
    NRS_EPI_BIAS_COL = 1, /* + bias[c]   (Linear bias, src/cuda/graph/add.rs:25-30)   */
    NRS_EPI_BIAS_ROW = 2, /* + bias[r]   (conv bias, src/cuda/nn/conv.rs:62-76)       */
    NRS_EPI_RELU = 4,     /* max(v, 0)   (src/cuda/graph/relu.rs:16-28)              */
};

/* ---------------------------------------------------------------- runtime */
/* Replaces backend::get() (src/cuda/backend.rs:19-28): select device, init. */
int nrs_init(int device);
/* Frees library scratch. */
int nrs_shutdown(void);
/* Stream all subsequent calls enqueue on (hipStream_t as void*); NULL = null stream. */
int nrs_set_stream(void *stream);
void *nrs_get_stream(void);
/* Message for the last non-zero status (thread-local, valid until the next call). */
const char *nrs_last_error(void);
/* Device buffers: replace stream.alloc_zeros / CudaSlice drop (runtime.rs:39-51).
 * A caching allocator: sizes round up to classes (512 B steps to 1 MiB, 2 MiB
 * steps above); nrs_free returns the block to its class's cache, and the next
 * nrs_malloc of that class reuses it in library-stream order. nrs_free of a
 * pointer that is not a live nrs_malloc buffer is an error. Memory is not
 * zeroed (alloc_zeros = nrs_malloc + nrs_memset_zero).                       */
int nrs_malloc(void **ptr, size_t bytes);
int nrs_free(void *ptr);
/* hipFree every cached idle block (live buffers are untouched); also done by
 * nrs_shutdown and, once, by an nrs_malloc that runs out of memory.          */
int nrs_empty_cache(void);
/* Bytes held by live buffers and by idle cached blocks (class-rounded).     */
int nrs_memory_stats(size_t *live_bytes, size_t *cached_bytes);
/* clone_htod / clone_dtoh (runtime.rs:39-63). dtoh synchronises the stream. */
int nrs_memcpy_htod(void *dst, const void *src, size_t bytes);
int nrs_memcpy_dtoh(void *dst, const void *src, size_t bytes);
int nrs_memcpy_dtod(void *dst, const void *src, size_t bytes);
/* memset_zeros (runtime.rs:108-117 zero_grad) -- a fill kernel, graph-capture safe. */
int nrs_memset_zero(void *ptr, size_t bytes);
/* runtime::synchronize (runtime.rs:122-124). */
int nrs_sync(void);

/* ------------------------------------------------------------------ GEMM */
/* mm(kernel, a, b, rows, cols, inner) (src/cuda/graph/matmul.rs:343-348) with
 * the layout selecting matmul_nn/nt/tn. Unlike the reference, C is not
 * freshly allocated: C = epi(A op B) + beta*C, so beta=1 fuses the
 * accumulate_into() that follows every backward GEMM (runtime.rs:67-83).
 * bias may be NULL unless a BIAS flag is set. rows/cols/inner may be 0.       */
int nrs_gemm(int layout, float *C, const float *A, const float *B,
             int64_t rows, int64_t cols, int64_t inner,
             float beta, const float *bias, int epilogue);

/* Several mm calls in one launch: the two gradient products of a matmul
 * node's backward closure (src/cuda/graph/matmul.rs:418-431: matmul_nt for dA
 * and matmul_tn for dB, each followed by accumulate_into) or the projections
 * of one input (src/cuda/nn/multihead.rs:64-66, three matmuls of x). Each
 * descriptor means exactly nrs_gemm with its fields; at most
 * NRS_GEMM_GROUP_MAX of them. When every call is dense, 16-byte aligned with
 * rows of whole float4s and no output overlaps another call's output or
 * operands, their workgroups share one grid (one problem's load latency,
 * barriers and epilogue overlap another's matrix-core work); otherwise the
 * calls run one after another in the order given. Results equal nrs_gemm's to
 * the GEMM tolerance (the tiling, hence the summation order, may differ).   */
#define NRS_GEMM_GROUP_MAX 4
typedef struct nrs_gemm_desc {
    int layout;
    float *C;
    const float *A;
    const float *B;
    int64_t rows, cols, inner;
    float beta;
    const float *bias;
    int epilogue;
} nrs_gemm_desc;
int nrs_gemm_group(const nrs_gemm_desc *descs, int count);

/* The backward of count (1 to 3) products sharing their left operand,
 * y_i = x . W_i: the Q, K and V projections of one input (src/cuda/nn/
 * multihead.rs:64-66), each with the matmul closure of src/cuda/graph/
 * matmul.rs:418-431 (replaces those closures run one after another).
 * x [rows, inner], W_i [inner, cols], g_i = dL/dy_i [rows, cols]:
 *   dx   = ((g_0 . W_0^T + beta_x * dx) + g_1 . W_1^T) + g_2 . W_2^T
 *   dW_i = x^T . g_i + beta_w[i] * dW_i
 * The input gradient adds the parts in index order: with index 0 the
 * closure that would run first, the bits are those of the closures run in
 * turn (each the nrs_gemm_group of its two products, the first adding to dx
 * with beta_x, the others with 1). All products run in one grouped launch
 * and the sums in a second. When an output overlaps another output or an
 * operand, or the products are small enough for the short-GEMM kernel, the
 * closures' sequence runs instead (same results). */
int nrs_matmul_shared_lhs_backward(float *dx, float *const *dw, const float *const *g,
                                   const float *x, const float *const *w, int count,
                                   int64_t rows, int64_t inner, int64_t cols, float beta_x,
                                   const float *beta_w);

/* The backward of Linear::forward = add(matmul(x, W), bias) (src/cuda/nn/
 * linear.rs:22-25; the closures of src/cuda/graph/matmul.rs:418-431 and
 * src/cuda/graph/add.rs:91-100), grad [batch, out_f], x [batch, in_f],
 * W [in_f, out_f]:
 *   dW = x^T . grad + beta_w * dW          (matmul_tn + accumulate_into)
 *   db = sum over rows of grad + beta_b*db (sum_axis0 + accumulate_into)
 *   dx = grad . W^T + beta_x * dx          (matmul_nt + accumulate_into)
 * in one grouped launch (plus a split-K reduce when the weight gradient is
 * split): db is computed as an extra output row of the weight-gradient
 * product whose x^T row is all ones, so it needs no column-sum launch, where
 * that row costs no extra tile row (in_f not a multiple of 64) or the
 * product is small (else the column sums follow as one nrs_sum_axis0). dx
 * and db may be NULL (not computed); dW may not. Results are within the GEMM
 * tolerance of the separate calls (db sums in the product's order).       */
int nrs_linear_backward(float *dx, float *dw, float *db, const float *grad,
                        const float *x, const float *w, int64_t batch, int64_t in_f,
                        int64_t out_f, float beta_x, float beta_w, float beta_b);

/* nrs_linear_backward of a Linear whose input is the output of a ReLU, with
 * the ReLU's backward (relu_grad, src/cuda/graph/relu.rs:16-28: the gradient
 * passes where the ReLU input is > 0) applied to dx:
 *   dx = (grad . W^T) * (mask > 0) + beta_x * dx
 * mask is the ReLU's input or its output [batch, in_f] (both are > 0 at the
 * same places), so dx is the gradient of the ReLU's INPUT, and the gradient
 * of the ReLU's output is never materialised. dW and db as in
 * nrs_linear_backward. One launch when both products are short (the mask
 * rides the input-gradient product's epilogue); else the products, then one
 * nrs_relu_backward pass. mask may be NULL only when dx is.               */
int nrs_linear_backward_relu(float *dx, float *dw, float *db, const float *grad,
                             const float *x, const float *w, const float *mask,
                             int64_t batch, int64_t in_f, int64_t out_f,
                             float beta_x, float beta_w, float beta_b);

/* The last Linear of a classifier followed by the fused cross-entropy seed:
 * Linear::forward (src/cuda/nn/linear.rs:22-25, matmul + bias add) then
 * cross_entropy_backward (src/cuda/loss/cross_entropy.rs:39-58):
 *   logits = x . W + bias                       [batch, classes]
 *   grad   = (softmax(logits) - target) / batch [batch, classes]
 * with the seed computed as ce_backward computes it (row max folded from
 * class 0, sum of expf(l - max) in class order). bias may be NULL. One launch
 * for at most 16 classes; else nrs_gemm then nrs_cross_entropy_backward.
 * logits, grad and target must not overlap.                               */
int nrs_linear_cross_entropy(float *logits, float *grad, const float *x, const float *w,
                             const float *bias, const float *target, int64_t batch,
                             int64_t in_f, int64_t classes);

/* The two-layer classifier of the reference's MNIST step
 * (examples/mnist_cuda.rs:34-37: relu(add(matmul(x, w1), b1)), then
 * add(matmul(h, w2), b2), then the fused cross-entropy seed of
 * src/cuda/loss/cross_entropy.rs:39-58) through the gradient of its hidden
 * layer, in one launch (everything here is row-local):
 *   h  = relu(x . w1 + b1)               [batch, hidden]
 *   z  = h . w2 + b2                     [batch, classes]  the logits
 *   gz = (softmax(z) - target) / batch   [batch, classes]  ce_backward's seed
 *   dh = (gz . w2^T) where h > 0         [batch, hidden]   relu_grad
 *                                          (src/cuda/graph/relu.rs:23-28)
 * One launch for hidden <= 256, classes <= 16 and in_f <= 4096; any other
 * shape gives the same quantities from three launches (layer 1 with bias and
 * ReLU, nrs_linear_cross_entropy, the masked dh product). b1, b2 may be NULL.
 * No output may overlap an input or another output.                          */
int nrs_mlp2_forward_seed(float *h, float *z, float *gz, float *dh, const float *x,
                          const float *w1, const float *b1, const float *w2, const float *b2,
                          const float *target, int64_t batch, int64_t in_f, int64_t hidden,
                          int64_t classes);
/* Its parameter and input gradients in one launch (both layers' matmul
 * backward closures, src/autograd/graph/matmul.rs:17-63 on the GPU path
 * src/cuda/graph/matmul.rs:386-436, and the bias add's column sums):
 *   dw1 = x^T . dh + beta_p * dw1      db1 = sum_rows(dh) + beta_p * db1
 *   dw2 = h^T . gz + beta_p * dw2      db2 = sum_rows(gz) + beta_p * db2
 *   dx  = dh . w1^T + beta_x * dx      (skipped when dx is NULL)
 * the products nrs_linear_backward runs for each layer, with their bits.
 * db1, db2 may be NULL.                                                      */
int nrs_mlp2_backward(float *dx, float *dw1, float *db1, float *dw2, float *db2,
                      const float *dh, const float *gz, const float *x, const float *w1,
                      const float *h, int64_t batch, int64_t in_f, int64_t hidden,
                      int64_t classes, float beta_x, float beta_p);

/* mm_nt_splitk(a, b, rows, cols, inner) (src/cuda/graph/matmul.rs:354-379):
 * C = A[rows,inner] . B[cols,inner]^T + beta*C for skinny outputs with a huge
 * inner dimension. The inner dimension is split across workgroups; partial
 * tiles go to library scratch and are combined in a fixed slice order, so the
 * result is deterministic (the reference uses float atomicAdd).               */
int nrs_gemm_nt_splitk(float *C, const float *A, const float *B,
                       int64_t rows, int64_t cols, int64_t inner, float beta);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): nrs_gemm_nt_splitk with the same plan, kernels and bits,
 * but its split-K partials go to a fixed 14 MiB per-GPU array compiled into
 * the library (its device address looked up once per device by nrs_init), so
 * the call allocates nothing. A plan whose partials (slices * rows * cols *
 * 4 bytes) exceed 14 MiB is rejected with NRS_ERR_ARG; every plan of the
 * convolution weight-gradient shapes fits (at most 12.7 MB at 64 x 576 over
 * 100352). All calls on one GPU share the array: calls that overlap on one
 * GPU (several streams or threads) race and must be serialised by the caller. */
int nrs_gemm_nt_splitk_noalloc(float *C, const float *A, const float *B,
                               int64_t rows, int64_t cols, int64_t inner, float beta);

/* ------------------------------------------------------------------- bmm */
/* bmm_forward / bmm_grad_a / bmm_grad_b (src/cuda/graph/bmm.rs:12-56), per
 * batch item b with the GEMM layouts above and contiguous items:
 *   NN : C[b] (m x n) = A[b] (m x k) . B[b] (k x n)          -- bmm_forward
 *   NT : C[b] (m x k) = G[b] (m x n) . B[b] (k x n)^T        -- bmm_grad_a
 *   TN : C[b] (k x n) = A[b] (m x k)^T . G[b] (m x n)        -- bmm_grad_b
 * Arguments use GEMM naming: C[b] is rows x cols, reduced over inner.
 * C = A op B + beta*C (beta=1 fuses accumulate_into, bmm.rs:104,118).         */
int nrs_bmm(int layout, float *C, const float *A, const float *B,
            int64_t batch, int64_t rows, int64_t cols, int64_t inner, float beta);

/* The backward closure of graph bmm (src/cuda/graph/bmm.rs:93-131): the two
 * gradients of a forward product per item, with G[b] (m x n) the gradient of
 * its output C[b] (m x n) and A[b] (m x k):
 *   NN (the reference's bmm, B[b] k x n, C = A . B):
 *     dA[b] (m x k) = G . B^T + beta*dA      (bmm_grad_a + accumulate_into)
 *     dB[b] (k x n) = A^T . G + beta*dB      (bmm_grad_b + accumulate_into)
 *   NT (bmm(A, transpose(B)) without the transpose, B[b] n x k, C = A . B^T):
 *     dA[b] (m x k) = G . B + beta*dA,   dB[b] (n x k) = G^T . A + beta*dB
 * Either of dA, dB may be NULL (that gradient is skipped). Items of at most
 * 128 x 128 x 128 compute both gradients in one launch. dA and dB must not
 * overlap each other or A, B, G.                                              */
int nrs_bmm_backward(int layout, float *dA, float *dB, const float *G, const float *A,
                     const float *B, int64_t batch, int64_t m, int64_t k, int64_t n,
                     float beta);

/* ------------------------------------------------- fused attention core */
/* attention_batch (src/cuda/nn/attention.rs:23-32: bmm(q, transpose(k)),
 * scale, softmax, bmm with v) for every head of MultiHeadAttention::
 * forward_batch (src/cuda/nn/multihead.rs:57-85) in one launch, reading and
 * writing the heads in place: q, k, v and out are row-major [batch*seq, ld]
 * with head h in columns [h*d_head, (h+1)*d_head), so the per-head
 * slice_cols / concat_cols copies (multihead.rs:43-52,72-81) disappear; with
 * heads = 1 and ld = d_head it is attention_batch on [batch, seq, d_head].
 *   out = softmax(scale * q . k^T) . v   per (batch item, head);
 *   stats [batch*heads*seq*2] receives, per query row, the softmax in base 2:
 *   max_j u_j and sum_j 2^(u_j - max) with u = scale * log2(e) * q . k^T; the
 *   backward recomputes the probabilities from them (the S x S matrix is
 *   never stored).
 * The fused path takes d_head 16 or 32 and seq up to 16384
 * (nrs_attention_supported): up to 128 one workgroup per (item, head) holds
 * the whole sequence; past it the keys stream through in tiles of 128 with
 * the softmax taken online, so no S x S matrix exists in any form (the
 * stats are the final max and sum of each row). Other shapes are refused
 * with NRS_ERR_ARG and the caller composes bmm / softmax / bmm instead.    */
int nrs_attention_supported(int64_t batch, int64_t heads, int64_t seq, int64_t d_head, int64_t ld);
int nrs_attention_forward(float *out, float *stats, const float *q, const float *k, const float *v,
                          int64_t batch, int64_t heads, int64_t seq, int64_t d_head, int64_t ld,
                          float scale);
/* Its backward (the closures of bmm.rs:93-131, softmax.rs:23-35 and
 * scale.rs:10-20 in the order attention composes them), from the forward's
 * stats: dq = dS . k, dk = dS^T . q, dv = P^T . dout with P recomputed and
 * dS = (P * (dP - rowsum(P * dP))) * scale, dP = dout . v^T; each gradient
 * = computed + beta * old (beta = 1 is accumulate_into). Same layouts as the
 * forward; dq, dk, dv must not overlap each other or the inputs. out is the
 * forward's output, required past seq 128 (rowsum(P * dP) = dout . out per
 * row, so the key tiles need no other tiles' scores) and unused up to it.
 * Past 128, each key tile's dq part goes to library scratch and a second
 * launch adds the parts in key-tile order (deterministic).                 */
int nrs_attention_backward(float *dq, float *dk, float *dv, const float *dout, const float *out,
                           const float *q, const float *k, const float *v, const float *stats,
                           int64_t batch, int64_t heads, int64_t seq, int64_t d_head, int64_t ld,
                           float scale, float beta);

/* ---------------------------------------------------------------- conv2d */
/* The five primitive launches of src/cuda/nn/conv.rs:161-236, same index
 * semantics (columns grouped by sample: col = ni*out_h*out_w + p).           */
int nrs_im2col(float *cols, const float *input, int64_t N, int64_t c_in,
               int64_t in_h, int64_t in_w, int64_t kh, int64_t kw,
               int64_t stride, int64_t pad);                         /* :27-58   */
int nrs_col2out(float *out, const float *mm_out, const float *bias,
                int64_t N, int64_t c_out, int64_t out_h, int64_t out_w); /* :62-76 */
int nrs_out2mm(float *mm_grad, const float *grad,
               int64_t N, int64_t c_out, int64_t out_h, int64_t out_w);  /* :94-108 */
int nrs_col2im(float *dinput, const float *dcols, int64_t N, int64_t c_in,
               int64_t in_h, int64_t in_w, int64_t kh, int64_t kw,
               int64_t stride, int64_t pad, float beta);             /* :113-149 */
int nrs_conv2d_bias_grad(float *dbias, const float *grad, int64_t N, int64_t c_out,
                         int64_t out_h, int64_t out_w, float beta);  /* :78-90   */

/* Whole-op entry points for nn::conv2d (src/cuda/nn/conv.rs:244-328):
 * forward  out[N,c_out,oh,ow] = conv(input, weight) + bias   (im2col + GEMM
 *          whose epilogue writes NCHW + bias, replacing col2out);
 * backward accumulates (+=) into dinput (if non-NULL; the reference skips it
 *          when input.requires_grad is false, :304), dweight and dbias.      */
int nrs_conv2d_forward(float *out, const float *input, const float *weight,
                       const float *bias, int64_t N, int64_t c_in, int64_t in_h,
                       int64_t in_w, int64_t c_out, int64_t kh, int64_t kw,
                       int64_t stride, int64_t pad);
int nrs_conv2d_backward(float *dinput, float *dweight, float *dbias,
                        const float *grad, const float *input, const float *weight,
                        int64_t N, int64_t c_in, int64_t in_h, int64_t in_w,
                        int64_t c_out, int64_t kh, int64_t kw, int64_t stride,
                        int64_t pad);

/* nrs_conv2d_backward with dinput = its gradient + beta_input * dinput: 1 is
 * nrs_conv2d_backward's accumulation (the backward closure's accumulate_into,
 * src/cuda/nn/conv.rs:298-312); 0 writes the gradient without reading dinput
 * (a gradient buffer that was just zeroed needs no zeroing launch). dweight
 * and dbias accumulate as in nrs_conv2d_backward.                          */
int nrs_conv2d_backward_beta(float *dinput, float *dweight, float *dbias,
                             const float *grad, const float *input, const float *weight,
                             int64_t N, int64_t c_in, int64_t in_h, int64_t in_w,
                             int64_t c_out, int64_t kh, int64_t kw, int64_t stride,
                             int64_t pad, float beta_input);
/* nrs_conv2d_backward_beta whose weight and bias gradients are likewise
 * dweight = gradient + beta_params * dweight (and dbias): 1 accumulates as
 * the reference does (conv.rs:314-322 into accumulate_into); 0 writes them
 * without reading the old values, for gradients that were just zeroed
 * (runtime.rs:108-117 zero_grad) and so need no clearing launch. Same
 * kernels and sums as nrs_conv2d_backward; no counterpart in the reference. */
int nrs_conv2d_backward_ex(float *dinput, float *dweight, float *dbias,
                           const float *grad, const float *input, const float *weight,
                           int64_t N, int64_t c_in, int64_t in_h, int64_t in_w,
                           int64_t c_out, int64_t kh, int64_t kw, int64_t stride,
                           int64_t pad, float beta_input, float beta_params);

/* nn::conv2d followed by max pooling (src/cuda/nn/conv.rs:244-277, then
 * src/cuda/nn/maxpool.rs:18-46 on the conv output) in one call: pooled
 * [N, c_out, oh/k', ow/k'] and argmax as nrs_maxpool_forward gives them for
 * the conv output (flat indices into [N, c_out, oh, ow], first maximum wins).
 * out receives the conv output when non-NULL; a CNN whose conv output only
 * feeds the pooling passes NULL and the conv output is never written. One
 * launch for "same" 3x3 stride-1 layers with c_in <= 3, width % 4 == 0, even
 * height and 2x2 stride-2 pooling (the conv values have the bits of
 * nrs_conv2d_forward's); any other shape runs the two ops (the conv output
 * in library scratch when out is NULL).                                     */
int nrs_conv2d_maxpool_forward(float *pooled, int32_t *argmax, float *out, const float *input,
                               const float *weight, const float *bias, int64_t N, int64_t c_in,
                               int64_t in_h, int64_t in_w, int64_t c_out, int64_t kh, int64_t kw,
                               int64_t stride, int64_t pad, int64_t pool_k, int64_t pool_stride);
/* The backward closures of that pair: nrs_conv2d_backward (accumulating
 * dinput, dweight, dbias; any may be NULL) with the conv output's gradient
 * taken as maxpool_backward of grad_pooled into zeros
 * (src/cuda/nn/maxpool.rs:48-66), which is never written when dinput is NULL
 * and the layer has few taps (<= 32 per output channel, 2x2 stride-2
 * pooling, width % 4 == 0): the weight and bias gradients then read the
 * pooled gradient and argmax and expand them while loading, one launch plus
 * the slice sum. Otherwise the unpooled gradient goes through library
 * scratch and the two backward calls.                                       */
int nrs_maxpool_conv2d_backward(float *dinput, float *dweight, float *dbias,
                                const float *grad_pooled, const int32_t *argmax,
                                const float *input, const float *weight, int64_t N, int64_t c_in,
                                int64_t in_h, int64_t in_w, int64_t c_out, int64_t kh, int64_t kw,
                                int64_t stride, int64_t pad, int64_t pool_k, int64_t pool_stride);

/* The same two calls with a ReLU between the conv and the pooling, the
 * reference CNN's maxpool2d(relu(conv2d(..)), 2, 2)
 * (examples/mnist_cuda_cnn.rs:125,127; src/cuda/graph/relu.rs:16-28 between
 * conv.rs:244-277 and maxpool.rs:18-46): pooled and argmax are the pooling of
 * relu(conv output), first maximum wins (windows of zeros keep their first
 * element); out, when non-NULL, receives the conv output before the ReLU.
 * The backward's relu_grad test (conv value > 0) is taken from the pooled
 * value at each window's argmax, which is that conv value's ReLU: pass the
 * forward's pooled output. Same single-launch shapes as above. dinput
 * accumulates; dweight and dbias take beta_params as nrs_conv2d_backward_ex
 * does (1 accumulates).                                                     */
int nrs_conv2d_relu_maxpool_forward(float *pooled, int32_t *argmax, float *out,
                                    const float *input, const float *weight, const float *bias,
                                    int64_t N, int64_t c_in, int64_t in_h, int64_t in_w,
                                    int64_t c_out, int64_t kh, int64_t kw, int64_t stride,
                                    int64_t pad, int64_t pool_k, int64_t pool_stride);
int nrs_maxpool_relu_conv2d_backward(float *dinput, float *dweight, float *dbias,
                                     const float *grad_pooled, const int32_t *argmax,
                                     const float *pooled, const float *input, const float *weight,
                                     int64_t N, int64_t c_in, int64_t in_h, int64_t in_w,
                                     int64_t c_out, int64_t kh, int64_t kw, int64_t stride,
                                     int64_t pad, int64_t pool_k, int64_t pool_stride,
                                     float beta_params);

/* The backward of a conv layer over that pooled output, with the lower
 * pair's parameter gradients: the reference CNN's
 * conv2d(maxpool2d(relu(conv2d(x)))) (examples/mnist_cuda_cnn.rs:123-138)
 * from the upper layer's output gradient down, when the lower layer's input
 * needs no gradient (mnist_cuda_cnn.rs:261). Equals
 *   nrs_conv2d_backward_ex(dpooled, dweight, dbias, grad, pooled, weight,
 *       N, c_mid, ph, pw, c_out, kh, kw, stride, pad, 0, beta_params);
 *   nrs_maxpool_relu_conv2d_backward(NULL, dweight_lo, dbias_lo, dpooled,
 *       argmax, pooled, input_lo, weight_lo, N, c_in_lo, in_h, in_w, c_mid,
 *       kh_lo, kw_lo, stride_lo, pad_lo, pool_k, pool_stride, beta_params);
 * (ph x pw the pooled size): dpooled is written (not added); the four
 * parameter gradients take beta_params. One launch plus one for both
 * weight-gradient sums when the upper layer is "same" 3x3 stride 1 over
 * pooled images of at most 14x14 (even width >= 4, whole pixel quads),
 * c_mid % 32 == 0 and c_out % 64 == 0, and the lower layer is "same" 3x3
 * stride 1 with 1 or 2 input channels under 2x2 stride-2 pooling of an even
 * image; the lower weight gradient then sums over each window's argmax
 * pixel in another order (the same values up to rounding; exact on
 * small-integer data). Any other shape runs the two calls. weight_lo is
 * read only by that path.                                                    */
int nrs_conv2d_maxpool_relu_conv2d_backward(
    float *dpooled, float *dweight, float *dbias, float *dweight_lo, float *dbias_lo,
    const float *grad, const float *pooled, const float *weight, const int32_t *argmax,
    const float *input_lo, const float *weight_lo, int64_t N, int64_t c_in_lo, int64_t in_h,
    int64_t in_w, int64_t c_mid, int64_t kh_lo, int64_t kw_lo, int64_t stride_lo,
    int64_t pad_lo, int64_t pool_k, int64_t pool_stride, int64_t c_out, int64_t kh, int64_t kw,
    int64_t stride, int64_t pad, float beta_params);

/* ------------------------------------------------------ gradient plumbing */
/* accumulate (src/cuda/runtime.rs:13-19): acc[i] += src[i].                  */
int nrs_accumulate(float *acc, const float *src, int64_t n);
/* vadd / bias_add (src/cuda/graph/add.rs:18-31).                             */
int nrs_vadd(float *out, const float *a, const float *b, int64_t n);
int nrs_bias_add(float *out, const float *a, const float *bias, int64_t rows, int64_t cols);
/* sum_axis0 (src/cuda/reduce.rs:12-21): out[c] = sum_r in[r,c] (+ beta*out). */
int nrs_sum_axis0(float *out, const float *in, int64_t rows, int64_t cols, float beta);

/* maxpool_forward / maxpool_backward (src/cuda/nn/maxpool.rs:18-52), the glue
 * between the two convolutions of the CNN workload. Forward records the flat
 * input index of the first maximum (strict >). Backward adds grad to the
 * winners: dinput += scatter(grad, argmax); done as a gather over the windows
 * that cover each input element, so it needs no atomics and is deterministic
 * (the reference scatters with atomicAdd).                                    */
int nrs_maxpool_forward(float *out, int32_t *argmax, const float *input, int64_t N,
                        int64_t C, int64_t in_h, int64_t in_w, int64_t k, int64_t stride);
int nrs_maxpool_backward(float *dinput, const float *grad, const int32_t *argmax,
                         int64_t N, int64_t C, int64_t in_h, int64_t in_w, int64_t k,
                         int64_t stride);


/* ------------------------------------------------------- attention / MLP glue */
/* transpose2d (src/cuda/graph/transpose.rs:10-24): out[b,j,i] = in[b,i,j] for
 * `batch` row-major rows x cols matrices; out must not alias in.             */
int nrs_transpose(float *out, const float *in, int64_t batch, int64_t rows, int64_t cols);
/* vscale / scale_grad (src/cuda/graph/scale.rs:10-20): out = x*s + beta*out. */
int nrs_scale(float *out, const float *x, float s, int64_t n, float beta);
/* softmax_forward (src/cuda/graph/softmax.rs:11-22): softmax over the last
 * dim of rows x width, max-subtracted.                                       */
int nrs_softmax_forward(float *out, const float *in, int64_t rows, int64_t width);
/* Cross-entropy of raw logits [batch, classes] against a one-hot target of
 * the same shape (src/cuda/loss/cross_entropy.rs:18-36, ce_forward): row_loss
 * [batch] gets sum_c -t*(l - logsumexp(l)) per row; the batch mean is the
 * caller's host-side sum / batch (cross_entropy.rs:74-88).                  */
int nrs_cross_entropy_forward(float *row_loss, const float *logits, const float *target,
                              int64_t batch, int64_t classes);
/* The fused seed of cross_entropy_backward (cross_entropy.rs:39-58,100-127):
 * grad = (softmax(logits) - target) / batch, written (not accumulated).     */
int nrs_cross_entropy_backward(float *grad, const float *logits, const float *target,
                               int64_t batch, int64_t classes);
/* softmax_backward (src/cuda/graph/softmax.rs:23-35), from the forward output
 * y: gin = y*(grad - sum(y*grad)) + beta*gin.                                */
int nrs_softmax_backward(float *gin, const float *y, const float *grad, int64_t rows,
                         int64_t width, float beta);
/* graph::scale then graph::softmax in one pass, the scaled-scores step of
 * attention and attention_batch (src/cuda/nn/attention.rs:17-18,29-30;
 * scale.rs:27, softmax.rs:43): out = softmax(scale*x) over the last dim. The
 * product x*scale is rounded to f32 first, so the bits equal nrs_scale
 * followed by nrs_softmax_forward.                                           */
int nrs_softmax_forward_scaled(float *out, const float *in, int64_t rows, int64_t width,
                               float scale);
/* The backward of that pair in one pass: softmax_backward followed by
 * scale_grad, gin = (y*(grad - sum(y*grad)))*scale + beta*gin. With beta 0
 * the bits equal nrs_softmax_backward followed by nrs_scale.                 */
int nrs_softmax_backward_scaled(float *gin, const float *y, const float *grad, int64_t rows,
                                int64_t width, float scale, float beta);
/* slice_fwd (src/cuda/graph/slice_cols.rs:12-20): out[r][c] = in[r][col_start
 * + c] for r < rows, c < width, in having total_cols columns.                */
int nrs_slice_cols(float *out, const float *in, int64_t rows, int64_t total_cols,
                   int64_t col_start, int64_t width);
/* slice_bwd + accumulate_into (slice_cols.rs:21-29,66-80): gin[r][col_start +
 * c] = grad[r][c] + beta*gin[r][col_start + c]; gin's other columns are left
 * as they are (the reference adds zeros there). beta = 1 is the reference.   */
int nrs_slice_cols_backward(float *gin, const float *grad, int64_t rows, int64_t total_cols,
                            int64_t col_start, int64_t width, float beta);
/* concat_write (src/cuda/graph/concat_cols.rs:12-20), one part:
 * out[r][col_offset + c] = part[r][c].                                       */
int nrs_concat_cols(float *out, const float *part, int64_t rows, int64_t total_cols,
                    int64_t col_offset, int64_t width);
/* concat_read + accumulate_into (concat_cols.rs:21-29 and its backward
 * closure): gpart[r][c] = grad[r][col_offset + c] + beta*gpart[r][c].        */
int nrs_concat_cols_backward(float *gpart, const float *grad, int64_t rows, int64_t total_cols,
                             int64_t col_offset, int64_t width, float beta);
/* The per-head slice_cols loop of MultiHeadAttention (src/cuda/nn/
 * multihead.rs:43-49,72-78) in one launch: out[h][r][c] = in[r][h*width + c]
 * + beta*out[h][r][c], for heads x rows x width. The heads' rows are then one
 * batched bmm of heads*batch items. beta = 1 is merge_heads' backward.       */
int nrs_split_heads(float *out, const float *in, int64_t rows, int64_t heads, int64_t width,
                    float beta);
/* Its inverse, the heads' concat_cols (multihead.rs:52,81): out[r][h*width +
 * c] = in[h][r][c] + beta*out[r][h*width + c]. beta = 1 is split_heads'
 * backward.                                                                  */
int nrs_merge_heads(float *out, const float *in, int64_t rows, int64_t heads, int64_t width,
                    float beta);
/* cuda::nn::layernorm forward (src/cuda/nn/normalization.rs:14-40 ln_forward,
 * 87-120), used by TransformerBlock: per row of `features`, mean, biased var,
 * inv_std = 1/sqrt(var + eps), x_norm = (x - mean)*inv_std, out = gamma*x_norm
 * + beta. x_norm [rows*features] and inv_std [rows] are saved for backward.  */
int nrs_layernorm_forward(float *out, float *x_norm, float *inv_std, const float *in,
                          const float *gamma, const float *beta, int64_t rows, int64_t features,
                          float eps);
/* The same LayerNorm of in + in2, the residual add before each norm of
 * TransformerBlock::forward (src/cuda/nn/transformer_block.rs:32-33, 41-42: add then
 * norm) in one pass: the sum is rounded to f32 as the add computes it and is
 * not written out. in2 may be NULL (nrs_layernorm_forward).                  */
int nrs_add_layernorm_forward(float *out, float *x_norm, float *inv_std, const float *in,
                              const float *in2, const float *gamma, const float *beta,
                              int64_t rows, int64_t features, float eps);
/* Its backward (ln_dx, ln_reduce and accumulate_into, normalization.rs:41-80,
 * 133-160): dxh = grad*gamma; dinput = inv_std*(dxh - mean(dxh) - x_norm*
 * mean(dxh*x_norm)); dgamma = sum over rows of grad*x_norm; dbeta = sum of
 * grad; each + acc*old (acc = 1 is the reference's accumulate). Null outputs
 * are skipped.                                                               */
int nrs_layernorm_backward(float *dinput, float *dgamma, float *dbeta, const float *grad,
                           const float *gamma, const float *x_norm, const float *inv_std,
                           int64_t rows, int64_t features, float acc);
/* The backward of norm(a + b) (transformer_block.rs:32-33, 41-42; the add's
 * backward, src/cuda/graph/add.rs:41-110, hands the input gradient to both a
 * and b): the input gradient of nrs_layernorm_backward stored to da (+ beta_a
 * * old) and, when db is not NULL, to db (+ beta_b * old) in the same pass;
 * the parameter gradients take beta_params. db needs da.                     */
int nrs_add_layernorm_backward(float *da, float *db, float *dgamma, float *dbeta,
                               const float *grad, const float *gamma, const float *x_norm,
                               const float *inv_std, int64_t rows, int64_t features, float beta_a,
                               float beta_b, float beta_params);
/* vrelu / relu_grad (src/cuda/graph/relu.rs:16-28): out = max(x, 0);
 * gin = (x > 0 ? grad : 0) + beta*gin.                                       */
int nrs_relu_forward(float *out, const float *x, int64_t n);
int nrs_relu_backward(float *gin, const float *grad, const float *x, int64_t n, float beta);

#ifdef __cplusplus
}
#endif

#endif /* NRS_HIP_H */
