// Fused scaled-dot-product attention over all heads, forward and backward:
// the attention_batch of src/cuda/nn/attention.rs:23-32 (bmm Q.K^T, scale,
// softmax, bmm P.V) run for every head of MultiHeadAttention::forward_batch
// (src/cuda/nn/multihead.rs:57-85) in one launch, with the heads read and
// written in place in the projections' [batch*seq, ld] rows (no slice_cols /
// concat_cols copies) and the S x S scores never leaving the chip.
//
// One workgroup owns one (batch item, head) and eight waves; wave w owns the
// 16 queries 16w..16w+15 (and in the backward also the keys 16w..16w+15).
// Products run on v_mfma_f32_16x16x4f32. Lane l = 16g + c (c = l % 16,
// g = l / 16) holds, in a 16x16 accumulator, rows 4g..4g+3 of column c.
//  * Scores are computed transposed, S^T[key][query] = K . Q^T, so a lane
//    holds 32 scores of ONE query (keys kb*16 + 4g + r): the row max and sum
//    of the softmax are lane-local plus two cross-lane steps.
//  * Those registers are directly the A operand of P.V (A[i][k] = P[query
//    c][key of group g]), so P never goes through memory.
//  * The reduction dim of Q.K^T is split so lane group g takes d = DG*g ..
//    DG*g + DG - 1: Q rows load as 128-bit fragments, K rows read from LDS
//    as 128-bit fragments.
//  * V (and in the backward K, Q, dO) is kept transposed in LDS, so the
//    B operand of a product over keys (or queries) is one 128-bit LDS read
//    per four MFMAs.
// The softmax runs in base 2: u = score * (scale * log2 e), P = 2^(u - max u)
// / sum, the exponential being one v_exp_f32 and the normalisation one
// reciprocal per row (the libm expf and an IEEE division per element cost as
// much as the matrix products). The statistics (max u, sum) are saved by the
// forward; the backward recomputes P from them bit for bit (same products,
// same order) instead of storing the 16.8 MB score matrix of the cfg4 block.
#include "buffer_ops.hpp"

namespace nrs {
namespace {

constexpr int kAttnSeq = 128;  // longest sequence of the fused path
constexpr int kAttnThreads = 512;
constexpr int kAttnTP = kAttnSeq + 4;  // pitch of the transposed LDS tiles ([d][seq])

struct AttnArgs {
    const float* q;
    const float* k;
    const float* v;
    const float* dout;  // backward: gradient of the output
    float* out;         // forward: output; unused by the backward
    float* stats;       // [items][seq][2]: row max and row sum of exp (read by the backward)
    float* dq;
    float* dk;
    float* dv;
    int S, H, ld;  // sequence length, heads, row stride of q/k/v/out (floats)
    float scale;   // the attention scale (the gradient of the scores carries it)
    float scale2;  // scale * log2(e): scores to base-2 exponents
    float beta;  // backward: gradients = computed + beta * old
};

__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Element offset of (row, col) of this item's head in a [batch*seq, ld] tensor.
__device__ __forceinline__ int64_t item_base(const AttnArgs& a, int item, int D) {
    const int b = item / a.H, h = item - b * a.H;
    return (int64_t)b * a.S * a.ld + (int64_t)h * D;
}

// S^T (scores transposed, 8 blocks of 16 keys x 16 queries) from K in LDS and
// the lane's Q fragment; lane (c, g) gets keys kb*16 + 4g + r of query c.
// The next block's LDS fragments are read before the current block's MFMAs.
template <int D>
__device__ __forceinline__ void scores_t(f32x4 (&acc)[8], const float* k_lds,
                                         const f32x4 (&qf)[D / 16], int c, int g) {
    constexpr int DG = D / 4, KP = D + 4, NF = D / 16;
    const float* kr = k_lds + c * KP + DG * g;
    f32x4 kf[2][NF];
#pragma unroll
    for (int i = 0; i < NF; ++i) kf[0][i] = *reinterpret_cast<const f32x4*>(kr + 4 * i);
#pragma unroll
    for (int kb = 0; kb < 8; ++kb) {
        if (kb + 1 < 8) {
#pragma unroll
            for (int i = 0; i < NF; ++i)
                kf[(kb + 1) & 1][i] =
                    *reinterpret_cast<const f32x4*>(kr + (kb + 1) * 16 * KP + 4 * i);
        }
        acc[kb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < NF; ++i)
#pragma unroll
            for (int p = 0; p < 4; ++p) acc[kb] = mfma16(kf[kb & 1][i][p], qf[i][p], acc[kb]);
    }
}

// Stages rows [0, S) of this item's head of `src` (zero past S): row-major
// [key][D + 4] into `rows` (may be null) and transposed [d][kAttnTP] into
// `cols` (may be null). `vals` holds the thread's loaded 128-bit units.
template <int D>
__device__ __forceinline__ void stage_load(f32x4 (&vals)[kAttnSeq * D / 4 / kAttnThreads],
                                           __amdgpu_buffer_rsrc_t rs, const AttnArgs& a) {
    constexpr int U = kAttnSeq * D / 4 / kAttnThreads;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int idx = threadIdx.x + kAttnThreads * u;
        const int row = idx / (D / 4), d4 = idx - row * (D / 4);
        vals[u] = buffer_load4(rs, row < a.S ? (row * a.ld + 4 * d4) * 4 : kOutOfRange);
    }
}

template <int D>
__device__ __forceinline__ void stage_store(const f32x4 (&vals)[kAttnSeq * D / 4 / kAttnThreads],
                                            float* rows, float* cols) {
    constexpr int U = kAttnSeq * D / 4 / kAttnThreads, KP = D + 4;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int idx = threadIdx.x + kAttnThreads * u;
        const int row = idx / (D / 4), d4 = idx - row * (D / 4);
        if (rows) *reinterpret_cast<f32x4*>(rows + row * KP + 4 * d4) = vals[u];
        if (cols) {
#pragma unroll
            for (int i = 0; i < 4; ++i) cols[(4 * d4 + i) * kAttnTP + row] = vals[u][i];
        }
    }
}

// The lane's 128-bit fragments of row `row` of a head: d = DG*g .. DG*g + DG - 1.
template <int D>
__device__ __forceinline__ void row_fragment(f32x4 (&f)[D / 16], __amdgpu_buffer_rsrc_t rs,
                                             const AttnArgs& a, int row, int g) {
    constexpr int DG = D / 4;
#pragma unroll
    for (int i = 0; i < D / 16; ++i)
        f[i] = buffer_load4(rs, row < a.S ? (row * a.ld + DG * g + 4 * i) * 4 : kOutOfRange);
}

template <int D>
__global__ __launch_bounds__(kAttnThreads) void attn_fwd_kernel(AttnArgs a) {
    // t = score * scale is rounded before the max subtraction, as graph::scale
    // followed by softmax computes it
#pragma clang fp contract(off)
    constexpr int KP = D + 4, NJ = D / 16;
    __shared__ float k_lds[kAttnSeq * KP];
    __shared__ float vt_lds[D * kAttnTP];
    const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int item = blockIdx.x, S = a.S;
    const int64_t base = item_base(a, item, D);
    const int64_t ext = ((int64_t)(S - 1) * a.ld + D) * 4;
    const auto rq = buffer_rsrc(a.q + base, ext), rk = buffer_rsrc(a.k + base, ext),
               rv = buffer_rsrc(a.v + base, ext);
    // one barrier: after it each wave runs scores, softmax and P.V on its
    // own, so the two waves of a SIMD overlap one's softmax with the other's
    // MFMAs (a second barrier before P.V would line them up again)
    f32x4 kv[kAttnSeq * D / 4 / kAttnThreads], vv[kAttnSeq * D / 4 / kAttnThreads], qf[NJ];
    const int qrow = 16 * w + c;
    row_fragment<D>(qf, rq, a, qrow, g);
    stage_load<D>(kv, rk, a);
    stage_load<D>(vv, rv, a);
    stage_store<D>(kv, k_lds, nullptr);
    stage_store<D>(vv, nullptr, vt_lds);
    __syncthreads();

    f32x4 p[8];
    scores_t<D>(p, k_lds, qf, c, g);
    float m = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float u = kb * 16 + 4 * g + r < S ? p[kb][r] * a.scale2 : -INFINITY;
            p[kb][r] = u;
            m = fmaxf(m, u);
        }
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    float sum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float e = __builtin_amdgcn_exp2f(p[kb][r] - m);  // 2^-inf = 0 for masked keys
            p[kb][r] = e;
            sum += e;
        }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    const float rs = 1.0f / sum;
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) p[kb][r] = p[kb][r] * rs;

    // O = P . V: A = P (registers), B = V^T from LDS, four keys per read,
    // the next block's read issued before the current block's MFMAs
    f32x4 o[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) o[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const float* vr = vt_lds + c * kAttnTP + 4 * g;
    f32x4 vf[2][NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) vf[0][j] = *reinterpret_cast<const f32x4*>(vr + j * 16 * kAttnTP);
#pragma unroll
    for (int kb = 0; kb < 8; ++kb) {
        if (kb + 1 < 8) {
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                vf[(kb + 1) & 1][j] =
                    *reinterpret_cast<const f32x4*>(vr + j * 16 * kAttnTP + (kb + 1) * 16);
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[j] = mfma16(p[kb][r], vf[kb & 1][j][r], o[j]);
    }
    float* out = a.out + base;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * w + 4 * g + r;
            if (row < S) __builtin_nontemporal_store(o[j][r], out + (int64_t)row * a.ld + j * 16 + c);
        }
    // last: vmcnt counts stores, so a store issued earlier would hold up the
    // waits for V
    if (g == 0 && qrow < S) {
        float* st = a.stats + ((int64_t)item * S + qrow) * 2;
        st[0] = m;
        st[1] = sum;
    }
}

// Gradient stores of a 16-row block: lane holds rows 16*blk + 4g + r, columns
// j*16 + c; dst = v + beta * dst (the old values were loaded beforehand).
template <int D>
__device__ __forceinline__ void load_old(f32x4 (&old)[D / 16], const float* dst, const AttnArgs& a,
                                         int blk, int c, int g) {
#pragma unroll
    for (int j = 0; j < D / 16; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * blk + 4 * g + r;
            old[j][r] = row < a.S ? dst[(int64_t)row * a.ld + j * 16 + c] : 0.0f;
        }
}

template <int D>
__device__ __forceinline__ void store_grad(float* dst, const f32x4 (&v)[D / 16],
                                           const f32x4 (&old)[D / 16], const AttnArgs& a, int blk,
                                           int c, int g) {
#pragma unroll
    for (int j = 0; j < D / 16; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * blk + 4 * g + r;
            const float x = a.beta != 0.0f ? v[j][r] + a.beta * old[j][r] : v[j][r];
            if (row < a.S) dst[(int64_t)row * a.ld + j * 16 + c] = x;
        }
}

// out[key or query block][d] = sum over the 128 columns of x_lds rows (16
// rows from `row0`) times the transposed operand `t_lds` ([d][seq]).
template <int D>
__device__ __forceinline__ void rows_times_t(f32x4 (&o)[D / 16], const float* x_lds,
                                             const float* t_lds, int row0, int c, int g) {
#pragma unroll
    for (int j = 0; j < D / 16; ++j) o[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int qc = 0; qc < 8; ++qc) {
        const f32x4 xf =
            *reinterpret_cast<const f32x4*>(x_lds + (row0 + c) * kAttnTP + qc * 16 + 4 * g);
#pragma unroll
        for (int j = 0; j < D / 16; ++j) {
            const f32x4 tf =
                *reinterpret_cast<const f32x4*>(t_lds + (j * 16 + c) * kAttnTP + qc * 16 + 4 * g);
#pragma unroll
            for (int r = 0; r < 4; ++r) o[j] = mfma16(xf[r], tf[r], o[j]);
        }
    }
}

template <int D>
__global__ __launch_bounds__(kAttnThreads) void attn_bwd_kernel(AttnArgs a) {
#pragma clang fp contract(off)
    constexpr int KP = D + 4, NJ = D / 16, U = kAttnSeq * D / 4 / kAttnThreads;
    __shared__ float k_lds[kAttnSeq * KP];     // K  [key][d]   (S^T recompute)
    __shared__ float v_lds[kAttnSeq * KP];     // V  [key][d]   (dP^T)
    __shared__ float kt_lds[D * kAttnTP];      // K^T [d][key]  (dQ)
    __shared__ float qt_lds[D * kAttnTP];      // Q^T [d][query] (dK)
    __shared__ float dot_lds[D * kAttnTP];     // dO^T [d][query] (dV)
    __shared__ float x_lds[kAttnSeq * kAttnTP];  // P^T, then dS^T [key][query]
    const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int item = blockIdx.x, S = a.S;
    const int64_t base = item_base(a, item, D);
    const int64_t ext = ((int64_t)(S - 1) * a.ld + D) * 4;
    const auto rq = buffer_rsrc(a.q + base, ext), rk = buffer_rsrc(a.k + base, ext),
               rv = buffer_rsrc(a.v + base, ext), rdo = buffer_rsrc(a.dout + base, ext);
    {
        f32x4 kv[U], vv[U], qv[U], dv[U];
        stage_load<D>(kv, rk, a);
        stage_load<D>(vv, rv, a);
        stage_load<D>(qv, rq, a);
        stage_load<D>(dv, rdo, a);
        stage_store<D>(kv, k_lds, kt_lds);
        stage_store<D>(vv, v_lds, nullptr);
        stage_store<D>(qv, nullptr, qt_lds);
        stage_store<D>(dv, nullptr, dot_lds);
    }
    const int qrow = 16 * w + c;
    f32x4 qf[NJ], df[NJ];
    row_fragment<D>(qf, rq, a, qrow, g);
    row_fragment<D>(df, rdo, a, qrow, g);
    float m = 0.0f, sum = 1.0f;
    if (qrow < S) {
        const float* st = a.stats + ((int64_t)item * S + qrow) * 2;
        m = st[0];
        sum = st[1];
    }
    const float rs = 1.0f / sum;
    f32x4 old_q[NJ], old_k[NJ], old_v[NJ];
    if (a.beta != 0.0f) {
        load_old<D>(old_q, a.dq + base, a, w, c, g);
        load_old<D>(old_k, a.dk + base, a, w, c, g);
        load_old<D>(old_v, a.dv + base, a, w, c, g);
    }
    __syncthreads();

    // P, recomputed exactly as the forward computed it
    f32x4 p[8];
    scores_t<D>(p, k_lds, qf, c, g);
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool live = kb * 16 + 4 * g + r < S && qrow < S;
            p[kb][r] = live ? __builtin_amdgcn_exp2f(p[kb][r] * a.scale2 - m) * rs : 0.0f;
        }
    // dP^T = V . dO^T, in the layout of P
    f32x4 ds[8];
    scores_t<D>(ds, v_lds, df, c, g);
    // softmax backward, then the scale: dS = (P * (dP - sum(P * dP))) * scale
    float dot = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) dot += p[kb][r] * ds[kb][r];
    dot += __shfl_xor(dot, 16, 64);
    dot += __shfl_xor(dot, 32, 64);
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) ds[kb][r] = (p[kb][r] * (ds[kb][r] - dot)) * a.scale;

    // dQ = dS . K (A = dS registers, B = K^T from LDS)
    {
        f32x4 o[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) o[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb < 8; ++kb)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const f32x4 kf = *reinterpret_cast<const f32x4*>(kt_lds + (j * 16 + c) * kAttnTP +
                                                                 kb * 16 + 4 * g);
#pragma unroll
                for (int r = 0; r < 4; ++r) o[j] = mfma16(ds[kb][r], kf[r], o[j]);
            }
        store_grad<D>(a.dq + base, o, old_q, a, w, c, g);
    }
    // P^T to LDS for dV = P^T . dO
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) x_lds[(kb * 16 + 4 * g + r) * kAttnTP + qrow] = p[kb][r];
    __syncthreads();
    {
        f32x4 o[NJ];
        rows_times_t<D>(o, x_lds, dot_lds, 16 * w, c, g);
        store_grad<D>(a.dv + base, o, old_v, a, w, c, g);
    }
    __syncthreads();
    // dS^T to LDS for dK = dS^T . Q
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) x_lds[(kb * 16 + 4 * g + r) * kAttnTP + qrow] = ds[kb][r];
    __syncthreads();
    {
        f32x4 o[NJ];
        rows_times_t<D>(o, x_lds, qt_lds, 16 * w, c, g);
        store_grad<D>(a.dk + base, o, old_k, a, w, c, g);
    }
}

bool attn_shape_ok(int64_t batch, int64_t heads, int64_t seq, int64_t d_head, int64_t ld) {
    return batch >= 0 && heads >= 1 && seq >= 1 && seq <= kAttnSeq && (d_head == 16 || d_head == 32) &&
           ld >= heads * d_head && ld <= (1 << 20) && batch * heads <= INT32_MAX;
}

int attn_check(const char* what, int64_t batch, int64_t heads, int64_t seq, int64_t d_head,
               int64_t ld) {
    NRS_ARG_CHECK(attn_shape_ok(batch, heads, seq, d_head, ld),
                  "%s: unsupported shape (batch %lld, heads %lld, seq %lld, d_head %lld, ld %lld): "
                  "the fused path takes seq <= %d, d_head 16 or 32, ld >= heads * d_head",
                  what, (long long)batch, (long long)heads, (long long)seq, (long long)d_head,
                  (long long)ld, kAttnSeq);
    return NRS_OK;
}

}  // namespace
}  // namespace nrs

extern "C" {

int nrs_attention_supported(int64_t batch, int64_t heads, int64_t seq, int64_t d_head, int64_t ld) {
    return nrs::attn_shape_ok(batch, heads, seq, d_head, ld) ? 1 : 0;
}

int nrs_attention_forward(float* out, float* stats, const float* q, const float* k, const float* v,
                          int64_t batch, int64_t heads, int64_t seq, int64_t d_head, int64_t ld,
                          float scale) {
    NRS_REQUIRE_INIT();
    if (int rc = nrs::attn_check("attention forward", batch, heads, seq, d_head, ld)) return rc;
    if (batch == 0) return NRS_OK;
    NRS_ARG_CHECK(out && stats && q && k && v, "attention forward: null pointer");
    nrs::AttnArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.stats = stats;
    a.S = (int)seq;
    a.H = (int)heads;
    a.ld = (int)ld;
    a.scale = scale;
    a.scale2 = scale * 1.4426950408889634f;
    const dim3 grid((unsigned)(batch * heads));
    if (d_head == 16)
        hipLaunchKernelGGL(nrs::attn_fwd_kernel<16>, grid, dim3(nrs::kAttnThreads), 0,
                           nrs::stream(), a);
    else
        hipLaunchKernelGGL(nrs::attn_fwd_kernel<32>, grid, dim3(nrs::kAttnThreads), 0,
                           nrs::stream(), a);
    NRS_LAUNCH_CHECK("attention forward");
    return NRS_OK;
}

int nrs_attention_backward(float* dq, float* dk, float* dv, const float* dout, const float* q,
                           const float* k, const float* v, const float* stats, int64_t batch,
                           int64_t heads, int64_t seq, int64_t d_head, int64_t ld, float scale,
                           float beta) {
    NRS_REQUIRE_INIT();
    if (int rc = nrs::attn_check("attention backward", batch, heads, seq, d_head, ld)) return rc;
    if (batch == 0) return NRS_OK;
    NRS_ARG_CHECK(dq && dk && dv && dout && q && k && v && stats,
                  "attention backward: null pointer");
    nrs::AttnArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.dout = dout;
    a.stats = const_cast<float*>(stats);  // only read by the backward
    a.dq = dq;
    a.dk = dk;
    a.dv = dv;
    a.S = (int)seq;
    a.H = (int)heads;
    a.ld = (int)ld;
    a.scale = scale;
    a.scale2 = scale * 1.4426950408889634f;  // as the forward computed it
    a.beta = beta;
    const dim3 grid((unsigned)(batch * heads));
    if (d_head == 16)
        hipLaunchKernelGGL(nrs::attn_bwd_kernel<16>, grid, dim3(nrs::kAttnThreads), 0,
                           nrs::stream(), a);
    else
        hipLaunchKernelGGL(nrs::attn_bwd_kernel<32>, grid, dim3(nrs::kAttnThreads), 0,
                           nrs::stream(), a);
    NRS_LAUNCH_CHECK("attention backward");
    return NRS_OK;
}

}  // extern "C"
