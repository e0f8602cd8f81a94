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
//  * K, V, Q and dO sit row-major in LDS ([row][D + 4], staged with 128-bit
//    stores); the B operand of a product over keys (or queries) is four rows
//    of one column, two conflict-free ds_read2_b32 per four MFMAs.
// The softmax runs in base 2: the query fragments are multiplied by
// scale * log2(e) once, so the scores come out as exponents u, and
// P = 2^(u - max u) / sum, the exponential being one v_exp_f32 (the libm expf
// and an IEEE division per element cost as much as the matrix products). The
// forward exponentiates each key block just before its P.V MFMAs, so that
// VALU work overlaps the matrix core, and divides the 16 or 32 outputs of a
// row by the sum instead of its 128 probabilities. Its keys are staged in two
// halves: Q.K^T of the first half runs while the second half and V arrive.
// The statistics (max u, sum) are saved by the forward; the backward
// recomputes the same exponents (same products, same order) instead of
// storing the 16.8 MB score matrix of the cfg4 block.
#include "buffer_ops.hpp"

namespace nrs {
namespace {

constexpr int kAttnSeq = 128;  // longest sequence of the fused path
constexpr int kAttnThreads = 512;
constexpr int kAttnTP = kAttnSeq + 4;  // pitch of the [key][query] score tile in LDS

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

// 128-bit units one thread stages of a [kAttnSeq][D] head tile; unit u holds
// rows [u * kAttnSeq / U, (u + 1) * kAttnSeq / U).
template <int D>
constexpr int stage_units() {
    return kAttnSeq * D / 4 / kAttnThreads;
}

// Loads rows [0, S) of this item's head of a tensor (zero past S).
template <int D>
__device__ __forceinline__ void stage_load(f32x4 (&vals)[stage_units<D>()],
                                           __amdgpu_buffer_rsrc_t rs, int ld, int S) {
#pragma unroll
    for (int u = 0; u < stage_units<D>(); ++u) {
        const int idx = threadIdx.x + kAttnThreads * u;
        const int row = idx / (D / 4), d4 = idx - row * (D / 4);
        vals[u] = buffer_load4(rs, row < S ? (row * ld + 4 * d4) * 4 : kOutOfRange);
    }
}

// Stores unit u of `vals` into a row-major [kAttnSeq][D + 4] LDS tile.
template <int D>
__device__ __forceinline__ void stage_store(const f32x4 (&vals)[stage_units<D>()], int u,
                                            float* lds) {
    const int idx = threadIdx.x + kAttnThreads * u;
    const int row = idx / (D / 4), d4 = idx - row * (D / 4);
    *reinterpret_cast<f32x4*>(lds + row * (D + 4) + 4 * d4) = vals[u];
}

// The lane's 128-bit fragments of row `row` of a head (global memory):
// d = D/4*g .. D/4*g + D/4 - 1.
template <int D>
__device__ __forceinline__ void row_fragment(f32x4 (&f)[D / 16], __amdgpu_buffer_rsrc_t rs, int ld,
                                             int row, int S, int g) {
    constexpr int DG = D / 4;
#pragma unroll
    for (int i = 0; i < D / 16; ++i)
        f[i] = buffer_load4(rs, row < S ? (row * ld + DG * g + 4 * i) * 4 : kOutOfRange);
}

// The same fragments from a row-major LDS tile.
template <int D>
__device__ __forceinline__ void lds_row_fragment(f32x4 (&f)[D / 16], const float* lds, int row,
                                                 int g) {
    constexpr int DG = D / 4, KP = D + 4;
#pragma unroll
    for (int i = 0; i < D / 16; ++i)
        f[i] = *reinterpret_cast<const f32x4*>(lds + row * KP + DG * g + 4 * i);
}

// B operand of a product that reduces over the rows of a row-major LDS tile:
// rows row0 + 4g .. row0 + 4g + 3 of column `col` (two ds_read2_b32; the
// 16 lanes of a group hit 16 distinct banks and the four groups are 16 banks
// apart at pitch D + 4).
template <int D>
__device__ __forceinline__ f32x4 col4(const float* lds, int row0, int col, int g) {
    constexpr int KP = D + 4;
    const float* p = lds + (row0 + 4 * g) * KP + col;
    return f32x4{p[0], p[KP], p[2 * KP], p[3 * KP]};
}

// Blocks kb in [KB0, KB1) of S^T (16 keys x 16 queries each) from the row-major
// tile `rows` ([key][D + 4]) and the lane's fragment `qf` of query c: lane
// (c, g) gets keys kb*16 + 4g + r of query c. The next block's LDS fragments
// are read before the current block's MFMAs.
template <int D, int KB0, int KB1>
__device__ __forceinline__ void scores_t(f32x4 (&acc)[8], const float* rows,
                                         const f32x4 (&qf)[D / 16], int c, int g) {
    constexpr int DG = D / 4, KP = D + 4, NF = D / 16;
    const float* kr = rows + c * KP + DG * g;
    f32x4 kf[2][NF];
#pragma unroll
    for (int i = 0; i < NF; ++i)
        kf[KB0 & 1][i] = *reinterpret_cast<const f32x4*>(kr + KB0 * 16 * KP + 4 * i);
#pragma unroll
    for (int kb = KB0; kb < KB1; ++kb) {
        if (kb + 1 < KB1) {
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

// Scores in base-2 exponent units: the query fragment times scale * log2(e),
// so S' = Q' . K^T needs no per-score scaling.
template <int D>
__device__ __forceinline__ void prescale(f32x4 (&qf)[D / 16], float s) {
#pragma unroll
    for (int i = 0; i < D / 16; ++i) qf[i] = qf[i] * s;
}

// FULL: seq == kAttnSeq, so no key, query or row is masked.
template <int D, bool FULL>
__global__ __launch_bounds__(kAttnThreads) void attn_fwd_kernel(AttnArgs a) {
    constexpr int KP = D + 4, NJ = D / 16, U = stage_units<D>();
    static_assert(U == 1 || U == 2, "one or two staging units per thread");
    // key blocks whose rows are staged before the first barrier
    constexpr int KBH = U == 2 ? 4 : 8;
    __shared__ float k_lds[kAttnSeq * KP];
    __shared__ float v_lds[kAttnSeq * KP];
    const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int item = blockIdx.x, S = FULL ? kAttnSeq : a.S;
    const int64_t base = item_base(a, item, D);
    const int64_t ext = ((int64_t)(S - 1) * a.ld + D) * 4;
    const auto rq = buffer_rsrc(a.q + base, ext), rk = buffer_rsrc(a.k + base, ext),
               rv = buffer_rsrc(a.v + base, ext);
    const int qrow = 16 * w + c;
    f32x4 qf[NJ], kv[U], vv[U];
    row_fragment<D>(qf, rq, a.ld, qrow, S, g);
    stage_load<D>(kv, rk, a.ld, S);
    stage_load<D>(vv, rv, a.ld, S);
    prescale<D>(qf, a.scale2);
    // the first half of the keys is multiplied while the second half and V
    // are still arriving (loads return in order)
    stage_store<D>(kv, 0, k_lds);
    if constexpr (U == 1) stage_store<D>(vv, 0, v_lds);
    __syncthreads();
    f32x4 p[8];
    scores_t<D, 0, KBH>(p, k_lds, qf, c, g);
    if constexpr (U == 2) {
        stage_store<D>(kv, 1, k_lds);
        stage_store<D>(vv, 0, v_lds);
        stage_store<D>(vv, 1, v_lds);
        __syncthreads();
        scores_t<D, KBH, 8>(p, k_lds, qf, c, g);
    }
    float m = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (!FULL && kb * 16 + 4 * g + r >= S) p[kb][r] = -INFINITY;
            m = fmaxf(m, p[kb][r]);
        }
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));

    // O = (E . V) / sum with E = 2^(S' - max): A = E (registers, each block
    // exponentiated just before its MFMAs, so the VALU work overlaps them),
    // B = rows of V from LDS, the next block's reads issued first
    f32x4 o[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) o[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float sum = 0.0f;
    f32x4 vf[2][NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) vf[0][j] = col4<D>(v_lds, 0, j * 16 + c, g);
#pragma unroll
    for (int kb = 0; kb < 8; ++kb) {
        if (kb + 1 < 8) {
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                vf[(kb + 1) & 1][j] = col4<D>(v_lds, (kb + 1) * 16, j * 16 + c, g);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float e = __builtin_amdgcn_exp2f(p[kb][r] - m);  // 2^-inf = 0 for masked keys
            p[kb][r] = e;
            sum += e;
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[j] = mfma16(p[kb][r], vf[kb & 1][j][r], o[j]);
    }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    const float rs = 1.0f / sum;
    // o[j][r] is query 16w + 4g + r, whose 1/sum lane 4g + r holds
    float rsr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) rsr[r] = __shfl(rs, 4 * g + r, 64);
    float* out = a.out + base;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * w + 4 * g + r;
            if (FULL || row < S)
                __builtin_nontemporal_store(o[j][r] * rsr[r], out + (int64_t)row * a.ld + j * 16 + c);
        }
    if (g == 0 && (FULL || qrow < S)) {
        float* st = a.stats + ((int64_t)item * S + qrow) * 2;
        st[0] = m;
        st[1] = sum;
    }
}

// Gradient stores of a 16-row block: lane holds rows 16*blk + 4g + r, columns
// j*16 + c; dst = v + beta * dst (the old values were loaded beforehand).
template <int D, bool FULL>
__device__ __forceinline__ void load_old(f32x4 (&old)[D / 16], const float* dst, const AttnArgs& a,
                                         int blk, int c, int g) {
#pragma unroll
    for (int j = 0; j < D / 16; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * blk + 4 * g + r;
            old[j][r] = FULL || row < a.S ? dst[(int64_t)row * a.ld + j * 16 + c] : 0.0f;
        }
}

template <int D, bool FULL>
__device__ __forceinline__ void store_grad(float* dst, const f32x4 (&v)[D / 16],
                                           const f32x4 (&old)[D / 16], const AttnArgs& a, int blk,
                                           int c, int g) {
#pragma unroll
    for (int j = 0; j < D / 16; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * blk + 4 * g + r;
            const float x = a.beta != 0.0f ? v[j][r] + a.beta * old[j][r] : v[j][r];
            if (FULL || row < a.S) dst[(int64_t)row * a.ld + j * 16 + c] = x;
        }
}

// o[d] = sum over the kAttnSeq columns of rows row0 .. row0 + 15 of x_lds
// ([key][query] or [query][key]) times the rows of the row-major tile `rows`.
template <int D>
__device__ __forceinline__ void rows_times(f32x4 (&o)[D / 16], const float* x_lds,
                                           const float* rows, int row0, int c, int g) {
#pragma unroll
    for (int j = 0; j < D / 16; ++j) o[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int qc = 0; qc < 8; ++qc) {
        const f32x4 xf =
            *reinterpret_cast<const f32x4*>(x_lds + (row0 + c) * kAttnTP + qc * 16 + 4 * g);
#pragma unroll
        for (int j = 0; j < D / 16; ++j) {
            const f32x4 tf = col4<D>(rows, qc * 16, j * 16 + c, g);
#pragma unroll
            for (int r = 0; r < 4; ++r) o[j] = mfma16(xf[r], tf[r], o[j]);
        }
    }
}

template <int D, bool FULL>
__global__ __launch_bounds__(kAttnThreads) void attn_bwd_kernel(AttnArgs a) {
    constexpr int KP = D + 4, NJ = D / 16, U = stage_units<D>();
    __shared__ float k_lds[kAttnSeq * KP];     // K  [key][d]
    __shared__ float q_lds[kAttnSeq * KP];     // Q  [query][d]
    __shared__ float v_lds[kAttnSeq * KP];     // V  [key][d]
    __shared__ float do_lds[kAttnSeq * KP];    // dO [query][d]
    __shared__ float x_lds[kAttnSeq * kAttnTP];  // P^T, then dS^T [key][query]
    const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int item = blockIdx.x, S = FULL ? kAttnSeq : a.S;
    const int64_t base = item_base(a, item, D);
    const int64_t ext = ((int64_t)(S - 1) * a.ld + D) * 4;
    const auto rq = buffer_rsrc(a.q + base, ext), rk = buffer_rsrc(a.k + base, ext),
               rv = buffer_rsrc(a.v + base, ext), rdo = buffer_rsrc(a.dout + base, ext);
    const int qrow = 16 * w + c;
    // K and Q first: the score recompute starts once they are staged, while
    // V and dO are still arriving
    f32x4 kv[U], qv[U], vv[U], dv[U];
    stage_load<D>(kv, rk, a.ld, S);
    stage_load<D>(qv, rq, a.ld, S);
    stage_load<D>(vv, rv, a.ld, S);
    stage_load<D>(dv, rdo, a.ld, S);
    float m = 0.0f, sum = 1.0f;
    if (FULL || qrow < S) {
        const float* st = a.stats + ((int64_t)item * S + qrow) * 2;
        m = st[0];
        sum = st[1];
    }
    f32x4 old_q[NJ], old_k[NJ], old_v[NJ];
    if (a.beta != 0.0f) {
        load_old<D, FULL>(old_q, a.dq + base, a, w, c, g);
        load_old<D, FULL>(old_k, a.dk + base, a, w, c, g);
        load_old<D, FULL>(old_v, a.dv + base, a, w, c, g);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        stage_store<D>(kv, u, k_lds);
        stage_store<D>(qv, u, q_lds);
    }
    __syncthreads();

    // S' recomputed exactly as the forward computed it
    f32x4 qf[NJ], p[8];
    lds_row_fragment<D>(qf, q_lds, qrow, g);
    prescale<D>(qf, a.scale2);
    scores_t<D, 0, 8>(p, k_lds, qf, c, g);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        stage_store<D>(vv, u, v_lds);
        stage_store<D>(dv, u, do_lds);
    }
    __syncthreads();
    // dP^T = V . dO^T, in the layout of P; P = 2^(S' - max) / sum meanwhile
    f32x4 df[NJ], ds[8];
    lds_row_fragment<D>(df, do_lds, qrow, g);
    scores_t<D, 0, 8>(ds, v_lds, df, c, g);
    const float rs = 1.0f / sum;
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool live = FULL || (kb * 16 + 4 * g + r < S && qrow < S);
            p[kb][r] = live ? __builtin_amdgcn_exp2f(p[kb][r] - m) * rs : 0.0f;
        }
    // P^T to LDS for dV = P^T . dO
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) x_lds[(kb * 16 + 4 * g + r) * kAttnTP + qrow] = p[kb][r];
    __syncthreads();
    // dV first: its MFMAs overlap the softmax backward's VALU work,
    // dS = (P * (dP - sum(P * dP))) * scale
    f32x4 o_v[NJ];
    rows_times<D>(o_v, x_lds, do_lds, 16 * w, c, g);
    float dot = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) dot = fmaf(p[kb][r], ds[kb][r], dot);
    dot += __shfl_xor(dot, 16, 64);
    dot += __shfl_xor(dot, 32, 64);
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) ds[kb][r] = (p[kb][r] * (ds[kb][r] - dot)) * a.scale;
    // dQ = dS . K (A = dS registers, B = rows of K)
    f32x4 o_q[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) o_q[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const f32x4 kf = col4<D>(k_lds, kb * 16, j * 16 + c, g);
#pragma unroll
            for (int r = 0; r < 4; ++r) o_q[j] = mfma16(ds[kb][r], kf[r], o_q[j]);
        }
    store_grad<D, FULL>(a.dv + base, o_v, old_v, a, w, c, g);
    store_grad<D, FULL>(a.dq + base, o_q, old_q, a, w, c, g);
    __syncthreads();
    // dS^T to LDS for dK = dS^T . Q
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) x_lds[(kb * 16 + 4 * g + r) * kAttnTP + qrow] = ds[kb][r];
    __syncthreads();
    f32x4 o_k[NJ];
    rows_times<D>(o_k, x_lds, q_lds, 16 * w, c, g);
    store_grad<D, FULL>(a.dk + base, o_k, old_k, a, w, c, g);
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
    const bool full = seq == nrs::kAttnSeq;
    auto kernel = d_head == 16 ? (full ? nrs::attn_fwd_kernel<16, true> : nrs::attn_fwd_kernel<16, false>)
                               : (full ? nrs::attn_fwd_kernel<32, true> : nrs::attn_fwd_kernel<32, false>);
    hipLaunchKernelGGL(kernel, grid, dim3(nrs::kAttnThreads), 0, nrs::stream(), a);
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
    const bool full = seq == nrs::kAttnSeq;
    auto kernel = d_head == 16 ? (full ? nrs::attn_bwd_kernel<16, true> : nrs::attn_bwd_kernel<16, false>)
                               : (full ? nrs::attn_bwd_kernel<32, true> : nrs::attn_bwd_kernel<32, false>);
    hipLaunchKernelGGL(kernel, grid, dim3(nrs::kAttnThreads), 0, nrs::stream(), a);
    NRS_LAUNCH_CHECK("attention backward");
    return NRS_OK;
}

}  // extern "C"
