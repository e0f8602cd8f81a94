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
#include <algorithm>

#include "buffer_ops.hpp"

namespace nrs {
namespace {

constexpr int kAttnSeq = 128;  // rows of a tile (the whole sequence of the short kernels)
constexpr int kAttnMaxSeq = 16384;  // longest sequence of the fused path (tiled past kAttnSeq)
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
    const float* o;     // long backward: the forward's output (softmax row term dO . O)
    float* dq_part;     // long backward: [key tiles][items][S][D] partial dQ
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

// ---------------------------------------------------------------- long sequences
// Sequences past kAttnSeq, flash style: the keys stream through LDS in tiles
// of kAttnSeq rows, so nothing of size S x S is ever stored.
//
// Forward: one workgroup per (item, head, tile of kAttnSeq queries), the
// short kernel's layout per tile (wave w owns 16 queries, scores transposed in
// registers). Key tiles are double-buffered (tile t+1's loads fly while tile
// t is reduced) and the softmax is taken online in base 2: per query the
// running max m and sum l; a new tile's max m' rescales the sum and the
// output accumulators by 2^(m - m') before the tile's probabilities
// 2^(u - m') are added. The saved statistics are the final (m, l), so the
// backward's P = 2^(u - m) / l is the softmax of the whole row.
//
// Backward: one workgroup per (item, head, tile of kAttnSeq keys); wave w
// owns 16 keys and loops over the query tiles. With the scores of its key
// held per lane for 32 queries (S^T), dV += P^T . dO and dK += dS^T . Q take
// their A operands straight from registers and accumulate over the query
// tiles; dQ = dS . K goes through an LDS tile ([query][key]) and each key
// tile writes its partial dQ, which a second launch adds in key-tile order
// (deterministic). The softmax backward's row term sum_j P_ij dP_ij is
// dO_i . O_i (the forward output), so no workgroup needs every key.

// Tile t (rows [t * kAttnSeq, ...) of this head) into registers.
template <int D>
__device__ __forceinline__ void tile_load(f32x4 (&vals)[stage_units<D>()], const float* head, int ld,
                                          int S, int t) {
    const int r0 = t * kAttnSeq, rows = min(kAttnSeq, S - r0);
    const auto rs = buffer_rsrc(head + (int64_t)r0 * ld, ((int64_t)(rows - 1) * ld + D) * 4);
    stage_load<D>(vals, rs, ld, rows);
}

template <int D>
__global__ __launch_bounds__(kAttnThreads) void attn_fwd_long_kernel(AttnArgs a) {
    constexpr int KP = D + 4, NJ = D / 16, U = stage_units<D>();
    __shared__ float k_lds[2][kAttnSeq * KP];
    __shared__ float v_lds[2][kAttnSeq * KP];
    const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int S = a.S, T = (S + kAttnSeq - 1) / kAttnSeq;
    const int item = blockIdx.x / T, qt = blockIdx.x - item * T;
    const int64_t base = item_base(a, item, D);
    const auto rq = buffer_rsrc(a.q + base, ((int64_t)(S - 1) * a.ld + D) * 4);
    const int qrow = qt * kAttnSeq + 16 * w + c;
    f32x4 qf[NJ], kv[U], vv[U];
    row_fragment<D>(qf, rq, a.ld, qrow, S, g);
    tile_load<D>(kv, a.k + base, a.ld, S, 0);
    tile_load<D>(vv, a.v + base, a.ld, S, 0);
    prescale<D>(qf, a.scale2);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        stage_store<D>(kv, u, k_lds[0]);
        stage_store<D>(vv, u, v_lds[0]);
    }
    if (T > 1) {
        tile_load<D>(kv, a.k + base, a.ld, S, 1);
        tile_load<D>(vv, a.v + base, a.ld, S, 1);
    }
    __syncthreads();

    float m = -INFINITY, l = 0.0f;  // running max and sum of query c (every g holds them)
    f32x4 o[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) o[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int t = 0; t < T; ++t) {
        const float* kl = k_lds[t & 1];
        const float* vl = v_lds[t & 1];
        f32x4 p[8];
        scores_t<D, 0, 8>(p, kl, qf, c, g);
        float mt = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 8; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (t * kAttnSeq + kb * 16 + 4 * g + r >= S) p[kb][r] = -INFINITY;
                mt = fmaxf(mt, p[kb][r]);
            }
        mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        const float mn = fmaxf(m, mt);
        // rescale of what the earlier tiles added (0 before the first tile)
        const float alpha = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
        m = mn;
        float al[4];  // the factor of accumulator row r: query 16w + 4g + r
#pragma unroll
        for (int r = 0; r < 4; ++r) al[r] = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[j][r] *= al[r];
        float sum = 0.0f;
        f32x4 vf[2][NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) vf[0][j] = col4<D>(vl, 0, j * 16 + c, g);
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) {
            if (kb + 1 < 8) {
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    vf[(kb + 1) & 1][j] = col4<D>(vl, (kb + 1) * 16, j * 16 + c, g);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = __builtin_amdgcn_exp2f(p[kb][r] - m);  // masked keys: 0
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
        l = l * alpha + sum;
        if (t + 1 < T) {
            // the other buffer was last read by tile t - 1, finished by every
            // wave before the previous barrier
#pragma unroll
            for (int u = 0; u < U; ++u) {
                stage_store<D>(kv, u, k_lds[(t + 1) & 1]);
                stage_store<D>(vv, u, v_lds[(t + 1) & 1]);
            }
            if (t + 2 < T) {
                tile_load<D>(kv, a.k + base, a.ld, S, t + 2);
                tile_load<D>(vv, a.v + base, a.ld, S, t + 2);
            }
            __syncthreads();
        }
    }
    const float rl = 1.0f / l;
    float rsr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) rsr[r] = __shfl(rl, 4 * g + r, 64);
    float* out = a.out + base;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = qt * kAttnSeq + 16 * w + 4 * g + r;
            if (row < S)
                __builtin_nontemporal_store(o[j][r] * rsr[r], out + (int64_t)row * a.ld + j * 16 + c);
        }
    if (g == 0 && qrow < S) {
        float* st = a.stats + ((int64_t)item * S + qrow) * 2;
        st[0] = m;
        st[1] = l;
    }
}

template <int D>
__global__ __launch_bounds__(kAttnThreads) void attn_bwd_long_kernel(AttnArgs a) {
    constexpr int KP = D + 4, NJ = D / 16, U = stage_units<D>();
    __shared__ float k_lds[kAttnSeq * KP];       // this workgroup's keys [key][d]
    __shared__ float v_lds[kAttnSeq * KP];       // and values
    __shared__ float q_lds[kAttnSeq * KP];       // the query tile [query][d]
    __shared__ float do_lds[kAttnSeq * KP];      // its output gradient
    __shared__ float x_lds[kAttnSeq * kAttnTP];  // dS [query][key]
    __shared__ f32x4 st_lds[kAttnSeq];           // per query: max, 1/sum, dO . O
    const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tid = threadIdx.x;
    const int S = a.S, T = (S + kAttnSeq - 1) / kAttnSeq;
    const int item = blockIdx.x / T, kt = blockIdx.x - item * T;
    const int64_t base = item_base(a, item, D);
    const int k0 = kt * kAttnSeq, krow = 16 * w + c;  // this lane's key (tile row)
    {
        f32x4 kv[U], vv[U];
        tile_load<D>(kv, a.k + base, a.ld, S, kt);
        tile_load<D>(vv, a.v + base, a.ld, S, kt);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            stage_store<D>(kv, u, k_lds);
            stage_store<D>(vv, u, v_lds);
        }
    }
    __syncthreads();
    // the lane's key row: scaled to base-2 exponents for the scores, plain
    // for dP^T = dO . V^T
    f32x4 kf[NJ], vf[NJ];
    lds_row_fragment<D>(kf, k_lds, krow, g);
    lds_row_fragment<D>(vf, v_lds, krow, g);
    prescale<D>(kf, a.scale2);
    const bool key_live = k0 + krow < S;
    f32x4 o_v[NJ], o_k[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        o_v[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        o_k[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    for (int qt = 0; qt < T; ++qt) {
        const int q0 = qt * kAttnSeq;
        {
            f32x4 qv[U], dv[U];
            tile_load<D>(qv, a.q + base, a.ld, S, qt);
            tile_load<D>(dv, a.dout + base, a.ld, S, qt);
            f32x4 stv = f32x4{0.0f, 1.0f, 0.0f, 0.0f};
            if (tid < kAttnSeq && q0 + tid < S) {
                const int64_t row = q0 + tid;
                const float* st = a.stats + ((int64_t)item * S + row) * 2;
                // the softmax backward's row term: dO . O of this query
                float dot = 0.0f;
                const auto ro = buffer_rsrc(a.o + base + row * a.ld, D * 4);
                const auto rd = buffer_rsrc(a.dout + base + row * a.ld, D * 4);
                float ov[D], dd[D];
#pragma unroll
                for (int d = 0; d < D; ++d) {
                    ov[d] = buffer_load1(ro, 4 * d);
                    dd[d] = buffer_load1(rd, 4 * d);
                }
#pragma unroll
                for (int d = 0; d < D; ++d) dot = fmaf(ov[d], dd[d], dot);
                stv = f32x4{st[0], 1.0f / st[1], dot, 0.0f};
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                stage_store<D>(qv, u, q_lds);
                stage_store<D>(dv, u, do_lds);
            }
            if (tid < kAttnSeq) st_lds[tid] = stv;
        }
        __syncthreads();
        // lane (c, g): key krow, queries qb*16 + 4g + r of the tile
        f32x4 p[8], dp[8];
        scores_t<D, 0, 8>(p, q_lds, kf, c, g);
        scores_t<D, 0, 8>(dp, do_lds, vf, c, g);
#pragma unroll
        for (int qb = 0; qb < 8; ++qb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int ql = qb * 16 + 4 * g + r;
                const f32x4 st = st_lds[ql];
                const bool live = key_live & (q0 + ql < S);
                const float pr = live ? __builtin_amdgcn_exp2f(p[qb][r] - st[0]) * st[1] : 0.0f;
                p[qb][r] = pr;
                dp[qb][r] = (pr * (dp[qb][r] - st[2])) * a.scale;  // dS
                x_lds[ql * kAttnTP + krow] = dp[qb][r];
            }
        // dV += P^T . dO and dK += dS^T . Q over this query tile
#pragma unroll
        for (int qb = 0; qb < 8; ++qb)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const f32x4 df = col4<D>(do_lds, qb * 16, j * 16 + c, g);
                const f32x4 qf = col4<D>(q_lds, qb * 16, j * 16 + c, g);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    o_v[j] = mfma16(p[qb][r], df[r], o_v[j]);
                    o_k[j] = mfma16(dp[qb][r], qf[r], o_k[j]);
                }
            }
        __syncthreads();
        // this key tile's part of dQ = dS . K for queries 16w + 4g + r
        f32x4 o_q[NJ];
        rows_times<D>(o_q, x_lds, k_lds, 16 * w, c, g);
        float* part = a.dq_part + (((int64_t)kt * (gridDim.x / T) + item) * S + q0) * D;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int ql = 16 * w + 4 * g + r;
                if (q0 + ql < S) part[(int64_t)ql * D + j * 16 + c] = o_q[j][r];
            }
        __syncthreads();  // q_lds, do_lds, x_lds and st_lds are restaged next
    }
    // dK, dV of this workgroup's keys (rows k0 + 16w + 4g + r)
    f32x4 old_k[NJ], old_v[NJ];
    AttnArgs t = a;
    t.S = S - k0;  // rows past the sequence are not stored
    if (a.beta != 0.0f) {
        load_old<D, false>(old_k, a.dk + base + (int64_t)k0 * a.ld, t, w, c, g);
        load_old<D, false>(old_v, a.dv + base + (int64_t)k0 * a.ld, t, w, c, g);
    }
    store_grad<D, false>(a.dk + base + (int64_t)k0 * a.ld, o_k, old_k, t, w, c, g);
    store_grad<D, false>(a.dv + base + (int64_t)k0 * a.ld, o_v, old_v, t, w, c, g);
}

// dq[item][row][d] = sum over key tiles of dq_part (in key-tile order)
// + beta * dq, one thread per element.
__global__ __launch_bounds__(256) void attn_dq_sum_kernel(AttnArgs a, int items, int D) {
    const int T = (a.S + kAttnSeq - 1) / kAttnSeq;
    const int64_t n = (int64_t)items * a.S * D;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
        float v = 0.0f;
        for (int t = 0; t < T; ++t) v += a.dq_part[(int64_t)t * n + e];
        const int64_t rd = e / D;
        const int d = (int)(e - rd * D);
        const int item = (int)(rd / a.S), row = (int)(rd - (int64_t)item * a.S);
        float* dst = a.dq + item_base(a, item, D) + (int64_t)row * a.ld + d;
        *dst = a.beta != 0.0f ? v + a.beta * *dst : v;
    }
}

bool attn_shape_ok(int64_t batch, int64_t heads, int64_t seq, int64_t d_head, int64_t ld) {
    return batch >= 0 && heads >= 1 && seq >= 1 && seq <= kAttnMaxSeq &&
           (d_head == 16 || d_head == 32) && ld >= heads * d_head && ld <= (1 << 20) &&
           seq * ld <= (1 << 29) && batch * heads * ((seq + kAttnSeq - 1) / kAttnSeq) <= INT32_MAX;
}

int attn_check(const char* what, int64_t batch, int64_t heads, int64_t seq, int64_t d_head,
               int64_t ld) {
    NRS_ARG_CHECK(attn_shape_ok(batch, heads, seq, d_head, ld),
                  "%s: unsupported shape (batch %lld, heads %lld, seq %lld, d_head %lld, ld %lld): "
                  "the fused path takes seq <= %d, d_head 16 or 32, ld >= heads * d_head, "
                  "seq * ld <= 2^29",
                  what, (long long)batch, (long long)heads, (long long)seq, (long long)d_head,
                  (long long)ld, kAttnMaxSeq);
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
    if (seq > nrs::kAttnSeq) {
        // query tiles of one head each stream every key tile
        const int64_t tiles = (seq + nrs::kAttnSeq - 1) / nrs::kAttnSeq;
        auto kernel = d_head == 16 ? nrs::attn_fwd_long_kernel<16> : nrs::attn_fwd_long_kernel<32>;
        hipLaunchKernelGGL(kernel, dim3((unsigned)(batch * heads * tiles)), dim3(nrs::kAttnThreads),
                           0, nrs::stream(), a);
        NRS_LAUNCH_CHECK("attention forward (tiled)");
        return NRS_OK;
    }
    const dim3 grid((unsigned)(batch * heads));
    const bool full = seq == nrs::kAttnSeq;
    auto kernel = d_head == 16 ? (full ? nrs::attn_fwd_kernel<16, true> : nrs::attn_fwd_kernel<16, false>)
                               : (full ? nrs::attn_fwd_kernel<32, true> : nrs::attn_fwd_kernel<32, false>);
    hipLaunchKernelGGL(kernel, grid, dim3(nrs::kAttnThreads), 0, nrs::stream(), a);
    NRS_LAUNCH_CHECK("attention forward");
    return NRS_OK;
}

int nrs_attention_backward(float* dq, float* dk, float* dv, const float* dout, const float* out,
                           const float* q, const float* k, const float* v, const float* stats,
                           int64_t batch, int64_t heads, int64_t seq, int64_t d_head, int64_t ld,
                           float scale, float beta) {
    NRS_REQUIRE_INIT();
    if (int rc = nrs::attn_check("attention backward", batch, heads, seq, d_head, ld)) return rc;
    if (batch == 0) return NRS_OK;
    NRS_ARG_CHECK(dq && dk && dv && dout && q && k && v && stats,
                  "attention backward: null pointer");
    NRS_ARG_CHECK(out || seq <= nrs::kAttnSeq,
                  "attention backward: sequences past %d need the forward output", nrs::kAttnSeq);
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
    if (seq > nrs::kAttnSeq) {
        // key tiles of one head each stream every query tile; their partial
        // dQ are added in key-tile order by a second launch
        const int64_t tiles = (seq + nrs::kAttnSeq - 1) / nrs::kAttnSeq;
        const int64_t items = batch * heads;
        float* part = nrs::workspace(sizeof(float) * (size_t)(tiles * items * seq * d_head), 0);
        if (!part) return NRS_ERR_ALLOC;
        a.o = out;
        a.dq_part = part;
        auto kernel = d_head == 16 ? nrs::attn_bwd_long_kernel<16> : nrs::attn_bwd_long_kernel<32>;
        hipLaunchKernelGGL(kernel, dim3((unsigned)(items * tiles)), dim3(nrs::kAttnThreads), 0,
                           nrs::stream(), a);
        NRS_LAUNCH_CHECK("attention backward (tiled)");
        const int64_t n = items * seq * d_head;
        hipLaunchKernelGGL(nrs::attn_dq_sum_kernel,
                           dim3((unsigned)std::min<int64_t>((n + 255) / 256, 4096)), dim3(256), 0,
                           nrs::stream(), a, (int)items, (int)d_head);
        NRS_LAUNCH_CHECK("attention backward (dQ sum)");
        return NRS_OK;
    }
    const dim3 grid((unsigned)(batch * heads));
    const bool full = seq == nrs::kAttnSeq;
    auto kernel = d_head == 16 ? (full ? nrs::attn_bwd_kernel<16, true> : nrs::attn_bwd_kernel<16, false>)
                               : (full ? nrs::attn_bwd_kernel<32, true> : nrs::attn_bwd_kernel<32, false>);
    hipLaunchKernelGGL(kernel, grid, dim3(nrs::kAttnThreads), 0, nrs::stream(), a);
    NRS_LAUNCH_CHECK("attention backward");
    return NRS_OK;
}

}  // extern "C"
