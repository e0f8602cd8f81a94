// Short GEMMs: products whose output covers only a few 64x64 tiles, e.g.
// the MLP's Linear layers at batch 256 (src/cuda/graph/matmul.rs:44-198
// through Linear::forward and the matmul backward closure, linear.rs:22-25,
// matmul.rs:418-431).
//
// On the tiled core such a product either runs a handful of workgroups down
// a long k loop (one memory round trip per k-tile) or is split over K into
// partial tiles that a second launch sums. Both cost several microseconds of
// round trips and launches for a few hundred nanoseconds of matrix-core
// work. Here a workgroup owns one 16x16 block of C and splits its reduction
// over its W waves:
//  * in round r, lane group g (lanes 16g..16g+15) of wave w reduces the S
//    consecutive k values starting at r*W*4S + w*4S + g*S, so the S A values
//    of a lane (row 16tm + lane%16) and its S B values (column 16tn +
//    lane%16) are contiguous in k: 128-bit loads where k is the contiguous
//    dimension, else one float per step with 16 lanes reading 64 contiguous
//    bytes. Every load of a round is issued before its first
//    v_mfma_f32_16x16x4f32, so a round costs one memory round trip; S
//    MFMAs consume it (step s takes k = base + g*S + s from lane group g);
//  * the W partial blocks meet in LDS and are added in wave order (a fixed
//    order: the result does not depend on timing), then the epilogue runs
//    with one thread per output element.
// Reduction-dim padding, rows past M and columns past N read zero through
// the buffer bounds. Epilogues: bias (column or row), ReLU, a mask (v = 0
// where mask <= 0: the ReLU backward of src/cuda/graph/relu.rs:16-28 fused
// into the product that feeds it), beta * old, a row of sums (row M of the
// product has an all-ones A row: the column sums of op(B), a Linear's bias
// gradient), and the fused cross-entropy seed of
// src/cuda/loss/cross_entropy.rs:39-58 for outputs of at most 16 columns.
// Up to kWsMax independent problems share one launch.
#include <algorithm>

#include "buffer_ops.hpp"
#include "gemm_call.hpp"
#include "gemm_wsplit.hpp"

namespace nrs {
namespace {

// Row of element e (mod 256) of a 16x16 block in the sums: a wave's 64
// elements are rows r, r + 4, r + 8, r + 12 (r = bits 6-7 of e) by 16
// columns, 16 banks apart at the pitch below, so the reads do not conflict;
// each store still covers whole 64-byte row segments.
__device__ __forceinline__ int ws_row(int e) { return ((e >> 4) & 3) * 4 + ((e >> 6) & 3); }

// LDS pitch of a 16x16 partial block. A wave stores rows 4g + r, columns c
// (g < 4, c < 16) at (4g + r) * pitch + c: with pitch = 4 (mod 16) the four
// row groups start 16 banks apart, so the 64 lanes hit 64 banks (17 put
// rows 4 apart and conflicted about 4-way).
constexpr int kWsPitch = 20;

__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Operand access of a problem, fixed per kernel body so that a round's
// loads are straight-line code (a branch between load forms made the
// compiler wait for the loads at the join): A's k-contiguous rows loaded
// 128 bits (AV) or 32 bits at a time, or A stored [K][M] (TN); likewise B.
enum WsMode { WS_NN_AV = 0, WS_NN_AS, WS_NT_AV_BV, WS_NT_AV_BS, WS_NT_AS_BV, WS_NT_AS_BS, WS_TN,
              WS_MODES };

// The S values of op(A) for row m at k = k0 .. k0+S-1 (zero past K and M).
template <int MODE, int S>
__device__ __forceinline__ void load_a(const WsProblem& p, __amdgpu_buffer_rsrc_t ra, int m, int k0,
                                       float (&av)[S]) {
    constexpr bool a_kc = MODE != WS_TN;
    constexpr bool a_vec = MODE == WS_NN_AV || MODE == WS_NT_AV_BV || MODE == WS_NT_AV_BS;
    const bool m_ok = m < p.M;
    if constexpr (a_vec) {
#pragma unroll
        for (int v = 0; v < S / 4; ++v) {
            const int k = k0 + 4 * v;
            const f32x4 x = buffer_load4(
                ra, (m_ok & (k < p.K)) ? (int)(((int64_t)m * p.lda + k) * 4) : kOutOfRange);
#pragma unroll
            for (int e = 0; e < 4; ++e) av[4 * v + e] = x[e];
        }
    } else {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int k = k0 + s;
            const int64_t off = a_kc ? (int64_t)m * p.lda + k : (int64_t)k * p.lda + m;
            av[s] = buffer_load1(ra, (m_ok & (k < p.K)) ? (int)(off * 4) : kOutOfRange);
        }
    }
}

// The S values of op(B) for column n at k = k0 .. k0+S-1 (zero past K and N).
template <int MODE, int S>
__device__ __forceinline__ void load_b(const WsProblem& p, __amdgpu_buffer_rsrc_t rb, int n, int k0,
                                       float (&bv)[S]) {
    constexpr bool b_kc = MODE >= WS_NT_AV_BV && MODE <= WS_NT_AS_BS;
    constexpr bool b_vec = MODE == WS_NT_AV_BV || MODE == WS_NT_AS_BV;
    const bool n_ok = n < p.N;
    if constexpr (b_vec) {
#pragma unroll
        for (int v = 0; v < S / 4; ++v) {
            const int k = k0 + 4 * v;
            const f32x4 x = buffer_load4(
                rb, (n_ok & (k < p.K)) ? (int)(((int64_t)n * p.ldb + k) * 4) : kOutOfRange);
#pragma unroll
            for (int e = 0; e < 4; ++e) bv[4 * v + e] = x[e];
        }
    } else {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int k = k0 + s;
            const int64_t off = b_kc ? (int64_t)n * p.ldb + k : (int64_t)k * p.ldb + n;
            bv[s] = buffer_load1(rb, (n_ok & (k < p.K)) ? (int)(off * 4) : kOutOfRange);
        }
    }
}

// This wave's partial 16x16 blocks (TM row blocks by TN column blocks from
// (m0, n0)) over its k values of every round. Each block sees the same MFMA
// sequence as a workgroup of one block would, so the grouping changes no
// bits. The lane holding the row of sums (row M) feeds 1 for k < K in place
// of A.
template <int W, int S, int MODE, int TM, int TN>
__device__ __forceinline__ void ws_reduce(const WsProblem& p, int m0, int n0, int w, int c, int g,
                                          f32x4 (&acc)[TM][TN]) {
    const auto ra = buffer_rsrc(p.A, p.a_bytes), rb = buffer_rsrc(p.B, p.b_bytes);
    bool ones[TM];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) ones[tm] = p.sum_row != nullptr && m0 + 16 * tm + c == p.M;
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = w * 4 * S + g * S; k0 < p.K + w * 4 * S + g * S; k0 += W * 4 * S) {
        float av[TM][S], bv[TN][S];
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) load_a<MODE, S>(p, ra, m0 + 16 * tm + c, k0, av[tm]);
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) load_b<MODE, S>(p, rb, n0 + 16 * tn + c, k0, bv[tn]);
        // every load of the round before the first MFMA (left alone, the
        // scheduler interleaves them to save registers: a round trip each)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
                const float a = ones[tm] ? (k0 + s < p.K ? 1.0f : 0.0f) : av[tm][s];
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = mfma16(a, bv[tn][s], acc[tm][tn]);
            }
    }
}

// One workgroup per TM x TN group of 16x16 blocks of one problem's output
// (TM = TN = 1 for the cross-entropy epilogue, whose rows are one block).
template <int W, int S, int TM, int TN>
__global__ __launch_bounds__(64 * W) void gemm_wsplit_kernel(WsArgs args) {
    constexpr int NBLK = TM * TN;
    __shared__ float red[W * NBLK * 16 * kWsPitch];
    __shared__ float row_stat[2][16];
    int q = 0;
#pragma unroll
    for (int i = 1; i < kWsMax; ++i)
        if (i < args.count && (int)blockIdx.x >= args.prob[i].first) q = i;
    const WsProblem& p = args.prob[q];
    const int tid = threadIdx.x, lane = tid & 63, c = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = (int)blockIdx.x - p.first;
    const int tm = tile / p.tiles_n, tn = tile - tm * p.tiles_n;
    const int m0 = 16 * TM * tm, n0 = 16 * TN * tn;
    f32x4 acc[TM][TN];
    switch (p.mode) {
        case WS_NN_AV: ws_reduce<W, S, WS_NN_AV, TM, TN>(p, m0, n0, w, c, g, acc); break;
        case WS_NN_AS: ws_reduce<W, S, WS_NN_AS, TM, TN>(p, m0, n0, w, c, g, acc); break;
        case WS_NT_AV_BV: ws_reduce<W, S, WS_NT_AV_BV, TM, TN>(p, m0, n0, w, c, g, acc); break;
        case WS_NT_AV_BS: ws_reduce<W, S, WS_NT_AV_BS, TM, TN>(p, m0, n0, w, c, g, acc); break;
        case WS_NT_AS_BV: ws_reduce<W, S, WS_NT_AS_BV, TM, TN>(p, m0, n0, w, c, g, acc); break;
        case WS_NT_AS_BS: ws_reduce<W, S, WS_NT_AS_BS, TM, TN>(p, m0, n0, w, c, g, acc); break;
        default: ws_reduce<W, S, WS_TN, TM, TN>(p, m0, n0, w, c, g, acc); break;
    }
    // lane (c, g) holds rows 4g..4g+3 of column c of each of this wave's
    // partial blocks
#pragma unroll
    for (int bm = 0; bm < TM; ++bm)
#pragma unroll
        for (int bn = 0; bn < TN; ++bn)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                red[((w * NBLK + bm * TN + bn) * 16 + 4 * g + r) * kWsPitch + c] = acc[bm][bn][r];
    __syncthreads();
    if constexpr (NBLK == 1) {
        if (p.epi & kWsCe) {
            // the fused seed (softmax(logits) - target) / batch, with the
            // reference kernel's arithmetic: the row max folded from class 0,
            // the sum of expf(l - max) in class order, then expf(l - max) / sum
            const int i = ws_row(tid), j = tid & 15;
            const int row = m0 + i, col = n0 + j;
            float v = 0.0f;
            if (tid < 256) {
#pragma unroll
                for (int ww = 0; ww < W; ++ww) v += red[(ww * 16 + i) * kWsPitch + j];
                if (p.epi & NRS_EPI_BIAS_COL) v += col < p.N ? p.bias[col] : 0.0f;
                if (p.epi & NRS_EPI_BIAS_ROW) v += row < p.M ? p.bias[row] : 0.0f;
            }
            __syncthreads();  // every wave is done reading its partial block
            if (tid < 256) red[i * kWsPitch + j] = v;
            __syncthreads();
            if (tid < 16 && m0 + tid < p.M) {
                const float* l = red + tid * kWsPitch;
                float mx = l[0];
                for (int cc = 1; cc < p.N; ++cc) mx = fmaxf(mx, l[cc]);
                float sum = 0.0f;
                for (int cc = 0; cc < p.N; ++cc) sum += expf(l[cc] - mx);
                row_stat[0][tid] = mx;
                row_stat[1][tid] = sum;
            }
            __syncthreads();
            if (tid < 256 && row < p.M && col < p.N) {
                const int64_t idx = (int64_t)row * p.ldc + col;
                const float t = p.target[idx];
                p.aux[idx] = (expf(v - row_stat[0][i]) / row_stat[1][i] - t) * p.inv_batch;
                if (p.C) p.C[idx] = v;
            }
            return;
        }
    }
    // one thread per output element: the W partials added in wave order
    for (int e = tid; e < NBLK * 256; e += 64 * W) {
        const int blk = e >> 8, i = ws_row(e), j = e & 15;
        const int bm = blk / TN, bn = blk - bm * TN;
        const int row = m0 + 16 * bm + i, col = n0 + 16 * bn + j;
        if (col >= p.N) continue;
        float v = 0.0f;
#pragma unroll
        for (int ww = 0; ww < W; ++ww) v += red[((ww * NBLK + blk) * 16 + i) * kWsPitch + j];
        if (p.epi & NRS_EPI_BIAS_COL) v += p.bias[col];
        if (p.epi & NRS_EPI_BIAS_ROW) v += row < p.M ? p.bias[row] : 0.0f;
        if (row < p.M) {
            if (p.epi & NRS_EPI_RELU) v = fmaxf(v, 0.0f);
            const int64_t idx = (int64_t)row * p.ldc + col;
            if ((p.epi & kWsMask) && !(p.mask[idx] > 0.0f)) v = 0.0f;
            if (p.beta != 0.0f) v = v + p.beta * p.C[idx];
            p.C[idx] = v;
        } else if (row == p.M && p.sum_row != nullptr) {
            if (p.sum_beta != 0.0f) v = v + p.sum_beta * p.sum_row[col];
            p.sum_row[col] = v;
        }
    }
}

using WsKernel = void (*)(WsArgs);

// (waves, k values per lane group per round) for a reduction of length K:
// the smallest round that covers K, else 8 waves of 32 (several rounds);
// `group`: each workgroup takes 2 x 2 blocks.
template <int TM, int TN>
WsKernel ws_kernel_for(int64_t K, int& threads) {
    if (K <= 128) {
        threads = 256;
        return gemm_wsplit_kernel<4, 8, TM, TN>;
    }
    threads = 512;
    if (K <= 256) return gemm_wsplit_kernel<8, 8, TM, TN>;
    if (K <= 512) return gemm_wsplit_kernel<8, 16, TM, TN>;
    return gemm_wsplit_kernel<8, 32, TM, TN>;
}

WsKernel ws_kernel_for(int64_t K, bool group, int& threads) {
    return group ? ws_kernel_for<2, 2>(K, threads) : ws_kernel_for<1, 1>(K, threads);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

bool wsplit_eligible(const GemmCall& c, bool automatic) {
    // (a caller-provided partials buffer does not matter: this kernel keeps
    // its partial sums on chip)
    if (c.amode != OP_DENSE || c.bmode != OP_DENSE || c.batch != 1 || c.nchw_P != 0 ||
        c.force_slices != 0 || c.K < 1 || c.M < 1 || c.N < 1)
        return false;
    if (c.epi & ~(NRS_EPI_BIAS_COL | NRS_EPI_BIAS_ROW | NRS_EPI_RELU)) return false;
    if (c.K > kWsMaxK || c.M >= (1 << 30) || c.N >= (1 << 30)) return false;
    if (automatic && c.K > kWsAutoMaxK) return false;
    // every valid element's byte offset must stay below the buffer bound
    const int64_t limit = int64_t(1) << 31;
    if (c.M * c.K * 4 >= limit || c.K * c.N * 4 >= limit || c.M * c.N * 4 >= limit) return false;
    if (!automatic) return true;
    // the tiled core's plan for this output: few 64x64 tiles means a split
    // over K (plus a reduce launch) or a short grid down a long k loop
    const int cus = num_cus();
    const int64_t mrows = c.M + (c.sum_row ? 1 : 0);
    const int64_t tiles64 = ((mrows + 63) / 64) * ((c.N + 63) / 64);
    const int64_t tiles16 = ((mrows + 15) / 16) * ((c.N + 15) / 16);
    return 2 * tiles64 <= cus && tiles16 <= 4 * (int64_t)cus;
}

int wsplit_run(const GemmCall* calls, int count, const WsExtra* extra) {
    NRS_ARG_CHECK(count >= 1 && count <= kWsMax, "short gemm: %d problems", count);
    WsArgs a{};
    int64_t total = 0, kmax = 0;
    for (int i = 0; i < count; ++i) {
        const GemmCall& c = calls[i];
        WsProblem& p = a.prob[i];
        p.A = c.A;
        p.B = c.B;
        p.C = c.C;
        p.bias = c.bias;
        p.sum_row = c.sum_row;
        p.sum_beta = c.sum_beta;
        p.M = (int)c.M;
        p.N = (int)c.N;
        p.K = (int)c.K;
        p.layout = c.layout;
        p.lda = c.layout == NRS_TN ? c.M : c.K;
        p.ldb = c.layout == NRS_NT ? c.K : c.N;
        p.ldc = c.N;
        p.a_bytes = c.M * c.K * 4;
        p.b_bytes = c.K * c.N * 4;
        const bool a_vec = c.layout != NRS_TN && aligned16(c.A) && c.K % 4 == 0;
        const bool b_vec = c.layout == NRS_NT && aligned16(c.B) && c.K % 4 == 0;
        p.mode = c.layout == NRS_TN   ? WS_TN
                 : c.layout == NRS_NN ? (a_vec ? WS_NN_AV : WS_NN_AS)
                 : a_vec              ? (b_vec ? WS_NT_AV_BV : WS_NT_AV_BS)
                                      : (b_vec ? WS_NT_AS_BV : WS_NT_AS_BS);
        p.beta = c.beta;
        p.epi = c.epi;
        if (c.mask) {
            p.mask = c.mask;
            p.epi |= kWsMask;
        }
        if (extra && extra[i].ce_grad) {
            NRS_ARG_CHECK(c.N <= 16 && c.sum_row == nullptr && c.beta == 0.0f,
                          "short gemm: the cross-entropy epilogue needs <= 16 columns");
            p.aux = extra[i].ce_grad;
            p.target = extra[i].ce_target;
            p.inv_batch = 1.0f / (float)c.M;
            p.epi |= kWsCe;
        }
        kmax = std::max<int64_t>(kmax, c.K);
    }
    // Outputs of many 16x16 blocks (more than two a CU) go 2 x 2 blocks a
    // workgroup: a quarter of the workgroups, each reusing its loads of A
    // and B twice, with every block's arithmetic unchanged. The
    // cross-entropy epilogue keeps one block a workgroup.
    int64_t blocks = 0;
    bool ce = false;
    for (int i = 0; i < count; ++i) {
        const int64_t mrows = calls[i].M + (calls[i].sum_row ? 1 : 0);
        blocks += ((mrows + 15) / 16) * ((calls[i].N + 15) / 16);
        ce = ce || (a.prob[i].epi & kWsCe);
    }
    const bool group = !ce && blocks > 2 * (int64_t)num_cus();
    const int bm = group ? 32 : 16, bn = group ? 32 : 16;
    for (int i = 0; i < count; ++i) {
        WsProblem& p = a.prob[i];
        const int64_t mrows = calls[i].M + (calls[i].sum_row ? 1 : 0);
        p.tiles_n = (int)((calls[i].N + bn - 1) / bn);
        p.first = (int)total;
        total += ((mrows + bm - 1) / bm) * p.tiles_n;
    }
    a.count = count;
    NRS_ARG_CHECK(total <= INT32_MAX, "short gemm: grid too large");
    int threads = 0;
    WsKernel fn = ws_kernel_for(kmax, group, threads);
    hipLaunchKernelGGL(fn, dim3((unsigned)total), dim3(threads), 0, stream(), a);
    NRS_LAUNCH_CHECK("short gemm");
    return NRS_OK;
}

}  // namespace nrs
