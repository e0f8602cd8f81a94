// The two-layer MLP step of the reference's MNIST example (cfg2,
// examples/mnist_cuda.rs:34-37: relu(x . w1 + b1) . w2 + b2, then the fused
// cross-entropy seed) in two launches:
//
//   nrs_mlp2_forward_seed  h  = relu(x . w1 + b1)               [batch, hidden]
//                          z  = h . w2 + b2                     [batch, classes]
//                          gz = (softmax(z) - target) / batch   [batch, classes]
//                          dh = (gz . w2^T) * (h > 0)           [batch, hidden]
//   nrs_mlp2_backward      dx = dh . w1^T, dw1 = x^T . dh, db1 = sum(dh),
//                          dw2 = h^T . gz, db2 = sum(gz)  (one short-GEMM launch)
//
// Everything up to dh is row-local, so the first launch gives each workgroup
// four rows of the batch and carries them from the input to the hidden
// gradient on chip. Its first product reads all of w1 per workgroup; one CU
// streams it from L2 at ~120 GB/s with 128-bit loads (401 KB in ~3.3 us at
// 784 x 128), and four rows are the most that v_mfma_f32_4x4x1f32 reduces
// within that time, so 64 workgroups run at batch 256. The reduction over
// in_f is split over the 8 waves (ranges of kw rows of w1), each wave
// requesting its next batch of rows before reducing the current one; the
// partial rows meet in LDS and are added in a fixed order. The rest is
// small: w2 is staged in LDS, the logits reduce their hidden dimension in 8
// parts added in order, the seed is ce_backward's arithmetic
// (src/cuda/loss/cross_entropy.rs:39-58: the row max folded from class 0,
// the sum of expf(l - max) in class order), and dh is relu_grad of
// src/cuda/graph/relu.rs:23-28 (the gradient where the pre-activation,
// equivalently h, is > 0) applied to gz . w2^T.
#include <algorithm>

#include "buffer_ops.hpp"
#include "gemm_call.hpp"
#include "nrs_internal.hpp"

namespace nrs {
namespace {

constexpr int kHeadRows = 4;                    // batch rows per workgroup
constexpr int kHeadWaves = 8;                   // waves splitting the first reduction
constexpr int kHeadThreads = 64 * kHeadWaves;
constexpr int kHeadMaxHidden = 256;
constexpr int kHeadMaxClasses = 16;
constexpr int kHeadMaxIn = 4096;                // the block's x rows staged in LDS (64 KB)
constexpr int kHeadSmallIn = 1024;
constexpr int kHeadXPad = 64;                   // zeros after the staged x rows

struct HeadArgs {
    const float* x;       // [B][I]
    const float* w1;      // [I][H]
    const float* b1;      // [H] or null
    const float* w2;      // [H][O]
    const float* b2;      // [O] or null
    const float* target;  // [B][O]
    float* h;
    float* z;
    float* gz;
    float* dh;
    int B, I, H, O;
    int kw;  // rows of w1 per wave, a multiple of 4
    float inv_batch;
};

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0);
}

// HP: hidden columns padded to 64, 128 or 256; FAST: hidden % 4 == 0 and
// in_f % 4 == 0 with 16-byte aligned x and w1 (128-bit loads); SMALLX:
// in_f <= kHeadSmallIn (fewer x load slots per thread).
//
// The first product streams w1 with 128-bit loads: one wave load covers
// P = 256 / HP consecutive rows of w1 (LPR = HP / 4 lanes a row), lane l
// holding row k + q, q = l / LPR, columns 4 (l % LPR) .. + 3. (A CU's
// L2 read rate follows load instructions, not bytes: 64-bit loads measured
// half the rate.) The 16 blocks of v_mfma_f32_4x4x1f32 are independent
// products, so block b of MFMA g (g = 0..3: element g of each lane's
// vector) reduces row k + q of the lanes it holds: lanes 4b..4b+3 share q,
// A = x[row0 + i][k + q] from lane 4b + i, B = w1[k + q][4 (l % LPR) + g]
// from lane l = 4b + j, D[i][j] in lane 4b + j, register i. Each lane's
// accumulator g thus sums hidden column 4 (l % LPR) + g over the rows
// k = q mod P of this wave's range; the P parities and the 8 waves are
// added in LDS in a fixed order. The block's 4 x rows are staged in LDS
// first, so A costs no global load instructions.
template <int HP, bool FAST, bool SMALLX>
__global__ __launch_bounds__(kHeadThreads) void mlp_head_kernel(HeadArgs a) {
    constexpr int P = 256 / HP, LPR = HP / 4, RP = HP + 4, NPART = kHeadWaves * P;
    constexpr int NB = 8;  // w1 loads per batch (8 KB a wave); two batches in flight
    extern __shared__ __attribute__((aligned(16))) float xs[];  // [4][I] x rows, then kHeadXPad zeros
    __shared__ float red[NPART * kHeadRows * RP];  // partial rows of h, then logit parts
    __shared__ float w2s[HP * kHeadMaxClasses];
    __shared__ float hs[kHeadRows * HP];
    __shared__ float zs[kHeadRows * kHeadMaxClasses];
    __shared__ float gs[kHeadRows * kHeadMaxClasses];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row0 = blockIdx.x * kHeadRows;
    const int H = a.H, O = a.O, I = a.I;
    const int q = lane / LPR, cb = 4 * (lane % LPR);
    const int k0 = w * a.kw, k1 = min(I, k0 + a.kw);
    const auto rw = buffer_rsrc(a.w1, (int64_t)I * H * 4);

    // this wave's w1 rows k .. k + P - 1 as one 128-bit load per lane
    auto load_w = [&](int k) -> f32x4 {
        const int kr = k + q;
        const bool ok = kr < k1;
        if constexpr (FAST) {
            return buffer_load4(rw, (ok & (cb < H)) ? (kr * H + cb) * 4 : kOutOfRange);
        } else {
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v[e] = buffer_load1(rw, (ok & (cb + e < H)) ? (kr * H + cb + e) * 4 : kOutOfRange);
            return v;
        }
    };
    constexpr int KB = NB * P;  // rows per batch
    // the x rows' loads first, then the first two batches of w1 (the x
    // stores wait only for the x loads)
    constexpr int XPT = (kHeadRows * (SMALLX ? kHeadSmallIn : kHeadMaxIn) / 4 + kHeadThreads - 1) /
                        kHeadThreads;
    const int xn = kHeadRows * I, xvalid = max(0, min(a.B - row0, kHeadRows)) * I;
    const auto rx = buffer_rsrc(a.x + (int64_t)row0 * I, (int64_t)xvalid * 4);
    f32x4 xv[FAST ? XPT : 1];
    if constexpr (FAST) {
        // unconditional (zero past the rows): no branch between the loads
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const int e = 4 * (tid + kHeadThreads * j);
            xv[j] = buffer_load4(rx, e < xn ? e * 4 : kOutOfRange);
        }
    }
    // the tail's operands from global memory, requested early (each would
    // otherwise be a round trip between two barriers): b1 for this thread's
    // h elements, and for wave 0 (logits and seed) b2 and the targets
    constexpr int HPT = (kHeadRows * HP + kHeadThreads - 1) / kHeadThreads;
    float b1v[HPT], b2v = 0.0f, tv = 0.0f;
    {
        const auto rb1 = buffer_rsrc(a.b1, a.b1 ? (int64_t)H * 4 : 0);
#pragma unroll
        for (int j = 0; j < HPT; ++j) {
            const int e = tid + kHeadThreads * j;
            b1v[j] = buffer_load1(rb1, e < kHeadRows * H ? (e % H) * 4 : kOutOfRange);
        }
        const int r = (tid >> 4) & 3, o = tid & 15;
        const auto rb2 = buffer_rsrc(a.b2, a.b2 ? (int64_t)O * 4 : 0);
        b2v = buffer_load1(rb2, o < O ? o * 4 : kOutOfRange);
        const int trow = row0 + r;
        const auto rt = buffer_rsrc(a.target, (int64_t)a.B * O * 4);
        tv = buffer_load1(rt, (o < O && trow < a.B) ? (trow * O + o) * 4 : kOutOfRange);
    }
    f32x4 wv[2][NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) wv[0][u] = load_w(k0 + P * u);
#pragma unroll
    for (int u = 0; u < NB; ++u) wv[1][u] = load_w(k0 + KB + P * u);
    if constexpr (FAST) {
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const int e = 4 * (tid + kHeadThreads * j);
            if (e < xn) *reinterpret_cast<f32x4*>(xs + e) = xv[j];
        }
    } else {
        for (int e = tid; e < xn; e += kHeadThreads) xs[e] = buffer_load1(rx, e * 4);
    }
    // past the last row: a batch may run up to KB - 1 rows past the wave's
    // range (plus the parity q), whose w1 values read as zero; their x
    // values must be finite (0 * NaN is NaN), so they read zeros
    static_assert(KB + P <= kHeadXPad, "zero pad past the x rows");
    if (tid < kHeadXPad) xs[xn + tid] = 0.0f;
    // w2 (read by the logits and dh) into registers; it goes to LDS after
    // the reduction, so no wait for it sits among the batches' loads
    constexpr int W2PT = HP * kHeadMaxClasses / kHeadThreads;
    float w2v[W2PT];
    {
        const auto r2 = buffer_rsrc(a.w2, (int64_t)H * O * 4);
#pragma unroll
        for (int j = 0; j < W2PT; ++j) {
            const int e = tid + kHeadThreads * j;
            w2v[j] = buffer_load1(r2, e < H * O ? e * 4 : kOutOfRange);
        }
    }
    __syncthreads();

    f32x4 acc[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) acc[g] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const float* xa = xs + (lane & 3) * I + q;
    auto reduce = [&](const f32x4 (&tb)[NB], int kb) {
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const float av = xa[kb + P * u];
#pragma unroll
            for (int g = 0; g < 4; ++g) acc[g] = mfma4(av, tb[u][g], acc[g]);
        }
    };
    // Two batches in registers: each is reduced, then refilled with the
    // batch two ahead. The loads are unconditional (past k1 they read zeros
    // without touching memory): a load under a branch would make the
    // compiler's count of outstanding loads at the join wait for the batch
    // just requested.
    int kb = k0;
    for (; kb + 2 * KB <= k1; kb += 2 * KB) {
        reduce(wv[0], kb);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < NB; ++u) wv[0][u] = load_w(kb + 2 * KB + P * u);
        __builtin_amdgcn_sched_barrier(0);
        reduce(wv[1], kb + KB);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < NB; ++u) wv[1][u] = load_w(kb + 3 * KB + P * u);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (kb < k1) {  // fewer than 2 * KB rows left, in wv[0] and maybe wv[1]
        reduce(wv[0], kb);
        if (kb + KB < k1) reduce(wv[1], kb + KB);
    }
#pragma unroll
    for (int j = 0; j < W2PT; ++j) {
        const int e = tid + kHeadThreads * j;
        if (e < H * O) w2s[e] = w2v[j];
    }
    // part (wave, parity): lane holds rows 0..3 of columns cb + g
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[((w * P + q) * kHeadRows + r) * RP + cb + g] = acc[g][r];
    __syncthreads();

    // h = relu(sum of the wave partials in wave order + b1)
#pragma unroll
    for (int j = 0; j < HPT; ++j) {
        const int e = tid + kHeadThreads * j;
        if (e >= kHeadRows * H) break;
        const int r = e / H, c = e - r * H;
        float v = red[r * RP + c];
#pragma unroll
        for (int pp = 1; pp < NPART; ++pp) v += red[(pp * kHeadRows + r) * RP + c];
        if (a.b1) v += b1v[j];
        v = fmaxf(v, 0.0f);
        hs[r * HP + c] = v;
        if (row0 + r < a.B) a.h[(int64_t)(row0 + r) * H + c] = v;
    }
    for (int e = tid; e < kHeadRows * (HP - H); e += kHeadThreads)
        hs[(e / (HP - H)) * HP + H + e % (HP - H)] = 0.0f;
    __syncthreads();

    // logits: pair (r, o) = (tid & 63) / 16, % 16; part p = tid >> 6 takes
    // hidden columns [p * HP / 8, (p + 1) * HP / 8) (h is 0 past H in hs);
    // the parts added in order
    {
        constexpr int CP = HP / kHeadWaves;
        const int pr = tid & 63, p = tid >> 6, r = pr >> 4, o = pr & 15;
        const int oc = min(o, O - 1);
        float v = 0.0f;
#pragma unroll
        for (int j = 0; j < CP; ++j) {
            const int c = p * CP + j;
            v = fmaf(hs[r * HP + c], c < H ? w2s[c * O + oc] : 0.0f, v);
        }
        red[p * 64 + pr] = v;
    }
    __syncthreads();
    if (tid < 64) {
        const int r = tid >> 4, o = tid & 15;
        if (o < O) {
            float v = red[tid];
#pragma unroll
            for (int p = 1; p < kHeadWaves; ++p) v += red[p * 64 + tid];
            if (a.b2) v += b2v;
            zs[r * kHeadMaxClasses + o] = v;
            if (row0 + r < a.B) a.z[(int64_t)(row0 + r) * O + o] = v;
        }
        // the seed, as ce_backward computes it: the row max folded from
        // class 0, the sum of expf(l - max) in class order, then
        // expf(l - max) / sum (each expf taken once). The same wave wrote
        // the logits: its LDS accesses complete in order, so no barrier.
        // all 16 slots read, the ones past O replaced by values that leave
        // the result unchanged (-inf for the max, +0 for the sum of
        // non-negative terms): no branch or wait per class
        const float* l = zs + r * kHeadMaxClasses;
        float lv[kHeadMaxClasses];
#pragma unroll
        for (int cc = 0; cc < kHeadMaxClasses; ++cc) lv[cc] = l[cc];
        float mx = lv[0];
#pragma unroll
        for (int cc = 1; cc < kHeadMaxClasses; ++cc) mx = fmaxf(mx, cc < O ? lv[cc] : -INFINITY);
        const float e = o < O ? expf(l[o] - mx) : 0.0f;
        float* es = gs + r * kHeadMaxClasses;
        es[o] = e;
        float ev[kHeadMaxClasses];
#pragma unroll
        for (int cc = 0; cc < kHeadMaxClasses; ++cc) ev[cc] = es[cc];
        float sum = 0.0f;
#pragma unroll
        for (int cc = 0; cc < kHeadMaxClasses; ++cc) sum += cc < O ? ev[cc] : 0.0f;
        float g = 0.0f;
        if (o < O && row0 + r < a.B) {
            const int64_t idx = (int64_t)(row0 + r) * O + o;
            g = (e / sum - tv) * a.inv_batch;
            a.gz[idx] = g;
        }
        es[o] = g;
    }
    __syncthreads();
    // dh = (gz . w2^T) where h > 0, classes in order
    for (int e = tid; e < kHeadRows * H; e += kHeadThreads) {
        const int r = e / H, c = e - r * H;
        if (row0 + r >= a.B) continue;
        // classes past O add fmaf(0, 0, v) = v (gs is 0 there)
        float v = 0.0f;
#pragma unroll
        for (int o = 0; o < kHeadMaxClasses; ++o)
            v = fmaf(gs[r * kHeadMaxClasses + o], o < O ? w2s[c * O + o] : 0.0f, v);
        a.dh[(int64_t)(row0 + r) * H + c] = hs[r * HP + c] > 0.0f ? v : 0.0f;
    }
}

}  // namespace
}  // namespace nrs

extern "C" {

int nrs_mlp2_forward_seed(float* h, float* z, float* gz, float* dh, const float* x,
                          const float* w1, const float* b1, const float* w2, const float* b2,
                          const float* target, int64_t batch, int64_t in_f, int64_t hidden,
                          int64_t classes) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(batch >= 0 && in_f >= 1 && hidden >= 1 && classes >= 1,
                  "mlp2 forward: bad shape (batch %lld, in %lld, hidden %lld, classes %lld)",
                  (long long)batch, (long long)in_f, (long long)hidden, (long long)classes);
    if (batch == 0) return NRS_OK;
    NRS_ARG_CHECK(h && z && gz && dh && x && w1 && w2 && target, "mlp2 forward: null pointer");
    // the outputs are written while other workgroups still read the inputs
    const size_t hb = sizeof(float) * (size_t)(batch * hidden);
    const size_t zb = sizeof(float) * (size_t)(batch * classes);
    struct Span {
        const void* p;
        size_t n;
    };
    const Span outs[] = {{h, hb}, {z, zb}, {gz, zb}, {dh, hb}};
    const Span ins[] = {{x, sizeof(float) * (size_t)(batch * in_f)},
                        {w1, sizeof(float) * (size_t)(in_f * hidden)},
                        {b1, b1 ? sizeof(float) * (size_t)hidden : 0},
                        {w2, sizeof(float) * (size_t)(hidden * classes)},
                        {b2, b2 ? sizeof(float) * (size_t)classes : 0},
                        {target, zb}};
    for (int i = 0; i < 4; ++i) {
        for (const Span& s : ins)
            NRS_ARG_CHECK(!nrs::overlaps(outs[i].p, outs[i].n, s.p, s.n),
                          "mlp2 forward: an output overlaps an input");
        for (int j = i + 1; j < 4; ++j)
            NRS_ARG_CHECK(!nrs::overlaps(outs[i].p, outs[i].n, outs[j].p, outs[j].n),
                          "mlp2 forward: outputs overlap");
    }
    const bool fused = in_f <= nrs::kHeadMaxIn && hidden <= nrs::kHeadMaxHidden &&
                       classes <= nrs::kHeadMaxClasses && batch * in_f < (int64_t(1) << 29) &&
                       in_f * hidden < (int64_t(1) << 29) && batch <= INT32_MAX;
    if (!fused) {
        // past the one-launch kernel's limits, the same quantities from three
        // launches: layer 1 with its bias and ReLU in the GEMM epilogue,
        // layer 2 with the seed (nrs_linear_cross_entropy), and dh = gz . w2^T
        // masked where h > 0 in the product's epilogue
        int rc = nrs_gemm(NRS_NN, h, x, w1, batch, hidden, in_f, 0.0f, b1,
                          (b1 ? NRS_EPI_BIAS_COL : NRS_EPI_NONE) | NRS_EPI_RELU);
        if (rc != NRS_OK) return rc;
        rc = nrs_linear_cross_entropy(z, gz, h, w2, b2, target, batch, hidden, classes);
        if (rc != NRS_OK) return rc;
        nrs::GemmCall c;
        c.layout = NRS_NT;
        c.C = dh;
        c.A = gz;
        c.B = w2;
        c.M = batch;
        c.N = hidden;
        c.K = classes;
        c.mask = h;
        return nrs::gemm_run(c);
    }
    nrs::HeadArgs a;
    a.x = x;
    a.w1 = w1;
    a.b1 = b1;
    a.w2 = w2;
    a.b2 = b2;
    a.target = target;
    a.h = h;
    a.z = z;
    a.gz = gz;
    a.dh = dh;
    a.B = (int)batch;
    a.I = (int)in_f;
    a.H = (int)hidden;
    a.O = (int)classes;
    const int64_t per = (in_f + nrs::kHeadWaves - 1) / nrs::kHeadWaves;
    a.kw = (int)((per + 3) / 4 * 4);  // a multiple of the rows one wave load covers
    a.inv_batch = 1.0f / (float)batch;
    const unsigned grid = (unsigned)((batch + nrs::kHeadRows - 1) / nrs::kHeadRows);
    // hidden columns padded to 64, 128 or 256 (w1 rows per 128-bit wave load: 4, 2, 1)
    const int hp = hidden <= 64 ? 64 : (hidden <= 128 ? 128 : 256);
    const bool fast = hidden % 4 == 0 && in_f % 4 == 0 && ((uintptr_t)x & 15) == 0 &&
                      ((uintptr_t)w1 & 15) == 0;
    using Fn = void (*)(nrs::HeadArgs);
    const bool small = in_f <= nrs::kHeadSmallIn;
    // [hp 64/128/256][fast][small]
    static const Fn kFns[3][2][2] = {
        {{nrs::mlp_head_kernel<64, false, false>, nrs::mlp_head_kernel<64, false, true>},
         {nrs::mlp_head_kernel<64, true, false>, nrs::mlp_head_kernel<64, true, true>}},
        {{nrs::mlp_head_kernel<128, false, false>, nrs::mlp_head_kernel<128, false, true>},
         {nrs::mlp_head_kernel<128, true, false>, nrs::mlp_head_kernel<128, true, true>}},
        {{nrs::mlp_head_kernel<256, false, false>, nrs::mlp_head_kernel<256, false, true>},
         {nrs::mlp_head_kernel<256, true, false>, nrs::mlp_head_kernel<256, true, true>}}};
    const int hi = hp == 64 ? 0 : (hp == 128 ? 1 : 2);
    const Fn fn = kFns[hi][fast ? 1 : 0][small ? 1 : 0];
    // the block's x rows and their zero pad in dynamic LDS, beside the static
    // LDS (at most ~54 KB): allowed up to the largest in_f once per kernel
    const size_t lds = sizeof(float) * (size_t)(nrs::kHeadRows * in_f + nrs::kHeadXPad);
    constexpr size_t kMaxDyn = sizeof(float) * (nrs::kHeadRows * nrs::kHeadMaxIn + nrs::kHeadXPad);
    static bool attr_set[12] = {};
    const int fi = hi * 4 + (fast ? 2 : 0) + (small ? 1 : 0);
    if (!attr_set[fi]) {
        hipFuncAttributes fa;
        NRS_HIP_CHECK(hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(fn)));
        NRS_ARG_CHECK(fa.sharedSizeBytes + kMaxDyn <= nrs::lds_limit(),
                      "mlp2 forward: the device's LDS is too small for this kernel");
        NRS_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxDyn));
        attr_set[fi] = true;
    }
    hipLaunchKernelGGL(fn, dim3(grid), dim3(nrs::kHeadThreads), lds, nrs::stream(), a);
    NRS_LAUNCH_CHECK("mlp2 forward");
    return NRS_OK;
}

int nrs_mlp2_backward(float* dx, float* dw1, float* db1, float* dw2, float* db2, const float* dh,
                      const float* gz, const float* x, const float* w1, const float* h,
                      int64_t batch, int64_t in_f, int64_t hidden, int64_t classes, float beta_x,
                      float beta_p) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(batch >= 0 && in_f >= 0 && hidden >= 0 && classes >= 0,
                  "mlp2 backward: negative size");
    NRS_ARG_CHECK(dw1 && dw2, "mlp2 backward: null weight gradient");
    if (batch == 0 || in_f == 0 || hidden == 0 || classes == 0) {
        // no rows (the sums are empty: beta_p * old), or a product with no
        // output rows to carry its row of sums: each layer's
        // nrs_linear_backward, which handles both
        const int rc = nrs::linear_backward(dx, dw1, db1, dh, x, w1, nullptr, batch, in_f,
                                            hidden, beta_x, beta_p, beta_p);
        if (rc != NRS_OK) return rc;
        return nrs::linear_backward(nullptr, dw2, db2, gz, h, nullptr, nullptr, batch, hidden,
                                    classes, 0.0f, beta_p, beta_p);
    }
    // dW1 = x^T . dh (+ db1 as its row of sums), dx = dh . w1^T,
    // dW2 = h^T . gz (+ db2): nrs_linear_backward's products for both layers
    nrs::GemmCall calls[3];
    int n = 0;
    nrs::GemmCall& c1 = calls[n++];
    c1.layout = NRS_TN;
    c1.C = dw1;
    c1.A = x;
    c1.B = dh;
    c1.M = in_f;
    c1.N = hidden;
    c1.K = batch;
    c1.beta = beta_p;
    c1.sum_row = db1;
    c1.sum_beta = beta_p;
    nrs::GemmCall& c2 = calls[n++];
    c2.layout = NRS_TN;
    c2.C = dw2;
    c2.A = h;
    c2.B = gz;
    c2.M = hidden;
    c2.N = classes;
    c2.K = batch;
    c2.beta = beta_p;
    c2.sum_row = db2;
    c2.sum_beta = beta_p;
    if (dx) {
        nrs::GemmCall& c3 = calls[n++];
        c3.layout = NRS_NT;
        c3.C = dx;
        c3.A = dh;
        c3.B = w1;
        c3.M = batch;
        c3.N = in_f;
        c3.K = hidden;
        c3.beta = beta_x;
    }
    return nrs::gemm_group_run(calls, n);
}

}  // extern "C"
