// Batched products of small matrices on the f32 matrix cores
// (v_mfma_f32_32x32x2f32): the per-item bmm of src/cuda/graph/bmm.rs:12-56
// (forward NN, grad_a NT, grad_b TN) for items of at most 128x128 outputs
// and K <= 128, e.g. attention's per-head Q.K^T, P.V and their gradients.
//
// These products are short: ~17 MB of traffic and ~1.7 us of f32
// matrix-core work over the whole chip, and a memory round trip under that
// load costs microseconds. Measured on MI355X, one round trip per wave beats
// every staged or pipelined form (LDS staging, phased loads with two phases
// in flight, K split over waves), so the kernel is built around it:
//  * a wave owns one 32-row block and JB 32-column blocks of an item and
//    issues every load of its fragments at once: an operand whose reduction
//    dim is contiguous in memory as 128-bit buffer loads, the other kind
//    four bytes per lane (a half-wave reads one 128-byte row segment);
//    the MFMA chain then consumes them in issue order;
//  * the output is written with non-temporal stores: the 16.8 MB score
//    matrices of attention would otherwise evict the operands from L2
//    (Q.K^T: 8.8 -> 6.9 us);
//  * reduction-dim padding (k >= K) and rows or columns past M and N read
//    zero through the buffer bounds; only rows < M and columns < N are
//    stored.
//
// MFMA mapping: lane half h takes k = 8g + 4h + p (p = 0..3), so one 128-bit
// fragment load feeds four MFMAs; accumulator element e holds row
// 8*(e/4) + 4h + e%4, column lane%32 of the block.
#include "buffer_ops.hpp"
#include "gemm_call.hpp"

namespace nrs {
namespace {

typedef float f32x16v __attribute__((ext_vector_type(16)));

constexpr int kSmallMax = 128;  // M, N and K limits of an item

struct SmallArgs {
    const float* A;
    const float* B;
    float* C;
    int64_t sA, sB, sC;  // item strides (elements)
    int M, N, K;
    int NJ;              // waves per row block (ceil(column blocks / JB))
    int waves;           // waves per item (row blocks * NJ)
    int wg_per_item;
    float beta;
};

// Fragment g of an operand for the lane's row r (m or n): k = 8g + 4h .. +3.
// KC: stored [rows][K] (reduction contiguous), else [K][rows].
template <bool KC>
__device__ __forceinline__ f32x4 fragment(__amdgpu_buffer_rsrc_t rs, int r, int R, int K, int g,
                                          int h) {
    const int k = 8 * g + 4 * h;
    if (KC) return buffer_load4(rs, ((r < R) & (k < K)) ? (r * K + k) * 4 : kOutOfRange);
    f32x4 v;
#pragma unroll
    for (int p = 0; p < 4; ++p)
        v[p] = buffer_load1(rs, ((r < R) & (k + p < K)) ? ((k + p) * R + r) * 4 : kOutOfRange);
    return v;
}

// One workgroup `wg` (of batch * wg_per_item) of the product described by a.
// ACC (beta != 0): the C values the product adds to are loaded with the
// fragments, before the MFMA chain, so their wait hides behind it (loading
// them in the epilogue made every store wait for a round trip, and for the
// stores before it).
template <bool AK, bool BKC, int G, int JB, bool ACC>
__device__ __forceinline__ void bmm_small_block(const SmallArgs& a, int wg) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    const int item = wg / a.wg_per_item;
    const int wi = (wg - item * a.wg_per_item) * 4 + wave;
    if (wi >= a.waves) return;  // wave-uniform; no barriers follow
    const int bm = wi / a.NJ, bn0 = (wi - bm * a.NJ) * JB;
    const int m = 32 * bm + l32;
    const auto ra = buffer_rsrc(a.A + item * a.sA, (int64_t)a.M * a.K * 4);
    const auto rb = buffer_rsrc(a.B + item * a.sB, (int64_t)a.N * a.K * 4);

    f32x4 af[G], bf[JB][G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        af[g] = fragment<AK>(ra, m, a.M, a.K, g, h);
#pragma unroll
        for (int j = 0; j < JB; ++j)
            bf[j][g] = fragment<BKC>(rb, 32 * (bn0 + j) + l32, a.N, a.K, g, h);
    }
    float* c = a.C + item * a.sC;
    const int row0 = 32 * bm + 4 * h;
    f32x16v old[JB];
    if constexpr (ACC) {
        const auto rc = buffer_rsrc(c, (int64_t)a.M * a.N * 4);
#pragma unroll
        for (int j = 0; j < JB; ++j) {
            const int n = 32 * (bn0 + j) + l32;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = row0 + 8 * (e >> 2) + (e & 3);
                old[j][e] = buffer_load1(rc, ((row < a.M) & (n < a.N)) ? (row * a.N + n) * 4
                                                                      : kOutOfRange);
            }
        }
    }
    // keep the loads ahead of the MFMA chain (left alone, the scheduler
    // interleaves them to save registers, which costs a round trip each)
    __builtin_amdgcn_sched_barrier(0);
    // every MFMA chain before any store: vmcnt counts stores too, so a wait
    // for a fragment issued after a store would also wait for the store
    f32x16v acc[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) {
        acc[j] = f32x16v{};
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int p = 0; p < 4; ++p)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[g][p], bf[j][g][p], acc[j], 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < JB; ++j) {
        const int n = 32 * (bn0 + j) + l32;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int row = row0 + 8 * (e >> 2) + (e & 3);
            const float v = ACC ? acc[j][e] + a.beta * old[j][e] : acc[j][e];
            if (row < a.M && n < a.N) __builtin_nontemporal_store(v, c + (int64_t)row * a.N + n);
        }
    }
}

template <bool AK, bool BKC, int G, int JB, bool ACC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void bmm_small_kernel(SmallArgs a) {
    bmm_small_block<AK, BKC, G, JB, ACC>(a, blockIdx.x);
}

// Both gradients of one bmm in one launch: the first product (NT, or NN
// with BKCA = false) takes workgroups [0, wg_a), the second (TN) the rest.
// The launch is paid once and the second product's first workgroups start
// while the first product's last ones drain. (Interleaving the two in
// proportion to their counts measured slower on attention's gradients:
// 27.7 vs 26.3 us for both pairs.)
template <bool BKCA, int GA, int JBA, int GB, bool ACC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void bmm_small_pair_kernel(SmallArgs ga, SmallArgs gb, int wg_a) {
    const int x = blockIdx.x;
    if (x < wg_a)  // uniform
        bmm_small_block<true, BKCA, GA, JBA, ACC>(ga, x);
    else
        bmm_small_block<false, false, GB, 1, ACC>(gb, x - wg_a);
}

template <bool AK, bool BKC, int JB, bool ACC>
void* pick_g(int G) {
    return G <= 4   ? reinterpret_cast<void*>(bmm_small_kernel<AK, BKC, 4, JB, ACC>)
           : G <= 8 ? reinterpret_cast<void*>(bmm_small_kernel<AK, BKC, 8, JB, ACC>)
                    : reinterpret_cast<void*>(bmm_small_kernel<AK, BKC, 16, JB, ACC>);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

namespace {

// Validates a small-item product and fills its kernel arguments (G, JB:
// k-groups and column blocks per wave); kBmmUnsupported when it does not
// qualify (anything unusual, including invalid arguments, which gemm_run
// reports, goes to the general path).
int small_args(const GemmCall& c, SmallArgs& a, int& G, int& JB) {
    const int64_t M = c.M, N = c.N, K = c.K, batch = c.batch;
    if (c.layout < NRS_NN || c.layout > NRS_TN || !c.A || !c.B || !c.C || c.amode != OP_DENSE ||
        c.bmode != OP_DENSE || c.nchw_P != 0 || c.epi != NRS_EPI_NONE)
        return kBmmUnsupported;
    if (M < 1 || N < 1 || K < 1 || M > kSmallMax || N > kSmallMax || K > kSmallMax || batch < 1)
        return kBmmUnsupported;
    const bool AK = c.layout != NRS_TN, BKC = c.layout == NRS_NT;
    // 128-bit fragment loads need 16-byte aligned rows of whole float4s
    if (AK && (!aligned16(c.A) || c.sA % 4 || K % 4)) return kBmmUnsupported;
    if (BKC && (!aligned16(c.B) || c.sB % 4 || K % 4)) return kBmmUnsupported;
    const int MB = (int)((M + 31) / 32), NB = (int)((N + 31) / 32);
    // two column blocks per wave for NT (its A fragments are then loaded
    // once for both): measured 6.9 vs 7.2 us on attention's Q.K^T
    JB = (c.layout == NRS_NT && NB >= 2) ? 2 : 1;
    G = (int)((K + 7) / 8);
    a.A = c.A;
    a.B = c.B;
    a.C = c.C;
    a.sA = c.sA;
    a.sB = c.sB;
    a.sC = c.sC;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.NJ = (NB + JB - 1) / JB;
    a.waves = MB * a.NJ;
    a.wg_per_item = (a.waves + 3) / 4;
    a.beta = c.beta;
    if (batch * a.wg_per_item > INT32_MAX) return kBmmUnsupported;
    return NRS_OK;
}

int g_index(int G) { return G <= 4 ? 0 : (G <= 8 ? 1 : 2); }

template <bool BKCA, int GA, int JBA>
void* pick_pair_b(int GB, bool acc) {
    switch (g_index(GB)) {
        case 0: return acc ? reinterpret_cast<void*>(bmm_small_pair_kernel<BKCA, GA, JBA, 4, true>)
                           : reinterpret_cast<void*>(bmm_small_pair_kernel<BKCA, GA, JBA, 4, false>);
        case 1: return acc ? reinterpret_cast<void*>(bmm_small_pair_kernel<BKCA, GA, JBA, 8, true>)
                           : reinterpret_cast<void*>(bmm_small_pair_kernel<BKCA, GA, JBA, 8, false>);
        default: return acc ? reinterpret_cast<void*>(bmm_small_pair_kernel<BKCA, GA, JBA, 16, true>)
                           : reinterpret_cast<void*>(bmm_small_pair_kernel<BKCA, GA, JBA, 16, false>);
    }
}

template <bool BKCA, int JBA>
void* pick_pair(int GA, int GB, bool acc) {
    switch (g_index(GA)) {
        case 0: return pick_pair_b<BKCA, 4, JBA>(GB, acc);
        case 1: return pick_pair_b<BKCA, 8, JBA>(GB, acc);
        default: return pick_pair_b<BKCA, 16, JBA>(GB, acc);
    }
}

}  // namespace

int bmm_small(const GemmCall& c) {
    SmallArgs a;
    int G = 0, JB = 1;
    const int rc = small_args(c, a, G, JB);
    if (rc) return rc;
    const bool acc = c.beta != 0.0f;
    void* fn;
    switch (c.layout) {
        case NRS_NN:
            fn = acc ? pick_g<true, false, 1, true>(G) : pick_g<true, false, 1, false>(G);
            break;
        case NRS_NT:
            fn = JB == 2 ? (acc ? pick_g<true, true, 2, true>(G) : pick_g<true, true, 2, false>(G))
                         : (acc ? pick_g<true, true, 1, true>(G) : pick_g<true, true, 1, false>(G));
            break;
        default:
            fn = acc ? pick_g<false, false, 1, true>(G) : pick_g<false, false, 1, false>(G);
            break;
    }
    hipLaunchKernelGGL(reinterpret_cast<void (*)(SmallArgs)>(fn),
                       dim3((unsigned)(c.batch * a.wg_per_item)), dim3(256), 0, stream(), a);
    NRS_LAUNCH_CHECK("bmm (small items)");
    return NRS_OK;
}

int bmm_small_pair(const GemmCall& ga, const GemmCall& gb) {
    if ((ga.layout != NRS_NT && ga.layout != NRS_NN) || gb.layout != NRS_TN || ga.beta != gb.beta)
        return kBmmUnsupported;
    SmallArgs a, b;
    int GA = 0, JBA = 1, GB = 0, JBB = 1;
    if (small_args(ga, a, GA, JBA) || small_args(gb, b, GB, JBB)) return kBmmUnsupported;
    const int64_t wg_a = ga.batch * a.wg_per_item, wg_b = gb.batch * b.wg_per_item;
    if (wg_a + wg_b > INT32_MAX) return kBmmUnsupported;
    const bool acc = ga.beta != 0.0f;
    void* fn = ga.layout == NRS_NN ? pick_pair<false, 1>(GA, GB, acc)
               : JBA == 2          ? pick_pair<true, 2>(GA, GB, acc)
                                   : pick_pair<true, 1>(GA, GB, acc);
    hipLaunchKernelGGL(reinterpret_cast<void (*)(SmallArgs, SmallArgs, int)>(fn),
                       dim3((unsigned)(wg_a + wg_b)), dim3(256), 0, stream(), a, b, (int)wg_a);
    NRS_LAUNCH_CHECK("bmm backward (small items)");
    return NRS_OK;
}

}  // namespace nrs
