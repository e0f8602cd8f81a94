// Slab-resident convolution on the f32 matrix cores (v_mfma_f32_16x16x4f32).
//
// The implicit GEMM of src/cuda/nn/conv.rs:266-277 (forward) and of the
// stride-1 input gradient (conv.rs:304-312 as a convolution of the output
// gradient with flipped weights) without a column matrix and without global
// loads inside the reduction: each workgroup owns one image, a band of `band`
// consecutive output pixels and BM output channels. Per chunk of CC input
// channels it stages
//   * the input slab: every input row the band's windows touch, full padded
//     width, zero outside the image, pixel-major with the chunk's channels
//     contiguous ([row][col][CC + 4 pad]);
//   * the weight block: [BM][kh*kw][CC] (+4 pad per row), flipped and
//     channel-transposed on the fly for the input gradient;
// once into LDS, then runs the whole chunk's reduction from LDS.
//
// MFMA mapping (16x16x4): A = weights (rows = output channels), B = slab
// windows (columns = output pixels). Lane l supplies A[m = l%16][k = l/16]
// and B[k = l/16][n = l%16]; the four lane quarters q = l/16 take channel
// quarters (channel = q*CC/4 + j at step j) of the same tap, so both operands
// come from one 128-bit LDS read per four steps: the four channels are
// contiguous in both layouts, and every address offset inside the loop is
// uniform across the wavefront. Lane l's accumulator holds
// D[m = 4*(l/16) + r][n = l%16], r < 4.
//
// The summation order per output is taps outer, channels inner (the
// reference sums channel-major); results agree to f32 rounding.
#include <algorithm>

#include "conv_slab_wgrad.hpp"

namespace nrs {
namespace {

struct SlabArgs {
    const float* x;
    const float* w;
    const float* bias;
    float* out;
    int C, H, W, M, kh, kw, taps, stride, pad_h, pad_w, OW, P;
    const float* wpack;    // weights packed per (chunk, channel block) in LDS layout
    int nblk;              // output-channel blocks (gridDim.y)
    float beta;
    int vec_out;           // 128-bit output stores (P % 4 == 0, 16-byte aligned output)
    int CC, CC4;           // channels per chunk (multiple of 16) and CC / 4
    int band;              // output pixels per band
    int slab_rows, slab_w; // LDS slab rows reserved and columns
    int ps, wrow;          // LDS floats per slab pixel and per weight row
    int x_items, w_items;  // staging items per chunk: 4-channel slab pixels, weight float4s
    FastDiv div_bands, div_ow, div_psn, div_slab_w;
};


template <int WM, int WN, int MSW, int NSW>
struct SlabCfg {
    static constexpr int NT = 64 * WM * WN;
    static constexpr int BM = 16 * WM * MSW;  // output channels per workgroup
    static constexpr int BN = 16 * WN * NSW;  // output pixels per workgroup (max band)
    // staging items per thread per round: input-slab pixels (4 loads each)
    // and weight float4s; smaller for the widest tile, whose accumulators
    // and operand sets leave fewer registers
    static constexpr int SB = NSW >= 7 ? 6 : 12;
    static constexpr int WB = NSW >= 7 ? 10 : 20;
};

// The work of workgroup (bx, by) = (image * bands + band, output-channel
// block), with 64 * WM * WN threads.
template <int WM, int WN, int MSW, int NSW>
__device__ __forceinline__ void slab_block(const SlabArgs& a, int bx, int by) {
    using Cfg = SlabCfg<WM, WN, MSW, NSW>;
    extern __shared__ __attribute__((aligned(16))) float lds[];
    // the wave index is uniform; readfirstlane lets the compiler know, so
    // per-wave conditions below are scalar branches
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WM, wn = wave / WM;
    const int q = lane >> 4, l16 = lane & 15;

    uint32_t img, bi;
    fast_divmod((uint32_t)bx, a.div_bands, img, bi);
    const int m0 = by * Cfg::BM;
    const int p0 = (int)bi * a.band;
    const int p_end = min(p0 + a.band, a.P);
    const int oy_first = (int)fast_div((uint32_t)p0, a.div_ow);
    const int oy_last = (int)fast_div((uint32_t)(p_end - 1), a.div_ow);
    const int rows = (oy_last - oy_first) * a.stride + a.kh;
    const int iy0 = oy_first * a.stride - a.pad_h;
    const int HW = a.H * a.W;
    float* xs = lds;
    float* ws = lds + a.slab_rows * a.slab_w * a.ps;
    const int CQ = a.CC4;  // channels per lane quarter

    // per-lane slab offsets of this wave's pixel columns (masked pixels read
    // row 0, which is always staged)
    int poff[NSW];
#pragma unroll
    for (int t = 0; t < NSW; ++t) {
        const int p = p0 + 16 * (wn * NSW + t) + l16;
        int o = 0;
        if (p < p_end) {
            uint32_t oy, ox;
            fast_divmod((uint32_t)p, a.div_ow, oy, ox);
            o = (((int)oy - oy_first) * a.stride * a.slab_w + (int)ox * a.stride) * a.ps;
        }
        poff[t] = o + q * CQ;
    }
    int aoff[MSW];
#pragma unroll
    for (int ms = 0; ms < MSW; ++ms) aoff[ms] = (16 * (wm * MSW + ms) + l16) * a.wrow + q * CQ;

    f32x4 acc[MSW][NSW];
#pragma unroll
    for (int ms = 0; ms < MSW; ++ms)
#pragma unroll
        for (int t = 0; t < NSW; ++t) acc[ms][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // the epilogue's biases, loaded now so the stores do not wait for them
    float bias[MSW][4];
#pragma unroll
    for (int ms = 0; ms < MSW; ++ms)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int oc = m0 + 16 * (wm * MSW + ms) + 4 * q + r;
            bias[ms][r] = (a.bias && oc < a.M) ? a.bias[oc] : 0.0f;
        }

    const float* ximg = a.x + (int64_t)img * a.C * HW;
    // the image as a buffer: a load at kOutOfRange returns zero, so the
    // padding needs no select after the load (a select would make the
    // compiler wait for each item's loads before issuing the next item's)
    const auto rx = buffer_rsrc(ximg, (int64_t)a.C * HW * 4);
    for (int c0 = 0; c0 < a.C; c0 += a.CC) {
        if (c0) __syncthreads();  // the previous chunk's reads are done
        // Staging: each round issues up to Cfg::SB slab items and
        // Cfg::WB weight float4s per thread, every load of the round
        // before any LDS store, so a thread waits for global memory once per
        // round (one round for the common shapes).
        // Input slab: item = (channel quad, slab pixel), pixels fastest so
        // consecutive lanes read consecutive input columns. Weight block: a
        // straight copy of its packed LDS image.
        const auto rw = buffer_rsrc(
            a.wpack + ((int64_t)(c0 / a.CC) * a.nblk + by) * Cfg::BM * a.wrow,
            (int64_t)a.w_items * 16);
        f32x4* wdst = reinterpret_cast<f32x4*>(ws);
        const int rounds = max((a.x_items + Cfg::NT * Cfg::SB - 1) / (Cfg::NT * Cfg::SB),
                               (a.w_items + Cfg::NT * Cfg::WB - 1) / (Cfg::NT * Cfg::WB));
        for (int rd = 0; rd < rounds; ++rd) {
            const int xbase = rd * Cfg::NT * Cfg::SB, wbase = rd * Cfg::NT * Cfg::WB;
            f32x4 v[Cfg::SB], wv[Cfg::WB];
            int dst[Cfg::SB];
            const bool xrun = xbase < a.x_items, wrun = wbase < a.w_items;  // uniform
            if (xrun) {
#pragma unroll
                for (int b = 0; b < Cfg::SB; ++b) {
                    dst[b] = -1;
                    // slots past the last item are skipped (uniform condition)
                    if (xbase + b * Cfg::NT >= a.x_items) continue;
                    const int idx = xbase + tid + b * Cfg::NT;
                    uint32_t c4, pos, r, col;
                    fast_divmod((uint32_t)min(idx, a.x_items - 1), a.div_psn, c4, pos);
                    fast_divmod(pos, a.div_slab_w, r, col);
                    const bool live = (idx < a.x_items) & ((int)r < rows);
                    const int iy = iy0 + (int)r, ix = (int)col - a.pad_w;
                    const bool in =
                        live & ((unsigned)iy < (unsigned)a.H) & ((unsigned)ix < (unsigned)a.W);
                    const int c = c0 + 4 * (int)c4;
                    const int off = (c * HW + iy * a.W + ix) * 4;  // bytes
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const bool ok = in & (c + u < a.C);
                        v[b][u] = buffer_load1(rx, ok ? off + u * HW * 4 : kOutOfRange);
                    }
                    dst[b] = live ? (int)(pos * a.ps + 4 * c4) : -1;
                }
            }
            if (wrun) {
                // a load past the block returns zero (those lanes store nothing)
#pragma unroll
                for (int b = 0; b < Cfg::WB; ++b)
                    if (wbase + b * Cfg::NT < a.w_items)  // uniform
                        wv[b] = buffer_load4(rw, (wbase + tid + b * Cfg::NT) * 16);
            }
            // every load before the first LDS store (the scheduler would
            // otherwise sink some past the stores' waits: a second round
            // trip)
            __builtin_amdgcn_sched_barrier(0);
            if (xrun) {
#pragma unroll
                for (int b = 0; b < Cfg::SB; ++b)
                    if (xbase + b * Cfg::NT < a.x_items && dst[b] >= 0)
                        *reinterpret_cast<f32x4*>(xs + dst[b]) = v[b];
            }
            if (wrun) {
#pragma unroll
                for (int b = 0; b < Cfg::WB; ++b) {
                    const int e = wbase + tid + b * Cfg::NT;
                    if (e < a.w_items) wdst[e] = wv[b];
                }
            }
            // nothing outstanding at the loop edge: otherwise the compiler
            // assumes the (conditional) stores may have left loads pending
            // and waits for all of a round's slab loads before its weight
            // loads
            __builtin_amdgcn_s_waitcnt(0);
        }
        __syncthreads();

        // The reduction runs over (tap, 4-channel group) steps, two per
        // iteration on two register sets: the operands of the next step are
        // read from LDS before the current step's MFMAs issue (scheduling
        // barriers keep them there), and the sets alternate, so no register
        // copies sit between the MFMA groups. Past the last step the reads go
        // to offset 0 (in bounds) and the A operand is zeroed.
        const int steps = a.taps * (CQ / 4);
        int tap = 0, j4 = 0, i = 0, j = 0;
        f32x4 a0[MSW], b0[NSW], a1[MSW], b1[NSW];
#pragma unroll
        for (int ms = 0; ms < MSW; ++ms)
            a0[ms] = *reinterpret_cast<const f32x4*>(ws + aoff[ms]);
#pragma unroll
        for (int t = 0; t < NSW; ++t) b0[t] = *reinterpret_cast<const f32x4*>(xs + poff[t]);
        for (int it = 0; it < steps; it += 2) {
            j4 += 4;
            if (j4 == CQ) {
                j4 = 0;
                ++tap;
                if (++j == a.kw) {
                    j = 0;
                    ++i;
                }
            }
            const bool has1 = it + 1 < steps;  // uniform
            {
                const int woff = has1 ? tap * a.CC + j4 : 0;
                const int toff = has1 ? (i * a.slab_w + j) * a.ps + j4 : 0;
#pragma unroll
                for (int ms = 0; ms < MSW; ++ms)
                    a1[ms] = *reinterpret_cast<const f32x4*>(ws + aoff[ms] + woff);
#pragma unroll
                for (int t = 0; t < NSW; ++t)
                    b1[t] = *reinterpret_cast<const f32x4*>(xs + poff[t] + toff);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int ms = 0; ms < MSW; ++ms)
#pragma unroll
                    for (int t = 0; t < NSW; ++t)
                        acc[ms][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[ms][s], b0[t][s],
                                                                          acc[ms][t], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            j4 += 4;
            if (j4 == CQ) {
                j4 = 0;
                ++tap;
                if (++j == a.kw) {
                    j = 0;
                    ++i;
                }
            }
            const bool has2 = it + 2 < steps;  // uniform
            {
                const int woff = has2 ? tap * a.CC + j4 : 0;
                const int toff = has2 ? (i * a.slab_w + j) * a.ps + j4 : 0;
#pragma unroll
                for (int ms = 0; ms < MSW; ++ms)
                    a0[ms] = *reinterpret_cast<const f32x4*>(ws + aoff[ms] + woff);
#pragma unroll
                for (int t = 0; t < NSW; ++t)
                    b0[t] = *reinterpret_cast<const f32x4*>(xs + poff[t] + toff);
            }
#pragma unroll
            for (int ms = 0; ms < MSW; ++ms)
                if (!has1) a1[ms] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int ms = 0; ms < MSW; ++ms)
#pragma unroll
                    for (int t = 0; t < NSW; ++t)
                        acc[ms][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[ms][s], b1[t][s],
                                                                          acc[ms][t], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // epilogue: NCHW store, + bias, + beta * out, with non-temporal stores
    // (the output would otherwise evict the operands of the workgroups still
    // running from L2)
    float* oimg = a.out + (int64_t)img * a.M * a.P;
    if (a.vec_out) {
        // Through a per-wave LDS tile [MSW*16 channels][NSW*16 pixels]: the
        // MFMA layout holds four channels of one pixel per lane, the tile
        // gives each lane four adjacent pixels of one channel, so a wave's
        // stores are 128-bit and cover whole row segments.
        constexpr int TR = NSW * 16 + 4;   // tile row stride (floats)
        constexpr int TW = MSW * 16 * TR;  // floats per wave
        const int pw0 = p0 + 16 * wn * NSW, ocw0 = m0 + 16 * wm * MSW;
        // beta != 0: the values the stores add to, loaded now (before the
        // tile round trip) and all before any store; loaded beside each
        // store they would cost a round trip per store
        f32x4 old[MSW * NSW];
        if (a.beta != 0.0f) {  // uniform
            const auto ro = buffer_rsrc(oimg, (int64_t)a.M * a.P * 4);
#pragma unroll
            for (int k = 0; k < MSW * NSW; ++k) {
                const int e = lane + 64 * k;
                const int row = e / (NSW * 4), c4 = e - row * (NSW * 4);
                const int oc = ocw0 + row, p = pw0 + 4 * c4;
                old[k] = buffer_load4(ro, ((oc < a.M) & (p < p_end)) ? (oc * a.P + p) * 4
                                                                   : kOutOfRange);
            }
        }
        __syncthreads();                   // every wave is done with the operands
        float* tile = lds + wave * TW;
#pragma unroll
        for (int ms = 0; ms < MSW; ++ms)
#pragma unroll
            for (int t = 0; t < NSW; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    tile[(16 * ms + 4 * q + r) * TR + 16 * t + l16] = acc[ms][t][r] + bias[ms][r];
        __syncthreads();
        // (P % 4 == 0 and bands of whole float4s: a float4 never straddles
        // the band's end)
#pragma unroll
        for (int k = 0; k < MSW * NSW; ++k) {
            const int e = lane + 64 * k;
            const int row = e / (NSW * 4), c4 = e - row * (NSW * 4);
            const int oc = ocw0 + row, p = pw0 + 4 * c4;
            if (oc >= a.M || p >= p_end) continue;
            f32x4 v = *reinterpret_cast<const f32x4*>(tile + row * TR + 4 * c4);
            if (a.beta != 0.0f) v = v + a.beta * old[k];
            __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(oimg + (int64_t)oc * a.P + p));
        }
        return;
    }
    if (a.beta == 0.0f) {
#pragma unroll
        for (int ms = 0; ms < MSW; ++ms)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int oc = m0 + 16 * (wm * MSW + ms) + 4 * q + r;
                if (oc >= a.M) continue;
#pragma unroll
                for (int t = 0; t < NSW; ++t) {
                    const int p = p0 + 16 * (wn * NSW + t) + l16;
                    if (p < p_end)
                        __builtin_nontemporal_store(acc[ms][t][r] + bias[ms][r],
                                                    oimg + (int64_t)oc * a.P + p);
                }
            }
    } else {
#pragma unroll
        for (int ms = 0; ms < MSW; ++ms)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int oc = m0 + 16 * (wm * MSW + ms) + 4 * q + r;
                if (oc >= a.M) continue;
#pragma unroll
                for (int t = 0; t < NSW; ++t) {
                    const int p = p0 + 16 * (wn * NSW + t) + l16;
                    if (p >= p_end) continue;
                    float* dst = oimg + (int64_t)oc * a.P + p;
                    __builtin_nontemporal_store(acc[ms][t][r] + bias[ms][r] + a.beta * *dst, dst);
                }
            }
    }
}

// Two waves per SIMD: the LDS budget targets two workgroups per CU, and the
// 256-VGPR cap keeps the accumulators in place in VGPRs.
template <int WM, int WN, int MSW, int NSW>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(2)))
void conv_slab_kernel(SlabArgs a) {
    slab_block<WM, WN, MSW, NSW>(a, blockIdx.x, blockIdx.y);
}

// The input gradient (a flipped slab convolution, d) and the weight
// gradient (w) of one backward call in one launch: workgroups [0, nw) are
// the weight gradient's, in its (x, y, z) grid order, the rest the input
// gradient's. The weight-gradient workgroups are the longer ones and start
// first; the input-gradient workgroups fill the CU slots beside them and
// after them, where the weight gradient alone would leave one workgroup
// slot per CU idle.
template <int WM, int WN, int MSW, int NSW, bool VEC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void conv_bwd_pair_kernel(WgradArgs w, SlabArgs d, int wgx, int wgy, int nw, int dgx) {
    static_assert(WM * WN == 4, "both bodies run 256 threads");
    const int x = blockIdx.x;
    if (x < nw) {  // uniform
        const int yz = x / wgx, y = yz % wgy;
        wgrad_block<kTapw, VEC>(w, x - yz * wgx, y, yz / wgy);
    } else {
        const int e = x - nw, by = e / dgx;
        slab_block<WM, WN, MSW, NSW>(d, e - by * dgx, by);
    }
}

// Packs the weights of a slab convolution into the LDS image the kernel
// stages: packed[((chunk * nblk + blk) * BM + m) * wrow + tap * CC + c] =
// weight (m0 + m, c0 + c, tap), zero outside the tensor and in the row pad,
// with m0 = blk * BM, c0 = chunk * CC. The weight element (m, c, tap) is
// w[m][c][tap] forward and w[c][m][taps-1-tap] for the input gradient.
__global__ __launch_bounds__(256) void pack_slab_weights_kernel(
    float* __restrict__ packed, const float* __restrict__ w, int C, int M, int taps, int CC,
    int BM, int nblk, int wrow, int flip, int total) {
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
        const int row = e / wrow, col = e - row * wrow;
        const int cb = row / BM, m = row - cb * BM;
        const int chunk = cb / nblk, blk = cb - chunk * nblk;
        const int tap = col / CC, c = col - tap * CC;
        const int mg = blk * BM + m, cg = chunk * CC + c;
        float v = 0.0f;
        if (tap < taps && mg < M && cg < C)
            v = flip ? w[((int64_t)cg * M + mg) * taps + (taps - 1 - tap)]
                     : w[((int64_t)mg * C + cg) * taps + tap];
        packed[e] = v;
    }
}

// LDS of one workgroup: at most 160 KiB (gfx950's whole LDS), and no more
// than the device allows.
int64_t lds_budget() { return (int64_t)std::min<size_t>(160 * 1024, lds_limit()); }

int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// Launch geometry of one configuration: bands, slab size, channel chunk and
// LDS bytes (0 when the configuration cannot take the convolution).
struct SlabPlan {
    int64_t band = 0, nb = 0, slab_rows = 0, slab_w = 0, CC = 0;
    size_t lds = 0;
};

template <int WM, int WN, int MSW, int NSW>
SlabPlan plan_slab(const SlabConv& s, int64_t lds_cap) {
    using Cfg = SlabCfg<WM, WN, MSW, NSW>;
    SlabPlan pl;
    const int64_t P = (int64_t)s.OH * s.OW, taps = (int64_t)s.kh * s.kw;
    const int64_t bands = (P + Cfg::BN - 1) / Cfg::BN;
    pl.band = std::min<int64_t>(Cfg::BN, round_up((P + bands - 1) / bands, 16));
    pl.nb = (P + pl.band - 1) / pl.band;
    // input rows the windows of one band touch: exact maximum over the bands
    // when there are few, else the bound for a band starting anywhere
    int64_t out_rows = std::min<int64_t>(s.OH, (pl.band - 1 + s.OW - 1) / s.OW + 1);
    if (pl.nb <= 4096) {
        out_rows = 0;
        for (int64_t b = 0; b < pl.nb; ++b) {
            const int64_t p0 = b * pl.band, p1 = std::min(p0 + pl.band, P) - 1;
            out_rows = std::max(out_rows, p1 / s.OW - p0 / s.OW + 1);
        }
    }
    pl.slab_rows = (out_rows - 1) * s.stride + s.kh;
    pl.slab_w = (int64_t)(s.OW - 1) * s.stride + s.kw;
    // the largest channel chunk (multiple of 16) whose slab and weights fit
    // in lds_cap bytes
    auto bytes = [&](int64_t cc) {
        return 4 * (pl.slab_rows * pl.slab_w * (cc + 4) + Cfg::BM * (taps * cc + 4));
    };
    int64_t CC = round_up(s.C, 16);
    while (CC > 16 && bytes(CC) > lds_cap) CC -= 16;
    const int64_t grid_x = s.N * pl.nb, grid_y = (s.M + Cfg::BM - 1) / Cfg::BM;
    // (the weight block's byte offsets must fit the buffer loads' 31 bits)
    if (bytes(CC) > lds_budget() || grid_x > INT32_MAX || grid_y > 65535 ||
        pl.slab_rows * pl.slab_w * (CC / 4) > INT32_MAX / 2 ||
        Cfg::BM * (taps * CC + 4) > INT32_MAX / 4)
        return SlabPlan{};
    pl.CC = CC;
    // the epilogue's per-wave tiles reuse the same LDS
    const int64_t tile = (int64_t)(Cfg::NT / 64) * (16 * MSW) * (16 * NSW + 4) * 4;
    pl.lds = (size_t)std::max<int64_t>(bytes(CC), tile);
    if ((int64_t)pl.lds > lds_budget()) return SlabPlan{};
    return pl;
}

// Packs the weights (one launch) and fills the kernel arguments and grid.
template <int WM, int WN, int MSW, int NSW>
int prepare_slab(const SlabConv& s, const SlabPlan& pl, SlabArgs& a, unsigned& gx,
                 unsigned& gy) {
    using Cfg = SlabCfg<WM, WN, MSW, NSW>;
    const int64_t P = (int64_t)s.OH * s.OW, taps = (int64_t)s.kh * s.kw;
    a.x = s.x;
    a.w = s.w;
    a.bias = s.bias;
    a.out = s.out;
    a.C = s.C;
    a.H = s.H;
    a.W = s.W;
    a.M = s.M;
    a.kh = s.kh;
    a.kw = s.kw;
    a.taps = (int)taps;
    a.stride = s.stride;
    a.pad_h = s.pad_h;
    a.pad_w = s.pad_w;
    a.OW = s.OW;
    a.P = (int)P;
    const int64_t nblk = (s.M + Cfg::BM - 1) / Cfg::BM, nchunk = (s.C + pl.CC - 1) / pl.CC;
    const int64_t wrow = taps * pl.CC + 4, packed_n = nchunk * nblk * Cfg::BM * wrow;
    if (packed_n > INT32_MAX) return kSlabUnsupported;
    float* packed = workspace(sizeof(float) * (size_t)packed_n, 4);
    if (!packed) return NRS_ERR_ALLOC;
    hipLaunchKernelGGL(pack_slab_weights_kernel,
                       dim3((unsigned)std::min<int64_t>((packed_n + 255) / 256, 4096)), dim3(256),
                       0, stream(), packed, s.w, s.C, s.M, (int)taps, (int)pl.CC, Cfg::BM,
                       (int)nblk, (int)wrow, s.flip ? 1 : 0, (int)packed_n);
    NRS_LAUNCH_CHECK("conv2d (slab weight pack)");
    a.wpack = packed;
    a.nblk = (int)nblk;
    a.beta = s.beta;
    a.vec_out = (P % 4 == 0 && ((uintptr_t)s.out & 15) == 0) ? 1 : 0;
    a.CC = (int)pl.CC;
    a.CC4 = (int)(pl.CC / 4);
    a.band = (int)pl.band;
    a.slab_rows = (int)pl.slab_rows;
    a.slab_w = (int)pl.slab_w;
    a.ps = (int)(pl.CC + 4);
    a.wrow = (int)(taps * pl.CC + 4);
    a.x_items = (int)(pl.slab_rows * pl.slab_w * (pl.CC / 4));
    a.w_items = (int)(Cfg::BM * wrow / 4);
    a.div_bands = make_fastdiv((uint32_t)pl.nb);
    a.div_ow = make_fastdiv((uint32_t)s.OW);
    a.div_psn = make_fastdiv((uint32_t)(pl.slab_rows * pl.slab_w));
    a.div_slab_w = make_fastdiv((uint32_t)pl.slab_w);
    gx = (unsigned)(s.N * pl.nb);
    gy = (unsigned)((s.M + Cfg::BM - 1) / Cfg::BM);
    return NRS_OK;
}

// Raises a kernel's dynamic LDS limit to the LDS budget, once per process.
template <typename F>
int allow_full_lds(F fn, bool& done) {
    if (!done) {
        NRS_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                          hipFuncAttributeMaxDynamicSharedMemorySize,
                                          (int)lds_budget()));
        done = true;
    }
    return NRS_OK;
}

template <int WM, int WN, int MSW, int NSW>
int launch_slab(const SlabConv& s, const SlabPlan& pl) {
    using Cfg = SlabCfg<WM, WN, MSW, NSW>;
    SlabArgs a;
    unsigned gx = 0, gy = 0;
    const int rc = prepare_slab<WM, WN, MSW, NSW>(s, pl, a, gx, gy);
    if (rc) return rc;
    auto fn = conv_slab_kernel<WM, WN, MSW, NSW>;
    static bool attr_set = false;
    if (allow_full_lds(fn, attr_set)) return NRS_ERR_HIP;
    hipLaunchKernelGGL(fn, dim3(gx, gy), dim3(Cfg::NT), pl.lds, stream(), a);
    NRS_LAUNCH_CHECK("conv2d (slab)");
    return NRS_OK;
}

template <int WM, int WN, int MSW, int NSW>
int launch_pair(const SlabConv& s, const SlabPlan& pl, const WgradPlan& wp) {
    SlabArgs a;
    unsigned gx = 0, gy = 0;
    const int rc = prepare_slab<WM, WN, MSW, NSW>(s, pl, a, gx, gy);
    if (rc) return rc;
    const int64_t nw = (int64_t)wp.gx * wp.gy * wp.gz, total = nw + (int64_t)gx * gy;
    auto fn = wp.a.vec_g ? conv_bwd_pair_kernel<WM, WN, MSW, NSW, true>
                         : conv_bwd_pair_kernel<WM, WN, MSW, NSW, false>;
    static bool attr_set[2] = {false, false};
    if (allow_full_lds(fn, attr_set[wp.a.vec_g])) return NRS_ERR_HIP;
    hipLaunchKernelGGL(fn, dim3((unsigned)total), dim3(256), std::max(pl.lds, wp.lds), stream(),
                       wp.a, a, (int)wp.gx, (int)wp.gy, (int)nw, (int)gx);
    NRS_LAUNCH_CHECK("conv2d backward (slab pair)");
    return NRS_OK;
}

// Slab configuration for a convolution: 0, 1, 2 for 64 x 112, 32 x 128 and
// 16 x 128 tiles (channels x pixels), -1 when none fits. Takes the widest
// whose LDS lets two workgroups share a CU (one stages while the other
// computes), else the widest that fits at all. With `chunked`, a tile may
// stage its channels in smaller chunks to fit half the LDS: beside the
// weight gradient's workgroups (one per CU) that keeps the input gradient to
// one round of wide tiles instead of two rounds of narrow ones.
int pick_slab(const SlabConv& s, SlabPlan& pl, bool chunked = false) {
    const size_t kHalf = (size_t)lds_budget() / 2;
    const int64_t cap = chunked ? (int64_t)kHalf : lds_budget();
    const SlabPlan p64 = s.M >= 48 ? plan_slab<4, 1, 1, 7>(s, cap) : SlabPlan{};
    const SlabPlan p32 = s.M > 16 ? plan_slab<2, 2, 1, 4>(s, cap) : SlabPlan{};
    const SlabPlan p16 = plan_slab<1, 4, 1, 2>(s, cap);
    const SlabPlan* plans[3] = {&p64, &p32, &p16};
    for (int k = 0; k < 3; ++k)
        if (plans[k]->lds && plans[k]->lds <= kHalf) return pl = *plans[k], k;
    for (int k = 0; k < 3; ++k)
        if (plans[k]->lds) return pl = *plans[k], k;
    return -1;
}

// The shape checks every slab convolution needs before planning.
bool slab_shape_ok(const SlabConv& s) {
    if (s.C <= 0 || s.kh <= 0 || s.kw <= 0 || s.stride <= 0) return false;
    // staged channel chunks must be at least a quarter real channels
    if (round_up(s.C, 16) > 4 * (int64_t)s.C) return false;
    // an image's byte offsets (input and output) fit the buffer loads' 31-bit
    // range
    return (int64_t)s.C * s.H * s.W <= INT32_MAX / 4 && (int64_t)s.M * s.OH * s.OW <= INT32_MAX / 4;
}

}  // namespace

int slab_conv(const SlabConv& s) {
    if (s.N == 0 || s.M == 0 || s.OH == 0 || s.OW == 0) return NRS_OK;
    if (!slab_shape_ok(s)) return kSlabUnsupported;
    SlabPlan pl;
    switch (pick_slab(s, pl)) {
        case 0: return launch_slab<4, 1, 1, 7>(s, pl);
        case 1: return launch_slab<2, 2, 1, 4>(s, pl);
        case 2: return launch_slab<1, 4, 1, 2>(s, pl);
        default: return kSlabUnsupported;
    }
}

int slab_backward_pair(const SlabConv& d, const SlabWgrad& w) {
    if (d.N == 0 || d.M == 0 || d.OH == 0 || d.OW == 0 || !slab_shape_ok(d))
        return kSlabUnsupported;
    SlabPlan pl;
    const int cfg = pick_slab(d, pl, true);
    if (cfg < 0) return kSlabUnsupported;
    const int64_t bm = cfg == 0 ? 64 : (cfg == 1 ? 32 : 16);
    const int64_t d_wgs = d.N * pl.nb * ((d.M + bm - 1) / bm);
    WgradPlan wp;
    int rc = plan_slab_wgrad(w, wp);
    if (rc) return rc;
    if ((int64_t)wp.gx * wp.gy * wp.gz + d_wgs > INT32_MAX || d.N * pl.nb > INT32_MAX)
        return kSlabUnsupported;
    switch (cfg) {
        case 0: rc = launch_pair<4, 1, 1, 7>(d, pl, wp); break;
        case 1: rc = launch_pair<2, 2, 1, 4>(d, pl, wp); break;
        default: rc = launch_pair<1, 4, 1, 2>(d, pl, wp); break;
    }
    if (rc) return rc;
    return slab_wgrad_sum(w, wp);
}

}  // namespace nrs
