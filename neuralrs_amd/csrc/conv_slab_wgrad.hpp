// Device side of the slab weight gradient (host side in conv_slab_wgrad.hip):
// its arguments, its launch plan and the per-workgroup body, shared by the
// standalone kernel and the backward pair kernel of conv_slab.hip.
//
// Slab-resident weight and bias gradient of a convolution on the f32 matrix
// cores (v_mfma_f32_16x16x4f32): the split-K weight-gradient GEMM of
// src/cuda/nn/conv.rs:314-320 (dW = G . cols^T, K = N*out_h*out_w) and the
// bias gradient of conv.rs:322, without the column matrix.
//
//   dW[m, c, i, j] += sum over (n, oy, ox) of g[n, m, oy, ox] * x[n, c, oy*s - pad + i, ox*s - pad + j]
//   db[m]          += sum over (n, oy, ox) of g[n, m, oy, ox]
//
// A workgroup owns one image's band of output rows (a K slice), 16 input
// channels, a group of TAPW taps and 64 output channels. It stages into LDS
//   * the gradient rows of its 64 channels, pixels contiguous ([m][KP + 4]),
//   * a table of each band pixel's offset inside the input slab,
//   * the input slab of its 16 channels (every input row the band's windows
//     touch, full padded width, zero outside the image),
// and runs the band's whole reduction from LDS. Wave w owns output channels
// 16w..16w+15 (A rows); each of its TAPW subtiles is one tap with the lanes
// on the 16 channels (B columns), so a lane's slab address is its channel's
// plane plus the tap offset plus the pixel offset, which is the same for the
// sixteen lanes of a quarter. Lane quarter q takes pixels q*KP/4 + j at step
// j, so both the A operand and the pixel offsets come from 128-bit LDS reads
// per four steps. Each slice writes its sums to a partial buffer; a second
// kernel adds the slices in a fixed order (deterministic, no atomics).
#pragma once

#include "buffer_ops.hpp"
#include "conv_slab.hpp"

namespace nrs {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kWgM = 64;  // output channels per workgroup: 4 waves x 16
constexpr int kWgC = 16;  // input channels per workgroup
constexpr int kWgStageG = 16;  // gradient float4 items per thread per staging round
constexpr int kWgStageX = 16;  // input-slab floats per thread per staging round

struct WgradArgs {
    const float* x;
    const float* g;
    float* part_w;  // [slice][M][taps][C]
    float* part_b;  // [slice][M]
    int C, H, W, M, kh, kw, taps, stride, pad_h, pad_w, OH, OW;
    int band_rows, bands, ntg;  // output rows per band, bands per image, tap groups
    int KP, KQ, KPP;            // padded band pixels, KP / 4, gradient row stride in LDS
    int slab_rows, slab_w, CS;  // input slab rows, columns and channel stride in LDS
    int vec_g;                  // gradient rows 16-byte aligned (128-bit staging loads)
    FastDiv div_bands, div_ntg, div_kp4, div_srw, div_slab_w, div_ow, div_kw;
};

constexpr int kTapw = 9;  // taps per workgroup (a 3x3 kernel in one group)

// The work of workgroup (bx, by, bz) = (slice, channel part * tap groups +
// tap group, output-channel block); 256 threads, with the LDS bytes of the
// launch plan below. VEC (= a.vec_g) stages the gradient rows with 128-bit
// loads; it is a template parameter so that each form is one straight run
// of loads (a branch between the two forms made the compiler wait for the
// loads at the join).
template <int TAPW, bool VEC>
__device__ __forceinline__ void wgrad_block(const WgradArgs& a, int bx, int by, int bz) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, l16 = lane & 15;

    uint32_t img, band, cp, tg;
    fast_divmod((uint32_t)bx, a.div_bands, img, band);
    fast_divmod((uint32_t)by, a.div_ntg, cp, tg);
    const int slice = bx;
    const int c0 = (int)cp * kWgC, t0 = (int)tg * TAPW, m0 = bz * kWgM;
    const int oy0 = (int)band * a.band_rows;
    const int rows_b = min(a.band_rows, a.OH - oy0);
    const int PB = rows_b * a.OW;
    const int iy0 = oy0 * a.stride - a.pad_h;
    const int srw = a.slab_rows * a.slab_w;

    float* gs = lds;                                   // [kWgM][KPP]
    int* pofs = reinterpret_cast<int*>(gs + kWgM * a.KPP);  // [KP]
    float* xs = reinterpret_cast<float*>(pofs + a.KP);      // [kWgC][CS]

    // Staging, in rounds that issue every load before any LDS store (one
    // memory round trip per round, one round for the common shapes):
    //  * gradient rows: the band's pixels are contiguous in each channel
    //    plane; item = (channel, pixel quad), one 128-bit load when the rows
    //    are 16-byte aligned (vec_g), else four masked loads; pixels past the
    //    band are zero;
    //  * input slab of the 16 channels: one float per item, zero outside the
    //    image.
    const float* gimg = a.g + ((int64_t)img * a.M + m0) * a.OH * a.OW + (int64_t)oy0 * a.OW;
    const int KP4 = a.KP >> 2, g_items = kWgM * KP4;
    const float* ximg = a.x + ((int64_t)img * a.C + c0) * a.H * a.W;
    // both as buffers: a load at kOutOfRange returns zero, so masked items
    // need no select after the load (which would make the compiler wait for
    // each item's load before issuing the next)
    const auto rg = buffer_rsrc(gimg, (int64_t)kWgM * a.OH * a.OW * 4);
    const auto rx = buffer_rsrc(ximg, (int64_t)kWgC * a.H * a.W * 4);
    const int x_items = kWgC * srw;
    const int rows_in = (rows_b - 1) * a.stride + a.kh;
    const int rounds = max((g_items + 256 * kWgStageG - 1) / (256 * kWgStageG),
                           (x_items + 256 * kWgStageX - 1) / (256 * kWgStageX));
    for (int rd = 0; rd < rounds; ++rd) {
        const int gbase = rd * 256 * kWgStageG, xbase = rd * 256 * kWgStageX;
        f32x4 gv[kWgStageG];
        float xv[kWgStageX];
        int gdst[kWgStageG], xdst[kWgStageX], goff[kWgStageG], glen[kWgStageG], xoff[kWgStageX];
        // addresses first, then every load of the round in straight-line
        // code (no per-item branch between two load forms), so a thread
        // issues them all before its first wait
#pragma unroll
        for (int b = 0; b < kWgStageG; ++b) {
            gdst[b] = -1;
            goff[b] = kOutOfRange;
            glen[b] = 0;
            if (gbase + b * 256 >= g_items) continue;  // uniform
            const int e = gbase + b * 256 + tid;
            uint32_t m, k4;
            fast_divmod((uint32_t)min(e, g_items - 1), a.div_kp4, m, k4);
            const int kk = 4 * (int)k4;
            const bool row = (e < g_items) & (m0 + (int)m < a.M);
            goff[b] = ((int)m * a.OH * a.OW + kk) * 4;  // bytes
            glen[b] = row ? PB - kk : 0;  // gradient floats from kk on (<= 0: none)
            gdst[b] = e < g_items ? (int)m * a.KPP + kk : -1;
        }
#pragma unroll
        for (int b = 0; b < kWgStageX; ++b) {
            xdst[b] = -1;
            xoff[b] = kOutOfRange;
            if (xbase + b * 256 >= x_items) continue;  // uniform
            const int e = xbase + b * 256 + tid;
            uint32_t c, pos, r, col;
            fast_divmod((uint32_t)min(e, x_items - 1), a.div_srw, c, pos);
            fast_divmod(pos, a.div_slab_w, r, col);
            const int iy = iy0 + (int)r, ix = (int)col - a.pad_w;
            const bool ok = (e < x_items) & ((int)r < rows_in) & (c0 + (int)c < a.C) &
                            ((unsigned)iy < (unsigned)a.H) & ((unsigned)ix < (unsigned)a.W);
            xoff[b] = ok ? (((int)c * a.H + iy) * a.W + ix) * 4 : kOutOfRange;
            xdst[b] = e < x_items ? (int)c * a.CS + (int)pos : -1;
        }
        if constexpr (VEC) {  // rows of whole float4s
#pragma unroll
            for (int b = 0; b < kWgStageG; ++b)
                if (gbase + b * 256 < g_items)
                    gv[b] = buffer_load4(rg, glen[b] > 0 ? goff[b] : kOutOfRange);
        } else {
#pragma unroll
            for (int b = 0; b < kWgStageG; ++b)
                if (gbase + b * 256 < g_items)
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        gv[b][u] = buffer_load1(rg, u < glen[b] ? goff[b] + 4 * u : kOutOfRange);
        }
#pragma unroll
        for (int b = 0; b < kWgStageX; ++b)
            if (xbase + b * 256 < x_items) xv[b] = buffer_load1(rx, xoff[b]);
        // every load before the first LDS store (the scheduler would
        // otherwise sink some past the stores' waits: a second round trip)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b < kWgStageG; ++b)
            if (gdst[b] >= 0) *reinterpret_cast<f32x4*>(gs + gdst[b]) = gv[b];
#pragma unroll
        for (int b = 0; b < kWgStageX; ++b)
            if (xdst[b] >= 0) xs[xdst[b]] = xv[b];
        // nothing outstanding at the loop edge (else the compiler waits for
        // the whole previous batch before the next round's first load)
        __builtin_amdgcn_s_waitcnt(0);
    }
    // slab offset of each band pixel (0 for the padding pixels, whose
    // gradient is zero)
    for (int kk = tid; kk < a.KP; kk += 256) {
        int o = 0;
        if (kk < PB) {
            uint32_t oy, ox;
            fast_divmod((uint32_t)kk, a.div_ow, oy, ox);
            o = (int)oy * a.stride * a.slab_w + (int)ox * a.stride;
        }
        pofs[kk] = o;
    }
    __syncthreads();

    // lane's B base per tap subtile: its channel's plane + the tap offset
    int bb[TAPW];
#pragma unroll
    for (int t = 0; t < TAPW; ++t) {
        const int tap = min(t0 + t, a.taps - 1);
        uint32_t ti, tj;
        fast_divmod((uint32_t)tap, a.div_kw, ti, tj);
        bb[t] = l16 * a.CS + (int)ti * a.slab_w + (int)tj;
    }
    const int aoff = (16 * wave + l16) * a.KPP + q * a.KQ;
    const int poff = q * a.KQ;
    f32x4 acc[TAPW];
#pragma unroll
    for (int t = 0; t < TAPW; ++t) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // Software-pipelined: the B values of the next step (and the pixel
    // offsets and A quad of the next group of four) are read from LDS
    // before this step's MFMAs issue; with one wave per SIMD nothing else
    // hides the LDS latency. Scheduling barriers keep the reads ahead. The
    // four steps of a group alternate between two B register sets, so the
    // first set is current again at the next group.
    i32x4 po = *reinterpret_cast<const i32x4*>(pofs + poff);
    f32x4 av = *reinterpret_cast<const f32x4*>(gs + aoff);
    // two B register sets, alternating over the (unrolled) steps, so no
    // copies sit between the MFMA groups
    float bset[2][TAPW];
#pragma unroll
    for (int t = 0; t < TAPW; ++t) bset[0][t] = xs[bb[t] + po[0]];
    for (int j = 0; j < a.KQ; j += 4) {
        const int jn = j + 4 < a.KQ ? j + 4 : j;  // the last group re-reads itself (unused)
        const i32x4 pon = *reinterpret_cast<const i32x4*>(pofs + poff + jn);
        const f32x4 avn = *reinterpret_cast<const f32x4*>(gs + aoff + jn);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int cur = s & 1, nxt = cur ^ 1;
            const int pn = s < 3 ? po[s + 1] : pon[0];
#pragma unroll
            for (int t = 0; t < TAPW; ++t) bset[nxt][t] = xs[bb[t] + pn];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < TAPW; ++t)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[s], bset[cur][t], acc[t], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        po = pon;
        av = avn;
    }

    // partial sums: lane holds D[m = 4q + r][channel l16] of each tap subtile
    const int c = c0 + l16;
#pragma unroll
    for (int t = 0; t < TAPW; ++t) {
        const int tap = t0 + t;
        if (tap >= a.taps || c >= a.C) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + 16 * wave + 4 * q + r;
            if (m < a.M)
                a.part_w[(((int64_t)slice * a.M + m) * a.taps + tap) * a.C + c] = acc[t][r];
        }
    }
    // bias: the first channel part and tap group of each slice sums the
    // gradient rows; thread (m, quarter) adds a quarter of the pixels, the
    // quarters are combined by a fixed butterfly
    if (a.part_b && cp == 0 && tg == 0) {
        const int m = tid >> 2, qq = tid & 3;
        const float* row = gs + m * a.KPP + qq * a.KQ;
        float s = 0.0f;
        for (int k = 0; k < a.KQ; k += 4) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(row + k);
            s += (v[0] + v[1]) + (v[2] + v[3]);
        }
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        if (qq == 0 && m0 + m < a.M) a.part_b[(int64_t)slice * a.M + m0 + m] = s;
    }
}

// Launch plan of one weight gradient: arguments (partials in the workspace),
// grid and LDS bytes.
struct WgradPlan {
    WgradArgs a;
    unsigned gx = 0, gy = 0, gz = 0;
    size_t lds = 0;
    int slices = 0;
    int64_t nw = 0;  // weight partials per slice (M * taps * C)
};

// Fills the plan and reserves the partials; kSlabUnsupported (nothing
// reserved or launched) for shapes outside the kernel's limits.
int plan_slab_wgrad(const SlabWgrad& s, WgradPlan& p);

// The fixed-order sum of a planned gradient's partials into dw (and db).
int slab_wgrad_sum(const SlabWgrad& s, const WgradPlan& p);

}  // namespace nrs
