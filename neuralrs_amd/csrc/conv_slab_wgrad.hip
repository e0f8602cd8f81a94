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
#include <algorithm>

#include "conv_slab.hpp"

namespace nrs {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
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

template <int TAPW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void conv_slab_wgrad_kernel(WgradArgs a) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, l16 = lane & 15;

    uint32_t img, band, cp, tg;
    fast_divmod(blockIdx.x, a.div_bands, img, band);
    fast_divmod(blockIdx.y, a.div_ntg, cp, tg);
    const int slice = blockIdx.x;
    const int c0 = (int)cp * kWgC, t0 = (int)tg * TAPW, m0 = blockIdx.z * kWgM;
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
    const int x_items = kWgC * srw;
    const int rows_in = (rows_b - 1) * a.stride + a.kh;
    const int rounds = max((g_items + 256 * kWgStageG - 1) / (256 * kWgStageG),
                           (x_items + 256 * kWgStageX - 1) / (256 * kWgStageX));
    for (int rd = 0; rd < rounds; ++rd) {
        const int gbase = rd * 256 * kWgStageG, xbase = rd * 256 * kWgStageX;
        f32x4 gv[kWgStageG];
        float xv[kWgStageX];
        int gdst[kWgStageG], xdst[kWgStageX];
#pragma unroll
        for (int b = 0; b < kWgStageG; ++b) {
            gdst[b] = -1;
            if (gbase + b * 256 >= g_items) continue;  // uniform
            const int e = gbase + b * 256 + tid;
            uint32_t m, k4;
            fast_divmod((uint32_t)min(e, g_items - 1), a.div_kp4, m, k4);
            const int kk = 4 * (int)k4;
            const bool row = (e < g_items) & (m0 + (int)m < a.M);
            const float* src = gimg + (int64_t)m * a.OH * a.OW + kk;
            if (a.vec_g) {
                const bool ok = row & (kk < PB);
                gv[b] = *reinterpret_cast<const f32x4*>(ok ? src : gimg);
                if (!ok) gv[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const bool ok = row & (kk + u < PB);
                    const float t = *(ok ? src + u : gimg);
                    gv[b][u] = ok ? t : 0.0f;
                }
            }
            gdst[b] = e < g_items ? (int)m * a.KPP + kk : -1;
        }
#pragma unroll
        for (int b = 0; b < kWgStageX; ++b) {
            xdst[b] = -1;
            if (xbase + b * 256 >= x_items) continue;  // uniform
            const int e = xbase + b * 256 + tid;
            uint32_t c, pos, r, col;
            fast_divmod((uint32_t)min(e, x_items - 1), a.div_srw, c, pos);
            fast_divmod(pos, a.div_slab_w, r, col);
            const int iy = iy0 + (int)r, ix = (int)col - a.pad_w;
            const bool ok = (e < x_items) & ((int)r < rows_in) & (c0 + (int)c < a.C) &
                            ((unsigned)iy < (unsigned)a.H) & ((unsigned)ix < (unsigned)a.W);
            const float t = ximg[ok ? ((int64_t)c * a.H + iy) * a.W + ix : 0];
            xv[b] = ok ? t : 0.0f;
            xdst[b] = e < x_items ? (int)c * a.CS + (int)pos : -1;
        }
#pragma unroll
        for (int b = 0; b < kWgStageG; ++b)
            if (gdst[b] >= 0) *reinterpret_cast<f32x4*>(gs + gdst[b]) = gv[b];
#pragma unroll
        for (int b = 0; b < kWgStageX; ++b)
            if (xdst[b] >= 0) xs[xdst[b]] = xv[b];
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

// dw[m][c][tap] += sum over slices of part_w[slice][m][tap][c] and
// db[m] += sum over slices of part_b[slice][m]: the slices are split into
// kSumGroups contiguous groups summed in parallel (ascending within a group),
// then the group sums are added in group order, so the result is
// deterministic. A thread issues the loads of up to kSumBatch slices (in
// runs of 8, as many runs as its group needs) before adding any, so a group
// of that size costs one memory round trip.
constexpr int kSumGroups = 16, kSumBatch = 32;

__global__ __launch_bounds__(64 * kSumGroups) void wgrad_sum_kernel(
    float* __restrict__ dw, float* __restrict__ db, const float* __restrict__ part_w,
    const float* __restrict__ part_b, int slices, int M, int C, int taps) {
    __shared__ float red[kSumGroups][64];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int nw = dw ? M * taps * C : 0, total = nw + (db ? M : 0);
    const int per = (slices + kSumGroups - 1) / kSumGroups;
    const int s0 = min(slices, ty * per), s1 = min(slices, s0 + per);
    for (int base = blockIdx.x * 64; base < total; base += gridDim.x * 64) {
        const int e = base + tx;
        const bool is_w = e < nw;
        const float* part = is_w ? part_w + e : part_b + (e - nw);
        const int64_t stride = is_w ? nw : M;
        float v = 0.0f;
        if (e < total) {
            for (int s = s0; s < s1; s += kSumBatch) {
                float t[kSumBatch];
#pragma unroll
                for (int b = 0; b < kSumBatch; b += 8) {
                    if (s + b < s1) {  // uniform over the wave (one slice group)
#pragma unroll
                        for (int u = b; u < b + 8; ++u)
                            t[u] = part[(int64_t)min(s + u, s1 - 1) * stride];
                    } else {
#pragma unroll
                        for (int u = b; u < b + 8; ++u) t[u] = 0.0f;
                    }
                }
#pragma unroll
                for (int u = 0; u < kSumBatch; ++u) v += s + u < s1 ? t[u] : 0.0f;
            }
        }
        red[ty][tx] = v;
        __syncthreads();
        if (ty == 0 && e < total) {
            float r = red[0][tx];
#pragma unroll
            for (int y = 1; y < kSumGroups; ++y) r += red[y][tx];
            float* dst;
            if (is_w) {
                const int c = e % C, mt = e / C, tap = mt % taps, m = mt / taps;
                dst = dw + ((int64_t)m * C + c) * taps + tap;
            } else {
                dst = db + (e - nw);
            }
            *dst = r + *dst;
        }
        __syncthreads();
    }
}

constexpr int kLdsBytes = 160 * 1024;
constexpr int kTapw = 9;  // taps per workgroup (a 3x3 kernel in one group)

}  // namespace

int slab_wgrad(const SlabWgrad& s) {
    if (!s.dw) return kSlabUnsupported;  // a bias-only gradient needs no matrix cores
    if (s.N == 0 || s.M == 0 || s.OH == 0 || s.OW == 0) return kSlabUnsupported;
    if (s.C <= 0 || s.kh <= 0 || s.kw <= 0 || s.stride <= 0) return kSlabUnsupported;
    const int64_t taps = (int64_t)s.kh * s.kw;
    // one 16-channel part per workgroup: mostly-empty parts waste the matrix
    // cores, and taps beyond one group multiply the slab staging
    if (s.C < 8 || taps > 2 * kTapw) return kSlabUnsupported;
    const int64_t slab_w = (int64_t)(s.OW - 1) * s.stride + s.kw;
    // the largest band of output rows whose tiles fit the LDS
    auto lds_bytes = [&](int64_t band_rows, int64_t& KP, int64_t& CS, int64_t& slab_rows) {
        KP = (band_rows * s.OW + 15) / 16 * 16;
        slab_rows = (band_rows - 1) * s.stride + s.kh;
        CS = (slab_rows * slab_w) | 1;
        return 4 * (kWgM * (KP + 4) + KP + kWgC * CS);
    };
    int64_t band_rows = s.OH, KP = 0, CS = 0, slab_rows = 0;
    while (band_rows > 1 && lds_bytes(band_rows, KP, CS, slab_rows) > kLdsBytes) --band_rows;
    if (lds_bytes(band_rows, KP, CS, slab_rows) > kLdsBytes) return kSlabUnsupported;
    const int64_t bands = (s.OH + band_rows - 1) / band_rows;
    const int64_t slices = s.N * bands;
    const int64_t cparts = (s.C + kWgC - 1) / kWgC, ntg = (taps + kTapw - 1) / kTapw;
    const int64_t mblocks = (s.M + kWgM - 1) / kWgM;
    const int64_t nw = (int64_t)s.M * taps * s.C;
    if (slices > INT32_MAX || cparts * ntg > 65535 || mblocks > 65535 ||
        slices * (nw + s.M) > ((int64_t)1 << 31) || (int64_t)s.C * s.H * s.W > INT32_MAX ||
        (int64_t)s.M * s.OH * s.OW > INT32_MAX || nw + s.M > INT32_MAX)
        return kSlabUnsupported;

    float* part = workspace(sizeof(float) * (size_t)(slices * (nw + s.M)), 3);
    if (!part) return NRS_ERR_ALLOC;
    WgradArgs a;
    a.x = s.x;
    a.g = s.g;
    a.part_w = part;
    a.part_b = s.db ? part + slices * nw : nullptr;
    a.C = s.C;
    a.H = s.H;
    a.W = s.W;
    a.M = s.M;
    a.kh = s.kh;
    a.kw = s.kw;
    a.taps = (int)taps;
    a.stride = s.stride;
    a.pad_h = s.pad;
    a.pad_w = s.pad;
    a.OH = s.OH;
    a.OW = s.OW;
    a.band_rows = (int)band_rows;
    a.bands = (int)bands;
    a.ntg = (int)ntg;
    a.KP = (int)KP;
    a.KQ = (int)(KP / 4);
    a.KPP = (int)(KP + 4);
    a.slab_rows = (int)slab_rows;
    a.slab_w = (int)slab_w;
    a.CS = (int)CS;
    a.div_bands = make_fastdiv((uint32_t)bands);
    a.div_ntg = make_fastdiv((uint32_t)ntg);
    a.div_kp4 = make_fastdiv((uint32_t)(KP / 4));
    // 16-byte aligned gradient rows: every band starts on a float4
    a.vec_g = ((int64_t)s.OH * s.OW % 4 == 0 && band_rows * s.OW % 4 == 0 &&
               ((uintptr_t)s.g & 15) == 0) ? 1 : 0;
    a.div_srw = make_fastdiv((uint32_t)(slab_rows * slab_w));
    a.div_slab_w = make_fastdiv((uint32_t)slab_w);
    a.div_ow = make_fastdiv((uint32_t)s.OW);
    a.div_kw = make_fastdiv((uint32_t)s.kw);

    const size_t lds = (size_t)lds_bytes(band_rows, KP, CS, slab_rows);
    auto fn = conv_slab_wgrad_kernel<kTapw>;
    static bool attr_set = false;
    if (!attr_set) {
        NRS_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes));
        attr_set = true;
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)slices, (unsigned)(cparts * ntg), (unsigned)mblocks),
                       dim3(256), lds, stream(), a);
    NRS_LAUNCH_CHECK("conv2d weight gradient (slab)");
    // dW and (when requested) dB from the partials
    return wgrad_partial_sum(s.dw, s.db, part, part + slices * nw, (int)slices, s.M, s.C,
                             (int)taps);
}

int wgrad_partial_sum(float* dw, float* db, const float* part_w, const float* part_b, int slices,
                      int M, int C, int taps) {
    const int64_t total = (dw ? (int64_t)M * taps * C : 0) + (db ? M : 0);
    if (total == 0) return NRS_OK;
    hipLaunchKernelGGL(wgrad_sum_kernel, dim3((unsigned)((total + 63) / 64)),
                       dim3(64 * kSumGroups), 0, stream(), dw, db, part_w, part_b, slices, M, C,
                       taps);
    NRS_LAUNCH_CHECK("conv2d weight gradient (sum)");
    return NRS_OK;
}

}  // namespace nrs
