// Image-resident convolution on the f32 matrix cores (v_mfma_f32_16x16x4f32)
// for small stride-1 3x3 layers: the implicit GEMM of nn::conv2d's forward
// (src/cuda/nn/conv.rs:266-277) and of its stride-1 input gradient
// (conv.rs:304-312, read as a convolution of the output gradient with the
// flipped, channel-transposed weights).
//
// One workgroup owns one image and MB output channels. It stages, once:
//   * the whole zero-padded image as rows of 16 floats, channel planes of
//     R = H + 2*PAD rows. Each thread copies whole rows: the source row is
//     read with 64-bit loads (32-bit for odd widths) and written with the
//     halo zeros as four 128-bit LDS stores, so no zero-fill pass, no barrier
//     before the copy and no per-element index arithmetic;
//   * the block's weights in their natural order [MB][C*9] (+4 pad per row),
//     or flipped and transposed for the input gradient;
// then reduces K = C*9 entirely from LDS.
//
// Reduction order: k = c*9 + tap, the weights' own order. Lane quarter q
// (lanes 16q..16q+15) takes the channels [q*C/4, (q+1)*C/4), so at step s
// of a quarter its k is q*(C/4)*9 + s:
//   * A (weights, rows = output channels): four consecutive steps are four
//     consecutive floats of the lane's weight row: one 128-bit LDS read per
//     four MFMAs;
//   * B (image, columns = output pixels): a pixel tile is one output row
//     (lane = column; lanes past the row's width compute values that are
//     never stored), so step s reads plane q*C/4 + s/9 at a compile-time
//     offset (s%9)/3 rows and s%3 columns from the lane's pixel. The
//     quarters' planes start 16 floats apart modulo 64, so the 64 lanes of a
//     read hit 64 different banks.
// Lane l's accumulator holds D[m = 4*(l/16) + r][column l%16 of its row].
#include <algorithm>

#include "buffer_ops.hpp"
#include "conv_slab.hpp"
#include "fastdiv.hpp"

namespace nrs {
namespace {

constexpr int kImgRow = 16;   // floats per staged row (padded width <= 16)
constexpr int kImgRpt = 4;    // staged rows per thread per round

struct ImgArgs {
    const float* x;     // NCHW [N][C][H][W]
    const float* w;     // [M][C][3][3], or [C][M][3][3] with FLIP
    const float* bias;  // [M] or null
    float* out;         // NCHW [N][M][OH][OW]
    int C, H, W, M, OH, OW, P;
    int R;              // staged rows per plane (H + 2*PAD)
    int plane;          // floats per staged plane (>= R*16 + 2, a multiple of 4)
    int qpitch;         // floats per lane quarter's C/4 planes (16 mod 64)
    int wrow;           // floats per staged weight row (C*9 + 4)
    int vec_out;        // 128-bit output stores (P % 4 == 0, 16-byte aligned output)
    float beta;
    FastDiv div_r;      // staged rows per plane
    FastDiv div_cq;     // channels per lane quarter
    FastDiv div_wq;     // forward: float4s per weight row (C*9/4)
    FastDiv div_p4;     // float4s per output channel plane
};

template <int PAD, int MB, int NSW, bool FLIP>
__global__ __launch_bounds__(256) void conv_img_kernel(ImgArgs a) {
    constexpr int OB = MB / 16, TSTEP = 4 / OB;
    constexpr int SEG = kImgRow - 2 * PAD;  // source floats loaded per staged row
    static_assert(MB == 16 || MB == 32, "16 or 32 output channels per workgroup");
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, l16 = lane & 15;
    const int img = blockIdx.x, m0 = blockIdx.y * MB;
    const int C = a.C, CQ = C >> 2;  // channels per lane quarter (multiple of 4)
    float* xs = lds;
    float* ws = lds + 4 * a.qpitch;

    // ---- staging: the image rows, then the weight block. A round issues
    // all of its loads before its first LDS store, so the common shapes pay
    // one memory round trip.
    {
        const float* ximg = a.x + (int64_t)img * C * a.H * a.W;
        const auto rx = buffer_rsrc(ximg, (int64_t)C * a.H * a.W * 4);
        const bool pairs = ((a.W & 1) == 0) && ((((uintptr_t)ximg) & 7) == 0);
        constexpr int WB = FLIP ? 4 : 9;  // weight items per thread in the first round
        const int wq = MB * (C * 9 / 4);  // forward: float4s of the [MB][C*9] block
        const int wpairs = MB * C;        // input gradient: (m, c) pairs of 9 taps
        // weight items [w0, w0 + WB*256): forward rows are straight 128-bit
        // copies; the input gradient gathers, per (row m, channel c), the 9
        // taps of w[c][m0 + m] (w is [C][M][3][3]) reversed
        auto load_weights = [&](int w0, f32x4 (&wv)[FLIP ? 1 : WB], float (&wf)[FLIP ? WB : 1][9],
                                int (&wd)[WB]) {
            if constexpr (!FLIP) {
                const float* wsrc = a.w + (int64_t)m0 * C * 9;
                const auto rw = buffer_rsrc(wsrc, (int64_t)max(0, min(MB, a.M - m0)) * C * 9 * 4);
#pragma unroll
                for (int b = 0; b < WB; ++b) {
                    const int e = w0 + b * 256 + tid;
                    wv[b] = buffer_load4(rw, e < wq ? e * 16 : kOutOfRange);
                }
#pragma unroll
                for (int b = 0; b < WB; ++b) {
                    const int e = w0 + b * 256 + tid;
                    // row m = e / (C*9/4): staged at m*wrow + 4*(e - m*C*9/4)
                    const int m = (int)fast_div((uint32_t)e, a.div_wq);
                    wd[b] = e < wq ? 4 * e + 4 * m : -1;
                }
            } else {
                const auto rw = buffer_rsrc(a.w, (int64_t)C * a.M * 9 * 4);
#pragma unroll
                for (int b = 0; b < WB; ++b) {
                    const int e = w0 + b * 256 + tid;
                    const int m = e % MB, c = e / MB;
                    const bool ok = (e < wpairs) & (m0 + m < a.M);
                    const int src = ((c * a.M + m0 + m) * 9) * 4;
#pragma unroll
                    for (int t = 0; t < 9; ++t)
                        wf[b][t] = buffer_load1(rw, ok ? src + t * 4 : kOutOfRange);
                    wd[b] = e < wpairs ? m * a.wrow + c * 9 : -1;
                }
            }
        };
        auto store_weights = [&](const f32x4 (&wv)[FLIP ? 1 : WB],
                                 const float (&wf)[FLIP ? WB : 1][9], const int (&wd)[WB]) {
#pragma unroll
            for (int b = 0; b < WB; ++b) {
                if (wd[b] < 0) continue;
                if constexpr (!FLIP) {
                    *reinterpret_cast<f32x4*>(ws + wd[b]) = wv[b];
                } else {
#pragma unroll
                    for (int t = 0; t < 9; ++t) ws[wd[b] + t] = wf[b][8 - t];
                }
            }
        };
        // staged row `row` = c*R + y holds source row y - PAD of channel c
        // (zeros outside the image) at columns PAD .. PAD+W-1; loads past the
        // row's W floats are masked to the buffer's zero
        const int nrows = C * a.R;
        for (int r0 = 0; r0 < nrows; r0 += 256 * kImgRpt) {
            float v[kImgRpt][SEG];
#pragma unroll
            for (int i = 0; i < kImgRpt; ++i) {
                if (r0 + i * 256 >= nrows) break;  // uniform
                const int row = r0 + i * 256 + tid;
                const uint32_t c = fast_div((uint32_t)row, a.div_r);
                const int y = row - (int)c * a.R - PAD;
                const bool ok = (row < nrows) & ((unsigned)y < (unsigned)a.H);
                const int src = ((int)c * a.H + y) * a.W;
                if (pairs) {
#pragma unroll
                    for (int k = 0; k < SEG / 2; ++k) {
                        const f32x2 t =
                            buffer_load2(rx, (ok & (2 * k < a.W)) ? (src + 2 * k) * 4 : kOutOfRange);
                        v[i][2 * k] = t[0];
                        v[i][2 * k + 1] = t[1];
                    }
                } else {
#pragma unroll
                    for (int k = 0; k < SEG; ++k)
                        v[i][k] = buffer_load1(rx, (ok & (k < a.W)) ? (src + k) * 4 : kOutOfRange);
                }
            }
            f32x4 wv[FLIP ? 1 : WB];
            float wf[FLIP ? WB : 1][9];
            int wd[WB];
            if (r0 == 0) load_weights(0, wv, wf, wd);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < kImgRpt; ++i) {
                if (r0 + i * 256 >= nrows) break;  // uniform
                const int row = r0 + i * 256 + tid;
                if (row >= nrows) continue;
                const uint32_t c = fast_div((uint32_t)row, a.div_r);
                const int y = row - (int)c * a.R;
                uint32_t qq, cl;
                fast_divmod(c, a.div_cq, qq, cl);
                float* dst = xs + (int)qq * a.qpitch + (int)cl * a.plane + y * kImgRow;
                // columns PAD .. PAD+SEG-1 carry the loaded floats (zero past
                // W), the rest is halo
                float r[kImgRow];
#pragma unroll
                for (int j = 0; j < kImgRow; ++j) r[j] = (j >= PAD && j < PAD + SEG) ? v[i][j - PAD] : 0.0f;
#pragma unroll
                for (int j = 0; j < kImgRow; j += 4)
                    *reinterpret_cast<f32x4*>(dst + j) = f32x4{r[j], r[j + 1], r[j + 2], r[j + 3]};
            }
            if (r0 == 0) store_weights(wv, wf, wd);
            __builtin_amdgcn_s_waitcnt(0);
        }
        const int witems = FLIP ? wpairs : wq;
        for (int w0 = WB * 256; w0 < witems; w0 += WB * 256) {
            f32x4 wv[FLIP ? 1 : WB];
            float wf[FLIP ? WB : 1][9];
            int wd[WB];
            load_weights(w0, wv, wf, wd);
            __builtin_amdgcn_sched_barrier(0);
            store_weights(wv, wf, wd);
            __builtin_amdgcn_s_waitcnt(0);
        }
    }

    const int ob = wave % OB, t0 = wave / OB;
    const int mrow = 16 * ob + l16;  // this lane's A row (weights)
    float bias[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = m0 + 16 * ob + 4 * q + r;
        bias[r] = (a.bias && m < a.M) ? a.bias[m] : 0.0f;
    }
    // per-tile LDS offset of this lane's pixel (quarter's first plane); tiles
    // past the last output row repeat it (their results are not stored)
    int pb[NSW];
#pragma unroll
    for (int k = 0; k < NSW; ++k) {
        const int oy = min(t0 + k * TSTEP, a.OH - 1);
        pb[k] = q * a.qpitch + oy * kImgRow + l16;
    }
    __syncthreads();

    f32x4 acc[NSW];
#pragma unroll
    for (int k = 0; k < NSW; ++k) acc[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const float* wrow = ws + mrow * a.wrow + q * CQ * 9;
    // groups of four channels: 36 steps, 9 MFMA groups of four steps
    for (int cg = 0; cg < CQ; cg += 4) {
        const float* wg = wrow + cg * 9;
        const int cbase = cg * a.plane;
        f32x4 af = *reinterpret_cast<const f32x4*>(wg);
        float bf[NSW][4];
#pragma unroll
        for (int k = 0; k < NSW; ++k)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                bf[k][r] = xs[pb[k] + cbase + (r / 9) * a.plane + ((r % 9) / 3) * kImgRow + r % 3];
#pragma unroll
        for (int u = 0; u < 9; ++u) {
            f32x4 an;
            float bn[NSW][4];
            if (u + 1 < 9) {
                an = *reinterpret_cast<const f32x4*>(wg + 4 * (u + 1));
#pragma unroll
                for (int k = 0; k < NSW; ++k)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int s = 4 * (u + 1) + r;
                        bn[k][r] =
                            xs[pb[k] + cbase + (s / 9) * a.plane + ((s % 9) / 3) * kImgRow + s % 3];
                    }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int k = 0; k < NSW; ++k)
                    acc[k] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[r], bf[k][r], acc[k], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (u + 1 < 9) {
                af = an;
#pragma unroll
                for (int k = 0; k < NSW; ++k)
#pragma unroll
                    for (int r = 0; r < 4; ++r) bf[k][r] = bn[k][r];
            }
        }
    }

    // epilogue: the block's [MB][P] output goes through LDS (the image
    // planes are no longer needed), so it leaves as 128-bit stores of whole
    // contiguous channel rows; + bias on the way in, + beta * old on the way
    // out (the old values are loaded before the tile round trip)
    float* oimg = a.out + (int64_t)img * a.M * a.P;
    const int mvalid = min(MB, a.M - m0);
    const int P4 = a.P / 4;
    const bool vec = a.vec_out != 0;
    constexpr int OV = 8;  // 128-bit outputs per thread held for beta
    f32x4 old[OV];
    if (a.beta != 0.0f && vec) {  // uniform
#pragma unroll
        for (int u = 0; u < OV; ++u) {
            const int e = u * 256 + tid;
            const int m = (int)fast_div((uint32_t)e, a.div_p4), p4 = e - m * P4;
            old[u] = (m < mvalid) ? *reinterpret_cast<const f32x4*>(oimg + (int64_t)(m0 + m) * a.P + 4 * p4)
                                  : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    __syncthreads();  // every wave is done with the image planes
    float* ot = lds;  // [MB][P]
    if (l16 < a.OW) {
#pragma unroll
        for (int k = 0; k < NSW; ++k) {
            const int oy = t0 + k * TSTEP;
            if (oy < a.OH) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = 16 * ob + 4 * q + r;
                    ot[m * a.P + oy * a.OW + l16] = acc[k][r] + bias[r];
                }
            }
        }
    }
    __syncthreads();
    if (vec) {
        const int total = mvalid * P4;
        for (int u0 = 0; u0 < total; u0 += OV * 256) {
#pragma unroll
            for (int u = 0; u < OV; ++u) {
                const int e = u0 + u * 256 + tid;
                if (e >= total) continue;
                const int m = (int)fast_div((uint32_t)e, a.div_p4), p4 = e - m * P4;
                f32x4 v = *reinterpret_cast<const f32x4*>(ot + m * a.P + 4 * p4);
                if (a.beta != 0.0f) {
                    const f32x4 o = u0 == 0 ? old[u]
                                            : *reinterpret_cast<const f32x4*>(
                                                  oimg + (int64_t)(m0 + m) * a.P + 4 * p4);
                    v = v + a.beta * o;
                }
                __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(
                                                   oimg + (int64_t)(m0 + m) * a.P + 4 * p4));
            }
        }
    } else {
        const int total = mvalid * a.P;
        for (int e = tid; e < total; e += 256) {
            const int m = e / a.P, p = e - m * a.P;
            float v = ot[m * a.P + p];
            float* dstp = oimg + (int64_t)(m0 + m) * a.P + p;
            if (a.beta != 0.0f) v = v + a.beta * *dstp;
            *dstp = v;
        }
    }
}

// LDS of one workgroup: at most 160 KiB (gfx950's whole LDS), and no more
// than the device allows.
size_t img_lds_budget() { return std::min<size_t>(160 * 1024, lds_limit()); }

template <int PAD, int MB, int NSW, bool FLIP>
int launch_img(const ImgArgs& a, int64_t N, size_t lds) {
    auto fn = conv_img_kernel<PAD, MB, NSW, FLIP>;
    static bool attr_set = false;
    if (!attr_set) {
        NRS_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                          hipFuncAttributeMaxDynamicSharedMemorySize,
                                          (int)img_lds_budget()));
        attr_set = true;
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)N, (unsigned)((a.M + MB - 1) / MB)), dim3(256), lds,
                       stream(), a);
    NRS_LAUNCH_CHECK("conv2d (image-resident)");
    return NRS_OK;
}

template <int PAD, bool FLIP>
int launch_img_pad(const ImgArgs& a, int64_t N, size_t lds, int MB, int NSW) {
    if (MB == 32) return NSW == 7 ? launch_img<PAD, 32, 7, FLIP>(a, N, lds)
                                  : launch_img<PAD, 32, 4, FLIP>(a, N, lds);
    return NSW == 7 ? launch_img<PAD, 16, 7, FLIP>(a, N, lds)
                    : launch_img<PAD, 16, 4, FLIP>(a, N, lds);
}

}  // namespace

int img_conv(const SlabConv& s) {
    // 3x3, stride 1, channel count a multiple of 16, rows of at most 16
    // staged floats, a handful of output rows per wave
    if (s.kh != 3 || s.kw != 3 || s.stride != 1 || s.pad_h != s.pad_w || s.pad_h > 2 ||
        s.C % 16 != 0 || s.C <= 0 || s.M <= 0 || s.N <= 0 || s.N > 65535)
        return kSlabUnsupported;
    const int pad = s.pad_h;
    const int R = s.H + 2 * pad, Wp = s.W + 2 * pad;
    if (Wp > kImgRow || s.OH != R - 2 || s.OW != Wp - 2 || s.OH < 1 || s.OW < 1)
        return kSlabUnsupported;
    const int P = s.OH * s.OW;
    // 32 output channels per workgroup when that leaves at least one
    // workgroup per CU, else 16
    const int MB = (s.M % 32 == 0 && s.N * (s.M / 32) >= num_cus()) ? 32 : 16;
    const int per_wave = (s.OH + (4 / (MB / 16)) - 1) / (4 / (MB / 16));
    const int NSW = per_wave <= 4 ? 4 : (per_wave <= 7 ? 7 : 0);
    if (NSW == 0) return kSlabUnsupported;
    // planes of R rows (+2 floats read by the lanes past the last column of
    // the last row); the four lane quarters' plane blocks start 16 floats
    // apart modulo 64 so a quarter-per-16-banks read has no conflicts
    const int CQ = s.C / 4;
    const int plane = (R * kImgRow + 2 + 3) / 4 * 4;
    const int qpitch = CQ * plane + (((16 - CQ * plane) % 64) + 64) % 64;
    const int wrow = s.C * 9 + 4;
    // (the epilogue's [MB][P] output tile reuses the image planes)
    const size_t lds = 4 * std::max((size_t)4 * qpitch + (size_t)MB * wrow, (size_t)MB * P);
    if (lds > img_lds_budget()) return kSlabUnsupported;
    ImgArgs a;
    a.x = s.x;
    a.w = s.w;
    a.bias = s.bias;
    a.out = s.out;
    a.C = s.C;
    a.H = s.H;
    a.W = s.W;
    a.M = s.M;
    a.OH = s.OH;
    a.OW = s.OW;
    a.P = P;
    a.R = R;
    a.plane = plane;
    a.qpitch = qpitch;
    a.wrow = wrow;
    a.beta = s.beta;
    a.vec_out = (P % 4 == 0 && ((uintptr_t)s.out & 15) == 0) ? 1 : 0;
    a.div_r = make_fastdiv((uint32_t)R);
    a.div_cq = make_fastdiv((uint32_t)CQ);
    a.div_wq = make_fastdiv((uint32_t)(s.C * 9 / 4));
    a.div_p4 = make_fastdiv((uint32_t)std::max(1, P / 4));
    switch (pad) {
        case 0: return s.flip ? launch_img_pad<0, true>(a, s.N, lds, MB, NSW)
                              : launch_img_pad<0, false>(a, s.N, lds, MB, NSW);
        case 1: return s.flip ? launch_img_pad<1, true>(a, s.N, lds, MB, NSW)
                              : launch_img_pad<1, false>(a, s.N, lds, MB, NSW);
        default: return s.flip ? launch_img_pad<2, true>(a, s.N, lds, MB, NSW)
                               : launch_img_pad<2, false>(a, s.N, lds, MB, NSW);
    }
}

}  // namespace nrs
