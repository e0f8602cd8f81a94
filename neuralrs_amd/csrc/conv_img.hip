// Image-resident convolution on the f32 matrix cores (v_mfma_f32_16x16x4f32)
// for small stride-1 3x3 layers: the implicit GEMM of nn::conv2d's forward
// (src/cuda/nn/conv.rs:266-277) and of its stride-1 input gradient
// (conv.rs:304-312, read as a convolution of the output gradient with the
// flipped, channel-transposed weights).
//
// One workgroup owns one image and MB output channels. It stages, once:
//   * the whole zero-padded image, channel planes [C][R][PW] (R = H + 2*pad
//     rows, PW >= W + 2*pad columns), read as contiguous 128-bit loads and
//     scattered into the zeroed planes;
//   * the block's weights in their natural order [MB][C*9] (+4 pad per row),
//     or flipped and transposed for the input gradient;
// then reduces K = C*9 entirely from LDS. No weight repacking launch and no
// per-item index arithmetic beyond the row copy.
//
// Reduction order: k = c*9 + tap, the weights' own order. Lane quarter q
// (lanes 16q..16q+15) takes the channels [q*C/4, (q+1)*C/4), so at step s
// of a quarter its k is q*(C/4)*9 + s:
//   * A (weights, rows = output channels): four consecutive steps are four
//     consecutive floats of the lane's weight row: one 128-bit LDS read per
//     four MFMAs;
//   * B (image, columns = output pixels): step s reads plane q*C/4 + s/9 at
//     tap (s%9)/3, s%3 from the lane's pixel: within a group of four
//     channels the 36 offsets are compile-time constants (immediate offsets
//     of the LDS reads).
// Lane l's accumulator holds D[m = 4*(l/16) + r][pixel = 16*tile + l%16].
#include <algorithm>

#include "buffer_ops.hpp"
#include "conv_slab.hpp"
#include "fastdiv.hpp"

namespace nrs {
namespace {

struct ImgArgs {
    const float* x;     // NCHW [N][C][H][W]
    const float* w;     // [M][C][3][3], or [C][M][3][3] with FLIP
    const float* bias;  // [M] or null
    float* out;         // NCHW [N][M][OH][OW]
    int C, H, W, M, pad, OH, OW, P;
    int R, plane;       // staged rows (H + 2*pad) and floats per staged plane (>= R * PW)
    int tiles;          // pixel tiles of 16 per image
    int wrow;           // floats per staged weight row (C*9 + 4)
    int vec_out;        // 128-bit output stores (P % 4 == 0, 16-byte aligned output)
    float beta;
    FastDiv div_ow, div_hw, div_w;
};

template <int PW>
__device__ __forceinline__ int tap_off(int tap) {
    return (tap / 3) * PW + tap % 3;
}

// MB output channels (OB = MB/16 blocks) per workgroup of 4 waves: wave w
// takes channel block w % OB and the pixel tiles w / OB + k * (4 / OB),
// k < NSW.
template <int PW, int MB, int NSW, bool FLIP>
__global__ __launch_bounds__(256) void conv_img_kernel(ImgArgs a) {
    constexpr int OB = MB / 16, TSTEP = 4 / OB;
    static_assert(MB == 16 || MB == 32, "16 or 32 output channels per workgroup");
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, l16 = lane & 15;
    const int img = blockIdx.x, m0 = blockIdx.y * MB;
    const int C = a.C, CQ = C >> 2;  // channels per lane quarter (multiple of 4)
    float* xs = lds;
    float* ws = lds + C * a.plane;

    // ---- staging: the image and the weight block. A round issues all of its
    // loads before its first LDS store, so the common shapes pay one memory
    // round trip.
    {
        const float* ximg = a.x + (int64_t)img * C * a.H * a.W;
        const int HW = a.H * a.W, nimg = C * HW;  // floats of this image
        const auto rx = buffer_rsrc(ximg, (int64_t)nimg * 4);
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
                const int per_row = C * 9 / 4;
#pragma unroll
                for (int b = 0; b < WB; ++b) {
                    const int e = w0 + b * 256 + tid;
                    const int m = e / per_row, k4 = e - m * per_row;
                    wv[b] = buffer_load4(rw, e < wq ? e * 16 : kOutOfRange);
                    wd[b] = e < wq ? m * a.wrow + 4 * k4 : -1;
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
        // The image is contiguous: it is read as 128-bit loads (XV per
        // thread per round, the weights in the first round too) and scattered
        // into the zeroed, padded planes; the last nimg % 4 floats are read
        // one by one.
        constexpr int XV = 8;
        const int n4 = nimg >> 2;
        const bool aligned = (((uintptr_t)ximg) & 15) == 0;
        for (int r0 = 0; r0 == 0 || r0 < n4; r0 += XV * 256) {
            f32x4 v[XV];
#pragma unroll
            for (int b = 0; b < XV; ++b) {
                const int e = r0 + b * 256 + tid;
                if (aligned) {
                    v[b] = buffer_load4(rx, e < n4 ? e * 16 : kOutOfRange);
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        v[b][u] = buffer_load1(rx, e < n4 ? (4 * e + u) * 4 : kOutOfRange);
                }
            }
            f32x4 wv[FLIP ? 1 : WB];
            float wf[FLIP ? WB : 1][9];
            int wd[WB];
            float tail = 0.0f;
            if (r0 == 0) {
                load_weights(0, wv, wf, wd);
                if (tid < (nimg & 3)) tail = buffer_load1(rx, (4 * n4 + tid) * 4);
                // zero the planes (halo included) while the loads fly
                f32x4* z = reinterpret_cast<f32x4*>(xs);
                for (int e = tid; e < (C * a.plane) / 4; e += 256) z[e] = f32x4{0.f, 0.f, 0.f, 0.f};
                for (int e = (C * a.plane) / 4 * 4 + tid; e < C * a.plane; e += 256) xs[e] = 0.0f;
                __syncthreads();
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int b = 0; b < XV; ++b) {
                const int e = r0 + b * 256 + tid;
                if (e >= n4) continue;
                uint32_t c, rem, r, col;
                fast_divmod((uint32_t)(4 * e), a.div_hw, c, rem);
                fast_divmod(rem, a.div_w, r, col);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    xs[(int)c * a.plane + ((int)r + a.pad) * PW + (int)col + a.pad] = v[b][u];
                    if (++col == (uint32_t)a.W) {
                        col = 0;
                        if (++r == (uint32_t)a.H) {
                            r = 0;
                            ++c;
                        }
                    }
                }
            }
            if (r0 == 0) {
                store_weights(wv, wf, wd);
                if (tid < (nimg & 3)) {
                    const int e = 4 * n4 + tid;
                    const int c = e / HW, rem = e - c * HW, r = rem / a.W, col = rem - r * a.W;
                    xs[c * a.plane + (r + a.pad) * PW + col + a.pad] = tail;
                }
            }
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
    // per-tile LDS offset of this lane's pixel window (quarter's first plane)
    int pb[NSW];
#pragma unroll
    for (int k = 0; k < NSW; ++k) {
        const int t = t0 + k * TSTEP;
        const int p = min(16 * t + l16, a.P - 1);  // masked pixels read pixel P-1
        uint32_t oy, ox;
        fast_divmod((uint32_t)p, a.div_ow, oy, ox);
        pb[k] = (q * CQ) * a.plane + (int)oy * PW + (int)ox;
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
                bf[k][r] = xs[pb[k] + cbase + (r / 9) * a.plane + tap_off<PW>(r % 9)];
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
                        bn[k][r] = xs[pb[k] + cbase + (s / 9) * a.plane + tap_off<PW>(s % 9)];
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
            const int m = e / max(P4, 1), p4 = e - m * P4;
            old[u] = (m < mvalid) ? *reinterpret_cast<const f32x4*>(oimg + (int64_t)(m0 + m) * a.P + 4 * p4)
                                  : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    __syncthreads();  // every wave is done with the image planes
    float* ot = lds;  // [MB][P]
#pragma unroll
    for (int k = 0; k < NSW; ++k)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int p = 16 * (t0 + k * TSTEP) + l16;
            const int m = 16 * ob + 4 * q + r;
            if (p < a.P) ot[m * a.P + p] = acc[k][r] + bias[r];
        }
    __syncthreads();
    if (vec) {
        const int total = mvalid * P4;
        for (int u0 = 0; u0 < total; u0 += OV * 256) {
#pragma unroll
            for (int u = 0; u < OV; ++u) {
                const int e = u0 + u * 256 + tid;
                if (e >= total) continue;
                const int m = e / P4, p4 = e - m * P4;
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

constexpr int kImgLdsBytes = 160 * 1024;

template <int PW, int MB, int NSW, bool FLIP>
int launch_img(const ImgArgs& a, int64_t N, size_t lds) {
    auto fn = conv_img_kernel<PW, MB, NSW, FLIP>;
    static bool attr_set = false;
    if (!attr_set) {
        NRS_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, kImgLdsBytes));
        attr_set = true;
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)N, (unsigned)((a.M + MB - 1) / MB)), dim3(256), lds,
                       stream(), a);
    NRS_LAUNCH_CHECK("conv2d (image-resident)");
    return NRS_OK;
}

}  // namespace

int img_conv(const SlabConv& s) {
    // 3x3, stride 1, channel count a multiple of 16, rows of at most 16
    // staged floats, a handful of 16-pixel tiles per wave
    if (s.kh != 3 || s.kw != 3 || s.stride != 1 || s.pad_h != s.pad_w || s.pad_h > 2 ||
        s.C % 16 != 0 || s.C <= 0 || s.M <= 0 || s.N <= 0 || s.N > 65535)
        return kSlabUnsupported;
    const int pad = s.pad_h;
    const int R = s.H + 2 * pad, Wp = s.W + 2 * pad;
    if (Wp > 16 || s.OH != R - 2 || s.OW != Wp - 2) return kSlabUnsupported;
    constexpr int PW = 16;
    const int P = s.OH * s.OW, tiles = (P + 15) / 16;
    // 32 output channels per workgroup when that leaves at least one
    // workgroup per CU, else 16
    const int MB = (s.M % 32 == 0 && s.N * (s.M / 32) >= num_cus()) ? 32 : 16;
    const int per_wave = (tiles + (4 / (MB / 16)) - 1) / (4 / (MB / 16));
    const int NSW = per_wave <= 4 ? 4 : (per_wave <= 7 ? 7 : 0);
    if (NSW == 0) return kSlabUnsupported;
    // plane pitch: the four lane quarters read four channel planes at once;
    // a pitch with quarters * planes = 16 (mod 64) floats puts them on
    // different LDS banks
    const int CQ = s.C / 4;
    int plane = R * PW;
    while ((CQ * plane) % 64 != 16) ++plane;
    const int wrow = s.C * 9 + 4;
    // (the epilogue's [MB][P] output tile reuses the image planes)
    const size_t lds = 4 * std::max((size_t)s.C * plane + (size_t)MB * wrow, (size_t)MB * P);
    if (lds > kImgLdsBytes) return kSlabUnsupported;
    ImgArgs a;
    a.x = s.x;
    a.w = s.w;
    a.bias = s.bias;
    a.out = s.out;
    a.C = s.C;
    a.H = s.H;
    a.W = s.W;
    a.M = s.M;
    a.pad = pad;
    a.OH = s.OH;
    a.OW = s.OW;
    a.P = P;
    a.R = R;
    a.plane = plane;
    a.tiles = tiles;
    a.wrow = wrow;
    a.beta = s.beta;
    a.vec_out = (P % 4 == 0 && ((uintptr_t)s.out & 15) == 0) ? 1 : 0;
    a.div_ow = make_fastdiv((uint32_t)s.OW);
    a.div_hw = make_fastdiv((uint32_t)(s.H * s.W));
    a.div_w = make_fastdiv((uint32_t)s.W);
    if (s.flip) {
        if (MB == 32) return NSW == 7 ? launch_img<PW, 32, 7, true>(a, s.N, lds)
                                      : launch_img<PW, 32, 4, true>(a, s.N, lds);
        return NSW == 7 ? launch_img<PW, 16, 7, true>(a, s.N, lds)
                        : launch_img<PW, 16, 4, true>(a, s.N, lds);
    }
    if (MB == 32) return NSW == 7 ? launch_img<PW, 32, 7, false>(a, s.N, lds)
                                  : launch_img<PW, 32, 4, false>(a, s.N, lds);
    return NSW == 7 ? launch_img<PW, 16, 7, false>(a, s.N, lds)
                    : launch_img<PW, 16, 4, false>(a, s.N, lds);
}

}  // namespace nrs
