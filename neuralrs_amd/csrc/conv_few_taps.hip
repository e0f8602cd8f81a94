// Weight and bias gradient of convolutions with few taps per output channel
// (c_in*kh*kw <= 15, e.g. a first layer over grayscale images): the
// reference's dW = G . cols^T and db = sum(G) (src/cuda/nn/conv.rs:314-322)
// without the cols matrix, on the f32 matrix cores.
//
//   dW[m][t] = sum_{n,p} g[n,m,p] * x_t(n,p)     db[m] = sum_{n,p} g[n,m,p]
//
// is a product with the output channels and the taps as its 2-D output and
// the N*P pixels as its reduction. v_mfma_f32_16x16x4f32 takes 16 channels
// (m = lane%16) by 16 taps (n = lane%16) per block; tap column `taps` reads
// the constant 1, so the same product yields the bias gradient. Lane group
// kq = lane/16 holds pixels p0 + 4kq .. p0 + 4kq + 3: one 128-bit load of the
// output gradient per channel block feeds four MFMAs. The input image is
// staged in LDS with a zero halo, so a tap reads x_t(p) branch-free.
//
// UNPOOL: the output gradient is the 2x2 max-pool backward of a pooled
// gradient, expanded while loading (the conv output's gradient is never
// written).
//
// A workgroup (4 waves) owns one image and `4*GPW` groups of 16 pixels.
// A wave issues all its gradient loads at once (one memory round trip) and
// then runs its MFMA chain over its pixel groups in order. The four waves'
// sums are added in wave order into per-workgroup partials
// pw[slice][m][t], pb[slice][m], which a second launch adds in slice order:
// the result is deterministic.
#include <algorithm>

#include "buffer_ops.hpp"
#include "conv_slab.hpp"

namespace nrs {
namespace {

typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int kFewTaps = 15;   // taps per channel (one MFMA column is the bias)
constexpr int kFewMaxM = 64;   // output channels (four blocks of 16)
constexpr int kFewImage = 16384;  // staged image floats (64 KB)
constexpr int kStageX = 4;        // image floats per thread per staging round

struct FewTapsArgs {
    const float* x;
    const float* g;
    const float* gp;     // UNPOOL: pooled gradient [N][M][OH/2][OW/2]
    const int32_t* am;   // UNPOOL: its argmax (flat conv-output indices)
    const float* pv;     // UNPOOL with a ReLU between conv and pool: the pooled values (or null)
    float* pw;  // [slices][M][taps]
    float* pb;  // [slices][M]
    int C, H, W, M, kh, kw, stride, pad, OH, OW, P, Hp, Wp, taps, chunks;
    FastDiv div_ow;
};

template <int NBLK, int GPW, bool UNPOOL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void wgrad_few_taps_kernel(FewTapsArgs a) {
    extern __shared__ __attribute__((aligned(16))) float xs[];  // [C][Hp][Wp]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = blockIdx.x / a.chunks, chunk = blockIdx.x - n * a.chunks;
    const int t = lane & 15, kq = lane >> 4;

    // the input image with a zero halo of `pad` (rows and columns), kStageX
    // items per thread per round (a load at kOutOfRange returns zero, so the
    // halo needs no select that would make each load wait for the previous).
    // An image of one round is requested before the gradient, so the two
    // round trips overlap (with the pooled gradient, expanding it waits for
    // its loads).
    const auto rimg =
        buffer_rsrc(a.x + (int64_t)n * a.C * a.H * a.W, (int64_t)a.C * a.H * a.W * 4);
    const int plane = a.Hp * a.Wp, xn = a.C * plane;
    auto stage_load = [&](int e0, float (&v)[kStageX]) {
#pragma unroll
        for (int k = 0; k < kStageX; ++k) {
            const int e = e0 + k * 256 + tid;
            const int c = e / plane, r = e - c * plane, yy = r / a.Wp, xx = r - yy * a.Wp;
            const int iy = yy - a.pad, ix = xx - a.pad;
            const bool ok = (e < xn) & ((unsigned)iy < (unsigned)a.H) & ((unsigned)ix < (unsigned)a.W);
            v[k] = buffer_load1(rimg, ok ? ((c * a.H + iy) * a.W + ix) * 4 : kOutOfRange);
        }
    };
    auto stage_store = [&](int e0, const float (&v)[kStageX]) {
#pragma unroll
        for (int k = 0; k < kStageX; ++k)
            if (e0 + k * 256 + tid < xn) xs[e0 + k * 256 + tid] = v[k];
    };
    const bool one_round = xn <= 256 * kStageX;
    float v0[kStageX];
    stage_load(0, v0);

    // gradient fragments: [group][block], pixels 16*gi + 4*kq .. +3 of
    // channel 16*b + t (zero past P and M through the buffer bounds)
    const int g0 = (chunk * 4 + wave) * GPW;
    f32x4v ga[GPW][NBLK];
    if constexpr (!UNPOOL) {
        const auto rg = buffer_rsrc(a.g + (int64_t)n * a.M * a.P, (int64_t)a.M * a.P * 4);
#pragma unroll
        for (int q = 0; q < GPW; ++q) {
            const int p = 16 * (g0 + q) + 4 * kq;
#pragma unroll
            for (int b = 0; b < NBLK; ++b) {
                const int oc = 16 * b + t;
                ga[q][b] =
                    buffer_load4(rg, ((p < a.P) & (oc < a.M)) ? (oc * a.P + p) * 4 : kOutOfRange);
            }
        }
        stage_store(0, v0);  // waits for the image only: the older loads
    } else {
        // pixels p .. p+3 (one row: OW % 4 == 0) lie in pooled columns
        // x/2 and x/2 + 1 of pooled row y/2: two pooled values and two
        // indices per quad, 64-bit loads; the quad's values are the pooled
        // value where the index names the pixel, else 0
        const int PP = (a.OH >> 1) * (a.OW >> 1);
        const auto rp = buffer_rsrc(a.gp + (int64_t)n * a.M * PP, (int64_t)a.M * PP * 4);
        const auto ri = buffer_rsrc(reinterpret_cast<const float*>(a.am) + (int64_t)n * a.M * PP,
                                    (int64_t)a.M * PP * 4);
        // with a ReLU between the conv and the pooling, a window's gradient
        // passes only where its pooled value (the ReLU of the conv value at
        // the index) is > 0, relu_grad's test on the conv value
        const bool relu = a.pv != nullptr;
        const auto rv = buffer_rsrc(relu ? a.pv + (int64_t)n * a.M * PP : a.gp,
                                    relu ? (int64_t)a.M * PP * 4 : 0);
        f32x2 gv[GPW][NBLK], iv[GPW][NBLK], vv[GPW][NBLK];
        int qy[GPW], qx[GPW];
#pragma unroll
        for (int q = 0; q < GPW; ++q) {
            const int p = 16 * (g0 + q) + 4 * kq;
            uint32_t y, x;
            fast_divmod((uint32_t)min(p, a.P - 1), a.div_ow, y, x);
            qy[q] = (int)y;
            qx[q] = (int)x;
            const int pw = (int)(y >> 1) * (a.OW >> 1) + (int)(x >> 1);
#pragma unroll
            for (int b = 0; b < NBLK; ++b) {
                const int oc = 16 * b + t;
                const bool ok = (p < a.P) & (oc < a.M);
                gv[q][b] = buffer_load2(rp, ok ? (oc * PP + pw) * 4 : kOutOfRange);
                iv[q][b] = buffer_load2(ri, ok ? (oc * PP + pw) * 4 : kOutOfRange);
                vv[q][b] = buffer_load2(rv, (ok & relu) ? (oc * PP + pw) * 4 : kOutOfRange);
            }
        }
        stage_store(0, v0);  // waits for the image only: the older loads
#pragma unroll
        for (int q = 0; q < GPW; ++q)
#pragma unroll
            for (int b = 0; b < NBLK; ++b) {
                const int oc = 16 * b + t;
                const int e0 = ((n * a.M + oc) * a.OH + qy[q]) * a.OW + qx[q];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    // the element first, then its bits (a bit_cast of the
                    // vector element expression read element 0 for every u)
                    const float raw = u < 2 ? iv[q][b].x : iv[q][b].y;
                    const int idx = __builtin_bit_cast(int, raw);
                    const float pval = u < 2 ? vv[q][b].x : vv[q][b].y;
                    const bool pass = (idx == e0 + u) & (!relu | (pval > 0.0f));
                    ga[q][b][u] = pass ? (u < 2 ? gv[q][b].x : gv[q][b].y) : 0.0f;
                }
            }
    }

    // the image's further rounds, every load of a round issued before its
    // stores
    if (!one_round) {
        for (int e0 = 256 * kStageX; e0 < xn; e0 += 256 * kStageX) {
            float v[kStageX];
            stage_load(e0, v);
            stage_store(e0, v);
            // nothing outstanding at the loop edge: the compiler would
            // otherwise wait for the gradient loads before the next round
            __builtin_amdgcn_s_waitcnt(0);
        }
    }
    // this lane's tap: offset in the staged image, or the bias column
    int toff = 0;
    const bool tap_live = t < a.taps, ones = t == a.taps;
    if (tap_live) {
        const int j = t % a.kw, i = (t / a.kw) % a.kh, c = t / (a.kw * a.kh);
        toff = (c * a.Hp + i) * a.Wp + j;
    }
    __syncthreads();

    f32x4v acc[NBLK];
#pragma unroll
    for (int b = 0; b < NBLK; ++b) acc[b] = f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int q = 0; q < GPW; ++q) {
        int p = 16 * (g0 + q) + 4 * kq;
        uint32_t oy, ox;
        fast_divmod((uint32_t)min(p, a.P - 1), a.div_ow, oy, ox);
        f32x4v xb;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const bool pl = p + s < a.P;
            const float v = xs[toff + (pl ? ((int)oy * a.Wp + (int)ox) * a.stride : 0)];
            xb[s] = pl ? (tap_live ? v : (ones ? 1.0f : 0.0f)) : 0.0f;
            if ((int)++ox == a.OW) {
                ox = 0;
                ++oy;
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int b = 0; b < NBLK; ++b)
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(ga[q][b][s], xb[s], acc[b], 0, 0, 0);
    }

    // lane holds D[m = 16b + 4kq + r][t]; the waves' sums in wave order
    __syncthreads();  // the staged image is no longer read
    float* red = xs;  // [4][NBLK*16][17]
    constexpr int RS = 17, WS = NBLK * 16 * RS;
#pragma unroll
    for (int b = 0; b < NBLK; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave * WS + (16 * b + 4 * kq + r) * RS + t] = acc[b][r];
    __syncthreads();
    const int slice = blockIdx.x;
    for (int e = tid; e < NBLK * 256; e += 256) {
        const int m = e >> 4, tt = e & 15;
        if (m >= a.M || tt > a.taps) continue;
        float v = red[m * RS + tt];
#pragma unroll
        for (int w = 1; w < 4; ++w) v += red[w * WS + m * RS + tt];
        if (tt < a.taps)
            a.pw[((int64_t)slice * a.M + m) * a.taps + tt] = v;
        else
            a.pb[(int64_t)slice * a.M + m] = v;
    }
}

template <int NBLK, bool UNPOOL>
void* pick_gpw(int gpw) {
    switch (gpw) {
        case 1: return reinterpret_cast<void*>(wgrad_few_taps_kernel<NBLK, 1, UNPOOL>);
        case 2: return reinterpret_cast<void*>(wgrad_few_taps_kernel<NBLK, 2, UNPOOL>);
        case 4: return reinterpret_cast<void*>(wgrad_few_taps_kernel<NBLK, 4, UNPOOL>);
        default: return reinterpret_cast<void*>(wgrad_few_taps_kernel<NBLK, 8, UNPOOL>);
    }
}

template <bool UNPOOL>
void* pick_kernel(int nblk, int gpw) {
    return nblk == 1 ? pick_gpw<1, UNPOOL>(gpw)
                     : (nblk == 2 ? pick_gpw<2, UNPOOL>(gpw) : pick_gpw<4, UNPOOL>(gpw));
}

}  // namespace

int few_taps_wgrad(const FewTapsWgrad& s) {
    const int taps = s.C * s.kh * s.kw;
    const int64_t P = (int64_t)s.OH * s.OW;
    const int Hp = s.H + 2 * s.pad, Wp = s.W + 2 * s.pad;
    if (taps > kFewTaps || s.M > kFewMaxM || s.M < 1 || P % 4 || P < 1 || s.N < 1 ||
        (int64_t)s.C * Hp * Wp > kFewImage || (int64_t)s.M * P > INT32_MAX / 4 ||
        (int64_t)(s.OH - 1) * s.stride + s.kh > Hp || (int64_t)(s.OW - 1) * s.stride + s.kw > Wp)
        return kSlabUnsupported;
    const bool unpool = s.g == nullptr;
    if (unpool && (!s.gp || !s.am || s.OH % 2 || s.OW % 4 || ((uintptr_t)s.gp & 7) ||
                   ((uintptr_t)s.am & 7) || ((uintptr_t)s.pv & 7) || s.N * s.M * P > INT32_MAX))
        return kSlabUnsupported;
    const int nblk = s.M <= 16 ? 1 : (s.M <= 32 ? 2 : 4);  // channel blocks instantiated
    const int64_t gpi = (P + 15) / 16;
    // pixel groups per wave: the largest that still gives two workgroups
    // per CU (fewer, longer waves amortise the staged image)
    int gpw = 8;
    auto chunks_for = [&](int gw) { return (gpi + 4 * gw - 1) / (4 * gw); };
    while (gpw > 1 && s.N * chunks_for(gpw) < 2 * num_cus()) gpw /= 2;
    const int64_t chunks = chunks_for(gpw), slices = s.N * chunks;
    if (slices > INT32_MAX || slices * s.M * (taps + 1) > INT32_MAX) return kSlabUnsupported;
    float* pw = workspace(sizeof(float) * (size_t)(slices * s.M * (taps + 1)), 3);
    if (!pw) return NRS_ERR_ALLOC;
    float* pb = pw + slices * s.M * taps;
    FewTapsArgs a;
    a.x = s.x;
    a.g = s.g;
    a.gp = s.gp;
    a.am = s.am;
    a.pv = s.pv;
    a.pw = pw;
    a.pb = pb;
    a.C = s.C;
    a.H = s.H;
    a.W = s.W;
    a.M = s.M;
    a.kh = s.kh;
    a.kw = s.kw;
    a.stride = s.stride;
    a.pad = s.pad;
    a.OH = s.OH;
    a.OW = s.OW;
    a.P = (int)P;
    a.Hp = Hp;
    a.Wp = Wp;
    a.taps = taps;
    a.chunks = (int)chunks;
    a.div_ow = make_fastdiv((uint32_t)s.OW);
    const size_t lds =
        sizeof(float) * (size_t)std::max<int64_t>((int64_t)s.C * Hp * Wp, 4 * nblk * 16 * 17);
    void* fn = unpool ? pick_kernel<true>(nblk, gpw) : pick_kernel<false>(nblk, gpw);
    hipLaunchKernelGGL(reinterpret_cast<void (*)(FewTapsArgs)>(fn), dim3((unsigned)slices),
                       dim3(256), lds, stream(), a);
    NRS_LAUNCH_CHECK("conv2d weight gradient (few taps)");
    return wgrad_partial_sum(s.dw, s.db, pw, pb, (int)slices, s.M, 1, taps, s.beta);
}

}  // namespace nrs
