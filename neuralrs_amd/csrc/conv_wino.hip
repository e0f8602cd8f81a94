// Winograd F(2x2, 3x3) convolution of "same" 3x3 stride-1 layers over small
// images on the f32 matrix cores: the forward of src/cuda/nn/conv.rs:244-277
// (im2col + GEMM there) with 2.25x fewer multiplies.
//
// Lavin and Gray, "Fast Algorithms for Convolutional Neural Networks" (2016):
// each 2x2 output tile is
//   Y = A^T [ sum_c (G g_c G^T) .* (B^T d_c B) ] A
// with d_c the 4x4 input patch of channel c over the tile (rows and columns
// -1 .. +2 around it, zero outside the image), g_c the 3x3 filter and
//   B^T = [1 0 -1 0; 0 1 1 0; 0 -1 1 0; 0 1 0 -1]
//   G   = [1 0 0; 1/2 1/2 1/2; 1/2 -1/2 1/2; 0 0 1]
//   A^T = [1 1 1 0; 0 1 -1 -1].
// For each of the 16 transform positions xi the channel sum is a product
// M_xi[m][t] = sum_c U_xi[m][c] V_xi[c][t] (m output channel, t tile), run on
// v_mfma_f32_16x16x4f32: 16 channels by 16 tiles, 4 input channels a step.
//
// Exactness: B^T and A^T hold only 0 and +-1 and G only halves, so on small
// integer data every transformed value and partial sum is a multiple of 1/4
// far inside f32's exact range, and the result equals the direct sum. On
// general data the transforms add a few roundings to each term; the tests
// bound the error against f64.
//
// Workgroup: one image and 32 output channels, 8 waves. Wave w owns output
// channel block w&1 (16 channels) and tile block w>>1 (16 of at most 64
// tiles: images up to 16x16) and keeps one accumulator per xi for that
// 16x16 block, so the output transform runs in registers: the lane holding
// M_xi[m][t] for one xi holds it for all 16.
//
// Input channels go in chunks of 8 (two MFMA steps of 4). A chunk's raw
// image planes (with a zero halo, so patch reads need no bounds checks) and
// its 32x8 raw filters are staged in LDS by coalesced loads, triple-buffered
// so one barrier per chunk suffices. Each lane builds its own operands from
// them: B = B^T d B of its 4x4 patch (channel 4s + l/16, tile l%16 of its
// block) and A = G g G^T of its filter (channel 16mb + l%16, the same input
// channel), the next step's while the matrix core runs the current step's
// products. The transforms are VALU work (repeated by the waves that share
// a patch or a filter), but they keep LDS traffic to the raw data: with
// the transformed operands staged in LDS instead, a chunk moved about twice
// the bytes and LDS, not the matrix core, set the pace.
#include <algorithm>
#include <type_traits>

#include "buffer_ops.hpp"
#include "conv_slab.hpp"

namespace nrs {
namespace {

constexpr int kWinoThreads = 512;                  // 8 waves
constexpr int kWinoMB = 32;                        // output channels per workgroup
constexpr int kWinoCC = 8;                         // input channels per chunk
constexpr int kWinoMaxTiles = 64;                  // 4 tile blocks of 16
constexpr int kWinoMaxSide = 16;                   // images up to 16x16
constexpr int kWinoPlane = 468;                    // padded plane and its pad (see wino_layout)
constexpr int kWinoImg = kWinoCC * kWinoPlane;     // floats of one image stage
constexpr int kWinoFPitch = kWinoMB * 9 + 16;      // raw filters of one channel (+16: no bank conflicts)
constexpr int kWinoFilt = kWinoCC * kWinoFPitch;   // floats of one filter stage
constexpr int kWinoStage = kWinoImg + kWinoFilt;
constexpr int kWinoStages = 3;
constexpr int kWinoImgLoads = kWinoCC * kWinoMaxSide * kWinoMaxSide / kWinoThreads;            // 4
constexpr int kWinoFiltLoads = (kWinoCC * kWinoMB * 9 + kWinoThreads - 1) / kWinoThreads;     // 5
constexpr int kWinoLds = kWinoStages * kWinoStage;  // floats

struct WinoArgs {
    const float* x;     // [N][C][H][W]
    const float* w;     // [M][C][3][3], or [C][M][3][3] read flipped
    const float* bias;  // [M] or null
    float* out;         // [N][M][H][W]
    int C, H, W, M;
    int TX, T;          // tiles per row, tiles per image
    int PW, PS;         // padded plane: row pitch and channel stride (floats)
    int mgroups;        // M / 32
    float beta;         // out = conv + beta * out (0: write without reading)
};

// V = B^T d B for a 4x4 patch d (row-major), in place.
__device__ __forceinline__ void input_transform(float (&d)[16]) {
    float s[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        s[0 + j] = d[0 + j] - d[8 + j];
        s[4 + j] = d[4 + j] + d[8 + j];
        s[8 + j] = d[8 + j] - d[4 + j];
        s[12 + j] = d[4 + j] - d[12 + j];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        d[4 * i + 0] = s[4 * i + 0] - s[4 * i + 2];
        d[4 * i + 1] = s[4 * i + 1] + s[4 * i + 2];
        d[4 * i + 2] = s[4 * i + 2] - s[4 * i + 1];
        d[4 * i + 3] = s[4 * i + 1] - s[4 * i + 3];
    }
}

// U = G g G^T for a 3x3 filter g (row-major).
__device__ __forceinline__ void filter_transform(const float (&g)[9], float (&u)[16]) {
    float t[12];  // G g: 4 x 3
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        t[0 + j] = g[j];
        t[3 + j] = 0.5f * (g[j] + g[3 + j] + g[6 + j]);
        t[6 + j] = 0.5f * (g[j] - g[3 + j] + g[6 + j]);
        t[9 + j] = g[6 + j];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        u[4 * i + 0] = t[3 * i];
        u[4 * i + 1] = 0.5f * (t[3 * i] + t[3 * i + 1] + t[3 * i + 2]);
        u[4 * i + 2] = 0.5f * (t[3 * i] - t[3 * i + 1] + t[3 * i + 2]);
        u[4 * i + 3] = t[3 * i + 2];
    }
}

template <bool FLIP>
__global__ __launch_bounds__(kWinoThreads) void conv_wino_kernel(WinoArgs a) {
    extern __shared__ __attribute__((aligned(16))) float lds[];  // kWinoStages x [image | filters]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // an image's output-channel groups are consecutive logical blocks, and
    // when the grid is a multiple of 8 logical block L runs on XCD
    // L / (grid / 8) (ids are dealt to the XCDs round-robin): the groups that
    // read one image share an L2
    const int grid = gridDim.x, bid = blockIdx.x;
    const int L = (grid & 7) == 0 ? (bid & 7) * (grid >> 3) + (bid >> 3) : bid;
    const int n = L / a.mgroups, mg = L - n * a.mgroups;
    const int mb = wave & 1, tb = wave >> 1;
    const int l16 = lane & 15, k = lane >> 4;
    const int HW = a.H * a.W, PW = a.PW, PS = a.PS, nch = a.C / kWinoCC;
    const auto rx = buffer_rsrc(a.x + (int64_t)n * a.C * HW, (int64_t)a.C * HW * 4);
    const auto rw = buffer_rsrc(a.w, (int64_t)a.M * a.C * 9 * 4);

    // staging maps, the same for every chunk: this thread's image elements
    // (consecutive threads on consecutive floats) and their places in the
    // padded planes; its filter elements (runs of 8*9 floats per output
    // channel in the forward's w[m][c][tap], of 32*9 per input channel in
    // the flipped w[c][m][tap]) and their places in [c][m][tap]
    const int img_n = kWinoCC * HW, filt_n = kWinoCC * kWinoMB * 9;
    int isrc[kWinoImgLoads], idst[kWinoImgLoads], fsrc[kWinoFiltLoads], fdst[kWinoFiltLoads];
#pragma unroll
    for (int q = 0; q < kWinoImgLoads; ++q) {
        const int e = q * kWinoThreads + tid;
        const int c = e / HW, r = e - c * HW, y = r / a.W, x = r - y * a.W;
        isrc[q] = e < img_n ? e : -1;
        idst[q] = e < img_n ? c * PS + (y + 1) * PW + x + 1 : 0;
    }
#pragma unroll
    for (int q = 0; q < kWinoFiltLoads; ++q) {
        const int e = q * kWinoThreads + tid;
        int c, m, tap, src;
        if (FLIP) {
            c = e / (kWinoMB * 9);
            const int r = e - c * (kWinoMB * 9);
            m = r / 9;
            tap = 8 - (r - m * 9);
            src = (c * a.M + mg * kWinoMB) * 9 + r;
        } else {
            m = e / (kWinoCC * 9);
            const int r = e - m * (kWinoCC * 9);
            c = r / 9;
            tap = r - c * 9;
            src = (mg * kWinoMB + m) * a.C * 9 + r;
        }
        fsrc[q] = e < filt_n ? src : -1;
        fdst[q] = e < filt_n ? c * kWinoFPitch + m * 9 + tap : 0;
    }
    const int fstep = FLIP ? kWinoCC * a.M * 9 : kWinoCC * 9;  // source advance per chunk
    // two register sets: chunk j's data is loaded into set j&1 three chunks
    // ahead and staged in LDS two chunks ahead
    struct Raw {
        float i[kWinoImgLoads], f[kWinoFiltLoads];
    } raw[2];
    auto stage_load = [&](Raw& r, int ch) {
#pragma unroll
        for (int q = 0; q < kWinoImgLoads; ++q)
            r.i[q] = buffer_load1(rx, isrc[q] >= 0 ? (isrc[q] + ch * img_n) * 4 : kOutOfRange);
#pragma unroll
        for (int q = 0; q < kWinoFiltLoads; ++q)
            r.f[q] = buffer_load1(rw, fsrc[q] >= 0 ? (fsrc[q] + ch * fstep) * 4 : kOutOfRange);
    };
    auto stage_store = [&](const Raw& r, int g) {
        float* st = lds + g * kWinoStage;
#pragma unroll
        for (int q = 0; q < kWinoImgLoads; ++q)
            if (isrc[q] >= 0) st[idst[q]] = r.i[q];
#pragma unroll
        for (int q = 0; q < kWinoFiltLoads; ++q)
            if (fsrc[q] >= 0) st[kWinoImg + fdst[q]] = r.f[q];
    };

    // this lane's operands of step s of the chunk in stage g: its patch of
    // channel 4s + k over tile 16tb + l16 (a pad tile, t >= T, reads tile
    // 0: its columns of the product are never stored), and its filter of
    // output channel 16mb + l16 over the same channel
    const int t = tb * 16 + l16, tt = t < a.T ? t : 0, tty = tt / a.TX, ttx = tt - tty * a.TX;
    const int poff = k * PS + 2 * tty * PW + 2 * ttx;
    const int foff = kWinoImg + k * kWinoFPitch + (mb * 16 + l16) * 9;
    auto make_b = [&](int g, int s, float (&b)[16]) {
        const float* src = lds + g * kWinoStage + 4 * s * PS + poff;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) b[4 * i + j] = src[i * PW + j];
        input_transform(b);
    };
    auto make_a = [&](int g, int s, float (&u)[16]) {
        const float* src = lds + g * kWinoStage + 4 * s * kWinoFPitch + foff;
        float f[9];
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) f[tap] = src[tap];
        filter_transform(f, u);
    };

    // prologue: chunks 0 and 1 loaded together; the planes' halos zeroed in
    // every stage (they stay zero; the stores never touch them, so no
    // barrier is needed between the two); chunks 0 and 1 staged, chunk 2
    // loaded, step 0 of chunk 0 built. A plane's halo: row -1, column -1
    // and W of rows 0 .. H-1, and rows H .. 2*TY (one more for odd H).
    stage_load(raw[0], 0);
    if (nch > 1) stage_load(raw[1], 1);
    {
        const int PH = 2 * ((a.H + 1) >> 1) + 2, row = a.W + 2;
        const int halo = row + 2 * a.H + (PH - 1 - a.H) * row;
        for (int e = tid; e < kWinoCC * halo; e += kWinoThreads) {
            const int c = e / halo, h = e - c * halo;
            int y, x;
            if (h < row) {
                y = 0;
                x = h;
            } else if (h < row + 2 * a.H) {
                y = 1 + ((h - row) >> 1);
                x = (h - row) & 1 ? a.W + 1 : 0;
            } else {
                const int r = h - row - 2 * a.H;
                y = a.H + 1 + r / row;
                x = r - (y - a.H - 1) * row;
            }
#pragma unroll
            for (int g = 0; g < kWinoStages; ++g) lds[g * kWinoStage + c * PS + y * PW + x] = 0.0f;
        }
    }
    stage_store(raw[0], 0);
    if (nch > 1) stage_store(raw[1], 1);
    if (nch > 2) stage_load(raw[0], 2);
    __syncthreads();
    float ac[16], bc[16], an[16], bn[16];
    make_a(0, 0, ac);
    make_b(0, 0, bc);

    f32x4 acc[16];
#pragma unroll
    for (int xi = 0; xi < 16; ++xi) acc[xi] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // the interleaving of one step's 16 MFMAs with the next operands'
    // build: the 13 LDS reads in the first five MFMA slots, the transforms'
    // VALU work in the other eleven, so no read is waited for right after
    // it is issued
    auto interleave = [] {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);  // LDS read
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
        for (int i = 0; i < 11; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // VALU
        }
    };
    // chunk ch in stage g; P = ch & 1 selects the register sets
    auto chunk = [&](int ch, int g, auto parity) {
        constexpr int P = decltype(parity)::value;
        const int gn = g == kWinoStages - 1 ? 0 : g + 1;
        // chunk ch+3's loads, into the set chunk ch+1 left (staged before
        // the last barrier)
        if (ch + 3 < nch) stage_load(raw[P ^ 1], ch + 3);
        __builtin_amdgcn_sched_barrier(0);
        // step 0's products while step 1's operands are built
#pragma unroll
        for (int xi = 0; xi < 16; ++xi)
            acc[xi] = __builtin_amdgcn_mfma_f32_16x16x4f32(ac[xi], bc[xi], acc[xi], 0, 0, 0);
        make_a(g, 1, an);
        make_b(g, 1, bn);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
        // step 1's products while the next chunk's step 0 operands are built
        // (its stage was filled before the last barrier; after the last
        // chunk this reads a stage nobody fills, and the result is unused:
        // no branch, which would stop the interleaving)
#pragma unroll
        for (int xi = 0; xi < 16; ++xi)
            acc[xi] = __builtin_amdgcn_mfma_f32_16x16x4f32(an[xi], bn[xi], acc[xi], 0, 0, 0);
        make_a(gn, 0, ac);
        make_b(gn, 0, bc);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
        if (ch + 2 < nch) {
            // chunk ch+2 (set P) into the stage chunk ch-1 used (every wave
            // finished reading it before the last barrier). Without a store
            // there is nothing to wait for: the next chunk's stage was filled
            // before the last barrier, and the chunk after it stores nothing.
            stage_store(raw[P], gn == kWinoStages - 1 ? 0 : gn + 1);
            __syncthreads();
        }
    };
    for (int ch = 0, g = 0; ch < nch; ch += 2) {
        chunk(ch, g, std::integral_constant<int, 0>());
        g = g == kWinoStages - 1 ? 0 : g + 1;
        if (ch + 1 < nch) chunk(ch + 1, g, std::integral_constant<int, 1>());
        g = g == kWinoStages - 1 ? 0 : g + 1;
    }

    // output transform: lane holds M_xi[m = 16mb + 4k + r][t = 16tb + l16]
    if (t >= a.T) return;
    const int ty = t / a.TX, tx = t - ty * a.TX;
    const bool row1 = 2 * ty + 1 < a.H;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int mo = mg * kWinoMB + mb * 16 + 4 * k + r;
        float T0[4], T1[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            T0[j] = acc[j][r] + acc[4 + j][r] + acc[8 + j][r];
            T1[j] = acc[4 + j][r] - acc[8 + j][r] - acc[12 + j][r];
        }
        const float bv = a.bias ? a.bias[mo] : 0.0f;
        f32x2 y0{T0[0] + T0[1] + T0[2] + bv, T0[1] - T0[2] - T0[3] + bv};
        f32x2 y1{T1[0] + T1[1] + T1[2] + bv, T1[1] - T1[2] - T1[3] + bv};
        float* o = a.out + ((int64_t)n * a.M + mo) * HW + (2 * ty) * a.W + 2 * tx;
        if (a.beta != 0.0f) {
            y0 += a.beta * *reinterpret_cast<const f32x2*>(o);
            if (row1) y1 += a.beta * *reinterpret_cast<const f32x2*>(o + a.W);
        }
        *reinterpret_cast<f32x2*>(o) = y0;
        if (row1) *reinterpret_cast<f32x2*>(o + a.W) = y1;
    }
}

// Padded plane layout of an image size: the row pitch PW >= W + 2 and the
// channel stride PS >= (2*TY + 2) * PW that spread a wave's patch reads
// (4 channels x 16 tiles, lane 16k + j on channel k, tile j) over the most
// LDS banks, counted as distinct addresses per bank over 64 banks and over
// 32 banks per half wave; the first best candidate wins. Memoized per size.
void wino_layout(int H, int W, int& PW, int& PS) {
    static int memo[kWinoMaxSide + 1][kWinoMaxSide + 1][2] = {};
    int* m = memo[H][W];
    if (m[0]) {
        PW = m[0];
        PS = m[1];
        return;
    }
    const int TX = W / 2, T = ((H + 1) / 2) * TX, PH = 2 * ((H + 1) / 2) + 2;
    int best = 1 << 30;
    for (int pw = W + 2; pw <= W + 24; ++pw)
        for (int ps = PH * pw; ps <= PH * pw + 63 && ps <= kWinoPlane; ++ps) {
            int worst = 0;
            for (int tb = 0; tb < 4; ++tb) {
                // distinct addresses (same-address lanes share one access)
                int offs[64], half[64], nd = 0;
                for (int l = 0; l < 64; ++l) {
                    int t = 16 * tb + (l & 15);
                    if (t >= T) t = 0;
                    const int o = (l >> 4) * ps + 2 * (t / TX) * pw + 2 * (t % TX);
                    bool dup = false;
                    for (int q = 0; q < nd; ++q) dup |= offs[q] == o && half[q] == (l >> 5);
                    if (!dup) {
                        offs[nd] = o;
                        half[nd++] = l >> 5;
                    }
                }
                int c64[64] = {}, c32[2][32] = {};
                for (int q = 0; q < nd; ++q) {
                    bool dup = false;  // across halves, for the 64-bank count
                    for (int r = 0; r < q; ++r) dup |= offs[r] == offs[q];
                    if (!dup) ++c64[offs[q] % 64];
                    ++c32[half[q]][offs[q] % 32];
                }
                int w64 = 0, w32 = 0;
                for (int b = 0; b < 64; ++b) w64 = std::max(w64, c64[b]);
                for (int b = 0; b < 32; ++b) w32 = std::max(w32, std::max(c32[0][b], c32[1][b]));
                worst = std::max(worst, w64 + w32);
            }
            if (worst < best) {
                best = worst;
                PW = pw;
                PS = ps;
            }
        }
    m[0] = PW;
    m[1] = PS;
}

}  // namespace

int wino_conv(const SlabConv& s) {
    if (s.kh != 3 || s.kw != 3 || s.stride != 1 || s.pad_h != 1 || s.pad_w != 1 || s.OH != s.H ||
        s.OW != s.W || s.H < 1 || s.W < 2 || s.W % 2 != 0 || s.C <= 0 || s.C % kWinoCC != 0 ||
        s.M <= 0 || s.M % kWinoMB != 0 || s.N <= 0 || ((uintptr_t)s.out & 7) != 0)
        return kSlabUnsupported;
    const int TY = (s.H + 1) / 2, TX = s.W / 2;
    const int64_t HW = (int64_t)s.H * s.W;
    if (TY * TX > kWinoMaxTiles || s.H > kWinoMaxSide || s.W > kWinoMaxSide || s.N * (s.M / kWinoMB) > INT32_MAX ||
        (int64_t)s.C * HW * 4 > INT32_MAX / 2 || (int64_t)s.M * s.C * 9 * 4 > INT32_MAX / 2 ||
        s.N * std::max(s.C, s.M) * HW > INT32_MAX)
        return kSlabUnsupported;
    const size_t lds = sizeof(float) * kWinoLds;
    if (lds > lds_limit()) return kSlabUnsupported;
    WinoArgs a;
    a.x = s.x;
    a.w = s.w;
    a.bias = s.bias;
    a.out = s.out;
    a.C = s.C;
    a.H = s.H;
    a.W = s.W;
    a.M = s.M;
    a.TX = TX;
    a.T = TY * TX;
    wino_layout(s.H, s.W, a.PW, a.PS);
    a.mgroups = s.M / kWinoMB;
    a.beta = s.beta;
    auto fn = s.flip ? conv_wino_kernel<true> : conv_wino_kernel<false>;
    static bool attr_set[2] = {false, false};
    if (!attr_set[s.flip]) {
        NRS_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        attr_set[s.flip] = true;
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)(s.N * a.mgroups)), dim3(kWinoThreads), lds, stream(), a);
    NRS_LAUNCH_CHECK("conv2d (Winograd F(2x2,3x3))");
    return NRS_OK;
}

}  // namespace nrs
