// Chunk-pipelined image-resident convolution for small "same" 3x3 layers
// (stride 1, pad 1, images of at most 14x14), on the f32 matrix cores
// (v_mfma_f32_16x16x4f32). One kernel body serves
//   * the forward of nn::conv2d (src/cuda/nn/conv.rs:266-277),
//   * its input gradient (conv.rs:304-312), read as a forward convolution of
//     the output gradient with the flipped, channel-transposed weights,
//   * its weight and bias gradient (conv.rs:314-322),
// and the backward runs both gradients' workgroups in one launch.
//
// Output workgroups ("D" blocks: forward or input gradient) own one image
// and 32 output channels. The reduction K = C*9 is walked in chunks of 16
// input channels, double-buffered in LDS: while the matrix cores reduce
// chunk j, the loads of chunk j+1 are in flight into registers, and they are
// written to the other buffer afterwards. A chunk is
//   * 16 zero-padded image planes of 16 rows x 16 floats (+4, so a plane is
//     4 floats past a multiple of 64 banks), each thread copying one row;
//   * the block's 32 weight rows of the chunk's 16 channels x 9 taps: a
//     straight 128-bit copy in the forward; in the input gradient the taps of
//     w[oc][c] are reversed and (oc, c) transposed while they are staged.
// Wave w owns output-channel block w & 1 (A rows) and output rows
// (w >> 1) * 7 .. +6 (one B tile per row: lane = column, so every tap offset
// is an immediate). Lane quarter q takes chunk channels 4q .. 4q+3, whose
// planes start 16 banks apart, so a B read of 64 lanes hits 64 banks.
//
// Weight-gradient workgroups ("W" blocks) own two consecutive images (a K
// slice), 16 input channels (N: channel x tap) and 64 output channels (M).
// K is the image's pixels: lane quarter q takes pixels 4s + q at step s, so
// the four quarters read four neighbouring pixels of their channel's plane
// (planes 4 banks apart: conflict-free). The gradient rows are staged
// de-interleaved by quarter ([oc][q][s]), so four steps of A are one 128-bit
// read. The bias gradient is the same A values summed on the vector ALU.
// Each slice writes [M][9][C] partials that wgrad_partial_sum adds in slice
// order (deterministic).
#include <algorithm>

#include "buffer_ops.hpp"
#include "conv_slab.hpp"
#include "fastdiv.hpp"

namespace nrs {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kPRow = 16;                       // floats per staged image row
constexpr int kPPlane = 260;                    // floats per staged plane (16 x 16 + 4)
constexpr int kPCC = 16;                        // channels per chunk / per W block
constexpr int kPImg = kPCC * kPPlane;           // a chunk's 16 staged planes
constexpr int kPMB = 32;                        // output channels per D block
constexpr int kPWrow = 148;                     // floats per staged weight row (144 + 4)
constexpr int kPDBuf = kPImg + kPMB * kPWrow;   // floats per D chunk buffer
constexpr int kPWM = 64;                        // output channels per W block
constexpr int kPGrow = 52;                      // floats per (oc, quarter) gradient row
constexpr int kPGs = kPWM * 4 * kPGrow;         // staged gradient floats per image
constexpr int kPWBuf = kPGs + kPImg;            // floats per W image buffer
constexpr int kPImgs = 2;                       // images per W block (K slice)
constexpr int kPMaxSide = 14;                   // largest image side (16 with the halo)

struct PipeArgs {
    // D blocks: out[n][m][y][x] = sum_{c,tap} Wt(m, c, tap) img[n][c][y+dy-1][x+dx-1]
    //           (+ bias[m]) + beta * out
    const float* dimg;   // [N][dC][H][W]
    const float* dw;     // forward: [dM][dC][3][3]; input gradient: [dC][dM][3][3]
    const float* dbias;  // [dM] or null
    float* dout;         // [N][dM][H][W]
    int dC, dM, nd;      // reduction channels, output channels, D blocks
    float beta;
    // W blocks: part_w[slice][m][tap][c] = sum over the slice's pixels of
    //           g[n][m][y][x] * x[n][c][y+dy-1][x+dx-1]; part_b[slice][m] = sum g
    const float* wx;     // [N][wC][H][W]
    const float* wg;     // [N][wM][H][W]
    float* part_w;
    float* part_b;       // or null
    int wC, wM, nw;      // input channels, output channels, W blocks
    int N, H, W, P;
    // D blocks of an input gradient whose input is the 2x2 stride-2 max pool
    // of relu(y), y a "same" 3x3 stride-1 convolution of lo_x (c_lo
    // channels, 2H x 2W): each D block also writes that layer's weight and
    // bias gradient over its image and channels, with the gradient it just
    // computed as the pooled gradient (a pooled value's gradient reaches
    // its window's argmax when the pooled value is > 0: relu_grad).
    const int32_t* lo_am;     // [N][dM][H][W]: flat indices into [N][dM][2H][2W]
    const float* lo_pooled;   // [N][dM][H][W]: the pooled values (this layer's input)
    const float* lo_x;        // [N][c_lo][2H][2W]
    float* lo_part_w;         // [N][dM][9][c_lo]: per-image partials
    float* lo_part_b;         // [N][dM], or null
    FastDiv lo_div_w2;        // 2W
    FastDiv lo_div_plane;     // (2H + 2) * (2W + 2): a zero-padded plane
    FastDiv lo_div_wp;        // 2W + 2
};

// Tap t of a 3x3 window as an offset in a staged plane.
__device__ constexpr int tap_off(int t) { return (t / 3) * kPRow + t % 3; }

// One padded image row (16 floats: halo, W values, zeros) for staging:
// thread -> (plane p = tid >> 4, padded row y = tid & 15); loads of channel
// `ch` of the image behind `r`, zero outside.
struct RowStage {
    f32x2 v[kPMaxSide / 2];
    __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t r, int ch, int y, int H, int W) {
        const bool ok = (y >= 1) & (y <= H);
        const int src = (ch * H + y - 1) * W;
#pragma unroll
        for (int k = 0; k < kPMaxSide / 2; ++k)
            v[k] = buffer_load2(r, (ok & (2 * k < W)) ? (src + 2 * k) * 4 : kOutOfRange);
    }
    __device__ __forceinline__ void store(float* dst) const {
        *reinterpret_cast<f32x4*>(dst) = f32x4{0.0f, v[0][0], v[0][1], v[1][0]};
        *reinterpret_cast<f32x4*>(dst + 4) = f32x4{v[1][1], v[2][0], v[2][1], v[3][0]};
        *reinterpret_cast<f32x4*>(dst + 8) = f32x4{v[3][1], v[4][0], v[4][1], v[5][0]};
        *reinterpret_cast<f32x4*>(dst + 12) = f32x4{v[5][1], v[6][0], v[6][1], 0.0f};
    }
};

// ---- D blocks -------------------------------------------------------------

constexpr int kPWItems = kPMB * kPCC * 9 / 4;            // weight float4s per chunk (1152)
constexpr int kPWSlots = (kPWItems + 255) / 256;         // per thread (5, the last partial)

template <bool FLIP>
struct WeightStage {
    f32x4 v[kPWSlots];
    // chunk j's weights of output channels m0 .. m0+31
    __device__ __forceinline__ void issue(const PipeArgs& a, __amdgpu_buffer_rsrc_t r, int j, int m0,
                                          int tid) {
#pragma unroll
        for (int i = 0; i < kPWSlots; ++i) {
            const int e = tid + 256 * i;
            int src;
            if constexpr (!FLIP) {
                // row m: the chunk's 144 floats w[m0+m][16j .. 16j+15][0..8]
                const int m = e / 36, f = e - 36 * m;
                src = ((m0 + m) * a.dC + kPCC * j) * 9 + 4 * f;
            } else {
                // oc = 16j + o: the 288 floats w[oc][m0 .. m0+31][0..8]
                const int o = e / 72, f = e - 72 * o;
                src = ((kPCC * j + o) * a.dM + m0) * 9 + 4 * f;
            }
            v[i] = buffer_load4(r, e < kPWItems ? src * 4 : kOutOfRange);
        }
    }
    __device__ __forceinline__ void store(float* ws, int tid) const {
#pragma unroll
        for (int i = 0; i < kPWSlots; ++i) {
            const int e = tid + 256 * i;
            if (e >= kPWItems) continue;
            if constexpr (!FLIP) {
                const int m = e / 36, f = e - 36 * m;
                *reinterpret_cast<f32x4*>(ws + m * kPWrow + 4 * f) = v[i];
            } else {
                // element u of the item is w[oc][m0 + c][tap] with 4f + u = 9c + tap;
                // staged at row c, column 9*o + 8 - tap
                const int o = e / 72, f = e - 72 * o;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int k = 4 * f + u;
                    const int c = (k * 7282) >> 16;  // k / 9 for k < 32768
                    const int tap = k - 9 * c;
                    ws[c * kPWrow + 9 * o + 8 - tap] = v[i][u];
                }
            }
        }
    }
};

// The lower layer's weight and bias gradient over one image and the D
// block's 32 channels (see PipeArgs), in two parts: issue() loads, per
// thread, the argmax and pooled value of its pooled positions and its share
// of the lower input image; finish() stages the image with a zero halo in
// free LDS (xs) and reduces, given ot, the block's [32][P] gradient of the
// pooled values. Thread t takes channel t / 8 and the positions
// p = t % 8 + 8i in ascending order; a position's gradient goes to its
// window's argmax pixel (y, x) and multiplies the nine input values around
// it; the eight threads of a channel then add their sums in a fixed
// butterfly order.
template <int CLO>
struct LowerWgrad {
    static constexpr int kPos = (kPMaxSide * kPMaxSide + 7) / 8;  // positions per thread
    static constexpr int kImgItems = (CLO * (2 * kPMaxSide + 2) * (2 * kPMaxSide + 2) + 255) / 256;
    static_assert(CLO * (2 * kPMaxSide + 2) * (2 * kPMaxSide + 2) <= kPDBuf,
                  "the padded lower input fits a chunk buffer");
    float amv[kPos], pvv[kPos], xv[kImgItems];

    __device__ __forceinline__ void issue(const PipeArgs& a, int img, int m0) {
        const int tid = threadIdx.x, m = tid >> 3, part = tid & 7;
        const int P = a.P, H2 = 2 * a.H, W2 = 2 * a.W, plane = (H2 + 2) * (W2 + 2);
        // buffer bases uniform over the workgroup (a per-lane base would
        // make the compiler loop over the distinct bases of each load); the
        // lane's channel goes into the offset
        const int64_t blk = ((int64_t)img * a.dM + m0) * P;
        const auto ram =
            buffer_rsrc(reinterpret_cast<const float*>(a.lo_am) + blk, (int64_t)kPMB * P * 4);
        const auto rpv = buffer_rsrc(a.lo_pooled + blk, (int64_t)kPMB * P * 4);
        const auto rx =
            buffer_rsrc(a.lo_x + (int64_t)img * CLO * H2 * W2, (int64_t)CLO * H2 * W2 * 4);
#pragma unroll
        for (int i = 0; i < kPos; ++i) {
            const int p = part + 8 * i;
            amv[i] = buffer_load1(ram, p < P ? (m * P + p) * 4 : kOutOfRange);
            pvv[i] = buffer_load1(rpv, p < P ? (m * P + p) * 4 : kOutOfRange);
        }
        // the image with its zero halo (a load at kOutOfRange returns zero)
#pragma unroll
        for (int k = 0; k < kImgItems; ++k) {
            const int e = tid + 256 * k;
            uint32_t c, r, yy, xx;
            fast_divmod((uint32_t)e, a.lo_div_plane, c, r);
            fast_divmod(r, a.lo_div_wp, yy, xx);
            const int iy = (int)yy - 1, ix = (int)xx - 1;
            const bool ok = (e < CLO * plane) & ((unsigned)iy < (unsigned)H2) &
                            ((unsigned)ix < (unsigned)W2);
            xv[k] = buffer_load1(rx, ok ? (((int)c * H2 + iy) * W2 + ix) * 4 : kOutOfRange);
        }
    }

    __device__ __forceinline__ void finish(const PipeArgs& a, int img, int m0, const float* ot,
                                           float* xs) const {
        const int tid = threadIdx.x, m = tid >> 3, part = tid & 7;
        const int P = a.P, H2 = 2 * a.H, W2 = 2 * a.W, Wp = W2 + 2, plane = (H2 + 2) * Wp;
#pragma unroll
        for (int k = 0; k < kImgItems; ++k) {
            const int e = tid + 256 * k;
            if (e < CLO * plane) xs[e] = xv[k];
        }
        __syncthreads();

        const int64_t row = (int64_t)img * a.dM + m0 + m;
        const int pix0 = (int)(row * H2 * W2);  // flat index of this channel's first pixel
        float acc[CLO * 9];
#pragma unroll
        for (int k = 0; k < CLO * 9; ++k) acc[k] = 0.0f;
        float bsum = 0.0f;
#pragma unroll
        for (int i = 0; i < kPos; ++i) {
            const int p = part + 8 * i;
            const bool live = p < P;
            // the argmax as this channel's pixel, clamped into the image (the
            // forward wrote it there; the clamp keeps the LDS reads in bounds)
            const int loc = min(max(__builtin_bit_cast(int, amv[i]) - pix0, 0), H2 * W2 - 1);
            uint32_t y, x;
            fast_divmod((uint32_t)loc, a.lo_div_w2, y, x);
            const float g = (live & (pvv[i] > 0.0f)) ? ot[m * P + (live ? p : 0)] : 0.0f;
            bsum += g;
            const float* xp = xs + (int)y * Wp + (int)x;
#pragma unroll
            for (int c = 0; c < CLO; ++c)
#pragma unroll
                for (int t = 0; t < 9; ++t)
                    acc[c * 9 + t] += g * xp[c * plane + (t / 3) * Wp + t % 3];
        }
#pragma unroll
        for (int sh = 1; sh < 8; sh <<= 1) {
#pragma unroll
            for (int k = 0; k < CLO * 9; ++k) acc[k] += __shfl_xor(acc[k], sh);
            bsum += __shfl_xor(bsum, sh);
        }
        if (part == 0) {
            // [img][m][tap][c], the layout of the slice-order partial sum
#pragma unroll
            for (int c = 0; c < CLO; ++c)
#pragma unroll
                for (int t = 0; t < 9; ++t) a.lo_part_w[(row * 9 + t) * CLO + c] = acc[c * 9 + t];
            if (a.lo_part_b) a.lo_part_b[row] = bsum;
        }
    }
};

// (no lower layer)
template <>
struct LowerWgrad<0> {};

template <bool FLIP, int CLO = 0>
__device__ __forceinline__ void pipe_d_block(const PipeArgs& a, int bid, float* lds) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, l16 = lane & 15;
    const int mblocks = a.dM / kPMB;
    const int img = bid / mblocks, m0 = (bid - img * mblocks) * kPMB;
    const int H = a.H, W = a.W, P = a.P, nch = a.dC / kPCC;

    const auto rimg = buffer_rsrc(a.dimg + (int64_t)img * a.dC * P, (int64_t)a.dC * P * 4);
    const auto rw = buffer_rsrc(a.dw, (int64_t)a.dC * a.dM * 9 * 4);
    const int sp = tid >> 4, sy = tid & 15;
    RowStage rs;
    WeightStage<FLIP> wst;

    // chunk 0 staged, chunk 1's loads in flight
    rs.issue(rimg, sp, sy, H, W);
    wst.issue(a, rw, 0, m0, tid);
    __builtin_amdgcn_sched_barrier(0);
    rs.store(lds + sp * kPPlane + sy * kPRow);
    wst.store(lds + kPImg, tid);
    if (nch > 1) {
        rs.issue(rimg, kPCC + sp, sy, H, W);
        wst.issue(a, rw, 1, m0, tid);
    }
    __syncthreads();

    const int mb = wave & 1, row0 = (wave >> 1) * 7;
    int boff[7];
#pragma unroll
    for (int t = 0; t < 7; ++t) boff[t] = 4 * q * kPPlane + min(row0 + t, H - 1) * kPRow + l16;
    const int aoff = kPImg + (mb * 16 + l16) * kPWrow + 36 * q;
    float bias[4];  // loaded now, used in the epilogue
#pragma unroll
    for (int r = 0; r < 4; ++r) bias[r] = a.dbias ? a.dbias[m0 + mb * 16 + 4 * q + r] : 0.0f;
    f32x4 acc[7];
#pragma unroll
    for (int t = 0; t < 7; ++t) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    for (int j = 0; j < nch; ++j) {
        const float* cb = lds + (j & 1) * kPDBuf;
        // 36 steps: step s of quarter q is channel 4q + s/9, tap s%9. The B
        // values of step s+1 are read while step s's MFMAs run.
        f32x4 av = *reinterpret_cast<const f32x4*>(cb + aoff);
        float bv[7];
#pragma unroll
        for (int t = 0; t < 7; ++t) bv[t] = cb[boff[t]];
        // The schedule is pinned per step: the next step's reads go one
        // after each of this step's MFMAs, so the wave issues them while the
        // matrix core is busy. Left alone, the compiler sinks every read to
        // just before its MFMA and the LDS latency shows; issued as a block
        // between MFMA groups, they leave the matrix core idle.
#pragma unroll
        for (int s = 0; s < 36; ++s) {
            float bn[7];
            f32x4 an = av;
            if (s + 1 < 36) {
                const int off = ((s + 1) / 9) * kPPlane + tap_off((s + 1) % 9);
#pragma unroll
                for (int t = 0; t < 7; ++t) bn[t] = cb[boff[t] + off];
                if ((s + 1) % 4 == 0) an = *reinterpret_cast<const f32x4*>(cb + aoff + s + 1);
            }
#pragma unroll
            for (int t = 0; t < 7; ++t)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[s & 3], bv[t], acc[t], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 7; ++t) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (s + 1 < 36) {
#pragma unroll
                for (int t = 0; t < 7; ++t) bv[t] = bn[t];
                av = an;
            }
        }
        if (j + 1 < nch) {
            // the other buffer was last read by chunk j-1, which every wave
            // finished before the previous barrier
            float* nb = lds + ((j + 1) & 1) * kPDBuf;
            rs.store(nb + sp * kPPlane + sy * kPRow);
            wst.store(nb + kPImg, tid);
            if (j + 2 < nch) {
                rs.issue(rimg, kPCC * (j + 2) + sp, sy, H, W);
                wst.issue(a, rw, j + 2, m0, tid);
            }
            __syncthreads();
        }
    }

    // the lower layer's loads fly while the tile is stored
    LowerWgrad<CLO> lower;
    if constexpr (CLO > 0) lower.issue(a, img, m0);

    // epilogue: lane holds D[m = 4q + r][column l16] of each row tile. The
    // block's [32][P] output goes through the chunk buffer the last chunk did
    // not use (every wave finished reading it before the last barrier), so it
    // leaves as 128-bit stores of contiguous channel rows; + bias on the way
    // in, + beta * old on the way out (old values loaded before the round trip).
    float* ot = lds + (nch & 1) * kPDBuf;
    float* oimg = a.dout + ((int64_t)img * a.dM + m0) * P;
    const int P4 = P >> 2, total = kPMB * P4;
    constexpr int kOV = (kPMB * kPMaxSide * kPMaxSide / 4 + 255) / 256;  // float4s per thread
    // e / P4 as a multiply-shift: exact for e < 2^11, P4 <= 49
    const uint32_t p4inv = ((1u << 20) + P4 - 1) / P4;
    f32x4 old[kOV];
    if (a.beta != 0.0f) {
#pragma unroll
        for (int u = 0; u < kOV; ++u) {
            const int e = tid + 256 * u;
            const int m = (int)(((uint32_t)e * p4inv) >> 20), p4 = e - m * P4;
            old[u] = e < total ? *reinterpret_cast<const f32x4*>(oimg + (int64_t)m * P + 4 * p4)
                               : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    if (l16 < W) {
#pragma unroll
        for (int t = 0; t < 7; ++t) {
            const int oy = row0 + t;
            if (oy < H) {
#pragma unroll
                for (int r = 0; r < 4; ++r) ot[(mb * 16 + 4 * q + r) * P + oy * W + l16] = acc[t][r] + bias[r];
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kOV; ++u) {
        const int e = tid + 256 * u;
        if (e >= total) continue;
        const int m = (int)(((uint32_t)e * p4inv) >> 20), p4 = e - m * P4;
        f32x4 v = *reinterpret_cast<const f32x4*>(ot + m * P + 4 * p4);
        if (a.beta != 0.0f) v = v + a.beta * old[u];
        *reinterpret_cast<f32x4*>(oimg + (int64_t)m * P + 4 * p4) = v;
    }
    // the lower layer's gradients from the tile just stored (beta is 0 on
    // this path, so the tile is the gradient as written); the other chunk
    // buffer was last read by the last chunk, before the barrier above
    if constexpr (CLO > 0) lower.finish(a, img, m0, ot, lds + ((nch + 1) & 1) * kPDBuf);
}

// ---- W blocks -------------------------------------------------------------

constexpr int kPGItems = kPWM * kPGrow / 4 * 4;    // gradient float4 slots per image (64 x 52)
constexpr int kPGSlots = kPGItems / 256;           // 13 per thread

struct GradStage {
    f32x4 v[kPGSlots];
    // item e = (oc, s'): g[n][m0 + oc][4s' .. 4s'+3], zero for s' >= P/4
    __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t r, int img, int m0, int M, int P,
                                          int tid) {
        const int S4 = P >> 2;
#pragma unroll
        for (int i = 0; i < kPGSlots; ++i) {
            const int e = tid + 256 * i;
            const int oc = e / kPGrow, s = e - kPGrow * oc;
            const int src = ((img * M + m0 + oc) * P + 4 * s) * 4;
            v[i] = buffer_load4(r, s < S4 ? src : kOutOfRange);
        }
    }
    // staged de-interleaved: gs[oc][q][s'] = g[oc][4s' + q]
    __device__ __forceinline__ void store(float* gs, int tid) const {
#pragma unroll
        for (int i = 0; i < kPGSlots; ++i) {
            const int e = tid + 256 * i;
            const int oc = e / kPGrow, s = e - kPGrow * oc;
            float* d = gs + oc * 4 * kPGrow + s;
#pragma unroll
            for (int u = 0; u < 4; ++u) d[u * kPGrow] = v[i][u];
        }
    }
};

__device__ __forceinline__ void pipe_w_block(const PipeArgs& a, int bid, float* lds) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, l16 = lane & 15;
    const int cblocks = a.wC / kPCC, mblocks = a.wM / kPWM;
    const int cblk = bid % cblocks, rest = bid / cblocks;
    const int mblk = rest % mblocks, slice = rest / mblocks;
    const int c0 = cblk * kPCC, m0 = mblk * kPWM;
    const int img0 = slice * kPImgs, nimg = min(kPImgs, a.N - img0);
    const int H = a.H, W = a.W, P = a.P;

    // the slice's images as buffers (loads past the last image return zero)
    const auto rg = buffer_rsrc(a.wg, (int64_t)a.N * a.wM * P * 4);
    const auto rx = buffer_rsrc(a.wx + (int64_t)c0 * P, ((int64_t)a.N * a.wC - c0) * P * 4);
    const int sp = tid >> 4, sy = tid & 15;
    RowStage rs;
    GradStage gst;
    // input plane of channel c0 + sp of image n: plane n * wC + sp in rx
    rs.issue(rx, img0 * a.wC + sp, sy, H, W);
    gst.issue(rg, img0, m0, a.wM, P, tid);
    __builtin_amdgcn_sched_barrier(0);
    rs.store(lds + kPGs + sp * kPPlane + sy * kPRow);
    gst.store(lds, tid);
    if (nimg > 1) {
        rs.issue(rx, (img0 + 1) * a.wC + sp, sy, H, W);
        gst.issue(rg, img0 + 1, m0, a.wM, P, tid);
    }
    // staged-plane offset of pixel 4s + q (clamped to the last pixel, whose
    // gradient rows are zero past the image): table [q][s]
    if (tid < 4 * kPGrow) {
        const int tq = tid / kPGrow, ts = tid - kPGrow * tq;
        const int p = min(4 * ts + tq, P - 1), y = p / W;
        reinterpret_cast<int*>(lds + 2 * kPWBuf)[tid] = y * kPRow + (p - y * W);
    }
    __syncthreads();

    const int gb = (16 * wave + l16) * 4 * kPGrow + q * kPGrow;
    const int xb = kPGs + l16 * kPPlane;
    const int* ptab = reinterpret_cast<const int*>(lds + 2 * kPWBuf) + q * kPGrow;
    const int G = (P >> 2) >> 2, T = (P >> 2) & 3;  // whole groups of four steps, tail steps
    f32x4 acc[9];
#pragma unroll
    for (int t = 0; t < 9; ++t) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float bsum = 0.0f;

    // One step: this step's nine MFMAs (A = av_u, B = bv), with the next
    // step's nine B reads (at pixel offset pnext) placed one after each MFMA,
    // so the wave issues them while the matrix core is busy.
    auto step = [&](float av_u, float (&bv)[9], int pnext, const float* cb) {
        float bn[9];
#pragma unroll
        for (int t = 0; t < 9; ++t) bn[t] = cb[xb + pnext + tap_off(t)];
#pragma unroll
        for (int t = 0; t < 9; ++t)
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av_u, bv[t], acc[t], 0, 0, 0);
        bsum += av_u;
#pragma unroll
        for (int t = 0; t < 9; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < 9; ++t) bv[t] = bn[t];
    };

    for (int i = 0; i < nimg; ++i) {
        const float* cb = lds + (i & 1) * kPWBuf;
        // step s of quarter q is pixel 4s + q; its offset in a staged plane
        // comes from the table, four steps per 128-bit read
        i32x4 pc = *reinterpret_cast<const i32x4*>(ptab);
        f32x4 av = *reinterpret_cast<const f32x4*>(cb + gb);
        float bv[9];
#pragma unroll
        for (int t = 0; t < 9; ++t) bv[t] = cb[xb + pc[0] + tap_off(t)];
        for (int g = 0; g < G; ++g) {
            const int gn = min(g + 1, kPGrow / 4 - 1);
            const f32x4 an = *reinterpret_cast<const f32x4*>(cb + gb + 4 * gn);
            const i32x4 pn = *reinterpret_cast<const i32x4*>(ptab + 4 * gn);
            step(av[0], bv, pc[1], cb);
            step(av[1], bv, pc[2], cb);
            step(av[2], bv, pc[3], cb);
            step(av[3], bv, pn[0], cb);
            av = an;
            pc = pn;
        }
        // the last P/4 % 4 steps
        if (T > 0) step(av[0], bv, pc[1], cb);
        if (T > 1) step(av[1], bv, pc[2], cb);
        if (T > 2) step(av[2], bv, pc[3], cb);
        if (i + 1 < nimg) {
            float* nb = lds + ((i + 1) & 1) * kPWBuf;
            rs.store(nb + kPGs + sp * kPPlane + sy * kPRow);
            gst.store(nb, tid);
            if (i + 2 < nimg) {
                rs.issue(rx, (img0 + i + 2) * a.wC + sp, sy, H, W);
                gst.issue(rg, img0 + i + 2, m0, a.wM, P, tid);
            }
            __syncthreads();
        }
    }

    // partials: lane holds D[oc = 4q + r][channel l16] of each tap
    const int c = c0 + l16;
#pragma unroll
    for (int t = 0; t < 9; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + 16 * wave + 4 * q + r;
            a.part_w[(((int64_t)slice * a.wM + m) * 9 + t) * a.wC + c] = acc[t][r];
        }
    if (a.part_b && cblk == 0) {
        bsum += __shfl_xor(bsum, 16);
        bsum += __shfl_xor(bsum, 32);
        if (q == 0) a.part_b[(int64_t)slice * a.wM + m0 + 16 * wave + l16] = bsum;
    }
}

// With W blocks (the backward), the blocks are ordered slice by slice: a
// slice's W blocks, then the D blocks of its images. The output gradient of
// a slice is read by all of them (the W blocks' gradient operand, the D
// blocks' image), so when the grid is a multiple of 8 logical index L runs
// on XCD L / (grid / 8): workgroup ids are dealt to the 8 XCDs round-robin
// (id % 8), and consecutive logical blocks then share one XCD's L2.
template <bool FLIP, bool HAS_W, int CLO = 0>
__global__ __launch_bounds__(256) void conv_pipe_kernel(PipeArgs a) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int bid = blockIdx.x;
    if constexpr (HAS_W) {
        const int total = a.nw + a.nd;
        const int L = (total & 7) == 0 ? (bid & 7) * (total >> 3) + (bid >> 3) : bid;
        const int cblocks = a.wC / kPCC, wmblocks = a.wM / kPWM, dmblocks = a.dM / kPMB;
        const int wper = cblocks * wmblocks, per = wper + (a.nd > 0 ? kPImgs * dmblocks : 0);
        const int slice = L / per, r = L - slice * per;
        if (r < wper) {
            // pipe_w_block's decode: cblk fastest, then m-block, then slice
            const int mblk = r / cblocks, cblk = r - mblk * cblocks;
            pipe_w_block(a, (slice * wmblocks + mblk) * cblocks + cblk, lds);
            return;
        }
        // the slice's images in order, m-blocks fastest (pipe_d_block's
        // decode); the last slice of an odd batch has one image, and L stays
        // below the grid, so r never reaches its missing image's blocks
        const int rd = r - wper, img = slice * kPImgs + rd / dmblocks, mblk = rd % dmblocks;
        pipe_d_block<FLIP, CLO>(a, img * dmblocks + mblk, lds);
    } else {
        // an image's m-blocks (consecutive ids) folded onto one XCD, as above
        const int total = a.nd;
        pipe_d_block<FLIP>(a, (total & 7) == 0 ? (bid & 7) * (total >> 3) + (bid >> 3) : bid, lds);
    }
}

// Dynamic LDS of a launch: two chunk buffers of the input-gradient blocks,
// and with weight-gradient blocks their two image buffers and pixel-offset
// table.
size_t pipe_lds(bool has_w) {
    return sizeof(float) * (size_t)(has_w ? std::max(2 * kPWBuf + 4 * kPGrow, 2 * kPDBuf) : 2 * kPDBuf);
}

// Whether the device gives one workgroup that much LDS.
bool pipe_lds_fits(bool has_w) { return pipe_lds(has_w) <= lds_limit(); }

template <bool FLIP, bool HAS_W, int CLO = 0>
int launch_pipe(const PipeArgs& a) {
    auto fn = conv_pipe_kernel<FLIP, HAS_W, CLO>;
    const size_t lds = pipe_lds(a.nw > 0);
    static bool attr_set = false;
    if (!attr_set) {
        NRS_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                          hipFuncAttributeMaxDynamicSharedMemorySize,
                                          (int)pipe_lds(HAS_W)));
        attr_set = true;
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)(a.nw + a.nd)), dim3(256), lds, stream(), a);
    NRS_LAUNCH_CHECK("conv2d (chunk-pipelined)");
    return NRS_OK;
}

// The shapes the kernel takes: "same" 3x3 stride 1 over images of at most
// 14x14 with an even width of at least 4 and whole pixel quads.
bool pipe_geometry(int kh, int kw, int stride, int pad_h, int pad_w, int H, int W, int OH, int OW) {
    return kh == 3 && kw == 3 && stride == 1 && pad_h == 1 && pad_w == 1 && OH == H && OW == W &&
           H >= 1 && H <= kPMaxSide && W >= 4 && W <= kPMaxSide && W % 2 == 0 && (H * W) % 4 == 0;
}

}  // namespace

int pipe_conv(const SlabConv& s) {
    if (!pipe_geometry(s.kh, s.kw, s.stride, s.pad_h, s.pad_w, s.H, s.W, s.OH, s.OW) ||
        s.C % kPCC != 0 || s.C <= 0 || s.M % kPMB != 0 || s.M <= 0 || s.N <= 0 ||
        s.N * (s.M / kPMB) > 0x7fffffff || s.N * (int64_t)std::max(s.C, s.M) * s.H * s.W > 0x1fffffff ||
        ((uintptr_t)s.x & 7) != 0 || ((uintptr_t)s.out & 15) != 0 || !pipe_lds_fits(false))
        return kSlabUnsupported;
    PipeArgs a{};
    a.dimg = s.x;
    a.dw = s.w;
    a.dbias = s.bias;
    a.dout = s.out;
    a.dC = s.C;
    a.dM = s.M;
    a.nd = (int)(s.N * (s.M / kPMB));
    a.beta = s.beta;
    a.N = (int)s.N;
    a.H = s.H;
    a.W = s.W;
    a.P = s.H * s.W;
    return s.flip ? launch_pipe<true, false>(a) : launch_pipe<false, false>(a);
}

int pipe_backward(const SlabConv* d, const SlabWgrad& w, const PipeLower* lo) {
    if (!pipe_geometry(w.kh, w.kw, w.stride, w.pad, w.pad, w.H, w.W, w.OH, w.OW) || !w.dw ||
        w.C % kPMB != 0 || w.C <= 0 || w.M % kPWM != 0 || w.M <= 0 || w.N <= 0 ||
        w.N * (int64_t)std::max(w.C, w.M) * w.H * w.W > 0x1fffffff || ((uintptr_t)w.x & 7) != 0 ||
        ((uintptr_t)w.g & 15) != 0 || !pipe_lds_fits(true))
        return kSlabUnsupported;
    if (d && (d->x != w.g || d->C != w.M || d->M != w.C || !d->flip || ((uintptr_t)d->out & 15) != 0))
        return kSlabUnsupported;
    // the lower layer: its gradients come from d's result as written
    // (beta 0), its argmax indices [N][C][2H][2W] within int32
    if (lo && (!d || d->beta != 0.0f || lo->c_lo < 1 || lo->c_lo > 2 || !lo->dw || !lo->am ||
               !lo->pooled || !lo->x || w.N * (int64_t)w.C * 4 * w.H * w.W > 0x7fffffff))
        return kSlabUnsupported;
    const int P = w.H * w.W;
    const int64_t slices = (w.N + kPImgs - 1) / kPImgs;
    const int64_t nw = slices * (w.C / kPCC) * (w.M / kPWM);
    const int64_t nd = d ? w.N * (w.C / kPMB) : 0;
    if (nw + nd > 0x7fffffff) return kSlabUnsupported;
    const int64_t npw = (int64_t)w.M * 9 * w.C;
    const int64_t nlo = lo ? w.N * (int64_t)w.C * (9 * lo->c_lo + 1) : 0;
    float* part = workspace(sizeof(float) * (size_t)(slices * (npw + w.M) + nlo), 3);
    if (!part) return NRS_ERR_ALLOC;
    PipeArgs a{};
    if (d) {
        a.dimg = d->x;
        a.dw = d->w;
        a.dout = d->out;
        a.dC = d->C;
        a.dM = d->M;
        a.beta = d->beta;
    }
    a.nd = (int)nd;
    a.wx = w.x;
    a.wg = w.g;
    a.part_w = part;
    a.part_b = w.db ? part + slices * npw : nullptr;
    a.wC = w.C;
    a.wM = w.M;
    a.nw = (int)nw;
    a.N = (int)w.N;
    a.H = w.H;
    a.W = w.W;
    a.P = P;
    if (!lo) {
        int rc = launch_pipe<true, true>(a);
        if (rc) return rc;
        return wgrad_partial_sum(w.dw, w.db, part, a.part_b, (int)slices, w.M, w.C, 9, w.beta);
    }
    a.lo_am = lo->am;
    a.lo_pooled = lo->pooled;
    a.lo_x = lo->x;
    a.lo_part_w = part + slices * (npw + w.M);
    a.lo_part_b = lo->db ? a.lo_part_w + w.N * (int64_t)w.C * 9 * lo->c_lo : nullptr;
    a.lo_div_w2 = make_fastdiv((uint32_t)(2 * w.W));
    a.lo_div_plane = make_fastdiv((uint32_t)((2 * w.H + 2) * (2 * w.W + 2)));
    a.lo_div_wp = make_fastdiv((uint32_t)(2 * w.W + 2));
    int rc = lo->c_lo == 1 ? launch_pipe<true, true, 1>(a) : launch_pipe<true, true, 2>(a);
    if (rc) return rc;
    const WgradSumArgs up{w.dw, w.db, part, a.part_b, (int)slices, w.M, w.C, 9, w.beta};
    const WgradSumArgs low{lo->dw, lo->db, a.lo_part_w, a.lo_part_b, (int)w.N, w.C, lo->c_lo, 9,
                           lo->beta};
    return wgrad_partial_sum_pair(up, low);
}

}  // namespace nrs
