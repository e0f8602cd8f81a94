// Slab weight gradient: the standalone kernel, the fixed-order partial sum
// and the host planner (the per-workgroup body is in conv_slab_wgrad.hpp).
#include <algorithm>

#include "conv_slab_wgrad.hpp"

namespace nrs {
namespace {

template <int TAPW, bool VEC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void conv_slab_wgrad_kernel(WgradArgs a) {
    wgrad_block<TAPW, VEC>(a, blockIdx.x, blockIdx.y, blockIdx.z);
}

// dw[m][c][tap] += sum over slices of part_w[slice][m][tap][c] and
// db[m] += sum over slices of part_b[slice][m]: the slices are split into
// kSumGroups contiguous groups summed in parallel (ascending within a group),
// then the group sums are added in group order, so the result is
// deterministic. A thread issues the loads of up to kSumBatch slices (in
// runs of 8, as many runs as its group needs) before adding any, so a group
// of that size costs one memory round trip.
constexpr int kSumGroups = 16, kSumBatch = 32;

// The 64 outputs from `base` on of one partial sum (every thread of the
// workgroup takes part: the barriers are uniform).
__device__ __forceinline__ void wgrad_sum_at(const WgradSumArgs& p, int base) {
    __shared__ float red[kSumGroups][64];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int M = p.M, C = p.C, taps = p.taps, slices = p.slices;
    const int nw = p.dw ? M * taps * C : 0, total = nw + (p.db ? M : 0);
    const int per = (slices + kSumGroups - 1) / kSumGroups;
    const int s0 = min(slices, ty * per), s1 = min(slices, s0 + per);
    const int e = base + tx;
    const bool is_w = e < nw;
    const float* part = is_w ? p.part_w + e : p.part_b + (e - nw);
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
            dst = p.dw + ((int64_t)m * C + c) * taps + tap;
        } else {
            dst = p.db + (e - nw);
        }
        // beta 0 writes without reading the old gradient
        *dst = p.beta != 0.0f ? r + p.beta * *dst : r;
    }
    __syncthreads();
}

__global__ __launch_bounds__(64 * kSumGroups) void wgrad_sum_kernel(WgradSumArgs p) {
    wgrad_sum_at(p, blockIdx.x * 64);
}

// Two partial sums in one launch: blocks [0, blocks0) take p0, the rest p1.
__global__ __launch_bounds__(64 * kSumGroups) void wgrad_sum_pair_kernel(WgradSumArgs p0,
                                                                         WgradSumArgs p1,
                                                                         int blocks0) {
    const int b = blockIdx.x;
    if (b < blocks0)
        wgrad_sum_at(p0, b * 64);
    else
        wgrad_sum_at(p1, (b - blocks0) * 64);
}

// LDS of one workgroup: at most 160 KiB (gfx950's whole LDS), and no more
// than the device allows.
int64_t lds_budget() { return (int64_t)std::min<size_t>(160 * 1024, lds_limit()); }

}  // namespace

int plan_slab_wgrad(const SlabWgrad& s, WgradPlan& p) {
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
    while (band_rows > 1 && lds_bytes(band_rows, KP, CS, slab_rows) > lds_budget()) --band_rows;
    if (lds_bytes(band_rows, KP, CS, slab_rows) > lds_budget()) return kSlabUnsupported;
    const int64_t bands = (s.OH + band_rows - 1) / band_rows;
    const int64_t slices = s.N * bands;
    const int64_t cparts = (s.C + kWgC - 1) / kWgC, ntg = (taps + kTapw - 1) / kTapw;
    const int64_t mblocks = (s.M + kWgM - 1) / kWgM;
    const int64_t nw = (int64_t)s.M * taps * s.C;
    if (slices > INT32_MAX || cparts * ntg > 65535 || mblocks > 65535 ||
        slices * cparts * ntg * mblocks > INT32_MAX ||
        slices * (nw + s.M) > ((int64_t)1 << 31) || (int64_t)s.C * s.H * s.W > INT32_MAX / 4 ||
        (int64_t)s.M * s.OH * s.OW > INT32_MAX / 4 || nw + s.M > INT32_MAX)
        return kSlabUnsupported;

    float* part = workspace(sizeof(float) * (size_t)(slices * (nw + s.M)), 3);
    if (!part) return NRS_ERR_ALLOC;
    WgradArgs& a = p.a;
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
    p.gx = (unsigned)slices;
    p.gy = (unsigned)(cparts * ntg);
    p.gz = (unsigned)mblocks;
    p.lds = (size_t)lds_bytes(band_rows, KP, CS, slab_rows);
    p.slices = (int)slices;
    p.nw = nw;
    return NRS_OK;
}

int slab_wgrad_sum(const SlabWgrad& s, const WgradPlan& p) {
    // dW and (when requested) dB from the partials
    return wgrad_partial_sum(s.dw, s.db, p.a.part_w, p.a.part_w + (int64_t)p.slices * p.nw,
                             p.slices, s.M, s.C, p.a.taps, s.beta);
}

int slab_wgrad(const SlabWgrad& s) {
    WgradPlan p;
    const int rc = plan_slab_wgrad(s, p);
    if (rc) return rc;
    auto fn = p.a.vec_g ? conv_slab_wgrad_kernel<kTapw, true> : conv_slab_wgrad_kernel<kTapw, false>;
    static bool attr_set[2] = {false, false};
    if (!attr_set[p.a.vec_g]) {
        NRS_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                          hipFuncAttributeMaxDynamicSharedMemorySize,
                                          (int)lds_budget()));
        attr_set[p.a.vec_g] = true;
    }
    hipLaunchKernelGGL(fn, dim3(p.gx, p.gy, p.gz), dim3(256), p.lds, stream(), p.a);
    NRS_LAUNCH_CHECK("conv2d weight gradient (slab)");
    return slab_wgrad_sum(s, p);
}

namespace {
int64_t sum_blocks(const WgradSumArgs& p) {
    const int64_t total = (p.dw ? (int64_t)p.M * p.taps * p.C : 0) + (p.db ? p.M : 0);
    return (total + 63) / 64;
}
}  // namespace

int wgrad_partial_sum(float* dw, float* db, const float* part_w, const float* part_b, int slices,
                      int M, int C, int taps, float beta) {
    const WgradSumArgs p{dw, db, part_w, part_b, slices, M, C, taps, beta};
    const int64_t blocks = sum_blocks(p);
    if (blocks == 0) return NRS_OK;
    hipLaunchKernelGGL(wgrad_sum_kernel, dim3((unsigned)blocks), dim3(64 * kSumGroups), 0,
                       stream(), p);
    NRS_LAUNCH_CHECK("conv2d weight gradient (sum)");
    return NRS_OK;
}

int wgrad_partial_sum_pair(const WgradSumArgs& p0, const WgradSumArgs& p1) {
    const int64_t b0 = sum_blocks(p0), b1 = sum_blocks(p1);
    if (b0 + b1 == 0) return NRS_OK;
    hipLaunchKernelGGL(wgrad_sum_pair_kernel, dim3((unsigned)(b0 + b1)), dim3(64 * kSumGroups), 0,
                       stream(), p0, p1, (int)b0);
    NRS_LAUNCH_CHECK("conv2d weight gradient (sum)");
    return NRS_OK;
}

}  // namespace nrs
