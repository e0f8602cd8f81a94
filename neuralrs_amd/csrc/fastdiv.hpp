// Division by a run-time constant without a division instruction sequence.
//
// A GPU has no integer divide: `n / d` with d a kernel argument expands to
// ~30 VALU instructions (64-bit: over 100). The index math of the gathered
// convolution operands divides every element, so the divisors are prepared
// once on the host and every division becomes one high multiply, one add and
// one shift (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, the round-up variant):
//
//   s = ceil(log2 d),  m = floor(2^32 * (2^s - d) / d) + 1,
//   n / d = (umulhi(n, m) + n) >> s        for 0 <= n < 2^31, 1 <= d < 2^31.
//
// With 2^(s-1) < d <= 2^s, m < 2^32 and umulhi(n, m) < n, so the sum cannot
// overflow 32 bits for n < 2^31. Usable from host and device code; the CPU
// test suite checks it exhaustively over small ranges and on edge values.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define NRS_HD __host__ __device__
#else
#define NRS_HD
#endif

namespace nrs {

struct FastDiv {
    uint32_t d = 1, m = 1, s = 0;
};

// Host side: prepares division by d (1 <= d < 2^31).
inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f;
    f.d = d;
    uint32_t s = 0;
    while ((1ull << s) < d) ++s;
    f.s = s;
    f.m = (uint32_t)((((1ull << s) - d) << 32) / d + 1);
    return f;
}

NRS_HD inline uint32_t fast_div(uint32_t n, const FastDiv& f) {
    // the high half of a 32x32 product: one v_mul_hi_u32 on the GPU
    const uint32_t hi = (uint32_t)(((uint64_t)n * f.m) >> 32);
    return (hi + n) >> f.s;
}

// n = q * d + r with q = n / d.
NRS_HD inline void fast_divmod(uint32_t n, const FastDiv& f, uint32_t& q, uint32_t& r) {
    q = fast_div(n, f);
    r = n - q * f.d;
}

}  // namespace nrs
