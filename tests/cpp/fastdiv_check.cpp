// Checks nrs::fast_div against the CPU's integer division: every divisor
// 1..4096 over every dividend 0..2^16 and the dividends next to each multiple
// near 2^31; the powers of two and their neighbours; and random pairs below
// 2^31. Prints "fastdiv ok" or the first mismatch; exit status 1 on mismatch.
#include <cstdio>
#include <random>

#include "fastdiv.hpp"

static bool check(uint32_t n, uint32_t d, const nrs::FastDiv& f) {
    const uint32_t q = nrs::fast_div(n, f);
    if (q != n / d) {
        std::printf("mismatch: %u / %u = %u, fast_div gives %u\n", n, d, n / d, q);
        return false;
    }
    return true;
}

int main() {
    const uint32_t top = 0x7fffffffu;  // largest dividend the contract allows
    for (uint32_t d = 1; d <= 4096; ++d) {
        const nrs::FastDiv f = nrs::make_fastdiv(d);
        for (uint32_t n = 0; n <= 65536; ++n)
            if (!check(n, d, f)) return 1;
        const uint32_t q = top / d;
        for (uint32_t k = (q > 2 ? q - 2 : 0); k <= q; ++k)
            for (int e = -1; e <= 1; ++e) {
                const int64_t n = (int64_t)k * d + e;
                if (n >= 0 && n <= top && !check((uint32_t)n, d, f)) return 1;
            }
    }
    for (int b = 0; b <= 30; ++b)
        for (int e = -1; e <= 1; ++e) {
            const int64_t d = (1ll << b) + e;
            if (d < 1 || d > top) continue;
            const nrs::FastDiv f = nrs::make_fastdiv((uint32_t)d);
            for (uint32_t n : {0u, 1u, (uint32_t)d - 1, (uint32_t)d, (uint32_t)d + 1, top - 1, top})
                if (n <= top && !check(n, (uint32_t)d, f)) return 1;
        }
    std::mt19937_64 rng(7);
    for (int it = 0; it < 20000000; ++it) {
        const uint32_t d = 1 + (uint32_t)(rng() % top);
        const uint32_t n = (uint32_t)(rng() % ((uint64_t)top + 1));
        if (!check(n, d, nrs::make_fastdiv(d))) return 1;
    }
    std::printf("fastdiv ok\n");
    return 0;
}
