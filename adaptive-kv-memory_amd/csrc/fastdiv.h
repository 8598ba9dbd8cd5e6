// Division of a non-negative integer n < 2^31 by a run-time constant d >= 1 as one
// high multiply, one add and one shift (Granlund and Montgomery, "Division by
// invariant integers using multiplication", PLDI 1994, section 4, the 33-bit
// multiplier m' = 2^32 + mul):
//
//   l = ceil(log2 d),  m' = floor(2^(32+l) / d) + 1,  n / d = floor(m' n / 2^(32+l))
//
// which holds for every 0 <= n < 2^32 because 2^(32+l) < m' d <= 2^(32+l) + 2^l.
// With mul = m' - 2^32 < 2^32 the quotient is (mulhi(mul, n) + n) >> l; mulhi(mul, n)
// <= n, so the add stays below 2^32 when n < 2^31.  The host computes (mul, l) once per
// launch; the kernels use it where a workgroup or lane id is split into coordinates.
// Plain constexpr C++ (usable on the host, in host tests, and in device code).
#pragma once

#include <stdint.h>

namespace akv {

struct FastDiv {
    uint32_t mul;    // m' - 2^32
    uint32_t shift;  // l
    uint32_t d;
};

constexpr FastDiv make_fast_div(uint32_t d) {
    uint32_t l = 0;
    while (l < 31 && ((uint64_t)1 << l) < d) ++l;
    const uint64_t m = ((((uint64_t)1 << 32) * (((uint64_t)1 << l) - d)) / d) + 1;
    return FastDiv{(uint32_t)m, l, d};
}

// n / d for 0 <= n < 2^31.
constexpr uint32_t fast_div(uint32_t n, FastDiv f) {
    return ((uint32_t)(((uint64_t)n * f.mul) >> 32) + n) >> f.shift;
}

}  // namespace akv
