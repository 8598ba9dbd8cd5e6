// Checks akv::fast_div (csrc/fastdiv.h) against the C++ '/' operator: every
// divisor 1..65536 with every n below 65536 and the quotient boundaries
// k*d - 1, k*d, k*d + 1 of many k; divisors near each power of two up to 2^31
// and random divisors with boundary and random n up to 2^31 - 1.  Prints the
// mismatch count; exits 1 on any mismatch.
#include <stdint.h>
#include <stdio.h>

#include "fastdiv.h"

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint32_t rnd() {
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return (uint32_t)rng_state;
}

static long long checked = 0, bad = 0;
static void check(uint32_t n, uint32_t d, akv::FastDiv f) {
    if (n >= (1u << 31)) return;
    ++checked;
    if (akv::fast_div(n, f) != n / d) {
        if (bad < 10) printf("mismatch n=%u d=%u got %u want %u\n", n, d, akv::fast_div(n, f), n / d);
        ++bad;
    }
}
static void boundaries(uint32_t d, akv::FastDiv f, int nk) {
    const uint64_t kmax = ((1ull << 31) - 1) / d;
    for (int i = 0; i < nk; ++i) {
        const uint64_t k = i < nk / 2 ? (uint64_t)i : kmax - (uint64_t)(i - nk / 2);
        if (k > kmax + 1) continue;
        const uint64_t b = k * d;
        for (int e = -1; e <= 1; ++e) {
            const int64_t n = (int64_t)b + e;
            if (n >= 0 && n < (1ll << 31)) check((uint32_t)n, d, f);
        }
    }
    for (int i = 0; i < 64; ++i) check(rnd() >> 1, d, f);
    check((1u << 31) - 1, d, f);
}

int main(int argc, char **argv) {
    const bool dense = argc > 1;  // every n below 2^16 for every small divisor
    for (uint32_t d = 1; d <= 65536; ++d) {
        const akv::FastDiv f = akv::make_fast_div(d);
        if (dense || d <= 1024)
            for (uint32_t n = 0; n < 65536; ++n) check(n, d, f);
        boundaries(d, f, 64);
    }
    for (int p = 0; p <= 31; ++p)
        for (int e = -3; e <= 3; ++e) {
            const int64_t d = (1ll << p) + e;
            if (d < 1 || d > (1ll << 31)) continue;
            boundaries((uint32_t)d, akv::make_fast_div((uint32_t)d), 2000);
        }
    for (int i = 0; i < 200000; ++i) {
        uint32_t d = rnd() >> (1 + rnd() % 31);
        if (d == 0) d = 1;
        boundaries(d, akv::make_fast_div(d), 8);
    }
    printf("checked %lld; mismatches %lld\n", checked, bad);
    return bad ? 1 : 0;
}
