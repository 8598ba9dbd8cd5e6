/*
 * Exhaustive check of the fast quantize kernel's reciprocal code path
 * (adaptive-kv-memory_amd/csrc/quant.hip: scale_of, mul_mix2, code2) against
 * the reference's fp16 arithmetic (akv/affine_quantizer.py:91-95):
 *
 *   reference:  scale = round16((max - min) / maxv)      (torch fp16: fp32 op, one RNE to fp16)
 *               code  = clamp(rint(round16(q / scale)), 0, maxv), NaN -> 0,  q = round16(x - min) >= 0
 *   kernel:     scale = round16(round32(d * round32(1 / maxv)))
 *               r     = round32(1 / scale)                          (IEEE fp32 division)
 *               t     = round16(q * r)                              (v_fma_mix: exact product, one rounding)
 *               code  = min(max(round16(t + 1024), 1024), 1024 + maxv) - 1024   (fp16 RNE at ulp 1)
 *
 * Part 1 runs over every finite fp16 d >= 0; part 2 over every q in
 * {non-negative finite fp16, +inf, NaN} and every scale in {0, positive finite
 * fp16} taken with stride `argv[1]` (1 = all 2^31 pairs).  Prints the counts of
 * mismatching scales and codes; exit status 1 if any.  With the argument
 * "round" it prints rnd16 of each hex double read from stdin (the test checks
 * this rounding against numpy's float16 conversion).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* fp16 bit pattern -> its exact value */
static double h2d(uint32_t b) {
    const int sgn = (b >> 15) & 1, e = (b >> 10) & 31, m = b & 1023;
    double v;
    if (e == 31) v = m ? NAN : INFINITY;
    else if (e == 0) v = ldexp((double)m, -24);
    else v = ldexp((double)(1024 + m), e - 25);
    return sgn ? -v : v;
}

/* x rounded to fp16 (round to nearest, ties to even; subnormal spacing 2^-24;
 * overflow to inf), returned as a double holding that fp16 value.  x must be
 * exactly representable in a double; the scaling by a power of two is exact and
 * nearbyint rounds ties to even in the default rounding mode. */
static double rnd16(double x) {
    if (x != x || isinf(x)) return x;
    const double a = fabs(x);
    if (a >= 65520.0) return copysign(INFINITY, x);
    int e;
    frexp(a, &e); /* a = f * 2^e, f in [0.5, 1) */
    int ue = e - 11;
    if (ue < -24) ue = -24;
    const double ulp = ldexp(1.0, ue);
    return copysign(nearbyint(a / ulp) * ulp, x);
}

static int code_ref(float q, float s, int maxv) {
    double d = rnd16((double)(q / s)); /* fp32 quotient, then RNE to fp16 */
    if (d != d) return 0;
    d = nearbyint(d);
    if (d < 0) d = 0;
    if (d > maxv) d = maxv;
    return (int)d;
}

static int code_kernel(float q, float s, int maxv) {
    const float r = 1.0f / s;
    const double t = rnd16((double)q * (double)r);   /* exact product (35 bits), one rounding */
    double u = rnd16((double)((float)t + 1024.0f));  /* fp16 add: fp32 sum (exact here) rounded once */
    if (u != u || u < 1024.0) u = 1024.0;            /* v_pk_max_f16 with 1024: NaN gives 1024 */
    if (u > 1024.0 + maxv) u = 1024.0 + maxv;
    return (int)(u - 1024.0);
}

int main(int argc, char **argv) {
    if (argc > 1 && strcmp(argv[1], "round") == 0) { /* rnd16 of each hex double on stdin */
        double x;
        while (scanf("%la", &x) == 1) printf("%a\n", rnd16(x));
        return 0;
    }
    const int stride = argc > 1 ? atoi(argv[1]) : 1;
    const int maxvs[3] = {3, 7, 15};
    long bad_scale = 0, bad_code = 0, pairs = 0;
    for (int m = 0; m < 3; ++m) {
        const float inv = 1.0f / (float)maxvs[m];
        for (uint32_t b = 0; b < 0x7C00; ++b) {
            const float d = (float)h2d(b);
            if (rnd16((double)(d / (float)maxvs[m])) != rnd16((double)(d * inv))) ++bad_scale;
        }
    }
    for (uint32_t sb = 0; sb < 0x7C00; sb += (uint32_t)stride) {
        const float s = (float)h2d(sb);
        for (uint32_t qb = 0; qb <= 0x7E00; ++qb) {
            if (qb > 0x7C00 && qb != 0x7E00) continue; /* +inf (0x7C00) and one NaN (0x7E00) */
            const float q = (float)h2d(qb);
            ++pairs;
            for (int m = 0; m < 3; ++m)
                if (code_ref(q, s, maxvs[m]) != code_kernel(q, s, maxvs[m])) ++bad_code;
        }
    }
    printf("scale mismatches %ld; code mismatches %ld over %ld (q, scale) pairs x 3 widths\n", bad_scale, bad_code,
           pairs);
    return (bad_scale || bad_code) ? 1 : 0;
}
