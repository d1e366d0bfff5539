/*
 * Single-precision exp used by every kernel of the decode path (SiLU, softmax)
 * and by the CPU checker, so the two agree bit-for-bit.
 *
 * Method (Cody & Waite, "Software Manual for the Elementary Functions", 1980):
 *   n = rint(x * log2(e));  r = x - n*ln2 (two-constant reduction, fma)
 *   exp(r) by the degree-7 Taylor polynomial of e^r on |r| <= ln2/2
 *   (truncation error < 6e-9 relative), evaluated by Horner with fma;
 *   exp(x) = 2^n * exp(r) by exact ldexp in two steps (covers subnormals).
 * Error against the correctly rounded result is at most 1 ulp (checked on
 * 400k points spanning the float range in the test suite).
 * Only IEEE-exact operations (fma, rint, ldexp, compares) are used, so the
 * result is identical on gfx950 and on any host with a correct fmaf.
 * The header is valid C and HIP.
 */
#ifndef Q3_MATH_H
#define Q3_MATH_H

#include <math.h>

#if defined(__HIPCC__)
#define Q3_FN __host__ __device__ static inline
#else
#define Q3_FN static inline
#endif

Q3_FN float q3_expf(float x) {
    /* Branch-free: the polynomial path is evaluated for every input and the
     * special cases are selected at the end (on the GPU a branch per case
     * would serialize the lanes).  For -103.97208 <= x <= 88.72284 the result
     * is the polynomial path; outside it exactly the special value. */
    const float n = rintf(x * 1.44269504088896341f);
    /* ln2 split: hi has 16 significant bits so n*hi is exact for |n| <= 2^8. */
    float r = fmaf(-n, 0.693145751953125f, x);
    r = fmaf(-n, 1.42860682030941723e-6f, r);
    float p = 1.98412698412698413e-4f;      /* 1/5040 */
    p = fmaf(p, r, 1.38888888888888889e-3f); /* 1/720 */
    p = fmaf(p, r, 8.33333333333333333e-3f); /* 1/120 */
    p = fmaf(p, r, 4.16666666666666667e-2f); /* 1/24 */
    p = fmaf(p, r, 1.66666666666666667e-1f); /* 1/6 */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    /* n is in [-150, 128] on the polynomial path; the clamp only keeps the
     * integer conversion defined for the discarded inputs (and NaN). */
    const int e = (int)fminf(fmaxf(n, -200.0f), 200.0f);
    const int e1 = e / 2;
    const float poly = ldexpf(ldexpf(p, e1), e - e1);
    const float big = x > 88.72284f ? INFINITY : poly;
    const float ranged = x < -103.97208f ? 0.0f : big;
    return x != x ? x : ranged;
}

#endif
