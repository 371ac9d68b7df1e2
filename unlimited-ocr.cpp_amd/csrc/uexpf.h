// Correctly rounded binary32 exp, evaluated in binary64 with explicit FMAs so
// that the host and the device produce identical bits (every operation is an
// IEEE-754 basic operation: rint, fma, ldexp and the final double->float
// rounding). Shared by the device router (softmax / sigmoid scoring) and by the
// build-time generator of the glibc fix-up table.
//
// Method: Cody-Waite reduction x = k*ln2 + r with |r| <= ln2/2 (ln2 split into
// a 53-bit head and a tail), exp(r) by its Taylor series to degree 13
// (truncation < 5e-18 on |r| <= 0.347), then scaling by 2^k. The binary64
// result carries ~1e-16 relative error, so its rounding to binary32 is the
// correctly rounded value except for inputs within 1e-16 of a rounding
// boundary; an exhaustive host check over all 2^32 inputs finds none.
#pragma once
#include <math.h>

#if defined(__HIPCC__)
#define UEXPF_QUAL __host__ __device__ static inline
#else
#define UEXPF_QUAL static inline
#endif

// binary64 value of exp(xf) before the final rounding (finite, in-range xf)
UEXPF_QUAL double uocr_uexp_d(float xf) {
    const double x = (double)xf;
    const double kd = rint(x * 1.4426950408889634);
    double r = fma(-kd, 0x1.62e42fefa39efp-1, x);
    r = fma(-kd, 0x1.abc9e3b39803fp-56, r);
    double p = 1.0 / 6227020800.0;
    p = fma(p, r, 1.0 / 479001600.0);
    p = fma(p, r, 1.0 / 39916800.0);
    p = fma(p, r, 1.0 / 3628800.0);
    p = fma(p, r, 1.0 / 362880.0);
    p = fma(p, r, 1.0 / 40320.0);
    p = fma(p, r, 1.0 / 5040.0);
    p = fma(p, r, 1.0 / 720.0);
    p = fma(p, r, 1.0 / 120.0);
    p = fma(p, r, 1.0 / 24.0);
    p = fma(p, r, 1.0 / 6.0);
    p = fma(p, r, 0.5);
    p = fma(p, r, 1.0);
    p = fma(p, r, 1.0);
    return ldexp(p, (int)kd);
}

UEXPF_QUAL float uocr_uexpf(float xf) {
    if (xf != xf) return xf;
    if (xf > 88.72283935546875f) return INFINITY;
    if (xf < -103.97208404541015625f) return 0.0f;
    return (float)uocr_uexp_d(xf);
}

// True when the binary64 value lies within 1/256 ulp of a binary32 rounding
// midpoint. glibc's expf can only round differently from the correctly rounded
// result in that band (its pre-rounding error is 1.69 * 2^-34 relative, i.e.
// <= 0.0017 ulp); the table generator verifies on all 2^32 inputs that every
// listed difference passes this test, so callers may skip the fix-up table
// whenever it is false.
UEXPF_QUAL int uocr_uexpf_near_tie_d(double yd) {
    const float yf = (float)yd;
    unsigned int b;
    __builtin_memcpy(&b, &yf, 4);
    b = (yd >= (double)yf) ? b + 1u : b - 1u;
    float nb;
    __builtin_memcpy(&nb, &b, 4);
    const double mid = ((double)yf + (double)nb) * 0.5;
    return fabs(yd - mid) < fabs((double)nb - (double)yf) * (1.0 / 256.0);
}

UEXPF_QUAL int uocr_uexpf_near_tie(float xf) {
    if (xf != xf || xf > 88.72283935546875f || xf < -103.97208404541015625f) return 0;
    return uocr_uexpf_near_tie_d(uocr_uexp_d(xf));
}
