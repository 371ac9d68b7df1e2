// glibc's binary32 expf, restated so that host and device produce identical
// bits. The reference's CPU softmax calls std::exp on floats
// (src/kernels/cpu_ops.cpp:100), i.e. glibc's expf, whose algorithm (glibc >=
// 2.28, published with ARM's optimized-routines) is:
//   z = x * 32/ln2 (binary64);  k = round(z) via the 1.5*2^52 shift;  r = z - k;
//   s = 2^(k/32) from a 32-entry table of 2^(i/32) with the exponent of k
//   folded in;  exp(x) = s * (1 + C2 r + (C0 r + C1) r^2), rounded to binary32.
// The x86-64 build runs the FMA variant (every a*b+c above is one fma). The
// table holds 2^(i/32) rounded to binary64, minus i << 47 (so adding
// k << 47 yields the scaled bits). An exhaustive comparison with the host
// expf over every binary32 input is run at build time by gen_expf_fixups.c,
// which writes the few inputs where this restatement and glibc still disagree
// into expf_exceptions.h.
// Provenance: the table values are 2^(i/32) (a mathematical constant set) and
// the polynomial is the degree-3 fit published in ARM optimized-routines
// (math/expf.c, exp2f_data.c; Copyright (c) 2017-2018 Arm Limited,
// SPDX-License-Identifier: MIT OR Apache-2.0 WITH LLVM-exception), the code
// glibc >= 2.28 ships as sysdeps/ieee754/flt-32/e_expf.c.
#pragma once
#include <math.h>
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define UEXPF_QUAL __host__ __device__ static inline
#else
#define UEXPF_QUAL static inline
#endif

#define UOCR_EXP2_TAB32                                                                  \
    {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
     0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
     0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
     0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
     0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
     0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
     0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
     0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

// Main path for finite x in [-0x1.9fe368p6, 0x1.62e42ep6]; `tab` = UOCR_EXP2_TAB32.
UEXPF_QUAL float uocr_expf_core(float x, const uint64_t* tab) {
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    const double z = inv_ln2_n * xd;
    double kd = z + shift;
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    const double r = z - kd;
    const uint64_t t = tab[ki & 31] + (ki << 47);
    double s;
    memcpy(&s, &t, 8);
    const double zz = fma(c0, r, c1);
    const double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(zz, r2, y);
    y = y * s;
    return (float)y;
}

// Special cases of glibc's expf: NaN propagates, overflow above 0x1.62e42ep6,
// underflow to +0 below -0x1.9fe368p6.
UEXPF_QUAL int uocr_expf_special(float x, float* out) {
    if (x != x) {
        *out = x;
        return 1;
    }
    if (x > 88.72283935546875f) {
        *out = INFINITY;
        return 1;
    }
    if (x < -103.97208404541015625f) {
        *out = 0.0f;
        return 1;
    }
    return 0;
}
