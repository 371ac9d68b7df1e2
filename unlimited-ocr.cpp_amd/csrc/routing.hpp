// Routing arithmetic shared by the router kernels: glibc-exact expf and the
// reference's greedy top-k order.
#pragma once
#include "common.hpp"
#include "expf_exceptions.h"

namespace uocr_hip {

// Correctly rounded binary32 square root. __fsqrt_rn / sqrtf compile to the
// hardware v_sqrt_f32 here, which is only faithful (<= 1 ulp); the reference's
// std::sqrt (sqrtss) is correctly rounded. The hardware value is corrected by
// comparing `a` with the squares of the neighbouring rounding midpoints, which
// binary64 holds exactly (25-bit midpoints, 50-bit squares).
__device__ __forceinline__ float sqrt_rn(float a) {
    float s = __builtin_sqrtf(a);
    if (!(a > 0.0f) || !(a < INFINITY)) return s;
    const double ad = (double)a;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const float up = __uint_as_float(__float_as_uint(s) + 1u);
        const float dn = __uint_as_float(__float_as_uint(s) - 1u);
        const double mu = ((double)s + (double)up) * 0.5, ml = ((double)s + (double)dn) * 0.5;
        if (ad > mu * mu) s = up;
        else if (ad < ml * ml) s = dn;
        else break;
    }
    return s;
}

// glibc's expf bits (uexpf.h restatement + the build-time exception list);
// `tab` is UOCR_EXP2_TAB32, staged in LDS by the caller.
__device__ __forceinline__ float ref_expf(float x, const uint64_t* tab) {
    float y;
    if (uocr_expf_special(x, &y)) return y;
    y = uocr_expf_core(x, tab);
    constexpr uint32_t exc[][2] = UOCR_EXPF_EXCEPTIONS;
    const uint32_t b = __float_as_uint(x);
#pragma unroll
    for (int i = 0; i < UOCR_EXPF_N_EXCEPTIONS; ++i)
        if (b == exc[i][0]) y = __uint_as_float(exc[i][1]);
    return y;
}

// 2^(i/32) table of the expf restatement, for staging into LDS
__device__ __constant__ static const uint64_t uocr_exp2_tab[32] = UOCR_EXP2_TAB32;

// Greedy top-k of the reference (strict '>' scan, first maximum wins,
// moe_decoder.cpp:264-277) selects experts in order of (p descending, index
// ascending); lane e's position in that order is the number of experts that
// beat it. p[] holds the scores in LDS; returns the rank of `pe` (lane e).
__device__ __forceinline__ int greedy_rank(const float* p, int E, int e, float pe) {
    int rank = 0;
    for (int j = 0; j < E; ++j) {
        const float q = p[j];
        rank += (q > pe || (q == pe && j < e)) ? 1 : 0;
    }
    return rank;
}

// The same rank over exactly 64 scores in LDS (16-byte aligned): the reads are
// independent 16-byte broadcasts, issued together.
__device__ __forceinline__ int greedy_rank64(const float* p, int e, float pe) {
    int part[4] = {0, 0, 0, 0};  // four independent counting chains
#pragma unroll
    for (int j4 = 0; j4 < 16; ++j4) {
        const f32x4 q = reinterpret_cast<const f32x4*>(p)[j4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = 4 * j4 + i;
            part[i] += (q[i] > pe || (q[i] == pe && j < e)) ? 1 : 0;
        }
    }
    return (part[0] + part[1]) + (part[2] + part[3]);
}

// sum of p[0..E) in index order (E <= 64; p 16-byte aligned, zero-padded to 64)
__device__ __forceinline__ float ordered_sum64(const float* p, int E) {
    f32x4 q[16];
#pragma unroll
    for (int j4 = 0; j4 < 16; ++j4) q[j4] = reinterpret_cast<const f32x4*>(p)[j4];
    float s = 0.0f;
#pragma unroll
    for (int j4 = 0; j4 < 16; ++j4)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (4 * j4 + i < E) s += q[j4][i];
    return s;
}

}  // namespace uocr_hip
