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


// Maximum of v over the 64 lanes, in every lane: DPP steps inside each 16-lane
// row (quad swaps, half-row and row mirrors), then the four row maxima. fmaxf
// drops NaN like the reference's strict '>' scan never picks one.
__device__ __forceinline__ float wave_max64(float v) {
    // (bound_ctrl off and every row enabled: each lane reads its partner)
#define UOCR_MAXSTEP(CTRL) \
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false)))
    UOCR_MAXSTEP(0xB1);   // quad_perm [1,0,3,2]
    UOCR_MAXSTEP(0x4E);   // quad_perm [2,3,0,1]
    UOCR_MAXSTEP(0x141);  // row_half_mirror
    UOCR_MAXSTEP(0x140);  // row_mirror
#undef UOCR_MAXSTEP
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Scoring (src/kernels/cpu_ops.cpp:93-106 softmax, or sigmoid) and greedy
// top-k (src/engine/moe_decoder.cpp:264-287) of one token by ONE wave, lane e
// holding expert e's logit `acc` (E <= 64). The greedy scan (strict '>', so
// the lowest index wins a tie; the pick is then removed) is K rounds of a wave
// maximum and the lowest lane holding it. sc: 64 floats of LDS, 16-byte
// aligned, private to the wave. Returns the lane's position in the selection
// (kTopkNone if not picked) and, in lanes j < K, the j-th pick's weight after
// the optional renormalisation and the scaling factor.
constexpr int kTopkNone = 64;
struct WaveTopk {
    int rank;
    float w;
};
__device__ __forceinline__ WaveTopk wave_topk(float acc, int E, int K, bool sigmoid, bool norm_topk_prob,
                                              float scaling, float* sc, const uint64_t* etab) {
    const int lane = threadIdx.x & 63;
    float p;
    if (sigmoid) {
        p = __fdiv_rn(1.0f, 1.0f + ref_expf(-acc, etab));
    } else {
        const float mx = wave_max64(lane < E ? acc : -INFINITY);
        const float ev = lane < E ? ref_expf(acc - mx, etab) : 0.0f;
        sc[lane] = ev;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        const float sum = ordered_sum64(sc, E);  // expert order
        p = ev * __fdiv_rn(1.0f, sum);
    }
    float rem = lane < E ? p : -INFINITY;
    float wsel = 0.0f, wsum = 0.0f;
    int rank = kTopkNone;
    for (int j = 0; j < K; ++j) {
        const float m = wave_max64(rem);
        const uint64_t tie = __ballot(rem == m);
        const int win = (int)__builtin_ctzll(tie);
        if (lane == win) {
            rank = j;
            rem = -INFINITY;
        }
        if (lane == j) wsel = m;
        wsum += m;  // moe_decoder.cpp:280-281, selection order
    }
    float wj = wsel;
    if (K > 1 && norm_topk_prob) {  // moe_decoder.cpp:280-284
        wj = __fdiv_rn(wj, wsum + 1e-20f) * scaling;
    } else {
        wj *= scaling;
    }
    return WaveTopk{rank, wj};
}

// One 128-column chunk of the router chain (lane e: its expert, columns
// ascending) with the multiply-accumulate step MAC(x, w) spelled by the caller.
#define UOCR_RCHUNK(MAC) \
    "s_waitcnt lgkmcnt(0)\n" \
    "ds_read_b128 v[64:67], %[w] offset:0\n" \
    "ds_read_b128 v[68:71], %[x] offset:0\n" \
    "ds_read_b128 v[72:75], %[w] offset:1024\n" \
    "ds_read_b128 v[76:79], %[x] offset:16\n" \
    "ds_read_b128 v[80:83], %[w] offset:2048\n" \
    "ds_read_b128 v[84:87], %[x] offset:32\n" \
    "ds_read_b128 v[88:91], %[w] offset:3072\n" \
    "ds_read_b128 v[92:95], %[x] offset:48\n" \
    "ds_read_b128 v[96:99], %[w] offset:4096\n" \
    "ds_read_b128 v[100:103], %[x] offset:64\n" \
    "ds_read_b128 v[104:107], %[w] offset:5120\n" \
    "ds_read_b128 v[108:111], %[x] offset:80\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v68", "v64") \
    MAC("v69", "v65") \
    MAC("v70", "v66") \
    MAC("v71", "v67") \
    "ds_read_b128 v[64:67], %[w] offset:6144\n" \
    "ds_read_b128 v[68:71], %[x] offset:96\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v76", "v72") \
    MAC("v77", "v73") \
    MAC("v78", "v74") \
    MAC("v79", "v75") \
    "ds_read_b128 v[72:75], %[w] offset:7168\n" \
    "ds_read_b128 v[76:79], %[x] offset:112\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v84", "v80") \
    MAC("v85", "v81") \
    MAC("v86", "v82") \
    MAC("v87", "v83") \
    "ds_read_b128 v[80:83], %[w] offset:8192\n" \
    "ds_read_b128 v[84:87], %[x] offset:128\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v92", "v88") \
    MAC("v93", "v89") \
    MAC("v94", "v90") \
    MAC("v95", "v91") \
    "ds_read_b128 v[88:91], %[w] offset:9216\n" \
    "ds_read_b128 v[92:95], %[x] offset:144\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v100", "v96") \
    MAC("v101", "v97") \
    MAC("v102", "v98") \
    MAC("v103", "v99") \
    "ds_read_b128 v[96:99], %[w] offset:10240\n" \
    "ds_read_b128 v[100:103], %[x] offset:160\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v108", "v104") \
    MAC("v109", "v105") \
    MAC("v110", "v106") \
    MAC("v111", "v107") \
    "ds_read_b128 v[104:107], %[w] offset:11264\n" \
    "ds_read_b128 v[108:111], %[x] offset:176\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v68", "v64") \
    MAC("v69", "v65") \
    MAC("v70", "v66") \
    MAC("v71", "v67") \
    "ds_read_b128 v[64:67], %[w] offset:12288\n" \
    "ds_read_b128 v[68:71], %[x] offset:192\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v76", "v72") \
    MAC("v77", "v73") \
    MAC("v78", "v74") \
    MAC("v79", "v75") \
    "ds_read_b128 v[72:75], %[w] offset:13312\n" \
    "ds_read_b128 v[76:79], %[x] offset:208\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v84", "v80") \
    MAC("v85", "v81") \
    MAC("v86", "v82") \
    MAC("v87", "v83") \
    "ds_read_b128 v[80:83], %[w] offset:14336\n" \
    "ds_read_b128 v[84:87], %[x] offset:224\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v92", "v88") \
    MAC("v93", "v89") \
    MAC("v94", "v90") \
    MAC("v95", "v91") \
    "ds_read_b128 v[88:91], %[w] offset:15360\n" \
    "ds_read_b128 v[92:95], %[x] offset:240\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v100", "v96") \
    MAC("v101", "v97") \
    MAC("v102", "v98") \
    MAC("v103", "v99") \
    "ds_read_b128 v[96:99], %[w] offset:16384\n" \
    "ds_read_b128 v[100:103], %[x] offset:256\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v108", "v104") \
    MAC("v109", "v105") \
    MAC("v110", "v106") \
    MAC("v111", "v107") \
    "ds_read_b128 v[104:107], %[w] offset:17408\n" \
    "ds_read_b128 v[108:111], %[x] offset:272\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v68", "v64") \
    MAC("v69", "v65") \
    MAC("v70", "v66") \
    MAC("v71", "v67") \
    "ds_read_b128 v[64:67], %[w] offset:18432\n" \
    "ds_read_b128 v[68:71], %[x] offset:288\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v76", "v72") \
    MAC("v77", "v73") \
    MAC("v78", "v74") \
    MAC("v79", "v75") \
    "ds_read_b128 v[72:75], %[w] offset:19456\n" \
    "ds_read_b128 v[76:79], %[x] offset:304\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v84", "v80") \
    MAC("v85", "v81") \
    MAC("v86", "v82") \
    MAC("v87", "v83") \
    "ds_read_b128 v[80:83], %[w] offset:20480\n" \
    "ds_read_b128 v[84:87], %[x] offset:320\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v92", "v88") \
    MAC("v93", "v89") \
    MAC("v94", "v90") \
    MAC("v95", "v91") \
    "ds_read_b128 v[88:91], %[w] offset:21504\n" \
    "ds_read_b128 v[92:95], %[x] offset:336\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v100", "v96") \
    MAC("v101", "v97") \
    MAC("v102", "v98") \
    MAC("v103", "v99") \
    "ds_read_b128 v[96:99], %[w] offset:22528\n" \
    "ds_read_b128 v[100:103], %[x] offset:352\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v108", "v104") \
    MAC("v109", "v105") \
    MAC("v110", "v106") \
    MAC("v111", "v107") \
    "ds_read_b128 v[104:107], %[w] offset:23552\n" \
    "ds_read_b128 v[108:111], %[x] offset:368\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v68", "v64") \
    MAC("v69", "v65") \
    MAC("v70", "v66") \
    MAC("v71", "v67") \
    "ds_read_b128 v[64:67], %[w] offset:24576\n" \
    "ds_read_b128 v[68:71], %[x] offset:384\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v76", "v72") \
    MAC("v77", "v73") \
    MAC("v78", "v74") \
    MAC("v79", "v75") \
    "ds_read_b128 v[72:75], %[w] offset:25600\n" \
    "ds_read_b128 v[76:79], %[x] offset:400\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v84", "v80") \
    MAC("v85", "v81") \
    MAC("v86", "v82") \
    MAC("v87", "v83") \
    "ds_read_b128 v[80:83], %[w] offset:26624\n" \
    "ds_read_b128 v[84:87], %[x] offset:416\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v92", "v88") \
    MAC("v93", "v89") \
    MAC("v94", "v90") \
    MAC("v95", "v91") \
    "ds_read_b128 v[88:91], %[w] offset:27648\n" \
    "ds_read_b128 v[92:95], %[x] offset:432\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v100", "v96") \
    MAC("v101", "v97") \
    MAC("v102", "v98") \
    MAC("v103", "v99") \
    "ds_read_b128 v[96:99], %[w] offset:28672\n" \
    "ds_read_b128 v[100:103], %[x] offset:448\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v108", "v104") \
    MAC("v109", "v105") \
    MAC("v110", "v106") \
    MAC("v111", "v107") \
    "ds_read_b128 v[104:107], %[w] offset:29696\n" \
    "ds_read_b128 v[108:111], %[x] offset:464\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v68", "v64") \
    MAC("v69", "v65") \
    MAC("v70", "v66") \
    MAC("v71", "v67") \
    "ds_read_b128 v[64:67], %[w] offset:30720\n" \
    "ds_read_b128 v[68:71], %[x] offset:480\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v76", "v72") \
    MAC("v77", "v73") \
    MAC("v78", "v74") \
    MAC("v79", "v75") \
    "ds_read_b128 v[72:75], %[w] offset:31744\n" \
    "ds_read_b128 v[76:79], %[x] offset:496\n" \
    "s_waitcnt lgkmcnt(10)\n" \
    MAC("v84", "v80") \
    MAC("v85", "v81") \
    MAC("v86", "v82") \
    MAC("v87", "v83") \
    "s_waitcnt lgkmcnt(8)\n" \
    MAC("v92", "v88") \
    MAC("v93", "v89") \
    MAC("v94", "v90") \
    MAC("v95", "v91") \
    "s_waitcnt lgkmcnt(6)\n" \
    MAC("v100", "v96") \
    MAC("v101", "v97") \
    MAC("v102", "v98") \
    MAC("v103", "v99") \
    "s_waitcnt lgkmcnt(4)\n" \
    MAC("v108", "v104") \
    MAC("v109", "v105") \
    MAC("v110", "v106") \
    MAC("v111", "v107") \
    "s_waitcnt lgkmcnt(2)\n" \
    MAC("v68", "v64") \
    MAC("v69", "v65") \
    MAC("v70", "v66") \
    MAC("v71", "v67") \
    "s_waitcnt lgkmcnt(0)\n" \
    MAC("v76", "v72") \
    MAC("v77", "v73") \
    MAC("v78", "v74") \
    MAC("v79", "v75")
// fused step: acc = fma(x, w, acc) (the reference's contracted bf16 chain)
#define UOCR_RMAC_FMA(X, W) "v_fmac_f32 %[acc], " X ", " W "\n"
// unfused step: acc = acc + round(x * w) (the reference's f32 matmul_t, whose
// build does not contract the loop; src/kernels/cpu_ops.cpp:11-24)
#define UOCR_RMAC_SEP(X, W) "v_mul_f32 v112, " X ", " W "\nv_add_f32 %[acc], %[acc], v112\n"

}  // namespace uocr_hip
