// Device helpers shared by the single-launch decode kernels (decode_fused.hip,
// decode_stream.hip): bounded waits, agent-coherent accesses for data that
// other workgroups of the same launch read, bf16 -> f16 staging of token rows
// and the candidate-expert bound.
#pragma once
#include "decode_common.hpp"

namespace uocr_hip {

constexpr int kSpinLimit = 1 << 20;    // bounded waits (~1 s)
constexpr int kFusedSteps = 1 << 12;   // progress advance per call (> steps of any workgroup)

// A bounded wait ran out: the sticky status bit, and this call's tag in
// call_fault so that the call's combine writes NaN instead of a result built
// from incomplete rows. Both stores are released (agent scope) before the
// caller publishes any further progress, so a workgroup that waited for that
// progress sees the fault.
__device__ __forceinline__ void report_timeout(FusedSync* sy, unsigned rtag) {
    __hip_atomic_fetch_or(&sy->error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&sy->call_fault, rtag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
}

// The same with the sticky bit in `status` (a kernel whose progress words
// live in another FusedSync than the layer's status word)
__device__ __forceinline__ void report_timeout_to(int* status, FusedSync* sy, unsigned rtag) {
    __hip_atomic_fetch_or(status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&sy->call_fault, rtag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
}

// Cross-workgroup data moves through agent-coherent accesses (sc1: written
// through to, and read from, the coherence point shared by every XCD's L2), so
// publishing needs no L2-wide writeback and reading no L2 invalidation -- both
// serialise per XCD and cost far more than the few rows exchanged. Publish =
// the stores, an explicit vmcnt(0) in every wave (the workgroup barrier does
// not wait for outstanding stores), the barrier, then a counter increment;
// consume = spin on the counter, then the loads. The workgroup-scope fences
// only keep the compiler from moving accesses across those points.
__device__ __forceinline__ void fence_wg_release() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup"); }
__device__ __forceinline__ void fence_wg_acquire() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup"); }

// Wait until every memory operation this wave issued has completed (stores
// included: on gfx9 vmcnt counts them). The asm carries a memory clobber, so
// the compiler keeps every earlier store before it; the waitcnt builtin alone
// would let a store sink past the wait.
__device__ __forceinline__ void store_fence() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <typename U>
__device__ __forceinline__ U load_cg(const U* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename U>
__device__ __forceinline__ void store_cg(U* p, U v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ f32x4 load4_cg(const float* p) {
    return f32x4{load_cg(p), load_cg(p + 1), load_cg(p + 2), load_cg(p + 3)};
}
__device__ __forceinline__ void store_cg_f16(f16* p, f16 v) {
    asm volatile("global_store_short %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
// 16-byte agent-coherent read of y (rows other workgroups wrote with sc1
// stores): a buffer load with the sc1 policy, so the compiler tracks its
// completion like any other load. `byte_off` < 2^31 (the y rows of one call).
__device__ __forceinline__ f32x4 load16_cg(const float* base, size_t byte_off) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, 0x7fffffff, 0x00020000);
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)byte_off, 0, 16 /* sc1 */));
}
// 16-byte global -> LDS DMA, agent-coherent read
__device__ __forceinline__ void load_lds16_cg(const void* src, void* lds_base) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)lds_base, 16, 0, 16 /* sc1 */);
}

// 32-bit LDS read by asm (a plain LDS read issued while LDS DMAs are in
// flight makes the compiler wait for every outstanding global load)
__device__ __forceinline__ uint32_t lds_read_u32(const void* p) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(p)) : "memory");
    return v;
}

// bf16 token rows DMA'd into As by this lane -> f16 in place (the lane's own
// 16 bytes of every k-tile; its DMA has landed once the caller has waited)
template <int KT>
__device__ __forceinline__ void convert_own_rows(f16* As, int wave, int lane) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
        const uint32_t ad = lds_addr(As + (size_t)(kt * 4 + wave) * 64 * 8 + (size_t)lane * 8);
        u32x4 v;
        asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(ad) : "memory");
        f16x8 h;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            h[2 * i] = (f16)__uint_as_float(v[i] << 16);
            h[2 * i + 1] = (f16)__uint_as_float(v[i] & 0xffff0000u);
        }
        asm volatile("ds_write_b128 %0, %1" ::"v"(ad), "v"(h) : "memory");
    }
}

// Every expert that can be among the token's top_k after the exact chain,
// from an estimate S of its logit and SA = sum |x w| (lane e: expert e, the
// whole wave calls). The chain's rounding error is at most 2^-24 * H * SA
// (recursive fma summation) and the estimate's at most 2^-24 * n_est * SA
// with n_est the estimate's terms per partial sum plus its merge depth;
// NTERMS = H + n_est + 64 bounds both with slack. Softmax: a candidate when
// its upper bound reaches the top_k-th largest lower bound, less the logit
// distance over which two probabilities can still round equal (equal scores go
// to the lower index). Sigmoid: the same in score space. Non-finite input: all.
__device__ __forceinline__ uint64_t candidate_mask(const DecodeArgs& a, float S, float SA, float nterms) {
    const int lane = threadIdx.x & 63;
    const int E = a.n_experts;
    const bool valid = lane < E;
    bool cand;
    if (__ballot(valid && !(__builtin_isfinite(S) && __builtin_isfinite(SA)))) {
        cand = valid;
    } else {
        const float B = nterms * 0x1p-24f * 1.02f * SA + 0x1p-22f * fabsf(S) + 1e-30f;
        float lo = S - B, hi = S + B;
        if (a.scoring_sigmoid) {
            lo = (1.0f - 1e-5f) / (1.0f + __expf(-lo));
            hi = (1.0f + 1e-5f) / (1.0f + __expf(-hi));
        }
        float rem = valid ? lo : -INFINITY, kth = -INFINITY;
        for (int j = 0; j < a.top_k && j < E; ++j) {
            kth = wave_max64(rem);
            const uint64_t tie = __ballot(rem == kth);
            if (lane == (int)__builtin_ctzll(tie)) rem = -INFINITY;
        }
        float slack = 0.0f;
        if (!a.scoring_sigmoid) {
            const float mx = wave_max64(valid ? fabsf(hi) : 0.0f);
            slack = 0x1p-21f * (2.0f + fabsf(kth) + mx);
        }
        cand = valid && hi + slack >= kth;
    }
    return __ballot(cand);
}


// Router of token t with the router matrix held in registers: wave w loads
// columns [w*SEG, (w+1)*SEG) (SEG = H / NW) of lane e's row (bf16, [H/8][E][8]) in one burst
// at kernel start, then the waves run the reference's sequential fmaf chain
// (columns ascending, src/kernels/cpu_ops.cpp:26-39) one segment after the
// other, handing the running sums on through LDS; the last wave scores and
// selects. The token row sits in LDS as f32 and reaches the chain as broadcast
// 16-byte reads one 8-column block ahead, so a column costs the weight's
// widening and the fmac. The router waves run at raised issue priority (the
// other workgroup on the CU dequantises expert weights meanwhile).
// PREP: the token row is f32 or bf16 (a.x_bf16), RMS-normalised when
// a.rms_weight is set (src/kernels/cpu_ops.cpp:58-67). The expert input
// (a.x16, f16, agent-coherent stores) and the candidates come first, from a
// scale whose sum of squares is added in parallel (it differs from the
// reference's column-order sum by at most about H unit roundoffs, which the
// candidate bound takes in, and the f16 input far less than its own
// rounding); then the reference's sequential sum, the exact row and the
// exact chain. part then needs kMaxHidden + 2 * H + 64 floats beyond its
// NW * 128 (rounded squares, the estimate's row).
// F32R: an f32 router (a.router_f32, [H/4][64][4]), held as f32 in registers;
// its chain is the reference's uncontracted f32 matmul_t, acc + round(x * w)
// (src/kernels/cpu_ops.cpp:11-24).
template <int KT, int NW = 4, bool PREP = false, bool F32R = false>
__device__ __forceinline__ void router_token_regs(const DecodeArgs& a, int t, float* hand, float* sc, float* topv,
                                                  uint64_t* etab, float* xs, float* part, unsigned rtag) {
    constexpr int SEG = KT * 128 / NW;  // columns per wave (H = KT * 128)
    constexpr int NL = SEG / 8;   // 16-byte weight loads per lane
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int E = a.n_experts, H = KT * 128;
    const int e = lane < E ? lane : 0;
    // token row first (the weight burst behind it is waited for only by the chain)
    static_assert(SEG % 8 == 0, "whole 16-byte weight loads per segment");
    constexpr int NXT = (KT * 128 + 64 * NW - 1) / (64 * NW);  // token-row passes of the workgroup
    __builtin_amdgcn_s_setprio(3);
    const uint16_t* x = static_cast<const uint16_t*>(a.x) + (size_t)t * H;
    const float* xf = static_cast<const float*>(a.x) + (size_t)t * H;
    const bool xbf = a.x_bf16;
    uint32_t xb[NXT];  // bf16 bits, or (f32 x) the float's bits
    float rw[NXT];     // PREP + RMSNorm: the weights of the thread's columns
#pragma unroll
    for (int i = 0; i < NXT; ++i) {
        const int c = tid + 64 * NW * i;
        if (a.x_bf16) {
            xb[i] = c < H ? (uint32_t)x[c] : 0u;
        } else {
            xb[i] = c < H ? __float_as_uint(xf[c]) : 0u;
        }
        rw[i] = PREP && a.rms_weight && c < H ? a.rms_weight[c] : 0.0f;
    }
    // bf16: 8 columns per 16-byte load; f32: 4 (two loads per 8 columns)
    constexpr int NLW = F32R ? 2 * NL : NL;
    u32x4 wr[NLW];
    if constexpr (F32R) {
        const float* wbase = a.router_f32 + ((size_t)wave * NLW * 64 + lane) * 4;
#pragma unroll
        for (int i = 0; i < NLW; ++i) wr[i] = *reinterpret_cast<const u32x4*>(wbase + (size_t)i * 64 * 4);
    } else {
        const uint16_t* wbase = a.router_t + ((size_t)wave * NL * E + e) * 8;
#pragma unroll
        for (int i = 0; i < NL; ++i) wr[i] = *reinterpret_cast<const u32x4*>(wbase + (size_t)i * E * 8);
    }
    asm volatile("" ::: "memory");  // the whole burst is issued before the row is waited for
#pragma unroll
    for (int i = 0; i < NXT; ++i) {
        asm volatile("" : "+v"(xb[i]));
        if (tid + 64 * NW * i < H) xs[tid + 64 * NW * i] = __uint_as_float(xbf ? xb[i] << 16 : xb[i]);
    }
    lds_barrier();
    float* pq = part + NW * 128;      // PREP + RMSNorm: rounded squares [H + 64]
    float* xe = pq + kMaxHidden + 64;  // the estimate's row
    const bool rms = PREP && a.rms_weight;
    if constexpr (PREP) {
        const float* xin = xs;
        if (rms) {
            float ps = 0.0f;
#pragma unroll
            for (int i = 0; i < NXT; ++i) {
                const int c = tid + 64 * NW * i;
                if (c < H) {
                    const float q = __fmul_rn(xs[c], xs[c]);
                    pq[c] = q;
                    ps += q;
                }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) ps += __shfl_xor(ps, o, 64);
            if (lane == 0) hand[wave] = ps;
            __syncthreads();
            float ssa = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; ++w) ssa += hand[w];
            const float inv_a = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ssa, (float)H), a.rms_eps)));
#pragma unroll
            for (int i = 0; i < NXT; ++i) {
                const int c = tid + 64 * NW * i;
                if (c < H) xe[c] = __fmul_rn(__fmul_rn(xs[c], inv_a), rw[i]);
            }
            __syncthreads();
            xin = xe;
        }
        // the f16 expert input, written through to the coherence point
        for (int c = tid * 8; c < H; c += 64 * NW * 8) {
            const f32x4 p = *reinterpret_cast<const f32x4*>(xin + c);
            const f32x4 q = *reinterpret_cast<const f32x4*>(xin + c + 4);
            const f16x8 h = {(f16)p[0], (f16)p[1], (f16)p[2], (f16)p[3], (f16)q[0], (f16)q[1], (f16)q[2], (f16)q[3]};
            // (the nops: wait states the hazard recognizer does not add around asm)
            asm volatile("s_nop 4\n\tglobal_store_dwordx4 %0, %1, off sc1\n\ts_nop 4" ::"v"(a.x16 + (size_t)t * H + c),
                         "v"(h)
                         : "memory");
        }
        store_fence();  // complete before the candidates are published
    }
    const uint32_t xa = lds_addr(xs + wave * SEG);
    const uint32_t xea = rms ? lds_addr(xe + wave * SEG) : xa;  // the estimate's row

    // Candidate experts of the token, ahead of the exact chain: this wave's
    // segment as a blocked sum (8 chains) and the sum of |x w| (part[wave]).
    auto early_partial = [&]() {
        float s8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, sa = 0.0f;
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            f32x4 c0, c1, w0, w1;
            asm volatile("ds_read_b128 %0, %2 offset:%3\n\tds_read_b128 %1, %2 offset:%4\n\ts_waitcnt lgkmcnt(0)"
                         : "=&v"(c0), "=&v"(c1) : "v"(xea), "i"(i * 32), "i"(i * 32 + 16) : "memory");
            if constexpr (F32R) {
                w0 = __builtin_bit_cast(f32x4, wr[2 * i]);
                w1 = __builtin_bit_cast(f32x4, wr[2 * i + 1]);
            } else {
                asm volatile(
                    "v_lshlrev_b32 %0, 16, %8\n\tv_and_b32 %1, 0xffff0000, %8\n\t"
                    "v_lshlrev_b32 %2, 16, %9\n\tv_and_b32 %3, 0xffff0000, %9\n\t"
                    "v_lshlrev_b32 %4, 16, %10\n\tv_and_b32 %5, 0xffff0000, %10\n\t"
                    "v_lshlrev_b32 %6, 16, %11\n\tv_and_b32 %7, 0xffff0000, %11"
                    : "=&v"(w0[0]), "=&v"(w0[1]), "=&v"(w0[2]), "=&v"(w0[3]), "=&v"(w1[0]), "=&v"(w1[1]),
                      "=&v"(w1[2]), "=&v"(w1[3])
                    : "v"(wr[i][0]), "v"(wr[i][1]), "v"(wr[i][2]), "v"(wr[i][3]));
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                s8[c] = fmaf(c0[c], w0[c], s8[c]);
                s8[4 + c] = fmaf(c1[c], w1[c], s8[4 + c]);
                sa = fmaf(fabsf(c0[c]), fabsf(w0[c]), sa);
                sa = fmaf(fabsf(c1[c]), fabsf(w1[c]), sa);
            }
        }
        part[wave * 128 + lane] = ((s8[0] + s8[1]) + (s8[2] + s8[3])) + ((s8[4] + s8[5]) + (s8[6] + s8[7]));
        part[wave * 128 + 64 + lane] = sa;
    };
    // the candidates: an expert whose logit interval can reach the top_k
    // (candidate_mask), published as two tagged 32-bit halves of the mask
    auto early_finish = [&]() {
        float S = part[lane], SA = part[64 + lane];
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            S += part[w * 128 + lane];
            SA += part[w * 128 + 64 + lane];
        }
        // (+ H + 16 terms: the approximate RMSNorm scale of the estimate's row;
        // F32R: + 16, the chain's rounded products add at most 2^-24 * SA)
        const uint64_t m =
            candidate_mask(a, S, SA, (float)(H + SEG / 8 + 64 + (rms ? H + 16 : 0) + (F32R ? 16 : 0)));
        if (lane < 2) {
            const uint64_t w = ((uint64_t)rtag << 32) | (uint32_t)(lane == 0 ? m : (m >> 32));
            __hip_atomic_store(a.sync->cand + 2 * t + lane, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    };

    // every wave estimates its segment first (in parallel); wave NW - 1 selects
    // the candidates beside wave 0's chain segment (PREP: before the exact
    // RMSNorm sum, which lane 0 adds meanwhile)
    early_partial();
    lds_barrier();
    if constexpr (PREP) {
        if (wave == NW - 1) early_finish();
        if (rms) {
            if (tid == 0) {
                const float ss = rms_sum_chain(pq, H);
                sc[0] = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)H), a.rms_eps)));
            }
            __syncthreads();
            const float inv = sc[0];
#pragma unroll
            for (int i = 0; i < NXT; ++i) {
                const int c = tid + 64 * NW * i;
                if (c < H) xs[c] = __fmul_rn(__fmul_rn(xs[c], inv), rw[i]);
            }
            __syncthreads();
        }
    }
    float acc = 0.0f;
    for (int w = 0; w < NW; ++w) {
        if (wave != w) {
            if constexpr (!PREP)
                if (w == 0 && wave == NW - 1) early_finish();
        } else {
            if (w > 0) acc = hand[lane];
            f32x4 c0, c1, n0, n1;
            asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:16\n\ts_waitcnt lgkmcnt(0)"
                         : "=&v"(c0), "=&v"(c1) : "v"(xa) : "memory");
#pragma unroll
            for (int i = 0; i < NL; ++i) {
                if (i + 1 < NL)
                    asm volatile("ds_read_b128 %0, %2 offset:%3\n\tds_read_b128 %1, %2 offset:%4"
                                 : "=&v"(n0), "=&v"(n1) : "v"(xa), "i"((i + 1) * 32), "i"((i + 1) * 32 + 16));
                f32x4 w0, w1;
                if constexpr (F32R) {
                    w0 = __builtin_bit_cast(f32x4, wr[2 * i]);
                    w1 = __builtin_bit_cast(f32x4, wr[2 * i + 1]);
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc = __fadd_rn(acc, __fmul_rn(c0[c], w0[c]));
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc = __fadd_rn(acc, __fmul_rn(c1[c], w1[c]));
                } else {
                    // widen at the point of use (volatile: not hoisted into a spill)
                    asm volatile(
                        "v_lshlrev_b32 %0, 16, %8\n\tv_and_b32 %1, 0xffff0000, %8\n\t"
                        "v_lshlrev_b32 %2, 16, %9\n\tv_and_b32 %3, 0xffff0000, %9\n\t"
                        "v_lshlrev_b32 %4, 16, %10\n\tv_and_b32 %5, 0xffff0000, %10\n\t"
                        "v_lshlrev_b32 %6, 16, %11\n\tv_and_b32 %7, 0xffff0000, %11"
                        : "=&v"(w0[0]), "=&v"(w0[1]), "=&v"(w0[2]), "=&v"(w0[3]), "=&v"(w1[0]), "=&v"(w1[1]),
                          "=&v"(w1[2]), "=&v"(w1[3])
                        : "v"(wr[i][0]), "v"(wr[i][1]), "v"(wr[i][2]), "v"(wr[i][3]));
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc = fmaf(c0[c], w0[c], acc);
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc = fmaf(c1[c], w1[c], acc);
                }
                if (i + 1 < NL) {
                    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(n0), "+v"(n1), "+v"(acc));
                    c0 = n0;
                    c1 = n1;
                }
            }
            if (w < NW - 1) hand[lane] = acc;
            // the expf table for the selection (wave 0's weight burst is drained)
            if (w == 0 && lane < 32) etab[lane] = uocr_exp2_tab[lane];
        }
        lds_barrier();
    }
    if (wave == NW - 1) router_select<true>(a, t, acc, sc, topv, etab);
    __builtin_amdgcn_s_setprio(0);
}

}  // namespace uocr_hip
