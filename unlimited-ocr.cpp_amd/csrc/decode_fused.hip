// Fused decode layer (1..16 tokens, bf16 input, no fused RMSNorm): router,
// gate/up, down and combine in ONE persistent launch (two workgroups per CU,
// the grid fully resident and the same on every call). The description below
// is the dense form (12..16 tokens); with fewer tokens the gate/up items cover
// only the candidate groups, after the candidate summary (up to 4 tokens the
// candidates come from per-expert estimate workgroups instead of the routers).
//
// The stand-alone decode path (decode_path.hip) runs four kernels in order. At
// 16 tokens the router is latency-bound (the reference's sequential fmaf chain
// per (token, expert), src/kernels/cpu_ops.cpp:26-39) and every kernel boundary
// drains the chip. Here every workgroup derives the same static schedule:
//
//   workgroups [0, T)   the router of token t: first the candidate experts (a
//                       bounded estimate of the logits, published at once),
//                       then the exact chain, scores and top_k
//   workgroups [T, P)   gate/up items (group g, 64 inter rows) for every group
//                       and all T tokens, round-robin: no wait for routing
//   every workgroup     then down items (live group, 128 hidden rows), live =
//                       a candidate of some token or shared, in slots ordered
//                       by when their workgroups are expected to be free; a
//                       down item waits for its group's gate/up items only
//   one slot per block  the weighted combine of 128 output columns with the
//                       exact routing (src/engine/moe_decoder.cpp:88-97,
//                       110-112), after the down items of the block
//
// Waiting is on per-workgroup progress words (FusedSync, layer-owned): a
// workgroup publishes S + steps done, S being its word at kernel start (every
// word ends a call at S + kFusedSteps). A workgroup only waits for steps that
// other resident workgroups reach without waiting for it, and every wait is
// bounded (kSpinLimit): a timeout sets a sticky flag in FusedSync::error and
// makes the call's outputs NaN (never a silently wrong result).
//
// Cross-workgroup data (candidate words, ids / weights, act rows, y rows) is
// written and read with agent-coherent (sc1) accesses around the progress
// stores; act and y rows are indexed by (group, token): g * T + t.
#include <hip/hip_runtime.h>
#include "fused_common.hpp"
#include "fused_schedule.hpp"

#include <algorithm>



namespace uocr_hip {

// LDS of the expert phase (the router phase uses the same bytes for its ring)
template <int GPT, int KTG, int KTD, bool ZP>
struct FusedLds {
    static constexpr int KTM = KTG > KTD ? KTG : KTD;
    static constexpr int GS = kTileK / GPT;
    static constexpr int NGG = scale_row_stride(KTG * kTileK, GS);
    static constexpr int NGD = scale_row_stride(KTD * kTileK, GS);
    static constexpr int SRM = kTileRows * (NGG > NGD ? NGG : NGD);
    static constexpr size_t as_bytes = (size_t)KTM * 4 * 64 * 8 * 2;
    // per wave: scale rows of the item's two matrices, then (ZP) their zero-offset rows
    static constexpr int SROWS = ZP ? 4 : 2;
    static constexpr size_t ss_bytes = ((size_t)4 * SROWS * SRM * 2 + 15) / 16 * 16;
    static constexpr int ZOFF = 2 * SRM * 2;  // bytes from a scale row to its zero-offset row
    static constexpr size_t cs_bytes = (size_t)KTM * GPT * 16 * 4;  // bias seeds [group][16 tokens] f32
    static constexpr int n_ints = 2 * kFusedMaxSeq + 2 * kMaxExperts + 4 * 16 + 4 + 2 * kFusedMaxSeq * kMaxTopK;
    static constexpr size_t bytes = as_bytes + ss_bytes + cs_bytes + (size_t)n_ints * 4;
};

// Logit estimates of expert e for the T tokens (one workgroup, up to
// kFusedEstMaxSeq tokens): thread i takes columns 8i .. 8i + 7 (an fma chain
// of 8 terms per token), the 256 partials then summed in a tree (8 levels);
// published as tagged words est[t][e][0..1] (estimate, sum of |x w|).
template <int KT>
__device__ __forceinline__ void estimate_expert(const DecodeArgs& a, int e, unsigned rtag, float* red) {
    constexpr int H = KT * 128;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int T = a.seq, E = a.n_experts;
    float s[kFusedEstMaxSeq], sa[kFusedEstMaxSeq];
#pragma unroll
    for (int t = 0; t < kFusedEstMaxSeq; ++t) s[t] = sa[t] = 0.0f;
    if (tid < H / 8) {
        const u32x4 wv = *reinterpret_cast<const u32x4*>(a.router_t + ((size_t)tid * E + e) * 8);
        float w[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[2 * i] = __uint_as_float(wv[i] << 16);
            w[2 * i + 1] = __uint_as_float(wv[i] & 0xffff0000u);
        }
        const uint16_t* xb = static_cast<const uint16_t*>(a.x);
        const float* xf = static_cast<const float*>(a.x);
#pragma unroll
        for (int t = 0; t < kFusedEstMaxSeq; ++t) {
            if (t < T) {
                float xv[8];  // the token's 8 columns (bf16 or f32 input)
                if (a.x_bf16) {
                    const u32x4 u = *reinterpret_cast<const u32x4*>(xb + (size_t)t * H + tid * 8);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        xv[2 * i] = __uint_as_float(u[i] << 16);
                        xv[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
                    }
                } else {
                    const f32x4 u0 = *reinterpret_cast<const f32x4*>(xf + (size_t)t * H + tid * 8);
                    const f32x4 u1 = *reinterpret_cast<const f32x4*>(xf + (size_t)t * H + tid * 8 + 4);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        xv[i] = u0[i];
                        xv[4 + i] = u1[i];
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float x0 = xv[2 * i], x1 = xv[2 * i + 1];
                    s[t] = fmaf(x0, w[2 * i], s[t]);
                    s[t] = fmaf(x1, w[2 * i + 1], s[t]);
                    sa[t] = fmaf(fabsf(x0), fabsf(w[2 * i]), sa[t]);
                    sa[t] = fmaf(fabsf(x1), fabsf(w[2 * i + 1]), sa[t]);
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < kFusedEstMaxSeq; ++t) {
        if (t >= T) break;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            s[t] += __shfl_xor(s[t], o, 64);
            sa[t] += __shfl_xor(sa[t], o, 64);
        }
        if (lane == 0) {
            red[(wave * kFusedEstMaxSeq + t) * 2] = s[t];
            red[(wave * kFusedEstMaxSeq + t) * 2 + 1] = sa[t];
        }
    }
    __syncthreads();
    if (tid < 2 * T) {
        const int t = tid >> 1, k = tid & 1;
        const float v = (red[(0 * kFusedEstMaxSeq + t) * 2 + k] + red[(1 * kFusedEstMaxSeq + t) * 2 + k]) +
                        (red[(2 * kFusedEstMaxSeq + t) * 2 + k] + red[(3 * kFusedEstMaxSeq + t) * 2 + k]);
        const uint64_t word = ((uint64_t)rtag << 32) | __float_as_uint(v);
        __hip_atomic_store(a.sync->est + ((size_t)t * 64 + e) * 2 + k, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
}

constexpr int kFusedWGPerCU = 2;  // workgroups per CU (the progress words need them all resident)
template <int GPT, int KTG, int KTD, bool ZP>
__global__ __launch_bounds__(256, kFusedWGPerCU) void decode_fused_kernel(DecodeArgs a) {
    using Lay = FusedLds<GPT, KTG, KTD, ZP>;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    f16* As = reinterpret_cast<f16*>(smem);
    f16* Ss = reinterpret_cast<f16*>(smem + Lay::as_bytes);  // [4 waves][SROWS][SRM]
    float* Cs = reinterpret_cast<float*>(smem + Lay::as_bytes + Lay::ss_bytes);
    // candidate masks per token, token masks per routed group, live groups
    uint32_t* cm32 = reinterpret_cast<uint32_t*>(smem + Lay::as_bytes + Lay::ss_bytes + Lay::cs_bytes);
    int* tokmask = reinterpret_cast<int*>(cm32 + 2 * kFusedMaxSeq);
    int* live = tokmask + kMaxExperts;
    int* ent = live + kMaxExperts;  // [4 waves][16]
    int* misc = ent + 4 * 16;       // routed live count
    int* ids_c = misc + 4;          // exact routing for the combine
    float* wts_c = reinterpret_cast<float*>(ids_c + kFusedMaxSeq * kMaxTopK);

    // wave index as a scalar: weight addresses become scalar bases + the lane offset
    int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, r = lane & 15;
    // per item: makes the thread indices opaque, so addresses derived from them
    // are recomputed in each item instead of hoisted (and spilled) across items
    auto fresh_indices = [&]() { asm volatile("" : "+v"(tid), "+v"(lane), "+v"(r), "+s"(wave)); };
    const int T = a.seq, E = a.n_experts, V = a.n_virtual, G = E + V, K = a.top_k, N = T * K;
    const int H = a.hidden, I = a.inter;
    // gate/up items: 64 rows (one 16-row tile per wave); down items: 128 rows
    // (two tiles per wave, one A staging)
    const int RBG = (I / kTileRows + 3) / 4, RBD = (H / kTileRows + 7) / 8;
    const int P = gridDim.x, b = blockIdx.x, PW = P - T;  // PW gate/up workers: T .. P-1
    FusedSync* sy = a.sync;
    int* prog = sy->progress;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const uint16_t* xb = static_cast<const uint16_t*>(a.x);

    // this call's base: every workgroup ended the previous call at the same value
    const int S = load_cg(prog + b);
    const unsigned rtag = (((unsigned)S >> 12) + 1u) & 0xFFFFFFu;  // routing words of this call
    int k = 0;  // steps published by this workgroup
    // publish: every wave waits for its own stores (a workgroup barrier does
    // not), the barrier, then one progress store
    auto publish = [&]() {
        store_fence();
        __syncthreads();
        ++k;
        if (tid == 0) {
            fence_wg_release();
            store_cg(prog + b, S + k);
        }
    };
    // An item's publish is deferred until the worker's next item has issued its
    // weights: flush(n) waits for everything but the n loads issued last (the
    // pending stores are older), so the store acknowledgements come back while
    // the next weights stream.
    bool pend = false;
    auto flush = [&](int n_after) {
        if (!pend) return;
        wait_vm_n(n_after);
        asm volatile("" ::: "memory");
        __syncthreads();
        ++k;
        if (tid == 0) {
            fence_wg_release();
            store_cg(prog + b, S + k);
        }
        pend = false;
    };
    // wave 0: until, for every lane with want, prog[owner] >= S + step; then the
    // whole workgroup proceeds
    auto wait_steps = [&](auto&& pair_of, int n) {
        if (wave == 0) {
            for (int base = 0; base < n; base += 64) {
                int owner = 0, step = 0;
                const bool want = base + lane < n;
                if (want) pair_of(base + lane, owner, step);
                int it = 0;
                while (__ballot(want && (int)(load_cg(prog + owner) - (S + step)) < 0)) {
                    if (++it > kSpinLimit) {
                        if (lane == 0) report_timeout(sy, rtag);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
        }
        __syncthreads();
        fence_wg_acquire();
    };

    bool have_summary = false;
    bool have_x = false;  // As holds all T token rows as f16
    int n_live_r = 0, n_live = 0;

    // Routing summary from the candidate masks (a superset of the routing,
    // published by the router workgroups before their exact chains): per
    // routed group the mask of its candidate tokens, the live routed groups
    // ascending, then the shared groups. Wave 0 holds the tagged words
    // (lane < 2T), prefetched under the last gate/up item and re-read until
    // every tag is this call's.
    uint64_t cw = 0;
    bool have_cw = false;
    auto cand_prefetch = [&]() {
        if (wave == 0) cw = lane < 2 * T ? __hip_atomic_load(sy->cand + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                         : ((uint64_t)rtag << 32);
        have_cw = true;
    };
    auto need_summary = [&]() {
        if (have_summary) return;
        if (T <= kFusedEstMaxSeq) {
            // few tokens: the candidates from the per-expert estimates, wave w
            // taking tokens w, w + 4, ... (each token's words requested
            // before any is checked)
            constexpr int TPW = (kFusedEstMaxSeq + 3) / 4;
            const bool want = lane < E;
            uint64_t w0[TPW], w1[TPW];
            int it = 0;
            while (true) {
                bool stale = false;
#pragma unroll
                for (int u = 0; u < TPW; ++u) {
                    const int t = wave + 4 * u;
                    if (t < T && want) {
                        w0[u] = __hip_atomic_load(sy->est + ((size_t)t * 64 + lane) * 2, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
                        w1[u] = __hip_atomic_load(sy->est + ((size_t)t * 64 + lane) * 2 + 1, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
                    } else {
                        w0[u] = w1[u] = 0;
                    }
                }
#pragma unroll
                for (int u = 0; u < TPW; ++u)
                    if (wave + 4 * u < T && want)
                        stale |= (uint32_t)(w0[u] >> 32) != rtag || (uint32_t)(w1[u] >> 32) != rtag;
                if (!__ballot(stale)) break;
                if (++it > kSpinLimit) {
                    if (lane == 0) report_timeout(sy, rtag);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
#pragma unroll
            for (int u = 0; u < TPW; ++u) {
                const int t = wave + 4 * u;
                if (t >= T) break;
                const uint64_t m = candidate_mask(a, __uint_as_float((uint32_t)w0[u]), __uint_as_float((uint32_t)w1[u]),
                                                  (float)(H + 16 + 64));
                if (lane == 0) {
                    cm32[2 * t] = (uint32_t)m;
                    cm32[2 * t + 1] = (uint32_t)(m >> 32);
                }
            }
            __syncthreads();
        }
        if (wave == 0) {
            if (T > kFusedEstMaxSeq) {
                if (!have_cw) cand_prefetch();
                int it = 0;
                while (__ballot((uint32_t)(cw >> 32) != rtag)) {
                    if (++it > kSpinLimit) {
                        if (lane == 0) report_timeout(sy, rtag);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                    if (lane < 2 * T) cw = __hip_atomic_load(sy->cand + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                if (lane < 2 * T) cm32[lane] = (uint32_t)cw;
            }
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            // lane e: the tokens whose candidates hold expert e
            int tm = 0;
            for (int t = 0; t < T; ++t) tm |= (int)((cm32[2 * t + (lane >> 5)] >> (lane & 31)) & 1u) << t;
            const bool hit = lane < E && tm != 0;
            tokmask[lane] = lane < E ? tm : 0;
            const uint64_t m = __ballot(hit);
            if (hit) live[__popcll(m & below)] = lane;
            const int run = __popcll(m);
            for (int v = lane; v < V; v += 64) live[run + v] = E + v;
            if (lane == 0) misc[0] = run;
        }
        __syncthreads();
        n_live_r = misc[0];
        n_live = n_live_r + V;
        have_summary = true;
    };

    // this wave's token list for group g (routed: its candidate tokens
    // ascending; shared or dense down: tokens 0..T-1) -> ent[wave][]; returns
    // the count
    auto token_list = [&](int g) {
        int* el = ent + wave * 16;
        if (g < E) {
            const int tm = tokmask[g];
            const bool hit = lane < T && ((tm >> lane) & 1);
            const uint64_t m = __ballot(hit);
            if (hit) el[__popcll(m & below)] = lane;
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            return (int)__popcll(m);
        }
        if (lane < T) el[lane] = lane;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        return T;
    };

    // ---- gate/up item: group g, 64 rows rb*64.. (all_tokens: A = all T rows)
    auto gate_up_item = [&](int g, int rb, bool prefetch_cand) {
        constexpr int KT = KTG;
        constexpr int NG = Lay::NGG;
        constexpr int SROW = kTileRows * NG;
        const int cnt = T;
        const int rbw = rb * 4 + wave;
        const bool wave_live = rbw * kTileRows < I;
        const int rbl = min(rbw, I / kTileRows - 1);
        const bool stage = !have_x;
        if (stage && r < cnt) {
            if (a.x_bf16) {
                const uint16_t* src = xb + (size_t)r * H + wave * 32 + 8 * (lane >> 4);
#pragma unroll
                for (int kt = 0; kt < KT; ++kt) load_lds16(src + kt * kTileK, As + (size_t)(kt * 4 + wave) * 64 * 8);
            } else {
                // f32 input: this wave's rows -> f16 into As before the weights are
                // requested (5 k-tiles of registers at a time)
                const float* src = static_cast<const float*>(a.x) + (size_t)r * H + wave * 32 + 8 * (lane >> 4);
#pragma unroll
                for (int k0 = 0; k0 < KT; k0 += 5) {
                    f32x4 v[5][2];
#pragma unroll
                    for (int i = 0; i < 5; ++i)
                        if (k0 + i < KT) {
                            v[i][0] = *reinterpret_cast<const f32x4*>(src + (k0 + i) * kTileK);
                            v[i][1] = *reinterpret_cast<const f32x4*>(src + (k0 + i) * kTileK + 4);
                        }
#pragma unroll
                    for (int i = 0; i < 5; ++i)
                        if (k0 + i < KT) {
                            const f16x8 h = {(f16)v[i][0][0], (f16)v[i][0][1], (f16)v[i][0][2], (f16)v[i][0][3],
                                             (f16)v[i][1][0], (f16)v[i][1][1], (f16)v[i][1][2], (f16)v[i][1][3]};
                            asm volatile("ds_write_b128 %0, %1" ::"v"(lds_addr(As + (size_t)((k0 + i) * 4 + wave) * 64 * 8 +
                                                                              (size_t)lane * 8)),
                                         "v"(h)
                                         : "memory");
                        }
                }
            }
        }
        f16* ssw = Ss + (size_t)wave * Lay::SROWS * Lay::SRM;
        const size_t sb = (size_t)g * a.gu_sstride + (size_t)rbl * SROW;
        for (int q = lane; q * 8 < SROW; q += 64) {
            load_lds16(a.gate_s + sb + q * 8, ssw + (q & ~63) * 8);
            load_lds16(a.up_s + sb + q * 8, ssw + Lay::SRM + (q & ~63) * 8);
            if constexpr (ZP) {
                load_lds16(a.gate_z + sb + q * 8, ssw + 2 * Lay::SRM + (q & ~63) * 8);
                load_lds16(a.up_z + sb + q * 8, ssw + 3 * Lay::SRM + (q & ~63) * 8);
            }
        }
        u32x4 bw0[KT], bw1[KT];
        const size_t toff = (size_t)g * a.gu_wstride + (size_t)rbl * KT * kTileBytes + (size_t)lane * 16;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
            bw0[kt] = *reinterpret_cast<const u32x4*>(a.gate + toff + (size_t)kt * kTileBytes);
            bw1[kt] = *reinterpret_cast<const u32x4*>(a.up + toff + (size_t)kt * kTileBytes);
        }
        flush(2 * KT);  // the previous item: its stores are older than the A rows and scales
        if (prefetch_cand) cand_prefetch();  // behind the weights: consumed after the item
        wait_vm_n(2 * KT + (prefetch_cand && wave == 0 ? 1 : 0));  // A rows and scales
        if (stage && a.x_bf16) convert_own_rows<KT>(As, wave, lane);
        lds_barrier();
        if (stage && !ZP) {
            bias_seeds<KT, GPT>(As, Cs, tid);
            lds_barrier();
        }
        if (wave_live) {
            f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
            item_mma<GPT, KT, true, ZP, Lay::ZOFF>(bw0, bw1, lds_addr(As + (size_t)lane * 8), lds_addr(ssw + r * NG),
                                                   lds_addr(ssw + Lay::SRM + r * NG),
                                                   lds_addr(Cs) + (uint32_t)(lane >> 4) * 16, acc0, acc1);
            const int col = rbw * kTileRows + r;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int m = 4 * (lane >> 4) + q;
                if (m < cnt) store_cg_f16(a.act + (size_t)(g * T + m) * I + col, (f16)silu_mul_f(acc0[q], acc1[q]));
            }
        }
        have_x = true;
    };

    // ---- down item: group g, 128 hidden rows rb*128.. (tiles rb*8 + wave and
    // rb*8 + 4 + wave of this wave)
    // Order of one item: wave 0 polls the gate/up workers of the group (issued
    // first, so its answer does not queue behind the weights), every wave
    // issues its weights, then -- once the group's act rows are complete --
    // the act rows and the scales go to LDS while the weights stream in.
    // ready(lane, owner, step) names the progress word lane < n_ready waits for.
    auto down_item = [&](int g, int rb, auto&& ready, int n_ready) {
        constexpr int KT = KTD;
        constexpr int NG = Lay::NGD;
        constexpr int SROW = kTileRows * NG;
        have_x = false;
        const int cnt = token_list(g);
        const int rbw0 = rb * 8 + wave, rbw1 = rbw0 + 4;
        const int rbl0 = min(rbw0, H / kTileRows - 1), rbl1 = min(rbw1, H / kTileRows - 1);
        int powner = 0, pstep = 0, pv = 0;
        const bool want = wave == 0 && lane < n_ready;
        if (want) {
            ready(lane, powner, pstep);
            pv = load_cg(prog + powner);
        }
        u32x4 bw0[KT], bw1[KT];
        const size_t toff0 = (size_t)g * a.dn_wstride + (size_t)rbl0 * KT * kTileBytes + (size_t)lane * 16;
        const size_t toff1 = (size_t)g * a.dn_wstride + (size_t)rbl1 * KT * kTileBytes + (size_t)lane * 16;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
            bw0[kt] = *reinterpret_cast<const u32x4*>(a.down + toff0 + (size_t)kt * kTileBytes);
            bw1[kt] = *reinterpret_cast<const u32x4*>(a.down + toff1 + (size_t)kt * kTileBytes);
        }
        flush(2 * KT);  // the previous item (its stores are older than these weights)
        if (wave == 0) {
            int it = 0;
            while (__ballot(want && (int)(pv - (S + pstep)) < 0)) {
                if (++it > kSpinLimit) {
                    if (lane == 0) report_timeout(sy, rtag);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
                if (want) pv = load_cg(prog + powner);
            }
        }
        lds_barrier();  // the other waves' weights stay in flight
        fence_wg_acquire();
        if (r < cnt) {
            const int tok = ent[wave * 16 + r];
            const f16* src = a.act + (size_t)(g * T + tok) * I + wave * 32 + 8 * (lane >> 4);
#pragma unroll
            for (int kt = 0; kt < KT; ++kt) load_lds16_cg(src + kt * kTileK, As + (size_t)(kt * 4 + wave) * 64 * 8);
        }
        f16* ssw = Ss + (size_t)wave * Lay::SROWS * Lay::SRM;
        const size_t sb0 = (size_t)g * a.dn_sstride + (size_t)rbl0 * SROW;
        const size_t sb1 = (size_t)g * a.dn_sstride + (size_t)rbl1 * SROW;
        for (int q = lane; q * 8 < SROW; q += 64) {
            load_lds16(a.down_s + sb0 + q * 8, ssw + (q & ~63) * 8);
            load_lds16(a.down_s + sb1 + q * 8, ssw + Lay::SRM + (q & ~63) * 8);
            if constexpr (ZP) {
                load_lds16(a.down_z + sb0 + q * 8, ssw + 2 * Lay::SRM + (q & ~63) * 8);
                load_lds16(a.down_z + sb1 + q * 8, ssw + 3 * Lay::SRM + (q & ~63) * 8);
            }
        }
        wait_vm<0>();
        lds_barrier();
        if constexpr (!ZP) {
            bias_seeds<KT, GPT>(As, Cs, tid);
            lds_barrier();
        }
        if (rbw0 * kTileRows < H) {
            // the two tiles share the A operand: the gate/up MMA shape
            f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
            item_mma<GPT, KT, true, ZP, Lay::ZOFF>(bw0, bw1, lds_addr(As + (size_t)lane * 8), lds_addr(ssw + r * NG),
                                                   lds_addr(ssw + Lay::SRM + r * NG),
                                                   lds_addr(Cs) + (uint32_t)(lane >> 4) * 16, acc0, acc1);
            const bool live1 = rbw1 * kTileRows < H;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int m = 4 * (lane >> 4) + q;
                if (m < cnt) {
                    const int yrow = g * T + ent[wave * 16 + m];  // (group, token)
                    store_cg(a.y + (size_t)yrow * H + rbw0 * kTileRows + r, acc0[q]);
                    if (live1) store_cg(a.y + (size_t)yrow * H + rbw1 * kTileRows + r, acc1[q]);
                }
            }
        }
    };

    // ---- combine of output columns rb*128 .. rb*128+127 for every token
    // (src/engine/moe_decoder.cpp:88-97, 110-112), y rows read agent-coherent.
    auto combine_block = [&](int rb) {
        // this thread: token t, columns c0 and c0 + 64 (both chunks' y rows are
        // requested before the one wait)
        const int t = tid >> 4;
        if (t >= T) return;
        // a timed-out wait anywhere in this call (reported before the progress
        // this combine waited for) makes every output of the call NaN
        bool bad = load_cg(&sy->call_fault) == rtag;
        constexpr int NY = kMaxTopK + 2;  // routed rows, then the first two shared rows
        const size_t sh0 = (size_t)E * T;  // first shared row
        const int c0 = rb * 128 + (tid & 15) * 4;
        float wt[kMaxTopK];
        f32x4 yv[2 * NY];
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j) {
            if (j < K) {
                wt[j] = wts_c[t * K + j];
                const int id = ids_c[t * K + j];
                // the exact pick is one of the token's candidates (else its y
                // row was not computed: flagged, never silent)
                if (!((cm32[2 * t + (id >> 5)] >> (id & 31)) & 1u)) {
                    __hip_atomic_fetch_or(&sy->error, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    bad = true;
                }
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    if (c0 + 64 * h < H) yv[h * NY + j] = load16_cg(a.y, (((size_t)id * T + t) * H + c0 + 64 * h) * 4);
            }
        }
#pragma unroll
        for (int v = 0; v < 2; ++v)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                if (v < V && c0 + 64 * h < H)
                    yv[h * NY + kMaxTopK + v] = load16_cg(a.y, ((sh0 + (size_t)v * T + t) * H + c0 + 64 * h) * 4);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int c = c0 + 64 * h;
            if (c >= H) continue;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < kMaxTopK; ++j)
                if (j < K)
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[q] = fmaf(wt[j], yv[h * NY + j][q], acc[q]);
            if (V > 0) {
                f32x4 sh = yv[h * NY + kMaxTopK];
                for (int v = 1; v < V; ++v) {
                    const f32x4 y2 = v < 2 ? yv[h * NY + kMaxTopK + 1] : load16_cg(a.y, ((sh0 + (size_t)v * T + t) * H + c) * 4);
#pragma unroll
                    for (int q = 0; q < 4; ++q) sh[q] += y2[q];
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) acc[q] += sh[q];
            }
            if (a.shared_y) {  // written by an earlier launch: a plain load
                const f32x4 sv = *reinterpret_cast<const f32x4*>(a.shared_y + (size_t)t * H + c);
#pragma unroll
                for (int q = 0; q < 4; ++q) acc[q] += sv[q];
            }
            if (bad) acc = f32x4{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")};
            *reinterpret_cast<f32x4*>(a.out + (size_t)t * H + c) = acc;
        }
    };

    // ---- 1. router (workgroups 0 .. T-1)
    if (b < T) {
        float* hand = reinterpret_cast<float*>(smem);
        float* sc = hand + 64;
        float* topv = sc + 64;
        uint64_t* etab = reinterpret_cast<uint64_t*>(topv + kMaxTopK);
        router_token_regs<KTG>(a, b, hand, sc, topv, etab, hand + 256, hand + 256 + kMaxHidden, rtag);
        publish();
    }

    // ---- 2. gate/up (workers T .. P-1). Dense (kFusedDenseMinSeq tokens and
    // more): every group for all tokens, no wait for the routing. Sparse (fewer
    // tokens): the live groups only, after the candidate summary -- a few
    // tokens touch few groups, so reading every group would cost more than
    // waiting for the candidates.
    const bool sparse = T < kFusedDenseMinSeq;
    // up to kFusedEstMaxSeq tokens: workgroups T .. T + E - 1 first estimate
    // one expert's logits each (a router's own estimate waits for the whole
    // router matrix; beyond a few tokens every workgroup's candidate
    // computation over the tokens costs more than that wait)
    if (T <= kFusedEstMaxSeq && b >= T && b < T + E) estimate_expert<KTG>(a, b - T, rtag, Cs);
    if (sparse) need_summary();
    const int n_gu_groups = sparse ? n_live : G;
    const int ngu_total = n_gu_groups * RBG;
    if (b >= T) {
        for (int i = b - T;; i += PW) {
            fresh_indices();
            if (i >= ngu_total) break;
            gate_up_item(sparse ? live[i / RBG] : i / RBG, i % RBG, !sparse && i + PW >= ngu_total);
            pend = true;
        }
    }

    // ---- 3. down (every workgroup) and the combine of each column block.
    // Dense: every group for all T tokens, item j = (group j / RBD, block
    // j % RBD); it waits only for its group's gate/up items, so the weight
    // stream runs on from gate/up into down while the router finishes. Sparse:
    // the live groups only (the routing summary first).
    need_summary();
    const int n_dn_groups = n_live;
    const FusedSchedule sch(T, P, n_gu_groups, RBG, RBD, n_live);  // identical in every workgroup
    const int ndn_total = sch.ndn_total;
    // position of gate/up item r of the group at down position gpos
    auto gu_index = [&](int gpos, int r_) { return (sparse ? gpos : live[gpos]) * RBG + r_; };
    const int my_slot = sch.slot_of(b);
    for (int j = my_slot; j < ndn_total; j += P) {
        fresh_indices();
        const int gpos = j / RBD, rb = j % RBD;
        down_item(
            live[gpos], rb,
            [&](int q, int& owner, int& step) { sch.gu_step(gu_index(gpos, q), owner, step); },
            RBG);
        pend = true;
    }
    flush(0);
    // combine of column block rb by slot (ndn_total + rb) % P, one with the
    // fewest down items, after all of its own (a combine waits only for down
    // items and the router, which never wait for a combine)
    bool have_route = false;
    for (int rb = 0; rb < RBD; ++rb) {
        if (sch.combine_slot(rb) != my_slot) continue;
        if (!have_route) {
            // the exact routing first (done long before the last down items),
            // so that the y rows are one round trip after the down items
            wait_steps([&](int q, int& owner, int& step) { owner = q; step = 1; }, T);
            for (int i = tid; i < T * K; i += 256) {
                ids_c[i] = load_cg(a.ids + i);
                wts_c[i] = load_cg(a.wts + i);
            }
            have_route = true;
        }
        wait_steps([&](int q, int& owner, int& step) { sch.dn_step(q * RBD + rb, owner, step); }, n_dn_groups);
        combine_block(rb);
    }

    // ---- leave: every workgroup ends the call at S + kFusedSteps
    __syncthreads();
    if (tid == 0) store_cg(prog + b, S + kFusedSteps);
}

template <int GPT, int KTG, int KTD, bool ZP>
static hipError_t launch_fused(const DecodeArgs& a, hipStream_t st) {
    using Lay = FusedLds<GPT, KTG, KTD, ZP>;
    const size_t lds = std::max(Lay::bytes, (size_t)a.hidden * 4 + 1024);
    static hipError_t attr = hipFuncSetAttribute((const void*)decode_fused_kernel<GPT, KTG, KTD, ZP>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, 80 * 1024);
    if (attr != hipSuccess) return attr;
    if (lds > 80 * 1024) return hipErrorInvalidValue;
    static int resident = [] {
        int dev = 0, cus = 0, per_cu = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_fused_kernel<GPT, KTG, KTD, ZP>, 256,
                                                           std::max(Lay::bytes, (size_t)kMaxHidden * 4 + 1024));
        return std::max(1, cus * std::max(1, per_cu));
    }();
    // the grid is the same on every call (the progress words advance together)
    // and fully resident (workgroups wait for one another)
    const int grid = std::min(resident, kFusedMaxGrid);
    if (grid <= a.seq) return hipErrorInvalidConfiguration;
    // up to kFusedEstMaxSeq tokens every expert needs its estimating workgroup
    if (a.seq <= kFusedEstMaxSeq && grid < a.seq + a.n_experts) return hipErrorInvalidConfiguration;
    // Plain launch: a cooperative launch (which refuses a grid that cannot be
    // resident at once) measured 53.6 us per call against 36.6 us on MI355X. The
    // grid is sized from the occupancy query; if other work keeps workgroups
    // from being resident, the bounded waits time out and the call's output
    // becomes NaN (status bit 0), never a silently wrong result.
    launch_k((decode_fused_kernel<GPT, KTG, KTD, ZP>), dim3(grid), dim3(256), (uint32_t)lds, st, a);
    return hipGetLastError();
}

bool decode_fused_ok(int hidden, int inter, int group) {
    return hidden == 1280 && inter == 896 && (group == 32 || group == 64 || group == 128);
}

hipError_t launch_decode_fused(const DecodeArgs& a, hipStream_t st) {
    if (a.seq < 1 || a.seq > kFusedMaxSeq || a.rms_weight || !a.sync) return hipErrorInvalidValue;
    if (a.n_experts + a.n_virtual > kMaxExperts || a.n_experts > 64 || a.top_k > kMaxTopK) return hipErrorInvalidValue;
    if (!decode_fused_ok(a.hidden, a.inter, a.group)) return hipErrorInvalidValue;
    const bool zp = a.gate_z != nullptr;
    switch (a.group) {
        case 32: return zp ? launch_fused<4, 10, 7, true>(a, st) : launch_fused<4, 10, 7, false>(a, st);
        case 64: return zp ? launch_fused<2, 10, 7, true>(a, st) : launch_fused<2, 10, 7, false>(a, st);
        default: return zp ? launch_fused<1, 10, 7, true>(a, st) : launch_fused<1, 10, 7, false>(a, st);
    }
}

}  // namespace uocr_hip
