// Device router: optional RMSNorm prologue, router logits, softmax / sigmoid
// scoring, greedy top-k, and the stable token->expert grouping.
//
// Bit-exactness contract with the reference CPU path:
//   logits   src/kernels/cpu_ops.cpp:26-39 -- one sequential fmaf chain per
//            (token, expert), k ascending (the -march=native build contracts
//            `acc += x * w`); one lane per expert runs exactly that chain.
//   rmsnorm  src/kernels/cpu_ops.cpp:58-67 -- sequential fmaf chain for the sum
//            of squares, correctly rounded divide and sqrt, (x * inv) * w.
//   softmax  src/kernels/cpu_ops.cpp:93-106 -- exp(l - max) with glibc's expf
//            bits (correctly rounded exp + the generated fix-up table), sum in
//            expert order, p = e * (1 / sum).
//   top-k    src/engine/moe_decoder.cpp:264-287 -- strict '>' greedy selection,
//            ties to the lowest expert index, optional renormalisation.
//   grouping src/engine/gpu_decoder.cu:602-609 -- per expert, tokens in
//            ascending (token, j) order: a stable counting sort, built here from
//            wave ballots (equal-expert masks) and per-wave LDS prefix counts.
#include "launch.hpp"

namespace uocr_hip {

__device__ __forceinline__ float apply_expf_fix(float x, float y, const uint32_t* __restrict__ offs,
                                                const uint32_t* __restrict__ ent) {
    const uint32_t b = __float_as_uint(x);
    uint32_t lo = offs[b >> 16], hi = offs[(b >> 16) + 1];
    const uint32_t key = b & 0xffffu;
    while (lo < hi) {  // entries of one bucket are sorted by their low 16 bits
        const uint32_t mid = (lo + hi) >> 1;
        const uint32_t v = ent[mid];
        const uint32_t k = v & 0xffffu;
        if (k == key) {
            const uint32_t yb = __float_as_uint(y);
            return __uint_as_float((v >> 16) ? yb + 1u : yb - 1u);
        }
        if (k < key) lo = mid + 1;
        else hi = mid;
    }
    return y;
}

__device__ __forceinline__ float ref_expf(float x, const uint32_t* offs, const uint32_t* ent) {
    return apply_expf_fix(x, uocr_uexpf(x), offs, ent);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// Argmax over the wave with the reference's tie rule (first maximum wins).
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(v, o, kWave);
        const int oi = __shfl_xor(i, o, kWave);
        if (ov > v || (ov == v && oi < i)) {
            v = ov;
            i = oi;
        }
    }
}

template <typename XT>
__device__ __forceinline__ void load8_f32(const XT* p, float* out);

template <>
__device__ __forceinline__ void load8_f32<uint16_t>(const uint16_t* p, float* out) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[2 * i] = __uint_as_float(v[i] << 16);
        out[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
    }
}

template <>
__device__ __forceinline__ void load8_f32<float>(const float* p, float* out) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
    const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[i] = a[i];
        out[4 + i] = b[i];
    }
}

// One wave routes TPW tokens; lane e owns expert e (E <= 64).
// LDS: [waves][TPW][H] f32 activations + [waves][64] scratch.
template <typename XT, bool RMS, int TPW>
__global__ __launch_bounds__(256) void router_kernel(RouterArgs a) {
    extern __shared__ float lds[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int H = a.hidden, E = a.n_experts, K = a.top_k;
    float* xs = lds + (size_t)wave * TPW * H;
    float* scr = lds + (size_t)(blockDim.x >> 6) * TPW * H + wave * 64;
    const int t0 = (blockIdx.x * (blockDim.x >> 6) + wave) * TPW;
    const XT* x = static_cast<const XT*>(a.x);

    // 1. stage the activations as f32
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
        const int t = t0 + tt;
        for (int c = lane * 8; c < H; c += 64 * 8) {
            float v[8];
            if (t < a.seq) {
                load8_f32<XT>(x + (size_t)t * H + c, v);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = 0.0f;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) xs[tt * H + c + i] = v[i];
        }
    }
    __syncthreads();

    // 2. RMSNorm: one lane per token runs the reference's sequential chain
    if constexpr (RMS) {
        if (lane < TPW) {
            const float* xr = xs + lane * H;
            float ss = 0.0f;
            for (int c = 0; c < H; c += 4) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(xr + c);
                ss = fmaf(v[0], v[0], ss);
                ss = fmaf(v[1], v[1], ss);
                ss = fmaf(v[2], v[2], ss);
                ss = fmaf(v[3], v[3], ss);
            }
            scr[lane] = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)H) + a.rms_eps));
        }
        __syncthreads();
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt) {
            const float inv = scr[tt];
            for (int c = lane; c < H; c += 64) xs[tt * H + c] = xs[tt * H + c] * inv * a.rms_weight[c];
        }
        __syncthreads();
    }

    // 3. f16 copy of the expert input for the MFMA kernels
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
        const int t = t0 + tt;
        if (t < a.seq) {
            for (int c = lane * 8; c < H; c += 64 * 8) {
                f16x8 h;
#pragma unroll
                for (int i = 0; i < 8; ++i) h[i] = (f16)xs[tt * H + c + i];
                *reinterpret_cast<f16x8*>(a.x16 + (size_t)t * H + c) = h;
            }
        }
    }

    // 4. logits: lane e, sequential fmaf over k (router W stored [H/8][E][8])
    float acc[TPW];
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) acc[tt] = 0.0f;
    if (lane < E) {
        const uint16_t* wp = a.router_t + (size_t)lane * 8;
        for (int c8 = 0; c8 < H / 8; ++c8) {
            float w[8];
            load8_f32<uint16_t>(wp + (size_t)c8 * E * 8, w);
#pragma unroll
            for (int tt = 0; tt < TPW; ++tt) {
                const f32x4 xa = *reinterpret_cast<const f32x4*>(xs + tt * H + c8 * 8);
                const f32x4 xb = *reinterpret_cast<const f32x4*>(xs + tt * H + c8 * 8 + 4);
                float s = acc[tt];
                s = fmaf(xa[0], w[0], s);
                s = fmaf(xa[1], w[1], s);
                s = fmaf(xa[2], w[2], s);
                s = fmaf(xa[3], w[3], s);
                s = fmaf(xb[0], w[4], s);
                s = fmaf(xb[1], w[5], s);
                s = fmaf(xb[2], w[6], s);
                s = fmaf(xb[3], w[7], s);
                acc[tt] = s;
            }
        }
    }

    // 5. scoring + greedy top-k, one token at a time
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
        const int t = t0 + tt;
        const float l = acc[tt];
        float p;
        if (a.scoring_sigmoid) {
            p = __fdiv_rn(1.0f, 1.0f + ref_expf(-l, a.fix_offsets, a.fix_entries));
        } else {
            const float mx = wave_max(lane < E ? l : -INFINITY);
            const float ev = ref_expf(l - mx, a.fix_offsets, a.fix_entries);
            scr[lane] = ev;
            __syncthreads();
            float sum = 0.0f;
            for (int e = 0; e < E; ++e) sum += scr[e];  // every lane: same order, same bits
            p = ev * __fdiv_rn(1.0f, sum);
            __syncthreads();
        }
        float sel = lane < E ? p : -INFINITY;
        float wj = 0.0f;
        int idj = 0;
        for (int j = 0; j < K; ++j) {
            float v = sel;
            int i = lane;
            wave_argmax(v, i);
            if (!(v > -1e30f)) i = -1;  // reference: no candidate above -1e30
            if (lane == j) {
                idj = i;
                wj = v;
            }
            if (lane == i) sel = -1e30f;
        }
        // renormalisation / scaling (moe_decoder.cpp:280-287)
        if (K > 1 && a.norm_topk_prob) {
            float s = 0.0f;
            for (int j = 0; j < K; ++j) s += __shfl(wj, j, kWave);
            const float denom = s + 1e-20f;
            wj = __fdiv_rn(wj, denom) * a.scaling;
        } else {
            wj *= a.scaling;
        }
        if (t < a.seq && lane < K) {
            a.ids[(size_t)t * K + lane] = idj;
            a.weights[(size_t)t * K + lane] = wj;
        }
    }
}

// Router from precomputed logits [seq, E] (mirror of moe_router_topk,
// src/kernels/cuda/moe_device.cu:24-98), any E: one wave per token, experts
// strided over lanes; reduction orders match the CPU reference.
__global__ __launch_bounds__(256) void router_from_logits_kernel(RouterArgs a, const float* logits) {
    extern __shared__ float lds[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int E = a.n_experts, K = a.top_k;
    float* row = lds + (size_t)wave * E;
    const int t = blockIdx.x * (blockDim.x >> 6) + wave;
    const bool live = t < a.seq;
    const float* src = logits + (size_t)(live ? t : 0) * E;
    if (a.scoring_sigmoid) {
        for (int e = lane; e < E; e += 64)
            row[e] = __fdiv_rn(1.0f, 1.0f + ref_expf(-src[e], a.fix_offsets, a.fix_entries));
    } else {
        float mx = -INFINITY;
        for (int e = lane; e < E; e += 64) mx = fmaxf(mx, src[e]);
        mx = wave_max(mx);
        for (int e = lane; e < E; e += 64) row[e] = ref_expf(src[e] - mx, a.fix_offsets, a.fix_entries);
        __syncthreads();
        float sum = 0.0f;
        for (int e = 0; e < E; ++e) sum += row[e];
        const float inv = __fdiv_rn(1.0f, sum);
        __syncthreads();
        for (int e = lane; e < E; e += 64) row[e] *= inv;
    }
    __syncthreads();
    float wj = 0.0f;
    int idj = 0;
    for (int j = 0; j < K; ++j) {
        float v = -INFINITY;
        int i = 0x7fffffff;
        for (int e = lane; e < E; e += 64)
            if (row[e] > v) {
                v = row[e];
                i = e;
            }
        wave_argmax(v, i);
        if (!(v > -1e30f)) i = -1;
        if (lane == j) {
            idj = i;
            wj = v;
        }
        __syncthreads();
        if (i >= 0 && lane == (i & 63)) row[i] = -1e30f;
        __syncthreads();
    }
    if (K > 1 && a.norm_topk_prob) {
        float s = 0.0f;
        for (int j = 0; j < K; ++j) s += __shfl(wj, j, kWave);
        wj = __fdiv_rn(wj, s + 1e-20f) * a.scaling;
    } else {
        wj *= a.scaling;
    }
    if (live && lane < K) {
        a.ids[(size_t)t * K + lane] = idj;
        a.weights[(size_t)t * K + lane] = wj;
    }
}

// ---------------------------------------------------------------------------
// Stable grouping (one workgroup of 1024 threads).
// ---------------------------------------------------------------------------
constexpr int kGroupThreads = 1024;
constexpr int kGroupWaves = kGroupThreads / 64;

__global__ __launch_bounds__(kGroupThreads) void group_kernel(GroupArgs g) {
    __shared__ int hist[kMaxExperts];
    __shared__ int offs[kMaxExperts + 1];
    __shared__ int run[kMaxExperts];
    __shared__ int wcnt[kGroupWaves][kMaxExperts];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int E = g.n_experts, N = g.seq * g.top_k;
    const int Ev = E + g.n_virtual;

    for (int e = tid; e < kMaxExperts; e += kGroupThreads) {
        hist[e] = 0;
        run[e] = 0;
    }
    __syncthreads();
    for (int i = tid; i < N; i += kGroupThreads) {
        const int e = g.ids[i];
        if (e >= 0 && e < E) atomicAdd(&hist[e], 1);
    }
    __syncthreads();
    if (tid == 0) {
        int s = 0;
        for (int e = 0; e < Ev; ++e) {
            offs[e] = s;
            s += (e < E) ? hist[e] : g.seq;
        }
        offs[Ev] = s;
    }
    __syncthreads();
    if (g.counts) {
        for (int e = tid; e < Ev; e += kGroupThreads) {
            g.counts[e] = (e < E) ? hist[e] : g.seq;
            g.offsets[e] = offs[e];
        }
        if (tid == 0) g.offsets[Ev] = offs[Ev];
    }
    // m-tile list: tiles of BM slots per expert, experts in index order
    if (g.tile_e) {
        if (tid == 0) {
            int nt = 0;
            for (int e = 0; e < Ev; ++e) {
                const int c = offs[e + 1] - offs[e];
                run[e] = nt;  // temporarily: first tile of e
                nt += (c + g.bm - 1) / g.bm;
            }
            *g.n_tiles = nt;
        }
        __syncthreads();
        for (int e = tid; e < Ev; e += kGroupThreads) {
            const int c = offs[e + 1] - offs[e];
            const int nt = (c + g.bm - 1) / g.bm;
            for (int m = 0; m < nt; ++m) {
                g.tile_e[run[e] + m] = e;
                g.tile_m0[run[e] + m] = m * g.bm;
            }
        }
        __syncthreads();
        for (int e = tid; e < kMaxExperts; e += kGroupThreads) run[e] = 0;
        __syncthreads();
    }
    // stable placement of the routed entries, kGroupThreads entries per round
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int base = 0; base < N; base += kGroupThreads) {
        for (int i = tid; i < kGroupWaves * kMaxExperts; i += kGroupThreads) (&wcnt[0][0])[i] = 0;
        __syncthreads();
        const int i = base + tid;
        const int e = (i < N) ? g.ids[i] : -1;
        const bool valid = e >= 0 && e < E;
        uint64_t m = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 7; ++b) {
            const uint64_t bal = __ballot(valid && ((e >> b) & 1));
            m &= (valid && ((e >> b) & 1)) ? bal : ~bal;
        }
        const int rank = __popcll(m & below);
        if (valid && rank == 0) wcnt[wave][e] = __popcll(m);
        __syncthreads();
        for (int ee = tid; ee < E; ee += kGroupThreads) {
            int acc = run[ee];
            for (int w = 0; w < kGroupWaves; ++w) {
                const int c = wcnt[w][ee];
                wcnt[w][ee] = acc;
                acc += c;
            }
            run[ee] = acc;
        }
        __syncthreads();
        if (valid) {
            const int r = wcnt[wave][e] + rank;  // position within expert e
            const float w = g.weights[i];
            if (g.slot_tok) {
                const int s = offs[e] + r;
                g.slot_tok[s] = i / g.top_k;
                g.slot_w[s] = w;
                if (g.pos) g.pos[i] = s;
            }
            if (g.assign_token && r < g.cap) {
                g.assign_token[(size_t)e * g.cap + r] = i / g.top_k;
                g.assign_w[(size_t)e * g.cap + r] = w;
            }
        }
        __syncthreads();
    }
    if (g.assign_count)
        for (int e = tid; e < E; e += kGroupThreads) g.assign_count[e] = min(hist[e], g.cap);
    // virtual (shared-expert) groups: every token, weight 1
    if (g.slot_tok) {
        for (int v = 0; v < g.n_virtual; ++v)
            for (int t = tid; t < g.seq; t += kGroupThreads) {
                g.slot_tok[offs[E + v] + t] = t;
                g.slot_w[offs[E + v] + t] = 1.0f;
            }
    }
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
hipError_t launch_router(const RouterArgs& a, bool x_is_bf16, hipStream_t st) {
    const int waves = 4;
    const bool rms = a.rms_weight != nullptr;
    const bool big = a.seq >= 1024;
    const int tpw = big ? 4 : 1;
    const int tokens_per_block = waves * tpw;
    const dim3 grid((a.seq + tokens_per_block - 1) / tokens_per_block);
    const size_t lds = ((size_t)waves * tpw * a.hidden + waves * 64) * sizeof(float);
    // the large-T variant needs > 64 KiB of dynamic LDS; raise the limit once per kernel
#define UOCR_ROUTER_CASE(XT, R, TPW)                                                                 \
    {                                                                                                \
        static hipError_t attr_ = hipFuncSetAttribute((const void*)router_kernel<XT, R, TPW>,        \
                                                      hipFuncAttributeMaxDynamicSharedMemorySize,    \
                                                      160 * 1024);                                   \
        if (attr_ != hipSuccess) return attr_;                                                       \
        hipLaunchKernelGGL((router_kernel<XT, R, TPW>), grid, dim3(64 * waves), lds, st, a);         \
    }
    if (x_is_bf16) {
        if (rms) {
            if (big) UOCR_ROUTER_CASE(uint16_t, true, 4) else UOCR_ROUTER_CASE(uint16_t, true, 1)
        } else {
            if (big) UOCR_ROUTER_CASE(uint16_t, false, 4) else UOCR_ROUTER_CASE(uint16_t, false, 1)
        }
    } else {
        if (rms) {
            if (big) UOCR_ROUTER_CASE(float, true, 4) else UOCR_ROUTER_CASE(float, true, 1)
        } else {
            if (big) UOCR_ROUTER_CASE(float, false, 4) else UOCR_ROUTER_CASE(float, false, 1)
        }
    }
#undef UOCR_ROUTER_CASE
    return hipGetLastError();
}

hipError_t launch_router_from_logits(const RouterArgs& a, const float* logits, hipStream_t st) {
    const int waves = 4;
    const dim3 grid((a.seq + waves - 1) / waves);
    const size_t lds = (size_t)waves * a.n_experts * sizeof(float);
    hipLaunchKernelGGL(router_from_logits_kernel, grid, dim3(64 * waves), lds, st, a, logits);
    return hipGetLastError();
}

hipError_t launch_group(const GroupArgs& g, hipStream_t st) {
    hipLaunchKernelGGL(group_kernel, dim3(1), dim3(kGroupThreads), 0, st, g);
    return hipGetLastError();
}

}  // namespace uocr_hip
