// Device router: optional RMSNorm prologue, router logits, softmax / sigmoid
// scoring, greedy top-k, and the stable token->expert grouping.
//
// Bit-exactness contract with the reference CPU path:
//   logits   src/kernels/cpu_ops.cpp:26-39 -- one sequential fmaf chain per
//            (token, expert), k ascending (the -march=native build contracts
//            `acc += x * w`); one lane per expert runs exactly that chain.
//   rmsnorm  src/kernels/cpu_ops.cpp:58-67 -- as the reference's -O3
//            -march=native build runs it: each x*x rounded, summed in column
//            order (only a scalar tail of H % 4 terms would be fused),
//            correctly rounded divide and sqrt, (x * inv) * w.
//   softmax  src/kernels/cpu_ops.cpp:93-106 -- exp(l - max) with glibc's expf
//            bits (correctly rounded exp + the generated fix-up table), sum in
//            expert order, p = e * (1 / sum).
//   top-k    src/engine/moe_decoder.cpp:264-287 -- strict '>' greedy selection,
//            ties to the lowest expert index, optional renormalisation.
//   grouping src/engine/gpu_decoder.cu:602-609 -- per expert, tokens in
//            ascending (token, j) order: a stable counting sort, built here from
//            wave ballots (equal-expert masks) and per-wave LDS prefix counts.
#include <mutex>

#include "launch.hpp"
#include "routing.hpp"

namespace uocr_hip {

// Sticky flag of the moe_router_topk mirror: set when an expert received more
// entries than the [n_experts, cap] tables hold (the reference drops them
// silently, src/kernels/cuda/moe_device.cu:90-95). Written with vector atomics,
// read and cleared by router_overflow_read.
__device__ int g_router_overflow;

// Grouping scratch of the moe_router_topk mirror, whose reference signature
// has no workspace: the multi-workgroup grouping's per-entry ranks and
// per-(chunk, expert) counts / bases for up to kMirrorGroupEntries routed
// entries (larger calls run the single-workgroup rounds). One copy per device;
// host code reaches it through hipGetSymbolAddress only.
constexpr int kMirrorGroupEntries = 1 << 17;
constexpr int kMirrorGroupChunks = kMirrorGroupEntries / 1024;
__device__ int g_mirror_lrank[kMirrorGroupEntries];
__device__ int g_mirror_chunk_count[kMirrorGroupChunks * kMaxExperts];
__device__ int g_mirror_chunk_base[kMirrorGroupChunks * kMaxExperts];

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

// ---------------------------------------------------------------------------
// Stable grouping body (one workgroup of 1024 threads), shared by the
// stand-alone group kernel and the router kernel's fused tail.
// ---------------------------------------------------------------------------
constexpr int kGroupThreads = 1024;
constexpr int kGroupWaves = kGroupThreads / 64;

struct GroupLds {
    int hist[kMaxExperts];
    int offs[kMaxExperts + 1];
    int tile0[kMaxExperts + 1];
    int short0[kMaxExperts + 1];
    int nshort[kMaxExperts];
    int run[kMaxExperts];
    int wcnt[kGroupWaves][kMaxExperts];   // per-wave counts of the round
    int wbase[kGroupWaves][kMaxExperts];  // exclusive per-wave prefix of the round
};

// Exclusive prefix sum of v[0..n) (n <= 128) by wave 0; out[n] = total.
__device__ __forceinline__ void wave0_exclusive_scan(const int* v, int* out, int n) {
    const int lane = threadIdx.x & 63;
    const int a = (2 * lane < n) ? v[2 * lane] : 0;
    const int b = (2 * lane + 1 < n) ? v[2 * lane + 1] : 0;
    int inc = a + b;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(inc, o, kWave);
        if (lane >= o) inc += u;
    }
    const int ex = inc - a - b;
    if (2 * lane < n) out[2 * lane] = ex;
    if (2 * lane + 1 < n) out[2 * lane + 1] = ex + a;
    if (lane == 63) out[n] = inc;
}

// Tile list order: every expert's tiles of more than bm/2 rows first, then
// each expert's short last tile (1 .. bm/2 rows), so the short tiles (which
// the large-tile prefill kernel runs in half mode) fill the grid's last round.
// Long / short tile counts of a group of c rows:
__device__ __forceinline__ int short_tiles(int c, int bm) {
    const int rem = c % bm;
    return (rem != 0 && rem <= bm / 2) ? 1 : 0;
}
__device__ __forceinline__ int long_tiles(int c, int bm) { return (c + bm - 1) / bm - short_tiles(c, bm); }
// Write the list from the exclusive scans of the long (tile0) and short
// (short0) counts over Ev groups of hist[] rows. Called by all threads.
__device__ __forceinline__ void write_tile_list(const GroupArgs& g, const int* hist, const int* offs,
                                                const int* tile0, const int* short0, int Ev) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int nlong = tile0[Ev];
    if (tid == 0) *g.n_tiles = nlong + short0[Ev];
    for (int e = wave; e < Ev; e += kGroupWaves) {
        const int nt = tile0[e + 1] - tile0[e];
        auto put = [&](int idx, int m0) {
            g.tile_e[idx] = e;
            g.tile_m0[idx] = m0;
            if (g.tile_info)
                *reinterpret_cast<int4*>(g.tile_info + 4 * idx) =
                    make_int4(e, m0, min(g.bm, hist[e] - m0), offs[e] + m0);
        };
        for (int m = lane; m < nt; m += 64) put(tile0[e] + m, m * g.bm);
        if (lane == 0 && short0[e + 1] > short0[e]) put(nlong + short0[e], nt * g.bm);
    }
}

// `ids` / `wts` may live in global memory or LDS. Must be called by all 1024 threads.
__device__ void group_body(const int* ids, const float* wts, const GroupArgs& g, GroupLds& s) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int E = g.n_experts, N = g.seq * g.top_k;
    const int Ev = E + g.n_virtual;

    for (int e = tid; e < kMaxExperts; e += kGroupThreads) {
        s.hist[e] = 0;
        s.run[e] = 0;
    }
    __syncthreads();
    for (int i = tid; i < N; i += kGroupThreads) {
        const int e = ids[i];
        if (e >= 0 && e < E) atomicAdd(&s.hist[e], 1);
    }
    __syncthreads();
    if (wave == 0) {
        for (int e = lane; e < g.n_virtual; e += 64) s.hist[E + e] = g.seq;  // virtual groups: all tokens
    }
    __syncthreads();
    if (wave == 0) wave0_exclusive_scan(s.hist, s.offs, Ev);
    if (wave == 1 && g.tile_e) {
        // tiles per expert into run[] (reset below), then scan into tile0[]
        for (int e = lane; e < Ev; e += 64) {
            s.run[e] = long_tiles(s.hist[e], g.bm);
            s.nshort[e] = short_tiles(s.hist[e], g.bm);
        }
    }
    __syncthreads();
    if (g.tile_e && wave == 1) wave0_exclusive_scan(s.run, s.tile0, Ev);
    if (g.tile_e && wave == 2) wave0_exclusive_scan(s.nshort, s.short0, Ev);
    __syncthreads();
    if (g.counts) {
        for (int e = tid; e < Ev; e += kGroupThreads) {
            g.counts[e] = s.hist[e];
            g.offsets[e] = s.offs[e];
        }
        if (tid == 0) g.offsets[Ev] = s.offs[Ev];
    }
    if (g.tile_e) write_tile_list(g, s.hist, s.offs, s.tile0, s.short0, Ev);
    for (int e = tid; e < kMaxExperts; e += kGroupThreads) s.run[e] = 0;
    __syncthreads();
    // stable placement of the routed entries, kGroupThreads entries per round
    // (entry i = base + tid, so lane order, then wave order, is (t, j) order)
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int nid = (tid < N) ? ids[tid] : -1;
    float nw = (tid < N) ? wts[tid] : 0.0f;
    for (int base = 0; base < N; base += kGroupThreads) {
        const int i = base + tid;
        const int e = nid;
        const float w = nw;
        if (base + kGroupThreads + tid < N) {  // next round's entry, in flight during this round
            nid = ids[base + kGroupThreads + tid];
            nw = wts[base + kGroupThreads + tid];
        }
        for (int k = tid; k < kGroupWaves * kMaxExperts; k += kGroupThreads) (&s.wcnt[0][0])[k] = 0;
        __syncthreads();
        // i < N: past the last round's end, nid still holds an earlier round's id
        const bool valid = i < N && e >= 0 && e < E;
        uint64_t m = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 7; ++b) {
            const bool bit = valid && ((e >> b) & 1);
            const uint64_t bal = __ballot(bit);
            m &= bit ? bal : ~bal;
        }
        const int rank = __popcll(m & below);
        if (valid && rank == 0) s.wcnt[wave][e] = __popcll(m);
        __syncthreads();
        // exclusive prefix over waves, one thread per (wave, expert)
        for (int ee = lane; ee < E; ee += 64) {
            int acc = s.run[ee];
            for (int w2 = 0; w2 < wave; ++w2) acc += s.wcnt[w2][ee];
            s.wbase[wave][ee] = acc;
        }
        __syncthreads();
        if (wave == kGroupWaves - 1)
            for (int ee = lane; ee < E; ee += 64) s.run[ee] = s.wbase[wave][ee] + s.wcnt[wave][ee];
        if (valid) {
            const int r = s.wbase[wave][e] + rank;  // position within expert e
            if (g.slot_tok) {
                const int sl = s.offs[e] + r;
                g.slot_tok[sl] = i / g.top_k;
                g.slot_w[sl] = w;
                if (g.pos) g.pos[i] = sl;
            }
            if (g.assign_token && r < g.cap) {
                g.assign_token[(size_t)e * g.cap + r] = i / g.top_k;
                g.assign_w[(size_t)e * g.cap + r] = w;
            }
        }
        __syncthreads();
    }
    if (g.assign_count)
        for (int e = tid; e < E; e += kGroupThreads) {
            g.assign_count[e] = min(s.hist[e], g.cap);
            if (s.hist[e] > g.cap) atomicOr(&g_router_overflow, 1);
        }
    if (g.slot_tok) {
        for (int v = 0; v < g.n_virtual; ++v)
            for (int t = tid; t < g.seq; t += kGroupThreads) {
                g.slot_tok[s.offs[E + v] + t] = t;
                g.slot_w[s.offs[E + v] + t] = 1.0f;
            }
    }
}

__global__ __launch_bounds__(kGroupThreads) void group_kernel(GroupArgs g) {
    __shared__ GroupLds s;
    group_body(g.ids, g.weights, g, s);
}

// ---------------------------------------------------------------------------
// Multi-workgroup stable grouping for large batches: three launches, each of
// which finishes all of its loads before its first store (on gfx9 the vmcnt
// wait for a load also waits for every earlier store).
//   rank:  per 1024-entry chunk, stable rank of each entry among the chunk's
//          entries of the same expert + the chunk's per-expert counts;
//   scan:  expert totals, offsets, tile list and per-(chunk, expert) bases;
//   place: slot = base[chunk][expert] + rank.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kGroupThreads) void group_rank_kernel(GroupArgs g) {
    __shared__ int wcnt[kGroupWaves][kMaxExperts];
    __shared__ int wbase[kGroupWaves][kMaxExperts];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int E = g.n_experts, N = g.seq * g.top_k;
    const int i = blockIdx.x * kGroupThreads + tid;
    const int e = (i < N) ? g.ids[i] : -1;
    for (int k = tid; k < kGroupWaves * kMaxExperts; k += kGroupThreads) (&wcnt[0][0])[k] = 0;
    __syncthreads();
    const bool valid = e >= 0 && e < E;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    uint64_t m = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 7; ++b) {
        const bool bit = valid && ((e >> b) & 1);
        const uint64_t bal = __ballot(bit);
        m &= bit ? bal : ~bal;
    }
    const int rank = __popcll(m & below);
    if (valid && rank == 0) wcnt[wave][e] = __popcll(m);
    __syncthreads();
    for (int ee = lane; ee < E; ee += 64) {
        int acc = 0;
        for (int w2 = 0; w2 < wave; ++w2) acc += wcnt[w2][ee];
        wbase[wave][ee] = acc;
    }
    __syncthreads();
    if (i < N) g.lrank[i] = valid ? wbase[wave][e] + rank : 0;
    if (wave == kGroupWaves - 1)
        for (int ee = lane; ee < E; ee += 64)
            g.chunk_count[(size_t)blockIdx.x * E + ee] = wbase[wave][ee] + wcnt[wave][ee];
}

__global__ __launch_bounds__(kGroupThreads) void group_scan_kernel(GroupArgs g, int n_chunks) {
    extern __shared__ int cc[];  // [n_chunks][E] counts, then bases
    __shared__ int hist[kMaxExperts], offs[kMaxExperts + 1], ntl[kMaxExperts], tile0[kMaxExperts + 1];
    __shared__ int nsh[kMaxExperts], short0[kMaxExperts + 1];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int E = g.n_experts, Ev = E + g.n_virtual;
    for (int k = tid; k < n_chunks * E; k += kGroupThreads) cc[k] = g.chunk_count[k];
    __syncthreads();
    for (int e = tid; e < Ev; e += kGroupThreads) {
        int acc = 0;
        if (e < E)
            for (int c = 0; c < n_chunks; ++c) {
                const int v = cc[c * E + e];
                cc[c * E + e] = acc;  // exclusive base within expert e
                acc += v;
            }
        else
            acc = g.seq;
        hist[e] = acc;
        ntl[e] = long_tiles(acc, g.bm);
        nsh[e] = short_tiles(acc, g.bm);
    }
    __syncthreads();
    if (wave == 0) wave0_exclusive_scan(hist, offs, Ev);
    if (wave == 1) wave0_exclusive_scan(ntl, tile0, Ev);
    if (wave == 2) wave0_exclusive_scan(nsh, short0, Ev);
    __syncthreads();
    for (int k = tid; k < n_chunks * E; k += kGroupThreads) g.chunk_base[k] = cc[k] + (g.slot_tok ? offs[k % E] : 0);
    for (int e = tid; e < Ev; e += kGroupThreads) {
        if (g.counts) {
            g.counts[e] = hist[e];
            g.offsets[e] = offs[e];
        }
        if (g.assign_count && e < E) {
            g.assign_count[e] = min(hist[e], g.cap);
            if (hist[e] > g.cap) atomicOr(&g_router_overflow, 1);
        }
    }
    if (tid == 0 && g.counts) g.offsets[Ev] = offs[Ev];
    if (g.tile_e) write_tile_list(g, hist, offs, tile0, short0, Ev);
    // virtual (shared-expert) groups: every token, weight 1
    if (g.slot_tok)
        for (int v = 0; v < g.n_virtual; ++v)
            for (int t = tid; t < g.seq; t += kGroupThreads) {
                g.slot_tok[offs[E + v] + t] = t;
                g.slot_w[offs[E + v] + t] = 1.0f;
            }
}

// Scan and place in one launch, for up to kGroupFusedMaxChunks chunks: every
// workgroup (one per 1024-entry chunk) reduces the per-(chunk, expert) counts
// itself (n_chunks x E ints from L2), so its bases need no other workgroup;
// workgroup 0 also writes the expert totals, offsets and tile list, and the
// virtual groups' slots are spread over all of them. All loads come before
// the first store.
constexpr int kGroupFusedMaxChunks = 64;

__global__ __launch_bounds__(kGroupThreads) void group_scan_place_kernel(GroupArgs g, int n_chunks) {
    extern __shared__ int cc[];  // [n_chunks][E] counts
    __shared__ int hist[kMaxExperts], offs[kMaxExperts + 1], base[kMaxExperts];
    __shared__ int ntl[kMaxExperts], tile0[kMaxExperts + 1], nsh[kMaxExperts], short0[kMaxExperts + 1];
    const int tid = threadIdx.x, wave = tid >> 6;
    const int E = g.n_experts, Ev = E + g.n_virtual, N = g.seq * g.top_k;
    const int b = blockIdx.x;
    const int i = b * kGroupThreads + tid;
    const int e_i = i < N ? g.ids[i] : -1;
    const bool valid = e_i >= 0 && e_i < E;
    const int lr = valid ? g.lrank[i] : 0;
    const float w_i = valid ? g.weights[i] : 0.0f;
    for (int k = tid; k < n_chunks * E; k += kGroupThreads) cc[k] = g.chunk_count[k];
    __syncthreads();
    for (int e = tid; e < Ev; e += kGroupThreads) {
        int acc = 0;
        if (e < E) {
            int mine = 0;
            for (int c = 0; c < n_chunks; ++c) {
                if (c == b) mine = acc;
                acc += cc[c * E + e];
            }
            base[e] = mine;  // entries of expert e in the chunks before this one
        } else {
            acc = g.seq;
        }
        hist[e] = acc;
        ntl[e] = long_tiles(acc, g.bm);
        nsh[e] = short_tiles(acc, g.bm);
    }
    __syncthreads();
    if (wave == 0) wave0_exclusive_scan(hist, offs, Ev);
    if (b == 0 && g.tile_e && wave == 1) wave0_exclusive_scan(ntl, tile0, Ev);
    if (b == 0 && g.tile_e && wave == 2) wave0_exclusive_scan(nsh, short0, Ev);
    __syncthreads();
    if (valid) {
        if (g.slot_tok) {  // the slot
            const int r = offs[e_i] + base[e_i] + lr;
            g.slot_tok[r] = i / g.top_k;
            g.slot_w[r] = w_i;
            if (g.pos) g.pos[i] = r;
        } else if (g.assign_token) {  // the position within expert e_i
            const int r = base[e_i] + lr;
            if (r < g.cap) {
                g.assign_token[(size_t)e_i * g.cap + r] = i / g.top_k;
                g.assign_w[(size_t)e_i * g.cap + r] = w_i;
            }
        }
    }
    if (b == 0) {
        for (int e = tid; e < Ev; e += kGroupThreads) {
            if (g.counts) {
                g.counts[e] = hist[e];
                g.offsets[e] = offs[e];
            }
            if (g.assign_count && e < E) {
                g.assign_count[e] = min(hist[e], g.cap);
                if (hist[e] > g.cap) atomicOr(&g_router_overflow, 1);
            }
        }
        if (tid == 0 && g.counts) g.offsets[Ev] = offs[Ev];
        if (g.tile_e) write_tile_list(g, hist, offs, tile0, short0, Ev);
    }
    // virtual (shared-expert) groups: every token, weight 1
    if (g.slot_tok)
        for (int v = 0; v < g.n_virtual; ++v)
            for (int t = i; t < g.seq; t += n_chunks * kGroupThreads) {
                g.slot_tok[offs[E + v] + t] = t;
                g.slot_w[offs[E + v] + t] = 1.0f;
            }
}

__global__ __launch_bounds__(256) void group_place_kernel(GroupArgs g) {
    const int E = g.n_experts, N = g.seq * g.top_k;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    const int e = g.ids[i];
    if (e < 0 || e >= E) return;
    const int r = g.chunk_base[(size_t)(i / kGroupThreads) * E + e] + g.lrank[i];
    const float w = g.weights[i];
    if (g.slot_tok) {  // r is the slot (bases include the expert offset)
        g.slot_tok[r] = i / g.top_k;
        g.slot_w[r] = w;
        if (g.pos) g.pos[i] = r;
    }
    if (g.assign_token && r < g.cap) {  // r is the position within expert e
        g.assign_token[(size_t)e * g.cap + r] = i / g.top_k;
        g.assign_w[(size_t)e * g.cap + r] = w;
    }
}

// ---------------------------------------------------------------------------
// Router: one wave per token, lane e owns expert e (E <= 64); a workgroup of W
// waves routes W tokens (W = 4 for small batches, so the FMA chains of
// different tokens run on different SIMDs and CUs; W = 16 for large batches,
// so each streamed weight chunk serves 16 tokens). The router matrix
// ([H/8][E][8] bf16) streams through LDS in double-buffered 128-column chunks,
// so every lane's FMA chain reads its weights from LDS instead of issuing one
// dependent global load per 8 columns.
// ---------------------------------------------------------------------------
constexpr int kChunkC8 = 16;  // 128 columns per chunk

__host__ __device__ constexpr size_t router_lds_bytes(int H, int waves) {
    return (size_t)waves * H * 4          // xs
           + 2ull * kChunkC8 * 64 * 16    // W chunks (E <= 64)
           + (size_t)waves * 64 * 4;      // per-wave scores
}

constexpr int kMaxChunks = 14;  // hidden <= 1792

template <typename XT, bool RMS, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void router_kernel(RouterArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    constexpr int NT = WAVES * 64;
    constexpr int UPT = kChunkC8 * 64 / NT;  // 16-byte chunk units per thread (E <= 64)
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, tid = threadIdx.x;
    const int H = a.hidden, E = a.n_experts, K = a.top_k;
    float* xs = reinterpret_cast<float*>(smem) + (size_t)wave * H;
    u32x4* wb = reinterpret_cast<u32x4*>(smem + (size_t)WAVES * H * 4);
    float* scr = reinterpret_cast<float*>(wb + 2 * kChunkC8 * 64) + wave * 64;
    __shared__ uint64_t etab[32];
    if (threadIdx.x < 32) etab[threadIdx.x] = uocr_exp2_tab[threadIdx.x];
    const int t = blockIdx.x * WAVES + wave;
    const bool live = t < a.seq;
    const XT* x = static_cast<const XT*>(a.x);
    const int chunk_units = kChunkC8 * E;
    const u32x4* wsrc = reinterpret_cast<const u32x4*>(a.router_t);
    const int n_chunks = H / (kChunkC8 * 8);

    // every router-weight load of this thread, all chunks, issued at once
    u32x4 wreg[kMaxChunks][UPT];
#pragma unroll
    for (int ch = 0; ch < kMaxChunks; ++ch)
#pragma unroll
        for (int j = 0; j < UPT; ++j) {
            const int u = tid + j * NT;
            if (ch < n_chunks && u < chunk_units) wreg[ch][j] = wsrc[(size_t)ch * chunk_units + u];
        }
    // this wave's token row, as f32
    for (int c = lane * 8; c < H; c += 64 * 8) {
        float v[8];
        if (live) {
            load8_f32<XT>(x + (size_t)t * H + c, v);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = 0.0f;
        }
        *reinterpret_cast<f32x4*>(xs + c) = f32x4{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f32x4*>(xs + c + 4) = f32x4{v[4], v[5], v[6], v[7]};
    }
#pragma unroll
    for (int j = 0; j < UPT; ++j)
        if (tid + j * NT < chunk_units) wb[tid + j * NT] = wreg[0][j];
    __syncthreads();

    if constexpr (RMS) {
        if (lane == 0) {
            float ss = 0.0f;
            for (int c = 0; c < H; c += 4) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(xs + c);
                // the reference build rounds each x*x and sums in order (H % 4 == 0 here)
#pragma unroll
                for (int i = 0; i < 4; ++i) ss = __fadd_rn(ss, __fmul_rn(v[i], v[i]));
            }
            scr[0] = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)H), a.rms_eps)));
        }
        __syncthreads();
        const float inv = scr[0];
        for (int c = lane; c < H; c += 64) xs[c] = __fmul_rn(__fmul_rn(xs[c], inv), a.rms_weight[c]);
        __syncthreads();
    }

    if (live) {
        for (int c = lane * 8; c < H; c += 64 * 8) {
            const f32x4 p = *reinterpret_cast<const f32x4*>(xs + c);
            const f32x4 q = *reinterpret_cast<const f32x4*>(xs + c + 4);
            f16x8 h = {(f16)p[0], (f16)p[1], (f16)p[2], (f16)p[3], (f16)q[0], (f16)q[1], (f16)q[2], (f16)q[3]};
            *reinterpret_cast<f16x8*>(a.x16 + (size_t)t * H + c) = h;
        }
    }

    // logits: lane e runs the sequential fmaf chain over all H columns
    float acc = 0.0f;
    if constexpr (!RMS && WAVES == 16) {
        // The token row is the same for every lane of the wave: it comes in
        // through scalar loads (16 dwords per block, the next block requested
        // while this one is consumed), so LDS serves only the weight reads.
        constexpr int DW = 2 * (int)sizeof(XT);  // dwords per 8 columns
        constexpr int BC = 16 / DW;               // 8-column steps per block
        constexpr int NB = kChunkC8 / BC;         // blocks per chunk
        const int n_blocks = n_chunks * NB;
        const int tu = min(__builtin_amdgcn_readfirstlane(t), a.seq - 1);
        const uint64_t row = (uint64_t)(x + (size_t)tu * H);
        auto block_load = [&](int b, u32x16& q) {
            const uint64_t ad = row + (uint64_t)min(b, n_blocks - 1) * 64u;
            asm volatile("s_load_dwordx16 %0, %1, 0x0" : "=s"(q) : "s"(ad) : "memory");
        };
        u32x16 c0;
        block_load(0, c0);
#pragma unroll
        for (int ch = 0; ch < kMaxChunks; ++ch) {
            if (ch < n_chunks) {
                const u32x4* cur = wb + (ch & 1) * kChunkC8 * 64;
#pragma unroll
                for (int bl = 0; bl < NB; ++bl) {
                    // (acc ties the previous block's chain to this point, so
                    // the loads are not all hoisted to the chunk's start)
                    asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(c0), "+v"(acc)::"memory");
                    u32x16 n0;
                    block_load(ch * NB + bl + 1, n0);
#pragma unroll
                    for (int i = 0; i < BC; ++i) {
                        const u32x4 wv = cur[(bl * BC + i) * E + lane];
                        float xv[8];
#pragma unroll
                        for (int k = 0; k < DW; ++k) {
                            const uint32_t d = c0[DW * i + k];
                            if constexpr (sizeof(XT) == 2) {
                                xv[2 * k] = __uint_as_float(d << 16);
                                xv[2 * k + 1] = __uint_as_float(d & 0xffff0000u);
                            } else {
                                xv[k] = __uint_as_float(d);
                            }
                        }
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            acc = fmaf(xv[2 * k], __uint_as_float(wv[k] << 16), acc);
                            acc = fmaf(xv[2 * k + 1], __uint_as_float(wv[k] & 0xffff0000u), acc);
                        }
                    }
                    c0 = n0;
                }
                if (ch + 1 < kMaxChunks && ch + 1 < n_chunks) {
#pragma unroll
                    for (int j = 0; j < UPT; ++j)
                        if (tid + j * NT < chunk_units)
                            wb[((ch + 1) & 1) * kChunkC8 * 64 + tid + j * NT] = wreg[ch + 1][j];
                }
                __syncthreads();
            }
        }
        // the last block's (clamped, repeated) loads must land before exit
        asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(c0)::"memory");
    } else
#pragma unroll
    for (int ch = 0; ch < kMaxChunks; ++ch) {
        if (ch < n_chunks) {
            const u32x4* cur = wb + (ch & 1) * kChunkC8 * 64;
            if (lane < E) {
#pragma unroll 4
                for (int c8 = 0; c8 < kChunkC8; ++c8) {
                    const u32x4 wv = cur[c8 * E + lane];
                    const float* xp = xs + (ch * kChunkC8 + c8) * 8;
                    const f32x4 xa = *reinterpret_cast<const f32x4*>(xp);
                    const f32x4 xb = *reinterpret_cast<const f32x4*>(xp + 4);
                    acc = fmaf(xa[0], __uint_as_float(wv[0] << 16), acc);
                    acc = fmaf(xa[1], __uint_as_float(wv[0] & 0xffff0000u), acc);
                    acc = fmaf(xa[2], __uint_as_float(wv[1] << 16), acc);
                    acc = fmaf(xa[3], __uint_as_float(wv[1] & 0xffff0000u), acc);
                    acc = fmaf(xb[0], __uint_as_float(wv[2] << 16), acc);
                    acc = fmaf(xb[1], __uint_as_float(wv[2] & 0xffff0000u), acc);
                    acc = fmaf(xb[2], __uint_as_float(wv[3] << 16), acc);
                    acc = fmaf(xb[3], __uint_as_float(wv[3] & 0xffff0000u), acc);
                }
            }
            if (ch + 1 < kMaxChunks && ch + 1 < n_chunks) {
#pragma unroll
                for (int j = 0; j < UPT; ++j)
                    if (tid + j * NT < chunk_units) wb[((ch + 1) & 1) * kChunkC8 * 64 + tid + j * NT] = wreg[ch + 1][j];
            }
            __syncthreads();
        }
    }

    // scoring and greedy top-k by the wave alone (no workgroup barrier)
    const WaveTopk pick = wave_topk(acc, E, K, a.scoring_sigmoid, a.norm_topk_prob, a.scaling, scr, etab);
    if (live && lane < K) a.weights[(size_t)t * K + lane] = pick.w;
    if (live && pick.rank < K) a.ids[(size_t)t * K + pick.rank] = lane;
}


// Router without the RMSNorm prologue for fewer than 4096 tokens: one token
// per wave, one wave per SIMD, where a wave issues one VALU op every several
// cycles whatever the dependences. The weights therefore come from the f32
// copy of the router ([H/4][64][4]: a 128-column chunk is one contiguous
// 32 KiB block), so a column costs one FMA and no widening; the chunks stream
// through LDS from a register ring as in router_kernel.
constexpr int kF32ChunkUnits = kChunkC8 * 2 * 64;  // 16-byte units per 128-column chunk

__host__ __device__ constexpr size_t router_f32w_lds_bytes(int H) {
    return (size_t)4 * H * 4                     // xs
           + 2ull * kF32ChunkUnits * 16         // W chunks
           + (size_t)4 * 64 * 4;                // per-wave scores
}

template <typename XT>
__global__ __launch_bounds__(256) void router_f32w_kernel(RouterArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    constexpr int WAVES = 4, NT = 256;
    constexpr int UPT = kF32ChunkUnits / NT;  // 8
    constexpr int RING = 3;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, tid = threadIdx.x;
    const int H = a.hidden, E = a.n_experts, K = a.top_k;
    float* xs = reinterpret_cast<float*>(smem) + (size_t)wave * H;
    f32x4* wb = reinterpret_cast<f32x4*>(smem + (size_t)WAVES * H * 4);
    float* scr = reinterpret_cast<float*>(wb + 2 * kF32ChunkUnits) + wave * 64;
    __shared__ uint64_t etab[32];
    if (threadIdx.x < 32) etab[threadIdx.x] = uocr_exp2_tab[threadIdx.x];
    const int t = blockIdx.x * WAVES + wave;
    const bool live = t < a.seq;
    const XT* x = static_cast<const XT*>(a.x);
    const f32x4* wsrc = reinterpret_cast<const f32x4*>(a.router_f32);
    const int n_chunks = H / (kChunkC8 * 8);

    f32x4 wreg[RING][UPT];
    auto issue_chunk = [&](int ch) {
#pragma unroll
        for (int j = 0; j < UPT; ++j)
            if (ch < n_chunks) wreg[ch % RING][j] = wsrc[(size_t)ch * kF32ChunkUnits + tid + j * NT];
    };
#pragma unroll
    for (int ch = 0; ch < RING; ++ch) issue_chunk(ch);
    // this wave's token row, as f32 (and as f16 for the experts)
    for (int c = lane * 8; c < H; c += 64 * 8) {
        float v[8];
        if (live) {
            load8_f32<XT>(x + (size_t)t * H + c, v);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = 0.0f;
        }
        *reinterpret_cast<f32x4*>(xs + c) = f32x4{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f32x4*>(xs + c + 4) = f32x4{v[4], v[5], v[6], v[7]};
        if (live)
            *reinterpret_cast<f16x8*>(a.x16 + (size_t)t * H + c) =
                f16x8{(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3], (f16)v[4], (f16)v[5], (f16)v[6], (f16)v[7]};
    }
#pragma unroll
    for (int j = 0; j < UPT; ++j) wb[tid + j * NT] = wreg[0][j];
    if (RING < kMaxChunks) issue_chunk(RING);
    __syncthreads();

    // logits: lane e runs the sequential fmaf chain over all H columns (lanes
    // >= E run the zero padding)
    float acc = 0.0f;
#pragma unroll
    for (int ch = 0; ch < kMaxChunks; ++ch) {
        if (ch < n_chunks) {
            const f32x4* cur = wb + (ch & 1) * kF32ChunkUnits;
            const float* xc = xs + ch * kChunkC8 * 8;
            // 32 steps of 4 columns; the LDS reads run 6 steps ahead of the
            // FMAs with explicit lgkmcnt waits (the compiler's schedule waits
            // on every read pair or hoists every read of the chunk)
            const uint32_t w_addr = lds_addr(cur) + lane * 16;
            const uint32_t x_addr = lds_addr(xc);
            asm volatile(UOCR_RCHUNK(UOCR_RMAC_FMA)
                : [acc] "+v"(acc)
                : [w] "v"(w_addr), [x] "v"(x_addr)
                : "v64", "v65", "v66", "v67", "v68", "v69", "v70", "v71", "v72", "v73", "v74", "v75", "v76", "v77",
                  "v78", "v79", "v80", "v81", "v82", "v83", "v84", "v85", "v86", "v87", "v88", "v89", "v90", "v91",
                  "v92", "v93", "v94", "v95", "v96", "v97", "v98", "v99", "v100", "v101", "v102", "v103", "v104",
                  "v105", "v106", "v107", "v108", "v109", "v110", "v111", "memory");
            if (ch + 1 < kMaxChunks && ch + 1 < n_chunks) {
#pragma unroll
                for (int j = 0; j < UPT; ++j) wb[((ch + 1) & 1) * kF32ChunkUnits + tid + j * NT] = wreg[(ch + 1) % RING][j];
                if (ch + 1 + RING < kMaxChunks) issue_chunk(ch + 1 + RING);
            }
            __syncthreads();
        }
    }

    const WaveTopk pick = wave_topk(acc, E, K, a.scoring_sigmoid, a.norm_topk_prob, a.scaling, scr, etab);
    if (live && lane < K) a.weights[(size_t)t * K + lane] = pick.w;
    if (live && pick.rank < K) a.ids[(size_t)t * K + pick.rank] = lane;
}

// Router from precomputed logits [seq, E] (mirror of moe_router_topk,
// src/kernels/cuda/moe_device.cu:24-98), any E: one wave per token, experts
// strided over lanes; reduction orders match the CPU reference.
__global__ __launch_bounds__(256) void router_from_logits_kernel(RouterArgs a, const float* logits) {
    extern __shared__ float lds[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int E = a.n_experts, K = a.top_k;
    float* row = lds + (size_t)wave * E;
    __shared__ uint64_t etab[32];
    if (threadIdx.x < 32) etab[threadIdx.x] = uocr_exp2_tab[threadIdx.x];
    __syncthreads();
    const int t = blockIdx.x * (blockDim.x >> 6) + wave;
    const bool live = t < a.seq;
    const float* src = logits + (size_t)(live ? t : 0) * E;
    if (a.scoring_sigmoid) {
        for (int e = lane; e < E; e += 64)
            row[e] = __fdiv_rn(1.0f, 1.0f + ref_expf(-src[e], etab));
    } else {
        float mx = -INFINITY;
        for (int e = lane; e < E; e += 64) mx = fmaxf(mx, src[e]);
        mx = wave_max(mx);
        for (int e = lane; e < E; e += 64) row[e] = ref_expf(src[e] - mx, etab);
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
// host launchers
// ---------------------------------------------------------------------------
size_t router_smem_bytes(int hidden) { return router_lds_bytes(hidden, 16); }

template <typename XT, bool RMS, int WAVES>
static hipError_t launch_router_t(const RouterArgs& a, hipStream_t st) {
    // > 64 KiB of dynamic LDS: raise the limit once per kernel
    static hipError_t attr = hipFuncSetAttribute((const void*)router_kernel<XT, RMS, WAVES>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);
    if (attr != hipSuccess) return attr;
    const dim3 grid((a.seq + WAVES - 1) / WAVES);
    launch_k((router_kernel<XT, RMS, WAVES>), grid, dim3(WAVES * 64), router_lds_bytes(a.hidden, WAVES),
                       st, a);
    return hipGetLastError();
}

template <typename XT>
static hipError_t launch_router_f32w(const RouterArgs& a, hipStream_t st) {
    static hipError_t attr = hipFuncSetAttribute((const void*)router_f32w_kernel<XT>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);
    if (attr != hipSuccess) return attr;
    launch_k((router_f32w_kernel<XT>), dim3((a.seq + 3) / 4), dim3(256), router_f32w_lds_bytes(a.hidden), st, a);
    return hipGetLastError();
}

template <typename XT, bool RMS>
static hipError_t launch_router_w(const RouterArgs& a, hipStream_t st) {
    if constexpr (!RMS) {
        if (a.seq < 4096 && a.router_f32) return launch_router_f32w<XT>(a, st);
    }
    // 4 tokens per workgroup spread the FMA chains over the CUs; once that
    // gives 4+ workgroups per CU (4096 tokens on 256 CUs), 16 tokens per
    // workgroup amortise the router-weight stream
    return a.seq >= 4096 ? launch_router_t<XT, RMS, 16>(a, st) : launch_router_t<XT, RMS, 4>(a, st);
}

hipError_t launch_router(const RouterArgs& a, bool x_is_bf16, hipStream_t st) {
    if (a.n_experts > 64 || a.hidden > kMaxChunks * kChunkC8 * 8 || a.hidden % (kChunkC8 * 8))
        return hipErrorInvalidValue;
    const bool rms = a.rms_weight != nullptr;
    if (x_is_bf16) return rms ? launch_router_w<uint16_t, true>(a, st) : launch_router_w<uint16_t, false>(a, st);
    return rms ? launch_router_w<float, true>(a, st) : launch_router_w<float, false>(a, st);
}

hipError_t launch_router_from_logits(const RouterArgs& a, const float* logits, hipStream_t st) {
    const int waves = 4;
    const dim3 grid((a.seq + waves - 1) / waves);
    const size_t lds = (size_t)waves * a.n_experts * sizeof(float);
    launch_k(router_from_logits_kernel, grid, dim3(64 * waves), lds, st, a, logits);
    return hipGetLastError();
}

int group_chunks(int seq, int top_k) { return (seq * top_k + kGroupThreads - 1) / kGroupThreads; }

bool group_fits(int seq, int top_k, int n_experts) {
    return (size_t)group_chunks(seq, top_k) * n_experts * sizeof(int) <= kGroupScanLds;
}

hipError_t router_overflow_read(int clear, int* flag) {
    hipError_t e = hipMemcpyFromSymbol(flag, HIP_SYMBOL(g_router_overflow), sizeof(int), 0, hipMemcpyDeviceToHost);
    if (e != hipSuccess || !clear) return e;
    const int zero = 0;
    return hipMemcpyToSymbol(HIP_SYMBOL(g_router_overflow), &zero, sizeof(int), 0, hipMemcpyHostToDevice);
}

hipError_t launch_group_mirror(GroupArgs g, hipStream_t st) {
    if (group_chunks(g.seq, g.top_k) > 1 && (long long)g.seq * g.top_k <= kMirrorGroupEntries) {
        static std::mutex mu;
        static void* addr[3][64] = {};
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return e;
        if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
        {
            std::lock_guard<std::mutex> lock(mu);
            if (!addr[0][dev]) {
                if ((e = hipGetSymbolAddress(&addr[0][dev], HIP_SYMBOL(g_mirror_lrank))) != hipSuccess ||
                    (e = hipGetSymbolAddress(&addr[1][dev], HIP_SYMBOL(g_mirror_chunk_count))) != hipSuccess ||
                    (e = hipGetSymbolAddress(&addr[2][dev], HIP_SYMBOL(g_mirror_chunk_base))) != hipSuccess) {
                    addr[0][dev] = nullptr;
                    return e;
                }
            }
        }
        g.lrank = static_cast<int*>(addr[0][dev]);
        g.chunk_count = static_cast<int*>(addr[1][dev]);
        g.chunk_base = static_cast<int*>(addr[2][dev]);
    }
    return launch_group(g, st);
}

hipError_t launch_group(const GroupArgs& g, hipStream_t st) {
    const int n_chunks = group_chunks(g.seq, g.top_k);
    // one workgroup for a single 1024-entry round (or without the multi-kernel
    // scratch); measured slower than rank / scan / place from 6 rounds on
    if (n_chunks <= 1 || !g.lrank) {
        launch_k(group_kernel, dim3(1), dim3(kGroupThreads), 0, st, g);
        return hipGetLastError();
    }
    if (g.slot_tok && g.assign_token) return hipErrorInvalidValue;  // bases are slots or positions, not both
    // checked before the first launch, so an oversized call enqueues nothing
    const size_t lds = (size_t)n_chunks * g.n_experts * sizeof(int);
    if (lds > kGroupScanLds) return hipErrorInvalidValue;
    launch_k(group_rank_kernel, dim3(n_chunks), dim3(kGroupThreads), 0, st, g);
    if (n_chunks <= kGroupFusedMaxChunks) {
        launch_k(group_scan_place_kernel, dim3(n_chunks), dim3(kGroupThreads), lds, st, g, n_chunks);
        return hipGetLastError();
    }
    static hipError_t attr = hipFuncSetAttribute((const void*)group_scan_kernel,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, kGroupScanLds);
    if (attr != hipSuccess) return attr;
    launch_k(group_scan_kernel, dim3(1), dim3(kGroupThreads), lds, st, g, n_chunks);
    const int n = g.seq * g.top_k;
    launch_k(group_place_kernel, dim3((n + 255) / 256), dim3(256), 0, st, g);
    return hipGetLastError();
}

}  // namespace uocr_hip
