// Decode-sized MoE layer (seq < 256): router, expert passes and combine with
// no grouping kernel and no cross-workgroup synchronisation.
//
// The reference routes a decode batch on the host and re-reads every weight row
// once per assigned token (src/engine/gpu_decoder.cu:591-609,
// src/kernels/cuda/moe_device.cu:199-268). Here:
//   * router_decode_kernel gives every token its own workgroup (lane e of wave 0
//     = expert e), so the reference's sequential fmaf chain per (token, expert)
//     runs on T different CUs at once; the f32 router matrix streams through an
//     LDS ring filled by all four waves;
//   * the expert kernels are launched over (expert, 64-row block) for every
//     expert. Each workgroup reads the routing ids (T*top_k ints) and derives
//     its expert's token list and slot base itself -- the stable grouping of
//     gpu_decoder.cu:602-609 (tokens ascending) -- so no grouping pass or tile
//     list sits between the router and the weight stream. An expert with no
//     tokens exits before loading anything; a live one loads its 64 weight rows
//     into registers ONCE and applies them to all of its 16-token m-tiles;
//   * the down pass writes y by entry ((t, j) at t*top_k + j, shared group v at
//     T*top_k + v*T + t), so the combine needs no routing lookups.
// act slot layout: shared-expert ("virtual") groups first, slot v*T + t, then
// the routed groups in expert order, slot n_virtual*T + offset(e) + rank.
#include "decode_common.hpp"

#include <algorithm>

namespace uocr_hip {

// Ring of four 32 KiB chunks for the stand-alone router kernel
constexpr int kRRing = 4;

template <typename XT, bool RMS>
__global__ __launch_bounds__(256) void router_decode_kernel(DecodeArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char rsmem[];
    router_token<XT, RMS, kRRing>(a, blockIdx.x, rsmem);
}

// ---------------------------------------------------------------------------
// Expert pass. Workgroup = (expert or virtual group, 64 output rows = 4 waves
// x 16 rows); weights in the tile-16x128 layout (common.hpp), held in
// registers across the expert's m-tiles.
// ---------------------------------------------------------------------------
constexpr int kDecBM = 16;
constexpr int kDecodeMaxEntries = 256 * kMaxTopK;  // seq < 256

template <int GPT, int KT, bool GU, bool ZP>
// three workgroups per CU (the routing ids are read from global memory, not
// staged, so the LDS fits three), except the gate/up pass at g32 or with zero
// points, which would spill at the register budget of three
__global__ __launch_bounds__(256, (GU && (GPT == 4 || ZP)) ? 2 : 3) void expert_decode_kernel(DecodeArgs a) {
    constexpr int K = KT * kTileK;
    constexpr int NG = scale_row_stride(K, kTileK / GPT);
    constexpr int SROW = kTileRows * NG;
    constexpr int NM = GU ? 2 : 1;  // weight matrices per item
    __shared__ __attribute__((aligned(16))) f16 As[KT * 4 * 64 * 8];
    // per wave: the scale rows of its NM matrices, then (ZP) their zero-offset rows
    __shared__ __attribute__((aligned(16))) f16 Ss[4][ZP ? 2 * NM : NM][SROW];
    constexpr int ZOFF = NM * SROW * 2;  // bytes from a scale row to its zero-offset row
    __shared__ int ent[256];
    __shared__ int hist[kMaxExperts], offs[kMaxExperts], live[kMaxExperts];
    __shared__ int n_live_s;
    __shared__ int ipre[kMaxExperts + 1];  // first item of live group i
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int T = a.seq, E = a.n_experts, N = T * a.top_k;
    const int n_rows = GU ? a.inter : a.hidden;
    const int RBG = (n_rows / kTileRows + 3) / 4;  // 64-row groups per expert

    // Routing summary, identical in every workgroup: per-expert counts, slot
    // offsets (stable grouping, experts ascending) and the list of live groups
    // (the shared-expert groups first -- every token, so the longest items --
    // then the routed experts with tokens).
    for (int e = tid; e < kMaxExperts; e += 256) hist[e] = 0;
    __syncthreads();
    // the ids of a 1024-entry chunk are all requested before the first use
    // (one L2 round trip per chunk, not per 256 entries)
    for (int i0 = 0; i0 < N; i0 += 1024) {
        int v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = i0 + tid + 256 * u < N ? a.ids[i0 + tid + 256 * u] : -1;
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (v[u] >= 0) atomicAdd(&hist[v[u]], 1);
    }
    __syncthreads();
    if (wave == 0) {
        int run_off = 0, run_live = a.n_virtual;
        for (int v = lane; v < a.n_virtual; v += 64) live[v] = E + v;
        for (int e0 = 0; e0 < E; e0 += 64) {
            const int e = e0 + lane;
            const int c = e < E ? hist[e] : 0;
            int inc = c;  // inclusive scan of counts over the wave
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int u = __shfl_up(inc, o, kWave);
                if (lane >= o) inc += u;
            }
            if (e < E) offs[e] = run_off + inc - c;
            run_off += __shfl(inc, 63, kWave);
            const uint64_t m = __ballot(c > 0);
            if (c > 0) live[run_live + __popcll(m & ((1ull << lane) - 1))] = e;
            run_live += __popcll(m);
        }
        if (lane == 0) n_live_s = run_live;
        // items per live group: RBG row blocks x its 16-token tiles
        int run_it = 0;
        for (int i0 = 0; i0 < run_live; i0 += 64) {
            const int i = i0 + lane;
            int n = 0;
            if (i < run_live) {
                const int g = live[i];
                const int c = g < E ? hist[g] : T;
                n = RBG * ((c + kDecBM - 1) / kDecBM);
            }
            int inc = n;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int u = __shfl_up(inc, o, kWave);
                if (lane >= o) inc += u;
            }
            if (i < run_live) ipre[i] = run_it + inc - n;
            run_it += __shfl(inc, 63, kWave);
        }
        if (lane == 0) ipre[run_live] = run_it;
    }
    __syncthreads();
    const int n_items = ipre[n_live_s];
    // Up to 512 routed entries: every wave keeps the ids in registers (lane l,
    // register u: entry 64u + l), read once here -- an item's entry list then
    // needs no global load, whose round trip would queue behind the weight
    // stream of the other workgroups (measured at 3-4 us per item).
    constexpr int kIdRegs = 8;
    const bool ids_in_regs = N <= 64 * kIdRegs;
    int idr[kIdRegs];
#pragma unroll
    for (int u = 0; u < kIdRegs; ++u) idr[u] = ids_in_regs && 64 * u + lane < N ? a.ids[64 * u + lane] : -1;

    const int r = lane & 15;
    const uint8_t* wsrc0 = GU ? a.gate : a.down;
    const uint16_t* ssrc0 = GU ? a.gate_s : a.down_s;
    const uint16_t* zsrc0 = GU ? a.gate_z : a.down_z;
    const long long wstr = GU ? a.gu_wstride : a.dn_wstride;
    const long long sstr = GU ? a.gu_sstride : a.dn_sstride;

    // work items (live group, 64-row block): grid-strided, so experts without
    // tokens never occupy a workgroup slot
    // one 16-token tile of one 64-row block per item, so groups with many
    // tokens (the shared ones see every token) spread over workgroups instead
    // of serialising their tiles
    for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
        int gi = 0;  // live group holding the item: ipre[gi] <= item < ipre[gi + 1]
        for (int i0 = 0; i0 < n_live_s; i0 += 64) {
            const int i = i0 + lane;
            gi += __popcll(__ballot(i < n_live_s && i > 0 && ipre[i] <= item));
        }
        const int g = live[gi];
        const int local = item - ipre[gi];
        const int m_item = (local / RBG) * kDecBM;
        const int rb = (local % RBG) * 4 + wave;
        const bool wave_live = rb * kTileRows < n_rows;
        const int cnt = g < E ? hist[g] : T;
        const int slot_base = g < E ? a.n_virtual * T + offs[g] : (g - E) * T;
        // the group's entries (t * top_k + j), ascending; every wave writes
        // the same values and reads back its own writes
        if (g < E) {
            const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
            int run = 0;
            // 512 entries per round: every id of the round is requested
            // before the first compare (one L2 round trip, not eight)
            for (int base = 0; base < N; base += 512) {
                int v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    v[u] = ids_in_regs ? idr[u] : (base + 64 * u + lane < N ? a.ids[base + 64 * u + lane] : -1);
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const bool hit = v[u] == g;
                    const uint64_t m = __ballot(hit);
                    if (hit) ent[run + __popcll(m & below)] = base + 64 * u + lane;
                    run += __popcll(m);
                }
            }
        } else {
            for (int i = lane; i < T; i += 64) ent[i] = i;
        }
        __builtin_amdgcn_wave_barrier();

        // A rows of an m-tile into LDS (fragments (kt, s = wave), row r = lane % 16)
        auto stage_a = [&](int m0) {
            const int rows = min(kDecBM, cnt - m0);
            if (r < rows) {
                // gate/up: x16 row of the entry's token; down: the slot's act row
                const int row = GU ? (g < E ? ent[m0 + r] / a.top_k : ent[m0 + r]) : slot_base + m0 + r;
                const f16* src = (GU ? a.x16 : a.act) + (size_t)row * K + wave * 32 + 8 * (lane >> 4);
#pragma unroll
                for (int kt = 0; kt < KT; ++kt) load_lds16(src + kt * kTileK, As + (size_t)(kt * 4 + wave) * 64 * 8);
            }
        };
        stage_a(m_item);

        // this wave's scale rows (LDS) and 16 x K weights (registers); no
        // branch around the weight loads (a wave past the last row block
        // reloads the last one and discards it), so the compiler tracks them
        // in issue order and waits k-tile by k-tile
        u32x4 bw0[KT], bw1[KT];
        {
            const int rbl = min(rb, n_rows / kTileRows - 1);
            const size_t sb = (size_t)g * sstr + (size_t)rbl * SROW;
            for (int i = lane; i * 8 < SROW; i += 64) {
                load_lds16(ssrc0 + sb + i * 8, &Ss[wave][0][(i & ~63) * 8]);
                if constexpr (GU) load_lds16(a.up_s + sb + i * 8, &Ss[wave][GU ? 1 : 0][(i & ~63) * 8]);
                if constexpr (ZP) {
                    load_lds16(zsrc0 + sb + i * 8, &Ss[wave][NM][(i & ~63) * 8]);
                    if constexpr (GU) load_lds16(a.up_z + sb + i * 8, &Ss[wave][NM + 1][(i & ~63) * 8]);
                }
            }
            const size_t toff = (size_t)g * wstr + (size_t)rbl * KT * kTileBytes + (size_t)lane * 16;
#pragma unroll
            for (int kt = 0; kt < KT; ++kt) {
                bw0[kt] = *reinterpret_cast<const u32x4*>(wsrc0 + toff + (size_t)kt * kTileBytes);
                if constexpr (GU) bw1[kt] = *reinterpret_cast<const u32x4*>(a.up + toff + (size_t)kt * kTileBytes);
            }
        }

        const f16* srow0 = &Ss[wave][0][r * NG];
        const f16* srow1 = &Ss[wave][GU ? 1 : 0][r * NG];
        const int col = rb * kTileRows + r;
        // one m-tile: MFMAs over all k-tiles and the stores
        auto tile = [&](int m0) {
            if (!wave_live) return;
            const int rows = min(kDecBM, cnt - m0);
            f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
            const uint32_t a_base = lds_addr(As + (size_t)lane * 8);
            const uint32_t s_base0 = lds_addr(srow0), s_base1 = lds_addr(srow1);
            TileRegs<GPT> tr[2];
            lds_issue_tile<GPT, ZP, ZOFF>(a_base, s_base0, s_base1, tr[0]);
#pragma unroll
            for (int kt = 0; kt < KT; ++kt) {
                f16 s0[4], s1[4], z0[4], z1[4];
                // this k-tile's LDS operands were issued one k-tile ahead; issue
                // the next k-tile's before waiting for these
                if (kt + 1 < KT) {
                    lds_issue_tile<GPT, ZP, ZOFF>(a_base + (uint32_t)((kt + 1) * 4096),
                                                  s_base0 + (uint32_t)((kt + 1) * GPT * 2),
                                                  s_base1 + (uint32_t)((kt + 1) * GPT * 2), tr[(kt + 1) & 1]);
                    lds_wait_tile<GPT, tile_reads<ZP>(), ZP>(tr[kt & 1], s0, s1, z0, z1);
                } else {
                    lds_wait_tile<GPT, 0, ZP>(tr[kt & 1], s0, s1, z0, z1);
                }
                const f16x8* av = tr[kt & 1].av;
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    if constexpr (ZP) {
                        acc0 = mfma16(av[s], dequant8z(bw0[kt][s], scale2(s0[s]), z0[s]), acc0);
                        if constexpr (GU) acc1 = mfma16(av[s], dequant8z(bw1[kt][s], scale2(s1[s]), z1[s]), acc1);
                    } else {
                        acc0 = mfma16(av[s], dequant8(bw0[kt][s], scale2(s0[s])), acc0);
                        if constexpr (GU) acc1 = mfma16(av[s], dequant8(bw1[kt][s], scale2(s1[s])), acc1);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 4 * (lane >> 4) + i;
                if (m < rows) {
                    if constexpr (GU) {
                        const float v = silu_mul_f(acc0[i], acc1[i]);
                        report_f16_overflow(a.status, f16_overflow(v));
                        a.act[(size_t)(slot_base + m0 + m) * n_rows + col] = (f16)v;
                    } else {
                        // y is indexed by entry: routed (t, j) at t*top_k + j,
                        // shared group v's token t at N + v*T + t
                        const int yrow = g < E ? ent[m0 + m] : N + slot_base + m0 + m;
                        a.y[(size_t)yrow * n_rows + col] = acc0[i];
                    }
                }
            }
        };
        // first m-tile: the A rows and scales (issued before the weights) are
        // waited for here, the weights k-tile by k-tile inside tile(), so the
        // dequant and MFMAs of early k-tiles overlap the arrival of later ones
        wait_vm_n(NM * KT);
        lds_barrier();
        tile(m_item);
        __syncthreads();  // As / Ss / ent are reused by the next item
    }
}

// ---------------------------------------------------------------------------
// Combine: out[t] = residual[t] + (sum_j fma(w[t,j], y[t*K + j]) in j order)
// + sum_v y[N + v*T + t]   (src/engine/moe_decoder.cpp:88-97,110-112,179)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void combine_decode_kernel(DecodeArgs a) {
    const int t = blockIdx.x, tid = threadIdx.x;
    const int T = a.seq, K = a.top_k, N = T * K, H = a.hidden;
    float wt[kMaxTopK];
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) wt[j] = j < K ? a.wts[(size_t)t * K + j] : 0.0f;
    const float* res = a.rms_weight ? static_cast<const float*>(a.x) + (size_t)t * H : nullptr;
    // one 16-byte column group per thread (the launch covers the row in one
    // pass); every row this thread needs is requested before the first FMA
    // (indices clamped, so no load sits behind a branch)
    for (int c = tid * 4; c < H; c += blockDim.x * 4) {
        f32x4 yv[kMaxTopK], ys[2];
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j)
            yv[j] = *reinterpret_cast<const f32x4*>(a.y + ((size_t)t * K + min(j, K - 1)) * H + c);
        // shared rows exist only with a shared MLP (y holds N + n_virtual*T rows)
        if (a.n_virtual > 0) {
#pragma unroll
            for (int v = 0; v < 2; ++v)
                ys[v] = *reinterpret_cast<const f32x4*>(a.y + ((size_t)N + (size_t)min(v, a.n_virtual - 1) * T + t) * H + c);
        }
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j)
            if (j < K)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] = fmaf(wt[j], yv[j][i], acc[i]);
        if (a.n_virtual > 0) {
            f32x4 sh = ys[0];
            for (int v = 1; v < a.n_virtual; ++v) {
                const f32x4 y2 = v < 2 ? ys[1] : *reinterpret_cast<const f32x4*>(a.y + ((size_t)N + (size_t)v * T + t) * H + c);
#pragma unroll
                for (int i = 0; i < 4; ++i) sh[i] += y2[i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += sh[i];
        }
        if (a.shared_y) {
            const f32x4 sv = *reinterpret_cast<const f32x4*>(a.shared_y + (size_t)t * H + c);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += sv[i];
        }
        if (res) {
            const f32x4 rv = *reinterpret_cast<const f32x4*>(res + c);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = rv[i] + acc[i];
        }
        *reinterpret_cast<f32x4*>(a.out + (size_t)t * H + c) = acc;
    }
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
template <int GPT, int KT, bool GU, bool ZP>
static void launch_expert(const DecodeArgs& a, int n_groups, int n_rows, hipStream_t st) {
    // one generation of resident workgroups (work items are grid-strided);
    // never more workgroups than the worst-case item count
    static int resident = [] {
        int dev = 0, cus = 0, per_cu = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, expert_decode_kernel<GPT, KT, GU, ZP>, 256, 0);
        return std::max(1, cus * std::max(1, per_cu));
    }();
    const int max_items = n_groups * ((n_rows / kTileRows + 3) / 4);
    launch_k((expert_decode_kernel<GPT, KT, GU, ZP>), dim3(std::min(resident, max_items)), dim3(256), 0, st, a);
}

template <bool GU, int GPT, bool ZP>
static hipError_t launch_expert_kt(const DecodeArgs& a, hipStream_t st) {
    const int K = GU ? a.hidden : a.inter;
    const int n_rows = GU ? a.inter : a.hidden;
    const int ng = a.n_experts + a.n_virtual;
    switch (K / kTileK) {
        case 1: launch_expert<GPT, 1, GU, ZP>(a, ng, n_rows, st); break;
        case 2: launch_expert<GPT, 2, GU, ZP>(a, ng, n_rows, st); break;
        case 4: launch_expert<GPT, 4, GU, ZP>(a, ng, n_rows, st); break;
        case 7: launch_expert<GPT, 7, GU, ZP>(a, ng, n_rows, st); break;
        case 10: launch_expert<GPT, 10, GU, ZP>(a, ng, n_rows, st); break;
        case 14: launch_expert<GPT, 14, GU, ZP>(a, ng, n_rows, st); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <bool GU, int GPT>
static hipError_t launch_expert_z(const DecodeArgs& a, hipStream_t st) {
    return a.gate_z ? launch_expert_kt<GU, GPT, true>(a, st) : launch_expert_kt<GU, GPT, false>(a, st);
}

template <bool GU>
static hipError_t launch_expert_g(const DecodeArgs& a, hipStream_t st) {
    switch (a.group) {
        case 32: return launch_expert_z<GU, 4>(a, st);
        case 64: return launch_expert_z<GU, 2>(a, st);
        case 128: return launch_expert_z<GU, 1>(a, st);
        default: return hipErrorInvalidValue;
    }
}

bool decode_shapes_ok(int hidden, int inter) {
    auto ok = [](int k) {
        const int kt = k / kTileK;
        return k % kTileK == 0 && (kt == 1 || kt == 2 || kt == 4 || kt == 7 || kt == 10 || kt == 14);
    };
    return ok(hidden) && ok(inter) && hidden <= kMaxHidden;
}

template <typename XT, bool RMS>
static hipError_t launch_rd(const DecodeArgs& a, dim3 grid, size_t lds, hipStream_t st) {
    // > 64 KiB of dynamic LDS: raise the limit once per instantiation
    static hipError_t attr = hipFuncSetAttribute((const void*)router_decode_kernel<XT, RMS>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);
    if (attr != hipSuccess) return attr;
    launch_k((router_decode_kernel<XT, RMS>), grid, dim3(256), lds, st, a);
    return hipGetLastError();
}

hipError_t launch_router_decode(const DecodeArgs& a, hipStream_t st) {
    if (a.n_experts > 64 || a.hidden > kMaxHidden || a.hidden % 8) return hipErrorInvalidValue;
    if (a.hidden % kRChunkCols) return hipErrorInvalidValue;
    const dim3 grid(a.seq);
    const size_t lds = (size_t)kRRing * kRChunkBytes + (size_t)a.hidden * 8 + 128;
    const bool rms = a.rms_weight != nullptr;
    if (a.x_bf16) {
        if (rms) return launch_rd<uint16_t, true>(a, grid, lds, st);
        return launch_rd<uint16_t, false>(a, grid, lds, st);
    }
    if (rms) return launch_rd<float, true>(a, grid, lds, st);
    return launch_rd<float, false>(a, grid, lds, st);
}

hipError_t launch_experts_decode2(const DecodeArgs& a, bool gate_up, hipStream_t st) {
    if (a.seq * a.top_k > 0x7fffffff / 2 || a.seq > 256) return hipErrorInvalidValue;
    return gate_up ? launch_expert_g<true>(a, st) : launch_expert_g<false>(a, st);
}

hipError_t launch_combine_decode(const DecodeArgs& a, hipStream_t st) {
    const int threads = std::min(1024, ((a.hidden / 4 + 63) / 64) * 64);
    launch_k(combine_decode_kernel, dim3(a.seq), dim3(threads), 0, st, a);
    return hipGetLastError();
}

}  // namespace uocr_hip
