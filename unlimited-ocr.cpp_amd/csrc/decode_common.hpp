// Device helpers shared by the decode kernels (decode_path.hip) and the fused
// decode-layer kernel (decode_fused.hip): operand loads, explicit memory-counter
// waits, the asm LDS reads of one MFMA k-tile, and the per-token router body.
#pragma once
#include "launch.hpp"
#include "routing.hpp"

#include <type_traits>

namespace uocr_hip {


// ---------------------------------------------------------------------------
// routing helpers shared with the router kernels
// ---------------------------------------------------------------------------

// ---------------------------------------------------------------------------
// Router: one token per workgroup of one wave.
// ---------------------------------------------------------------------------
constexpr int kMaxHidden = 1792;

template <typename XT>
__device__ __forceinline__ void load8(const XT* p, float* out);
template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t* p, float* out) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[2 * i] = __uint_as_float(v[i] << 16);
        out[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
    }
}
template <>
__device__ __forceinline__ void load8<float>(const float* p, float* out) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
    const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[i] = a[i];
        out[4 + i] = b[i];
    }
}

// The router matrix streams through an LDS ring of 16 KiB chunks (64 columns x
// 64 experts x f32, [H/4][64][4] in HBM) filled by direct global->LDS loads
// from all four waves; wave 0 runs the 64 FMA chains out of LDS. Eight chunks
// (512 columns) are in flight at a time.
constexpr int kRChunkCols = 128;
constexpr int kRChunkBytes = kRChunkCols * 64 * 4;  // 32 KiB
constexpr int kRChunkLoads = kRChunkBytes / 1024;   // 1 KiB per wave load
// DMA loads per chunk issued by producer wave w (1..3): units w-1, w+2, ...
__host__ __device__ constexpr int router_loads_of(int wave) { return (kRChunkLoads - (wave - 1) + 2) / 3; }

// s_waitcnt vmcnt(n) (n <= 63), leaving expcnt / lgkmcnt unconstrained
template <int N>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
// s_waitcnt vmcnt(n) for a wave-uniform runtime n (values above 63 wait for 0)
__device__ __forceinline__ void wait_vm_n(int n) {
    switch (n) {
#define UOCR_VM(k) case k: wait_vm<k>(); break;
#define UOCR_VM8(b) UOCR_VM(b) UOCR_VM(b + 1) UOCR_VM(b + 2) UOCR_VM(b + 3) UOCR_VM(b + 4) UOCR_VM(b + 5) UOCR_VM(b + 6) UOCR_VM(b + 7)
        UOCR_VM8(1) UOCR_VM8(9) UOCR_VM8(17) UOCR_VM8(25) UOCR_VM8(33) UOCR_VM8(41) UOCR_VM8(49)
        UOCR_VM(57) UOCR_VM(58) UOCR_VM(59) UOCR_VM(60) UOCR_VM(61) UOCR_VM(62) UOCR_VM(63)
#undef UOCR_VM8
#undef UOCR_VM
        default: wait_vm<0>(); break;
    }
}

template <int RING>
__device__ __forceinline__ void router_issue_chunk(const float* w, int chunk, unsigned char* ring, int wave, int lane) {
    const unsigned char* src = reinterpret_cast<const unsigned char*>(w) + (size_t)chunk * kRChunkBytes;
    unsigned char* dst = ring + (size_t)(chunk % RING) * kRChunkBytes;
    for (int unit = wave - 1; unit < kRChunkLoads; unit += 3)  // 1 KiB per wave instruction
        load_lds16(src + ((size_t)unit * 64 + lane) * 16, dst + (size_t)unit * 1024);
}


// LDS operands of one k-tile: four A fragments (1 KiB apart) and the scale
// words of one or two scale rows (the GPT groups of the k-tile; MFMA step s
// uses group (s * GPT) / 4), plus, with ZP, the zero-offset words of the same
// rows ZOFF bytes after the scales. lds_issue_tile only issues the reads (the
// registers must not be used before lds_wait_tile); reading through asm keeps
// the compiler's LDS-DMA tracking from turning the first read into a wait for
// every outstanding global load.
template <int GPT>
struct TileRegs {
    f16x8 av[4];
    // GPT 4: four scales in 64 bits; GPT 2 / 1: two / one in 32 bits
    typedef typename std::conditional<GPT == 4, uint64_t, uint32_t>::type SW;
    SW w0, w1, z0, z1;
};
// LDS reads lds_issue_tile issues
template <bool ZP>
constexpr int tile_reads() { return ZP ? 8 : 6; }

template <int GPT, bool ZP = false, int ZOFF = 0>
__device__ __forceinline__ void lds_issue_tile(uint32_t a_addr, uint32_t s0_addr, uint32_t s1_addr, TileRegs<GPT>& t) {
#define UOCR_TILE_READS(SREAD)                                                                        \
    asm volatile("ds_read_b128 %0, %6\n"                                                             \
                 "ds_read_b128 %1, %6 offset:1024\n"                                                 \
                 "ds_read_b128 %2, %6 offset:2048\n"                                                 \
                 "ds_read_b128 %3, %6 offset:3072\n" SREAD " %4, %7\n" SREAD " %5, %8\n"             \
                 : "=&v"(t.av[0]), "=&v"(t.av[1]), "=&v"(t.av[2]), "=&v"(t.av[3]), "=&v"(t.w0), "=&v"(t.w1) \
                 : "v"(a_addr), "v"(s0_addr), "v"(s1_addr)                                          \
                 : "memory")
#define UOCR_ZERO_READS(SREAD)                                                                        \
    asm volatile(SREAD " %0, %2 offset:%4\n" SREAD " %1, %3 offset:%4\n"                              \
                 : "=&v"(t.z0), "=&v"(t.z1)                                                         \
                 : "v"(s0_addr), "v"(s1_addr), "n"(ZOFF)                                            \
                 : "memory")
    if constexpr (GPT == 4) {
        UOCR_TILE_READS("ds_read_b64");
        if constexpr (ZP) UOCR_ZERO_READS("ds_read_b64");
    } else if constexpr (GPT == 2) {
        UOCR_TILE_READS("ds_read_b32");
        if constexpr (ZP) UOCR_ZERO_READS("ds_read_b32");
    } else {
        UOCR_TILE_READS("ds_read_u16");
        if constexpr (ZP) UOCR_ZERO_READS("ds_read_u16");
    }
#undef UOCR_TILE_READS
#undef UOCR_ZERO_READS
}

template <int GPT>
__device__ __forceinline__ void unpack_tile_words(uint64_t x0, uint64_t x1, f16* s0, f16* s1) {
    const uint32_t w0[2] = {(uint32_t)x0, (uint32_t)(x0 >> 32)};
    const uint32_t w1[2] = {(uint32_t)x1, (uint32_t)(x1 >> 32)};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int gi = (s * GPT) >> 2;  // group within the k-tile
        s0[s] = __builtin_bit_cast(f16, (uint16_t)((w0[gi >> 1] >> (16 * (gi & 1))) & 0xffffu));
        s1[s] = __builtin_bit_cast(f16, (uint16_t)((w1[gi >> 1] >> (16 * (gi & 1))) & 0xffffu));
    }
}

// Wait until at most `later` LDS reads (issued after this tile's) are
// outstanding, then unpack the scales (and, with ZP, the zero offsets).
template <int GPT, int LATER, bool ZP = false>
__device__ __forceinline__ void lds_wait_tile(TileRegs<GPT>& t, f16* s0, f16* s1, f16* z0 = nullptr,
                                              f16* z1 = nullptr) {
    if constexpr (ZP) {
        asm volatile("s_waitcnt lgkmcnt(%8)"
                     : "+v"(t.av[0]), "+v"(t.av[1]), "+v"(t.av[2]), "+v"(t.av[3]), "+v"(t.w0), "+v"(t.w1), "+v"(t.z0),
                       "+v"(t.z1)
                     : "n"(LATER));
        unpack_tile_words<GPT>(t.z0, t.z1, z0, z1);
    } else {
        asm volatile("s_waitcnt lgkmcnt(%6)"
                     : "+v"(t.av[0]), "+v"(t.av[1]), "+v"(t.av[2]), "+v"(t.av[3]), "+v"(t.w0), "+v"(t.w1)
                     : "n"(LATER));
    }
    unpack_tile_words<GPT>(t.w0, t.w1, s0, s1);
}

// Workgroup barrier that orders LDS only: __syncthreads() would also wait for
// every outstanding global load (vmcnt(0)), draining the ring.
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt unconstrained
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Bias seeds of the staged A rows (As, the MFMA fragment layout: region
// kt*4 + s holds k = kt*128 + s*32 .. +32, lane t + 16c the eight k from 8c of
// token t): for scale group g of the item and token t, Cs[g][t] =
// -(1032 * sum of A at the positions that dequant8_biased biases by 1024 +
// 72 * sum at the positions biased by 64), summed with v_dot2_f32_f16.
template <int KT, int GPT, int NT = 256>
__device__ __forceinline__ void bias_seeds(const f16* As, float* Cs, int tid) {
    constexpr int NGI = KT * GPT;
    const f16x2 one = {(f16)1.0f, (f16)1.0f};
    for (int p = tid; p < NGI * 16; p += NT) {
        const int g = p >> 4, t = p & 15, kt = g / GPT, gi = g % GPT;
        float xe = 0.0f, xo = 0.0f;
#pragma unroll
        for (int s = gi * 4 / GPT; s < (gi + 1) * 4 / GPT; ++s)
            {
                // asm reads: a plain LDS read after the DMA staging would wait
                // for every outstanding global load (the weights in flight)
                u32x4 v[4];
                asm volatile("ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:256\n\t"
                             "ds_read_b128 %2, %4 offset:512\n\tds_read_b128 %3, %4 offset:768\n\t"
                             "s_waitcnt lgkmcnt(0)"
                             : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
                             : "v"(lds_addr(As + ((size_t)(kt * 4 + s) * 64 + t) * 8))
                             : "memory");
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    xe = __builtin_amdgcn_fdot2(as_h2(v[c][0]), one, xe, false);
                    xo = __builtin_amdgcn_fdot2(as_h2(v[c][1]), one, xo, false);
                    xe = __builtin_amdgcn_fdot2(as_h2(v[c][2]), one, xe, false);
                    xo = __builtin_amdgcn_fdot2(as_h2(v[c][3]), one, xo, false);
                }
            }
        Cs[p] = -(1032.0f * xe + 72.0f * xo);
    }
}

// The seeds of the GPT groups of one k-tile for this lane's four tokens
template <int GPT>
__device__ __forceinline__ void lds_issue_seeds(uint32_t c_addr, f32x4 (&c)[GPT]) {
    if constexpr (GPT == 4) {
        asm volatile("ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:64\n\t"
                     "ds_read_b128 %2, %4 offset:128\n\tds_read_b128 %3, %4 offset:192"
                     : "=&v"(c[0]), "=&v"(c[1]), "=&v"(c[2]), "=&v"(c[3]) : "v"(c_addr) : "memory");
    } else if constexpr (GPT == 2) {
        asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:64"
                     : "=&v"(c[0]), "=&v"(c[1]) : "v"(c_addr) : "memory");
    } else {
        asm volatile("ds_read_b128 %0, %1" : "=&v"(c[0]) : "v"(c_addr) : "memory");
    }
}

// One wave's 16 rows x KT k-tiles (two weight tiles sharing the A rows, or
// one: TWO = false) against the staged A rows. Per scale group the MFMAs run
// on the biased nibbles from the group's bias seed (ZP: on the exact integers
// q - zero from a zero seed), then the group result is scaled into the
// accumulator (f16 scale x f32, one fma per element). LDS operands are read
// one k-tile ahead (asm reads, explicit lgkmcnt waits). ZOFF: bytes from a
// scale row to its zero-offset row.
struct NoHook {
    __device__ __forceinline__ void operator()(int) const {}
};
// hook(kt) runs once the MFMAs of k-tile kt are issued (its weight registers
// are then free: a caller may load the next item's tile kt into them)
// item_mma_f: the weight words of k-tile kt come from w0(kt) / w1(kt); ZC:
// every zero point is 8 (symmetric layer) and the MFMAs run on the exact
// integers q - 8 from a zero seed, with neither bias seeds nor zero-offset
// rows (c_base unused)
// PF: the LDS operands of k-tile kt + 1 are read while k-tile kt computes
// (else each k-tile's are read and waited for in turn: fewer registers)
template <int GPT, int KT, bool TWO, bool ZP, int ZOFF, bool ZC, bool PF, typename W0, typename W1, typename Hook>
__device__ __forceinline__ void item_mma_f(W0 w0, W1 w1, uint32_t a_base, uint32_t s_base0, uint32_t s_base1,
                                           uint32_t c_base, f32x4& acc0, f32x4& acc1, Hook hook);
template <int GPT, int KT, bool TWO = true, bool ZP = false, int ZOFF = 0, typename Hook = NoHook>
__device__ __forceinline__ void item_mma(const u32x4 (&bw0)[KT], const u32x4 (&bw1)[KT], uint32_t a_base,
                                         uint32_t s_base0, uint32_t s_base1, uint32_t c_base, f32x4& acc0,
                                         f32x4& acc1, Hook hook = Hook()) {
    item_mma_f<GPT, KT, TWO, ZP, ZOFF, false, true>([&](int kt) -> const u32x4& { return bw0[kt]; },
                                       [&](int kt) -> const u32x4& { return bw1[kt]; }, a_base, s_base0, s_base1,
                                       c_base, acc0, acc1, hook);
}
template <int GPT, int KT, bool TWO, bool ZP, int ZOFF, bool ZC, bool PF, typename W0, typename W1, typename Hook>
__device__ __forceinline__ void item_mma_f(W0 w0, W1 w1, uint32_t a_base, uint32_t s_base0, uint32_t s_base1,
                                           uint32_t c_base, f32x4& acc0, f32x4& acc1, Hook hook) {
    static_assert(!(ZP && ZC), "one zero-point form");
    constexpr bool SEEDS = !ZP && !ZC;
    constexpr int NSEED = SEEDS ? GPT : 0;  // seed reads per k-tile
    TileRegs<GPT> tr[2];
    f32x4 cr[2][GPT];
    lds_issue_tile<GPT, ZP, ZOFF>(a_base, s_base0, s_base1, tr[0]);
    if constexpr (SEEDS) lds_issue_seeds<GPT>(c_base, cr[0]);
    // the previous group's results, scaled in after the next group's MFMAs
    // are issued (the MFMA latency is then covered)
    f32x4 p0 = {0.f, 0.f, 0.f, 0.f}, p1 = {0.f, 0.f, 0.f, 0.f};
    float ps0 = 0.0f, ps1 = 0.0f;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
        f16 s0[4], s1[4], z0[4], z1[4];
        if constexpr (!PF) {
            if (kt > 0) {
                lds_issue_tile<GPT, ZP, ZOFF>(a_base + (uint32_t)(kt * 4096), s_base0 + (uint32_t)(kt * GPT * 2),
                                              s_base1 + (uint32_t)(kt * GPT * 2), tr[0]);
                if constexpr (SEEDS) lds_issue_seeds<GPT>(c_base + (uint32_t)(kt * GPT * 64), cr[0]);
            }
            lds_wait_tile<GPT, 0, ZP>(tr[0], s0, s1, z0, z1);
        } else if (kt + 1 < KT) {
            lds_issue_tile<GPT, ZP, ZOFF>(a_base + (uint32_t)((kt + 1) * 4096), s_base0 + (uint32_t)((kt + 1) * GPT * 2),
                                          s_base1 + (uint32_t)((kt + 1) * GPT * 2), tr[(kt + 1) & 1]);
            if constexpr (SEEDS) lds_issue_seeds<GPT>(c_base + (uint32_t)((kt + 1) * GPT * 64), cr[(kt + 1) & 1]);
            lds_wait_tile<GPT, tile_reads<ZP>() + NSEED, ZP>(tr[kt & 1], s0, s1, z0, z1);
        } else {
            lds_wait_tile<GPT, 0, ZP>(tr[kt & 1], s0, s1, z0, z1);
        }
        constexpr int B = PF ? 1 : 0;  // buffer mask
        if constexpr (SEEDS) {
#pragma unroll
            for (int gi = 0; gi < GPT; ++gi) asm volatile("" : "+v"(cr[kt & B][gi]));  // landed with the tile
        }
        const f16x8* av = tr[kt & B].av;
#pragma unroll
        for (int gi = 0; gi < GPT; ++gi) {
            f32x4 r0, r1;
            if constexpr (!SEEDS) {
                r0 = f32x4{0.f, 0.f, 0.f, 0.f};
                r1 = r0;
            } else {
                r0 = cr[kt & B][gi];
                r1 = r0;
            }
#pragma unroll
            for (int s = gi * 4 / GPT; s < (gi + 1) * 4 / GPT; ++s) {
                if constexpr (ZP) {
                    r0 = mfma16(av[s], dequant8z_unscaled(w0(kt)[s], z0[s]), r0);
                    if constexpr (TWO) r1 = mfma16(av[s], dequant8z_unscaled(w1(kt)[s], z1[s]), r1);
                } else if constexpr (ZC) {
                    const f16 zo = (f16)-1032.0f;  // -(1024 + 8)
                    r0 = mfma16(av[s], dequant8z_unscaled(w0(kt)[s], zo), r0);
                    if constexpr (TWO) r1 = mfma16(av[s], dequant8z_unscaled(w1(kt)[s], zo), r1);
                } else {
                    r0 = mfma16(av[s], dequant8_biased(w0(kt)[s]), r0);
                    if constexpr (TWO) r1 = mfma16(av[s], dequant8_biased(w1(kt)[s]), r1);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc0[i] = fmaf(ps0, p0[i], acc0[i]);
                if constexpr (TWO) acc1[i] = fmaf(ps1, p1[i], acc1[i]);
            }
            asm volatile("" : "+v"(acc0), "+v"(acc1));  // scaled here, not deferred
            p0 = r0;
            p1 = r1;
            ps0 = (float)s0[gi * 4 / GPT];
            ps1 = (float)s1[gi * 4 / GPT];
        }
        hook(kt);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        acc0[i] = fmaf(ps0, p0[i], acc0[i]);
        if constexpr (TWO) acc1[i] = fmaf(ps1, p1[i], acc1[i]);
    }
}



// Scoring (src/kernels/cpu_ops.cpp:93-106 softmax, or sigmoid) and greedy
// top-k (src/engine/moe_decoder.cpp:264-287) of token t by ONE wave, lane e
// holding expert e's logit `acc`; sc (64 floats), topv (unused) and etab (the
// expf table) are LDS of the caller. The greedy scan (strict '>', so the lowest
// index wins a tie; the pick is then removed) is K rounds of a wave maximum and
// the lowest lane holding it. COHERENT: ids / weights are written with
// agent-scope stores that other workgroups read without a cache invalidation.
template <bool COHERENT>
__device__ __forceinline__ void router_select(const DecodeArgs& a, int t, float acc, float* sc, float* topv,
                                              const uint64_t* etab) {
    (void)topv;
    const int lane = threadIdx.x & 63;
    const int K = a.top_k;
    const WaveTopk pick = wave_topk(acc, a.n_experts, K, a.scoring_sigmoid, a.norm_topk_prob, a.scaling, sc, etab);
    const int rank = pick.rank;
    if (lane < K) {
        const float wj = pick.w;
        if constexpr (COHERENT) {
            __hip_atomic_store(a.wts + (size_t)t * K + lane, wj, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            a.wts[(size_t)t * K + lane] = wj;
        }
    }
    if (rank < K) {
        if constexpr (COHERENT) {
            __hip_atomic_store(a.ids + (size_t)t * K + rank, lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            a.ids[(size_t)t * K + rank] = lane;
        }
    }
}


// The sum of the rounded squares pq[0 .. H) in column order, by one lane
// (src/kernels/cpu_ops.cpp:58-67 as the reference build computes it; H is a
// multiple of 64 and pq has 64 readable floats past H). The LDS reads run one
// 32-column step ahead of the adds (asm reads with explicit waits: the
// compiler's schedule waited on every read).
__device__ __forceinline__ float rms_sum_chain(const float* pq, int H) {
    // 32 columns per step: eight 16-byte reads at immediate offsets,
    // the next step's issued before this step's adds (one instruction
    // per column beyond the add)
    uint32_t pb = lds_addr(pq);
    f32x4 cur[8], nxt[8];
    asm volatile("ds_read_b128 %0, %8\n\tds_read_b128 %1, %8 offset:16\n\t"
                 "ds_read_b128 %2, %8 offset:32\n\tds_read_b128 %3, %8 offset:48\n\t"
                 "ds_read_b128 %4, %8 offset:64\n\tds_read_b128 %5, %8 offset:80\n\t"
                 "ds_read_b128 %6, %8 offset:96\n\tds_read_b128 %7, %8 offset:112\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(cur[0]), "=&v"(cur[1]), "=&v"(cur[2]), "=&v"(cur[3]), "=&v"(cur[4]), "=&v"(cur[5]),
                   "=&v"(cur[6]), "=&v"(cur[7])
                 : "v"(pb)
                 : "memory");
    // Two 32-column steps per iteration with the two buffers swapping
    // roles (no register copies between the adds; H / 32 is even).
    auto read8 = [&](f32x4 (&d)[8], uint32_t p) {
        asm volatile("ds_read_b128 %0, %8\n\tds_read_b128 %1, %8 offset:16\n\t"
                     "ds_read_b128 %2, %8 offset:32\n\tds_read_b128 %3, %8 offset:48\n\t"
                     "ds_read_b128 %4, %8 offset:64\n\tds_read_b128 %5, %8 offset:80\n\t"
                     "ds_read_b128 %6, %8 offset:96\n\tds_read_b128 %7, %8 offset:112"
                     : "=&v"(d[0]), "=&v"(d[1]), "=&v"(d[2]), "=&v"(d[3]), "=&v"(d[4]), "=&v"(d[5]),
                       "=&v"(d[6]), "=&v"(d[7])
                     : "v"(p)
                     : "memory");
    };
    auto wait8 = [&](f32x4 (&d)[8], float& acc) {
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3]), "+v"(d[4]), "+v"(d[5]), "+v"(d[6]),
                       "+v"(d[7]), "+v"(acc));
    };
    float ss = 0.0f;
    for (int c = 0; c < H; c += 64) {
        read8(nxt, pb + 128u);  // the next step
#pragma unroll
        for (int k = 0; k < 8; ++k)
#pragma unroll
            for (int q = 0; q < 4; ++q) ss = __fadd_rn(ss, cur[k][q]);
        wait8(nxt, ss);
        read8(cur, pb + 256u);  // the step after (past the end: the pad, never added)
#pragma unroll
        for (int k = 0; k < 8; ++k)
#pragma unroll
            for (int q = 0; q < 4; ++q) ss = __fadd_rn(ss, nxt[k][q]);
        wait8(cur, ss);
        pb += 256u;
    }
    return ss;
}

// One token's routing by one 256-thread workgroup: rsmem = RING chunks of the
// router matrix, then the token row as f32 (H floats), then H + 32 floats of
// scratch for the RMSNorm. Waves 1..3 return after
// the logits; wave 0 scores, selects and writes ids / weights (and x16) --
// COHERENT: as agent-scope stores that other workgroups read without a cache
// invalidation.
template <typename XT, bool RMS, int RING, bool COHERENT = false>
__device__ __forceinline__ void router_token(const DecodeArgs& a, int t, unsigned char* rsmem) {
    unsigned char* ring = rsmem;
    float* xs = reinterpret_cast<float*>(rsmem + RING * kRChunkBytes);
    __shared__ __attribute__((aligned(16))) float sc[64];
    __shared__ float topv[kMaxTopK];
    __shared__ uint64_t etab[32];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int H = a.hidden;
    if (tid < 32) etab[tid] = uocr_exp2_tab[tid];
    const int NCH = H / kRChunkCols;
    const XT* x = static_cast<const XT*>(a.x) + (size_t)t * H;

    // waves 1..3 start the router-matrix ring; wave 0 loads the token row -> xs (f32)
    if (wave != 0) {
        for (int ch = 0; ch < RING && ch < NCH; ++ch) router_issue_chunk<RING>(a.router_f32, ch, ring, wave, lane);
    } else {
        for (int c = lane * 8; c < H; c += 64 * 8) {
            float v[8];
            load8<XT>(x + c, v);
            *reinterpret_cast<f32x4*>(xs + c) = f32x4{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<f32x4*>(xs + c + 4) = f32x4{v[4], v[5], v[6], v[7]};
        }
    }
    lds_barrier();  // xs

    if constexpr (RMS) {
        // src/kernels/cpu_ops.cpp:58-67 as the reference build computes it: the
        // products x*x rounded, summed in column order (the last H % 4 terms would
        // be fused; H is a multiple of 128 on this path)
        // The rounded products in parallel (LDS after the token row), then one
        // lane adds them in column order, its LDS reads one 32-column step
        // ahead of the adds (asm reads with explicit waits: the compiler's
        // schedule waited on every read). H is a multiple of 128 here.
        float* pq = xs + H;
        for (int c = tid; c < H; c += 256) pq[c] = __fmul_rn(xs[c], xs[c]);
        __syncthreads();
        if (tid == 0) {
            const float ss = rms_sum_chain(pq, H);
            sc[0] = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)H), a.rms_eps)));
        }
        __syncthreads();
        const float inv = sc[0];
        for (int c = tid; c < H; c += 256) xs[c] = __fmul_rn(__fmul_rn(xs[c], inv), a.rms_weight[c]);
        __syncthreads();
    }

    // f16 expert input (waves 1..3; wave 0 starts its chains)
    if (wave > 0)
        for (int c = (tid - 64) * 8; c < H; c += 192 * 8) {
            const f32x4 p = *reinterpret_cast<const f32x4*>(xs + c);
            const f32x4 q = *reinterpret_cast<const f32x4*>(xs + c + 4);
            const f16x8 h = {(f16)p[0], (f16)p[1], (f16)p[2], (f16)p[3], (f16)q[0], (f16)q[1], (f16)q[2], (f16)q[3]};
            *reinterpret_cast<f16x8*>(a.x16 + (size_t)t * H + c) = h;
        }

    // logits: lane e of wave 0 runs the reference's sequential chain, columns
    // ascending: fmaf steps for a bf16 router (matmul_t_bf16,
    // src/kernels/cpu_ops.cpp:26-39, contracted by the -march=native build),
    // acc + round(x * w) for an f32 router (matmul_t, cpu_ops.cpp:11-24, whose
    // build leaves the loop uncontracted; H % 4 == 0 here, so no fused tail). Waves 1..3 keep the ring filled; wave 0 only
    // computes.
    float acc = 0.0f;
    const int my_loads = wave == 0 ? 0 : router_loads_of(wave);
    for (int ch = 0; ch < NCH; ++ch) {
        // chunks this wave has issued so far: 0 .. last
        const int last = min(NCH - 1, max(RING - 1, ch - 2 + RING));
        if (wave != 0) wait_vm_n(my_loads * (last - ch));
        lds_barrier();
        if (wave != 0 && ch >= 1 && ch - 1 + RING < NCH)
            router_issue_chunk<RING>(a.router_f32, ch - 1 + RING, ring, wave, lane);
        if (wave == 0) {
            // 32 steps of 4 columns: the LDS reads run 6 steps (12 reads) ahead
            // of the FMA chain, with explicit lgkmcnt waits (the compiler's own
            // schedule waits for every read pair)
            const uint32_t w_addr = lds_addr(ring + (size_t)(ch % RING) * kRChunkBytes) + lane * 16;
            const uint32_t x_addr = lds_addr(xs + ch * kRChunkCols);
            if (a.router_unfused) {
                asm volatile(UOCR_RCHUNK(UOCR_RMAC_SEP)
                : [acc] "+v"(acc)
                : [w] "v"(w_addr), [x] "v"(x_addr)
                : "v64", "v65", "v66", "v67", "v68", "v69", "v70", "v71", "v72", "v73", "v74", "v75", "v76", "v77", "v78", "v79", "v80", "v81", "v82", "v83", "v84", "v85", "v86", "v87", "v88", "v89", "v90", "v91", "v92", "v93", "v94", "v95", "v96", "v97", "v98", "v99", "v100", "v101", "v102", "v103", "v104", "v105", "v106", "v107", "v108", "v109", "v110", "v111", "v112", "memory");
            } else {
                asm volatile(UOCR_RCHUNK(UOCR_RMAC_FMA)
                : [acc] "+v"(acc)
                : [w] "v"(w_addr), [x] "v"(x_addr)
                : "v64", "v65", "v66", "v67", "v68", "v69", "v70", "v71", "v72", "v73", "v74", "v75", "v76", "v77", "v78", "v79", "v80", "v81", "v82", "v83", "v84", "v85", "v86", "v87", "v88", "v89", "v90", "v91", "v92", "v93", "v94", "v95", "v96", "v97", "v98", "v99", "v100", "v101", "v102", "v103", "v104", "v105", "v106", "v107", "v108", "v109", "v110", "v111", "memory");
            }
        }
    }
    // scoring and top-k by wave 0 alone
    if (wave != 0) return;
    router_select<COHERENT>(a, t, acc, sc, topv, etab);
}


}  // namespace uocr_hip
