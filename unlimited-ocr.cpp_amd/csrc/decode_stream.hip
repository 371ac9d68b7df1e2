// Streamed decode layer: router, gate/up, down and combine in ONE persistent
// launch of one 8-wave workgroup per CU (two where the registers and LDS
// allow), organised so that the weight stream never waits on another
// workgroup. Two modes:
//   16-token mode (WIDE = false): up to kStreamMaxSeq tokens, bf16 or f32
//     input, no RMSNorm; every item covers all T tokens;
//   wide mode (WIDE = true): up to kStreamWideMaxSeq tokens, any input, the
//     RMSNorm prologue and the residual; an item covers one 16-token block of
//     its group's candidate tokens.
//
// The work unit is an ITEM (group g, slice s): 128 inter rows of one expert
// group (a routed expert, or one of the shared MLP's virtual groups). One
// workgroup computes, for its tokens,
//   act[t, s*128 .. s*128+127] = silu(gate_rows . x_t) * (up_rows . x_t)
// and right away the down projection restricted to those 128 inter columns,
//   part[.][s][t][0 .. H) = down[:, s*128 .. s*128+127] . act[t, slice]
// (the split-K partial of the expert's output; src/engine/moe_decoder.cpp:62-74
// sums over all inter columns, here the partials of the slices are added in
// slice order by the combine). Gate/up rows and the matching down columns
// stream in together; nothing waits for another item. Routing is needed only
// (1) to know which tokens' partial rows to store (wide mode: which tokens an
// item computes) -- the candidate experts that the routers publish before
// their exact chains -- and (2) by the combine.
//
//   workgroups [0, T)   the router of token t (candidates, then the exact
//                       chain, scores and top_k); wide mode: afterwards they
//                       take items from the end of the item list
//   workgroups [T, P)   16-token mode: item w (w = b - T), group-major,
//                       then the w-th, (w + PW)-th, ... item from PW on whose
//                       group some token's candidates name (or a shared
//                       group); wide mode: item w, then items drawn from a
//                       per-call ticket counter. Each worker issues the next
//                       item's weights while it computes the current item's
//                       down partial
//   combine units       16-token mode: (token t, 128 output columns); wide
//                       mode: (token t, several column blocks), one per
//                       workgroup from the last one down: after the exact
//                       routing of t and the items of t's picks and of the
//                       shared groups,
//                       out[t] = sum_j w[t,j] * sum_s part[id_j][s][t]
//                              + sum_v sum_s part[E+v][s][t] (+ shared_y)
//                              (+ the residual)
//                       in the reference's j order (moe_decoder.cpp:88-97,
//                       110-112, 179).
//
// Cross-workgroup data goes through agent-coherent accesses with bounded
// waits (fused_common.hpp): per-workgroup progress words (a workgroup
// publishes S + steps, every word ends the call at S + kFusedSteps), tagged
// candidate words and tagged per-item completion words.
#include <hip/hip_runtime.h>
#include "fused_common.hpp"

#include <algorithm>
#include <type_traits>

namespace uocr_hip {

constexpr int kStreamWaves = 8;
// weight units (1 KiB each) in flight per wave. A CU streams about (bytes in
// flight) / (memory latency): 6 units per wave keep a kernel within 128 VGPRs,
// so that two workgroups (16 waves) share a CU where the rest of the kernel
// fits (group 64 / 128, 16-token mode); where it does not (group 32, wide
// mode), one workgroup per CU keeps 10 units per wave in flight. A unit and
// the unit kRing further on share a ring slot, so kRing divides the units of
// an item.
template <int GPT, bool WIDE>
constexpr int ring_units() { return (WIDE || GPT == 4) ? 10 : 6; }
constexpr int kStreamThreads = 64 * kStreamWaves;
constexpr size_t align_up_c(size_t v, size_t a) { return (v + a - 1) / a * a; }

// LDS of a worker (the router role uses the first bytes for its own data)
template <int GPT, int KTG, int KTD, bool ZP>
struct StreamLds {
    static constexpr int GS = kTileK / GPT;                    // group size
    static constexpr int NGG = scale_row_stride(KTG * kTileK, GS);
    static constexpr int SRM = kTileRows * NGG;                // one wave's scale rows of one matrix
    static constexpr int NTD = KTG * kTileK / kTileRows / kStreamWaves;  // down tiles per wave (10 at H = 1280)
    static constexpr size_t as_bytes = (size_t)KTG * 4 * 64 * 8 * 2;   // x rows (f16, MFMA A layout)
    static constexpr int SROWS = ZP ? 4 : 2;                   // gate, up (, gate zeros, up zeros)
    static constexpr size_t ss_bytes = (size_t)kStreamWaves * SROWS * SRM * 2;
    static constexpr int ZOFF_G = 2 * SRM * 2;                 // scale row -> zero-offset row (gate/up)
    static constexpr size_t ad_bytes = (size_t)4 * 64 * 8 * 2; // act of the slice (down A operand)
    static constexpr int DSW = NTD * kTileRows * GPT;          // one wave's down scales (f16)
    static constexpr size_t ds_bytes = (size_t)kStreamWaves * DSW * 2 * (ZP ? 2 : 1);
    static constexpr int ZOFF_D = kStreamWaves * DSW * 2;      // scale -> zero offset (down)
    static constexpr int n_ints = 2 * kFusedMaxSeq + kMaxExperts + 2 * kMaxTopK + 2;
    static constexpr size_t o_ss = as_bytes;
    static constexpr size_t o_ad = o_ss + ss_bytes;
    static constexpr size_t o_ds = o_ad + ad_bytes;
    static constexpr size_t o_int = o_ds + ds_bytes;
    // wide mode: every token's expert mask, per group its token count, first partial row, 16-token blocks and first extra block,
    // each wave's token list, a combine unit's rows and items
    static constexpr size_t o_mask = align_up_c(o_int + (size_t)n_ints * 4, 8);
    static constexpr size_t o_tab = o_mask + (size_t)kStreamWideMaxSeq * 8;
    static constexpr size_t o_wl = o_tab + (size_t)4 * kMaxExperts * 4;
    static constexpr size_t o_cu = o_wl + (size_t)kStreamWaves * 16 * 4;
    static constexpr size_t bytes = o_cu + (size_t)2 * (kMaxTopK + kMaxExperts) * 4 + 16;
};

// 16-byte global -> LDS DMA per lane (to lds_base + 16 * lane; lds_base
// wave-uniform) written as asm for the same reason: with an LDS DMA pending,
// the compiler waits for every outstanding load before any use of a loaded
// register. Only the explicit counter waits order the LDS data.
// (M0 is a reserved register to the compiler, which sets it before each of
// its own uses, so the clobber is a note for the reader; clang warns about it)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* src, const void* lds_base) {
    const uint32_t m = __builtin_amdgcn_readfirstlane(lds_addr(lds_base));
    // (an M0 write needs a wait state before the LDS DMA that reads it)
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m) : "memory", "m0");
}
// the same, agent-coherent (rows other workgroups of the launch wrote)
__device__ __forceinline__ void dma16_sc1(const void* src, const void* lds_base) {
    const uint32_t m = __builtin_amdgcn_readfirstlane(lds_addr(lds_base));
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 1\n\tglobal_load_lds_dwordx4 %0, off sc1" ::"v"(src), "s"(m)
                 : "memory", "m0");
}
#pragma clang diagnostic pop
// asm LDS word write (see lds_read_u32)
__device__ __forceinline__ void lds_write_u32(void* p, int v) {
    asm volatile("ds_write_b32 %0, %1" ::"v"(lds_addr(p)), "v"(v) : "memory");
}
// Stores whose completion only the explicit counter waits track: written as
// asm, so the compiler's own waits for loaded registers do not see pending
// stores (with both loads and stores pending it would wait for everything).
// buffer_desc: a raw buffer over 2 GiB from `base`; an offset past that range
// (0x80000000) is dropped by the hardware.
__device__ __forceinline__ u32x4 buffer_desc(const void* base) {
    const uint64_t p = (uint64_t)base;
    return u32x4{(uint32_t)p, (uint32_t)(p >> 32) & 0xffffu, 0x7fffffffu, 0x00020000u};
}
// The compiler's hazard recognizer does not look into asm, so these spell out
// the wait states around them: a wide store's data registers must not be
// rewritten right after it, nor used right after their VALU write (without
// the nops the first dword of a 16-byte store was seen to carry the offset).
__device__ __forceinline__ void store16_sc1(const u32x4& desc, int off, const f32x4& v) {
    asm volatile("s_nop 4\n\tbuffer_store_dwordx4 %0, %1, %2, 0 offen sc1\n\ts_nop 4" ::"v"(v), "v"(off), "s"(desc)
                 : "memory");
}
__device__ __forceinline__ void store_sc1(int* p, int v) {
    asm volatile("s_nop 4\n\tglobal_store_dword %0, %1, off sc1\n\ts_nop 4" ::"v"(p), "v"(v) : "memory");
}

// Down partials of two 16-row tiles at the item's k-tile (128 inter columns):
// D[row][token] = sum_k W[row][k] * act[token][k] with the weights as the A
// operand (lane l: row l % 16, k 8(l/16) ..) and act as B (lane l: token
// l % 16, the same k -- the lane's fragment of Ad as staged for the gate/up
// layout), so lane l ends with rows 4(l/16) .. +3 of token l % 16: one 16-byte
// store per tile. Per scale group the MFMAs run from zero on the exact
// integers q - zero (ZP: the stored zero offsets of row l % 16, else 8), and
// the group result is scaled per row into the accumulator. sc0 / sc1: LDS byte
// addresses of the scale rows 4(l/16) .. of the two tiles ([row][GPT] f16);
// zr0 / zr1 (ZP): of the scale row l % 16, whose zero offsets sit ZOFF bytes on.
template <int GPT, bool ZP, int ZOFF>
__device__ __forceinline__ void down_pair(const u32x4& w0, const u32x4& w1, const f16x8 (&av)[4], uint32_t sc0,
                                          uint32_t sc1, uint32_t zr0, uint32_t zr1, f32x4& acc0, f32x4& acc1) {
    constexpr int SPG = 4 / GPT;  // MFMA steps per scale group
    // scales of the lane's 4 rows (GPT per row, f16): GPT 4: 32 bytes per
    // tile, GPT 2: 16, GPT 1: 8
    u32x4 s0[2], s1[2];
    uint64_t z0 = 0, z1 = 0;  // ZP: zero offsets of row l % 16 (GPT halves)
    if constexpr (GPT == 4) {
        asm volatile("ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:16\n\tds_read_b128 %2, %5\n\tds_read_b128 %3, %5 offset:16"
                     : "=&v"(s0[0]), "=&v"(s0[1]), "=&v"(s1[0]), "=&v"(s1[1]) : "v"(sc0), "v"(sc1) : "memory");
    } else if constexpr (GPT == 2) {
        asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3" : "=&v"(s0[0]), "=&v"(s1[0]) : "v"(sc0), "v"(sc1) : "memory");
    } else {
        uint64_t a0, a1;
        asm volatile("ds_read_b64 %0, %2\n\tds_read_b64 %1, %3" : "=&v"(a0), "=&v"(a1) : "v"(sc0), "v"(sc1) : "memory");
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a0), "+v"(a1)::"memory");
        s0[0] = u32x4{(uint32_t)a0, (uint32_t)(a0 >> 32), 0u, 0u};
        s1[0] = u32x4{(uint32_t)a1, (uint32_t)(a1 >> 32), 0u, 0u};
    }
    if constexpr (ZP) {
        if constexpr (GPT == 4) {
            asm volatile("ds_read_b64 %0, %2 offset:%4\n\tds_read_b64 %1, %3 offset:%4"
                         : "=&v"(z0), "=&v"(z1) : "v"(zr0), "v"(zr1), "n"(ZOFF) : "memory");
        } else if constexpr (GPT == 2) {
            uint32_t a0, a1;
            asm volatile("ds_read_b32 %0, %2 offset:%4\n\tds_read_b32 %1, %3 offset:%4"
                         : "=&v"(a0), "=&v"(a1) : "v"(zr0), "v"(zr1), "n"(ZOFF) : "memory");
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a0), "+v"(a1)::"memory");
            z0 = a0;
            z1 = a1;
        } else {
            uint32_t a0, a1;
            asm volatile("ds_read_u16 %0, %2 offset:%4\n\tds_read_u16 %1, %3 offset:%4"
                         : "=&v"(a0), "=&v"(a1) : "v"(zr0), "v"(zr1), "n"(ZOFF) : "memory");
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a0), "+v"(a1)::"memory");
            z0 = a0;
            z1 = a1;
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(s0[0]), "+v"(s0[1]), "+v"(s1[0]), "+v"(s1[1]), "+v"(z0), "+v"(z1)::"memory");
    // scale of the lane's row q (0..3) in group gi
    auto scale_of = [&](const u32x4* sv, int q, int gi) -> float {
        const int h = q * GPT + gi;  // half index
        const uint32_t word = sv[h >> 3][(h >> 1) & 3];
        return (float)__builtin_bit_cast(f16, (uint16_t)(word >> (16 * (h & 1))));
    };
    // the zero offset -(1024 + zero) of group gi
    auto zero_of = [&](uint64_t z, int gi) -> f16 {
        if constexpr (ZP) return __builtin_bit_cast(f16, (uint16_t)(z >> (16 * gi)));
        else return (f16)-1032.0f;
    };
    f32x4 p0 = {0.f, 0.f, 0.f, 0.f}, p1 = p0;
#pragma unroll
    for (int gi = 0; gi < GPT; ++gi) {
        f32x4 r0 = {0.f, 0.f, 0.f, 0.f}, r1 = r0;
#pragma unroll
        for (int s = gi * SPG; s < (gi + 1) * SPG; ++s) {
            r0 = mfma16(dequant8z_unscaled(w0[s], zero_of(z0, gi)), av[s], r0);
            r1 = mfma16(dequant8z_unscaled(w1[s], zero_of(z1, gi)), av[s], r1);
        }
        // the previous group's results, scaled in now (their MFMA latency is covered)
        if (gi > 0) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc0[q] = fmaf(scale_of(s0, q, gi - 1), p0[q], acc0[q]);
                acc1[q] = fmaf(scale_of(s1, q, gi - 1), p1[q], acc1[q]);
            }
            asm volatile("" : "+v"(acc0), "+v"(acc1));
        }
        p0 = r0;
        p1 = r1;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        acc0[q] = fmaf(scale_of(s0, q, GPT - 1), p0[q], acc0[q]);
        acc1[q] = fmaf(scale_of(s1, q, GPT - 1), p1[q], acc1[q]);
    }
}

// Combine of one unit (token t, output columns cb*128 ..): thread (slot jj,
// column quad q); slot j < K holds the routed pick j, slot K the sum of the
// shared groups. Rows are read agent-coherent (written by other workgroups).
// Partial rows: [group][slice][token] (rows = null), or (wide mode) row
// rows[jj] of [row][slice] for routed pick jj < K and shared group jj - K.
// With an RMSNorm prologue the layer adds its input (the residual) last.
template <int NS>
__device__ __forceinline__ void stream_combine(const DecodeArgs& a, int t, int cb, const int* ids_t,
                                               const float* wts_t, const int* rows, bool bad, float* ys) {
    const int tid = threadIdx.x;
    const int T = a.seq, E = a.n_experts, V = a.n_virtual, K = a.top_k, H = a.hidden;
    const int q = tid & 31, tg = tid >> 5;  // 16 thread groups of 32 column quads
    const int c = cb * 128 + q * 4;
    const bool colv = c < H;
    // byte offset of slice 0 of pick / shared group jj
    auto row_off = [&](int jj) -> size_t {
        if (rows) return ((size_t)rows[jj] * NS * H + c) * 4;
        const size_t g = jj < K ? (size_t)ids_t[jj] : (size_t)(E + jj - K);
        return (((g * NS) * T + t) * H + c) * 4;
    };
    const size_t s_step = (rows ? (size_t)H : (size_t)T * H) * 4;  // bytes between slices
    for (int jj = tg; jj <= K; jj += kStreamThreads / 32) {
        f32x4 y = {0.f, 0.f, 0.f, 0.f};
        if (colv) {
            for (int jv = jj; jv < (jj < K ? jj + 1 : K + V); ++jv) {
                const size_t o = row_off(jv);
                f32x4 v[NS];
#pragma unroll
                for (int s = 0; s < NS; ++s) v[s] = load16_cg(a.y, o + s * s_step);
#pragma unroll
                for (int s = 0; s < NS; ++s)
#pragma unroll
                    for (int i = 0; i < 4; ++i) y[i] += v[s][i];
            }
        }
        *reinterpret_cast<f32x4*>(ys + jj * 128 + q * 4) = y;
    }
    __syncthreads();
    if (tid < 32 && colv) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int j = 0; j < K; ++j) {
            const float w = wts_t[j];
            const f32x4 y = *reinterpret_cast<const f32x4*>(ys + j * 128 + q * 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = fmaf(w, y[i], acc[i]);
        }
        if (V > 0) {
            const f32x4 sh = *reinterpret_cast<const f32x4*>(ys + K * 128 + q * 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += sh[i];
        }
        if (a.shared_y) {  // written by an earlier launch: a plain load
            const f32x4 sv = *reinterpret_cast<const f32x4*>(a.shared_y + (size_t)t * H + c);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += sv[i];
        }
        if (a.rms_weight) {  // the residual (f32 input)
            const f32x4 rv = *reinterpret_cast<const f32x4*>(static_cast<const float*>(a.x) + (size_t)t * H + c);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = rv[i] + acc[i];
        }
        if (bad) acc = f32x4{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")};
        *reinterpret_cast<f32x4*>(a.out + (size_t)t * H + c) = acc;
    }
    __syncthreads();
}

// Wide-mode combine of token t, output columns c0 .. c0 + ncol: first every
// (slot jj, column quad) -- slot j < K the routed pick j, K + v shared group v
// -- sums its partial rows over the slices in order (row rows[jj] of
// [row][slice], agent-coherent reads, two tasks per thread with all their
// loads in flight) into ys [K + V][ncol]; then out = sum_j w_j * ys[j] in j
// order + (ys[K] + ys[K + 1] + ...) (+ shared_y) (+ the residual).
template <int NS>
__device__ __forceinline__ void stream_combine_wide(const DecodeArgs& a, int t, int c0, int ncol, const float* wts_t,
                                                    const int* rows, bool bad, float* ys) {
    const int tid = threadIdx.x;
    const int V = a.n_virtual, K = a.top_k, H = a.hidden;
    const int nq = ncol >> 2, ntask = (K + V) * nq;
    for (int k0 = tid; k0 < ntask; k0 += 2 * kStreamThreads) {
        const int k1 = min(k0 + kStreamThreads, ntask - 1);  // (a repeat of the last task when past the end)
        const int j0 = k0 / nq, q0 = k0 - j0 * nq, j1 = k1 / nq, q1 = k1 - j1 * nq;
        const size_t o0 = ((size_t)rows[j0] * NS * H + c0 + 4 * q0) * 4, o1 = ((size_t)rows[j1] * NS * H + c0 + 4 * q1) * 4;
        f32x4 v0[NS], v1[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            v0[s] = load16_cg(a.y, o0 + (size_t)s * H * 4);
            v1[s] = load16_cg(a.y, o1 + (size_t)s * H * 4);
        }
        f32x4 y0 = {0.f, 0.f, 0.f, 0.f}, y1 = y0;
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                y0[i] += v0[s][i];
                y1[i] += v1[s][i];
            }
        *reinterpret_cast<f32x4*>(ys + (size_t)j0 * ncol + 4 * q0) = y0;
        *reinterpret_cast<f32x4*>(ys + (size_t)j1 * ncol + 4 * q1) = y1;
    }
    __syncthreads();
    for (int q = tid; q < nq; q += kStreamThreads) {
        const int c = c0 + 4 * q;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int j = 0; j < K; ++j) {
            const float w = wts_t[j];
            const f32x4 y = *reinterpret_cast<const f32x4*>(ys + (size_t)j * ncol + 4 * q);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = fmaf(w, y[i], acc[i]);
        }
        if (V > 0) {
            f32x4 sh = *reinterpret_cast<const f32x4*>(ys + (size_t)K * ncol + 4 * q);
            for (int v = 1; v < V; ++v) {
                const f32x4 y = *reinterpret_cast<const f32x4*>(ys + (size_t)(K + v) * ncol + 4 * q);
#pragma unroll
                for (int i = 0; i < 4; ++i) sh[i] += y[i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += sh[i];
        }
        if (a.shared_y) {
            const f32x4 sv = *reinterpret_cast<const f32x4*>(a.shared_y + (size_t)t * H + c);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += sv[i];
        }
        if (a.rms_weight) {  // the residual (f32 input)
            const f32x4 rv = *reinterpret_cast<const f32x4*>(static_cast<const float*>(a.x) + (size_t)t * H + c);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = rv[i] + acc[i];
        }
        if (bad) acc = f32x4{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")};
        *reinterpret_cast<f32x4*>(a.out + (size_t)t * H + c) = acc;
    }
    __syncthreads();
}

// One item of a worker: expert group g, slice s, and in wide mode the
// 16-token block tb of the group's tokens (n of them, partial rows row0 ..);
// wi = g * NS + s indexes the weights; tok: the token of the lane's row
struct StreamItem {
    int g, s, tb, wi, n, row0, tok;
};

template <int GPT, int KTG, int KTD, bool ZP, bool WIDE, bool F32R>
__global__ __launch_bounds__(kStreamThreads, 2) void decode_stream_kernel(DecodeArgs a) {
    using Lay = StreamLds<GPT, KTG, KTD, ZP>;
    constexpr int kRing = ring_units<GPT, WIDE>();
    constexpr int NS = KTD;             // slices per group (128 inter rows each)
    constexpr int NTD = Lay::NTD;       // down tiles per wave
    constexpr int NGG = Lay::NGG;
    constexpr int SROW = kTileRows * NGG;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    f16* As = reinterpret_cast<f16*>(smem);
    f16* Ss = reinterpret_cast<f16*>(smem + Lay::o_ss);
    f16* Ad = reinterpret_cast<f16*>(smem + Lay::o_ad);
    f16* Ds = reinterpret_cast<f16*>(smem + Lay::o_ds);
    uint32_t* cm32 = reinterpret_cast<uint32_t*>(smem + Lay::o_int);  // candidate masks per token
    int* tokmask = reinterpret_cast<int*>(cm32 + 2 * kFusedMaxSeq);  // per routed group: candidate tokens
    int* misc = tokmask + kMaxExperts;
    // wide mode tables
    uint64_t* masks = reinterpret_cast<uint64_t*>(smem + Lay::o_mask);  // [token] picked experts
    int* cntL = reinterpret_cast<int*>(smem + Lay::o_tab);               // [group] tokens
    int* baseL = cntL + kMaxExperts;                                     // [group] first partial row
    int* nbL = baseL + kMaxExperts;                                      // [group] 16-token blocks
    int* extL = nbL + kMaxExperts;                                       // [group] first extra block
    int* cuL = reinterpret_cast<int*>(smem + Lay::o_cu);  // combine unit: rows [K + V], first items [K + V]
    int* ntotL = cuL + 2 * (kMaxTopK + kMaxExperts);

    int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, r = lane & 15;
    auto fresh_indices = [&]() { asm volatile("" : "+v"(tid), "+v"(lane), "+v"(r), "+s"(wave)); };
    const int T = a.seq, E = a.n_experts, V = a.n_virtual, G = E + V, K = a.top_k;
    const int H = a.hidden, I = a.inter;
    const int P = gridDim.x, b = blockIdx.x, PW = P - T;
    const int NI = G * NS;  // items
    FusedSync* sy = a.sync;
    int* prog = sy->progress;
    const uint16_t* xb = static_cast<const uint16_t*>(a.x);
    (void)I;

    const int S = load_cg(prog + b);
    const unsigned rtag = (((unsigned)S >> 12) + 1u) & 0xFFFFFFu;
    // wide mode: this call's item tickets; the other counter is cleared for the next call
    unsigned long long* queue = sy->queue + (((unsigned)S >> 12) & 1u);
    if (WIDE && b == 0 && tid == 0) store_cg(sy->queue + ((((unsigned)S >> 12) & 1u) ^ 1u), 0ull);
    int k = 0;  // steps published by this workgroup
    auto publish_now = [&]() {
        __syncthreads();
        ++k;
        if (tid == 0) store_sc1(prog + b, S + k);
    };
    auto wait_steps = [&](auto&& pair_of, int n) {
        if (wave == 0) {
            for (int base = 0; base < n; base += 64) {
                int owner = 0, step = 0;
                const bool want = base + lane < n;
                if (want) pair_of(base + lane, owner, step);
                int it = 0;
                while (__ballot(want && (int)(load_cg(prog + owner) - (S + step)) < 0)) {
                    if (++it > kSpinLimit) {
                        if (lane == 0) report_timeout_to(a.status, sy, rtag);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
        }
        __syncthreads();
        fence_wg_acquire();
    };

    // candidate masks of every token (tagged words the routers publish before
    // their exact chains) -> cm32, and per routed group the mask of its
    // candidate tokens -> tokmask
    bool have_cand = false;
    auto need_cand = [&]() {
        if (have_cand) return;
        if (wave == 0) {
            uint64_t cw = lane < 2 * T ? __hip_atomic_load(sy->cand + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                       : ((uint64_t)rtag << 32);
            int it = 0;
            while (__ballot((uint32_t)(cw >> 32) != rtag)) {
                if (++it > kSpinLimit) {
                    if (lane == 0) report_timeout_to(a.status, sy, rtag);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
                if (lane < 2 * T) cw = __hip_atomic_load(sy->cand + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (lane < 2 * T) cm32[lane] = (uint32_t)cw;
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            int tm = 0;
            for (int t = 0; t < T; ++t) tm |= (int)((cm32[2 * t + (lane >> 5)] >> (lane & 31)) & 1u) << t;
            tokmask[lane] = lane < E ? tm : 0;
        }
        __syncthreads();
        have_cand = true;
    };

    // Wide mode: every token's candidate experts (tagged words the routers
    // publish with the expert input rows, before their exact chains) -> the
    // token masks; then per group its token count, first partial row (groups
    // in order, tokens ascending: routed rows first, then T rows per shared
    // group), 16-token blocks and first extra block. Items: (g, s) for every
    // group and slice (block 0), then (g, block tb >= 1, s) in group order ->
    // NTOT. When the candidates' rows exceed the partial-row budget
    // (kStreamCandRows per token), the exact picks take their place (every
    // workgroup sees the same words and decides alike).
    int NTOT = NI;
    uint64_t my_mask = 0;  // lane t: token t's experts (every wave)
    bool wide_ready = false;
    auto wide_tables = [&]() -> int {  // the routed rows
        my_mask = masks[lane];
        for (int g = wave; g < E; g += kStreamWaves) {
            const uint64_t bb = __ballot((my_mask >> g) & 1);
            if (lane == 0) cntL[g] = (int)__popcll(bb);
        }
        __syncthreads();
        if (wave == 0) {
            int run_n = 0, run_x = 0;
            for (int h = 0; h < G; h += 64) {
                const int g = h + lane;
                const int n = g < E ? cntL[g] : (g < G ? T : 0);
                const int nb = (n + 15) >> 4;
                const int xb = nb > 1 ? nb - 1 : 0;
                int sn = n, sx = xb;
                for (int d = 1; d < 64; d <<= 1) {
                    const int u1 = __shfl_up(sn, d, 64), u2 = __shfl_up(sx, d, 64);
                    if (lane >= d) {
                        sn += u1;
                        sx += u2;
                    }
                }
                if (g < G) {
                    baseL[g] = run_n + sn - n;
                    nbL[g] = nb;
                    extL[g] = run_x + sx - xb;
                }
                run_n += __shfl(sn, 63, 64);
                run_x += __shfl(sx, 63, 64);
            }
            if (lane == 0) {
                ntotL[0] = NI + run_x * NS;
                ntotL[1] = run_n - V * T;  // the shared groups hold T rows each
            }
        }
        __syncthreads();
        // (readfirstlane: values read from LDS look divergent to the compiler, and a
        // loop bound on them made it place wave-uniform values in vector registers)
        NTOT = __builtin_amdgcn_readfirstlane(ntotL[0]);
        return __builtin_amdgcn_readfirstlane(ntotL[1]);
    };
    auto wide_setup = [&]() {
        if (wave == 0) {
            uint64_t c0 = (uint64_t)rtag << 32, c1 = c0;
            int it = 0;
            while (true) {
                if (lane < T) {
                    c0 = __hip_atomic_load(sy->cand + 2 * lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    c1 = __hip_atomic_load(sy->cand + 2 * lane + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                if (!__ballot((uint32_t)(c0 >> 32) != rtag || (uint32_t)(c1 >> 32) != rtag)) break;
                if (++it > kSpinLimit) {
                    if (lane == 0) report_timeout_to(a.status, sy, rtag);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            masks[lane] = lane < T ? (uint64_t)(uint32_t)c0 | ((uint64_t)(uint32_t)c1 << 32) : 0ull;
        }
        __syncthreads();
        fence_wg_acquire();  // the expert input rows published with the words
        if (wide_tables() > T * kStreamCandRows) {
            // the exact picks (all routers done)
            if (wave == 0) {
                int it = 0;
                while (__ballot(lane < T && (int)(load_cg(prog + lane) - (S + 1)) < 0)) {
                    if (++it > kSpinLimit) {
                        if (lane == 0) report_timeout_to(a.status, sy, rtag);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
            __syncthreads();
            fence_wg_acquire();
            if (wave == 0) {
                uint64_t m = 0;
                if (lane < T)
                    for (int j = 0; j < K; ++j) m |= 1ull << (load_cg(a.ids + (size_t)lane * K + j) & 63);
                masks[lane] = m;
            }
            __syncthreads();
            wide_tables();
        }
        wide_ready = true;
    };

    // ---- 1. router (workgroups 0 .. T-1)
    if (b < T) {
        float* hand = reinterpret_cast<float*>(smem);
        float* sc = hand + 64;
        float* topv = sc + 64;
        uint64_t* etab = reinterpret_cast<uint64_t*>(topv + kMaxTopK);
        float* xs = hand + 256;
        router_token_regs<KTG, kStreamWaves, WIDE, F32R>(a, b, hand, sc, topv, etab, xs, xs + kMaxHidden, rtag);
        store_fence();
        publish_now();
    }

    // ---- 2. items (workers T .. P-1)
    // gate/up rows of the item's slice: wave w owns the 16 rows s*128 + 16w ..;
    // down: wave w owns the NTD 16-row tiles w*NTD .. of the hidden outputs,
    // k-tile s of the down matrix (= the slice's 128 inter columns).
    //
    // Pipeline (per wave, no wait on another workgroup): a wave's weights of
    // an item are kUnits 1 KiB units in order of use -- gate k-tile 0, up
    // k-tile 0, ..., up k-tile KTG-1, then the NTD down tiles -- read from the
    // streamed copy (a.sw: unit u of every item and wave side by side, so that
    // all workgroups read one compact window at a time). They pass through a
    // ring of kRing registers: consuming unit u issues unit u + kRing (of this
    // item, or of the next one), so every wave keeps kRing units in flight.
    // Scales go to LDS by DMA: the next item's gate/up scales once the current
    // gate/up MMA is done, its down scales once the current down MMA is done.
    // An item's partial rows are published (progress step) at the next item's
    // down phase, when the counter wait that precedes it has covered those
    // stores.
    constexpr int kUnits = 2 * KTG + NTD;
    static_assert(kUnits % kRing == 0 && kRing <= 2 * KTG, "ring slots repeat every item");
    u32x4 ring[kRing];
    // unit u of the item with weight index i (u < kUnits) into its ring slot u % kRing
    auto unit = [&](int i, int u) {
        ring[u % kRing] = *reinterpret_cast<const u32x4*>(
            a.sw + (((size_t)u * NI + i) * kStreamWaves + wave) * kTileBytes + (size_t)lane * 16);
    };
    // after consuming unit u of weight item i: the unit kRing further on (of
    // i, or of the next item nx)
    auto advance = [&](int i, int u, int nx, bool more) {
        const int v = u + kRing;
        asm volatile("" ::: "memory");
        if (v < kUnits) {
            unit(i, v);
        } else if (more) {
            unit(nx, v - kUnits);
        }
        asm volatile("" ::: "memory");
    };
    f16* ssw = Ss + (size_t)wave * Lay::SROWS * Lay::SRM;
    f16* dsw = Ds + (size_t)wave * Lay::DSW;
    // gate/up scales (, zero offsets) of the wave's 16 rows: 2 (4) DMA instructions per matrix
    auto gu_scales = [&](int i) {
        const int g = i / NS, s = i % NS;
        const size_t sb = (size_t)g * a.gu_sstride + (size_t)(s * 8 + wave) * SROW;
        for (int q = lane; q * 8 < SROW; q += 64) {
            dma16(a.gate_s + sb + q * 8, ssw + (q & ~63) * 8);
            dma16(a.up_s + sb + q * 8, ssw + Lay::SRM + (q & ~63) * 8);
            if constexpr (ZP) {
                dma16(a.gate_z + sb + q * 8, ssw + 2 * Lay::SRM + (q & ~63) * 8);
                dma16(a.up_z + sb + q * 8, ssw + 3 * Lay::SRM + (q & ~63) * 8);
            }
        }
    };
    // down scales (, zero offsets) of k-tile s for the wave's rows: [g][s][row][GPT]
    auto dn_scales = [&](int i) {
        const int g = i / NS, s = i % NS;
        const size_t sb = ((size_t)g * KTD + s) * (size_t)(NTD * kStreamWaves * kTileRows) * GPT +
                          (size_t)wave * Lay::DSW;
        for (int q = lane; q * 8 < Lay::DSW; q += 64) {
            dma16(a.down_skt + sb + q * 8, dsw + (q & ~63) * 8);
            if constexpr (ZP) dma16(a.down_zkt + sb + q * 8, dsw + Lay::ZOFF_D / 2 + (q & ~63) * 8);
        }
    };

    // the item at list position idx (wide mode; every wave, after wide_setup)
    int* wlw = reinterpret_cast<int*>(smem + Lay::o_wl) + wave * 16;  // this wave's token list
    auto witem = [&](int idx) -> StreamItem {
        StreamItem it;
        if (idx < NI) {
            it.g = idx / NS;
            it.s = idx - it.g * NS;
            it.tb = 0;
        } else {
            const int e = idx - NI, xbk = e / NS;
            it.s = e - xbk * NS;
            it.g = 0;
            for (int h = 0; h < G; h += 64) {
                const int gg = h + lane;
                const int eb = (int)lds_read_u32(extL + gg), nb = (int)lds_read_u32(nbL + gg);
                const uint64_t hit = __ballot(gg < G && xbk >= eb && xbk < eb + nb - 1);
                if (hit) {
                    it.g = h + (int)__builtin_ctzll(hit);
                    break;
                }
            }
            it.tb = xbk - (int)lds_read_u32(extL + it.g) + 1;
        }
        it.wi = it.g * NS + it.s;
        const int ng = it.g < E ? (int)lds_read_u32(cntL + it.g) : T;
        it.n = min(16, ng - 16 * it.tb);
        it.row0 = (int)lds_read_u32(baseL + it.g) + 16 * it.tb;
        if (it.g < E) {
            const bool mem = (my_mask >> it.g) & 1;
            const uint64_t bal = __ballot(mem);
            const int rank = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                             __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
            if (mem && rank >= 16 * it.tb && rank < 16 * it.tb + 16) lds_write_u32(wlw + rank - 16 * it.tb, lane);
            it.tok = it.n > 0 ? (int)lds_read_u32(wlw + (r < it.n ? r : 0)) : 0;
        } else {
            it.tok = 16 * it.tb + (r < it.n ? r : 0);
        }
        return it;
    };
    // StreamItem of list position i (streamed mode: every item is block 0 of all tokens)
    auto sitem = [&](int i) -> StreamItem {
        StreamItem it;
        it.g = i / NS;
        it.s = i - it.g * NS;
        it.tb = 0;
        it.wi = i;
        it.n = T;
        it.row0 = 0;
        it.tok = r;
        return it;
    };
    // wide mode: the f16 token rows of an item's block -> As (the MFMA A
    // layout; wave w stages blocks w, w + 8, ...: k-tile blk / 4, step blk % 4)
    constexpr int NXD = KTG * 4 / kStreamWaves;  // x DMAs per wave
    static_assert(KTG * 4 % kStreamWaves == 0, "x blocks per wave");
    auto x_rows = [&](int tok) {
        const f16* src = a.x16 + (size_t)tok * H + 8 * (lane >> 4);
#pragma unroll
        for (int q = 0; q < NXD; ++q) {
            const int blk = wave + kStreamWaves * q;
            dma16_sc1(src + (blk >> 2) * kTileK + (blk & 3) * 32, As + (size_t)blk * 64 * 8);
        }
    };
    // the first kRing units and the scales of weight item wi
    auto prefetch = [&](int wi) {
        asm volatile("" ::: "memory");
        gu_scales(wi);
        dn_scales(wi);
        asm volatile("" ::: "memory");
        // (one compiler barrier per unit: the issue order is the order of use)
#pragma unroll
        for (int u = 0; u < kRing; ++u) {
            unit(wi, u);
            asm volatile("" ::: "memory");
        }
    };

    // Wide mode: the routers join the workers once their routing is done.
    // Worker w's first item is item w; every further item (routers: every
    // item) comes from a ticket of the call's counter, drawn one item ahead:
    // workers take items PW, PW + 1, ... from the front, routers (late) take
    // them from the end, NTOT - 1, NTOT - 2, ... A ticket is the counter
    // before the draw (front draws in the low half, end draws in the high
    // half), so the two sides never take the same item.
    int* tkL = ntotL + 2;          // a drawn item, shared through LDS
    unsigned long long tkn = 0;    // thread 0: the ticket drawn during the current item
    const unsigned long long tk_step = b < T ? (1ull << 32) : 1ull;
    auto draw = [&]() { return __hip_atomic_fetch_add(queue, tk_step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    auto tk_item = [&](unsigned long long tk) -> int {  // (after wide_setup: NTOT)
        const int lo = (int)(uint32_t)tk, hi = (int)(tk >> 32);
        if (lo + hi >= NTOT - PW) return NTOT;
        return b < T ? NTOT - 1 - hi : PW + lo;
    };
    // 16-token mode: the first PW items are static (worker w: item w); worker
    // w's k-th further item is the (w + (k - 1) PW)-th item from PW on whose
    // group is live (a candidate token, or a shared group), so a group that no
    // token can pick is not streamed past the first round. Wave 0, after the
    // candidates are resolved (tokmask).
    auto live_item = [&](int j) -> int {
        int base = 0;
        for (int g0 = 0; g0 < G; g0 += 64) {
            const int g = g0 + lane;
            int n = 0;
            if (g < G && (g >= E || (int)lds_read_u32(tokmask + g) != 0)) n = max(0, (g + 1) * NS - max(PW, g * NS));
            int sn = n;
            for (int d = 1; d < 64; d <<= 1) {
                const int u = __shfl_up(sn, d, 64);
                if (lane >= d) sn += u;
            }
            const int tot = __builtin_amdgcn_readfirstlane(__shfl(sn, 63, 64));
            if (j < base + tot) {
                const uint64_t hit = __ballot(n > 0 && j < base + sn);
                const int l = (int)__builtin_ctzll(hit);
                const int before = __builtin_amdgcn_readfirstlane(__shfl(sn - n, l, 64));
                return max(PW, (g0 + l) * NS) + (j - base - before);
            }
            base += tot;
        }
        return NTOT;
    };
    int n_more = 0;  // 16-token mode: further items taken so far
    if (WIDE || (b >= T && b - T < NI)) {
        const int w = b - T;
        StreamItem first_item;
        int i0 = w;  // the first item
        if constexpr (WIDE) {
            // weights first (block 0 items exist whatever the routing), then
            // the routing, then this item's token rows
            if (b >= T && w < NI) prefetch(w);
            unsigned long long tk0 = 0;
            if (tid == 0 && b < T) tk0 = draw();  // a router's first item
            wide_setup();
            if (tid == 0) tkL[0] = tk_item(tk0);
            __syncthreads();
            i0 = __builtin_amdgcn_readfirstlane(b >= T ? w : tkL[0]);
            if (i0 < NTOT) {
                first_item = witem(i0);
                if (b < T || i0 >= NI) prefetch(first_item.wi);
                x_rows(first_item.tok);
            }
        } else {
            // the token rows (all T, once): bf16 DMA, then f16 in place; f32
            // input: into registers, f16 into As at the first item. Wave w
            // stages MFMA step w & 3 of k-tiles w >> 2, (w >> 2) + 2, ...
            if (a.x_bf16) {
                if (r < T) {
                    const uint16_t* src = xb + (size_t)r * H + (wave & 3) * 32 + 8 * (lane >> 4);
                    for (int kt = wave >> 2; kt < KTG; kt += 2)
                        dma16(src + kt * kTileK, As + (size_t)(kt * 4 + (wave & 3)) * 64 * 8);
                }
            }
            // issue order = the order the explicit counter waits assume
            prefetch(w);
            if (!a.x_bf16) {
                // f32 input: this wave's rows -> f16 into As, behind the
                // prefetch (the compiler's wait for them covers it too)
                constexpr int NKX = (KTG + 1) / 2;
                f32x4 xf[NKX][2];
                const float* src = static_cast<const float*>(a.x) + (size_t)min(r, T - 1) * H + (wave & 3) * 32 + 8 * (lane >> 4);
#pragma unroll
                for (int q = 0; q < NKX; ++q) {
                    const int kt = (wave >> 2) + 2 * q;
                    if (kt < KTG) {
                        xf[q][0] = *reinterpret_cast<const f32x4*>(src + kt * kTileK);
                        xf[q][1] = *reinterpret_cast<const f32x4*>(src + kt * kTileK + 4);
                    }
                }
#pragma unroll
                for (int q = 0; q < NKX; ++q) {
                    const int kt = (wave >> 2) + 2 * q;
                    if (kt < KTG) {
                        const f16x8 h = {(f16)xf[q][0][0], (f16)xf[q][0][1], (f16)xf[q][0][2], (f16)xf[q][0][3],
                                         (f16)xf[q][1][0], (f16)xf[q][1][1], (f16)xf[q][1][2], (f16)xf[q][1][3]};
                        asm volatile("ds_write_b128 %0, %1" ::"v"(lds_addr(As + (size_t)(kt * 4 + (wave & 3)) * 64 * 8 +
                                                                          (size_t)lane * 8)),
                                     "v"(h)
                                     : "memory");
                    }
                }
            }
            first_item = sitem(w);
        }
      if (i0 < NTOT) {

        // candidates: wave 0 requests the tagged words here, ahead of their
        // use in the first item's down phase, so waiting for them is part of
        // the in-order wait for older loads; words of an earlier call are
        // requested again (blocking) there. The first check is outside the
        // retry loop and each path stores the result itself: the compiler's
        // counter waits then never merge with the loop's.
        uint64_t cw = 0;
        if (!WIDE && wave == 0)
            cw = lane < 2 * T ? __hip_atomic_load(sy->cand + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                              : ((uint64_t)rtag << 32);
        // -> cm32 (every token's candidate mask) and tokmask, wave 0 (the
        // caller's barrier shares them)
        auto cand_store = [&](uint64_t c) {
            if (lane < 2 * T) cm32[lane] = (uint32_t)c;
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            int tm = 0;
            for (int t = 0; t < T; ++t) tm |= (int)((cm32[2 * t + (lane >> 5)] >> (lane & 31)) & 1u) << t;
            tokmask[lane] = lane < E ? tm : 0;
        };
        auto cand_resolve = [&]() {
            if (wave != 0) return;
            asm volatile("" : "+v"(cw));  // consumed here, not where it was requested
            if (!__ballot((uint32_t)(cw >> 32) != rtag)) {
                cand_store(cw);
                return;
            }
            uint64_t c2 = cw;
            int it = 0;
            do {
                if (++it > kSpinLimit) {
                    if (lane == 0) report_timeout_to(a.status, sy, rtag);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
                if (lane < 2 * T) c2 = __hip_atomic_load(sy->cand + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } while (__ballot((uint32_t)(c2 >> 32) != rtag));
            cand_store(c2);
        };

        bool ovf = false;  // an act value left f16's range (reported once at the end)
        // One item; MORE: a next item exists (its weights stream under this
        // item's work). The last item is a separate copy, so that the
        // compiler's own counter waits see one fixed issue order.
        // item i (list position) with nx after it and pi before it (-1: none)
        // The first half of an item: up to its gate/up MMA (wide mode: thread 0
        // draws the ticket of the next item at the start and shares it before
        // the closing barrier). The gate/up phase takes ring units of this
        // item only (kRing <= NTD).
        static_assert(kRing <= NTD, "the gate/up phase stays within its item's units");
        auto item_a = [&](const StreamItem& cur, bool first, f32x4& acc0, f32x4& acc1) {
            fresh_indices();
            const int wi = cur.wi;
            // this item's gate/up scales (and, first item, the token rows and
            // down scales): older than the last kRing ops (first item: the
            // ring's loads) or 2 * NTD ops (later items: the previous down
            // phase's NTD unit loads and NTD partial stores, and its down-scale
            // DMA)
            if (first) {
                if constexpr (WIDE) {
                    wait_vm<0>();  // (the routing wait came between)
                } else {
                    wait_vm<kRing>();
                }
            } else {
                wait_vm<2 * NTD>();
            }
            if constexpr (WIDE) {
                lds_barrier();  // every wave's token-row DMA has landed
                // (its counter wait, the compiler's, lets this phase's 2 * KTG unit loads run on)
                if (tid == 0) tkn = draw();
            } else if (first && !a.x_bf16) {
                lds_barrier();  // (f32 input: the rows went to As in the prologue)
            } else if (first) {
                // this wave's DMA'd rows -> f16 in place
                for (int kt = wave >> 2; kt < KTG; kt += 2) {
                    const uint32_t ad = lds_addr(As + (size_t)(kt * 4 + (wave & 3)) * 64 * 8 + (size_t)lane * 8);
                    u32x4 v;
                    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(ad) : "memory");
                    f16x8 h;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        h[2 * q] = (f16)__uint_as_float(v[q] << 16);
                        h[2 * q + 1] = (f16)__uint_as_float(v[q] & 0xffff0000u);
                    }
                    asm volatile("ds_write_b128 %0, %1" ::"v"(ad), "v"(h) : "memory");
                }
                lds_barrier();
            }
            // gate/up of the wave's 16 rows -> act (f16) into Ad in the down
            // A layout (inter column kl = 16 * wave + r of the slice); each
            // consumed k-tile's registers take the next item's k-tile
            acc0 = f32x4{0.f, 0.f, 0.f, 0.f};
            acc1 = acc0;
            item_mma_f<GPT, KTG, true, ZP, Lay::ZOFF_G, !ZP, false>(
                [&](int kt) -> const u32x4& { return ring[(2 * kt) % kRing]; },
                [&](int kt) -> const u32x4& { return ring[(2 * kt + 1) % kRing]; }, lds_addr(As + (size_t)lane * 8),
                lds_addr(ssw + r * NGG), lds_addr(ssw + Lay::SRM + r * NGG), 0u,
                acc0, acc1, [&](int kt) {
                    advance(wi, 2 * kt, 0, false);
                    advance(wi, 2 * kt + 1, 0, false);
                });
            if constexpr (WIDE) {
                if (tid == 0) lds_write_u32(tkL, tk_item(tkn));
                // every wave is past this item's gate/up (As reads) and the
                // previous item's down (Ad reads); the next item is known
                lds_barrier();
            } else {
                if (first) cand_resolve();
                if (wave == 0) {
                    const int nx = live_item((b - T) + n_more * PW);
                    if (lane == 0) lds_write_u32(tkL, nx);
                }
                ++n_more;
                lds_barrier();  // (also shares cm32 / tokmask)
            }
        };
        // The second half: act, the next item's scales and token rows, the
        // down phase. MORE: a next item nx exists.
        auto item_b = [&](int i, int nx, int pi, const StreamItem& cur, StreamItem& nxt, bool first, const f32x4& acc0,
                          const f32x4& acc1, auto more_tag) {
            constexpr bool MORE = decltype(more_tag)::value;
            fresh_indices();
            const int g = cur.g, s = cur.s, wi = cur.wi;
            int wnx = WIDE ? 0 : nx;  // the next item's weight index
            (void)i;
            {
                const int kl = 16 * wave + r;
                const int sp = kl >> 5, cp = (kl & 31) >> 3, ip = kl & 7;
                // every wave is past the previous item's down (Ad reads)
                if (!WIDE && !first) lds_barrier();
                if constexpr (WIDE && MORE) {
                    nxt = witem(nx);
                    wnx = nxt.wi;
                    x_rows(nxt.tok);
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int t = 4 * (lane >> 4) + q;
                    const float v = silu_mul_f(acc0[q], acc1[q]);
                    ovf |= t < cur.n && f16_overflow(v);
                    // asm write: a plain LDS access after the DMAs would make the
                    // compiler wait for every outstanding global load
                    const f16 hv = (f16)v;
                    asm volatile("ds_write_b16 %0, %1" ::"v"(lds_addr(Ad + ((size_t)sp * 64 + t + 16 * cp) * 8 + ip)),
                                 "v"(hv)
                                 : "memory");
                }
            }
            // the next item's gate/up scales (this wave's gate/up MMA is done)
            asm volatile("" ::: "memory");
            if constexpr (MORE) gu_scales(wnx);
            asm volatile("" ::: "memory");
            // this item's down scales and the previous item's partial stores:
            // older than the 2 * KTG unit loads of this gate/up phase (and the
            // next item's token rows and gate/up scales)
            wait_vm<2 * KTG + (WIDE && MORE ? NXD : 0)>();
            lds_barrier();  // Ad complete; every wave's older stores done
            // the previous item (no fence: the counter waits ordered its stores)
            if (!first && tid == 0) store_sc1(reinterpret_cast<int*>(sy->item_done + pi), (int)rtag);
            have_cand = true;
            const int tm = WIDE ? 0 : (g < E ? (int)lds_read_u32(tokmask + g) : (int)((1u << T) - 1u));
            // down: the act fragments (B operand) once for the item, then the
            // tile pairs; each consumed pair takes the next units of the ring.
            // A pair's partial rows of the candidate tokens are stored right
            // away (on the last item the loads after them are the last few ring
            // units, whose wait then includes those stores' acknowledgements,
            // which the final publish waits for anyway). Buffer stores whose
            // masked lanes carry an out-of-range offset (the hardware drops
            // them), so every wave issues the same stores on every path.
            f16x8 av[4];
            {
                const uint32_t aa = lds_addr(Ad + (size_t)lane * 8);
                asm volatile("ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:1024\n\t"
                             "ds_read_b128 %2, %4 offset:2048\n\tds_read_b128 %3, %4 offset:3072\n\ts_waitcnt lgkmcnt(0)"
                             : "=&v"(av[0]), "=&v"(av[1]), "=&v"(av[2]), "=&v"(av[3]) : "v"(aa) : "memory");
            }
            const int rq = 4 * (lane >> 4);  // the lane's first row in a tile
            const u32x4 prs = buffer_desc(a.y);
            const bool keep = WIDE ? r < cur.n : r < T && ((tm >> r) & 1);
            const size_t prow = WIDE ? ((size_t)(cur.row0 + r) * NS + s) : (((size_t)g * NS + s) * T + r);
            const int off0 = keep ? (int)((prow * H + wave * NTD * kTileRows + rq) * 4) : (int)0x80000000;
            auto store_pair = [&](int j, const f32x4& v0, const f32x4& v1) {
                store16_sc1(prs, keep ? off0 + j * kTileRows * 4 : off0, v0);
                store16_sc1(prs, keep ? off0 + (j + 1) * kTileRows * 4 : off0, v1);
            };
#pragma unroll
            for (int j = 0; j < NTD; j += 2) {
                f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
                down_pair<GPT, ZP, Lay::ZOFF_D>(ring[(2 * KTG + j) % kRing], ring[(2 * KTG + j + 1) % kRing], av,
                                                lds_addr(dsw + (j * 16 + rq) * GPT),
                                                lds_addr(dsw + ((j + 1) * 16 + rq) * GPT), lds_addr(dsw + (j * 16 + r) * GPT),
                                                lds_addr(dsw + ((j + 1) * 16 + r) * GPT), acc0, acc1);
                advance(wi, 2 * KTG + j, wnx, MORE);
                advance(wi, 2 * KTG + j + 1, wnx, MORE);
                store_pair(j, acc0, acc1);
            }
            // the next item's down scales (this wave's down MMA is done)
            asm volatile("" ::: "memory");
            if constexpr (MORE) dn_scales(wnx);
            asm volatile("" ::: "memory");
        };
        int i = i0;
        StreamItem cur = first_item, nxt = first_item;
        f32x4 acc0, acc1;
        int pi = -1;
        bool first = true;
        while (true) {
            item_a(cur, first, acc0, acc1);
            const int nx = __builtin_amdgcn_readfirstlane((int)lds_read_u32(tkL));  // (uniform: see NTOT)
            if (nx >= NTOT) break;
            item_b(i, nx, pi, cur, nxt, first, acc0, acc1, std::true_type{});
            pi = i;
            i = nx;
            if constexpr (WIDE) {
                cur = nxt;
            } else {
                cur = sitem(nx);
            }
            first = false;
        }
        item_b(i, NTOT, pi, cur, nxt, first, acc0, acc1, std::false_type{});
        report_f16_overflow(a.status, ovf);
        // the last item: its stores, then the step and its completion word
        store_fence();
        publish_now();
        if (tid == 0) store_sc1(reinterpret_cast<int*>(sy->item_done + i), (int)rtag);
      }
    }

    // ---- 3. combine units (token t, column block cb), one per workgroup from
    // the grid's end; the routers are the last to get one
    // (wide mode: CPU column blocks per unit, so that every workgroup has one
    // unit where the LDS for the unit's sums allows)
    const int NCB = (H + 127) / 128;
    const int CPU = WIDE ? max(1, min((NCB * T + P - 1) / P, (int)(Lay::as_bytes / (512 * (K + V))))) : 1;
    const int UPT = (NCB + CPU - 1) / CPU;  // units per token
    const int n_units = T * UPT;
    for (int u = P - 1 - b; u < n_units; u += P) {
        fresh_indices();
        const int t = u / UPT, cb = u % UPT;
        int* ids_c = misc;                                   // [K]
        float* wts_c = reinterpret_cast<float*>(misc + kMaxTopK);
        float* ys = reinterpret_cast<float*>(smem + Lay::o_ad);  // (K + 1) x 128 floats (Ad, Ds)
        if constexpr (WIDE) {
            if (!wide_ready) wide_setup();
            // the exact routing of token t
            wait_steps([&](int, int& owner, int& step) { owner = t; step = 1; }, 1);
            bool bad = false;
            // the partial rows and first items of token t's picks and of the
            // shared groups; an exact pick outside the token's candidates has
            // no rows (status bit 2, NaN output)
            if (wave == 0) {
                const int idl = lane < K ? load_cg(a.ids + (size_t)t * K + lane) : 0;
                const float wtl = lane < K ? load_cg(a.wts + (size_t)t * K + lane) : 0.0f;
                for (int jj = 0; jj < K + V; ++jj) {
                    const int g = jj < K ? __shfl(idl, jj, 64) : E + jj - K;
                    int slot = t;
                    if (jj < K) {
                        const uint64_t bal = __ballot((my_mask >> g) & 1);
                        slot = (int)__popcll(bal & ((1ull << t) - 1ull));
                        bad |= !((bal >> t) & 1);
                    }
                    const int tb = slot >> 4;
                    if (lane == 0) {
                        cuL[jj] = baseL[g] + slot;
                        cuL[kMaxTopK + kMaxExperts + jj] = tb == 0 ? g * NS : NI + (extL[g] + tb - 1) * NS;
                    }
                }
                if (lane < K) {
                    ids_c[lane] = idl;
                    wts_c[lane] = wtl;
                }
                if (lane == 0) {
                    misc[2 * kMaxTopK] = bad;
                    if (bad) __hip_atomic_fetch_or(a.status, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            __syncthreads();
            bad = misc[2 * kMaxTopK] != 0;
            const int* ib = cuL + kMaxTopK + kMaxExperts;
            if (wave == 0) {
                const int nq = (K + V) * NS;
                for (int q0 = 0; q0 < nq; q0 += 64) {
                    const int q = q0 + lane;
                    const bool want = q < nq;
                    const int i = want ? ib[q / NS] + q % NS : 0;
                    int it = 0;
                    while (__ballot(want && load_cg(sy->item_done + i) != rtag)) {
                        if (++it > kSpinLimit) {
                            if (lane == 0) report_timeout_to(a.status, sy, rtag);
                            break;
                        }
                        __builtin_amdgcn_s_sleep(1);
                    }
                }
            }
            __syncthreads();
            fence_wg_acquire();
            bad |= load_cg(&sy->call_fault) == rtag;
            const int c0 = cb * CPU * 128;
            stream_combine_wide<NS>(a, t, c0, min(H - c0, CPU * 128), wts_c, cuL, bad, reinterpret_cast<float*>(smem));
            continue;
        }
        need_cand();
        // the exact routing of token t
        wait_steps([&](int, int& owner, int& step) { owner = t; step = 1; }, 1);
        if (tid < K) {
            ids_c[tid] = load_cg(a.ids + (size_t)t * K + tid);
            wts_c[tid] = load_cg(a.wts + (size_t)t * K + tid);
        }
        __syncthreads();
        // the items of the picked groups and of the shared groups (a group no
        // token can pick has only its first-round items: an exact pick there
        // is outside the candidates, flagged below)
        if (wave == 0) {
            const int n_wait = (K + V) * NS;
            for (int q0 = 0; q0 < n_wait; q0 += 64) {
                const int q = q0 + lane;
                const int jj = q / NS, s = q % NS;
                const int g = q >= n_wait ? 0 : jj < K ? ids_c[jj] : E + (jj - K);
                const bool want = q < n_wait && (g >= E || g * NS + s < PW || (int)lds_read_u32(tokmask + g) != 0);
                const int i = g * NS + s;
                int it = 0;
                while (__ballot(want && load_cg(sy->item_done + i) != rtag)) {
                    if (++it > kSpinLimit) {
                        if (lane == 0) report_timeout_to(a.status, sy, rtag);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
        }
        __syncthreads();
        fence_wg_acquire();
        bool bad = load_cg(&sy->call_fault) == rtag;
        for (int j = 0; j < K; ++j) {
            const int id = ids_c[j];
            // an exact pick outside the candidates: its rows were not stored
            if (!((cm32[2 * t + (id >> 5)] >> (id & 31)) & 1u)) {
                if (tid == 0) __hip_atomic_fetch_or(a.status, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                bad = true;
            }
        }
        stream_combine<NS>(a, t, cb, ids_c, wts_c, nullptr, bad, ys);
    }

    // ---- leave: every workgroup ends the call at S + kFusedSteps
    __syncthreads();
    if (tid == 0) store_sc1(prog + b, S + kFusedSteps);
}

template <int GPT, int KTG, int KTD, bool ZP, bool WIDE, bool F32R>
static hipError_t launch_stream(const DecodeArgs& a, hipStream_t st) {
    using Lay = StreamLds<GPT, KTG, KTD, ZP>;
    constexpr size_t lds = Lay::bytes;
    static_assert(lds <= 160 * 1024, "stream kernel LDS");
    static_assert((KTG * kTileK / kTileRows) % kStreamWaves == 0 && Lay::NTD % 2 == 0, "down tiles per wave");
    auto kern = decode_stream_kernel<GPT, KTG, KTD, ZP, WIDE, F32R>;
    static hipError_t attr = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return attr;
    static int resident = [&] {
        int dev = 0, cus = 0, per_cu = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kStreamThreads, lds);
        return std::max(1, cus * std::max(1, per_cu));
    }();
    const int grid = std::min(resident, kFusedMaxGrid);
    if (grid <= a.seq) return hipErrorInvalidConfiguration;
    launch_k(kern, dim3(grid), dim3(kStreamThreads), (uint32_t)lds, st, a);
    return hipGetLastError();
}

bool decode_stream_ok(int hidden, int inter, int group) {
    return hidden == 1280 && inter == 896 && (group == 32 || group == 64 || group == 128);
}

bool decode_stream_wide(const DecodeArgs& a) { return a.seq > kStreamMaxSeq || a.rms_weight; }

// F32R: the layer's router is f32 (no bf16 copy): its own instantiation,
// since the f32 weights need twice the router registers
template <bool WIDE, bool F32R>
static hipError_t launch_stream_g(const DecodeArgs& a, hipStream_t st) {
    const bool zp = a.gate_z != nullptr;
    switch (a.group) {
        case 32:
            return zp ? launch_stream<4, 10, 7, true, WIDE, F32R>(a, st) : launch_stream<4, 10, 7, false, WIDE, F32R>(a, st);
        case 64:
            return zp ? launch_stream<2, 10, 7, true, WIDE, F32R>(a, st) : launch_stream<2, 10, 7, false, WIDE, F32R>(a, st);
        default:
            return zp ? launch_stream<1, 10, 7, true, WIDE, F32R>(a, st) : launch_stream<1, 10, 7, false, WIDE, F32R>(a, st);
    }
}

hipError_t launch_decode_stream(const DecodeArgs& a, hipStream_t st) {
    const bool wide = decode_stream_wide(a);
    if (a.seq < 1 || a.seq > (wide ? kStreamWideMaxSeq : kStreamMaxSeq) || !a.sync || !(a.router_t || a.router_f32) || !a.status)
        return hipErrorInvalidValue;
    // wide mode: the f16 expert input rows; with an RMSNorm the residual is the f32 input
    if (wide && (!a.x16 || (a.rms_weight && a.x_bf16))) return hipErrorInvalidValue;
    if (!a.down_skt || !a.sw || (a.gate_z && !a.down_zkt)) return hipErrorInvalidValue;
    if (a.n_experts + a.n_virtual > kMaxExperts || a.n_experts > 64 || a.top_k > kMaxTopK) return hipErrorInvalidValue;
    if (!decode_stream_ok(a.hidden, a.inter, a.group)) return hipErrorInvalidValue;
    if (!a.router_t) return wide ? launch_stream_g<true, true>(a, st) : launch_stream_g<false, true>(a, st);
    return wide ? launch_stream_g<true, false>(a, st) : launch_stream_g<false, false>(a, st);
}

}  // namespace uocr_hip
