// Prefill-sized grouped INT4 expert GEMM (MFMA-bound): dequantise the INT4
// weights into LDS-staged f16 tiles feeding v_mfma_f32_16x16x32_f16.
//
// Counterpart of the reference's grouped pair moe_grouped_gate_up_int4 /
// moe_grouped_down_int4 (src/kernels/cuda/moe_gemm_int4.cu:535-732), which
// stages bf16 panels for mma.sync m16n8k16. Here:
//   * work items are (m-tile of up to 128 grouped slots of one expert, n-tile)
//     taken from the device tile list, so skewed experts (Zipf routing) simply
//     own more m-tiles and every CU gets full 128-row tiles;
//   * a workgroup (4 waves, 2 x 2) computes 128 slots x 128 weight rows; the
//     fused gate/up pass pairs 64 gate rows with the same 64 up rows so SiLU(g)*u
//     is formed in registers and written once as f16 `act`;
//   * per 128-column k-tile, activation rows are copied global->LDS directly
//     (gathered through the slot->token list) and the 8 KiB of packed weights
//     are dequantised once per workgroup, exactly, into f16 fragments; both land
//     in MFMA fragment order (1 KiB per 16x32 fragment, lane-contiguous), so every
//     LDS read is a linear 1 KiB wave read.
#include <type_traits>
#include <utility>

#pragma once
#include "launch.hpp"

namespace uocr_hip {

// Global load issued by inline asm (the caller waits with vm_wait and tie):
// 16, 8 or 4 bytes by the destination's size, at byte offset OFF.
template <int OFF, typename T>
__device__ __forceinline__ void gload(T& d, const void* p) {
    if constexpr (sizeof(T) == 16)
        asm volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=v"(d) : "v"(p), "n"(OFF));
    else if constexpr (sizeof(T) == 8)
        asm volatile("global_load_dwordx2 %0, %1, off offset:%2" : "=v"(d) : "v"(p), "n"(OFF));
    else if constexpr (sizeof(T) == 4)
        asm volatile("global_load_dword %0, %1, off offset:%2" : "=v"(d) : "v"(p), "n"(OFF));
}
// 2 bytes, zero-extended
template <int OFF>
__device__ __forceinline__ void gload_u16(uint32_t& d, const void* p) {
    asm volatile("global_load_ushort %0, %1, off offset:%2" : "=v"(d) : "v"(p), "n"(OFF));
}
// wait until at most N global loads are outstanding
template <int N>
__device__ __forceinline__ void vm_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N));
}
// wait until at most N LDS operations are outstanding
template <int N>
__device__ __forceinline__ void lgkm_wait() {
    asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N));
}
// 16-byte LDS read issued by inline asm (waited for with lgkm_wait and tie)
template <int OFF>
__device__ __forceinline__ void lds_read16(f16x8& d, uint32_t addr) {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(d) : "v"(addr), "n"(OFF));
}
// 16-byte LDS write issued by inline asm
template <int OFF>
__device__ __forceinline__ void lds_write16(uint32_t addr, f16x8 v) {
    asm volatile("ds_write_b128 %0, %1 offset:%2" ::"v"(addr), "v"(v), "n"(OFF));
}
// the value is used only after this point (orders a use after a vm_wait)
template <typename T>
__device__ __forceinline__ void tie(T& v) {
    asm volatile("" : "+v"(v));
}

template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
// f(std::integral_constant<int, i>) for i = 0 .. N-1, in order
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

constexpr int kPreBM = 128;               // slots per m-tile (generic kernel)
constexpr int kPreBN = 128;               // weight rows per workgroup
constexpr int kBigBM = kPrefillBigTileRows; // slots per m-tile (large-tile kernel)
constexpr int kFragHalfs = 64 * 8;        // f16 per 1 KiB fragment

template <int GPT, bool GU, bool ZP>
__global__ __launch_bounds__(256) void experts_prefill_kernel(ExpertArgs a) {
    // A: 8 m-subtiles x 4 k-steps; B: 8 row blocks x 4 k-steps (fragments of 1 KiB)
    __shared__ __attribute__((aligned(16))) f16 As[8 * 4 * kFragHalfs];
    __shared__ __attribute__((aligned(16))) f16 Bs[8 * 4 * kFragHalfs];
    const int n_ntiles = GU ? (a.n_rows / (kPreBN / 2)) : (a.n_rows / kPreBN);
    const int tile = blockIdx.x / n_ntiles, ntile = blockIdx.x % n_ntiles;
    const int n_tiles = *a.n_tiles;
    const int e = a.tile_e[tile], m0 = a.tile_m0[tile];
    if (tile >= n_tiles) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int rows = min(kPreBM, a.counts[e] - m0);
    const int slot0 = a.offsets[e] + m0;
    const int K = a.k, KT = K / kTileK;
    const int NG = scale_row_stride(K, kTileK / GPT);

    // this wave's A rows for the DMA: m-subtiles (wave + 4i), row lane % 16
    const f16* arow[2];
    bool alive[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int m = (wave + 4 * i) * 16 + (lane & 15);
        alive[i] = m < rows;
        const int slot = slot0 + (alive[i] ? m : 0);
        const int row = a.gather ? a.slot_tok[slot] : slot;
        arow[i] = a.a + (size_t)row * K + 8 * (lane >> 4);
    }
    // this thread's B row blocks for the dequant: rb = wave and rb = wave + 4
    // (GU: 0..3 gate rows n0..n0+63, 4..7 the same up rows)
    const uint8_t* bsrc[2];
    const f16* ssrc[2];
    const f16* zsrc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int rbl = wave + 4 * i;
        int grow;  // global weight row block
        const uint8_t* wbase;
        const uint16_t* sbase;
        const uint16_t* zbase;
        if constexpr (GU) {
            grow = ntile * 4 + (rbl & 3);
            wbase = (rbl < 4 ? a.w0 : a.w1) + (size_t)e * a.w_stride;
            sbase = (rbl < 4 ? a.s0 : a.s1) + (size_t)e * a.s_stride;
            zbase = (rbl < 4 ? a.z0 : a.z1) + (size_t)e * a.s_stride;
        } else {
            grow = ntile * 8 + rbl;
            wbase = a.w0 + (size_t)e * a.w_stride;
            sbase = a.s0 + (size_t)e * a.s_stride;
            zbase = a.z0 + (size_t)e * a.s_stride;
        }
        bsrc[i] = wbase + (size_t)grow * KT * kTileBytes + (size_t)lane * 16;
        const size_t so = (size_t)(grow * kTileRows + (lane & 15)) * NG;
        ssrc[i] = reinterpret_cast<const f16*>(sbase) + so;
        zsrc[i] = ZP ? reinterpret_cast<const f16*>(zbase) + so : nullptr;
    }

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int kt = 0; kt < KT; ++kt) {
        // activations straight into LDS (fragment (msub, s) at ((msub * 4 + s) * 64 + lane) * 16 B)
#pragma unroll
        for (int i = 0; i < 2; ++i)
            if (alive[i]) {
                const int msub = wave + 4 * i;
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    load_lds16(arow[i] + kt * kTileK + s * 32, As + (size_t)(msub * 4 + s) * kFragHalfs);
            }
        // weights: 16 bytes per lane per row block -> four exact f16 fragments
        u32x4 wv[2];
        f16 sc[2][4], zc[2][4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            wv[i] = *reinterpret_cast<const u32x4*>(bsrc[i] + (size_t)kt * kTileBytes);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                sc[i][s] = ssrc[i][kt * GPT + ((s * GPT) >> 2)];
                if constexpr (ZP) zc[i][s] = zsrc[i][kt * GPT + ((s * GPT) >> 2)];
            }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int rbl = wave + 4 * i;
#pragma unroll
            for (int s = 0; s < 4; ++s)
                *reinterpret_cast<f16x8*>(Bs + ((size_t)(rbl * 4 + s) * 64 + lane) * 8) =
                    ZP ? dequant8z(wv[i][s], scale2(sc[i][s]), zc[i][s]) : dequant8(wv[i][s], scale2(sc[i][s]));
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            f16x8 af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                af[i] = *reinterpret_cast<const f16x8*>(As + ((size_t)((wm * 4 + i) * 4 + s) * 64 + lane) * 8);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                // GU: j = 0,1 gate row blocks 2wn, 2wn+1; j = 2,3 the matching up blocks
                const int rbl = GU ? ((j < 2) ? (2 * wn + j) : (4 + 2 * wn + (j - 2))) : (4 * wn + j);
                bf[j] = *reinterpret_cast<const f16x8*>(Bs + ((size_t)(rbl * 4 + s) * 64 + lane) * 8);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma16(af[i], bf[j], acc[i][j]);
        }
        __syncthreads();
    }

    // epilogue: lane holds C[m = msub*16 + 4*(lane/16) + r][n = nsub*16 + lane%16]
    bool ovf = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = (wm * 4 + i) * 16 + 4 * (lane >> 4) + r;
            if (m >= rows) continue;
            const size_t orow = (size_t)(slot0 + m) * a.n_rows;
            if constexpr (GU) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int col = ntile * 64 + wn * 32 + j * 16 + (lane & 15);
                    const float v = silu_mul_f(acc[i][j][r], acc[i][j + 2][r]);
                    ovf |= f16_overflow(v);
                    a.act_out[orow + col] = (f16)v;
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int col = ntile * kPreBN + wn * 64 + j * 16 + (lane & 15);
                    ovf |= f16_overflow(acc[i][j][r]);
                    a.y_out[orow + col] = (f16)acc[i][j][r];
                }
            }
        }
    }
    report_f16_overflow(a.status, ovf);
}

// ---------------------------------------------------------------------------
// Large-tile variant (K = 896 or 1280): 256 slots x 256 weight rows per
// workgroup, v_mfma_f32_32x32x16_f16 (the faster gfx950 f16 MFMA shape).
//   * the 4 waves stack along M (64 slots each) and each covers all 256 weight
//     rows (8 32-row blocks, 256 accumulator registers), so every activation
//     byte fetched from L2 feeds 256 output columns and every weight is
//     dequantised once per workgroup -- one dequant per 8 MFMAs -- into LDS in
//     32x32x16 B-fragment order, double-buffered one k-tile ahead;
//   * activation fragments are private to a wave, so they go global ->
//     registers (gathered through the slot->token list) one k-tile ahead and
//     never touch LDS;
//   * the k-tile loop is fully unrolled (exact waits) and blockIdx is remapped
//     so the n-tiles of one m-tile share an XCD's L2.
// Output layout of the 32x32x16 MFMA (verified on gfx950): lane l, register r
// holds C[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32].
// ---------------------------------------------------------------------------
constexpr int kBigBN = 256;  // weight rows per workgroup
constexpr int kBigNB = kBigBN / 32;
constexpr int kEpStride = 288;  // epilogue staging: bytes per row (256 + 32 of padding)

__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// lgkmcnt for the wait on B fragment f (f = k-step * 8 + 32-row block) of the
// large-tile k-loop: the ring's reads issued after it, f+1 .. f+3. Staging
// writes issued meanwhile are not counted: an LDS write can retire before an
// older read (measured: counting them as if LDS operations retired in issue
// order lets the wait pass early), while reads return in order among
// themselves. With the writes uncounted, the count cannot reach the limit
// before fragment f has landed, whatever the writes do.
constexpr int kRingAhead = 4;               // B fragments read ahead of their use
constexpr int kRing = kRingAhead + 2;       // register ring size
constexpr int lds_reads_after(int f) { return 63 - f < kRingAhead - 1 ? 63 - f : kRingAhead - 1; }

// DW: unquantised experts (the reference's BF16 expert format, uploaded as
// f16, row-major [rows][K], a.w_stride bytes per expert): the B fragments go
// global -> LDS by 16-byte DMA, one k-tile ahead, in the same fragment order
// (lane l of fragment (k-step, n-block): weight row n-block * 32 + l % 32,
// columns k-step * 16 + 8 * (l / 32) ..), so there is no dequantisation and no
// weight register; GPT and ZP are unused.
template <int GPT, bool GU, int KT, bool ZP, bool DW = false>
__global__ __launch_bounds__(256) void experts_prefill_big_kernel(ExpertArgs a) {
    // B fragments: [buffer][k-step 0..7][n-block 0..7][64 lanes][8 f16]
    __shared__ __attribute__((aligned(16))) f16 Bs[2][8 * kBigNB * kFragHalfs];
    constexpr int K = KT * kTileK;
    constexpr int NG = scale_row_stride(K, kTileK / GPT);
    constexpr int UNITS = kBigBN / kTileRows * 64 / 256;  // dequant units per thread (4)
    const int n_ntiles = GU ? (a.n_rows / (kBigBN / 2)) : (a.n_rows / kBigBN);
    const int b = blockIdx.x, xcd = b & 7, local = b >> 3;
    const int tile = (local / n_ntiles) * 8 + xcd, ntile = local % n_ntiles;
    const int n_tiles = *a.n_tiles;
    if (tile >= n_tiles) return;
    // one 16-byte record per tile: expert, first row, live rows, first slot
    const int4 ti = *reinterpret_cast<const int4*>(a.tile_info + 4 * tile);
    const int e = ti.x, rows = ti.z, slot0 = ti.w;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

    // A tile of at most 128 live rows runs in half mode: each wave takes 32
    // rows (JN = 1) instead of 64 (JN = 2), so it costs half the MFMAs and
    // activation loads; the tile list puts such tiles last so they fill the
    // grid's final round.
    auto body = [&](auto jnc) {
        constexpr int JN = decltype(jnc)::value;
        // A: wave rows wave*32*JN + j*32 + lane%32 (j < JN); k offset 8 * (lane / 32) in a k-step
        const f16* arow[JN];
        bool alive[JN];
#pragma unroll
        for (int j = 0; j < JN; ++j) {
            const int m = wave * 32 * JN + j * 32 + (lane & 31);
            alive[j] = m < rows;
            const int slot = slot0 + (alive[j] ? m : 0);
            const int row = a.gather ? a.slot_tok[slot] : slot;
            arow[j] = a.a + (size_t)row * K + 8 * (lane >> 5);
        }
        // B dequant units: u = tid + 256 i -> local row block rbl = u / 64, tile lane q = u % 64
        // (GU: row blocks 0..7 are gate rows of the n-tile's 128 act columns, 8..15 the same up rows)
        const uint8_t* bsrc[UNITS];
        const f16* ssrc[UNITS];
        // zero offsets sit at the same index of the zero array (ZP layers)
        const ptrdiff_t zdelta = ZP ? (GU ? 0 : a.z0 - a.s0) : 0;
#pragma unroll
        for (int i = 0; i < UNITS; ++i) {
            const int u = tid + 256 * i, rbl = u >> 6, q = u & 63;
            int grow;
            const uint8_t* wbase;
            const uint16_t* sbase;
            if constexpr (GU) {
                grow = ntile * 8 + (rbl & 7);
                wbase = (rbl < 8 ? a.w0 : a.w1) + (size_t)e * a.w_stride;
                sbase = (rbl < 8 ? a.s0 : a.s1) + (size_t)e * a.s_stride;
            } else {
                grow = ntile * 16 + rbl;
                wbase = a.w0 + (size_t)e * a.w_stride;
                sbase = a.s0 + (size_t)e * a.s_stride;
            }
            bsrc[i] = wbase + (size_t)grow * KT * kTileBytes + (size_t)q * 16;
            ssrc[i] = reinterpret_cast<const f16*>(sbase) + (size_t)(grow * kTileRows + (q & 15)) * NG;
        }
        // gate/up: unit i's matrix is gate for i < UNITS / 2 (row blocks 0..7), up after
        auto zsrc_of = [&](int i) -> const f16* {
            if constexpr (GU) return ssrc[i] + (i < UNITS / 2 ? a.z0 - a.s0 : a.z1 - a.s1);
            else return ssrc[i] + zdelta;
        };
        // LDS destination of unit i's 8-column run s (columns s*32 + 8*(q/16) ..
        // +7 of local weight row n = (wave + 4i) * 16 + q % 16, in 32x32x16
        // B-fragment order): byte offset bdst0 + s * 16384 + i * 2048
        uint32_t bdst0;
        {
            const int n = wave * 16 + (lane & 15), q4 = lane >> 4;
            bdst0 = (uint32_t)((((q4 >> 1) * kBigNB + (n >> 5)) * 64 + (n & 31) + 32 * (q4 & 1)) * 16);
        }
        // DW: this wave DMAs the fragments of n-blocks 2 * wave and 2 * wave + 1
        // (all 8 k-steps); the lane's row of each and its first column
        const f16* drow[2];
        if constexpr (DW) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int n = (2 * wave + h) * 32 + (lane & 31);  // local weight row
                const f16* base;
                int grow;
                if constexpr (GU) {
                    base = reinterpret_cast<const f16*>((n < kBigBN / 2 ? a.w0 : a.w1) + (size_t)e * a.w_stride);
                    grow = ntile * (kBigBN / 2) + (n & (kBigBN / 2 - 1));
                } else {
                    base = reinterpret_cast<const f16*>(a.w0 + (size_t)e * a.w_stride);
                    grow = ntile * kBigBN + n;
                }
                drow[h] = base + (size_t)grow * K + 8 * (lane >> 5);
            }
        }

        // The k-tile pipeline keeps its own load schedule: every global load is
        // issued by inline asm at a fixed point and every wait is an explicit
        // vmcnt tied to the registers it guards. Left to itself the compiler sinks
        // the prefetches to their first use under this register pressure, so each
        // wait also covers the loads just issued and the pipeline loses its depth.
        //   * activations: one register pair per k-step (a ring over the k-tile);
        //     the pair of k-step ks is reloaded with k-tile kt+1's columns right
        //     after k-tile kt's MFMAs have read it, so every load has most of a
        //     k-tile to land;
        //   * weights: B(kt+2) (UNITS weight loads, then UNITS scale loads) at the
        //     start of k-tile kt, staged into LDS during k-tile kt+1.
        // Issue order within k-tile kt: B(kt+2), then A(kt+1, ks) after k-step ks.
        constexpr int AK = JN;         // activation loads per k-step
        constexpr int NB = DW ? 16 : (ZP ? 3 : 2) * UNITS;  // loads (DW: DMAs) per k-tile of weights
        u32x4 braw[2][UNITS];
        typename std::conditional<GPT == 4, u32x2, uint32_t>::type bscr[2][UNITS], bzr[2][UNITS];
        f16x8 areg[JN][8];
        f16x8 bring[kRing];
        auto issue_a = [&](auto ktc, auto ksc) {
            constexpr int kt = decltype(ktc)::value, ks = decltype(ksc)::value;
#pragma unroll
            for (int j = 0; j < JN; ++j) {
                gload<kt * kTileK * 2 + ks * 32>(areg[j][ks], arow[j]);
            }
        };
        // DW: the 16 fragment DMAs of k-tile kt into buffer kt & 1
        auto issue_bd = [&](auto ktc) {
            constexpr int kt = decltype(ktc)::value;
#pragma unroll
            for (int ks = 0; ks < 8; ++ks)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    load_lds16(drow[h] + kt * kTileK + ks * 16,
                               reinterpret_cast<uint8_t*>(&Bs[kt & 1][0]) + (ks * kBigNB + 2 * wave + h) * 1024);
        };
        auto issue_b = [&](auto ktc) {
            constexpr int kt = decltype(ktc)::value;
#pragma unroll
            for (int i = 0; i < UNITS; ++i) {
                gload<0>(braw[kt & 1][i], bsrc[i] + (size_t)kt * kTileBytes);
            }
#pragma unroll
            for (int i = 0; i < UNITS; ++i) {
                if constexpr (GPT == 1)
                    gload_u16<kt * 2>(bscr[kt & 1][i], ssrc[i]);
                else
                    gload<kt * GPT * 2>(bscr[kt & 1][i], ssrc[i]);
            }
            if constexpr (ZP) {
#pragma unroll
                for (int i = 0; i < UNITS; ++i) {
                    if constexpr (GPT == 1)
                        gload_u16<kt * 2>(bzr[kt & 1][i], zsrc_of(i));
                    else
                        gload<kt * GPT * 2>(bzr[kt & 1][i], zsrc_of(i));
                }
            }
        };
        // wait until at most N loads are outstanding, then let the guarded values be used
        auto wait_a = [&](auto nc, int ks) {
            vm_wait<decltype(nc)::value>();
#pragma unroll
            for (int j = 0; j < JN; ++j) tie(areg[j][ks]);
        };
        auto wait_b = [&](auto nc, int buf) {
            vm_wait<decltype(nc)::value>();
#pragma unroll
            for (int i = 0; i < UNITS; ++i) {
                tie(braw[buf][i]);
                tie(bscr[buf][i]);
                if constexpr (ZP) tie(bzr[buf][i]);
            }
        };
        auto word_of = [&](const auto& words, int buf, int i, int s) -> f16 {
            const int g = (s * GPT) >> 2;  // group within the k-tile
            uint32_t w;
            if constexpr (GPT == 4) w = words[buf][i][g >> 1];
            else w = words[buf][i];
            const uint16_t h = (uint16_t)((g & 1) ? (w >> 16) : (w & 0xffffu));
            return __builtin_bit_cast(f16, h);
        };
        // dequantise run s (8 columns) of unit i of k-tile kt into its LDS buffer
        auto stage_run = [&](int kt, auto ic, auto sc) {
            constexpr int i = decltype(ic)::value, s = decltype(sc)::value;
            const uint32_t dst = lds_addr(Bs[kt & 1]) + bdst0;
            const f16 scl = word_of(bscr, kt & 1, i, s);
            if constexpr (ZP)
                lds_write16<s * 16384 + i * 2048>(dst, dequant8z(braw[kt & 1][i][s], scale2(scl), word_of(bzr, kt & 1, i, s)));
            else
                lds_write16<s * 16384 + i * 2048>(dst, dequant8(braw[kt & 1][i][s], scale2(scl)));
        };

        f32x16 acc[JN][kBigNB];
#pragma unroll
        for (int j = 0; j < JN; ++j)
#pragma unroll
            for (int nb = 0; nb < kBigNB; ++nb) acc[j][nb] = f32x16{};

        if constexpr (DW) {
            // prologue: B(0) by DMA, A(0); B(0) landed in every wave's part
            issue_bd(std::integral_constant<int, 0>{});
            static_for<8>([&](auto ksc) { issue_a(std::integral_constant<int, 0>{}, ksc); });
            vm_wait<8 * AK>();
        } else {
            // prologue: B(0), B(1), A(0); stage B(0)
            issue_b(std::integral_constant<int, 0>{});
            if constexpr (KT > 1) issue_b(std::integral_constant<int, 1>{});
            static_for<8>([&](auto ksc) { issue_a(std::integral_constant<int, 0>{}, ksc); });
            wait_b(std::integral_constant<int, (KT > 1 ? NB : 0) + 8 * AK>{}, 0);
            static_for<UNITS>([&](auto ic) { static_for<4>([&](auto sc) { stage_run(0, ic, sc); }); });
            lgkm_wait<0>();
        }
        __syncthreads();
        static_for<KT>([&](auto ktc) {
            constexpr int kt = decltype(ktc)::value;
            constexpr bool more = kt + 1 < KT;
            // weight loads issued after A(kt, *) and before A(kt + 1, *): DW the
            // DMAs of B(kt + 1) (into the buffer the last k-tile read), else B(kt + 2)
            constexpr int nB2 = DW ? (more ? NB : 0) : (kt + 2 < KT ? NB : 0);
            if constexpr (DW) {
                if constexpr (more) issue_bd(std::integral_constant<int, kt + 1>{});
            } else {
                if constexpr (kt + 2 < KT) issue_b(std::integral_constant<int, kt + 2>{});
            }
            // B fragments stream from LDS through a 6-deep register ring, read
            // 4 fragments (8 MFMAs) ahead of their use: fragment f = ks * 8 + nb
            const uint32_t bb = lds_addr(Bs[kt & 1]) + lane * 16;
            static_for<kRingAhead>([&](auto fc) { lds_read16<decltype(fc)::value * 1024>(bring[decltype(fc)::value], bb); });
            static_for<8 * kBigNB>([&](auto fc) {
                constexpr int f = decltype(fc)::value, ks = f / kBigNB, nb = f % kBigNB;
                if constexpr (nb == 0)  // A(kt, ks) was issued before A(kt, ks+1 .. 7), B(kt+2) and A(kt+1, 0 .. ks-1)
                    wait_a(std::integral_constant<int, AK * (7 - ks) + nB2 + (more ? AK * ks : 0)>{}, ks);
                lgkm_wait<lds_reads_after(f)>();
                tie(bring[f % kRing]);
#pragma unroll
                for (int j = 0; j < JN; ++j) acc[j][nb] = mfma32(areg[j][ks], bring[f % kRing], acc[j][nb]);
                if constexpr (f + kRingAhead < 8 * kBigNB)
                    lds_read16<(f + kRingAhead) * 1024>(bring[(f + kRingAhead) % kRing], bb);
                if constexpr (nb == kBigNB - 1 && more)
                    issue_a(std::integral_constant<int, kt + 1>{}, std::integral_constant<int, ks>{});
                // next k-tile's weights go to the other buffer (last read before the
                // previous barrier): one 8-column run (one dequant8, one LDS write)
                // every third fragment from fragment 8 on, so the VALU work
                // interleaves with the MFMAs in flight
                constexpr int run = (f - 8) / 3;
                if constexpr (!DW && more && f >= 8 && (f - 8) % 3 == 0 && run < 4 * UNITS) {
                    // B(kt+1) was issued before A(kt), B(kt+2) and A(kt+1, 0)
                    if constexpr (run == 0) wait_b(std::integral_constant<int, 8 * AK + nB2 + AK>{}, (kt + 1) & 1);
                    stage_run(kt + 1, std::integral_constant<int, run / 4>{}, std::integral_constant<int, run % 4>{});
                }
            });
            lgkm_wait<0>();  // this k-tile's staging writes (asm, not tracked by the compiler)
            // DW: B(kt + 1)'s DMAs, older than A(kt + 1, *), have landed
            if constexpr (DW && more) vm_wait<8 * AK>();
            __syncthreads();
        });

        // Epilogue: each wave stages its 32*JN output rows in LDS, row-major
        // with a 288-byte row stride (rows 4 apart land 32 banks apart), then
        // every lane stores 16 contiguous bytes: one store instruction covers
        // 4 rows x 256 bytes. The k-loop's last barrier has retired every read
        // of Bs, and each wave only touches its own region.
        uint8_t* ep = reinterpret_cast<uint8_t*>(&Bs[0][0]) + wave * (64 * kEpStride);
        const int er = lane >> 4, ec = (lane & 15) * 16;  // store lane: row within 4, byte column
        auto stage_rows = [&](auto write_vals) {
#pragma unroll
            for (int j = 0; j < JN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    write_vals(j, r, ep + (j * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * kEpStride);
        };
        bool ovf = false;
        if constexpr (GU) {
            stage_rows([&](int j, int r, uint8_t* row) {
#pragma unroll
                for (int nb = 0; nb < kBigNB / 2; ++nb)
                    reinterpret_cast<f16*>(row)[nb * 32 + (lane & 31)] =
                        (f16)silu_mul_f(acc[j][nb][r], acc[j][nb + kBigNB / 2][r]);
            });
#pragma unroll
            for (int i = 0; i < 8 * JN; ++i) {
                const int m = wave * 32 * JN + i * 4 + er;
                const u32x4 v = *reinterpret_cast<const u32x4*>(ep + (i * 4 + er) * kEpStride + ec);
                // an f16 with an all-ones exponent: the value left f16's range
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    ovf |= m < rows && ((v[q] & 0x7c00u) == 0x7c00u || (v[q] & 0x7c000000u) == 0x7c000000u);
                if (m < rows)
                    *reinterpret_cast<u32x4*>(a.act_out + (size_t)(slot0 + m) * a.n_rows + ntile * (kBigBN / 2) + ec / 2) = v;
            }
        } else {
            // 64 output columns per pass
#pragma unroll
            for (int pass = 0; pass < kBigNB / 2; ++pass) {
                stage_rows([&](int j, int r, uint8_t* row) {
#pragma unroll
                    for (int q = 0; q < 2; ++q)
                        reinterpret_cast<float*>(row)[q * 32 + (lane & 31)] = acc[j][2 * pass + q][r];
                });
#pragma unroll
                for (int i = 0; i < 8 * JN; ++i) {
                    const int m = wave * 32 * JN + i * 4 + er;
                    const f32x4 v = *reinterpret_cast<const f32x4*>(ep + (i * 4 + er) * kEpStride + ec);
                    // f16 rows (8 bytes per lane, 128 contiguous bytes per row)
                    const f16x4 h = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
                    ovf |= m < rows && (f16_overflow(v[0]) || f16_overflow(v[1]) || f16_overflow(v[2]) ||
                                        f16_overflow(v[3]));
                    if (m < rows)
                        *reinterpret_cast<f16x4*>(a.y_out + (size_t)(slot0 + m) * a.n_rows + ntile * kBigBN + pass * 64 +
                                                  ec / 4) = h;
                }
            }
        }
        report_f16_overflow(a.status, ovf);
    };
    if (rows <= kBigBM / 2)
        body(std::integral_constant<int, 1>{});
    else
        body(std::integral_constant<int, 2>{});
}

template <int GPT, bool GU, bool ZP>
static bool launch_big(const ExpertArgs& a, int max_tiles, hipStream_t st) {
    const int n_ntiles = GU ? (a.n_rows / (kBigBN / 2)) : (a.n_rows / kBigBN);
    if (n_ntiles * (GU ? kBigBN / 2 : kBigBN) != a.n_rows) return false;
    const dim3 grid(((max_tiles + 7) / 8) * 8 * n_ntiles);
    switch (a.k / kTileK) {
        case 7: launch_k((experts_prefill_big_kernel<GPT, GU, 7, ZP>), grid, dim3(256), 0, st, a); return true;
        case 10: launch_k((experts_prefill_big_kernel<GPT, GU, 10, ZP>), grid, dim3(256), 0, st, a); return true;
        default: return false;
    }
}

template <bool GU, bool ZP>
static hipError_t launch_prefill_g(const ExpertArgs& a, int max_tiles, hipStream_t st) {
    const int n_ntiles = GU ? (a.n_rows / (kPreBN / 2)) : (a.n_rows / kPreBN);
    const dim3 grid(max_tiles * n_ntiles);
    if (a.bm == kBigBM) {
        bool done = false;
        switch (a.group) {
            case 32: done = launch_big<4, GU, ZP>(a, max_tiles, st); break;
            case 64: done = launch_big<2, GU, ZP>(a, max_tiles, st); break;
            case 128: done = launch_big<1, GU, ZP>(a, max_tiles, st); break;
            default: return hipErrorInvalidValue;
        }
        return done ? hipGetLastError() : hipErrorInvalidValue;
    }
    if (a.bm != kPreBM) return hipErrorInvalidValue;
    switch (a.group) {
        case 32: launch_k((experts_prefill_kernel<4, GU, ZP>), grid, dim3(256), 0, st, a); break;
        case 64: launch_k((experts_prefill_kernel<2, GU, ZP>), grid, dim3(256), 0, st, a); break;
        case 128: launch_k((experts_prefill_kernel<1, GU, ZP>), grid, dim3(256), 0, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace uocr_hip
