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
#include "launch.hpp"

namespace uocr_hip {

constexpr int kPreBM = kPrefillTileRows;  // 128 slots per m-tile
constexpr int kPreBN = 128;               // weight rows per workgroup
constexpr int kFragHalfs = 64 * 8;        // f16 per 1 KiB fragment

template <int GPT, bool GU>
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
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int rbl = wave + 4 * i;
        int grow;  // global weight row block
        const uint8_t* wbase;
        const f16* sbase;
        if constexpr (GU) {
            grow = ntile * 4 + (rbl & 3);
            wbase = (rbl < 4 ? a.w0 : a.w1) + (size_t)e * a.w_stride;
            sbase = reinterpret_cast<const f16*>(rbl < 4 ? a.s0 : a.s1) + (size_t)e * a.s_stride;
        } else {
            grow = ntile * 8 + rbl;
            wbase = a.w0 + (size_t)e * a.w_stride;
            sbase = reinterpret_cast<const f16*>(a.s0) + (size_t)e * a.s_stride;
        }
        bsrc[i] = wbase + (size_t)grow * KT * kTileBytes + (size_t)lane * 16;
        ssrc[i] = sbase + (size_t)(grow * kTileRows + (lane & 15)) * NG;
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
        f16 sc[2][4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            wv[i] = *reinterpret_cast<const u32x4*>(bsrc[i] + (size_t)kt * kTileBytes);
#pragma unroll
            for (int s = 0; s < 4; ++s) sc[i][s] = ssrc[i][kt * GPT + ((s * GPT) >> 2)];
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int rbl = wave + 4 * i;
#pragma unroll
            for (int s = 0; s < 4; ++s)
                *reinterpret_cast<f16x8*>(Bs + ((size_t)(rbl * 4 + s) * 64 + lane) * 8) =
                    dequant8(wv[i][s], scale2(sc[i][s]));
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
                    a.act_out[orow + col] = (f16)silu_mul_f(acc[i][j][r], acc[i][j + 2][r]);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int col = ntile * kPreBN + wn * 64 + j * 16 + (lane & 15);
                    a.y_out[orow + col] = acc[i][j][r];
                }
            }
        }
    }
}

template <bool GU>
static hipError_t launch_prefill_g(const ExpertArgs& a, int max_tiles, hipStream_t st) {
    const int n_ntiles = GU ? (a.n_rows / (kPreBN / 2)) : (a.n_rows / kPreBN);
    const dim3 grid(max_tiles * n_ntiles);
    switch (a.group) {
        case 32: hipLaunchKernelGGL((experts_prefill_kernel<4, GU>), grid, dim3(256), 0, st, a); break;
        case 64: hipLaunchKernelGGL((experts_prefill_kernel<2, GU>), grid, dim3(256), 0, st, a); break;
        case 128: hipLaunchKernelGGL((experts_prefill_kernel<1, GU>), grid, dim3(256), 0, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_experts_prefill(const ExpertArgs& a, bool gate_up, int max_tiles, hipStream_t st) {
    if (max_tiles <= 0) return hipSuccess;
    if ((gate_up && a.n_rows % (kPreBN / 2)) || (!gate_up && a.n_rows % kPreBN)) return hipErrorInvalidValue;
    return gate_up ? launch_prefill_g<true>(a, max_tiles, st) : launch_prefill_g<false>(a, max_tiles, st);
}

}  // namespace uocr_hip
