// Decode-sized grouped INT4 expert kernels (bandwidth-bound) and the combine.
//
// Counterpart of the reference's masked expert pair
// (src/kernels/cuda/moe_device.cu:199-268, launched at :299-320), which re-reads
// each weight row once per assigned token. Here a wave owns one 16-row block
// of one expert's matrix, streams its tile-16x128 bytes once with 16-byte
// loads (1 KiB per wave instruction), unpacks the nibbles in registers, and
// multiplies them against the tile's tokens (up to 16 slots = one 16-row MFMA
// A operand) with v_mfma_f32_16x16x32_f16. Work items come from the
// device tile list, so the grid depends only on static shapes (graph-capturable);
// tiles beyond the live count exit at once.
#include "launch.hpp"

#if defined(UOCR_DECODE_PROFILE)
__device__ unsigned long long uocr_dbg_ts[4096 * 8];
extern "C" hipError_t uocr_dbg_read(void* host, size_t bytes) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(uocr_dbg_ts), bytes, 0, hipMemcpyDeviceToHost);
}
#define DBG_TS(i)                                                                                  \
    if (GU && threadIdx.x == 0) uocr_dbg_ts[(blockIdx.x + blockIdx.y * gridDim.x) * 8 + (i)] = wall_clock64();
#else
#define DBG_TS(i)
#endif

namespace uocr_hip {

constexpr int kDecodeBM = 16;

// Weight stream loads (read once per call). UOCR_NT_LOADS selects the
// non-temporal variant.
__device__ __forceinline__ u32x4 stream_load(const u32x4* p) {
#if defined(UOCR_NT_LOADS)
    return __builtin_nontemporal_load(p);
#else
    return *p;
#endif
}

// One workgroup = one m-tile (<= 16 slots of one expert) x 4 row blocks (one
// per wave). The activation rows and the wave's scale rows are copied straight
// into LDS with direct global->LDS loads (no registers); the activations land
// in MFMA A-fragment order (1 KiB per 16x32 fragment, lane-contiguous) for
// conflict-free reads. The wave's weight tiles stream into registers. All of
// it is issued before the first wait. Only live rows are loaded (rows beyond
// the tile's count only feed output rows that are never stored).
template <int GPT, int KT, bool GU>
__global__ __launch_bounds__(256) void experts_decode_kernel(ExpertArgs a) {
    constexpr int K = KT * kTileK;
    constexpr int NG = scale_row_stride(K, kTileK / GPT);  // padded groups per row
    constexpr int SROW = kTileRows * NG;                    // f16 scales per row block
    __shared__ __attribute__((aligned(16))) f16 As[KT * 4 * 64 * 8];
    __shared__ __attribute__((aligned(16))) f16 Ss[4][GU ? 2 : 1][SROW];
    DBG_TS(0)
    const int tile = blockIdx.x;
    // the tile list is sized for the worst case, so its entries can be read
    // together with the live count (one memory latency instead of two)
    const int n_tiles = *a.n_tiles;
    const int e = a.tile_e[tile], m0 = a.tile_m0[tile];
    DBG_TS(1)
    if (tile >= n_tiles) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int rb = blockIdx.y * 4 + wave;
    const bool wave_live = rb * kTileRows < a.n_rows;
    const int rows = min(kDecodeBM, a.counts[e] - m0);
    const int slot0 = a.offsets[e] + m0;
    const int r = lane & 15;

    // activations: this wave fills fragments (kt, s = wave) with row r = lane % 16
    if (r < rows) {
        const int row = a.gather ? a.slot_tok[slot0 + r] : slot0 + r;
        const f16* src = a.a + (size_t)row * K + wave * 32 + 8 * (lane >> 4);
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) load_lds16(src + kt * kTileK, As + (size_t)(kt * 4 + wave) * 64 * 8);
    }
    u32x4 bw0[KT], bw1[KT];
    if (wave_live) {
        // this wave's 16 scale rows are one contiguous block of SROW f16
        const size_t sb = (size_t)e * a.s_stride + (size_t)rb * SROW;
        for (int i = lane; i * 8 < SROW; i += 64) {
            load_lds16(a.s0 + sb + i * 8, &Ss[wave][0][(i & ~63) * 8]);
            if constexpr (GU) load_lds16(a.s1 + sb + i * 8, &Ss[wave][GU ? 1 : 0][(i & ~63) * 8]);
        }
        const size_t toff = (size_t)rb * KT * kTileBytes + (size_t)lane * 16;
        const uint8_t* w0 = a.w0 + (size_t)e * a.w_stride + toff;
        const uint8_t* w1 = GU ? a.w1 + (size_t)e * a.w_stride + toff : nullptr;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
            bw0[kt] = stream_load(reinterpret_cast<const u32x4*>(w0 + (size_t)kt * kTileBytes));
            if constexpr (GU) bw1[kt] = stream_load(reinterpret_cast<const u32x4*>(w1 + (size_t)kt * kTileBytes));
        }
    }
    DBG_TS(2)
    __builtin_amdgcn_s_waitcnt(0);  // direct-to-LDS data of this wave has landed
    __syncthreads();
    DBG_TS(3)
    if (!wave_live) return;

    const f16* srow0 = &Ss[wave][0][r * NG];
    const f16* srow1 = &Ss[wave][GU ? 1 : 0][r * NG];
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int g = kt * GPT + ((s * GPT) >> 2);  // group of MFMA step (kt, s)
            const f16x8 av = *reinterpret_cast<const f16x8*>(As + ((size_t)(kt * 4 + s) * 64 + lane) * 8);
            acc0 = mfma16(av, dequant8(bw0[kt][s], scale2(srow0[g])), acc0);
            if constexpr (GU) acc1 = mfma16(av, dequant8(bw1[kt][s], scale2(srow1[g])), acc1);
        }
    }

    const int col = rb * kTileRows + (lane & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = 4 * (lane >> 4) + i;
        if (m < rows) {
            const size_t o = (size_t)(slot0 + m) * a.n_rows + col;
            if constexpr (GU)
                a.act_out[o] = (f16)silu_mul_f(acc0[i], acc1[i]);
            else
                a.y_out[o] = acc0[i];
        }
    }
    DBG_TS(4)
}

// out[t] = residual[t] + (sum_j fma(w[t,j], y[pos[t,j]]) in j order) + shared(t)
// (src/engine/moe_decoder.cpp:88-97,111-112,179).
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs c) {
    const int t = blockIdx.x;
    const int H = c.hidden;
    for (int col = threadIdx.x * 4; col < H; col += blockDim.x * 4) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int j = 0; j < c.top_k; ++j) {
            const int slot = c.pos[(size_t)t * c.top_k + j];
            const float w = c.weights[(size_t)t * c.top_k + j];
            const f32x4 yv = *reinterpret_cast<const f32x4*>(c.y + (size_t)slot * H + col);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = fmaf(w, yv[i], acc[i]);
        }
        if (c.n_virtual > 0) {
            f32x4 sh = *reinterpret_cast<const f32x4*>(c.y + (size_t)(c.offsets[c.n_experts] + t) * H + col);
            for (int v = 1; v < c.n_virtual; ++v) {
                const f32x4 yv =
                    *reinterpret_cast<const f32x4*>(c.y + (size_t)(c.offsets[c.n_experts + v] + t) * H + col);
#pragma unroll
                for (int i = 0; i < 4; ++i) sh[i] += yv[i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += sh[i];
        }
        if (c.residual) {
            const f32x4 r = *reinterpret_cast<const f32x4*>(c.residual + (size_t)t * H + col);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = r[i] + acc[i];
        }
        *reinterpret_cast<f32x4*>(c.out + (size_t)t * H + col) = acc;
    }
}

template <int GPT, bool GU>
static hipError_t launch_decode_kt(const ExpertArgs& a, int max_tiles, hipStream_t st) {
    const dim3 grid(max_tiles, (a.n_rows / kTileRows + 3) / 4);
    const int kt = a.k / kTileK;
    switch (kt) {
        case 7: hipLaunchKernelGGL((experts_decode_kernel<GPT, 7, GU>), grid, dim3(256), 0, st, a); break;
        case 10: hipLaunchKernelGGL((experts_decode_kernel<GPT, 10, GU>), grid, dim3(256), 0, st, a); break;
        case 14: hipLaunchKernelGGL((experts_decode_kernel<GPT, 14, GU>), grid, dim3(256), 0, st, a); break;
        case 4: hipLaunchKernelGGL((experts_decode_kernel<GPT, 4, GU>), grid, dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL((experts_decode_kernel<GPT, 2, GU>), grid, dim3(256), 0, st, a); break;
        case 1: hipLaunchKernelGGL((experts_decode_kernel<GPT, 1, GU>), grid, dim3(256), 0, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <bool GU>
static hipError_t launch_decode_g(const ExpertArgs& a, int max_tiles, hipStream_t st) {
    switch (a.group) {
        case 32: return launch_decode_kt<4, GU>(a, max_tiles, st);
        case 64: return launch_decode_kt<2, GU>(a, max_tiles, st);
        case 128: return launch_decode_kt<1, GU>(a, max_tiles, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_experts_decode(const ExpertArgs& a, bool gate_up, int max_tiles, hipStream_t st) {
    if (max_tiles <= 0) return hipSuccess;
    return gate_up ? launch_decode_g<true>(a, max_tiles, st) : launch_decode_g<false>(a, max_tiles, st);
}

hipError_t launch_combine(const CombineArgs& c, hipStream_t st) {
    if (c.seq <= 0) return hipSuccess;
    hipLaunchKernelGGL(combine_kernel, dim3(c.seq), dim3(256), 0, st, c);
    return hipGetLastError();
}

}  // namespace uocr_hip
