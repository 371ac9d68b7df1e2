// Decode-sized grouped INT4 expert kernels (bandwidth-bound) and the combine.
//
// Counterpart of the reference's masked expert pair
// (src/kernels/cuda/moe_device.cu:199-268, launched at :299-320), which re-reads
// each weight row once per assigned token. Here a wave owns one 16-row block
// of one expert's matrix, streams its tile-16x128 bytes once with 16-byte
// loads (1 KiB per wave instruction), unpacks the nibbles in registers, and
// multiplies them against ALL of that expert's tokens (up to 64 slots = four
// 16-row MFMA A tiles) with v_mfma_f32_16x16x32_f16. Work items come from the
// device tile list, so the grid depends only on static shapes (graph-capturable);
// tiles beyond the live count exit at once.
#include "launch.hpp"

namespace uocr_hip {

constexpr int kDecodeBM = 64;

template <int GPT>
__device__ __forceinline__ uint32_t scale_bits(const uint16_t* sp, int s) {
    // group index inside the 128-column tile for MFMA step s
    return sp[(s * GPT) >> 2];
}

template <int GPT, int KT, bool GU>
__global__ __launch_bounds__(256) void experts_decode_kernel(ExpertArgs a) {
    const int tile = blockIdx.x;
    if (tile >= *a.n_tiles) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rb = blockIdx.y * 4 + wave;
    if (rb * kTileRows >= a.n_rows) return;
    const int e = a.tile_e[tile], m0 = a.tile_m0[tile];
    const int rows = min(kDecodeBM, a.counts[e] - m0);
    const int slot0 = a.offsets[e] + m0;
    const int K = KT * kTileK;
    const int nsub = (rows + 15) >> 4;

    const size_t toff = (size_t)rb * KT * kTileBytes + (size_t)lane * 16;
    const uint8_t* w0 = a.w0 + (size_t)e * a.w_stride + toff;
    const uint8_t* w1 = GU ? a.w1 + (size_t)e * a.w_stride + toff : nullptr;
    const size_t soff = (size_t)rb * KT * kTileRows * GPT + (size_t)(lane & 15) * GPT;
    const uint16_t* s0 = a.s0 + (size_t)e * a.s_stride + soff;
    const uint16_t* s1 = GU ? a.s1 + (size_t)e * a.s_stride + soff : nullptr;

    const f16* arow[4];
    bool aval[4];
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
        const int m = sub * 16 + (lane & 15);
        aval[sub] = m < rows;
        const int slot = slot0 + (aval[sub] ? m : 0);
        const int row = a.gather ? a.slot_tok[slot] : slot;
        arow[sub] = a.a + (size_t)row * K + 8 * (lane >> 4);
    }

    // issue every weight load of the wave up front
    u32x4 bw0[KT], bw1[KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
        bw0[kt] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(w0 + (size_t)kt * kTileBytes));
        if constexpr (GU)
            bw1[kt] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(w1 + (size_t)kt * kTileBytes));
    }

    f32x4 acc0[4], acc1[4];
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
        acc0[sub] = f32x4{0.f, 0.f, 0.f, 0.f};
        acc1[sub] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const f16x8 zero8 = {};

#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
        const uint16_t* sp0 = s0 + kt * kTileRows * GPT;
        const uint16_t* sp1 = GU ? s1 + kt * kTileRows * GPT : nullptr;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const f16x8 b0 = dequant8(bw0[kt][s], scale2(scale_bits<GPT>(sp0, s)));
            f16x8 b1;
            if constexpr (GU) b1 = dequant8(bw1[kt][s], scale2(scale_bits<GPT>(sp1, s)));
#pragma unroll
            for (int sub = 0; sub < 4; ++sub) {
                if (sub < nsub) {
                    const f16x8 av =
                        aval[sub] ? *reinterpret_cast<const f16x8*>(arow[sub] + kt * kTileK + s * 32) : zero8;
                    acc0[sub] = mfma16(av, b0, acc0[sub]);
                    if constexpr (GU) acc1[sub] = mfma16(av, b1, acc1[sub]);
                }
            }
        }
    }

    const int col = rb * kTileRows + (lane & 15);
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
        if (sub < nsub) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = sub * 16 + 4 * (lane >> 4) + i;
                if (m < rows) {
                    const size_t o = (size_t)(slot0 + m) * a.n_rows + col;
                    if constexpr (GU)
                        a.act_out[o] = (f16)silu_mul_f(acc0[sub][i], acc1[sub][i]);
                    else
                        a.y_out[o] = acc0[sub][i];
                }
            }
        }
    }
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
