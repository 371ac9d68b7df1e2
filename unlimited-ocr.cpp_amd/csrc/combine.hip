// Combine of the prefill path: out[t] = residual + weighted routed rows +
// shared-expert rows, from the grouped [slots, hidden] expert outputs.
#include <algorithm>

#include "launch.hpp"

namespace uocr_hip {

// out[t] = residual[t] + (sum_j fma(w[t,j], y[pos[t,j]]) in j order) + shared(t)
// (src/engine/moe_decoder.cpp:88-97,111-112,179); the y rows are f16, widened
// exactly, and every sum is in f32. One thread per 8 columns (16-byte y
// loads), kCombineTok tokens per workgroup.
constexpr int kCombineTok = 2;

__device__ __forceinline__ void load_y8(const f16* p, float* v) {
    const f16x8 h = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)h[i];
}

__global__ __launch_bounds__(1024) void combine_kernel(CombineArgs c) {
    const int H = c.hidden;
    const int per_tok = H / 8;  // threads of one token
    const int t = blockIdx.x * kCombineTok + threadIdx.x / per_tok;
    const int col = (threadIdx.x % per_tok) * 8;
    if (t >= c.seq || threadIdx.x >= kCombineTok * per_tok) return;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < c.top_k; ++j) {
        const int slot = c.pos[(size_t)t * c.top_k + j];
        const float w = c.weights[(size_t)t * c.top_k + j];
        float yv[8];
        load_y8(c.y + (size_t)slot * H + col, yv);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = fmaf(w, yv[i], acc[i]);
    }
    if (c.n_virtual > 0) {
        float sh[8];
        load_y8(c.y + (size_t)(c.offsets[c.n_experts] + t) * H + col, sh);
        for (int v = 1; v < c.n_virtual; ++v) {
            float yv[8];
            load_y8(c.y + (size_t)(c.offsets[c.n_experts + v] + t) * H + col, yv);
#pragma unroll
            for (int i = 0; i < 8; ++i) sh[i] += yv[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += sh[i];
    }
    if (c.shared_y) {
        const f32x4 s0 = *reinterpret_cast<const f32x4*>(c.shared_y + (size_t)t * H + col);
        const f32x4 s1 = *reinterpret_cast<const f32x4*>(c.shared_y + (size_t)t * H + col + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[i] += s0[i];
            acc[4 + i] += s1[i];
        }
    }
    if (c.residual) {
        const f32x4 r0 = *reinterpret_cast<const f32x4*>(c.residual + (size_t)t * H + col);
        const f32x4 r1 = *reinterpret_cast<const f32x4*>(c.residual + (size_t)t * H + col + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[i] = r0[i] + acc[i];
            acc[4 + i] = r1[i] + acc[4 + i];
        }
    }
    *reinterpret_cast<f32x4*>(c.out + (size_t)t * H + col) = f32x4{acc[0], acc[1], acc[2], acc[3]};
    *reinterpret_cast<f32x4*>(c.out + (size_t)t * H + col + 4) = f32x4{acc[4], acc[5], acc[6], acc[7]};
}

hipError_t launch_combine(const CombineArgs& c, hipStream_t st) {
    if (c.seq <= 0) return hipSuccess;
    if (c.hidden % 8 || c.hidden / 8 * kCombineTok > 1024) return hipErrorInvalidValue;
    const int threads = ((c.hidden / 8 * kCombineTok + 63) / 64) * 64;
    launch_k(combine_kernel, dim3((c.seq + kCombineTok - 1) / kCombineTok), dim3(threads), 0, st, c);
    return hipGetLastError();
}

}  // namespace uocr_hip
