// Combine of the prefill path: out[t] = residual + weighted routed rows +
// shared-expert rows, from the grouped [slots, hidden] expert outputs.
#include <algorithm>

#include "launch.hpp"

namespace uocr_hip {

// out[t] = residual[t] + (sum_j fma(w[t,j], y[pos[t,j]]) in j order) + shared(t)
// (src/engine/moe_decoder.cpp:88-97,111-112,179); the y rows are f16, widened
// exactly, and every sum is in f32.
__device__ __forceinline__ f32x4 load_y4(const f16* p) {
    const f16x4 h = *reinterpret_cast<const f16x4*>(p);
    return f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
}

__global__ __launch_bounds__(1024) void combine_kernel(CombineArgs c) {
    const int t = blockIdx.x;
    const int H = c.hidden;
    for (int col = threadIdx.x * 4; col < H; col += blockDim.x * 4) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int j = 0; j < c.top_k; ++j) {
            const int slot = c.pos[(size_t)t * c.top_k + j];
            const float w = c.weights[(size_t)t * c.top_k + j];
            const f32x4 yv = load_y4(c.y + (size_t)slot * H + col);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = fmaf(w, yv[i], acc[i]);
        }
        if (c.n_virtual > 0) {
            f32x4 sh = load_y4(c.y + (size_t)(c.offsets[c.n_experts] + t) * H + col);
            for (int v = 1; v < c.n_virtual; ++v) {
                const f32x4 yv = load_y4(c.y + (size_t)(c.offsets[c.n_experts + v] + t) * H + col);
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

hipError_t launch_combine(const CombineArgs& c, hipStream_t st) {
    if (c.seq <= 0) return hipSuccess;
    // one 16-byte column group per thread, the whole row in one pass
    // (hidden / 4 threads rounded up to whole waves, at most 1024)
    const int threads = std::min(1024, ((c.hidden / 4 + 63) / 64) * 64);
    launch_k(combine_kernel, dim3(c.seq), dim3(threads), 0, st, c);
    return hipGetLastError();
}

}  // namespace uocr_hip
