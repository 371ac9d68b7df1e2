// Operator mirrors of the reference's expert calls on the REFERENCE device
// layout (include/uocr/cuda_ops.h:134-239): per-expert tables as the engine
// uploads them (GpuDecoder::upload_expert_table, src/engine/gpu_decoder.cu:316-358)
// -- INT4 packed rows [E][rows][ceil(cols/2)] (low nibble = even column, stride
// pstride bytes), f32 scales and zeros [E][rows][ng] (stride sstride floats) --
// or bf16 row-major matrices behind device pointer arrays, the [n_experts, cap]
// assignment tables of moe_router_topk, f32 activations in and out.
//
// One kernel family serves every call: a workgroup owns (64 output rows, one
// expert) and walks the expert's assigned rows in m-tiles of 64. Per 128-column
// k-chunk it stages the gathered activation rows (f32 -> f16) and the weight
// panel (INT4: (q - zero) * scale in f32, rounded once to f16, where the
// reference dequantises to bf16, moe_gemm_int4.cu:456-473; bf16 weights:
// converted to f16, exact for |w| in the f16 normal range) into LDS in MFMA
// fragment order, and runs v_mfma_f32_16x16x32_f16 with f32 accumulation.
// f16 operands carry 3 more significand bits than the reference's bf16 ones;
// values beyond the f16 range (|x| > 65504) become infinite, so such inputs
// give non-finite outputs, never silently wrong finite ones.
// Epilogues: gate/up -> silu(g) * u into act [E, cap, N] (cpu_ops.cpp:108-113);
// down -> out[token] += w * y with f32 atomics (the reference's scatter-add,
// moe_device.cu:261-266; the order of the adds is not fixed); plain GEMM -> y.
#include "launch.hpp"

#include <algorithm>

namespace uocr_hip {

namespace {

constexpr int kMBM = 64;   // assigned rows per m-tile
constexpr int kMBN = 64;   // output rows per workgroup
constexpr int kMKC = 128;  // k columns per staged chunk
constexpr int kMFrag = 64 * 8;  // f16 per 1 KiB fragment

enum MirrorMode { kGateUp = 0, kDown = 1, kPlain = 2 };

struct MirrorArgs {
    const float* a;  // gate/up, plain: x [rows, K]; down: act [E, cap, K]
    int wfmt;        // 0: INT4 reference layout, 1: bf16 pointer arrays
    // INT4 tables (second set = up, gate/up only)
    const uint8_t* p0;
    const float* s0;
    const float* z0;
    const uint8_t* p1;
    const float* s1;
    const float* z1;
    long long pstride0, sstride0, pstride1, sstride1;
    int ng0, ng1;
    // bf16 tables
    const uint16_t* const* w0;
    const uint16_t* const* w1;
    const uint16_t* wplain;   // plain bf16 GEMM: W [N, K]
    const float* bias;        // plain GEMM: optional bias [N]
    const int* assign_token;  // [E, cap]
    const float* assign_w;    // [E, cap]
    const int* count;         // [E]
    int cap;
    int K, N, group;
    int m_plain;  // plain GEMM: rows of x
    float* out;   // gate/up: act [E, cap, N]; down: out [T, N] (+=); plain: y [m, N]
};

__device__ __forceinline__ float silu_mul_ref(float g, float u) { return g / (1.0f + expf(-g)) * u; }

template <int MODE, int WFMT>
__global__ __launch_bounds__(256) void mirror_kernel(MirrorArgs a) {
    constexpr int NM = MODE == kGateUp ? 2 : 1;  // weight matrices
    // A: [4 m-subtiles][4 k-steps] fragments; B: [NM][4 n-subtiles][4 k-steps]
    __shared__ __attribute__((aligned(16))) f16 As[16 * kMFrag];
    __shared__ __attribute__((aligned(16))) f16 Bs[NM * 16 * kMFrag];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int e = MODE == kPlain ? 0 : blockIdx.y;
    const int n0 = blockIdx.x * kMBN;
    const int rows = MODE == kPlain ? a.m_plain : min(a.count[e], a.cap);
    const int K = a.K, N = a.N;
    const int packed_row = (K + 1) / 2;

    // m-tiles blockIdx.z, + gridDim.z, ...: a skewed expert's rows spread over
    // gridDim.z workgroups per column block
    for (int m0 = blockIdx.z * kMBM; m0 < rows; m0 += gridDim.z * kMBM) {
        f32x4 acc[NM][4];
#pragma unroll
        for (int j = 0; j < NM; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};

        for (int k0 = 0; k0 < K; k0 += kMKC) {
            const int kc = min(kMKC, K - k0);  // a multiple of 32
            // activations: 64 rows x 16 runs of 8 columns
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                const int u = tid + 256 * it, m = u >> 4, c8 = u & 15;
                f16x8 v;
                const int slot = m0 + m;
                if (slot < rows && c8 * 8 < kc) {
                    long long row;
                    if constexpr (MODE == kGateUp) row = a.assign_token[(size_t)e * a.cap + slot];
                    else if constexpr (MODE == kDown) row = (long long)e * a.cap + slot;
                    else row = slot;
                    const float* src = a.a + (size_t)row * K + k0 + c8 * 8;
                    const f32x4 p = *reinterpret_cast<const f32x4*>(src);
                    const f32x4 q = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        v[i] = (f16)p[i];
                        v[4 + i] = (f16)q[i];
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) v[i] = (f16)0.0f;
                }
                // fragment (m / 16, k-step c8 / 4), lane (m % 16) + 16 * (c8 % 4)
                const int frag = (m >> 4) * 4 + (c8 >> 2);
                *reinterpret_cast<f16x8*>(As + (size_t)frag * kMFrag + ((m & 15) + 16 * (c8 & 3)) * 8) = v;
            }
            // weights
            if constexpr (WFMT == 0) {
                // NM x 64 rows x 4 runs of 32 columns (16 packed bytes)
#pragma unroll
                for (int it = 0; it < NM; ++it) {
                    const int u = tid + 256 * it, mat = u >> 8, n = (u >> 2) & 63, c32 = u & 3;
                    const uint8_t* P = mat ? a.p1 : a.p0;
                    const float* S = mat ? a.s1 : a.s0;
                    const float* Z = mat ? a.z1 : a.z0;
                    const long long ps = mat ? a.pstride1 : a.pstride0, ss = mat ? a.sstride1 : a.sstride0;
                    const int ng = mat ? a.ng1 : a.ng0;
                    const int kk = k0 + c32 * 32;
                    f16x8 v[4];
                    if (c32 * 32 < kc) {
                        const uint8_t* prow = P + (size_t)e * ps + (size_t)(n0 + n) * packed_row + kk / 2;
                        u32x4 w;
                        __builtin_memcpy(&w, prow, 16);  // 16-byte aligned when K % 32 == 0
                        const size_t sidx = (size_t)e * ss + (size_t)(n0 + n) * ng;
#pragma unroll
                        for (int r8 = 0; r8 < 4; ++r8) {
                            const int g = (kk + r8 * 8) / a.group;
                            const float sc = S[sidx + g], zr = Z[sidx + g];
#pragma unroll
                            for (int i = 0; i < 8; ++i) {
                                const uint32_t byte = (w[(r8 * 8 + i) >> 3] >> (8 * (((r8 * 8 + i) & 7) >> 1))) & 0xffu;
                                const uint32_t q = (i & 1) ? (byte >> 4) : (byte & 0x0fu);
                                v[r8][i] = (f16)(((float)q - zr) * sc);
                            }
                        }
                    } else {
#pragma unroll
                        for (int r8 = 0; r8 < 4; ++r8)
#pragma unroll
                            for (int i = 0; i < 8; ++i) v[r8][i] = (f16)0.0f;
                    }
                    // run r8 of k-step c32 -> lane (n % 16) + 16 * r8
#pragma unroll
                    for (int r8 = 0; r8 < 4; ++r8) {
                        const int frag = (mat * 4 + (n >> 4)) * 4 + c32;
                        *reinterpret_cast<f16x8*>(Bs + (size_t)frag * kMFrag + ((n & 15) + 16 * r8) * 8) = v[r8];
                    }
                }
            } else {
                // NM x 64 rows x 16 runs of 8 bf16
#pragma unroll
                for (int it = 0; it < 4 * NM; ++it) {
                    const int u = tid + 256 * it, mat = u >> 10, n = (u >> 4) & 63, c8 = u & 15;
                    u32x4 w = {0u, 0u, 0u, 0u};
                    if (c8 * 8 < kc) {
                        const uint16_t* wm = MODE == kPlain ? a.wplain : (mat ? a.w1 : a.w0)[e];
                        const uint16_t* row = wm + (size_t)(n0 + n) * K + k0 + c8 * 8;
                        w = *reinterpret_cast<const u32x4*>(row);
                    }
                    f16x8 v;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        v[2 * i] = (f16)bf16_bits_to_f32(w[i] & 0xffffu);
                        v[2 * i + 1] = (f16)__uint_as_float(w[i] & 0xffff0000u);
                    }
                    const int frag = (mat * 4 + (n >> 4)) * 4 + (c8 >> 2);
                    *reinterpret_cast<f16x8*>(Bs + (size_t)frag * kMFrag + ((n & 15) + 16 * (c8 & 3)) * 8) = v;
                }
            }
            __syncthreads();
            // wave w: n-subtile w of every matrix, all four m-subtiles
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                if (ks * 32 >= kc) break;
                f16x8 bf[NM];
#pragma unroll
                for (int j = 0; j < NM; ++j)
                    bf[j] = *reinterpret_cast<const f16x8*>(Bs + (size_t)((j * 4 + wave) * 4 + ks) * kMFrag + lane * 8);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const f16x8 af = *reinterpret_cast<const f16x8*>(As + (size_t)(i * 4 + ks) * kMFrag + lane * 8);
#pragma unroll
                    for (int j = 0; j < NM; ++j)
                        acc[j][i] = mfma16(af, bf[j], acc[j][i]);
                }
            }
            __syncthreads();
        }

        // epilogue: lane holds C[m = 16 i + 4 (lane / 16) + r][n = 16 wave + lane % 16]
        const int col = n0 + wave * 16 + (lane & 15);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int slot = m0 + i * 16 + 4 * (lane >> 4) + r;
                if (slot >= rows) continue;
                if constexpr (MODE == kGateUp) {
                    a.out[((size_t)e * a.cap + slot) * N + col] = silu_mul_ref(acc[0][i][r], acc[1][i][r]);
                } else if constexpr (MODE == kDown) {
                    const size_t ai = (size_t)e * a.cap + slot;
                    atomicAdd(a.out + (size_t)a.assign_token[ai] * N + col, a.assign_w[ai] * acc[0][i][r]);
                } else {
                    a.out[(size_t)slot * N + col] = acc[0][i][r] + (a.bias ? a.bias[col] : 0.0f);
                }
            }
    }
}

template <int MODE, int WFMT>
hipError_t launch_mirror(const MirrorArgs& a, int n_experts, hipStream_t st) {
    // m-tile workgroups per (column block, expert): every m-tile of a plain
    // GEMM; up to 32 per expert of the grouped calls (cap bounds the rows)
    const int mt = ((MODE == kPlain ? a.m_plain : a.cap) + kMBM - 1) / kMBM;
    const int mz = MODE == kPlain ? std::min(mt, 65535) : std::min(mt, 32);
    const dim3 grid(a.N / kMBN, MODE == kPlain ? 1 : n_experts, std::max(mz, 1));
    launch_k((mirror_kernel<MODE, WFMT>), grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace

// shape preconditions shared by every mirror (K multiple of 32, N of 64)
bool mirror_shapes_ok(int k, int n, int group, bool int4) {
    return k > 0 && n > 0 && k % 32 == 0 && n % kMBN == 0 && (!int4 || (group > 0 && group % 32 == 0));
}

hipError_t mirror_gate_up_int4(const float* x, const uint8_t* gp, const float* gs, const float* gz, long long gps,
                               long long gss, int gng, const uint8_t* up, const float* us, const float* uz,
                               long long ups, long long uss, int ung, const int* assign_token, const int* count,
                               int n_experts, int cap, int hidden, int inter, int group, float* act, hipStream_t st) {
    MirrorArgs a{};
    a.a = x;
    a.wfmt = 0;
    a.p0 = gp, a.s0 = gs, a.z0 = gz, a.pstride0 = gps, a.sstride0 = gss, a.ng0 = gng;
    a.p1 = up, a.s1 = us, a.z1 = uz, a.pstride1 = ups, a.sstride1 = uss, a.ng1 = ung;
    a.assign_token = assign_token, a.count = count, a.cap = cap;
    a.K = hidden, a.N = inter, a.group = group, a.out = act;
    return launch_mirror<kGateUp, 0>(a, n_experts, st);
}

hipError_t mirror_down_int4(const float* act, const uint8_t* p, const float* s, const float* z, long long ps,
                            long long ss, int ng, const int* assign_token, const float* assign_w, const int* count,
                            int n_experts, int cap, int hidden, int inter, int group, float* out, hipStream_t st) {
    MirrorArgs a{};
    a.a = act;
    a.wfmt = 0;
    a.p0 = p, a.s0 = s, a.z0 = z, a.pstride0 = ps, a.sstride0 = ss, a.ng0 = ng;
    a.assign_token = assign_token, a.assign_w = assign_w, a.count = count, a.cap = cap;
    a.K = inter, a.N = hidden, a.group = group, a.out = out;
    return launch_mirror<kDown, 0>(a, n_experts, st);
}

hipError_t mirror_gemm_int4(const float* x, const uint8_t* p, const float* s, const float* z, int m, int n, int k,
                            int group, float* y, hipStream_t st) {
    MirrorArgs a{};
    a.a = x;
    a.wfmt = 0;
    a.p0 = p, a.s0 = s, a.z0 = z, a.pstride0 = 0, a.sstride0 = 0, a.ng0 = (k + group - 1) / group;
    a.K = k, a.N = n, a.group = group, a.m_plain = m, a.out = y;
    return launch_mirror<kPlain, 0>(a, 1, st);
}

hipError_t mirror_gemm_bf16(const float* x, const uint16_t* w, const float* bias, int m, int n, int k, float* y,
                            hipStream_t st) {
    MirrorArgs a{};
    a.a = x;
    a.wfmt = 1;
    a.wplain = w;
    a.bias = bias;
    a.K = k, a.N = n, a.m_plain = m, a.out = y;
    return launch_mirror<kPlain, 1>(a, 1, st);
}

// ---------------------------------------------------------------------------
// Elementwise helpers of the host-grouping decode branch (the reference's
// gpu_ops.cu:12-45,85-111): 4 elements per thread where the row length allows.
// ---------------------------------------------------------------------------
__global__ void silu_mul_kernel(const float* g, const float* u, float* out, long long n) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = silu_mul_ref(g[i], u[i]);
}

__global__ void add_scaled_kernel(float* dst, const float* src, float scale, long long n) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = fmaf(scale, src[i], dst[i]);
}

// out[row_idx[r], c] += w[r] * vals[r, c]; rows that name the same output row
// add atomically (the reference's plain += leaves that case undefined)
__global__ void scatter_add_scaled_kernel(float* out, const float* vals, const int* row_idx, const float* w, int rows,
                                          int cols) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)rows * cols) return;
    const int r = (int)(i / cols), c = (int)(i - (long long)r * cols);
    atomicAdd(out + (size_t)row_idx[r] * cols + c, w[r] * vals[i]);
}

__global__ void gather_rows_kernel(float* dst, const float* src, const int* row_idx, int rows, int cols) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)rows * cols) return;
    const int r = (int)(i / cols), c = (int)(i - (long long)r * cols);
    dst[i] = src[(size_t)row_idx[r] * cols + c];
}

static dim3 grid_for(long long n) { return dim3((unsigned)((n + 255) / 256)); }

hipError_t mirror_silu_mul(const float* g, const float* u, float* out, long long n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    launch_k(silu_mul_kernel, grid_for(n), dim3(256), 0, st, g, u, out, n);
    return hipGetLastError();
}

hipError_t mirror_add_scaled(float* dst, const float* src, float scale, long long n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    launch_k(add_scaled_kernel, grid_for(n), dim3(256), 0, st, dst, src, scale, n);
    return hipGetLastError();
}

hipError_t mirror_scatter_add_scaled(float* out, const float* vals, const int* row_idx, const float* w, int rows,
                                     int cols, hipStream_t st) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    launch_k(scatter_add_scaled_kernel, grid_for((long long)rows * cols), dim3(256), 0, st, out, vals, row_idx, w,
             rows, cols);
    return hipGetLastError();
}

hipError_t mirror_gather_rows(float* dst, const float* src, const int* row_idx, int rows, int cols, hipStream_t st) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    launch_k(gather_rows_kernel, grid_for((long long)rows * cols), dim3(256), 0, st, dst, src, row_idx, rows, cols);
    return hipGetLastError();
}

hipError_t mirror_gate_up_bf16(const float* x, const uint16_t* const* gw, const uint16_t* const* uw,
                               const int* assign_token, const int* count, int n_experts, int cap, int hidden,
                               int inter, float* act, hipStream_t st) {
    MirrorArgs a{};
    a.a = x;
    a.wfmt = 1;
    a.w0 = gw, a.w1 = uw;
    a.assign_token = assign_token, a.count = count, a.cap = cap;
    a.K = hidden, a.N = inter, a.out = act;
    return launch_mirror<kGateUp, 1>(a, n_experts, st);
}

hipError_t mirror_down_bf16(const float* act, const uint16_t* const* dw, const int* assign_token,
                            const float* assign_w, const int* count, int n_experts, int cap, int hidden, int inter,
                            float* out, hipStream_t st) {
    MirrorArgs a{};
    a.a = act;
    a.wfmt = 1;
    a.w0 = dw;
    a.assign_token = assign_token, a.assign_w = assign_w, a.count = count, a.cap = cap;
    a.K = inter, a.N = hidden, a.out = out;
    return launch_mirror<kDown, 1>(a, n_experts, st);
}

}  // namespace uocr_hip
