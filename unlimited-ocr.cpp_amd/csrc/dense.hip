// Unquantised expert weights: the reference's BF16 (and, after the AWQ fold,
// F32) matrices on f16 MFMA.
//
// The reference keeps the shared expert unquantised (src/runtime/weights.cpp:
// 289-292; F32 after scale_columns, weights.cpp:185-207) and runs it as three
// bf16 linear_forward calls (src/engine/gpu_decoder.cu:647-652); its default
// routed-expert format is BF16 too (include/uocr/config.h:111), grouped by
// moe_grouped_gate_up_bf16 / _down_bf16 (src/kernels/cuda/moe_gemm_bf16.cu:
// 122-353). Here those matrices are uploaded once as f16, row-major
// [rows][cols] (exact for every bf16 value in f16's normal range; finer than
// bf16 for f32 values), and multiplied with f16 activations on
// v_mfma_f32_*_f16 with f32 accumulation. Two kernels share one argument
// block and one work description (the grouping's tile list, or consecutive
// slot tiles for the shared MLP, which sees every token):
//   * dense_skinny_kernel -- up to 16 slots per tile (decode). A workgroup owns
//     16 output columns of one tile and splits K across its waves; every wave
//     issues all of its weight and activation loads at once (16-byte
//     fragments straight from global memory into MFMA operand order), so the
//     weight stream is limited by HBM, not by latency; the waves' partial sums
//     meet in LDS.
//   * dense_tiled_kernel -- 128 slots per tile (prefill). Activations are
//     staged in LDS per 128-column k-tile, one k-tile ahead (double-buffered);
//     each wave loads its own weight rows for the k-tile into registers and
//     runs v_mfma_f32_32x32x16_f16 against the 4 staged 32-slot subtiles. Two
//     workgroups per CU hide each other's load latency (measured faster than
//     one workgroup per CU with the weights double-buffered in registers, and
//     than 192-slot tiles).
// Gate/up (GU) pairs a gate block with the same up rows and writes
// silu(g) * u as f16 act; down writes y (f16 per slot for the combine of the
// grouped path, f32 per token for the shared MLP).
#include "launch.hpp"

#include <utility>

namespace uocr_hip {

namespace {

template <typename F, int... I>
__device__ __forceinline__ void sfor_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void sfor(F&& f) {
    sfor_impl(f, std::make_integer_sequence<int, N>{});
}

// 8 consecutive activations as f16: f16 rows (AK 0) or bf16 rows (AK 1,
// converted exactly within f16's range)
template <int AK>
__device__ __forceinline__ f16x8 load_a8(const void* base, size_t idx) {
    if constexpr (AK == 0) {
        return *reinterpret_cast<const f16x8*>(static_cast<const f16*>(base) + idx);
    } else {
        const u32x4 v = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + idx);
        f16x8 r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            r[2 * i] = (f16)__uint_as_float(v[i] << 16);
            r[2 * i + 1] = (f16)__uint_as_float(v[i] & 0xffff0000u);
        }
        return r;
    }
}

__device__ __forceinline__ f16x8 load_w8(const f16* p) { return *reinterpret_cast<const f16x8*>(p); }

__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

struct TileDesc {
    int e, m0, rows, slot0;
};

// tile `tile` of the work list; false past its end
__device__ __forceinline__ bool tile_desc(const DenseArgs& a, int tile, int bm, TileDesc& t) {
    if (a.tile_info) {
        if (tile >= *a.n_tiles) return false;
        const int4 ti = *reinterpret_cast<const int4*>(a.tile_info + 4 * tile);
        t = TileDesc{ti.x, ti.y, ti.z, ti.w};
        return true;
    }
    const int m0 = tile * bm;
    if (m0 >= a.seq) return false;
    t = TileDesc{0, m0, min(bm, a.seq - m0), m0};
    return true;
}

// four values staged as f16 (a value beyond f16's range is reported)
__device__ __forceinline__ void store_f16x4(f16* p, float v0, float v1, float v2, float v3, int* status) {
    f16x4 h = {(f16)v0, (f16)v1, (f16)v2, (f16)v3};
    *reinterpret_cast<f16x4*>(p) = h;
    report_f16_overflow(status, f16_overflow(v0) || f16_overflow(v1) || f16_overflow(v2) || f16_overflow(v3));
}

}  // namespace

// ---------------------------------------------------------------------------
// Decode-sized tiles (<= 16 slots). Workgroup = (tile, 16 output columns),
// NW waves; wave w covers k-steps [w * KSW, (w + 1) * KSW) of 32 columns.
// KSW == 0: runtime k-step count, in chunks of 8.
// ---------------------------------------------------------------------------
template <int NW, int KSW, bool GU, int AK>
__global__ __launch_bounds__(64 * NW) void dense_skinny_kernel(DenseArgs a) {
    constexpr int CH = KSW > 0 ? KSW : 8;
    __shared__ f32x4 red[NW > 1 ? NW - 1 : 1][GU ? 2 : 1][64];
    const int n_nb = a.n_out / 16;
    const int tile = blockIdx.x / n_nb, nb = blockIdx.x % n_nb;
    TileDesc t;
    if (!tile_desc(a, tile, 16, t)) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int K = a.k;
    const int ksw = KSW > 0 ? KSW : (K / 32) / NW;
    const int kc0 = wave * ksw * 32 + 8 * (lane >> 4);  // this lane's first column
    const int m = lane & 15;
    const int slot = t.slot0 + min(m, t.rows - 1);
    const int arow = a.slot_tok ? a.slot_tok[slot] : slot;
    const size_t abase = (size_t)arow * K + kc0;
    const size_t wbase = (size_t)t.e * a.w_stride + (size_t)(nb * 16 + m) * K + kc0;
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < ksw; c += CH) {
        f16x8 b0[CH], b1[CH], af[CH];
        // the weight stream first (HBM), then the activations (L2)
#pragma unroll
        for (int i = 0; i < CH; ++i)
            if (KSW > 0 || c + i < ksw) {
                b0[i] = load_w8(a.w0 + wbase + (c + i) * 32);
                if constexpr (GU) b1[i] = load_w8(a.w1 + wbase + (c + i) * 32);
            }
#pragma unroll
        for (int i = 0; i < CH; ++i)
            if (KSW > 0 || c + i < ksw) af[i] = load_a8<AK>(a.a, abase + (c + i) * 32);
        // every load of the chunk is in flight before the first use (left to
        // itself the scheduler sinks loads to their uses, one round trip each)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < CH; ++i)
            if (KSW > 0 || c + i < ksw) {
                acc0 = mfma16(b0[i], af[i], acc0);
                if constexpr (GU) acc1 = mfma16(b1[i], af[i], acc1);
            }
    }
    if constexpr (NW > 1) {
        if (wave > 0) {
            red[wave - 1][0][lane] = acc0;
            if constexpr (GU) red[wave - 1][1][lane] = acc1;
        }
        __syncthreads();
        if (wave > 0) return;
#pragma unroll
        for (int w = 0; w < NW - 1; ++w) {
            acc0 += red[w][0][lane];
            if constexpr (GU) acc1 += red[w][1][lane];
        }
    }
    // lane holds D[weight row 4 * (lane / 16) + r][slot lane % 16]
    if (m >= t.rows) return;
    const size_t o = (size_t)(t.slot0 + m) * a.n_out + nb * 16 + 4 * (lane >> 4);
    if constexpr (GU) {
        store_f16x4(a.out16 + o, silu_mul_f(acc0[0], acc1[0]), silu_mul_f(acc0[1], acc1[1]),
                    silu_mul_f(acc0[2], acc1[2]), silu_mul_f(acc0[3], acc1[3]), a.status);
    } else if (a.out32) {
        *reinterpret_cast<f32x4*>(a.out32 + o) = acc0;
    } else {
        store_f16x4(a.out16 + o, acc0[0], acc0[1], acc0[2], acc0[3], a.status);
    }
}

// ---------------------------------------------------------------------------
// Prefill-sized tiles (128 slots), two workgroups per CU. Workgroup = (tile,
// output columns: GU 128 act columns = 4 waves x (32 gate + 32 up rows); down
// 256 = 4 waves x 64 rows). Activations: wave w stages 32-slot subtile w of each 128-column
// k-tile into LDS in 32x32x16 operand order (fragment (msub, s) = 1 KiB,
// lane l: slot l % 32, columns s * 16 + 8 * (l / 32) .. + 8).
// ---------------------------------------------------------------------------
template <bool GU>
__global__ __launch_bounds__(256, 2) void dense_tiled_kernel(DenseArgs a) {
    constexpr int NS = 8;  // k16-steps per 128-column k-tile
    constexpr int WB = 2;  // 32-row weight blocks per wave
    __shared__ __attribute__((aligned(16))) f16 As[2][4 * NS * 512];
    const int cols_wg = GU ? 128 : 256;
    const int n_nt = a.n_out / cols_wg;
    // XCD-aware order: the grid is a multiple of 8 and block b runs on XCD
    // b % 8, so XCD x gets a contiguous run of (n-tile, tile) items: the tiles
    // of one n-tile share its weight rows in that XCD's L2
    const int per_xcd = gridDim.x / 8;
    const int item = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    const int n_tiles_grid = gridDim.x / n_nt;  // unused tail items exit below
    (void)n_tiles_grid;
    const int nt = item / (gridDim.x / n_nt), tile = item % (gridDim.x / n_nt);
    if (nt >= n_nt) return;
    TileDesc t;
    if (!tile_desc(a, tile, kDenseTiledBM, t)) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int K = a.k, KT = K / kTileK;
    const int l32 = lane & 31, lh = lane >> 5;
    // A: this wave's 32-slot subtile
    const int am = wave * 32 + l32;
    const int slot = t.slot0 + min(am, t.rows - 1);
    const int arow = a.slot_tok ? a.slot_tok[slot] : slot;
    const f16* asrc = static_cast<const f16*>(a.a) + (size_t)arow * K + 8 * lh;
    // B: this wave's weight rows
    const f16* bsrc[WB];
#pragma unroll
    for (int b = 0; b < WB; ++b) {
        const int row = GU ? (nt * 128 + wave * 32 + l32) : (nt * 256 + wave * 64 + b * 32 + l32);
        const f16* w = (GU && b == 1) ? a.w1 : a.w0;
        bsrc[b] = w + (size_t)t.e * a.w_stride + (size_t)row * K + 8 * lh;
    }
    f32x16 acc[WB][4];
#pragma unroll
    for (int b = 0; b < WB; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[b][i][r] = 0.f;
    f16x8 ar[NS];
    f16x8 bq[WB][NS];
    auto load_a = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < NS; ++s) ar[s] = *reinterpret_cast<const f16x8*>(asrc + kt * kTileK + s * 16);
    };
    auto write_a = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < NS; ++s) *reinterpret_cast<f16x8*>(&As[buf][((wave * NS + s) * 64 + lane) * 8]) = ar[s];
    };
    auto load_b = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
        for (int b = 0; b < WB; ++b)
#pragma unroll
            for (int s = 0; s < NS; ++s) bq[b][s] = load_w8(bsrc[b] + kt * kTileK + s * 16);
    };
    auto compute = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            f16x8 af[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) af[i] = *reinterpret_cast<const f16x8*>(&As[buf][((i * NS + s) * 64 + lane) * 8]);
#pragma unroll
            for (int b = 0; b < WB; ++b)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[b][i] = mfma32(bq[b][s], af[i], acc[b][i]);
        }
    };
    // the weights of k-tile kt are issued at the top of its own iteration (no
    // register double buffer: two workgroups per CU hide each other's
    // latency), the activations one k-tile ahead through LDS
    load_a(0);
    write_a(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const bool more = kt + 1 < KT;
        load_b(kt);
        if (more) load_a(kt + 1);
        compute(kt & 1);
        if (more) write_a((kt + 1) & 1);
        __syncthreads();
    }
    // D lane l: weight row 8 * (r / 4) + 4 * (l / 32) + r % 4 of the block, slot l % 32 of subtile i
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int mm = i * 32 + l32;
        if (mm >= t.rows) continue;
        const size_t orow = (size_t)(t.slot0 + mm) * a.n_out;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r0 = 8 * q + 4 * lh;
            if constexpr (GU) {
                const size_t o = orow + nt * 128 + wave * 32 + r0;
                store_f16x4(a.out16 + o, silu_mul_f(acc[0][i][4 * q], acc[1][i][4 * q]),
                            silu_mul_f(acc[0][i][4 * q + 1], acc[1][i][4 * q + 1]),
                            silu_mul_f(acc[0][i][4 * q + 2], acc[1][i][4 * q + 2]),
                            silu_mul_f(acc[0][i][4 * q + 3], acc[1][i][4 * q + 3]), a.status);
            } else {
#pragma unroll
                for (int b = 0; b < WB; ++b) {
                    const size_t o = orow + nt * 256 + wave * 64 + b * 32 + r0;
                    if (a.out32)
                        *reinterpret_cast<f32x4*>(a.out32 + o) =
                            f32x4{acc[b][i][4 * q], acc[b][i][4 * q + 1], acc[b][i][4 * q + 2], acc[b][i][4 * q + 3]};
                    else
                        store_f16x4(a.out16 + o, acc[b][i][4 * q], acc[b][i][4 * q + 1], acc[b][i][4 * q + 2],
                                    acc[b][i][4 * q + 3], a.status);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
bool dense_shapes_ok(int k, int n_out, bool gate_up, int bm) {
    if (k <= 0 || n_out <= 0 || k % kTileK) return false;
    if (bm == kDenseSkinnyBM) return n_out % 16 == 0 && (k / 32) % 4 == 0;
    if (bm == kDenseTiledBM) return n_out % (gate_up ? 128 : 256) == 0;
    return false;
}

template <bool GU, int AK>
static hipError_t launch_skinny(const DenseArgs& a, int n_tiles, hipStream_t st) {
    const int ks = a.k / 32;
    const dim3 grid(n_tiles * (a.n_out / 16));
    if (ks == 40)
        launch_k(dense_skinny_kernel<4, 10, GU, AK>, grid, dim3(256), 0, st, a);
    else if (ks == 28)
        launch_k(dense_skinny_kernel<4, 7, GU, AK>, grid, dim3(256), 0, st, a);
    else if (ks == 56)
        launch_k(dense_skinny_kernel<8, 7, GU, AK>, grid, dim3(512), 0, st, a);
    else
        launch_k(dense_skinny_kernel<4, 0, GU, AK>, grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// The f16 input rows of an unquantised shared MLP that runs ahead of the
// single-kernel decode, for f32 hidden states or the RMSNorm prologue
// (src/kernels/cpu_ops.cpp:58-67: (x * inv) * w with inv = 1 / sqrt(mean(x^2)
// + eps)). One workgroup per token; the sum of squares is added in parallel,
// which moves inv by a few units of f32 roundoff, far below the f16 rounding
// of the result.
// ---------------------------------------------------------------------------
constexpr int kPrepThreads = 256;
constexpr int kPrepCols = 8;  // columns per thread (hidden <= 2048)

__global__ __launch_bounds__(kPrepThreads) void x16_prep_kernel(const void* x, int x_bf16, const float* rms_w,
                                                                float eps, int H, f16* x16) {
    __shared__ float wsum[kPrepThreads / 64];
    const int t = blockIdx.x, tid = threadIdx.x;
    float v[kPrepCols];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kPrepCols; ++i) {
        const int c = tid + kPrepThreads * i;
        v[i] = 0.0f;
        if (c < H)
            v[i] = x_bf16 ? __uint_as_float((uint32_t)static_cast<const uint16_t*>(x)[(size_t)t * H + c] << 16)
                          : static_cast<const float*>(x)[(size_t)t * H + c];
        ss += v[i] * v[i];
    }
    float inv = 1.0f;
    if (rms_w) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        if ((tid & 63) == 0) wsum[tid >> 6] = ss;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < kPrepThreads / 64; ++w) tot += wsum[w];
        inv = 1.0f / sqrtf(tot / (float)H + eps);
    }
#pragma unroll
    for (int i = 0; i < kPrepCols; ++i) {
        const int c = tid + kPrepThreads * i;
        if (c < H) x16[(size_t)t * H + c] = (f16)(rms_w ? (v[i] * inv) * rms_w[c] : v[i]);
    }
}

hipError_t launch_x16_prep(const void* x, bool x_bf16, const float* rms_w, float eps, int seq, int H, f16* x16,
                           hipStream_t st) {
    if (seq <= 0) return hipSuccess;
    if (H > kPrepThreads * kPrepCols || !x || !x16) return hipErrorInvalidValue;
    launch_k(x16_prep_kernel, dim3(seq), dim3(kPrepThreads), 0, st, x, x_bf16 ? 1 : 0, rms_w, eps, H, x16);
    return hipGetLastError();
}

hipError_t launch_dense(const DenseArgs& a, bool gate_up, int bm, int max_tiles, hipStream_t st) {
    if (!dense_shapes_ok(a.k, a.n_out, gate_up, bm)) return hipErrorInvalidValue;
    if (gate_up ? !(a.out16 && a.w1) : !(a.out16 || a.out32)) return hipErrorInvalidValue;
    const int n_tiles = a.tile_info ? max_tiles : (a.seq + bm - 1) / bm;
    if (n_tiles <= 0) return hipSuccess;
    if (bm == kDenseSkinnyBM) {
        if (a.a_kind == 1) return gate_up ? launch_skinny<true, 1>(a, n_tiles, st) : launch_skinny<false, 1>(a, n_tiles, st);
        return gate_up ? launch_skinny<true, 0>(a, n_tiles, st) : launch_skinny<false, 0>(a, n_tiles, st);
    }
    if (a.a_kind != 0) return hipErrorInvalidValue;
    const int n_nt = a.n_out / (gate_up ? 128 : 256);
    const int blocks = (n_tiles * n_nt + 7) / 8 * 8;
    // the in-kernel item map needs blocks to be a multiple of n_nt as well
    int grid = blocks;
    while (grid % n_nt) grid += 8;
    if (gate_up)
        launch_k(dense_tiled_kernel<true>, dim3(grid), dim3(256), 0, st, a);
    else
        launch_k(dense_tiled_kernel<false>, dim3(grid), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace uocr_hip
