// R-SWA attention and KV-cache writes (the step after the MoE path):
// counterparts of src/kernels/cuda/rswa_attention.cu and the host cache
// semantics of src/scheduler/kv_cache.cpp. Cache layout as the reference's:
// [capacity, kv_heads, head_dim] f32 per request (a batch of requests: slot s
// at base + s * batch_cap * kv_heads * head_dim); rows 0..P-1 hold the first
// prefill ("reference tokens"), rows P..P+W-1 a ring of the last W decoded
// tokens.
//
// Attention: one workgroup per (query row, head), 8 waves splitting the keys.
// A wave takes groups of 8 consecutive keys (groups w, w + 8, ...): lane
// (j, p) = (lane / 8, lane % 8) holds key j's dims 4p + 32i .. + 3 (i < HDP / 32)
// of K and V (each load: the 8 lanes of a key read one contiguous 128-byte run),
// with the next two groups' K and V loads (one for head_dim > 128) issued
// before the current group is used. Scores reduce over the 8 lanes of a key, the online softmax runs per
// wave (max, rescale, sum over the group's keys), and each lane accumulates
// p * V for its own key slot; the 8 key slots and then the 8 waves are
// combined at the end (flash-decoding). Decode is HBM-bound: every (row, head)
// streams kv_len * head_dim * 8 bytes of K and V.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <initializer_list>
#include <mutex>
#include <string>

#include "common.hpp"
#include "launch.hpp"
#include "uocr_hip/moe_capi.h"

namespace uocr_hip {
namespace {

constexpr int kRswaWaves = 8;

struct RswaArgs {
    const float* q;
    const float* kc;
    const float* vc;
    float* out;
    int heads, kv_heads, head_dim;
    float scale;
    int mode;  // 0: one cache, kv_len (causal: q_start); 1: same, kv_len = *d_len;
               // 2: batch (slot d_slots[b], length d_len[slot]); 3: ragged (slot d_slots[t], rows 0..d_pos[t])
    int kv_len, q_start, causal;
    const int* d_len;
    const int* d_slots;
    const int* d_pos;
    int batch_cap;
    int n_chunks;  // > 1: keys split over blockIdx.z, partial (m, l, o) records to part
    float* part;   // [rows][heads][n_chunks][kRswaRec]
};

// one partial record: m, l, (pad), then o[head_dim]
constexpr int kRswaRec = 256 + 4;

template <int HDP>
__global__ __launch_bounds__(kRswaWaves * 64) void rswa_kernel(RswaArgs a) {
    constexpr int D = HDP / 8;  // dims per lane
    constexpr int NV = D / 4;   // float4 per lane per row
    const int row = blockIdx.x, head = blockIdx.y;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int j = lane >> 3, p = lane & 7;
    const int hd = a.head_dim, stride = a.kv_heads * hd;
    const int kvh = head / (a.heads / a.kv_heads);
    const float* kc = a.kc;
    const float* vc = a.vc;
    int limit;
    if (a.mode <= 1) {
        const int kv_len = a.mode == 1 ? *a.d_len : a.kv_len;
        limit = a.causal ? min(kv_len, a.q_start + row + 1) : kv_len;
    } else {
        const int slot = a.d_slots[row];
        limit = a.mode == 2 ? a.d_len[slot] : a.d_pos[row] + 1;
        kc += (size_t)slot * a.batch_cap * stride;
        vc += (size_t)slot * a.batch_cap * stride;
    }
    const size_t qoff = ((size_t)row * a.heads + head) * hd;
    kc += (size_t)kvh * hd;
    vc += (size_t)kvh * hd;
    // lane p's dims: 4 at 4p + 32i (i < NV), so the 8 lanes of a key read one
    // contiguous 128-byte run per load
    auto dim_of = [&](int i) { return 4 * p + 32 * i; };

    f32x4 qv[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i)
        qv[i] = dim_of(i) < hd ? *reinterpret_cast<const f32x4*>(a.q + qoff + dim_of(i)) : f32x4{0.f, 0.f, 0.f, 0.f};

    float m = -INFINITY, l = 0.0f;
    f32x4 acc[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    // this workgroup's keys [kbeg, kend): chunk blockIdx.z of n_chunks (chunks
    // of whole 8-key groups; a chunk past the limit has no keys)
    int kbeg = 0, kend = limit;
    if (a.n_chunks > 1) {
        const int cs = ((limit + a.n_chunks - 1) / a.n_chunks + 7) & ~7;
        kbeg = min(limit, (int)blockIdx.z * cs);
        kend = min(limit, kbeg + cs);
    }
    const int n_groups = (kend - kbeg + 7) / 8;
    // Unpredicated loads (a lane-predicated load makes the compiler wait for
    // every outstanding load before the first use, defeating the prefetch):
    // keys past the limit re-read the last valid row (their weight is 0),
    // dims past head_dim re-read the last 4 (their q is 0 and they are never
    // stored). Called only with limit >= 1.
    auto load = [&](int g, f32x4 (&kv)[NV], f32x4 (&vv)[NV]) {
        const int t = min(kbeg + g * 8 + j, kend - 1);
        const float* kr = kc + (size_t)t * stride;
        const float* vr = vc + (size_t)t * stride;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int d = min(dim_of(i), hd - 4);
            kv[i] = *reinterpret_cast<const f32x4*>(kr + d);
            vv[i] = *reinterpret_cast<const f32x4*>(vr + d);
        }
    };
    f32x4 k0[NV], v0[NV], k1[NV], v1[NV], k2[NV], v2[NV];
    constexpr float kLog2e = 1.4426950408889634f;
    auto step = [&](int g, const f32x4 (&kv)[NV], const f32x4 (&vv)[NV]) {
        float part = 0.0f;
#pragma unroll
        for (int i = 0; i < NV; ++i)
#pragma unroll
            for (int c = 0; c < 4; ++c) part = fmaf(qv[i][c], kv[i][c], part);
        part += __shfl_xor(part, 1, 64);
        part += __shfl_xor(part, 2, 64);
        part += __shfl_xor(part, 4, 64);
        const bool valid = kbeg + g * 8 + j < kend;
        const float s = valid ? part * a.scale : -INFINITY;
        float mg = fmaxf(s, __shfl_xor(s, 8, 64));
        mg = fmaxf(mg, __shfl_xor(mg, 16, 64));
        mg = fmaxf(mg, __shfl_xor(mg, 32, 64));
        const float m_new = fmaxf(m, mg);  // finite: key 0 of the group is valid
        const float alpha = __builtin_amdgcn_exp2f((m - m_new) * kLog2e);
        const float beta = valid ? __builtin_amdgcn_exp2f((s - m_new) * kLog2e) : 0.0f;
        float bs = beta + __shfl_xor(beta, 8, 64);
        bs += __shfl_xor(bs, 16, 64);
        bs += __shfl_xor(bs, 32, 64);
        l = fmaf(l, alpha, bs);
#pragma unroll
        for (int i = 0; i < NV; ++i)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[i][c] = fmaf(acc[i][c], alpha, beta * vv[i][c]);
        m = m_new;
    };
    // groups wave, wave + 8, ...; two groups' loads in flight beyond the one in
    // use (three register buffers in rotation), one for head_dim > 128
    constexpr int GS = kRswaWaves;
    int g = wave;
    if constexpr (HDP <= 128) {
        if (g < n_groups) {
            load(g, k0, v0);
            load(g + GS, k1, v1);
        }
        while (g < n_groups) {
            load(g + 2 * GS, k2, v2);
            step(g, k0, v0);
            g += GS;
            if (g >= n_groups) break;
            load(g + 2 * GS, k0, v0);
            step(g, k1, v1);
            g += GS;
            if (g >= n_groups) break;
            load(g + 2 * GS, k1, v1);
            step(g, k2, v2);
            g += GS;
        }
    } else {
        if (g < n_groups) load(g, k0, v0);
        while (g < n_groups) {
            load(g + GS, k1, v1);
            step(g, k0, v0);
            g += GS;
            if (g >= n_groups) break;
            load(g + GS, k0, v0);
            step(g, k1, v1);
            g += GS;
        }
    }
    // sum the 8 key slots of the wave (same m within the wave)
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float x = acc[i][c];
            x += __shfl_xor(x, 8, 64);
            x += __shfl_xor(x, 16, 64);
            x += __shfl_xor(x, 32, 64);
            acc[i][c] = x;
        }
    __shared__ float wm[kRswaWaves], wl[kRswaWaves];
    __shared__ __attribute__((aligned(16))) float wacc[kRswaWaves][HDP];
    if (lane < 8) {
#pragma unroll
        for (int i = 0; i < NV; ++i) *reinterpret_cast<f32x4*>(&wacc[wave][dim_of(i)]) = acc[i];
    }
    if (lane == 0) {
        wm[wave] = m;
        wl[wave] = l;
    }
    __syncthreads();
    // combine the waves (a wave without keys has m = -inf and weight 0)
    float* rec = a.n_chunks > 1 ? a.part + (((size_t)row * a.heads + head) * a.n_chunks + blockIdx.z) * kRswaRec
                                : nullptr;
    if (rec && tid == 0) {
        float M = -INFINITY, L = 0.0f;
#pragma unroll
        for (int w = 0; w < kRswaWaves; ++w) M = fmaxf(M, wm[w]);
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < kRswaWaves; ++w)
                L = fmaf(wl[w], wm[w] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((wm[w] - M) * kLog2e), L);
        }
        rec[0] = M;
        rec[1] = L;
    }
    for (int d = tid; d < hd; d += kRswaWaves * 64) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kRswaWaves; ++w) M = fmaxf(M, wm[w]);
        float L = 0.0f, o = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < kRswaWaves; ++w) {
                const float f = wm[w] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((wm[w] - M) * kLog2e);
                L = fmaf(wl[w], f, L);
                o = fmaf(wacc[w][d], f, o);
            }
        }
        if (rec)
            rec[4 + d] = o;  // unnormalised, relative to this chunk's max
        else
            a.out[qoff + d] = L > 0.0f ? o / L : 0.0f;
    }
}

// Merge of the n_chunks partial records of each (row, head): the
// flash-decoding combine, chunks in key order.
__global__ __launch_bounds__(256) void rswa_merge_kernel(const float* part, float* out, int heads, int head_dim,
                                                         int n_chunks) {
    constexpr float kLog2e = 1.4426950408889634f;
    const int row = blockIdx.x, head = blockIdx.y;
    const float* rec = part + ((size_t)row * heads + head) * n_chunks * kRswaRec;
    float M = -INFINITY;
    for (int c = 0; c < n_chunks; ++c) M = fmaxf(M, rec[(size_t)c * kRswaRec]);
    for (int d = threadIdx.x; d < head_dim; d += blockDim.x) {
        float L = 0.0f, o = 0.0f;
        if (M != -INFINITY) {
            for (int c = 0; c < n_chunks; ++c) {
                const float m = rec[(size_t)c * kRswaRec];
                const float f = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m - M) * kLog2e);
                L = fmaf(rec[(size_t)c * kRswaRec + 1], f, L);
                o = fmaf(rec[(size_t)c * kRswaRec + 4 + d], f, o);
            }
        }
        out[((size_t)row * heads + head) * head_dim + d] = L > 0.0f ? o / L : 0.0f;
    }
}

// Row copy of one token's K and V (stride floats each) into a cache row.
__device__ __forceinline__ void copy_row(const float* k, const float* v, float* kd, float* vd, int stride) {
    for (int i = threadIdx.x * 4; i < stride; i += blockDim.x * 4) {
        *reinterpret_cast<f32x4*>(kd + i) = *reinterpret_cast<const f32x4*>(k + i);
        *reinterpret_cast<f32x4*>(vd + i) = *reinterpret_cast<const f32x4*>(v + i);
    }
}

// The cache row an append writes, with the ring state advanced: grow until
// prefill_len + window, then overwrite prefill_len + ring_pos circularly
// (kv_cache.cpp:54-82; rswa_attention.cu:409-420). One thread updates the
// state; the row reaches the others through LDS.
__device__ __forceinline__ int append_row(int* d_len, int* d_ring_pos, int prefill_len, int window) {
    __shared__ int row_s;
    if (threadIdx.x == 0) {
        const int len = *d_len;
        int row;
        if (len < prefill_len + window) {
            row = len;
            *d_len = len + 1;
            if (len + 1 >= prefill_len + window) *d_ring_pos = 0;
        } else {
            const int rp = *d_ring_pos;
            row = prefill_len + rp;
            *d_ring_pos = (rp + 1) % window;
        }
        row_s = row;
    }
    __syncthreads();
    return row_s;
}

__global__ __launch_bounds__(256) void rswa_append_kernel(const float* k, const float* v, float* kc, float* vc,
                                                          int* d_len, int* d_ring_pos, int prefill_len, int window,
                                                          int stride) {
    const int row = append_row(d_len, d_ring_pos, prefill_len, window);
    copy_row(k, v, kc + (size_t)row * stride, vc + (size_t)row * stride, stride);
}

__global__ __launch_bounds__(256) void rswa_append_batch_kernel(const float* k, const float* v, float* kc, float* vc,
                                                                int* d_len, int* d_ring_pos, const int* d_prefill_len,
                                                                const int* d_slots, int batch_cap, int window,
                                                                int stride) {
    const int b = blockIdx.x, slot = d_slots[b];
    const int row = append_row(d_len + slot, d_ring_pos + slot, d_prefill_len[slot], window);
    const size_t dst = ((size_t)slot * batch_cap + row) * stride;
    copy_row(k + (size_t)b * stride, v + (size_t)b * stride, kc + dst, vc + dst, stride);
}

__global__ __launch_bounds__(256) void rswa_write_ragged_kernel(const float* k, const float* v, float* kc, float* vc,
                                                                const int* d_slots, const int* d_pos, int batch_cap,
                                                                int stride) {
    const int t = blockIdx.x;
    const size_t dst = ((size_t)d_slots[t] * batch_cap + d_pos[t]) * stride;
    copy_row(k + (size_t)t * stride, v + (size_t)t * stride, kc + dst, vc + dst, stride);
}

int check_shape(int heads, int kv_heads, int head_dim) {
    if (heads <= 0 || kv_heads <= 0 || heads % kv_heads)
        return set_error(UOCR_HIP_EINVAL, "heads must be a positive multiple of kv_heads");
    if (head_dim <= 0 || head_dim > 256 || head_dim % 4)
        return set_error(UOCR_HIP_EUNSUPPORTED, "head_dim must be a multiple of 4 in [4, 256]");
    return UOCR_HIP_OK;
}

int check_ptrs(std::initializer_list<const void*> ps) {
    for (const void* p : ps) {
        if (!p) return set_error(UOCR_HIP_EINVAL, "null pointer");
        if ((uintptr_t)p % 16) return set_error(UOCR_HIP_EINVAL, "q, k/v caches and out must be 16-byte aligned");
    }
    return UOCR_HIP_OK;
}

// Partial records of the key-split attention: a library-owned device buffer
// (the reference's attention signatures carry no workspace). Calls that split
// on one device share it, so split calls on different streams of one device
// must not overlap; a call whose records would not fit runs unsplit.
constexpr int kRswaPartRecs = 4096;
__device__ float g_rswa_part[(size_t)kRswaPartRecs * kRswaRec];
std::mutex g_rswa_mu;
float* g_rswa_part_ptr[64] = {};
int g_rswa_cus[64] = {};

// device address of g_rswa_part and the CU count of the current device
int rswa_device(float** part, int* cus) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= 64) return -1;
    std::lock_guard<std::mutex> lock(g_rswa_mu);
    if (!g_rswa_part_ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_rswa_part)) != hipSuccess) return -1;
        if (hipDeviceGetAttribute(&g_rswa_cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
        g_rswa_part_ptr[dev] = static_cast<float*>(p);
    }
    *part = g_rswa_part_ptr[dev];
    *cus = g_rswa_cus[dev];
    return 0;
}

// max_len: an upper bound of any row's key count (0: unknown). When rows x
// heads workgroups cannot fill the chip (decode), the keys of each (row, head)
// are split into chunks of at least 128 keys over up to 8 workgroups, then
// merged by a second kernel.
int launch_attention(RswaArgs a, int rows, hipStream_t st, int max_len) {
    if (rows <= 0) return UOCR_HIP_OK;
    a.scale = 1.0f / sqrtf((float)a.head_dim);
    a.n_chunks = 1;
    float* part = nullptr;
    int cus = 0;
    const long long wgs = (long long)rows * a.heads;
    if (wgs < 512 && rswa_device(&part, &cus) == 0) {
        int n = (int)((2LL * cus + wgs - 1) / wgs);
        if (max_len > 0) n = std::min(n, max_len / 128);
        n = std::min(n, 8);
        while (n > 1 && wgs * n > kRswaPartRecs) --n;
        if (n > 1) {
            a.n_chunks = n;
            a.part = part;
        }
    }
    const dim3 grid(rows, a.heads, a.n_chunks), block(kRswaWaves * 64);
    if (a.head_dim <= 64) launch_k(rswa_kernel<64>, grid, block, 0, st, a);
    else if (a.head_dim <= 128) launch_k(rswa_kernel<128>, grid, block, 0, st, a);
    else launch_k(rswa_kernel<256>, grid, block, 0, st, a);
    if (a.n_chunks > 1)
        launch_k(rswa_merge_kernel, dim3(rows, a.heads), dim3(std::min(256, (a.head_dim + 63) / 64 * 64)), 0, st,
                 (const float*)a.part, a.out, a.heads, a.head_dim, a.n_chunks);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? UOCR_HIP_OK : set_error(UOCR_HIP_EHIP, std::string("rswa launch: ") + hipGetErrorString(e));
}

int launch_done(const char* what) {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? UOCR_HIP_OK : set_error(UOCR_HIP_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace
}  // namespace uocr_hip

using namespace uocr_hip;

extern "C" {

int uocr_hip_rswa_attention_decode(const float* q, const float* kcache, const float* vcache, int kv_len, int heads,
                                   int kv_heads, int head_dim, float* out, void* stream) {
    if (int rc = check_shape(heads, kv_heads, head_dim)) return rc;
    if (int rc = check_ptrs({q, kcache, vcache, out})) return rc;
    if (kv_len < 0) return set_error(UOCR_HIP_EINVAL, "kv_len must be >= 0");
    RswaArgs a{q, kcache, vcache, out, heads, kv_heads, head_dim, 0.f, 0, kv_len, 0, 0, nullptr, nullptr, nullptr, 0};
    return launch_attention(a, 1, (hipStream_t)stream, kv_len);
}

int uocr_hip_rswa_attention(const float* q, const float* kcache, const float* vcache, int kv_len, int seq,
                            int q_start, int heads, int kv_heads, int head_dim, int causal, float* out,
                            void* stream) {
    if (int rc = check_shape(heads, kv_heads, head_dim)) return rc;
    if (int rc = check_ptrs({q, kcache, vcache, out})) return rc;
    if (kv_len < 0 || seq < 0) return set_error(UOCR_HIP_EINVAL, "kv_len and seq must be >= 0");
    RswaArgs a{q, kcache, vcache, out, heads, kv_heads, head_dim, 0.f, 0, kv_len, q_start, causal != 0,
               nullptr, nullptr, nullptr, 0};
    return launch_attention(a, seq, (hipStream_t)stream, kv_len);
}

int uocr_hip_rswa_attention_devlen(const float* q, const float* kcache, const float* vcache, const int* d_len,
                                   int seq, int q_start, int heads, int kv_heads, int head_dim, int causal,
                                   float* out, void* stream) {
    if (int rc = check_shape(heads, kv_heads, head_dim)) return rc;
    if (int rc = check_ptrs({q, kcache, vcache, out})) return rc;
    if (!d_len || seq < 0) return set_error(UOCR_HIP_EINVAL, "null d_len or negative seq");
    RswaArgs a{q, kcache, vcache, out, heads, kv_heads, head_dim, 0.f, 1, 0, q_start, causal != 0,
               d_len, nullptr, nullptr, 0};
    return launch_attention(a, seq, (hipStream_t)stream, 0);
}

int uocr_hip_rswa_attention_batch(const float* q, const float* kcache_base, const float* vcache_base,
                                  const int* d_len, const int* d_slots, int batch, int batch_cap, int heads,
                                  int kv_heads, int head_dim, float* out, void* stream) {
    if (batch <= 0) return UOCR_HIP_OK;  // as the reference: nothing to do
    if (int rc = check_shape(heads, kv_heads, head_dim)) return rc;
    if (int rc = check_ptrs({q, kcache_base, vcache_base, out})) return rc;
    if (!d_len || !d_slots || batch_cap <= 0) return set_error(UOCR_HIP_EINVAL, "null d_len/d_slots or batch_cap <= 0");
    RswaArgs a{q, kcache_base, vcache_base, out, heads, kv_heads, head_dim, 0.f, 2, 0, 0, 0,
               d_len, d_slots, nullptr, batch_cap};
    return launch_attention(a, batch, (hipStream_t)stream, batch_cap);
}

int uocr_hip_rswa_attention_ragged(const float* q, const float* kcache_base, const float* vcache_base,
                                   const int* d_slots, const int* d_pos, int total, int batch_cap, int heads,
                                   int kv_heads, int head_dim, float* out, void* stream) {
    if (total <= 0) return UOCR_HIP_OK;
    if (int rc = check_shape(heads, kv_heads, head_dim)) return rc;
    if (int rc = check_ptrs({q, kcache_base, vcache_base, out})) return rc;
    if (!d_slots || !d_pos || batch_cap <= 0) return set_error(UOCR_HIP_EINVAL, "null d_slots/d_pos or batch_cap <= 0");
    RswaArgs a{q, kcache_base, vcache_base, out, heads, kv_heads, head_dim, 0.f, 3, 0, 0, 0,
               nullptr, d_slots, d_pos, batch_cap};
    return launch_attention(a, total, (hipStream_t)stream, batch_cap);
}

int uocr_hip_rswa_append_decode(const float* k, const float* v, float* kcache, float* vcache, int* d_len,
                                int* d_ring_pos, int prefill_len, int window, int kv_heads, int head_dim,
                                void* stream) {
    if (int rc = check_shape(kv_heads, kv_heads, head_dim)) return rc;
    if (int rc = check_ptrs({k, v, kcache, vcache})) return rc;
    if (!d_len || !d_ring_pos || window <= 0 || prefill_len < 0)
        return set_error(UOCR_HIP_EINVAL, "null state or window <= 0");
    launch_k(rswa_append_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, k, v, kcache, vcache, d_len, d_ring_pos,
             prefill_len, window, kv_heads * head_dim);
    return launch_done("rswa append");
}

int uocr_hip_rswa_append_decode_batch(const float* k, const float* v, float* kcache_base, float* vcache_base,
                                      int* d_len, int* d_ring_pos, const int* d_prefill_len, const int* d_slots,
                                      int batch, int batch_cap, int window, int kv_heads, int head_dim,
                                      void* stream) {
    if (batch <= 0) return UOCR_HIP_OK;
    if (int rc = check_shape(kv_heads, kv_heads, head_dim)) return rc;
    if (int rc = check_ptrs({k, v, kcache_base, vcache_base})) return rc;
    if (!d_len || !d_ring_pos || !d_prefill_len || !d_slots || window <= 0 || batch_cap <= 0)
        return set_error(UOCR_HIP_EINVAL, "null state arrays, window <= 0 or batch_cap <= 0");
    launch_k(rswa_append_batch_kernel, dim3(batch), dim3(256), 0, (hipStream_t)stream, k, v, kcache_base, vcache_base,
             d_len, d_ring_pos, d_prefill_len, d_slots, batch_cap, window, kv_heads * head_dim);
    return launch_done("rswa batch append");
}

int uocr_hip_rswa_write_prefill_ragged(const float* k, const float* v, float* kcache_base, float* vcache_base,
                                       const int* d_slots, const int* d_pos, int total, int batch_cap, int kv_heads,
                                       int head_dim, void* stream) {
    if (total <= 0) return UOCR_HIP_OK;
    if (int rc = check_shape(kv_heads, kv_heads, head_dim)) return rc;
    if (int rc = check_ptrs({k, v, kcache_base, vcache_base})) return rc;
    if (!d_slots || !d_pos || batch_cap <= 0) return set_error(UOCR_HIP_EINVAL, "null d_slots/d_pos or batch_cap <= 0");
    launch_k(rswa_write_ragged_kernel, dim3(total), dim3(256), 0, (hipStream_t)stream, k, v, kcache_base, vcache_base,
             d_slots, d_pos, batch_cap, kv_heads * head_dim);
    return launch_done("rswa ragged write");
}

}  // extern "C"
