// Decode-sized MoE layer (seq < 256): router, expert passes and combine with
// no grouping kernel and no cross-workgroup synchronisation.
//
// The reference routes a decode batch on the host and re-reads every weight row
// once per assigned token (src/engine/gpu_decoder.cu:591-609,
// src/kernels/cuda/moe_device.cu:199-268). Here:
//   * router_decode_kernel gives every token its own workgroup (lane e of wave 0
//     = expert e), so the reference's sequential fmaf chain per (token, expert)
//     runs on T different CUs at once; the f32 router matrix streams through an
//     LDS ring filled by all four waves;
//   * the expert kernels are launched over (expert, 64-row block) for every
//     expert. Each workgroup reads the routing ids (T*top_k ints) and derives
//     its expert's token list and slot base itself -- the stable grouping of
//     gpu_decoder.cu:602-609 (tokens ascending) -- so no grouping pass or tile
//     list sits between the router and the weight stream. An expert with no
//     tokens exits before loading anything; a live one loads its 64 weight rows
//     into registers ONCE and applies them to all of its 16-token m-tiles;
//   * the down pass writes y by entry ((t, j) at t*top_k + j, shared group v at
//     T*top_k + v*T + t), so the combine needs no routing lookups.
// act slot layout: shared-expert ("virtual") groups first, slot v*T + t, then
// the routed groups in expert order, slot n_virtual*T + offset(e) + rank.
#include "launch.hpp"
#include "routing.hpp"

#include <algorithm>
#include <type_traits>

#if defined(UOCR_DBG)
__device__ unsigned long long uocr_dbg_ts[64 * 64];
extern "C" hipError_t uocr_dbg_read(void* host, size_t bytes) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(uocr_dbg_ts), bytes, 0, hipMemcpyDeviceToHost);
}
#define RDBG(i) \
    if (threadIdx.x == 0 && blockIdx.x < 64) uocr_dbg_ts[blockIdx.x * 64 + (i)] = wall_clock64();
__device__ unsigned long long uocr_dbg_ex[2][80 * 20 * 8];
extern "C" hipError_t uocr_dbg_read_ex(void* host, size_t bytes) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(uocr_dbg_ex), bytes, 0, hipMemcpyDeviceToHost);
}
#define EDBG(i) \
    if (threadIdx.x == 0 && blockIdx.x < 80 && blockIdx.y < 20) uocr_dbg_ex[GU ? 0 : 1][(blockIdx.y * 80 + blockIdx.x) * 8 + (i)] = wall_clock64();
#else
#define RDBG(i)
#define EDBG(i)
#endif

namespace uocr_hip {

// ---------------------------------------------------------------------------
// routing helpers shared with the router kernels
// ---------------------------------------------------------------------------

// ---------------------------------------------------------------------------
// Router: one token per workgroup of one wave.
// ---------------------------------------------------------------------------
constexpr int kMaxHidden = 1792;

template <typename XT>
__device__ __forceinline__ void load8(const XT* p, float* out);
template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t* p, float* out) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[2 * i] = __uint_as_float(v[i] << 16);
        out[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
    }
}
template <>
__device__ __forceinline__ void load8<float>(const float* p, float* out) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
    const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[i] = a[i];
        out[4 + i] = b[i];
    }
}

// The router matrix streams through an LDS ring of 16 KiB chunks (64 columns x
// 64 experts x f32, [H/4][64][4] in HBM) filled by direct global->LDS loads
// from all four waves; wave 0 runs the 64 FMA chains out of LDS. Eight chunks
// (512 columns) are in flight at a time.
constexpr int kRChunkCols = 128;
constexpr int kRChunkBytes = kRChunkCols * 64 * 4;  // 32 KiB
constexpr int kRRing = 4;
constexpr int kRChunkLoads = kRChunkBytes / 1024;   // 1 KiB per wave load
// DMA loads per chunk issued by producer wave w (1..3): units w-1, w+2, ...
__host__ __device__ constexpr int router_loads_of(int wave) { return (kRChunkLoads - (wave - 1) + 2) / 3; }

// s_waitcnt vmcnt(n) (n <= 63), leaving expcnt / lgkmcnt unconstrained
template <int N>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
// s_waitcnt vmcnt(n) for a wave-uniform runtime n (values above 31 wait for 0)
__device__ __forceinline__ void wait_vm_n(int n) {
    switch (n) {
#define UOCR_VM(k) case k: wait_vm<k>(); break;
        UOCR_VM(1) UOCR_VM(2) UOCR_VM(3) UOCR_VM(4) UOCR_VM(5) UOCR_VM(6) UOCR_VM(7) UOCR_VM(8)
        UOCR_VM(9) UOCR_VM(10) UOCR_VM(11) UOCR_VM(12) UOCR_VM(13) UOCR_VM(14) UOCR_VM(15) UOCR_VM(16)
        UOCR_VM(17) UOCR_VM(18) UOCR_VM(19) UOCR_VM(20) UOCR_VM(21) UOCR_VM(22) UOCR_VM(23) UOCR_VM(24)
        UOCR_VM(25) UOCR_VM(26) UOCR_VM(27) UOCR_VM(28) UOCR_VM(29) UOCR_VM(30) UOCR_VM(31)
#undef UOCR_VM
        default: wait_vm<0>(); break;
    }
}

__device__ __forceinline__ void router_issue_chunk(const float* w, int chunk, unsigned char* ring, int wave, int lane) {
    const unsigned char* src = reinterpret_cast<const unsigned char*>(w) + (size_t)chunk * kRChunkBytes;
    unsigned char* dst = ring + (size_t)(chunk % kRRing) * kRChunkBytes;
    for (int unit = wave - 1; unit < kRChunkLoads; unit += 3)  // 1 KiB per wave instruction
        load_lds16(src + ((size_t)unit * 64 + lane) * 16, dst + (size_t)unit * 1024);
}

// LDS byte address of a __shared__ object
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// LDS operands of one k-tile: four A fragments (1 KiB apart) and the scale
// words of one or two scale rows (the GPT groups of the k-tile; MFMA step s
// uses group (s * GPT) / 4). lds_issue_tile only issues the six reads (the
// registers must not be used before lds_wait_tile); reading through asm keeps
// the compiler's LDS-DMA tracking from turning the first read into a wait for
// every outstanding global load.
template <int GPT>
struct TileRegs {
    f16x8 av[4];
    // GPT 4: four scales in 64 bits; GPT 2 / 1: two / one in 32 bits
    typename std::conditional<GPT == 4, uint64_t, uint32_t>::type w0, w1;
};

template <int GPT>
__device__ __forceinline__ void lds_issue_tile(uint32_t a_addr, uint32_t s0_addr, uint32_t s1_addr, TileRegs<GPT>& t) {
#define UOCR_TILE_READS(SREAD)                                                                        \
    asm volatile("ds_read_b128 %0, %6\n"                                                             \
                 "ds_read_b128 %1, %6 offset:1024\n"                                                 \
                 "ds_read_b128 %2, %6 offset:2048\n"                                                 \
                 "ds_read_b128 %3, %6 offset:3072\n" SREAD " %4, %7\n" SREAD " %5, %8\n"             \
                 : "=&v"(t.av[0]), "=&v"(t.av[1]), "=&v"(t.av[2]), "=&v"(t.av[3]), "=&v"(t.w0), "=&v"(t.w1) \
                 : "v"(a_addr), "v"(s0_addr), "v"(s1_addr)                                          \
                 : "memory")
    if constexpr (GPT == 4) {
        UOCR_TILE_READS("ds_read_b64");
    } else if constexpr (GPT == 2) {
        UOCR_TILE_READS("ds_read_b32");
    } else {
        UOCR_TILE_READS("ds_read_u16");
    }
#undef UOCR_TILE_READS
}

// Wait until at most `later` LDS reads (issued after this tile's) are
// outstanding, then unpack the scales.
template <int GPT, int LATER>
__device__ __forceinline__ void lds_wait_tile(TileRegs<GPT>& t, f16* s0, f16* s1) {
    asm volatile("s_waitcnt lgkmcnt(%6)"
                 : "+v"(t.av[0]), "+v"(t.av[1]), "+v"(t.av[2]), "+v"(t.av[3]), "+v"(t.w0), "+v"(t.w1)
                 : "n"(LATER));
    const uint64_t x0 = t.w0, x1 = t.w1;
    const uint32_t w0[2] = {(uint32_t)x0, (uint32_t)(x0 >> 32)};
    const uint32_t w1[2] = {(uint32_t)x1, (uint32_t)(x1 >> 32)};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int gi = (s * GPT) >> 2;  // group within the k-tile
        s0[s] = __builtin_bit_cast(f16, (uint16_t)((w0[gi >> 1] >> (16 * (gi & 1))) & 0xffffu));
        s1[s] = __builtin_bit_cast(f16, (uint16_t)((w1[gi >> 1] >> (16 * (gi & 1))) & 0xffffu));
    }
}

// Workgroup barrier that orders LDS only: __syncthreads() would also wait for
// every outstanding global load (vmcnt(0)), draining the ring.
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt unconstrained
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <typename XT, bool RMS>
__global__ __launch_bounds__(256) void router_decode_kernel(DecodeArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char rsmem[];
    unsigned char* ring = rsmem;
    float* xs = reinterpret_cast<float*>(rsmem + kRRing * kRChunkBytes);
    __shared__ __attribute__((aligned(16))) float sc[64];
    __shared__ float topv[kMaxTopK];
    __shared__ uint64_t etab[32];
    const int t = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int H = a.hidden, E = a.n_experts, K = a.top_k;
    if (tid < 32) etab[tid] = uocr_exp2_tab[tid];
    const int NCH = H / kRChunkCols;
    const XT* x = static_cast<const XT*>(a.x) + (size_t)t * H;
    RDBG(0)

    // waves 1..3 start the router-matrix ring; wave 0 loads the token row -> xs (f32)
    if (wave != 0) {
        for (int ch = 0; ch < kRRing && ch < NCH; ++ch) router_issue_chunk(a.router_f32, ch, ring, wave, lane);
    } else {
        for (int c = lane * 8; c < H; c += 64 * 8) {
            float v[8];
            load8<XT>(x + c, v);
            *reinterpret_cast<f32x4*>(xs + c) = f32x4{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<f32x4*>(xs + c + 4) = f32x4{v[4], v[5], v[6], v[7]};
        }
    }
    lds_barrier();  // xs
    RDBG(1)

    if constexpr (RMS) {
        // src/kernels/cpu_ops.cpp:58-67 as the reference build computes it: the
        // products x*x rounded, summed in column order; the last H % 4 terms fused
        if (tid == 0) {
            float ss = 0.0f;
            const int h4 = H & ~3;
            for (int c = 0; c < h4; c += 4) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(xs + c);
#pragma unroll
                for (int i = 0; i < 4; ++i) ss = __fadd_rn(ss, __fmul_rn(v[i], v[i]));
            }
            for (int c = h4; c < H; ++c) ss = fmaf(xs[c], xs[c], ss);
            sc[0] = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)H), a.rms_eps)));
        }
        __syncthreads();
        const float inv = sc[0];
        for (int c = tid; c < H; c += 256) xs[c] = __fmul_rn(__fmul_rn(xs[c], inv), a.rms_weight[c]);
        __syncthreads();
    }

    // f16 expert input (waves 1..3; wave 0 starts its chains)
    if (wave > 0)
        for (int c = (tid - 64) * 8; c < H; c += 192 * 8) {
            const f32x4 p = *reinterpret_cast<const f32x4*>(xs + c);
            const f32x4 q = *reinterpret_cast<const f32x4*>(xs + c + 4);
            const f16x8 h = {(f16)p[0], (f16)p[1], (f16)p[2], (f16)p[3], (f16)q[0], (f16)q[1], (f16)q[2], (f16)q[3]};
            *reinterpret_cast<f16x8*>(a.x16 + (size_t)t * H + c) = h;
        }

    // logits: lane e of wave 0 runs the reference's sequential fmaf chain,
    // columns ascending (src/kernels/cpu_ops.cpp:26-39, contracted by the
    // -march=native build). Waves 1..3 keep the ring filled; wave 0 only
    // computes.
    float acc = 0.0f;
    const int my_loads = wave == 0 ? 0 : router_loads_of(wave);
    for (int ch = 0; ch < NCH; ++ch) {
        // chunks this wave has issued so far: 0 .. last
        const int last = min(NCH - 1, max(kRRing - 1, ch - 2 + kRRing));
        if (wave != 0) wait_vm_n(my_loads * (last - ch));
        lds_barrier();
        if (wave != 0 && ch >= 1 && ch - 1 + kRRing < NCH)
            router_issue_chunk(a.router_f32, ch - 1 + kRRing, ring, wave, lane);
        if (wave == 0) {
            // 32 steps of 4 columns: the LDS reads run 6 steps (12 reads) ahead
            // of the FMA chain, with explicit lgkmcnt waits (the compiler's own
            // schedule waits for every read pair)
            const uint32_t w_addr = lds_addr(ring + (size_t)(ch % kRRing) * kRChunkBytes) + lane * 16;
            const uint32_t x_addr = lds_addr(xs + ch * kRChunkCols);
            asm volatile(
                "s_waitcnt lgkmcnt(0)\n"
                "ds_read_b128 v[64:67], %[w] offset:0\n"
                "ds_read_b128 v[68:71], %[x] offset:0\n"
                "ds_read_b128 v[72:75], %[w] offset:1024\n"
                "ds_read_b128 v[76:79], %[x] offset:16\n"
                "ds_read_b128 v[80:83], %[w] offset:2048\n"
                "ds_read_b128 v[84:87], %[x] offset:32\n"
                "ds_read_b128 v[88:91], %[w] offset:3072\n"
                "ds_read_b128 v[92:95], %[x] offset:48\n"
                "ds_read_b128 v[96:99], %[w] offset:4096\n"
                "ds_read_b128 v[100:103], %[x] offset:64\n"
                "ds_read_b128 v[104:107], %[w] offset:5120\n"
                "ds_read_b128 v[108:111], %[x] offset:80\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v68, v64\n"
                "v_fmac_f32 %[acc], v69, v65\n"
                "v_fmac_f32 %[acc], v70, v66\n"
                "v_fmac_f32 %[acc], v71, v67\n"
                "ds_read_b128 v[64:67], %[w] offset:6144\n"
                "ds_read_b128 v[68:71], %[x] offset:96\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v76, v72\n"
                "v_fmac_f32 %[acc], v77, v73\n"
                "v_fmac_f32 %[acc], v78, v74\n"
                "v_fmac_f32 %[acc], v79, v75\n"
                "ds_read_b128 v[72:75], %[w] offset:7168\n"
                "ds_read_b128 v[76:79], %[x] offset:112\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v84, v80\n"
                "v_fmac_f32 %[acc], v85, v81\n"
                "v_fmac_f32 %[acc], v86, v82\n"
                "v_fmac_f32 %[acc], v87, v83\n"
                "ds_read_b128 v[80:83], %[w] offset:8192\n"
                "ds_read_b128 v[84:87], %[x] offset:128\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v92, v88\n"
                "v_fmac_f32 %[acc], v93, v89\n"
                "v_fmac_f32 %[acc], v94, v90\n"
                "v_fmac_f32 %[acc], v95, v91\n"
                "ds_read_b128 v[88:91], %[w] offset:9216\n"
                "ds_read_b128 v[92:95], %[x] offset:144\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v100, v96\n"
                "v_fmac_f32 %[acc], v101, v97\n"
                "v_fmac_f32 %[acc], v102, v98\n"
                "v_fmac_f32 %[acc], v103, v99\n"
                "ds_read_b128 v[96:99], %[w] offset:10240\n"
                "ds_read_b128 v[100:103], %[x] offset:160\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v108, v104\n"
                "v_fmac_f32 %[acc], v109, v105\n"
                "v_fmac_f32 %[acc], v110, v106\n"
                "v_fmac_f32 %[acc], v111, v107\n"
                "ds_read_b128 v[104:107], %[w] offset:11264\n"
                "ds_read_b128 v[108:111], %[x] offset:176\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v68, v64\n"
                "v_fmac_f32 %[acc], v69, v65\n"
                "v_fmac_f32 %[acc], v70, v66\n"
                "v_fmac_f32 %[acc], v71, v67\n"
                "ds_read_b128 v[64:67], %[w] offset:12288\n"
                "ds_read_b128 v[68:71], %[x] offset:192\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v76, v72\n"
                "v_fmac_f32 %[acc], v77, v73\n"
                "v_fmac_f32 %[acc], v78, v74\n"
                "v_fmac_f32 %[acc], v79, v75\n"
                "ds_read_b128 v[72:75], %[w] offset:13312\n"
                "ds_read_b128 v[76:79], %[x] offset:208\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v84, v80\n"
                "v_fmac_f32 %[acc], v85, v81\n"
                "v_fmac_f32 %[acc], v86, v82\n"
                "v_fmac_f32 %[acc], v87, v83\n"
                "ds_read_b128 v[80:83], %[w] offset:14336\n"
                "ds_read_b128 v[84:87], %[x] offset:224\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v92, v88\n"
                "v_fmac_f32 %[acc], v93, v89\n"
                "v_fmac_f32 %[acc], v94, v90\n"
                "v_fmac_f32 %[acc], v95, v91\n"
                "ds_read_b128 v[88:91], %[w] offset:15360\n"
                "ds_read_b128 v[92:95], %[x] offset:240\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v100, v96\n"
                "v_fmac_f32 %[acc], v101, v97\n"
                "v_fmac_f32 %[acc], v102, v98\n"
                "v_fmac_f32 %[acc], v103, v99\n"
                "ds_read_b128 v[96:99], %[w] offset:16384\n"
                "ds_read_b128 v[100:103], %[x] offset:256\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v108, v104\n"
                "v_fmac_f32 %[acc], v109, v105\n"
                "v_fmac_f32 %[acc], v110, v106\n"
                "v_fmac_f32 %[acc], v111, v107\n"
                "ds_read_b128 v[104:107], %[w] offset:17408\n"
                "ds_read_b128 v[108:111], %[x] offset:272\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v68, v64\n"
                "v_fmac_f32 %[acc], v69, v65\n"
                "v_fmac_f32 %[acc], v70, v66\n"
                "v_fmac_f32 %[acc], v71, v67\n"
                "ds_read_b128 v[64:67], %[w] offset:18432\n"
                "ds_read_b128 v[68:71], %[x] offset:288\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v76, v72\n"
                "v_fmac_f32 %[acc], v77, v73\n"
                "v_fmac_f32 %[acc], v78, v74\n"
                "v_fmac_f32 %[acc], v79, v75\n"
                "ds_read_b128 v[72:75], %[w] offset:19456\n"
                "ds_read_b128 v[76:79], %[x] offset:304\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v84, v80\n"
                "v_fmac_f32 %[acc], v85, v81\n"
                "v_fmac_f32 %[acc], v86, v82\n"
                "v_fmac_f32 %[acc], v87, v83\n"
                "ds_read_b128 v[80:83], %[w] offset:20480\n"
                "ds_read_b128 v[84:87], %[x] offset:320\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v92, v88\n"
                "v_fmac_f32 %[acc], v93, v89\n"
                "v_fmac_f32 %[acc], v94, v90\n"
                "v_fmac_f32 %[acc], v95, v91\n"
                "ds_read_b128 v[88:91], %[w] offset:21504\n"
                "ds_read_b128 v[92:95], %[x] offset:336\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v100, v96\n"
                "v_fmac_f32 %[acc], v101, v97\n"
                "v_fmac_f32 %[acc], v102, v98\n"
                "v_fmac_f32 %[acc], v103, v99\n"
                "ds_read_b128 v[96:99], %[w] offset:22528\n"
                "ds_read_b128 v[100:103], %[x] offset:352\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v108, v104\n"
                "v_fmac_f32 %[acc], v109, v105\n"
                "v_fmac_f32 %[acc], v110, v106\n"
                "v_fmac_f32 %[acc], v111, v107\n"
                "ds_read_b128 v[104:107], %[w] offset:23552\n"
                "ds_read_b128 v[108:111], %[x] offset:368\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v68, v64\n"
                "v_fmac_f32 %[acc], v69, v65\n"
                "v_fmac_f32 %[acc], v70, v66\n"
                "v_fmac_f32 %[acc], v71, v67\n"
                "ds_read_b128 v[64:67], %[w] offset:24576\n"
                "ds_read_b128 v[68:71], %[x] offset:384\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v76, v72\n"
                "v_fmac_f32 %[acc], v77, v73\n"
                "v_fmac_f32 %[acc], v78, v74\n"
                "v_fmac_f32 %[acc], v79, v75\n"
                "ds_read_b128 v[72:75], %[w] offset:25600\n"
                "ds_read_b128 v[76:79], %[x] offset:400\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v84, v80\n"
                "v_fmac_f32 %[acc], v85, v81\n"
                "v_fmac_f32 %[acc], v86, v82\n"
                "v_fmac_f32 %[acc], v87, v83\n"
                "ds_read_b128 v[80:83], %[w] offset:26624\n"
                "ds_read_b128 v[84:87], %[x] offset:416\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v92, v88\n"
                "v_fmac_f32 %[acc], v93, v89\n"
                "v_fmac_f32 %[acc], v94, v90\n"
                "v_fmac_f32 %[acc], v95, v91\n"
                "ds_read_b128 v[88:91], %[w] offset:27648\n"
                "ds_read_b128 v[92:95], %[x] offset:432\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v100, v96\n"
                "v_fmac_f32 %[acc], v101, v97\n"
                "v_fmac_f32 %[acc], v102, v98\n"
                "v_fmac_f32 %[acc], v103, v99\n"
                "ds_read_b128 v[96:99], %[w] offset:28672\n"
                "ds_read_b128 v[100:103], %[x] offset:448\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v108, v104\n"
                "v_fmac_f32 %[acc], v109, v105\n"
                "v_fmac_f32 %[acc], v110, v106\n"
                "v_fmac_f32 %[acc], v111, v107\n"
                "ds_read_b128 v[104:107], %[w] offset:29696\n"
                "ds_read_b128 v[108:111], %[x] offset:464\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v68, v64\n"
                "v_fmac_f32 %[acc], v69, v65\n"
                "v_fmac_f32 %[acc], v70, v66\n"
                "v_fmac_f32 %[acc], v71, v67\n"
                "ds_read_b128 v[64:67], %[w] offset:30720\n"
                "ds_read_b128 v[68:71], %[x] offset:480\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v76, v72\n"
                "v_fmac_f32 %[acc], v77, v73\n"
                "v_fmac_f32 %[acc], v78, v74\n"
                "v_fmac_f32 %[acc], v79, v75\n"
                "ds_read_b128 v[72:75], %[w] offset:31744\n"
                "ds_read_b128 v[76:79], %[x] offset:496\n"
                "s_waitcnt lgkmcnt(10)\n"
                "v_fmac_f32 %[acc], v84, v80\n"
                "v_fmac_f32 %[acc], v85, v81\n"
                "v_fmac_f32 %[acc], v86, v82\n"
                "v_fmac_f32 %[acc], v87, v83\n"
                "s_waitcnt lgkmcnt(8)\n"
                "v_fmac_f32 %[acc], v92, v88\n"
                "v_fmac_f32 %[acc], v93, v89\n"
                "v_fmac_f32 %[acc], v94, v90\n"
                "v_fmac_f32 %[acc], v95, v91\n"
                "s_waitcnt lgkmcnt(6)\n"
                "v_fmac_f32 %[acc], v100, v96\n"
                "v_fmac_f32 %[acc], v101, v97\n"
                "v_fmac_f32 %[acc], v102, v98\n"
                "v_fmac_f32 %[acc], v103, v99\n"
                "s_waitcnt lgkmcnt(4)\n"
                "v_fmac_f32 %[acc], v108, v104\n"
                "v_fmac_f32 %[acc], v109, v105\n"
                "v_fmac_f32 %[acc], v110, v106\n"
                "v_fmac_f32 %[acc], v111, v107\n"
                "s_waitcnt lgkmcnt(2)\n"
                "v_fmac_f32 %[acc], v68, v64\n"
                "v_fmac_f32 %[acc], v69, v65\n"
                "v_fmac_f32 %[acc], v70, v66\n"
                "v_fmac_f32 %[acc], v71, v67\n"
                "s_waitcnt lgkmcnt(0)\n"
                "v_fmac_f32 %[acc], v76, v72\n"
                "v_fmac_f32 %[acc], v77, v73\n"
                "v_fmac_f32 %[acc], v78, v74\n"
                "v_fmac_f32 %[acc], v79, v75\n"
                : [acc] "+v"(acc)
                : [w] "v"(w_addr), [x] "v"(x_addr)
                : "v64", "v65", "v66", "v67", "v68", "v69", "v70", "v71", "v72", "v73", "v74", "v75", "v76", "v77", "v78", "v79", "v80", "v81", "v82", "v83", "v84", "v85", "v86", "v87", "v88", "v89", "v90", "v91", "v92", "v93", "v94", "v95", "v96", "v97", "v98", "v99", "v100", "v101", "v102", "v103", "v104", "v105", "v106", "v107", "v108", "v109", "v110", "v111", "memory");
        }
    }
    RDBG(40)
    // scoring (src/kernels/cpu_ops.cpp:93-106 softmax, or sigmoid) and greedy
    // top-k (src/engine/moe_decoder.cpp:264-287) by wave 0 alone: its LDS
    // accesses are ordered within the wave, so no workgroup barrier is needed
    if (wave != 0) return;
    float p;
    if (a.scoring_sigmoid) {
        p = __fdiv_rn(1.0f, 1.0f + ref_expf(-acc, etab));
    } else {
        float mx = lane < E ? acc : -INFINITY;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
        const float ev = lane < E ? ref_expf(acc - mx, etab) : 0.0f;
        sc[lane] = ev;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        const float sum = ordered_sum64(sc, E);  // expert order
        p = ev * __fdiv_rn(1.0f, sum);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
    RDBG(42)
    sc[lane] = lane < E ? p : -1.0f;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const int rank = lane < E ? greedy_rank64(sc, lane, p) : 64;  // sc[E..64) holds -1 (below every score)
    if (rank < K) topv[rank] = p;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    RDBG(43)
    if (lane < K) {
        float wj = topv[lane];
        if (K > 1 && a.norm_topk_prob) {  // moe_decoder.cpp:280-284
            float s = 0.0f;
            for (int j = 0; j < K; ++j) s += topv[j];
            wj = __fdiv_rn(wj, s + 1e-20f) * a.scaling;
        } else {
            wj *= a.scaling;
        }
        a.wts[(size_t)t * K + lane] = wj;
    }
    if (rank < K) a.ids[(size_t)t * K + rank] = lane;
    RDBG(41)
}

// ---------------------------------------------------------------------------
// Expert pass. Workgroup = (expert or virtual group, 64 output rows = 4 waves
// x 16 rows); weights in the tile-16x128 layout (common.hpp), held in
// registers across the expert's m-tiles.
// ---------------------------------------------------------------------------
constexpr int kDecBM = 16;
constexpr int kDecodeMaxEntries = 256 * kMaxTopK;  // seq < 256

template <int GPT, int KT, bool GU>
__global__ __launch_bounds__(256) void expert_decode_kernel(DecodeArgs a) {
    constexpr int K = KT * kTileK;
    constexpr int NG = scale_row_stride(K, kTileK / GPT);
    constexpr int SROW = kTileRows * NG;
    __shared__ __attribute__((aligned(16))) f16 As[KT * 4 * 64 * 8];
    __shared__ __attribute__((aligned(16))) f16 Ss[4][GU ? 2 : 1][SROW];
    __shared__ int ent[256];
    __shared__ int ids_s[kDecodeMaxEntries];
    __shared__ int hist[kMaxExperts], offs[kMaxExperts], live[kMaxExperts];
    __shared__ int n_live_s;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int T = a.seq, E = a.n_experts, N = T * a.top_k;
    const int n_rows = GU ? a.inter : a.hidden;
    const int RBG = (n_rows / kTileRows + 3) / 4;  // 64-row groups per expert

    // Routing summary, identical in every workgroup: per-expert counts, slot
    // offsets (stable grouping, experts ascending) and the list of live groups
    // (routed experts with tokens, then the shared-expert groups).
    for (int e = tid; e < kMaxExperts; e += 256) hist[e] = 0;
    for (int i = tid; i < N; i += 256) ids_s[i] = a.ids[i];
    __syncthreads();
    for (int i = tid; i < N; i += 256) atomicAdd(&hist[ids_s[i]], 1);
    __syncthreads();
    if (wave == 0) {
        int run_off = 0, run_live = 0;
        for (int e0 = 0; e0 < E; e0 += 64) {
            const int e = e0 + lane;
            const int c = e < E ? hist[e] : 0;
            int inc = c;  // inclusive scan of counts over the wave
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int u = __shfl_up(inc, o, kWave);
                if (lane >= o) inc += u;
            }
            if (e < E) offs[e] = run_off + inc - c;
            run_off += __shfl(inc, 63, kWave);
            const uint64_t m = __ballot(c > 0);
            if (c > 0) live[run_live + __popcll(m & ((1ull << lane) - 1))] = e;
            run_live += __popcll(m);
        }
        for (int v = lane; v < a.n_virtual; v += 64) live[run_live + v] = E + v;
        if (lane == 0) n_live_s = run_live + a.n_virtual;
    }
    __syncthreads();
    const int n_items = n_live_s * RBG;

    const int r = lane & 15;
    const uint8_t* wsrc0 = GU ? a.gate : a.down;
    const uint16_t* ssrc0 = GU ? a.gate_s : a.down_s;
    const long long wstr = GU ? a.gu_wstride : a.dn_wstride;
    const long long sstr = GU ? a.gu_sstride : a.dn_sstride;

    // work items (live group, 64-row block): grid-strided, so experts without
    // tokens never occupy a workgroup slot
    for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
        const int g = live[item / RBG];
        const int rb = (item % RBG) * 4 + wave;
        const bool wave_live = rb * kTileRows < n_rows;
        const int cnt = g < E ? hist[g] : T;
        const int slot_base = g < E ? a.n_virtual * T + offs[g] : (g - E) * T;
        // the group's entries (t * top_k + j), ascending; every wave writes
        // the same values and reads back its own writes
        if (g < E) {
            const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
            int run = 0;
            for (int base = 0; base < N; base += 64) {
                const int i = base + lane;
                const bool hit = i < N && ids_s[i] == g;
                const uint64_t m = __ballot(hit);
                if (hit) ent[run + __popcll(m & below)] = i;
                run += __popcll(m);
            }
        } else {
            for (int i = lane; i < T; i += 64) ent[i] = i;
        }
        __builtin_amdgcn_wave_barrier();

        // A rows of an m-tile into LDS (fragments (kt, s = wave), row r = lane % 16)
        auto stage_a = [&](int m0) {
            const int rows = min(kDecBM, cnt - m0);
            if (r < rows) {
                // gate/up: x16 row of the entry's token; down: the slot's act row
                const int row = GU ? (g < E ? ent[m0 + r] / a.top_k : ent[m0 + r]) : slot_base + m0 + r;
                const f16* src = (GU ? a.x16 : a.act) + (size_t)row * K + wave * 32 + 8 * (lane >> 4);
#pragma unroll
                for (int kt = 0; kt < KT; ++kt) load_lds16(src + kt * kTileK, As + (size_t)(kt * 4 + wave) * 64 * 8);
            }
        };
        stage_a(0);

        // this wave's scale rows (LDS) and 16 x K weights (registers); no
        // branch around the weight loads (a wave past the last row block
        // reloads the last one and discards it), so the compiler tracks them
        // in issue order and waits k-tile by k-tile
        u32x4 bw0[KT], bw1[KT];
        {
            const int rbl = min(rb, n_rows / kTileRows - 1);
            const size_t sb = (size_t)g * sstr + (size_t)rbl * SROW;
            for (int i = lane; i * 8 < SROW; i += 64) {
                load_lds16(ssrc0 + sb + i * 8, &Ss[wave][0][(i & ~63) * 8]);
                if constexpr (GU) load_lds16(a.up_s + sb + i * 8, &Ss[wave][GU ? 1 : 0][(i & ~63) * 8]);
            }
            const size_t toff = (size_t)g * wstr + (size_t)rbl * KT * kTileBytes + (size_t)lane * 16;
#pragma unroll
            for (int kt = 0; kt < KT; ++kt) {
#if defined(UOCR_NOLOAD)
                bw0[kt] = u32x4{(uint32_t)(toff + kt), 1u, 2u, 3u};
                if constexpr (GU) bw1[kt] = u32x4{(uint32_t)(toff * 3 + kt), 1u, 2u, 3u};
#else
                bw0[kt] = *reinterpret_cast<const u32x4*>(wsrc0 + toff + (size_t)kt * kTileBytes);
                if constexpr (GU) bw1[kt] = *reinterpret_cast<const u32x4*>(a.up + toff + (size_t)kt * kTileBytes);
#endif
            }
        }

        const f16* srow0 = &Ss[wave][0][r * NG];
        const f16* srow1 = &Ss[wave][GU ? 1 : 0][r * NG];
        const int col = rb * kTileRows + r;
        // one m-tile: MFMAs over all k-tiles and the stores
        auto tile = [&](int m0, bool first) {
            if (!wave_live) return;
            const int rows = min(kDecBM, cnt - m0);
            f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
            const uint32_t a_base = lds_addr(As + (size_t)lane * 8);
            const uint32_t s_base0 = lds_addr(srow0), s_base1 = lds_addr(srow1);
            TileRegs<GPT> tr[2];
            lds_issue_tile<GPT>(a_base, s_base0, s_base1, tr[0]);
#pragma unroll
            for (int kt = 0; kt < KT; ++kt) {
                // for later m-tiles the weights are opaque to the optimiser:
                // hoisting their unpacking out of the m-tile loop would quadruple
                // the registers they occupy
                if (!first) {
                    asm volatile("" : "+v"(bw0[kt]));
                    if constexpr (GU) asm volatile("" : "+v"(bw1[kt]));
                }
                f16 s0[4], s1[4];
                // this k-tile's LDS operands were issued one k-tile ahead; issue
                // the next k-tile's before waiting for these
                if (kt + 1 < KT) {
                    lds_issue_tile<GPT>(a_base + (uint32_t)((kt + 1) * 4096), s_base0 + (uint32_t)((kt + 1) * GPT * 2),
                                        s_base1 + (uint32_t)((kt + 1) * GPT * 2), tr[(kt + 1) & 1]);
                    lds_wait_tile<GPT, 6>(tr[kt & 1], s0, s1);
                } else {
                    lds_wait_tile<GPT, 0>(tr[kt & 1], s0, s1);
                }
                const f16x8* av = tr[kt & 1].av;
#if defined(UOCR_NOCOMPUTE)
                acc0[0] += __uint_as_float(bw0[kt][0] ^ bw0[kt][1] ^ bw0[kt][2] ^ bw0[kt][3]) + (float)av[0][0] + (float)s0[0];
                if constexpr (GU) acc1[0] += __uint_as_float(bw1[kt][0] ^ bw1[kt][1] ^ bw1[kt][2] ^ bw1[kt][3]) + (float)s1[0];
#else
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    acc0 = mfma16(av[s], dequant8(bw0[kt][s], scale2(s0[s])), acc0);
                    if constexpr (GU) acc1 = mfma16(av[s], dequant8(bw1[kt][s], scale2(s1[s])), acc1);
                }
#endif
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 4 * (lane >> 4) + i;
                if (m < rows) {
                    if constexpr (GU) {
                        a.act[(size_t)(slot_base + m0 + m) * n_rows + col] = (f16)silu_mul_f(acc0[i], acc1[i]);
                    } else {
                        // y is indexed by entry: routed (t, j) at t*top_k + j,
                        // shared group v's token t at N + v*T + t
                        const int yrow = g < E ? ent[m0 + m] : N + slot_base + m0 + m;
                        a.y[(size_t)yrow * n_rows + col] = acc0[i];
                    }
                }
            }
        };
        // first m-tile: the A rows and scales (issued before the weights) are
        // waited for here, the weights k-tile by k-tile inside tile(), so the
        // dequant and MFMAs of early k-tiles overlap the arrival of later ones
        wait_vm_n((GU ? 2 : 1) * KT);
        lds_barrier();
        tile(0, true);
        for (int m0 = kDecBM; m0 < cnt; m0 += kDecBM) {
            __syncthreads();  // every wave is done with the previous tile's As
            stage_a(m0);
            wait_vm<0>();
            lds_barrier();
            tile(m0, false);
        }
        __syncthreads();  // As / Ss / ent are reused by the next item
    }
}

// ---------------------------------------------------------------------------
// Combine: out[t] = residual[t] + (sum_j fma(w[t,j], y[t*K + j]) in j order)
// + sum_v y[N + v*T + t]   (src/engine/moe_decoder.cpp:88-97,110-112,179)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void combine_decode_kernel(DecodeArgs a) {
    const int t = blockIdx.x, tid = threadIdx.x;
    const int T = a.seq, K = a.top_k, N = T * K, H = a.hidden;
    float wt[kMaxTopK];
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) wt[j] = j < K ? a.wts[(size_t)t * K + j] : 0.0f;
    const float* res = a.rms_weight ? static_cast<const float*>(a.x) + (size_t)t * H : nullptr;
    for (int c = tid * 4; c < H; c += 256 * 4) {
        f32x4 yv[kMaxTopK];
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j)
            if (j < K) yv[j] = *reinterpret_cast<const f32x4*>(a.y + ((size_t)t * K + j) * H + c);
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j)
            if (j < K)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] = fmaf(wt[j], yv[j][i], acc[i]);
        if (a.n_virtual > 0) {
            f32x4 sh = *reinterpret_cast<const f32x4*>(a.y + ((size_t)N + t) * H + c);
            for (int v = 1; v < a.n_virtual; ++v) {
                const f32x4 y2 = *reinterpret_cast<const f32x4*>(a.y + ((size_t)N + (size_t)v * T + t) * H + c);
#pragma unroll
                for (int i = 0; i < 4; ++i) sh[i] += y2[i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += sh[i];
        }
        if (res) {
            const f32x4 rv = *reinterpret_cast<const f32x4*>(res + c);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = rv[i] + acc[i];
        }
        *reinterpret_cast<f32x4*>(a.out + (size_t)t * H + c) = acc;
    }
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
template <int GPT, int KT, bool GU>
static void launch_expert(const DecodeArgs& a, int n_groups, int n_rows, hipStream_t st) {
    // one generation of resident workgroups (work items are grid-strided);
    // never more workgroups than the worst-case item count
    static int resident = [] {
        int dev = 0, cus = 0, per_cu = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, expert_decode_kernel<GPT, KT, GU>, 256, 0);
        return std::max(1, cus * std::max(1, per_cu));
    }();
    const int max_items = n_groups * ((n_rows / kTileRows + 3) / 4);
    launch_k((expert_decode_kernel<GPT, KT, GU>), dim3(std::min(resident, max_items)), dim3(256), 0, st, a);
}

template <bool GU, int GPT>
static hipError_t launch_expert_kt(const DecodeArgs& a, hipStream_t st) {
    const int K = GU ? a.hidden : a.inter;
    const int n_rows = GU ? a.inter : a.hidden;
    const int ng = a.n_experts + a.n_virtual;
    switch (K / kTileK) {
        case 1: launch_expert<GPT, 1, GU>(a, ng, n_rows, st); break;
        case 2: launch_expert<GPT, 2, GU>(a, ng, n_rows, st); break;
        case 4: launch_expert<GPT, 4, GU>(a, ng, n_rows, st); break;
        case 7: launch_expert<GPT, 7, GU>(a, ng, n_rows, st); break;
        case 10: launch_expert<GPT, 10, GU>(a, ng, n_rows, st); break;
        case 14: launch_expert<GPT, 14, GU>(a, ng, n_rows, st); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <bool GU>
static hipError_t launch_expert_g(const DecodeArgs& a, hipStream_t st) {
    switch (a.group) {
        case 32: return launch_expert_kt<GU, 4>(a, st);
        case 64: return launch_expert_kt<GU, 2>(a, st);
        case 128: return launch_expert_kt<GU, 1>(a, st);
        default: return hipErrorInvalidValue;
    }
}

bool decode_shapes_ok(int hidden, int inter) {
    auto ok = [](int k) {
        const int kt = k / kTileK;
        return k % kTileK == 0 && (kt == 1 || kt == 2 || kt == 4 || kt == 7 || kt == 10 || kt == 14);
    };
    return ok(hidden) && ok(inter) && hidden <= kMaxHidden;
}

template <typename XT, bool RMS>
static hipError_t launch_rd(const DecodeArgs& a, dim3 grid, size_t lds, hipStream_t st) {
    // > 64 KiB of dynamic LDS: raise the limit once per instantiation
    static hipError_t attr = hipFuncSetAttribute((const void*)router_decode_kernel<XT, RMS>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);
    if (attr != hipSuccess) return attr;
    launch_k((router_decode_kernel<XT, RMS>), grid, dim3(256), lds, st, a);
    return hipGetLastError();
}

hipError_t launch_router_decode(const DecodeArgs& a, hipStream_t st) {
    if (a.n_experts > 64 || a.hidden > kMaxHidden || a.hidden % 8) return hipErrorInvalidValue;
    if (a.hidden % kRChunkCols) return hipErrorInvalidValue;
    const dim3 grid(a.seq);
    const size_t lds = (size_t)kRRing * kRChunkBytes + (size_t)a.hidden * 4;
    const bool rms = a.rms_weight != nullptr;
    if (a.x_bf16) {
        if (rms) return launch_rd<uint16_t, true>(a, grid, lds, st);
        return launch_rd<uint16_t, false>(a, grid, lds, st);
    }
    if (rms) return launch_rd<float, true>(a, grid, lds, st);
    return launch_rd<float, false>(a, grid, lds, st);
}

hipError_t launch_experts_decode2(const DecodeArgs& a, bool gate_up, hipStream_t st) {
    if (a.seq * a.top_k > 0x7fffffff / 2 || a.seq > 256) return hipErrorInvalidValue;
    return gate_up ? launch_expert_g<true>(a, st) : launch_expert_g<false>(a, st);
}

hipError_t launch_combine_decode(const DecodeArgs& a, hipStream_t st) {
    launch_k(combine_decode_kernel, dim3(a.seq), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace uocr_hip
