// Device-side building blocks shared by the MoE kernels (gfx950 / CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "uexpf.h"

namespace uocr_hip {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Device weight layout ("tile-16x128"): the contract between the host repack
// (capi.cpp) and every INT4 kernel.
//
// A matrix of R rows (output features) x K columns (input features) is cut
// into 16-row blocks `rb` and 128-column k-tiles `kt`; each (rb, kt) tile is
// 1024 bytes, stored at ((rb * KT + kt) * 64 + lane) * 16. Lane `l` of a wave
// owns row rb*16 + l%16 and, for MFMA step s = 0..3, the 8 columns
//   kt*128 + s*32 + 8*(l/16) + i,  i = 0..7,
// packed into 32-bit word s of its 16 bytes with nibble i at bit
// (i & 1) * 16 + (i >> 1) * 4. With that order one AND-OR per pair turns
// (word >> 4j) into two f16 values 1024 + q (the f16 with exponent 2^10 has an
// integer ulp), ready for the v_mfma_f32_16x16x32_f16 B operand, and one
// 1 KiB tile is one fully coalesced wave load.
//
// Scales: one per (row, group), stored as f16 (the bf16-valued reference
// scales convert exactly whenever they are normal f16 numbers), row-major
// [rows][scale_row_stride(K, group)] (K / group rounded up to 8, so every row
// starts 16-byte aligned and a lane fetches all scales of its row with whole
// 16-byte loads); the zero point is the implicit 8 of the reference's
// symmetric layout (src/runtime/quant.cpp:82-116).
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int scale_row_stride(int k, int group) { return ((k / group) + 7) / 8 * 8; }

constexpr int kTileRows = 16;
constexpr int kTileK = 128;
constexpr int kTileBytes = 1024;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ f16x2 nib_pair(uint32_t w) {
    // (w & 0x000F000F) | 0x64006400 holds two f16 values 1024 + q; one
    // v_bfi_b32 (the high nibbles of 0x64006400 are zero where the mask is set)
    uint32_t v;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(v) : "v"(0x000F000Fu), "v"(w), "v"(0x64006400u));
    f16x2 h;
    __builtin_memcpy(&h, &v, 4);
    return h;
}

// Eight nibbles of one packed word -> f16x8 of (q - 8) * scale. Exact whenever
// the scale is a normal f16: (q - 8) has <= 3 significant bits and a bf16 scale
// 8, so the product fits the 11-bit f16 significand.
// (Scalar words on purpose: a __builtin_bit_cast of an ext_vector element was
// miscompiled by this toolchain into a copy of element 0.)
__device__ __forceinline__ f16x8 dequant8(uint32_t w, f16x2 s2) {
    const f16x2 off = {(f16)-1032.0f, (f16)-1032.0f};
    const f16x2 h0 = (nib_pair(w) + off) * s2;
    const f16x2 h1 = (nib_pair(w >> 4) + off) * s2;
    const f16x2 h2 = (nib_pair(w >> 8) + off) * s2;
    const f16x2 h3 = (nib_pair(w >> 12) + off) * s2;
    f16x8 r;
    r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
    r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
    return r;
}

__device__ __forceinline__ f16x2 scale2(f16 s) { return f16x2{s, s}; }

__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float silu_mul_f(float g, float u) { return g / (1.0f + __expf(-g)) * u; }

// gfx950 direct global->LDS load: each active lane copies 16 bytes from `src`
// to lds_base + 16 * lane (lds_base must be wave-uniform). No VGPRs are used;
// completion is tracked by vmcnt like any global load.
__device__ __forceinline__ void load_lds16(const void* src, void* lds_base) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)lds_base, 16, 0, 0);
}

}  // namespace uocr_hip
