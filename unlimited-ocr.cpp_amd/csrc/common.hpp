// Device-side building blocks shared by the MoE kernels (gfx950 / CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "uexpf.h"

namespace uocr_hip {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
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
// Scales: one per (row, group), the reference's f32 scale rounded to f16
// (exact for bf16-valued scales that are normal f16 numbers), row-major
// [rows][scale_row_stride(K, group)] (K / group rounded up to 8, so every row
// starts 16-byte aligned and a lane fetches all scales of its row with whole
// 16-byte loads).
// Zero points: a layer whose zeros are all 8 (quantize_int4_symmetric,
// src/runtime/quant.cpp:82-116) stores none -- 8 is implicit. Any other layer
// (quantize_int4_awq, src/runtime/quant.cpp:39-80, and the GPTQ files, whose
// zeros are integers in [0, 15]) stores one f16 per (row, group) in the scale
// layout, holding -(1024 + zero): the offset that turns the biased nibble
// 1024 + q into q - zero exactly (see dequant8z).
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int scale_row_stride(int k, int group) { return ((k / group) + 7) / 8 * 8; }

constexpr int kTileRows = 16;
constexpr int kTileK = 128;
constexpr int kTileBytes = 1024;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ f16x2 as_h2(uint32_t v) {
    f16x2 h;
    __builtin_memcpy(&h, &v, 4);
    return h;
}

// Eight nibbles of one packed word -> f16x8 of (q - 8) * scale, in the order of
// the tile layout (nibble i of the word at bit (i & 1) * 16 + (i >> 1) * 4).
// One AND-OR per nibble pair builds two f16 values directly: a nibble in bits
// [3:0] under the exponent of 1024 (0x6400, unit ulp) is 1024 + q, a nibble in
// bits [7:4] under the exponent of 64 (0x5400, ulp 1/16) is 64 + q -- so one
// shift by 8 serves all four pairs. Subtracting 1032 / 72 gives q - 8 exactly,
// and the product with a bf16-valued scale is exact in f16: (q - 8) has <= 3
// significant bits and the scale 8, within the 11-bit significand.
__device__ __forceinline__ f16x8 dequant8(uint32_t w, f16x2 s2) {
    const f16x2 off0 = {(f16)-1032.0f, (f16)-1032.0f}, off1 = {(f16)-72.0f, (f16)-72.0f};
    // (w & mask) | magic as one v_bitop3_b32 (truth table 0xEA = (a & b) | c)
    const uint32_t w8 = w >> 8;
    const f16x2 h0 = (as_h2(__builtin_amdgcn_bitop3_b32(w, 0x000F000Fu, 0x64006400u, 0xEA)) + off0) * s2;
    const f16x2 h1 = (as_h2(__builtin_amdgcn_bitop3_b32(w, 0x00F000F0u, 0x54005400u, 0xEA)) + off1) * s2;
    const f16x2 h2 = (as_h2(__builtin_amdgcn_bitop3_b32(w8, 0x000F000Fu, 0x64006400u, 0xEA)) + off0) * s2;
    const f16x2 h3 = (as_h2(__builtin_amdgcn_bitop3_b32(w8, 0x00F000F0u, 0x54005400u, 0xEA)) + off1) * s2;
    f16x8 r;
    r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
    r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
    return r;
}

// Eight nibbles -> f16x8 of (q - zero) * scale for a stored zero offset
// zo = -(1024 + zero) (an integer zero in [0, 15]): the biased values 1024 + q
// and 64 + q of dequant8 plus zo and zo + 960 give q - zero exactly; the
// product with the f16 scale rounds once (to f16) unless it is exact.
__device__ __forceinline__ f16x8 dequant8z(uint32_t w, f16x2 s2, f16 zo) {
    const f16x2 off0 = {zo, zo};
    const f16 zo1 = zo + (f16)960.0f;
    const f16x2 off1 = {zo1, zo1};
    const uint32_t w8 = w >> 8;
    const f16x2 h0 = (as_h2(__builtin_amdgcn_bitop3_b32(w, 0x000F000Fu, 0x64006400u, 0xEA)) + off0) * s2;
    const f16x2 h1 = (as_h2(__builtin_amdgcn_bitop3_b32(w, 0x00F000F0u, 0x54005400u, 0xEA)) + off1) * s2;
    const f16x2 h2 = (as_h2(__builtin_amdgcn_bitop3_b32(w8, 0x000F000Fu, 0x64006400u, 0xEA)) + off0) * s2;
    const f16x2 h3 = (as_h2(__builtin_amdgcn_bitop3_b32(w8, 0x00F000F0u, 0x54005400u, 0xEA)) + off1) * s2;
    f16x8 r;
    r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
    r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
    return r;
}

// Eight nibbles -> f16x8 of the exact integers q - zero (zo as in dequant8z),
// the scale left to the caller.
__device__ __forceinline__ f16x8 dequant8z_unscaled(uint32_t w, f16 zo) {
    const f16 zo1 = zo + (f16)960.0f;
    const f16x2 off0 = {zo, zo}, off1 = {zo1, zo1};
    const uint32_t w8 = w >> 8;
    const f16x2 h0 = as_h2(__builtin_amdgcn_bitop3_b32(w, 0x000F000Fu, 0x64006400u, 0xEA)) + off0;
    const f16x2 h1 = as_h2(__builtin_amdgcn_bitop3_b32(w, 0x00F000F0u, 0x54005400u, 0xEA)) + off1;
    const f16x2 h2 = as_h2(__builtin_amdgcn_bitop3_b32(w8, 0x000F000Fu, 0x64006400u, 0xEA)) + off0;
    const f16x2 h3 = as_h2(__builtin_amdgcn_bitop3_b32(w8, 0x00F000F0u, 0x54005400u, 0xEA)) + off1;
    f16x8 r;
    r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
    r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
    return r;
}

// The same eight nibbles as biased f16 values without the zero point and the
// scale: positions 0, 1, 4, 5 hold 1024 + q, positions 2, 3, 6, 7 hold 64 + q
// (the magic exponents of dequant8). A caller that seeds the MFMA accumulator
// with -(1032 * sum of its A values at the first positions + 72 * sum at the
// others) over a scale group, then scales the group's result, gets the same
// product as with dequant8 at four operations per word instead of twelve.
__device__ __forceinline__ f16x8 dequant8_biased(uint32_t w) {
    const uint32_t w8 = w >> 8;
    u32x4 p;
    p[0] = __builtin_amdgcn_bitop3_b32(w, 0x000F000Fu, 0x64006400u, 0xEA);
    p[1] = __builtin_amdgcn_bitop3_b32(w, 0x00F000F0u, 0x54005400u, 0xEA);
    p[2] = __builtin_amdgcn_bitop3_b32(w8, 0x000F000Fu, 0x64006400u, 0xEA);
    p[3] = __builtin_amdgcn_bitop3_b32(w8, 0x00F000F0u, 0x54005400u, 0xEA);
    f16x8 r;
    __builtin_memcpy(&r, &p, 16);
    return r;
}

__device__ __forceinline__ f16x2 scale2(f16 s) { return f16x2{s, s}; }

__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// An f32 value staged as f16 that leaves f16's finite range (rounds to +-inf,
// or is NaN): the kernels that stage act / y rows in f16 report it once per
// lane with atomicOr(status, kStatusF16Overflow) on the layer's status word.
constexpr int kStatusF16Overflow = 4;
__device__ __forceinline__ bool f16_overflow(float v) { return !(__builtin_fabsf(v) < 65520.0f); }
__device__ __forceinline__ void report_f16_overflow(int* status, bool ovf) {
    if (ovf && status) atomicOr(status, kStatusF16Overflow);
}

// silu(g) * u with the hardware reciprocal (1 ulp) in place of an IEEE divide
__device__ __forceinline__ float silu_mul_f(float g, float u) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u; }

// gfx950 direct global->LDS load: each active lane copies 16 bytes from `src`
// to lds_base + 16 * lane (lds_base must be wave-uniform). No VGPRs are used;
// completion is tracked by vmcnt like any global load.
__device__ __forceinline__ void load_lds16(const void* src, void* lds_base) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)lds_base, 16, 0, 0);
}

// LDS byte address of a __shared__ object
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

}  // namespace uocr_hip
