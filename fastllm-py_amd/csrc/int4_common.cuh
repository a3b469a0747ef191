// INT4 nibble helpers shared by the Marlin-ABI kernels and the fused MoE.
//
// Both libraries' tile layouts keep 8 consecutive k of one weight row in one
// u32 with k-offset r in nibble slot {0,4,1,5,2,6,3,7}[r].  Then
// (w & 0x000F000F) and (w & 0x00F000F0) (and the same of w >> 8) are the
// fp16 pairs (k0,k1), (k2,k3), (k4,k5), (k6,k7) once OR-ed with the exponent
// of 1024 (bits 0-3, ulp 1) or of 64 (bits 4-7, ulp 1/16), so one v_and_or
// and one packed add of -(1024+z) / -(64+z) give q - z exactly in fp16.
#pragma once

#include "common.cuh"

// nibble slot of k-offset r inside a tile-layout u32 (and, as it happens, the
// inverse of Marlin's zero-point interleave {0,2,4,6,1,3,5,7}).
__host__ __device__ constexpr int slot_of(int r) {
    return (r & 1) ? 4 + (r >> 1) : (r >> 1);
}

FL_DEV uint32_t gptq_word_to_tile_word(uint32_t w) {
    uint32_t o = 0;
#pragma unroll
    for (int r = 0; r < 8; ++r) o |= ((w >> (4 * r)) & 0xFu) << (4 * slot_of(r));
    return o;
}

FL_DEV uint32_t tile_word_to_gptq_word(uint32_t w) {
    uint32_t o = 0;
#pragma unroll
    for (int r = 0; r < 8; ++r) o |= ((w >> (4 * slot_of(r))) & 0xFu) << (4 * r);
    return o;
}

// (a & m) | c in one VALU op.
FL_DEV uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(c));
    return r;
}

// Dequantize with the zero point folded into fp16 constants: zlo = -(1024+z),
// zhi = -(64+z) as fp16 pairs (exact), magic_lo/hi = 0x64006400 / 0x54005400.
FL_DEV f16x8 dequant_word_fast(uint32_t w, uint32_t zlo, uint32_t zhi, uint32_t mlo,
                               uint32_t mhi) {
    const uint32_t w8 = w >> 8;
    const f16x2 p0 = bitcast<f16x2>(and_or(w, 0x000F000Fu, mlo)) + bitcast<f16x2>(zlo);
    const f16x2 p1 = bitcast<f16x2>(and_or(w, 0x00F000F0u, mhi)) + bitcast<f16x2>(zhi);
    const f16x2 p2 = bitcast<f16x2>(and_or(w8, 0x000F000Fu, mlo)) + bitcast<f16x2>(zlo);
    const f16x2 p3 = bitcast<f16x2>(and_or(w8, 0x00F000F0u, mhi)) + bitcast<f16x2>(zhi);
    const u32x4 r{bitcast<uint32_t>(p0), bitcast<uint32_t>(p1), bitcast<uint32_t>(p2),
                  bitcast<uint32_t>(p3)};
    return bitcast<f16x8>(r);
}

// fp16-pair bit patterns of -(1024+z) and -(64+z) for a zero point z in 0..15.
FL_DEV void zero_bits(uint32_t z, uint32_t& zlo, uint32_t& zhi) {
    const uint32_t lo = 0xE400u | z;         // -(1024 + z): exponent 10, mantissa z
    const uint32_t hi = 0xD400u | (z << 4);  // -(64 + z): exponent 6, ulp 1/16
    zlo = lo | (lo << 16);
    zhi = hi | (hi << 16);
}

