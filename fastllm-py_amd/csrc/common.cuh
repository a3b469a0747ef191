// Shared device/host helpers for the gfx950 (CDNA4) quantized-matmul library.
//
// Everything here is written for wave64 / MFMA on gfx950 only. Conventions:
//   * all entry points are extern "C", take raw device pointers, and launch on
//     the stream they are given (nullptr = the null stream);
//   * floating-point contraction is disabled for the whole library
//     (-ffp-contract=off); fused multiply-adds are written explicitly with
//     __builtin_fmaf where they are wanted, so the packers keep the exact
//     two-rounding arithmetic of the numpy formulas they restate.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// 16-byte vector that only promises 4-byte alignment (rows of the inline-scale
// FP8 format start every 132 bytes).
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

#define FL_WAVE 64

#define FL_DEV __device__ __forceinline__

template <typename T, typename S>
FL_DEV T bitcast(S s) {
    static_assert(sizeof(T) == sizeof(S), "bitcast size");
    return __builtin_bit_cast(T, s);
}

// v_mfma_f32_16x16x32_f16: D[16x16] += A[16x32] * B[32x16].
// Operand layout (wave64): lane l holds A[l%16][8*(l/16) .. +7] and
// B[8*(l/16) .. +7][l%16]; D lane l holds D[4*(l/16) + i][l%16], i = 0..3.
FL_DEV f32x4 mfma_f16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
FL_DEV f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

FL_DEV float half_bits_to_float(uint16_t h) { return (float)bitcast<f16>(h); }

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] and
// vmcnt[5:4] at bits 15:14; expcnt and lgkmcnt left at their maxima).
template <int N>
FL_DEV void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

typedef void __attribute__((address_space(3)))* lptr_t;

// Workgroup barrier that hands LDS data to the other waves without draining
// this wave's outstanding global loads: it waits for the wave's LDS accesses
// (lgkmcnt(0)) and then s_barrier.  __syncthreads() would also wait for
// vmcnt(0) (its release fence), i.e. for every weight load issued before it.
FL_DEV void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4) | (0 << 8));
    asm volatile("s_barrier" ::: "memory");
}

// Raw buffer resource over [base, base + bytes) (gfx9 descriptor, dword 3 =
// 0x00020000): loads take a 32-bit per-lane offset plus a wave-uniform SGPR
// offset, so the per-block address step is one scalar add; offsets at or
// past `bytes` read 0.
FL_DEV __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}

// Copy rings of the MFMA GEMMs.  With the buffer_load ... lds builtin the
// compiler cannot tell which LDS bytes a copy in flight will write, so
// before every LDS read it waits for all of them (s_waitcnt vmcnt(0)): a
// ring of several stages then drains on every block and holds one block in
// flight.  These copies are issued from inline asm, which the compiler's
// wait insertion does not see; the kernels that use them order every LDS
// read after its copies themselves (s_waitcnt vmcnt(n) + s_barrier), and
// read nothing else through the vector memory counter inside the ring (a
// vector load issued behind the copies would return only after them).
typedef int i32x4_t __attribute__((ext_vector_type(4)));
// Buffer descriptor as four SGPR words (same fields as buf_rsrc).
FL_DEV i32x4_t raw_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)base;
    return i32x4_t{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xFFFFu), (int)bytes, 0x00020000};
}
// BYTES (16 or 4) per lane from rsrc + voff + soff into LDS at lds_addr +
// BYTES lane (lds_addr and soff wave-uniform; offsets past the buffer read 0).
template <int BYTES = 16>
FL_DEV void lds_copy(i32x4_t rsrc, uint32_t lds_addr, uint32_t voff, uint32_t soff = 0) {
    static_assert(BYTES == 16 || BYTES == 4, "copy width");
    if constexpr (BYTES == 16)
        asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                     :
                     : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voff), "s"(rsrc),
                       "s"(__builtin_amdgcn_readfirstlane(soff))
                     : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
                     :
                     : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voff), "s"(rsrc),
                       "s"(__builtin_amdgcn_readfirstlane(soff))
                     : "memory", "m0");
}

// Host-side launch error check: returns the HIP error of the last launch.
static inline hipError_t fl_last_error() { return hipGetLastError(); }

static inline int fl_ceil_div(int a, int b) { return (a + b - 1) / b; }

// Workgroup index regrouped by XCD: the hardware deals workgroup b to XCD
// b % 8, so with the grid a multiple of 8 XCD x takes the contiguous range
// [x G/8, (x+1) G/8) and neighbouring tiles share that XCD's L2.
FL_DEV int xcd_block() {
    return (gridDim.x & 7) ? (int)blockIdx.x
                           : (int)(blockIdx.x & 7) * (int)(gridDim.x >> 3) + (int)(blockIdx.x >> 3);
}
