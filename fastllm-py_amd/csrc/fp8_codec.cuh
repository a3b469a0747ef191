// E4M3 (e4m3fn) codecs used by the FP8 packers and kernels.
#pragma once

#include "common.cuh"

// fp32 -> e4m3 byte, the reference numpy encoder (fastllm_py/quantizer.py:26-51):
// clip to +-448; normals round-to-nearest-even at mantissa bit 20
// (em = |x|bits + 0x7FFFF + bit20), code clipped to 0x7E; values below 2^-6
// become rint(|x| * 512) clipped to 7 (so |x| in [7.5*2^-9, 2^-6) encodes
// 0x07, not 0x08); sign bit of the clipped fp32 copied to bit 7.
__host__ __device__ inline uint8_t e4m3_encode_ref(float x) {
    const float xc = x < -448.0f ? -448.0f : (x > 448.0f ? 448.0f : x);  // np.clip
    uint32_t f;
    __builtin_memcpy(&f, &xc, 4);
    const uint32_t sign = (f >> 24) & 0x80u;
    const int64_t em_in = (int64_t)(f & 0x7FFFFFFFu);
    const float ax = fabsf(xc);
    uint32_t out;
    if (ax >= 0.015625f) {
        const int64_t em = em_in + 0x7FFFF + ((em_in >> 20) & 1);
        const int64_t e = ((em >> 23) & 0xFF) - 127 + 7;
        const int64_t m = (em >> 20) & 0x7;
        int64_t val = (e << 3) | m;
        val = val < 0 ? 0 : (val > 0x7E ? 0x7E : val);
        out = (uint32_t)val;
    } else {
        const float t = rintf(ax * 512.0f);
        out = t > 7.0f ? 7u : (uint32_t)t;
    }
    return (uint8_t)(out | sign);
}

// fp32 -> e4m3 byte with IEEE round-to-nearest-even over the whole range
// (subnormals included) and saturation to +-448; NaN -> 0x7F.  This is the
// conversion the reference's inline-scale FP8 quantizer asks of its GPU
// (native/fastllm_fp8_block128.cu:93-94: satfinite E4M3).
__host__ __device__ inline uint8_t e4m3_encode_rne_sat(float x) {
    uint32_t f;
    __builtin_memcpy(&f, &x, 4);
    const uint32_t sign = (f >> 24) & 0x80u;
    const float ax = fabsf(x);
    if (ax != ax) return (uint8_t)(sign | 0x7F);
    if (ax >= 448.0f) return (uint8_t)(sign | 0x7E);
    uint32_t out;
    if (ax >= 0.015625f) {
        const uint32_t a = f & 0x7FFFFFFFu;
        const uint32_t em = a + 0x7FFFFu + ((a >> 20) & 1u);
        const uint32_t e = ((em >> 23) & 0xFFu) - 120u;
        const uint32_t m = (em >> 20) & 0x7u;
        out = (e << 3) | m;
    } else {
        out = (uint32_t)rintf(ax * 512.0f);  // 0..8; 8 is the normal 2^-6 = 0x08
    }
    return (uint8_t)(out | sign);
}

// e4m3 byte -> fp32, exact; 0x7F/0xFF decode to +-480 like the reference
// (fastllm_py/quantizer.py:54-62).
__host__ __device__ inline float e4m3_decode_exact(uint8_t b) {
    const int e = (b >> 3) & 0xF;
    const int m = b & 0x7;
    const float v = e > 0 ? ldexpf(1.0f + (float)m * 0.125f, e - 7) : (float)m * 0.001953125f;
    return (b & 0x80) ? -v : v;
}
