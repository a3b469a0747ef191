// GPU packers and unpackers of the quantized-weight formats, bit-exact with the
// reference's numpy formulas (all fp32 arithmetic is IEEE with one rounding per
// numpy operation: the library is built with -ffp-contract=off and HIP's
// correctly-rounded fp32 division).
//
//   quantize_int4_group / dequantize_int4_group   fastllm_py/quantizer.py:97-129
//   quantize_marlin_matrix (quantization part)     fastllm_py/moe.py:30-46
//   pack_gptq_qweight                              fastllm_py/kernels/marlin.py:113-127
//   build_marlin_scales_zeros                      fastllm_py/kernels/marlin.py:130-159
//   quantize_int4_rowmajor (+ batched) / dequant   fastllm_py/kernels/moe_int4.py:24-54,97-113
//   _fp8_e4m3_encode / _fp8_e4m3_decode            fastllm_py/quantizer.py:26-62
//   quantize_fp8_block / dequantize_fp8_block      fastllm_py/quantizer.py:65-94
#include "common.cuh"
#include "device.cuh"
#include "fp8_codec.cuh"

namespace {

// ---------------------------------------------------------------- reductions
FL_DEV float wave_min(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
    return v;
}
FL_DEV float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// min/max of one quantization group, one wave per group (lanes stride 64).
FL_DEV void group_minmax(const float* __restrict__ g, int gs, int lane, float& mn, float& mx) {
    float a = INFINITY, b = -INFINITY;
    for (int i = lane; i < gs; i += 64) {
        const float v = g[i];
        a = fminf(a, v);
        b = fmaxf(b, v);
    }
    mn = wave_min(a);
    mx = wave_max(b);
}

// (wmax - wmin) / 15, 1 where that is 0 (quantizer.py:108-109, moe.py:42-43,
// moe_int4.py:31-32).
FL_DEV float rtn_scale(float mn, float mx) {
    const float s = (mx - mn) / 15.0f;
    return s == 0.0f ? 1.0f : s;
}

// np.clip(v, 0, 15): replaces only values strictly outside the range, so a
// -0.0 (rint of a small negative) stays -0.0 like in numpy.
FL_DEV float clip015(float v) { return v < 0.0f ? 0.0f : (v > 15.0f ? 15.0f : v); }

// ---------------------------------------------------------------- int4 group
// q = clip(rint((g - wmin) / scale), 0, 15); even column in the low nibble;
// scales = scale (fp32), zeros = wmin (fp32).
__global__ void quantize_int4_group_k(const float* __restrict__ w, uint8_t* __restrict__ packed,
                                      float* __restrict__ scales, float* __restrict__ zeros,
                                      int rows, int cols, int gs) {
    const int lane = threadIdx.x & 63;
    const int ng = cols / gs;
    const long task = (long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (task >= (long)rows * ng) return;
    const int row = (int)(task / ng), gi = (int)(task % ng);
    const float* g = w + (size_t)row * cols + (size_t)gi * gs;
    float mn, mx;
    group_minmax(g, gs, lane, mn, mx);
    const float s = rtn_scale(mn, mx);
    uint8_t* out = packed + (size_t)row * (cols / 2) + (size_t)gi * (gs / 2);
    for (int p = lane; p < gs / 2; p += 64) {
        const float q0 = clip015(rintf((g[2 * p] - mn) / s));
        const float q1 = clip015(rintf((g[2 * p + 1] - mn) / s));
        out[p] = (uint8_t)((uint32_t)q0 | ((uint32_t)q1 << 4));
    }
    if (lane == 0) {
        scales[(size_t)row * ng + gi] = s;
        zeros[(size_t)row * ng + gi] = mn;
    }
}

// q * scale + zero, multiply and add rounded separately (quantizer.py:120-129).
__global__ void dequantize_int4_group_k(const uint8_t* __restrict__ packed,
                                        const float* __restrict__ scales,
                                        const float* __restrict__ zeros, float* __restrict__ out,
                                        int rows, int cols, int gs) {
    const size_t total = (size_t)rows * cols / 2;
    const int ng = cols / gs;
    for (size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x; p < total;
         p += (size_t)gridDim.x * blockDim.x) {
        const size_t row = p / (cols / 2);
        const int c = (int)(p % (cols / 2)) * 2;
        const uint8_t b = packed[p];
        const size_t gidx = row * ng + c / gs;
        const float s = scales[gidx], z = zeros[gidx];
        const float q0 = (float)(b & 0xF), q1 = (float)(b >> 4);
        float* o = out + row * cols + c;
        const float t0 = q0 * s;
        const float t1 = q1 * s;
        o[0] = t0 + z;
        o[1] = t1 + z;
    }
}

// ------------------------------------------------- Marlin-style integer zero
// zero = clip(rint(-wmin / scale), 0, 15); q = clip(rint(g / scale) + zero, 0, 15)
// (moe.py:40-46).  Outputs unpacked q [N, K] u8, scale [N, G] f32, zero [N, G] i32.
__global__ void quantize_int4_marlin_k(const float* __restrict__ w, uint8_t* __restrict__ q,
                                       float* __restrict__ scale, int32_t* __restrict__ zero,
                                       int rows, int cols, int gs) {
    const int lane = threadIdx.x & 63;
    const int ng = cols / gs;
    const long task = (long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (task >= (long)rows * ng) return;
    const int row = (int)(task / ng), gi = (int)(task % ng);
    const float* g = w + (size_t)row * cols + (size_t)gi * gs;
    float mn, mx;
    group_minmax(g, gs, lane, mn, mx);
    const float s = rtn_scale(mn, mx);
    const float z = clip015(rintf(-mn / s));
    uint8_t* out = q + (size_t)row * cols + (size_t)gi * gs;
    for (int i = lane; i < gs; i += 64) {
        const float r = rintf(g[i] / s);
        out[i] = (uint8_t)clip015(r + z);  // integer-valued, exact in fp32
    }
    if (lane == 0) {
        scale[(size_t)row * ng + gi] = s;
        zero[(size_t)row * ng + gi] = (int32_t)z;
    }
}

// ----------------------------------------------------- row-major int4 format
// zero = clip(rint(-wmin / scale), 0, 15) (fp32); q = clip(rint(g / scale + zero), 0, 15);
// scales, zeros stored fp16 (moe_int4.py:24-40, batched :97-113).
__global__ void quantize_int4_rowmajor_k(const float* __restrict__ w, uint8_t* __restrict__ packed,
                                         f16* __restrict__ scales, f16* __restrict__ zeros,
                                         long rows, int cols, int gs) {
    const int lane = threadIdx.x & 63;
    const int ng = cols / gs;
    const long task = (long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (task >= rows * ng) return;
    const long row = task / ng;
    const int gi = (int)(task % ng);
    const float* g = w + (size_t)row * cols + (size_t)gi * gs;
    float mn, mx;
    group_minmax(g, gs, lane, mn, mx);
    const float s = rtn_scale(mn, mx);
    const float z = clip015(rintf(-mn / s));
    uint8_t* out = packed + (size_t)row * (cols / 2) + (size_t)gi * (gs / 2);
    for (int p = lane; p < gs / 2; p += 64) {
        const float a0 = g[2 * p] / s;
        const float a1 = g[2 * p + 1] / s;
        const float q0 = clip015(rintf(a0 + z));
        const float q1 = clip015(rintf(a1 + z));
        out[p] = (uint8_t)((uint32_t)q0 | ((uint32_t)q1 << 4));
    }
    if (lane == 0) {
        scales[(size_t)row * ng + gi] = (f16)s;
        zeros[(size_t)row * ng + gi] = (f16)z;
    }
}

// (q - zero) * scale with fp16 scale/zero widened to fp32 (moe_int4.py:43-54).
__global__ void dequantize_int4_rowmajor_k(const uint8_t* __restrict__ packed,
                                           const f16* __restrict__ scales,
                                           const f16* __restrict__ zeros, float* __restrict__ out,
                                           long rows, int cols, int gs) {
    const size_t total = (size_t)rows * cols / 2;
    const int ng = cols / gs;
    for (size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x; p < total;
         p += (size_t)gridDim.x * blockDim.x) {
        const size_t row = p / (cols / 2);
        const int c = (int)(p % (cols / 2)) * 2;
        const uint8_t b = packed[p];
        const size_t gidx = row * ng + c / gs;
        const float s = (float)scales[gidx], z = (float)zeros[gidx];
        float* o = out + row * cols + c;
        const float d0 = (float)(b & 0xF) - z;
        const float d1 = (float)(b >> 4) - z;
        o[0] = d0 * s;
        o[1] = d1 * s;
    }
}

// ----------------------------------------------------------- GPTQ packing
// word [k/8, n] = sum_i q[n, 8(k/8) + i] << 4i  (mod 2^32, marlin.py:113-127).
__global__ void pack_gptq_k(const uint32_t* __restrict__ q, uint32_t* __restrict__ out, int N,
                            int K) {
    const size_t total = (size_t)K / 8 * N;
    for (size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x; o < total;
         o += (size_t)gridDim.x * blockDim.x) {
        const size_t kw = o / N;
        const size_t n = o % N;
        const uint32_t* src = q + n * K + kw * 8;
        uint32_t acc = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc += src[i] << (4 * i);
        out[o] = acc;
    }
}

// --------------------------------------------- Marlin scale/zero permutation
// scales_out[g, c*64 + 8i + j] = fp16(scale[c*64 + 8j + i, g]);
// zeros_out[g, c*8 + w] = sum_s zero[c*64 + 8*zpi[s] + w, g] << 4s (mod 2^32),
// zpi = {0,2,4,6,1,3,5,7}  (marlin.py:41-51,138-159).
__global__ void marlin_scales_zeros_k(const float* __restrict__ scale, const int32_t* __restrict__ zero,
                                      f16* __restrict__ scales_out, uint32_t* __restrict__ zeros_out,
                                      int N, int G) {
    const size_t total = (size_t)G * N;
    for (size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x; o < total;
         o += (size_t)gridDim.x * blockDim.x) {
        const int g = (int)(o / N);
        const int p = (int)(o % N);
        const int c = p >> 6, loc = p & 63;
        const int src_n = c * 64 + 8 * (loc & 7) + (loc >> 3);
        scales_out[o] = (f16)scale[(size_t)src_n * G + g];
        if ((p & 7) == 0) {
            // this thread also builds zero word (g, p/8)
            const int word = p >> 3;  // = c*8 + w
            const int wc = word >> 3, wi = word & 7;
            constexpr int zpi[8] = {0, 2, 4, 6, 1, 3, 5, 7};
            uint32_t acc = 0;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const int pp = wi * 8 + zpi[s];  // position in the scalePerm-ed chunk
                const int sn = wc * 64 + 8 * (pp & 7) + (pp >> 3);
                acc += (uint32_t)zero[(size_t)sn * G + g] << (4 * s);
            }
            zeros_out[(size_t)g * (N >> 3) + word] = acc;
        }
    }
}

// --------------------------------------------------------------- E4M3 codec
__global__ void fp8_encode_k(const float* __restrict__ x, uint8_t* __restrict__ out, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = e4m3_encode_ref(x[i]);
}
__global__ void fp8_decode_k(const uint8_t* __restrict__ b, float* __restrict__ out, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = e4m3_decode_exact(b[i]);
}

// ------------------------------------------------------- 128x128 block FP8
// One workgroup per (bs x bs) block: amax over the block (zero padding outside
// the matrix), scale = amax / 448 (1 if amax == 0), q = encode(w / scale)
// (quantizer.py:65-85).  Scales [ceil(R/bs), ceil(C/bs)] fp32.
__global__ void quantize_fp8_block_k(const float* __restrict__ w, uint8_t* __restrict__ q,
                                     float* __restrict__ scales, int rows, int cols, int bs) {
    __shared__ float red[1024 / 64];
    const int bi = blockIdx.y, bj = blockIdx.x;
    const int nbj = gridDim.x;
    const int r0 = bi * bs, c0 = bj * bs;
    float amax = 0.0f;
    for (int e = threadIdx.x; e < bs * bs; e += blockDim.x) {
        const int r = r0 + e / bs, c = c0 + e % bs;
        if (r < rows && c < cols) amax = fmaxf(amax, fabsf(w[(size_t)r * cols + c]));
    }
    amax = wave_max(amax);
    const int wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wid] = amax;
    __syncthreads();
    float m = 0.0f;
    for (int i = 0; i < nw; ++i) m = fmaxf(m, red[i]);
    const float s = (m == 0.0f) ? 1.0f : m / 448.0f;
    if (threadIdx.x == 0) scales[(size_t)bi * nbj + bj] = s;
    for (int e = threadIdx.x; e < bs * bs; e += blockDim.x) {
        const int r = r0 + e / bs, c = c0 + e % bs;
        if (r < rows && c < cols) q[(size_t)r * cols + c] = e4m3_encode_ref(w[(size_t)r * cols + c] / s);
    }
}

// decode(q) * scale (quantizer.py:88-94).
__global__ void dequantize_fp8_block_k(const uint8_t* __restrict__ q, const float* __restrict__ scales,
                                       float* __restrict__ out, int rows, int cols, int bs) {
    const size_t total = (size_t)rows * cols;
    const int nbj = (cols + bs - 1) / bs;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / cols), c = (int)(i % cols);
        out[i] = e4m3_decode_exact(q[i]) * scales[(size_t)(r / bs) * nbj + c / bs];
    }
}

// ------------------------------------------------------------- MXFP4 (OCP MX)
// Blocks of 32 consecutive elements of a row share an E8M0 scale X =
// 2^(floor(log2 amax) - 2) (exponent clamped to [-127, 127]; X = 1 for an
// all-zero block); elements are v / X rounded to E2M1 to nearest, ties to
// the even code, saturating at 6, with the sign of v.  Codes: two per byte,
// the lower column in the low nibble.  Finite inputs only.
FL_DEV int mx_exponent(float amax) {
    if (amax == 0.0f) return 0;
    const int biased = (int)((__float_as_uint(amax) >> 23) & 0xFFu);
    const int e = biased - 129;
    return e < -127 ? -127 : (e > 127 ? 127 : e);
}

FL_DEV uint32_t e2m1_code(float p) {
    const float a = fabsf(p);
    const uint32_t c = (uint32_t)(a > 0.25f) + (uint32_t)(a >= 0.75f) + (uint32_t)(a > 1.25f) +
                       (uint32_t)(a >= 1.75f) + (uint32_t)(a > 2.5f) + (uint32_t)(a >= 3.5f) +
                       (uint32_t)(a > 5.0f);
    return c | ((__float_as_uint(p) >> 28) & 8u);
}

// one thread per (row, 32-column block)
__global__ void quantize_mxfp4_k(const float* __restrict__ w, uint8_t* __restrict__ codes,
                                 uint8_t* __restrict__ e8, size_t nblk, int cols) {
    const int bpr = cols / 32;
    for (size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x; b < nblk;
         b += (size_t)gridDim.x * blockDim.x) {
        const size_t r = b / bpr;
        const int g = (int)(b - r * bpr);
        const f32x4* src = reinterpret_cast<const f32x4*>(w + r * cols + 32 * g);
        f32x4 v[8];
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[i] = src[i];
#pragma unroll
            for (int e = 0; e < 4; ++e) amax = fmaxf(amax, fabsf(v[i][e]));
        }
        const int ex = mx_exponent(amax);
        const float inv = __uint_as_float((uint32_t)(127 - ex) << 23);  // 2^-ex, ex in [-127, 125]
        u32x4 out;
#pragma unroll
        for (int wd = 0; wd < 4; ++wd) {
            uint32_t word = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) word |= e2m1_code(v[2 * wd + i / 4][i % 4] * inv) << (4 * i);
            out[wd] = word;
        }
        *reinterpret_cast<u32x4*>(codes + r * (cols / 2) + 16 * g) = out;
        e8[b] = (uint8_t)(ex + 127);
    }
}

__global__ void dequantize_mxfp4_k(const uint8_t* __restrict__ codes, const uint8_t* __restrict__ e8,
                                   float* __restrict__ out, size_t n, int cols) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / cols;
        const int c = (int)(i - r * cols);
        const uint32_t code = (codes[r * (cols / 2) + c / 2] >> (4 * (c & 1))) & 0xFu;
        const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
        const float v = (code & 8u) ? -mag[code & 7u] : mag[code & 7u];
        out[i] = v * ldexpf(1.0f, (int)e8[r * (cols / 32) + c / 32] - 127);
    }
}

unsigned grid_for(size_t n, int threads) {
    size_t b = (n + threads - 1) / threads;
    if (b > 65536) b = 65536;
    if (b < 1) b = 1;
    return (unsigned)b;
}

int finish(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fprintf(stderr, "%s launch error: %s\n", what, hipGetErrorString(e));
        return 2;
    }
    return 0;
}

// one wave per (row, group) task, 4 waves per workgroup
unsigned wave_task_grid(long tasks) { return (unsigned)((tasks + 3) / 4); }

}  // namespace

extern "C" {

int fastllm_pack_gptq_qweight(const uint32_t* q, uint32_t* out, int size_n, int size_k,
                              void* stream) {
    if (!q || !out || size_n <= 0 || size_k <= 0 || size_k % 8) return 1;
    hipLaunchKernelGGL(pack_gptq_k, dim3(grid_for((size_t)size_k / 8 * size_n, 256)), dim3(256), 0,
                       (hipStream_t)stream, q, out, size_n, size_k);
    return finish("fastllm_pack_gptq_qweight");
}

int fastllm_build_marlin_scales_zeros(const float* scale, const int32_t* zero, void* scales_out,
                                      uint32_t* zeros_out, int size_n, int num_groups,
                                      void* stream) {
    if (!scale || !zero || !scales_out || !zeros_out || size_n <= 0 || num_groups <= 0 ||
        size_n % 64)
        return 1;
    hipLaunchKernelGGL(marlin_scales_zeros_k, dim3(grid_for((size_t)size_n * num_groups, 256)),
                       dim3(256), 0, (hipStream_t)stream, scale, zero, (f16*)scales_out, zeros_out,
                       size_n, num_groups);
    return finish("fastllm_build_marlin_scales_zeros");
}

int fastllm_quantize_int4_group(const float* w, uint8_t* packed, float* scales, float* zeros,
                                int rows, int cols, int group_size, void* stream) {
    if (!w || !packed || !scales || !zeros || rows <= 0 || cols <= 0 || group_size <= 0 ||
        cols % group_size || cols % 2 || group_size % 2)
        return 1;
    const long tasks = (long)rows * (cols / group_size);
    hipLaunchKernelGGL(quantize_int4_group_k, dim3(wave_task_grid(tasks)), dim3(256), 0,
                       (hipStream_t)stream, w, packed, scales, zeros, rows, cols, group_size);
    return finish("fastllm_quantize_int4_group");
}

int fastllm_dequantize_int4_group(const uint8_t* packed, const float* scales, const float* zeros,
                                  float* out, int rows, int cols, int group_size, void* stream) {
    if (!packed || !scales || !zeros || !out || rows <= 0 || cols <= 0 || group_size <= 0 ||
        cols % group_size || cols % 2 || group_size % 2)
        return 1;
    hipLaunchKernelGGL(dequantize_int4_group_k, dim3(grid_for((size_t)rows * cols / 2, 256)),
                       dim3(256), 0, (hipStream_t)stream, packed, scales, zeros, out, rows, cols,
                       group_size);
    return finish("fastllm_dequantize_int4_group");
}

int fastllm_quantize_int4_marlin(const float* w, uint8_t* q, float* scale, int32_t* zero,
                                 int size_n, int size_k, int group_size, void* stream) {
    if (!w || !q || !scale || !zero || size_n <= 0 || size_k <= 0 || group_size <= 0 ||
        size_k % group_size)
        return 1;
    const long tasks = (long)size_n * (size_k / group_size);
    hipLaunchKernelGGL(quantize_int4_marlin_k, dim3(wave_task_grid(tasks)), dim3(256), 0,
                       (hipStream_t)stream, w, q, scale, zero, size_n, size_k, group_size);
    return finish("fastllm_quantize_int4_marlin");
}

int fastllm_quantize_int4_rowmajor(const float* w, uint8_t* packed, void* scales, void* zeros,
                                   int batch, int out_f, int in_f, int group_size, void* stream) {
    if (!w || !packed || !scales || !zeros || batch <= 0 || out_f <= 0 || in_f <= 0 ||
        group_size <= 0 || in_f % group_size || in_f % 2 || group_size % 2)
        return 1;
    const long rows = (long)batch * out_f;
    const long tasks = rows * (in_f / group_size);
    hipLaunchKernelGGL(quantize_int4_rowmajor_k, dim3(wave_task_grid(tasks)), dim3(256), 0,
                       (hipStream_t)stream, w, packed, (f16*)scales, (f16*)zeros, rows, in_f,
                       group_size);
    return finish("fastllm_quantize_int4_rowmajor");
}

int fastllm_dequantize_int4_rowmajor(const uint8_t* packed, const void* scales, const void* zeros,
                                     float* out, int batch, int out_f, int in_f, int group_size,
                                     void* stream) {
    if (!packed || !scales || !zeros || !out || batch <= 0 || out_f <= 0 || in_f <= 0 ||
        group_size <= 0 || in_f % group_size || in_f % 2 || group_size % 2)
        return 1;
    const long rows = (long)batch * out_f;
    hipLaunchKernelGGL(dequantize_int4_rowmajor_k, dim3(grid_for((size_t)rows * in_f / 2, 256)),
                       dim3(256), 0, (hipStream_t)stream, packed, (const f16*)scales,
                       (const f16*)zeros, out, rows, in_f, group_size);
    return finish("fastllm_dequantize_int4_rowmajor");
}

int fastllm_fp8_e4m3_encode(const float* x, uint8_t* out, long n, void* stream) {
    if (!x || !out || n < 0) return 1;
    if (n == 0) return 0;
    hipLaunchKernelGGL(fp8_encode_k, dim3(grid_for((size_t)n, 256)), dim3(256), 0,
                       (hipStream_t)stream, x, out, (size_t)n);
    return finish("fastllm_fp8_e4m3_encode");
}

int fastllm_fp8_e4m3_decode(const uint8_t* b, float* out, long n, void* stream) {
    if (!b || !out || n < 0) return 1;
    if (n == 0) return 0;
    hipLaunchKernelGGL(fp8_decode_k, dim3(grid_for((size_t)n, 256)), dim3(256), 0,
                       (hipStream_t)stream, b, out, (size_t)n);
    return finish("fastllm_fp8_e4m3_decode");
}

int fastllm_quantize_fp8_block(const float* w, uint8_t* q, float* scales, int rows, int cols,
                               int block_size, void* stream) {
    if (!w || !q || !scales || rows <= 0 || cols <= 0 || block_size <= 0 || block_size > 1024)
        return 1;
    const dim3 grid((cols + block_size - 1) / block_size, (rows + block_size - 1) / block_size);
    hipLaunchKernelGGL(quantize_fp8_block_k, grid, dim3(1024), 0, (hipStream_t)stream, w, q,
                       scales, rows, cols, block_size);
    return finish("fastllm_quantize_fp8_block");
}

int fastllm_quantize_mxfp4(const float* w, uint8_t* codes, uint8_t* e8, long rows, int cols,
                           void* stream) {
    if (!w || !codes || !e8 || rows <= 0 || cols <= 0 || cols % 32) return 1;
    if (!fl_aligned(w, 16) || !fl_aligned(codes, 16)) return 1;
    if (!fl_current_device_supported()) return 2;
    const size_t nblk = (size_t)rows * (cols / 32);
    hipLaunchKernelGGL(quantize_mxfp4_k, dim3(grid_for(nblk, 256)), dim3(256), 0, (hipStream_t)stream,
                       w, codes, e8, nblk, cols);
    return finish("fastllm_quantize_mxfp4");
}

int fastllm_dequantize_mxfp4(const uint8_t* codes, const uint8_t* e8, float* out, long rows, int cols,
                             void* stream) {
    if (!codes || !e8 || !out || rows <= 0 || cols <= 0 || cols % 32) return 1;
    if (!fl_current_device_supported()) return 2;
    const size_t n = (size_t)rows * cols;
    hipLaunchKernelGGL(dequantize_mxfp4_k, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t)stream,
                       codes, e8, out, n, cols);
    return finish("fastllm_dequantize_mxfp4");
}

int fastllm_dequantize_fp8_block(const uint8_t* q, const float* scales, float* out, int rows,
                                 int cols, int block_size, void* stream) {
    if (!q || !scales || !out || rows <= 0 || cols <= 0 || block_size <= 0) return 1;
    hipLaunchKernelGGL(dequantize_fp8_block_k, dim3(grid_for((size_t)rows * cols, 256)), dim3(256),
                       0, (hipStream_t)stream, q, scales, out, rows, cols, block_size);
    return finish("fastllm_dequantize_fp8_block");
}

}  // extern "C"
