// INT4 group-32/128 weight-only matmul behind the Marlin C-ABI of
// libfastllm_kernels.so (reference: fastllm_py/kernels/marlin.py:56-95,
// native/marlin_stream_entry.inc:8-33).
//
//   C[M, N] (fp16) = A[M, K] (fp16) @ dequant(W)^T,
//   dequant(W)[n, k] = s[g, n] * (q[n, k] - z[g, n]),  g = k / group_size.
//
// The caller-visible formats are the reference's: GPTQ-packed q (u32
// [K/8, N], value k at bits 4*(k%8) of word [k/8, n]) goes in to the repack;
// scales are fp16 [G, N] and zeros packed u32 [G, N/8], both in the Marlin
// 64-column permutation produced by build_marlin_scales_zeros.
//
// The repacked weight is this library's own tile layout (same u32 count as the
// GPTQ input, so callers' buffer sizes are unchanged).  It is shaped for the
// gfx950 MFMA v_mfma_f32_16x16x32_f16 B operand so a wave reads one 16-byte
// vector per lane per 128-k block:
//   * n-tile t (16 output columns) owns u32 [t*2K, (t+1)*2K);
//   * full 128-k block kb at +kb*256: u32 lane*4 + j holds column 16t + lane%16,
//     k = 128kb + 32j + 8(lane/16) + r for r = 0..7;
//   * a trailing 64-k block (K % 128 == 64) at +(K/128)*256: u32 lane*2 + j;
//   * inside a u32, offset r sits in nibble slot {0,4,1,5,2,6,3,7}[r], so
//     (w & 0x000F000F) and (w & 0x00F000F0) (and the same of w >> 8) are the
//     fp16 pairs (k0,k1), (k2,k3), (k4,k5), (k6,k7) once OR-ed with the
//     exponent of 1024 (bits 0-3) or of 64 (bits 4-7).
#include "common.cuh"
#include "device.cuh"

namespace {

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

// Position of (tile-layout u32 index o) in GPTQ coordinates: returns the
// source word index (k/8)*N + n.
FL_DEV size_t tile_index_to_gptq_word(size_t o, int K, int N) {
    const size_t per_tile = 2 * (size_t)K;
    const int t = (int)(o / per_tile);
    const int rem = (int)(o % per_tile);
    const int nfull = K >> 7;
    int kb, lane, j;
    if (rem < nfull * 256) {
        kb = rem >> 8;
        lane = (rem & 255) >> 2;
        j = rem & 3;
    } else {
        kb = nfull;
        const int r2 = rem - nfull * 256;
        lane = r2 >> 1;
        j = r2 & 1;
    }
    const int n = 16 * t + (lane & 15);
    const int k0 = 128 * kb + 32 * j + 8 * (lane >> 4);
    return (size_t)(k0 >> 3) * N + n;
}

__global__ void repack_gptq_to_tile(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst,
                                    int K, int N) {
    const size_t total = (size_t)K * N / 8;
    for (size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x; o < total;
         o += (size_t)gridDim.x * blockDim.x) {
        dst[o] = gptq_word_to_tile_word(src[tile_index_to_gptq_word(o, K, N)]);
    }
}

__global__ void unrepack_tile_to_gptq(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst,
                                      int K, int N) {
    const size_t total = (size_t)K * N / 8;
    for (size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x; o < total;
         o += (size_t)gridDim.x * blockDim.x) {
        dst[tile_index_to_gptq_word(o, K, N)] = tile_word_to_gptq_word(src[o]);
    }
}

// Marlin 64-column permutation: column n of a [G, N] scale row is stored at
// (n & ~63) + 8*(n%8) + (n%64)/8 (marlin.py:41-50,149-150).
FL_DEV int marlin_scale_pos(int n) {
    const int cl = n & 63;
    return (n & ~63) + 8 * (cl & 7) + (cl >> 3);
}
// Packed zero of column n lives in u32 word (n/64)*8 + n%8 of the group row,
// nibble slot slot_of((n%64)/8) (marlin.py:152-158).
FL_DEV int marlin_zero(const uint32_t* __restrict__ zrow, int n) {
    const int cl = n & 63;
    const uint32_t w = zrow[((n >> 6) << 3) + (cl & 7)];
    return (int)((w >> (4 * slot_of(cl >> 3))) & 0xFu);
}

// Dequantize one tile-layout u32 into the 8 fp16 B-operand values q - z
// (exact small integers).  zlo = -(1024+z), zhi = -(64+z) as fp16 pairs.
FL_DEV f16x8 dequant_tile_word(uint32_t w, f16x2 zlo, f16x2 zhi) {
    const uint32_t w8 = w >> 8;
    const f16x2 p0 = bitcast<f16x2>((w & 0x000F000Fu) | 0x64006400u) + zlo;
    const f16x2 p1 = bitcast<f16x2>((w & 0x00F000F0u) | 0x54005400u) + zhi;
    const f16x2 p2 = bitcast<f16x2>((w8 & 0x000F000Fu) | 0x64006400u) + zlo;
    const f16x2 p3 = bitcast<f16x2>((w8 & 0x00F000F0u) | 0x54005400u) + zhi;
    f16x8 r;
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
}

FL_DEV void zero_consts(int z, f16x2& zlo, f16x2& zhi) {
    const f16 lo = (f16)(-(1024.0f + (float)z));
    const f16 hi = (f16)(-(64.0f + (float)z));
    zlo = f16x2{lo, lo};
    zhi = f16x2{hi, hi};
}

// One workgroup = W waves on one strip of T n-tiles (16*T output columns).
// The waves split the 128-k blocks of the strip round-robin, each keeping
// MT 16-row m-tiles x T n-tiles of fp32 accumulators, and reduce through LDS
// at the end in a fixed wave order (deterministic, no atomics).
// Per block and tile the four 32-k MFMAs of a group-128 block accumulate q-z
// products, then the fp32 accumulator takes s * partial; group-32 weights
// scale every 32-k MFMA separately.
template <int T, int MT, bool G32>
__global__ __launch_bounds__(1024) void int4_tile_mm(
    const f16* __restrict__ A, const uint32_t* __restrict__ Wq, const f16* __restrict__ S,
    const uint32_t* __restrict__ Z, f16* __restrict__ C, int M, int N, int K, int nwaves) {
    extern __shared__ float red[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int strip = blockIdx.x;
    const int nfull = K >> 7;
    const int nkb = nfull + ((K & 127) ? 1 : 0);
    const int col = lane & 15;  // B/D column and A row within the 16x16 tile
    const int kq = lane >> 4;   // 8-k sub-chunk of each 32-k MFMA step
    const int zwords = N >> 3;

    f32x4 acc[MT][T];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int kb = wave; kb < nkb; kb += nwaves) {
        const bool tail = kb >= nfull;
        u32x4 wv[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const uint32_t* tb = Wq + (size_t)(strip * T + t) * (2 * (size_t)K);
            if (!tail) {
                wv[t] = *reinterpret_cast<const u32x4*>(tb + kb * 256 + lane * 4);
            } else {
                const u32x2 v = *reinterpret_cast<const u32x2*>(tb + nfull * 256 + lane * 2);
                wv[t] = u32x4{v[0], v[1], 0u, 0u};
            }
        }
        f16x8 av[MT][4];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int m = mt * 16 + col;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int k = kb * 128 + 32 * j + 8 * kq;
                if (m < M && (j < 2 || !tail))
                    av[mt][j] = *reinterpret_cast<const f16x8*>(A + (size_t)m * K + k);
                else
                    av[mt][j] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int n = (strip * T + t) * 16 + col;
            const int spos = marlin_scale_pos(n);
            if (!G32) {
                const float s = (float)S[(size_t)kb * N + spos];
                const int z = marlin_zero(Z + (size_t)kb * zwords, n);
                f16x2 zlo, zhi;
                zero_consts(z, zlo, zhi);
                f32x4 part[MT];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) part[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f16x8 b = dequant_tile_word(wv[t][j], zlo, zhi);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) part[mt] = mfma_f16(av[mt][j], b, part[mt]);
                }
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[mt][t][i] = __builtin_fmaf(s, part[mt][i], acc[mt][t][i]);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (tail && j >= 2) break;
                    const int g = kb * 4 + j;
                    const float s = (float)S[(size_t)g * N + spos];
                    const int z = marlin_zero(Z + (size_t)g * zwords, n);
                    f16x2 zlo, zhi;
                    zero_consts(z, zlo, zhi);
                    const f16x8 b = dequant_tile_word(wv[t][j], zlo, zhi);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const f32x4 part = mfma_f16(av[mt][j], b, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            acc[mt][t][i] = __builtin_fmaf(s, part[i], acc[mt][t][i]);
                    }
                }
            }
        }
    }

    // cross-wave reduction, fixed order
    constexpr int PER_WAVE = MT * T * 256;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                red[wave * PER_WAVE + (mt * T + t) * 256 + lane * 4 + i] = acc[mt][t][i];
    __syncthreads();
    for (int idx = threadIdx.x; idx < PER_WAVE; idx += blockDim.x) {
        float v = 0.f;
        for (int w = 0; w < nwaves; ++w) v += red[w * PER_WAVE + idx];
        const int mt = idx / (T * 256);
        const int t = (idx / 256) % T;
        const int l = (idx & 255) >> 2;
        const int i = idx & 3;
        const int m = mt * 16 + 4 * (l >> 4) + i;
        const int n = (strip * T + t) * 16 + (l & 15);
        if (m < M) C[(size_t)m * N + n] = (f16)v;
    }
}

template <int T, int MT, bool G32>
hipError_t launch_tile_mm(const f16* A, const uint32_t* Wq, const f16* S, const uint32_t* Z, f16* C,
                          int M, int N, int K, int nwaves, hipStream_t stream) {
    const int strips = N / (16 * T);
    const size_t lds = (size_t)nwaves * MT * T * 256 * sizeof(float);
    hipLaunchKernelGGL((int4_tile_mm<T, MT, G32>), dim3(strips), dim3(64 * nwaves), lds, stream, A,
                       Wq, S, Z, C, M, N, K, nwaves);
    return hipGetLastError();
}

template <int MT, bool G32>
hipError_t dispatch_t(int T, const f16* A, const uint32_t* Wq, const f16* S, const uint32_t* Z,
                      f16* C, int M, int N, int K, int nwaves, hipStream_t stream) {
    switch (T) {
        case 1: return launch_tile_mm<1, MT, G32>(A, Wq, S, Z, C, M, N, K, nwaves, stream);
        case 2: return launch_tile_mm<2, MT, G32>(A, Wq, S, Z, C, M, N, K, nwaves, stream);
        default: return launch_tile_mm<4, MT, G32>(A, Wq, S, Z, C, M, N, K, nwaves, stream);
    }
}

template <bool G32>
hipError_t dispatch_mt(int MT, int T, const f16* A, const uint32_t* Wq, const f16* S,
                       const uint32_t* Z, f16* C, int M, int N, int K, int nwaves,
                       hipStream_t stream) {
    switch (MT) {
        case 1: return dispatch_t<1, G32>(T, A, Wq, S, Z, C, M, N, K, nwaves, stream);
        case 2: return dispatch_t<2, G32>(T, A, Wq, S, Z, C, M, N, K, nwaves, stream);
        case 3: return dispatch_t<3, G32>(T, A, Wq, S, Z, C, M, N, K, nwaves, stream);
        default: return dispatch_t<4, G32>(T, A, Wq, S, Z, C, M, N, K, nwaves, stream);
    }
}

bool int4_marlin_abi_gemm(const void* a, const uint32_t* q, const void* scales,
                          const uint32_t* zeros, void* c, int M, int N, int K, int group_size,
                          hipStream_t stream) {
    if (M <= 0 || N <= 0 || K <= 0) return false;
    if (group_size != 32 && group_size != 128) return false;
    if (K % group_size != 0 || N % 64 != 0 || K % 64 != 0) return false;
    if (!a || !q || !scales || !zeros || !c) return false;
    if (!fl_aligned(a, 16) || !fl_aligned(q, 16) || !fl_aligned(c, 2) || !fl_aligned(scales, 2) ||
        !fl_aligned(zeros, 4))
        return false;
    if (!fl_current_device_supported()) return false;
    const int nkb = (K + 127) / 128;
    const bool g32 = group_size == 32;
    const f16* A = static_cast<const f16*>(a);
    f16* Cp = static_cast<f16*>(c);
    for (int m0 = 0; m0 < M; m0 += 64) {
        const int Mc = (M - m0) < 64 ? (M - m0) : 64;
        const int MT = (Mc + 15) / 16;
        const int T = 1;
        int nwaves = 16 / MT;
        if (nwaves > nkb) nwaves = nkb;
        if (nwaves < 1) nwaves = 1;
        const hipError_t e =
            g32 ? dispatch_mt<true>(MT, T, A + (size_t)m0 * K, q, static_cast<const f16*>(scales),
                                    zeros, Cp + (size_t)m0 * N, Mc, N, K, nwaves, stream)
                : dispatch_mt<false>(MT, T, A + (size_t)m0 * K, q, static_cast<const f16*>(scales),
                                     zeros, Cp + (size_t)m0 * N, Mc, N, K, nwaves, stream);
        if (e != hipSuccess) {
            fprintf(stderr, "FastllmCudaMarlinHalfInt4Gemm launch error: %s\n", hipGetErrorString(e));
            return false;
        }
    }
    return true;
}

bool int4_repack(const uint32_t* src, uint32_t* dst, int K, int N, bool inverse,
                 hipStream_t stream) {
    if (!src || !dst || K <= 0 || N <= 0 || K % 64 != 0 || N % 64 != 0) return false;
    if (!fl_current_device_supported()) return false;
    const size_t total = (size_t)K * N / 8;
    const int threads = 256;
    size_t blocks = (total + threads - 1) / threads;
    if (blocks > 65536) blocks = 65536;
    if (inverse)
        hipLaunchKernelGGL(unrepack_tile_to_gptq, dim3((unsigned)blocks), dim3(threads), 0, stream,
                           src, dst, K, N);
    else
        hipLaunchKernelGGL(repack_gptq_to_tile, dim3((unsigned)blocks), dim3(threads), 0, stream,
                           src, dst, K, N);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fprintf(stderr, "FastllmCudaGptqMarlinRepack launch error: %s\n", hipGetErrorString(e));
        return false;
    }
    return true;
}

}  // namespace

extern "C" {

bool FastllmCudaGptqMarlinRepack(const uint32_t* b_q_weight, uint32_t* out, int size_k,
                                 int size_n) {
    return int4_repack(b_q_weight, out, size_k, size_n, false, nullptr);
}

bool FastllmCudaGptqMarlinRepackStream(const uint32_t* b_q_weight, uint32_t* out, int size_k,
                                       int size_n, void* stream) {
    return int4_repack(b_q_weight, out, size_k, size_n, false, (hipStream_t)stream);
}

bool fastllm_int4_tile_unrepack(const uint32_t* tile_q, uint32_t* gptq_out, int size_k, int size_n,
                                void* stream) {
    return int4_repack(tile_q, gptq_out, size_k, size_n, true, (hipStream_t)stream);
}

bool FastllmCudaMarlinHalfInt4Gemm(const void* a, const uint32_t* b_q_weight, const void* b_scales,
                                   const uint32_t* b_zeros, void* c, int size_m, int size_n,
                                   int size_k, int group_size, int* workspace) {
    (void)workspace;
    return int4_marlin_abi_gemm(a, b_q_weight, b_scales, b_zeros, c, size_m, size_n, size_k,
                                group_size, nullptr);
}

bool FastllmCudaMarlinHalfInt4GemmStream(const void* a, const uint32_t* b_q_weight,
                                         const void* b_scales, const uint32_t* b_zeros, void* c,
                                         int size_m, int size_n, int size_k, int group_size,
                                         int* workspace, void* stream) {
    (void)workspace;
    return int4_marlin_abi_gemm(a, b_q_weight, b_scales, b_zeros, c, size_m, size_n, size_k,
                                group_size, (hipStream_t)stream);
}

}  // extern "C"
