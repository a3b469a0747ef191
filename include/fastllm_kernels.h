/*
 * libfastllm_kernels.so — MI355X (gfx950) quantized-weight matmul library.
 *
 * C ABI, drop-in for the ctypes entry points of the reference's
 * native/libfastllm_kernels.so, plus entry points for the kernels the
 * reference launches as CuPy RawKernels.  Every pointer is a device pointer
 * on the calling thread's current HIP device; every `stream` argument is a
 * hipStream_t (nullptr = the null stream).  The library allocates no device
 * memory in any entry point below; callers own every buffer.
 *
 * Reference citations are path:line in codemk8/fastllm-py.
 */
#ifndef FASTLLM_KERNELS_H
#define FASTLLM_KERNELS_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------
 * INT4 group-32/128 weight-only GEMM, Marlin ABI
 * ------------------------------------------------------------------------ */

/* Repack GPTQ-packed INT4 (u32 [size_k/8, size_n], value k at bits 4*(k%8)
 * of word [k/8, n]) into this library's tile layout, same u32 count.
 * size_k % 64 == 0, size_n % 64 == 0.  Null stream, asynchronous.
 * Replaces: FastllmCudaGptqMarlinRepack, bound at
 * fastllm_py/kernels/marlin.py:68-70, called at :182. */
bool FastllmCudaGptqMarlinRepack(const uint32_t *b_q_weight, uint32_t *out,
                                 int size_k, int size_n);

/* Same as FastllmCudaGptqMarlinRepack on an explicit stream.
 * Replaces: FastllmCudaGptqMarlinRepackStream of the Marlin file the
 * reference builds (documented in docs/fastllm-internals.md:399-401). */
bool FastllmCudaGptqMarlinRepackStream(const uint32_t *b_q_weight,
                                       uint32_t *out, int size_k, int size_n,
                                       void *stream);

/* C[size_m, size_n] (fp16) = A[size_m, size_k] (fp16) @ dequant(W)^T with
 * dequant(W)[n,k] = scales[g,n] * (q[n,k] - zeros[g,n]), g = k/group_size.
 * b_q_weight: tile layout from FastllmCudaGptqMarlinRepack.
 * b_scales: fp16 [G, size_n], b_zeros: u32 [G, size_n/8], both in the Marlin
 * permutation built by build_marlin_scales_zeros.
 * Returns false (no launch) for size_n % 64, size_k % 64, group_size not in
 * {32, 128}, size_k % group_size, a/b_q_weight not 16-byte aligned, or a
 * non-gfx950 device.  workspace is accepted for ABI compatibility and is not
 * written.  Null stream, asynchronous.
 * Replaces: FastllmCudaMarlinHalfInt4Gemm, bound at
 * fastllm_py/kernels/marlin.py:72-82, called at :238 and :285. */
bool FastllmCudaMarlinHalfInt4Gemm(const void *a, const uint32_t *b_q_weight,
                                   const void *b_scales,
                                   const uint32_t *b_zeros, void *c,
                                   int size_m, int size_n, int size_k,
                                   int group_size, int *workspace);

/* FastllmCudaMarlinHalfInt4Gemm on an explicit stream (graph-capturable).
 * Replaces: FastllmCudaMarlinHalfInt4GemmStream,
 * native/marlin_stream_entry.inc:8-33, bound at
 * fastllm_py/kernels/marlin.py:86-93, called at :227. */
bool FastllmCudaMarlinHalfInt4GemmStream(const void *a,
                                         const uint32_t *b_q_weight,
                                         const void *b_scales,
                                         const uint32_t *b_zeros, void *c,
                                         int size_m, int size_n, int size_k,
                                         int group_size, int *workspace,
                                         void *stream);

/* FastllmCudaMarlinHalfInt4GemmStream with an explicit launch configuration
 * for size_m <= 16: `tiles` 16-column n-tiles per workgroup (1 or 2), `waves`
 * waves per workgroup (1..16), `nb` the register budget in 128-k blocks per
 * wave (1, 2, 4, 6 or 8; at least ceil((size_k/128)/waves); 4 at most for
 * group 32).
 * Returns false for configurations the shape cannot take.  No counterpart in
 * the reference (Marlin picks its tiling internally); used to tune the
 * default launch table. */
bool fastllm_int4_gemm_config(const void *a, const uint32_t *b_q_weight,
                              const void *b_scales, const uint32_t *b_zeros,
                              void *c, int size_m, int size_n, int size_k,
                              int group_size, int tiles, int waves, int nb,
                              void *stream);

/* Inverse of the repack: tile layout -> GPTQ u32 [size_k/8, size_n].
 * No counterpart in the reference (its repacked layout is opaque); used to
 * prove the repack is a bijection. */
bool fastllm_int4_tile_unrepack(const uint32_t *tile_q, uint32_t *gptq_out,
                                int size_k, int size_n, void *stream);

/* ------------------------------------------------------------------------
 * Packers / unpackers (GPU, bit-exact with the reference's numpy formulas).
 * Return 0 on success, 1 on bad arguments, 2 on a launch error.  All are
 * asynchronous on `stream`.  The reference computes these on the host with
 * numpy (or CuPy through the same expressions); the cited function is the
 * one each entry replaces.
 * ------------------------------------------------------------------------ */

/* q u32 [size_n, size_k] (values 0..15) -> u32 [size_k/8, size_n],
 * value k at bits 4*(k%8).  Replaces: pack_gptq_qweight,
 * fastllm_py/kernels/marlin.py:113-127. */
int fastllm_pack_gptq_qweight(const uint32_t *q, uint32_t *out, int size_n,
                              int size_k, void *stream);

/* scale f32 [size_n, G], zero i32 [size_n, G] -> scales fp16 [G, size_n] and
 * zeros u32 [G, size_n/8] in the Marlin 64-column permutation.
 * Replaces: build_marlin_scales_zeros, fastllm_py/kernels/marlin.py:130-159. */
int fastllm_build_marlin_scales_zeros(const float *scale, const int32_t *zero,
                                      void *scales_out, uint32_t *zeros_out,
                                      int size_n, int num_groups,
                                      void *stream);

/* w f32 [rows, cols] -> packed u8 [rows, cols/2], scales f32 and zeros
 * (= group minimum) f32 [rows, cols/group_size].
 * Replaces: quantize_int4_group, fastllm_py/quantizer.py:97-117. */
int fastllm_quantize_int4_group(const float *w, uint8_t *packed, float *scales,
                                float *zeros, int rows, int cols,
                                int group_size, void *stream);

/* q*scale + zero -> f32 [rows, cols].
 * Replaces: dequantize_int4_group, fastllm_py/quantizer.py:120-129. */
int fastllm_dequantize_int4_group(const uint8_t *packed, const float *scales,
                                  const float *zeros, float *out, int rows,
                                  int cols, int group_size, void *stream);

/* Integer-zero-point RTN of the engine's Marlin packer: w f32 [size_n, size_k]
 * -> q u8 [size_n, size_k], scale f32 [size_n, G], zero i32 [size_n, G].
 * Replaces: the quantization in quantize_marlin_matrix,
 * fastllm_py/moe.py:40-46. */
int fastllm_quantize_int4_marlin(const float *w, uint8_t *q, float *scale,
                                 int32_t *zero, int size_n, int size_k,
                                 int group_size, void *stream);

/* Row-major INT4 format, batched over `batch` matrices: w f32
 * [batch, out_f, in_f] -> packed u8 [batch, out_f, in_f/2], scales/zeros fp16
 * [batch, out_f, in_f/group_size].
 * Replaces: quantize_int4_rowmajor / _quantize_int4_rowmajor_batched,
 * fastllm_py/kernels/moe_int4.py:24-40,97-113. */
int fastllm_quantize_int4_rowmajor(const float *w, uint8_t *packed,
                                   void *scales, void *zeros, int batch,
                                   int out_f, int in_f, int group_size,
                                   void *stream);

/* (q - zero) * scale -> f32 [batch, out_f, in_f].
 * Replaces: dequantize_int4_rowmajor, fastllm_py/kernels/moe_int4.py:43-54. */
int fastllm_dequantize_int4_rowmajor(const uint8_t *packed, const void *scales,
                                     const void *zeros, float *out, int batch,
                                     int out_f, int in_f, int group_size,
                                     void *stream);

/* f32 -> e4m3fn bytes with the reference's rounding and subnormal clip.
 * Replaces: _fp8_e4m3_encode, fastllm_py/quantizer.py:26-51. */
int fastllm_fp8_e4m3_encode(const float *x, uint8_t *out, long n,
                            void *stream);

/* e4m3fn bytes -> f32, exact.
 * Replaces: _fp8_e4m3_decode, fastllm_py/quantizer.py:54-62. */
int fastllm_fp8_e4m3_decode(const uint8_t *b, float *out, long n,
                            void *stream);

/* (block_size x block_size) block FP8: w f32 [rows, cols] -> q u8 [rows, cols]
 * and scales f32 [ceil(rows/bs), ceil(cols/bs)].
 * Replaces: quantize_fp8_block, fastllm_py/quantizer.py:65-85. */
int fastllm_quantize_fp8_block(const float *w, uint8_t *q, float *scales,
                               int rows, int cols, int block_size,
                               void *stream);

/* decode(q) * block scale -> f32 [rows, cols].
 * Replaces: dequantize_fp8_block, fastllm_py/quantizer.py:88-94. */
int fastllm_dequantize_fp8_block(const uint8_t *q, const float *scales,
                                 float *out, int rows, int cols,
                                 int block_size, void *stream);

/* ------------------------------------------------------------------------
 * FP8-E4M3 block-scaled GEMV
 * Return 0 on success, 1 on bad arguments, 2 on a device/launch error
 * (3 for a quantize kernel error), like the reference entries.
 * ------------------------------------------------------------------------ */

/* Quantize a [rows, columns] fp16 (isBf16 == 0) or bf16 device matrix into
 * the inline layout: per row, [128 e4m3 codes][f32 scale] x columns/128;
 * scale = amax/448 (1 if not > 0), codes = satfinite round-to-nearest-even
 * e4m3 of x * (1/scale).  columns % 128 == 0.  Null stream; synchronizes.
 * Replaces: fastllm_fp8_block128_quantize, native/fastllm_fp8_block128.cu:226,
 * bound at fastllm_py/kernels/fp8.py:45-47. */
int fastllm_fp8_block128_quantize(const void *input, void *output, int rows,
                                  int columns, int isBf16);

/* fastllm_fp8_block128_quantize on an explicit stream, asynchronous.  No
 * counterpart in the reference (its entry always synchronizes); for callers
 * that capture graphs. */
int fastllm_fp8_block128_quantize_stream(const void *input, void *output,
                                         int rows, int columns, int isBf16,
                                         void *stream);

/* m + (m/128)*4.  Replaces: fastllm_fp8_block128_packed_row_bytes,
 * native/fastllm_fp8_block128.cu:262, bound at fastllm_py/kernels/fp8.py:49-50. */
int fastllm_fp8_block128_packed_row_bytes(int m);

/* C[n, k] (fp16) = A[n, m] (fp16) @ dequant(W)[k, m]^T (+ bias[k] fp16).
 * W: k rows of perRow bytes in the inline layout; m % 128 == 0; any n.
 * Null stream; synchronizes.  Replaces: fastllm_fp8_block128_gemv_fp16,
 * native/fastllm_fp8_block128.cu:273, bound at fastllm_py/kernels/fp8.py:52-55. */
int fastllm_fp8_block128_gemv_fp16(const void *A, const void *weight, void *C,
                                   const void *bias, int n, int m, int k,
                                   int perRow);

/* fastllm_fp8_block128_gemv_fp16 on an explicit stream (asynchronous), with
 * bf16 activations/outputs/bias when isBf16 != 0.  No counterpart in the
 * reference .so (the reference has the bf16 kernel pair only inside upstream
 * fastllm, docs/fastllm-internals.md:597-612). */
int fastllm_fp8_block128_gemv_stream(const void *A, const void *weight,
                                     void *C, const void *bias, int n, int m,
                                     int k, int perRow, int isBf16,
                                     void *stream);

/* C[M, N] = A[M, K] @ dequant(Wq)^T (+ bias[N]) for the separate-scale
 * 128x128 block format of quantize_fp8_block: Wq u8 [N, K] row-major, scales
 * f32 [ceil(N/128), ceil(K/128)].  A, C, bias fp16 (isBf16 == 0) or bf16.
 * K % 64 == 0 and K >= 128 (a trailing 64-wide block is allowed); any N, M.
 * Asynchronous on `stream`.  No counterpart in the reference's C ABI: it is
 * the GPU consumer of fastllm_py/quantizer.py:65-94's format. */
int fastllm_fp8_b128x128_gemv(const void *A, const uint8_t *Wq,
                              const float *scales, const void *bias, void *C,
                              int M, int N, int K, int isBf16, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* FASTLLM_KERNELS_H */
