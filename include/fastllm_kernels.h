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
#include <stddef.h>
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
 * for size_m <= 16: `tiles` 16-column n-tiles per workgroup (1, 2 or 4;
 * 4 only with nb <= 4), `waves`
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

/* The Marlin-format GEMM of FastllmCudaMarlinHalfInt4Gemm[Stream] (same
 * arguments and result) with a caller workspace that lets the decode shapes
 * (size_m <= 16) split K over several workgroups: each split stores its fp32
 * partial, the last split of each output strip sums them in split order
 * (deterministic) and writes c.  workspace: device memory of at least
 * fastllm_int4_gemm_ws_bytes(size_m, size_n, size_k, group_size) bytes,
 * 256-byte aligned, zero-filled once before first use (its counters are left
 * at zero by every call, in a fixed 64 KiB region whatever the shape, so
 * calls of different shapes may share one workspace); calls sharing a
 * workspace must not overlap.  A
 * workspace of 0 bytes (or NULL) runs the unsplit kernels.  cfg (NULL for
 * the built-in choice) forces {tiles, waves, blocks per wave, splits} for
 * tuning; a forced shape the kernels cannot take returns 2.  Returns 0, 1
 * for bad arguments, 2 for a device or launch error.
 * No reference counterpart: the reference's workspace (N/64*16 ints,
 * fastllm_py/kernels/marlin.py:162-167) is too small for fp32 partials; the
 * Python layer's gemm_fast passes a sized workspace here. */
size_t fastllm_int4_gemm_ws_bytes(int size_m, int size_n, int size_k, int group_size);
int fastllm_int4_gemm_ws(const void *a, const uint32_t *b_q_weight,
                         const void *b_scales, const uint32_t *b_zeros, void *c,
                         int size_m, int size_n, int size_k, int group_size,
                         void *workspace, size_t workspace_bytes, const int *cfg,
                         void *stream);

/* Gate/up projection with the SwiGLU epilogue, decode-shaped (size_m <= 16):
 * the Marlin-format weight holds size_n = 2 I output columns, gate rows
 * [0, I) then up rows [I, 2 I) (I % 64 == 0, size_k % 128 == 0); writes
 * h[size_m, I] (fp16) = silu(g) * u from the fp16 g, u the plain GEMV would
 * store -- one launch instead of the GEMV and the swiglu kernel.
 * Limits: size_k <= 8192 above size_m = 4 (and for group 32); size_k <= 12288
 * up to size_m = 4 with group 128.  Beyond them it returns 1 and the caller
 * runs the plain GEMV then fastllm_swiglu.
 * Returns 0, 1 for arguments the kernel cannot take, 2 for a device or
 * launch error.
 * Replaces: the gate_up GEMV + swiglu pair of the reference's decode MLP
 * (fastllm_py/kernels/ops.py:144-163, fastllm_py/graph_decode.py's dense
 * FFN); no single reference entry. */
int fastllm_int4_gemm_swiglu(const void *a, const uint32_t *b_q_weight,
                             const void *b_scales, const uint32_t *b_zeros,
                             void *h, int size_m, int size_n, int size_k,
                             int group_size, void *stream);

/* Residual add + RMSNorm feeding a decode GEMV:
 *   xnew = x + delta (fp32), h = fp16(xnew * (1/sqrt(mean(xnew^2) + eps)) * w)
 * per row of `dim`; x, delta, w each fp32 (*_f32 = 1) or fp16 (0).  One
 * workgroup per row with the reference's thread count and summation order
 * (sum of squares bit-identical; 1/sqrt(mean + eps) in double rounded once,
 * where the reference uses rsqrtf).  Returns 0, 1 for bad arguments, 2 for a device or launch
 * error.
 * Replaces: add_rmsnorm / GraphDecoder._add_rmsnorm
 * (fastllm_py/graph_decode.py:291-326, 715-731). */
int fastllm_add_rmsnorm(const void *x, int x_f32, const void *delta, int delta_f32,
                        const void *w, int w_f32, float *xnew, uint16_t *h, int rows,
                        int dim, float eps, void *stream);

/* out[r, i] = fp16(silu(g) * u), g = gate[r * ld_gate + i],
 * u = up[r * ld_up + i], computed in fp32 as g / (1 + exp(-g)) * u; fp16
 * in and out, row strides in elements.  Returns 0, 1 for bad arguments,
 * 2 for a device or launch error.
 * Replaces: swiglu (fastllm_py/kernels/ops.py:144-163). */
int fastllm_swiglu(const void *gate, const void *up, void *out, int rows, int cols,
                   int ld_gate, int ld_up, int ld_out, void *stream);

/* add_rmsnorm fused into the prologue of one decode row's Marlin GEMV (M = 1):
 * xnew = x + delta (fp32, stored), h = fp16(xnew * inv * norm_w) with
 * inv = 1/sqrt(sum(xnew^2)/size_k + eps), and c = h @ dequant(W)^T (fp16,
 * 1 x size_n) -- or, with swiglu != 0, the SwiGLU epilogue of
 * fastllm_int4_gemm_swiglu (c is then 1 x size_n/2).  x fp32, delta and
 * norm_w fp16, 16-byte aligned; size_k % 128 == 0.  h never leaves the chip:
 * every workgroup forms its own blocks of it while its weight loads are in
 * flight (the sum of squares is taken in a different order from the
 * standalone op, so h may differ from it in the last bit).  xnew must not
 * overlap x or delta: workgroup 0 stores it while other workgroups still read
 * them (rc 1 otherwise).  Shapes whose per-wave LDS slots and reduction area
 * exceed 160 KB (group 128, size_k > 12288 with swiglu) return 1; the caller
 * then runs fastllm_add_rmsnorm and the unfused projection.  Returns 0, 1 for
 * arguments the kernel cannot take, 2 for a device or launch error.
 * Replaces: the add_rmsnorm launch before a projection plus that projection
 * (fastllm_py/graph_decode.py:818-826, 858-866); no single reference entry. */
int fastllm_int4_gemm_add_rmsnorm(const float *x, const void *delta, const void *norm_w,
                                  float eps, float *xnew, const uint32_t *b_q_weight,
                                  const void *b_scales, const uint32_t *b_zeros, void *c,
                                  int size_n, int size_k, int group_size, int swiglu,
                                  void *stream);

/* Marlin payload of one matrix (this library's repacked qweight, permuted
 * fp16 scales, packed zeros; size_n % 64 == 0, size_k % 128 == 0, group 32 or
 * 128) -> the fused MoE's stacked tile layout for those rows: qtile
 * (size_n/16, size_k/128, 1024) u8 and sz (size_n/16, size_k/group, 16) u32
 * (fp16 scale | fp16 zero << 16).  Bit-exact: the payload's own integers,
 * scales and zeros, no fp16 round trip.  Returns 0, 1 for bad arguments, 2
 * for a device or launch error.
 * Replaces: build_stacked_experts's dequantize-Marlin-to-fp16 then
 * requantize path for resident Marlin experts (fastllm_py/kernels/
 * moe_int4.py:116-133; docs/next-optimizations.md:108-135). */
int fastllm_marlin_to_moe_tile(const uint32_t *b_q_weight, const void *b_scales,
                               const uint32_t *b_zeros, uint8_t *qtile, uint32_t *sz,
                               int size_n, int size_k, int group_size, void *stream);

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

/* MXFP4 (OCP Microscaling v1.0, section 6.3): w f32 [rows, cols], cols % 32
 * == 0 -> codes u8 [rows, cols/2] (E2M1, column 2i in the low nibble of byte
 * i) and e8 u8 [rows, cols/32] (E8M0 exponent + 127 of each 32-column
 * block).  Block scale X = 2^(floor(log2 amax) - 2), exponent clamped to
 * [-127, 127], X = 1 for an all-zero block; codes = w / X rounded to
 * nearest E2M1, ties to the even code, saturating at 6, sign kept.  Finite
 * inputs only.
 * No reference counterpart: the reference plans MXFP4 expert weights
 * (docs/next-optimizations.md:160-184) without a format of its own. */
int fastllm_quantize_mxfp4(const float *w, uint8_t *codes, uint8_t *e8,
                           long rows, int cols, void *stream);
/* E2M1(code) * 2^(e8 - 127) -> f32 [rows, cols]. */
int fastllm_dequantize_mxfp4(const uint8_t *codes, const uint8_t *e8,
                             float *out, long rows, int cols, void *stream);

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

/* fastllm_fp8_b128x128_gemv with a caller workspace for the prefill GEMM's
 * split-K (M > 64 with fewer than 256 64x128 output tiles: the 2048-wide
 * outputs): up to 4 splits of the 128-k blocks, each storing fp32 partials;
 * the last split of each tile sums them in split order (deterministic) and
 * writes C.  workspace: fastllm_fp8_b128x128_gemm_ws_bytes(M, N, K) bytes
 * (0: no split for this shape), 256-byte aligned, zero-filled once (the
 * tile counters sit in its first 1 KB for every shape and are left at
 * zero, so one workspace serves calls of any shape); calls sharing a
 * workspace must not overlap.  A smaller workspace runs unsplit.  Other arguments and
 * return codes as fastllm_fp8_b128x128_gemv.
 * No reference counterpart (the reference has no FP8 prefill GEMM). */
size_t fastllm_fp8_b128x128_gemm_ws_bytes(int M, int N, int K);
int fastllm_fp8_b128x128_gemm_ws(const void *A, const uint8_t *Wq,
                                 const float *scales, const void *bias,
                                 void *C, int M, int N, int K, int isBf16,
                                 void *workspace, size_t workspace_bytes,
                                 void *stream);

/* ------------------------------------------------------------------------
 * Row-major INT4 GEMV, router, fused selective INT4 MoE
 * (kernels the reference launches as CuPy RawKernels).  Return 0 on
 * success, 1 on bad arguments, 2 on a device/launch error.  Asynchronous.
 * ------------------------------------------------------------------------ */

/* y[M, out_f] = x[M, in_f] @ dequant(W)^T for the row-major INT4 format
 * (qweight u8 [out_f, in_f/2], scales/zeros fp16 [out_f, in_f/group]).
 * x fp32 (x_fp32 = 1) or fp16, y fp32 (y_fp32 = 1) or fp16.  in_f % 128 == 0,
 * in_f <= 16384, group in {32, 64, 128}.
 * Replaces: gemv_int4 (fastllm_py/kernels/moe_int4.py:57-94,490-506) and
 * dgemv (fastllm_py/graph_decode.py:170-216,748-765). */
int fastllm_int4_rowmajor_gemv(const void *x, int x_fp32, const uint8_t *qweight,
                               const void *scales, const void *zeros, void *y,
                               int y_fp32, int M, int out_f, int in_f,
                               int group_size, void *stream);

/* y[M, out_f] = x[M, in_f] @ dequant(W)^T for quantize_int4_group's format
 * (fastllm_py/quantizer.py:97-129): data u8 [out_f, in_f/2], even column in
 * the low nibble; scales and zeros (the group minimum) f32
 * [out_f, in_f/group]; dequant(W) = q * scale + zero.  x fp32 (x_fp32 = 1) or
 * fp16, y fp32 (y_fp32 = 1) or fp16.  in_f % 128 == 0, in_f <= 16384,
 * group in {32, 64} or a multiple of 128 dividing in_f.  The reference has no
 * GPU consumer of this format: its CPU path is dequantize_int4_group
 * (quantizer.py:120-129) followed by a matmul. */
int fastllm_int4_group_gemv(const void *x, int x_fp32, const uint8_t *data,
                            const float *scales, const float *zeros, void *y,
                            int y_fp32, int M, int out_f, int in_f,
                            int group_size, void *stream);

/* logits[T, E] = x[T, hidden] (f32) @ gate_w[E, hidden]^T (fp16), fp32
 * accumulate; with shared_gate_w (fp16 [hidden]) also shared_logit[T].
 * Replaces: gate_matvec (fastllm_py/kernels/moe_int4.py:139-169) and the
 * shared-gate matvec of fastllm_py/graph_decode.py:695-697. */
int fastllm_gate_matvec(const float *x, const void *gate_w,
                        const void *shared_gate_w, float *logits,
                        float *shared_logit, int T, int E, int hidden,
                        void *stream);

/* Top-k routing of logits[T, E] (fp32), E <= 256, top_k <= 16, with numpy's
 * float32 exp/sum arithmetic: scoring 0 = softmax, 1 = sigmoid (+ optional
 * e_score_bias[E] on the selection value); n_group/topk_group = DeepSeek
 * group-limited selection; norm = renormalise over the k weights (+1e-20);
 * times routed_scaling.  Selection and order follow np.argpartition as numpy
 * 2.x runs it for float32 rows of <= 256 on an AVX512_SKX host (its bitonic
 * key/index network decides ties).
 * Outputs: topk_ids/topk_w [T, top_k] (descending selection), optional dense
 * rw [T, E]; optional shared_coef[T] = sigmoid(shared_logit); optional
 * expert-major MoE lists (all or none): n_active[1], active[E] ascending,
 * offsets[E+1], tok[T*top_k] ascending within an expert, tokw[T*top_k].
 * Replaces: route_topk (fastllm_py/expert_router.py:22-71) and
 * _route_topk_kernel (fastllm_py/graph_decode.py:242-285). */
int fastllm_route_topk(const float *logits, int T, int E, int top_k,
                       int scoring, int norm, float routed_scaling,
                       const float *e_score_bias, int n_group, int topk_group,
                       int *topk_ids, float *topk_w, float *rw,
                       const float *shared_logit, float *shared_coef,
                       int *n_active, int *active, int *offsets, int *tok,
                       float *tokw, void *stream);

/* MoE lists (layout of fastllm_route_topk's) for S caller-chosen slots,
 * T <= 16, S <= 256: slot s is expert cand[s] (or s when cand is null) and
 * token t joins it with weight rw[t, expert] (dense rw [T, E], slot_coef
 * null) or slot_coef[s, t] when that weight is nonzero.  Slots keep their
 * order; empty slots and experts outside [0, E) are dropped.  Capacities:
 * active[S], offsets[S+1], tok/tokw[S*T].
 * Replaces: the active-expert scan of fused_moe_weighted
 * (fastllm_py/kernels/moe_int4.py:263-294) and the (eidx, rw) inputs of
 * fused_moe_ffn2 (:372-396). */
int fastllm_moe_build_lists(const float *rw, const float *slot_coef,
                            const int *cand, int T, int E, int S,
                            int *n_active, int *active, int *offsets,
                            int *tok, float *tokw, void *stream);

/* Row-major INT4 (qweight u8 [rows, in_f/2], scales/zeros fp16
 * [rows, in_f/group]) -> the fused MoE's tile layout: qtile u8
 * [rows/16, in_f/128, 1024] (block (R/16, kb) holds at byte 16*(c + 16*q)
 * the row-major bytes [64*kb + 16*q, +16) of row 16*(R/16) + c) and sz u32
 * [rows/16, in_f/group, 16] (scale bits | zero bits << 16).  rows % 16 == 0,
 * in_f % 128 == 0.  fastllm_moe_int4_tile_unpack is the exact inverse.
 * Replaces: the layout step of build_stacked_experts
 * (fastllm_py/kernels/moe_int4.py:116-133); the reference's kernels read
 * the row-major arrays directly. */
int fastllm_moe_int4_tile_repack(const uint8_t *qweight, const void *scales,
                                 const void *zeros, uint8_t *qtile,
                                 uint32_t *sz, long rows, int in_f,
                                 int group_size, void *stream);
int fastllm_moe_int4_tile_unpack(const uint8_t *qtile, const uint32_t *sz,
                                 uint8_t *qweight, void *scales, void *zeros,
                                 long rows, int in_f, int group_size,
                                 void *stream);

/* Low-precision expert tiles for fastllm_moe_lowp_* (rows % 16 == 0,
 * in_f % 128 == 0; stacked experts are rows e * out + r):
 *  - FP8: row-major e4m3 codes q u8 [rows, in_f] (fastllm_quantize_fp8_block
 *    with 128x128 blocks, out % 128 == 0 so no block straddles two experts)
 *    -> qtile u8 [rows/16, in_f/128, 2048]: half h of block (t, kb) holds
 *    at byte 1024*h + 16*(c + 16*q) the 16 codes of row 16*t + c,
 *    k = 128*kb + 32*q + 16*h .. + 15 (each 16-byte load or copy of a lane
 *    then reads whole cache lines with its wave).
 *    The block scales f32 [rows/128, in_f/128] are used as they are.
 *  - MXFP4: codes u8 [rows, in_f/2] and e8 u8 [rows, in_f/32] from
 *    fastllm_quantize_mxfp4 -> qtile u8 [rows/16, in_f/128, 1024] whose
 *    block (t, kb) holds at byte 16*(c + 16*q) + 4*j the 8 codes of row
 *    16*t + c, k = 128*kb + 32*j + 8*q .. + 7 (row-major bytes
 *    64*kb + 16*j + 4*q .. + 3), and e8w u32 [rows/16, in_f/128, 16] whose
 *    word (t, kb, c) holds the E8M0 bytes of blocks 4*kb + j, byte j.
 * No reference counterpart (the layouts feed this library's MFMA kernels). */
int fastllm_moe_fp8_tile_repack(const uint8_t *q, uint8_t *qtile, long rows,
                                int in_f, void *stream);
int fastllm_moe_mxfp4_tile_repack(const uint8_t *codes, const uint8_t *e8,
                                  uint8_t *qtile, uint32_t *e8w, long rows,
                                  int in_f, void *stream);

/* Dense MXFP4 GEMV / GEMM: C[M, N] = A[M, K] @ dequant(W)^T with W in the
 * MXFP4 tile layout above (qtile [N/16, K/128, 1024], e8w [N/16, K/128, 16],
 * one expert's worth), A and C fp16 row-major.  N % 16 == 0, K % 128 == 0.
 * Up to 64 rows (K <= 12288) the decode GEMV, which reads the weights once
 * per 16 rows of A (fast for M <= 16), above 64 rows (M K and N K / 2 below
 * 2^31 bytes) the prefill GEMM on the matrix cores.  Both feed the MFMAs
 * fp16(code * scale) (exact for E8M0 scales from 2^-14 up, rounded below)
 * and accumulate in fp32 in a fixed order, rounded once to fp16.
 * Returns 0, 1 for bad arguments, 2 for a device or launch error.
 * Asynchronous on `stream`.
 * No reference counterpart: the dense decode GEMV and prefill GEMM of the
 * MXFP4 weights that docs/next-optimizations.md:160-184 plans (MXFP4 exists
 * in the reference only as that plan). */
int fastllm_mxfp4_gemv(const void *A, const uint8_t *qtile,
                       const uint32_t *e8w, void *C, int M, int N, int K,
                       void *stream);

/* Bytes of device workspace fastllm_moe_int4_fused needs for this shape
 * (0 when the shape is unsupported). */
size_t fastllm_moe_int4_workspace_bytes(int T, int hidden, int inter,
                                        int shared_inter, int max_entries);

/* Fused selective INT4 MoE FFN (x fp32 [T, hidden], hidden % 128 == 0):
 *   y[t] = sum_{entries p of t} tokw[p] * down_e(silu(gate_e x_t) * up_e x_t)
 *          + shared_coef[t] * shared(x_t)          (y fp32 [T, hidden])
 * driven by MoE lists (fastllm_route_topk / fastllm_moe_build_lists) with at
 * most max_slots (<= 256) slots and max_entries entries.  Experts in the tile
 * layout (fastllm_moe_int4_tile_repack of the stacked row-major arrays):
 * gq/gsz, uq/usz over rows E*inter, in_f hidden; dq/dsz over rows E*hidden,
 * in_f inter; the shared expert the same with E = 1 and shared_inter (0 =
 * none; shared_coef null = 1).  workspace: fastllm_moe_int4_workspace_bytes(
 * T, hidden, inter, shared_inter, max_entries) bytes, 16-byte aligned; calls
 * sharing one workspace must not overlap.
 * T <= 16 (decode; hidden <= 4096, inter <= 8192): two launches --
 * gate/up + SwiGLU over the routed tokens only (also zeroes y), then the
 * down projection adding each term into y with fp32 atomics, as the
 * reference's moew_down does (the last bits of y depend on the order of
 * arrival).
 * T > 16 (prefill, hidden % 256 == 0): grouped GEMM kernels on the matrix
 * cores (fp16 copy of x, gate/up per slot in 64-row chunks, down).
 * Replaces: fused_moe_weighted (fastllm_py/kernels/moe_int4.py:175-294),
 * fused_moe_ffn2 (:300-396), fused_moe_ffn (:402-487) and the routed+shared
 * part of _moe_branch (fastllm_py/graph_decode.py:688-699). */
int fastllm_moe_int4_fused(const float *x, int T, int hidden, int group_size,
                           int E, int inter, const uint8_t *gq,
                           const uint32_t *gsz, const uint8_t *uq,
                           const uint32_t *usz, const uint8_t *dq,
                           const uint32_t *dsz, int shared_inter,
                           const uint8_t *sgq, const uint32_t *sgsz,
                           const uint8_t *suq, const uint32_t *susz,
                           const uint8_t *sdq, const uint32_t *sdsz,
                           const float *shared_coef, const int *n_active,
                           const int *active, const int *offsets,
                           const int *tok, const float *tokw, int max_slots,
                           int max_entries, void *workspace,
                           size_t workspace_bytes, float *y, void *stream);

/* Router + fused MoE in one call: fastllm_route_topk (same arguments, same
 * outputs topk_ids/topk_w/rw/shared_coef and lists, bit for bit) followed by
 * fastllm_moe_int4_fused over its lists with max_slots = min(E, T * top_k),
 * max_entries = T * top_k and, when shared_logit is given, shared_coef =
 * sigmoid(shared_logit) (shared_coef must then be given).  Every argument is
 * checked before the first launch.  Expert arguments and workspace as
 * fastllm_moe_int4_fused.  Above 16 tokens (T * top_k <= 4096,
 * E * ceil(T / 32) <= 4096) the router's last workgroup builds the lists and
 * its spare workgroups write the fp16 copy of x, so the call is three
 * launches; the workspace then holds the router's arrival counter and must
 * be zero-filled before its first use (every call leaves the counter at
 * zero).
 * Replaces: the router + routed/shared expert launches of _moe_branch
 * (fastllm_py/graph_decode.py:669-700). */
int fastllm_moe_int4_routed(const float *logits, int top_k, int scoring,
                            int norm, float routed_scaling,
                            const float *e_score_bias, int n_group,
                            int topk_group, const float *shared_logit,
                            int *topk_ids, float *topk_w, float *rw,
                            float *shared_coef, int *n_active, int *active,
                            int *offsets, int *tok, float *tokw,
                            const float *x, int T, int hidden, int group_size,
                            int E, int inter, const uint8_t *gq,
                            const uint32_t *gsz, const uint8_t *uq,
                            const uint32_t *usz, const uint8_t *dq,
                            const uint32_t *dsz, int shared_inter,
                            const uint8_t *sgq, const uint32_t *sgsz,
                            const uint8_t *suq, const uint32_t *susz,
                            const uint8_t *sdq, const uint32_t *sdsz,
                            void *workspace, size_t workspace_bytes, float *y,
                            void *stream);

/* The fused MoE with FP8 or MXFP4 expert weights: the decode kernels up to
 * 16 tokens, the grouped MFMA kernels above (the workspace is sized as for
 * INT4 by fastllm_moe_int4_workspace_bytes; fastllm_moe_lowp_routed takes
 * the batches of fastllm_moe_int4_routed, with the same workspace rule).  format FASTLLM_MOE_FP8 (group_size
 * must be 128): gq/uq/dq are the FP8 tiles and gsz/usz/dsz the f32 block
 * scales (passed as uint32 pointers); FASTLLM_MOE_MXFP4 (group_size 32):
 * the MXFP4 tiles and scale words.  The codes become fp16 exactly and run on
 * the f16 matrix cores against the fp16 activations; block scales multiply
 * the fp32 results.  Other arguments, outputs and return codes as
 * fastllm_moe_int4_fused / fastllm_moe_int4_routed; other formats return 1.
 * No single reference counterpart: the tensor-core fused MoE with FP8 /
 * MXFP4 experts of docs/next-optimizations.md:160-184 (the reference's
 * graph path runs INT4 experts only, fastllm_py/graph_decode.py:669-700). */
#define FASTLLM_MOE_FP8 1
#define FASTLLM_MOE_MXFP4 2
int fastllm_moe_lowp_fused(int format, const float *x, int T, int hidden,
                           int group_size, int E, int inter,
                           const uint8_t *gq, const uint32_t *gsz,
                           const uint8_t *uq, const uint32_t *usz,
                           const uint8_t *dq, const uint32_t *dsz,
                           int shared_inter, const uint8_t *sgq,
                           const uint32_t *sgsz, const uint8_t *suq,
                           const uint32_t *susz, const uint8_t *sdq,
                           const uint32_t *sdsz, const float *shared_coef,
                           const int *n_active, const int *active,
                           const int *offsets, const int *tok,
                           const float *tokw, int max_slots, int max_entries,
                           void *workspace, size_t workspace_bytes, float *y,
                           void *stream);
int fastllm_moe_lowp_routed(int format, const float *logits, int top_k,
                            int scoring, int norm, float routed_scaling,
                            const float *e_score_bias, int n_group,
                            int topk_group, const float *shared_logit,
                            int *topk_ids, float *topk_w, float *rw,
                            float *shared_coef, int *n_active, int *active,
                            int *offsets, int *tok, float *tokw,
                            const float *x, int T, int hidden, int group_size,
                            int E, int inter, const uint8_t *gq,
                            const uint32_t *gsz, const uint8_t *uq,
                            const uint32_t *usz, const uint8_t *dq,
                            const uint32_t *dsz, int shared_inter,
                            const uint8_t *sgq, const uint32_t *sgsz,
                            const uint8_t *suq, const uint32_t *susz,
                            const uint8_t *sdq, const uint32_t *sdsz,
                            void *workspace, size_t workspace_bytes, float *y,
                            void *stream);

/* The fused MoE entries with a weight format (0 INT4, FASTLLM_MOE_FP8,
 * FASTLLM_MOE_MXFP4) and call flags.  FASTLLM_MOE_DETERMINISTIC: the down
 * projections store each term into the workspace instead of adding it into
 * y with fp32 atomics, and one more launch sums every token's terms in a
 * fixed order (its list entries in ascending entry order, i.e. ascending
 * expert, then the shared expert's pieces), so repeated calls on the same
 * inputs give bit-identical y; it needs max_slots <= 256 and the workspace
 * of fastllm_moe_workspace_bytes_ex with the same flags (more than without:
 * (max_entries + pieces*T) x hidden fp32 term rows).  flags 0 is exactly the
 * entries above.  Unknown flags or formats return 1 (0 bytes).
 * No reference counterpart: the reference's moew_down adds with atomicAdd
 * (fastllm_py/kernels/moe_int4.py:250), whose order varies between calls. */
#define FASTLLM_MOE_DETERMINISTIC 1
size_t fastllm_moe_workspace_bytes_ex(int T, int hidden, int inter,
                                      int shared_inter, int max_entries,
                                      int flags);
int fastllm_moe_fused_ex(int format, int flags, const float *x, int T,
                         int hidden, int group_size, int E, int inter,
                         const uint8_t *gq, const uint32_t *gsz,
                         const uint8_t *uq, const uint32_t *usz,
                         const uint8_t *dq, const uint32_t *dsz,
                         int shared_inter, const uint8_t *sgq,
                         const uint32_t *sgsz, const uint8_t *suq,
                         const uint32_t *susz, const uint8_t *sdq,
                         const uint32_t *sdsz, const float *shared_coef,
                         const int *n_active, const int *active,
                         const int *offsets, const int *tok,
                         const float *tokw, int max_slots, int max_entries,
                         void *workspace, size_t workspace_bytes, float *y,
                         void *stream);
int fastllm_moe_routed_ex(int format, int flags, const float *logits,
                          int top_k, int scoring, int norm,
                          float routed_scaling, const float *e_score_bias,
                          int n_group, int topk_group,
                          const float *shared_logit, int *topk_ids,
                          float *topk_w, float *rw, float *shared_coef,
                          int *n_active, int *active, int *offsets, int *tok,
                          float *tokw, const float *x, int T, int hidden,
                          int group_size, int E, int inter, const uint8_t *gq,
                          const uint32_t *gsz, const uint8_t *uq,
                          const uint32_t *usz, const uint8_t *dq,
                          const uint32_t *dsz, int shared_inter,
                          const uint8_t *sgq, const uint32_t *sgsz,
                          const uint8_t *suq, const uint32_t *susz,
                          const uint8_t *sdq, const uint32_t *sdsz,
                          void *workspace, size_t workspace_bytes, float *y,
                          void *stream);

/* fastllm_moe_int4_routed without the workspace argument: the workspace is a
 * static device array of the library, FASTLLM_MOE_SCRATCH_BYTES (16 MiB) per
 * GPU, held until the process ends, so the call allocates nothing (no
 * hipMalloc/hipFree, no allocating library routine).  Shapes whose workspace
 * (fastllm_moe_int4_workspace_bytes) exceeds it return 1 with a message on
 * stderr.  Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (different streams or threads) race and must not be issued.
 * The first call on each device resolves the array's address on that device
 * (hipGetSymbolAddress); make it outside graph capture.  Other arguments,
 * outputs and return codes as fastllm_moe_int4_routed.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). */
#define FASTLLM_MOE_SCRATCH_BYTES ((size_t)16 << 20)
int fastllm_moe_int4_routed_noalloc(const float *logits, int top_k, int scoring,
                                    int norm, float routed_scaling,
                                    const float *e_score_bias, int n_group,
                                    int topk_group, const float *shared_logit,
                                    int *topk_ids, float *topk_w, float *rw,
                                    float *shared_coef, int *n_active,
                                    int *active, int *offsets, int *tok,
                                    float *tokw, const float *x, int T,
                                    int hidden, int group_size, int E,
                                    int inter, const uint8_t *gq,
                                    const uint32_t *gsz, const uint8_t *uq,
                                    const uint32_t *usz, const uint8_t *dq,
                                    const uint32_t *dsz, int shared_inter,
                                    const uint8_t *sgq, const uint32_t *sgsz,
                                    const uint8_t *suq, const uint32_t *susz,
                                    const uint8_t *sdq, const uint32_t *sdsz,
                                    float *y, void *stream);

/* ------------------------------------------------------------------------
 * Measurement
 * ------------------------------------------------------------------------ */

/* HBM streaming-read probe: reads `bytes` (a multiple of 16) from `src`
 * (16-byte aligned) with the decode GEMVs' access shape (contiguous 1 KB per
 * wave load, non-temporal), `loads_per_lane` (4, 8 or 16) loads per lane all
 * in flight, and writes nothing (sink: 1024 words, written only if the
 * folded data equals a fixed constant).  Its per-launch time at a GEMV's
 * byte count is the floor that GEMV's launch can reach.  loads_per_lane + 64:
 * every wave also stores one word once its loads have landed (the dependent
 * store a GEMV ends with).  0 ok, 1 bad arguments, 2 device /
 * launch error.
 * No counterpart in the reference: bench.py's calibration of the GEMV
 * figures against the device's own streaming rate. */
int fastllm_hbm_read_probe(const void *src, size_t bytes, uint32_t *sink,
                           int loads_per_lane, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* FASTLLM_KERNELS_H */
