// Residual add + RMSNorm on gfx950, the op that feeds every decode GEMV's
// input (reference: fastllm_py/graph_decode.py:291-326 `add_rmsnorm`,
// graph_decode.py:715-731 `_add_rmsnorm`):
//
//   xnew[r, :] = x[r, :] + delta[r, :]                      (fp32, stored)
//   h[r, :]    = fp16(xnew[r, :] * (1 / sqrt(mean(xnew[r, :]^2) + eps)) * w)
//
// x, delta and w are each fp32 or fp16.  One workgroup per row with the
// reference's thread count (256, or 128 below dim 256) and its summation
// order: thread t accumulates v*v (fused multiply-add) over i = t, t + nt, ...
// in order, then the nt partials are summed by the halving tree
// p[t] += p[t + s], s = nt/2 .. 1.  So the sum of squares, and xnew, are
// bit-identical to the reference's; 1/sqrt(mean + eps) is taken in double and
// rounded once to float, where the reference uses the hardware approximation
// rsqrtf on a float quotient.
// Bandwidth-bound (3 reads + 2 writes per element); rows are independent.
#include "common.cuh"
#include "device.cuh"

namespace {

constexpr int kRegPer = 32;  // values per thread kept in registers (dim <= 32 nt)

template <bool XF, bool DF, bool WF>
__global__ __launch_bounds__(256) void add_rmsnorm_k(const void* __restrict__ xv,
                                                     const void* __restrict__ dv,
                                                     const void* __restrict__ wv,
                                                     float* __restrict__ xnew,
                                                     uint16_t* __restrict__ h, int dim, float eps) {
    __shared__ float part[256];
    const int row = blockIdx.x, tid = threadIdx.x, nt = blockDim.x;
    const size_t base = (size_t)row * dim;
    auto ld = [](const void* p, size_t i, bool f32) {
        return f32 ? static_cast<const float*>(p)[i]
                   : (float)bitcast<f16>(static_cast<const uint16_t*>(p)[i]);
    };
    // a thread's values stay in registers when they fit (one global pass)
    const bool regs = dim <= kRegPer * nt;
    float vr[kRegPer], wr[kRegPer];
    float acc = 0.0f;
    if (regs) {
        // every load unconditional (index clamped into the row; values past
        // dim are never used), so all of them go out before the first wait --
        // a guarded load becomes a branch with its own wait, one round trip
        // per value.  w is loaded here too, ahead of the reduction.
#pragma unroll
        for (int j = 0; j < kRegPer; ++j) {
            const int i = tid + j * nt;
            const int ic = i < dim ? i : dim - 1;
            vr[j] = ld(xv, base + ic, XF) + ld(dv, base + ic, DF);
            wr[j] = ld(wv, ic, WF);
        }
#pragma unroll
        for (int j = 0; j < kRegPer; ++j) {
            const int i = tid + j * nt;
            if (i < dim) {
                xnew[base + i] = vr[j];
                acc = __builtin_fmaf(vr[j], vr[j], acc);
            }
        }
    } else {
        for (int i = tid; i < dim; i += nt) {
            const float v = ld(xv, base + i, XF) + ld(dv, base + i, DF);
            xnew[base + i] = v;
            acc = __builtin_fmaf(v, v, acc);
        }
    }
    // the halving tree p[t] += p[t + s], s = nt/2 .. 1: levels s >= 64 across
    // waves through LDS, the rest inside wave 0 (lane t < s adds lane t + s)
    part[tid] = acc;
    __syncthreads();
    for (int s = nt >> 1; s >= 64; s >>= 1) {
        if (tid < s) part[tid] += part[tid + s];
        __syncthreads();
    }
    if (tid < 64) {
        float p = part[tid];
        for (int s = 32; s > 0; s >>= 1) {
            const float o = __shfl_down(p, s, 64);
            if (tid < s) p += o;
        }
        if (tid == 0) part[0] = p;
    }
    __syncthreads();
    // 1 / sqrt(mean + eps) in double, rounded once to float: the same value
    // on any IEEE machine (the oracle computes it the same way)
    const float inv = (float)(1.0 / sqrt((double)part[0] / (double)dim + (double)eps));
    // y is rounded to fp32 before the fp16 conversion, as the reference does;
    // without the asm the compiler may fold the last multiply and the
    // conversion into one mixed-precision instruction that rounds once, which
    // differs from the reference on fp16 ties
    if (regs) {
#pragma unroll
        for (int j = 0; j < kRegPer; ++j) {
            const int i = tid + j * nt;
            if (i < dim) {
                float y = vr[j] * inv * wr[j];
                asm volatile("" : "+v"(y));
                h[base + i] = bitcast<uint16_t>((f16)y);
            }
        }
    } else {
        for (int i = tid; i < dim; i += nt) {
            float y = xnew[base + i] * inv * ld(wv, i, WF);
            asm volatile("" : "+v"(y));
            h[base + i] = bitcast<uint16_t>((f16)y);
        }
    }
}

template <bool XF, bool DF>
void launch_w(bool wf, const void* x, const void* d, const void* w, float* xnew, uint16_t* h,
              int rows, int dim, float eps, int th, hipStream_t st) {
    if (wf)
        hipLaunchKernelGGL((add_rmsnorm_k<XF, DF, true>), dim3(rows), dim3(th), 0, st, x, d, w, xnew, h,
                           dim, eps);
    else
        hipLaunchKernelGGL((add_rmsnorm_k<XF, DF, false>), dim3(rows), dim3(th), 0, st, x, d, w, xnew, h,
                           dim, eps);
}



// out[r, i] = fp16(silu(g) * u) for g = gate[r, i], u = up[r, i] (fp16 in),
// computed in fp32 as g / (1 + exp(-g)) * u -- the reference's swiglu
// (fastllm_py/kernels/ops.py:157-163) and the SwiGLU epilogue of the fused
// gate/up GEMV.  Elementwise, 8 halves per thread where the row allows.
__global__ void swiglu_k(const uint16_t* __restrict__ gate, const uint16_t* __restrict__ up,
                         uint16_t* __restrict__ out, int rows, int cols, int ldg, int ldu, int ldo) {
    const long total = (long)rows * cols;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (long)gridDim.x * blockDim.x) {
        const int r = (int)(i / cols), c = (int)(i - (long)r * cols);
        const float g = (float)bitcast<f16>(gate[(size_t)r * ldg + c]);
        const float u = (float)bitcast<f16>(up[(size_t)r * ldu + c]);
        out[(size_t)r * ldo + c] = bitcast<uint16_t>((f16)(g / (1.0f + expf(-g)) * u));
    }
}

}  // namespace

extern "C" {

int fastllm_swiglu(const void* gate, const void* up, void* out, int rows, int cols, int ld_gate,
                   int ld_up, int ld_out, void* stream) {
    if (!gate || !up || !out || rows <= 0 || cols <= 0) return 1;
    if (ld_gate < cols || ld_up < cols || ld_out < cols) return 1;
    if (!fl_current_device_supported()) return 2;
    const long total = (long)rows * cols;
    const int grid = (int)((total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192);
    hipLaunchKernelGGL(swiglu_k, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                       static_cast<const uint16_t*>(gate), static_cast<const uint16_t*>(up),
                       static_cast<uint16_t*>(out), rows, cols, ld_gate, ld_up, ld_out);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fprintf(stderr, "fastllm_swiglu launch error: %s\n", hipGetErrorString(e));
        return 2;
    }
    return 0;
}

// 0 ok, 1 bad arguments, 2 device / launch error.  *_f32: 1 = fp32, 0 = fp16.
int fastllm_add_rmsnorm(const void* x, int x_f32, const void* delta, int delta_f32, const void* w,
                        int w_f32, float* xnew, uint16_t* h, int rows, int dim, float eps,
                        void* stream) {
    if (!x || !delta || !w || !xnew || !h || rows <= 0 || dim <= 0) return 1;
    if (rows > 0x7FFFFFFF / dim) return 1;
    if (!fl_current_device_supported()) return 2;
    const int th = dim >= 256 ? 256 : 128;
    hipStream_t st = (hipStream_t)stream;
    if (x_f32)
        delta_f32 ? launch_w<true, true>(w_f32, x, delta, w, xnew, h, rows, dim, eps, th, st)
                  : launch_w<true, false>(w_f32, x, delta, w, xnew, h, rows, dim, eps, th, st);
    else
        delta_f32 ? launch_w<false, true>(w_f32, x, delta, w, xnew, h, rows, dim, eps, th, st)
                  : launch_w<false, false>(w_f32, x, delta, w, xnew, h, rows, dim, eps, th, st);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fprintf(stderr, "fastllm_add_rmsnorm launch error: %s\n", hipGetErrorString(e));
        return 2;
    }
    return 0;
}

}  // extern "C"
