/* Residual add + RMSNorm, restated from fastllm_py/graph_decode.py:300-322
 * (test oracle only).  Per row: v = x + d (fp32); thread t of nt (256, or
 * 128 below dim 256) accumulates fmaf(v, v, acc) over i = t, t + nt, ... in
 * order; the nt partials are summed by the halving tree p[t] += p[t + s];
 * inv = 1 / sqrt(sum / dim + eps) in double, rounded once to float (the
 * reference's rsqrtf is the hardware approximation on a float quotient);
 * y = (v * inv) * w, returned in fp32 (the caller rounds it to fp16). */
#include <math.h>

void oracle_add_rmsnorm(const float* x, const float* d, const float* w, float* xnew, float* y,
                        int rows, int dim, float eps) {
    const int nt = dim >= 256 ? 256 : 128;
    float part[256];
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (long)r * dim;
        const float* dr = d + (long)r * dim;
        float* xo = xnew + (long)r * dim;
        float* yo = y + (long)r * dim;
        for (int t = 0; t < nt; ++t) {
            float acc = 0.0f;
            for (int i = t; i < dim; i += nt) {
                const float v = xr[i] + dr[i];
                xo[i] = v;
                acc = fmaf(v, v, acc);
            }
            part[t] = acc;
        }
        for (int s = nt >> 1; s > 0; s >>= 1)
            for (int t = 0; t < s; ++t) part[t] += part[t + s];
        const float inv = (float)(1.0 / sqrt((double)part[0] / (double)dim + (double)eps));
        for (int i = 0; i < dim; ++i) {
            const float a = xo[i] * inv;
            yo[i] = a * w[i];
        }
    }
}
