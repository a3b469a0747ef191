/* numpy's float32 SIMD exp and pairwise sum, restated in C — TEST ORACLE ONLY.
 *
 * The reference's expert router (fastllm_py/expert_router.py:40-42) computes
 * softmax with np.exp and ndarray.sum on float32 rows.  On x86-64 builds with
 * AVX2/AVX512F, numpy evaluates float32 exp with a Cody-Waite reduction
 * (ln2 split in two), a degree-5 / degree-2 rational approximation in fp32
 * FMAs, an IEEE division and an exact power-of-two scaling; and it sums a
 * contiguous float32 row with an 8-accumulator pairwise summation.  This file
 * restates both so the GPU router can be checked bit for bit independently of
 * which SIMD path the numpy of a given host dispatches.  Pinned against the
 * installed np.exp / np.sum in tests/test_oracle_router.py.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static const float kLog2e = 1.442695040888963407359924681001892137f;
static const float kMagic = 12582912.0f; /* 1.5 * 2^23 */
static const float kLn2Hi = -6.93145752e-1f;
static const float kLn2Lo = -1.42860677e-6f;
static const float kP0 = 9.999999999980870924916e-01f;
static const float kP1 = 7.257664613233124478488e-01f;
static const float kP2 = 2.473615434895520810817e-01f;
static const float kP3 = 5.114512081637298353406e-02f;
static const float kP4 = 6.757896990527504603057e-03f;
static const float kP5 = 5.082762527590693718096e-04f;
static const float kQ0 = 1.0f;
static const float kQ1 = -2.742335390411667452936e-01f;
static const float kQ2 = 2.159509375685829852307e-02f;

float np_expf(float x) {
    if (x != x) return x;
    if (x >= 88.72283935546875f) return INFINITY;
    if (x <= -103.97208404541015625f) return 0.0f;
    volatile float q = x * kLog2e;
    q = (q + kMagic) - kMagic;
    float r = fmaf(q, kLn2Hi, x);
    r = fmaf(q, kLn2Lo, r);
    float num = fmaf(kP5, r, kP4);
    num = fmaf(num, r, kP3);
    num = fmaf(num, r, kP2);
    num = fmaf(num, r, kP1);
    num = fmaf(num, r, kP0);
    float den = fmaf(kQ2, r, kQ1);
    den = fmaf(den, r, kQ0);
    float p = num / den;
    return ldexpf(p, (int)q);
}

void np_expf_array(const float* x, float* y, long n) {
    for (long i = 0; i < n; ++i) y[i] = np_expf(x[i]);
}

/* numpy pairwise summation of n contiguous float32 values (block 128). */
static float pairwise(const float* a, long n) {
    if (n < 8) {
        float res = 0.0f;
        for (long i = 0; i < n; ++i) res += a[i];
        return res;
    } else if (n <= 128) {
        float r[8];
        for (int j = 0; j < 8; ++j) r[j] = a[j];
        long i;
        for (i = 8; i < n - (n % 8); i += 8)
            for (int j = 0; j < 8; ++j) r[j] += a[i + j];
        float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        for (; i < n; ++i) res += a[i];
        return res;
    } else {
        long n2 = n / 2;
        n2 -= n2 % 8;
        return pairwise(a, n2) + pairwise(a + n2, n - n2);
    }
}

float np_sum_f32(const float* a, long n) { return pairwise(a, n); }

void np_sum_rows_f32(const float* a, float* out, long rows, long cols) {
    for (long r = 0; r < rows; ++r) out[r] = pairwise(a + r * cols, cols);
}
