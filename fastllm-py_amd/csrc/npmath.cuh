// Device versions of the two numpy float32 primitives the reference's expert
// router depends on (fastllm_py/expert_router.py:37-42,58): np.exp on a
// contiguous float32 array and the row sum of a float32 array.  Both follow
// numpy's published algorithms so the GPU router reproduces the CPU router
// bit for bit:
//   * exp: Cody-Waite reduction by ln2 split in a high and a low part,
//     degree-5 / degree-2 rational approximation evaluated with fp32 FMAs,
//     IEEE division, exact scaling by 2^q (numpy's AVX2/AVX512F float32 exp);
//   * sum: pairwise summation with 8 accumulators, blocks of 128, and a
//     plain left-to-right loop (starting from 0) below 8 elements.
#pragma once

#include "common.cuh"

__host__ __device__ inline float np_expf(float x) {
    if (x != x) return x;
    if (x >= 88.72283935546875f) return __builtin_inff();
    if (x <= -103.97208404541015625f) return 0.0f;
    float q = x * 1.442695040888963407359924681001892137f;
    q = (q + 12582912.0f) - 12582912.0f;  // round to nearest even integer
    float r = __builtin_fmaf(q, -6.93145752e-1f, x);
    r = __builtin_fmaf(q, -1.42860677e-6f, r);
    float num = __builtin_fmaf(5.082762527590693718096e-04f, r, 6.757896990527504603057e-03f);
    num = __builtin_fmaf(num, r, 5.114512081637298353406e-02f);
    num = __builtin_fmaf(num, r, 2.473615434895520810817e-01f);
    num = __builtin_fmaf(num, r, 7.257664613233124478488e-01f);
    num = __builtin_fmaf(num, r, 9.999999999980870924916e-01f);
    float den = __builtin_fmaf(2.159509375685829852307e-02f, r, -2.742335390411667452936e-01f);
    den = __builtin_fmaf(den, r, 1.0f);
    return ldexpf(num / den, (int)q);
}

// numpy pairwise sum of n contiguous floats (n <= 1024), sequential.
__host__ __device__ inline float np_pairwise_block(const float* a, int n) {
    if (n < 8) {
        float res = 0.0f;
        for (int i = 0; i < n; ++i) res += a[i];
        return res;
    }
    float r[8];
    for (int j = 0; j < 8; ++j) r[j] = a[j];
    int i;
    for (i = 8; i < n - (n % 8); i += 8)
        for (int j = 0; j < 8; ++j) r[j] += a[i + j];
    float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n; ++i) res += a[i];
    return res;
}

// numpy's recursion: a row longer than 128 splits at n/2 rounded down to a
// multiple of 8; each side <= 128 is one block.  Depth 3 covers n <= 1024.
template <int D>
__host__ __device__ inline float np_sum_rec(const float* a, int n) {
    if (D == 0 || n <= 128) return np_pairwise_block(a, n);
    int n2 = n / 2;
    n2 -= n2 % 8;
    return np_sum_rec<(D > 0 ? D - 1 : 0)>(a, n2) + np_sum_rec<(D > 0 ? D - 1 : 0)>(a + n2, n - n2);
}

__host__ __device__ inline float np_sum_f32(const float* a, int n) { return np_sum_rec<3>(a, n); }

// np_sum_f32 for n <= 256 evaluated by one wave, same result bit for bit.
// The recursion's leaves (at most three for n <= 256: [0, n2) and the right
// part, split once more when longer than 128) go to lane groups of 8; lane j
// of a group forms accumulator r[j] over its leaf in numpy's order, the
// groups fold ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)) with xor-shuffles (the
// same sums: float addition is commutative), add the leaf's tail, and lane 0
// joins the leaves as the recursion does.  `a` may be LDS.  All lanes return
// the sum.
__device__ inline float np_sum_wave(const float* a, int n, int lane) {
    int s1 = 0, l0 = n, l1 = 0, s2 = 0, l2 = 0, nl = 1;
    if (n > 128) {
        const int h = n / 2, n2 = h - h % 8, m = n - n2;
        l0 = n2;
        s1 = n2;
        nl = 2;
        l1 = m;
        if (m > 128) {
            const int hm = m / 2, m2 = hm - hm % 8;
            l1 = m2;
            s2 = n2 + m2;
            l2 = m - m2;
            nl = 3;
        }
    }
    const int leaf = lane >> 3, j = lane & 7;
    const int ls = leaf == 0 ? 0 : (leaf == 1 ? s1 : s2);
    const int ll = leaf == 0 ? l0 : (leaf == 1 ? l1 : (leaf == 2 ? l2 : 0));
    const bool blk = leaf < nl && ll >= 8;
    float r = 0.0f;
    if (blk) {
        r = a[ls + j];
        for (int i = 8; i < ll - ll % 8; i += 8) r += a[ls + i + j];
    }
    r = r + __shfl_xor(r, 1, 64);
    r = r + __shfl_xor(r, 2, 64);
    r = r + __shfl_xor(r, 4, 64);
    float res = 0.0f;
    if (j == 0 && leaf < nl) {
        res = blk ? r : 0.0f;
        for (int i = blk ? ll - ll % 8 : 0; i < ll; ++i) res += a[ls + i];
    }
    const float f0 = __shfl(res, 0, 64), f1 = __shfl(res, 8, 64), f2 = __shfl(res, 16, 64);
    return nl == 1 ? f0 : (nl == 2 ? f0 + f1 : f0 + (f1 + f2));
}
