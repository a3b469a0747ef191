// Pieces shared by the decode-shaped (M <= 16) MFMA GEMV kernels.
//
// Work split: one workgroup = `nwaves` waves on a strip of T 16-column
// n-tiles; the strip's full 128-k blocks are dealt to the waves round-robin;
// the waves meet in LDS at the end and reduce in a fixed order.
#pragma once

#include "common.cuh"

// Staging of the M x K activations (16-bit elements) into LDS rows of stride
// `lda` halves by the first `sw = ceil(M*K/8 / 256)` waves, split in two so
// the weight loads go out in between: load() issues this lane's 4 chunk
// loads (8 halves each) before the wave's weight loads, store() writes them
// to LDS after.  Vector loads retire in issue order, so the store waits only
// for the activation loads while the weight loads stay in flight.  Indices
// are clamped so every lane loads and stores (duplicates rewrite the same
// value).
struct RowStager {
    u32x4 v[4];
    int dst[4];
    template <typename E>
    FL_DEV void load(const E* __restrict__ A, int M, int K, int lda, int wave, int lane) {
        const int k8 = K >> 3;
        const int nchunks = M * k8;
        const float inv_k8 = 1.0f / (float)k8;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            int c = (wave * 64 + lane) * 4 + r;
            c = c < nchunks ? c : nchunks - 1;
            int m = (int)((float)c * inv_k8);
            m -= (m * k8 > c) ? 1 : 0;
            m += ((m + 1) * k8 <= c) ? 1 : 0;
            const int c8 = c - m * k8;
            v[r] = *reinterpret_cast<const u32x4*>(A + (size_t)m * K + c8 * 8);
            dst[r] = m * lda + c8 * 8;
        }
    }
    template <typename E>
    FL_DEV void store(E* __restrict__ As) const {
#pragma unroll
        for (int r = 0; r < 4; ++r) *reinterpret_cast<u32x4*>(As + dst[r]) = v[r];
    }
};

template <typename E>
FL_DEV void stage_rows_loop(const E* __restrict__ A, E* __restrict__ As, int M, int K, int lda) {
    const int k8 = K >> 3;
    for (int idx = threadIdx.x; idx < M * k8; idx += blockDim.x) {
        const int m = idx / k8, c8 = idx - m * k8;
        *reinterpret_cast<u32x4*>(As + (size_t)m * lda + c8 * 8) =
            *reinterpret_cast<const u32x4*>(A + (size_t)m * K + c8 * 8);
    }
}

// Waves needed to stage M x K activations early (4 x 16 B per lane).
__host__ __device__ inline int stage_waves(int M, int K) { return (M * (K >> 3) + 255) >> 8; }

// Cross-wave reduction of T 16x16 fp32 accumulator tiles and the store of
// the rows < M.  out(m, t, c) receives the reduced value of output row m,
// tile t, tile column c.
template <int T, typename Store>
FL_DEV void reduce_and_store(float* __restrict__ red, const f32x4 (&acc)[T], int M, int wave,
                             int nwaves, int lane, Store out) {
#pragma unroll
    for (int t = 0; t < T; ++t)
        *reinterpret_cast<f32x4*>(red + (wave * T + t) * 256 + lane * 4) = acc[t];
    __syncthreads();
    for (int idx = threadIdx.x; idx < T * 256; idx += blockDim.x) {
        const int l = (idx & 255) >> 2, e = idx & 3, t = idx >> 8;
        const int m = 4 * (l >> 4) + e;
        if (m >= M) continue;
        float v = 0.f;
        for (int w = 0; w < nwaves; ++w) v += red[(w * T + t) * 256 + (idx & 255)];
        out(m, t, l & 15, v);
    }
}
