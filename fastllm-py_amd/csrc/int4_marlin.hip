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
#include "gemv_common.cuh"
#include "int4_common.cuh"

namespace {

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

// Decode-shaped GEMV (M <= 16): one 16-row m-tile, W waves per workgroup on a
// strip of T n-tiles; the full 128-k blocks of the strip are dealt to the
// waves round-robin, NB at most per wave.
//   * Each wave issues ALL of its weight, scale and zero loads before doing
//     anything else (indices clamped so the issue is unconditional), so HBM
//     latency is paid once per wave and a workgroup keeps W*NB KB in flight.
//   * Activations (AM = activation mode):
//       AM 0 (M <= 4): each wave copies the rows of ITS OWN blocks into its
//         own LDS slot -- one global->LDS copy (buffer_load ... lds, no
//         VGPRs) of 1 KB = 4 rows x 128 k per block, issued before its weight
//         loads -- so no workgroup barrier separates the load issue from the
//         first MFMA.  A barrier there makes every wave wait until the
//         slowest wave has issued all of its loads into a saturated memory
//         system, which serialises the compute tail behind the stream;
//       AM 1: the M x K rows are staged once per workgroup in LDS (row stride
//         K+8 halves) behind an LDS-only barrier;
//       AM 2 (M > 4, NB > 4, M x K too large for AM 1): a ring of three
//         register slots -- the A operands of a wave's first three blocks
//         are loaded ahead of its weights, and block i + 3's are issued once
//         block i's MFMAs have read slot i % 3.  Loads complete in issue
//         order, so the first three blocks wait only for their own weights,
//         and by the time the later blocks' weights have arrived so have
//         their activations (loaded at use, each block would wait a full L2
//         round trip after all of the wave's weights);
//       AM 5 (4 < M <= 8): AM 0's per-wave copies, two per block (rows 0-7
//         in MFMA fragment order, so the 8 distinct rows do not share LDS
//         banks).  Against AM 3 it moves the unique 2 KB per block instead
//         of 16 rows' fragments and holds no VGPRs: Qwen3-8B M = 8 qkv 6.38
//         -> 5.99, o 5.41 -> 5.00, gate_up 14.8 -> 13.8, down 10.5 -> 9.9 us.
//       AM 6 (8 < M <= 16): the block's 16 rows as whole 256-byte rows,
//         4 per copy (16-byte k chunks XOR-swizzled by row), 4 KB per block:
//         Qwen3-8B M = 16 qkv 7.56 -> 6.34, o 6.64 -> 5.27 us.  Copies of
//         16 rows x 64 B (the MFMA fragment order) were no faster than AM 3:
//         such a copy costs the CU's vector-cache path four times the
//         accesses of whole lines;
//       AM 3 (M > 4, NB <= 4): each lane loads its own MFMA A operands of all
//         its blocks from global memory into registers (4 x 16 B per block),
//         first of all, so they arrive ahead of the weights in issue order;
//         no LDS and no barrier -- the whole M x K staging of AM 1 needs so
//         much LDS per workgroup (64 KB at M = 8, K = 4096) that only one
//         workgroup fits a CU.
//     MFMA rows >= M read row M-1: C rows are independent and rows >= M are
//     never stored, so no masking is needed.
//   * A trailing 64-k block (group 32 only) is done by wave 0 at the end.
//   * Cross-wave reduction through LDS in fixed wave order.
// SWI (T = 2): gate/up with the SwiGLU epilogue -- N = 2 I columns, gate
// rows [0, I) and up rows [I, 2 I); strip s pairs gate n-tile s (tile 0)
// with up n-tile I/16 + s (tile 1) and stores H[m, 16 s + c] =
// fp16(silu(g) * u) from the fp16-rounded g and u, which is what the
// unfused GEMV followed by the reference's swiglu computes
// (fastllm_py/kernels/ops.py:157-163).  C is then H, M x I.
// AM 4 (M = 1): the activation row is add_rmsnorm's output, formed in the
// prologue from the residual x (fp32), the branch output d (fp16) and the
// norm weight w (fp16): v = x + d, h = fp16((v * inv) * w) with
// inv = 1 / sqrt(sum(v^2) / K + eps) (reference: graph_decode.py:300-322).
struct NormArgs {
    const float* x;
    const uint16_t* d;
    const uint16_t* w;
    float* xnew;  // x + d, stored by workgroup 0
    float eps;
};

// Split-K (gridDim.y > 1, plain GEMV with register activations only): split
// s of S covers full blocks [s * nb_s, (s + 1) * nb_s); each split stores its
// fp32 partial of the strip with agent-scope atomic stores (coherent across
// XCDs without cache flushes) into ws[(s * M + m) * N + n], waits for them to
// complete, then bumps the strip's counter; the split that finds S - 1 sums the S partials in split
// order (deterministic), writes C and resets the counter to 0.  Nothing
// waits on another workgroup.  The counters start at zero (the caller's
// workspace is zero-filled once) and are left at zero.
struct SplitArgs {
    float* ws = nullptr;
    int* cnt = nullptr;
};

// Sum of the nsplit (<= 16) partials p[0], p[stride], ... in split order,
// read with agent-coherent loads that all issue before the first add (a
// loop of dependent loads costs one memory round trip per split).
constexpr int kMaxSplits = 16;
template <int NS>
FL_DEV float split_sum_n(const float* p, size_t stride) {
    float pv[NS];
#pragma unroll
    for (int q = 0; q < NS; ++q) pv[q] = __hip_atomic_load(p + q * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float v = 0.f;
#pragma unroll
    for (int q = 0; q < NS; ++q) v += pv[q];
    return v;
}

FL_DEV float split_sum(const float* p, size_t stride, int nsplit) {
    switch (nsplit) {
        case 1: return split_sum_n<1>(p, stride);
        case 2: return split_sum_n<2>(p, stride);
        case 3: return split_sum_n<3>(p, stride);
        case 4: return split_sum_n<4>(p, stride);
        case 5: return split_sum_n<5>(p, stride);
        case 6: return split_sum_n<6>(p, stride);
        case 7: return split_sum_n<7>(p, stride);
        case 8: return split_sum_n<8>(p, stride);
        case 9: return split_sum_n<9>(p, stride);
        case 10: return split_sum_n<10>(p, stride);
        case 11: return split_sum_n<11>(p, stride);
        case 12: return split_sum_n<12>(p, stride);
        case 13: return split_sum_n<13>(p, stride);
        case 14: return split_sum_n<14>(p, stride);
        case 15: return split_sum_n<15>(p, stride);
        default: return split_sum_n<16>(p, stride);
    }
}

template <int T, int NB, bool G32, int AM, bool SWI>
__device__ __forceinline__ void int4_gemv_body(const f16* __restrict__ A, const uint32_t* __restrict__ Wq,
                                               const uint16_t* __restrict__ S, const uint32_t* __restrict__ Z,
                                               f16* __restrict__ C, int M, int N, int K,
                                               const NormArgs& nrm = NormArgs{},
                                               const SplitArgs& sp = SplitArgs{}) {
    constexpr int SPB = G32 ? 4 : 1;  // scale groups per 128-k block
    extern __shared__ __align__(16) unsigned char smem[];
    const int nwaves = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // XCD-grouped strips: workgroup b runs on XCD b % 8, so each XCD takes a
    // contiguous range of strips and neighbours share its L2 (scale / zero
    // lines cover 64 columns, the activations every strip)
    const int strip = xcd_block();
    const int nsplit = gridDim.y;
    const int nfull = (K >> 7) / nsplit;  // full 128-k blocks of this split
    const int col = lane & 15;
    const int kq = lane >> 4;
    const int zwords = N >> 3;
    if (nsplit > 1) {  // this split's k-range: shift every block-indexed base
        const int kbo = blockIdx.y * nfull;
        A += (size_t)kbo * 128;
        Wq += (size_t)kbo * 256;
        S += (size_t)kbo * SPB * N;
        Z += (size_t)kbo * SPB * zwords;
    }
    constexpr bool ALDS = AM == 1;
    // per-wave LDS copies of the wave's own blocks: ACP 1 KB copies per block
    constexpr bool ACOPY = AM == 0 || AM == 4 || AM == 5 || AM == 6;
    constexpr int ACP = AM == 5 ? 2 : (AM == 6 ? 4 : 1);
    const int lda = K + 8;
    f16* As = reinterpret_cast<f16*>(smem);
    // AM 0/4/5/6: wave w's slot of NB blocks x ACP KB at w * NB * ACP KB
    const size_t abytes = ACOPY ? (size_t)nwaves * NB * ACP * 1024
                                : (ALDS ? (((size_t)M * lda * 2 + 15) & ~(size_t)15) : 0);
    // AM 6 with four tiles: the cross-wave reduction reuses the activation
    // slots once every wave is past its blocks (a barrier first), so the
    // launch needs the larger of the two, not their sum -- two workgroups
    // per CU where the sum allowed one (down M = 16, four tiles, three K
    // splits: 11.0 us against 11.95 with register fragments).  With one or
    // two tiles the extra barrier cost more than it saved.
    constexpr bool RALIAS = AM == 6 && T == 4;
    float* red = reinterpret_cast<float*>(smem + (RALIAS ? 0 : abytes));

    const int nb = wave < nfull ? (nfull - wave + nwaves - 1) / nwaves : 0;

    int spos[T], zw[T], zsh[T];
    const uint32_t* tbase[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int nt = SWI ? t * (N >> 5) + strip : strip * T + t;  // n-tile of tile t
        const int n = nt * 16 + col;
        if (SWI && t > 0) {
            // the up column n + N/2 lies in the same place of a 64-column
            // chunk N/128 chunks on (N % 128 == 0): scale and zero word
            // positions shift by uniform amounts, the nibble slot stays
            spos[t] = spos[0] + (N >> 1);
            zw[t] = zw[0] + (N >> 4);
            zsh[t] = zsh[0];
        } else {
            spos[t] = marlin_scale_pos(n);
            const int cl = n & 63;
            zw[t] = ((n >> 6) << 3) + (cl & 7);
            zsh[t] = 4 * slot_of(cl >> 3);
        }
        tbase[t] = Wq + (size_t)nt * (2 * (size_t)K);
    }

    // Activations are staged by the first `sw` waves (RowStager: their
    // activation loads go out before their weight loads, the LDS stores
    // after them, so the stores wait only for the activations and the LDS
    // barrier does not drain the weight loads).  M*K too large for that goes
    // through a plain staging loop.
    const int k8 = K >> 3;
    const int nchunks = ALDS ? M * k8 : 0;
    const int sw = (nchunks + 255) >> 8;
    const bool early = sw <= nwaves;
    RowStager stg;
    const bool stager = ALDS && early && wave < sw;
    if (stager) stg.load(A, M, K, lda, wave, lane);
    // AM 0: lane l of block slot i copies row min(l / 16, M - 1), 16-byte
    // piece l % 16 of the block into this wave's LDS slot
    unsigned char* aslot = smem + (size_t)wave * NB * ACP * 1024;
    const int arow_m = col < M ? col : M - 1;
    f16x8 ar[NB][4];
    constexpr int kRing = 3;  // AM 2 register slots
    f16x8 rg[kRing][4];
    if (AM == 2) {
        const f16* ap = A + (size_t)arow_m * K + 8 * kq;
#pragma unroll
        for (int i = 0; i < (NB < kRing ? NB : kRing); ++i) {
            int kb = wave + (i < nb ? i : (nb > 0 ? nb - 1 : 0)) * nwaves;
            kb = kb < nfull ? kb : nfull - 1;
#pragma unroll
            for (int j = 0; j < 4; ++j) rg[i][j] = *reinterpret_cast<const f16x8*>(ap + kb * 128 + 32 * j);
        }
    }
    if (AM == 3) {
        const f16* ap = A + (size_t)arow_m * K + 8 * kq;
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            int kb = wave + (i < nb ? i : (nb > 0 ? nb - 1 : 0)) * nwaves;
            kb = kb < nfull ? kb : nfull - 1;
#pragma unroll
            for (int j = 0; j < 4; ++j) ar[i][j] = *reinterpret_cast<const f16x8*>(ap + kb * 128 + 32 * j);
        }
    }
    if (AM == 0) {
        const int own_m = (lane >> 4) < M ? (lane >> 4) : M - 1;
        const __amdgpu_buffer_rsrc_t rA = buf_rsrc(A, (uint32_t)M * K * 2);
        const uint32_t ao = 2u * ((uint32_t)own_m * K + 8 * (lane & 15));
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            int kb = wave + (i < nb ? i : (nb > 0 ? nb - 1 : 0)) * nwaves;
            kb = kb < nfull ? kb : nfull - 1;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lptr_t)(aslot + i * 1024), 16, ao, kb * 256, 0, 0);
        }
    }
    if (AM == 5) {
        // fragment-major copies of rows 0-7, read back by each lane at its
        // own 16 bytes (the row-major slot of AM 0 would put 8 distinct rows
        // on the same LDS banks): copy p of a block holds MFMA steps 2p and
        // 2p + 1 -- lane l takes row l & 7, k 32 (2p + l / 32) + 8 ((l / 8) & 3)
        // -- and MFMA lanes c and c + 8 read the same piece (rows >= 8 are
        // never stored).  Rows past M repeat row M - 1.
        const __amdgpu_buffer_rsrc_t rA = buf_rsrc(A, (uint32_t)M * K * 2);
        const int r = lane & 7;
        const uint32_t ao = 2u * ((uint32_t)(r < M ? r : M - 1) * K + 32 * (lane >> 5) + 8 * ((lane >> 3) & 3));
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            int kb = wave + (i < nb ? i : (nb > 0 ? nb - 1 : 0)) * nwaves;
            kb = kb < nfull ? kb : nfull - 1;
#pragma unroll
            for (int p = 0; p < 2; ++p)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lptr_t)(aslot + (i * 2 + p) * 1024), 16,
                                                         ao + 128u * p, kb * 256, 0, 0);
        }
    }
    if (AM == 6) {
        // the block's 16 rows (rows past M repeat row M - 1) as whole 256-byte
        // rows, 4 per copy: lane l of copy p takes row r = 4 p + l / 16 and
        // its 16-byte k chunk (l % 16) ^ r into position l % 16 of that row
        // (16 rows x 64 B per copy, the MFMA fragment order, cost the CU's
        // vector-cache path four times the accesses)
        const __amdgpu_buffer_rsrc_t rA = buf_rsrc(A, (uint32_t)M * K * 2);
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            int kb = wave + (i < nb ? i : (nb > 0 ? nb - 1 : 0)) * nwaves;
            kb = kb < nfull ? kb : nfull - 1;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int r = 4 * p + (lane >> 4);
                const uint32_t ao = 2u * ((uint32_t)(r < M ? r : M - 1) * K + 8 * ((lane & 15) ^ r));
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lptr_t)(aslot + (i * 4 + p) * 1024), 16, ao,
                                                         kb * 256, 0, 0);
            }
        }
    }
    if (AM == 4) {
        // slot i of this wave's blocks: [x: 128 fp32][d: 128 fp16][w: 128 fp16];
        // a copy writes lane l's 16 B at slot + 16 l, so lanes 0-31 carry x,
        // 32-47 d and 48-63 w (three copies, each with its lanes active)
        const __amdgpu_buffer_rsrc_t rX = buf_rsrc(nrm.x, (uint32_t)K * 4);
        const __amdgpu_buffer_rsrc_t rD = buf_rsrc(nrm.d, (uint32_t)K * 2);
        const __amdgpu_buffer_rsrc_t rW = buf_rsrc(nrm.w, (uint32_t)K * 2);
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            int kb = wave + (i < nb ? i : (nb > 0 ? nb - 1 : 0)) * nwaves;
            kb = kb < nfull ? kb : nfull - 1;
            lptr_t dst = (lptr_t)(aslot + i * 1024);
            if (lane < 32)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rX, dst, 16, 4u * (kb * 128 + 4 * lane), 0, 0, 0);
            else if (lane < 48)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rD, dst, 16, 2u * (kb * 128 + 8 * (lane - 32)), 0, 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rW, dst, 16, 2u * (kb * 128 + 8 * (lane - 48)), 0, 0, 0);
        }
    }

    // the activation copies above stay ahead of every load below: the wait
    // that hands a wave its copies counts the loads issued after them
    __builtin_amdgcn_sched_barrier(0);

    // One straight-line issue of every load this wave will need (block
    // indices clamped into range: no guard, so nothing derived from the loaded
    // values can be hoisted up here by the compiler).  The tiles of one strip
    // lie in one 64-column chunk unless SWI, so they share each zero word:
    // it is loaded once (zv[i][0]) -- the load count the copy wait relies on
    // is then the count the compiler emits, with nothing left to merge.
    constexpr bool ZSHARE = !SWI && T > 1;
    u32x4 wv[NB][T];
    uint32_t sv[NB][T][SPB], zv[NB][T][SPB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        int kb = wave + (i < nb ? i : (nb > 0 ? nb - 1 : 0)) * nwaves;
        kb = kb < nfull ? kb : nfull - 1;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            wv[i][t] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(tbase[t] + kb * 256 + lane * 4));
#pragma unroll
            for (int g = 0; g < SPB; ++g) {
                const size_t grp = (size_t)kb * SPB + g;
                sv[i][t][g] = S[grp * N + spos[t]];
                zv[i][t][g] = (ZSHARE && t > 0) ? zv[i][0][g] : Z[grp * zwords + zw[t]];
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    if (ACOPY) {
        // this wave's activation copies, issued before its weight, scale and
        // zero loads, are done once at most those loads are outstanding (no
        // barrier: only this wave reads its slot)
        constexpr int WL = NB * (T * (1 + SPB) + (ZSHARE ? 1 : T) * SPB);
        wait_vmcnt<(WL < 63 ? WL : 63)>();
    }
    if (AM == 4) {
        // add_rmsnorm of the one row: sum of v^2 over this wave's live
        // blocks (lane l: elements 2l, 2l + 1), the waves' partials summed in
        // wave order through LDS (an LDS-only barrier: the weights stay in
        // flight), then h of each block into row 0 of its slot
        float* npart = reinterpret_cast<float*>(smem + abytes + (size_t)nwaves * T * 1024);
        float ss = 0.0f;
        float2 v[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const unsigned char* sl = aslot + (size_t)i * 1024;
            const float2 xv = *reinterpret_cast<const float2*>(sl + 8 * lane);
            const uint32_t dv = *reinterpret_cast<const uint32_t*>(sl + 512 + 4 * lane);
            v[i].x = xv.x + (float)bitcast<f16>((uint16_t)(dv & 0xFFFFu));
            v[i].y = xv.y + (float)bitcast<f16>((uint16_t)(dv >> 16));
            if (i < nb) {
                ss = __builtin_fmaf(v[i].x, v[i].x, ss);
                ss = __builtin_fmaf(v[i].y, v[i].y, ss);
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
        if (lane == 0) npart[wave] = ss;
        lds_barrier();
        // the partials in wave order: four 16-byte reads (the launch gives
        // npart 64 floats, so all 16 slots are in the allocation), slots of
        // absent waves masked -- not one dependent LDS read per wave
        float pw[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 f = reinterpret_cast<const float4*>(npart)[q];
            pw[4 * q] = f.x;
            pw[4 * q + 1] = f.y;
            pw[4 * q + 2] = f.z;
            pw[4 * q + 3] = f.w;
        }
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < 16; ++w) tot += w < nwaves ? pw[w] : 0.0f;
        const float inv = (float)(1.0 / sqrt((double)tot / (double)K + (double)nrm.eps));
        uint32_t hv[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const uint32_t wv2 = *reinterpret_cast<const uint32_t*>(aslot + (size_t)i * 1024 + 768 + 4 * lane);
            float y0 = v[i].x * inv * (float)bitcast<f16>((uint16_t)(wv2 & 0xFFFFu));
            float y1 = v[i].y * inv * (float)bitcast<f16>((uint16_t)(wv2 >> 16));
            // rounded to fp32 first, as the reference does (no fused
            // multiply-and-convert)
            asm volatile("" : "+v"(y0), "+v"(y1));
            hv[i] = (uint32_t)bitcast<uint16_t>((f16)y0) | ((uint32_t)bitcast<uint16_t>((f16)y1) << 16);
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < NB; ++i) *reinterpret_cast<uint32_t*>(aslot + (size_t)i * 1024 + 4 * lane) = hv[i];
        if (blockIdx.x == 0) {
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const int kb = wave + i * nwaves;
                if (i < nb) *reinterpret_cast<float2*>(nrm.xnew + kb * 128 + 2 * lane) = v[i];
            }
        }
    }
    if (ALDS) {
        if (stager) stg.store(As);
        if (!early) {
            for (int idx = threadIdx.x; idx < nchunks; idx += blockDim.x) {
                const int m = idx / k8, c8 = idx - m * k8;
                *reinterpret_cast<f16x8*>(As + (size_t)m * lda + c8 * 8) =
                    *reinterpret_cast<const f16x8*>(A + (size_t)m * K + c8 * 8);
            }
        }
        lds_barrier();  // the weight loads stay in flight
    }

    const uint32_t mlo = 0x64006400u, mhi = 0x54005400u;
    const f16* arow = ALDS ? As + (size_t)arow_m * lda + 8 * kq : A + (size_t)arow_m * K + 8 * kq;
    (void)aslot;
    f32x4 acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Straight-line over all NB register slots (no per-block branch, so the
    // compiler cannot hoist the scale/zero unpacking of later blocks next to
    // their loads and wait on them early); slots past this wave's nb repeat
    // its last block with a zero scale.
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const bool live = i < nb;
        int kb = wave + (live ? i : (nb > 0 ? nb - 1 : 0)) * nwaves;
        kb = kb < nfull ? kb : nfull - 1;
        f16x8 a[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (AM == 0 || AM == 4)
                a[j] = *reinterpret_cast<const f16x8*>(aslot + (size_t)i * 1024 + arow_m * 256 +
                                                       2 * (32 * j + 8 * kq));
            else if (AM == 6)
                a[j] = *reinterpret_cast<const f16x8*>(aslot + (size_t)i * 4096 + arow_m * 256 +
                                                       16 * ((4 * j + kq) ^ arow_m));
            else if (AM == 5)
                a[j] = *reinterpret_cast<const f16x8*>(aslot + (size_t)(i * 2 + (j >> 1)) * 1024 +
                                                       16 * ((col & 7) + 8 * kq + 32 * (j & 1)));
            else if (AM == 3)
                a[j] = ar[i][j];
            else if (AM == 2)
                a[j] = rg[i % kRing][j];
            else
                a[j] = *reinterpret_cast<const f16x8*>(arow + kb * 128 + 32 * j);
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            if (!G32) {
                uint32_t zlo, zhi;
                zero_bits((zv[i][t][0] >> zsh[t]) & 0xFu, zlo, zhi);
                f32x4 part = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    part = mfma_f16(a[j], dequant_word_fast(wv[i][t][j], zlo, zhi, mlo, mhi), part);
                const float s = live ? (float)bitcast<f16>((uint16_t)sv[i][t][0]) : 0.0f;
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[t][e] = __builtin_fmaf(s, part[e], acc[t][e]);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    uint32_t zlo, zhi;
                    zero_bits((zv[i][t][j] >> zsh[t]) & 0xFu, zlo, zhi);
                    const f32x4 part = mfma_f16(a[j], dequant_word_fast(wv[i][t][j], zlo, zhi, mlo, mhi),
                                                f32x4{0.f, 0.f, 0.f, 0.f});
                    const float s = live ? (float)bitcast<f16>((uint16_t)sv[i][t][j]) : 0.0f;
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[t][e] = __builtin_fmaf(s, part[e], acc[t][e]);
                }
            }
        }
        if (AM == 2 && i + kRing < NB) {
            // refill the slot block i has just consumed with block i + 3's rows
            __builtin_amdgcn_sched_barrier(0);
            const int ii = i + kRing;
            int kn = wave + (ii < nb ? ii : (nb > 0 ? nb - 1 : 0)) * nwaves;
            kn = kn < nfull ? kn : nfull - 1;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                rg[i % kRing][j] = *reinterpret_cast<const f16x8*>(arow + kn * 128 + 32 * j);
        }
        // keep block i's work in its own scheduling region: blocks then wait
        // only for their own loads, in arrival order
        __builtin_amdgcn_sched_barrier(0);
    }

    if (G32 && (K & 127) && wave == 0) {
        // trailing 64-k block: two 32-k groups
        f16x8 a[2];
        const f16* arow_t = (AM == 0 || AM == 3 || AM == 5 || AM == 6) ? A + (size_t)arow_m * K + 8 * kq : arow;
#pragma unroll
        for (int j = 0; j < 2; ++j)
            a[j] = *reinterpret_cast<const f16x8*>(arow_t + nfull * 128 + 32 * j);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const u32x2 w2 = *reinterpret_cast<const u32x2*>(tbase[t] + nfull * 256 + lane * 2);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const size_t grp = (size_t)nfull * 4 + j;
                uint32_t zlo, zhi;
                zero_bits((Z[grp * zwords + zw[t]] >> zsh[t]) & 0xFu, zlo, zhi);
                const f32x4 part = mfma_f16(a[j], dequant_word_fast(w2[j], zlo, zhi, mlo, mhi),
                                            f32x4{0.f, 0.f, 0.f, 0.f});
                const float s = (float)bitcast<f16>(S[grp * N + spos[t]]);
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[t][e] = __builtin_fmaf(s, part[e], acc[t][e]);
            }
        }
    }

    // cross-wave reduction in fixed wave order; only rows < M are written
    if (RALIAS) __syncthreads();  // the activation slots are dead
#pragma unroll
    for (int t = 0; t < T; ++t)
        *reinterpret_cast<f32x4*>(red + (wave * T + t) * 256 + lane * 4) = acc[t];
    __syncthreads();
    if (SWI) {
        for (int idx = threadIdx.x; idx < 256; idx += blockDim.x) {
            const int l = idx >> 2, e = idx & 3;
            const int m = 4 * (l >> 4) + e;
            if (m >= M) continue;
            float g = 0.f, u = 0.f;
            for (int w = 0; w < nwaves; ++w) {
                g += red[(w * T) * 256 + idx];
                u += red[(w * T + 1) * 256 + idx];
            }
            const float gf = (float)(f16)g, uf = (float)(f16)u;
            C[(size_t)m * (N >> 1) + strip * 16 + (l & 15)] = (f16)(gf / (1.0f + expf(-gf)) * uf);
        }
        return;
    }
    if (nsplit == 1) {
        for (int idx = threadIdx.x; idx < T * 256; idx += blockDim.x) {
            const int l = (idx & 255) >> 2, e = idx & 3, t = idx >> 8;
            const int m = 4 * (l >> 4) + e;
            if (m >= M) continue;
            float v = 0.f;
            for (int w = 0; w < nwaves; ++w) v += red[(w * T + t) * 256 + (idx & 255)];
            C[(size_t)m * N + (strip * T + t) * 16 + (l & 15)] = (f16)v;
        }
        return;
    }
    for (int idx = threadIdx.x; idx < T * 256; idx += blockDim.x) {
        const int l = (idx & 255) >> 2, e = idx & 3, t = idx >> 8;
        const int m = 4 * (l >> 4) + e;
        if (m >= M) continue;
        float v = 0.f;
        for (int w = 0; w < nwaves; ++w) v += red[(w * T + t) * 256 + (idx & 255)];
        __hip_atomic_store(sp.ws + ((size_t)blockIdx.y * M + m) * N + (strip * T + t) * 16 + (l & 15), v,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // this wave's partial stores are complete (agent-coherent stores: no
    // cache write-back needed; an agent-scope release fence would write back
    // the XCD's whole L2 from every wave, measured 2-50x slower)
    wait_vmcnt<0>();
    __syncthreads();
    int* last = reinterpret_cast<int*>(red);
    if (threadIdx.x == 0)
        last[0] = __hip_atomic_fetch_add(sp.cnt + strip, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                  nsplit - 1;
    __syncthreads();
    if (!last[0]) return;
    for (int idx = threadIdx.x; idx < T * 256; idx += blockDim.x) {
        const int l = (idx & 255) >> 2, e = idx & 3, t = idx >> 8;
        const int m = 4 * (l >> 4) + e;
        if (m >= M) continue;
        const size_t n = (size_t)(strip * T + t) * 16 + (l & 15);
        C[(size_t)m * N + n] = (f16)split_sum(sp.ws + (size_t)m * N + n, (size_t)M * N, nsplit);
    }
    if (threadIdx.x == 0) __hip_atomic_store(sp.cnt + strip, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int T, int NB, bool G32, int AM, bool SWI = false>
__global__ __launch_bounds__(1024) void int4_gemv_nb(
    const f16* __restrict__ A, const uint32_t* __restrict__ Wq, const uint16_t* __restrict__ S,
    const uint32_t* __restrict__ Z, f16* __restrict__ C, int M, int N, int K,
    SplitArgs sp = SplitArgs{}) {
    int4_gemv_body<T, NB, G32, AM, SWI>(A, Wq, S, Z, C, M, N, K, NormArgs{}, sp);
}

// One decode row (M = 1) with add_rmsnorm in the prologue (AM 4): the GEMV of
// h = add_rmsnorm(x, d, w) without h ever leaving the chip.
template <int T, int NB, bool G32, bool SWI>
__global__ __launch_bounds__(1024) void int4_gemv_norm(NormArgs nrm, const uint32_t* __restrict__ Wq,
                                                       const uint16_t* __restrict__ S,
                                                       const uint32_t* __restrict__ Z,
                                                       f16* __restrict__ C, int N, int K) {
    int4_gemv_body<T, NB, G32, 4, SWI>(nullptr, Wq, S, Z, C, 1, N, K, nrm);
}

// Column-split GEMV for wide outputs (N / 16 >= kCsMinTiles), 5..16 rows,
// group 128: each wave owns one 16-column n-tile and streams all K / 128
// blocks of it itself, so there is no cross-wave reduction, no split and
// no barrier after the start, and one generation of workgroups covers the
// matrix (gate_up 24576 x 4096: 1536 tiles, 192 workgroups of 8 waves;
// 6 waves on all 256 CUs, two-block chunks, or more chunks in flight each
// measured slower).
// The MR activation rows (rows past M repeat row M - 1) are copied whole
// into LDS first, as activation mode 6 does per block: [block][row][256 B],
// the 16-byte k chunks of row r XOR-swizzled by r.  Weights, scales and zero
// words are compiler-visible buffer loads (scalar block offsets, lane
// offsets fixed per wave), kCsCH blocks per chunk, kCsD chunks in flight; the
// chunk loop's first pass only issues, so each buffer is written in one
// place and the compiler's waits leave the later chunks in flight.
constexpr int kCsWaves = 8;       // waves (n-tiles) per workgroup
constexpr int kCsCH = 1;          // 128-k blocks per chunk
constexpr int kCsD = 4;           // chunks in flight
constexpr int kCsMinTiles = 1024;  // narrower outputs keep the split-k GEMV

struct CsBlk {
    u32x4 w;
    uint32_t z;
    uint16_t s;
};

template <int MR>
__global__ __launch_bounds__(64 * kCsWaves) void int4_gemv_cs(const f16* __restrict__ A,
                                                              const uint32_t* __restrict__ Wq,
                                                              const uint16_t* __restrict__ S,
                                                              const uint32_t* __restrict__ Z,
                                                              f16* __restrict__ C, int M, int N, int K) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kq = lane >> 4;
    const int nkb = K >> 7, ntiles = N >> 4, zwords = N >> 3;
    const int tb = xcd_block() * kCsWaves + wave;  // this wave's n-tile
    const bool tlive = tb < ntiles;
    const int nt = tlive ? tb : ntiles - 1;
    // activation rows into LDS: one copy = 4 rows x 256 B of one block
    {
        const i32x4_t rA = raw_rsrc(A, (uint32_t)M * (uint32_t)K * 2u);
        const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
        const int ncp = nkb * (MR / 4);
        for (int c = wave; c < ncp; c += kCsWaves) {
            const int kb = c / (MR / 4), p = c - kb * (MR / 4);
            const int r = 4 * p + (lane >> 4);
            const int m = r < M ? r : M - 1;
            lds_copy(rA, lds0 + (uint32_t)(kb * MR + 4 * p) * 256u,
                     2u * ((uint32_t)m * (uint32_t)K + (uint32_t)kb * 128u + 8u * (uint32_t)((lane & 15) ^ r)));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    const int n = nt * 16 + col;
    const uint32_t voS = 2u * (uint32_t)marlin_scale_pos(n);
    const int cl = n & 63;
    const uint32_t voZ = 4u * (uint32_t)(((n >> 6) << 3) + (cl & 7));
    const int zsh = 4 * slot_of(cl >> 3);
    const __amdgpu_buffer_rsrc_t rW = buf_rsrc(Wq, (uint32_t)((size_t)N * K / 2));
    const __amdgpu_buffer_rsrc_t rS = buf_rsrc(S, (uint32_t)nkb * (uint32_t)N * 2u);
    const __amdgpu_buffer_rsrc_t rZ = buf_rsrc(Z, (uint32_t)nkb * (uint32_t)zwords * 4u);
    const uint32_t wt = (uint32_t)nt * 8u * (uint32_t)K;  // the tile's bytes
    const int nch = (nkb + kCsCH - 1) / kCsCH;
    // block i of chunk c: min(c kCsCH + i, nkb - 1); a block past the end
    // repeats the last one and counts zero
    auto issue = [&](CsBlk (&b)[kCsCH], int c) {
        c = c < nch ? c : nch - 1;
#pragma unroll
        for (int i = 0; i < kCsCH; ++i) {
            const int kb = c * kCsCH + i < nkb ? c * kCsCH + i : nkb - 1;
            b[i].w = bitcast<u32x4>(__builtin_amdgcn_raw_buffer_load_b128(rW, (int)(16u * lane),
                                                                          (int)(wt + 1024u * kb), 2));
            b[i].s = __builtin_amdgcn_raw_buffer_load_b16(rS, (int)voS, (int)(2u * (uint32_t)N * kb), 0);
            b[i].z = __builtin_amdgcn_raw_buffer_load_b32(rZ, (int)voZ, (int)(4u * (uint32_t)zwords * kb), 0);
        }
    };
    const uint32_t mlo = 0x64006400u, mhi = 0x54005400u;
    const int arow = col < M ? col : M - 1;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    CsBlk buf[kCsD][kCsCH];
    const int passes = (nch + kCsD - 1) / kCsD + 1;
    for (int it = 0; it < passes; ++it) {
#pragma unroll
        for (int d = 0; d < kCsD; ++d) {
            const int c = (it - 1) * kCsD + d;  // the chunk computed here
            if (it == 1 && d == 0) {
                // the copies went out before every weight load: once the
                // first weight word has landed (the asm names it, so the
                // compiler waits for it) they have too; the barrier publishes
                // every wave's rows
                asm volatile("" : : "v"(buf[0][0].w) : "memory");
                lds_barrier();
            }
            if (it > 0 && c < nch) {
#pragma unroll
                for (int i = 0; i < kCsCH; ++i) {
                    const int kr = c * kCsCH + i;
                    const int kb = kr < nkb ? kr : nkb - 1;
                    const unsigned char* ab = smem + ((size_t)kb * MR + arow) * 256;
                    f16x8 a[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) a[j] = *reinterpret_cast<const f16x8*>(ab + 16 * ((4 * j + kq) ^ arow));
                    uint32_t zlo, zhi;
                    zero_bits((buf[d][i].z >> zsh) & 0xFu, zlo, zhi);
                    f32x4 part = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        part = mfma_f16(a[j], dequant_word_fast(buf[d][i].w[j], zlo, zhi, mlo, mhi), part);
                    const float sc = kr < nkb ? (float)bitcast<f16>(buf[d][i].s) : 0.0f;
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(sc, part[e], acc[e]);
                    // keeps the scaled add here: the compiler would otherwise
                    // sink every block's add to the end and keep each block's
                    // partial MFMA result live until then
                    asm volatile("" : "+v"(acc));
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            issue(buf[d], it * kCsD + d);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (tlive) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int m = 4 * kq + e;
            if (m < M) C[(size_t)m * N + nt * 16 + col] = (f16)acc[e];
        }
    }
}

// Prefill-shaped GEMM (M > 64, K % 128 == 0) on the matrix cores.
//
// Workgroup tile 64 (m) x 256 (n): eight waves side by side along n, each
// with a 64 x 32 wave tile (4 m-tiles x 2 n-tiles of 16 x 16 fp32
// accumulators), two waves per SIMD so one wave's dequantization overlaps
// the other's MFMAs.  The tile shape follows from traffic: a 128-k block
// brings 256 B per activation row (fp16) but 64 B per weight column (int4),
// so 64 x 256 moves 2 B of L2 traffic per output element and block where
// 128 x 128 moves 2.5, and the workgroup reuses its A rows 256 times.
// Every main-loop global load goes straight to LDS (buffer_load ... lds), so
// nothing in the loop waits on a VGPR load: kGemmAhead blocks are in flight
// into a ring of kGemmAhead + 1 LDS stages, and one vmcnt wait plus one
// barrier per block hand a finished stage to all waves.  A stage holds, for
// one 128-k block:
//   * A  (16 KB): the 64 x 128 fp16 activation tile, row-major (256 B per
//     row) with the 16-byte k chunks of row r XOR-swizzled by r % 16: each
//     copy moves 4 whole rows (8 full cache lines, where a fragment-major
//     order touches 16 half-used lines per copy: M512 N8192 K2048 21.3-21.9
//     -> 21.1-21.2 us), and the 16 lanes of an MFMA operand read hit 16
//     different bank groups;
//   * B  (16 KB): the 16 n-tiles' 1 KB tile-layout blocks as they lie;
//   * S  (2 KB): per group row of the block, the strip's 256 fp16 scales
//     (Marlin positions 256 nb .. 256 nb + 255; the permutation stays inside
//     64-column chunks);
//   * Z  (1 KB): per group row, the strip's 32 packed zero words.
// B is dequantized in registers: (q - z) exactly in fp16, times the fp16
// group scale (the B operand is s * (q - z) rounded to fp16, as a Marlin
// kernel feeds its tensor cores); 32 v_mfma_f32_16x16x32_f16 per wave and
// block accumulate in fp32.
// Rows >= M read row M-1 and are not stored; n-tiles >= N read the last
// n-tile and are not stored; blocks past the end re-read the last block
// with a zero scale (uniform load counts and trip structure).
// Workgroup-to-tile order: the hardware deals workgroup b to XCD b % 8, so
// when the tile count is a multiple of 8 the tiles of one XCD are a
// contiguous run in (n-block major, m-block minor) order, and the m-blocks
// that share a weight strip share one L2.
constexpr int kGemmBM = 64, kGemmBN = 256;
constexpr int kGemmMfmaMinM = 64;   // M above this takes the MFMA GEMM
// one block ahead in two 35 KB stages: two workgroups per CU (M512 N8192
// K2048 21.5 us) against 23.8 us for two blocks ahead in three stages (one
// workgroup per CU; copies from inline asm, so the ring really holds two
// blocks: see lds_copy) -- the second workgroup's dequantization work hides
// more than the deeper ring
constexpr int kGemmAhead = 1;       // blocks in flight ahead of the one computed
constexpr int kGemmStages = kGemmAhead + 1;
constexpr int kStA = 0, kStB = 16384, kStS = kStB + 16384, kStZ = kStS + 2048;
constexpr int kStageBytes = kStZ + 1024;
constexpr size_t kGemmLds = (size_t)kGemmStages * kStageBytes;

FL_DEV f16x8 dequant_word_scaled(uint32_t w, uint32_t zlo, uint32_t zhi, f16x2 s2) {
    const uint32_t w8 = w >> 8;
    const f16x2 p0 = (bitcast<f16x2>(and_or(w, 0x000F000Fu, 0x64006400u)) + bitcast<f16x2>(zlo)) * s2;
    const f16x2 p1 = (bitcast<f16x2>(and_or(w, 0x00F000F0u, 0x54005400u)) + bitcast<f16x2>(zhi)) * s2;
    const f16x2 p2 = (bitcast<f16x2>(and_or(w8, 0x000F000Fu, 0x64006400u)) + bitcast<f16x2>(zlo)) * s2;
    const f16x2 p3 = (bitcast<f16x2>(and_or(w8, 0x00F000F0u, 0x54005400u)) + bitcast<f16x2>(zhi)) * s2;
    const u32x4 r{bitcast<uint32_t>(p0), bitcast<uint32_t>(p1), bitcast<uint32_t>(p2),
                  bitcast<uint32_t>(p3)};
    return bitcast<f16x8>(r);
}

template <bool G32>
__global__ __launch_bounds__(512) void int4_gemm_mfma(
    const f16* __restrict__ A, const uint32_t* __restrict__ Wq, const uint16_t* __restrict__ S,
    const uint32_t* __restrict__ Z, f16* __restrict__ C, int M, int N, int K) {
    constexpr int D = kGemmAhead, NS = kGemmStages;
    constexpr int SPB = G32 ? 4 : 1;  // group rows per block
    // DMA loads per block and wave: 2 A fragments, 2 B tiles, 2 scale/zero
    // pieces (3 * SPB pieces are needed; waves past them repeat one)
    constexpr int LPB = 2 + 2 + 2;
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kq = lane >> 4;
    const int nkb = K >> 7;
    const int zwords = N >> 3;
    const int ntiles = N >> 4;
    const int G = K / (G32 ? 32 : 128);

    const int nblk = (N + kGemmBN - 1) / kGemmBN, mblk = (M + kGemmBM - 1) / kGemmBM;
    const int total = nblk * mblk;
    int lin = blockIdx.x;
    if ((total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);
    const int nb_i = lin / mblk, mb_i = lin - nb_i * mblk;
    const int m0 = mb_i * kGemmBM;
    const int nt_base = nb_i * 16;

    const i32x4_t rA = raw_rsrc(A, (uint32_t)M * K * 2);
    const i32x4_t rW = raw_rsrc(Wq, (uint32_t)N * K / 2);
    const i32x4_t rS = raw_rsrc(S, (uint32_t)G * N * 2);
    const i32x4_t rZ = raw_rsrc(Z, (uint32_t)G * zwords * 4);
    const uint32_t lds0 = (uint32_t)(uintptr_t)smem;

    // DMA sources of this wave: A rows 4 q .. 4 q + 3, q = 2 wave + i (whole
    // 256-byte rows of the block, so every copy reads 8 full cache lines),
    // and B n-tiles 2 wave + i of the strip.  Lane l of copy q lands at LDS
    // row r = 4 q + l / 16, position p = l % 16 and brings the row's 16-byte
    // k chunk p ^ (r % 16): the XOR swizzle that keeps the MFMA reads below
    // conflict-free.
    uint32_t ao[2], bo[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = 4 * (wave * 2 + i) + (lane >> 4);
        int m = m0 + r;
        m = m < M ? m : M - 1;
        ao[i] = 2u * ((uint32_t)m * K) + 16u * ((lane & 15) ^ (r & 15));
        int nt = nt_base + wave * 2 + i;
        nt = nt < ntiles ? nt : ntiles - 1;
        bo[i] = (uint32_t)nt * (8u * K) + lane * 16;
    }
    // scale/zero pieces: piece p < 3 SPB is (row g = p / 3, part p % 3):
    // parts 0, 1 = scale positions [128 part, +128) of the strip (64 lanes x
    // 4 B), part 2 = the strip's 32 zero words (lanes 32..63 repeat them).
    // Wave w moves pieces 2 w and 2 w + 1 (modulo 3 SPB).
    uint32_t pvo[2], prow_bytes[2], pgrp[2];
    int pdst[2];
    bool pis_s[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int p = (wave * 2 + i) % (3 * SPB);
        const int g = p / 3, part = p % 3;
        pgrp[i] = g;
        pis_s[i] = part < 2;
        if (part < 2) {
            int q = nb_i * 256 + part * 128 + 2 * lane;
            q = q < N ? q : N - 2;
            pvo[i] = 2u * q;
            prow_bytes[i] = 2u * N;
            pdst[i] = kStS + g * 512 + part * 256;
        } else {
            int w = nb_i * 32 + (lane & 31);
            w = w < zwords ? w : zwords - 1;
            pvo[i] = 4u * w;
            prow_bytes[i] = 4u * zwords;
            pdst[i] = kStZ + g * 256;
        }
    }

    auto issue = [&](int kb, int slot) {
        kb = kb < nkb ? kb : nkb - 1;
        const uint32_t st = lds0 + (uint32_t)slot * kStageBytes;
#pragma unroll
        for (int i = 0; i < 2; ++i) lds_copy(rA, st + kStA + (wave * 2 + i) * 1024, ao[i], kb * 256);
#pragma unroll
        for (int i = 0; i < 2; ++i) lds_copy(rW, st + kStB + (wave * 2 + i) * 1024, bo[i], kb * 1024);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t grp = (uint32_t)kb * SPB + pgrp[i];
            lds_copy<4>(pis_s[i] ? rS : rZ, st + pdst[i], pvo[i], grp * prow_bytes[i]);
        }
    };

    // this wave's 2 n-tiles: scale/zero positions inside the stage's rows
    int sp[2], zp[2], zsh[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int n = (nt_base + wave * 2 + t) * 16 + col;
        sp[t] = marlin_scale_pos(n) - nb_i * 256;
        const int cl = n & 63;
        zp[t] = ((n >> 6) << 3) + (cl & 7) - nb_i * 32;
        zsh[t] = 4 * slot_of(cl >> 3);
    }

    f32x4 acc[4][2];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int d = 0; d < D; ++d) issue(d, d);

    // A operand of m-tile mt, step j for lane (col, kq): row 16 mt + col, k
    // chunk 4 j + kq, stored at position (4 j + kq) ^ col of that row
    const int afrag = kStA + col * 256 + 16 * (kq ^ (col & 3));
    const int ajx = col >> 2;
    for (int kb0 = 0; kb0 < nkb; kb0 += NS) {
#pragma unroll
        for (int u = 0; u < NS; ++u) {
            const int kb = kb0 + u;
            const f16 live = kb < nkb ? (f16)1.0f : (f16)0.0f;
            wait_vmcnt<(D - 1) * LPB>();
            asm volatile("s_barrier" ::: "memory");
            issue(kb + D, (u + D) % NS);
            const unsigned char* st = smem + (size_t)u * kStageBytes;
            u32x4 wv[2];
            uint32_t zl[2][SPB], zh[2][SPB];
            f16 sc[2][SPB];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                wv[t] = *reinterpret_cast<const u32x4*>(st + kStB + (wave * 2 + t) * 1024 + lane * 16);
#pragma unroll
                for (int g = 0; g < SPB; ++g) {
                    const uint16_t sb = *reinterpret_cast<const uint16_t*>(st + kStS + g * 512 + 2 * sp[t]);
                    const uint32_t zw = *reinterpret_cast<const uint32_t*>(st + kStZ + g * 256 + 4 * zp[t]);
                    sc[t][g] = bitcast<f16>(sb) * live;
                    zero_bits((zw >> zsh[t]) & 0xFu, zl[t][g], zh[t][g]);
                }
            }
            const unsigned char* as = st + afrag;
            f16x8 a[2][4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) a[0][mt] = *reinterpret_cast<const f16x8*>(as + mt * 4096 + 64 * ajx);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (j < 3) {
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt)
                        a[(j + 1) & 1][mt] =
                            *reinterpret_cast<const f16x8*>(as + mt * 4096 + 64 * ((j + 1) ^ ajx));
                }
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int g = G32 ? j : 0;
                    const f16x8 b = dequant_word_scaled(wv[t][j], zl[t][g], zh[t][g],
                                                        f16x2{sc[t][g], sc[t][g]});
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) acc[mt][t] = mfma_f16(a[j & 1][mt], b, acc[mt][t]);
                }
            }
        }
    }
    wait_vmcnt<0>();  // no LDS copy may still be in flight when the workgroup ends

#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int nt = nt_base + wave * 2 + t;
        if (nt >= ntiles) continue;
        const int n = nt * 16 + col;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = m0 + mt * 16 + 4 * kq + e;
                if (m < M) C[(size_t)m * N + n] = (f16)acc[mt][t][e];
            }
    }
}

hipError_t launch_gemm_mfma(const f16* A, const uint32_t* Wq, const uint16_t* S, const uint32_t* Z,
                            f16* C, int M, int N, int K, bool g32, hipStream_t stream) {
    const int tiles = ((N + kGemmBN - 1) / kGemmBN) * ((M + kGemmBM - 1) / kGemmBM);
    if (g32)
        hipLaunchKernelGGL((int4_gemm_mfma<true>), dim3(tiles), dim3(512), kGemmLds, stream, A, Wq,
                           S, Z, C, M, N, K);
    else
        hipLaunchKernelGGL((int4_gemm_mfma<false>), dim3(tiles), dim3(512), kGemmLds, stream, A, Wq,
                           S, Z, C, M, N, K);
    return hipGetLastError();
}

struct GemvCfg {
    int tiles;      // n-tiles (16 columns) per workgroup: 1, 2 or 4
    int waves;      // waves per workgroup, 1..16
    int nb;         // max full 128-k blocks per wave (register budget): 1,2,4,6,8
    int split = 1;  // k-splits (gridDim.y), each over (K/128)/split blocks
};

// Workspace of a split-K launch: the strip counters in a fixed region at
// offset 0 (one int per strip, kSplitStrips of them whatever N, M, the tiles
// and the split), then the fp32 partials [split][M][N].  The counter of strip
// s is then at the same place for every call, and no call's partials reach
// another's counters, so calls of any shape may share one workspace as long
// as they do not overlap; every call leaves its counters at zero.
constexpr int kSplitStrips = 16384;  // N <= 16 * kSplitStrips with a split
constexpr size_t splitk_part_off(int) { return (size_t)kSplitStrips * 4; }
constexpr size_t splitk_ws_bytes(int M, int N, int split) {
    return splitk_part_off(N) + (size_t)split * M * N * 4;
}

constexpr size_t kGemvLdsCap = 96 * 1024;  // activations staged in LDS up to this size

// A split-K launch (split > 1) uses per-wave activations (AM 0 / AM 5 copies
// up to M = 8, AM 3 / AM 2 above): the whole-row LDS staging of AM 1 would
// read past the shifted activation base.
template <int T, int NB, bool G32>
hipError_t launch_gemv_nb(const f16* A, const uint32_t* Wq, const uint16_t* S, const uint32_t* Z,
                          f16* C, int M, int N, int K, int waves, int split, SplitArgs sp,
                          hipStream_t stream) {
    const size_t red = (size_t)waves * T * 256 * sizeof(float);
    const dim3 grid(N / (16 * T), split), block(64 * waves);
    const size_t own = (size_t)waves * NB * 1024;
    const size_t shared = (((size_t)M * (K + 8) * 2 + 15) & ~(size_t)15);
    if (M <= 4 && own + red <= 160 * 1024)
        hipLaunchKernelGGL((int4_gemv_nb<T, NB, G32, 0>), grid, block, own + red, stream, A, Wq, S, Z,
                           C, M, N, K, sp);
    else if (M <= 8 && 2 * own + red <= 160 * 1024)
        hipLaunchKernelGGL((int4_gemv_nb<T, NB, G32, 5>), grid, block, 2 * own + red, stream, A, Wq, S, Z,
                           C, M, N, K, sp);
    else if (M > 8 && 4 * own + red <= 160 * 1024)
        hipLaunchKernelGGL((int4_gemv_nb<T, NB, G32, 6>), grid, block, 4 * own + red, stream, A, Wq, S, Z,
                           C, M, N, K, sp);
    else if (NB <= 4)
        hipLaunchKernelGGL((int4_gemv_nb<T, NB, G32, 3>), grid, block, red, stream, A, Wq, S, Z, C, M,
                           N, K, sp);
    else if (shared <= kGemvLdsCap && split == 1)
        hipLaunchKernelGGL((int4_gemv_nb<T, NB, G32, 1>), grid, block, shared + red, stream, A, Wq, S,
                           Z, C, M, N, K, sp);
    else
        hipLaunchKernelGGL((int4_gemv_nb<T, NB, G32, 2>), grid, block, red, stream, A, Wq, S, Z, C, M,
                           N, K, sp);
    return hipGetLastError();
}

template <int T, bool G32>
hipError_t dispatch_nb(int nb, const f16* A, const uint32_t* Wq, const uint16_t* S,
                       const uint32_t* Z, f16* C, int M, int N, int K, int waves, int split,
                       SplitArgs sp, hipStream_t stream) {
    switch (nb) {
        case 1: return launch_gemv_nb<T, 1, G32>(A, Wq, S, Z, C, M, N, K, waves, split, sp, stream);
        case 2: return launch_gemv_nb<T, 2, G32>(A, Wq, S, Z, C, M, N, K, waves, split, sp, stream);
        case 3: return launch_gemv_nb<T, 3, G32>(A, Wq, S, Z, C, M, N, K, waves, split, sp, stream);
        case 4: return launch_gemv_nb<T, 4, G32>(A, Wq, S, Z, C, M, N, K, waves, split, sp, stream);
        case 5: return launch_gemv_nb<T, 5, G32>(A, Wq, S, Z, C, M, N, K, waves, split, sp, stream);
        case 6: return launch_gemv_nb<T, 6, G32>(A, Wq, S, Z, C, M, N, K, waves, split, sp, stream);
        default: return launch_gemv_nb<T, 8, G32>(A, Wq, S, Z, C, M, N, K, waves, split, sp, stream);
    }
}

// Four n-tiles per workgroup: half the workgroups of two tiles, so half the
// activation reads per output (each workgroup reads all of A: M x K x 2
// bytes, 128 KB at M = 16, K = 4096).  Register activations (AM 3) only.
template <int NB, bool G32>
hipError_t launch_gemv_t4(const f16* A, const uint32_t* Wq, const uint16_t* S, const uint32_t* Z,
                          f16* C, int M, int N, int K, int waves, int split, SplitArgs sp,
                          hipStream_t stream) {
    const size_t red = (size_t)waves * 4 * 256 * sizeof(float);
    const size_t own = (size_t)waves * NB * 1024;
    const dim3 grid(N / 64, split), block(64 * waves);
    // above M = 8: AM 6 with the reduction in the activation slots from two
    // blocks per wave; one block per wave measured even with register
    // fragments (gate_up M = 16, split 2: 16.4 against 16.3 us)
    if (M <= 8 && 2 * own + red <= 160 * 1024)
        hipLaunchKernelGGL((int4_gemv_nb<4, NB, G32, 5>), grid, block, 2 * own + red, stream, A, Wq, S, Z,
                           C, M, N, K, sp);
    else if (M > 8 && NB >= 2 && (4 * own > red ? 4 * own : red) <= 160 * 1024)
        hipLaunchKernelGGL((int4_gemv_nb<4, NB, G32, 6>), grid, block, 4 * own > red ? 4 * own : red, stream,
                           A, Wq, S, Z, C, M, N, K, sp);
    else
        hipLaunchKernelGGL((int4_gemv_nb<4, NB, G32, 3>), grid, block, red, stream, A, Wq, S, Z, C, M, N,
                           K, sp);
    return hipGetLastError();
}

template <bool G32>
hipError_t dispatch_gemv(const GemvCfg& c, const f16* A, const uint32_t* Wq, const uint16_t* S,
                         const uint32_t* Z, f16* C, int M, int N, int K, hipStream_t stream,
                         SplitArgs sp = SplitArgs{}) {
    if (c.tiles == 4) {
        switch (c.nb) {
            case 1: return launch_gemv_t4<1, G32>(A, Wq, S, Z, C, M, N, K, c.waves, c.split, sp, stream);
            case 2: return launch_gemv_t4<2, G32>(A, Wq, S, Z, C, M, N, K, c.waves, c.split, sp, stream);
            default: return launch_gemv_t4<4, G32>(A, Wq, S, Z, C, M, N, K, c.waves, c.split, sp, stream);
        }
    }
    if (c.tiles == 2)
        return dispatch_nb<2, G32>(c.nb, A, Wq, S, Z, C, M, N, K, c.waves, c.split, sp, stream);
    return dispatch_nb<1, G32>(c.nb, A, Wq, S, Z, C, M, N, K, c.waves, c.split, sp, stream);
}

// register-slot counts with a kernel instance (slots beyond a wave's share
// are wasted work, so the launcher picks the exact count when it can)
int nb_bucket(int need) {
    if (need <= 6) return need < 1 ? 1 : need;
    return 8;
}

// Launch heuristic for M <= 16, from a sweep on MI355X at the Qwen3-8B
// shapes (graph-timed, weights rotated through HBM): wide outputs
// (N >= 16384) take 2 n-tiles per strip and 8 waves while M <= 4; otherwise 16
// waves, 2 n-tiles once N >= 6144 and M >= 4 (activation fragments then feed
// two tiles).  The register-slot count is the exact per-wave block share.
GemvCfg default_gemv_cfg(int M, int N, int K, bool g32, bool can_split = false) {
    GemvCfg c;
    if (can_split && M > 4 && !g32 && K % 128 == 0 && N % 64 == 0) {
        // Splitting K over workgroups costs the last split of each strip a
        // chain of device-coherent round trips (partials out, counter, partials
        // back): ~2-3 us, so it pays only where the unsplit kernel re-reads
        // the activations heavily.  Long K (the down projection): two splits
        // of two tiles (M = 8: 11.8 -> 10.5 us, M = 16: 15.7 -> 12.6 at
        // 4096 x 12288); wide N above M = 8: four tiles, two splits of one
        // block per wave (18.6 -> 16.7 us at 24576 x 4096, M = 16).
        const int nall = K / 128;
        if (M > 8 && nall >= 64 && nall % 3 == 0 && nall / 3 <= 16 * 2) {
            // above eight rows: four tiles, three splits of two blocks per
            // wave, activations copied in whole rows (4096 x 12288, M = 16:
            // 12.35 -> 11.0 us)
            c.tiles = 4;
            c.waves = 16;
            c.nb = nb_bucket((nall / 3 + 15) / 16);
            c.split = 3;
            return c;
        }
        if (nall >= 64 && nall % 2 == 0 && nall / 2 <= 16 * 8) {
            c.tiles = 2;
            c.waves = 16;
            c.nb = nb_bucket((nall / 2 + 15) / 16);
            c.split = 2;
            return c;
        }
        if (N >= 16384 && M > 8 && nall % 2 == 0 && nall / 2 <= 16) {
            c.tiles = 4;
            c.waves = nall / 2;
            c.nb = 1;
            c.split = 2;
            return c;
        }
    }
    // four tiles above M = 8 on wide N: each workgroup reads all of A, and
    // the A bytes (M x K x 2 per workgroup) load the L1/TD path more than
    // the weights do there
    c.tiles = N >= 16384 ? (M > 8 ? 4 : 2) : (N >= 6144 ? 2 : 1);
    if (N % (16 * c.tiles)) c.tiles = 1;
    const int nfull = K / 128 > 0 ? K / 128 : 1;
    const int cap = g32 ? 4 : 8;
    // eight waves of four blocks beat sixteen of two where K <= 4096 (M <= 4:
    // qkv 5.85 -> 5.40 us, o 4.36 -> 4.26; one tile at any M: o 5.67 -> 5.52
    // at M = 8; above eight rows: qkv 6.51 -> 6.34 at M = 16)
    int waves = ((N >= 16384 && M <= 8) || (nfull <= 32 && (M <= 4 || M > 8 || c.tiles == 1))) ? 8 : 16;
    while (waves > 1 && nfull < waves) waves /= 2;  // at least one block per wave
    while ((nfull + waves - 1) / waves > cap && waves < 16) waves *= 2;
    c.waves = waves;
    c.nb = nb_bucket((nfull + waves - 1) / waves);
    if (c.nb > cap) c.nb = cap;
    if (c.tiles == 4 && c.nb > 4) c.tiles = 2;  // four tiles take register activations: nb <= 4
    return c;
}

bool gemv_cfg_ok(const GemvCfg& c, int M, int N, int K, bool g32) {
    if (c.tiles != 1 && c.tiles != 2 && c.tiles != 4) return false;
    if (c.tiles == 4 && c.nb > 4) return false;
    if (c.waves < 1 || c.waves > 16) return false;
    if (N % (16 * c.tiles)) return false;
    if (c.split < 1 || c.split > kMaxSplits) return false;
    if (c.split > 1 && (K % 128 || (K / 128) % c.split)) return false;  // whole blocks per split
    const int nfull = K / 128 / c.split;
    if (nfull < 1 && !(g32 && K == 64)) return false;
    const int need = (nfull + c.waves - 1) / c.waves;
    if (need > c.nb || c.nb > (g32 ? 4 : 8)) return false;
    if (c.nb == 7) return false;
    (void)M;
    return true;
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

bool int4_args_ok(const void* a, const uint32_t* q, const void* scales, const uint32_t* zeros,
                  void* c, int M, int N, int K, int group_size) {
    if (M <= 0 || N <= 0 || K <= 0) return false;
    if (group_size != 32 && group_size != 128) return false;
    if (K % group_size != 0 || N % 64 != 0 || K % 64 != 0) return false;
    if (!a || !q || !scales || !zeros || !c) return false;
    if (!fl_aligned(a, 16) || !fl_aligned(q, 16) || !fl_aligned(c, 2) || !fl_aligned(scales, 2) ||
        !fl_aligned(zeros, 4))
        return false;
    return fl_current_device_supported();
}

bool report(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        fprintf(stderr, "%s launch error: %s\n", what, hipGetErrorString(e));
        return false;
    }
    return true;
}

// M > 16: slabs of up to 64 rows through the multi-m-tile kernel.
bool int4_gemm_large_m(const f16* A, const uint32_t* q, const f16* S, const uint32_t* Z, f16* C,
                       int M, int N, int K, bool g32, hipStream_t stream) {
    const int nkb = (K + 127) / 128;
    for (int m0 = 0; m0 < M; m0 += 64) {
        const int Mc = (M - m0) < 64 ? (M - m0) : 64;
        const int MT = (Mc + 15) / 16;
        int nwaves = 16 / MT;
        if (nwaves > nkb) nwaves = nkb;
        if (nwaves < 1) nwaves = 1;
        const hipError_t e =
            g32 ? dispatch_mt<true>(MT, 1, A + (size_t)m0 * K, q, S, Z, C + (size_t)m0 * N, Mc, N,
                                    K, nwaves, stream)
                : dispatch_mt<false>(MT, 1, A + (size_t)m0 * K, q, S, Z, C + (size_t)m0 * N, Mc,
                                     N, K, nwaves, stream);
        if (!report(e, "FastllmCudaMarlinHalfInt4Gemm")) return false;
    }
    return true;
}

bool int4_marlin_abi_gemm(const void* a, const uint32_t* q, const void* scales,
                          const uint32_t* zeros, void* c, int M, int N, int K, int group_size,
                          hipStream_t stream, const GemvCfg* forced, void* ws = nullptr,
                          size_t ws_bytes = 0) {
    if (!int4_args_ok(a, q, scales, zeros, c, M, N, K, group_size)) return false;
    const bool g32 = group_size == 32;
    const f16* A = static_cast<const f16*>(a);
    f16* Cp = static_cast<f16*>(c);
    if (M > kGemmMfmaMinM && K % 128 == 0 && (size_t)N * K / 2 < (1ull << 31)) {
        // the kernel addresses A through a 32-bit buffer range: launch rows in
        // chunks (multiples of its 64-row tile) of fewer than 2^31 bytes
        const size_t rows_cap = ((1ull << 31) - 1) / ((size_t)K * 2);
        const int mchunk = rows_cap >= (size_t)M ? M : (int)(rows_cap / kGemmBM * kGemmBM);
        for (int m0 = 0; m0 < M; m0 += mchunk) {
            const int Mc = (M - m0) < mchunk ? (M - m0) : mchunk;
            if (!report(launch_gemm_mfma(A + (size_t)m0 * K, q, static_cast<const uint16_t*>(scales),
                                         zeros, Cp + (size_t)m0 * N, Mc, N, K, g32, stream),
                        "FastllmCudaMarlinHalfInt4Gemm"))
                return false;
        }
        return true;
    }
    if (M > 16)
        return int4_gemm_large_m(A, q, static_cast<const f16*>(scales), zeros, Cp, M, N, K, g32,
                                 stream);
    if (!forced && !g32 && M > 4 && K % 128 == 0 && N / 16 >= kCsMinTiles && (size_t)N * K / 2 < (1ull << 31)) {
        // wide output, 5..16 rows: the column-split GEMV, all rows in LDS
        const int mr = M > 8 ? 16 : 8;
        const size_t lds = (size_t)(K / 128) * mr * 256;
        if (lds <= 128 * 1024) {
            const dim3 grid((N / 16 + kCsWaves - 1) / kCsWaves), block(64 * kCsWaves);
            const uint16_t* S = static_cast<const uint16_t*>(scales);
            if (mr == 16)
                hipLaunchKernelGGL(int4_gemv_cs<16>, grid, block, lds, stream, A, q, S, zeros, Cp, M, N, K);
            else
                hipLaunchKernelGGL(int4_gemv_cs<8>, grid, block, lds, stream, A, q, S, zeros, Cp, M, N, K);
            return report(hipGetLastError(), "FastllmCudaMarlinHalfInt4Gemm");
        }
    }
    GemvCfg cfg = forced ? *forced : default_gemv_cfg(M, N, K, g32, ws != nullptr);
    if (cfg.split > 1 && (!ws || !fl_aligned(ws, 256) || N / 16 > kSplitStrips ||
                          ws_bytes < splitk_ws_bytes(M, N, cfg.split))) {
        if (forced) return false;
        cfg = default_gemv_cfg(M, N, K, g32, false);
    }
    if (!gemv_cfg_ok(cfg, M, N, K, g32)) {
        if (forced) return false;
        return int4_gemm_large_m(A, q, static_cast<const f16*>(scales), zeros, Cp, M, N, K, g32,
                                 stream);
    }
    SplitArgs sp;
    if (cfg.split > 1) {
        sp.cnt = static_cast<int*>(ws);
        sp.ws = reinterpret_cast<float*>(static_cast<char*>(ws) + splitk_part_off(N));
    }
    const uint16_t* S = static_cast<const uint16_t*>(scales);
    const hipError_t e = g32 ? dispatch_gemv<true>(cfg, A, q, S, zeros, Cp, M, N, K, stream, sp)
                             : dispatch_gemv<false>(cfg, A, q, S, zeros, Cp, M, N, K, stream, sp);
    return report(e, "FastllmCudaMarlinHalfInt4Gemm");
}

// gate/up GEMV + SwiGLU (M <= 16, N = 2 I, I % 64 == 0): two n-tiles per
// workgroup (gate s, up s), per-wave activation copies up to M = 4, register
// activations above.
template <int NB, bool G32>
hipError_t launch_gemv_swiglu(const f16* A, const uint32_t* Wq, const uint16_t* S, const uint32_t* Z,
                              f16* H, int M, int N, int K, int waves, hipStream_t stream) {
    const size_t red = (size_t)waves * 2 * 256 * sizeof(float);
    const size_t own = (size_t)waves * NB * 1024;
    const dim3 grid(N / 32), block(64 * waves);
    if (own + red > kMaxLds) return hipErrorInvalidValue;
    // LDS activation copies (AM 0; AM 5 above four rows, AM 6 above eight,
    // while their 2 or 4 KB per block fit), register activations otherwise
    // (NB <= 4: more blocks per wave spill there)
    if (M <= 4) {
        hipLaunchKernelGGL((int4_gemv_nb<2, NB, G32, 0, true>), grid, block, own + red, stream, A, Wq, S,
                           Z, H, M, N, K);
    } else if constexpr (NB <= 4) {
        if (M <= 8 && 2 * own + red <= kMaxLds)
            hipLaunchKernelGGL((int4_gemv_nb<2, NB, G32, 5, true>), grid, block, 2 * own + red, stream, A,
                               Wq, S, Z, H, M, N, K);
        else if (M > 8 && 4 * own + red <= kMaxLds)
            hipLaunchKernelGGL((int4_gemv_nb<2, NB, G32, 6, true>), grid, block, 4 * own + red, stream, A, Wq,
                               S, Z, H, M, N, K);
        else
            hipLaunchKernelGGL((int4_gemv_nb<2, NB, G32, 3, true>), grid, block, red, stream, A, Wq, S, Z,
                               H, M, N, K);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <bool G32>
hipError_t dispatch_swiglu(const f16* A, const uint32_t* Wq, const uint16_t* S, const uint32_t* Z,
                           f16* H, int M, int N, int K, hipStream_t stream) {
    // the decode config of this shape.  Up to M = 8 (LDS activation copies)
    // eight waves on wide N, and six blocks per wave fit the registers at 16
    // waves, so K <= 12288 (16 x 6 x 128).  Above M = 8 (register
    // activations) sixteen waves of at most four blocks (K <= 8192): the NB =
    // 4 register-A instantiation at eight waves needs more than 128 VGPRs
    // and spills.  Larger K is refused (rc 1): the caller runs the plain GEMV
    // and the standalone SwiGLU.
    const int nfull = K / 128 > 0 ? K / 128 : 1;
    const int cap = (M <= 8 && !G32) ? 6 : 4;
    int waves = (N >= 16384 && M <= 8) ? 8 : 16;
    while (waves > 1 && nfull < waves) waves /= 2;
    while ((nfull + waves - 1) / waves > 4 && waves < 16) waves *= 2;
    int nb = (nfull + waves - 1) / waves;
    if (nb > 4 && nb <= cap) nb = 6;
    switch (nb) {
        case 1: return launch_gemv_swiglu<1, G32>(A, Wq, S, Z, H, M, N, K, waves, stream);
        case 2: return launch_gemv_swiglu<2, G32>(A, Wq, S, Z, H, M, N, K, waves, stream);
        case 3: return launch_gemv_swiglu<3, G32>(A, Wq, S, Z, H, M, N, K, waves, stream);
        case 4: return launch_gemv_swiglu<4, G32>(A, Wq, S, Z, H, M, N, K, waves, stream);
        case 6:
            if constexpr (!G32)
                if (M <= 4) return launch_gemv_swiglu<6, G32>(A, Wq, S, Z, H, M, N, K, waves, stream);
            return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

// Marlin payload of one expert matrix -> its slot of the fused MoE's stacked
// tile layout, with the payload's own integers, scales and zeros (no fp16
// round trip, no requantization).  Both layouts keep, per 16-row tile and
// 128-k block, 256 u32 of 8 nibbles each in the same nibble order; the u32
// holding k = 128 kb + 32 a + 8 b + r (r = 0..7) of column c sits at index
// 4 c + 64 b + a in the Marlin block and 4 c + 64 a + b in the MoE block, so
// the blocks differ by a 4 x 4 transpose of (a, b) per column.
//   sz[tile][g][c] = fp16 scale bits | fp16(zero) bits << 16 of row 16 tile + c.
__global__ void marlin_to_moe_tile_k(const uint32_t* __restrict__ qw, const uint16_t* __restrict__ S,
                                     const uint32_t* __restrict__ Z, uint32_t* __restrict__ qt,
                                     uint32_t* __restrict__ sz, int N, int K, int G) {
    const long nq = (long)N * K / 8, nsz = (long)(N / 16) * G * 16;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < nq + nsz;
         i += (long)gridDim.x * blockDim.x) {
        if (i < nq) {
            const long blk = i >> 8;
            const int w = (int)(i & 255);
            const int c = (w >> 2) & 15, a = w >> 6, b = w & 3;
            qt[i] = qw[(blk << 8) + 4 * c + 64 * b + a];
        } else {
            const long j = i - nq;
            const int c = (int)(j & 15);
            const long tg = j >> 4;
            const int g = (int)(tg % G);
            const int n = (int)(tg / G) * 16 + c;
            const uint32_t sb = S[(size_t)g * N + marlin_scale_pos(n)];
            const int z = marlin_zero(Z + (size_t)g * (N / 8), n);
            sz[j] = sb | ((uint32_t)bitcast<uint16_t>((f16)(float)z) << 16);
        }
    }
}

// LDS bytes of int4_gemv_norm: a 1 KB slot per block of every wave, the
// cross-wave reduction area and the per-wave norm partials.
constexpr size_t gemv_norm_lds(int T, int NB, int waves) {
    return (size_t)waves * NB * 1024 + (size_t)waves * T * 1024 + 256;
}

template <int T, int NB, bool G32, bool SWI>
hipError_t launch_gemv_norm(const NormArgs& nrm, const uint32_t* Wq, const uint16_t* S,
                            const uint32_t* Z, f16* C, int N, int K, int waves, hipStream_t st) {
    const size_t lds = gemv_norm_lds(T, NB, waves);
    if (lds > kMaxLds) return hipErrorInvalidValue;
    const dim3 grid(SWI ? N / 32 : N / (16 * T)), block(64 * waves);
    hipLaunchKernelGGL((int4_gemv_norm<T, NB, G32, SWI>), grid, block, lds, st, nrm, Wq, S, Z, C, N, K);
    return hipGetLastError();
}

template <int T, bool G32, bool SWI>
hipError_t dispatch_gemv_norm(int nb, const NormArgs& nrm, const uint32_t* Wq, const uint16_t* S,
                              const uint32_t* Z, f16* C, int N, int K, int waves, hipStream_t st) {
    switch (nb) {
        case 1: return launch_gemv_norm<T, 1, G32, SWI>(nrm, Wq, S, Z, C, N, K, waves, st);
        case 2: return launch_gemv_norm<T, 2, G32, SWI>(nrm, Wq, S, Z, C, N, K, waves, st);
        case 3: return launch_gemv_norm<T, 3, G32, SWI>(nrm, Wq, S, Z, C, N, K, waves, st);
        case 4: return launch_gemv_norm<T, 4, G32, SWI>(nrm, Wq, S, Z, C, N, K, waves, st);
        case 6: return launch_gemv_norm<T, 6, G32, SWI>(nrm, Wq, S, Z, C, N, K, waves, st);
        default: return launch_gemv_norm<T, 8, G32, SWI>(nrm, Wq, S, Z, C, N, K, waves, st);
    }
}

// add_rmsnorm + one decode row's GEMV (or gate/up GEMV with the SwiGLU
// epilogue).  The plain GEMV's M = 1 shape choice, four blocks per wave at
// most with 32-groups and eight otherwise.
template <bool G32>
hipError_t gemv_norm(const NormArgs& nrm, const uint32_t* Wq, const uint16_t* S, const uint32_t* Z,
                     f16* C, int N, int K, bool swi, hipStream_t st) {
    const int nfull = K / 128;
    const int cap = G32 ? 4 : 8;
    int waves, tiles;
    if (swi) {
        tiles = 2;
        waves = N >= 16384 ? 8 : 16;
        while (waves > 1 && nfull < waves) waves /= 2;
        while ((nfull + waves - 1) / waves > cap && waves < 16) waves *= 2;
    } else {
        const GemvCfg c = default_gemv_cfg(1, N, K, G32);
        tiles = c.tiles == 2 ? 2 : 1;
        waves = c.waves;
    }
    int nb = nb_bucket((nfull + waves - 1) / waves);
    if (nb > cap) return hipErrorInvalidValue;
    // two tiles per workgroup need 1 KB more reduction space per wave; where
    // that overflows the LDS (16 waves of 8 blocks: K > 12288) the plain GEMV
    // takes one tile, and the SwiGLU pair is refused (the caller runs the
    // standalone norm and the unfused kernels instead)
    if (tiles == 2 && gemv_norm_lds(2, nb, waves) > kMaxLds) {
        if (swi) return hipErrorInvalidValue;
        tiles = 1;
    }
    if (gemv_norm_lds(tiles, nb, waves) > kMaxLds) return hipErrorInvalidValue;
    if (swi) return dispatch_gemv_norm<2, G32, true>(nb, nrm, Wq, S, Z, C, N, K, waves, st);
    if (tiles == 2) return dispatch_gemv_norm<2, G32, false>(nb, nrm, Wq, S, Z, C, N, K, waves, st);
    return dispatch_gemv_norm<1, G32, false>(nb, nrm, Wq, S, Z, C, N, K, waves, st);
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
                                group_size, nullptr, nullptr);
}

bool FastllmCudaMarlinHalfInt4GemmStream(const void* a, const uint32_t* b_q_weight,
                                         const void* b_scales, const uint32_t* b_zeros, void* c,
                                         int size_m, int size_n, int size_k, int group_size,
                                         int* workspace, void* stream) {
    (void)workspace;
    return int4_marlin_abi_gemm(a, b_q_weight, b_scales, b_zeros, c, size_m, size_n, size_k,
                                group_size, (hipStream_t)stream, nullptr);
}

bool fastllm_int4_gemm_config(const void* a, const uint32_t* b_q_weight, const void* b_scales,
                              const uint32_t* b_zeros, void* c, int size_m, int size_n, int size_k,
                              int group_size, int tiles, int waves, int nb, void* stream) {
    GemvCfg cfg{tiles, waves, nb};
    if (size_m > 16) return false;
    return int4_marlin_abi_gemm(a, b_q_weight, b_scales, b_zeros, c, size_m, size_n, size_k,
                                group_size, (hipStream_t)stream, &cfg);
}

size_t fastllm_int4_gemm_ws_bytes(int size_m, int size_n, int size_k, int group_size) {
    if (size_m < 1 || size_m > 16 || size_n <= 0 || size_k <= 0) return 0;
    if (group_size != 32 && group_size != 128) return 0;
    const GemvCfg c = default_gemv_cfg(size_m, size_n, size_k, group_size == 32, true);
    return c.split > 1 && size_n / 16 <= kSplitStrips ? splitk_ws_bytes(size_m, size_n, c.split) : 0;
}

int fastllm_int4_gemm_ws(const void* a, const uint32_t* b_q_weight, const void* b_scales,
                         const uint32_t* b_zeros, void* c, int size_m, int size_n, int size_k,
                         int group_size, void* workspace, size_t workspace_bytes, const int* cfg,
                         void* stream) {
    if (!int4_args_ok(a, b_q_weight, b_scales, b_zeros, c, size_m, size_n, size_k, group_size)) return 1;
    if (cfg && size_m > 16) return 1;
    GemvCfg forced;
    if (cfg) {
        forced.tiles = cfg[0];
        forced.waves = cfg[1];
        forced.nb = cfg[2];
        forced.split = cfg[3];
    }
    return int4_marlin_abi_gemm(a, b_q_weight, b_scales, b_zeros, c, size_m, size_n, size_k, group_size,
                                (hipStream_t)stream, cfg ? &forced : nullptr, workspace, workspace_bytes)
               ? 0
               : 2;
}

int fastllm_int4_gemm_swiglu(const void* a, const uint32_t* b_q_weight, const void* b_scales,
                             const uint32_t* b_zeros, void* h, int size_m, int size_n, int size_k,
                             int group_size, void* stream) {
    if (size_m < 1 || size_m > 16 || size_n % 128 != 0 || size_k % 128 != 0 || size_k > 65536)
        return 1;
    if (group_size != 32 && group_size != 128) return 1;
    if (!a || !b_q_weight || !b_scales || !b_zeros || !h) return 1;
    if (!fl_aligned(a, 16) || !fl_aligned(b_q_weight, 16) || !fl_aligned(h, 2) ||
        !fl_aligned(b_scales, 2) || !fl_aligned(b_zeros, 4))
        return 1;
    if (!fl_current_device_supported()) return 2;
    const f16* A = static_cast<const f16*>(a);
    const uint16_t* S = static_cast<const uint16_t*>(b_scales);
    f16* H = static_cast<f16*>(h);
    const hipError_t e =
        group_size == 32
            ? dispatch_swiglu<true>(A, b_q_weight, S, b_zeros, H, size_m, size_n, size_k, (hipStream_t)stream)
            : dispatch_swiglu<false>(A, b_q_weight, S, b_zeros, H, size_m, size_n, size_k, (hipStream_t)stream);
    if (e == hipErrorInvalidValue) return 1;  // shape beyond the fused kernel (see dispatch_swiglu)
    return report(e, "fastllm_int4_gemm_swiglu") ? 0 : 2;
}

int fastllm_marlin_to_moe_tile(const uint32_t* b_q_weight, const void* b_scales,
                               const uint32_t* b_zeros, uint8_t* qtile, uint32_t* sz, int size_n,
                               int size_k, int group_size, void* stream) {
    if (!b_q_weight || !b_scales || !b_zeros || !qtile || !sz) return 1;
    if (size_n <= 0 || size_n % 64 || size_k <= 0 || size_k % 128) return 1;
    if (group_size != 32 && group_size != 128) return 1;
    if (!fl_aligned(b_q_weight, 4) || !fl_aligned(qtile, 4) || !fl_aligned(sz, 4)) return 1;
    if (!fl_current_device_supported()) return 2;
    const long work = (long)size_n * size_k / 8 + (long)(size_n / 16) * (size_k / group_size) * 16;
    const int grid = (int)((work + 255) / 256 < 16384 ? (work + 255) / 256 : 16384);
    hipLaunchKernelGGL(marlin_to_moe_tile_k, dim3(grid), dim3(256), 0, (hipStream_t)stream, b_q_weight,
                       static_cast<const uint16_t*>(b_scales), b_zeros, reinterpret_cast<uint32_t*>(qtile),
                       sz, size_n, size_k, size_k / group_size);
    return report(hipGetLastError(), "fastllm_marlin_to_moe_tile") ? 0 : 2;
}

int fastllm_int4_gemm_add_rmsnorm(const float* x, const void* delta, const void* norm_w, float eps,
                                  float* xnew, const uint32_t* b_q_weight, const void* b_scales,
                                  const uint32_t* b_zeros, void* c, int size_n, int size_k,
                                  int group_size, int swiglu, void* stream) {
    if (!x || !delta || !norm_w || !xnew || !b_q_weight || !b_scales || !b_zeros || !c) return 1;
    if (size_k < 128 || size_k % 128 || size_k > 65536 || size_n <= 0 || size_n % 64) return 1;
    if (swiglu && size_n % 128) return 1;
    if (group_size != 32 && group_size != 128) return 1;
    if (!fl_aligned(x, 16) || !fl_aligned(delta, 16) || !fl_aligned(norm_w, 16) || !fl_aligned(xnew, 16) ||
        !fl_aligned(b_q_weight, 16))
        return 1;
    // workgroup 0 stores xnew while later workgroups still read x and delta:
    // an in-place update would feed them x + 2 delta
    if (fl_overlap(xnew, (size_t)size_k * 4, x, (size_t)size_k * 4) ||
        fl_overlap(xnew, (size_t)size_k * 4, delta, (size_t)size_k * 2))
        return 1;
    if (!fl_current_device_supported()) return 2;
    const NormArgs nrm{x, static_cast<const uint16_t*>(delta), static_cast<const uint16_t*>(norm_w), xnew,
                       eps};
    const uint16_t* S = static_cast<const uint16_t*>(b_scales);
    f16* C = static_cast<f16*>(c);
    const hipError_t e =
        group_size == 32
            ? gemv_norm<true>(nrm, b_q_weight, S, b_zeros, C, size_n, size_k, swiglu != 0, (hipStream_t)stream)
            : gemv_norm<false>(nrm, b_q_weight, S, b_zeros, C, size_n, size_k, swiglu != 0, (hipStream_t)stream);
    if (e == hipErrorInvalidValue) return 1;
    return report(e, "fastllm_int4_gemm_add_rmsnorm") ? 0 : 2;
}

}  // extern "C"
