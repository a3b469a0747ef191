// FP8-E4M3 weight-only GEMV/GEMM on gfx950.
//
// Two weight formats (reference: native/fastllm_fp8_block128.cu,
// fastllm_py/kernels/fp8.py, fastllm_py/quantizer.py:65-94):
//   * "inline" 1x128: every weight row is [128 codes][f32 scale] x K/128,
//     row stride perRow = K + 4K/128 bytes; one scale per (row, 128-k block).
//     This is the reference .so's C ABI (fastllm_fp8_block128_*).
//   * "128x128": codes [N, K] row-major, scales f32 [ceil(N/128), ceil(K/128)]
//     (quantize_fp8_block's format); K may end in a 64-wide block.
//
//   C[M, N] = A[M, K] @ dequant(W)^T (+ bias), A/C fp16 or bf16.
//
// Kernel: same decomposition as the INT4 GEMV (strip of T 16-row weight
// tiles per workgroup, waves splitting the 128-k blocks, every load of a wave
// issued up front, activations staged in LDS, fixed-order LDS reduction).  A
// lane (q = lane/16, c = lane%16) of the v_mfma_f32_16x16x32_{f16,bf16} B
// operand owns column c (a weight row) and ends up with bytes [32q, 32q+32)
// of each 128-byte block; its A fragments are taken at the same k offsets.
// Weights are loaded whole-line: each load instruction reads eight complete
// 128-byte block rows (the 16 B pieces 2q and 2q+1 of columns c and c^8 come
// in through lanes c and c^8, one of the two in the other's place), and one
// DPP row rotation by 8 trades the misplaced pieces (trade_pieces).  Reading
// only half of each line per instruction -- the 64 B a column's four lanes
// own -- costs a quarter of the bandwidth on row-major weights.
// e4m3 codes become fp16/bf16 exactly through v_cvt_scalef32_pk_*_fp8
// (scale 1.0); the block scale multiplies the fp32 partial.
#include "common.cuh"
#include "device.cuh"
#include "fp8_codec.cuh"
#include "gemv_common.cuh"

namespace {

template <bool BF16>
FL_DEV u32x4 fp8x8_to_16(uint32_t w0, uint32_t w1) {
    if (BF16) {
        return u32x4{bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false)),
                     bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true)),
                     bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false)),
                     bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true))};
    } else {
        return u32x4{bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false)),
                     bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true)),
                     bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false)),
                     bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true))};
    }
}

// Whole-line weight loads.  Columns c < 8 and c >= 8 of a 16-lane row form
// pairs (c, c^8).  Load i0 of lane (q, c) holds piece 2q + (c >= 8) of the
// lower block of the pair, load i1 piece 2q + 1 - (c >= 8) of the upper one,
// so each load reads the full 128 B of eight blocks.  Afterwards lane (q, c)
// keeps its own piece 2q (own) and receives piece 2q + 1 of its own block
// from lane c^8 (mate); "lower" and "upper" are whatever column groups the
// kernel pairs.
FL_DEV void trade_pieces(const u32x4& i0, const u32x4& i1, bool up, u32x4& own, u32x4& mate) {
    const u32x4 send = up ? i0 : i1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        own[e] = up ? i1[e] : i0[e];
        mate[e] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)send[e], 0x128 /* row_ror:8 */, 0xF,
                                                        0xF, false);
    }
}

template <bool BF16>
FL_DEV f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    if (BF16) return mfma_bf16(bitcast<bf16x8>(a), bitcast<bf16x8>(b), c);
    return mfma_f16(bitcast<f16x8>(a), bitcast<f16x8>(b), c);
}

template <bool BF16>
FL_DEV uint16_t f32_to_act(float v) {
    if (BF16) return bitcast<uint16_t>((__bf16)v);
    return bitcast<uint16_t>((f16)v);
}
template <bool BF16>
FL_DEV float act_to_f32(uint16_t v) {
    if (BF16) return (float)bitcast<__bf16>(v);
    return (float)bitcast<f16>(v);
}

// INLINE: row stride `rs` bytes, block stride 132, scale after the codes.
// !INLINE: row stride rs (= K), block stride 128, scales [N/128, nks].
// Activations (AM):
//   AM 0 (M <= 4): each wave copies the rows of its own blocks global -> LDS
//     (buffer_load ... lds, 1 KB = 4 rows x 128 k per block) before its
//     weight loads and waits only for them -- no workgroup barrier;
//   AM 1: M x K staged in LDS per workgroup (barrier that waits for LDS only);
//   AM 2: MFMA A fragments read from global memory (L2) at use;
//   AM 3 (M > 4, NB <= 4): each lane loads its own A fragments of all its
//     blocks into registers first of all (no LDS, no barrier);
//   AM 5 (4 < M <= 8): AM 0's per-wave copies of the block's 8 rows as whole
//     256-byte rows, two copies of 4 rows (the 16-byte k chunks of row r
//     XOR-swizzled by r), 2 KB per block.  AM 3's fragment loads read four
//     16-byte pieces 64 B apart per row and cost the CU's vector-cache path
//     several times the accesses of whole lines: 10944 x 2048, M = 8
//     8.67 -> 7.51 us.
template <int T, int NB, bool INLINE, bool BF16, int AM>
__global__ __launch_bounds__(1024) void fp8_gemv_nb(
    const uint16_t* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ Sc,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ C, int M, int N, int K, int rs,
    int nks) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int BSTRIDE = INLINE ? 132 : 128;
    const int nwaves = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int strip = xcd_block();  // XCD-grouped: neighbours share scale rows in L2
    const int nfull = K >> 7;
    const int col = lane & 15;
    const int kq = lane >> 4;
    const int lda = K + 8;
    constexpr bool ALDS = AM == 1;
    uint16_t* As = reinterpret_cast<uint16_t*>(smem);
    constexpr int SLOT = AM == 5 ? 2048 : 1024;  // per-wave LDS bytes per block (AM 0 / 5)
    const size_t abytes = (AM == 0 || AM == 5) ? (size_t)nwaves * NB * SLOT
                                               : (ALDS ? (((size_t)M * lda * 2 + 15) & ~(size_t)15) : 0);
    float* red = reinterpret_cast<float*>(smem + abytes);

    const int nb = wave < nfull ? (nfull - wave + nwaves - 1) / nwaves : 0;
    const int sw = ALDS ? stage_waves(M, K) : 0;
    const bool early = sw <= nwaves;
    RowStager stg;
    const bool stager = ALDS && early && wave < sw;
    if (stager) stg.load(A, M, K, lda, wave, lane);
    const int arow_m = col < M ? col : M - 1;
    // AM 0: lane l of block slot i copies row min(l / 16, M - 1), 16-byte
    // piece l % 16 of the block into this wave's LDS slot
    unsigned char* aslot = smem + (size_t)wave * NB * SLOT;
    if (AM == 5) {
        // copy p of block slot i: lane l brings row r = 4 p + l / 16 (rows
        // past M repeat row M - 1), k chunk (l % 16) ^ r, to position l % 16
        const __amdgpu_buffer_rsrc_t rA = buf_rsrc(A, (uint32_t)M * K * 2);
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            int kb = wave + (i < nb ? i : (nb > 0 ? nb - 1 : 0)) * nwaves;
            kb = kb < nfull ? kb : nfull - 1;
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const int r = 4 * p + (lane >> 4);
                const uint32_t ao = 2u * ((uint32_t)(r < M ? r : M - 1) * K + 8 * ((lane & 15) ^ r));
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lptr_t)(aslot + i * 2048 + p * 1024), 16, ao,
                                                         kb * 256, 0, 0);
            }
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
    u32x4 ar[NB][4];
    if (AM == 3) {
        const uint16_t* ap = A + (size_t)arow_m * K + 32 * kq;
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            int kb = wave + (i < nb ? i : (nb > 0 ? nb - 1 : 0)) * nwaves;
            kb = kb < nfull ? kb : nfull - 1;
#pragma unroll
            for (int j = 0; j < 4; ++j) ar[i][j] = *reinterpret_cast<const u32x4*>(ap + kb * 128 + 8 * j);
        }
    }

    // tile rows paired (c, c + 8): load 0 reads rows 0..7 of the tile, load 1
    // rows 8..15, each all 128 B of its block
    const bool up = col >= 8;
    const int p0 = 16 * (2 * kq + (up ? 1 : 0)), p1 = 16 * (2 * kq + (up ? 0 : 1));
    const uint8_t* rb0[T];
    const uint8_t* rb1[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int n0 = (strip * T + t) * 16 + (col & 7), n1 = n0 + 8;
        rb0[t] = W + (size_t)(n0 < N ? n0 : N - 1) * rs;
        rb1[t] = W + (size_t)(n1 < N ? n1 : N - 1) * rs;
    }

    u32x4 ld0[NB][T], ld1[NB][T];
    float sv[NB][T];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        int kb = wave + (i < nb ? i : (nb > 0 ? nb - 1 : 0)) * nwaves;
        kb = kb < nfull ? kb : nfull - 1;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const size_t bo = (size_t)kb * BSTRIDE;
            ld0[i][t] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_a4*>(rb0[t] + bo + p0));
            ld1[i][t] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_a4*>(rb1[t] + bo + p1));
            // inline: the scale of the lane's own row (rb0 for c < 8, rb1 for
            // c >= 8); 128 x 128: the tile's 16 rows share one scale band
            if (INLINE)
                sv[i][t] = *reinterpret_cast<const float*>((up ? rb1[t] : rb0[t]) + bo + 128);
            else
                sv[i][t] = Sc[(size_t)(((strip * T + t) * 16) >> 7) * nks + kb];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (AM == 0 || AM == 5) {
        // this wave's activation copies, issued before its weight loads, are
        // done once at most the weight loads are outstanding: two vector
        // loads per (block, tile) of codes; the block scale may be a third
        // (inline rows) or a scalar load (uniform address in the 128 x 128
        // format), so count only the two -- a stricter wait, never a shorter
        constexpr int WL = NB * T * 2;
        wait_vmcnt<(WL < 63 ? WL : 63)>();
    }
    if (ALDS) {
        if (stager) stg.store(As);
        if (!early) stage_rows_loop(A, As, M, K, lda);
        lds_barrier();  // the weight loads stay in flight
    }

    const uint16_t* arow = ALDS ? As + (size_t)arow_m * lda : A + (size_t)arow_m * K;
    f32x4 acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const bool live = i < nb;
        int kb = wave + (live ? i : (nb > 0 ? nb - 1 : 0)) * nwaves;
        kb = kb < nfull ? kb : nfull - 1;
        // k offsets 32 kq + 8 j of the block (bytes [32 kq, 32 kq + 32))
        u32x4 a[4];
        if (AM == 0) {
            const unsigned char* ak = aslot + (size_t)i * 1024 + arow_m * 256 + 64 * kq;
#pragma unroll
            for (int j = 0; j < 4; ++j) a[j] = *reinterpret_cast<const u32x4*>(ak + 16 * j);
        } else if (AM == 5) {
            const unsigned char* ak = aslot + (size_t)i * 2048 + arow_m * 256;
#pragma unroll
            for (int j = 0; j < 4; ++j) a[j] = *reinterpret_cast<const u32x4*>(ak + 16 * ((4 * kq + j) ^ arow_m));
        } else if (AM == 3) {
#pragma unroll
            for (int j = 0; j < 4; ++j) a[j] = ar[i][j];
        } else {
            const uint16_t* ak = arow + kb * 128 + 32 * kq;
#pragma unroll
            for (int j = 0; j < 4; ++j) a[j] = *reinterpret_cast<const u32x4*>(ak + 8 * j);
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            u32x4 lo, hi;
            trade_pieces(ld0[i][t], ld1[i][t], up, lo, hi);
            f32x4 part = f32x4{0.f, 0.f, 0.f, 0.f};
            part = mfma16<BF16>(a[0], fp8x8_to_16<BF16>(lo[0], lo[1]), part);
            part = mfma16<BF16>(a[1], fp8x8_to_16<BF16>(lo[2], lo[3]), part);
            part = mfma16<BF16>(a[2], fp8x8_to_16<BF16>(hi[0], hi[1]), part);
            part = mfma16<BF16>(a[3], fp8x8_to_16<BF16>(hi[2], hi[3]), part);
            const float s = live ? sv[i][t] : 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[t][e] = __builtin_fmaf(s, part[e], acc[t][e]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    if (!INLINE && (K & 127) && wave == 0) {
        // trailing 64-wide block: bytes [16q, 16q+16) only (four lanes read
        // a row's 64 B)
        const uint16_t* ak = (AM == 0 || AM == 3 || AM == 5 ? A + (size_t)arow_m * K : arow) + nfull * 128 + 16 * kq;
        const u32x4 a0 = *reinterpret_cast<const u32x4*>(ak);
        const u32x4 a1 = *reinterpret_cast<const u32x4*>(ak + 8);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int n = (strip * T + t) * 16 + col;
            const uint8_t* bp = W + (size_t)(n < N ? n : N - 1) * rs + (size_t)nfull * BSTRIDE;
            const u32x4 w = *reinterpret_cast<const u32x4_a4*>(bp + 16 * kq);
            f32x4 part = f32x4{0.f, 0.f, 0.f, 0.f};
            part = mfma16<BF16>(a0, fp8x8_to_16<BF16>(w[0], w[1]), part);
            part = mfma16<BF16>(a1, fp8x8_to_16<BF16>(w[2], w[3]), part);
            const float s = Sc[(size_t)(((strip * T + t) * 16) >> 7) * nks + nfull];
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[t][e] = __builtin_fmaf(s, part[e], acc[t][e]);
        }
    }

    reduce_and_store<T>(red, acc, M, wave, nwaves, lane, [&](int m, int t, int c, float v) {
        const int n = (strip * T + t) * 16 + c;
        if (n >= N) return;
        if (bias) v += act_to_f32<BF16>(bias[n]);
        C[(size_t)m * N + n] = f32_to_act<BF16>(v);
    });
}

// Decode GEMV for M <= 4 on 4-row tiles ("quartered" MFMA).
//
// A 16 x 16 MFMA tile normally needs 16 weight rows, so N = 2048 gives only
// 128 workgroups -- half of the GPU's CUs.  Here the 16 B-operand columns are
// (row r, k-quarter h) = column 4 h + r of a 4-row tile, and the 16 A-operand
// rows are (k-quarter h', activation row m) = row 4 h' + m: lane column
// 4 h + r reads the weights of row r in quarter h of K, lane row 4 h' + m the
// activations of row m in quarter h'.  The diagonal blocks h' == h of the
// product are the quarter partial sums; summing them over h gives the
// output.  The off-diagonal blocks are discarded.  So one 128-k MFMA step
// covers 4 rows x 4 quarters, and a workgroup needs only 4 weight rows.
//   * Quarter h holds blocks [h QB, (h + 1) QB) of the nfull full 128-k
//     blocks (QB = ceil(nfull / 4)); waves take block slots b of a quarter
//     round-robin, NB at most.  Blocks past nfull repeat the last one with a
//     zero scale.
//   * Each wave copies the activations of its own slots global -> LDS
//     (buffer_load ... lds, 1 KB = 4 quarters x 128 k per activation row)
//     before issuing its weight loads; no workgroup barrier precedes the
//     MFMAs.
//   * A trailing 64-wide block (128 x 128 format) is added by wave 0 through
//     quarter 0.
//   * Lane l holds the diagonal element of column l % 16 when
//     l / 16 == (l % 16) / 4; waves and quarters are summed through LDS in a
//     fixed order.
template <int NB, bool INLINE, bool BF16>
__global__ __launch_bounds__(1024) void fp8_gemv_q4(
    const uint16_t* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ Sc,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ C, int M, int N, int K, int rs,
    int nks) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int BSTRIDE = INLINE ? 132 : 128;
    const int nwaves = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = xcd_block() * 4;
    const int nfull = K >> 7;
    const int QB = (nfull + 3) >> 2;
    const int col = lane & 15, kq = lane >> 4;
    const int r = col & 3, h = col >> 2;  // B column (row, quarter)
    const int am = col & 3, ah = col >> 2;  // A row (quarter ah, activation row am)

    // this wave's slots b = wave + i * nwaves (< QB), block of quarter q: q QB + b
    const int nb = wave < QB ? (QB - wave + nwaves - 1) / nwaves : 0;
    auto slot_b = [&](int i) { return wave + (i < nb ? i : (nb > 0 ? nb - 1 : 0)) * nwaves; };

    // activation copies: slot i, row m -> 1 KB at aslot + (i * 4 + m) KB,
    // lane l = 16 quarter + piece: k = (quarter QB + b) 128 + 8 piece
    unsigned char* aslot = smem + (size_t)wave * NB * 4096;
    {
        const __amdgpu_buffer_rsrc_t rA = buf_rsrc(A, (uint32_t)M * K * 2);
        const int q = lane >> 4, piece = lane & 15;
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int b = slot_b(i);
            int kb = q * QB + b;
            kb = kb < nfull ? kb : nfull - 1;
            for (int m = 0; m < M; ++m)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rA, (lptr_t)(aslot + (i * 4 + m) * 1024), 16,
                    2u * ((uint32_t)m * K + kb * 128 + 8 * piece), 0, 0, 0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // every copy is issued before any weight load

    const int wrow = row0 + r < N ? row0 + r : N - 1;
    const uint8_t* rbase = W + (size_t)wrow * rs;
    // whole-line loads: columns (r, h) and (r, h + 2) are paired; load 0
    // reads quarters 0 and 1, load 1 quarters 2 and 3
    const bool up = h >= 2;
    const int p0 = 16 * (2 * kq + (up ? 1 : 0)), p1 = 16 * (2 * kq + (up ? 0 : 1));
    // block scales first, then the codes: the live select below waits for
    // the scales only (loads return in issue order), with the codes still
    // in flight.  A select right after each scale load, among the code
    // loads, waited for all of them before the first MFMA; a scale used
    // only at its block was moved past the copy wait below.
    u32x4 ld0[NB], ld1[NB];
    float sv[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const int kbr = h * QB + slot_b(i);  // the lane's own block
        const int kb = kbr < nfull ? kbr : nfull - 1;
        sv[i] = INLINE ? *reinterpret_cast<const float*>(rbase + (size_t)kb * BSTRIDE + 128)
                       : Sc[(size_t)(wrow >> 7) * nks + kb];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const int b = slot_b(i);
        const int k0 = (h & 1) * QB + b, k1 = (2 + (h & 1)) * QB + b;
        ld0[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_a4*>(
            rbase + (size_t)(k0 < nfull ? k0 : nfull - 1) * BSTRIDE + p0));
        ld1[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_a4*>(
            rbase + (size_t)(k1 < nfull ? k1 : nfull - 1) * BSTRIDE + p1));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NB; ++i) sv[i] = (i < nb && h * QB + slot_b(i) < nfull) ? sv[i] : 0.0f;
    __builtin_amdgcn_sched_barrier(0);
    // the activation copies went out first: done once at most the code
    // loads (two per slot, issued last) are outstanding; the scale loads
    // between them and the copies are then done too (the select above
    // needs them anyway), whichever memory path they take
    {
        constexpr int WL = NB * 2;  // lo, hi
        wait_vmcnt<(WL < 63 ? WL : 63)>();
    }

    const int arow = am < M ? am : M - 1;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const unsigned char* ab = aslot + (i * 4 + arow) * 1024 + ah * 256 + 64 * kq;
        u32x4 lo, hi;
        trade_pieces(ld0[i], ld1[i], up, lo, hi);
        f32x4 part = f32x4{0.f, 0.f, 0.f, 0.f};
        part = mfma16<BF16>(*reinterpret_cast<const u32x4*>(ab), fp8x8_to_16<BF16>(lo[0], lo[1]), part);
        part = mfma16<BF16>(*reinterpret_cast<const u32x4*>(ab + 16), fp8x8_to_16<BF16>(lo[2], lo[3]), part);
        part = mfma16<BF16>(*reinterpret_cast<const u32x4*>(ab + 32), fp8x8_to_16<BF16>(hi[0], hi[1]), part);
        part = mfma16<BF16>(*reinterpret_cast<const u32x4*>(ab + 48), fp8x8_to_16<BF16>(hi[2], hi[3]), part);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(sv[i], part[e], acc[e]);
        __builtin_amdgcn_sched_barrier(0);
    }

    if (!INLINE && (K & 127) && wave == 0) {
        // trailing 64-wide block, through quarter 0 only (columns and A rows
        // of other quarters carry zeros)
        const int kt = nfull * 128;
        u32x4 a0 = u32x4{0u, 0u, 0u, 0u}, a1 = a0, w = a0;
        if (ah == 0) {
            const uint16_t* ar = A + (size_t)arow * K + kt + 16 * kq;
            a0 = *reinterpret_cast<const u32x4*>(ar);
            a1 = *reinterpret_cast<const u32x4*>(ar + 8);
        }
        if (h == 0) w = *reinterpret_cast<const u32x4_a4*>(rbase + (size_t)nfull * BSTRIDE + 16 * kq);
        f32x4 part = f32x4{0.f, 0.f, 0.f, 0.f};
        part = mfma16<BF16>(a0, fp8x8_to_16<BF16>(w[0], w[1]), part);
        part = mfma16<BF16>(a1, fp8x8_to_16<BF16>(w[2], w[3]), part);
        const float st = Sc[(size_t)(wrow >> 7) * nks + nfull];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(st, part[e], acc[e]);
    }

    // diagonal lanes (kq == h) hold rows m = 0..3 of column (r, h)
    float* red = reinterpret_cast<float*>(smem + (size_t)nwaves * NB * 4096);
    if (kq == h) {
#pragma unroll
        for (int e = 0; e < 4; ++e) red[(wave * 16 + col) * 4 + e] = acc[e];
    }
    __syncthreads();
    if (threadIdx.x < 16) {
        const int rr = threadIdx.x >> 2, m = threadIdx.x & 3;
        const int n = row0 + rr;
        if (m < M && n < N) {
            float v = 0.f;
            for (int w = 0; w < nwaves; ++w)
#pragma unroll
                for (int q = 0; q < 4; ++q) v += red[(w * 16 + 4 * q + rr) * 4 + m];
            if (bias) v += act_to_f32<BF16>(bias[n]);
            C[(size_t)m * N + n] = f32_to_act<BF16>(v);
        }
    }
}

// Decode GEMV for M <= 8 (above four rows, or up to four when K >= 8192) on
// 8-row tiles ("halved" MFMA), the q4 scheme
// with two k-parts: B column 8 h + r = weight row r in half h of K, A row
// 8 h' + m = activation row m in half h'; the diagonal blocks h' == h are the
// half partial sums.  A workgroup needs 8 weight rows (N = 2048: 256
// workgroups instead of 128).  M x K activations are too large for LDS here
// (8 x 10944 bf16 = 175 KB), so above four rows each lane loads its own A
// fragments of all its slots into registers, ahead of its weight loads.  Up
// to four rows (ALDS) each wave first copies the activation bytes its slots
// need (M rows x 2 halves x 256 B per slot) into its LDS slot, 64 chunks of
// 16 B per buffer_load ... lds, and its lanes read their fragments there:
// sixteen lanes share each fragment, so the register loads moved 8 x the
// unique bytes through the address path and held every wave's weight loads
// back (2048 x 10944, M = 1: the last wave's loads went out 5.4 us in).
//   * Half h holds blocks [h HB, (h + 1) HB) (HB = ceil(nfull / 2)); waves
//     take slots round-robin, NB at most; blocks past nfull repeat the last
//     one with a zero scale.
//   * Accumulator element e of lane l is A row 4 (l / 16) + e: half
//     (l / 16) / 2, activation row 4 ((l / 16) % 2) + e; it is a diagonal
//     element when that half equals the lane's column half.
//   * RING (4 < M <= 8, where the slots' 4 KB of activations each do not
//     fit the LDS): a ring of two LDS slots per wave, each slot's 8 rows x 2
//     halves as whole 256-byte rows (16-byte k chunks of row-half rh
//     XOR-swizzled by rh), slots 0 and 1 copied before the weight loads and
//     slot i + 2 once slot i has been read.  M = 8: 2048 x 10944 10.08 ->
//     8.37 us, 2048 x 2048 3.56 -> 3.28 us against register fragments.
template <int NB, bool INLINE, bool BF16, bool ALDS, bool RING = false>
__global__ __launch_bounds__(1024) void fp8_gemv_q2(
    const uint16_t* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ Sc,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ C, int M, int N, int K, int rs,
    int nks) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int BSTRIDE = INLINE ? 132 : 128;
    const int nwaves = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = xcd_block() * 8;
    const int nfull = K >> 7;
    const int HB = (nfull + 1) >> 1;
    const int col = lane & 15, kq = lane >> 4;
    const int r = col & 7, h = col >> 3;  // B column (row, half) and A row (half, activation row)
    const int nb = wave < HB ? (HB - wave + nwaves - 1) / nwaves : 0;
    auto slot_b = [&](int i) { return wave + (i < nb ? i : (nb > 0 ? nb - 1 : 0)) * nwaves; };

    // A fragments first: lane (col, kq) = activation row col % 8 (clamped),
    // half col / 8, k 32 kq + {0, 8, 16, 24} of the slot's block
    const int arow = (col & 7) < M ? (col & 7) : M - 1;
    u32x4 ar[NB][4];
    unsigned char* aslot = smem + (size_t)wave * (RING ? 2 * 4096 : NB * 2048);
    const __amdgpu_buffer_rsrc_t rAr = buf_rsrc(A, (uint32_t)M * K * 2);
    // RING: the four copies of slot i into ring position i & 1 -- copy c
    // lane l: row-half rh = 4 c + l / 16 (row rh / 2 clamped to M - 1, half
    // rh % 2), k chunk (l % 16) ^ rh of the half's block, to position l % 16
    auto ring_copy = [&](int i) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int rh = 4 * c + (lane >> 4);
            const int m = (rh >> 1) < M ? (rh >> 1) : M - 1;
            int kb = (rh & 1) * HB + slot_b(i);
            kb = kb < nfull ? kb : nfull - 1;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rAr, (lptr_t)(aslot + (i & 1) * 4096 + c * 1024), 16,
                2u * ((uint32_t)m * K + kb * 128 + 8 * ((lane & 15) ^ rh)), 0, 0, 0);
        }
    };
    if (RING) {
        ring_copy(0);
        if (NB > 1) ring_copy(1);
    }
    if (ALDS) {
        // chunk q = ((i M + m) 2 + half) 16 + p (16 B each) lands at 16 q
        const int total = NB * M * 32;
        const int ncp = (total + 63) >> 6;
        const __amdgpu_buffer_rsrc_t rA = buf_rsrc(A, (uint32_t)M * K * 2);
        for (int c = 0; c < ncp; ++c) {
            int q = c * 64 + lane;
            q = q < total ? q : total - 1;
            const int i = q / (M * 32), rem = q - i * M * 32;
            const int m = rem >> 5, hh = (rem >> 4) & 1, pc = q & 15;
            int kb = hh * HB + slot_b(i);
            kb = kb < nfull ? kb : nfull - 1;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lptr_t)(aslot + c * 1024), 16,
                                                     2u * ((uint32_t)m * K + kb * 128 + pc * 8), 0, 0, 0);
        }
    } else if (!RING) {
        const uint16_t* ap = A + (size_t)arow * K + 32 * kq;
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            int kb = h * HB + slot_b(i);
            kb = kb < nfull ? kb : nfull - 1;
#pragma unroll
            for (int j = 0; j < 4; ++j) ar[i][j] = *reinterpret_cast<const u32x4*>(ap + kb * 128 + 8 * j);
        }
    }
    const int wrow = row0 + r < N ? row0 + r : N - 1;
    const uint8_t* rbase = W + (size_t)wrow * rs;
    // whole-line loads: columns (r, 0) and (r, 1) are paired; load 0 reads
    // half 0, load 1 half 1
    const bool up = h == 1;
    const int p0 = 16 * (2 * kq + h), p1 = 16 * (2 * kq + 1 - h);
    // block scales first, then the codes (as in the quartered kernel)
    u32x4 ld0[NB], ld1[NB];
    float sv[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const int kbr = h * HB + slot_b(i);  // the lane's own block
        const int kb = kbr < nfull ? kbr : nfull - 1;
        sv[i] = INLINE ? *reinterpret_cast<const float*>(rbase + (size_t)kb * BSTRIDE + 128)
                       : Sc[(size_t)(wrow >> 7) * nks + kb];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const int b = slot_b(i);
        const int k0 = b, k1 = HB + b;
        ld0[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_a4*>(
            rbase + (size_t)(k0 < nfull ? k0 : nfull - 1) * BSTRIDE + p0));
        ld1[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_a4*>(
            rbase + (size_t)(k1 < nfull ? k1 : nfull - 1) * BSTRIDE + p1));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NB; ++i) sv[i] = (i < nb && h * HB + slot_b(i) < nfull) ? sv[i] : 0.0f;
    __builtin_amdgcn_sched_barrier(0);
    if (ALDS) {
        // this wave's copies went out first: done once at most its code loads
        // (two per slot, issued after the scale loads) are outstanding
        constexpr int WL = NB * 2;
        wait_vmcnt<(WL < 63 ? WL : 63)>();
    }
    const int rhl = 2 * arow + h;  // RING: this lane's row-half

    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        u32x4 lo, hi;
        trade_pieces(ld0[i], ld1[i], up, lo, hi);
        if (RING) {
            // slot i's copies are done once at most the loads issued after
            // them are outstanding: slot 0 -- slot 1's copies and every code
            // load; slot 1 -- the code loads and slot 2's copies; slot i >= 2
            // -- slot i + 1's copies
            if (i == 0)
                wait_vmcnt<((NB > 1 ? 4 : 0) + 2 * NB < 63 ? (NB > 1 ? 4 : 0) + 2 * NB : 63)>();
            else if (i == 1)
                wait_vmcnt<(2 * NB + (NB > 2 ? 4 : 0) < 63 ? 2 * NB + (NB > 2 ? 4 : 0) : 63)>();
            else if (i + 1 < NB)
                wait_vmcnt<4>();
            else
                wait_vmcnt<0>();
        }
        u32x4 a[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            a[j] = ALDS ? *reinterpret_cast<const u32x4*>(aslot + (size_t)(((i * M + arow) * 2 + h) * 16 + 4 * kq + j) * 16)
                 : RING ? *reinterpret_cast<const u32x4*>(aslot + (i & 1) * 4096 + rhl * 256 +
                                                          16 * ((4 * kq + j) ^ rhl))
                        : ar[i][j];
        f32x4 part = f32x4{0.f, 0.f, 0.f, 0.f};
        part = mfma16<BF16>(a[0], fp8x8_to_16<BF16>(lo[0], lo[1]), part);
        part = mfma16<BF16>(a[1], fp8x8_to_16<BF16>(lo[2], lo[3]), part);
        part = mfma16<BF16>(a[2], fp8x8_to_16<BF16>(hi[0], hi[1]), part);
        part = mfma16<BF16>(a[3], fp8x8_to_16<BF16>(hi[2], hi[3]), part);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(sv[i], part[e], acc[e]);
        __builtin_amdgcn_sched_barrier(0);
        // slot i has been read (its MFMAs consumed the reads): its ring
        // position takes slot i + 2
        if (RING && i + 2 < NB) {
            ring_copy(i + 2);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    if (!INLINE && (K & 127) && wave == 0) {
        // trailing 64-wide block, through half 0 only (columns and A rows of
        // half 1 carry zeros)
        const int kt = nfull * 128;
        u32x4 a0 = u32x4{0u, 0u, 0u, 0u}, a1 = a0, w = a0;
        if (h == 0) {
            const uint16_t* at = A + (size_t)arow * K + kt + 16 * kq;
            a0 = *reinterpret_cast<const u32x4*>(at);
            a1 = *reinterpret_cast<const u32x4*>(at + 8);
            w = *reinterpret_cast<const u32x4_a4*>(rbase + (size_t)nfull * BSTRIDE + 16 * kq);
        }
        f32x4 part = f32x4{0.f, 0.f, 0.f, 0.f};
        part = mfma16<BF16>(a0, fp8x8_to_16<BF16>(w[0], w[1]), part);
        part = mfma16<BF16>(a1, fp8x8_to_16<BF16>(w[2], w[3]), part);
        const float st = Sc[(size_t)(wrow >> 7) * nks + nfull];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(st, part[e], acc[e]);
    }

    // diagonal elements: half (kq / 2) == h, activation row 4 (kq % 2) + e
    float* red = reinterpret_cast<float*>(smem + (ALDS ? (size_t)nwaves * NB * 2048
                                                        : RING ? (size_t)nwaves * 2 * 4096 : 0));
    if ((kq >> 1) == h) {
#pragma unroll
        for (int e = 0; e < 4; ++e) red[(wave * 16 + col) * 8 + 4 * (kq & 1) + e] = acc[e];
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const int rr = threadIdx.x >> 3, m = threadIdx.x & 7;
        const int n = row0 + rr;
        if (m < M && n < N) {
            float v = 0.f;
            for (int w = 0; w < nwaves; ++w)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) v += red[(w * 16 + 8 * hh + rr) * 8 + m];
            if (bias) v += act_to_f32<BF16>(bias[n]);
            C[(size_t)m * N + n] = f32_to_act<BF16>(v);
        }
    }
}

template <int NB, bool INLINE, bool BF16>
hipError_t launch_fp8_q2(const uint16_t* A, const uint8_t* W, const float* Sc, const uint16_t* bias,
                         uint16_t* C, int M, int N, int K, int rs, int nks, int waves,
                         hipStream_t st) {
    const size_t red = (size_t)waves * 16 * 8 * sizeof(float);
    if (M <= 4)
        hipLaunchKernelGGL((fp8_gemv_q2<NB, INLINE, BF16, true>), dim3((N + 7) / 8), dim3(64 * waves),
                           (size_t)waves * NB * 2048 + red, st, A, W, Sc, bias, C, M, N, K, rs, nks);
    else if ((size_t)waves * 2 * 4096 + red <= 160 * 1024)
        hipLaunchKernelGGL((fp8_gemv_q2<NB, INLINE, BF16, false, true>), dim3((N + 7) / 8), dim3(64 * waves),
                           (size_t)waves * 2 * 4096 + red, st, A, W, Sc, bias, C, M, N, K, rs, nks);
    else
        hipLaunchKernelGGL((fp8_gemv_q2<NB, INLINE, BF16, false>), dim3((N + 7) / 8), dim3(64 * waves), red, st,
                           A, W, Sc, bias, C, M, N, K, rs, nks);
    return hipGetLastError();
}

// 4 < M <= 8 and few 16-row strips: the halved 8-row kernel
template <bool INLINE, bool BF16>
hipError_t fp8_q2(const uint16_t* A, const uint8_t* W, const float* Sc, const uint16_t* bias,
                  uint16_t* C, int M, int N, int K, int rs, int nks, hipStream_t st) {
    const int HB = ((K >> 7) + 1) >> 1;
    const int nb = (HB + 15) / 16;
    const int waves = (HB + nb - 1) / nb;
    switch (nb) {
        case 1: return launch_fp8_q2<1, INLINE, BF16>(A, W, Sc, bias, C, M, N, K, rs, nks, waves, st);
        case 2: return launch_fp8_q2<2, INLINE, BF16>(A, W, Sc, bias, C, M, N, K, rs, nks, waves, st);
        case 3: return launch_fp8_q2<3, INLINE, BF16>(A, W, Sc, bias, C, M, N, K, rs, nks, waves, st);
        case 4: return launch_fp8_q2<4, INLINE, BF16>(A, W, Sc, bias, C, M, N, K, rs, nks, waves, st);
        default: return hipErrorInvalidValue;
    }
}

template <int NB, bool INLINE, bool BF16>
hipError_t launch_fp8_q4(const uint16_t* A, const uint8_t* W, const float* Sc, const uint16_t* bias,
                         uint16_t* C, int M, int N, int K, int rs, int nks, int waves,
                         hipStream_t st) {
    const size_t lds = (size_t)waves * NB * 4096 + (size_t)waves * 16 * 4 * sizeof(float);
    hipLaunchKernelGGL((fp8_gemv_q4<NB, INLINE, BF16>), dim3((N + 3) / 4), dim3(64 * waves), lds, st,
                       A, W, Sc, bias, C, M, N, K, rs, nks);
    return hipGetLastError();
}

// M <= 4 and few 16-row strips: the quartered kernel, as many waves as a
// quarter has blocks (up to 16), the fewest slots per wave that cover it
template <bool INLINE, bool BF16>
hipError_t fp8_q4(const uint16_t* A, const uint8_t* W, const float* Sc, const uint16_t* bias,
                  uint16_t* C, int M, int N, int K, int rs, int nks, hipStream_t st) {
    const int QB = ((K >> 7) + 3) >> 2;
    const int nb = (QB + 15) / 16;
    const int waves = (QB + nb - 1) / nb;
    if (nb > 4) return hipErrorInvalidValue;
    switch (nb) {
        case 1: return launch_fp8_q4<1, INLINE, BF16>(A, W, Sc, bias, C, M, N, K, rs, nks, waves, st);
        case 2: return launch_fp8_q4<2, INLINE, BF16>(A, W, Sc, bias, C, M, N, K, rs, nks, waves, st);
        case 3: return launch_fp8_q4<3, INLINE, BF16>(A, W, Sc, bias, C, M, N, K, rs, nks, waves, st);
        default: return launch_fp8_q4<4, INLINE, BF16>(A, W, Sc, bias, C, M, N, K, rs, nks, waves, st);
    }
}

struct Fp8Cfg {
    int tiles, waves, nb;
};

Fp8Cfg fp8_cfg(int M, int N, int K) {
    Fp8Cfg c;
    const int nfull = K / 128 > 0 ? K / 128 : 1;
    // one 16-row tile per workgroup (twice the workgroups of two: 10944 x 2048
    // measured 7.4 us against 8.2 at M = 1); on wide N eight waves up to
    // M = 8 and four above (10944 x 2048, M = 8: 6.9-7.1 us against 7.4-7.5
    // with four, 9.0 with sixteen)
    c.tiles = 1;
    int waves = N >= 8192 ? (M <= 8 ? 8 : 4) : 16;
    while (waves > 1 && nfull < waves) waves /= 2;
    while ((nfull + waves - 1) / waves > 6 && waves < 16) waves *= 2;
    c.waves = waves;
    int need = (nfull + waves - 1) / waves;
    c.nb = need <= 6 ? (need < 1 ? 1 : need) : 8;
    return c;
}

constexpr size_t kFp8LdsCap = 96 * 1024;

// Prefill-shaped FP8 GEMM (M > kF8MinM, 128 x 128 block format, K % 128 ==
// 0) on the matrix cores: the INT4 MFMA GEMM's structure with e4m3 weights.
//   * Workgroup tile BM (m) x 128 (n), eight waves side by side along n, a
//     BM x 16 wave tile (BM / 16 m-tiles x one n-tile of 16 x 16 fp32).
//     BM = 64, or 32 where the 64-row grid has at most 128 tiles and no K
//     split (2048 x 2048, M = 512: 13.6 -> 10.0 us; the copies bound the
//     kernel per CU, and twice the workgroups reach every CU for 1.5x the
//     lines copied in all).
//   * Every main-loop load goes global -> LDS (lds_copy: buffer_load ...
//     lds from inline asm) D 128-k blocks ahead into D + 1 stages of 32 KB
//     (D = 1: two workgroups per CU; D = 3: one), one vmcnt wait and one
//     barrier per block.  With the builtin copies the compiler drained them
//     all before each block's LDS reads, so no ring held more than one block.
//   * A stage holds the 64 x 128 activation tile row-major (256 B per row,
//     the 16-byte k chunks of row r XOR-swizzled by r % 16) and the strip's
//     128 weight rows x 128 codes row-major (128 B per row, the 16-code
//     chunks of row r swizzled by r % 8), so every copy moves whole cache
//     lines: 4 activation rows or 8 code rows.  The kernel is bound by its
//     copies (a variant without the MFMA loop ran as long as the kernel,
//     one without the copies half as long), and a copy that reads 16 rows x
//     64 B (the fragment-major order this replaced) costs a CU as much as
//     one of 8 full lines: M = 512, 2048 x 2048 / 10944 x 2048 / 2048 x
//     10944 19.7 / 56.5 / 53.7 -> 13.6 / 35.6 / 43.6 us (ring depths below).
//   * Codes become fp16/bf16 exactly (v_cvt_scalef32_pk_*_fp8, scale 1); each
//     block's MFMAs accumulate into a fresh partial that the fp32 block scale
//     then adds into the accumulator, as the GEMV does.
//   * A trailing 64-wide block is a 128-k block whose second half is read as
//     zeros (source offsets past the buffer end), activations and codes both.
constexpr int kF8BM = 64, kF8BN = 128, kF8MinM = 64;
// n-tiles per wave and waves per workgroup: one tile each for eight waves.
// Two tiles for four waves (half the LDS reads of activations per block)
// measured slower at M = 512: 26.7 / 65.0 / 132.4 us, with half the waves
// per SIMD to hide the LDS and conversion latencies.
constexpr int kF8NTW = 1, kF8Waves = 8 / kF8NTW;
// Blocks in flight ahead of the one computed (the ring holds D + 1 stages
// of 32 KB).  Grids of more than 256 workgroups take one block ahead, so
// two workgroups share a CU; smaller grids (at most one per CU) three.  With
// whole-line copies, M = 512: 10944 x 2048 (688 workgroups) 35.6 us one
// ahead, 41.3 two, 39.7 three; 2048 x 2048 (128) 15.7 / 14.7 / 13.6;
// 2048 x 10944 (two K splits, 256) 52.1 / 43.6 / 44.2.
// stage = BM x 128 activations (bf16) + 128 x 128 codes
constexpr size_t fp8_gemm_lds(int ahead, int bm) { return (size_t)(ahead + 1) * (bm * 256 + 16384); }

// Split-K (gridDim.y > 1, grids of fewer than 256 tiles): split y takes 128-k
// blocks [y kb_per, (y + 1) kb_per); each split stores its fp32 64 x 128
// accumulator tile (thread order) with device-coherent stores, waits for
// them, and bumps the tile's counter; the split that finds gridDim.y - 1
// sums the tiles in split order (deterministic), finishes the epilogue and
// resets the counter.  Nothing waits on another workgroup.
constexpr int kF8TileF = kF8BM * kF8BN;  // fp32 partials per tile and split

template <bool BF16, int D, int BM = 64>
__global__ __launch_bounds__(512) void fp8_gemm_mfma(const uint16_t* __restrict__ A,
                                                     const uint8_t* __restrict__ W,
                                                     const float* __restrict__ Sc,
                                                     const uint16_t* __restrict__ bias,
                                                     uint16_t* __restrict__ C, int M, int N, int K,
                                                     int nks, int kb_per, float* __restrict__ part,
                                                     int* __restrict__ cnt) {
    static_assert(BM == 32 || BM == 64, "tile height");
    constexpr int NS = D + 1, NTW = kF8NTW;
    constexpr int AF = BM / 32;          // A copies (4 rows each) per block and wave
    constexpr int MT = BM / 16;          // m-tiles each wave computes
    constexpr int LPB = AF + 2 * NTW;    // copies per block and wave: A rows, 2 halves per code tile
    constexpr int STB = BM * 256;        // codes after the activation rows
    constexpr int STG = STB + 16384;     // stage bytes
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kq = lane >> 4;
    const int nkb_all = (K + 127) >> 7;  // a trailing 64-wide block counts as one
    const int kb_lo = (int)blockIdx.y * kb_per;
    const int nkb = (nkb_all - kb_lo) < kb_per ? (nkb_all - kb_lo) : kb_per;  // this split's blocks
    const int ntiles = (N + 15) >> 4;

    const int nblk = (N + kF8BN - 1) / kF8BN, mblk = (M + BM - 1) / BM;
    const int total = nblk * mblk;
    int lin = blockIdx.x;
    if ((total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);  // XCD-grouped
    const int nb_i = lin / mblk, mb_i = lin - nb_i * mblk;
    const int m0 = mb_i * BM;
    const int nt_base = nb_i * 8;

    const i32x4_t rA = raw_rsrc(A, (uint32_t)M * K * 2);
    const i32x4_t rW = raw_rsrc(W, (uint32_t)N * K);
    const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
    // per-lane source offsets; a piece at k >= K (the second half of a
    // trailing 64-wide block) points past the buffer, and the copy reads zeros
    // Every copy reads whole 128-byte lines: A copy f brings rows 4 f ..
    // 4 f + 3 (256 B each), lane l row 4 f + l / 16 and its 16-byte k chunk
    // (l % 16) ^ (row % 16) into LDS position l % 16 of that row; code copy
    // (tile s, half h) brings rows 8 h .. 8 h + 7 of n-tile s (128 B each),
    // lane l row 8 h + l / 8 and its 16-code chunk (l % 8) ^ (l / 8).  The
    // XOR swizzles keep the MFMA reads below off shared banks.
    constexpr uint32_t kOut = 0x80000000u;
    uint32_t ao[AF], bo[NTW][2];
    int ak[AF], bk[NTW][2];
#pragma unroll
    for (int i = 0; i < AF; ++i) {
        const int r = 4 * (wave * AF + i) + (lane >> 4);  // tile row
        int m = m0 + r;
        m = m < M ? m : M - 1;
        ak[i] = 8 * ((lane & 15) ^ (r & 15));
        ao[i] = 2u * ((uint32_t)m * K + ak[i]);
    }
#pragma unroll
    for (int t = 0; t < NTW; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            int n = (nt_base + wave * NTW + t) * 16 + 8 * h + (lane >> 3);
            n = n < N ? n : N - 1;
            bk[t][h] = 16 * ((lane & 7) ^ (lane >> 3));
            bo[t][h] = (uint32_t)n * K + bk[t][h];
        }
    auto issue = [&](int kb, int slot) {
        kb = kb_lo + (kb < nkb ? kb : nkb - 1);
        const uint32_t st = lds0 + (uint32_t)slot * STG;
#pragma unroll
        for (int i = 0; i < AF; ++i)
            lds_copy(rA, st + (wave * AF + i) * 1024, kb * 128 + ak[i] < K ? ao[i] + kb * 256 : kOut);
#pragma unroll
        for (int i = 0; i < NTW; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                lds_copy(rW, st + STB + (wave * NTW + i) * 2048 + h * 1024,
                         kb * 128 + bk[i][h] < K ? bo[i][h] + kb * 128 : kOut);
    };
    // block-scale rows of this wave's two n-tiles (a 16-row tile lies in one band)
    const float* srow[NTW];
#pragma unroll
    for (int t = 0; t < NTW; ++t) {
        int nt = nt_base + wave * NTW + t;
        nt = nt < ntiles ? nt : ntiles - 1;
        srow[t] = Sc + (size_t)((nt * 16) >> 7) * nks;
    }

    f32x4 acc[MT][NTW];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < NTW; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < D; ++d) issue(d, d);

    // A operand of (m-tile mt, step j), lane (col, kq): row 16 mt + col, k
    // chunk 4 j + kq at position (4 j + kq) ^ col; codes of step j for n-tile
    // row col: chunk 2 j + kq / 2 at position (2 j + kq / 2) ^ (col % 8),
    // half kq % 2
    const int arow = col * 256, brow = col * 128 + 8 * (kq & 1);
    for (int kb0 = 0; kb0 < nkb; kb0 += NS) {
#pragma unroll
        for (int u = 0; u < NS; ++u) {
            const int kb = kb0 + u;
            const bool live = kb < nkb;
            wait_vmcnt<(D - 1) * LPB>();
            asm volatile("s_barrier" ::: "memory");
            issue(kb + D, (u + D) % NS);
            const unsigned char* st = smem + (size_t)u * STG;
            f32x4 part[MT][NTW];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int t = 0; t < NTW; ++t) part[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                u32x4 a[MT];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    a[mt] = *reinterpret_cast<const u32x4*>(st + mt * 4096 + arow + 16 * ((4 * j + kq) ^ col));
#pragma unroll
                for (int t = 0; t < NTW; ++t) {
                    const uint2 w8 = *reinterpret_cast<const uint2*>(
                        st + STB + (wave * NTW + t) * 2048 + brow + 16 * ((2 * j + (kq >> 1)) ^ (col & 7)));
                    const u32x4 b = fp8x8_to_16<BF16>(w8.x, w8.y);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) part[mt][t] = mfma16<BF16>(a[mt], b, part[mt][t]);
                }
            }
#pragma unroll
            for (int t = 0; t < NTW; ++t) {
                const float s = live ? srow[t][kb_lo + (kb < nkb ? kb : nkb - 1)] : 0.0f;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[mt][t][e] = __builtin_fmaf(s, part[mt][t][e], acc[mt][t][e]);
            }
        }
    }
    wait_vmcnt<0>();  // no LDS copy may still be in flight when the workgroup ends

    if (gridDim.y > 1) {
        static_assert(NTW == 1, "split-K partials assume one n-tile per wave");
        __shared__ int last;
        const int nsplit = (int)gridDim.y;
        const size_t tile_off = (size_t)blockIdx.x * (BM * kF8BN);
        const size_t split_stride = (size_t)gridDim.x * (BM * kF8BN);
        float* mine = part + (size_t)blockIdx.y * split_stride + tile_off;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                __hip_atomic_store(mine + ((wave * MT + mt) * 4 + e) * 64 + lane, acc[mt][0][e], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        // this wave's partial stores are complete (device-coherent stores: no
        // cache write-back needed)
        wait_vmcnt<0>();
        __syncthreads();
        if (threadIdx.x == 0)
            last = __hip_atomic_fetch_add(cnt + blockIdx.x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   nsplit - 1;
        __syncthreads();
        if (!last) return;
        // splits outermost: each pass issues the tile's loads together (one
        // memory round trip per split, not per element and split); every
        // element still sums its partials in split order
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[mt][0][e] = 0.0f;
        for (int q = 0; q < nsplit; ++q) {
            float pv[MT][4];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    pv[mt][e] = __hip_atomic_load(part + q * split_stride + tile_off +
                                                      ((wave * MT + mt) * 4 + e) * 64 + lane,
                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[mt][0][e] += pv[mt][e];
        }
        if (threadIdx.x == 0) __hip_atomic_store(cnt + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

#pragma unroll
    for (int t = 0; t < NTW; ++t) {
        const int n = (nt_base + wave * NTW + t) * 16 + col;
        if (n >= N) continue;
        const float bv = bias ? act_to_f32<BF16>(bias[n]) : 0.0f;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = m0 + mt * 16 + 4 * kq + e;
                if (m < M) C[(size_t)m * N + n] = f32_to_act<BF16>(acc[mt][t][e] + bv);
            }
    }
}

template <int T, int NB, bool INLINE, bool BF16>
hipError_t launch_fp8(const uint16_t* A, const uint8_t* W, const float* Sc, const uint16_t* bias,
                      uint16_t* C, int M, int N, int K, int rs, int nks, int waves,
                      hipStream_t st) {
    const size_t abytes = (((size_t)M * (K + 8) * 2 + 15) & ~(size_t)15);
    const size_t red = (size_t)waves * T * 1024;
    const size_t own = (size_t)waves * NB * 1024;
    const int strips = (N + 16 * T - 1) / (16 * T);
    if (M > 4 && M <= 8 && 2 * own + red <= 160 * 1024)
        hipLaunchKernelGGL((fp8_gemv_nb<T, NB, INLINE, BF16, 5>), dim3(strips), dim3(64 * waves),
                           2 * own + red, st, A, W, Sc, bias, C, M, N, K, rs, nks);
    else if (M <= 4 && own + red <= 160 * 1024)
        hipLaunchKernelGGL((fp8_gemv_nb<T, NB, INLINE, BF16, 0>), dim3(strips), dim3(64 * waves),
                           own + red, st, A, W, Sc, bias, C, M, N, K, rs, nks);
    else if (NB <= 4)
        hipLaunchKernelGGL((fp8_gemv_nb<T, NB, INLINE, BF16, 3>), dim3(strips), dim3(64 * waves), red,
                           st, A, W, Sc, bias, C, M, N, K, rs, nks);
    else if (abytes <= kFp8LdsCap)
        hipLaunchKernelGGL((fp8_gemv_nb<T, NB, INLINE, BF16, 1>), dim3(strips), dim3(64 * waves),
                           abytes + red, st, A, W, Sc, bias, C, M, N, K, rs, nks);
    else
        hipLaunchKernelGGL((fp8_gemv_nb<T, NB, INLINE, BF16, 2>), dim3(strips), dim3(64 * waves), red,
                           st, A, W, Sc, bias, C, M, N, K, rs, nks);
    return hipGetLastError();
}

template <int T, bool INLINE, bool BF16>
hipError_t fp8_dispatch_nb(int nb, const uint16_t* A, const uint8_t* W, const float* Sc,
                           const uint16_t* bias, uint16_t* C, int M, int N, int K, int rs, int nks,
                           int waves, hipStream_t st) {
    switch (nb) {
        case 1: return launch_fp8<T, 1, INLINE, BF16>(A, W, Sc, bias, C, M, N, K, rs, nks, waves, st);
        case 2: return launch_fp8<T, 2, INLINE, BF16>(A, W, Sc, bias, C, M, N, K, rs, nks, waves, st);
        case 3: return launch_fp8<T, 3, INLINE, BF16>(A, W, Sc, bias, C, M, N, K, rs, nks, waves, st);
        case 4: return launch_fp8<T, 4, INLINE, BF16>(A, W, Sc, bias, C, M, N, K, rs, nks, waves, st);
        case 5: return launch_fp8<T, 5, INLINE, BF16>(A, W, Sc, bias, C, M, N, K, rs, nks, waves, st);
        case 6: return launch_fp8<T, 6, INLINE, BF16>(A, W, Sc, bias, C, M, N, K, rs, nks, waves, st);
        default: return launch_fp8<T, 8, INLINE, BF16>(A, W, Sc, bias, C, M, N, K, rs, nks, waves, st);
    }
}

// K splits of the prefill GEMM for M x N x K: grids under 256 tiles split
// until they reach 256 workgroups, at most 4 splits of >= 16 blocks each
// (1: no split).  M = 512: 2048 x 10944 118.6 -> 79.3 us with two splits
// (one block ahead); 2048 x 2048 (16 blocks) is slower in two halves (24.0
// us against 19.7 whole, three blocks ahead), so short K stays whole.
int fp8_gemm_splits(int M, int N, int K) {
    const int tiles = ((N + kF8BN - 1) / kF8BN) * ((M + kF8BM - 1) / kF8BM);
    const int nkb = (K + 127) / 128;
    if (tiles >= 256) return 1;
    int s = (256 + tiles - 1) / tiles;
    s = s > 4 ? 4 : s;
    while (s > 1 && nkb / s < 16) --s;
    if (s > 1) s = (nkb + (nkb + s - 1) / s - 1) / ((nkb + s - 1) / s);  // no empty split
    return s;
}

// workspace: the tile counters in a fixed 1 KB (only grids under 256 tiles
// split), so calls of any shape on one workspace find theirs at zero, then
// fp32 partials [split][tile][64 x 128]
constexpr size_t kF8CntBytes = 256 * 4;
size_t fp8_gemm_ws_bytes(int M, int N, int K) {
    const int s = fp8_gemm_splits(M, N, K);
    if (s <= 1) return 0;
    const size_t tiles = (size_t)((N + kF8BN - 1) / kF8BN) * ((M + kF8BM - 1) / kF8BM);
    return kF8CntBytes + (size_t)s * tiles * kF8TileF * 4;
}

template <bool INLINE, bool BF16>
hipError_t fp8_gemm(const uint16_t* A, const uint8_t* W, const float* Sc, const uint16_t* bias,
                    uint16_t* C, int M, int N, int K, int rs, int nks, hipStream_t st,
                    void* ws = nullptr, size_t ws_bytes = 0) {
    // few 16-row strips and M <= 4: the quartered 4-row kernel up to
    // K = 8192; beyond, the halved kernel's activation traffic (half of the
    // quartered one's per weight byte) wins (2048 x 10944, M = 1: 8.4 us
    // against 8.8; re-measured 6.8 against 8.2)
    if (M <= 4 && K >= 512 && K < 8192 && N < 8192 && N % 4 == 0)
        return fp8_q4<INLINE, BF16>(A, W, Sc, bias, C, M, N, K, rs, nks, st);
    // M <= 8 there: the halved 8-row kernel (K <= 128 x 2 x 64)
    if (M <= 8 && K >= 512 && K <= 16384 && N < 8192 && N % 8 == 0)
        return fp8_q2<INLINE, BF16>(A, W, Sc, bias, C, M, N, K, rs, nks, st);
    // prefill-shaped: the MFMA GEMM (128 x 128 format; K % 64 == 0)
    if (!INLINE && M > kF8MinM && K % 64 == 0 && (size_t)N * K < (1ull << 31) &&
        (size_t)M * K * 2 < (1ull << 31)) {
        const int tiles = ((N + kF8BN - 1) / kF8BN) * ((M + kF8BM - 1) / kF8BM);
        const int nkb = (K + 127) / 128;
        int s = fp8_gemm_splits(M, N, K);
        if (s > 1 && (!ws || !fl_aligned(ws, 256) || ws_bytes < fp8_gemm_ws_bytes(M, N, K))) s = 1;
        const int kb_per = (nkb + s - 1) / s;
        int* cnt = s > 1 ? static_cast<int*>(ws) : nullptr;
        float* part = s > 1 ? reinterpret_cast<float*>(static_cast<char*>(ws) + kF8CntBytes) : nullptr;
        if (s == 1 && tiles <= 128) {
            // at most half the chip with 64-row tiles and no K split: 32-row
            // tiles, twice the workgroups (1.5x the lines copied in all, but
            // on every CU)
            const int t32 = ((N + kF8BN - 1) / kF8BN) * ((M + 31) / 32);
            hipLaunchKernelGGL((fp8_gemm_mfma<BF16, 3, 32>), dim3(t32, 1), dim3(64 * kF8Waves), fp8_gemm_lds(3, 32),
                               st, A, W, Sc, bias, C, M, N, K, nks, kb_per, part, cnt);
        } else if (tiles * s > 256) {
            hipLaunchKernelGGL((fp8_gemm_mfma<BF16, 1>), dim3(tiles, s), dim3(64 * kF8Waves), fp8_gemm_lds(1, 64), st,
                               A, W, Sc, bias, C, M, N, K, nks, kb_per, part, cnt);
        } else {
            hipLaunchKernelGGL((fp8_gemm_mfma<BF16, 3>), dim3(tiles, s), dim3(64 * kF8Waves), fp8_gemm_lds(3, 64), st,
                               A, W, Sc, bias, C, M, N, K, nks, kb_per, part, cnt);
        }
        return hipGetLastError();
    }
    // decode-shaped kernel, 16 activation rows per launch
    for (int m0 = 0; m0 < M; m0 += 16) {
        const int Mc = (M - m0) < 16 ? (M - m0) : 16;
        const Fp8Cfg c = fp8_cfg(Mc, N, K);
        const uint16_t* Am = A + (size_t)m0 * K;
        uint16_t* Cm = C + (size_t)m0 * N;
        const hipError_t e =
            c.tiles == 2
                ? fp8_dispatch_nb<2, INLINE, BF16>(c.nb, Am, W, Sc, bias, Cm, Mc, N, K, rs, nks,
                                                   c.waves, st)
                : fp8_dispatch_nb<1, INLINE, BF16>(c.nb, Am, W, Sc, bias, Cm, Mc, N, K, rs, nks,
                                                   c.waves, st);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// ---------------------------------------------- inline 1x128 quantization
// One wave per (row, 128-column block): scale = amax/448 (1 if not > 0), codes
// = satfinite-RNE e4m3 of x * (1/scale) (native/fastllm_fp8_block128.cu:52-97).
template <bool BF16>
__global__ void fp8_inline_quantize_k(const uint16_t* __restrict__ in, uint8_t* __restrict__ out,
                                      int rows, int cols, int packed_row_bytes) {
    const int lane = threadIdx.x & 63;
    const int bpr = cols / 128;
    const long total = (long)rows * bpr;
    for (long task = (long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); task < total;
         task += (long)gridDim.x * (blockDim.x >> 6)) {
        const int row = (int)(task / bpr), blk = (int)(task % bpr);
        const uint16_t* src = in + (size_t)row * cols + blk * 128;
        const float v0 = act_to_f32<BF16>(src[2 * lane]);
        const float v1 = act_to_f32<BF16>(src[2 * lane + 1]);
        float m = fmaxf(fabsf(v0), fabsf(v1));
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        float scale = m / 448.0f;
        if (!(scale > 0.0f)) scale = 1.0f;
        const float inv = 1.0f / scale;
        uint8_t* dst = out + (size_t)row * packed_row_bytes + (size_t)blk * 132;
        const uint16_t pair = (uint16_t)e4m3_encode_rne_sat(v0 * inv) |
                              ((uint16_t)e4m3_encode_rne_sat(v1 * inv) << 8);
        // 132-byte block stride: 2-byte stores are aligned, 4-byte ones are
        reinterpret_cast<uint16_t*>(dst)[lane] = pair;
        if (lane == 0) *reinterpret_cast<float*>(dst + 128) = scale;
    }
}

}  // namespace

extern "C" {

int fastllm_fp8_block128_packed_row_bytes(int m) { return m + (m / 128) * (int)sizeof(float); }

static int fp8_inline_quantize(const void* input, void* output, int rows, int columns, int isBf16,
                               hipStream_t st) {
    if (!input || !output || rows <= 0 || columns <= 0 || (columns % 128) != 0) return 1;
    if (!fl_current_device_supported()) return 2;
    const long tasks = (long)rows * (columns / 128);
    long grid = (tasks + 3) / 4;
    const long cap = (long)fl_current_device_cu_count() * 32;
    if (grid > cap) grid = cap;
    const int prb = fastllm_fp8_block128_packed_row_bytes(columns);
    if (isBf16)
        hipLaunchKernelGGL(fp8_inline_quantize_k<true>, dim3((unsigned)grid), dim3(256), 0, st,
                           (const uint16_t*)input, (uint8_t*)output, rows, columns, prb);
    else
        hipLaunchKernelGGL(fp8_inline_quantize_k<false>, dim3((unsigned)grid), dim3(256), 0, st,
                           (const uint16_t*)input, (uint8_t*)output, rows, columns, prb);
    return hipGetLastError() == hipSuccess ? 0 : 3;
}

int fastllm_fp8_block128_quantize(const void* input, void* output, int rows, int columns,
                                  int isBf16) {
    const int rc = fp8_inline_quantize(input, output, rows, columns, isBf16, nullptr);
    if (rc) return rc;
    const hipError_t e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) {
        fprintf(stderr, "fastllm_fp8_block128_quantize kernel error: %s\n", hipGetErrorString(e));
        return 3;
    }
    return 0;
}

int fastllm_fp8_block128_quantize_stream(const void* input, void* output, int rows, int columns,
                                         int isBf16, void* stream) {
    return fp8_inline_quantize(input, output, rows, columns, isBf16, (hipStream_t)stream);
}

static int fp8_inline_gemv(const void* A, const void* weight, void* C, const void* bias, int n,
                           int m, int k, int perRow, int isBf16, hipStream_t st) {
    if (n <= 0 || m <= 0 || k <= 0 || (m % 128) != 0 || !A || !weight || !C) return 1;
    if (perRow < fastllm_fp8_block128_packed_row_bytes(m) || (perRow & 3)) return 1;
    if (!fl_aligned(A, 16) || !fl_aligned(weight, 4)) return 1;
    if (!fl_current_device_supported()) return 2;
    const hipError_t e =
        isBf16 ? fp8_gemm<true, true>((const uint16_t*)A, (const uint8_t*)weight, nullptr,
                                      (const uint16_t*)bias, (uint16_t*)C, n, k, m, perRow, 0, st)
               : fp8_gemm<true, false>((const uint16_t*)A, (const uint8_t*)weight, nullptr,
                                       (const uint16_t*)bias, (uint16_t*)C, n, k, m, perRow, 0, st);
    if (e != hipSuccess) {
        fprintf(stderr, "fastllm_fp8_block128_gemv launch error: %s\n", hipGetErrorString(e));
        return 2;
    }
    return 0;
}

int fastllm_fp8_block128_gemv_fp16(const void* A, const void* weight, void* C, const void* bias,
                                   int n, int m, int k, int perRow) {
    const int rc = fp8_inline_gemv(A, weight, C, bias, n, m, k, perRow, 0, nullptr);
    if (rc) return rc;
    const hipError_t e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) {
        fprintf(stderr, "fastllm_fp8_block128_gemv_fp16 kernel error: %s\n", hipGetErrorString(e));
        return 2;
    }
    return 0;
}

int fastllm_fp8_block128_gemv_stream(const void* A, const void* weight, void* C, const void* bias,
                                     int n, int m, int k, int perRow, int isBf16, void* stream) {
    return fp8_inline_gemv(A, weight, C, bias, n, m, k, perRow, isBf16, (hipStream_t)stream);
}

static int fp8_b128x128_impl(const void* A, const uint8_t* Wq, const float* scales,
                             const void* bias, void* C, int M, int N, int K, int isBf16,
                             void* stream, void* ws, size_t ws_bytes) {
    if (M <= 0 || N <= 0 || K <= 0 || (K % 64) != 0 || !A || !Wq || !scales || !C) return 1;
    if (K < 128) return 1;
    if (!fl_aligned(A, 16) || !fl_aligned(Wq, 16) || (K % 16) != 0) return 1;
    if (!fl_current_device_supported()) return 2;
    const int nks = (K + 127) / 128;
    const hipError_t e =
        isBf16 ? fp8_gemm<false, true>((const uint16_t*)A, Wq, scales, (const uint16_t*)bias,
                                       (uint16_t*)C, M, N, K, K, nks, (hipStream_t)stream, ws, ws_bytes)
               : fp8_gemm<false, false>((const uint16_t*)A, Wq, scales, (const uint16_t*)bias,
                                        (uint16_t*)C, M, N, K, K, nks, (hipStream_t)stream, ws, ws_bytes);
    if (e != hipSuccess) {
        fprintf(stderr, "fastllm_fp8_b128x128_gemv launch error: %s\n", hipGetErrorString(e));
        return 2;
    }
    return 0;
}

int fastllm_fp8_b128x128_gemv(const void* A, const uint8_t* Wq, const float* scales,
                              const void* bias, void* C, int M, int N, int K, int isBf16,
                              void* stream) {
    return fp8_b128x128_impl(A, Wq, scales, bias, C, M, N, K, isBf16, stream, nullptr, 0);
}

size_t fastllm_fp8_b128x128_gemm_ws_bytes(int M, int N, int K) {
    if (M <= kF8MinM || N <= 0 || K <= 0 || K % 64) return 0;
    return fp8_gemm_ws_bytes(M, N, K);
}

int fastllm_fp8_b128x128_gemm_ws(const void* A, const uint8_t* Wq, const float* scales,
                                 const void* bias, void* C, int M, int N, int K, int isBf16,
                                 void* workspace, size_t workspace_bytes, void* stream) {
    return fp8_b128x128_impl(A, Wq, scales, bias, C, M, N, K, isBf16, stream, workspace,
                             workspace_bytes);
}

}  // extern "C"
