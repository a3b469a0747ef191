// Row-major INT4 GEMV, router and fused selective INT4 MoE on gfx950.
//
// Row-major INT4 format (fastllm_py/kernels/moe_int4.py:12-16, kept because
// the reference's callers build, cache and dequantize it themselves):
//   qweight (.., out, in/2) u8, two nibbles per byte, even column low;
//   scales, zeros (.., out, in/gs) fp16;  dequant = (q - zero) * scale.
//
// MFMA mapping (v_mfma_f32_16x16x32_f16, wave64): the B-operand lane l owns
// weight row 16t + l%16 and, per 128-k block, the 16 bytes at [16q, 16q+16)
// of that row's 64-byte block (q = l/16), i.e. k = 32q + 8j + r for u32 j
// and nibble r; its A fragments are read at the same k, so both operands see
// one permutation of k.  With group 128 the four lanes of a column share the
// group and the scale multiplies the fp32 MFMA partial; with groups of 32/64
// the weights are scaled in fp16 before the MFMA.
#include "common.cuh"
#include "device.cuh"
#include "gemv_common.cuh"
#include "int4_common.cuh"
#include "npmath.cuh"

#include <atomic>
#include <mutex>

namespace {

// 8 row-major nibbles (bytes b0..b3 of w; byte b = k 2b low, 2b+1 high) ->
// fp16 (q - z) in k order.  magic = {1024 (lo), 64 (hi)} exponent pair,
// zc = fp16 pair {-(1024+z), -(64+z)}.
FL_DEV u32x4 rm_dequant(uint32_t w, uint32_t zc, uint32_t magic) {
    const uint32_t t01 = __builtin_amdgcn_perm(w, w, 0x01000100u);  // b0 b1 b0 b1
    const uint32_t t23 = __builtin_amdgcn_perm(w, w, 0x03020302u);  // b2 b3 b2 b3
    const f16x2 z = bitcast<f16x2>(zc);
    const f16x2 p0 = bitcast<f16x2>(and_or(t01, 0x00F0000Fu, magic)) + z;
    const f16x2 p1 = bitcast<f16x2>(and_or(t01 >> 8, 0x00F0000Fu, magic)) + z;
    const f16x2 p2 = bitcast<f16x2>(and_or(t23, 0x00F0000Fu, magic)) + z;
    const f16x2 p3 = bitcast<f16x2>(and_or(t23 >> 8, 0x00F0000Fu, magic)) + z;
    return u32x4{bitcast<uint32_t>(p0), bitcast<uint32_t>(p1), bitcast<uint32_t>(p2),
                 bitcast<uint32_t>(p3)};
}

FL_DEV uint32_t rm_zero_consts(uint16_t z16) {
    const uint32_t z = (uint32_t)(float)bitcast<f16>(z16);
    return (0xE400u | z) | ((0xD400u | (z << 4)) << 16);
}

FL_DEV u32x4 scale_f16x8(u32x4 v, uint16_t s16) {
    const f16 s = bitcast<f16>(s16);
    const f16x2 ss{s, s};
    return u32x4{bitcast<uint32_t>(bitcast<f16x2>(v[0]) * ss), bitcast<uint32_t>(bitcast<f16x2>(v[1]) * ss),
                 bitcast<uint32_t>(bitcast<f16x2>(v[2]) * ss), bitcast<uint32_t>(bitcast<f16x2>(v[3]) * ss)};
}

constexpr uint32_t kRmMagic = 0x54006400u;

// One 128-k block of one 16-row tile: B lanes dequantized, 4 MFMAs, scale
// applied (group 128: on the fp32 partial; smaller groups: in fp16 before).
template <bool G128>
FL_DEV void rm_block_mma(f32x4& acc, const u32x4 (&a)[4], u32x4 w, uint16_t s16, uint16_t z16,
                         float live) {
    const uint32_t zc = rm_zero_consts(z16);
    if (G128) {
        f32x4 part = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j)
            part = mfma_f16(bitcast<f16x8>(a[j]), bitcast<f16x8>(rm_dequant(w[j], zc, kRmMagic)), part);
        const float s = (float)bitcast<f16>(s16) * live;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(s, part[e], acc[e]);
    } else {
        f32x4 part = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j)
            part = mfma_f16(bitcast<f16x8>(a[j]),
                            bitcast<f16x8>(scale_f16x8(rm_dequant(w[j], zc, kRmMagic), s16)), part);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(live, part[e], acc[e]);
    }
}

// Zero point of a stacked-expert group (fp16 holding an integer 0..15) as
// the fp16 pairs -(1024+z) and -(64+z).
FL_DEV void tile_zero_bits(uint16_t z16, uint32_t& zlo, uint32_t& zhi) {
    zero_bits((uint32_t)(float)bitcast<f16>(z16), zlo, zhi);
}

// One 128-k block of one 16-row tile of the stacked-expert tile layout
// (nibbles interleaved like the Marlin tile layout): B lanes dequantized,
// 4 MFMAs, scale applied (group 128: on the fp32 partial; smaller groups: in
// fp16 before).
template <bool G128>
FL_DEV void tile_block_mma(f32x4& acc, const u32x4 (&a)[4], u32x4 w, uint16_t s16, uint16_t z16,
                           float live) {
    uint32_t zlo, zhi;
    tile_zero_bits(z16, zlo, zhi);
    f32x4 part = f32x4{0.f, 0.f, 0.f, 0.f};
    if (G128) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            part = mfma_f16(bitcast<f16x8>(a[j]), dequant_word_fast(w[j], zlo, zhi, 0x64006400u, 0x54005400u),
                            part);
        const float s = (float)bitcast<f16>(s16) * live;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(s, part[e], acc[e]);
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            part = mfma_f16(bitcast<f16x8>(a[j]),
                            bitcast<f16x8>(scale_f16x8(bitcast<u32x4>(dequant_word_fast(
                                                           w[j], zlo, zhi, 0x64006400u, 0x54005400u)),
                                                       s16)),
                            part);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(live, part[e], acc[e]);
    }
}

// One 128-k block of one 16-row tile in quantize_int4_group's format
// (quantizer.py:97-129): fp32 scale s and fp32 group minimum mn, w = q*s + mn.
// Groups of 128 or more: s * sum(x*q) + mn * sum(x), both sums on the matrix
// cores (the second against a B operand of ones), scaled in fp32.  Groups of
// 32/64: w formed in fp16 by one fused multiply-add before the MFMA.
template <bool G128>
FL_DEV void a_block_mma(f32x4& acc, const u32x4 (&a)[4], u32x4 w, float s, float mn, float live) {
    const uint32_t zc = rm_zero_consts(0);
    f32x4 part = f32x4{0.f, 0.f, 0.f, 0.f};
    if (G128) {
        f32x4 xsum = f32x4{0.f, 0.f, 0.f, 0.f};
        const u32x4 ones = u32x4{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            part = mfma_f16(bitcast<f16x8>(a[j]), bitcast<f16x8>(rm_dequant(w[j], zc, kRmMagic)), part);
            xsum = mfma_f16(bitcast<f16x8>(a[j]), bitcast<f16x8>(ones), xsum);
        }
        const float ss = s * live, mm = mn * live;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(mm, xsum[e], __builtin_fmaf(ss, part[e], acc[e]));
    } else {
        const f16 s16 = (f16)s, m16 = (f16)mn;
        const f16x2 ss{s16, s16}, mm{m16, m16};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u32x4 q = rm_dequant(w[j], zc, kRmMagic);
            u32x4 v;
#pragma unroll
            for (int h = 0; h < 4; ++h)
                v[h] = bitcast<uint32_t>(__builtin_elementwise_fma(bitcast<f16x2>(q[h]), ss, mm));
            part = mfma_f16(bitcast<f16x8>(a[j]), bitcast<f16x8>(v), part);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(live, part[e], acc[e]);
    }
}

// ------------------------------------------------------ row-major INT4 GEMV
// Y[M, N] = X[M, K] @ dequant(W)^T, M <= 16, X/Y fp32 or fp16 (XF32/YF32).
// K % 128 == 0.  AFMT false: moe_int4.py's format, fp16 scale and zero,
// group gs in {32, 64, 128}.  AFMT true: quantize_int4_group's format
// (same nibbles), fp32 scale and minimum, gs in {32, 64} or a multiple of
// 128 (G128 then means "one group per 128-k block").
template <int NB, bool G128, bool XF32, bool YF32, bool AFMT>
__global__ __launch_bounds__(1024) void rm_gemv_nb(const void* __restrict__ Xv,
                                                   const uint8_t* __restrict__ Wq,
                                                   const void* __restrict__ Sv,
                                                   const void* __restrict__ Zv, void* __restrict__ Yv,
                                                   int M, int N, int K, int gs) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int nwaves = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nfull = K >> 7;
    const int col = lane & 15, kq = lane >> 4;
    const int lda = K + 8;
    f16* As = reinterpret_cast<f16*>(smem);
    float* red = reinterpret_cast<float*>(smem + (((size_t)M * lda * 2 + 15) & ~(size_t)15));
    const int G = K / gs;

    // stage X (converted to fp16) into LDS before issuing the weight loads:
    // loads retire in issue order, so staging after them would wait for all.
    {
        const int k8 = K >> 3;
        const int nchunks = M * k8;
        for (int c = threadIdx.x; c < nchunks; c += blockDim.x) {
            const int m = c / k8, c8 = c - m * k8;
            f16x8 v;
            if (XF32) {
                const float* src = reinterpret_cast<const float*>(Xv) + (size_t)m * K + c8 * 8;
                const f32x4 lo = *reinterpret_cast<const f32x4*>(src);
                const f32x4 hi = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[e] = (f16)lo[e];
                    v[4 + e] = (f16)hi[e];
                }
            } else {
                v = *reinterpret_cast<const f16x8*>(reinterpret_cast<const f16*>(Xv) + (size_t)m * K + c8 * 8);
            }
            *reinterpret_cast<f16x8*>(As + (size_t)m * lda + c8 * 8) = v;
        }
    }

    const int n = blockIdx.x * 16 + col;
    const int nc = n < N ? n : N - 1;
    const uint8_t* wrow = Wq + (size_t)nc * (K / 2);
    const int nb = wave < nfull ? (nfull - wave + nwaves - 1) / nwaves : 0;

    using P = typename std::conditional<AFMT, float, uint16_t>::type;
    const P* __restrict__ S = static_cast<const P*>(Sv);
    const P* __restrict__ Z = static_cast<const P*>(Zv);
    u32x4 wv[NB];
    P sv[NB], zv[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        int kb = wave + (i < nb ? i : (nb > 0 ? nb - 1 : 0)) * nwaves;
        kb = kb < nfull ? kb : nfull - 1;
        wv[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + kb * 64 + 16 * kq));
        const int g = (kb * 128 + (G128 ? 0 : 32 * kq)) / gs;
        sv[i] = S[(size_t)nc * G + g];
        zv[i] = Z[(size_t)nc * G + g];
    }
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();  // the weight loads stay in flight

    const f16* arow = As + (size_t)(col < M ? col : M - 1) * lda + 32 * kq;
    f32x4 acc[1] = {f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const bool live = i < nb;
        int kb = wave + (live ? i : (nb > 0 ? nb - 1 : 0)) * nwaves;
        kb = kb < nfull ? kb : nfull - 1;
        u32x4 a[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) a[j] = *reinterpret_cast<const u32x4*>(arow + kb * 128 + 8 * j);
        if constexpr (AFMT)
            a_block_mma<G128>(acc[0], a, wv[i], sv[i], zv[i], live ? 1.0f : 0.0f);
        else
            rm_block_mma<G128>(acc[0], a, wv[i], sv[i], zv[i], live ? 1.0f : 0.0f);
        __builtin_amdgcn_sched_barrier(0);
    }

    reduce_and_store<1>(red, acc, M, wave, nwaves, lane, [&](int m, int, int c, float v) {
        const int nn = blockIdx.x * 16 + c;
        if (nn >= N) return;
        if (YF32)
            reinterpret_cast<float*>(Yv)[(size_t)m * N + nn] = v;
        else
            reinterpret_cast<f16*>(Yv)[(size_t)m * N + nn] = (f16)v;
    });
}

// ------------------------------- row-major INT4 GEMV, whole-line loads (M <= 4)
// The decode shape of the row-major GEMV (the graph decoder's dgemv,
// graph_decode.py:170-216, M = 1).  A 128-byte line of a weight row holds
// two 128-k blocks (2p, 2p + 1), so the waves take k in pairs of blocks and
// every load instruction reads eight whole lines: load 0 of lane (q, c)
// reads 16-byte piece q + 4 [c >= 8] of tile row c mod 8, load 1 piece
// q + 4 [c < 8] of row 8 + c mod 8, and one DPP row rotation by 8 trades
// the misplaced pieces between lanes c and c ^ 8 (trade_rm).  Lane (q, c)
// then holds bytes [16q, 16q + 16) of row c's block 2p and of its block
// 2p + 1, i.e. k = 32q + 8j + r for word j, nibble position r.
//   * Dequantization in the nibbles' own order: (w & 0x000F000F) etc. give
//     the fp16 pairs (k0, k4), (k1, k5), (k2, k6), (k3, k7) of a word
//     (dequant_word_fast), so the MFMA reads the activations in that order:
//     fp16 rows are permuted in place once they land in LDS, fp32 rows are
//     paired that way when rounded to fp16.
//   * Wave w takes the NP consecutive pairs [w NP, w NP + NP), so the scales
//     and zeros of its blocks are one 16-byte piece per row (two where the
//     range crosses a piece): one copy global -> LDS per piece carries both
//     arrays for all its rows (lane = (array, tile, row)).  Per-block dword
//     loads of them put 16 requests on each scale line (one per pair) and
//     measured 1-4 us slower per launch.
//     fp16 scale/zero (group 128), or quantize_int4_group's fp32 scale and
//     minimum (group 128: s*sum(x q) + min*sum(x), the second sum against a
//     B operand of ones).
//   * Activations: each wave copies the rows of its own blocks global -> LDS
//     (buffer_load ... lds).  XC 0: fp16 rows, one copy = 4 rows x 128 k;
//     XC 1: fp32 rows, one copy = 2 rows x 128 k (M <= 2); XC 2: fp32, two
//     copies (M <= 4).  fp32 rows are rounded to fp16 at the MFMA, as
//     rm_gemv_nb stages them.
//   * All copies go out before the weight loads and a wave waits only for
//     its own (vmcnt = its weight loads); no workgroup barrier until the
//     reduction, whose partials go into each wave's own activation slots.
//   * Strips of T tiles, XCD-grouped.
FL_DEV void trade_rm(const u32x4& i0, const u32x4& i1, bool up, u32x4& own, u32x4& mate) {
    const u32x4 send = up ? i0 : i1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        own[e] = up ? i1[e] : i0[e];
        mate[e] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)send[e], 0x128 /* row_ror:8 */, 0xF, 0xF,
                                                        false);
    }
}

// 8 consecutive k (h0..h7) in the order dequant_word_fast produces them
FL_DEV f16x8 nib_order(f16x8 v) { return f16x8{v[0], v[4], v[1], v[5], v[2], v[6], v[3], v[7]}; }

template <int XC>
constexpr int rm_slot_bytes() {
    return XC == 2 ? 2048 : 1024;
}
// 16-byte scale/zero pieces a range of NP consecutive pairs can span (PP
// pairs per piece: 4 for fp16 values, 2 for fp32)
constexpr int rm_sz_pieces(int np, int pp) {
    int worst = 1;
    for (int w = 0; w < pp; ++w) {  // wave w starts at pair w np: offset (w np) mod pp
        const int n = ((w * np) % pp + np + pp - 1) / pp;
        worst = n > worst ? n : worst;
    }
    return worst;
}
// LDS bytes of one wave: activation slots (NP x 2 blocks; the reduction
// partials reuse them) and its scale/zero pieces
__host__ __device__ inline size_t rm_line_wave_lds(int np, int slot, int T, int pieces) {
    const size_t a = (size_t)np * 2 * slot;
    const size_t r = (size_t)T * 1024;
    return (a > r ? a : r) + (size_t)pieces * 1024;
}

template <int T, int NP, int XC, bool AFMT>
__global__ __launch_bounds__(1024) void rm_gemv_line(const void* __restrict__ Xv,
                                                     const uint8_t* __restrict__ Wq,
                                                     const void* __restrict__ Sv,
                                                     const void* __restrict__ Zv, void* __restrict__ Yv,
                                                     int y_fp32, int M, int N, int K) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int BSL = rm_slot_bytes<XC>();  // LDS bytes of one block's activation rows
    constexpr int ES = AFMT ? 4 : 2;          // bytes per scale / zero value
    constexpr int PP = 16 / (2 * ES);         // pairs per 16-byte scale piece
    constexpr int NPC = rm_sz_pieces(NP, PP);
    const int nwaves = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int strip = xcd_block();
    const int npairs = K >> 8;
    const int G = K >> 7;
    const int col = lane & 15, kq = lane >> 4;
    const int p_first = wave * NP;
    const int np = p_first < npairs ? (npairs - p_first < NP ? npairs - p_first : NP) : 0;
    const size_t wl = rm_line_wave_lds(NP, BSL, T, NPC);
    unsigned char* aslot = smem + (size_t)wave * wl;
    unsigned char* szl = aslot + (wl - (size_t)NPC * 1024);
    auto pair_of = [&](int i) {
        const int p = p_first + (i < np ? i : (np > 0 ? np - 1 : 0));
        return p < npairs ? p : npairs - 1;
    };

    // scale / zero pieces of this wave's pairs: copy c, lane (array, tile,
    // row) -> 16 B at szl + c KB + 16 lane
    const int piece0 = pair_of(0) / PP;
    {
        const int arr = lane >> 5, t = (lane >> 4) & 1, c = lane & 15;
        const int row = (strip * T + (t < T ? t : T - 1)) * 16 + c;
        const uint32_t rowoff = (uint32_t)(row < N ? row : N - 1) * G * ES;
        const uint32_t nbytes = (uint32_t)N * G * ES;
        const __amdgpu_buffer_rsrc_t r = buf_rsrc(arr ? Zv : Sv, nbytes);
#pragma unroll
        for (int c2 = 0; c2 < NPC; ++c2)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lptr_t)(szl + c2 * 1024), 16, rowoff + 16 * (piece0 + c2),
                                                     0, 0, 0);
    }
    // activation copies of this wave's blocks
    if (XC == 0) {
        const __amdgpu_buffer_rsrc_t rA = buf_rsrc(Xv, (uint32_t)M * K * 2);
        const int own_m = (lane >> 4) < M ? (lane >> 4) : M - 1;
        const uint32_t ao = 2u * ((uint32_t)own_m * K + 8 * (lane & 15));
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int p = pair_of(i);
#pragma unroll
            for (int h = 0; h < 2; ++h)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lptr_t)(aslot + (2 * i + h) * BSL), 16, ao,
                                                         (2 * p + h) * 256, 0, 0);
        }
    } else {
        const __amdgpu_buffer_rsrc_t rA = buf_rsrc(Xv, (uint32_t)M * K * 4);
#pragma unroll
        for (int c = 0; c < XC; ++c) {
            const int m = 2 * c + (lane >> 5);
            const int own_m = m < M ? m : M - 1;
            const uint32_t ao = 4u * ((uint32_t)own_m * K + 4 * (lane & 31));
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int p = pair_of(i);
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(
                        rA, (lptr_t)(aslot + (2 * i + h) * BSL + c * 1024), 16, ao, (2 * p + h) * 512, 0, 0);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // the copies go out before every load below

    const bool up = col >= 8;
    const int p0 = 16 * (kq + (up ? 4 : 0)), p1 = 16 * (kq + (up ? 0 : 4));
    const size_t rs = (size_t)(K >> 1);
    const uint8_t* rb0[T];
    const uint8_t* rb1[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int n0 = (strip * T + t) * 16 + (col & 7), n1 = n0 + 8;
        rb0[t] = Wq + (size_t)(n0 < N ? n0 : N - 1) * rs + p0;
        rb1[t] = Wq + (size_t)(n1 < N ? n1 : N - 1) * rs + p1;
    }
    u32x4 ld0[NP][T], ld1[NP][T];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const int p = pair_of(i);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            ld0[i][t] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rb0[t] + (size_t)p * 128));
            ld1[i][t] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rb1[t] + (size_t)p * 128));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // this wave's copies are done once at most its weight loads (two per
    // pair and tile) are outstanding
    constexpr int WL = NP * T * 2;
    wait_vmcnt<(WL < 63 ? WL : 63)>();
    if (XC == 0) {
        // fp16 rows into the nibble order, in place: lane l owns 16 B of
        // every block slot
#pragma unroll
        for (int s = 0; s < 2 * NP; ++s) {
            f16x8* pv = reinterpret_cast<f16x8*>(aslot + s * BSL + 16 * lane);
            *pv = nib_order(*pv);
        }
    }

    const int arow_m = col < M ? col : M - 1;
    const uint32_t mlo = 0x64006400u, mhi = 0x54005400u;
    uint32_t zlo0, zhi0;
    zero_bits(0, zlo0, zhi0);
    f32x4 acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const float live = i < np ? 1.0f : 0.0f;
        const int p = pair_of(i);
        u32x4 wb[T][2];  // blocks 2p and 2p + 1 of each tile
#pragma unroll
        for (int t = 0; t < T; ++t) trade_rm(ld0[i][t], ld1[i][t], up, wb[t][0], wb[t][1]);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            // k offsets 32 kq + 8 j of block 2p + h, in the nibble order
            f16x8 a[4];
            const unsigned char* ak = aslot + (2 * i + h) * BSL;
            if (XC == 0) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    a[j] = *reinterpret_cast<const f16x8*>(ak + arow_m * 256 + 64 * kq + 16 * j);
            } else {
                const float* af = reinterpret_cast<const float*>(ak + arow_m * 512) + 32 * kq;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x4 lo = *reinterpret_cast<const f32x4*>(af + 8 * j);
                    const f32x4 hi = *reinterpret_cast<const f32x4*>(af + 8 * j + 4);
                    a[j] = f16x8{(f16)lo[0], (f16)hi[0], (f16)lo[1], (f16)hi[1],
                                 (f16)lo[2], (f16)hi[2], (f16)lo[3], (f16)hi[3]};
                }
            }
            // value index of block 2p + h in this wave's pieces of its row
            const int vi = 2 * p + h - 2 * PP * piece0;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const unsigned char* rowp = szl + (vi / (2 * PP)) * 1024 + (t * 16 + col) * 16;
                const int vo = (vi % (2 * PP)) * ES;
                f32x4 part = f32x4{0.f, 0.f, 0.f, 0.f};
                if constexpr (AFMT) {
                    const float s = *reinterpret_cast<const float*>(rowp + vo) * live;
                    const float mn = *reinterpret_cast<const float*>(rowp + 512 + vo) * live;
                    f32x4 xsum = f32x4{0.f, 0.f, 0.f, 0.f};
                    const f16x8 ones = f16x8{1, 1, 1, 1, 1, 1, 1, 1};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        part = mfma_f16(a[j], dequant_word_fast(wb[t][h][j], zlo0, zhi0, mlo, mhi), part);
                        xsum = mfma_f16(a[j], ones, xsum);
                    }
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        acc[t][e] = __builtin_fmaf(mn, xsum[e], __builtin_fmaf(s, part[e], acc[t][e]));
                } else {
                    const uint16_t s16 = *reinterpret_cast<const uint16_t*>(rowp + vo);
                    const uint16_t z16 = *reinterpret_cast<const uint16_t*>(rowp + 512 + vo);
                    uint32_t zlo, zhi;
                    zero_bits((uint32_t)(float)bitcast<f16>(z16), zlo, zhi);
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        part = mfma_f16(a[j], dequant_word_fast(wb[t][h][j], zlo, zhi, mlo, mhi), part);
                    const float s = (float)bitcast<f16>(s16) * live;
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[t][e] = __builtin_fmaf(s, part[e], acc[t][e]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // cross-wave reduction: wave w's partials into its own slots (their
    // activations are consumed), read back by all after one barrier
#pragma unroll
    for (int t = 0; t < T; ++t) *reinterpret_cast<f32x4*>(aslot + t * 1024 + lane * 16) = acc[t];
    __syncthreads();
    for (int idx = threadIdx.x; idx < T * 256; idx += blockDim.x) {
        const int l = (idx & 255) >> 2, e = idx & 3, t = idx >> 8;
        const int m = 4 * (l >> 4) + e;
        const int n = (strip * T + t) * 16 + (l & 15);
        if (m >= M || n >= N) continue;
        float v = 0.f;
        for (int w = 0; w < nwaves; ++w)
            v += reinterpret_cast<const float*>(smem + (size_t)w * wl + t * 1024)[idx & 255];
        if (y_fp32)
            reinterpret_cast<float*>(Yv)[(size_t)m * N + n] = v;
        else
            reinterpret_cast<f16*>(Yv)[(size_t)m * N + n] = (f16)v;
    }
}

// ------------------------------------------------------------- gate matvec
// logits[t, e] = sum_h x[t, h] * W[e, h] in fp32 (fp16 W), t < T, for the E
// router rows and, when sgw is given, one more row (shared-expert gate) into
// slogit[t] (moe_int4.py:139-169).  One workgroup per row, 256 threads.
__global__ void gate_matvec_k(const float* __restrict__ x, const uint16_t* __restrict__ gw,
                              const uint16_t* __restrict__ sgw, float* __restrict__ logits,
                              float* __restrict__ slogit, int T, int E, int hidden) {
    __shared__ float red[4][16];
    const int e = blockIdx.x;
    const uint16_t* w = (e < E) ? gw + (size_t)e * hidden : sgw;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    for (int t0 = 0; t0 < T; t0 += 16) {
        const int tn = (T - t0) < 16 ? (T - t0) : 16;
        float acc[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) acc[t] = 0.f;
        for (int h = threadIdx.x; h < hidden; h += blockDim.x) {
            const float wf = (float)bitcast<f16>(w[h]);
#pragma unroll
            for (int t = 0; t < 16; ++t)
                if (t < tn) acc[t] = __builtin_fmaf(x[(size_t)(t0 + t) * hidden + h], wf, acc[t]);
        }
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            float v = acc[t];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
            if (lane == 0) red[wv][t] = v;
        }
        __syncthreads();
        if (threadIdx.x < tn) {
            const float v = red[0][threadIdx.x] + red[1][threadIdx.x] + red[2][threadIdx.x] + red[3][threadIdx.x];
            if (e < E)
                logits[(size_t)(t0 + threadIdx.x) * E + e] = v;
            else
                slogit[t0 + threadIdx.x] = v;
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------ router
// One wave per token, numpy's arithmetic (fastllm_py/expert_router.py:22-71):
//   softmax: p = exp(s - max) / pairwise_sum(exp(s - max));
//   sigmoid: p = 1 / (1 + exp(-s)), selection value p + bias;
//   group-limited: keep the topk_group groups with the largest
//   (second largest + largest) selection value, others -inf;
//   top-k by (value desc, index asc), weights p[idx], optional
//   w / (sum(w) + 1e-20) in selection order, times `scale`.
// Up to 256 experts (4 per lane), k <= 16.
//
// Expert-major lists ("MoE lists"), consumed by the fused MoE kernels:
//   n_active; active[s] expert of slot s; offsets[s..s+1] its entries;
//   tok/tokw[p] token and weight of entry p (tokens ascending within a slot).
constexpr int kMaxTopK = 16;

struct MoeLists {
    int* n_active;
    int* active;
    int* offsets;
    int* tok;
    float* tokw;
};

struct RouteArgs {
    const float* logits;
    const float* bias;
    const float* slogit;  // shared-expert gate logits, optional
    int T, E, K, scoring, norm, n_group, topk_group;
    float scale;
    int* topk_ids;
    float* topk_w;
    float* rw;       // dense [T, E], optional
    float* scoef;    // sigmoid(slogit) [T], optional
    MoeLists lists;  // built by route_k itself when the batch is one workgroup
    // optional: the last xh_blocks workgroups of route_k's grid store
    // xh[t, :] = fp16(x[t, :]) while the others route
    const float* x;
    uint16_t* xh;
    int hidden, xh_blocks;
    // batches of several routing workgroups: an arrival counter (zero before
    // the launch, left at zero) -- the last routing workgroup builds the
    // lists from every workgroup's picks (nullptr: route_lists_k does)
    int* arrive;
};

// Inclusive prefix sum over the wave: shifts by 1, 2, 4, 8 inside each
// 16-lane row (DPP), then the totals of the rows before a lane's row.
FL_DEV int wave_incl_scan(int x, int lane) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
    const int t0 = __builtin_amdgcn_readlane(x, 15);
    const int t1 = __builtin_amdgcn_readlane(x, 31);
    const int t2 = __builtin_amdgcn_readlane(x, 47);
    const int row = lane >> 4;
    return x + (row == 0 ? 0 : (row == 1 ? t0 : (row == 2 ? t0 + t1 : t0 + t1 + t2)));
}

// MoE lists from the T*K routed entries of one workgroup (ids/ws
// token-major, T <= 32, each token's K experts distinct, all < E <= 256,
// blockDim.x >= 64).  Entry (t, k) of expert e goes to
//   base[e] + #{t' < t : t' chose e},
// the popcount of the expert's token mask sel[e] below bit t: one pass of
// LDS atomics (counts, masks), one scan of the counts by the first wave
// (slot offsets, active list), one pass of placements.  cnt/base/sel: E
// words of LDS each.
FL_DEV void build_lists(const int* ids, const float* ws, int T, int K, int E, MoeLists L,
                        int* cnt, int* base, unsigned* sel) {
    const int TK = T * K;
    const int tid = threadIdx.x, bd = blockDim.x;
    for (int e = tid; e < E; e += bd) {
        cnt[e] = 0;
        sel[e] = 0u;
    }
    __syncthreads();
    for (int i = tid; i < TK; i += bd) {
        const int e = ids[i];
        atomicAdd(&cnt[e], 1);
        atomicOr(&sel[e], 1u << (i / K));
    }
    __syncthreads();
    if (tid < 64) {
        int c[4], tot = 0, act = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int ee = 4 * tid + q;
            c[q] = ee < E ? cnt[ee] : 0;
            tot += c[q];
            act += c[q] > 0 ? 1 : 0;
        }
        const int it = wave_incl_scan(tot, tid), ia = wave_incl_scan(act, tid);
        int off = it - tot, na = ia - act;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int ee = 4 * tid + q;
            if (ee < E) {
                base[ee] = off;
                if (c[q] > 0) {
                    L.active[na] = ee;
                    L.offsets[na] = off;
                    ++na;
                }
                off += c[q];
            }
        }
        if (tid == 63) {
            L.offsets[ia] = it;
            *L.n_active = ia;
        }
    }
    __syncthreads();
    for (int i = tid; i < TK; i += bd) {
        const int e = ids[i], t = i / K;
        const int pos = base[e] + __builtin_popcount(sel[e] & ((1u << t) - 1u));
        L.tok[pos] = t;
        L.tokw[pos] = ws[i];
    }
}

// Order-preserving map of a float to an unsigned key (larger float, larger
// key; -inf above 0, so 0 marks "removed").
FL_DEV uint32_t order_key(float v) {
    const uint32_t u = bitcast<uint32_t>(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

FL_DEV float key_float(uint32_t k) {
    return bitcast<float>((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

FL_DEV uint32_t umax4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t x = a > b ? a : b, y = c > d ? c : d;
    return x > y ? x : y;
}

// Wave-wide unsigned maximum, uniform: DPP butterflies inside each 16-lane
// row (xor 1, xor 2, half-row mirror, row mirror), then the four row results
// read into scalar registers.
FL_DEV uint32_t wave_umax(uint32_t k) {
    uint32_t o;
    o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0xB1, 0xF, 0xF, false);  // quad_perm 1,0,3,2
    k = k > o ? k : o;
    o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0x4E, 0xF, 0xF, false);  // quad_perm 2,3,0,1
    k = k > o ? k : o;
    o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0x141, 0xF, 0xF, false);  // row_half_mirror
    k = k > o ? k : o;
    o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0x140, 0xF, 0xF, false);  // row_mirror
    k = k > o ? k : o;
    const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)k, 0);
    const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)k, 16);
    const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)k, 32);
    const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)k, 48);
    return umax4(r0, r1, r2, r3);
}

// np_sum_f32 of n <= 64 values held one per lane in v0, also stored at a[e]
// (LDS): np_sum_wave128 with at most eight 8-value blocks.
FL_DEV float np_sum_wave64(const float* a, int n, int lane, float v0) {
    float res = 0.0f;
    int i0 = 0;
    if (n >= 8) {
        const int q = n >> 3;  // 8-value blocks, 1..8
        const int j = lane & 7;
        float x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = a[8 * i + j];
        float r = x[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) r = i < q ? r + x[i] : r;
        r = r + bitcast<float>(__builtin_amdgcn_update_dpp(0, bitcast<int>(r), 0xB1, 0xF, 0xF, false));
        r = r + bitcast<float>(__builtin_amdgcn_update_dpp(0, bitcast<int>(r), 0x4E, 0xF, 0xF, false));
        r = r + bitcast<float>(__builtin_amdgcn_update_dpp(0, bitcast<int>(r), 0x141, 0xF, 0xF, false));
        res = bitcast<float>(__builtin_amdgcn_readlane(bitcast<int>(r), 0));
        i0 = 8 * q;
    }
    for (int i = i0; i < n; ++i) res += bitcast<float>(__builtin_amdgcn_readlane(bitcast<int>(v0), i));
    return res;
}

// numpy's float32 row sum (np_sum_f32) of n <= 128 values held one per lane
// in v[0] (e < 64) and v[1] (e >= 64), also stored at a[e] (LDS): lanes
// j < 8 read their accumulator's values a[j + 8 i] at once and add them in
// order, three DPP butterflies form ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)) (the
// same sums: float addition is commutative), the tail comes from lane reads.
// Every lane returns the sum.
FL_DEV float np_sum_wave128(const float* a, int n, int lane, float v0, float v1) {
    float res = 0.0f;
    int i0 = 0;
    if (n >= 8) {
        const int q = n >> 3;  // 8-value blocks, 1..16
        const int j = lane & 7;
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] = a[8 * i + j];
        float r = x[0];
#pragma unroll
        for (int i = 1; i < 16; ++i) r = i < q ? r + x[i] : r;
        r = r + bitcast<float>(__builtin_amdgcn_update_dpp(0, bitcast<int>(r), 0xB1, 0xF, 0xF, false));
        r = r + bitcast<float>(__builtin_amdgcn_update_dpp(0, bitcast<int>(r), 0x4E, 0xF, 0xF, false));
        r = r + bitcast<float>(__builtin_amdgcn_update_dpp(0, bitcast<int>(r), 0x141, 0xF, 0xF, false));
        res = bitcast<float>(__builtin_amdgcn_readlane(bitcast<int>(r), 0));
        i0 = 8 * q;
    }
    for (int i = i0; i < n; ++i) {
        const int l = i & 63;
        const int xv = i < 64 ? __builtin_amdgcn_readlane(bitcast<int>(v0), l)
                              : __builtin_amdgcn_readlane(bitcast<int>(v1), l);
        res += bitcast<float>(xv);
    }
    return res;
}

// ---- numpy's argpartition tie order (float32 rows of <= 256 elements)
// numpy 2.x sends a single-kth float32 argpartition on an AVX512_SKX host to
// x86-simd-sort, which fully sorts rows of <= 256 elements with a bitonic
// key/index network on 8-lane registers: pad to maxN = max(8, next power of
// two) with +inf keys and index 0; sort each 8-lane register (6 steps); merge
// registers in groups of 2, 4, .. maxN/8 (register i against register n-1-i
// read lane-reversed, half-cleaners across registers, then each register's
// 3-step in-lane merge).  A step keeps the max where the lane's mask bit is
// set, else the min, and a lane whose result equals its own key keeps its own
// index, so equal keys never trade places and ties end where the wiring puts
// them.  The selection of argpartition(keys, k-1)[:k] is the first k
// positions.  Here position x = 64 c + lane sits in slot c of the lane;
// partners come through ds_bpermute (the partner slot is uniform per slot
// and step).  Used only for rows with a tied maximum in some top-k round.
FL_DEV float bperm_f(float v, int src_lane) {
    return bitcast<float>(__builtin_amdgcn_ds_bpermute(src_lane << 2, bitcast<int>(v)));
}

// One cross-register network step over the NSL slots in use: part(c, &pc,
// &pl, &mx) gives the partner slot pc (uniform) and lane pl of this lane's
// slot-c position, mx = keep the max.  Every slot's partner reads issue
// before the first compare.
template <int NSL, typename Part>
FL_DEV void net_step(float (&kf)[4], int (&ix)[4], Part part) {
    float ok[NSL];
    int oi[NSL];
    bool mxv[NSL];
#pragma unroll
    for (int c = 0; c < NSL; ++c) {
        int pc, pl;
        bool mx;
        part(c, pc, pl, mx);
        const float sk = pc == 0 ? kf[0] : pc == 1 ? kf[1] : pc == 2 ? kf[2] : kf[3];
        const int si = pc == 0 ? ix[0] : pc == 1 ? ix[1] : pc == 2 ? ix[2] : ix[3];
        ok[c] = bperm_f(sk, pl);
        oi[c] = __builtin_amdgcn_ds_bpermute(pl << 2, si);
        mxv[c] = mx;
    }
#pragma unroll
    for (int c = 0; c < NSL; ++c) {
        const float r = mxv[c] ? fmaxf(kf[c], ok[c]) : fminf(kf[c], ok[c]);
        ix[c] = r == kf[c] ? ix[c] : oi[c];
        kf[c] = r;
    }
}

// Partners inside 8-lane registers by DPP: l ^ 1, l ^ 2, 3 - l within four,
// 7 - l (half-row mirror), l ^ 4 (a shift left or right by four inside the
// 16-lane row, picked by lane bit 2).
enum { kNetX1, kNetX2, kNetR4, kNetR8, kNetX4 };
template <int P>
FL_DEV int net_dpp(int v, int lane) {
    if constexpr (P == kNetX1) return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm 1,0,3,2
    else if constexpr (P == kNetX2) return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // quad_perm 2,3,0,1
    else if constexpr (P == kNetR4) return __builtin_amdgcn_update_dpp(0, v, 0x1B, 0xF, 0xF, false);  // quad_perm 3,2,1,0
    else if constexpr (P == kNetR8) return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);  // row_half_mirror
    else {
        const int up = __builtin_amdgcn_update_dpp(0, v, 0x104, 0xF, 0xF, false);  // row_shl:4: lane l + 4
        const int dn = __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4: lane l - 4
        return (lane & 4) ? dn : up;
    }
}

// In-register step: partner P inside each 8-lane register, max where
// `mask` has bit l % 8.
template <int NSL, int P>
FL_DEV void net_lane_step(float (&kf)[4], int (&ix)[4], int lane, int mask) {
    const bool mx = (mask >> (lane & 7)) & 1;
#pragma unroll
    for (int c = 0; c < NSL; ++c) {
        const float ok = bitcast<float>(net_dpp<P>(bitcast<int>(kf[c]), lane));
        const int oi = net_dpp<P>(ix[c], lane);
        const float r = mx ? fmaxf(kf[c], ok) : fminf(kf[c], ok);
        ix[c] = r == kf[c] ? ix[c] : oi;
        kf[c] = r;
    }
}

// Full network over maxN (8..64 NSL) positions held as described above.
template <int NSL>
FL_DEV void net_argsort(float (&kf)[4], int (&ix)[4], int maxN, int lane) {
    const int nv = maxN >> 3;
    net_lane_step<NSL, kNetX1>(kf, ix, lane, 0xAA);
    net_lane_step<NSL, kNetR4>(kf, ix, lane, 0xCC);
    net_lane_step<NSL, kNetX1>(kf, ix, lane, 0xAA);
    net_lane_step<NSL, kNetR8>(kf, ix, lane, 0xF0);
    net_lane_step<NSL, kNetX2>(kf, ix, lane, 0xCC);
    net_lane_step<NSL, kNetX1>(kf, ix, lane, 0xAA);
    const int l = lane & 7;
    for (int n = 2; n <= nv; n <<= 1) {
        // register R against register g + n - 1 - (R - g), lanes reversed
        net_step<NSL>(kf, ix, [&](int c, int& pc, int& pl, bool& mx) {
            const int R = 8 * c + (lane >> 3);
            const int g = R & ~(n - 1), a = R - g;
            const int R2 = g + n - 1 - a;
            mx = a >= (n >> 1);
            pc = R2 >> 3;
            pl = ((R2 & 7) << 3) | (7 - l);
        });
        for (int m = n >> 1; m >= 2; m >>= 1) {
            const int d = m >> 1;
            net_step<NSL>(kf, ix, [&](int c, int& pc, int& pl, bool& mx) {
                const int R = 8 * c + (lane >> 3);
                const bool hi = (R & (m - 1)) >= d;  // m: a power of two
                const int R2 = hi ? R - d : R + d;
                mx = hi;
                pc = R2 >> 3;
                pl = ((R2 & 7) << 3) | l;
            });
        }
        net_lane_step<NSL, kNetX4>(kf, ix, lane, 0xF0);
        net_lane_step<NSL, kNetX2>(kf, ix, lane, 0xCC);
        net_lane_step<NSL, kNetX1>(kf, ix, lane, 0xAA);
    }
}

// Keys -v (numpy's -select) of n <= 64 NSL values (lane + 64 c), padded to
// the network's size, sorted; returns maxN.  Inlined: called out of line it
// cost config 5's router (T = 512, 18 tied tokens) 7.6 us, and the smaller
// routing code it gave the one-token path measured no faster.
template <int NSL>
FL_DEV int net_load_sort(const float (&v)[4], int n, int lane, float (&kf)[4], int (&ix)[4]) {
    int maxN = 8;
    while (maxN < n) maxN <<= 1;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int x = lane + 64 * c;
        kf[c] = x < n ? -v[c] : __builtin_inff();
        ix[c] = x < n ? x : 0;
    }
    net_argsort<NSL>(kf, ix, maxN, lane);
    return maxN;
}

// Route token t with one wave.  `exw` is the wave's 256-float LDS row.
// Lane i < K ends with the i-th selection (expert `my_id`, final weight
// `my_w`), which it also stores to sids/sws[tl*K + i] and, when `store`, to
// topk_ids/topk_w (and scoef, rw).
// Values sit one per lane in nc <= 4 slots (expert lane + 64 c); slots past
// nc are skipped by uniform branches.  Everything stays in registers except
// the exp row of the softmax sum.  NC = route_slots(E): 1 (E <= 64) and 2
// (E <= 128) fix nc at compile time, which removes the per-slot branches and
// the E-dependent sum paths of the general (NC = 4) body.
__host__ __device__ constexpr int route_slots(int E) { return E <= 64 ? 1 : (E <= 128 ? 2 : 4); }

template <int NC>
FL_DEV void route_token(const RouteArgs& a, int t, int tl, int lane, float* exw, int* sids,
                        float* sws, int& my_id, float& my_w, bool store = true) {
    const int E = a.E, K = a.K;
    const int nc = NC < 4 ? NC : (E + 63) >> 6;
    float sel[4], p[4];
    const float* s = a.logits + (size_t)t * E;
    // the logit (and bias) loads go out together, indices clamped
    float lv[4], bv4[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int e = lane + 64 * c;
        const int ec = e < E ? e : E - 1;
        lv[c] = c < nc ? s[ec] : 0.0f;
        bv4[c] = (c < nc && a.bias) ? a.bias[ec] : 0.0f;
    }
    const float slog = (a.scoef && a.slogit) ? a.slogit[t] : 0.0f;
    if (a.scoring == 0) {
        uint32_t mk = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t k = order_key(lv[c]);
            if (c < nc && lane + 64 * c < E && k > mk) mk = k;
        }
        const float m = key_float(wave_umax(mk));
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            p[c] = 0.0f;
            if (c < nc) {
                const int e = lane + 64 * c;
                p[c] = e < E ? np_expf(lv[c] - m) : 0.0f;
                exw[e] = p[c];
            }
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        const float z = NC == 1   ? np_sum_wave64(exw, E, lane, p[0])
                        : NC == 2 ? np_sum_wave128(exw, E, lane, p[0], p[1])
                                  : np_sum_wave(exw, E, lane);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int e = lane + 64 * c;
            p[c] = (c < nc && e < E) ? p[c] / z : 0.f;
            sel[c] = (c < nc && e < E) ? p[c] : -__builtin_inff();
        }
    } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int e = lane + 64 * c;
            p[c] = 0.f;
            sel[c] = -__builtin_inff();
            if (c < nc && e < E) {
                const float d = 1.0f + np_expf(-lv[c]);
                p[c] = 1.0f / d;
                sel[c] = a.bias ? p[c] + bv4[c] : p[c] + 0.0f;
            }
        }
    }
    if (a.n_group > 1 && a.topk_group > 0 && a.topk_group < a.n_group) {
        const int gsz = E / a.n_group;
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int e = lane + 64 * c;
            if (e < E) exw[e] = sel[c];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // lane g scores group g: second largest + largest (numpy sums the
        // ascending top-2)
        float gscore = -__builtin_inff();
        if (lane < a.n_group) {
            float b1 = -__builtin_inff(), b2 = -__builtin_inff();
            for (int i = 0; i < gsz; ++i) {
                const float v = exw[lane * gsz + i];
                if (v > b1) {
                    b2 = b1;
                    b1 = v;
                } else if (v > b2) {
                    b2 = v;
                }
            }
            gscore = gsz >= 2 ? (0.0f + b2) + b1 : 0.0f + b1;
        }
        // keep topk_group groups: rank = #groups strictly better; tied
        // group scores take numpy's argpartition order (the network)
        int rank = 0, same = 0;
        for (int g2 = 0; g2 < a.n_group; ++g2) {
            const float o = __shfl(gscore, g2, 64);
            rank += (o > gscore || (o == gscore && g2 < lane)) ? 1 : 0;
            same += (o == gscore && g2 != lane) ? 1 : 0;
        }
        int keep = (lane < a.n_group && rank < a.topk_group) ? 1 : 0;
        if (__ballot(lane < a.n_group && same > 0)) {
            float gv[4] = {gscore, 0.f, 0.f, 0.f}, kf[4];
            int ix[4];
            net_load_sort<1>(gv, a.n_group, lane, kf, ix);
            unsigned long long km = 0ull;
            for (int j = 0; j < a.topk_group; ++j) km |= 1ull << __builtin_amdgcn_readlane(ix[0], j);
            keep = (lane < a.n_group && ((km >> lane) & 1ull)) ? 1 : 0;
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int e = lane + 64 * c;
            const int kg = __shfl(keep, e < E ? e / gsz : 0, 64);
            if (e < E && !kg) sel[c] = -__builtin_inff();
        }
    }
    // top-k by (value desc, index asc): K rounds of a wave-wide maximum over
    // order-preserving integer keys, the lowest expert index among equal
    // keys through a ballot; round i's pick lands in lane i.
    uint32_t key[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int e = lane + 64 * c;
        key[c] = (c < nc && e < E) ? order_key(sel[c]) : 0u;  // 0: never picked
    }
    my_id = 0;
    my_w = 0.f;
    bool tie = false;  // some round's maximum held by more than one expert
    if (NC == 1) {
        // one expert per lane (E <= 64): the same rounds without slot loops
        uint32_t k0 = key[0];
        for (int i = 0; i < K; ++i) {
            const uint32_t m = wave_umax(k0);
            const unsigned long long bm = __ballot(k0 == m);
            const int l = __builtin_ctzll(bm);
            tie |= (bm & (bm - 1ull)) != 0ull;
            const float w = bitcast<float>(__builtin_amdgcn_readlane(bitcast<int>(p[0]), l));
            k0 = lane == l ? 0u : k0;
            if (lane == i) {
                my_id = l;
                my_w = w;
            }
        }
    } else {
    for (int i = 0; i < K; ++i) {
        const uint32_t m = wave_umax(umax4(key[0], key[1], key[2], key[3]));
        int e = 0, holders = 0;
        float w = 0.f;
#pragma unroll
        for (int c = 3; c >= 0; --c) {  // the lowest slot c holding m wins
            if (c < nc) {
                const unsigned long long bm = __ballot(key[c] == m);
                holders += __builtin_popcountll(bm);
                if (bm) {
                    const int l = __builtin_ctzll(bm);
                    e = 64 * c + l;
                    w = bitcast<float>(__builtin_amdgcn_readlane(bitcast<int>(p[c]), l));
                }
            }
        }
        tie |= holders > 1;
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (lane + 64 * c == e) key[c] = 0u;
        if (lane == i) {
            my_id = e;
            my_w = w;
        }
    }
    }
    if (tie) {
        // numpy's argpartition(-select)[:K]: the set at a tied k-th value and
        // the order of tied picks (which the weight sum follows) come from
        // its network
        float kf[4];
        int ix[4];
        float sv[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) sv[c] = sel[c];
        net_load_sort<(NC < 4 ? NC : 4)>(sv, E, lane, kf, ix);
        my_id = ix[0];
        float w = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float pc = bperm_f(p[c], my_id & 63);
            if (c < nc && (my_id >> 6) == c) w = pc;
        }
        my_w = lane < K ? w : 0.f;
        if (lane >= K) my_id = 0;
    }
    if (a.norm) {
        // numpy row sum of the k weights (selection order), + 1e-20: below 8
        // a plain loop; else 8 accumulators (a second round of 8 when
        // k == 16), their tree, then the leftovers one by one
        const int wbits = bitcast<int>(my_w);
        float den;
        if (K < 8) {
            den = 0.0f;
            for (int i = 0; i < K; ++i) den += bitcast<float>(__builtin_amdgcn_readlane(wbits, i));
        } else {
            float r[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) r[j] = bitcast<float>(__builtin_amdgcn_readlane(wbits, j));
            if (K == 16) {
#pragma unroll
                for (int j = 0; j < 8; ++j) r[j] += bitcast<float>(__builtin_amdgcn_readlane(wbits, 8 + j));
            }
            den = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
            if (K < 16)
                for (int i = 8; i < K; ++i) den += bitcast<float>(__builtin_amdgcn_readlane(wbits, i));
        }
        den = den + 1e-20f;
        my_w = my_w / den;
    }
    my_w = my_w * a.scale;
    if (lane < K) {
        if (store) {  // agent-coherent: the lists may be built on another XCD
            __hip_atomic_store(a.topk_ids + (size_t)t * K + lane, my_id, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.topk_w + (size_t)t * K + lane, my_w, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
        sids[tl * K + lane] = my_id;
        sws[tl * K + lane] = my_w;
    }
    if (!store) return;
    if (lane == 0 && a.scoef && a.slogit) a.scoef[t] = 1.0f / (1.0f + expf(-slog));
    if (a.rw) {
        float w[4] = {0.f, 0.f, 0.f, 0.f};
        for (int i = 0; i < K; ++i) {
            const int id = __builtin_amdgcn_readlane(my_id, i);
            const float wi = bitcast<float>(__builtin_amdgcn_readlane(bitcast<int>(my_w), i));
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (lane + 64 * c == id) w[c] = wi;
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int e = lane + 64 * c;
            if (c < nc && e < E) a.rw[(size_t)t * E + e] = w[c];
        }
    }
}

// One token: its K picks are the K slots, ordered by expert id (the experts
// are distinct, so the ranks are too).  Returns the lane's slot.
FL_DEV int one_token_rank(int K, int my_id) {
    int rank = 0;
    for (int j = 0; j < K; ++j) rank += __builtin_amdgcn_readlane(my_id, j) < my_id ? 1 : 0;
    return rank;
}

FL_DEV void one_token_lists(const RouteArgs& a, int lane, int my_id, float my_w) {
    const int K = a.K;
    const int rank = one_token_rank(K, my_id);
    if (lane < K) {
        a.lists.active[rank] = my_id;
        a.lists.offsets[rank] = rank;
        a.lists.tok[rank] = 0;
        a.lists.tokw[rank] = my_w;
        if (lane == 0) {
            a.lists.offsets[K] = K;
            *a.lists.n_active = K;
        }
    }
}

// MoE lists for batches routed by several workgroups (entries read from the
// router's topk_ids / topk_w), one workgroup of 1024 threads.  Entries of an
// expert are its tokens in ascending order (a token's K experts are
// distinct), so entry (t, k) of expert e sits at
//   base[e] + #{t' < t : t' chose e},
// and that count is a popcount over a token bitmap sel[e] of the expert:
//   1. every thread loads its entries, counts experts (LDS atomics) and sets
//      the token bits of sel;
//   2. the first wave scans the expert counts (slot offsets, active list)
//      while the others form pc[e][w], the bits of sel[e] below word w;
//   3. every entry writes itself at base[e] + pc[e][t/32] + the popcount
//      of sel[e][t/32] below bit t%32 -- no serial walk anywhere.
// Limits: T * K <= kListIds, E * ceil(T / 32) <= kListSel.
constexpr int kListIds = 4096;
constexpr int kListSel = 4096;
// The placement of route_lists_k by NT threads of one workgroup; COHERENT:
// the picks are read with agent-coherent loads (written by other workgroups
// of the same launch, possibly on other XCDs).
template <int NT, bool COHERENT>
FL_DEV void lists_multi(const int* __restrict__ ids, const float* __restrict__ tw, int T, int K, int E,
                        MoeLists L) {
    constexpr int R = kListIds / NT;  // entries per thread
    __shared__ int cnt[256];
    __shared__ int base[256];
    __shared__ uint32_t sel[kListSel];
    __shared__ int pc[kListSel];
    const int TK = T * K;
    const int tw32 = (T + 31) >> 5;  // bitmap words per expert
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += NT) cnt[e] = 0;
    for (int i = tid; i < E * tw32; i += NT) sel[i] = 0u;
    int ev[R], tv[R];
    float wv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = tid + NT * r;
        const int ic = i < TK ? i : TK - 1;
        if (COHERENT) {
            ev[r] = __hip_atomic_load(ids + ic, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            wv[r] = __hip_atomic_load(tw + ic, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            ev[r] = ids[ic];
            wv[r] = tw[ic];
        }
        tv[r] = (int)(((float)ic + 0.5f) * (1.0f / (float)K));  // ic / K (exact: ic < 2^12)
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (tid + NT * r < TK) {
            atomicAdd(&cnt[ev[r]], 1);
            atomicOr(&sel[ev[r] * tw32 + (tv[r] >> 5)], 1u << (tv[r] & 31));
        }
    }
    __syncthreads();
    if (tid < 64) {
        int c[4], tot = 0, act = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = 4 * tid + q;
            c[q] = e < E ? cnt[e] : 0;
            tot += c[q];
            act += c[q] > 0 ? 1 : 0;
        }
        int it = tot, ia = act;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int vt = __shfl_up(it, o, 64), va = __shfl_up(ia, o, 64);
            if (tid >= o) {
                it += vt;
                ia += va;
            }
        }
        int off = it - tot, na = ia - act;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = 4 * tid + q;
            if (e < E) {
                base[e] = off;
                if (c[q] > 0) {
                    L.active[na] = e;
                    L.offsets[na] = off;
                    ++na;
                }
                off += c[q];
            }
        }
        if (tid == 63) {
            L.offsets[ia] = it;
            *L.n_active = ia;
        }
    } else {
        // pc[e][w] = popcount of sel[e][0..w): one expert per thread
        for (int e = tid - 64; e < E; e += NT - 64) {
            int run = 0;
            for (int w = 0; w < tw32; ++w) {
                pc[e * tw32 + w] = run;
                run += __popc(sel[e * tw32 + w]);
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (tid + NT * r < TK) {
            const int e = ev[r], t = tv[r], w = e * tw32 + (t >> 5);
            const int p = base[e] + pc[w] + __popc(sel[w] & ((1u << (t & 31)) - 1u));
            L.tok[p] = t;
            L.tokw[p] = wv[r];
        }
    }
}

// One wave per token; a batch of one workgroup (up to 16 tokens) also
// builds the MoE lists, larger batches take kRouteTpb tokens per workgroup
// (one wave each), so T = 512 routes on 128 CUs instead of 32 (16.5 us on 32
// workgroups of 16 waves).
constexpr int kRouteTpb = 4;
template <int NC>
__global__ __launch_bounds__(1024) void route_k(RouteArgs a) {
    __shared__ float ex[16][256];
    __shared__ int sids[16 * kMaxTopK];
    __shared__ float sws[16 * kMaxTopK];
    __shared__ int cnt[256];
    __shared__ int base[256];
    __shared__ unsigned selm[256];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rb = gridDim.x - a.xh_blocks;  // routing workgroups
    if ((int)blockIdx.x >= rb) {
        // fp16 copy of the token rows, beside the routing
        const int n8 = a.T * a.hidden / 8;
        for (int i = (blockIdx.x - rb) * blockDim.x + threadIdx.x; i < n8; i += a.xh_blocks * blockDim.x) {
            const f32x4 lo = reinterpret_cast<const f32x4*>(a.x)[2 * i];
            const f32x4 hi = reinterpret_cast<const f32x4*>(a.x)[2 * i + 1];
            f16x8 v;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                v[q] = (f16)lo[q];
                v[4 + q] = (f16)hi[q];
            }
            reinterpret_cast<f16x8*>(a.xh)[i] = v;
        }
        return;
    }
    int my_id = 0;
    float my_w = 0.f;
    const int tpb = rb > 1 ? kRouteTpb : 16;  // tokens per routing workgroup
    // every launch has a wave per token of its workgroup (tpb <= waves), so
    // a wave routes at most one token: no loop, whose preheader would take
    // every loop-invariant piece of the routing (group sizes, the tie
    // network's lane constants) ahead of the first load
    {
        const int tl = wv;
        const int t = blockIdx.x * tpb + tl;
        if (tl < tpb && t < a.T) route_token<NC>(a, t, tl, lane, ex[wv], sids, sws, my_id, my_w);
    }
    if (rb > 1 && a.arrive && a.lists.n_active) {
        // the last routing workgroup to arrive builds the lists: each wave's
        // pick stores are complete (agent-coherent), then one counter bump
        __shared__ int s_last;
        wait_vmcnt<0>();
        __syncthreads();
        if (threadIdx.x == 0)
            s_last = __hip_atomic_fetch_add(a.arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == rb - 1;
        __syncthreads();
        if (!s_last) return;
        lists_multi<64 * kRouteTpb, true>(a.topk_ids, a.topk_w, a.T, a.K, a.E, a.lists);
        if (threadIdx.x == 0) __hip_atomic_store(a.arrive, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    if (rb == 1 && a.lists.n_active) {
        if (a.T == 1) {
            one_token_lists(a, lane, my_id, my_w);
            return;
        }
        __syncthreads();
        build_lists(sids, sws, a.T, a.K, a.E, a.lists, cnt, base, selm);
    }
}

void launch_route(const RouteArgs& a, int grid, int threads, hipStream_t st) {
    switch (route_slots(a.E)) {
        case 1: hipLaunchKernelGGL(route_k<1>, dim3(grid), dim3(threads), 0, st, a); break;
        case 2: hipLaunchKernelGGL(route_k<2>, dim3(grid), dim3(threads), 0, st, a); break;
        default: hipLaunchKernelGGL(route_k<4>, dim3(grid), dim3(threads), 0, st, a); break;
    }
}

// The lists of a batch routed by several workgroups, one launch after the router.
__global__ __launch_bounds__(1024) void route_lists_k(const int* __restrict__ ids,
                                                      const float* __restrict__ tw, int T, int K,
                                                      int E, MoeLists L) {
    lists_multi<1024, false>(ids, tw, T, K, E, L);
}

// MoE lists from an explicit slot list: slot s is expert cand[s] (or s when
// cand is null); token t is routed to it with weight rw[t, expert] (dense
// weights) or coef[s, t] (per-slot weights) when that weight is nonzero.
// Slots keep the given order; slots without tokens, or whose expert is
// outside [0, E), are dropped.  T <= 16, S <= 256, one workgroup of 256.
__global__ __launch_bounds__(256) void slot_lists_k(const float* __restrict__ rw,
                                                    const float* __restrict__ coef,
                                                    const int* __restrict__ cand, int T, int E,
                                                    int S, MoeLists L) {
    __shared__ int start[256];
    const int s = threadIdx.x;
    int e = -1;
    if (s < S) {
        e = cand ? cand[s] : s;
        if (e < 0 || e >= E) e = -1;
        int c = 0;
        if (e >= 0)
            for (int t = 0; t < T; ++t) {
                const float w = coef ? coef[(size_t)s * T + t] : rw[(size_t)t * E + e];
                c += (w != 0.0f) ? 1 : 0;
            }
        start[s] = c;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int na = 0, off = 0;
        for (int q = 0; q < S; ++q) {
            const int c = start[q];
            if (c > 0) {
                L.active[na] = cand ? cand[q] : q;
                L.offsets[na] = off;
                start[q] = off;
                off += c;
                ++na;
            } else {
                start[q] = -1;
            }
        }
        L.offsets[na] = off;
        *L.n_active = na;
    }
    __syncthreads();
    if (s < S && start[s] >= 0) {
        int p = start[s];
        for (int t = 0; t < T; ++t) {
            const float w = coef ? coef[(size_t)s * T + t] : rw[(size_t)t * E + e];
            if (w != 0.0f) {
                L.tok[p] = t;
                L.tokw[p] = w;
                ++p;
            }
        }
    }
}

// Row-major e4m3 codes (rows, in_f) -> FP8 tiles (rows/16, in_f/128, 2048):
// one thread per 16 bytes; lane (c, q) of tile t, block kb takes row 16 t + c,
// k 128 kb + 32 q .. + 31.  The 128x128 block scales are not moved.
__global__ void moe_fp8_tile_repack_k(const uint8_t* __restrict__ q, uint8_t* __restrict__ qt, long rows,
                                      int in_f) {
    const int nkb = in_f / 128;
    const size_t n = (size_t)rows * in_f / 16;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        // destination piece i: block (t, kb), half h, lane l = c + 16 q
        const size_t blk = i / 128;
        const int within = (int)(i % 128), h = within >> 6, l = within & 63;
        const size_t t = blk / nkb;
        const int kb = (int)(blk % nkb), c = l & 15, qq = l >> 4;
        const size_t src = (16 * t + c) * (size_t)in_f + 128 * kb + 32 * qq + 16 * h;
        reinterpret_cast<u32x4*>(qt)[i] = *reinterpret_cast<const u32x4*>(q + src);
    }
}

// Row-major MXFP4 (codes (rows, in_f/2), e8 (rows, in_f/32)) -> tiles
// (rows/16, in_f/128, 1024) + scale words (rows/16, in_f/128, 16): lane
// (c, q)'s word j holds the codes of row 16 t + c, k 128 kb + 32 j + 8 q ..
// + 7 (row-major bytes 64 kb + 16 j + 4 q .. + 3); scale word (t, kb, c)
// holds the E8M0 bytes of blocks 4 kb .. 4 kb + 3 of that row.
__global__ void moe_mxfp4_tile_repack_k(const uint8_t* __restrict__ codes, const uint8_t* __restrict__ e8,
                                        uint8_t* __restrict__ qt, uint32_t* __restrict__ ew, long rows,
                                        int in_f) {
    const int nkb = in_f / 128;
    const size_t n = (size_t)rows * nkb * 4;  // lanes (c, q) per block: 64 per 16 rows
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const size_t blk = i / 64;
        const int l = (int)(i % 64), c = l & 15, qq = l >> 4;
        const size_t t = blk / nkb;
        const int kb = (int)(blk % nkb);
        const size_t row = 16 * t + c;
        const uint32_t* src = reinterpret_cast<const uint32_t*>(codes + row * (in_f / 2) + 64 * kb + 4 * qq);
        reinterpret_cast<u32x4*>(qt)[i] = u32x4{src[0], src[4], src[8], src[12]};
        if (qq == 0)
            ew[blk * 16 + c] = *reinterpret_cast<const uint32_t*>(e8 + row * (in_f / 32) + 4 * kb);
    }
}

// ------------------------------------------------------- fused MoE layer
// Stacked-expert tile layout (this library's device layout for the fused MoE;
// build_stacked_experts produces it from the row-major format):
//   qtile (rows/16, in/128, 1024) u8: block (R/16, kb) holds, at byte
//     16 * (c + 16 * q), the 16 row-major bytes [64 kb + 16 q, +16) of row
//     16 (R/16) + c -- what MFMA B-lane c + 16 q dequantizes -- so one wave
//     load reads a whole 1 KB block;
//   sz (rows/16, in/gs, 16) u32: scale bits | zero bits << 16 of row
//     16 (R/16) + c, group g, at [R/16][g][c].
// Rows of all experts are stacked (R = e * out + r); out % 16 == 0.
__global__ void moe_tile_repack_k(const uint8_t* __restrict__ q, const uint16_t* __restrict__ s,
                                  const uint16_t* __restrict__ z, uint8_t* __restrict__ qt,
                                  uint32_t* __restrict__ sz, long rows, int in_f, int G) {
    const long stride = (long)gridDim.x * blockDim.x;
    const int cpr = in_f / 32;  // 16-byte chunks per row
    const long nchunk = rows * cpr;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < nchunk; i += stride) {
        const long R = i / cpr;
        const int c = (int)(i - R * cpr), kb = c >> 2, kq = c & 3;
        const long dst = ((R >> 4) * (in_f / 128) + kb) * 1024 + ((R & 15) + 16 * kq) * 16;
        const u32x4 v = *reinterpret_cast<const u32x4*>(q + R * (in_f / 2) + c * 16);
        *reinterpret_cast<u32x4*>(qt + dst) =
            u32x4{gptq_word_to_tile_word(v[0]), gptq_word_to_tile_word(v[1]),
                  gptq_word_to_tile_word(v[2]), gptq_word_to_tile_word(v[3])};
    }
    const long nsz = rows * G;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < nsz; i += stride) {
        const long R = i / G;
        const int g = (int)(i - R * G);
        sz[((R >> 4) * G + g) * 16 + (R & 15)] = (uint32_t)s[i] | ((uint32_t)z[i] << 16);
    }
}

__global__ void moe_tile_unpack_k(const uint8_t* __restrict__ qt, const uint32_t* __restrict__ sz,
                                  uint8_t* __restrict__ q, uint16_t* __restrict__ s,
                                  uint16_t* __restrict__ z, long rows, int in_f, int G) {
    const long stride = (long)gridDim.x * blockDim.x;
    const int cpr = in_f / 32;
    const long nchunk = rows * cpr;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < nchunk; i += stride) {
        const long R = i / cpr;
        const int c = (int)(i - R * cpr), kb = c >> 2, kq = c & 3;
        const long src = ((R >> 4) * (in_f / 128) + kb) * 1024 + ((R & 15) + 16 * kq) * 16;
        const u32x4 v = *reinterpret_cast<const u32x4*>(qt + src);
        *reinterpret_cast<u32x4*>(q + R * (in_f / 2) + c * 16) =
            u32x4{tile_word_to_gptq_word(v[0]), tile_word_to_gptq_word(v[1]),
                  tile_word_to_gptq_word(v[2]), tile_word_to_gptq_word(v[3])};
    }
    const long nsz = rows * G;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < nsz; i += stride) {
        const long R = i / G;
        const int g = (int)(i - R * G);
        const uint32_t v = sz[((R >> 4) * G + g) * 16 + (R & 15)];
        s[i] = (uint16_t)(v & 0xFFFFu);
        z[i] = (uint16_t)(v >> 16);
    }
}

// Expert set in the tile layout, shared by the two MoE kernels.
struct MoeExperts {
    const uint8_t* gq;    // gate (E * inter / 16, hidden / 128, 1024)
    const uint32_t* gsz;  // gate (E * inter / 16, hidden / gs, 16)
    const uint8_t* uq;    // up, as gate
    const uint32_t* usz;
    const uint8_t* dq;    // down (E * hidden / 16, inter / 128, 1024)
    const uint32_t* dsz;  // down (E * hidden / 16, inter / gs, 16)
    int inter;
};

// Weight formats of the fused-MoE tiles (16 rows x 128 k per tile block):
//   INT4  -- 1 KB nibbles + per (row, group) fp16 scale|zero words (sz);
//   FP8   -- 2 KB e4m3 codes, lane (c, q) holding k 32 q .. 32 q + 31 of row
//            c; sz is the fp32 128x128-block scale array of
//            quantize_fp8_block (quantizer.py:65-85), one per (row/128, kb);
//   MXFP4 -- 1 KB E2M1 nibbles, lane (c, q)'s word j holding k 32 j + 8 q ..
//            + 7 (so MFMA step j covers MX block 4 kb + j) and sz one word
//            per (tile, kb, row) with the four E8M0 scales in bytes j.
// FP8 codes become fp16 exactly (scale-1 conversions) and the block scale
// multiplies the fp32 MFMA result; MXFP4 codes are converted with their
// block scale to fp16(code * scale) (mx_operand_scaled).
constexpr int kFmtInt4 = 0, kFmtFp8 = 1, kFmtMx4 = 2;
// Call flags of the fused MoE entries
constexpr int kMoeDeterministic = 1;  // ordered combine: bit-identical repeats
constexpr int kMoeFlags = kMoeDeterministic;

template <int FMT>
struct WBlk {  // one lane's share of a tile block
    u32x4 w;
    u32x4 w2;  // FP8: bytes 16..31
    uint32_t sz;
};

// Tile block `tile` x `kb` of a matrix (q, sz) with nkb 128-k blocks per row
// tile; INT4 group index g of this lane (G groups per row).
template <int FMT>
FL_DEV WBlk<FMT> wblk_load(const uint8_t* q, const uint32_t* sz, size_t tile, int nkb, int kb, int g,
                           int G, int lane, int col) {
    WBlk<FMT> b;
    const size_t blk = tile * nkb + kb;
    if (FMT == kFmtFp8) {
        // the lane's two 16-byte halves, 1 KB apart: each load reads whole lines
        const u32x4* p = reinterpret_cast<const u32x4*>(q + blk * 2048 + lane * 16);
        b.w = __builtin_nontemporal_load(p);
        b.w2 = __builtin_nontemporal_load(p + 64);
        b.sz = sz[(tile >> 3) * nkb + kb];  // fp32 bits of the 128x128 block scale
    } else {
        b.w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(q + blk * 1024 + lane * 16));
        b.sz = FMT == kFmtMx4 ? sz[blk * 16 + col] : sz[(tile * G + g) * 16 + col];
    }
    return b;
}

// fp16 pair of e4m3 bytes (hi: bytes 2, 3 of w, else 0, 1), exact
FL_DEV uint32_t fp8x2_f16(uint32_t w, bool hi) {
    return hi ? bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true))
              : bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
}

// fp16 pair of the E2M1 nibbles of byte `bs` of w (low nibble first), exact
template <int BS>
FL_DEV uint32_t fp4x2_f16(uint32_t w) {
    return bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, BS));
}

// 2^(e - 127) for an E8M0 byte (e = 0 gives 2^-127, a subnormal fp32)
FL_DEV float e8m0_float(uint32_t e) { return e ? __uint_as_float(e << 23) : __uint_as_float(0x00400000u); }

// MFMA step j's fp16 B operand of an FP8 / MXFP4 tile block (exact codes)
template <int FMT>
FL_DEV f16x8 wblk_operand(const WBlk<FMT>& b, int j) {
    if (FMT == kFmtFp8) {
        const uint32_t lo = j < 2 ? b.w[2 * j] : b.w2[2 * j - 4];
        const uint32_t hi = j < 2 ? b.w[2 * j + 1] : b.w2[2 * j - 3];
        return bitcast<f16x8>(u32x4{fp8x2_f16(lo, false), fp8x2_f16(lo, true), fp8x2_f16(hi, false),
                                    fp8x2_f16(hi, true)});
    }
    const uint32_t w = b.w[j];
    return bitcast<f16x8>(u32x4{fp4x2_f16<0>(w), fp4x2_f16<1>(w), fp4x2_f16<2>(w), fp4x2_f16<3>(w)});
}

// MXFP4: the scale of MFMA step j (the E8M0 byte j of the lane's column)
FL_DEV float mx_step_scale(uint32_t sz, int j) { return e8m0_float((sz >> (8 * j)) & 0xFFu); }
// MFMA operand of MXFP4 step j: fp16(code * s) of the 8 E2M1 codes of word
// w, the scale applied by the conversion itself (exact while code * s is an
// fp16 normal, i.e. for block scales from 2^-14 up; below, rounded), so the
// four steps of a tile block chain in one accumulator with no fp32 rescale
// (config 5 with MXFP4 experts 134.5 -> 120.7 us against exact codes scaled
// in fp32)
FL_DEV f16x8 mx_operand_scaled(uint32_t w, float s) {
    return bitcast<f16x8>(u32x4{bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 0)),
                                bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 1)),
                                bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 2)),
                                bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 3))});
}

// acc += live * (tile block of weights) x (activation fragments a[j]): a[j]
// is MFMA step j's A operand (k 32 q + 8 j for INT4 / FP8, 32 j + 8 q for
// MXFP4, q the lane's quarter).
template <int FMT, bool G128>
FL_DEV void wblk_mma(f32x4& acc, const u32x4 (&a)[4], const WBlk<FMT>& b, float live) {
    if (FMT == kFmtInt4) {
        tile_block_mma<G128>(acc, a, b.w, (uint16_t)(b.sz & 0xFFFFu), (uint16_t)(b.sz >> 16), live);
    } else if (FMT == kFmtFp8) {
        f32x4 part = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) part = mfma_f16(bitcast<f16x8>(a[j]), wblk_operand(b, j), part);
        const float s = __uint_as_float(b.sz) * live;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(s, part[e], acc[e]);
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc = mfma_f16(bitcast<f16x8>(a[j]), mx_operand_scaled(b.w[j], mx_step_scale(b.sz, j) * live), acc);
    }
}

// activation offset (halves, within a 128-k block) of MFMA step j for lane quarter q
template <int FMT>
FL_DEV int a_koff(int q, int j) { return FMT == kFmtMx4 ? 32 * j + 8 * q : 32 * q + 8 * j; }

// inter_buf (caller workspace) fp16 [max_entries + T][inter_pad] holds
// silu(g) * u * w per list entry and, from row max_entries, per token of the
// shared expert.  y is zeroed by the gate/up kernel and accumulated by the
// down kernel with fp32 atomics.
struct MoeArgs {
    const float* x;  // (T, hidden) fp32
    int T, hidden, gs, E;
    MoeExperts routed, shared;
    int has_shared, pieces;  // shared-expert down projection split into `pieces` K ranges
    const float* scoef;      // shared-expert per-token coefficient (T), or null (1.0)
    const int* n_active;
    const int* active;
    const int* offsets;
    const int* tok;
    const float* tokw;
    int max_slots, max_entries, inter_pad;
    uint16_t* inter_buf;
    const uint16_t* xh;  // (T, hidden) fp16 copy of x (grouped kernels; decode kernels for T > 4)
    int xh_ready;        // xh already written (by the router) before the launch
    float* y;  // (T, hidden) fp32
    // T == 1 with routing: every routed gate/up workgroup routes the token
    // itself (no router launch before it); workgroup 0 stores the router
    // outputs and the lists the down kernel reads
    int fuse_route;
    RouteArgs ra;
    int fmt;  // weight format of both expert stacks (kFmt*)
    // deterministic combine: the down projections store their terms into
    // `part` (rows [0, max_entries): list entry p; row max_entries + q T + t:
    // shared-expert piece q of token t) and moe_combine_k sums them per
    // token in one fixed order, instead of fp32 atomics into y
    int det, nq;
    float* part;
};

// Fused routing of the one token (T == 1) in a routed gate/up workgroup:
// wave 0 routes it, workgroup 0 also stores the router outputs and lists;
// returns the expert of slot `slot` (the slot-th smallest of the K picks) and
// its combine weight to every thread.
FL_DEV void fused_route_slot(const RouteArgs& r, int slot, bool store, int& e, float& w) {
    __shared__ float exw[256];
    __shared__ int sids[kMaxTopK];
    __shared__ float sws[kMaxTopK];
    __shared__ int s_e;
    __shared__ float s_w;
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        int my_id = 0;
        float my_w = 0.f;
        switch (route_slots(r.E)) {
            case 1: route_token<1>(r, 0, 0, lane, exw, sids, sws, my_id, my_w, store); break;
            case 2: route_token<2>(r, 0, 0, lane, exw, sids, sws, my_id, my_w, store); break;
            default: route_token<4>(r, 0, 0, lane, exw, sids, sws, my_id, my_w, store); break;
        }
        const int rank = one_token_rank(r.K, my_id);
        if (lane < r.K && rank == slot) {
            s_e = my_id;
            s_w = my_w;
        }
        if (store) one_token_lists(r, lane, my_id, my_w);
    }
    __syncthreads();
    e = s_e;
    w = s_w;
}

// 16-row tiles of gate and of up per gate/up workgroup: one for up to
// kGuOwnT tokens (more, smaller workgroups: one generation of them covers
// the chip), four above (fewer, larger ones: more bytes per dispatch).
constexpr int gu_tiles(int T) { return T <= 4 ? 1 : 4; }
constexpr int kGuOwnT = 4;    // up to this many tokens each wave stages its own activations

FL_DEV int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// Slot `slot` of the lists: expert, first entry and entry count (clamped to
// the workspace); false when the slot is at or past n_active.  The four index
// loads issue together.
FL_DEV bool moe_slot(const MoeArgs& a, int slot, int& e, int& row0, int& M) {
    const int na = __builtin_amdgcn_readfirstlane(*a.n_active);
    const int ee = __builtin_amdgcn_readfirstlane(a.active[slot]);
    const int r0 = __builtin_amdgcn_readfirstlane(a.offsets[slot]);
    const int r1 = __builtin_amdgcn_readfirstlane(a.offsets[slot + 1]);
    if (slot >= clampi(na, 0, a.max_slots)) return false;
    e = clampi(ee, 0, a.E - 1);
    row0 = clampi(r0, 0, a.max_entries);
    const int end = clampi(r1, row0, a.max_entries);
    M = end - row0 < a.T ? end - row0 : a.T;
    return true;
}

// 128-k block handled by wave `wave` at step i.  With an even NB a wave takes
// adjacent block pairs; blocks [0, nwaves * NB) are covered once either way.
template <int NB>
FL_DEV int moe_kb(int wave, int i, int nwaves) {
    return (NB % 2 == 0) ? 2 * (wave + (i >> 1) * nwaves) + (i & 1) : wave + i * nwaves;
}

FL_DEV uint16_t sz_scale(uint32_t v) { return (uint16_t)(v & 0xFFFFu); }
FL_DEV uint16_t sz_zero(uint32_t v) { return (uint16_t)(v >> 16); }

// gate/up for TR 16-row tiles of one slot's expert over only the tokens
// routed to it: h = silu(x Wg^T) * (x Wu^T) * w, stored fp16 in inter_buf.
// The waves split the hidden (K) blocks, NB each; every weight load of a wave
// (one 1 KB block per load) is issued before the token rows are gathered
// into LDS.  Workgroup 0 also zeroes y for the down kernel's accumulation.
template <int FMT, bool G128, int NB, int TR>
__global__ __launch_bounds__(512) void moe_gate_up_k(MoeArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int nwaves = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kq = lane >> 4;
    const int K = a.hidden;
    const int nfull = K >> 7;
    // Every wave stages all T token rows of its own blocks in its own LDS
    // slot (NB blocks x Tp rows x 128 halves, Tp = T rounded up to 4) and
    // reads them back without a workgroup barrier:
    //   T <= 4: fp32 rows loaded first of all into registers (they depend on
    //     nothing), converted and stored once the weight loads are out;
    //   T > 4: copies global -> LDS (buffer_load ... lds) of the fp16 rows
    //     of xh, issued right before the weight loads and waited for with a
    //     vmcnt that leaves the weight loads in flight.
    // Either way a block's MFMAs wait only for that block's weights.
    const bool own = a.T <= kGuOwnT;
    const int Tp = (a.T + 3) & ~3;
    f32x4 xs[NB][2];
    if (own) {
        const int m = (lane >> 4) < a.T ? (lane >> 4) : a.T - 1;
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            int kb = moe_kb<NB>(wave, i, nwaves);
            kb = kb < nfull ? kb : nfull - 1;
            const float* src = a.x + (size_t)m * K + kb * 128 + 8 * (lane & 15);
            xs[i][0] = *reinterpret_cast<const f32x4*>(src);
            xs[i][1] = *reinterpret_cast<const f32x4*>(src + 4);
        }
    }

    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i < a.T * a.hidden / 4; i += blockDim.x)
            reinterpret_cast<f32x4*>(a.y)[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Order of the grid (the hardware dispatches workgroups in index order):
    // with the lists given, shared-expert workgroups first -- they depend on
    // nothing and stream while the routed ones read their lists (T = 16:
    // 60.8 -> 57.6 us per layer); with the routing fused (one token), the
    // routed workgroups first, so their routing overlaps the shared stream
    // (shared first measured 17.1 against 16.0 us)
    const int groups_r = a.routed.inter / (16 * TR);
    const int n_r = a.max_slots * groups_r;
    const int n_sh = a.has_shared ? a.shared.inter / (16 * TR) : 0;
    int slot, grp, e = 0, M = 0, row0 = 0;
    float fw = 0.f;  // fused routing: the slot's combine weight
    const MoeExperts* ex;
    const int b = blockIdx.x;
    const bool routed = a.fuse_route ? b < n_r : b >= n_sh;
    if (routed) {
        const int br = a.fuse_route ? b : b - n_sh;
        slot = br / groups_r;
        grp = br - slot * groups_r;
        if (a.fuse_route) {
            fused_route_slot(a.ra, slot, br == 0, e, fw);
            e = clampi(e, 0, a.E - 1);
            row0 = slot;
            M = 1;
        } else if (!moe_slot(a, slot, e, row0, M)) {
            return;
        }
        ex = &a.routed;
    } else {
        slot = -1;
        grp = a.fuse_route ? b - n_r : b;
        row0 = a.max_entries;
        M = a.T;
        ex = &a.shared;
    }
    if (M <= 0) return;
    const int G = K / a.gs;
    const size_t tb0 = (size_t)e * (ex->inter / 16) + (size_t)grp * TR;  // first row tile
    unsigned char* oslot = smem + (size_t)wave * NB * Tp * 256;
    if (!own) {
        // lane l copies 16 B piece l % 16 of row m0 + l / 16 (rows past T
        // repeat row T - 1 into the padding)
        const __amdgpu_buffer_rsrc_t rX = buf_rsrc(a.xh, (uint32_t)a.T * K * 2);
        const int rq = lane >> 4;
        const uint32_t po = 16u * (lane & 15);
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            int kb = moe_kb<NB>(wave, i, nwaves);
            kb = kb < nfull ? kb : nfull - 1;
            for (int m0 = 0; m0 < a.T; m0 += 4) {
                const int m = m0 + rq < a.T ? m0 + rq : a.T - 1;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rX, (lptr_t)(oslot + ((size_t)i * Tp + m0) * 256), 16,
                                                         2u * ((uint32_t)m * K + kb * 128) + po, 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // the copies go out before the weight loads
    }
    // the token of this lane's MFMA row and the entry weights, loaded now so
    // neither waits at the end
    const int jr = col < M ? col : M - 1;
    const int tok_r = (slot >= 0 && !a.fuse_route) ? clampi(a.tok[row0 + jr], 0, a.T - 1) : jr;
    const int jw = (int)threadIdx.x < M ? (int)threadIdx.x : 0;
    float wpre;
    if (slot >= 0)
        wpre = a.fuse_route ? fw : a.tokw[row0 + jw];
    else if (a.fuse_route)  // the router has not stored scoef yet: sigmoid of the shared logit here
        wpre = (a.scoef && a.ra.slogit) ? 1.0f / (1.0f + expf(-a.ra.slogit[jw])) : 1.0f;
    else
        wpre = a.scoef ? a.scoef[jw] : 1.0f;

    WBlk<FMT> wg[NB][TR], wu[NB][TR];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        int kb = moe_kb<NB>(wave, i, nwaves);
        kb = kb < nfull ? kb : nfull - 1;
        const int g = (kb * 128 + 32 * kq) / a.gs;
#pragma unroll
        for (int r = 0; r < TR; ++r) {
            wg[i][r] = wblk_load<FMT>(ex->gq, ex->gsz, tb0 + r, nfull, kb, g, G, lane, col);
            wu[i][r] = wblk_load<FMT>(ex->uq, ex->usz, tb0 + r, nfull, kb, g, G, lane, col);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (own) {
        if ((lane >> 4) < a.T) {
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                f16x8 v;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    v[q] = (f16)xs[i][0][q];
                    v[4 + q] = (f16)xs[i][1][q];
                }
                *reinterpret_cast<f16x8*>(oslot + ((size_t)i * Tp + (lane >> 4)) * 256 + 16 * (lane & 15)) = v;
            }
        }
    } else {
        // the copies went out before this wave's weight loads (wg, wu: 2 per
        // tile and block, 4 for FP8; the scale words only make the wait
        // stricter)
        constexpr int WL = NB * TR * (FMT == kFmtFp8 ? 4 : 2);
        wait_vmcnt<(WL < 63 ? WL : 63)>();
    }

    f32x4 acc[2 * TR];
#pragma unroll
    for (int r = 0; r < 2 * TR; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        int kb = moe_kb<NB>(wave, i, nwaves);
        const float live = kb < nfull ? 1.0f : 0.0f;
        kb = kb < nfull ? kb : nfull - 1;
        u32x4 av[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            av[j] = *reinterpret_cast<const u32x4*>(oslot + ((size_t)i * Tp + tok_r) * 256 + 2 * a_koff<FMT>(kq, j));
#pragma unroll
        for (int r = 0; r < TR; ++r) {
            wblk_mma<FMT, G128>(acc[2 * r], av, wg[i][r], live);
            wblk_mma<FMT, G128>(acc[2 * r + 1], av, wu[i][r], live);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();  // the token rows are dead: the reduction reuses their LDS

    // reduce the 2*TR tiles over the waves, then h = silu(g) * u * w
    float* red = reinterpret_cast<float*>(smem);
    const size_t red_bytes = (size_t)nwaves * 2 * TR * 1024;
    const size_t as_bytes = (size_t)nwaves * NB * Tp * 256;
    float* gu = reinterpret_cast<float*>(smem + (red_bytes > as_bytes ? red_bytes : as_bytes));
    float* wsm = gu + 2 * TR * 256;
    if ((int)threadIdx.x < M) wsm[threadIdx.x] = wpre;
    reduce_and_store<2 * TR>(red, acc, M, wave, nwaves, lane,
                             [&](int m, int t, int c, float v) { gu[t * 256 + m * 16 + c] = v; });
    __syncthreads();
    for (int idx = threadIdx.x; idx < TR * M * 16; idx += blockDim.x) {
        const int r = idx / (16 * M), rem = idx - r * (16 * M);
        const int m = rem >> 4, c = rem & 15;
        const float g = gu[(2 * r) * 256 + m * 16 + c];
        const float u = gu[(2 * r + 1) * 256 + m * 16 + c];
        const float h = (g / (1.0f + expf(-g))) * u * wsm[m];
        a.inter_buf[(size_t)(row0 + m) * a.inter_pad + (grp * TR + r) * 16 + c] =
            bitcast<uint16_t>((f16)h);
    }
}

// Down projection of one slot (blockIdx.y < max_slots) or one K piece of the
// shared expert (blockIdx.y - max_slots) for TRD 16-row output tiles
// (blockIdx.x), over that slot's entries; results are added to y[token] with
// fp32 atomics (like the reference's moew_down), so the summation order of
// a token's terms varies between calls.
template <int FMT, bool G128, int NB, int TRD>
__global__ __launch_bounds__(512) void moe_down_k(MoeArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int toks[16];
    constexpr int W = 16 * TRD;  // output columns per workgroup
    const int nwaves = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kq = lane >> 4;
    // shared-expert pieces first (rows y < pieces) with the lists given, as
    // in the gate/up grid; last with the routing fused
    const int npc = a.has_shared ? a.pieces : 0;
    const int yb = (int)blockIdx.y;
    const bool is_shared = a.fuse_route ? yb >= a.max_slots : yb < npc;
    const int y_slot = a.fuse_route ? yb : (is_shared ? a.max_slots + yb : yb - npc);
    const int o0 = blockIdx.x * W;

    int e = 0, row0 = 0, M = 0, kb0, nfull;
    const MoeExperts* ex;
    if (!is_shared) {
        if (!moe_slot(a, y_slot, e, row0, M)) return;
        ex = &a.routed;
        kb0 = 0;
        nfull = ex->inter >> 7;
    } else {
        const int p = y_slot - a.max_slots;
        row0 = a.max_entries;
        M = a.T;
        ex = &a.shared;
        kb0 = p * nwaves * NB;
        const int left = (ex->inter >> 7) - kb0;
        nfull = left < nwaves * NB ? left : nwaves * NB;
    }
    if (M <= 0 || nfull <= 0) return;
    const int inter = ex->inter;
    const int nkb = inter >> 7;  // 128-k blocks per row of the expert
    const int G = inter / a.gs;
    const int mrow = col < M ? col : M - 1;
    const uint16_t* arow = a.inter_buf + (size_t)(row0 + mrow) * a.inter_pad;
    const size_t tb0 = (size_t)e * (a.hidden / 16) + o0 / 16;  // first row tile
    if (threadIdx.x < 16)
        toks[threadIdx.x] = is_shared ? threadIdx.x
                                      : clampi(a.tok[row0 + (threadIdx.x < M ? threadIdx.x : 0)], 0, a.T - 1);

    u32x4 av[NB][4];
    WBlk<FMT> wv[NB][TRD];
    // activations first (L2 hits), then weights (HBM): loads retire in
    // issue order, so each block then waits only for its own weights
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        int kb = moe_kb<NB>(wave, i, nwaves);
        kb = kb0 + (kb < nfull ? kb : nfull - 1);
#pragma unroll
        for (int j = 0; j < 4; ++j) av[i][j] = *reinterpret_cast<const u32x4*>(arow + kb * 128 + a_koff<FMT>(kq, j));
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        int kb = moe_kb<NB>(wave, i, nwaves);
        kb = kb0 + (kb < nfull ? kb : nfull - 1);
        const int g = (kb * 128 + 32 * kq) / a.gs;
#pragma unroll
        for (int r = 0; r < TRD; ++r) wv[i][r] = wblk_load<FMT>(ex->dq, ex->dsz, tb0 + r, nkb, kb, g, G, lane, col);
    }
    __builtin_amdgcn_sched_barrier(0);
    f32x4 acc[TRD];
#pragma unroll
    for (int r = 0; r < TRD; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const float live = moe_kb<NB>(wave, i, nwaves) < nfull ? 1.0f : 0.0f;
#pragma unroll
        for (int r = 0; r < TRD; ++r) wblk_mma<FMT, G128>(acc[r], av[i], wv[i][r], live);
        __builtin_amdgcn_sched_barrier(0);
    }
    float* red = reinterpret_cast<float*>(smem);
    if (a.det) {
        float* dst = a.part + (size_t)(is_shared ? a.max_entries + (y_slot - a.max_slots) * a.T : row0) * a.hidden + o0;
        reduce_and_store<TRD>(red, acc, M, wave, nwaves, lane, [&](int m, int t, int c, float v) {
            dst[(size_t)m * a.hidden + 16 * t + c] = v;
        });
    } else {
        reduce_and_store<TRD>(red, acc, M, wave, nwaves, lane, [&](int m, int t, int c, float v) {
            unsafeAtomicAdd(&a.y[(size_t)toks[m] * a.hidden + o0 + 16 * t + c], v);
        });
    }
}

// ---- dense MXFP4 GEMV / small-M GEMM
// C[M, N] = A[M, K] @ dequant(W)^T, W in the MXFP4 tile layout of the MoE
// experts (one expert: qtile [N/16, K/128, 1KB], e8w [N/16, K/128, 16]).
// Workgroup (bx, by): TR 16-row tiles of W (bx) against the 16 rows of A
// from 16 by; its waves split the K blocks, NB each (moe_kb), every lane
// loading its activation fragments (L2 hits) and then its weight blocks, so
// each block waits only for its own weights; the four MX blocks of a 128-k
// block chain their MFMAs on fp16(code * scale), like the MoE kernels; the
// waves' partials are summed in wave order (deterministic) and stored as
// fp16.
template <int NB, int TR, int PH, int RS>
__global__ __launch_bounds__(1024) void mx4_gemv_k(const uint16_t* __restrict__ A, const uint8_t* __restrict__ q,
                                                   const uint32_t* __restrict__ e8w, uint16_t* __restrict__ C,
                                                   int M, int N, int K) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int nwaves = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kq = lane >> 4;
    const int nkb = K >> 7;
    const int m0 = blockIdx.y * 16;
    const int Mc = M - m0 < 16 ? M - m0 : 16;
    const uint16_t* arow = A + (size_t)(m0 + (col < Mc ? col : Mc - 1)) * K;
    const size_t t0 = (size_t)blockIdx.x * TR;  // first 16-row tile of W
    // RS = 4, 8 or 16 (the rows of A rounded up): each wave first copies RS
    // activation rows of its blocks into its own LDS slots as whole 256-byte rows
    // (block i: [row][256 B], the 16-byte k chunks of row r XOR-swizzled by
    // r, so the rows of an MFMA operand read hit distinct bank groups), four
    // rows per copy, issued before its weight loads and waited for with a
    // count that leaves those in flight; no barrier (only the wave reads its
    // slots).  With RS < 16 the lanes of MFMA rows RS..15 read rows 0..RS-1
    // again (their outputs are not stored).  RS = 0 (the two-phase long-K
    // shape, whose slots do not fit): register fragments, which load every
    // activation byte once per lane quarter that uses it.
    constexpr bool LDSA = RS > 0;
    constexpr int SB = RS * 256;  // slot bytes per block
    unsigned char* aslot = smem + (size_t)wave * NB * SB;
    const size_t abytes = LDSA ? (size_t)nwaves * NB * SB : 0;
    f32x4 acc[TR];
#pragma unroll
    for (int r = 0; r < TR; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    // PH phases of NB blocks (the 128-VGPR budget of 16-wave workgroups
    // holds the registers of up to four blocks at once)
#pragma unroll
    for (int ph = 0; ph < PH; ++ph) {
        u32x4 av[NB][4];
        WBlk<kFmtMx4> wv[NB][TR];
        if (LDSA) {
            const i32x4_t rA = raw_rsrc(A + (size_t)m0 * K, (uint32_t)Mc * (uint32_t)K * 2u);
            const uint32_t lds = (uint32_t)(uintptr_t)aslot;
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                int kb = moe_kb<NB * PH>(wave, ph * NB + i, nwaves);
                kb = kb < nkb ? kb : nkb - 1;
#pragma unroll
                for (int p = 0; p < RS / 4; ++p) {
                    const int r = 4 * p + (lane >> 4);
                    const int m = r < Mc ? r : Mc - 1;
                    lds_copy(rA, lds + (uint32_t)(i * SB + p * 1024),
                             2u * (uint32_t)m * (uint32_t)K + 16u * (uint32_t)((lane & 15) ^ r), (uint32_t)kb * 256u);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                int kb = moe_kb<NB * PH>(wave, ph * NB + i, nwaves);
                kb = kb < nkb ? kb : nkb - 1;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    av[i][j] = *reinterpret_cast<const u32x4*>(arow + kb * 128 + a_koff<kFmtMx4>(kq, j));
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            int kb = moe_kb<NB * PH>(wave, ph * NB + i, nwaves);
            kb = kb < nkb ? kb : nkb - 1;
#pragma unroll
            for (int r = 0; r < TR; ++r) wv[i][r] = wblk_load<kFmtMx4>(q, e8w, t0 + r, nkb, kb, 0, 0, lane, col);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (LDSA) {
            // the copies are older than the NB * TR 16-byte weight loads
            // (and their scale words): done once at most that many are left
            wait_vmcnt<(NB * TR < 63 ? NB * TR : 63)>();
            asm volatile("" ::: "memory");  // no LDS read moves above the wait
#pragma unroll
            for (int i = 0; i < NB; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    av[i][j] = *reinterpret_cast<const u32x4*>(aslot + i * SB + (col & (RS - 1)) * 256 +
                                                               16 * ((4 * j + kq) ^ (col & (RS - 1))));
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const float live = moe_kb<NB * PH>(wave, ph * NB + i, nwaves) < nkb ? 1.0f : 0.0f;
#pragma unroll
            for (int r = 0; r < TR; ++r) wblk_mma<kFmtMx4, true>(acc[r], av[i], wv[i][r], live);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    reduce_and_store<TR>(reinterpret_cast<float*>(smem + abytes), acc, Mc, wave, nwaves, lane,
                         [&](int m, int t, int c, float v) {
                             C[(size_t)(m0 + m) * N + (t0 + t) * 16 + c] = bitcast<uint16_t>((f16)v);
                         });
}

// Dense MXFP4 prefill GEMM (M > 64) on the matrix cores.  Workgroup tile 64
// (m) x 256 (n), eight waves side by side along n, each 64 x 32 (4 m-tiles x
// 2 n-tiles of 16 x 16 fp32 accumulators); the 128-k blocks stream through
// two LDS stages by buffer_load ... lds copies (one block in flight while
// the other is computed, one vmcnt wait and one barrier per block).  A
// stage holds, for one 128-k block:
//   * A (16 KB): the 64 x 128 fp16 rows, 256 B per row, the 16-byte k
//     chunks of row r XOR-swizzled by r % 16 (conflict-free MFMA reads);
//   * B (16 KB): the strip's 16 tile blocks as they lie (1 KB each);
//   * E (1 KB): the strip's 16 tiles' e8w words for the block (64 B each).
// MFMA step j of a block covers MX block 4 kb + j: the lane's word j of its
// tile block is converted with the block's scale in the conversion itself
// (v_cvt_scalef32_pk_f16_fp4: fp16(code * 2^(e - 127)), exact while that
// value is an fp16 normal, i.e. for scales from 2^-14 up -- weights below
// ~1e-4 in magnitude round), and the four steps of a block accumulate in
// one MFMA chain per tile.  Rows >=
// M read row M - 1 and are not stored; n-tiles >= N / 16 read the last
// n-tile and are not stored.  Workgroup order as the INT4 GEMM: the tiles of
// one XCD are a contiguous (n-block major, m-block minor) run.
constexpr int kMxBM = 64, kMxBN = 256;
constexpr int kMxStA = 0, kMxStB = 16384, kMxStE = 32768, kMxStage = kMxStE + 1024;

__global__ __launch_bounds__(512) void mx4_gemm_mfma(const f16* __restrict__ A, const uint8_t* __restrict__ Wq,
                                                     const uint32_t* __restrict__ E, f16* __restrict__ C, int M,
                                                     int N, int K) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kq = lane >> 4;
    const int nkb = K >> 7;
    const int ntiles = N >> 4;
    const int nblk = (N + kMxBN - 1) / kMxBN, mblk = (M + kMxBM - 1) / kMxBM;
    const int total = nblk * mblk;
    int lin = blockIdx.x;
    if ((total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);
    const int nb_i = lin / mblk, mb_i = lin - nb_i * mblk;
    const int m0 = mb_i * kMxBM;
    const int nt_base = nb_i * 16;

    const i32x4_t rA = raw_rsrc(A, (uint32_t)M * K * 2);
    const i32x4_t rW = raw_rsrc(Wq, (uint32_t)ntiles * nkb * 1024);
    const i32x4_t rE = raw_rsrc(E, (uint32_t)ntiles * nkb * 64);
    const uint32_t lds0 = (uint32_t)(uintptr_t)smem;

    // copy sources of this wave: A rows 4 q .. 4 q + 3 (q = 2 wave + i) as
    // whole 256-byte rows, lane l of a copy landing at row 4 q + l / 16,
    // position l % 16 with the row's k chunk (l % 16) ^ (row % 16); B tiles
    // 2 wave + i of the strip; wave 0 also the strip's E words (lane l: tile
    // l / 4, 16 bytes (l % 4) of its 64).
    uint32_t ao[2], bo[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = 4 * (wave * 2 + i) + (lane >> 4);
        int m = m0 + r;
        m = m < M ? m : M - 1;
        ao[i] = 2u * ((uint32_t)m * K) + 16u * ((lane & 15) ^ (r & 15));
        int nt = nt_base + wave * 2 + i;
        nt = nt < ntiles ? nt : ntiles - 1;
        bo[i] = (uint32_t)nt * (uint32_t)nkb * 1024u + lane * 16;
    }
    int et = nt_base + (lane >> 2);
    et = et < ntiles ? et : ntiles - 1;
    const uint32_t eo = (uint32_t)et * (uint32_t)nkb * 64u + 16u * (lane & 3);

    auto issue = [&](int kb, int slot) {
        const uint32_t st = lds0 + (uint32_t)slot * kMxStage;
#pragma unroll
        for (int i = 0; i < 2; ++i) lds_copy(rA, st + kMxStA + (wave * 2 + i) * 1024, ao[i], kb * 256);
#pragma unroll
        for (int i = 0; i < 2; ++i) lds_copy(rW, st + kMxStB + (wave * 2 + i) * 1024, bo[i], kb * 1024);
        if (wave == 0) lds_copy(rE, st + kMxStE, eo, kb * 64);
    };

    f32x4 acc[4][2];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    issue(0, 0);
    // A operand of m-tile mt, step j for lane (col, kq): row 16 mt + col, k
    // chunk 4 j + kq (k 32 j + 8 kq, the MX tile's order), stored at
    // position (4 j + kq) ^ col of that row
    const int afrag = kMxStA + col * 256 + 16 * (kq ^ (col & 3));
    const int ajx = col >> 2;
    for (int kb = 0; kb < nkb; ++kb) {
        const int u = kb & 1;
        wait_vmcnt<0>();  // this wave's copies of block kb have landed
        lds_barrier();    // ... and every wave's; block kb - 1's stage is free
        if (kb + 1 < nkb) issue(kb + 1, u ^ 1);
        const unsigned char* st = smem + (size_t)u * kMxStage;
        u32x4 wv[2];
        uint32_t ew[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            wv[t] = *reinterpret_cast<const u32x4*>(st + kMxStB + (wave * 2 + t) * 1024 + lane * 16);
            ew[t] = *reinterpret_cast<const uint32_t*>(st + kMxStE + (wave * 2 + t) * 64 + col * 4);
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
                    a[(j + 1) & 1][mt] = *reinterpret_cast<const f16x8*>(as + mt * 4096 + 64 * ((j + 1) ^ ajx));
            }
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const float s = e8m0_float((ew[t] >> (8 * j)) & 0xFFu);
                const uint32_t w = wv[t][j];
                const f16x8 b = bitcast<f16x8>(u32x4{
                    bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 0)),
                    bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 1)),
                    bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 2)),
                    bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 3))});
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) acc[mt][t] = mfma_f16(a[j & 1][mt], b, acc[mt][t]);
            }
        }
    }
    wait_vmcnt<0>();  // no copy may still be in flight when the workgroup ends

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
constexpr size_t kMxGemmLds = 2 * (size_t)kMxStage;
constexpr int kMxGemmMinM = 64;  // M above this takes the MFMA GEMM

// Launch shape of mx4_gemv_k: blocks per wave so that at most 16 waves cover
// K (1, 2 or 4 in one phase, 6 in two phases of 3), two tiles per workgroup
// from 384 tiles on (never with the two-phase blocks).  Measured at the
// Qwen3-8B shapes, M = 1 (us): qkv 6144x4096 two tiles, 16 waves of two
// blocks 5.3 (one tile 6.0); gate_up 24576x4096 8 waves of four blocks 11.9
// (16 of two 12.8); o 4096x4096 one tile, 16 waves of two 4.4.
struct Mx4Cfg {
    int nb, waves, tr;
};
Mx4Cfg mx4_cfg(int N, int K) {
    const int nkb = K / 128, tiles = N / 16;
    Mx4Cfg c;
    c.nb = nkb <= 16 ? 1 : (nkb <= 32 ? (tiles >= 1024 ? 4 : 2) : (nkb <= 64 ? 4 : 6));
    c.waves = (nkb + c.nb - 1) / c.nb;
    c.tr = (c.nb <= 4 && tiles >= 384 && tiles % 2 == 0) ? 2 : 1;
    return c;
}

template <int NB, int TR, int PH>
void launch_mx4_gemv(const Mx4Cfg& c, const uint16_t* A, const uint8_t* q, const uint32_t* e8w, uint16_t* C, int M,
                     int N, int K, hipStream_t st) {
    const dim3 grid(N / (16 * TR), (M + 15) / 16);
    const size_t red = (size_t)c.waves * TR * 1024;
    const int rs = M > 8 ? 16 : (M > 4 ? 8 : 4);  // rows staged per block
    const size_t slots = (size_t)c.waves * NB * rs * 256;
    // the activations go through LDS where the slots fit
    if (PH == 1 && slots + red <= 160 * 1024) {
        if (rs == 4)
            hipLaunchKernelGGL((mx4_gemv_k<NB, TR, PH, 4>), grid, dim3(64 * c.waves), slots + red, st, A, q, e8w,
                               C, M, N, K);
        else if (rs == 8)
            hipLaunchKernelGGL((mx4_gemv_k<NB, TR, PH, 8>), grid, dim3(64 * c.waves), slots + red, st, A, q, e8w,
                               C, M, N, K);
        else
            hipLaunchKernelGGL((mx4_gemv_k<NB, TR, PH, 16>), grid, dim3(64 * c.waves), slots + red, st, A, q,
                               e8w, C, M, N, K);
    } else {
        hipLaunchKernelGGL((mx4_gemv_k<NB, TR, PH, 0>), grid, dim3(64 * c.waves), red, st, A, q, e8w, C, M, N,
                           K);
    }
}

// Weight loads of the column-split down kernel: compiler-visible buffer
// loads, so the compiler tracks their destination registers and places the
// waits itself (loads issued from inline asm are invisible to it, and it may
// then copy a destination register before the data has landed).  The
// descriptor (a whole matrix, in SGPRs) is built once; a block adds a scalar
// tile offset to a lane offset, so a load costs no 64-bit vector address
// arithmetic.  Offsets past the descriptor's size read 0.
typedef __amdgpu_buffer_rsrc_t wb_rsrc_t;
FL_DEV u32x4 wb_ld16(wb_rsrc_t r, uint32_t voff, uint32_t soff = 0) {  // non-temporal
    return bitcast<u32x4>(__builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 2));
}
FL_DEV uint32_t wb_ld4(wb_rsrc_t r, uint32_t voff, uint32_t soff = 0) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
}

// A lane's byte offsets into one tile for 128-k block kb: the weight bytes
// of the block and the lane's scale word.
struct BlkOff {
    uint32_t w, s;
};
template <int FMT>
FL_DEV BlkOff blk_offsets(int kb, int g, int lane, int col) {
    BlkOff o;
    o.w = (uint32_t)kb * (FMT == kFmtFp8 ? 2048u : 1024u) + 16u * lane;
    o.s = FMT == kFmtFp8 ? 0u : 4u * (16u * (uint32_t)(FMT == kFmtMx4 ? kb : g) + col);
    return o;
}

// Block kb of tile `tile` of the matrix (rq, scales rs), with a fixed number
// of vector loads: the 16-byte weight load and, INT4 / MXFP4, the lane's
// scale word; FP8 the second 16-byte half and the block scale (the same
// word in every lane).
template <int FMT>
FL_DEV WBlk<FMT> wb_blk(wb_rsrc_t rq, wb_rsrc_t rs, uint32_t tile, int nkb, int kb, int G, BlkOff o) {
    constexpr uint32_t TB = FMT == kFmtFp8 ? 2048u : 1024u;
    WBlk<FMT> b;
    const uint32_t tw = tile * (uint32_t)nkb * TB;
    b.w = wb_ld16(rq, o.w, tw);
    if (FMT == kFmtFp8) {
        b.w2 = wb_ld16(rq, o.w + 1024u, tw);
        b.sz = wb_ld4(rs, 0u, ((tile >> 3) * (uint32_t)nkb + (uint32_t)kb) * 4u);
    } else {
        b.sz = wb_ld4(rs, o.s, tile * (uint32_t)(FMT == kFmtMx4 ? nkb : G) * 64u);
    }
    return b;
}

// ---- down projection for 4 < T <= 16 tokens, output columns split over waves
// One workgroup per (slot or shared-expert piece, kDnWaves * kDnTPW output
// tiles); each wave owns kDnTPW output tiles and streams the slot's whole k
// range itself (kDnCH blocks per chunk, dn_depth chunks in flight), so there
// is no cross-wave reduction and no barrier after the start.  The slot's
// activation rows (inter_buf, row0 .. row0 + M) over the k range are copied
// into LDS once per workgroup.  Against the split-k kernel (moe_down_k) this
// runs twice the waves, each with fewer bytes in flight, and the live
// workgroups of a 16-token batch fit in one generation.  Weight loads are
// compiler-visible buffer loads in straight-line code (the chunk loop is
// unrolled), so the compiler's waits leave the later chunks in flight.
constexpr int kDnWaves = 8;  // waves per workgroup
constexpr int kDnTPW = 1;    // 16-column output tiles per wave
constexpr int kDnCH = 2;     // 128-k blocks per chunk
// chunks in flight: three, two for FP8 (its 2 KB blocks take twice the registers)
constexpr int dn_depth(int fmt) { return fmt == kFmtFp8 ? 2 : 3; }
constexpr int kDnMaxCh = 8;  // chunks per slot (k range <= 16 blocks)

// pieces of the shared expert's k range for this kernel (NCH chunks each)
constexpr int dn_kp(int nch) { return nch * kDnCH; }

// Descriptors of expert e's down matrix and its scales (hidden / 16 tiles,
// a multiple of 16: at most hidden x inter bytes each, so 32-bit sizes and
// offsets hold for any expert count).
struct DnRs {
    wb_rsrc_t q, s;
};
template <int FMT>
FL_DEV DnRs dn_rsrcs(const MoeExperts& ex, int e, int hidden, int nkb, int G) {
    const uint32_t tiles = (uint32_t)(hidden / 16);
    const uint32_t wb = tiles * (uint32_t)nkb * (FMT == kFmtFp8 ? 2048u : 1024u);
    const uint32_t sw = FMT == kFmtFp8 ? (tiles >> 3) * (uint32_t)nkb : tiles * (uint32_t)(FMT == kFmtMx4 ? nkb : G) * 16u;
    return DnRs{buf_rsrc(ex.dq + (size_t)e * wb, wb), buf_rsrc(ex.dsz + (size_t)e * sw, sw * 4u)};
}

template <int FMT, bool G128, int NCH>
__global__ __launch_bounds__(64 * kDnWaves, 4) void moe_down_ns(MoeArgs a) {  // 4 waves per SIMD: two workgroups per CU
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int toks[16];
    constexpr int KP = dn_kp(NCH);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kq = lane >> 4;
    const int npc = a.has_shared ? a.pieces : 0;  // shared-expert pieces first
    const int yb = (int)blockIdx.y;
    const bool is_shared = yb < npc;
    int e = 0, row0, M, kb0, KR;
    const MoeExperts* ex;
    if (!is_shared) {
        if (!moe_slot(a, yb - npc, e, row0, M)) return;
        ex = &a.routed;
        kb0 = 0;
        KR = ex->inter >> 7;
    } else {
        row0 = a.max_entries;
        M = a.T;
        ex = &a.shared;
        kb0 = yb * KP;
        const int left = (ex->inter >> 7) - kb0;
        KR = left < KP ? left : KP;
    }
    if (M <= 0 || KR <= 0) return;
    const int nkb = ex->inter >> 7;
    const int G = ex->inter / a.gs;
    // the entries' tokens: loaded first, stored to LDS once the weights are
    // in flight (the store waits for the load)
    const int tok_ld = is_shared ? 0 : a.tok[row0 + (lane < M ? lane : 0)];
    // activation rows -> LDS [M][KR blocks][256 B]: 256-byte pieces, four per
    // wave copy (lane l: 16 bytes l % 16 of piece 4 i + l / 16); a tail past
    // M KR pieces repeats the last one into the slack
    const int npieces = M * KR;
    {
        const i32x4_t rA = raw_rsrc(a.inter_buf, (uint32_t)(a.max_entries + a.T) * (uint32_t)a.inter_pad * 2u);
        const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
        for (int p0 = 4 * wave; p0 < npieces; p0 += 4 * kDnWaves) {
            int p = p0 + (lane >> 4);
            p = p < npieces ? p : npieces - 1;
            const int m = p / KR, kl = p - m * KR;
            lds_copy(rA, lds0 + (uint32_t)p0 * 256u,
                     2u * ((uint32_t)(row0 + m) * (uint32_t)a.inter_pad + (uint32_t)(kb0 + kl) * 128u) +
                         16u * (uint32_t)(lane & 15));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    const DnRs rs = dn_rsrcs<FMT>(*ex, e, a.hidden, nkb, G);
    const uint32_t tile0 = blockIdx.x * (kDnWaves * kDnTPW) + wave * kDnTPW;  // within expert e
    // block i of chunk c: k block kb0 + min(c kDnCH + i, KR - 1) (a block past
    // KR repeats the last one and counts zero)
    auto issue = [&](WBlk<FMT> (&w)[kDnCH][kDnTPW], int c) {
#pragma unroll
        for (int i = 0; i < kDnCH; ++i) {
            const int kl = c * kDnCH + i < KR ? c * kDnCH + i : KR - 1;
            const int kb = kb0 + kl;
            const BlkOff o = blk_offsets<FMT>(kb, (kb * 128 + 32 * kq) / a.gs, lane, col);
#pragma unroll
            for (int t = 0; t < kDnTPW; ++t) w[i][t] = wb_blk<FMT>(rs.q, rs.s, tile0 + t, nkb, kb, G, o);
        }
    };
    constexpr int kDnD = dn_depth(FMT);
    WBlk<FMT> wb[kDnD][kDnCH][kDnTPW];
#pragma unroll
    for (int c = 0; c < kDnD && c < NCH; ++c) {
        issue(wb[c], c);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (threadIdx.x < 16) toks[threadIdx.x] = is_shared ? threadIdx.x : clampi(tok_ld, 0, a.T - 1);
    // the copies were issued before every weight load: once the first weight
    // word has landed (the asm names it, so the compiler waits for it) they
    // have too; the barrier then publishes every wave's pieces and toks
    asm volatile("" : : "v"(wb[0][0][0].w) : "memory");
    lds_barrier();
    const int mrow = col < M ? col : M - 1;
    const unsigned char* arow = smem + (size_t)mrow * KR * 256;
    f32x4 acc[kDnTPW];
#pragma unroll
    for (int t = 0; t < kDnTPW; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
#pragma unroll
        for (int i = 0; i < kDnCH; ++i) {
            const int kl = c * kDnCH + i < KR ? c * kDnCH + i : KR - 1;
            const float live = c * kDnCH + i < KR ? 1.0f : 0.0f;
            u32x4 av[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                av[j] = *reinterpret_cast<const u32x4*>(arow + (size_t)kl * 256 + 2 * a_koff<FMT>(kq, j));
#pragma unroll
            for (int t = 0; t < kDnTPW; ++t) {
                wblk_mma<FMT, G128>(acc[t], av, wb[c % kDnD][i][t], live);
                // keeps the scaled add here: the compiler otherwise sinks every
                // block's add to the epilogue and keeps each block's partial
                // MFMA result live until then
                asm volatile("" : "+v"(acc[t]));
            }
            __builtin_amdgcn_sched_barrier(0);  // one block's operands live at a time
        }
        if (c + kDnD < NCH) issue(wb[c % kDnD], c + kDnD);
        __builtin_amdgcn_sched_barrier(0);
    }
    // lane: rows 4 (lane / 16) + r of tile t, column lane % 16
    const uint32_t c0 = (blockIdx.x * (kDnWaves * kDnTPW) + wave * kDnTPW) * 16u + (uint32_t)col;
#pragma unroll
    for (int t = 0; t < kDnTPW; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 4 * kq + r;
            if (m < M) {
                if (a.det) {
                    const size_t prow = is_shared ? (size_t)a.max_entries + (size_t)yb * a.T + m : (size_t)row0 + m;
                    a.part[prow * a.hidden + c0 + 16 * t] = acc[t][r];
                } else {
                    unsafeAtomicAdd(&a.y[(size_t)toks[m] * a.hidden + c0 + 16 * t], acc[t][r]);
                }
            }
        }
    }
}

// ---- gate/up for 4 < T <= 16 tokens (hidden <= 2048), columns split over waves
// The same split as moe_down_ns: one workgroup per (shared-expert or slot
// column group of 16 kDnWaves intermediate columns); each wave owns one gate
// and one up tile and streams all hidden / 128 k blocks of both itself, so
// h = silu(g) u w is formed in registers with no cross-wave reduction.  The
// T token rows of the fp16 copy of x (all of them: they do not depend on the
// lists) are copied into LDS at the start, before the weights.
template <int FMT>
FL_DEV DnRs gu_rsrcs(const uint8_t* q, const uint32_t* sz, int e, int inter, int nkb, int G) {
    const uint32_t tiles = (uint32_t)(inter / 16);  // a multiple of 8
    const uint32_t wb = tiles * (uint32_t)nkb * (FMT == kFmtFp8 ? 2048u : 1024u);
    const uint32_t sw = FMT == kFmtFp8 ? (tiles >> 3) * (uint32_t)nkb : tiles * (uint32_t)(FMT == kFmtMx4 ? nkb : G) * 16u;
    return DnRs{buf_rsrc(q + (size_t)e * wb, wb), buf_rsrc(sz + (size_t)e * sw, sw * 4u)};
}

template <int FMT, bool G128, int NCH>
__global__ __launch_bounds__(64 * kDnWaves, 4) void moe_gate_up_ns(MoeArgs a) {  // two workgroups per CU
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kq = lane >> 4;
    const int K = a.hidden, KB = K >> 7, T = a.T;
    constexpr int GW = 16 * kDnWaves;  // intermediate columns per workgroup
    // grid: shared-expert groups first (they need no lists), then (slot, group)
    const int n_sh = a.has_shared ? a.shared.inter / GW : 0;
    const int groups_r = a.routed.inter / GW;
    const int b = (int)blockIdx.x;
    // y zeroed for the down kernel's accumulation, spread over the whole grid
    // before any workgroup can leave (these stores are older than every
    // weight load, so the waits below do not count them)
    for (int i = b * 64 * kDnWaves + (int)threadIdx.x; i < T * K / 4; i += (int)gridDim.x * 64 * kDnWaves)
        reinterpret_cast<f32x4*>(a.y)[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const bool routed = b >= n_sh;
    int e = 0, row0, M, grp;
    const MoeExperts* ex;
    if (routed) {
        const int slot = (b - n_sh) / groups_r;
        grp = b - n_sh - slot * groups_r;
        if (!moe_slot(a, slot, e, row0, M)) return;
        ex = &a.routed;
    } else {
        grp = b;
        row0 = a.max_entries;
        M = T;
        ex = &a.shared;
    }
    if (M <= 0) return;
    // token rows -> LDS [T][KB][256 B]: 256-byte pieces, four per wave copy
    // (lane l: 16 bytes l % 16 of piece 4 i + l / 16); a tail repeats the
    // last piece into the slack
    const int npieces = T * KB;
    {
        const i32x4_t rX = raw_rsrc(a.xh, (uint32_t)T * (uint32_t)K * 2u);
        const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
        for (int p0 = 4 * wave; p0 < npieces; p0 += 4 * kDnWaves) {
            int p = p0 + (lane >> 4);
            p = p < npieces ? p : npieces - 1;
            lds_copy(rX, lds0 + (uint32_t)p0 * 256u, 2u * (uint32_t)p * 128u + 16u * (uint32_t)(lane & 15));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // the lane's MFMA row: entry jr of the unit (token tok_ld) and its weight
    // (unconditional loads: values not used are replaced after the barrier)
    const int jr = col < M ? col : M - 1;
    const int tok_ld = a.tok[routed ? row0 + jr : 0];
    const float w_ld = *(routed ? a.tokw + row0 + jr : (a.scoef ? a.scoef + jr : a.tokw));
    const int G = K / a.gs;
    const int inter = ex->inter;
    const DnRs rg = gu_rsrcs<FMT>(ex->gq, ex->gsz, e, inter, KB, G);
    const DnRs ru = gu_rsrcs<FMT>(ex->uq, ex->usz, e, inter, KB, G);
    const uint32_t tile = (uint32_t)(grp * kDnWaves + wave);  // within expert e
    auto issue = [&](WBlk<FMT> (&w)[kDnCH][2], int c) {
#pragma unroll
        for (int i = 0; i < kDnCH; ++i) {
            const int kb = c * kDnCH + i < KB ? c * kDnCH + i : KB - 1;
            const BlkOff o = blk_offsets<FMT>(kb, (kb * 128 + 32 * kq) / a.gs, lane, col);
            w[i][0] = wb_blk<FMT>(rg.q, rg.s, tile, KB, kb, G, o);
            w[i][1] = wb_blk<FMT>(ru.q, ru.s, tile, KB, kb, G, o);
        }
    };
    // each chunk holds gate and up: one chunk fewer in flight than the down
    constexpr int kD = dn_depth(FMT) > 2 ? dn_depth(FMT) - 1 : 2;
    WBlk<FMT> wb[kD][kDnCH][2];
#pragma unroll
    for (int c = 0; c < kD && c < NCH; ++c) {
        issue(wb[c], c);
        __builtin_amdgcn_sched_barrier(0);
    }
    // the copies were issued before every weight load: once the first weight
    // word has landed (the asm names it, so the compiler waits for it) they
    // have too; the barrier publishes every wave's pieces
    asm volatile("" : : "v"(wb[0][0][0].w) : "memory");
    lds_barrier();
    // first uses of the token and weight words only here (through the asm),
    // so their wait does not move above the weight loads
    int tk = tok_ld;
    float wl = w_ld;
    asm volatile("" : "+v"(tk), "+v"(wl));
    tk = routed ? tk : jr;
    wl = (routed || a.scoef) ? wl : 1.0f;
    const unsigned char* arow = smem + (size_t)clampi(tk, 0, T - 1) * KB * 256;
    f32x4 acc[2];
    acc[0] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
#pragma unroll
        for (int i = 0; i < kDnCH; ++i) {
            const int kb = c * kDnCH + i < KB ? c * kDnCH + i : KB - 1;
            const float live = c * kDnCH + i < KB ? 1.0f : 0.0f;
            u32x4 av[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                av[j] = *reinterpret_cast<const u32x4*>(arow + (size_t)kb * 256 + 2 * a_koff<FMT>(kq, j));
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                wblk_mma<FMT, G128>(acc[t], av, wb[c % kD][i][t], live);
                asm volatile("" : "+v"(acc[t]));  // keeps the scaled add here (see moe_down_ns)
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (c + kD < NCH) issue(wb[c % kD], c + kD);
        __builtin_amdgcn_sched_barrier(0);
    }
    // lane: rows 4 (lane / 16) + r, column lane % 16; entry m's weight from
    // lane m (its MFMA row was entry m)
    const uint32_t c0 = (uint32_t)(grp * GW + wave * 16 + col);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = 4 * kq + r;
        const float wm = __shfl(wl, m);
        if (m < M) {
            const float g = acc[0][r], u = acc[1][r];
            const float h = (g / (1.0f + expf(-g))) * u * wm;
            a.inter_buf[(size_t)(row0 + m) * a.inter_pad + c0] = bitcast<uint16_t>((f16)h);
        }
    }
}

// Deterministic combine (MoeArgs::det): y[t, c] = the terms of token t's
// list entries in ascending entry order (ascending expert), then its shared-
// expert pieces in order -- one fixed summation order, so repeated calls give
// bit-identical y.  Grid (hidden / 256 column blocks, T); the workgroup
// gathers token t's entries from tok[] with ballots (ascending by
// construction) before any thread sums.
constexpr int kCombineMaxEnt = 256;  // entries of one token (<= max_slots)
__global__ __launch_bounds__(256) void moe_combine_k(MoeArgs a) {
    __shared__ int ents[kCombineMaxEnt];
    __shared__ int wcount[4];
    const int t = blockIdx.y;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int na = clampi(*a.n_active, 0, a.max_slots);
    const int n_ent = clampi(a.offsets[na], 0, a.max_entries);
    int cnt = 0;
    for (int base = 0; base < n_ent; base += 256) {
        const int i = base + tid;
        const bool hit = i < n_ent && a.tok[i] == t;
        const unsigned long long bm = __ballot(hit);
        if (lane == 0) wcount[wave] = __builtin_popcountll(bm);
        __syncthreads();
        int off = cnt;
        for (int w = 0; w < wave; ++w) off += wcount[w];
        const int pos = off + __builtin_popcountll(bm & ((1ull << lane) - 1ull));
        if (hit && pos < kCombineMaxEnt) ents[pos] = i;
        cnt += wcount[0] + wcount[1] + wcount[2] + wcount[3];
        __syncthreads();
    }
    const int c = blockIdx.x * 256 + tid;
    if (c >= a.hidden) return;
    const int n = cnt < kCombineMaxEnt ? cnt : kCombineMaxEnt;
    float sum = 0.f;
    for (int j = 0; j < n; ++j) sum += a.part[(size_t)ents[j] * a.hidden + c];
    for (int q = 0; q < a.nq; ++q) sum += a.part[(size_t)(a.max_entries + q * a.T + t) * a.hidden + c];
    a.y[(size_t)t * a.hidden + c] = sum;
}

// ------------------------------------------- grouped MoE GEMM (prefill)
// The two fused-MoE kernels for T > 16 tokens: per list slot a grouped GEMM
// over the slot's entries, in chunks of 64 rows (4 m-tiles).
//   PHASE 0 (gate/up): one workgroup per (slot, 128 intermediate columns);
//     wave w computes gate tile 8 strip + w and up tile 8 strip + w over all
//     of hidden, so h = silu(g) * u * w_entry is formed in registers and
//     stored fp16 to inter_buf (no cross-wave reduction: waves split N).
//     Its token rows come from xh, the fp16 copy of x made by x_to_f16_k.
//   PHASE 1 (down): one workgroup per (slot, 256 hidden columns); wave w
//     computes tiles 16 strip + 2 w, + 1 over the slot's inter_buf rows and
//     adds them into y[token] with fp32 atomics, like the decode kernel.
// Slot indices >= max_slots are the shared expert (rows max_entries + t,
// tokens t = 0..T-1, coefficient scoef[t] or 1).
// Every main-loop load goes global -> LDS (lds_copy: buffer_load ... lds
// from inline asm, see common.cuh), kMgAhead blocks ahead, into a ring of
// kMgAhead + 1 stages; one vmcnt wait and one barrier per 128-k block hand
// a stage to all waves.  One block ahead in two stages (two workgroups per
// CU): config 5 148.8-154.2 us per layer, against 190.9 us two blocks ahead
// in three stages (one workgroup per CU).  A stage holds
//   * A (16 KB): 64 rows x 128 k fp16.  FP8 / MXFP4: row-major (256 B per
//     row) with the 16-byte k chunks of row r XOR-swizzled by r % 16, so
//     each copy moves 4 whole rows and the 16 lanes of an MFMA operand read
//     hit 16 different bank groups -- lane (c, q) of MFMA step j of m-tile
//     mt reads row 16 mt + c, chunk a_koff(q, j) / 8 at position chunk ^ c.
//     INT4: fragment-major -- lane (c, q) of MFMA step j reads row c, k
//     32 q + 8 j .. + 7 at 16 (64 (4 mt + j) + c + 16 q);
//   * per wave (2.5 KB): its two 1 KB tile blocks and the tiles' 16 x
//     (128 / gs) scale|zero words.
// B is dequantized in registers to s * (q - z) in fp16 (lane (c, q)'s 32 k
// lie in one group for every group size >= 32) and 32 MFMAs per wave and
// block accumulate in fp32; m-tiles past the chunk's rows skip their MFMAs.
constexpr int kMgAhead = 1, kMgStages = kMgAhead + 1;
constexpr int kMgWaves = 8;                     // waves per workgroup
// per wave and stage: two tile blocks (1 KB, FP8 2 KB) + two 256-byte scale rows
constexpr int mg_wave_stage(int fmt) { return 2 * (fmt == kFmtFp8 ? 2048 : 1024) + 2 * 256; }
constexpr int kMgABytes = 64 * 128 * 2;            // A tile of one stage
constexpr int mg_stage(int fmt) { return kMgABytes + kMgWaves * mg_wave_stage(fmt); }
constexpr size_t mg_lds(int fmt) { return (size_t)kMgStages * mg_stage(fmt); }

// xh[t, :] = fp16(x[t, :]) for the grouped kernels' A copies
__global__ void x_to_f16_k(const float* __restrict__ x, uint16_t* __restrict__ xh, int n8) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += gridDim.x * blockDim.x) {
        const f32x4 lo = reinterpret_cast<const f32x4*>(x)[2 * i];
        const f32x4 hi = reinterpret_cast<const f32x4*>(x)[2 * i + 1];
        f16x8 h;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            h[q] = (f16)lo[q];
            h[4 + q] = (f16)hi[q];
        }
        reinterpret_cast<f16x8*>(xh)[i] = h;
    }
}

template <int PHASE, bool G128, int FMT = kFmtInt4>
__global__ __launch_bounds__(64 * kMgWaves) void moe_gemm_k(MoeArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int D = kMgAhead, NS = kMgStages;
    constexpr int NW = kMgWaves, FPW = 16 / NW;  // waves, A fragments copied per wave
    constexpr int BPT = FMT == kFmtFp8 ? 2 : 1;  // 1 KB copies per tile block
    constexpr int TB = 1024 * BPT;               // tile block bytes
    constexpr int WST = mg_wave_stage(FMT), STG = mg_stage(FMT);
    constexpr int LPB = FPW + 2 * BPT + 2;  // per block and wave: A fragments, B copies, 2 scale rows
    // FP8 / MXFP4 stage A row-major in whole rows (config 5: FP8 204 -> 198,
    // MXFP4 150 -> 147 us per layer); INT4 keeps the MFMA fragment order,
    // whose reads need no per-step lane addressing (its dequantization keeps
    // the VALU busy: 146 against 160 us with whole rows)
    constexpr bool ROWA = FMT != kFmtInt4;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kq = lane >> 4;
    // XCD-grouped units, as in moe_gemm_rk
    const int lin = blockIdx.y * gridDim.x + blockIdx.x, units = gridDim.x * gridDim.y;
    const int unit = (units & 7) ? lin : (lin & 7) * (units >> 3) + (lin >> 3);
    const int slot = unit / gridDim.x, strip = unit - slot * gridDim.x;
    if (PHASE == 0) {
        // every workgroup zeroes its share of y for the down phase's atomics
        const int nwg = gridDim.x * gridDim.y;
        const int wg = blockIdx.y * gridDim.x + blockIdx.x;
        const int n4 = a.T * a.hidden / 4;
        for (int i = wg * 64 * NW + threadIdx.x; i < n4; i += nwg * 64 * NW)
            reinterpret_cast<f32x4*>(a.y)[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const bool is_shared = slot >= a.max_slots;
    if (is_shared && !a.has_shared) return;
    int e = 0, row0, M;
    const MoeExperts* ex;
    if (!is_shared) {
        if (!moe_slot(a, slot, e, row0, M)) return;
        // moe_slot caps M at T for the decode kernels; a prefill slot holds
        // every entry routed to its expert
        const int r1 = clampi(__builtin_amdgcn_readfirstlane(a.offsets[slot + 1]), row0, a.max_entries);
        M = r1 - row0;
        ex = &a.routed;
    } else {
        row0 = a.max_entries;
        M = a.T;
        ex = &a.shared;
    }
    const int inter = ex->inter;
    const int K = PHASE == 0 ? a.hidden : inter;
    const int Nrows = PHASE == 0 ? inter : a.hidden;  // output rows of the weight
    const int ncols = PHASE == 0 ? 16 * NW : 32 * NW;  // columns per workgroup
    if (M <= 0 || strip * ncols >= Nrows) return;
    const int nkb = K >> 7;
    const int G = K / a.gs;
    const int spb = 128 / a.gs;  // groups per 128-k block

    // this wave's two weight tiles
    i32x4_t rq[2], rz[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        size_t tile;
        const uint8_t* tq;
        const uint32_t* tsz;
        if (PHASE == 0) {
            tile = (size_t)e * (inter / 16) + strip * NW + wave;
            tq = t == 0 ? ex->gq : ex->uq;
            tsz = t == 0 ? ex->gsz : ex->usz;
        } else {
            tile = (size_t)e * (a.hidden / 16) + strip * 2 * NW + wave * 2 + t;
            tq = ex->dq;
            tsz = ex->dsz;
        }
        rq[t] = raw_rsrc(tq + tile * nkb * TB, nkb * TB);
        if (FMT == kFmtFp8)  // one fp32 scale per (128-row band, block)
            rz[t] = raw_rsrc(tsz + (tile >> 3) * nkb, nkb * 4);
        else if (FMT == kFmtMx4)  // 16 E8M0 words per block
            rz[t] = raw_rsrc(tsz + tile * nkb * 16, nkb * 64);
        else
            rz[t] = raw_rsrc(tsz + tile * G * 16, G * 64);
    }
    // A rows: PHASE 0 token rows of xh, PHASE 1 the slot's inter_buf rows
    const uint16_t* abase = PHASE == 0 ? a.xh : a.inter_buf;
    const int astride = PHASE == 0 ? a.hidden : a.inter_pad;  // halves
    const int arows = PHASE == 0 ? a.T : a.max_entries + a.T;
    const i32x4_t rA = raw_rsrc(abase, (uint32_t)arows * astride * 2);
    const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
    // scale-row copy: INT4 16 words per group, MXFP4 16 words, FP8 the one
    // block scale (every lane copies it)
    const uint32_t zlane = FMT == kFmtFp8 ? 0u
                         : FMT == kFmtMx4 ? 4u * (lane < 16 ? lane : 15)
                                          : 4u * (lane < 16 * spb ? lane : 16 * spb - 1);
    const int zstep = FMT == kFmtFp8 ? 4 : (FMT == kFmtMx4 ? 64 : spb * 64);  // scale bytes per block
    const int g_local = kq * 32 / a.gs;  // this lane's group within a block

    for (int mc = 0; mc < M; mc += 64) {
        const int mt_live = (M - mc + 15) >> 4;  // m-tiles holding rows of this chunk
        // A copies f = FPW wave + i of this wave.  FP8 / MXFP4 (ROWA): chunk
        // rows 4 f .. 4 f + 3 (m-tile f / 4), each the row's whole 256 bytes
        // of the block (two full cache lines); lane l takes row 4 f + l / 16
        // and its 16-byte k chunk (l % 16) ^ (row % 16).  INT4: fragment f =
        // 4 m-tile + j in MFMA order (16 rows x four 16-byte pieces).
        // lane l holds row mc + l's token and combine weight (rows past M
        // repeat row M - 1), read once per chunk and handed out by shuffles
        const int ml = mc + lane < M ? mc + lane : M - 1;
        const int ltok = is_shared ? ml : clampi(a.tok[row0 + ml], 0, a.T - 1);
        const float lw = PHASE != 0 ? 0.0f : (!is_shared ? a.tokw[row0 + ml] : (a.scoef ? a.scoef[ml] : 1.0f));
        uint32_t ao[4];
#pragma unroll
        for (int i = 0; i < FPW; ++i) {
            const int f = wave * FPW + i;
            const int r = ROWA ? 4 * f + (lane >> 4) : 16 * (f >> 2) + col;
            int m = mc + r;
            m = m < M ? m : M - 1;
            const int row = PHASE == 0 ? __shfl(ltok, m - mc, 64) : row0 + m;
            ao[i] = 2u * ((uint32_t)row * astride +
                          (ROWA ? 8 * ((lane & 15) ^ (r & 15)) : a_koff<FMT>(kq, f & 3)));
        }
        // blocks past the end keep the copy count with lane offsets past
        // every buffer's range: they read zeros without touching memory
        auto issue = [&](int kb, int stg) {
            const uint32_t oob = kb < nkb ? 0u : 0x80000000u;
            kb = kb < nkb ? kb : nkb - 1;
            const uint32_t st = lds0 + (uint32_t)stg * STG;
#pragma unroll
            for (int i = 0; i < FPW; ++i)
                if (kMgAhead > 1 || wave * FPW + i < 4 * mt_live)  // dead m-tiles: no copy
                    lds_copy(rA, st + (wave * FPW + i) * 1024, ao[i] | oob, kb * 256);
            const uint32_t wst = st + kMgABytes + wave * WST;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int h = 0; h < BPT; ++h)  // FP8: the block's two 1 KB halves
                    lds_copy(rq[t], wst + t * TB + h * 1024, (h * 1024 + lane * 16) | oob, kb * TB);
#pragma unroll
            for (int t = 0; t < 2; ++t) lds_copy<4>(rz[t], wst + 2 * TB + t * 256, zlane | oob, kb * zstep);
        };

        f32x4 acc[4][2];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int t = 0; t < 2; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
        for (int d = 0; d < D; ++d) issue(d, d);
        for (int kb = 0; kb < nkb; ++kb) {
            wait_vmcnt<(D - 1) * LPB>();
            asm volatile("s_barrier" ::: "memory");
            issue(kb + D, (kb + D) % NS);
            const unsigned char* st = smem + (size_t)(kb % NS) * STG;
            const unsigned char* wst = st + kMgABytes + wave * WST;
            if constexpr (FMT != kFmtInt4) {
                // FP8 / MXFP4: codes to fp16 once per (tile, step) for the
                // four m-tiles; FP8 scales the block's partial once, MXFP4
                // every step (one MX block per step)
                WBlk<FMT> bl[2];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    bl[t].w = *reinterpret_cast<const u32x4*>(wst + t * TB + lane * 16);
                    if (FMT == kFmtFp8) bl[t].w2 = *reinterpret_cast<const u32x4*>(wst + t * TB + 1024 + lane * 16);
                    bl[t].sz = *reinterpret_cast<const uint32_t*>(wst + 2 * TB + t * 256 +
                                                                  (FMT == kFmtMx4 ? 4 * col : 0));
                }
                const unsigned char* ab = st + col * 256;  // ROWA (FP8 / MXFP4)
                f32x4 part[4][2];
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int t = 0; t < 2; ++t) part[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    f16x8 av[4];
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt)
                        av[mt] = *reinterpret_cast<const f16x8*>(ab + mt * 4096 + 16 * ((a_koff<FMT>(kq, j) >> 3) ^ col));
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        if (FMT == kFmtMx4) {
                            const f16x8 b = mx_operand_scaled(bl[t].w[j], mx_step_scale(bl[t].sz, j));
#pragma unroll
                            for (int mt = 0; mt < 4; ++mt)
                                if (mt < mt_live) acc[mt][t] = mfma_f16(av[mt], b, acc[mt][t]);
                        } else {
                            const f16x8 b = wblk_operand(bl[t], j);
#pragma unroll
                            for (int mt = 0; mt < 4; ++mt)
                                if (mt < mt_live) part[mt][t] = mfma_f16(av[mt], b, part[mt][t]);
                        }
                    }
                }
                if (FMT == kFmtFp8) {
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        const float sv = __uint_as_float(bl[t].sz);
#pragma unroll
                        for (int mt = 0; mt < 4; ++mt)
                            if (mt < mt_live)
#pragma unroll
                                for (int i = 0; i < 4; ++i) acc[mt][t][i] = __builtin_fmaf(sv, part[mt][t][i], acc[mt][t][i]);
                    }
                }
                continue;
            }
            u32x4 wv[2];
            uint32_t zlo[2], zhi[2];
            uint16_t sc[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                wv[t] = *reinterpret_cast<const u32x4*>(wst + t * 1024 + lane * 16);
                const uint32_t szw =
                    *reinterpret_cast<const uint32_t*>(wst + 2048 + t * 256 + 4 * (g_local * 16 + col));
                tile_zero_bits(sz_zero(szw), zlo[t], zhi[t]);
                sc[t] = sz_scale(szw);
            }
            const unsigned char* ab = st + lane * 16;  // INT4: fragment order
            // group 128: q - z products accumulate in a per-block fp32 partial
            // that takes the column scale once; smaller groups scale B in fp16
            f32x4 part[4][2];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int t = 0; t < 2; ++t) part[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f16x8 av[4];
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
                    av[mt] = *reinterpret_cast<const f16x8*>(ab + (mt * 4 + j) * 1024);
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    f16x8 b = dequant_word_fast(wv[t][j], zlo[t], zhi[t], 0x64006400u, 0x54005400u);
                    if (!G128) b = bitcast<f16x8>(scale_f16x8(bitcast<u32x4>(b), sc[t]));
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt)
                        if (mt < mt_live) {
                            if (G128)
                                part[mt][t] = mfma_f16(av[mt], b, part[mt][t]);
                            else
                                acc[mt][t] = mfma_f16(av[mt], b, acc[mt][t]);
                        }
                }
            }
            if (G128) {
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const float sv = (float)bitcast<f16>(sc[t]);
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt)
                        if (mt < mt_live)
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                acc[mt][t][i] = __builtin_fmaf(sv, part[mt][t][i], acc[mt][t][i]);
                }
            }
        }
        wait_vmcnt<0>();

        // epilogue: rows mc + 16 mt + 4 kq + i of the chunk
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = mc + 16 * mt + 4 * kq + i;
                // shuffles with every lane active (a lane whose row is past M
                // may hold the row another lane reads)
                const float w = __shfl(lw, 16 * mt + 4 * kq + i, 64);
                const int tkn = __shfl(ltok, 16 * mt + 4 * kq + i, 64);
                if (m >= M) continue;
                if (PHASE == 0) {
                    const float g = acc[mt][0][i], u = acc[mt][1][i];
                    const float h = (g / (1.0f + expf(-g))) * u * w;
                    a.inter_buf[(size_t)(row0 + m) * a.inter_pad + strip * 16 * NW + wave * 16 + col] =
                        bitcast<uint16_t>((f16)h);
                } else {
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        const int cc = strip * 32 * NW + wave * 32 + t * 16 + col;
                        if (a.det)  // the shared slot's rows max_entries + t are piece 0's
                            a.part[(size_t)(row0 + m) * a.hidden + cc] = acc[mt][t][i];
                        else
                            unsafeAtomicAdd(&a.y[(size_t)tkn * a.hidden + cc], acc[mt][t][i]);
                    }
                }
            }
        asm volatile("s_barrier" ::: "memory");  // the chunk's LDS is reused by the next chunk
    }
}

// INT4 grouped MoE GEMM with the weights streamed into registers.  The same
// units, tiles and epilogue as moe_gemm_k, but only the activation tile (the
// operand all waves share) goes through the LDS ring; each wave's two tile
// blocks and their scale|zero words (its own, read back by no other wave)
// are compiler-visible buffer loads into a register ring kMrD blocks deep.
// The LDS then holds kMrD + 1 activation stages (16 KB each), so two
// workgroups per CU keep kMrD blocks of weights in flight where the shared
// stages of moe_gemm_k (36 KB each) allow one.  B is s * (q - z) rounded to
// fp16 (the Marlin operand) and the MFMAs accumulate in fp32.
// Hand-off per block c: the compiler waits for the wave's first weight word
// of c (named by an empty asm), and the activation copies of c went out just
// before it, so they have landed too; one barrier then publishes every
// wave's copies and retires the stage of block c - 1, which the copies of
// block c + kMrD (issued after the barrier) overwrite.
constexpr int kMrD = 3;              // blocks in flight ahead
// Waves per workgroup and blocks ahead of each launch.  Config 5 (INT4):
// 8 / 3 for both 111-112 us per layer; four-wave workgroups two blocks ahead
// (three per CU, 95 / 82 VGPRs) 119 us for down alone, 124 for gate/up
// alone, 131 for both; three ahead at four waves 129 us.
constexpr int kMrGuWaves = 8, kMrGuD = 3;  // gate/up: waves (16 columns each), blocks ahead
constexpr int kMrDnWaves = 8, kMrDnD = 3;  // down: waves (32 columns each), blocks ahead

template <int V>
struct IntC {
    static constexpr int value = V;
};

struct MrBlk {
    u32x4 w[2];      // the two tiles' 1 KB blocks, this lane's 16 bytes
    uint32_t sz[2];  // this lane's scale|zero word of each tile
};

template <int PHASE, bool G128, int NW = kMgWaves, int D = kMrD>
__global__ __launch_bounds__(64 * NW) void moe_gemm_rk(MoeArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int NS = D + 1, FPW = 16 / NW;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kq = lane >> 4;
    // XCD-grouped units: the hardware deals workgroup L (linear index) to XCD
    // L % 8, so with the unit count a multiple of 8 XCD x takes the
    // contiguous units [x U/8, (x+1) U/8): whole slots, whose strips then
    // share the slot's activation rows in one L2
    const int lin = blockIdx.y * gridDim.x + blockIdx.x, units = gridDim.x * gridDim.y;
    const int unit = (units & 7) ? lin : (lin & 7) * (units >> 3) + (lin >> 3);
    const int slot = unit / gridDim.x, strip = unit - slot * gridDim.x;
    if (PHASE == 0) {
        // every workgroup zeroes its share of y for the down phase's atomics
        const int nwg = gridDim.x * gridDim.y;
        const int wg = blockIdx.y * gridDim.x + blockIdx.x;
        const int n4 = a.T * a.hidden / 4;
        for (int i = wg * 64 * NW + threadIdx.x; i < n4; i += nwg * 64 * NW)
            reinterpret_cast<f32x4*>(a.y)[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const bool is_shared = slot >= a.max_slots;
    if (is_shared && !a.has_shared) return;
    int e = 0, row0, M;
    const MoeExperts* ex;
    if (!is_shared) {
        if (!moe_slot(a, slot, e, row0, M)) return;
        const int r1 = clampi(__builtin_amdgcn_readfirstlane(a.offsets[slot + 1]), row0, a.max_entries);
        M = r1 - row0;
        ex = &a.routed;
    } else {
        row0 = a.max_entries;
        M = a.T;
        ex = &a.shared;
    }
    const int inter = ex->inter;
    const int K = PHASE == 0 ? a.hidden : inter;
    const int Nrows = PHASE == 0 ? inter : a.hidden;
    const int ncols = PHASE == 0 ? 16 * NW : 32 * NW;
    if (M <= 0 || strip * ncols >= Nrows) return;
    const int nkb = K >> 7;
    const int G = K / a.gs;
    const int spb = 128 / a.gs;  // groups per 128-k block

    // this wave's two weight tiles: blocks and scale|zero words
    __amdgpu_buffer_rsrc_t rq[2], rz[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        size_t tile;
        const uint8_t* tq;
        const uint32_t* tsz;
        if (PHASE == 0) {
            tile = (size_t)e * (inter / 16) + strip * NW + wave;
            tq = t == 0 ? ex->gq : ex->uq;
            tsz = t == 0 ? ex->gsz : ex->usz;
        } else {
            tile = (size_t)e * (a.hidden / 16) + strip * 2 * NW + wave * 2 + t;
            tq = ex->dq;
            tsz = ex->dsz;
        }
        rq[t] = buf_rsrc(tq + tile * nkb * 1024, (uint32_t)nkb * 1024u);
        rz[t] = buf_rsrc(tsz + tile * G * 16, (uint32_t)G * 64u);
    }
    const uint32_t zoff = 4u * (uint32_t)((kq * 32 / a.gs) * 16 + col);  // this lane's word in a block
    const uint32_t zstep = (uint32_t)spb * 64u;                           // scale bytes per block
    // A rows: PHASE 0 token rows of xh, PHASE 1 the slot's inter_buf rows
    const uint16_t* abase = PHASE == 0 ? a.xh : a.inter_buf;
    const int astride = PHASE == 0 ? a.hidden : a.inter_pad;  // halves
    const int arows = PHASE == 0 ? a.T : a.max_entries + a.T;
    const i32x4_t rA = raw_rsrc(abase, (uint32_t)arows * astride * 2);
    const uint32_t lds0 = (uint32_t)(uintptr_t)smem;

    for (int mc = 0; mc < M; mc += 64) {
        const int mt_live = (M - mc + 15) >> 4;  // m-tiles holding rows of this chunk
        // lane l holds row mc + l's token and combine weight (rows past M
        // repeat row M - 1), read once per chunk and handed out by shuffles
        const int ml = mc + lane < M ? mc + lane : M - 1;
        const int ltok = is_shared ? ml : clampi(a.tok[row0 + ml], 0, a.T - 1);
        const float lw = PHASE != 0 ? 0.0f : (!is_shared ? a.tokw[row0 + ml] : (a.scoef ? a.scoef[ml] : 1.0f));
        // A copies f = FPW wave + i of this wave: fragment f = 4 m-tile + j in
        // MFMA order (16 rows x four 16-byte pieces)
        uint32_t ao[FPW];
#pragma unroll
        for (int i = 0; i < FPW; ++i) {
            const int f = wave * FPW + i;
            const int r = 16 * (f >> 2) + col;  // chunk row
            const int row = PHASE == 0 ? __shfl(ltok, r, 64) : row0 + (mc + r < M ? mc + r : M - 1);
            ao[i] = 2u * ((uint32_t)row * astride + a_koff<kFmtInt4>(kq, f & 3));
        }
        // block b: activation copies into stage b % NS, then the wave's weight
        // and scale loads into r.  Blocks past the end keep the weight and
        // scale load count (so the compiler's waits stay exact) with lane
        // offsets past every buffer's range: the loads return zeros without
        // touching memory, into a ring slot nobody reads.  They issue no
        // activation copy: with fewer blocks than the ring is deep, no
        // barrier separates a past-end block's stage from the waves still
        // reading an earlier block there (the copies come from inline asm,
        // which the compiler's waits do not count).
        auto issue = [&](MrBlk& r, int b) {
            const int kb = b < nkb ? b : nkb - 1;
            const uint32_t oob = b < nkb ? 0u : 0x80000000u;
            const uint32_t st = lds0 + (uint32_t)(b % NS) * kMgABytes;
            if (b < nkb) {
#pragma unroll
                for (int i = 0; i < FPW; ++i)
                    if (wave * FPW + i < 4 * mt_live)  // dead m-tiles: no copy
                        lds_copy(rA, st + (wave * FPW + i) * 1024, ao[i], kb * 256);
            }
#pragma unroll
            for (int t = 0; t < 2; ++t)
                r.w[t] = bitcast<u32x4>(__builtin_amdgcn_raw_buffer_load_b128(rq[t], (int)(16u * lane | oob),
                                                                              (int)(1024u * kb), 2));
#pragma unroll
            for (int t = 0; t < 2; ++t)
                r.sz[t] = __builtin_amdgcn_raw_buffer_load_b32(rz[t], (int)(zoff | oob), (int)(zstep * kb), 0);
        };

        f32x4 acc[4][2];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int t = 0; t < 2; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

        // the block loop for ML live m-tiles (a compile-time count: no
        // per-MFMA branches, no activation reads of dead m-tiles)
        auto run = [&](auto mlc) {
            constexpr int ML = decltype(mlc)::value;
            MrBlk ring[D];
            const int passes = (nkb + D - 1) / D + 1;
            for (int it = 0; it < passes; ++it) {
#pragma unroll
                for (int d = 0; d < D; ++d) {
                    const int c = (it - 1) * D + d;  // the block computed here
                    if (it > 0 && c < nkb) {
                        asm volatile("" : : "v"(ring[d].w[0]) : "memory");
                        asm volatile("s_barrier" ::: "memory");
                        const unsigned char* ab = smem + (size_t)(c % NS) * kMgABytes + lane * 16;
                        uint32_t zlo[2], zhi[2];
#pragma unroll
                        for (int t = 0; t < 2; ++t) tile_zero_bits(sz_zero(ring[d].sz[t]), zlo[t], zhi[t]);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            f16x8 av[ML];
#pragma unroll
                            for (int mt = 0; mt < ML; ++mt)
                                av[mt] = *reinterpret_cast<const f16x8*>(ab + (mt * 4 + j) * 1024);
#pragma unroll
                            for (int t = 0; t < 2; ++t) {
                                const f16x8 b = bitcast<f16x8>(scale_f16x8(
                                    bitcast<u32x4>(dequant_word_fast(ring[d].w[t][j], zlo[t], zhi[t], 0x64006400u,
                                                                     0x54005400u)),
                                    sz_scale(ring[d].sz[t])));
#pragma unroll
                                for (int mt = 0; mt < ML; ++mt) acc[mt][t] = mfma_f16(av[mt], b, acc[mt][t]);
                            }
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    issue(ring[d], it * D + d);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        };
        switch (mt_live) {
            case 1: run(IntC<1>{}); break;
            case 2: run(IntC<2>{}); break;
            case 3: run(IntC<3>{}); break;
            default: run(IntC<4>{}); break;
        }
        wait_vmcnt<0>();

        // epilogue: rows mc + 16 mt + 4 kq + i of the chunk
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = mc + 16 * mt + 4 * kq + i;
                // shuffles with every lane active (a lane whose row is past M
                // may hold the row another lane reads)
                const float w = __shfl(lw, 16 * mt + 4 * kq + i, 64);
                const int tkn = __shfl(ltok, 16 * mt + 4 * kq + i, 64);
                if (m >= M) continue;
                if (PHASE == 0) {
                    const float g = acc[mt][0][i], u = acc[mt][1][i];
                    const float h = (g / (1.0f + expf(-g))) * u * w;
                    a.inter_buf[(size_t)(row0 + m) * a.inter_pad + strip * 16 * NW + wave * 16 + col] =
                        bitcast<uint16_t>((f16)h);
                } else {
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        const int cc = strip * 32 * NW + wave * 32 + t * 16 + col;
                        if (a.det)
                            a.part[(size_t)(row0 + m) * a.hidden + cc] = acc[mt][t][i];
                        else
                            unsafeAtomicAdd(&a.y[(size_t)tkn * a.hidden + cc], acc[mt][t][i]);
                    }
                }
            }
        asm volatile("s_barrier" ::: "memory");  // the chunk's LDS is reused by the next chunk
    }
}

int finish(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fprintf(stderr, "%s launch error: %s\n", what, hipGetErrorString(e));
        return 2;
    }
    return 0;
}

template <int NB, bool G128, bool XF32, bool YF32, bool AFMT>
void launch_rm(const void* X, const uint8_t* W, const void* S, const void* Z, void* Y, int M,
               int N, int K, int gs, int waves, hipStream_t st) {
    const size_t lds = (((size_t)M * (K + 8) * 2 + 15) & ~(size_t)15) + (size_t)waves * 1024;
    hipLaunchKernelGGL((rm_gemv_nb<NB, G128, XF32, YF32, AFMT>), dim3((N + 15) / 16),
                       dim3(64 * waves), lds, st, X, W, S, Z, Y, M, N, K, gs);
}

template <bool G128, bool XF32, bool YF32, bool AFMT>
void rm_dispatch(int nb, const void* X, const uint8_t* W, const void* S, const void* Z, void* Y,
                 int M, int N, int K, int gs, int waves, hipStream_t st) {
    switch (nb) {
        case 1: launch_rm<1, G128, XF32, YF32, AFMT>(X, W, S, Z, Y, M, N, K, gs, waves, st); break;
        case 2: launch_rm<2, G128, XF32, YF32, AFMT>(X, W, S, Z, Y, M, N, K, gs, waves, st); break;
        case 3: launch_rm<3, G128, XF32, YF32, AFMT>(X, W, S, Z, Y, M, N, K, gs, waves, st); break;
        case 4: launch_rm<4, G128, XF32, YF32, AFMT>(X, W, S, Z, Y, M, N, K, gs, waves, st); break;
        case 5: launch_rm<5, G128, XF32, YF32, AFMT>(X, W, S, Z, Y, M, N, K, gs, waves, st); break;
        case 6: launch_rm<6, G128, XF32, YF32, AFMT>(X, W, S, Z, Y, M, N, K, gs, waves, st); break;
        default: launch_rm<8, G128, XF32, YF32, AFMT>(X, W, S, Z, Y, M, N, K, gs, waves, st); break;
    }
}

template <int T, int XC, bool AFMT>
void launch_rm_line_np(int np, dim3 grid, dim3 block, size_t lds, const void* X, const uint8_t* W,
                       const void* S, const void* Z, void* Y, int y_fp32, int M, int N, int K,
                       hipStream_t st) {
    switch (np) {
        case 1: hipLaunchKernelGGL((rm_gemv_line<T, 1, XC, AFMT>), grid, block, lds, st, X, W, S, Z, Y, y_fp32, M, N, K); break;
        case 2: hipLaunchKernelGGL((rm_gemv_line<T, 2, XC, AFMT>), grid, block, lds, st, X, W, S, Z, Y, y_fp32, M, N, K); break;
        default:
            if constexpr (T == 1) {  // two tiles take at most two pairs per wave
                if (np == 3)
                    hipLaunchKernelGGL((rm_gemv_line<1, 3, XC, AFMT>), grid, block, lds, st, X, W, S, Z, Y, y_fp32, M, N, K);
                else
                    hipLaunchKernelGGL((rm_gemv_line<1, 4, XC, AFMT>), grid, block, lds, st, X, W, S, Z, Y, y_fp32, M, N, K);
            }
            break;
    }
}

// The whole-line kernel for M <= 4, K % 256 == 0 and one group per 128-k
// block; false (nothing launched) for shapes it does not take.  Sixteen
// waves of one pair up to K = 4096 (4096 x 4096: 4.75 us against 5.15 with
// eight of two), eight of two on wide N (24576 x 4096: 12.3 against 13.4
// us), more pairs per wave above; two tiles per workgroup from N = 6144.
template <bool AFMT>
bool launch_rm_line(const void* X, int x_fp32, const uint8_t* W, const void* S, const void* Z, void* Y,
                    int y_fp32, int M, int N, int K, bool g128, hipStream_t st) {
    if (M > 4 || K % 256 || !g128) return false;
    if (!fl_aligned(S, AFMT ? 8 : 4) || !fl_aligned(Z, AFMT ? 8 : 4)) return false;
    const int npairs = K / 256;
    int waves = (npairs <= 16 && N >= 16384) ? 8 : 16;
    while (waves > 1 && npairs < waves) waves /= 2;
    const int np = (npairs + waves - 1) / waves;
    if (np > 4) return false;
    const int xc = x_fp32 ? (M <= 2 ? 1 : 2) : 0;
    // two tiles take 2x the weight registers: at most two pairs per wave
    const int T = (N >= 6144 && N % 32 == 0 && np <= 2) ? 2 : 1;
    const int pieces = rm_sz_pieces(np, AFMT ? 2 : 4);
    const size_t lds = (size_t)waves * rm_line_wave_lds(np, xc == 2 ? 2048 : 1024, T, pieces);
    if (lds > 160 * 1024) return false;
    const dim3 grid((N + 16 * T - 1) / (16 * T)), block(64 * waves);
#define RM_LINE(TT, XCC) \
    if (T == TT && xc == XCC) launch_rm_line_np<TT, XCC, AFMT>(np, grid, block, lds, X, W, S, Z, Y, y_fp32, M, N, K, st);
    RM_LINE(1, 0) RM_LINE(1, 1) RM_LINE(1, 2) RM_LINE(2, 0) RM_LINE(2, 1) RM_LINE(2, 2)
#undef RM_LINE
    return true;
}

// Shared body of the two row-major GEMV entries: M in chunks whose fp16 rows
// fit the LDS staging area, one launch per chunk.
template <bool AFMT>
int rm_gemv_entry(const char* what, const void* x, int x_fp32, const uint8_t* qweight,
                  const void* scales, const void* zeros, void* y, int y_fp32, int M, int out_f,
                  int in_f, int group_size, bool g128, void* stream) {
    if (launch_rm_line<AFMT>(x, x_fp32, qweight, scales, zeros, y, y_fp32, M, out_f, in_f,
                             g128 && group_size == 128, (hipStream_t)stream))
        return finish(what);
    const int nfull = in_f / 128;
    int waves = 16;
    while (waves > 1 && nfull < waves) waves /= 2;
    while ((nfull + waves - 1) / waves > 8 && waves < 16) waves *= 2;
    if ((nfull + waves - 1) / waves > 8) return 1;  // in_f > 16384
    const int need = (nfull + waves - 1) / waves;
    const int nb = need <= 6 ? need : 8;
    hipStream_t st = (hipStream_t)stream;
    const size_t xe = x_fp32 ? 4 : 2, ye = y_fp32 ? 4 : 2;
    int mcap = (int)((96 * 1024) / ((size_t)(in_f + 8) * 2));
    mcap = mcap > 16 ? 16 : (mcap < 1 ? 1 : mcap);
    for (int m0 = 0; m0 < M; m0 += mcap) {
        const int Mc = (M - m0) < mcap ? (M - m0) : mcap;
        const void* xm = static_cast<const char*>(x) + (size_t)m0 * in_f * xe;
        void* ym = static_cast<char*>(y) + (size_t)m0 * out_f * ye;
#define RM_CASE(G, XF, YF)                                                                       \
    if (g128 == G && (x_fp32 != 0) == XF && (y_fp32 != 0) == YF)                                 \
        rm_dispatch<G, XF, YF, AFMT>(nb, xm, qweight, scales, zeros, ym, Mc, out_f, in_f,         \
                                     group_size, waves, st);
        RM_CASE(true, true, true)
        RM_CASE(true, true, false)
        RM_CASE(true, false, true)
        RM_CASE(true, false, false)
        RM_CASE(false, true, true)
        RM_CASE(false, true, false)
        RM_CASE(false, false, true)
        RM_CASE(false, false, false)
#undef RM_CASE
        const int rc = finish(what);
        if (rc) return rc;
    }
    return 0;
}

// Launch plan of the fused MoE for one problem shape (host side).
struct MoePlan {
    bool grouped;   // T > 16: the grouped-GEMM kernels
    size_t xh_off;  // grouped, or T > 4: workspace offset of the fp16 copy of x (else 0)
    int nb_gu, waves_gu, tr_gu, nb_d, trd, waves_d, pieces, inter_pad;
    size_t lds_gu, lds_d, bytes;
    size_t part_off;  // deterministic combine: workspace offset of the term rows (else 0)
    int nq;           // shared-expert pieces of the down projection
    bool dn_ns;       // down by the column-split kernel (moe_down_ns), nch chunks
    int nch;
    size_t lds_dn;
    bool gu_ns;       // gate/up by the column-split kernel (moe_gate_up_ns), nch_gu chunks
    int nch_gu;
    size_t lds_gun;
    size_t inter_off;   // workspace offset of inter_buf (after the counter region)
};

// The first kMoeCounterBytes of every fused-MoE workspace hold the routed
// entry's arrival counter (batches above 16 tokens).  Every plan leaves them
// out, so a workspace shared by calls of any shape keeps them as the last
// call left them: zero, once the workspace was zero-filled before its first
// use.
constexpr size_t kMoeCounterBytes = 256;

// The deterministic combine's term rows after the rest of the workspace:
// (max_entries + nq T) x hidden fp32, 256-byte aligned.
void plan_part(MoePlan& p, bool det, int T, int hidden, int max_entries) {
    p.part_off = 0;
    if (!det) return;
    p.part_off = (p.bytes + 255) & ~(size_t)255;
    p.bytes = p.part_off + (size_t)(max_entries + (size_t)p.nq * T) * hidden * 4;
}

// 16-row output tiles per down-projection workgroup for NB blocks per wave
// (Qwen1.5-MoE down, NB = 2: two tiles measured 14.8 / 60.0 us per layer at
// T = 1 / 16 against 15.5 / 60.3 with four and 15.3 / 64.1 with one).
constexpr int down_tiles(int nb) { return nb <= 4 ? 2 : 1; }

// false when the shape is outside what the kernels support.
bool moe_plan(int T, int hidden, int inter, int shared_inter, int max_entries, MoePlan& p,
              int fmt = kFmtInt4, bool det = false) {
    if (T <= 0 || hidden <= 0 || hidden % 128 || inter <= 0 || inter % 128) return false;
    if (shared_inter < 0 || shared_inter % 128 || max_entries <= 0) return false;
    p.grouped = T > 16;
    p.xh_off = 0;
    p.inter_pad = inter > shared_inter ? inter : shared_inter;
    p.inter_off = kMoeCounterBytes;
    p.bytes = p.inter_off + (size_t)(max_entries + T) * p.inter_pad * 2;
    if (p.grouped) {
        // + the fp16 copy of x, 256-byte aligned after inter_buf
        p.xh_off = (p.bytes + 255) & ~(size_t)255;
        p.bytes = p.xh_off + (size_t)T * hidden * 2;
        p.nq = shared_inter > 0 ? 1 : 0;  // the shared slot covers all of its K
        plan_part(p, det, T, hidden, max_entries);
        return hidden % 256 == 0;  // grouped GEMM: 256-column down strips
    }
    const int nfh = hidden / 128;
    p.nb_gu = (nfh + 7) / 8;
    if (p.nb_gu > 4) return false;  // hidden <= 4096
    p.waves_gu = (nfh + p.nb_gu - 1) / p.nb_gu;
    const size_t as_bytes = (size_t)p.waves_gu * p.nb_gu * ((T + 3) & ~3) * 256;
    // FP8 blocks take twice the weight registers: four tiles only with two
    // blocks per wave, two with more
    p.tr_gu = gu_tiles(T);
    if (fmt == kFmtFp8 && p.tr_gu > 1 && (hidden / 128 + 7) / 8 > 2) p.tr_gu = 2;
    const size_t red_bytes = (size_t)p.waves_gu * 2 * p.tr_gu * 1024;
    p.lds_gu = (as_bytes > red_bytes ? as_bytes : red_bytes) + (size_t)2 * p.tr_gu * 1024 + 16 * 4;
    if (p.lds_gu > 160 * 1024) return false;
    const int nfr = inter / 128;
    const int nb = (nfr + 7) / 8;
    if (nb > 8) return false;  // inter <= 8192
    p.nb_d = nb == 5 ? 6 : (nb == 7 ? 8 : nb);
    p.trd = down_tiles(p.nb_d);
    if (hidden % (16 * p.trd)) return false;
    p.waves_d = (nfr + p.nb_d - 1) / p.nb_d;
    const int span = p.waves_d * p.nb_d;
    p.pieces = shared_inter > 0 ? (shared_inter / 128 + span - 1) / span : 0;
    p.lds_d = (size_t)p.waves_d * p.trd * 1024;
    p.inter_pad = inter > shared_inter ? inter : shared_inter;
    p.bytes = p.inter_off + (size_t)(max_entries + T) * p.inter_pad * 2;
    if (T > kGuOwnT) {  // + the fp16 copy of x the gate/up kernel stages from
        p.xh_off = (p.bytes + 255) & ~(size_t)255;
        p.bytes = p.xh_off + (size_t)T * hidden * 2;
    }
    // 5..16 tokens: the column-split down kernel when a slot's k range fits
    // its chunks (the shared expert then splits into pieces of that size)
    const int nch = (nfr + kDnCH - 1) / kDnCH;
    p.dn_ns = T > kGuOwnT && nch <= kDnMaxCh && hidden % (16 * kDnWaves * kDnTPW) == 0;
    p.nch = nch;
    p.lds_dn = 0;
    if (p.dn_ns) {
        const int kp = dn_kp(nch);
        p.pieces = shared_inter > 0 ? (shared_inter / 128 + kp - 1) / kp : 0;
        p.lds_dn = (size_t)T * kp * 256 + 768;
    }
    p.nq = p.pieces;
    plan_part(p, det, T, hidden, max_entries);
    // 5..16 tokens, hidden <= 2048: the column-split gate/up
    p.nch_gu = (nfh + kDnCH - 1) / kDnCH;
    p.gu_ns = T > kGuOwnT && p.nch_gu <= kDnMaxCh && inter % (16 * kDnWaves) == 0 &&
              shared_inter % (16 * kDnWaves) == 0;
    p.lds_gun = (size_t)T * nfh * 256 + 768;
    return true;
}

template <int FMT, bool G128, int NB>
void launch_gate_up(const MoeArgs& a, const MoePlan& p, hipStream_t st) {
    const int TR = p.tr_gu;
    const int grid = a.max_slots * (a.routed.inter / (16 * TR)) +
                     (a.has_shared ? a.shared.inter / (16 * TR) : 0);
    if (TR == 1)
        hipLaunchKernelGGL((moe_gate_up_k<FMT, G128, NB, 1>), dim3(grid), dim3(64 * p.waves_gu), p.lds_gu, st, a);
    else if (FMT == kFmtFp8 && TR == 2)
        hipLaunchKernelGGL((moe_gate_up_k<FMT, G128, NB, 2>), dim3(grid), dim3(64 * p.waves_gu), p.lds_gu, st, a);
    else
        hipLaunchKernelGGL((moe_gate_up_k<FMT, G128, NB, 4>), dim3(grid), dim3(64 * p.waves_gu), p.lds_gu, st, a);
}

template <int FMT, bool G128, int NB>
void launch_down(const MoeArgs& a, const MoePlan& p, hipStream_t st) {
    const dim3 grid(a.hidden / (16 * down_tiles(NB)), a.max_slots + (a.has_shared ? p.pieces : 0));
    hipLaunchKernelGGL((moe_down_k<FMT, G128, NB, down_tiles(NB)>), grid, dim3(64 * p.waves_d), p.lds_d,
                       st, a);
}

template <int FMT, bool G128>
void launch_gate_up_ns(const MoeArgs& a, const MoePlan& p, hipStream_t st) {
    const int gw = 16 * kDnWaves;
    const dim3 grid(a.max_slots * (a.routed.inter / gw) + (a.has_shared ? a.shared.inter / gw : 0));
    const dim3 blk(64 * kDnWaves);
    switch (p.nch_gu) {
#define GU_CASE(n) \
    case n: hipLaunchKernelGGL((moe_gate_up_ns<FMT, G128, n>), grid, blk, p.lds_gun, st, a); break;
        GU_CASE(1) GU_CASE(2) GU_CASE(3) GU_CASE(4) GU_CASE(5) GU_CASE(6) GU_CASE(7)
        default: hipLaunchKernelGGL((moe_gate_up_ns<FMT, G128, 8>), grid, blk, p.lds_gun, st, a); break;
#undef GU_CASE
    }
}

template <int FMT, bool G128>
void launch_down_ns(const MoeArgs& a, const MoePlan& p, hipStream_t st) {
    const dim3 grid(a.hidden / (16 * kDnWaves * kDnTPW), a.max_slots + (a.has_shared ? p.pieces : 0));
    const dim3 blk(64 * kDnWaves);
    switch (p.nch) {
#define DN_CASE(n) \
    case n: hipLaunchKernelGGL((moe_down_ns<FMT, G128, n>), grid, blk, p.lds_dn, st, a); break;
        DN_CASE(1) DN_CASE(2) DN_CASE(3) DN_CASE(4) DN_CASE(5) DN_CASE(6) DN_CASE(7)
        default: hipLaunchKernelGGL((moe_down_ns<FMT, G128, 8>), grid, blk, p.lds_dn, st, a); break;
#undef DN_CASE
    }
}

template <int FMT, bool G128>
void launch_grouped_pair(const MoeArgs& a, dim3 gu, dim3 dn, hipStream_t st) {
    if constexpr (FMT == kFmtInt4) {
        constexpr int GW = kMrGuWaves, GD = kMrGuD, DW = kMrDnWaves, DD = kMrDnD;
        hipLaunchKernelGGL((moe_gemm_rk<0, G128, GW, GD>), dim3(gu.x * kMgWaves / GW, gu.y), dim3(64 * GW),
                           (size_t)(GD + 1) * kMgABytes, st, a);
        hipLaunchKernelGGL((moe_gemm_rk<1, G128, DW, DD>), dim3(dn.x * kMgWaves / DW, dn.y), dim3(64 * DW),
                           (size_t)(DD + 1) * kMgABytes, st, a);
    } else {
        hipLaunchKernelGGL((moe_gemm_k<0, G128, FMT>), gu, dim3(64 * kMgWaves), mg_lds(FMT), st, a);
        hipLaunchKernelGGL((moe_gemm_k<1, G128, FMT>), dn, dim3(64 * kMgWaves), mg_lds(FMT), st, a);
    }
}

void launch_combine(const MoeArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(moe_combine_k, dim3((a.hidden + 255) / 256, a.T), dim3(256), 0, st, a);
}

void moe_launch_grouped(const MoeArgs& a, hipStream_t st) {
    const int n8 = a.T * a.hidden / 8;
    if (!a.xh_ready)
        hipLaunchKernelGGL(x_to_f16_k, dim3((n8 + 255) / 256 < 1024 ? (n8 + 255) / 256 : 1024), dim3(256), 0,
                           st, a.x, const_cast<uint16_t*>(a.xh), n8);
    const int slots = a.max_slots + (a.has_shared ? 1 : 0);
    const int inter_max = a.routed.inter > a.shared.inter ? a.routed.inter : a.shared.inter;
    const dim3 gu(inter_max / (16 * kMgWaves), slots), dn(a.hidden / (32 * kMgWaves), slots);
    if (a.fmt == kFmtFp8)
        launch_grouped_pair<kFmtFp8, true>(a, gu, dn, st);
    else if (a.fmt == kFmtMx4)
        launch_grouped_pair<kFmtMx4, true>(a, gu, dn, st);
    else if (a.gs == 128)
        launch_grouped_pair<kFmtInt4, true>(a, gu, dn, st);
    else
        launch_grouped_pair<kFmtInt4, false>(a, gu, dn, st);
    if (a.det) launch_combine(a, st);
}

template <int FMT, bool G128>
void moe_launch(const MoeArgs& a, const MoePlan& p, hipStream_t st) {
    if (a.T > kGuOwnT && !a.xh_ready) {
        const int n8 = a.T * a.hidden / 8;
        hipLaunchKernelGGL(x_to_f16_k, dim3((n8 + 255) / 256), dim3(256), 0, st, a.x,
                           const_cast<uint16_t*>(a.xh), n8);
    }
    if (p.gu_ns) {
        launch_gate_up_ns<FMT, G128>(a, p, st);
    } else {
        switch (p.nb_gu) {
            case 1: launch_gate_up<FMT, G128, 1>(a, p, st); break;
            case 2: launch_gate_up<FMT, G128, 2>(a, p, st); break;
            case 3: launch_gate_up<FMT, G128, 3>(a, p, st); break;
            default: launch_gate_up<FMT, G128, 4>(a, p, st); break;
        }
    }
    if (p.dn_ns) {
        launch_down_ns<FMT, G128>(a, p, st);
    } else {
        switch (p.nb_d) {
            case 1: launch_down<FMT, G128, 1>(a, p, st); break;
            case 2: launch_down<FMT, G128, 2>(a, p, st); break;
            case 3: launch_down<FMT, G128, 3>(a, p, st); break;
            case 4: launch_down<FMT, G128, 4>(a, p, st); break;
            case 6: launch_down<FMT, G128, 6>(a, p, st); break;
            default: launch_down<FMT, G128, 8>(a, p, st); break;
        }
    }
    if (a.det) launch_combine(a, st);
}

}  // namespace

extern "C" {

int fastllm_int4_rowmajor_gemv(const void* x, int x_fp32, const uint8_t* qweight,
                               const void* scales, const void* zeros, void* y, int y_fp32, int M,
                               int out_f, int in_f, int group_size, void* stream) {
    if (!x || !qweight || !scales || !zeros || !y || M <= 0 || out_f <= 0 || in_f <= 0) return 1;
    if (in_f % 128 || (group_size != 32 && group_size != 64 && group_size != 128)) return 1;
    if (!fl_aligned(x, 16) || !fl_aligned(qweight, 16)) return 1;
    if (!fl_current_device_supported()) return 2;
    return rm_gemv_entry<false>("fastllm_int4_rowmajor_gemv", x, x_fp32, qweight, scales, zeros, y,
                                y_fp32, M, out_f, in_f, group_size, group_size == 128, stream);
}

int fastllm_int4_group_gemv(const void* x, int x_fp32, const uint8_t* data, const float* scales,
                            const float* zeros, void* y, int y_fp32, int M, int out_f, int in_f,
                            int group_size, void* stream) {
    if (!x || !data || !scales || !zeros || !y || M <= 0 || out_f <= 0 || in_f <= 0) return 1;
    if (in_f % 128 || group_size <= 0 || in_f % group_size) return 1;
    if (group_size != 32 && group_size != 64 && group_size % 128) return 1;
    if (!fl_aligned(x, 16) || !fl_aligned(data, 16)) return 1;
    if (!fl_current_device_supported()) return 2;
    return rm_gemv_entry<true>("fastllm_int4_group_gemv", x, x_fp32, data, scales, zeros, y, y_fp32,
                               M, out_f, in_f, group_size, group_size % 128 == 0, stream);
}

int fastllm_gate_matvec(const float* x, const void* gate_w, const void* shared_gate_w,
                        float* logits, float* shared_logit, int T, int E, int hidden,
                        void* stream) {
    if (!x || !gate_w || !logits || T <= 0 || E <= 0 || hidden <= 0) return 1;
    if (shared_gate_w && !shared_logit) return 1;
    if (!fl_current_device_supported()) return 2;
    const int rows = E + (shared_gate_w ? 1 : 0);
    hipLaunchKernelGGL(gate_matvec_k, dim3(rows), dim3(256), 0, (hipStream_t)stream, x,
                       (const uint16_t*)gate_w, (const uint16_t*)shared_gate_w, logits,
                       shared_logit, T, E, hidden);
    return finish("fastllm_gate_matvec");
}

int fastllm_route_topk(const float* logits, int T, int E, int top_k, int scoring, int norm,
                       float routed_scaling, const float* e_score_bias, int n_group,
                       int topk_group, int* topk_ids, float* topk_w, float* rw,
                       const float* shared_logit, float* shared_coef, int* n_active,
                       int* active, int* offsets, int* tok, float* tokw, void* stream) {
    if (!logits || T <= 0 || E <= 0 || E > 256 || top_k <= 0 || top_k > 16 || top_k > E) return 1;
    if (!topk_ids || !topk_w) return 1;
    if (scoring != 0 && scoring != 1) return 1;
    if (n_group > 1 && (E % n_group || n_group > 64)) return 1;
    if (n_active && (!active || !offsets || !tok || !tokw)) return 1;
    // the multi-workgroup list builder stages ids, weights and a token bitmap in LDS
    if (n_active && T > 16 && ((long)T * top_k > kListIds || (long)E * ((T + 31) / 32) > kListSel))
        return 1;
    if (!fl_current_device_supported()) return 2;
    const MoeLists lists{n_active, active, offsets, tok, tokw};
    RouteArgs a{logits, e_score_bias, shared_logit, T, E, top_k, scoring, norm, n_group,
                topk_group, routed_scaling, topk_ids, topk_w, rw, shared_coef, lists};
    hipStream_t st = (hipStream_t)stream;
    const int wpb = T <= 16 ? T : kRouteTpb;
    const int grid = T <= 16 ? 1 : (T + kRouteTpb - 1) / kRouteTpb;
    launch_route(a, grid, 64 * wpb, st);
    int rc = finish("fastllm_route_topk");
    if (rc) return rc;
    if (grid > 1 && n_active) {
        hipLaunchKernelGGL(route_lists_k, dim3(1), dim3(1024), 0, st, topk_ids, topk_w, T, top_k,
                           E, lists);
        rc = finish("fastllm_route_topk");
    }
    return rc;
}

int fastllm_moe_build_lists(const float* rw, const float* slot_coef, const int* cand, int T,
                            int E, int S, int* n_active, int* active, int* offsets, int* tok,
                            float* tokw, void* stream) {
    if (T <= 0 || T > 16 || E <= 0 || S <= 0 || S > 256 || (!rw && !slot_coef)) return 1;
    if (rw && !cand && S > E) return 1;
    if (!n_active || !active || !offsets || !tok || !tokw) return 1;
    if (!fl_current_device_supported()) return 2;
    const MoeLists lists{n_active, active, offsets, tok, tokw};
    hipLaunchKernelGGL(slot_lists_k, dim3(1), dim3(256), 0, (hipStream_t)stream,
                       slot_coef ? nullptr : rw, slot_coef, cand, T, E, S, lists);
    return finish("fastllm_moe_build_lists");
}

int fastllm_moe_int4_tile_repack(const uint8_t* qweight, const void* scales, const void* zeros,
                                 uint8_t* qtile, uint32_t* sz, long rows, int in_f,
                                 int group_size, void* stream) {
    if (!qweight || !scales || !zeros || !qtile || !sz || rows <= 0 || rows % 16) return 1;
    if (in_f <= 0 || in_f % 128 || (group_size != 32 && group_size != 64 && group_size != 128))
        return 1;
    if (!fl_aligned(qweight, 16) || !fl_aligned(qtile, 16)) return 1;
    if (!fl_current_device_supported()) return 2;
    const long work = rows * (in_f / 32);
    const int grid = (int)((work + 255) / 256 < 8192 ? (work + 255) / 256 : 8192);
    hipLaunchKernelGGL(moe_tile_repack_k, dim3(grid), dim3(256), 0, (hipStream_t)stream, qweight,
                       (const uint16_t*)scales, (const uint16_t*)zeros, qtile, sz, rows, in_f,
                       in_f / group_size);
    return finish("fastllm_moe_int4_tile_repack");
}

int fastllm_moe_fp8_tile_repack(const uint8_t* q, uint8_t* qtile, long rows, int in_f, void* stream) {
    if (!q || !qtile || rows <= 0 || rows % 16 || in_f <= 0 || in_f % 128) return 1;
    if (!fl_aligned(q, 16) || !fl_aligned(qtile, 16)) return 1;
    if (!fl_current_device_supported()) return 2;
    const size_t n = (size_t)rows * in_f / 16;
    const int grid = (int)((n + 255) / 256 < 8192 ? (n + 255) / 256 : 8192);
    hipLaunchKernelGGL(moe_fp8_tile_repack_k, dim3(grid), dim3(256), 0, (hipStream_t)stream, q, qtile, rows,
                       in_f);
    return finish("fastllm_moe_fp8_tile_repack");
}

int fastllm_moe_mxfp4_tile_repack(const uint8_t* codes, const uint8_t* e8, uint8_t* qtile, uint32_t* e8w,
                                  long rows, int in_f, void* stream) {
    if (!codes || !e8 || !qtile || !e8w || rows <= 0 || rows % 16 || in_f <= 0 || in_f % 128) return 1;
    if (!fl_aligned(codes, 4) || !fl_aligned(e8, 4) || !fl_aligned(qtile, 16) || !fl_aligned(e8w, 4))
        return 1;
    if (!fl_current_device_supported()) return 2;
    const size_t n = (size_t)rows * (in_f / 128) * 4;
    const int grid = (int)((n + 255) / 256 < 8192 ? (n + 255) / 256 : 8192);
    hipLaunchKernelGGL(moe_mxfp4_tile_repack_k, dim3(grid), dim3(256), 0, (hipStream_t)stream, codes, e8,
                       qtile, e8w, rows, in_f);
    return finish("fastllm_moe_mxfp4_tile_repack");
}

int fastllm_mxfp4_gemv(const void* A, const uint8_t* qtile, const uint32_t* e8w, void* C, int M, int N, int K,
                       void* stream) {
    if (!A || !qtile || !e8w || !C || M <= 0 || N <= 0 || N % 16 || K <= 0 || K % 128) return 1;
    if (M <= kMxGemmMinM && K > 16 * 6 * 128) return 1;  // the GEMV: at most 16 waves of 6 blocks
    if (!fl_aligned(A, 16) || !fl_aligned(qtile, 16) || !fl_aligned(e8w, 4) || !fl_aligned(C, 2)) return 1;
    if (!fl_current_device_supported()) return 2;
    const uint16_t* a = static_cast<const uint16_t*>(A);
    uint16_t* y = static_cast<uint16_t*>(C);
    hipStream_t st = (hipStream_t)stream;
    if (M > kMxGemmMinM) {
        if ((size_t)M * K * 2 >= (1ull << 31) || (size_t)N * K / 2 >= (1ull << 31)) return 1;  // 32-bit buffer ranges
        const int tiles = ((N + kMxBN - 1) / kMxBN) * ((M + kMxBM - 1) / kMxBM);
        hipLaunchKernelGGL(mx4_gemm_mfma, dim3(tiles), dim3(512), kMxGemmLds, st, reinterpret_cast<const f16*>(a),
                           qtile, e8w, reinterpret_cast<f16*>(y), M, N, K);
        return finish("fastllm_mxfp4_gemv");
    }
    const Mx4Cfg c = mx4_cfg(N, K);
#define MX4_CASE(nb)                                                           \
    case nb:                                                                   \
        if (c.tr == 2)                                                         \
            launch_mx4_gemv<nb, 2, 1>(c, a, qtile, e8w, y, M, N, K, st);       \
        else                                                                   \
            launch_mx4_gemv<nb, 1, 1>(c, a, qtile, e8w, y, M, N, K, st);       \
        break;
    switch (c.nb) {
        MX4_CASE(1) MX4_CASE(2) MX4_CASE(4)
        default: launch_mx4_gemv<3, 1, 2>(c, a, qtile, e8w, y, M, N, K, st); break;
    }
#undef MX4_CASE
    return finish("fastllm_mxfp4_gemv");
}

int fastllm_moe_int4_tile_unpack(const uint8_t* qtile, const uint32_t* sz, uint8_t* qweight,
                                 void* scales, void* zeros, long rows, int in_f, int group_size,
                                 void* stream) {
    if (!qweight || !scales || !zeros || !qtile || !sz || rows <= 0 || rows % 16) return 1;
    if (in_f <= 0 || in_f % 128 || (group_size != 32 && group_size != 64 && group_size != 128))
        return 1;
    if (!fl_aligned(qweight, 16) || !fl_aligned(qtile, 16)) return 1;
    if (!fl_current_device_supported()) return 2;
    const long work = rows * (in_f / 32);
    const int grid = (int)((work + 255) / 256 < 8192 ? (work + 255) / 256 : 8192);
    hipLaunchKernelGGL(moe_tile_unpack_k, dim3(grid), dim3(256), 0, (hipStream_t)stream, qtile, sz,
                       qweight, (uint16_t*)scales, (uint16_t*)zeros, rows, in_f, in_f / group_size);
    return finish("fastllm_moe_int4_tile_unpack");
}

size_t fastllm_moe_int4_workspace_bytes(int T, int hidden, int inter, int shared_inter,
                                        int max_entries) {
    MoePlan p;
    return moe_plan(T, hidden, inter, shared_inter, max_entries, p) ? p.bytes : 0;
}

size_t fastllm_moe_workspace_bytes_ex(int T, int hidden, int inter, int shared_inter,
                                      int max_entries, int flags) {
    if (flags & ~kMoeFlags) return 0;
    MoePlan p;
    return moe_plan(T, hidden, inter, shared_inter, max_entries, p, kFmtInt4,
                    (flags & kMoeDeterministic) != 0)
               ? p.bytes
               : 0;
}

// The fused MoE entry; launch = false only validates the arguments.
static int moe_fused_impl(const float* x, int T, int hidden, int group_size, int E, int inter,
                          const uint8_t* gq, const uint32_t* gsz, const uint8_t* uq,
                          const uint32_t* usz, const uint8_t* dq, const uint32_t* dsz,
                          int shared_inter, const uint8_t* sgq, const uint32_t* sgsz,
                          const uint8_t* suq, const uint32_t* susz, const uint8_t* sdq,
                          const uint32_t* sdsz, const float* shared_coef, const int* n_active,
                          const int* active, const int* offsets, const int* tok,
                          const float* tokw, int max_slots, int max_entries, void* workspace,
                          size_t workspace_bytes, float* y, void* stream, bool launch,
                          const RouteArgs* fuse = nullptr, bool xh_ready = false,
                          int fmt = kFmtInt4, int flags = 0) {
    if (!x || !y || E <= 0 || !gq || !gsz || !uq || !usz || !dq || !dsz) return 1;
    if (fmt == kFmtInt4 && group_size != 32 && group_size != 64 && group_size != 128) return 1;
    if (fmt == kFmtFp8 && group_size != 128) return 1;
    if (fmt == kFmtMx4 && group_size != 32) return 1;
    if (fmt != kFmtInt4 && (inter % 128 || hidden % 128)) return 1;
    if (fmt < kFmtInt4 || fmt > kFmtMx4) return 1;
    if (!n_active || !active || !offsets || !tok || !tokw) return 1;
    if (max_slots <= 0 || max_entries <= 0) return 1;
    if (flags & ~kMoeFlags) return 1;
    const bool det = (flags & kMoeDeterministic) != 0;
    if (det && max_slots > kCombineMaxEnt) return 1;  // a token's entries fit the combine's list
    const bool has_shared = shared_inter > 0;
    if (has_shared && (!sgq || !sgsz || !suq || !susz || !sdq || !sdsz)) return 1;
    MoePlan p;
    if (!moe_plan(T, hidden, inter, has_shared ? shared_inter : 0, max_entries, p, fmt, det)) return 1;
    if (!workspace || workspace_bytes < p.bytes || !fl_aligned(workspace, 16)) return 1;
    if (!fl_aligned(x, 16) || !fl_aligned(y, 16)) return 1;
    const bool al = fl_aligned(gq, 16) && fl_aligned(uq, 16) && fl_aligned(dq, 16) &&
                    (!has_shared || (fl_aligned(sgq, 16) && fl_aligned(suq, 16) && fl_aligned(sdq, 16)));
    if (!al) return 1;
    if (!fl_current_device_supported()) return 2;
    if (!launch) return 0;
    MoeArgs a;
    a.x = x;
    a.T = T;
    a.hidden = hidden;
    a.gs = group_size;
    a.E = E;
    a.routed = MoeExperts{gq, gsz, uq, usz, dq, dsz, inter};
    a.shared = MoeExperts{sgq, sgsz, suq, susz, sdq, sdsz, has_shared ? shared_inter : 0};
    a.has_shared = has_shared ? 1 : 0;
    a.pieces = p.pieces;
    a.scoef = shared_coef;
    a.n_active = n_active;
    a.active = active;
    a.offsets = offsets;
    a.tok = tok;
    a.tokw = tokw;
    a.max_slots = max_slots;
    a.max_entries = max_entries;
    a.inter_pad = p.inter_pad;
    a.inter_buf = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + p.inter_off);
    a.xh = p.xh_off ? reinterpret_cast<const uint16_t*>(static_cast<char*>(workspace) + p.xh_off)
                    : nullptr;
    a.xh_ready = xh_ready ? 1 : 0;
    a.y = y;
    a.fuse_route = (fuse && T == 1 && !p.grouped) ? 1 : 0;
    if (a.fuse_route) a.ra = *fuse;
    a.fmt = fmt;
    a.det = det ? 1 : 0;
    a.nq = p.nq;
    a.part = det ? reinterpret_cast<float*>(static_cast<char*>(workspace) + p.part_off) : nullptr;
    hipStream_t st = (hipStream_t)stream;
    if (p.grouped)
        moe_launch_grouped(a, st);
    else if (fmt == kFmtFp8)
        moe_launch<kFmtFp8, true>(a, p, st);
    else if (fmt == kFmtMx4)
        moe_launch<kFmtMx4, true>(a, p, st);
    else if (group_size == 128)
        moe_launch<kFmtInt4, true>(a, p, st);
    else
        moe_launch<kFmtInt4, false>(a, p, st);
    return finish("fastllm_moe_int4_fused");
}

int fastllm_moe_int4_fused(const float* x, int T, int hidden, int group_size, int E, int inter,
                           const uint8_t* gq, const uint32_t* gsz, const uint8_t* uq,
                           const uint32_t* usz, const uint8_t* dq, const uint32_t* dsz,
                           int shared_inter, const uint8_t* sgq, const uint32_t* sgsz,
                           const uint8_t* suq, const uint32_t* susz, const uint8_t* sdq,
                           const uint32_t* sdsz, const float* shared_coef, const int* n_active,
                           const int* active, const int* offsets, const int* tok,
                           const float* tokw, int max_slots, int max_entries, void* workspace,
                           size_t workspace_bytes, float* y, void* stream) {
    return moe_fused_impl(x, T, hidden, group_size, E, inter, gq, gsz, uq, usz, dq, dsz, shared_inter,
                          sgq, sgsz, suq, susz, sdq, sdsz, shared_coef, n_active, active, offsets,
                          tok, tokw, max_slots, max_entries, workspace, workspace_bytes, y, stream,
                          true);
}

int fastllm_moe_lowp_fused(int format, const float* x, int T, int hidden, int group_size, int E,
                           int inter, const uint8_t* gq, const uint32_t* gsz, const uint8_t* uq,
                           const uint32_t* usz, const uint8_t* dq, const uint32_t* dsz, int shared_inter,
                           const uint8_t* sgq, const uint32_t* sgsz, const uint8_t* suq,
                           const uint32_t* susz, const uint8_t* sdq, const uint32_t* sdsz,
                           const float* shared_coef, const int* n_active, const int* active,
                           const int* offsets, const int* tok, const float* tokw, int max_slots,
                           int max_entries, void* workspace, size_t workspace_bytes, float* y,
                           void* stream) {
    if (format != kFmtFp8 && format != kFmtMx4) return 1;
    return moe_fused_impl(x, T, hidden, group_size, E, inter, gq, gsz, uq, usz, dq, dsz, shared_inter,
                          sgq, sgsz, suq, susz, sdq, sdsz, shared_coef, n_active, active, offsets,
                          tok, tokw, max_slots, max_entries, workspace, workspace_bytes, y, stream,
                          true, nullptr, false, format);
}

// Router + fused MoE (body of fastllm_moe_int4_routed and of its
// static-scratch variant): up to 16 tokens the decode kernels, above that
// the grouped GEMMs, the router's spare workgroups writing the fp16 copy of
// x and its last routing workgroup the lists (a counter in the workspace,
// which must be zero-filled once; every call leaves it at zero).  `scratch_of`, when given, supplies the
// workspace once every argument has been validated (nullptr -> rc 2).
static int moe_routed_impl(const float* logits, int top_k, int scoring, int norm,
                           float routed_scaling, const float* e_score_bias, int n_group,
                           int topk_group, const float* shared_logit, int* topk_ids,
                           float* topk_w, float* rw, float* shared_coef, int* n_active,
                           int* active, int* offsets, int* tok, float* tokw, const float* x,
                           int T, int hidden, int group_size, int E, int inter,
                           const uint8_t* gq, const uint32_t* gsz, const uint8_t* uq,
                           const uint32_t* usz, const uint8_t* dq, const uint32_t* dsz,
                           int shared_inter, const uint8_t* sgq, const uint32_t* sgsz,
                           const uint8_t* suq, const uint32_t* susz, const uint8_t* sdq,
                           const uint32_t* sdsz, void* workspace, size_t workspace_bytes,
                           float* y, void* stream, void* (*scratch_of)() = nullptr,
                           int fmt = kFmtInt4, int flags = 0) {
    if (!logits || T <= 0 || E <= 0 || E > 256 || top_k <= 0 || top_k > 16 || top_k > E) return 1;
    // above 16 tokens the router's last workgroup builds the lists in LDS
    if (T > 16 && ((long)T * top_k > kListIds || (long)E * ((T + 31) / 32) > kListSel)) return 1;
    if (!topk_ids || !topk_w || !n_active || !active || !offsets || !tok || !tokw) return 1;
    if (scoring != 0 && scoring != 1) return 1;
    if (n_group > 1 && (E % n_group || n_group > 64)) return 1;
    if (shared_inter > 0 && shared_logit && !shared_coef) return 1;
    const int max_entries = T * top_k, max_slots = E < max_entries ? E : max_entries;
    if (scratch_of) {
        MoePlan sp;
        if (!moe_plan(T, hidden, inter, shared_inter > 0 ? shared_inter : 0, max_entries, sp, fmt,
                      (flags & kMoeDeterministic) != 0))
            return 1;
        if (sp.bytes > workspace_bytes) {
            fprintf(stderr,
                    "fastllm_moe_int4_routed_noalloc: this shape needs %zu bytes of scratch; the "
                    "static scratch holds %zu (use fastllm_moe_int4_routed with a workspace)\n",
                    sp.bytes, workspace_bytes);
            return 1;
        }
        if (!fl_current_device_supported()) return 2;
        workspace = scratch_of();
        if (!workspace) return 2;
    }
    // the MoE arguments are checked before anything is launched
    const int rc = moe_fused_impl(x, T, hidden, group_size, E, inter, gq, gsz, uq, usz, dq, dsz,
                                  shared_inter, sgq, sgsz, suq, susz, sdq, sdsz, shared_coef,
                                  n_active, active, offsets, tok, tokw, max_slots, max_entries,
                                  workspace, workspace_bytes, y, stream, false, nullptr, false, fmt,
                                  flags);
    if (rc) return rc;
    const MoeLists lists{n_active, active, offsets, tok, tokw};
    const RouteArgs r{logits, e_score_bias, shared_logit, T, E, top_k, scoring, norm, n_group,
                      topk_group, routed_scaling, topk_ids, topk_w, rw, shared_coef, lists};
    if (T == 1)  // routed inside the gate/up launch
        return moe_fused_impl(x, T, hidden, group_size, E, inter, gq, gsz, uq, usz, dq, dsz,
                              shared_inter, sgq, sgsz, suq, susz, sdq, sdsz,
                              shared_logit ? shared_coef : nullptr, n_active, active, offsets, tok,
                              tokw, max_slots, max_entries, workspace, workspace_bytes, y, stream,
                              true, &r, false, fmt, flags);
    // T > 4: the router also writes the fp16 token rows the gate/up kernel
    // stages (the plan was validated above)
    MoePlan p;
    moe_plan(T, hidden, inter, shared_inter > 0 ? shared_inter : 0, max_entries, p, fmt,
             (flags & kMoeDeterministic) != 0);
    RouteArgs rx = r;
    // routing workgroups: one of T waves (T <= 16), else kRouteTpb tokens
    // each, the last to finish building the lists
    const int tpw = T <= 16 ? T : kRouteTpb;
    const int rgrid = T <= 16 ? 1 : (T + kRouteTpb - 1) / kRouteTpb;
    if (T > 16) rx.arrive = static_cast<int*>(workspace);  // the counter region
    if (p.xh_off) {
        rx.x = x;
        rx.xh = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + p.xh_off);
        rx.hidden = hidden;
        const int n8 = T * hidden / 8, per = 64 * tpw;
        rx.xh_blocks = (n8 + per - 1) / per;
    }
    hipStream_t st = (hipStream_t)stream;
    launch_route(rx, rgrid + rx.xh_blocks, 64 * tpw, st);
    const int rr = finish("fastllm_moe_int4_routed");
    if (rr) return rr;
    return moe_fused_impl(x, T, hidden, group_size, E, inter, gq, gsz, uq, usz, dq, dsz,
                          shared_inter, sgq, sgsz, suq, susz, sdq, sdsz,
                          shared_logit ? shared_coef : nullptr, n_active, active, offsets, tok, tokw,
                          max_slots, max_entries, workspace, workspace_bytes, y, stream, true,
                          nullptr, p.xh_off != 0, fmt, flags);
}

}  // extern "C"

// ---------------------------------------------- static scratch (no-alloc entry)
// Workspace of fastllm_moe_int4_routed_noalloc: one copy per GPU, held until
// the process ends.  In host code `scratch` only names the symbol; kernels
// get the device address that hipGetSymbolAddress returns for the current
// device (moe_scratch_ptr).  Every call on a GPU shares it, so calls that
// overlap on one GPU (two streams, two threads) race on it.
constexpr size_t kMoeScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kMoeScratchBytes];

// Device address of `scratch` on the calling thread's current device,
// resolved once per device with that device current (nullptr on failure).
static void* moe_scratch_ptr() {
    static std::atomic<void*> addr[64];
    static std::mutex mu;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        (void)hipGetLastError();
        return nullptr;
    }
    void* p = addr[dev].load(std::memory_order_acquire);
    if (p) return p;
    std::lock_guard<std::mutex> lock(mu);
    p = addr[dev].load(std::memory_order_relaxed);
    if (!p) {
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            fprintf(stderr, "fastllm_moe_int4_routed_noalloc: scratch address on device %d: %s\n",
                    dev, hipGetErrorString(e));
            (void)hipGetLastError();
            return nullptr;
        }
        addr[dev].store(p, std::memory_order_release);
    }
    return p;
}

extern "C" {

int fastllm_moe_int4_routed(const float* logits, int top_k, int scoring, int norm,
                            float routed_scaling, const float* e_score_bias, int n_group,
                            int topk_group, const float* shared_logit, int* topk_ids,
                            float* topk_w, float* rw, float* shared_coef, int* n_active,
                            int* active, int* offsets, int* tok, float* tokw, const float* x,
                            int T, int hidden, int group_size, int E, int inter,
                            const uint8_t* gq, const uint32_t* gsz, const uint8_t* uq,
                            const uint32_t* usz, const uint8_t* dq, const uint32_t* dsz,
                            int shared_inter, const uint8_t* sgq, const uint32_t* sgsz,
                            const uint8_t* suq, const uint32_t* susz, const uint8_t* sdq,
                            const uint32_t* sdsz, void* workspace, size_t workspace_bytes, float* y,
                            void* stream) {
    return moe_routed_impl(logits, top_k, scoring, norm, routed_scaling, e_score_bias, n_group,
                           topk_group, shared_logit, topk_ids, topk_w, rw, shared_coef, n_active,
                           active, offsets, tok, tokw, x, T, hidden, group_size, E, inter, gq, gsz,
                           uq, usz, dq, dsz, shared_inter, sgq, sgsz, suq, susz, sdq, sdsz,
                           workspace, workspace_bytes, y, stream);
}

int fastllm_moe_lowp_routed(int format, const float* logits, int top_k, int scoring, int norm,
                            float routed_scaling, const float* e_score_bias, int n_group,
                            int topk_group, const float* shared_logit, int* topk_ids,
                            float* topk_w, float* rw, float* shared_coef, int* n_active,
                            int* active, int* offsets, int* tok, float* tokw, const float* x,
                            int T, int hidden, int group_size, int E, int inter,
                            const uint8_t* gq, const uint32_t* gsz, const uint8_t* uq,
                            const uint32_t* usz, const uint8_t* dq, const uint32_t* dsz,
                            int shared_inter, const uint8_t* sgq, const uint32_t* sgsz,
                            const uint8_t* suq, const uint32_t* susz, const uint8_t* sdq,
                            const uint32_t* sdsz, void* workspace, size_t workspace_bytes, float* y,
                            void* stream) {
    if (format != kFmtFp8 && format != kFmtMx4) return 1;
    return moe_routed_impl(logits, top_k, scoring, norm, routed_scaling, e_score_bias, n_group,
                           topk_group, shared_logit, topk_ids, topk_w, rw, shared_coef, n_active,
                           active, offsets, tok, tokw, x, T, hidden, group_size, E, inter, gq, gsz,
                           uq, usz, dq, dsz, shared_inter, sgq, sgsz, suq, susz, sdq, sdsz,
                           workspace, workspace_bytes, y, stream, nullptr, format);
}

int fastllm_moe_int4_routed_noalloc(const float* logits, int top_k, int scoring, int norm,
                                    float routed_scaling, const float* e_score_bias, int n_group,
                                    int topk_group, const float* shared_logit, int* topk_ids,
                                    float* topk_w, float* rw, float* shared_coef, int* n_active,
                                    int* active, int* offsets, int* tok, float* tokw,
                                    const float* x, int T, int hidden, int group_size, int E,
                                    int inter, const uint8_t* gq, const uint32_t* gsz,
                                    const uint8_t* uq, const uint32_t* usz, const uint8_t* dq,
                                    const uint32_t* dsz, int shared_inter, const uint8_t* sgq,
                                    const uint32_t* sgsz, const uint8_t* suq, const uint32_t* susz,
                                    const uint8_t* sdq, const uint32_t* sdsz, float* y,
                                    void* stream) {
    return moe_routed_impl(logits, top_k, scoring, norm, routed_scaling, e_score_bias, n_group,
                           topk_group, shared_logit, topk_ids, topk_w, rw, shared_coef, n_active,
                           active, offsets, tok, tokw, x, T, hidden, group_size, E, inter, gq, gsz,
                           uq, usz, dq, dsz, shared_inter, sgq, sgsz, suq, susz, sdq, sdsz, nullptr,
                           kMoeScratchBytes, y, stream, moe_scratch_ptr);
}

int fastllm_moe_fused_ex(int format, int flags, const float* x, int T, int hidden, int group_size,
                         int E, int inter, const uint8_t* gq, const uint32_t* gsz, const uint8_t* uq,
                         const uint32_t* usz, const uint8_t* dq, const uint32_t* dsz, int shared_inter,
                         const uint8_t* sgq, const uint32_t* sgsz, const uint8_t* suq,
                         const uint32_t* susz, const uint8_t* sdq, const uint32_t* sdsz,
                         const float* shared_coef, const int* n_active, const int* active,
                         const int* offsets, const int* tok, const float* tokw, int max_slots,
                         int max_entries, void* workspace, size_t workspace_bytes, float* y,
                         void* stream) {
    if (format < kFmtInt4 || format > kFmtMx4) return 1;
    return moe_fused_impl(x, T, hidden, group_size, E, inter, gq, gsz, uq, usz, dq, dsz, shared_inter,
                          sgq, sgsz, suq, susz, sdq, sdsz, shared_coef, n_active, active, offsets,
                          tok, tokw, max_slots, max_entries, workspace, workspace_bytes, y, stream,
                          true, nullptr, false, format, flags);
}

int fastllm_moe_routed_ex(int format, int flags, const float* logits, int top_k, int scoring,
                          int norm, float routed_scaling, const float* e_score_bias, int n_group,
                          int topk_group, const float* shared_logit, int* topk_ids, float* topk_w,
                          float* rw, float* shared_coef, int* n_active, int* active, int* offsets,
                          int* tok, float* tokw, const float* x, int T, int hidden, int group_size,
                          int E, int inter, const uint8_t* gq, const uint32_t* gsz,
                          const uint8_t* uq, const uint32_t* usz, const uint8_t* dq,
                          const uint32_t* dsz, int shared_inter, const uint8_t* sgq,
                          const uint32_t* sgsz, const uint8_t* suq, const uint32_t* susz,
                          const uint8_t* sdq, const uint32_t* sdsz, void* workspace,
                          size_t workspace_bytes, float* y, void* stream) {
    if (format < kFmtInt4 || format > kFmtMx4) return 1;
    return moe_routed_impl(logits, top_k, scoring, norm, routed_scaling, e_score_bias, n_group,
                           topk_group, shared_logit, topk_ids, topk_w, rw, shared_coef, n_active,
                           active, offsets, tok, tokw, x, T, hidden, group_size, E, inter, gq, gsz,
                           uq, usz, dq, dsz, shared_inter, sgq, sgsz, suq, susz, sdq, sdsz,
                           workspace, workspace_bytes, y, stream, nullptr, format, flags);
}

}  // extern "C"
