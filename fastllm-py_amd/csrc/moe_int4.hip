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
#include "npmath.cuh"

namespace {

FL_DEV uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(c));
    return r;
}

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

// ------------------------------------------------------ row-major INT4 GEMV
// Y[M, N] = X[M, K] @ dequant(W)^T, M <= 16, X/Y fp32 or fp16 (XF32/YF32).
// K % 128 == 0; group gs in {32, 64, 128}.
template <int NB, bool G128, bool XF32, bool YF32>
__global__ __launch_bounds__(1024) void rm_gemv_nb(const void* __restrict__ Xv,
                                                   const uint8_t* __restrict__ Wq,
                                                   const uint16_t* __restrict__ S,
                                                   const uint16_t* __restrict__ Z, void* __restrict__ Yv,
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

    u32x4 wv[NB];
    uint16_t sv[NB], zv[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        int kb = wave + (i < nb ? i : (nb > 0 ? nb - 1 : 0)) * nwaves;
        kb = kb < nfull ? kb : nfull - 1;
        wv[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + kb * 64 + 16 * kq));
        const int g = (kb * 128 + 32 * kq) / gs;
        sv[i] = S[(size_t)nc * G + g];
        zv[i] = Z[(size_t)nc * G + g];
    }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();

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
// Up to 256 experts (4 per lane), k <= 32.
struct RouteArgs {
    const float* logits;
    const float* bias;
    const float* slogit;  // shared-expert gate logits, optional
    int T, E, K, scoring, norm, n_group, topk_group;
    float scale;
    int* topk_ids;
    float* topk_w;
    float* rw;     // dense [T, E], optional
    float* scoef;  // sigmoid(slogit) [T], optional
    // expert-major lists (filled when the whole batch is one workgroup)
    int* n_active;
    int* active;
    int* offsets;
    int* tok;
    float* tokw;
};

__global__ __launch_bounds__(1024) void route_k(RouteArgs a) {
    __shared__ float ex[16][256];
    __shared__ int cnt[256];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int t = blockIdx.x * (blockDim.x >> 6) + wv;
    const int E = a.E;
    if (t < a.T) {
        float sel[4], p[4];
        const float* s = a.logits + (size_t)t * E;
        if (a.scoring == 0) {
            float m = -__builtin_inff();
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int e = lane + 64 * c;
                if (e < E) m = fmaxf(m, s[e]);
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int e = lane + 64 * c;
                if (e < E) ex[wv][e] = np_expf(s[e] - m);
            }
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            float z = 0.f;
            if (lane == 0) z = np_sum_f32(ex[wv], E);
            z = __shfl(z, 0, 64);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int e = lane + 64 * c;
                p[c] = (e < E) ? ex[wv][e] / z : 0.f;
                sel[c] = (e < E) ? p[c] : -__builtin_inff();
            }
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int e = lane + 64 * c;
                if (e < E) {
                    const float d = 1.0f + np_expf(-s[e]);
                    p[c] = 1.0f / d;
                    sel[c] = a.bias ? p[c] + a.bias[e] : p[c] + 0.0f;
                } else {
                    p[c] = 0.f;
                    sel[c] = -__builtin_inff();
                }
            }
        }
        if (a.n_group > 1 && a.topk_group > 0 && a.topk_group < a.n_group) {
            const int gsz = E / a.n_group;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int e = lane + 64 * c;
                if (e < E) ex[wv][e] = sel[c];
            }
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            // lane g scores group g: second largest + largest (ascending sum)
            float gscore = -__builtin_inff();
            if (lane < a.n_group) {
                float b1 = -__builtin_inff(), b2 = -__builtin_inff();
                for (int i = 0; i < gsz; ++i) {
                    const float v = ex[wv][lane * gsz + i];
                    if (v > b1) {
                        b2 = b1;
                        b1 = v;
                    } else if (v > b2) {
                        b2 = v;
                    }
                }
                gscore = gsz >= 2 ? (0.0f + b2) + b1 : 0.0f + b1;
            }
            // keep topk_group groups: rank = #groups strictly better (ties -> lower index)
            int rank = 0;
            for (int g2 = 0; g2 < a.n_group; ++g2) {
                const float o = __shfl(gscore, g2, 64);
                rank += (o > gscore || (o == gscore && g2 < lane)) ? 1 : 0;
            }
            const int keep = (lane < a.n_group && rank < a.topk_group) ? 1 : 0;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int e = lane + 64 * c;
                if (e < E) {
                    const int kg = __shfl(keep, e / gsz, 64);
                    if (!kg) sel[c] = -__builtin_inff();
                }
            }
        }
        // top-k: value desc, index asc
        int ids[16];
        float ws[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            ids[i] = 0;
            ws[i] = 0.f;
            if (i >= a.K) continue;
            float bv = -__builtin_inff();
            int bi = 0x7fffffff;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int e = lane + 64 * c;
                if (e < E && (sel[c] > bv || (sel[c] == bv && e < bi))) {
                    bv = sel[c];
                    bi = e;
                }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(bv, o, 64);
                const int oi = __shfl_xor(bi, o, 64);
                if (ov > bv || (ov == bv && oi < bi)) {
                    bv = ov;
                    bi = oi;
                }
            }
            ids[i] = bi;
            float pw = 0.f;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int e = lane + 64 * c;
                if (e == bi) {
                    pw = p[c];
                    sel[c] = -__builtin_inff();
                }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) pw += __shfl_xor(pw, o, 64);  // single nonzero lane
            ws[i] = pw;
        }
        if (a.norm) {
            // numpy row sum of the k weights (selection order), + 1e-20
            float den;
            if (a.K < 8) {
                den = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (i < a.K) den += ws[i];
            } else {
                // 8 accumulators, one more round of 8 when k == 16, then the
                // leftover elements one by one (numpy's pairwise block)
                float r[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) r[j] = ws[j];
                if (a.K == 16) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) r[j] += ws[8 + j];
                }
                den = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
#pragma unroll
                for (int i = 8; i < 16; ++i)
                    if (i < a.K && a.K < 16) den += ws[i];
            }
            den = den + 1e-20f;
#pragma unroll
            for (int i = 0; i < 16; ++i) ws[i] = ws[i] / den;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) ws[i] = ws[i] * a.scale;
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                if (i >= a.K) continue;
                a.topk_ids[(size_t)t * a.K + i] = ids[i];
                a.topk_w[(size_t)t * a.K + i] = ws[i];
            }
            if (a.scoef && a.slogit) a.scoef[t] = 1.0f / (1.0f + expf(-a.slogit[t]));
        }
        if (a.rw) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int e = lane + 64 * c;
                if (e < E) {
                    float w = 0.f;
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (i < a.K && ids[i] == e) w = ws[i];
                    a.rw[(size_t)t * E + e] = w;
                }
            }
        }
    }
    if (gridDim.x == 1 && a.n_active) {
        // expert-major lists: experts ascending, tokens ascending within one
        __syncthreads();
        __threadfence_block();
        const int TK = a.T * a.K;
        for (int e = threadIdx.x; e < E; e += blockDim.x) {
            int c = 0;
            for (int i = 0; i < TK; ++i) c += (a.topk_ids[i] == e) ? 1 : 0;
            cnt[e] = c;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            int na = 0, off = 0;
            for (int e = 0; e < E; ++e) {
                if (cnt[e] > 0) {
                    a.active[na] = e;
                    a.offsets[na] = off;
                    off += cnt[e];
                    cnt[e] = na;  // slot of expert e
                    ++na;
                } else {
                    cnt[e] = -1;
                }
            }
            a.offsets[na] = off;
            *a.n_active = na;
        }
        __syncthreads();
        for (int e = threadIdx.x; e < E; e += blockDim.x) {
            const int slot = cnt[e];
            if (slot < 0) continue;
            int w = a.offsets[slot];
            for (int tt = 0; tt < a.T; ++tt)
                for (int i = 0; i < a.K; ++i)
                    if (a.topk_ids[(size_t)tt * a.K + i] == e) {
                        a.tok[w] = tt;
                        a.tokw[w] = a.topk_w[(size_t)tt * a.K + i];
                        ++w;
                    }
        }
    }
}

// Expert-major lists for batches routed by several workgroups (same layout
// as the single-workgroup path above).
__global__ __launch_bounds__(1024) void route_lists_k(const int* __restrict__ ids,
                                                      const float* __restrict__ tw, int T, int K,
                                                      int E, int* n_active, int* active,
                                                      int* offsets, int* tok, float* tokw) {
    __shared__ int cnt[1024];
    const int TK = T * K;
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        int c = 0;
        for (int i = 0; i < TK; ++i) c += (ids[i] == e) ? 1 : 0;
        cnt[e] = c;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int na = 0, off = 0;
        for (int e = 0; e < E; ++e) {
            if (cnt[e] > 0) {
                active[na] = e;
                offsets[na] = off;
                off += cnt[e];
                cnt[e] = na;
                ++na;
            } else {
                cnt[e] = -1;
            }
        }
        offsets[na] = off;
        *n_active = na;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        const int slot = cnt[e];
        if (slot < 0) continue;
        int w = offsets[slot];
        for (int tt = 0; tt < T; ++tt)
            for (int i = 0; i < K; ++i)
                if (ids[(size_t)tt * K + i] == e) {
                    tok[w] = tt;
                    tokw[w] = tw[(size_t)tt * K + i];
                    ++w;
                }
    }
}

// ------------------------------------------------------- fused MoE layer
// Expert set description shared by the two MoE kernels.
struct MoeExperts {
    const uint8_t* gq;  // gate qweight (E, inter, hidden/2)
    const uint16_t* gs_;
    const uint16_t* gz;
    const uint8_t* uq;  // up
    const uint16_t* us;
    const uint16_t* uz;
    const uint8_t* dq;  // down qweight (E, hidden, inter/2)
    const uint16_t* ds;
    const uint16_t* dz;
    int inter;
};

struct MoeArgs {
    const float* x;  // (T, hidden) fp32
    int T, hidden, gs;
    MoeExperts routed, shared;
    int has_shared;
    int E;
    const int* n_active;  // device count of active slots (or null: host_active)
    int host_active;
    const int* active;    // expert id per slot
    const float* rw;      // dense (T, E) weights (coef_mode 0)
    const float* coef;    // per-slot (S, T) weights (coef_mode 1)
    int coef_mode;
    const float* scoef;   // shared-expert per-token coefficient (T), or null (1.0)
    int max_active;       // slots reserved in inter_buf before the shared slot
    int inter_pad;
    uint16_t* inter_buf;  // fp16 (max_active + has_shared, T, inter_pad)
    float* y;             // (T, hidden) fp32
};

FL_DEV int moe_n_active(const MoeArgs& a) {
    return a.n_active ? __builtin_amdgcn_readfirstlane(*a.n_active) : a.host_active;
}

FL_DEV float moe_coef(const MoeArgs& a, int slot, int e, int t) {
    return a.coef_mode == 0 ? a.rw[(size_t)t * a.E + e] : a.coef[(size_t)slot * a.T + t];
}

// gate/up for one 16-row tile of one expert slot: h = silu(g) * u * coef,
// stored fp16 in inter_buf.  Workgroup = 8 waves splitting hidden blocks.
template <bool G128>
__global__ __launch_bounds__(512) void moe_gate_up_k(MoeArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int NB = 2;  // hidden blocks per wave and matrix (hidden <= 8 waves * 2 * 128)
    const int nwaves = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kq = lane >> 4;
    const int K = a.hidden;
    const int nfull = K >> 7;
    const int lda = K + 8;
    const int M = a.T;

    // which slot / tile
    const int tiles_r = a.routed.inter / 16;
    int slot, tile;
    const MoeExperts* ex;
    int e = 0;
    const int b = blockIdx.x;
    if (b < a.max_active * tiles_r) {
        slot = b / tiles_r;
        tile = b % tiles_r;
        if (slot >= moe_n_active(a)) return;
        e = a.active[slot];
        ex = &a.routed;
    } else {
        if (!a.has_shared) return;
        slot = a.max_active;
        tile = b - a.max_active * tiles_r;
        ex = &a.shared;
    }
    const int inter = ex->inter;
    const int G = K / a.gs;
    const size_t wbase = (size_t)e * inter * (K / 2);
    const size_t sbase = (size_t)e * inter * G;

    f16* As = reinterpret_cast<f16*>(smem);
    float* red = reinterpret_cast<float*>(smem + (((size_t)M * lda * 2 + 15) & ~(size_t)15));
    // stage x as fp16
    {
        const int k8 = K >> 3;
        const int nchunks = M * k8;
        for (int c = threadIdx.x; c < nchunks; c += blockDim.x) {
            const int m = c / k8, c8 = c - m * k8;
            const float* src = a.x + (size_t)m * K + c8 * 8;
            const f32x4 lo = *reinterpret_cast<const f32x4*>(src);
            const f32x4 hi = *reinterpret_cast<const f32x4*>(src + 4);
            f16x8 v;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                v[q] = (f16)lo[q];
                v[4 + q] = (f16)hi[q];
            }
            *reinterpret_cast<f16x8*>(As + (size_t)m * lda + c8 * 8) = v;
        }
    }

    const int row = tile * 16 + col;
    const int nb = wave < nfull ? (nfull - wave + nwaves - 1) / nwaves : 0;
    u32x4 wg[NB], wu[NB];
    uint16_t sg[NB], zg[NB], su[NB], zu[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        int kb = wave + (i < nb ? i : (nb > 0 ? nb - 1 : 0)) * nwaves;
        kb = kb < nfull ? kb : nfull - 1;
        const size_t off = wbase + (size_t)row * (K / 2) + kb * 64 + 16 * kq;
        wg[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ex->gq + off));
        wu[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ex->uq + off));
        const size_t so = sbase + (size_t)row * G + (kb * 128 + 32 * kq) / a.gs;
        sg[i] = ex->gs_[so];
        zg[i] = ex->gz[so];
        su[i] = ex->us[so];
        zu[i] = ex->uz[so];
    }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();

    const f16* arow = As + (size_t)(col < M ? col : M - 1) * lda + 32 * kq;
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const bool live = i < nb;
        int kb = wave + (live ? i : (nb > 0 ? nb - 1 : 0)) * nwaves;
        kb = kb < nfull ? kb : nfull - 1;
        u32x4 av[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) av[j] = *reinterpret_cast<const u32x4*>(arow + kb * 128 + 8 * j);
        rm_block_mma<G128>(acc[0], av, wg[i], sg[i], zg[i], live ? 1.0f : 0.0f);
        rm_block_mma<G128>(acc[1], av, wu[i], su[i], zu[i], live ? 1.0f : 0.0f);
        __builtin_amdgcn_sched_barrier(0);
    }

    reduce_and_store<2>(red, acc, M, wave, nwaves, lane, [&](int m, int t, int c, float v) {
        // t == 0: gate, t == 1: up; combine through LDS slot of the gate value
        if (t == 0) red[nwaves * 512 + m * 16 + c] = v;
        else red[nwaves * 512 + 256 + m * 16 + c] = v;
    });
    __syncthreads();
    for (int idx = threadIdx.x; idx < M * 16; idx += blockDim.x) {
        const int m = idx >> 4, c = idx & 15;
        const float g = red[nwaves * 512 + idx];
        const float u = red[nwaves * 512 + 256 + idx];
        float cf;
        if (slot < a.max_active)
            cf = moe_coef(a, slot, e, m);
        else
            cf = a.scoef ? a.scoef[m] : 1.0f;
        const float h = (g / (1.0f + expf(-g))) * u * cf;
        a.inter_buf[((size_t)slot * a.T + m) * a.inter_pad + tile * 16 + c] = bitcast<uint16_t>((f16)h);
    }
}

// down projection of every active slot (and the shared expert) for one
// 16-row output tile, summed in the MFMA accumulator in a fixed order:
// y[t, o] = sum_slots sum_i inter_buf[slot, t, i] * dequant(Wd)[o, i].
template <bool G128>
__global__ __launch_bounds__(1024) void moe_down_k(MoeArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int CH = 4;  // items issued together per wave
    const int nwaves = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kq = lane >> 4;
    const int M = a.T;
    const int o = blockIdx.x * 16 + col;  // output row of this lane's B column
    const int na = moe_n_active(a);
    const int nkb_r = a.routed.inter >> 7;
    const int nkb_s = a.has_shared ? (a.shared.inter >> 7) : 0;
    const int items = na * nkb_r + nkb_s;
    const int mrow = col < M ? col : M - 1;
    float* red = reinterpret_cast<float*>(smem);

    f32x4 acc[1] = {f32x4{0.f, 0.f, 0.f, 0.f}};
    const int my = wave < items ? (items - wave + nwaves - 1) / nwaves : 0;
    for (int base = 0; base < my; base += CH) {
        u32x4 av[CH][4];
        u32x4 wv[CH];
        uint16_t sv[CH], zv[CH];
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            int it = base + i;
            it = it < my ? it : my - 1;
            const int item = wave + it * nwaves;
            int slot, kb;
            const MoeExperts* ex;
            int e = 0;
            if (item < na * nkb_r) {
                slot = item / nkb_r;
                kb = item - slot * nkb_r;
                e = a.active[slot];
                ex = &a.routed;
            } else {
                slot = a.max_active;
                kb = item - na * nkb_r;
                ex = &a.shared;
            }
            const int inter = ex->inter;
            const uint16_t* ar = a.inter_buf + ((size_t)slot * a.T + mrow) * a.inter_pad + kb * 128 + 32 * kq;
#pragma unroll
            for (int j = 0; j < 4; ++j) av[i][j] = *reinterpret_cast<const u32x4*>(ar + 8 * j);
            const int G = inter / a.gs;
            const size_t woff = (size_t)e * a.hidden * (inter / 2) + (size_t)o * (inter / 2) + kb * 64 + 16 * kq;
            wv[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ex->dq + woff));
            const size_t so = (size_t)e * a.hidden * G + (size_t)o * G + (kb * 128 + 32 * kq) / a.gs;
            sv[i] = ex->ds[so];
            zv[i] = ex->dz[so];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const float live = (base + i < my) ? 1.0f : 0.0f;
            rm_block_mma<G128>(acc[0], av[i], wv[i], sv[i], zv[i], live);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    reduce_and_store<1>(red, acc, M, wave, nwaves, lane, [&](int m, int, int c, float v) {
        a.y[(size_t)m * a.hidden + blockIdx.x * 16 + c] = v;
    });
}

int finish(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fprintf(stderr, "%s launch error: %s\n", what, hipGetErrorString(e));
        return 2;
    }
    return 0;
}

template <int NB, bool G128, bool XF32, bool YF32>
void launch_rm(const void* X, const uint8_t* W, const uint16_t* S, const uint16_t* Z, void* Y,
               int M, int N, int K, int gs, int waves, hipStream_t st) {
    const size_t lds = (((size_t)M * (K + 8) * 2 + 15) & ~(size_t)15) + (size_t)waves * 1024;
    hipLaunchKernelGGL((rm_gemv_nb<NB, G128, XF32, YF32>), dim3((N + 15) / 16), dim3(64 * waves),
                       lds, st, X, W, S, Z, Y, M, N, K, gs);
}

template <bool G128, bool XF32, bool YF32>
void rm_dispatch(int nb, const void* X, const uint8_t* W, const uint16_t* S, const uint16_t* Z,
                 void* Y, int M, int N, int K, int gs, int waves, hipStream_t st) {
    switch (nb) {
        case 1: launch_rm<1, G128, XF32, YF32>(X, W, S, Z, Y, M, N, K, gs, waves, st); break;
        case 2: launch_rm<2, G128, XF32, YF32>(X, W, S, Z, Y, M, N, K, gs, waves, st); break;
        case 3: launch_rm<3, G128, XF32, YF32>(X, W, S, Z, Y, M, N, K, gs, waves, st); break;
        case 4: launch_rm<4, G128, XF32, YF32>(X, W, S, Z, Y, M, N, K, gs, waves, st); break;
        case 5: launch_rm<5, G128, XF32, YF32>(X, W, S, Z, Y, M, N, K, gs, waves, st); break;
        case 6: launch_rm<6, G128, XF32, YF32>(X, W, S, Z, Y, M, N, K, gs, waves, st); break;
        default: launch_rm<8, G128, XF32, YF32>(X, W, S, Z, Y, M, N, K, gs, waves, st); break;
    }
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
    const int nfull = in_f / 128;
    int waves = 16;
    while (waves > 1 && nfull < waves) waves /= 2;
    while ((nfull + waves - 1) / waves > 8 && waves < 16) waves *= 2;
    if ((nfull + waves - 1) / waves > 8) return 1;  // in_f > 16384
    const int need = (nfull + waves - 1) / waves;
    const int nb = need <= 6 ? need : 8;
    const bool g128 = group_size == 128;
    hipStream_t st = (hipStream_t)stream;
    const size_t xe = x_fp32 ? 4 : 2, ye = y_fp32 ? 4 : 2;
    int mcap = (int)((96 * 1024) / ((size_t)(in_f + 8) * 2));
    mcap = mcap > 16 ? 16 : (mcap < 1 ? 1 : mcap);
    for (int m0 = 0; m0 < M; m0 += mcap) {
        const int Mc = (M - m0) < mcap ? (M - m0) : mcap;
        const void* xm = static_cast<const char*>(x) + (size_t)m0 * in_f * xe;
        void* ym = static_cast<char*>(y) + (size_t)m0 * out_f * ye;
        const uint16_t* S = static_cast<const uint16_t*>(scales);
        const uint16_t* Z = static_cast<const uint16_t*>(zeros);
#define RM_CASE(G, XF, YF)                                                                       \
    if (g128 == G && (x_fp32 != 0) == XF && (y_fp32 != 0) == YF)                                 \
        rm_dispatch<G, XF, YF>(nb, xm, qweight, S, Z, ym, Mc, out_f, in_f, group_size, waves, st);
        RM_CASE(true, true, true)
        RM_CASE(true, true, false)
        RM_CASE(true, false, true)
        RM_CASE(true, false, false)
        RM_CASE(false, true, true)
        RM_CASE(false, true, false)
        RM_CASE(false, false, true)
        RM_CASE(false, false, false)
#undef RM_CASE
        const int rc = finish("fastllm_int4_rowmajor_gemv");
        if (rc) return rc;
    }
    return 0;
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
    if (!fl_current_device_supported()) return 2;
    RouteArgs a{logits, e_score_bias, shared_logit, T, E, top_k, scoring, norm, n_group,
                topk_group, routed_scaling, topk_ids, topk_w, rw, shared_coef,
                n_active, active, offsets, tok, tokw};
    hipStream_t st = (hipStream_t)stream;
    const int wpb = T < 16 ? T : 16;
    const int grid = (T + 15) / 16;
    hipLaunchKernelGGL(route_k, dim3(grid), dim3(64 * wpb), 0, st, a);
    int rc = finish("fastllm_route_topk");
    if (rc) return rc;
    if (grid > 1 && n_active) {
        hipLaunchKernelGGL(route_lists_k, dim3(1), dim3(1024), 0, st, topk_ids, topk_w, T, top_k,
                           E, n_active, active, offsets, tok, tokw);
        rc = finish("fastllm_route_topk");
    }
    return rc;
}

// Fused selective INT4 MoE FFN for up to 16 tokens (see MoeArgs).
int fastllm_moe_int4_fused(const float* x, int T, int hidden, int group_size, int E,
                           int inter, const uint8_t* gq, const void* gsc, const void* gz,
                           const uint8_t* uq, const void* usc, const void* uz,
                           const uint8_t* dq, const void* dsc, const void* dz,
                           int shared_inter, const uint8_t* sgq, const void* sgs, const void* sgz,
                           const uint8_t* suq, const void* sus, const void* suz,
                           const uint8_t* sdq, const void* sds, const void* sdz,
                           const float* shared_coef, const int* n_active, int host_active,
                           const int* active, int max_active, const float* rw,
                           const float* slot_coef, void* inter_buf, int inter_pad, float* y,
                           void* stream) {
    if (!x || T <= 0 || T > 16 || hidden <= 0 || hidden % 128 || hidden > 2048) return 1;
    if (E <= 0 || inter <= 0 || inter % 128 || !gq || !uq || !dq || !active || !inter_buf || !y)
        return 1;
    if (group_size != 32 && group_size != 64 && group_size != 128) return 1;
    if (max_active < 0 || (!rw && !slot_coef)) return 1;
    const bool has_shared = shared_inter > 0;
    if (has_shared && (shared_inter % 128 || !sgq || !suq || !sdq)) return 1;
    const int need_pad = inter > shared_inter ? inter : shared_inter;
    if (inter_pad < need_pad) return 1;
    if (!fl_aligned(x, 16) || !fl_aligned(inter_buf, 16)) return 1;
    if (!fl_current_device_supported()) return 2;
    MoeArgs a;
    a.x = x;
    a.T = T;
    a.hidden = hidden;
    a.gs = group_size;
    a.routed = MoeExperts{gq, (const uint16_t*)gsc, (const uint16_t*)gz, uq, (const uint16_t*)usc,
                          (const uint16_t*)uz, dq, (const uint16_t*)dsc, (const uint16_t*)dz, inter};
    a.shared = MoeExperts{sgq, (const uint16_t*)sgs, (const uint16_t*)sgz, suq, (const uint16_t*)sus,
                          (const uint16_t*)suz, sdq, (const uint16_t*)sds, (const uint16_t*)sdz,
                          has_shared ? shared_inter : 0};
    a.has_shared = has_shared ? 1 : 0;
    a.E = E;
    a.n_active = n_active;
    a.host_active = host_active;
    a.active = active;
    a.rw = rw;
    a.coef = slot_coef;
    a.coef_mode = rw ? 0 : 1;
    a.scoef = shared_coef;
    a.max_active = max_active;
    a.inter_pad = inter_pad;
    a.inter_buf = (uint16_t*)inter_buf;
    a.y = y;
    hipStream_t st = (hipStream_t)stream;
    const bool g128 = group_size == 128;
    // gate/up: one workgroup per (slot, 16-row tile)
    const int tiles = max_active * (inter / 16) + (has_shared ? shared_inter / 16 : 0);
    const int waves_gu = 8;
    const size_t lds_gu = (((size_t)T * (hidden + 8) * 2 + 15) & ~(size_t)15) +
                          (size_t)waves_gu * 2 * 1024 + 2 * 1024;
    if (tiles > 0) {
        if (g128)
            hipLaunchKernelGGL(moe_gate_up_k<true>, dim3(tiles), dim3(64 * waves_gu), lds_gu, st, a);
        else
            hipLaunchKernelGGL(moe_gate_up_k<false>, dim3(tiles), dim3(64 * waves_gu), lds_gu, st, a);
        const int rc = finish("fastllm_moe_int4_fused(gate_up)");
        if (rc) return rc;
    }
    const int waves_d = 16;
    const size_t lds_d = (size_t)waves_d * 1024;
    if (g128)
        hipLaunchKernelGGL(moe_down_k<true>, dim3(hidden / 16), dim3(64 * waves_d), lds_d, st, a);
    else
        hipLaunchKernelGGL(moe_down_k<false>, dim3(hidden / 16), dim3(64 * waves_d), lds_d, st, a);
    return finish("fastllm_moe_int4_fused(down)");
}

}  // extern "C"
