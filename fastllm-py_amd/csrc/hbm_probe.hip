// HBM streaming-read probe: the floor a decode GEMV launch of a given byte
// count can reach on this device.
//
// A GEMV at M = 1 reads its packed weights once and does little else, so a
// kernel that only reads the same number of bytes, with the GEMVs' access
// shape (every wave load a contiguous 1 KB: 64 lanes x 16 B, non-temporal),
// bounds it from below: launch, wave dispatch, first-load latency, the
// stream itself and the drain at the end, with no compute, reduction or
// store.  Each workgroup of 4 waves reads one contiguous range of NL KB per
// wave (all loads issued before the first use) and folds the words into one
// value.  The read-only form stores it only when it equals a constant no
// input produces in practice, so the loads cannot be dropped and nothing is
// written; the storing form (STORE) has every wave write its value once
// its loads have landed, as a GEMV workgroup writes its outputs, so
// the difference between the two is the cost of a dependent store at the
// end of a launch.
#include "common.cuh"
#include "device.cuh"

namespace {

constexpr int kProbeThreads = 256;

// XOR of x over the wave: DPP exchanges within each 16-lane row (quad
// pairs, quads, half-rows), then the four row results read by lane.
FL_DEV uint32_t wave_xor(uint32_t x) {
    x ^= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false);   // quad_perm 1,0,3,2
    x ^= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false);   // quad_perm 2,3,0,1
    x ^= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x141, 0xF, 0xF, false);  // row_half_mirror
    x ^= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x140, 0xF, 0xF, false);  // row_mirror
    return (uint32_t)(__builtin_amdgcn_readlane((int)x, 0) ^ __builtin_amdgcn_readlane((int)x, 16) ^
                      __builtin_amdgcn_readlane((int)x, 32) ^ __builtin_amdgcn_readlane((int)x, 48));
}

template <int NL, bool STORE>
__global__ __launch_bounds__(kProbeThreads) void hbm_read_k(const u32x4* __restrict__ src, size_t n16,
                                                             uint32_t* __restrict__ sink) {
    const size_t base = (size_t)blockIdx.x * kProbeThreads * NL + threadIdx.x;
    u32x4 v[NL];
#pragma unroll
    for (int r = 0; r < NL; ++r) {
        size_t i = base + (size_t)r * kProbeThreads;
        i = i < n16 ? i : n16 - 1;
        v[r] = __builtin_nontemporal_load(src + i);
    }
    uint32_t x = 0;
#pragma unroll
    for (int r = 0; r < NL; ++r) x ^= v[r][0] ^ v[r][1] ^ v[r][2] ^ v[r][3];
    if (STORE) {
        // every lane's loads feed the stored value (folded over the wave
        // first: a value of lane 0 alone would let the compiler drop the
        // other lanes' loads), written by lane 0 once the loads have landed
        x = wave_xor(x);
        if ((threadIdx.x & 63) == 0) sink[(blockIdx.x * 4 + (threadIdx.x >> 6)) & 1023] = x;
    } else if (x == 0x9E3779B9u) {
        sink[blockIdx.x & 1023] = x;
    }
}

template <int NL>
void launch_probe(const void* src, size_t n16, uint32_t* sink, bool store, hipStream_t st) {
    const size_t per = (size_t)kProbeThreads * NL;
    const unsigned grid = (unsigned)((n16 + per - 1) / per);
    if (store)
        hipLaunchKernelGGL((hbm_read_k<NL, true>), dim3(grid), dim3(kProbeThreads), 0, st,
                           static_cast<const u32x4*>(src), n16, sink);
    else
        hipLaunchKernelGGL((hbm_read_k<NL, false>), dim3(grid), dim3(kProbeThreads), 0, st,
                           static_cast<const u32x4*>(src), n16, sink);
}

}  // namespace

extern "C" {

// Read `bytes` (a multiple of 16, > 0) from `src` (16-byte aligned) with
// `loads_per_lane` (4, 8 or 16) 16-byte loads per lane, plus 64 when every
// wave stores its folded value (into sink, wave index mod 1024) at the end;
// without it `sink` (1024 words) is written only in the practically
// impossible case noted above.  0 ok, 1 bad arguments, 2 device / launch
// error.
int fastllm_hbm_read_probe(const void* src, size_t bytes, uint32_t* sink, int loads_per_lane,
                           void* stream) {
    const bool store = loads_per_lane & 64;
    loads_per_lane &= ~64;
    if (!src || !sink || bytes == 0 || bytes % 16 || !fl_aligned(src, 16)) return 1;
    const size_t n16 = bytes / 16;
    if (n16 / ((size_t)kProbeThreads * 4) >= 0x7FFFFFFFu) return 1;
    if (!fl_current_device_supported()) return 2;
    hipStream_t st = (hipStream_t)stream;
    switch (loads_per_lane) {
        case 4: launch_probe<4>(src, n16, sink, store, st); break;
        case 8: launch_probe<8>(src, n16, sink, store, st); break;
        case 16: launch_probe<16>(src, n16, sink, store, st); break;
        default: return 1;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fprintf(stderr, "fastllm_hbm_read_probe launch error: %s\n", hipGetErrorString(e));
        return 2;
    }
    return 0;
}

}  // extern "C"
