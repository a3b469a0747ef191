// Per-device capability checks shared by every entry point.
#pragma once

#include "common.cuh"
#include <string.h>

// Returns true when the calling thread's current HIP device is a gfx950 part.
// The answer is cached per device ordinal (the check reads device properties,
// which is too slow for a per-call path).
static inline bool fl_current_device_supported() {
    static int cached[64];  // 0 = unknown, 1 = yes, -1 = no
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        (void)hipGetLastError();
        return false;
    }
    if (cached[dev] == 0) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
            (void)hipGetLastError();
            return false;
        }
        cached[dev] = (strncmp(prop.gcnArchName, "gfx950", 6) == 0) ? 1 : -1;
    }
    return cached[dev] == 1;
}

static inline int fl_current_device_cu_count() {
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        (void)hipGetLastError();
        return 256;
    }
    if (cached[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0) {
            (void)hipGetLastError();
            cus = 256;
        }
        cached[dev] = cus;
    }
    return cached[dev];
}

static inline bool fl_aligned(const void* p, size_t a) {
    return ((uintptr_t)p % a) == 0;
}

// True when the byte ranges [a, a + na) and [b, b + nb) intersect.
static inline bool fl_overlap(const void* a, size_t na, const void* b, size_t nb) {
    const uintptr_t pa = (uintptr_t)a, pb = (uintptr_t)b;
    return pa < pb + nb && pb < pa + na;
}

// LDS per workgroup on gfx950 (160 KB).
constexpr size_t kMaxLds = 160 * 1024;
