/*
 * lds_limit.h — the dynamic LDS limit of a kernel, raised once per device.
 *
 * hipFuncSetAttribute(hipFuncAttributeMaxDynamicSharedMemorySize) is made
 * on a kernel's first launch on each device (the device of the launch's
 * stream, or the current one for the null stream); `done` holds one bit per
 * device ordinal and is updated atomically, so concurrent first launches
 * from several threads are safe (at worst the attribute is set twice).
 */
#ifndef WARP_LDS_LIMIT_H
#define WARP_LDS_LIMIT_H

#include <hip/hip_runtime.h>

#include <atomic>
#include <stdint.h>

static inline int lds_limit(const void *fn, int bytes, std::atomic<uint64_t> &done, void *stream) {
    int d = 0;
    const hipError_t g = stream ? hipStreamGetDevice((hipStream_t)stream, &d) : hipGetDevice(&d);
    if (g != hipSuccess) return -(int)g - 1000;
    const uint64_t bit = 1ull << (d & 63);
    if (done.load(std::memory_order_acquire) & bit) return 0;
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return -(int)e - 1000;
    done.fetch_or(bit, std::memory_order_acq_rel);
    return 0;
}

#endif
