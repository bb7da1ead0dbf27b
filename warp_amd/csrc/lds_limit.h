/*
 * lds_limit.h — the dynamic LDS limit of a kernel, raised once per device.
 *
 * hipFuncSetAttribute(hipFuncAttributeMaxDynamicSharedMemorySize) is made
 * on a kernel's first launch on each device (the device of the launch's
 * stream, or the current one for the null stream), to all the LDS a block
 * may have (160 KiB less the kernel's static LDS), so that later launches
 * of the same kernel with more dynamic LDS than the first are allowed too
 * (the limit does not change what a launch allocates); `done` holds one bit
 * per device ordinal and is updated atomically, so concurrent first
 * launches from several threads are safe (at worst the attribute is set
 * twice).
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
    hipFuncAttributes fa;
    int lim = bytes;
    if (hipFuncGetAttributes(&fa, fn) == hipSuccess && 163840 - (int)fa.sharedSizeBytes > lim)
        lim = 163840 - (int)fa.sharedSizeBytes;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lim);
    if (e != hipSuccess && lim != bytes) e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return -(int)e - 1000;
    done.fetch_or(bit, std::memory_order_acq_rel);
    return 0;
}

#endif
