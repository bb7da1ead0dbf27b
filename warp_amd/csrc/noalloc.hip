// noalloc.hip — the allocation-free variant of the device encoder
// (warp_hip_vq_encode_dev_noalloc, include/warp_hip.h), for callers that
// cannot allocate device memory: code under HIP graph capture, serving loops,
// harnesses that forbid hipMalloc.
//
// The residuals that the multi-stage encoder carries from one stage to the
// next live in `scratch`, a file-scope device array of a fixed size, instead
// of a workspace the caller brings. Each device holds its own copy of the
// array for the life of the process. Its address on a device comes from
// hipGetSymbolAddress, asked once per device with that device current and
// kept in scratch_dev[]; host code uses only that address (the array's name
// is a host-side stand-in, not a device address). Calls on one device share
// the array, so calls that overlap on one device (two streams at once) race;
// nothing in it needs clearing (every stage writes the rows it reads next).

#include <hip/hip_runtime.h>
#include <pthread.h>
#include <stdint.h>

#include "warp_hip.h"
#include "warp_internal.h"

static __device__ __align__(256) float scratch[(size_t)WARP_HIP_NOALLOC_MAX_VECTORS * 8];

#define MAX_DEVICES 64
static float *scratch_dev[MAX_DEVICES];
static pthread_mutex_t scratch_mu = PTHREAD_MUTEX_INITIALIZER;

// The device address of this device's `scratch`, looked up on the first call
// on the device (the current one); NULL when the lookup fails.
static float *scratch_of_current(void) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return nullptr;
    pthread_mutex_lock(&scratch_mu);
    float *p = scratch_dev[dev];
    if (!p) {
        void *q = nullptr;
        if (hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)) == hipSuccess) p = scratch_dev[dev] = (float *)q;
    }
    pthread_mutex_unlock(&scratch_mu);
    return p;
}

extern "C" int warp_hip_vq_encode_dev_noalloc(const float *X_dev, long n, const float *books_dev, int stages,
                                              int entries, uint16_t *codes_dev, void *stream) {
    if (!X_dev || !books_dev || !codes_dev || n <= 0 || stages < 1 || entries < 1 || entries > 4096)
        return WARP_HIP_E_ARG;
    // one stage carries no residual; more need n rows of scratch
    if (stages > 1 && n > WARP_HIP_NOALLOC_MAX_VECTORS) return WARP_HIP_E_ARG;
    float *cur = nullptr;
    if (stages > 1 && !(cur = scratch_of_current())) return WARP_HIP_E_DEVICE;
    return wk_vq_encode(X_dev, n, books_dev, stages, entries, cur, codes_dev, stream) ? WARP_HIP_E_DEVICE : 0;
}
