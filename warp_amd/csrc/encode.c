/* The encoder on the device: drop-ins for waste_vq_encode and
 * waste_vq_lloyd (src/vq.c:96-136), the conversion-time half of the VQ
 * format. Host buffers in and out, one call per matrix; the device
 * buffers are allocated per call. The kernels are in kernels.hip. */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "warp_hip.h"
#include "warp_internal.h"

#define HIPOK(x) ((x) == hipSuccess)

typedef struct {
    float *X, *cur, *books;
    uint16_t *codes;
} enc_bufs;

static void enc_free(enc_bufs *b)
{
    if (b->X) (void)hipFree(b->X);
    if (b->cur) (void)hipFree(b->cur);
    if (b->books) (void)hipFree(b->books);
    if (b->codes) (void)hipFree(b->codes);
    memset(b, 0, sizeof *b);
}

/* codes [n][stages] on the host, 16-bit */
static int encode16(const float *X, long n, const float *books, int stages, int entries, uint16_t *out)
{
    enc_bufs b;
    memset(&b, 0, sizeof b);
    const size_t xb = (size_t)n * 8 * sizeof(float), bb = (size_t)stages * entries * 8 * sizeof(float);
    const size_t cb = (size_t)n * stages * sizeof(uint16_t);
    int rc = WARP_HIP_E_NOMEM;
    if (!HIPOK(hipMalloc((void **)&b.X, xb)) || !HIPOK(hipMalloc((void **)&b.books, bb)) ||
        !HIPOK(hipMalloc((void **)&b.codes, cb)) || (stages > 1 && !HIPOK(hipMalloc((void **)&b.cur, xb))))
        goto out;
    rc = WARP_HIP_E_DEVICE;
    if (!HIPOK(hipMemcpy(b.X, X, xb, hipMemcpyHostToDevice)) ||
        !HIPOK(hipMemcpy(b.books, books, bb, hipMemcpyHostToDevice)))
        goto out;
    if (wk_vq_encode(b.X, n, b.books, stages, entries, b.cur, b.codes, NULL)) goto out;
    if (!HIPOK(hipMemcpy(out, b.codes, cb, hipMemcpyDeviceToHost))) goto out;
    rc = 0;
out:
    enc_free(&b);
    return rc;
}

int warp_hip_vq_encode(const float *X, int n, const float *books, int stages, int entries, int dim, uint8_t *out,
                       int nthreads)
{
    (void)nthreads;
    if (!X || !books || !out || n < 0 || stages < 1 || entries < 1 || entries > 256 || dim != 8)
        return WARP_HIP_E_ARG;
    if (n == 0) return 0;
    uint16_t *c16 = (uint16_t *)malloc((size_t)n * stages * sizeof(uint16_t));
    if (!c16) return WARP_HIP_E_NOMEM;
    int rc = encode16(X, n, books, stages, entries, c16);
    if (!rc)
        for (size_t i = 0; i < (size_t)n * stages; i++) out[i] = (uint8_t)c16[i];
    free(c16);
    return rc;
}

int warp_hip_vq_encode16(const float *X, long n, const float *books, int stages, int entries, int dim, uint16_t *out)
{
    if (!X || !books || !out || n < 0 || stages < 1 || entries < 1 || entries > 4096 || dim != 8)
        return WARP_HIP_E_ARG;
    if (n == 0) return 0;
    return encode16(X, n, books, stages, entries, out);
}

int warp_hip_vq_encode_dev(const float *X_dev, long n, const float *books_dev, int stages, int entries,
                           float *resid_dev, uint16_t *codes_dev, void *stream)
{
    if (!X_dev || !books_dev || !codes_dev || n <= 0 || stages < 1 || entries < 1 || entries > 4096 ||
        (stages > 1 && !resid_dev))
        return WARP_HIP_E_ARG;
    return wk_vq_encode(X_dev, n, books_dev, stages, entries, resid_dev, codes_dev, stream) ? WARP_HIP_E_DEVICE : 0;
}

int warp_hip_vq_lloyd(const float *X, int n, float *C, int entries, int dim, int nthreads)
{
    (void)nthreads;
    if (!X || !C || n <= 0 || entries < 1 || entries > 4096 || dim != 8) return WARP_HIP_E_ARG;
    const int nchunk = (n + 4095) / 4096;
    const size_t xb = (size_t)n * 8 * sizeof(float), cb = (size_t)entries * 8 * sizeof(float);
    float *dX = NULL, *dC = NULL;
    uint16_t *asg = NULL;
    int *counts = NULL, *total = NULL, *base = NULL, *sorted = NULL, *live = NULL;
    int rc = WARP_HIP_E_NOMEM, h_live = 0;
    if (!HIPOK(hipMalloc((void **)&dX, xb)) || !HIPOK(hipMalloc((void **)&dC, cb)) ||
        !HIPOK(hipMalloc((void **)&asg, (size_t)n * sizeof(uint16_t))) ||
        !HIPOK(hipMalloc((void **)&counts, (size_t)nchunk * entries * sizeof(int))) ||
        !HIPOK(hipMalloc((void **)&total, (size_t)entries * sizeof(int))) ||
        !HIPOK(hipMalloc((void **)&base, (size_t)entries * sizeof(int))) ||
        !HIPOK(hipMalloc((void **)&sorted, (size_t)n * sizeof(int))) || !HIPOK(hipMalloc((void **)&live, sizeof(int))))
        goto out;
    rc = WARP_HIP_E_DEVICE;
    if (!HIPOK(hipMemcpy(dX, X, xb, hipMemcpyHostToDevice)) || !HIPOK(hipMemcpy(dC, C, cb, hipMemcpyHostToDevice)))
        goto out;
    if (wk_vq_lloyd(dX, n, dC, entries, dim, asg, counts, total, base, sorted, live, NULL)) goto out;
    if (!HIPOK(hipMemcpy(C, dC, cb, hipMemcpyDeviceToHost)) ||
        !HIPOK(hipMemcpy(&h_live, live, sizeof(int), hipMemcpyDeviceToHost)))
        goto out;
    rc = h_live;
out:
    if (dX) (void)hipFree(dX);
    if (dC) (void)hipFree(dC);
    if (asg) (void)hipFree(asg);
    if (counts) (void)hipFree(counts);
    if (total) (void)hipFree(total);
    if (base) (void)hipFree(base);
    if (sorted) (void)hipFree(sorted);
    if (live) (void)hipFree(live);
    return rc;
}
