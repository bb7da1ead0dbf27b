/*
 * expf_check.c -- test infrastructure: checks the device's expf restatement
 * (warp_amd/csrc/expf_glibc.h, compiled here as plain C) against the host's
 * glibc expf, the function the reference calls for its router scores and
 * SiLU (src/model.c:2724, src/model.c:501). Built into liboracle.so; nothing
 * in the product links it.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

#include "../warp_amd/csrc/expf_glibc.h"

typedef struct {
    uint64_t lo, n;
    int step, k;
    uint64_t bad;
    uint32_t first;
} job_t;

static void *scan(void *p)
{
    job_t *j = (job_t *)p;
    for (uint64_t i = (uint64_t)j->k; i < j->n; i += (uint64_t)j->step) {
        const uint32_t u = (uint32_t)(j->lo + i);
        float x, a, b;
        memcpy(&x, &u, 4);
        a = expf(x);
        b = warp_expf(x);
        uint32_t ua, ub;
        memcpy(&ua, &a, 4);
        memcpy(&ub, &b, 4);
        if (ua != ub && !(a != a && b != b)) {
            if (!j->bad) j->first = u;
            j->bad++;
        }
    }
    return NULL;
}

/* Inputs with bit patterns lo .. lo+n-1 (n <= 2^32) on which warp_expf and
 * glibc's expf differ (two NaNs count as equal); *first gets the lowest
 * such pattern each thread met first, or is left alone. */
uint64_t or_expf_mismatches(uint32_t lo, uint64_t n, int nthreads, uint32_t *first)
{
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 64) nthreads = 64;
    pthread_t th[64];
    job_t jb[64];
    for (int k = 0; k < nthreads; k++) {
        jb[k] = (job_t){ lo, n, nthreads, k, 0, 0 };
        pthread_create(&th[k], NULL, scan, &jb[k]);
    }
    uint64_t bad = 0;
    for (int k = 0; k < nthreads; k++) {
        pthread_join(th[k], NULL);
        if (jb[k].bad && first && (bad == 0 || jb[k].first < *first)) *first = jb[k].first;
        bad += jb[k].bad;
    }
    return bad;
}

/* glibc's expf and the reference's sigmoid score 1/(1+expf(-x)) over arrays */
void or_expf_array(const float *x, float *y, long n)
{
    for (long i = 0; i < n; i++) y[i] = expf(x[i]);
}

void or_sigmoid_array(const float *x, float *y, long n)
{
    for (long i = 0; i < n; i++) y[i] = 1.0f / (1.0f + expf(-x[i]));
}
