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

/* Pairs of neighbouring floats (in value order, -inf .. +inf) on which
 * glibc's expf decreases: the certified router takes the score at the ends
 * of a logit interval as bounds of the score anywhere inside it. Ranks r in
 * [0, 2^32 - 2^24) walk the non-NaN patterns in value order. */
typedef struct {
    uint64_t lo, hi;
    uint64_t bad;
} mono_t;

static uint32_t pattern_of_rank(uint64_t r)
{
    /* ranks 0 .. 0x7f800000: -inf .. -0 (patterns 0xff800000 down to
     * 0x80000000); then +0 .. +inf (0 .. 0x7f800000) */
    const uint64_t nneg = 0x7f800001ull;
    return r < nneg ? (uint32_t)(0xff800000ull - r) : (uint32_t)(r - nneg);
}

static void *mono_scan(void *p)
{
    mono_t *j = (mono_t *)p;
    float prev;
    uint32_t u = pattern_of_rank(j->lo);
    memcpy(&prev, &u, 4);
    prev = expf(prev);
    for (uint64_t r = j->lo + 1; r < j->hi; r++) {
        float x;
        u = pattern_of_rank(r);
        memcpy(&x, &u, 4);
        const float v = expf(x);
        if (v < prev) j->bad++;
        prev = v;
    }
    return NULL;
}

uint64_t or_expf_decreases(int nthreads)
{
    const uint64_t nr = 2ull * 0x7f800001ull;             /* -inf .. -0, +0 .. +inf */
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 64) nthreads = 64;
    pthread_t th[64];
    mono_t jb[64];
    for (int k = 0; k < nthreads; k++) {
        const uint64_t a = nr * (uint64_t)k / (uint64_t)nthreads, b = nr * (uint64_t)(k + 1) / (uint64_t)nthreads;
        jb[k] = (mono_t){ a, k + 1 < nthreads ? b + 1 : b, 0 };   /* overlapping by one: every pair is seen */
        pthread_create(&th[k], NULL, mono_scan, &jb[k]);
    }
    uint64_t bad = 0;
    for (int k = 0; k < nthreads; k++) {
        pthread_join(th[k], NULL);
        bad += jb[k].bad;
    }
    return bad;
}
