/*
 * moe_table.c — the MoE slots of waste_moe_kernels (include/warp_hip.h,
 * section 1b): moe_layer and moe_chunk (src/model.c:2713-2940,
 * 3512-3693) behind a table the engine calls, with the engine's CPU path as
 * the default and the fallback.
 *
 * Each slot call carries the layer's host tensors (warp_moe_args). Device
 * state is kept per engine model: one context (warp_hip_open) per
 * `model` pointer, opened on its first call with the model's shapes, and
 * per layer the device copies of its codebooks, router, bias, shared
 * expert and latent projections, made on the layer's first call and made
 * again when a host pointer changes (the way src/metal.m:98-150 keys its
 * buffers by host pointer). Expert records enter the context's HBM cache
 * through the engine's own fetch function on a miss. Everything is dropped
 * by waste_hip_release_host_buffers(). One mutex serialises the slots, as
 * the Metal backend serialises its table (src/metal.m:173).
 *
 * A call this backend cannot take (a format or tensor type it does not
 * run, codebooks it cannot hold, a device error, a selection whose records
 * name codebooks other than their layer's) goes to the slot's previous
 * value with the same arguments; with none, the slot returns the negative
 * code and the engine runs its own CPU code.
 */
#include <hip/hip_runtime_api.h>

#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "warp_hip.h"
#include "warp_internal.h"

#define HIPOK(x) ((x) == hipSuccess)
#define MOE_MAX_MODELS 8
#define MOE_MIN_TOKENS 64       /* a chunk of the reference's prefill (src/model.h:285) */

typedef struct {
    const float *books;         /* host pointers the device copies were made from */
    int cb_base;
    const void *router, *bias, *shared[3], *latent[2], *norm;
    int set;
} layer_key;

typedef struct {
    const void *model;
    warp_hip_ctx *c;
    warp_hip_cfg cfg;           /* the configuration it was opened with */
    layer_key *lk;
    float *x_dev, *out_dev;     /* one token's input and output */
} moe_dev;

static pthread_mutex_t g_moe_mu = PTHREAD_MUTEX_INITIALIZER;
static moe_dev g_moe[MOE_MAX_MODELS];
static int (*g_prev_decode)(const warp_moe_args *);
static int (*g_prev_batch)(const warp_moe_args *);
static uint64_t g_moe_calls, g_moe_fallbacks;

static void moe_drop(moe_dev *d)
{
    if (d->c) warp_hip_close(d->c);
    if (d->x_dev) (void)hipFree(d->x_dev);
    if (d->out_dev) (void)hipFree(d->out_dev);
    free(d->lk);
    memset(d, 0, sizeof *d);
}

/* The container format of waste_model's index width, stages and entries. */
static int moe_fmt(const warp_moe_args *a)
{
    if (a->vec_dim != 8) return 0;
    if (a->index_bits == 8 && a->cb_entries == 256) return a->stages == 3 ? WARP_HIP_VQ3R : a->stages == 2 ? WARP_HIP_VQ2R : 0;
    if (a->index_bits == 6 && a->stages == 4 && a->cb_entries == 64) return WARP_HIP_VQ4P;
    if (a->index_bits == 12 && a->stages == 2 && a->cb_entries == 4096) return WARP_HIP_VQ12;
    return 0;
}

static int quantised(const warp_trunk_tensor *t)
{
    return t->q && t->qs && (t->bits == 8 || t->bits == 4 || t->bits == 3) && t->group > 0;
}

/* The configuration a model's context is opened with. */
static int moe_cfg(const warp_moe_args *a, int tokens, warp_hip_cfg *g)
{
    memset(g, 0, sizeof *g);
    g->fmt = moe_fmt(a);
    if (!g->fmt || a->layer < 0 || a->layer >= a->n_layers || !a->codebooks || !a->fetch || a->rec_bytes == 0)
        return WARP_HIP_E_ARG;
    g->hidden = a->hidden;
    g->inter = a->moe_inter;
    g->n_experts = a->n_experts;
    g->top_k = a->top_k;
    g->n_layers = a->n_layers;
    g->renorm = a->renorm;
    g->routed_scale = a->routed_scale;
    g->router_act = WARP_HIP_ROUTE_SIGMOID;
    /* the selection is the reference's on every input: chunks sum the F32
     * router's logits in the reference's sequential order, decode certifies
     * its picks against that order (recomputing rows only where needed) */
    g->router_strict = 2;
    g->act_situ = a->act_situ;
    g->situ_beta = a->situ_beta;
    g->situ_linear_beta = a->situ_linear_beta;
    g->max_tokens = tokens;
    g->rec_bytes = a->rec_bytes;
    g->verify = a->verify;
    g->lookahead = a->lookahead;
    g->device = 0;
    g->latent = a->latent_dim;
    g->latent_norm = a->latent_norm;
    g->norm_eps = a->norm_eps;
    g->n_books = a->n_books;
    g->cache_bytes = a->cache_bytes;
    if (!g->cache_bytes) {
        /* every record of the model, or 80% of the free HBM */
        size_t fr = 0, tot = 0;
        if (!HIPOK(hipMemGetInfo(&fr, &tot))) return WARP_HIP_E_DEVICE;
        const size_t all = (size_t)a->n_layers * a->n_experts * a->rec_bytes;
        g->cache_bytes = all < fr / 10 * 8 ? all : fr / 10 * 8;
    }
    return 0;
}

static int same_cfg(const warp_hip_cfg *x, const warp_hip_cfg *y)
{
    warp_hip_cfg a = *x, b = *y;
    a.max_tokens = b.max_tokens = 0;
    a.cache_bytes = b.cache_bytes = 0;
    return memcmp(&a, &b, sizeof a) == 0;
}

/* The model's context, opened (or opened again, larger or reshaped) as the
 * call needs. */
static int moe_dev_of(const warp_moe_args *a, moe_dev **out)
{
    const int tokens = a->n_tokens > MOE_MIN_TOKENS ? a->n_tokens : MOE_MIN_TOKENS;
    warp_hip_cfg g;
    int rc = moe_cfg(a, tokens, &g);
    if (rc) return rc;
    moe_dev *d = NULL, *free_slot = NULL;
    for (int i = 0; i < MOE_MAX_MODELS; i++) {
        if (g_moe[i].model == a->model && g_moe[i].c) d = &g_moe[i];
        else if (!g_moe[i].c && !free_slot) free_slot = &g_moe[i];
    }
    if (d && (!same_cfg(&d->cfg, &g) || d->cfg.max_tokens < a->n_tokens)) {
        if (d->cfg.max_tokens > g.max_tokens) g.max_tokens = d->cfg.max_tokens;
        moe_drop(d);
        free_slot = d;
        d = NULL;
    }
    if (!d) {
        if (!free_slot) return WARP_HIP_E_NOMEM;
        d = free_slot;
        if ((rc = warp_hip_open(&g, &d->c)) != 0) {
            d->c = NULL;
            return rc;
        }
        d->model = a->model;
        d->cfg = g;
        d->lk = (layer_key *)calloc((size_t)a->n_layers, sizeof(layer_key));
        if (!d->lk || !HIPOK(hipMalloc((void **)&d->x_dev, (size_t)a->hidden * sizeof(float))) ||
            !HIPOK(hipMalloc((void **)&d->out_dev, (size_t)a->hidden * sizeof(float)))) {
            moe_drop(d);
            return WARP_HIP_E_NOMEM;
        }
    }
    *out = d;
    return 0;
}

/* f32 codebook values back to the fp16 bits they were loaded from: the
 * inverse of the loader's conversion (exponent + 112, mantissa << 13, zero
 * for a zero exponent, src/model.c:1281-1285), exact for every value it
 * makes; anything else (not from fp16) is refused. */
static int books_to_f16(const float *f, size_t n, uint16_t *h)
{
    for (size_t i = 0; i < n; i++) {
        uint32_t u;
        memcpy(&u, &f[i], 4);
        const uint32_t s = u >> 31, e = (u >> 23) & 0xffu, m = u & 0x7fffffu;
        if (e == 0 && m == 0) { h[i] = (uint16_t)(s << 15); continue; }
        if (e < 113 || e > 143 || (m & 0x1fffu)) return WARP_HIP_E_ARG;
        h[i] = (uint16_t)((s << 15) | ((e - 112) << 10) | (m >> 13));
    }
    return 0;
}

/* The layer's weights on the device, copied again if a host pointer moved. */
static int moe_layer_weights(moe_dev *d, const warp_moe_args *a)
{
    warp_hip_ctx *c = d->c;
    const int L = a->layer;
    layer_key k;
    memset(&k, 0, sizeof k);
    k.books = a->codebooks;
    k.cb_base = a->cb_base;
    k.router = a->router.data ? (const void *)a->router.data : (const void *)a->router.q;
    k.bias = a->bias;
    for (int i = 0; i < 3; i++) k.shared[i] = a->shared[i].q;
    for (int i = 0; i < 2; i++) k.latent[i] = a->latent[i].q;
    k.norm = a->latent_norm_w;
    k.set = 1;
    if (memcmp(&k, &d->lk[L], sizeof k) == 0) return 0;
    d->lk[L].set = 0;
    int rc;
    /* codebooks: the bank's 3 x stages books */
    if (a->cb_base < 0 || a->cb_base + 3 * a->stages > a->n_books) return WARP_HIP_E_ARG;
    const size_t nb = (size_t)3 * a->stages * a->cb_entries * 8;
    uint16_t *h = (uint16_t *)malloc(nb * sizeof(uint16_t));
    if (!h) return WARP_HIP_E_NOMEM;
    rc = books_to_f16(a->codebooks + (size_t)a->cb_base * a->cb_entries * 8, nb, h);
    if (!rc) rc = warp_hip_set_codebooks(c, L, a->cb_base, h);
    free(h);
    if (rc) return rc;
    /* router */
    if (a->router.data) rc = warp_hip_set_router(c, L, a->router.data, a->bias);
    else if (quantised(&a->router))
        rc = warp_hip_set_router_q(c, L, a->router.bits, a->router.group, a->router.q, a->router.qs,
                                   a->router.rowbytes, a->bias);
    else rc = WARP_HIP_E_ARG;
    if (rc) return rc;
    /* shared expert: quantised rows, all three of one type, or none */
    const int nsh = (a->shared[0].q != NULL) + (a->shared[1].q != NULL) + (a->shared[2].q != NULL);
    if (a->shared[0].data || a->shared[1].data || a->shared[2].data) return WARP_HIP_E_ARG;
    if (nsh == 3) {
        for (int i = 0; i < 3; i++)
            if (!quantised(&a->shared[i]) || a->shared[i].bits != a->shared[0].bits ||
                a->shared[i].group != a->shared[0].group)
                return WARP_HIP_E_ARG;
        const int8_t *q[3] = { a->shared[0].q, a->shared[1].q, a->shared[2].q };
        const uint16_t *s[3] = { a->shared[0].qs, a->shared[1].qs, a->shared[2].qs };
        const size_t rb[3] = { a->shared[0].rowbytes, a->shared[1].rowbytes, a->shared[2].rowbytes };
        if ((rc = warp_hip_set_shared(c, L, a->shared[0].bits, a->shared[0].group, a->inter_shared, q, s, rb)))
            return rc;
    } else if (nsh != 0) {
        return WARP_HIP_E_ARG;
    }
    if (a->latent_dim) {
        const warp_trunk_tensor *dn = &a->latent[0], *up = &a->latent[1];
        if (!quantised(dn) || !quantised(up) || dn->bits != up->bits || dn->group != up->group) return WARP_HIP_E_ARG;
        if ((rc = warp_hip_set_latent(c, L, dn->bits, dn->group, dn->q, dn->qs, dn->rowbytes, up->q, up->qs,
                                      up->rowbytes, a->latent_norm_w)))
            return rc;
    }
    d->lk[L] = k;
    return 0;
}

static int moe_run(const warp_moe_args *a, int batch)
{
    if (!a || !a->x || !a->out || a->n_tokens < 1 || (!batch && a->n_tokens != 1)) return WARP_HIP_E_ARG;
    moe_dev *d;
    int rc = moe_dev_of(a, &d);
    if (rc) return rc;
    warp_hip_ctx *c = d->c;
    if ((rc = moe_layer_weights(d, a))) return rc;
    if ((rc = warp_hip_set_fetch(c, (warp_hip_fetch_fn)a->fetch, a->fetch_user))) return rc;
    const int K = a->top_k;
    if (batch) return warp_hip_moe_chunk_host(c, a->layer, a->x, a->out, a->n_tokens, a->route, a->rw);
    int idx[WARP_MAX_K];
    float w[WARP_MAX_K];
    hipStream_t st = (hipStream_t)warp_hip_stream(c);
    if (!HIPOK(hipMemcpyAsync(d->x_dev, a->x, (size_t)a->hidden * sizeof(float), hipMemcpyHostToDevice, st)))
        return WARP_HIP_E_DEVICE;
    /* with idx and w the call waits and reports a pick without a record */
    if ((rc = warp_hip_moe_decode(c, a->layer, d->x_dev, d->out_dev, NULL, idx, w))) return rc;
    if (!HIPOK(hipMemcpyAsync(a->out, d->out_dev, (size_t)a->hidden * sizeof(float), hipMemcpyDeviceToHost, st)) ||
        !HIPOK(hipStreamSynchronize(st)))
        return WARP_HIP_E_DEVICE;
    if ((rc = warp_hip_sync(c))) return rc;
    if (a->route) memcpy(a->route, idx, (size_t)K * sizeof(int));
    if (a->rw) memcpy(a->rw, w, (size_t)K * sizeof(float));
    return 0;
}

static int slot(const warp_moe_args *a, int batch)
{
    pthread_mutex_lock(&g_moe_mu);
    const int rc = moe_run(a, batch);
    if (rc == 0) g_moe_calls++; else g_moe_fallbacks++;
    int (*prev)(const warp_moe_args *) = batch ? g_prev_batch : g_prev_decode;
    pthread_mutex_unlock(&g_moe_mu);
    if (rc == 0) return 0;
    return prev ? prev(a) : rc;
}

static int hip_moe_ffn_decode(const warp_moe_args *a) { return slot(a, 0); }
static int hip_moe_ffn_batch(const warp_moe_args *a) { return slot(a, 1); }

const char *waste_register_hip_moe(waste_moe_kernels *t)
{
    int n = 0;
    if (!t || !HIPOK(hipGetDeviceCount(&n)) || n < 1) return NULL;
    char arch[64];
    if (wk_device_arch(0, arch, sizeof arch) || strncmp(arch, "gfx950", 6) != 0) return NULL;
    pthread_mutex_lock(&g_moe_mu);
    if (t->moe_ffn_decode != hip_moe_ffn_decode) g_prev_decode = t->moe_ffn_decode;
    if (t->moe_ffn_batch != hip_moe_ffn_batch) g_prev_batch = t->moe_ffn_batch;
    pthread_mutex_unlock(&g_moe_mu);
    t->moe_ffn_decode = hip_moe_ffn_decode;
    t->moe_ffn_batch = hip_moe_ffn_batch;
    t->on_device = 1;
    return "HIP gfx950";
}

void warp_hip_moe_table_stats(uint64_t *device_calls, uint64_t *fallback_calls)
{
    pthread_mutex_lock(&g_moe_mu);
    if (device_calls) *device_calls = g_moe_calls;
    if (fallback_calls) *fallback_calls = g_moe_fallbacks;
    pthread_mutex_unlock(&g_moe_mu);
}

/* Drops every model's context (called by waste_hip_release_host_buffers). */
void warp_moe_release(void)
{
    pthread_mutex_lock(&g_moe_mu);
    for (int i = 0; i < MOE_MAX_MODELS; i++)
        if (g_moe[i].c || g_moe[i].lk) moe_drop(&g_moe[i]);
    pthread_mutex_unlock(&g_moe_mu);
}
