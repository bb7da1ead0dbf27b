/*
 * backend.c — host side of the MI355X backend, in C, over the HIP runtime
 * API. Implements include/warp_hip.h: the reference's dispatch-table
 * registration, the device context that keeps codebooks, routers, shared
 * experts and an expert cache resident in HBM, the miss path (pinned
 * staging, copies on a side stream, lookahead prefetch), and the layer and
 * chunk orchestration over the kernels of kernels.hip.
 */
#define _GNU_SOURCE
#include <hip/hip_runtime_api.h>

#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "warp_hip.h"
#include "warp_internal.h"

#define SLOT_LEAD 80            /* record start in its slot: header + 80 = 128 */

#define HIPOK(x) ((x) == hipSuccess)

/* ---- small utilities ----------------------------------------------------- */

static int fmt_stages(int fmt)
{
    switch (fmt) {
    case WARP_HIP_VQ3R: return 3;
    case WARP_HIP_VQ2R: return 2;
    case WARP_HIP_VQ4P: return 4;
    case WARP_HIP_VQ12: return 2;
    }
    return 0;
}

static int fmt_entries(int fmt)
{
    switch (fmt) {
    case WARP_HIP_VQ3R: case WARP_HIP_VQ2R: return 256;
    case WARP_HIP_VQ4P: return 64;
    case WARP_HIP_VQ12: return 4096;
    }
    return 0;
}

static int fmt_slot(int fmt)
{
    switch (fmt) {
    case WARP_HIP_VQ3R: return 3;
    case WARP_HIP_VQ2R: return 2;
    case WARP_HIP_VQ4P: return 3;
    case WARP_HIP_VQ12: return 3;
    }
    return 0;
}

static size_t index_bytes(int fmt, int M, int N)
{
    return ((size_t)(M + WARP_TILE - 1) / WARP_TILE) * (size_t)(N / 8) * WARP_TILE * fmt_slot(fmt);
}

/* ---- 1. the dispatch-table slot ---------------------------------------------- */

/* mvq_arg, src/simd.h:35-39 (same member order and types) */
typedef struct {
    float *y; const int8_t *W; const uint16_t *ws;
    const int8_t *xq; const float *xs; int in, ng, group, bits;
    size_t rowbytes;
} mvq_arg_t;

typedef struct {
    const void *host;
    size_t bytes;
    void *dev;
} mirror_t;

static pthread_mutex_t g_tab_mu = PTHREAD_MUTEX_INITIALIZER;
static void (*g_prev_mvq)(int, int, void *);
typedef void (*kda_fn)(int, int, int, const float *, const float *, const float *, const float *, const float *,
                       float *, float *, float *);
static kda_fn g_prev_kda;
static float *g_kda_buf;
static size_t g_kda_cap;
static float *g_kda_stage;        /* pinned: the stepped state and output before they are committed */
static size_t g_kda_stage_cap;
static uint64_t g_kda_calls, g_kda_fallbacks;
static mirror_t *g_mirrors;
static int g_n_mirrors, g_cap_mirrors;
static hipStream_t g_tab_stream;
static float *g_tab_x, *g_tab_y;
static size_t g_tab_x_cap, g_tab_y_cap;
static uint64_t g_dev_calls, g_fallback_calls;

/* Device copy of a host buffer, keyed by its pointer (the Metal backend's
 * no-copy buffers, src/metal.m:98-150, are the precedent: trunk tensors do
 * not change while a model is open). Grows when a longer range is asked. */
static void *mirror_of(const void *host, size_t bytes)
{
    for (int i = 0; i < g_n_mirrors; i++)
        if (g_mirrors[i].host == host) {
            if (g_mirrors[i].bytes >= bytes) return g_mirrors[i].dev;
            (void)hipFree(g_mirrors[i].dev);
            g_mirrors[i] = g_mirrors[--g_n_mirrors];
            break;
        }
    if (g_n_mirrors == g_cap_mirrors) {
        const int cap = g_cap_mirrors ? 2 * g_cap_mirrors : 64;
        mirror_t *m = (mirror_t *)realloc(g_mirrors, (size_t)cap * sizeof *m);
        if (!m) return NULL;
        g_mirrors = m;
        g_cap_mirrors = cap;
    }
    void *dev = NULL;
    if (!HIPOK(hipMalloc(&dev, bytes))) return NULL;
    if (!HIPOK(hipMemcpy(dev, host, bytes, hipMemcpyHostToDevice))) { (void)hipFree(dev); return NULL; }
    g_mirrors[g_n_mirrors++] = (mirror_t){ host, bytes, dev };
    return dev;
}

static int grow(float **p, size_t *cap, size_t n)
{
    if (*cap >= n) return 0;
    if (*p) (void)hipFree(*p);
    *p = NULL;
    *cap = 0;
    if (!HIPOK(hipMalloc((void **)p, n * sizeof(float)))) return -1;
    *cap = n;
    return 0;
}

static int mvq_on_device(int b, int e, const mvq_arg_t *a)
{
    if (!g_tab_stream && !HIPOK(hipStreamCreate(&g_tab_stream))) return -1;
    const size_t rows = (size_t)e;
    const int8_t *W = (const int8_t *)mirror_of(a->W, rows * a->rowbytes);
    const uint16_t *ws = (const uint16_t *)mirror_of(a->ws, rows * (size_t)a->ng * sizeof(uint16_t));
    if (!W || !ws) return -1;
    if (grow(&g_tab_x, &g_tab_x_cap, (size_t)a->in) || grow(&g_tab_y, &g_tab_y_cap, rows)) return -1;
    if (!HIPOK(hipMemcpyAsync(g_tab_x, a->xs, (size_t)a->in * sizeof(float), hipMemcpyHostToDevice, g_tab_stream)))
        return -1;
    if (wk_mvq(W + (size_t)b * a->rowbytes, ws + (size_t)b * a->ng, a->rowbytes, a->group, a->bits, g_tab_x,
               e - b, a->in, 1, g_tab_y, g_tab_stream))
        return -1;
    if (!HIPOK(hipMemcpyAsync(a->y + b, g_tab_y, (size_t)(e - b) * sizeof(float), hipMemcpyDeviceToHost,
                              g_tab_stream)))
        return -1;
    return HIPOK(hipStreamSynchronize(g_tab_stream)) ? 0 : -1;
}

/* The mvq_rows_f32 slot (src/simd.h:15-19, src/model.c:385-399). */
static void hip_mvq_rows_f32(int b, int e, void *p)
{
    const mvq_arg_t *a = (const mvq_arg_t *)p;
    if (e <= b) return;
    pthread_mutex_lock(&g_tab_mu);
    const int rc = mvq_on_device(b, e, a);
    if (rc == 0) g_dev_calls++; else g_fallback_calls++;
    pthread_mutex_unlock(&g_tab_mu);
    if (rc != 0 && g_prev_mvq) g_prev_mvq(b, e, p);
}

/* The kda_step slot (src/waste_backend.h:69-72): host pointers, so the
 * inputs and the state go to the device and the state and output come back
 * on every call; one block per head does the step (wk_kda). The results
 * land in a pinned staging buffer and reach the caller's S and o only once
 * the stream has completed, so a failure leaves S as it was and the CPU
 * fallback steps it exactly once. */
static int kda_on_device(int H, int K, int V, const float *q, const float *k, const float *v, const float *g,
                         const float *beta, float *S, float *o)
{
    if (!g_tab_stream && !HIPOK(hipStreamCreate(&g_tab_stream))) return -1;
    const size_t hk = (size_t)H * K, hv = (size_t)H * V, ns = (size_t)H * K * V;
    const size_t need = 3 * hk + 2 * hv + (size_t)H + ns;
    if (g_kda_cap < need) {
        if (g_kda_buf) (void)hipFree(g_kda_buf);
        g_kda_buf = NULL;
        g_kda_cap = 0;
        if (!HIPOK(hipMalloc((void **)&g_kda_buf, need * sizeof(float)))) return -1;
        g_kda_cap = need;
    }
    float *dq = g_kda_buf, *dk = dq + hk, *dg = dk + hk, *dv = dg + hk, *dob = dv + hv, *db = dob + hv, *dS = db + H;
    const struct { float *d; const float *h; size_t n; } in[] = {
        { dq, q, hk }, { dk, k, hk }, { dg, g, hk }, { dv, v, hv }, { db, beta, (size_t)H }, { dS, S, ns } };
    for (size_t i = 0; i < sizeof in / sizeof in[0]; i++)
        if (!HIPOK(hipMemcpyAsync(in[i].d, in[i].h, in[i].n * sizeof(float), hipMemcpyHostToDevice, g_tab_stream)))
            return -1;
    if (wk_kda(1, H, K, V, dq, dk, dv, dg, db, dS, dob, g_tab_stream)) return -1;
    if (g_kda_stage_cap < ns + hv) {
        if (g_kda_stage) (void)hipHostFree(g_kda_stage);
        g_kda_stage = NULL;
        g_kda_stage_cap = 0;
        if (!HIPOK(hipHostMalloc((void **)&g_kda_stage, (ns + hv) * sizeof(float), 0))) return -1;
        g_kda_stage_cap = ns + hv;
    }
    if (!HIPOK(hipMemcpyAsync(g_kda_stage, dS, ns * sizeof(float), hipMemcpyDeviceToHost, g_tab_stream)) ||
        !HIPOK(hipMemcpyAsync(g_kda_stage + ns, dob, hv * sizeof(float), hipMemcpyDeviceToHost, g_tab_stream)) ||
        !HIPOK(hipStreamSynchronize(g_tab_stream)))
        return -1;
    memcpy(S, g_kda_stage, ns * sizeof(float));
    memcpy(o, g_kda_stage + ns, hv * sizeof(float));
    return 0;
}

static void hip_kda_step(int H, int K, int V, const float *q, const float *k, const float *v, const float *g_log,
                         const float *beta, float *S, float *o, float *scratch)
{
    pthread_mutex_lock(&g_tab_mu);
    const int rc = kda_on_device(H, K, V, q, k, v, g_log, beta, S, o);
    if (rc == 0) g_kda_calls++; else g_kda_fallbacks++;
    pthread_mutex_unlock(&g_tab_mu);
    if (rc != 0 && g_prev_kda) g_prev_kda(H, K, V, q, k, v, g_log, beta, S, o, scratch);
}

static int device_is_gfx950(int dev)
{
    char arch[64];
    if (wk_device_arch(dev, arch, sizeof arch)) return 0;
    return strncmp(arch, "gfx950", 6) == 0;
}

const char *waste_register_hip(waste_kernels *t)
{
    int n = 0;
    if (!HIPOK(hipGetDeviceCount(&n)) || n < 1) return NULL;
    if (!device_is_gfx950(0)) return NULL;
    pthread_mutex_lock(&g_tab_mu);
    if (t->mvq_rows_f32 != hip_mvq_rows_f32) g_prev_mvq = t->mvq_rows_f32;
    if (t->kda_step != hip_kda_step) g_prev_kda = t->kda_step;
    pthread_mutex_unlock(&g_tab_mu);
    t->mvq_rows_f32 = hip_mvq_rows_f32;
    t->kda_step = hip_kda_step;
    t->on_device = 1;
    return "HIP gfx950";
}

void waste_hip_release_host_buffers(void)
{
    pthread_mutex_lock(&g_tab_mu);
    for (int i = 0; i < g_n_mirrors; i++) (void)hipFree(g_mirrors[i].dev);
    g_n_mirrors = 0;
    pthread_mutex_unlock(&g_tab_mu);
    warp_moe_release();
}

void warp_hip_table_stats(uint64_t *device_calls, uint64_t *fallback_calls)
{
    pthread_mutex_lock(&g_tab_mu);
    if (device_calls) *device_calls = g_dev_calls;
    if (fallback_calls) *fallback_calls = g_fallback_calls;
    pthread_mutex_unlock(&g_tab_mu);
}

void warp_hip_kda_stats(uint64_t *device_calls, uint64_t *fallback_calls)
{
    pthread_mutex_lock(&g_tab_mu);
    if (device_calls) *device_calls = g_kda_calls;
    if (fallback_calls) *fallback_calls = g_kda_fallbacks;
    pthread_mutex_unlock(&g_tab_mu);
}

int warp_hip_kda_forward(int T, int H, int K, int V, const float *q_dev, const float *k_dev, const float *v_dev,
                         const float *g_dev, const float *beta_dev, float *S_dev, float *o_dev, void *stream)
{
    if (!q_dev || !k_dev || !v_dev || !g_dev || !beta_dev || !S_dev || !o_dev) return WARP_HIP_E_ARG;
    const int rc = wk_kda(T, H, K, V, q_dev, k_dev, v_dev, g_dev, beta_dev, S_dev, o_dev, stream);
    return rc == -1 ? WARP_HIP_E_ARG : rc ? WARP_HIP_E_DEVICE : 0;
}

/* ---- 2. the context ---------------------------------------------------------------- */

typedef struct {
    uint16_t *books;            /* [3][S][E][8] fp16, flushed              */
    int books_x31;              /* some book value has exponent 31         */
    int cb_base, has_books;
    float *router;              /* [E][H] or NULL                          */
    int8_t *rq; uint16_t *rs;   /* quantised router                        */
    size_t r_rowbytes; int r_bits, r_group;
    float *bias;                /* [E] or NULL                             */
    int8_t *sq[3]; uint16_t *ss[3];
    size_t s_rowbytes[3]; int s_bits, s_group, s_inter;
    int s_small;    /* every shared scale finite and below 256 in magnitude */
    int8_t *lq[2]; uint16_t *ls[2];  /* latent down [latent][H], up [H][latent] */
    size_t l_rowbytes[2]; int l_bits, l_group;
    float *lnorm;               /* [latent] or NULL                        */
    int resident;               /* records of this layer in the cache      */
} layer_t;

#define N_STAGE 32
#define N_TQ 4                  /* pinned lists of table updates in flight */
#define CRC_MAX_BYTES ((size_t)16 << 30)   /* longest buffer warp_hip_crc32 takes */
#define WARP_TIMING_N 2048
#define WARP_TIMING_CLS 4

struct warp_hip_ctx {
    warp_hip_cfg cfg;
    int He;                     /* the experts' width: cfg.latent, or cfg.hidden */
    int S, En, SB, P6, P_max, max_jobs;
    size_t gate_bytes, down_bytes;
    hipStream_t st, cp, la;
    hipStream_t sx;                 /* a chunk's shared expert, beside its routed experts */
    hipEvent_t ev_sx0, ev_sx1;      /* fork from st, join back into st */
    int sx_pending;                 /* a fork whose join a failed call skipped */
    hipEvent_t ev_copy, ev_before, ev_after, ev_la, ev_x, ev_stage[N_STAGE];
    int copy_pending;
    layer_t *L;
    /* expert cache */
    uint8_t *pool;
    int n_slots, next_free, n_empty;   /* n_empty: freed slots below next_free */
    size_t slot_stride;         /* bytes between slots (see slot_rec)       */
    int *slot_key, *key_slot;
    uint16_t *rec_cb;           /* [layer][expert]: the codebook_id of the
                                 * record the key last placed             */
    int n_books;                /* cfg.n_books, or n_layers * 3 * stages  */
    uint32_t *hits;
    uint64_t *last, clock;
    unsigned rng;
    warp_slot *table_dev;       /* [layer][expert] residency and offsets  */
    uint8_t *staging;           /* pinned, N_STAGE records                 */
    int stage_next, stage_used[N_STAGE];
    /* Expert-table updates of a batch of fills, applied by one launch on
     * the copy stream after the batch's copies (each key once, the last
     * value): the copies are not interleaved with kernels. */
    warp_slot_upd *tq_host[N_TQ];   /* pinned                             */
    warp_slot_upd *tq_dev;
    hipEvent_t ev_tq[N_TQ];
    int tq_used[N_TQ], tq_cur, tq_n, tq_cap;
    int *tq_pos;                    /* [layer][expert]: index in the list, or -1 */
    warp_hip_fetch_fn fetch;
    void *fetch_user;
    warp_hip_fetch_host_fn fetch_host;  /* records read in place from pinned host memory */
    void *fetch_host_user;
    warp_hip_cache_stats stats;
    /* device crc32 of records entering the cache (cfg.verify): per key the
     * verdict of its last checked fill, and the keys the table refused */
    uint32_t *crc_tmp;              /* block sums, then one output word    */
    int8_t *crc_bad;                /* [layer][expert]                     */
    warp_crc_err *crc_err, *h_crc_err;
    uint32_t *h_word;               /* pinned: one result word             */
    int crc_pending;                /* checked fills not yet read back     */
    /* Holds keep records from eviction: `hold` is the selection of the
     * layer in flight, `spec_hold` what the last lookahead brought in or
     * found resident. A key is held when its pin_gen equals either; 0 is
     * no hold. */
    uint32_t *pin_gen;              /* [layer][expert]                     */
    uint32_t hold, spec_hold, hold_next;
    int pin_layer;                  /* the layer `hold` belongs to, or -1  */
    /* device scratch */
    float *logits;
    unsigned long long *cert_ctr;  /* certified decode routings that recomputed, rows recomputed */
    unsigned *cert_sync;           /* the certifying router's launch counter and tagged rows (after cert_ctr) */
    unsigned cert_polls;           /* its poll limit (0: the kernel's default) */
    warp_hip_route_stats route_stats;
    int *idx;
    float *w;
    warp_job *jobs;
    int *njobs, *missing;
    uint16_t *xs;
    float *xscale;
    float *yg, *yu, *yd;
    uint16_t *xsh;
    float *xscaleh, *hbuf;
    uint16_t *xsp;                /* prefill_fp16: x per pair slot, position-group-major */
    float *xscalep;
    float *shg, *shu, *shh, *sho;
    uint16_t *shxs;               /* the shared expert's h split for the matrix cores */
    float *shxscale;
    uint16_t *shxin;              /* its x split (a chunk's routed experts use xs meanwhile) */
    float *shxinscale;
    int sh_cap;
    int8_t *lut8, *lut8d;
    float *lscale, *lscaled;
    float *part;                /* LUT matvec partial sums                 */
    unsigned *fz_sync;          /* the fused decode launch's counters (zero between launches) */
    unsigned *run_queue;        /* the prefill run launches' unit queues (zero between launches) */
    size_t part_cap;            /* floats                                  */
    int n_cu, lut_ok, mv_path;
    int *counts, *offsets, *pair_tok, *pair_exp;
    int *tok_slots;               /* per token, its pair slots in ascending expert id */
    int *runs;                    /* prefill: runs of one expert's jobs (first << 3 | count) */
    float *pair_w;
    float *xin, *xout;
    float *xlat, *ylat, *yup;     /* latent MoE: experts' input and output, up projection */
    float *la_logits;
    int *la_idx;
    float *la_w;
    int la_T;                     /* tokens of the lookahead in flight      */
    int *la_votes, *la_order;     /* [E] host: per expert, tokens predicting it; ids in prefetch order */
    /* pinned host */
    int *h_idx, *h_la_idx, *h_missing;
    float *h_w;
    /* optional per-launch timing of the expert matvecs (HIP events on the
     * compute stream) */
    int missing_pending;          /* a sticky device flag may be set        */
    int timing;
    hipEvent_t *tev;              /* [WARP_TIMING_N][2]                    */
    int tev_cls[WARP_TIMING_N], tev_n;
    double t_ms[WARP_TIMING_CLS];
    uint64_t t_cnt[WARP_TIMING_CLS];
    char err[256];
    int err_layer, err_expert;
};

static int set_err(warp_hip_ctx *c, int code, int layer, int expert, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(c->err, sizeof c->err, fmt, ap);
    va_end(ap);
    c->err_layer = layer;
    c->err_expert = expert;
    return code;
}

static int dev_err(warp_hip_ctx *c, const char *what, hipError_t e)
{
    return set_err(c, WARP_HIP_E_DEVICE, -1, -1, "%s: %s", what, hipGetErrorString(e));
}

#define DEV(c, call)                                               \
    do {                                                           \
        hipError_t e__ = (call);                                   \
        if (e__ != hipSuccess) return dev_err((c), #call, e__);    \
    } while (0)

#define KRN(c, call)                                                          \
    do {                                                                      \
        int r__ = (call);                                                     \
        if (r__) return set_err((c), r__ == -1 ? WARP_HIP_E_ARG : WARP_HIP_E_DEVICE, -1, -1, \
                                "%s failed (%d)", #call, r__);                \
    } while (0)

const char *warp_hip_error(const warp_hip_ctx *c, int *layer, int *expert)
{
    if (layer) *layer = c ? c->err_layer : -1;
    if (expert) *expert = c ? c->err_expert : -1;
    return c ? c->err : "no context";
}

void *warp_hip_stream(warp_hip_ctx *c) { return c ? (void *)c->st : NULL; }

static int dmalloc(warp_hip_ctx *c, void **p, size_t bytes)
{
    *p = NULL;
    if (!bytes) bytes = 16;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
        *p = NULL;
        return set_err(c, WARP_HIP_E_NOMEM, -1, -1, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    }
    return 0;
}

#define DMALLOC(c, p, bytes) do { if (dmalloc((c), (void **)&(p), (bytes))) return WARP_HIP_E_NOMEM; } while (0)

/* A chunk's reduced-precision mode, while its inputs by pair slot stay
 * under 2 GiB (32-bit buffer offsets); past that, chunks keep the exact
 * by-token kernel. */
static int prefill_fp16(const warp_hip_ctx *c)
{
    const size_t w = (size_t)(c->He > c->cfg.inter ? c->He : c->cfg.inter);
    return c->cfg.prefill_fp16 && !c->P6 &&
           (size_t)c->cfg.max_tokens * c->cfg.top_k * w * 2 < ((size_t)1 << 31);
}

static int ctx_alloc(warp_hip_ctx *c)
{
    const warp_hip_cfg *g = &c->cfg;
    const int E = g->n_experts, K = g->top_k, H = g->hidden, I = g->inter, T = g->max_tokens;
    const int He = c->He, Hm = H > He ? H : He;    /* experts' width; the wider of the two */
    const size_t P = (size_t)T * K;
    c->P_max = (int)P;
    c->max_jobs = (int)(P / WARP_TPJ + (size_t)E + 1);
    if (c->max_jobs < K) c->max_jobs = K;
    const size_t nvH = (size_t)He / 8, nvI = (size_t)I / 8;
    const size_t nblkH = (nvH + WARP_LUT_BLK - 1) / WARP_LUT_BLK, nblkI = (nvI + WARP_LUT_BLK - 1) / WARP_LUT_BLK;
    /* at least four rows: one token's scores, biased scores and their
     * bounds (wk_router_cert) */
    DMALLOC(c, c->logits, (size_t)(T > 4 ? T : 4) * E * 4);
    /* the certification's counters, then the certifier's launch counter and
     * tagged rows */
    DMALLOC(c, c->cert_ctr, 2 * sizeof(unsigned long long) + WK_CERT_SYNC_WORDS(E) * sizeof(unsigned));
    DEV(c, hipMemset(c->cert_ctr, 0, 2 * sizeof(unsigned long long) + WK_CERT_SYNC_WORDS(E) * sizeof(unsigned)));
    c->cert_sync = (unsigned *)(c->cert_ctr + 2);
    DMALLOC(c, c->idx, P * 4);
    DMALLOC(c, c->w, P * 4);
    DMALLOC(c, c->jobs, (size_t)3 * c->max_jobs * sizeof(warp_job));
    /* zeroed, with the counts: lists read before any routing has written
     * them hold no jobs and NULL records */
    DEV(c, hipMemset(c->jobs, 0, (size_t)3 * c->max_jobs * sizeof(warp_job)));
    DMALLOC(c, c->njobs, 4 * sizeof(int));
    DEV(c, hipMemset(c->njobs, 0, 4 * sizeof(int)));
    DMALLOC(c, c->missing, sizeof(int));
    DMALLOC(c, c->xs, (size_t)T * Hm * 2 * 2);
    DMALLOC(c, c->xscale, (size_t)T * 4);
    DMALLOC(c, c->yg, P * I * 4);
    DMALLOC(c, c->yu, P * I * 4);
    DMALLOC(c, c->yd, P * He * 4);
    DMALLOC(c, c->xsh, P * I * 2 * 2);
    DMALLOC(c, c->xscaleh, P * 4);
    DMALLOC(c, c->hbuf, P * I * 4);
    if (prefill_fp16(c)) {
        DMALLOC(c, c->xsp, P * He * 2);
        DMALLOC(c, c->xscalep, P * 4);
    }
    DMALLOC(c, c->sho, (size_t)T * H * 4);
    DMALLOC(c, c->xin, (size_t)T * H * 4);
    DMALLOC(c, c->xout, (size_t)T * H * 4);
    if (g->latent) {
        DMALLOC(c, c->xlat, (size_t)T * He * 4);
        DMALLOC(c, c->ylat, (size_t)T * He * 4);
        DMALLOC(c, c->yup, (size_t)T * H * 4);
    }
    DMALLOC(c, c->counts, ((size_t)E + 1) * 4);
    DMALLOC(c, c->offsets, ((size_t)E + 1) * 4);
    DMALLOC(c, c->pair_tok, P * 4);
    DMALLOC(c, c->pair_exp, P * 4);
    DMALLOC(c, c->pair_w, P * 4);
    DMALLOC(c, c->tok_slots, P * 4);
    DMALLOC(c, c->runs, (size_t)c->max_jobs * 4);
    DMALLOC(c, c->la_logits, (size_t)T * E * 4);
    DMALLOC(c, c->la_idx, (size_t)T * WARP_MAX_K * 4);
    DMALLOC(c, c->la_w, (size_t)T * WARP_MAX_K * 4);
    if (c->lut_ok) {
        /* decode: gate+up over K jobs sharing x, then down per job */
        int gr, sp;
        size_t need = 0;
        if (!wk_lut_plan(I, He, K, 2, 1, c->n_cu, (size_t)-1, &gr, &sp))
            need = (size_t)2 * sp * K * (((size_t)I + 63) / 64) * 64;
        if (!wk_lut_plan(He, I, K, 1, 0, c->n_cu, (size_t)-1, &gr, &sp))
            need += (size_t)sp * K * (((size_t)He + 63) / 64) * 64;   /* down partials after the gate/up ones */
        c->part_cap = need;
        DMALLOC(c, c->part, need * sizeof(float));
    }
    if (c->P6) {
        DMALLOC(c, c->lut8, (size_t)T * 2 * nvH * 256);
        DMALLOC(c, c->lscale, (size_t)T * 2 * nblkH * 4);
        DMALLOC(c, c->lut8d, P * nvI * 256);
        DMALLOC(c, c->lscaled, P * nblkI * 4);
    }
    DMALLOC(c, c->run_queue, WARP_RUNQ_WORDS * sizeof(unsigned));
    DEV(c, hipMemset(c->run_queue, 0, WARP_RUNQ_WORDS * sizeof(unsigned)));
    if (c->lut_ok) {
        DMALLOC(c, c->fz_sync, WARP_FZ_WORDS * sizeof(unsigned));
        DEV(c, hipMemset(c->fz_sync, 0, WARP_FZ_WORDS * sizeof(unsigned)));
    }
    DEV(c, hipMemset(c->missing, 0, sizeof(int)));
    DEV(c, hipHostMalloc((void **)&c->h_idx, P * 4, 0));
    DEV(c, hipHostMalloc((void **)&c->h_w, P * 4, 0));
    DEV(c, hipHostMalloc((void **)&c->h_la_idx, (size_t)T * WARP_MAX_K * 4, 0));
    DEV(c, hipHostMalloc((void **)&c->h_missing, 4 * sizeof(int), 0));
    /* expert cache */
    c->n_slots = g->rec_bytes ? (int)(g->cache_bytes / g->rec_bytes) : 0;
    const size_t nkeys = (size_t)g->n_layers * E;
    c->key_slot = (int *)malloc(nkeys * sizeof(int));
    c->slot_key = (int *)malloc(((size_t)c->n_slots + 1) * sizeof(int));
    c->hits = (uint32_t *)calloc((size_t)c->n_slots + 1, sizeof(uint32_t));
    c->pin_gen = (uint32_t *)calloc(nkeys, sizeof(uint32_t));
    c->rec_cb = (uint16_t *)calloc(nkeys, sizeof(uint16_t));
    c->la_votes = (int *)calloc((size_t)E, sizeof(int));
    c->la_order = (int *)calloc((size_t)E, sizeof(int));
    c->last = (uint64_t *)calloc((size_t)c->n_slots + 1, sizeof(uint64_t));
    if (!c->key_slot || !c->slot_key || !c->hits || !c->last || !c->pin_gen || !c->rec_cb || !c->la_votes ||
        !c->la_order)
        return set_err(c, WARP_HIP_E_NOMEM, -1, -1, "host allocation failed");
    for (size_t i = 0; i < nkeys; i++) c->key_slot[i] = -1;
    for (int i = 0; i < c->n_slots; i++) c->slot_key[i] = -1;
    DMALLOC(c, c->table_dev, nkeys * sizeof(warp_slot));
    DEV(c, hipMemset(c->table_dev, 0, nkeys * sizeof(warp_slot)));
    DMALLOC(c, c->crc_tmp, (wk_crc32_tmp_words(CRC_MAX_BYTES) + 1) * sizeof(uint32_t));
    DMALLOC(c, c->crc_bad, nkeys);
    DEV(c, hipMemset(c->crc_bad, 0, nkeys));
    DMALLOC(c, c->crc_err, sizeof(warp_crc_err));
    DEV(c, hipMemset(c->crc_err, 0, sizeof(warp_crc_err)));
    DEV(c, hipHostMalloc((void **)&c->h_crc_err, sizeof(warp_crc_err), 0));
    DEV(c, hipHostMalloc((void **)&c->h_word, sizeof(uint32_t), 0));
    c->slot_stride = (g->rec_bytes + SLOT_LEAD + 255) / 256 * 256;
    if (c->n_slots > 0) DMALLOC(c, c->pool, (size_t)c->n_slots * c->slot_stride);
    DEV(c, hipHostMalloc((void **)&c->staging, (size_t)N_STAGE * g->rec_bytes, 0));
    /* a batch touches each expert of one layer at most twice over (the
     * records it places and the ones they evict) */
    c->tq_cap = 2 * E + 2;
    for (int i = 0; i < N_TQ; i++) DEV(c, hipHostMalloc((void **)&c->tq_host[i], (size_t)c->tq_cap * sizeof(warp_slot_upd), 0));
    DMALLOC(c, c->tq_dev, (size_t)c->tq_cap * sizeof(warp_slot_upd));
    c->tq_pos = (int *)malloc(nkeys * sizeof(int));
    if (!c->tq_pos) return set_err(c, WARP_HIP_E_NOMEM, -1, -1, "host allocation failed");
    for (size_t i = 0; i < nkeys; i++) c->tq_pos[i] = -1;
    return 0;
}

int warp_hip_open(const warp_hip_cfg *cfg, warp_hip_ctx **out)
{
    *out = NULL;
    warp_hip_ctx *c = (warp_hip_ctx *)calloc(1, sizeof *c);
    if (!c) return WARP_HIP_E_NOMEM;
    c->cfg = *cfg;
    c->err_layer = c->err_expert = -1;
    c->pin_layer = -1;
    c->rng = 0x9E3779B9u;
    warp_hip_cfg *g = &c->cfg;
    c->S = fmt_stages(g->fmt);
    c->En = fmt_entries(g->fmt);
    c->SB = fmt_slot(g->fmt);
    c->P6 = g->fmt == WARP_HIP_VQ4P;
    if (g->max_tokens < 1) g->max_tokens = 1;
    c->He = g->latent > 0 ? g->latent : g->hidden;
    const int He = c->He;
    int rc = WARP_HIP_E_ARG;
    if (!c->S || g->hidden <= 0 || g->inter <= 0 || g->n_experts <= 0 || g->top_k <= 0 ||
        g->top_k > WARP_MAX_K || g->top_k > g->n_experts || g->n_layers <= 0 || g->n_layers > 65535 ||
        g->n_experts > 65535 || (g->rec_bytes % 4096) != 0 || g->lookahead < 0 || g->latent < 0 ||
        (g->latent && g->latent_norm && !(g->norm_eps > 0.0f)) || g->n_books < 0) {
        set_err(c, rc, -1, -1, "configuration out of range");
        goto fail;
    }
    c->n_books = g->n_books > 0 ? g->n_books : g->n_layers * 3 * c->S;
    if (!c->P6 && (He % 32 || g->inter % 32 || g->hidden % 32)) {
        set_err(c, rc, -1, -1, "hidden, latent and inter must be multiples of 32 (4 vector positions)");
        goto fail;
    }
    if (He % 8 || g->inter % 8 || g->hidden % 8) {
        set_err(c, rc, -1, -1, "hidden, latent and inter must be multiples of vec_dim 8");
        goto fail;
    }
    c->gate_bytes = index_bytes(g->fmt, g->inter, He);
    c->down_bytes = index_bytes(g->fmt, He, g->inter);
    if (g->rec_bytes && WARP_HDR_BYTES + 2 * c->gate_bytes + c->down_bytes +
                            2 * (2 * (size_t)g->inter + He) > g->rec_bytes) {
        set_err(c, rc, -1, -1, "rec_bytes %zu cannot hold a record of this shape", g->rec_bytes);
        goto fail;
    }
    int ndev = 0;
    if (!HIPOK(hipGetDeviceCount(&ndev)) || g->device < 0 || g->device >= ndev) {
        set_err(c, WARP_HIP_E_DEVICE, -1, -1, "no HIP device %d", g->device);
        rc = WARP_HIP_E_DEVICE;
        goto fail;
    }
    if (!device_is_gfx950(g->device)) {
        set_err(c, WARP_HIP_E_DEVICE, -1, -1, "device %d is not gfx950", g->device);
        rc = WARP_HIP_E_DEVICE;
        goto fail;
    }
    if (!HIPOK(hipSetDevice(g->device)) || !HIPOK(hipStreamCreateWithFlags(&c->st, hipStreamNonBlocking)) ||
        !HIPOK(hipStreamCreateWithFlags(&c->cp, hipStreamNonBlocking)) ||
        !HIPOK(hipStreamCreateWithFlags(&c->la, hipStreamNonBlocking)) ||
        !HIPOK(hipStreamCreateWithFlags(&c->sx, hipStreamNonBlocking)) ||
        !HIPOK(hipEventCreateWithFlags(&c->ev_sx0, hipEventDisableTiming)) ||
        !HIPOK(hipEventCreateWithFlags(&c->ev_sx1, hipEventDisableTiming)) ||
        !HIPOK(hipEventCreateWithFlags(&c->ev_copy, hipEventDisableTiming)) ||
        !HIPOK(hipEventCreateWithFlags(&c->ev_before, hipEventDisableTiming)) ||
        !HIPOK(hipEventCreateWithFlags(&c->ev_after, hipEventDisableTiming)) ||
        !HIPOK(hipEventCreateWithFlags(&c->ev_la, hipEventDisableTiming)) ||
        !HIPOK(hipEventCreateWithFlags(&c->ev_x, hipEventDisableTiming))) {
        set_err(c, WARP_HIP_E_DEVICE, -1, -1, "stream/event creation failed");
        rc = WARP_HIP_E_DEVICE;
        goto fail;
    }
    for (int i = 0; i < N_STAGE; i++)
        if (!HIPOK(hipEventCreateWithFlags(&c->ev_stage[i], hipEventDisableTiming))) {
            rc = WARP_HIP_E_DEVICE;
            goto fail;
        }
    for (int i = 0; i < N_TQ; i++)
        if (!HIPOK(hipEventCreateWithFlags(&c->ev_tq[i], hipEventDisableTiming))) {
            rc = WARP_HIP_E_DEVICE;
            goto fail;
        }
    if (!HIPOK(hipDeviceGetAttribute(&c->n_cu, hipDeviceAttributeMultiprocessorCount, g->device)) || c->n_cu < 1)
        c->n_cu = 256;
    /* the LUT matvec serves decode for the float-LUT formats; it walks the
     * positions two at a time */
    c->lut_ok = !c->P6 && He % 16 == 0 && g->inter % 16 == 0;
    c->L = (layer_t *)calloc((size_t)g->n_layers, sizeof(layer_t));
    if (!c->L) { rc = WARP_HIP_E_NOMEM; goto fail; }
    if ((rc = ctx_alloc(c)) != 0) goto fail;
    *out = c;
    return 0;
fail:
    fprintf(stderr, "warp_hip_open: %s\n", c->err);
    warp_hip_close(c);
    return rc;
}

static void hfree(void *p) { if (p) (void)hipFree(p); }
static void hhfree(void *p) { if (p) (void)hipHostFree(p); }

void warp_hip_close(warp_hip_ctx *c)
{
    if (!c) return;
    if (c->st) (void)hipStreamSynchronize(c->st);
    if (c->cp) (void)hipStreamSynchronize(c->cp);
    if (c->la) (void)hipStreamSynchronize(c->la);
    if (c->sx) (void)hipStreamSynchronize(c->sx);
    if (c->L)
        for (int l = 0; l < c->cfg.n_layers; l++) {
            layer_t *L = &c->L[l];
            hfree(L->books); hfree(L->router); hfree(L->rq); hfree(L->rs); hfree(L->bias);
            for (int k = 0; k < 3; k++) { hfree(L->sq[k]); hfree(L->ss[k]); }
            for (int k = 0; k < 2; k++) { hfree(L->lq[k]); hfree(L->ls[k]); }
            hfree(L->lnorm);
        }
    free(c->L);
    void *d[] = { c->logits, c->idx, c->w, c->jobs, c->njobs, c->missing, c->xs, c->xscale, c->xsp, c->xscalep,
                  c->yg, c->yu,
                  c->yd, c->xsh, c->xscaleh, c->hbuf, c->shg, c->shu, c->shh, c->sho, c->lut8, c->lut8d,
                  c->lscale, c->lscaled, c->counts, c->offsets, c->pair_tok, c->pair_exp, c->pair_w, c->tok_slots, c->runs,
                  c->xin, c->xout, c->la_logits, c->la_idx, c->la_w, c->table_dev, c->pool, c->part,
                  c->shxs, c->shxscale, c->shxin, c->shxinscale, c->tq_dev, c->crc_tmp, c->crc_bad, c->crc_err, c->xlat, c->ylat, c->yup,
                  c->fz_sync, c->run_queue, c->cert_ctr };
    for (size_t i = 0; i < sizeof d / sizeof d[0]; i++) hfree(d[i]);
    hhfree(c->h_idx); hhfree(c->h_w); hhfree(c->h_la_idx); hhfree(c->h_missing); hhfree(c->staging);
    hhfree(c->h_crc_err); hhfree(c->h_word);
    for (int i = 0; i < N_TQ; i++) hhfree(c->tq_host[i]);
    free(c->tq_pos);
    free(c->key_slot); free(c->slot_key); free(c->hits); free(c->last); free(c->pin_gen); free(c->rec_cb);
    free(c->la_votes); free(c->la_order);
    if (c->tev) {
        for (int i = 0; i < 2 * WARP_TIMING_N; i++) if (c->tev[i]) (void)hipEventDestroy(c->tev[i]);
        free(c->tev);
    }
    for (int i = 0; i < N_STAGE; i++) if (c->ev_stage[i]) (void)hipEventDestroy(c->ev_stage[i]);
    for (int i = 0; i < N_TQ; i++) if (c->ev_tq[i]) (void)hipEventDestroy(c->ev_tq[i]);
    if (c->ev_copy) (void)hipEventDestroy(c->ev_copy);
    if (c->ev_before) (void)hipEventDestroy(c->ev_before);
    if (c->ev_after) (void)hipEventDestroy(c->ev_after);
    if (c->ev_la) (void)hipEventDestroy(c->ev_la);
    if (c->ev_x) (void)hipEventDestroy(c->ev_x);
    if (c->st) (void)hipStreamDestroy(c->st);
    if (c->cp) (void)hipStreamDestroy(c->cp);
    if (c->la) (void)hipStreamDestroy(c->la);
    if (c->ev_sx0) (void)hipEventDestroy(c->ev_sx0);
    if (c->ev_sx1) (void)hipEventDestroy(c->ev_sx1);
    if (c->sx) (void)hipStreamDestroy(c->sx);
    free(c);
}

/* Where slot s's record starts. Slots are SLOT_LEAD + rec_bytes rounded up
 * to 256 bytes apart (the pool is 256-byte aligned), and a record starts
 * SLOT_LEAD bytes into its slot, so that its first index block, right after
 * the 48-byte header, starts on a 128-byte line: a chunk's code words of
 * one row block (a multiple of 128 bytes at the K3 shapes) then never share
 * a line with the next chunk's, which another block of the launch reads. */
static uint8_t *slot_rec(const warp_hip_ctx *c, int s)
{
    return c->pool + (size_t)s * c->slot_stride + SLOT_LEAD;
}

/* Reads and clears the sticky missing-expert flag once the compute stream
 * is idle. */
static int crc_report(warp_hip_ctx *c);

static int take_missing(warp_hip_ctx *c)
{
    int rc = crc_report(c);
    if (rc) return rc;
    if (!c->missing_pending) return 0;
    DEV(c, hipMemcpy(c->h_missing, c->missing, sizeof(int), hipMemcpyDeviceToHost));
    c->missing_pending = 0;
    if (*c->h_missing) {
        const int flag = *c->h_missing;
        DEV(c, hipMemset(c->missing, 0, sizeof(int)));
        if ((flag & 4) && c->cert_sync) {
            /* a certifying router that gave up advanced its launch counter
             * with a row possibly not yet written; written late, that row
             * carries the next launch's tag: once every launch is done, the
             * counter and the tagged rows start again from zero */
            DEV(c, hipStreamSynchronize(c->st));
            DEV(c, hipMemset(c->cert_sync, 0, WK_CERT_SYNC_WORDS(c->cfg.n_experts) * sizeof(unsigned)));
        }
        if (flag & 4)
            return set_err(c, WARP_HIP_E_DEVICE, -1, -1,
                           "a decode launch gave up waiting (the fused launch for its work items, or the "
                           "certifying router for its rows): its outputs are not valid");
        return set_err(c, WARP_HIP_E_MISSING, -1, -1,
                       "a selected expert was not resident: the affected layers were not computed");
    }
    return 0;
}

int warp_hip_sync(warp_hip_ctx *c)
{
    DEV(c, hipStreamSynchronize(c->la));
    DEV(c, hipStreamSynchronize(c->cp));
    DEV(c, hipStreamSynchronize(c->st));
    return take_missing(c);
}

/* ---- layer weights ------------------------------------------------------------------ */

static int check_layer(warp_hip_ctx *c, int layer)
{
    if (!c || layer < 0 || layer >= c->cfg.n_layers)
        return c ? set_err(c, WARP_HIP_E_ARG, layer, -1, "layer %d out of range", layer) : WARP_HIP_E_ARG;
    /* a chunk that failed after forking its shared expert left the side
     * stream unjoined: nothing on the compute stream may overtake it */
    if (c->sx_pending) {
        c->sx_pending = 0;
        DEV(c, hipStreamWaitEvent(c->st, c->ev_sx1, 0));
    }
    return 0;
}

static int upload(warp_hip_ctx *c, void **dst, const void *src, size_t bytes)
{
    if (*dst) { (void)hipFree(*dst); *dst = NULL; }
    if (dmalloc(c, dst, bytes)) return WARP_HIP_E_NOMEM;
    DEV(c, hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice));
    return 0;
}

int warp_hip_set_codebooks(warp_hip_ctx *c, int layer, int cb_base, const uint16_t *books)
{
    int rc = check_layer(c, layer);
    if (rc) return rc;
    /* the bank's codebook_base, bounded as the loader bounds it
     * (src/model.c:1341-1343) */
    if (!books || cb_base < 0 || cb_base > c->n_books - 3 * c->S)
        return set_err(c, WARP_HIP_E_ARG, layer, -1, "codebook base %d with %d books of %d stages", cb_base,
                       c->n_books, c->S);
    const size_t n = (size_t)3 * c->S * c->En * 8;
    uint16_t *tmp = (uint16_t *)malloc(n * sizeof(uint16_t));
    if (!tmp) return set_err(c, WARP_HIP_E_NOMEM, layer, -1, "host allocation failed");
    /* fp16 subnormals flush to signed zero, as the codebook load does
     * (src/model.c:1277-1286); exponent-31 values keep their bits and the
     * kernels rebias them as the reference does. */
    for (size_t i = 0; i < n; i++) tmp[i] = ((books[i] >> 10) & 0x1f) ? books[i] : (uint16_t)(books[i] & 0x8000);
    rc = upload(c, (void **)&c->L[layer].books, tmp, n * sizeof(uint16_t));
    /* the reference reads exponent 31 as a finite power of two; the LUT
     * kernel then needs its exact (slower) conversion */
    c->L[layer].books_x31 = 0;
    for (size_t i = 0; i < n; i++)
        if (((tmp[i] >> 10) & 0x1f) == 0x1f) { c->L[layer].books_x31 = 1; break; }
    free(tmp);
    if (rc) return rc;
    c->L[layer].cb_base = cb_base;
    c->L[layer].has_books = 1;
    return 0;
}

int warp_hip_set_router(warp_hip_ctx *c, int layer, const float *w, const float *bias)
{
    int rc = check_layer(c, layer);
    if (rc) return rc;
    if (!w) return set_err(c, WARP_HIP_E_ARG, layer, -1, "router weights missing");
    layer_t *L = &c->L[layer];
    if ((rc = upload(c, (void **)&L->router, w, (size_t)c->cfg.n_experts * c->cfg.hidden * 4))) return rc;
    hfree(L->rq); hfree(L->rs);
    L->rq = NULL; L->rs = NULL;
    if (bias) return upload(c, (void **)&L->bias, bias, (size_t)c->cfg.n_experts * 4);
    hfree(L->bias);
    L->bias = NULL;
    return 0;
}

int warp_hip_set_router_q(warp_hip_ctx *c, int layer, int bits, int group, const int8_t *q,
                          const uint16_t *scales, size_t rowbytes, const float *bias)
{
    int rc = check_layer(c, layer);
    if (rc) return rc;
    if ((bits != 8 && bits != 4 && bits != 3) || group <= 0 || !q || !scales)
        return set_err(c, WARP_HIP_E_ARG, layer, -1, "quantised router arguments");
    layer_t *L = &c->L[layer];
    const int E = c->cfg.n_experts, ng = (c->cfg.hidden + group - 1) / group;
    if ((rc = upload(c, (void **)&L->rq, q, (size_t)E * rowbytes))) return rc;
    if ((rc = upload(c, (void **)&L->rs, scales, (size_t)E * ng * 2))) return rc;
    L->r_rowbytes = rowbytes;
    L->r_bits = bits;
    L->r_group = group;
    hfree(L->router);
    L->router = NULL;
    if (bias) return upload(c, (void **)&L->bias, bias, (size_t)E * 4);
    hfree(L->bias);
    L->bias = NULL;
    return 0;
}

int warp_hip_set_latent(warp_hip_ctx *c, int layer, int bits, int group, const int8_t *down_q,
                        const uint16_t *down_s, size_t down_rowbytes, const int8_t *up_q, const uint16_t *up_s,
                        size_t up_rowbytes, const float *norm_w)
{
    int rc = check_layer(c, layer);
    if (rc) return rc;
    const warp_hip_cfg *g = &c->cfg;
    if (!g->latent) return set_err(c, WARP_HIP_E_ARG, layer, -1, "the context has no latent width");
    if ((bits != 8 && bits != 4 && bits != 3) || group <= 0 || !down_q || !down_s || !up_q || !up_s ||
        (g->latent_norm && !norm_w))
        return set_err(c, WARP_HIP_E_ARG, layer, -1, "latent projection arguments");
    layer_t *L = &c->L[layer];
    const int H = g->hidden, lat = g->latent;
    const int rows[2] = { lat, H }, cols[2] = { H, lat };
    const int8_t *q[2] = { down_q, up_q };
    const uint16_t *sc[2] = { down_s, up_s };
    const size_t rb[2] = { down_rowbytes, up_rowbytes };
    for (int k = 0; k < 2; k++) {
        const int ng = (cols[k] + group - 1) / group;
        if ((rc = upload(c, (void **)&L->lq[k], q[k], (size_t)rows[k] * rb[k]))) return rc;
        if ((rc = upload(c, (void **)&L->ls[k], sc[k], (size_t)rows[k] * ng * 2))) return rc;
        L->l_rowbytes[k] = rb[k];
    }
    L->l_bits = bits;
    L->l_group = group;
    if (g->latent_norm) return upload(c, (void **)&L->lnorm, norm_w, (size_t)lat * sizeof(float));
    return 0;
}

int warp_hip_set_shared(warp_hip_ctx *c, int layer, int bits, int group, int inter_shared,
                        const int8_t *const q[3], const uint16_t *const scales[3], const size_t rowbytes[3])
{
    int rc = check_layer(c, layer);
    if (rc) return rc;
    if ((bits != 8 && bits != 4 && bits != 3) || group <= 0 || inter_shared <= 0)
        return set_err(c, WARP_HIP_E_ARG, layer, -1, "shared expert arguments");
    layer_t *L = &c->L[layer];
    const int H = c->cfg.hidden, Is = inter_shared;
    const int rows[3] = { Is, Is, H }, cols[3] = { H, H, Is };
    int small = 1;
    for (int k = 0; k < 3; k++) {
        const int ng = (cols[k] + group - 1) / group;
        if ((rc = upload(c, (void **)&L->sq[k], q[k], (size_t)rows[k] * rowbytes[k]))) return rc;
        if ((rc = upload(c, (void **)&L->ss[k], scales[k], (size_t)rows[k] * ng * 2))) return rc;
        L->s_rowbytes[k] = rowbytes[k];
        /* fp16 magnitude below 256 = 2^8: biased exponent below 23 */
        for (size_t i = 0; i < (size_t)rows[k] * ng; i++)
            small &= (scales[k][i] & 0x7fffu) < 0x5c00u;
    }
    L->s_small = small;
    L->s_bits = bits;
    L->s_group = group;
    L->s_inter = Is;
    /* scratch for the shared expert, sized for the widest one set so far */
    int max_is = 0;
    for (int l = 0; l < c->cfg.n_layers; l++) if (c->L[l].s_inter > max_is) max_is = c->L[l].s_inter;
    if (max_is > c->sh_cap) {
        hfree(c->shg); hfree(c->shu); hfree(c->shh); hfree(c->shxs); hfree(c->shxscale);
        hfree(c->shxin); hfree(c->shxinscale);
        c->shg = c->shu = c->shh = NULL;
        c->shxs = c->shxin = NULL;
        c->shxscale = c->shxinscale = NULL;
        c->sh_cap = 0;
        const size_t bytes = (size_t)c->cfg.max_tokens * max_is * 4;
        DMALLOC(c, c->shg, bytes);
        DMALLOC(c, c->shu, bytes);
        DMALLOC(c, c->shh, bytes);
        DMALLOC(c, c->shxs, bytes);
        DMALLOC(c, c->shxscale, (size_t)c->cfg.max_tokens * 4);
        DMALLOC(c, c->shxin, (size_t)c->cfg.max_tokens * c->cfg.hidden * 2 * 2);
        DMALLOC(c, c->shxinscale, (size_t)c->cfg.max_tokens * 4);
        c->sh_cap = max_is;
    }
    return 0;
}

/* ---- expert cache ----------------------------------------------------------------------- */

/* record_check (src/model.c:1698-1745), its conditions in its order, then
 * one more that the kernels need: every index block at least as long as its
 * shape, and the scales after them (the reference accepts any increasing
 * offsets, and a short block then reads into the next one; here a kernel
 * would read past what the header describes). The payload checksum is taken
 * on the device (publish_slot), the codebook_id kept per key (rec_cb). */
static int check_record(warp_hip_ctx *c, const uint8_t *rec, int layer, int expert)
{
    const warp_hip_cfg *g = &c->cfg;
    uint32_t magic, blocks, off[4];
    uint16_t lay, eid, cbid, lowrank;
    uint8_t fmt;
    memcpy(&magic, rec + 0, 4);
    memcpy(&lay, rec + 4, 2);
    memcpy(&eid, rec + 6, 2);
    memcpy(&fmt, rec + 8, 1);
    memcpy(&cbid, rec + 10, 2);
    memcpy(&lowrank, rec + 12, 2);
    memcpy(&blocks, rec + 16, 4);
    memcpy(off, rec + 20, 16);
    if (g->rec_bytes < WARP_HDR_BYTES || magic != 0x50584557u)
        return set_err(c, WARP_HIP_E_HEADER, layer, expert, "record header: magic");
    if (lay != (uint16_t)layer || eid != (uint16_t)expert)
        return set_err(c, WARP_HIP_E_HEADER, layer, expert, "record header names layer %u expert %u", lay, eid);
    if ((size_t)blocks * 4096u != g->rec_bytes)
        return set_err(c, WARP_HIP_E_HEADER, layer, expert, "record of %u 4 KiB blocks, stride %zu", blocks,
                       g->rec_bytes);
    /* the label must be the one the container's index width implies; byte
     * codes also take the 2-stage label (the stage count is the
     * container's, not the record's) */
    const int bits8 = g->fmt == WARP_HIP_VQ3R || g->fmt == WARP_HIP_VQ2R;
    const int want = g->fmt == WARP_HIP_VQ4P ? WARP_HIP_VQ4P : g->fmt == WARP_HIP_VQ12 ? WARP_HIP_VQ12
                                                                                        : WARP_HIP_VQ3R;
    if (fmt != want && !(bits8 && fmt == WARP_HIP_VQ2R))
        return set_err(c, WARP_HIP_E_HEADER, layer, expert, "record fmt %d in a container of fmt %d", fmt, g->fmt);
    if (lowrank != 0) return set_err(c, WARP_HIP_E_HEADER, layer, expert, "record lowrank_id %u", lowrank);
    if ((long)cbid + 3L * c->S > c->n_books)
        return set_err(c, WARP_HIP_E_HEADER, layer, expert, "record codebook_id %u with %d books", cbid,
                       c->n_books);
    if (!(off[0] == WARP_HDR_BYTES && off[0] < off[1] && off[1] < off[2] && off[2] < off[3] &&
          off[3] <= g->rec_bytes))
        return set_err(c, WARP_HIP_E_HEADER, layer, expert, "record offsets out of order");
    const size_t scales = 2u * (2 * (size_t)g->inter + c->He);
    if (scales > g->rec_bytes - off[3])
        return set_err(c, WARP_HIP_E_HEADER, layer, expert, "record scales past its end");
    if (!((size_t)off[0] + c->gate_bytes <= off[1] && (size_t)off[1] + c->gate_bytes <= off[2] &&
          (size_t)off[2] + c->down_bytes <= off[3]))
        return set_err(c, WARP_HIP_E_HEADER, layer, expert, "record index blocks shorter than the shape");
    return 0;
}

/* A key whose resident record names codebooks other than its layer's. */
static int key_foreign(const warp_hip_ctx *c, int key)
{
    const layer_t *L = &c->L[key / c->cfg.n_experts];
    return c->key_slot[key] >= 0 && c->rec_cb[key] != (uint16_t)L->cb_base;
}

/* Any resident record of `layer` whose codebook_id is not the layer's. */
static int layer_foreign(const warp_hip_ctx *c, int layer)
{
    const int E = c->cfg.n_experts;
    if (c->L[layer].resident == 0) return 0;
    for (int e = 0; e < E; e++)
        if (key_foreign(c, layer * E + e)) return 1;
    return 0;
}

/* The codebooks the resident records `ids` of `layer` decode with. The
 * reference builds the gate/up tables from the first selected record's
 * codebook_id and each down table from the record's own (src/model.c:
 * 2886-2907, 3612-3653). When every record of the selection names the same
 * id, that is one set: the codebooks given to the layer whose cb_base it is
 * (normally `layer` itself). Mixed ids, an id no layer has codebooks for, or
 * a set that would change the kernel choice (exponent-31 values) give
 * E_BOOKS, and the caller's CPU path runs the layer. */
static const layer_t *books_by_id(const warp_hip_ctx *c, const layer_t *L, int cb)
{
    if (cb == L->cb_base) return L;
    for (int l = 0; l < c->cfg.n_layers; l++)
        if (c->L[l].has_books && c->L[l].cb_base == cb && c->L[l].books_x31 == L->books_x31) return &c->L[l];
    return NULL;
}

static int books_of(warp_hip_ctx *c, int layer, const int *ids, int n, const layer_t **B)
{
    const int E = c->cfg.n_experts;
    const layer_t *L = &c->L[layer];
    int cb = -1, bad = -1;
    for (int j = 0; j < n && bad < 0; j++) {
        if (ids[j] < 0 || ids[j] >= E || c->key_slot[layer * E + ids[j]] < 0) continue;
        const int id = c->rec_cb[layer * E + ids[j]];
        if (cb < 0) cb = id;
        else if (id != cb) bad = ids[j];
    }
    *B = L;
    if (bad < 0 && cb < 0) return 0;
    if (bad < 0 && (*B = books_by_id(c, L, cb)) != NULL) return 0;
    if (bad < 0) bad = ids[0];
    *B = L;
    return set_err(c, WARP_HIP_E_BOOKS, layer, bad, "selected records name codebook_id %u; layer codebook base %d",
                   c->rec_cb[layer * E + bad], L->cb_base);
}

static int is_pinned(const warp_hip_ctx *c, int key)
{
    const uint32_t h = c->pin_gen[key];
    return h != 0 && (h == c->hold || h == c->spec_hold);
}

static uint32_t new_hold(warp_hip_ctx *c)
{
    if (++c->hold_next == 0) ++c->hold_next;
    return c->hold_next;
}

/* A slot to fill, as the reference's ec_victim chooses one
 * (src/ecache.c:432-460): the lowest-numbered empty slot, else the
 * least-frequent (then least recently used) of 16 slots sampled with its
 * generator (rng * 1664525 + 1013904223, rng % n_slots, seeded 0x9e3779b9)
 * that no hold keeps, else the first such slot. A hold keeps the selection
 * in flight whole, where the reference, which multiplies one record at a
 * time, keeps only the record in use. */
static int pick_victim(warp_hip_ctx *c)
{
    if (c->n_empty > 0) {
        /* slots freed by a refused record, below the never-used ones */
        for (int s = 0; s < c->next_free; s++)
            if (c->slot_key[s] < 0) { c->n_empty--; return s; }
        c->n_empty = 0;
    }
    if (c->next_free < c->n_slots) return c->next_free++;
    int best = -1;
    for (int k = 0; k < 16; k++) {
        c->rng = c->rng * 1664525u + 1013904223u;
        const int s = (int)(c->rng % (unsigned)c->n_slots);
        if (c->slot_key[s] >= 0 && is_pinned(c, c->slot_key[s])) continue;
        if (best < 0 || c->hits[s] < c->hits[best] || (c->hits[s] == c->hits[best] && c->last[s] < c->last[best]))
            best = s;
    }
    if (best < 0)
        for (int s = 0; s < c->n_slots; s++)
            if (c->slot_key[s] < 0 || !is_pinned(c, c->slot_key[s])) { best = s; break; }
    return best;
}

/* Apply the queued table updates after everything queued on the copy
 * stream so far (the batch's copies). Kernels that read the table wait for
 * ev_copy (wait_copies). */
static int flush_table(warp_hip_ctx *c)
{
    if (!c->tq_n) return 0;
    const int i = c->tq_cur, n = c->tq_n;
    warp_slot_upd *u = c->tq_host[i];
    for (int q = 0; q < n; q++) c->tq_pos[u[q].key] = -1;
    c->tq_n = 0;
    c->tq_cur = (i + 1) % N_TQ;
    DEV(c, hipMemcpyAsync(c->tq_dev, u, (size_t)n * sizeof *u, hipMemcpyHostToDevice, c->cp));
    DEV(c, hipEventRecord(c->ev_tq[i], c->cp));
    c->tq_used[i] = 1;
    if (wk_set_slots(c->table_dev, c->tq_dev, n, c->crc_bad, c->crc_err, c->cp))
        return set_err(c, WARP_HIP_E_DEVICE, -1, -1, "table update");
    DEV(c, hipEventRecord(c->ev_copy, c->cp));
    c->copy_pending = 1;
    return 0;
}

/* Queue table[key] = {rec, off} for the batch's update launch; checked: the
 * record's device checksum decides whether the entry is taken. */
static int queue_slot(warp_hip_ctx *c, int key, const uint8_t *rec, const uint32_t off[4], int checked)
{
    int rc;
    if (c->tq_n == c->tq_cap && (rc = flush_table(c)) != 0) return rc;
    if (c->tq_n == 0 && c->tq_used[c->tq_cur]) {
        DEV(c, hipEventSynchronize(c->ev_tq[c->tq_cur]));   /* its previous list has been copied */
        c->tq_used[c->tq_cur] = 0;
    }
    warp_slot_upd *u = c->tq_host[c->tq_cur];
    int i = c->tq_pos[key];
    if (i < 0) {
        i = c->tq_n++;
        c->tq_pos[key] = i;
        u[i].key = key;
    }
    u[i].checked = checked;
    u[i].v.rec = rec;
    memcpy(u[i].v.off, off, sizeof u[i].v.off);
    return 0;
}

/* Assign (layer, expert) a slot, evicting if needed. Returns the slot or a
 * negative code. The caller fills it; the eviction reaches the device
 * table with the batch's updates. */
static int claim_slot(warp_hip_ctx *c, int layer, int expert)
{
    const int E = c->cfg.n_experts, key = layer * E + expert;
    if (c->n_slots <= 0) return set_err(c, WARP_HIP_E_NOSLOT, layer, expert, "no cache slots");
    const int s = pick_victim(c);
    if (s < 0) return set_err(c, WARP_HIP_E_NOSLOT, layer, expert, "every sampled slot is in use");
    const int old = c->slot_key[s];
    if (old >= 0) {
        c->key_slot[old] = -1;
        c->L[old / E].resident--;
        c->stats.evictions++;
        static const uint32_t none[4] = { 0, 0, 0, 0 };
        int rc = queue_slot(c, old, NULL, none, 0);
        if (rc) return rc;
    }
    c->slot_key[s] = key;
    c->key_slot[key] = s;
    c->hits[s] = 1;                 /* a claim counts as a use (src/ecache.c:489,508) */
    c->last[s] = ++c->clock;
    c->L[layer].resident++;
    return s;
}

/* A slot's claim undone: the device refused its record. */
static void unclaim(warp_hip_ctx *c, int key)
{
    const int s = c->key_slot[key];
    if (s < 0) return;
    c->key_slot[key] = -1;
    c->slot_key[s] = -1;
    c->hits[s] = 0;
    c->n_empty++;
    c->L[key / c->cfg.n_experts].resident--;
}

/* hdr: a host copy of the record's (checked) header; the record is in slot
 * s, or on its way there on the copy stream. With cfg.verify the payload's
 * crc32 is taken on the device next (record_check's checksum,
 * src/model.c:1742-1744), after the copy, and the batch's table update
 * refuses a record whose checksum differs from its header's; the host
 * learns of it at crc_report. The entry reaches the device with the batch's
 * flush_table. */
static int publish_slot(warp_hip_ctx *c, int layer, int expert, int s, const uint8_t *hdr)
{
    uint32_t off[4];
    memcpy(off, hdr + WARP_HDR_GATE_OFF, sizeof off);
    const int key = layer * c->cfg.n_experts + expert;
    memcpy(&c->rec_cb[key], hdr + 10, sizeof c->rec_cb[key]);
    const uint8_t *slot = slot_rec(c, s);
    if (c->cfg.verify) {
        const size_t scales = 2u * (2 * (size_t)c->cfg.inter + c->He);
        KRN(c, wk_crc32(slot + WARP_HDR_BYTES, (size_t)off[3] + scales - WARP_HDR_BYTES, c->crc_tmp, NULL,
                        (const uint32_t *)(slot + WARP_HDR_CRC_OFF), key, c->crc_bad, c->cp));
        c->crc_pending = 1;
    }
    return queue_slot(c, key, slot, off, c->cfg.verify);
}

/* Waits for the copy stream and reports the records whose device checksum
 * failed since the last report: their slots are freed and the call fails
 * with E_CRC naming the first of them. Updates still queued are applied
 * first, so every checked fill has had its verdict. The device lists the
 * first WARP_CRC_ERR_KEYS refused keys; past that, the per-key verdicts
 * (crc_bad: 1 exactly where a key's last table update was a refusal) are
 * read back whole, so no refused key stays claimed on the host. */
static int crc_report(warp_hip_ctx *c)
{
    if (!c->crc_pending) return 0;
    int rc = flush_table(c);
    if (rc) return rc;
    DEV(c, hipMemcpyAsync(c->h_crc_err, c->crc_err, sizeof *c->h_crc_err, hipMemcpyDeviceToHost, c->cp));
    DEV(c, hipStreamSynchronize(c->cp));
    c->crc_pending = 0;
    const int n = c->h_crc_err->n;
    if (n == 0) return 0;
    int first = c->h_crc_err->keys[0];
    if (n <= WARP_CRC_ERR_KEYS) {
        for (int i = 0; i < n; i++) unclaim(c, c->h_crc_err->keys[i]);
    } else {
        const size_t nkeys = (size_t)c->cfg.n_layers * c->cfg.n_experts;
        int8_t *bad = (int8_t *)malloc(nkeys);
        if (!bad) return set_err(c, WARP_HIP_E_NOMEM, -1, -1, "host allocation failed");
        hipError_t e = hipMemcpy(bad, c->crc_bad, nkeys, hipMemcpyDeviceToHost);
        if (e != hipSuccess) { free(bad); return dev_err(c, "crc verdicts", e); }
        for (size_t k = 0; k < nkeys; k++)
            if (bad[k] && c->key_slot[k] >= 0) unclaim(c, (int)k);
        free(bad);
    }
    DEV(c, hipMemsetAsync(c->crc_err, 0, sizeof c->crc_err->n, c->cp));
    DEV(c, hipStreamSynchronize(c->cp));
    const int E = c->cfg.n_experts;
    return set_err(c, WARP_HIP_E_CRC, first / E, first % E, "record payload checksum (%d record%s refused)", n,
                   n > 1 ? "s" : "");
}

int warp_hip_put_expert(warp_hip_ctx *c, int layer, int expert, const uint8_t *rec)
{
    int rc = check_layer(c, layer);
    if (rc) return rc;
    if (expert < 0 || expert >= c->cfg.n_experts || !rec)
        return set_err(c, WARP_HIP_E_ARG, layer, expert, "expert id");
    if ((rc = check_record(c, rec, layer, expert))) return rc;
    const int key = layer * c->cfg.n_experts + expert;
    /* the eviction's table update and the overwrite wait for everything
     * already queued on the compute stream, which may still read the
     * slot's previous record */
    DEV(c, hipEventRecord(c->ev_before, c->st));
    DEV(c, hipStreamWaitEvent(c->cp, c->ev_before, 0));
    int s = c->key_slot[key];
    if (s < 0 && (s = claim_slot(c, layer, expert)) < 0) return s;
    DEV(c, hipMemcpyAsync(slot_rec(c, s), rec, c->cfg.rec_bytes, hipMemcpyHostToDevice, c->cp));
    DEV(c, hipStreamSynchronize(c->cp));
    if ((rc = publish_slot(c, layer, expert, s, rec)) || (rc = flush_table(c))) return rc;
    return crc_report(c);
}

int warp_hip_put_expert_dev(warp_hip_ctx *c, int layer, int expert, const uint8_t *rec_dev)
{
    int rc = check_layer(c, layer);
    if (rc) return rc;
    if (expert < 0 || expert >= c->cfg.n_experts || !rec_dev)
        return set_err(c, WARP_HIP_E_ARG, layer, expert, "expert id");
    /* the header is checked on a host copy of its first bytes before any
     * slot is touched: a refused record leaves the cache as it was (a
     * record already resident for the key stays resident) */
    uint8_t hdr[WARP_HDR_BYTES];
    DEV(c, hipMemcpy(hdr, rec_dev, sizeof hdr, hipMemcpyDeviceToHost));
    if ((rc = check_record(c, hdr, layer, expert))) return rc;
    const int key = layer * c->cfg.n_experts + expert;
    DEV(c, hipEventRecord(c->ev_before, c->st));
    DEV(c, hipStreamWaitEvent(c->cp, c->ev_before, 0));
    int s = c->key_slot[key];
    if (s < 0 && (s = claim_slot(c, layer, expert)) < 0) return s;
    DEV(c, hipMemcpyAsync(slot_rec(c, s), rec_dev, c->cfg.rec_bytes,
                          hipMemcpyDeviceToDevice, c->cp));
    DEV(c, hipStreamSynchronize(c->cp));
    if ((rc = publish_slot(c, layer, expert, s, hdr)) || (rc = flush_table(c))) return rc;
    return crc_report(c);
}

int warp_hip_put_expert_synth(warp_hip_ctx *c, int layer, int expert, uint64_t seed, const uint16_t *scales)
{
    int rc = check_layer(c, layer);
    if (rc) return rc;
    const warp_hip_cfg *g = &c->cfg;
    if (expert < 0 || expert >= g->n_experts || !scales) return set_err(c, WARP_HIP_E_ARG, layer, expert, "expert id");
    /* header of waste_expert_hdr (src/waste_format.h:98-130) for this shape */
    uint8_t hdr[WARP_HDR_BYTES];
    memset(hdr, 0, sizeof hdr);
    const uint32_t magic = 0x50584557u, blocks = (uint32_t)(g->rec_bytes / 4096u);
    const uint16_t lay = (uint16_t)layer, eid = (uint16_t)expert, cb = (uint16_t)c->L[layer].cb_base;
    const uint8_t fmt = (uint8_t)g->fmt;
    uint32_t off[4];
    off[0] = WARP_HDR_BYTES;
    off[1] = off[0] + (uint32_t)c->gate_bytes;
    off[2] = off[1] + (uint32_t)c->gate_bytes;
    off[3] = off[2] + (uint32_t)c->down_bytes;
    memcpy(hdr, &magic, 4);
    memcpy(hdr + 4, &lay, 2);
    memcpy(hdr + 6, &eid, 2);
    memcpy(hdr + 8, &fmt, 1);
    memcpy(hdr + 10, &cb, 2);
    memcpy(hdr + 16, &blocks, 4);
    memcpy(hdr + 20, off, 16);
    if ((rc = check_record(c, hdr, layer, expert))) return rc;
    const int key = layer * g->n_experts + expert;
    DEV(c, hipEventRecord(c->ev_before, c->st));
    DEV(c, hipStreamWaitEvent(c->cp, c->ev_before, 0));
    int s = c->key_slot[key];
    if (s < 0 && (s = claim_slot(c, layer, expert)) < 0) return s;
    uint8_t *slot = slot_rec(c, s);
    KRN(c, wk_fill_random(slot, g->rec_bytes, seed, c->cp));
    DEV(c, hipMemcpyAsync(slot, hdr, sizeof hdr, hipMemcpyHostToDevice, c->cp));
    DEV(c, hipMemcpyAsync(slot + off[3], scales, 2 * (2 * (size_t)g->inter + c->He), hipMemcpyHostToDevice, c->cp));
    DEV(c, hipStreamSynchronize(c->cp));
    /* a synthetic record carries no checksum: never verified */
    c->rec_cb[key] = cb;
    if ((rc = queue_slot(c, key, slot, off, 0))) return rc;
    return flush_table(c);
}

const uint8_t *warp_hip_resident(warp_hip_ctx *c, int layer, int expert)
{
    if (!c || layer < 0 || layer >= c->cfg.n_layers || expert < 0 || expert >= c->cfg.n_experts) return NULL;
    const int s = c->key_slot[layer * c->cfg.n_experts + expert];
    return s < 0 ? NULL : slot_rec(c, s);
}

int warp_hip_set_fetch(warp_hip_ctx *c, warp_hip_fetch_fn fetch, void *user)
{
    if (!c) return WARP_HIP_E_ARG;
    c->fetch = fetch;
    c->fetch_user = user;
    if (fetch) c->fetch_host = NULL;
    return 0;
}

int warp_hip_set_fetch_host(warp_hip_ctx *c, warp_hip_fetch_host_fn fetch, void *user)
{
    if (!c) return WARP_HIP_E_ARG;
    c->fetch_host = fetch;
    c->fetch_host_user = user;
    if (fetch) c->fetch = NULL;
    return 0;
}

void *warp_hip_host_alloc(warp_hip_ctx *c, size_t bytes)
{
    void *p = NULL;
    if (!c || !bytes) return NULL;
    if (hipSetDevice(c->cfg.device) != hipSuccess || hipHostMalloc(&p, bytes, 0) != hipSuccess) {
        set_err(c, WARP_HIP_E_NOMEM, -1, -1, "pinned host allocation of %zu bytes", bytes);
        return NULL;
    }
    return p;
}

void warp_hip_host_free(warp_hip_ctx *c, void *p)
{
    (void)c;
    if (p) (void)hipHostFree(p);
}

static int can_fetch(const warp_hip_ctx *c) { return c->fetch != NULL || c->fetch_host != NULL; }

void warp_hip_get_cache_stats(const warp_hip_ctx *c, warp_hip_cache_stats *st)
{
    if (!c || !st) return;
    *st = c->stats;
    st->n_slots = c->n_slots;
    int r = 0;
    for (int l = 0; l < c->cfg.n_layers; l++) r += c->L[l].resident;
    st->resident = r;
}

int warp_hip_get_route_stats(warp_hip_ctx *c, warp_hip_route_stats *st)
{
    if (!c || !st) return WARP_HIP_E_ARG;
    unsigned long long d[2];
    DEV(c, hipStreamSynchronize(c->st));
    DEV(c, hipMemcpy(d, c->cert_ctr, sizeof d, hipMemcpyDeviceToHost));
    *st = c->route_stats;
    st->recomputed = d[0];
    st->rows = d[1];
    return 0;
}

/* Fetch (layer, expert) through the caller's fetch function into a pinned
 * staging buffer (or find it in the caller's pinned memory), check it, and
 * copy it into a slot on the copy stream. The caller orders the copy stream
 * after the compute that may still read the victim, and ends the batch
 * with flush_table. */
static int fill_from_fetch(warp_hip_ctx *c, int layer, int expert)
{
    if (!can_fetch(c))
        return set_err(c, WARP_HIP_E_MISSING, layer, expert, "expert not resident and no fetch function");
    if (c->fetch_host) {
        /* the record is copied from where the caller keeps it (pinned host
         * memory from warp_hip_host_alloc), no staging copy */
        const uint8_t *src = c->fetch_host(c->fetch_host_user, layer, expert);
        if (!src) return set_err(c, WARP_HIP_E_READ, layer, expert, "fetch failed");
        int rc = check_record(c, src, layer, expert);
        if (rc) return rc;
        const int s = claim_slot(c, layer, expert);
        if (s < 0) return s;
        DEV(c, hipMemcpyAsync(slot_rec(c, s), src, c->cfg.rec_bytes, hipMemcpyHostToDevice,
                              c->cp));
        c->stats.bytes_read += c->cfg.rec_bytes;
        return publish_slot(c, layer, expert, s, src);
    }
    const int i = c->stage_next;
    c->stage_next = (c->stage_next + 1) % N_STAGE;
    if (c->stage_used[i]) DEV(c, hipEventSynchronize(c->ev_stage[i]));
    uint8_t *dst = c->staging + (size_t)i * c->cfg.rec_bytes;
    if (c->fetch(c->fetch_user, layer, expert, dst) != 0)
        return set_err(c, WARP_HIP_E_READ, layer, expert, "fetch failed");
    int rc = check_record(c, dst, layer, expert);
    if (rc) return rc;
    const int s = claim_slot(c, layer, expert);
    if (s < 0) return s;
    DEV(c, hipMemcpyAsync(slot_rec(c, s), dst, c->cfg.rec_bytes, hipMemcpyHostToDevice, c->cp));
    DEV(c, hipEventRecord(c->ev_stage[i], c->cp));
    c->stage_used[i] = 1;
    c->stats.bytes_read += c->cfg.rec_bytes;
    return publish_slot(c, layer, expert, s, dst);
}

/* Speculative fills of `ids` in order, until the cache has no slot left
 * that no hold keeps. With `hold`, every id is kept under spec_hold: the
 * resident ones first, so that no fill of this batch evicts another record
 * the batch asks for. */
static int prefetch_after(warp_hip_ctx *c, int layer, const int *ids, int n, hipEvent_t after, int hold)
{
    const int E = c->cfg.n_experts;
    int rc = 0;
    if (n <= 0) return 0;
    if (hold)
        for (int i = 0; i < n; i++)
            if (ids[i] >= 0 && ids[i] < E && c->key_slot[layer * E + ids[i]] >= 0)
                c->pin_gen[layer * E + ids[i]] = c->spec_hold;
    /* every eviction and copy of the batch waits for `after` */
    if (after) DEV(c, hipStreamWaitEvent(c->cp, after, 0));
    for (int i = 0; i < n; i++) {
        if (ids[i] < 0 || ids[i] >= E) continue;
        if (c->key_slot[layer * E + ids[i]] >= 0) continue;
        /* a guess: not a miss, and never allowed to stall on a full cache */
        if ((rc = fill_from_fetch(c, layer, ids[i])) != 0) {
            if (rc == WARP_HIP_E_NOSLOT) rc = 0;
            break;
        }
        if (hold) c->pin_gen[layer * E + ids[i]] = c->spec_hold;
        c->stats.spec_issued++;
    }
    const int f = flush_table(c);
    return rc ? rc : f;
}

int warp_hip_prefetch(warp_hip_ctx *c, int layer, const int *ids, int n)
{
    int rc = check_layer(c, layer);
    if (rc) return rc;
    /* everything queued so far may still read the slots it would evict */
    DEV(c, hipEventRecord(c->ev_after, c->st));
    return prefetch_after(c, layer, ids, n, c->ev_after, 0);
}

/* Demand residency for `n` experts of `layer`, all pinned against eviction
 * until the next layer pins its own. Hits and misses are counted per record
 * asked for, as waste_ecache_get counts them (src/ecache.c:596-669). */
static int ensure_selected(warp_hip_ctx *c, int layer, const int *ids, int n)
{
    const int E = c->cfg.n_experts;
    for (int j = 0; j < n; j++)
        if (ids[j] < 0 || ids[j] >= E) return set_err(c, WARP_HIP_E_ARG, layer, ids[j], "expert id from the router");
    /* this selection is held until the next one; the lookahead's guesses
     * are now either in it or wrong */
    c->pin_layer = layer;
    c->hold = new_hold(c);
    c->spec_hold = 0;
    for (int j = 0; j < n; j++) c->pin_gen[layer * E + ids[j]] = c->hold;
    for (int j = 0; j < n; j++) {
        const int e = ids[j];
        const int s = c->key_slot[layer * E + e];
        if (s >= 0) {
            c->stats.hits++;
            c->hits[s]++;
            c->last[s] = ++c->clock;
            continue;
        }
        c->stats.misses++;
        int rc = fill_from_fetch(c, layer, e);
        if (rc) {
            (void)flush_table(c);      /* what was placed before the failure */
            return rc;
        }
    }
    int rc = flush_table(c);
    /* records the device checksum refused are reported before any kernel
     * reads the table */
    return rc ? rc : crc_report(c);
}

/* A layer that selects without the host (all resident, or nothing to
 * fetch with) ends its own earlier hold. */
static void release_hold(warp_hip_ctx *c, int layer)
{
    if (c->pin_layer == layer) {
        c->pin_layer = -1;
        c->hold = 0;
    }
}

static int wait_copies(warp_hip_ctx *c)
{
    if (c->copy_pending) {
        DEV(c, hipStreamWaitEvent(c->st, c->ev_copy, 0));
        c->copy_pending = 0;
    }
    return 0;
}

/* ---- launch timing ---------------------------------------------------------------------------- */

static int timing_fold(warp_hip_ctx *c)
{
    for (int i = 0; i < c->tev_n; i++) {
        float ms = 0.0f;
        DEV(c, hipEventSynchronize(c->tev[2 * i + 1]));
        DEV(c, hipEventElapsedTime(&ms, c->tev[2 * i], c->tev[2 * i + 1]));
        c->t_ms[c->tev_cls[i]] += ms;
        c->t_cnt[c->tev_cls[i]]++;
    }
    c->tev_n = 0;
    return 0;
}

/* Bracket one launch of class `cls` with events on the compute stream. */
static int timing_begin(warp_hip_ctx *c, int cls)
{
    if (!c->timing) return 0;
    if (c->tev_n == WARP_TIMING_N) {
        int rc = timing_fold(c);
        if (rc) return rc;
    }
    c->tev_cls[c->tev_n] = cls;
    DEV(c, hipEventRecord(c->tev[2 * c->tev_n], c->st));
    return 0;
}

static int timing_end(warp_hip_ctx *c)
{
    if (!c->timing) return 0;
    DEV(c, hipEventRecord(c->tev[2 * c->tev_n + 1], c->st));
    c->tev_n++;
    return 0;
}

int warp_hip_set_matvec_path(warp_hip_ctx *c, int path)
{
    if (!c || (path != WARP_HIP_PATH_AUTO && path != WARP_HIP_PATH_MFMA && path != WARP_HIP_PATH_LUT_FUSED &&
               path != WARP_HIP_PATH_GATHER))
        return WARP_HIP_E_ARG;
    c->mv_path = path;
    return 0;
}

int warp_hip_set_router_fast(warp_hip_ctx *c, int fast)
{
    if (!c) return WARP_HIP_E_ARG;
    c->cfg.router_fast = fast != 0;
    return 0;
}

int warp_hip_set_cert_polls(warp_hip_ctx *c, unsigned polls)
{
    if (!c) return WARP_HIP_E_ARG;
    c->cert_polls = polls;
    return 0;
}

int warp_hip_set_timing(warp_hip_ctx *c, int on)
{
    if (!c) return WARP_HIP_E_ARG;
    if (on && !c->tev) {
        c->tev = (hipEvent_t *)calloc(2 * WARP_TIMING_N, sizeof(hipEvent_t));
        if (!c->tev) return set_err(c, WARP_HIP_E_NOMEM, -1, -1, "host allocation failed");
        for (int i = 0; i < 2 * WARP_TIMING_N; i++) DEV(c, hipEventCreate(&c->tev[i]));
    }
    c->timing = on;
    c->tev_n = 0;
    memset(c->t_ms, 0, sizeof c->t_ms);
    memset(c->t_cnt, 0, sizeof c->t_cnt);
    return 0;
}

int warp_hip_get_timing(warp_hip_ctx *c, double ms[4], uint64_t launches[4])
{
    if (!c) return WARP_HIP_E_ARG;
    int rc = timing_fold(c);
    if (rc) return rc;
    for (int k = 0; k < WARP_TIMING_CLS; k++) {
        if (ms) ms[k] = c->t_ms[k];
        if (launches) launches[k] = c->t_cnt[k];
    }
    return 0;
}

/* ---- the layer ------------------------------------------------------------------------------ */

static const uint16_t *books_kind(const warp_hip_ctx *c, const layer_t *L, int kind)
{
    return L->books + (size_t)kind * c->S * c->En * 8;
}

static int logits_of(warp_hip_ctx *c, const layer_t *L, const float *x, int T, float *logits, hipStream_t s)
{
    const warp_hip_cfg *g = &c->cfg;
    if (L->router)
        return wk_router_logits(L->router, x, g->n_experts, g->hidden, T, g->router_strict, logits, s);
    if (L->rq)
        return wk_mvq(L->rq, L->rs, L->r_rowbytes, L->r_group, L->r_bits, x, g->n_experts, g->hidden, T, logits, s);
    return -1;
}

/* Whether a decode of this layer certifies its selection: sigmoid scores
 * from an fp32 router, neither strict logits (router_strict 1) nor plain
 * fast ones asked for, a shape the certifying kernels take. */
static int cert_ok(const warp_hip_ctx *c, const layer_t *L)
{
    const warp_hip_cfg *g = &c->cfg;
    return L->router && g->router_strict != 1 && !g->router_fast && g->router_act == WARP_HIP_ROUTE_SIGMOID &&
           g->hidden % 4 == 0 && g->hidden <= 16384 && g->n_experts <= 4096;
}

/* The layer's shared expert as the fused decode kernels take it: an fp32
 * router with the fast (tree) sum or the certifying one, the hidden state
 * in shh. */
static int shared_args(const warp_hip_ctx *c, const layer_t *L, warp_shared_args *sa)
{
    const warp_hip_cfg *g = &c->cfg;
    memset(sa, 0, sizeof *sa);
    if (!L->sq[0] || !L->router || (g->router_strict && !cert_ok(c, L)) || !c->shh) return 0;
    for (int k = 0; k < 3; k++) {
        sa->q[k] = L->sq[k];
        sa->s[k] = L->ss[k];
        sa->rowbytes[k] = L->s_rowbytes[k];
    }
    sa->bits = L->s_bits;
    sa->group = L->s_group;
    sa->inter = L->s_inter;
    sa->situ = g->act_situ;
    sa->beta = g->situ_beta;
    sa->lbeta = g->situ_linear_beta;
    sa->h = c->shh;
    return 1;
}

/* The shared expert of T tokens into sho, on stream s; it touches only the
 * shared expert's own scratch (sh*), so it may run beside the routed
 * experts. */
static int shared_ffn(warp_hip_ctx *c, const layer_t *L, const float *x, int T, hipStream_t s)
{
    const warp_hip_cfg *g = &c->cfg;
    const int H = g->hidden, Is = L->s_inter;
    /* a batch: on the matrix cores, x and h split into fp16 halves */
    if (T >= 8 && L->s_bits != 3 && L->s_small && L->s_group % 32 == 0 && H % L->s_group == 0 &&
        Is % L->s_group == 0) {
        const int8_t *wq[2] = {L->sq[0], L->sq[1]};
        const uint16_t *wsc[2] = {L->ss[0], L->ss[1]};
        float *gu[2] = {c->shg, c->shu};
        KRN(c, wk_split(x, T, H, c->shxin, c->shxinscale, s));
        /* gate and up in one launch: they share x */
        KRN(c, wk_mvq_gemm(2, wq, wsc, L->s_rowbytes, L->s_group, L->s_bits, c->shxin, c->shxinscale, Is, H, T, gu,
                           s));
        KRN(c, wk_act_split(c->shg, c->shu, T, Is, g->act_situ, g->situ_beta, g->situ_linear_beta, c->shxs,
                            c->shxscale, NULL, s));
        const int8_t *dq = L->sq[2];
        const uint16_t *dsc = L->ss[2];
        float *dy = c->sho;
        KRN(c, wk_mvq_gemm(1, &dq, &dsc, &L->s_rowbytes[2], L->s_group, L->s_bits, c->shxs, c->shxscale, H, Is, T,
                           &dy, s));
        return 0;
    }
    KRN(c, wk_mvq(L->sq[0], L->ss[0], L->s_rowbytes[0], L->s_group, L->s_bits, x, Is, H, T, c->shg, s));
    KRN(c, wk_mvq(L->sq[1], L->ss[1], L->s_rowbytes[1], L->s_group, L->s_bits, x, Is, H, T, c->shu, s));
    KRN(c, wk_act(c->shg, c->shu, T, Is, g->act_situ, g->situ_beta, g->situ_linear_beta, c->shh, s));
    KRN(c, wk_mvq(L->sq[2], L->ss[2], L->s_rowbytes[2], L->s_group, L->s_bits, c->shh, H, Is, T, c->sho, s));
    return 0;
}

/* The next layer's router on this layer's input, each of T tokens' top n
 * by sigmoid + bias (predict_next_moe, src/model.c:2680-2711), on the
 * lookahead stream while this layer computes. */
static int lookahead_launch(warp_hip_ctx *c, int layer, const float *x_dev, int T)
{
    const warp_hip_cfg *g = &c->cfg;
    if (!g->lookahead || !can_fetch(c) || layer + 1 >= g->n_layers) return 0;
    const layer_t *N = &c->L[layer + 1];
    if (!N->router && !N->rq) return 0;
    if (N->resident == g->n_experts) return 0;
    const int n = g->lookahead < g->n_experts ? (g->lookahead < WARP_MAX_K ? g->lookahead : WARP_MAX_K) : g->n_experts;
    DEV(c, hipEventRecord(c->ev_x, c->st));
    DEV(c, hipStreamWaitEvent(c->la, c->ev_x, 0));
    KRN(c, logits_of(c, N, x_dev, T, c->la_logits, c->la));
    KRN(c, wk_route(c->la_logits, N->bias, g->n_experts, n, T, WARP_HIP_ROUTE_SIGMOID, 0, 1.0f, c->la_idx, c->la_w,
                    NULL, NULL, NULL, NULL, 0, c->la));
    DEV(c, hipMemcpyAsync(c->h_la_idx, c->la_idx, (size_t)T * n * sizeof(int), hipMemcpyDeviceToHost, c->la));
    DEV(c, hipEventRecord(c->ev_la, c->la));
    c->la_T = T;
    return n;
}

/* The guesses are fetched once this layer's own work is queued (as
 * src/model.c:2922-2931 issues them last) and held until the next layer
 * selects. One token's go in rank order; a batch's are each expert once,
 * the most-predicted first, ties by id. When this layer's selection is held
 * (it went through the host), the fills need only wait for the work queued
 * before this layer's expert kernels, and so overlap them; otherwise they
 * wait for the whole layer. */
static int lookahead_issue(warp_hip_ctx *c, int layer, int n)
{
    if (n <= 0) return 0;
    DEV(c, hipEventSynchronize(c->ev_la));
    const int E = c->cfg.n_experts, T = c->la_T;
    const int *ids = c->h_la_idx;
    int m = n;
    if (T > 1) {
        int top = 0;
        memset(c->la_votes, 0, (size_t)E * sizeof(int));
        for (int q = 0; q < T * n; q++) {
            const int e = c->h_la_idx[q];
            if (e >= 0 && e < E && ++c->la_votes[e] > top) top = c->la_votes[e];
        }
        m = 0;
        for (int v = top; v >= 1; v--)
            for (int e = 0; e < E; e++)
                if (c->la_votes[e] == v) c->la_order[m++] = e;
        ids = c->la_order;
    }
    c->spec_hold = new_hold(c);
    return prefetch_after(c, layer + 1, ids, m, c->pin_layer == layer ? c->ev_before : c->ev_after, 1);
}

/* The latent MoE's tail (src/model.c:2913-2921, 2934-2939): the combined
 * expert outputs ylat [T][latent], RMS-normalised with routed_expert_norm,
 * projected up to H, plus the shared expert's output, plus the caller's
 * residual, in that order. */
static int latent_tail(warp_hip_ctx *c, const layer_t *L, int T, const float *resid, float *out)
{
    const warp_hip_cfg *g = &c->cfg;
    if (g->latent_norm) KRN(c, wk_rmsnorm(c->ylat, L->lnorm, T, c->He, g->norm_eps, c->ylat, c->st));
    KRN(c, wk_mvq(L->lq[1], L->ls[1], L->l_rowbytes[1], L->l_group, L->l_bits, c->ylat, g->hidden, c->He, T, c->yup,
                  c->st));
    KRN(c, wk_add3(c->yup, L->sq[0] ? c->sho : NULL, resid, (size_t)T * g->hidden, out, c->st));
    return 0;
}

/* Codebook values with exponent 31 are finite in the reference (its fp16
 * conversion rebiases every exponent, src/simd.h:49-67) but inf/NaN as the
 * fp16 operands of the matrix-core kernels: such a layer's expert matvecs
 * take the table kernel (its exact conversion) on every path. */
static int use_table(const warp_hip_ctx *c, const layer_t *L)
{
    return c->lut_ok && L->books && (c->mv_path != WARP_HIP_PATH_MFMA || L->books_x31);
}

/* The row kernel (decode-then-dot, whole rows per wave, the codebook in
 * LDS) instead of the table kernel, for `experts` experts of a decode:
 * where few rows share each position's tables, building them costs more
 * than gathering the rows' codebook vectors. */
static int use_gather(const warp_hip_ctx *c, const layer_t *L, int experts)
{
    if (!use_table(c, L) || L->books_x31 || c->He % 32 || c->cfg.inter % 32) return 0;
    /* its LDS: the kind's codebook when staged (2 x 4096 entries: 128 KiB)
     * and the input */
    const size_t in = (size_t)(c->He > c->cfg.inter ? c->He : c->cfg.inter) * sizeof(float);
    if ((c->cfg.fmt == WARP_HIP_VQ12 ? (size_t)131072 : 0) + in > 160 * 1024 - 1024) return 0;
    if (c->mv_path == WARP_HIP_PATH_GATHER) return 1;
    /* AUTO: one expert's matvecs (an expert FFN or one matrix: 1.3-1.8x the
     * table kernel at [1024 x 2304]); from two experts on, the tables are
     * shared by enough rows to pay for themselves */
    return c->mv_path == WARP_HIP_PATH_AUTO && experts == 1;
}

const char *warp_hip_matvec_kernel(warp_hip_ctx *c, int layer, int experts)
{
    if (!c || layer < 0 || layer >= c->cfg.n_layers) return "none";
    const layer_t *L = &c->L[layer];
    if (use_gather(c, L, experts)) return "k_vq_rows";
    if (use_table(c, L)) return c->mv_path == WARP_HIP_PATH_LUT_FUSED && experts > 1 ? "k_moe_fused" : "k_vq_lut";
    return c->P6 ? "k_apply_p6" : "k_vq_mfma";
}

/* E_ARG where such a layer's shapes rule the table kernel out. */
static int x31_check(warp_hip_ctx *c, const layer_t *L, int layer)
{
    if (L->books_x31 && !c->P6 && !c->lut_ok)
        return set_err(c, WARP_HIP_E_ARG, layer, -1,
                       "codebooks with exponent-31 values need the table kernel (widths multiples of 16)");
    return 0;
}

/* One token's routing from c->logits into idx / w, and with jobs = 1 the
 * job lists from the layer's table (ra->table); certified where ra says so. */
static int route_one(warp_hip_ctx *c, const warp_route_args *ra, int K, int jobs, hipStream_t s)
{
    const warp_hip_cfg *g = &c->cfg;
    if (ra->scored == 2) {
        warp_route_args r = *ra;
        if (!jobs) {
            r.cctr = NULL;                     /* counted on the call with the job lists */
            r.table = NULL;
            r.jobs = NULL;
            r.njobs = NULL;
            r.missing = NULL;
        }
        return wk_route_cert(&r, K, s);
    }
    return wk_route(ra->logits, ra->bias, ra->E, K, 1, g->router_act, g->renorm, g->routed_scale, ra->idx, ra->w,
                    jobs ? ra->table : NULL, jobs ? ra->jobs : NULL, jobs ? ra->njobs : NULL,
                    jobs ? ra->missing : NULL, ra->inter, s);
}

int warp_hip_moe_decode(warp_hip_ctx *c, int layer, const float *x_dev, float *out_dev, const float *resid_dev,
                        int *idx, float *w)
{
    int rc = check_layer(c, layer);
    if (rc) return rc;
    const warp_hip_cfg *g = &c->cfg;
    const layer_t *L = &c->L[layer];
    const int E = g->n_experts, K = g->top_k, H = g->hidden, I = g->inter;
    if (!L->has_books || (!L->router && !L->rq))
        return set_err(c, WARP_HIP_E_ARG, layer, -1, "layer %d has no codebooks or router", layer);
    const warp_slot *table = c->table_dev + (size_t)layer * E;
    if ((rc = x31_check(c, L, layer))) return rc;
    /* fills since the last report that the device refused leave the cache
     * now, before this layer reads the table */
    if (c->crc_pending && (rc = crc_report(c))) return rc;
    const int use_lut = use_table(c, L);
    /* the row kernel reads x in f32 and leaves its partial sums where the
     * table kernel does; it routes in a launch of its own */
    const int gat = use_gather(c, L, K);
    /* a resident record naming other codebooks than the layer's: the
     * selection goes through the host, which picks the codebooks */
    const int foreign = layer_foreign(c, layer);
    const layer_t *B = L;
    /* the latent MoE: the experts see xe = down . x and return into the
     * latent width He; routing and the shared expert stay on x */
    const int lat = g->latent > 0, He = c->He;
    if (lat && !L->lq[0]) return set_err(c, WARP_HIP_E_ARG, layer, -1, "layer %d has no latent projections", layer);
    const float *xe = x_dev;
    if (lat) {
        KRN(c, wk_mvq(L->lq[0], L->ls[0], L->l_rowbytes[0], L->l_group, L->l_bits, x_dev, He, H, 1, c->xlat, c->st));
        xe = c->xlat;
    }

    /* inputs for the gate/up matvecs, then the router */
    if (use_lut) {
        /* the table kernel reads x in f32 */
    } else if (c->P6) {
        const size_t nvH = (size_t)He / 8, nblkH = (nvH + WARP_LUT_BLK - 1) / WARP_LUT_BLK;
        KRN(c, wk_lut_p6(xe, 1, He, books_kind(c, L, 0), c->lut8, c->lscale, c->st));
        KRN(c, wk_lut_p6(xe, 1, He, books_kind(c, L, 1), c->lut8 + nvH * 256, c->lscale + nblkH, c->st));
    } else {
        KRN(c, wk_split(xe, 1, He, c->xs, c->xscale, c->st));
    }
    /* with the table kernel, a Q8G/Q4G shared expert runs inside the router
     * launch (gate, up, act) and the combine (down) */
    warp_shared_args sa;
    int fuse_shared = use_lut && !lat && shared_args(c, L, &sa) && wk_shared_fast_ok(H, &sa);
    /* sigmoid scores from an fp32 router: the selection is certified (the
     * router launch bounds every logit against the reference's sequential
     * sum, and its last block recomputes the rows those bounds leave
     * unordered), unless the caller asked for the plain fast logits or
     * strict ones. Where the device routes with the expert table and the
     * layer has no shared expert, that last block also routes (picks,
     * weights, job lists) */
    const int cert = cert_ok(c, L);
    const int cert_route = cert && !foreign && (L->resident == E || !can_fetch(c)) && !L->sq[0];
    /* else, where the device routes with the expert table, the table
     * kernel's gate/up launch does the routing itself (one launch less) */
    const int fuse_route = use_lut && !gat && !cert_route && !foreign && (L->resident == E || !can_fetch(c)) &&
                           wk_lut_route_ok(g->fmt, E, K, 1, 0, 2);
    /* and where that launch leaves CUs idle, one more row of its blocks
     * computes the shared expert's gate/up rows (one row per wave) instead
     * of the router launch, and blocks appended to the down launch its down
     * rows (four per wave) instead of the combine */
    int sh_in_gu = 0;
    if (fuse_shared && fuse_route) {
        int gr, sp;
        sh_in_gu = !wk_lut_plan(I, He, K, 2, 1, c->n_cu, c->part_cap, &gr, &sp) && 2 * gr * sp < c->n_cu &&
                   gr * sp * 16 >= sa.inter && (size_t)H * sizeof(float) <= 64 * 1024 &&
                   (size_t)sa.inter * sizeof(float) <= 64 * 1024 && sa.inter / (sa.bits == 8 ? 16 : 32) <= 256 &&
                   (H + 63) / 64 < c->n_cu / 2;
    }
    /* (the certifying router launch computes no shared expert) */
    if (cert && fuse_shared && !sh_in_gu) fuse_shared = 0;
    /* else, for sigmoid scores from an fp32 router, the router launch also
     * scores (one pass less in the routing prologue) */
    const int scored = fuse_route && (!fuse_shared || sh_in_gu) && L->router && !g->router_strict &&
                       g->router_act == WARP_HIP_ROUTE_SIGMOID;
    if (cert_route) KRN(c, wait_copies(c));       /* (the router's last block reads the expert table) */
    if ((rc = timing_begin(c, 2))) return rc;
    if (cert) {
        const warp_route_args pick = { NULL, NULL, table, E, g->router_act, g->renorm, I, g->routed_scale, c->idx,
                                       c->w, c->jobs, c->njobs, c->missing, 2, NULL, NULL, 0, NULL };
        KRN(c, wk_router_cert(L->router, x_dev, E, H, L->bias, c->logits, c->cert_sync, K, c->cert_ctr, c->missing,
                              cert_route ? &pick : NULL, c->cert_polls, c->st));
    }
    else if (fuse_shared && !sh_in_gu) KRN(c, wk_router_shared(L->router, x_dev, E, H, c->logits, &sa, c->st));
    else if (scored) KRN(c, wk_router_scored(L->router, x_dev, E, H, L->bias, c->logits, c->st));
    else KRN(c, logits_of(c, L, x_dev, 1, c->logits, c->st));
    if ((rc = timing_end(c))) return rc;
    if (cert) {
        c->route_stats.certified++;
        c->missing_pending = 1;            /* (the flag's bit 2 if the router's last block gave up) */
    }
    /* the routing's arguments: the table kernel's fused routing reads the
     * (certified) scores and biased scores, the routing launch all four
     * certified arrays; table and jobs are set where the job lists are
     * wanted */
    warp_route_args ra = { c->logits, L->bias, table, E, g->router_act, g->renorm, I, g->routed_scale,
                           c->idx, c->w, c->jobs, c->njobs, c->missing, cert ? (fuse_route ? 1 : 2) : scored,
                           L->router, x_dev, H, c->cert_ctr };
    const int n_la = lookahead_launch(c, layer, x_dev, 1);
    if (n_la < 0) return n_la;
    if (L->resident == E && !foreign) {
        /* everything resident: route and build the jobs on the device, no
         * host round trip */
        KRN(c, wait_copies(c));
        if (!fuse_route && !cert_route) KRN(c, route_one(c, &ra, K, 1, c->st));
        c->stats.hits += (uint64_t)K;
        release_hold(c, layer);
    } else if (!can_fetch(c) && !foreign) {
        /* nothing to fetch with: the device flags a selected expert that is
         * not resident (sticky), the combine poisons this layer's output with
         * NaN, and the next synchronising call reports E_MISSING */
        KRN(c, wait_copies(c));
        if (!fuse_route && !cert_route) KRN(c, route_one(c, &ra, K, 1, c->st));
        c->missing_pending = 1;
        release_hold(c, layer);
    } else {
        KRN(c, route_one(c, &ra, K, 0, c->st));
        DEV(c, hipMemcpyAsync(c->h_idx, c->idx, (size_t)K * sizeof(int), hipMemcpyDeviceToHost, c->st));
        DEV(c, hipStreamSynchronize(c->st));
        if ((rc = ensure_selected(c, layer, c->h_idx, K))) return rc;
        if ((rc = books_of(c, layer, c->h_idx, K, &B))) return rc;
        if (B != L && c->P6 && !use_lut) {
            /* the gate/up tables again, from the selection's codebooks */
            const size_t nvH = (size_t)He / 8, nblkH = (nvH + WARP_LUT_BLK - 1) / WARP_LUT_BLK;
            KRN(c, wk_lut_p6(xe, 1, He, books_kind(c, B, 0), c->lut8, c->lscale, c->st));
            KRN(c, wk_lut_p6(xe, 1, He, books_kind(c, B, 1), c->lut8 + nvH * 256, c->lscale + nblkH, c->st));
        }
        KRN(c, wait_copies(c));
        /* (the selection again, now with the job lists: the same picks) */
        KRN(c, route_one(c, &ra, K, 1, c->st));
    }
    DEV(c, hipEventRecord(c->ev_before, c->st));

    /* the weighted sum of the experts: into the latent width first on a
     * latent MoE, else straight into out with the shared expert and residual */
    const float *add0 = lat ? NULL : L->sq[0] && !fuse_shared ? c->sho : NULL, *add1 = lat ? NULL : resid_dev;
    float *ysum = lat ? c->ylat : out_dev;
    if (use_lut && fuse_route && !fuse_shared && c->mv_path == WARP_HIP_PATH_LUT_FUSED) {
        /* gate/up, down and the combine in one launch */
        if (L->sq[0] && (rc = shared_ffn(c, L, x_dev, 1, c->st))) return rc;
        if ((rc = timing_begin(c, 0))) return rc;
        KRN(c, wk_moe_fused(g->fmt, B->books, B->books_x31, xe, K, I, He, c->part, c->part_cap, c->n_cu,
                            g->act_situ, g->situ_beta, g->situ_linear_beta, &ra, add0, add1, ysum, c->fz_sync,
                            WARP_FZ_WORDS, c->st));
        if ((rc = timing_end(c))) return rc;
        c->missing_pending = 1;
        goto tail;
    }

    /* gate and up, activation, down */
    float *yk[3] = { c->yg, c->yu, c->yd };
    int sp_d = 0;
    size_t d_off = 0;
    if (gat && !B->books_x31) {
        /* the row kernel: the picks' gate and up rows (scaled), then their down
         * rows from act(gate, up), unscaled, as one split of partial sums for
         * the combine */
        float *ykr[3] = { c->yg, c->yu, NULL };
        if ((size_t)K * (((size_t)He + 63) / 64) * 64 > c->part_cap)
            return set_err(c, WARP_HIP_E_ARG, layer, -1, "partial-sum buffer");
        if ((rc = timing_begin(c, 0))) return rc;
        KRN(c, wk_vq_rows(g->fmt, c->jobs, c->njobs, K, 0, 2, B->books, xe, I, He, NULL, 0, 0, 0.0f, 0.0f, ykr, NULL,
                          NULL, c->n_cu, c->st));
        if ((rc = timing_end(c))) return rc;
        if ((rc = timing_begin(c, 1))) return rc;
        KRN(c, wk_vq_rows(g->fmt, c->jobs, c->njobs, K, 2, 1, B->books, NULL, He, I, NULL, 0, g->act_situ,
                          g->situ_beta, g->situ_linear_beta, ykr, c->part, NULL, c->n_cu, c->st));
        if ((rc = timing_end(c))) return rc;
        sp_d = 1;
        d_off = 0;
    } else if (use_lut) {
        int sp_gu = 0;
        if ((rc = timing_begin(c, 0))) return rc;
        KRN(c, wk_vq_lut(g->fmt, c->jobs, c->njobs, K, 0, 2, B->books, B->books_x31, xe, 1, c->part, c->part_cap, I, He,
                         c->n_cu, NULL, 0, 0, 0.0f, 0.0f, fuse_route ? &ra : NULL, sh_in_gu ? &sa : NULL, NULL, &sp_gu,
                         c->st));
        if ((rc = timing_end(c))) return rc;
        /* the down launch makes its inputs from the gate/up partials (SwiGLU
         * in its prologue); its partials go after the gate/up ones */
        const size_t gu_floats = (size_t)2 * sp_gu * K * (((size_t)I + 63) / 64) * 64;
        if ((rc = timing_begin(c, 1))) return rc;
        KRN(c, wk_vq_lut(g->fmt, c->jobs, c->njobs, K, 2, 1, B->books, B->books_x31, NULL, 0, c->part + gu_floats,
                         c->part_cap - gu_floats, He, I, c->n_cu, c->part, sp_gu, g->act_situ, g->situ_beta,
                         g->situ_linear_beta, NULL, sh_in_gu ? &sa : NULL, sh_in_gu ? c->sho : NULL, &sp_d,
                         c->st));
        d_off = gu_floats;
        if ((rc = timing_end(c))) return rc;
    } else if (c->P6) {
        const size_t nvH = (size_t)He / 8, nblkH = (nvH + WARP_LUT_BLK - 1) / WARP_LUT_BLK;
        KRN(c, wk_apply_p6(c->jobs, c->njobs, K, 0, c->lut8, c->lscale, c->yg, I, He, c->st));
        KRN(c, wk_apply_p6(c->jobs, c->njobs, K, 1, c->lut8 + nvH * 256, c->lscale + nblkH, c->yu, I, He, c->st));
        KRN(c, wk_act(c->yg, c->yu, K, I, g->act_situ, g->situ_beta, g->situ_linear_beta, c->hbuf, c->st));
        KRN(c, wk_lut_p6(c->hbuf, K, I, books_kind(c, B, 2), c->lut8d, c->lscaled, c->st));
        KRN(c, wk_apply_p6(c->jobs, c->njobs, K, 2, c->lut8d, c->lscaled, c->yd, He, I, c->st));
    } else {
        if ((rc = timing_begin(c, 0))) return rc;
        KRN(c, wk_vq_matvec(g->fmt, c->jobs, c->njobs, K, 0, 2, B->books, c->xs, c->xscale, yk, I, He, 1, c->st));
        if ((rc = timing_end(c))) return rc;
        KRN(c, wk_act_split(c->yg, c->yu, K, I, g->act_situ, g->situ_beta, g->situ_linear_beta, c->xsh, c->xscaleh,
                            NULL, c->st));
        if ((rc = timing_begin(c, 1))) return rc;
        KRN(c, wk_vq_matvec(g->fmt, c->jobs, c->njobs, K, 2, 1, B->books, c->xsh, c->xscaleh, yk, He, I, 1, c->st));
        if ((rc = timing_end(c))) return rc;
    }
    if (L->sq[0] && !fuse_shared && (rc = shared_ffn(c, L, x_dev, 1, c->st))) return rc;
    if (use_lut)
        KRN(c, wk_combine_lut(c->jobs + 2 * (size_t)K, c->part + d_off, sp_d, K, c->w, K, He,
                              sh_in_gu ? c->sho : add0, add1, c->missing, fuse_shared && !sh_in_gu ? &sa : NULL, ysum,
                              c->st));
    else
        KRN(c, wk_combine(c->yd, c->w, K, He, add0, add1, c->missing, ysum, c->st));
tail:
    if (lat && (rc = latent_tail(c, L, 1, resid_dev, out_dev))) return rc;
    DEV(c, hipEventRecord(c->ev_after, c->st));

    if ((rc = lookahead_issue(c, layer, n_la))) return rc;
    if (idx || w) {
        if (idx) DEV(c, hipMemcpyAsync(c->h_idx, c->idx, (size_t)K * sizeof(int), hipMemcpyDeviceToHost, c->st));
        if (w) DEV(c, hipMemcpyAsync(c->h_w, c->w, (size_t)K * sizeof(float), hipMemcpyDeviceToHost, c->st));
        DEV(c, hipStreamSynchronize(c->st));
        if ((rc = take_missing(c))) return rc;
        if (idx) memcpy(idx, c->h_idx, (size_t)K * sizeof(int));
        if (w) memcpy(w, c->h_w, (size_t)K * sizeof(float));
    }
    return 0;
}

int warp_hip_expert_ffn(warp_hip_ctx *c, int layer, int expert, const float *x_dev, float *out_dev)
{
    int rc = check_layer(c, layer);
    if (rc) return rc;
    const warp_hip_cfg *g = &c->cfg;
    const layer_t *L = &c->L[layer];
    const int H = c->He, I = g->inter; /* the expert's width: latent on a latent MoE */
    if (expert < 0 || expert >= g->n_experts || !x_dev || !out_dev)
        return set_err(c, WARP_HIP_E_ARG, layer, expert, "expert_ffn arguments");
    if (!L->has_books) return set_err(c, WARP_HIP_E_ARG, layer, -1, "layer %d has no codebooks", layer);
    if (c->key_slot[layer * g->n_experts + expert] < 0)
        return set_err(c, WARP_HIP_E_MISSING, layer, expert, "expert not resident");
    /* the record's own codebook_id names its codebooks (src/model.c:2889-2907) */
    const layer_t *B;
    if ((rc = books_of(c, layer, &expert, 1, &B))) return rc;
    /* the record's table entry may still be on its way (copy stream) */
    KRN(c, wait_copies(c));
    const warp_slot *entry = c->table_dev + (size_t)layer * g->n_experts + expert;
    c->missing_pending = 1;
    if ((rc = x31_check(c, B, layer))) return rc;
    if (use_gather(c, B, 1)) {
        /* two launches of the row kernel, from the expert's table entry (no
         * job-list launch): gate and up rows, then the down rows from
         * act(gate, up) straight into out (no combine launch); a missing
         * record sets the flag and out to NaN */
        float *yk[3] = { c->yg, c->yu, out_dev };
        if ((rc = timing_begin(c, 0))) return rc;
        KRN(c, wk_vq_rows(g->fmt, NULL, NULL, 1, 0, 2, B->books, x_dev, I, H, entry, I, 0, 0.0f, 0.0f, yk, NULL,
                          c->missing, c->n_cu, c->st));
        if ((rc = timing_end(c))) return rc;
        if ((rc = timing_begin(c, 1))) return rc;
        KRN(c, wk_vq_rows(g->fmt, NULL, NULL, 1, 2, 1, B->books, NULL, H, I, entry, I, g->act_situ, g->situ_beta,
                          g->situ_linear_beta, yk, NULL, c->missing, c->n_cu, c->st));
        if ((rc = timing_end(c))) return rc;
        return 0;
    }
    KRN(c, wk_expert_jobs(entry, I, c->jobs, c->njobs, c->w, c->missing, c->st));
    if (use_table(c, B)) {
        int sp_gu = 0, sp_d = 0;
        if ((rc = timing_begin(c, 0))) return rc;
        KRN(c, wk_vq_lut(g->fmt, c->jobs, c->njobs, 1, 0, 2, B->books, B->books_x31, x_dev, 1, c->part, c->part_cap,
                         I, H, c->n_cu, NULL, 0, 0, 0.0f, 0.0f, NULL, NULL, NULL, &sp_gu, c->st));
        if ((rc = timing_end(c))) return rc;
        const size_t gu_floats = (size_t)2 * sp_gu * (((size_t)I + 63) / 64) * 64;
        if ((rc = timing_begin(c, 1))) return rc;
        KRN(c, wk_vq_lut(g->fmt, c->jobs, c->njobs, 1, 2, 1, B->books, B->books_x31, NULL, 0, c->part + gu_floats,
                         c->part_cap - gu_floats, H, I, c->n_cu, c->part, sp_gu, g->act_situ, g->situ_beta,
                         g->situ_linear_beta, NULL, NULL, NULL, &sp_d, c->st));
        if ((rc = timing_end(c))) return rc;
        KRN(c, wk_combine_lut(c->jobs + 2, c->part + gu_floats, sp_d, 1, c->w, 1, H, NULL, NULL, c->missing, NULL,
                              out_dev, c->st));
        return 0;
    }
    float *yk[3] = { c->yg, c->yu, out_dev };
    if (c->P6) {
        const size_t nvH = (size_t)H / 8, nblkH = (nvH + WARP_LUT_BLK - 1) / WARP_LUT_BLK;
        KRN(c, wk_lut_p6(x_dev, 1, H, books_kind(c, B, 0), c->lut8, c->lscale, c->st));
        KRN(c, wk_lut_p6(x_dev, 1, H, books_kind(c, B, 1), c->lut8 + nvH * 256, c->lscale + nblkH, c->st));
        KRN(c, wk_apply_p6(c->jobs, c->njobs, 1, 0, c->lut8, c->lscale, c->yg, I, H, c->st));
        KRN(c, wk_apply_p6(c->jobs, c->njobs, 1, 1, c->lut8 + nvH * 256, c->lscale + nblkH, c->yu, I, H, c->st));
        KRN(c, wk_act(c->yg, c->yu, 1, I, g->act_situ, g->situ_beta, g->situ_linear_beta, c->hbuf, c->st));
        KRN(c, wk_lut_p6(c->hbuf, 1, I, books_kind(c, B, 2), c->lut8d, c->lscaled, c->st));
        KRN(c, wk_apply_p6(c->jobs, c->njobs, 1, 2, c->lut8d, c->lscaled, out_dev, H, I, c->st));
        return 0;
    }
    KRN(c, wk_split(x_dev, 1, H, c->xs, c->xscale, c->st));
    KRN(c, wk_vq_matvec(g->fmt, c->jobs, c->njobs, 1, 0, 2, B->books, c->xs, c->xscale, yk, I, H, 1, c->st));
    KRN(c, wk_act_split(c->yg, c->yu, 1, I, g->act_situ, g->situ_beta, g->situ_linear_beta, c->xsh, c->xscaleh, NULL,
                        c->st));
    KRN(c, wk_vq_matvec(g->fmt, c->jobs, c->njobs, 1, 2, 1, B->books, c->xsh, c->xscaleh, yk, H, I, 1, c->st));
    return 0;
}

int warp_hip_moe_decode_host(warp_hip_ctx *c, int layer, const float *x, float *out, int *routed)
{
    if (!c) return WARP_HIP_E_ARG;
    const int H = c->cfg.hidden;
    DEV(c, hipMemcpyAsync(c->xin, x, (size_t)H * 4, hipMemcpyHostToDevice, c->st));
    int rc = warp_hip_moe_decode(c, layer, c->xin, c->xout, NULL, routed, NULL);
    if (rc) return rc;
    DEV(c, hipMemcpyAsync(out, c->xout, (size_t)H * 4, hipMemcpyDeviceToHost, c->st));
    DEV(c, hipStreamSynchronize(c->st));
    return take_missing(c);
}

/* The routed experts of a chunk whose experts e_lo..e_hi (in the windowed
 * case, the window's) are resident and held: grouping, then the matvecs of
 * their pairs into the pair rows of yd. */
static int chunk_experts(warp_hip_ctx *c, int layer, const layer_t *B, const float *X_dev, int T, int e_lo, int e_hi,
                         int first)
{
    const warp_hip_cfg *g = &c->cfg;
    const int E = g->n_experts, K = g->top_k, H = c->He, I = g->inter, P = T * K; /* H: the experts' width */
    const warp_slot *table = c->table_dev + (size_t)layer * E;
    KRN(c, wait_copies(c));
    KRN(c, wk_plan_chunk(c->idx, c->w, T, K, E, table, c->counts, c->offsets, c->pair_tok, c->pair_exp, c->pair_w,
                         c->tok_slots, c->jobs, c->max_jobs, c->njobs, c->runs, c->missing, I, e_lo, e_hi, !first,
                         c->st));
    DEV(c, hipEventRecord(c->ev_before, c->st));
    float *yk[3] = { c->yg, c->yu, c->yd };
    if (c->P6) {
        const size_t nvH = (size_t)H / 8, nblkH = (nvH + WARP_LUT_BLK - 1) / WARP_LUT_BLK;
        if (first) {
            /* per token: gate LUT at [t][0], up LUT at [t][1] */
            KRN(c, wk_lut_p6(X_dev, T, H, books_kind(c, B, 0), c->lut8, c->lscale, c->st));
            KRN(c, wk_lut_p6(X_dev, T, H, books_kind(c, B, 1), c->lut8 + (size_t)T * nvH * 256,
                             c->lscale + (size_t)T * nblkH, c->st));
        }
        KRN(c, wk_apply_p6(c->jobs, c->njobs, c->max_jobs, 0, c->lut8, c->lscale, c->yg, I, H, c->st));
        KRN(c, wk_apply_p6(c->jobs, c->njobs, c->max_jobs, 1, c->lut8 + (size_t)T * nvH * 256,
                           c->lscale + (size_t)T * nblkH, c->yu, I, H, c->st));
        KRN(c, wk_act(c->yg, c->yu, P, I, g->act_situ, g->situ_beta, g->situ_linear_beta, c->hbuf, c->st));
        KRN(c, wk_lut_p6(c->hbuf, P, I, books_kind(c, B, 2), c->lut8d, c->lscaled, c->st));
        KRN(c, wk_apply_p6(c->jobs, c->njobs, c->max_jobs, 2, c->lut8d, c->lscaled, c->yd, H, I, c->st));
    } else {
        /* by runs: each expert's records decoded once per WARP_RUN_J jobs */
        if (prefill_fp16(c)) {
            /* reduced precision: inputs by pair slot, position-group-major
             * (x replicated per pair once the first plan has placed them) */
            if (first && H <= 4096)
                KRN(c, wk_split_pgm_pairs(X_dev, c->tok_slots, T, K, H, c->xsp, c->xscalep, c->st));
            else if (first)
                KRN(c, wk_split_pgm(X_dev, NULL, c->pair_tok, c->offsets + E, P, H, 0, 0, 0.0f, 0.0f, c->xsp,
                                    c->xscalep, c->st));
            KRN(c, wk_vq_runs(g->fmt, c->jobs, c->njobs, c->max_jobs, c->runs, 0, 2, B->books, c->xsp, c->xscalep,
                              yk, I, H, P, c->run_queue, c->st));
            KRN(c, wk_split_pgm(c->yg, c->yu, NULL, c->offsets + E, P, I, 1, g->act_situ, g->situ_beta,
                                g->situ_linear_beta, c->xsh, c->xscaleh, c->st));
            KRN(c, wk_vq_runs(g->fmt, c->jobs, c->njobs, c->max_jobs, c->runs, 2, 1, B->books, c->xsh, c->xscaleh,
                              yk, H, I, P, c->run_queue, c->st));
        } else {
            if (first) KRN(c, wk_split(X_dev, T, H, c->xs, c->xscale, c->st));
            KRN(c, wk_vq_runs(g->fmt, c->jobs, c->njobs, c->max_jobs, c->runs, 0, 2, B->books, c->xs, c->xscale, yk,
                              I, H, 0, c->run_queue, c->st));
            KRN(c, wk_act_split(c->yg, c->yu, P, I, g->act_situ, g->situ_beta, g->situ_linear_beta, c->xsh,
                                c->xscaleh, NULL, c->st));
            KRN(c, wk_vq_runs(g->fmt, c->jobs, c->njobs, c->max_jobs, c->runs, 2, 1, B->books, c->xsh, c->xscaleh,
                              yk, H, I, 0, c->run_queue, c->st));
        }
    }
    return 0;
}

int warp_hip_moe_chunk(warp_hip_ctx *c, int layer, const float *X_dev, float *out_dev, const float *resid_dev, int T,
                       int *route, float *rw)
{
    int rc = check_layer(c, layer);
    if (rc) return rc;
    const warp_hip_cfg *g = &c->cfg;
    const layer_t *L = &c->L[layer];
    const int E = g->n_experts, K = g->top_k, H = g->hidden;
    if (T < 1 || T > g->max_tokens) return set_err(c, WARP_HIP_E_ARG, layer, -1, "T = %d, max_tokens = %d", T, g->max_tokens);
    if (!L->has_books || (!L->router && !L->rq))
        return set_err(c, WARP_HIP_E_ARG, layer, -1, "layer %d has no codebooks or router", layer);
    const int P = T * K;
    const int lat = g->latent > 0;
    if (lat && !L->lq[0]) return set_err(c, WARP_HIP_E_ARG, layer, -1, "layer %d has no latent projections", layer);
    /* a missing pick an earlier decode left unreported: this chunk's plan
     * rewrites the device flag, so report it first */
    if (c->missing_pending && (rc = take_missing(c))) return rc;
    /* fills since the last report that the device refused leave the cache
     * now, before this chunk reads the table (a lookahead's claims raise
     * resident before their checksums are known) */
    if (c->crc_pending && (rc = crc_report(c))) return rc;
    const layer_t *B = L;
    const int foreign = layer_foreign(c, layer);
    if (L->books_x31 && !c->P6) {
        /* the chunk's matrix-core kernels cannot take exponent-31 codebook
         * values: the tokens go one at a time through the table kernel,
         * each with the chunk's routing (the same rule per token) */
        if ((rc = x31_check(c, L, layer))) return rc;
        for (int t = 0; t < T; t++) {
            rc = warp_hip_moe_decode(c, layer, X_dev + (size_t)t * H, out_dev + (size_t)t * H,
                                     resid_dev ? resid_dev + (size_t)t * H : NULL, route ? route + (size_t)t * K : NULL,
                                     rw ? rw + (size_t)t * K : NULL);
            if (rc) return rc;
        }
        DEV(c, hipStreamSynchronize(c->st));
        return take_missing(c);
    }
    /* the experts' inputs: x itself, or its latent projection */
    const float *Xe = X_dev;
    if (lat) {
        KRN(c, wk_mvq(L->lq[0], L->ls[0], L->l_rowbytes[0], L->l_group, L->l_bits, X_dev, c->He, H, T, c->xlat, c->st));
        Xe = c->xlat;
    }

    /* the shared expert on its own stream, beside routing, grouping and the
     * routed experts; the combine waits for it */
    if (L->sq[0]) {
        DEV(c, hipEventRecord(c->ev_sx0, c->st));
        DEV(c, hipStreamWaitEvent(c->sx, c->ev_sx0, 0));
        if ((rc = shared_ffn(c, L, X_dev, T, c->sx))) return rc;
        DEV(c, hipEventRecord(c->ev_sx1, c->sx));
        c->sx_pending = 1;
    }
    KRN(c, logits_of(c, L, X_dev, T, c->logits, c->st));
    KRN(c, wk_route(c->logits, L->bias, E, K, T, g->router_act, g->renorm, g->routed_scale, c->idx, c->w, NULL, NULL,
                    NULL, NULL, 0, c->st));
    const int n_la = lookahead_launch(c, layer, X_dev, T);
    if (n_la < 0) return n_la;
    if ((L->resident != E && can_fetch(c)) || foreign) {
        DEV(c, hipMemcpyAsync(c->h_idx, c->idx, (size_t)P * sizeof(int), hipMemcpyDeviceToHost, c->st));
        DEV(c, hipStreamSynchronize(c->st));
        /* each distinct record once, ascending (src/model.c:3595-3603) */
        int *ids = (int *)malloc((size_t)E * sizeof(int));
        if (!ids) return set_err(c, WARP_HIP_E_NOMEM, layer, -1, "host allocation failed");
        char *used = (char *)calloc((size_t)E, 1);
        if (!used) { free(ids); return set_err(c, WARP_HIP_E_NOMEM, layer, -1, "host allocation failed"); }
        for (int q = 0; q < P; q++)
            if (c->h_idx[q] >= 0 && c->h_idx[q] < E) used[c->h_idx[q]] = 1;
        int n = 0;
        for (int e = 0; e < E; e++) if (used[e]) ids[n++] = e;
        free(used);
        if (n == 0) {
            rc = chunk_experts(c, layer, B, Xe, T, 0, E - 1, 1);
        } else {
            /* Windows of distinct experts that the cache holds at once, in
             * ascending id: the reference streams a chunk's experts through
             * its cache the same way, whatever the cache size
             * (src/model.c:3595-3606). Each window is held while its
             * matvecs run; the next window's fills wait for them. Pairs are
             * independent, so the windows fill disjoint pair rows and the
             * combine below sees what one window would give, bit for bit. */
            const int win = c->n_slots < n ? c->n_slots : n;
            if (win < 1) rc = set_err(c, WARP_HIP_E_NOSLOT, layer, ids[0], "no cache slots");
            for (int a = 0; rc == 0 && a < n; a += win) {
                const int b = a + win < n ? a + win : n;
                if (a > 0) {
                    hipError_t e = hipEventRecord(c->ev_before, c->st);
                    if (e == hipSuccess) e = hipStreamWaitEvent(c->cp, c->ev_before, 0);
                    if (e != hipSuccess) { rc = dev_err(c, "window order", e); break; }
                }
                if ((rc = ensure_selected(c, layer, ids + a, b - a)) != 0) break;
                /* one codebook set for the whole chunk: the first window's */
                const layer_t *Bw;
                if ((rc = books_of(c, layer, ids + a, b - a, &Bw)) != 0) break;
                if (a == 0) B = Bw;
                else if (Bw != B) {
                    rc = set_err(c, WARP_HIP_E_BOOKS, layer, ids[a], "a chunk's records name different codebooks");
                    break;
                }
                rc = chunk_experts(c, layer, B, Xe, T, ids[a], ids[b - 1], a == 0);
            }
        }
        free(ids);
        if (rc) return rc;
    } else {
        release_hold(c, layer);
        if ((rc = chunk_experts(c, layer, B, Xe, T, 0, E - 1, 1))) return rc;
    }
    if (L->sq[0]) {
        c->sx_pending = 0;
        DEV(c, hipStreamWaitEvent(c->st, c->ev_sx1, 0));
    }
    if (lat) {
        KRN(c, wk_combine_chunk(c->yd, c->tok_slots, c->pair_w, T, K, c->He, NULL, NULL, c->ylat, c->st));
        if ((rc = latent_tail(c, L, T, resid_dev, out_dev))) return rc;
    } else {
        KRN(c, wk_combine_chunk(c->yd, c->tok_slots, c->pair_w, T, K, H, L->sq[0] ? c->sho : NULL, resid_dev, out_dev,
                                c->st));
    }
    DEV(c, hipEventRecord(c->ev_after, c->st));
    if ((rc = lookahead_issue(c, layer, n_la))) return rc;
    /* every record of the layer resident and no selection asked for: no
     * pick can miss and the plan's job count always fits, so there is
     * nothing to report and the stream is not waited for (the outputs are
     * ready when the stream is) */
    if (!route && !rw && L->resident == E) return 0;
    DEV(c, hipMemcpyAsync(c->h_missing, c->missing, sizeof(int), hipMemcpyDeviceToHost, c->st));
    if (route) DEV(c, hipMemcpyAsync(c->h_idx, c->idx, (size_t)P * sizeof(int), hipMemcpyDeviceToHost, c->st));
    if (rw) DEV(c, hipMemcpyAsync(c->h_w, c->w, (size_t)P * sizeof(float), hipMemcpyDeviceToHost, c->st));
    DEV(c, hipStreamSynchronize(c->st));
    if (*c->h_missing)
        return set_err(c, WARP_HIP_E_MISSING, layer, -1,
                       *c->h_missing == 2 ? "chunk needs more jobs than planned" : "a selected expert is not resident");
    if (route) memcpy(route, c->h_idx, (size_t)P * sizeof(int));
    if (rw) memcpy(rw, c->h_w, (size_t)P * sizeof(float));
    return 0;
}

int warp_hip_moe_chunk_host(warp_hip_ctx *c, int layer, const float *X, float *out, int T, int *route, float *rw)
{
    if (!c) return WARP_HIP_E_ARG;
    if (T < 1 || T > c->cfg.max_tokens) return set_err(c, WARP_HIP_E_ARG, layer, -1, "T out of range");
    const size_t bytes = (size_t)T * c->cfg.hidden * 4;
    DEV(c, hipMemcpyAsync(c->xin, X, bytes, hipMemcpyHostToDevice, c->st));
    int rc = warp_hip_moe_chunk(c, layer, c->xin, c->xout, NULL, T, route, rw);
    if (rc) return rc;
    DEV(c, hipMemcpyAsync(out, c->xout, bytes, hipMemcpyDeviceToHost, c->st));
    DEV(c, hipStreamSynchronize(c->st));
    return 0;
}

/* ---- finer-grained entry points -------------------------------------------------------------- */

static int matrix_shape(const warp_hip_ctx *c, int kind, int *M, int *N)
{
    if (kind < 0 || kind > 2) return -1;
    *M = kind == 2 ? c->He : c->cfg.inter;
    *N = kind == 2 ? c->cfg.inter : c->He;
    return 0;
}

int warp_hip_vq_matvec(warp_hip_ctx *c, int layer, int kind, const uint8_t *rec_dev, const float *x_dev, float *y_dev)
{
    int rc = check_layer(c, layer);
    if (rc) return rc;
    const layer_t *L = &c->L[layer];
    int M, N;
    if (matrix_shape(c, kind, &M, &N) || !rec_dev || !L->has_books)
        return set_err(c, WARP_HIP_E_ARG, layer, -1, "vq_matvec arguments");
    uint8_t hdr[WARP_HDR_BYTES];
    DEV(c, hipMemcpy(hdr, rec_dev, sizeof hdr, hipMemcpyDeviceToHost));
    uint32_t off[4];
    memcpy(off, hdr + 20, 16);
    /* decoded with the record's own codebook_id (src/model.c:2286, 2907) */
    uint16_t cbid;
    memcpy(&cbid, hdr + 10, sizeof cbid);
    const layer_t *B = books_by_id(c, L, cbid);
    if (!B) return set_err(c, WARP_HIP_E_BOOKS, layer, -1, "record codebook_id %u: no layer has those codebooks", cbid);
    if (off[3] + 2 * (2 * (size_t)c->cfg.inter + c->He) > c->cfg.rec_bytes ||
        (size_t)off[kind] + (kind == 2 ? c->down_bytes : c->gate_bytes) > off[3])
        return set_err(c, WARP_HIP_E_HEADER, layer, -1, "record offsets");
    warp_job jb;
    memset(&jb, 0, sizeof jb);
    jb.idx = rec_dev + off[kind];
    jb.scale = (const uint16_t *)(rec_dev + off[3]) + (kind == 0 ? 0 : kind == 1 ? c->cfg.inter : 2 * c->cfg.inter);
    jb.n = 1;
    int nj[3] = { 0, 0, 0 };
    nj[kind] = 1;
    /* one job of this kind, list stride 1 */
    warp_job jl[3];
    memset(jl, 0, sizeof jl);
    jl[kind] = jb;
    DEV(c, hipMemcpyAsync(c->jobs, jl, sizeof jl, hipMemcpyHostToDevice, c->st));
    DEV(c, hipMemcpyAsync(c->njobs, nj, sizeof nj, hipMemcpyHostToDevice, c->st));
    /* scratch sized for the input width: hidden for gate/up, inter for down */
    if (c->P6) {
        int8_t *lut = kind == 2 ? c->lut8d : c->lut8;
        float *ls = kind == 2 ? c->lscaled : c->lscale;
        KRN(c, wk_lut_p6(x_dev, 1, N, books_kind(c, B, kind), lut, ls, c->st));
        KRN(c, wk_apply_p6(c->jobs, c->njobs, 1, kind, lut, ls, y_dev, M, N, c->st));
    } else if (use_gather(c, B, 1) && N % 32 == 0) {
        /* one launch of the row kernel: the whole matvec */
        float *yk[3] = { y_dev, y_dev, y_dev };
        KRN(c, wk_vq_rows(c->cfg.fmt, c->jobs, c->njobs, 1, kind, 1, B->books, x_dev, M, N, NULL, 0, 0, 0.0f, 0.0f,
                          yk, NULL, NULL, c->n_cu, c->st));
    } else if (use_table(c, B)) {
        float *yk[3] = { y_dev, y_dev, y_dev };
        int sp = 0;
        KRN(c, wk_vq_lut(c->cfg.fmt, c->jobs, c->njobs, 1, kind, 1, B->books, B->books_x31, x_dev, 1, c->part, c->part_cap, M, N,
                         c->n_cu, NULL, 0, 0, 0.0f, 0.0f, NULL, NULL, NULL, &sp, c->st));
        KRN(c, wk_lut_reduce(c->jobs, c->njobs, 1, kind, 1, c->part, sp, M, yk, c->st));
    } else {
        float *yk[3] = { y_dev, y_dev, y_dev };
        uint16_t *xs = kind == 2 ? c->xsh : c->xs;
        float *xsc = kind == 2 ? c->xscaleh : c->xscale;
        KRN(c, wk_split(x_dev, 1, N, xs, xsc, c->st));
        KRN(c, wk_vq_matvec(c->cfg.fmt, c->jobs, c->njobs, 1, kind, 1, B->books, xs, xsc, yk, M, N, 1, c->st));
    }
    DEV(c, hipStreamSynchronize(c->st));
    return 0;
}

int warp_hip_decode_weights(warp_hip_ctx *c, int layer, int kind, const uint8_t *rec_dev, float *W_dev)
{
    int rc = check_layer(c, layer);
    if (rc) return rc;
    const layer_t *L = &c->L[layer];
    int M, N;
    if (matrix_shape(c, kind, &M, &N) || !rec_dev || !L->has_books)
        return set_err(c, WARP_HIP_E_ARG, layer, -1, "decode_weights arguments");
    uint8_t hdr[WARP_HDR_BYTES];
    DEV(c, hipMemcpy(hdr, rec_dev, sizeof hdr, hipMemcpyDeviceToHost));
    uint32_t off[4];
    memcpy(off, hdr + 20, 16);
    /* decoded with the record's own codebook_id (src/model.c:2286, 2907) */
    uint16_t cbid;
    memcpy(&cbid, hdr + 10, sizeof cbid);
    const layer_t *B = books_by_id(c, L, cbid);
    if (!B) return set_err(c, WARP_HIP_E_BOOKS, layer, -1, "record codebook_id %u: no layer has those codebooks", cbid);
    const size_t soff = kind == 0 ? 0 : kind == 1 ? (size_t)c->cfg.inter : 2 * (size_t)c->cfg.inter;
    if (off[3] + 2 * (2 * (size_t)c->cfg.inter + c->He) > c->cfg.rec_bytes ||
        (size_t)off[kind] + (kind == 2 ? c->down_bytes : c->gate_bytes) > off[3])
        return set_err(c, WARP_HIP_E_HEADER, layer, -1, "record offsets");
    KRN(c, wk_decode_weights(c->cfg.fmt, rec_dev + off[kind], (const uint16_t *)(rec_dev + off[3]) + soff,
                             books_kind(c, B, kind), M, N, W_dev, c->st));
    DEV(c, hipStreamSynchronize(c->st));
    return 0;
}

int warp_hip_router_logits(warp_hip_ctx *c, int layer, const float *x_dev, int T, float *logits_dev)
{
    int rc = check_layer(c, layer);
    if (rc) return rc;
    KRN(c, logits_of(c, &c->L[layer], x_dev, T, logits_dev, c->st));
    DEV(c, hipStreamSynchronize(c->st));
    return 0;
}

int warp_hip_router_cert(warp_hip_ctx *c, int layer, const float *x_dev, float *out_dev)
{
    int rc = check_layer(c, layer);
    if (rc) return rc;
    const warp_hip_cfg *g = &c->cfg;
    const layer_t *L = &c->L[layer];
    if (!L->router || g->router_act != WARP_HIP_ROUTE_SIGMOID)
        return set_err(c, WARP_HIP_E_ARG, layer, -1, "certified router needs an F32 router and sigmoid scores");
    KRN(c, wk_router_cert(L->router, x_dev, g->n_experts, g->hidden, L->bias, out_dev, NULL, 0, NULL, NULL, NULL, 0,
                          c->st));
    DEV(c, hipStreamSynchronize(c->st));
    return 0;
}

int warp_hip_route(warp_hip_ctx *c, int layer, const float *logits_dev, int T, int *idx_dev, float *w_dev)
{
    int rc = check_layer(c, layer);
    if (rc) return rc;
    const warp_hip_cfg *g = &c->cfg;
    KRN(c, wk_route(logits_dev, c->L[layer].bias, g->n_experts, g->top_k, T, g->router_act, g->renorm, g->routed_scale,
                    idx_dev, w_dev, NULL, NULL, NULL, NULL, 0, c->st));
    DEV(c, hipStreamSynchronize(c->st));
    return 0;
}

int warp_hip_mvq(warp_hip_ctx *c, int bits, int group, const int8_t *q_dev, const uint16_t *scales_dev,
                 size_t rowbytes, const float *x_dev, int M, int N, int T, float *y_dev)
{
    if (!c) return WARP_HIP_E_ARG;
    KRN(c, wk_mvq(q_dev, scales_dev, rowbytes, group, bits, x_dev, M, N, T, y_dev, c->st));
    DEV(c, hipStreamSynchronize(c->st));
    return 0;
}

int warp_hip_fill_random(warp_hip_ctx *c, void *dev, size_t n, uint64_t seed)
{
    if (!c) return WARP_HIP_E_ARG;
    KRN(c, wk_fill_random((uint8_t *)dev, n, seed, c->st));
    return 0;
}

/* ---- checksums and the learned hotlist ------------------------------------------------------ */

int warp_hip_crc32(warp_hip_ctx *c, const void *p_dev, size_t n, uint32_t *crc)
{
    if (!c || !crc || (n && !p_dev)) return c ? set_err(c, WARP_HIP_E_ARG, -1, -1, "crc32 arguments") : WARP_HIP_E_ARG;
    if (n == 0) {
        *crc = 0;                      /* zlib's crc32 of nothing */
        return 0;
    }
    if (n > CRC_MAX_BYTES) return set_err(c, WARP_HIP_E_ARG, -1, -1, "crc32 of %zu bytes: at most %zu", n, CRC_MAX_BYTES);
    /* on the copy stream, in order with the record checksums that share
     * the scratch; the result goes after the block sums */
    uint32_t *out = c->crc_tmp + wk_crc32_tmp_words(CRC_MAX_BYTES);
    KRN(c, wk_crc32((const uint8_t *)p_dev, n, c->crc_tmp, out, NULL, -1, NULL, c->cp));
    DEV(c, hipMemcpyAsync(c->h_word, out, sizeof(uint32_t), hipMemcpyDeviceToHost, c->cp));
    DEV(c, hipStreamSynchronize(c->cp));
    *crc = *c->h_word;
    return 0;
}

/* waste_usage_hdr / waste_usage_ent (src/waste_format.h:173-187) */
typedef struct {
    uint32_t magic, version;
    uint64_t total_tokens;
} usage_hdr;
typedef struct {
    uint16_t layer, expert_id;
    uint32_t hits, last_seen, next_layer_top;
} usage_ent;
#define USAGE_MAGIC 0x47535557u

int warp_hip_save_usage(warp_hip_ctx *c, const char *path, uint64_t tokens)
{
    if (!c || !path) return WARP_HIP_E_ARG;
    FILE *f = fopen(path, "wb");
    if (!f) return set_err(c, WARP_HIP_E_READ, -1, -1, "cannot write %s", path);
    const usage_hdr h = { USAGE_MAGIC, 1, tokens };
    int ok = fwrite(&h, sizeof h, 1, f) == 1;
    const int E = c->cfg.n_experts;
    for (int s = 0; ok && s < c->n_slots; s++) {
        const int key = c->slot_key[s];
        if (key < 0) continue;
        const usage_ent e = { (uint16_t)(key / E), (uint16_t)(key % E), c->hits[s], (uint32_t)c->last[s], 0 };
        ok = fwrite(&e, sizeof e, 1, f) == 1;
    }
    ok &= fclose(f) == 0;
    if (!ok) {
        remove(path);
        return set_err(c, WARP_HIP_E_READ, -1, -1, "writing %s failed", path);
    }
    return 0;
}

/* hits descending, then (layer, expert) ascending: the order
 * src/ecache.c:749-760 warms in, the same for any sort */
static int usage_cmp(const void *a, const void *b)
{
    const usage_ent *x = (const usage_ent *)a, *y = (const usage_ent *)b;
    if (x->hits != y->hits) return x->hits > y->hits ? -1 : 1;
    if (x->layer != y->layer) return x->layer < y->layer ? -1 : 1;
    if (x->expert_id != y->expert_id) return x->expert_id < y->expert_id ? -1 : 1;
    return 0;
}

int warp_hip_warm(warp_hip_ctx *c, const char *path)
{
    if (!c || !path) return WARP_HIP_E_ARG;
    if (!can_fetch(c)) return set_err(c, WARP_HIP_E_ARG, -1, -1, "warming needs a fetch function");
    FILE *f = fopen(path, "rb");
    if (!f) return set_err(c, WARP_HIP_E_READ, -1, -1, "cannot read %s", path);
    usage_hdr h;
    long n = 0;
    usage_ent *ent = NULL;
    int bad = fread(&h, sizeof h, 1, f) != 1 || h.magic != USAGE_MAGIC;
    if (!bad) {
        const long start = ftell(f);
        bad = fseek(f, 0, SEEK_END) != 0;
        n = bad ? 0 : (ftell(f) - start) / (long)sizeof(usage_ent);
        bad |= fseek(f, start, SEEK_SET) != 0;
    }
    if (!bad && n > 0) {
        ent = (usage_ent *)malloc((size_t)n * sizeof *ent);
        bad = !ent || fread(ent, sizeof *ent, (size_t)n, f) != (size_t)n;
    }
    fclose(f);
    if (bad) {
        free(ent);
        return set_err(c, WARP_HIP_E_READ, -1, -1, "%s is not a usage file", path);
    }
    qsort(ent, (size_t)n, sizeof *ent, usage_cmp);
    const int want = n < c->n_slots ? (int)n : c->n_slots;
    const int E = c->cfg.n_experts;
    int loaded = 0;
    /* the fills overwrite nothing a kernel may still read */
    DEV(c, hipEventRecord(c->ev_before, c->st));
    DEV(c, hipStreamWaitEvent(c->cp, c->ev_before, 0));
    for (int i = 0; i < want; i++) {
        const int L = ent[i].layer, e = ent[i].expert_id;
        /* ids from a file that travels beside a container: a stale entry
         * is skipped, not an error (src/model.c:1770-1783, :2983-2988) */
        if (L >= c->cfg.n_layers || e >= E || !c->L[L].has_books) continue;
        if (c->key_slot[L * E + e] >= 0) continue;
        const int rc = fill_from_fetch(c, L, e);
        if (rc == WARP_HIP_E_NOSLOT) break;
        if (rc) continue;
        const int s = c->key_slot[L * E + e];
        c->hits[s] = ent[i].hits;          /* the recorded frequency seeds the LFRU */
        c->stats.prefetched++;
        loaded++;
    }
    free(ent);
    int rc = flush_table(c);
    if (rc) return rc;
    /* warming is best effort: records refused by their checksum are
     * dropped, not reported */
    if (c->cfg.verify && crc_report(c) == WARP_HIP_E_CRC) loaded -= c->h_crc_err->n;
    c->err[0] = 0;
    c->err_layer = c->err_expert = -1;
    return loaded;
}
