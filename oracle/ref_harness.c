/*
 * ref_harness.c — exposes the reference's static MoE functions for golden
 * vectors. TEST INFRASTRUCTURE ONLY, built into oracle/_ref/ by
 * oracle/Makefile from the reference sources where they lie (nothing is
 * copied): this file includes the reference's src/model.c so that its
 * static vq_build_lut, vq_apply, vq_matvec, moe_layer and moe_chunk can be
 * called on a model loaded by waste_model_load from a synthetic container.
 * Built with the flags the reference gives model.c (-O2 -std=gnu11).
 */
#include "model.c"

void *ref_open(const char *dir, size_t cache_bytes, int n_threads)
{
    waste_model *m = (waste_model *)calloc(1, sizeof *m);
    if (!m) return NULL;
    waste_load_opts o;
    memset(&o, 0, sizeof o);
    o.cache_bytes = cache_bytes;
    o.direct_io = 0;
    o.n_threads = n_threads;   /* 0: the reference's default, one per CPU */
    if (waste_model_load(m, dir, 64, &o) != 0) { free(m); return NULL; }
    /* the router's scratch must still hold this layer's logits and scores
     * when moe_layer returns, so no lookahead into it; set after the load,
     * whose one-time option parsing would otherwise reset it */
    waste_model_set_lookahead(0);
    return m;
}

void ref_close(void *p)
{
    waste_model *m = (waste_model *)p;
    if (m) { waste_model_free(m); free(m); }
}

const char *ref_backend(void) { return waste_backend_name(); }

int ref_threads(void) { return waste_pool_threads(); }

int ref_read_error(void *p) { return ((waste_model *)p)->read_error; }

/* moe_layer for one token. logits/scores get n_experts floats each. */
int ref_moe_layer(void *p, int L, const float *in, float *out, int *routed,
                  float *logits, float *scores)
{
    waste_model *m = (waste_model *)p;
    const int E = m->cfg.n_experts;
    moe_layer(m, L, in, out, routed);
    const float *sc = m->att + WASTE_ATT_ROUTER_OFF;
    if (logits) memcpy(logits, sc, (size_t)E * sizeof(float));
    if (scores) memcpy(scores, sc + E, (size_t)E * sizeof(float));
    return m->read_error;
}

/* moe_chunk over nT tokens; route/rw receive [nT][top_k]. */
int ref_moe_chunk(void *p, int L, const float *in, float *out, int nT, int *route,
                  float *rw)
{
    waste_model *m = (waste_model *)p;
    if (prefill_alloc(m, nT) != 0) return -1;
    moe_chunk(m, L, in, out, nT);
    const int K = m->cfg.top_k;
    memcpy(route, m->croute, (size_t)nT * K * sizeof(int));
    memcpy(rw, m->crw, (size_t)nT * K * sizeof(float));
    return m->read_error;
}

/* The LUT of one matrix kind (0 gate, 1 up, 2 down) for input x of width N,
 * built with the layer's codebook base. lut gets N/vd * stages * entries. */
int ref_build_lut(void *p, int L, int kind, const float *x, int N, float *lut)
{
    waste_model *m = (waste_model *)p;
    const int cb = m->bank[L].cb_base + kind * m->stages;
    vq_build_lut(m, lut, cb, x, N, m->stages, m->cb_entries, m->vec_dim, NULL, NULL);
    return 0;
}

/* vq_matvec of one matrix of one expert record: y = W_kind(expert) x. */
int ref_vq_matvec(void *p, int L, int expert, int kind, const float *x, float *y)
{
    waste_model *m = (waste_model *)p;
    const uint8_t *rec = read_expert(m, L, expert);
    if (!rec) return -1;
    const waste_expert_hdr *h = (const waste_expert_hdr *)rec;
    const uint16_t *sc = (const uint16_t *)(rec + h->chan_corr_off);
    /* the experts' width: the latent size on a latent MoE */
    const int inter = m->cfg.moe_inter, hid = m->cfg.latent_dim ? m->cfg.latent_dim : m->cfg.hidden;
    const uint32_t off = kind == 0 ? h->gate_off : kind == 1 ? h->up_off : h->down_off;
    const int M = kind == 2 ? hid : inter, N = kind == 2 ? inter : hid;
    const uint16_t *s = sc + (kind == 0 ? 0 : kind == 1 ? inter : 2 * inter);
    const size_t lsz = (size_t)(N / m->vec_dim) * m->stages * m->cb_entries;
    float *lut = (float *)malloc(lsz * sizeof(float));
    int8_t *q = m->index_bits == 6 ? (int8_t *)malloc(lsz) : NULL;
    float *qs = m->index_bits == 6 ? (float *)malloc((lsz / (m->stages * m->cb_entries) / WASTE_VQ_LUT_BLK + 2) * sizeof(float)) : NULL;
    if (!lut || (m->index_bits == 6 && (!q || !qs))) { free(lut); free(q); free(qs); return -1; }
    vq_matvec(m, y, rec + off, s, x, M, N, h->codebook_id + kind * m->stages, lut, q, qs);
    free(lut); free(q); free(qs);
    return 0;
}

/* The shared expert's three projections through matvec_t, as moe_layer
 * runs them (the backend's mvq_rows_f32 for a quantised trunk). */
int ref_trunk_matvec(void *p, const char *name, const float *x, float *y, int out, int in)
{
    waste_model *m = (waste_model *)p;
    const waste_tensor *t = waste_find(m, name);
    if (!t) return -1;
    matvec_t(m, y, t, x, out, in);
    return 0;
}

/* One expert's FFN as moe_layer runs it for each routed expert
 * (src/model.c:2886-2909): the gate and up tables of x, their gather
 * applies, SiLU(gate) * up, then the down matvec; y [hidden], unweighted. */
int ref_expert_ffn(void *p, int L, int expert, const float *x, float *y)
{
    waste_model *m = (waste_model *)p;
    const uint8_t *rec = read_expert(m, L, expert);
    if (!rec) return -1;
    const waste_expert_hdr *h = (const waste_expert_hdr *)rec;
    const uint16_t *sc = (const uint16_t *)(rec + h->chan_corr_off);
    const int inter = m->cfg.moe_inter, hid = m->cfg.latent_dim ? m->cfg.latent_dim : m->cfg.hidden;
    const size_t lin = (size_t)(hid / m->vec_dim) * m->stages * m->cb_entries;
    const size_t ldn = (size_t)(inter / m->vec_dim) * m->stages * m->cb_entries;
    float *lg = (float *)malloc(lin * sizeof(float)), *lu = (float *)malloc(lin * sizeof(float));
    float *ld = (float *)malloc(ldn * sizeof(float));
    float *ga = (float *)malloc((size_t)inter * sizeof(float)), *ub = (float *)malloc((size_t)inter * sizeof(float));
    if (!lg || !lu || !ld || !ga || !ub || m->index_bits == 6) {
        free(lg); free(lu); free(ld); free(ga); free(ub);
        return -1;
    }
    vq_build_lut(m, lg, h->codebook_id + 0 * m->stages, x, hid, m->stages, m->cb_entries, m->vec_dim, NULL, NULL);
    vq_build_lut(m, lu, h->codebook_id + 1 * m->stages, x, hid, m->stages, m->cb_entries, m->vec_dim, NULL, NULL);
    vq_apply(m, ga, rec + h->gate_off, sc, inter, hid, lg, NULL, NULL);
    vq_apply(m, ub, rec + h->up_off, sc + inter, inter, hid, lu, NULL, NULL);
    for (int i = 0; i < inter; i++) ga[i] = silu(ga[i]) * ub[i];
    vq_matvec(m, y, rec + h->down_off, sc + 2 * inter, ga, hid, inter, h->codebook_id + 2 * m->stages, ld, NULL,
              NULL);
    free(lg); free(lu); free(ld); free(ga); free(ub);
    return 0;
}

/* Ends the process-wide thread pool, so that the next ref_open sizes a new
 * one (the pool is otherwise fixed by the first model opened). */
void ref_pool_reset(void) { waste_pool_shutdown(); }

/* The reference's usage file of its expert cache (waste_model_save_usage,
 * src/model.c:2991-2995). */
int ref_save_usage(void *p, const char *path) { return waste_model_save_usage((waste_model *)p, path); }

/* The reference's record_check (src/model.c:1698-1745) on a record of layer
 * L's bank, with its checksum switch (m->verify) set to `verify` for the
 * call. Returns its rec_status: 0 OK, 2 E_HEADER, 3 E_CRC. */
int ref_record_check(void *p, int L, int expert, const uint8_t *rec, int verify)
{
    waste_model *m = (waste_model *)p;
    const int keep = m->verify;
    m->verify = verify;
    const int st = (int)record_check(m, L, expert, rec);
    m->verify = keep;
    return st;
}

/* The container's codebook count (src/model.c:1274). */
int ref_n_books(void *p) { return ((waste_model *)p)->n_books; }

/* The reference's expert cache (src/ecache.c) driven by a routing trace the
 * way moe_layer drives it with read-ahead off and no lookahead: for every
 * token, every layer, one waste_ecache_get per selected expert in order
 * (src/model.c:2862-2868). ids [n_tok][n_layers][K]; a cache of n_slots
 * records under the LFRU policy; the fetch reads nothing. out: hits,
 * misses, evictions, bytes_read / rec_bytes. */
static int replay_fetch(void *user, int layer, int expert, uint8_t *dst)
{
    (void)user; (void)layer; (void)expert; (void)dst;
    return 0;
}

int ref_ecache_replay(const int *ids, int n_tok, int n_layers, int K, int n_slots, uint64_t out[4])
{
    waste_ecache c;
    const size_t rec = 4096;
    if (waste_ecache_init(&c, (size_t)n_slots * rec, rec, 0) != 0) return -1;
    for (int t = 0; t < n_tok; t++)
        for (int L = 0; L < n_layers; L++)
            for (int j = 0; j < K; j++)
                if (!waste_ecache_get(&c, L, ids[((size_t)t * n_layers + L) * K + j], replay_fetch, NULL)) {
                    waste_ecache_free(&c);
                    return -2;
                }
    out[0] = c.hits;
    out[1] = c.misses;
    out[2] = c.evictions;
    out[3] = c.bytes_read / rec;
    waste_ecache_free(&c);
    return 0;
}
