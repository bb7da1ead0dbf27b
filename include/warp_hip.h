/*
 * warp_hip.h — C ABI of the MI355X (gfx950) backend for WARP's routed-expert
 * MoE path. Plain C, plain pointers and sizes.
 *
 * Two halves:
 *
 *  1. The reference's dispatch table (src/waste_backend.h:67-94) and a
 *     registration function in its style (src/waste_backend.h:116-120,
 *     called from src/backend.c:198-211 under WASTE_ENABLE_HIP). It fills
 *     the mvq_rows_f32 slot with a device implementation and sets
 *     on_device, so run_rows hands it whole row ranges (src/model.c:356-360).
 *
 *  2. The MoE slots the table does not have. The gather apply, routing,
 *     combine and chunk loop are static functions of src/model.c
 *     (vq_apply :2264, moe_layer :2713, moe_chunk :3512); these entry points
 *     replace them behind a context that keeps the codebooks, routers,
 *     shared experts and an expert cache resident in HBM.
 *
 * Device pointers are named *_dev and live in the memory of the context's
 * device; everything else is host memory borrowed for the duration of the
 * call. Functions returning int return 0 on success or a negative
 * WARP_HIP_E_* code; the reason is available from warp_hip_error().
 * A context is not thread-safe (as a waste_ctx is not, src/waste.h:25-26);
 * distinct contexts are independent.
 */
#ifndef WARP_HIP_H
#define WARP_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- 1. the reference's dispatch table ---------------------------------- */

#ifndef WASTE_BACKEND_H
/* Identical layout to src/waste_backend.h:67-90 for a build that does not
 * include the reference's header. */
typedef struct {
    void (*kda_step)(int H, int K, int V, const float *q, const float *k, const float *v,
                     const float *g_log, const float *beta, float *S, float *o, float *scratch);
    void (*short_conv_step)(int C, int KS, const float *w, const float *bias, float *ring,
                            const float *x, float *y);
    void (*rmsnorm_gated)(int C, const float *x, const float *gate, const float *weight,
                          float eps, float *y);
    void (*mvq_rows_f32)(int b, int e, void *arg);
    void (*lutb_range)(int lo, int hi, void *arg);
    int on_device;
} waste_kernels;
#endif

/* Replaces: the registration shape of src/waste_backend.h:116-120 (a new
 * waste_register_hip beside waste_register_metal, src/metal.m). Probes for a
 * gfx950 device and returns NULL (declines) without one; otherwise fills
 * mvq_rows_f32 (argument struct mvq_arg, src/simd.h:35-39, host pointers) and
 * kda_step (src/waste_backend.h:69-72: waste_kda_step's arguments, host
 * pointers; the state goes to the device and back on every call, and the
 * results are bit-identical to src/kda.c:26-68), sets on_device = 1, and
 * returns "HIP gfx950". Each slot keeps the table's previous function and
 * calls it with the same arguments if a device call fails, as the
 * reference's accelerator contract requires (src/metal.m:177-181);
 * warp_hip_table_stats() and warp_hip_kda_stats() report how many calls ran
 * where. */
const char *waste_register_hip(waste_kernels *t);

/* Replaces: src/waste_backend.h:112-114 for this backend. Drops the device
 * mirrors of trunk tensors keyed by host pointer and the MoE slots' device
 * state (their contexts, keyed by model); call before the model frees its
 * host buffers. */
void waste_hip_release_host_buffers(void);

/* Calls of the mvq_rows_f32 slot that ran on the device / fell back. */
void warp_hip_table_stats(uint64_t *device_calls, uint64_t *fallback_calls);
/* The same for the kda_step slot. */
void warp_hip_kda_stats(uint64_t *device_calls, uint64_t *fallback_calls);

/* Replaces waste_kda_forward (src/kda.c:70-82) for state and inputs already in
 * device memory: T steps of the recurrence in one launch on `stream` (a
 * hipStream_t, NULL for the null stream), the state S [H][K][V] updated in
 * place and kept on chip between the steps; q, k, g_log [T][H][K], v, o
 * [T][H][V], beta [T][H]. K <= 256, V <= 1024, K*V <= 38400. Bit-identical to
 * T calls of waste_kda_step. */
int warp_hip_kda_forward(int T, int H, int K, int V, const float *q_dev, const float *k_dev, const float *v_dev,
                         const float *g_dev, const float *beta_dev, float *S_dev, float *o_dev, void *stream);

/* ---- 1b. the MoE path behind a table of the same style -----------------------
 *
 * The reference's table has no slot for the routed-expert path: moe_layer
 * (src/model.c:2713) and moe_chunk (src/model.c:3512) are static, and call
 * vq_apply, the routing and the combine directly. This second table, beside
 * waste_kernels and in its style (function pointers the engine calls,
 * defaults that leave the CPU path in charge, filled by a registration
 * function), gives the engine one backend-neutral call per call site:
 *
 *     if (waste_km.moe_ffn_decode && waste_km.moe_ffn_decode(&a) == 0) return;
 *
 * at the top of moe_layer, and the same with moe_ffn_batch in moe_chunk.
 * A slot returns 0 when it has written every output, or a negative
 * WARP_HIP_E_* code when it declined or failed, having written nothing the
 * caller reads: the caller then runs its own CPU code with the same
 * arguments. A separate struct, rather than members appended to
 * waste_kernels, keeps waste_kernels' layout, so a registration function
 * never writes past the end of an engine's older table. */

/* A trunk tensor as waste_tensor holds it (src/model.h:30-45): F32 rows in
 * `data`, or quantised rows (Q8G, Q4G, Q3G) in q / qs. */
typedef struct {
    const float *data;        /* F32 [out][in], or NULL                     */
    const int8_t *q;          /* quantised rows, `rowbytes` apart           */
    const uint16_t *qs;       /* fp16 scale per group of `group`            */
    int group, bits;          /* bits 8, 4 or 3 when quantised              */
    size_t rowbytes;
} warp_trunk_tensor;

/* Everything moe_layer / moe_chunk read for one MoE layer, as plain host
 * pointers into the engine's model (waste_model), and the call's own
 * inputs and outputs. The backend keeps device copies keyed by `model`
 * and by these pointers (the way src/metal.m:98-150 keys its buffers),
 * until waste_hip_release_host_buffers. */
typedef struct {
    const void *model;        /* identity of the engine's model            */
    int layer, n_layers;
    /* waste_config (src/model.h) */
    int hidden, moe_inter, n_experts, top_k;
    int latent_dim;           /* 0: the experts run on hidden               */
    int latent_norm;          /* latent_moe_use_norm                        */
    float norm_eps;
    int renorm;               /* moe_renormalize present                    */
    float routed_scale;
    int act_situ;
    float situ_beta, situ_linear_beta;
    /* the expert format: index_bits 8 (stages 3 or 2, entries 256) or 6
     * (4 x 64), as waste_model keeps them; 12 with 2 x 4096 for the
     * 12-bit extension */
    int index_bits, stages, cb_entries, vec_dim;
    /* m->codebooks: [n_books][cb_entries][vec_dim] f32, flushed as the
     * loader flushes (src/model.c:1277-1286); this layer's bank base */
    const float *codebooks;
    int n_books, cb_base;
    /* block_sparse_moe.gate.weight and .e_score_correction_bias (NULL) */
    warp_trunk_tensor router;
    const float *bias;
    /* shared_experts.{gate,up,down}_proj (q NULL and data NULL: none),
     * inter_shared = moe_inter * n_shared */
    warp_trunk_tensor shared[3];
    int inter_shared;
    /* routed_expert_{down,up}_proj and routed_expert_norm (latent only) */
    warp_trunk_tensor latent[2];
    const float *latent_norm_w;
    /* expert records: the bank's stride, and how a miss is read
     * (bank_fetch and its model, src/model.c:1767-1812); the HBM cache
     * size the backend may use, and the engine's verify and lookahead */
    size_t rec_bytes, cache_bytes;
    int verify, lookahead;
    int (*fetch)(void *user, int layer, int expert, uint8_t *dst);
    void *fetch_user;
    /* the call: n_tokens inputs [n_tokens][hidden] -> out [n_tokens][hidden]
     * (routed sum plus the shared expert; not the residual), and per token
     * its top_k ids (route) and weights (rw, may be NULL) in selection
     * order. moe_ffn_decode takes n_tokens = 1. */
    int n_tokens;
    const float *x;
    float *out;
    int *route;
    float *rw;
} warp_moe_args;

typedef struct {
    int (*moe_ffn_decode)(const warp_moe_args *a);  /* moe_layer, one token   */
    int (*moe_ffn_batch)(const warp_moe_args *a);   /* moe_chunk              */
    int on_device;
} waste_moe_kernels;

/* Fills both slots with this backend's (when a gfx950 device is present;
 * otherwise returns NULL and leaves the table), keeping each slot's previous
 * value: a call this backend declines or fails goes to it with the same
 * arguments, and with the CPU default (NULL) the slot returns the negative
 * code and the engine runs its CPU path. Returns "HIP gfx950". The device
 * state it builds is dropped by waste_hip_release_host_buffers(). No
 * counterpart in the reference beyond the style of
 * waste_register_metal (src/waste_backend.h:116-120). */
const char *waste_register_hip_moe(waste_moe_kernels *t);
/* Calls of the MoE slots that ran on the device / were declined or failed
 * (and went to the previous slot or the CPU path). */
void warp_hip_moe_table_stats(uint64_t *device_calls, uint64_t *fallback_calls);

/* ---- 2. MoE slots ---------------------------------------------------------- */

/* Expert formats: waste_fmt codes (src/waste_format.h:41-71) plus one. */
enum {
    WARP_HIP_VQ3R = 4,   /* 3 stages x 256 entries, byte codes                 */
    WARP_HIP_VQ2R = 5,   /* 2 stages x 256 entries, byte codes                 */
    WARP_HIP_VQ4P = 8,   /* 4 stages x 64 entries, 4x6 bits in 3 bytes         */
    WARP_HIP_VQ12 = 9,   /* extension: 2 stages x 4096, two 12-bit codes in the
                          * little-endian 3-byte word s0 | s1 << 12; same
                          * blocked layout, same 3.00 bits per weight          */
};

enum {
    WARP_HIP_OK = 0,
    WARP_HIP_E_ARG = -1,       /* a size or pointer the call cannot accept     */
    WARP_HIP_E_DEVICE = -2,    /* a HIP call failed                            */
    WARP_HIP_E_NOMEM = -3,     /* device or pinned allocation failed           */
    WARP_HIP_E_READ = -4,      /* fetch short or failed   (REC_E_READ)         */
    WARP_HIP_E_HEADER = -5,    /* record header invalid   (REC_E_HEADER)       */
    WARP_HIP_E_CRC = -6,       /* record payload checksum (REC_E_CRC)          */
    WARP_HIP_E_NOSLOT = -7,    /* cache could not free a slot (REC_E_NOSLOT)   */
    WARP_HIP_E_MISSING = -8,   /* a selected expert is neither resident nor
                                * fetchable: the layer was not computed       */
    WARP_HIP_E_BOOKS = -9,     /* a selected record names codebooks other than
                                * its layer's (its codebook_id is not the
                                * layer's cb_base): the reference decodes it
                                * with its own (src/model.c:2889-2907), this
                                * backend with one set per layer, so the layer
                                * was not computed and the caller's CPU path
                                * runs it                                    */
};

enum { WARP_HIP_ROUTE_SIGMOID = 0, WARP_HIP_ROUTE_SOFTMAX = 1 };

typedef struct {
    int hidden;            /* H: the router's, shared expert's and output width */
    int inter;             /* moe_intermediate_size                            */
    int n_experts;         /* E                                                */
    int top_k;             /* K <= 64                                          */
    int n_layers;
    int fmt;               /* WARP_HIP_VQ*                                     */
    int renorm;            /* moe_renormalize present (src/model.c:977-978)    */
    float routed_scale;    /* routed_scaling_factor                            */
    int router_act;        /* WARP_HIP_ROUTE_SIGMOID is the reference; SOFTMAX
                            * is the extension                                 */
    int router_strict;     /* 1: F32 router logits in the reference's
                            * sequential fp32 order (bit-identical logits)
                            * everywhere; 2: so in chunks, while decode
                            * certifies its selection (router_fast)          */
    int act_situ;          /* hidden_act == "situ"                             */
    float situ_beta, situ_linear_beta;
    int max_tokens;        /* largest chunk warp_hip_moe_chunk will be given   */
    size_t rec_bytes;      /* expert record stride, a 4 KiB multiple           */
    size_t cache_bytes;    /* HBM budget for expert records                    */
    int verify;            /* crc32 every record entering the cache
                            * (WASTE_VERIFY, src/model.c:1742-1744), on the
                            * device after its copy; a refused record is
                            * reported as E_CRC by the call that fetched it
                            * (or, for a prefetch, by the next call that
                            * waits) and leaves the cache                    */
    int lookahead;         /* experts of layer L+1 to prefetch per token from
                            * layer L's input (WASTE_LOOKAHEAD,
                            * src/model.c:2680-2711)                           */
    int device;            /* HIP device ordinal                               */
    int latent;            /* routed_expert_hidden_size: the experts run on a
                            * latent projection of this width (0: on H); see
                            * warp_hip_set_latent                              */
    int latent_norm;       /* latent_moe_use_norm: RMS norm of the experts'
                            * combined latent output                          */
    float norm_eps;        /* rms_norm_eps for that norm                       */
    int prefill_fp16;      /* chunks (warp_hip_moe_chunk*): the routed experts'
                            * matrix-core products in fp16 -- the stages'
                            * codebook vectors added into one fp16 value, x's
                            * fp16 high half only, SwiGLU's SiLU with the
                            * hardware exp -- a quarter of the MFMAs,
                            * outputs within 2e-3 of the reference instead of
                            * 1e-4 (the reference CPU path has no such mode;
                            * 0 keeps the exact products). Needs max_tokens x
                            * top_k x max(hidden, inter) x 2 bytes under 2 GiB
                            * (else chunks stay exact) and allocates that much
                            * at open; VQ4P chunks stay on their int8 tables */
    int n_books;           /* codebooks in the container (codebooks.bin,
                            * src/model.c:1274): a record's codebook_id must
                            * satisfy codebook_id + 3*stages <= n_books, as
                            * record_check requires (src/model.c:1721-1723);
                            * 0: n_layers * 3 * stages, one set per layer    */
    int router_fast;       /* decode with an F32 router and sigmoid scores
                            * certifies its selection by default: the router
                            * launch bounds each logit's distance from the
                            * reference's sequential sum, and the routing
                            * recomputes, in the reference's order, the rows
                            * whose bounds leave the picks or their order
                            * open, so the picks are the reference's (see
                            * warp_hip_get_route_stats). 1: the fast logits'
                            * picks as they are (a near-tie may order
                            * differently); router_strict overrides both.
                            * Chunks take the fast logits unless
                            * router_strict                                  */
} warp_hip_cfg;

typedef struct warp_hip_ctx warp_hip_ctx;

/* Fills `rec_bytes` at dst with record (layer, expert) and returns 0; the
 * reference's waste_fetch_fn (src/ecache.h:35-38), e.g. bank_fetch. */
typedef int (*warp_hip_fetch_fn)(void *user, int layer, int expert, uint8_t *dst);

/* Returns where record (layer, expert) already sits in pinned host memory
 * (from warp_hip_host_alloc), or NULL when it cannot. The miss copies it to
 * HBM from there, without a staging copy: the ecache's host slots as the DMA
 * source (src/ecache.c:347-349). It must stay unchanged until the next
 * synchronising call. No counterpart in the reference's interface. */
typedef const uint8_t *(*warp_hip_fetch_host_fn)(void *user, int layer, int expert);

typedef struct {
    uint64_t hits, misses, bytes_read, evictions;
    uint64_t prefetched, spec_issued;      /* as waste_ecache (src/ecache.h:69-71) */
    int n_slots, resident;
} warp_hip_cache_stats;

/* Replaces the MoE half of waste_model_load (src/model.c:1058-1493) for
 * this backend: a context with device scratch for cfg->max_tokens tokens and
 * an expert cache of cfg->cache_bytes / cfg->rec_bytes slots. */
int warp_hip_open(const warp_hip_cfg *cfg, warp_hip_ctx **out);
void warp_hip_close(warp_hip_ctx *c);

/* Replaces waste_model_read_error (src/model.c:1815): the last failure, and
 * the layer and expert it concerns (-1 when none). Never NULL. */
const char *warp_hip_error(const warp_hip_ctx *c, int *layer, int *expert);

/* The context's compute stream (a hipStream_t) for callers that enqueue
 * around it. */
void *warp_hip_stream(warp_hip_ctx *c);

/* Layer weights, copied to HBM once.
 * books: the layer's 3*stages codebooks as codebooks.bin stores them without
 * headers, [3][stages][entries][8] fp16 (gate, up, down), ids cb_base..;
 * fp16 subnormals are flushed to signed zero on upload (src/model.c:1277-1286).
 * Replaces the codebook load of src/model.c:1269-1304. */
int warp_hip_set_codebooks(warp_hip_ctx *c, int layer, int cb_base, const uint16_t *books);
/* F32 router [E][H] and optional e_score_correction_bias [E]
 * (block_sparse_moe.gate.weight / .e_score_correction_bias). */
int warp_hip_set_router(warp_hip_ctx *c, int layer, const float *w, const float *bias);
/* Quantised router: Q8G (bits 8), Q4G (4) or Q3G (3) rows as the trunk stores
 * them (src/model.c:601-625). */
int warp_hip_set_router_q(warp_hip_ctx *c, int layer, int bits, int group, const int8_t *q,
                          const uint16_t *scales, size_t rowbytes, const float *bias);
/* Shared expert (block_sparse_moe.shared_experts.{gate,up,down}_proj), quantised
 * trunk rows; inter_shared = moe_inter * n_shared. q/scales/rowbytes: gate, up, down.
 * Batches of 8 tokens or more run it on the matrix cores when every scale is finite
 * and below 256 in magnitude (checked here, on the host copies); otherwise, and for
 * Q3G, on the vector units. Both meet the same bar. */
int warp_hip_set_shared(warp_hip_ctx *c, int layer, int bits, int group, int inter_shared,
                        const int8_t *const q[3], const uint16_t *const scales[3],
                        const size_t rowbytes[3]);

/* The latent MoE of real K3 (src/model.c:2789-2795, 2913-2921), for a context
 * with cfg.latent: routed_expert_down_proj [latent][H] and
 * routed_expert_up_proj [H][latent] as quantised trunk rows (Q8G, Q4G or Q3G,
 * one bits/group for both), routed_expert_norm [latent] f32 (read when
 * cfg.latent_norm). The layer then routes on x, runs its experts on
 * down . x, combines them in the latent width, normalises, and adds up .
 * (that) to the shared expert's output. Expert records have the latent shape
 * (gate/up [inter][latent], down [latent][inter]). */
int warp_hip_set_latent(warp_hip_ctx *c, int layer, int bits, int group, const int8_t *down_q,
                        const uint16_t *down_s, size_t down_rowbytes, const int8_t *up_q, const uint16_t *up_s,
                        size_t up_rowbytes, const float *norm_w);

/* Expert records. put copies one record into the cache now (checked as
 * record_check does, src/model.c:1698-1745, plus the offsets the kernels
 * rely on). fetch is how misses are filled. */
int warp_hip_set_fetch(warp_hip_ctx *c, warp_hip_fetch_fn fetch, void *user);
/* Misses read in place from pinned host records instead (replaces a
 * fetch function set before, and is replaced by one set after). */
int warp_hip_set_fetch_host(warp_hip_ctx *c, warp_hip_fetch_host_fn fetch, void *user);
/* Pinned host memory the device copies from directly (hipHostMalloc), for
 * records kept on the host; NULL on failure. */
void *warp_hip_host_alloc(warp_hip_ctx *c, size_t bytes);
void warp_hip_host_free(warp_hip_ctx *c, void *p);
int warp_hip_put_expert(warp_hip_ctx *c, int layer, int expert, const uint8_t *rec);
/* Replaces waste_ecache_prefetch (src/ecache.h:160-164): speculative fills on
 * the copy stream; not counted as misses. */
int warp_hip_prefetch(warp_hip_ctx *c, int layer, const int *ids, int n);
void warp_hip_get_cache_stats(const warp_hip_ctx *c, warp_hip_cache_stats *st);

/* The certified router's arrays for one token of `layer` (sigmoid scores,
 * F32 router): out_dev [4][E] = point scores, point biased scores, and
 * lower and upper bounds of the biased score that the reference's
 * sequential logit gives (src/model.c:155-160, 2723-2726). For checking and
 * for callers that rank themselves; no counterpart in the reference. */
int warp_hip_router_cert(warp_hip_ctx *c, int layer, const float *x_dev, float *out_dev);

/* Certified selection's counters since open: decode routings certified,
 * how many of them recomputed rows, and the rows recomputed. Waits for the
 * context's stream. No counterpart in the reference (whose router is the
 * sequential sum itself). */
typedef struct {
    uint64_t certified, recomputed, rows;
} warp_hip_route_stats;
int warp_hip_get_route_stats(warp_hip_ctx *c, warp_hip_route_stats *st);

/* Replaces moe_layer (src/model.c:2713-2940) for one token: router, top-k,
 * K expert FFNs, combine in selection order, shared expert. x_dev, out_dev:
 * [H] f32; resid_dev (may be NULL) is added to out (the caller's residual).
 * idx/w (host, may be NULL) receive the selection; passing them costs a
 * device->host copy and a wait. Experts not resident are fetched. */
int warp_hip_moe_decode(warp_hip_ctx *c, int layer, const float *x_dev, float *out_dev,
                        const float *resid_dev, int *idx, float *w);
/* The same on host buffers: the drop-in for moe_layer's call site
 * (src/model.c:3929-3934). `routed` (may be NULL) gets the K ids. */
int warp_hip_moe_decode_host(warp_hip_ctx *c, int layer, const float *x, float *out, int *routed);

/* Replaces the per-expert part of moe_layer (src/model.c:2886-2909): one
 * resident expert's SwiGLU FFN on one token, out_dev [H] = W_down .
 * (act(W_gate x) * (W_up x)), unweighted, in the reference's arithmetic
 * (the gate and up tables of x, the gather apply, SiLU/SiTU, the down
 * table of h). No routing, no shared expert. E_MISSING if the record is not
 * resident. Queued on the compute stream; nothing waits. */
int warp_hip_expert_ffn(warp_hip_ctx *c, int layer, int expert, const float *x_dev, float *out_dev);

/* Replaces moe_chunk (src/model.c:3512-3693) for T <= max_tokens tokens:
 * per-token routing, pairs grouped by expert on the GPU, matrix-core
 * matvecs over tiles of up to 8 tokens per expert, per-token combine in
 * ascending expert id, shared expert. resid_dev ([T][H], may be NULL) is
 * added to out. route/rw (host, may be NULL) get [T][K]. With lookahead,
 * the next layer's experts predicted for each token are fetched while this
 * layer computes (the reference has no lookahead on this path). Returns
 * after the layer's work is queued without waiting for it when every record
 * of the layer is resident and route and rw are NULL (no pick can miss);
 * otherwise it waits and reports E_MISSING for a pick without a record. */
int warp_hip_moe_chunk(warp_hip_ctx *c, int layer, const float *X_dev, float *out_dev,
                       const float *resid_dev, int T, int *route, float *rw);
int warp_hip_moe_chunk_host(warp_hip_ctx *c, int layer, const float *X, float *out, int T,
                            int *route, float *rw);

/* ---- finer-grained entry points (device pointers) -------------------------- */

/* Replaces vq_matvec (src/model.c:2282-2289) on one matrix of one record:
 * kind 0 gate, 1 up, 2 down; rec_dev is a record in device memory; x_dev
 * [N] f32, y_dev [M] f32 with (M, N) = (inter, hidden) for gate/up and
 * (hidden, inter) for down. Uses the layer's codebooks. */
int warp_hip_vq_matvec(warp_hip_ctx *c, int layer, int kind, const uint8_t *rec_dev,
                       const float *x_dev, float *y_dev);
/* Decoded weights of one matrix, W_dev [M][N] f32, bit for bit the closed
 * form of docs/FORMAT.md:186-189 (stage sum in fp32 from stage 0, then the
 * subnormal-keeping row scale); the reference never materialises it. */
int warp_hip_decode_weights(warp_hip_ctx *c, int layer, int kind, const uint8_t *rec_dev,
                            float *W_dev);
/* Router logits of the layer for T tokens: logits_dev [T][E]
 * (matvec_t on the gate tensor, src/model.c:2721). */
int warp_hip_router_logits(warp_hip_ctx *c, int layer, const float *x_dev, int T,
                           float *logits_dev);
/* Scoring, top-k and weights (src/model.c:2720-2747) on given logits:
 * idx_dev/w_dev [T][K]. */
int warp_hip_route(warp_hip_ctx *c, int layer, const float *logits_dev, int T, int *idx_dev,
                   float *w_dev);
/* Quantised rows times f32 activations on the device (the mvq_rows_f32 slot's
 * arithmetic): y_dev [T][M]. */
int warp_hip_mvq(warp_hip_ctx *c, int bits, int group, const int8_t *q_dev,
                 const uint16_t *scales_dev, size_t rowbytes, const float *x_dev, int M, int N,
                 int T, float *y_dev);

/* Replaces waste_crc32 (src/crc32.c:176) for n bytes of device memory: zlib's
 * crc32, computed on the device (the payload checksum that cfg.verify takes
 * of every record entering the cache runs the same kernels). n <= 16 GiB.
 * Synchronous. */
int warp_hip_crc32(warp_hip_ctx *c, const void *p_dev, size_t n, uint32_t *crc);

/* Replaces waste_ecache_save_usage / waste_ecache_warm (src/ecache.c:730-816)
 * for the HBM cache: save writes the usage file of the reference's format
 * (waste_usage_hdr then one waste_usage_ent per resident record: layer,
 * expert, hit count, last use; src/waste_format.h:173-187); warm reads one,
 * sorts it by hits descending then (layer, expert), and fills the cache
 * through the fetch function with the hottest records until it is full,
 * seeding each slot's hit count from the file. Warming is best effort:
 * entries naming experts the context does not have, records that fail to
 * read or fail their checksum are skipped. Returns the records loaded or a
 * negative code (no fetch function, unreadable file). */
int warp_hip_save_usage(warp_hip_ctx *c, const char *path, uint64_t tokens);
int warp_hip_warm(warp_hip_ctx *c, const char *path);

/* Fill n bytes of device memory with deterministic noise (synthetic expert
 * data for benchmarks that cannot afford host generation). */
int warp_hip_fill_random(warp_hip_ctx *c, void *dev, size_t n, uint64_t seed);
/* Direct pointer to the cache slot holding (layer, expert), NULL if not
 * resident; and making a slot resident from bytes already in device memory. */
const uint8_t *warp_hip_resident(warp_hip_ctx *c, int layer, int expert);
int warp_hip_put_expert_dev(warp_hip_ctx *c, int layer, int expert, const uint8_t *rec_dev);
/* A resident record of synthetic content for benchmarks: a valid header for
 * the context's shape, codes drawn on the device from `seed`, the given row
 * scales ((2*inter + hidden) fp16, gate then up then down). */
int warp_hip_put_expert_synth(warp_hip_ctx *c, int layer, int expert, uint64_t seed,
                              const uint16_t *scales);
/* Expert matvec kernels for single-token decode (no counterpart in the
 * reference, which has one CPU path). AUTO (the default) runs the LUT
 * kernel -- the reference's LUT algorithm, fp32 tables in LDS -- for the
 * float-LUT formats when hidden and inter are multiples of 16, as gate/up,
 * down and combine launches; MFMA forces the decode-then-dot matrix-core
 * kernel that prefill always uses; LUT_FUSED runs the LUT kernel's gate/up,
 * down and combine as work items of one launch per layer where the token's
 * routing runs inside it (the same results bit for bit; slower than AUTO at
 * the K3 shape, where the waits between its work items cost more than the
 * launch boundaries they replace); GATHER forces the row kernel
 * (decode-then-dot, no tables: whole rows per wave, each lane decoding its
 * rows' weights from the kind's fp16 codebook staged in LDS), which AUTO
 * takes for one expert (warp_hip_expert_ffn, warp_hip_vq_matvec). Applies to
 * warp_hip_moe_decode*, warp_hip_expert_ffn and warp_hip_vq_matvec. */
enum { WARP_HIP_PATH_AUTO = 0, WARP_HIP_PATH_MFMA = 1, WARP_HIP_PATH_LUT_FUSED = 2, WARP_HIP_PATH_GATHER = 3 };
int warp_hip_set_matvec_path(warp_hip_ctx *c, int path);
/* cfg.router_fast after open: 1 decodes from the fast logits' picks without
 * certifying them, 0 certifies (the default). For measuring what the
 * certificate costs; no counterpart in the reference. */
int warp_hip_set_router_fast(warp_hip_ctx *c, int fast);
/* The certifying router's limit on polls for its rows (0: the default,
 * 65,536). A launch that reaches it gives up: that layer's outputs are NaN,
 * and the next synchronising call reports E_DEVICE and resets the router's
 * launch counter and tagged rows, so later launches certify as before. For
 * tests of that path; no counterpart in the reference. */
int warp_hip_set_cert_polls(warp_hip_ctx *c, unsigned polls);
/* The expert matvec kernel the current path runs for a decode of `layer`
 * (experts = 1: warp_hip_expert_ffn's single expert, else the layer's
 * top_k): "k_vq_lut", "k_vq_rows", "k_moe_fused", "k_vq_mfma" or "k_apply_p6". For
 * reports; never NULL. */
const char *warp_hip_matvec_kernel(warp_hip_ctx *c, int layer, int experts);
/* Per-launch timing with HIP events on the compute stream: when on, every
 * warp_hip_moe_decode brackets its launches of class 0 (gate/up expert
 * matvec), 1 (down expert matvec) and 2 (router logits). get returns the
 * summed milliseconds and launch counts per class since timing was turned
 * on (waiting for the events). */
int warp_hip_set_timing(warp_hip_ctx *c, int on);
int warp_hip_get_timing(warp_hip_ctx *c, double ms[4], uint64_t launches[4]);
/* Blocks until the context's streams are idle. */
int warp_hip_sync(warp_hip_ctx *c);

/* ---- the encoder (conversion time; no context) ----------------------------
 * Replaces waste_vq_encode (src/vq.c:96-103), same arguments, dim 8: X
 * [n][8], books [stages][entries][8] (entries <= 256), out [n][stages]; per
 * stage the nearest entry under squared L2 with unfused fp32 arithmetic in
 * dimension order, the first minimum winning, the residual feeding the next
 * stage; bit-identical codes. nthreads is ignored. Host buffers; returns 0
 * or a negative WARP_HIP_E_* code. */
int warp_hip_vq_encode(const float *X, int n, const float *books, int stages, int entries, int dim,
                       uint8_t *out, int nthreads);
/* The same with 16-bit codes and up to 4096 entries (the 12-bit format's
 * codebooks); no counterpart in the reference, whose codes are 8-bit. */
int warp_hip_vq_encode16(const float *X, long n, const float *books, int stages, int entries, int dim,
                         uint16_t *out);
/* The same on device buffers (16-byte aligned) on `stream` (a hipStream_t,
 * NULL for the null stream), for callers that keep the matrix in HBM;
 * resid_dev [n][8] is scratch for stages > 1. */
int warp_hip_vq_encode_dev(const float *X_dev, long n, const float *books_dev, int stages, int entries,
                           float *resid_dev, uint16_t *codes_dev, void *stream);
/* The same as warp_hip_vq_encode_dev without the resid_dev workspace, and
 * allocating nothing: no counterpart in the reference. For callers that
 * cannot allocate device memory (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc). The residuals between stages live
 * in a fixed device array of WARP_HIP_NOALLOC_MAX_VECTORS x 8 floats (16 MiB)
 * that each device keeps until the process ends; with stages > 1, n above
 * that maximum is refused with WARP_HIP_E_ARG (encode a larger matrix in
 * pieces). Every call on one device shares the array: calls that overlap on
 * one device (on two streams at once) race. Codes bit-identical to
 * warp_hip_vq_encode_dev's. */
#define WARP_HIP_NOALLOC_MAX_VECTORS (1L << 19)
int warp_hip_vq_encode_dev_noalloc(const float *X_dev, long n, const float *books_dev, int stages, int entries,
                                   uint16_t *codes_dev, void *stream);
/* Replaces waste_vq_lloyd (src/vq.c:109-136), same arguments, dim 8: one
 * iteration (assign, then each non-empty cluster's centroid = the mean of
 * its members summed in double in index order, bit-identical to the
 * reference); returns the number of non-empty clusters, or a negative
 * WARP_HIP_E_* code. entries <= 4096. */
int warp_hip_vq_lloyd(const float *X, int n, float *C, int entries, int dim, int nthreads);

#ifdef __cplusplus
}
#endif
#endif /* WARP_HIP_H */
