/*
 * warp_internal.h — the interface between the C host backend (backend.c)
 * and the HIP kernels (kernels.hip). Not installed; include/warp_hip.h is
 * the public ABI.
 *
 * Device data the kernels read:
 *   - expert records, byte for byte as the container stores them: a 48-byte
 *     header, then the gate, up and down index blocks in the blocked
 *     [row_block=64][position][row_in_block][slot] layout, then one fp16 row
 *     scale per output row of each matrix;
 *   - per layer codebooks as fp16 [3 kinds][stages][entries][8], with fp16
 *     subnormals already flushed to signed zero (the reference flushes them
 *     when it loads codebooks.bin);
 *   - activations split for the fp16 matrix cores: a vector x of width N is
 *     stored as [N/8][2][8] fp16 (hi = fp16(x*2^k), lo = fp16(x*2^k - hi))
 *     with one float 2^-k per vector, so that the products on the matrix
 *     cores are exact and the sum keeps about 22 bits of x.
 */
#ifndef WARP_INTERNAL_H
#define WARP_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Formats (the reference's waste_fmt codes plus the 12-bit extension). */
#define WARP_FMT_VQ3R 4
#define WARP_FMT_VQ2R 5
#define WARP_FMT_VQ4P 8
#define WARP_FMT_VQ12 9

#define WARP_TILE 64          /* index_block of the container format     */
#define WARP_LUT_BLK 32       /* positions per int8 LUT scale (VQ4P)     */
#define WARP_TPJ 8            /* token slots per matvec job              */
#define WARP_RUN_J 4          /* jobs of one expert per prefill run      */
#define WARP_MAX_K 64         /* top-k bound (the reference's cfg_sane)  */

/* One matvec job: one matrix (kind) of one expert record against up to
 * WARP_TPJ input vectors. idx/scale point at that matrix's index block and
 * row scales inside the record; xi[t] indexes the split inputs, yi[t] the
 * output rows block ([y_index][M]). The list a job sits in gives its kind. */
typedef struct {
    const uint8_t *idx;
    const uint16_t *scale;
    int n;                    /* token slots in use, 1..WARP_TPJ         */
    int rsv;
    int xi[WARP_TPJ];
    int yi[WARP_TPJ];
} warp_job;

/* One expert of the device-side expert table: where its record sits in the
 * HBM cache (NULL when it is not resident) and the header's byte offsets of
 * the gate, up and down index blocks and of the row scales, copied from the
 * header when the record is placed, so that routing needs no dependent
 * reads of the record itself. */
typedef struct {
    const uint8_t *rec;
    uint32_t off[4];
} warp_slot;

/* Byte offsets of the header fields the kernels read (waste_expert_hdr). */
#define WARP_HDR_GATE_OFF 20
#define WARP_HDR_UP_OFF 24
#define WARP_HDR_DOWN_OFF 28
#define WARP_HDR_CORR_OFF 32
#define WARP_HDR_CRC_OFF 36
#define WARP_HDR_BYTES 48

/* Every launcher returns 0 or a negative hipError_t-derived code, and
 * launches on `stream` (a hipStream_t). */

/* x [T][N] f32 -> xs [T][N/8][2][8] fp16, xscale [T]. */
int wk_split(const float *x, int T, int N, uint16_t *xs, float *xscale, void *stream);

/* Batched quantised rows on the matrix cores (Q8G and Q4G with groups of a
 * multiple of 32, N a multiple of the group, every scale finite and below
 * 256 in magnitude, which the caller checks): y_k [T][M] = dequant(W_k) . x
 * for nmat (1 or 2) matrices of one shape sharing x, x given split as
 * [T][N/8][2][8] fp16 with xscale [T] (wk_split). Returns -1 for shapes it
 * does not take (the caller uses wk_mvq). */
int wk_mvq_gemm(int nmat, const int8_t *const *W, const uint16_t *const *ws, const size_t *rowbytes, int group,
                int bits, const uint16_t *xs, const float *xscale, int M, int N, int T, float *const *y,
                void *stream);

/* Router logits [T][E] = W [E][H] . x [T][H]. strict = 1 reproduces the
 * reference's sequential, unfused fp32 sum (dotf on x86); 0 is a parallel
 * fixed-order tree, or for batches of WARP_ROUTER_MFMA_T tokens or more
 * (H a multiple of 16) a fixed order of fp32 matrix-core steps. */
#define WARP_ROUTER_MFMA_T 16
int wk_router_logits(const float *W, const float *x, int E, int H, int T, int strict,
                     float *logits, void *stream);
/* One token's router rows with the fast sum, then its sigmoid scores
 * out[0..E) and biased scores out[E..2E) (score + bias, bias may be NULL), as
 * the routing computes them: the input of warp_route_args with scored = 1. */
int wk_router_scored(const float *W, const float *x, int E, int H, const float *bias, float *out, void *stream);
/* Certified routing inputs of one token (sigmoid scores, fp32 router): out
 * [4][E] = point scores, point biased scores, and the lower and upper bounds
 * of the biased score the reference's sequential logit gives. H % 4 == 0,
 * H <= 16384. sync (WK_CERT_SYNC_WORDS(E) words, 8-byte aligned, zeroed
 * before the first launch and kept between launches; or NULL): the
 * last block also certifies the top-K selection and rewrites the rows whose
 * order the bounds leave open with their exact (sequential) values, so that
 * a routing from [0, 2E) (scored = 1) picks the reference's experts in its
 * order; cctr as in warp_route_args; flag (or NULL): bit 2 (value 4) set
 * when the last block's wait for the rows gives up, after polls polls (0:
 * 65,536). E <= 4096 with sync.
 * pick (with sync, or NULL): the last block also writes what wk_route
 * writes from those arrays -- pick->idx and pick->w (renorm, routed_scale),
 * and with pick->table the job lists (pick->jobs, njobs, inter; a pick
 * without a record sets *flag; a wait that gave up leaves them empty) --
 * so that no routing launch follows. */
struct warp_route_args_s;
#define WK_CERT_SYNC_WORDS(E) (2 + 8 * (size_t)(E))  /* a launch counter, then [E][4] 64-bit tagged values */
int wk_router_cert(const float *W, const float *x, int E, int H, const float *bias, float *out, unsigned *sync,
                   int K, unsigned long long *cctr, int *flag, const struct warp_route_args_s *pick, unsigned polls,
                   void *stream);

/* Quantised router / dense trunk rows (Q8G, Q4G, Q3G with the reference's
 * packing): y [T][M] = dequant(W) [M][N] . x [T][N]. */
int wk_mvq(const int8_t *W, const uint16_t *ws, size_t rowbytes, int group, int bits,
           const float *x, int M, int N, int T, float *y, void *stream);

/* The encoder (waste_vq_encode for 8-dim vectors): one launch per stage; codes
 * [n][stages] 16-bit; cur [n][8] holds the residual between stages (unused
 * for one stage). X, books and cur 16-byte aligned; entries <= 4096. */
int wk_vq_encode(const float *X, long n, const float *books, int stages, int entries, float *cur,
                 uint16_t *codes, void *stream);
/* One Lloyd iteration (waste_vq_lloyd) on device buffers: assignment into asg,
 * the new centroids into C (empty clusters keep theirs), the number of
 * non-empty clusters into *live. Scratch: counts [ceil(n/4096)][entries],
 * total, base [entries], sorted [n]. dim 8. */
int wk_vq_lloyd(const float *X, long n, float *C, int entries, int dim, uint16_t *asg, int *counts, int *total,
                int *base, int *sorted, int *live, void *stream);

/* A layer's shared expert for one decode token, folded into the router and
 * combine launches: h = act(gate . x, up . x), then down . h. */
typedef struct {
    const int8_t *q[3];         /* gate, up, down rows (Q8G or Q4G)    */
    const uint16_t *s[3];       /* their fp16 group scales, [rows][N/group] */
    size_t rowbytes[3];
    int bits, group, inter;
    int situ;
    float beta, lbeta;
    float *h;                   /* [inter]                             */
} warp_shared_args;
/* Whether the fused kernels take this shape: bits 8 or 4, 16-byte rows,
 * a group a multiple of one 16-byte chunk's weights, rows short enough. */
int wk_shared_fast_ok(int H, const warp_shared_args *sa);
/* Router logits [E] of one token (the fast fixed-order tree) and, in the
 * same launch, the shared expert's h. */
int wk_router_shared(const float *W, const float *x, int E, int H, float *logits, const warp_shared_args *sa,
                     void *stream);

/* Routing for T tokens: scores, top-k by score + bias (strict >, lowest
 * index wins), weights, renorm, scale. When `table` is not NULL (decode,
 * T == 1) it also writes the decode job lists: jobs[0..K) gate, [K..2K) up,
 * [2K..3K) down, and njobs[3] = {K, K, K}, or {0, 0, 0} plus *missing = 1
 * when a selected expert has no resident record. */
int wk_route(const float *logits, const float *bias, int E, int K, int T, int act,
             int renorm, float routed_scale, int *idx, float *w,
             const warp_slot *table, warp_job *jobs, int *njobs, int *missing,
             int inter, void *stream);

/* The MFMA decode-then-dot matvec over a job list, one launch per group of
 * kinds: kind_lo..kind_lo+nkinds-1. jobs[k] / njobs[k] are the lists of
 * kind kind_lo + k, at most max_jobs each. books: the layer's fp16 codebooks.
 * y[k] gets the outputs of kind kind_lo + k: [y_index][M]. The output is
 * the full matvec, scaled by the row scale and the input's xscale. */
int wk_vq_matvec(int fmt, const warp_job *jobs, const int *njobs, int max_jobs,
                 int kind_lo, int nkinds, const uint16_t *books, const uint16_t *xs,
                 const float *xscale, float *const *y, int M, int N, int tokens_per_job,
                 void *stream);
/* The same for prefill by runs: runs[0..njobs[3]) = (first job << 3) | jobs,
 * up to WARP_RUN_J consecutive jobs of one expert (wk_plan_chunk writes
 * them); each run's records are decoded once for all its jobs.
 * fp16_rows = 0: exact products, xs/xscale as for wk_vq_matvec (rows by
 * xi). fp16_rows > 0: the reduced-precision products (stage vectors added
 * in fp16, x's fp16 high half), xs [N/32][fp16_rows][32] and xscale
 * [fp16_rows] by pair slot (yi), from wk_split_pgm.
 * queue: WARP_RUNQ_WORDS words, zero before the first launch; the launch
 * hands units out through it (a ticket and a waves-done counter per kind
 * and XCD) and leaves it zero (launches on one queue must not overlap). */
#define WARP_RUNQ_WORDS 1536
int wk_vq_runs(int fmt, const warp_job *jobs, const int *njobs, int max_jobs, const int *runs,
               int kind_lo, int nkinds, const uint16_t *books, const uint16_t *xs, const float *xscale,
               float *const *y, int M, int N, int fp16_rows, unsigned *queue, void *stream);
/* Inputs of the reduced-precision products: rows p < *nrows of
 * act(g, u) (act = 1, pair rows; SiLU with the hardware exp, SiTU exact)
 * or of x row rowmap[p] (act = 0, u NULL),
 * each scaled by a power of two (2^-k to xscale[p]) and rounded to fp16,
 * into xs [N/32][P][32]. N % 32 == 0, pointers 16-byte aligned. */
int wk_split_pgm(const float *g, const float *u, const int *rowmap, const int *nrows, int P, int N,
                 int act, int act_situ, float beta, float lbeta, uint16_t *xs, float *xscale,
                 void *stream);
/* The x rows of the same, walked by pair in token order: pair q = t K + k
 * takes x row t to its slot tok_slots[q] (the grouping's slots; -1: not
 * computed), so a token's pairs run in neighbouring blocks and its row is
 * fetched by few XCDs. The values of wk_split_pgm with rowmap = pair_tok,
 * into xs [N/32][T K][32] and xscale [T K]. N <= 4096, else -1. */
int wk_split_pgm_pairs(const float *x, const int *tok_slots, int T, int K, int N, uint16_t *xs, float *xscale,
                       void *stream);

/* The LUT matvec (decode, one input per job): for each kind
 * kind_lo..kind_lo+nkinds-1, every job's rows against the f32 input
 * x + xi[0] * N, as per-split partial sums part[kind - kind_lo][split]
 * [job][nrb * 64]. books: the layer's fp16 codebooks (flushed);
 * books_x31 = 1 when they hold exponent-31 values, which the reference
 * converts to finite floats (a slower exact conversion). shared_x = 1 when all
 * jobs of a list read the same input (row groups then span jobs).
 * cap_floats bounds part; target_blocks is the CU count. *splits_out gets
 * the split count the consumers must be given. N % 16 == 0. */
int wk_lut_plan(int M, int N, int max_jobs, int nkinds, int shared_x, int target_blocks,
                size_t cap_floats, int *groups_out, int *splits_out);
/* Routing done inside the gate/up launch of a decode step (see wk_vq_lut):
 * the arguments of wk_route with a table, for one token. scored = 1: logits
 * holds the sigmoid scores [E] and the biased scores [E] (wk_router_scored),
 * not the logits. scored = 2 (certified selection): logits holds the four
 * arrays of wk_router_cert, and cw [E][ch] / cx [ch] are the router rows
 * and the token's input the routing recomputes ambiguous logits from
 * (sequentially, as the reference sums); cctr (or NULL) [2] counts the
 * routings that recomputed and the rows recomputed. */
typedef struct warp_route_args_s {
    const float *logits, *bias;
    const warp_slot *table;
    int E, act, renorm, inter;
    float routed_scale;
    int *idx;
    float *w;
    warp_job *jobs;           /* written: the lists of all three kinds */
    int *njobs, *missing;
    int scored;
    const float *cw, *cx;
    int ch;
    unsigned long long *cctr;
} warp_route_args;
int wk_vq_lut(int fmt, const warp_job *jobs, const int *njobs, int max_jobs, int kind_lo,
              int nkinds, const uint16_t *books, int books_x31, const float *x, int shared_x, float *part,
              size_t cap_floats, int M, int N, int target_blocks, const float *act_part,
              int act_splits, int act_situ, float act_beta, float act_lbeta,
              const warp_route_args *route, const warp_shared_args *sh, float *sh_out, int *splits_out,
              void *stream);
/* (sh, with route: one more grid row of blocks computes the shared
 * expert's h = act(gate . x, up . x) into sh->h, as wk_router_shared does,
 * one row per wave; the launch must have as many waves per row as the
 * shared expert has rows, else -1. sh with sh_out, on a down launch
 * (act_part): M / 64 blocks appended to the plan's (which gets that many
 * fewer) compute the shared expert's down rows sh_out [M] = down . sh->h,
 * as wk_combine_lut does with its sa. NULL otherwise.
 * act_part: the down launch makes each job's input itself, h = act(gate,
 * up) from the gate/up partial sums -- kinds 0 and 1 of the previous launch
 * with act_splits splits -- instead of reading x; NULL otherwise.
 * route: the gate/up launch (kinds 0 and 1, shared input x) also routes the
 * token, K = max_jobs picks, as wk_route would with the table, instead of
 * reading jobs/njobs; route->jobs/njobs/idx/w/missing get what wk_route
 * writes. Only where wk_lut_route_ok says so; NULL otherwise.) */
int wk_lut_route_ok(int fmt, int E, int K, int shared_x, int kind_lo, int nkinds);
/* Expert matvecs by whole rows per wave, the kind's codebook staged in LDS
 * (or, at most 16 KiB, read through L1): jobs/njobs (max_jobs per kind, one
 * input each: x shared, or act inputs), or slot (one expert's expert-table
 * entry, inter giving the scale arrays' places; a missing record sets
 * *missing and its rows to NaN). y[kind] [max_jobs][M] = the rows times
 * their scales, for kinds kind_lo .. kind_lo + nkinds - 1; x NULL (kind 2
 * only): job j's inputs are act(y[0], y[1]) at j N. part (kind 2 only, or
 * NULL): the rows unscaled at part + j (M rounded up to 64) instead, the
 * table kernel's one-split partial sums that wk_combine_lut reads. About
 * target_blocks blocks; N % 32 == 0. */
int wk_vq_rows(int fmt, const warp_job *jobs, const int *njobs, int max_jobs, int kind_lo, int nkinds,
               const uint16_t *books, const float *x, int M, int N, const warp_slot *slot, int inter, int act_situ,
               float act_beta, float act_lbeta, float *const *y, float *part, int *missing, int target_blocks,
               void *stream);
/* Certified routing of one decode token (route->scored == 2, sigmoid): what
 * wk_route writes, with route->table (or NULL) for the job lists, from
 * wk_router_cert's arrays; ambiguous rows recomputed from cw / cx. E <= 4096. */
int wk_route_cert(const warp_route_args *route, int K, void *stream);
/* One decode step of a layer in one launch (the table kernel's gate/up
 * units with the routing, its down units, the combine), bit for bit what
 * wk_vq_lut (gate/up, routed), wk_vq_lut (down, act) and wk_combine_lut
 * give: out [H] = sum_j w_j y_j + add0 + add1, NaN when a pick has no
 * record (the missing flag as wk_route sets it). route as for wk_vq_lut;
 * part and cap_floats hold both launches' partial sums. sync: WARP_FZ_WORDS
 * zeroed words the launch leaves zeroed; a wait that exceeds its poll limit
 * sets bit 2 (value 4) of route->missing. Only where wk_lut_route_ok holds. */
#define WARP_FZ_WORDS 16384
int wk_moe_fused(int fmt, const uint16_t *books, int books_x31, const float *x, int K, int I, int H,
                 float *part, size_t cap_floats, int n_cu, int act_situ, float act_beta,
                 float act_lbeta, const warp_route_args *route, const float *add0, const float *add1,
                 float *out, unsigned *sync, int sync_words, void *stream);
/* y[k][yi][r] = (sum over splits) * row scale, for the kinds of one LUT launch. */
int wk_lut_reduce(const warp_job *jobs, const int *njobs, int max_jobs, int kind_lo, int nkinds,
                  const float *part, int splits, int M, float *const *y, void *stream);
/* Decode: down partials -> out [H] = sum_j w[j] * y_j in j order, + add0 + add1;
 * NaN everywhere when *missing is set. jobs2: the down job list. With `sa`
 * (add0 NULL), add0 is the shared expert's down . sa->h, computed here. */
int wk_combine_lut(const warp_job *jobs2, const float *part, int splits, int max_jobs,
                   const float *w, int K, int H, const float *add0, const float *add1,
                   const int *missing, const warp_shared_args *sa, float *out, void *stream);

/* Decoded weights of one matrix, bit for bit the reference's closed form
 * (stage sum in fp32 from stage 0, then times the subnormal-keeping fp16
 * row scale). books: fp16 [stages][entries][8] of this kind. W [M][N]. */
int wk_decode_weights(int fmt, const uint8_t *idx, const uint16_t *scale,
                      const uint16_t *books, int M, int N, float *W, void *stream);

/* h = act(g, u) per pair, then split: g, u [P][I] -> xs [P][I/8][2][8],
 * xscale [P]; h_out (may be NULL) gets h in f32. act_situ selects SiTU. */
int wk_act_split(const float *g, const float *u, int P, int I, int act_situ,
                 float beta, float lbeta, uint16_t *xs, float *xscale, float *h_out,
                 void *stream);

/* out [H] = sum_j w[j] * y[j][H] in j order (unfused, as the reference's
 * combine), then + add0[H] and + add1[H] when given; NaN everywhere when
 * *missing is set (a selected expert was not computed). */
int wk_combine(const float *y, const float *w, int K, int H, const float *add0,
               const float *add1, const int *missing, float *out, void *stream);

/* VQ4P: int8 LUT of x for one kind (4 stages x 64 entries, one scale per 32
 * positions), bit-identical to the reference's fused LUT build and
 * quantisation. x [V][N] f32 -> lut8 [V][N/8][4][64], lscale [V][nblk]. */
int wk_lut_p6(const float *x, int V, int N, const uint16_t *books_kind, int8_t *lut8,
              float *lscale, void *stream);
/* VQ4P apply over a job list of one kind: y[yi] = apply(rec kind, lut8[xi]). */
int wk_apply_p6(const warp_job *jobs, const int *njobs, int max_jobs, int kind,
                const int8_t *lut8, const float *lscale, float *y, int M, int N,
                void *stream);
/* silu/SiTU pairs for VQ4P: h [P][I] = act(g, u), exactly as the reference. */
int wk_act(const float *g, const float *u, int P, int I, int act_situ, float beta,
           float lbeta, float *h, void *stream);

/* Prefill: token-to-expert grouping on the GPU. From route idx/w [T][K]:
 * counts per expert, exclusive scan, pairs sorted by (expert, token) into
 * pair_tok/pair_exp/pair_w [T*K], and tok_slots [T][K]: each token's pair
 * slots in ascending expert id; gate/up jobs (tiles of WARP_TPJ tokens of
 * one expert; xi = token, yi = pair slot) and down jobs (xi = yi = pair
 * slot) written to jobs[kind*max_jobs ..], counts to njobs[0..3); the runs
 * of up to WARP_RUN_J jobs of one expert to runs, their count to njobs[3].
 * *missing is written every call: 1 when a pair's expert has no resident
 * record, 2 when the jobs exceed max_jobs, else 0 (with or_missing, only a
 * nonzero value is written). Jobs and runs are made for the experts
 * e_lo..e_hi only (a window of a chunk whose experts do not fit the cache
 * at once); every pair gets its place and slot either way, so the windows
 * of one chunk fill disjoint pair rows of one layout. */
int wk_plan_chunk(const int *idx, const float *w, int T, int K, int E,
                  const warp_slot *table, int *counts, int *offsets, int *pair_tok,
                  int *pair_exp, float *pair_w, int *tok_slots, warp_job *jobs,
                  int max_jobs, int *njobs, int *runs, int *missing, int inter,
                  int e_lo, int e_hi, int or_missing, void *stream);
/* out [T][H] = per token, sum over its pairs in ascending expert id (tok_slots)
 * of w * y[pair], then + add0 [T][H] when given. */
int wk_combine_chunk(const float *y, const int *tok_slots, const float *pair_w, int T, int K, int H,
                     const float *add0, const float *add1, float *out, void *stream);

/* The latent MoE's tail: RMS norm per token of [T][n] (o may be x), and
 * out = (y + a0) + a1 over n floats (a0, a1 may be NULL). */
int wk_rmsnorm(const float *x, const float *w, int T, int n, float eps, float *o, void *stream);
int wk_add3(const float *y, const float *a0, const float *a1, size_t n, float *out, void *stream);

/* The single-expert FFN's jobs from one device table entry: jobs[0..2] =
 * gate, up, down (list stride 1, input 0, output 0), njobs = {1, 1, 1, 0},
 * w[0] = 1; a missing record gives empty lists and sets *missing. */
int wk_expert_jobs(const warp_slot *entry, int inter, warp_job *jobs, int *njobs, float *w, int *missing,
                   void *stream);

/* Synthetic device data for benchmarks: fill n bytes with a counter-based
 * hash of (seed, offset). */
int wk_fill_random(uint8_t *p, size_t n, uint64_t seed, void *stream);

/* A batch of expert-table updates, each key at most once: table[key] = v.
 * checked = 1: the record was checksummed on the device (wk_crc32 with this
 * key); if crc_bad[key] is set, the entry becomes NULL (not resident) and the
 * key is appended to err (the first WARP_CRC_ERR_KEYS keys; n counts every
 * failure). checked = 0 clears crc_bad[key], so that after the launch
 * crc_bad[key] is 1 exactly for the keys whose last update was refused (the
 * complete list when more than WARP_CRC_ERR_KEYS were). */
typedef struct {
    warp_slot v;
    int key;
    int checked;
} warp_slot_upd;
#define WARP_CRC_ERR_KEYS 255
typedef struct {
    int n;
    int keys[WARP_CRC_ERR_KEYS];
} warp_crc_err;
int wk_set_slots(warp_slot *table, const warp_slot_upd *u, int n, int8_t *crc_bad, warp_crc_err *err,
                 void *stream);

/* zlib's crc32 of p[0, n) in device memory (crc.hip). tmp holds
 * wk_crc32_tmp_words(n) words. key < 0: the checksum to *out (device);
 * key >= 0: bad[key] = (checksum != *expect), both in device memory. */
size_t wk_crc32_tmp_words(size_t n);
int wk_crc32(const uint8_t *p, size_t n, uint32_t *tmp, uint32_t *out, const uint32_t *expect, int key,
             int8_t *bad, void *stream);

/* T steps of the Kimi Delta Attention recurrence (kda.hip), one block per
 * head, state S [H][K][V] in place: inputs of step t at q/k/g + t*H*K,
 * v + t*H*V, beta + t*H, output o + t*H*V. K <= 256, V <= 1024, K*V*4 <=
 * 150 KiB. */
int wk_kda(int T, int H, int K, int V, const float *q, const float *k, const float *v, const float *g,
           const float *beta, float *S, float *o, void *stream);

/* Device properties the host needs: returns the gfx name into buf. */
int wk_device_arch(int device, char *buf, int n);

/* Drops the MoE table slots' device state (moe_table.c). */
void warp_moe_release(void);

#ifdef __cplusplus
}
#endif
#endif /* WARP_INTERNAL_H */
