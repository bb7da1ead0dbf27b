/*
 * oracle.h — CPU restatement of the reference's routed-expert MoE path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the shipped library links, loads or
 * calls this code: it is the checker that the HIP path is compared against,
 * used by tests/, __graft_entry__.smoke() and the cpu_baseline leg of
 * bench.py, and nowhere else.
 *
 * Every function restates one reference function (file:line given at each
 * declaration) with the same arithmetic order, so that on x86-64 it is
 * bit-identical to the compiled reference with its own build flags
 * (model.c at -O2 -std=gnu11 without FMA; simd_avx512.c with AVX-512F,
 * where GCC contracts scalar a*b+c into an FMA). The build of this file
 * uses -ffp-contract=off and spells every fused multiply-add as fmaf().
 *
 * The 2-stage x 4096-entry, 12-bit-code format (OR_VQ12) has no
 * counterpart in the reference: the reference loader refuses entries > 256
 * (src/model.c:1172-1180). For it this file generalises the reference
 * algorithm in stage count, entry count and index width only.
 *
 * Pinning (how each function is checked, see tests/test_oracle_*.py):
 *  - f16 conversions, code packing, weight decode, LUT build, gather apply,
 *    VQ4P quantised apply, routing, mvq_rows_f32, the whole moe_layer and
 *    moe_chunk: golden vectors written by the compiled reference
 *    (oracle/_ref) on synthetic containers, compared bit for bit;
 *  - OR_VQ12 apply and decode: a brute-force float64 decode-then-dot on
 *    small shapes, plus an encode -> decode round trip through
 *    or_vq_encode, plus the bit-identity of VQ12 with VQ2R-style code
 *    packing when every code is < 256 (the reference runs that case);
 *  - crc32: zlib's published check value for "123456789".
 */
#ifndef WARP_ORACLE_H
#define WARP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Expert record formats: the reference's waste_fmt codes
 * (src/waste_format.h:41-71) plus one extension. */
enum {
    OR_VQ3R = 4,   /* 3 stages x 256, one byte per stage                   */
    OR_VQ2R = 5,   /* 2 stages x 256, one byte per stage                   */
    OR_VQ4P = 8,   /* 4 stages x 64, 4x6 bits packed in 3 bytes            */
    OR_VQ12 = 9,   /* extension: 2 stages x 4096, 2x12 bits in 3 bytes     */
};

#define OR_TILE 64          /* index_block: src/model.c:1937 (VQ_TILE)     */
#define OR_LUT_BLK 32       /* src/model.h:60 (WASTE_VQ_LUT_BLK)           */

/* ---- scalars ------------------------------------------------------------ */

/* waste_f16, subnormals kept (src/simd.h:49-67). */
float or_f16_keep(uint16_t h);
/* Codebook decode at load, subnormals flushed to signed zero
 * (src/model.c:1277-1286). */
float or_f16_flush(uint16_t h);
/* silu (src/model.c:501) and SiTU (src/model.c:505-509). */
float or_silu(float v);
float or_situ_pair(float g, float u, float beta, float lbeta);

/* ---- formats -------------------------------------------------------------- */

int or_fmt_stages(int fmt);
int or_fmt_entries(int fmt);
/* Bytes per (row, vector position) slot in the blocked index layout. */
int or_slot_bytes(int fmt);
/* Bytes of one [M x N] matrix's index block, rows padded to 64
 * (docs/FORMAT.md:194-201, tools/make_test_container.py:169-186). */
size_t or_index_bytes(int fmt, int M, int N);
/* codes: [stages][M * N/8] row-major per stage (code of row r, position v at
 * r*nv + v). Writes the blocked [M/64][nv][64][slot] layout; padding rows
 * stay zero. VQ4P packing follows docs/FORMAT.md:215-226; VQ12 packs the
 * little-endian 24-bit word s0 | s1 << 12. */
void or_pack_indices(int fmt, const uint16_t *codes, int M, int N, uint8_t *out);
/* Code of (row r, position v, stage s) from a blocked index block. */
unsigned or_code_at(int fmt, const uint8_t *idx, int N, int r, int v, int s);

/* ---- codebooks ------------------------------------------------------------ */

/* raw: n_books records of entries*vec_dim fp16 (headers stripped).
 * books: [n_books][entries][vec_dim] f32 (flushed); booksT: [n_books][vec_dim]
 * [entries] (src/model.c:1269-1304). Either output may be NULL. */
void or_books_decode(const uint16_t *raw, int n_books, int entries, int vec_dim,
                     float *books, float *booksT);

/* ---- the VQ matvec -------------------------------------------------------- */

/* Decoded weight, closed form (docs/FORMAT.md:186-189):
 * W[r][8v+d] = (C_0[i0][d] + C_1[i1][d] + ...) * f16_keep(scale[r]), the
 * stage sum in fp32 from stage 0 upwards. W is [M][N]. */
void or_decode_weights(int fmt, const uint8_t *idx, const uint16_t *scale,
                       const float *books, int cb_base, int M, int N, float *W);

/* lutb_range (src/model.c:1862-1901 portable, fused = 0;
 * src/simd_avx512.c:90-123 and src/simd_avx2.c:100-133, fused = 1):
 * lut[v][s][c] = sum_d x[8v+d] * CT[cb_base+s][d][c] for v in [lo, hi). */
void or_lutb_range(int lo, int hi, float *lut, const float *booksT, const float *x,
                   int cb_base, int stages, int entries, int vec_dim, int fused);

/* vq_rows over all M rows (src/model.c:1956-2024): for each row the stage
 * terms of a position are summed first, then added to the row accumulator
 * in ascending position order, then scaled. Generalised to any fmt whose
 * LUT is float (VQ3R, VQ2R, VQ12). */
void or_vq_apply(int fmt, float *y, const uint8_t *idx, const uint16_t *scale,
                 const float *lut, int M, int N);

/* vq_quant_range over the whole LUT (src/model.c:2048-2121): int8 table,
 * one scale per 32 positions, ties-to-even, clamp +-127. */
void or_vq_quant_lut(const float *lut, int nv, int st, int en, int8_t *q, float *qs);
/* vq_rows_p6 (src/model.c:2136-2229, the portable branch). */
void or_vq_apply_p6(float *y, const uint8_t *idx, const uint16_t *scale,
                    const int8_t *lut8, const float *lscale, int M, int N);

/* vq_matvec (src/model.c:2282-2289): LUT build then apply. Scratch sizes:
 * lut nv*S*E floats; for VQ4P also q8 (same count) and qs (nv/32+2). */
void or_vq_matvec(int fmt, float *y, const uint8_t *idx, const uint16_t *scale,
                  const float *x, const float *booksT, int cb_base, int M, int N,
                  int fused, float *lut, int8_t *q8, float *qs);

/* ---- dense pieces --------------------------------------------------------- */

/* dotf on x86 (src/model.c:155-160): sequential, unfused. */
float or_dotf(const float *a, const float *b, int n);
/* mvq_rows_f32: isa 0 = portable (src/model.c:265-320), 1 = AVX2
 * (src/simd_avx2.c:32-98), 2 = AVX-512 (src/simd_avx512.c:20-88). */
void or_mvq_rows_f32(int b, int e, float *y, const int8_t *W, const uint16_t *ws,
                     const float *x, int in, int ng, int group, int bits,
                     size_t rowbytes, int isa);
/* mmq_rows with T = 1 (src/model.c:3366-3398): the row is dequantised to
 * f32 first, then dotf. This is what moe_chunk's shared expert runs. */
void or_mmq_rows(int b, int e, float *y, const int8_t *W, const uint16_t *ws,
                 const float *x, int in, int ng, int group, int bits, size_t rowbytes);

/* ---- routing -------------------------------------------------------------- */

enum { OR_ROUTE_SIGMOID = 0, OR_ROUTE_SOFTMAX = 1 };

/* moe_layer scoring and selection (src/model.c:2720-2747): sigmoid scores,
 * top-k by score + bias with strict > (lowest index wins ties), weight =
 * unbiased score, optional renormalisation, times routed_scale.
 * OR_ROUTE_SOFTMAX is the extension: scores are a max-subtracted softmax
 * over all experts; selection and weights otherwise follow the same rules.
 * score_out (E floats) may be NULL. */
void or_route(const float *logits, const float *bias, int E, int K, int act,
              int renorm, float routed_scale, int *idx, float *w, float *score_out);

/* ---- the layer ------------------------------------------------------------ */

typedef struct {
    int fmt;
    int hidden, inter, n_experts, top_k;
    int renorm;               /* moe_renormalize present                  */
    float routed_scale;
    int router_act;           /* OR_ROUTE_*                               */
    int act_situ;             /* hidden_act == "situ"                     */
    float situ_beta, situ_lbeta;
    const float *booksT;      /* all books, [n_books][vd][E]              */
    const float *router;      /* [E][hidden] f32, or NULL if quantised    */
    const int8_t *router_q;   /* Q8G/Q4G router rows (router == NULL)     */
    const uint16_t *router_s;
    size_t router_rowbytes;
    int router_bits, router_group;
    const float *bias;        /* [E] or NULL                              */
    const uint8_t *const *recs;  /* [E] expert records (48-byte header)   */
    /* shared expert; sh_q[0] == NULL means none. kinds: gate, up, down    */
    const int8_t *sh_q[3];
    const uint16_t *sh_s[3];
    size_t sh_rowbytes[3];
    int sh_group, sh_bits, sh_inter;
    int fused_lutb;           /* 1: the AVX-512/AVX2 LUT build            */
    int mvq_isa;              /* which mvq_rows_f32 the host would run    */
    /* latent MoE (src/model.c:2789-2795, 2913-2921): latent > 0 runs the
     * experts on lat_q[0] . x (rows [latent][hidden]), then rmsnorm with
     * lat_norm (NULL: none) and eps, then lat_q[1] (rows [hidden][latent]) */
    int latent;
    const int8_t *lat_q[2];
    const uint16_t *lat_s[2];
    size_t lat_rowbytes[2];
    int lat_bits, lat_group;
    const float *lat_norm;
    float eps;
} or_layer;

/* One routed expert on one input (the body of the loop at
 * src/model.c:2874-2911): gate/up apply, activation, down matvec.
 * acc gets [hidden]; lut_gate/lut_up must have been built from x.
 * Scratch: ga, ub [inter]; lut_down, q8_down, qs_down as or_vq_matvec. */
void or_expert_ffn(const or_layer *L, const uint8_t *rec, const float *lut_gate,
                   const float *lut_up, const int8_t *q_gate, const float *qs_gate,
                   const int8_t *q_up, const float *qs_up, float *acc);

/* waste_rmsnorm (src/model.c:132-138): o = x * (1/sqrt(sum x^2 / n + eps)) * w. */
void or_rmsnorm(float *o, const float *x, const float *w, int n, float eps);

/* moe_layer (src/model.c:2713-2940), decode, with the latent projection when
 * L->latent.
 * logits (E floats) may be NULL. Returns 0, or -1 on allocation failure. */
int or_moe_layer(const or_layer *L, const float *in, float *out, int *idx,
                 float *w, float *logits);

/* moe_chunk (src/model.c:3512-3693) over nT tokens; route/rw get [nT][K]. */
int or_moe_chunk(const or_layer *L, const float *in, float *out, int nT,
                 int *route, float *rw);

/* ---- encoder, checksum, records ------------------------------------------ */

/* waste_vq_encode (src/vq.c:50-105), serial, generalised to uint16 codes:
 * out is [n][stages]. books is [stages][entries][dim]. */
void or_vq_encode(const float *X, int n, const float *books, int stages,
                  int entries, int dim, uint16_t *out);

/* zlib crc32 (src/crc32.c:176; record payload at src/model.c:1742-1744). */
uint32_t or_crc32(const uint8_t *p, size_t n);

/* Kimi Delta Attention step (src/kda.c:19-68): S [H][K][V] in place, o [H][V]. */
void or_kda_step(int H, int K, int V, const float *q, const float *k, const float *v, const float *g_log,
                 const float *beta, float *S, float *o);

/* expf_check.c: the device expf restatement against glibc's expf */
uint64_t or_expf_mismatches(uint32_t lo, uint64_t n, int nthreads, uint32_t *first);
void or_expf_array(const float *x, float *y, long n);
void or_sigmoid_array(const float *x, float *y, long n);

/* record_check (src/model.c:1698-1745). Returns 0 ok, 2 header, 3 crc.
 * index_bits 8, 6 or 12 (the last for the extension format). */
int or_record_check(const uint8_t *rec, size_t rec_bytes, int layer, int expert,
                    int index_bits, int stages, int n_books, const int expert_m[3],
                    int verify);

#ifdef __cplusplus
}
#endif
#endif /* WARP_ORACLE_H */
