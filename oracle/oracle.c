/*
 * oracle.c — CPU restatement of the reference's routed-expert MoE path.
 * TEST INFRASTRUCTURE ONLY: see oracle.h for what uses it and how each
 * function is pinned. Build with -ffp-contract=off (oracle/Makefile).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- scalars ------------------------------------------------------------- */

/* src/simd.h:49-67: exponent 0 is mantissa * 2^-24 (kept, not flushed); any
 * other exponent, 31 included, is rebiased as a normal number. */
float or_f16_keep(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1f, mn = h & 0x3ff;
    if (e == 0) {
        float f = (float)mn * 5.9604644775390625e-08f;
        return sign ? -f : f;
    }
    const uint32_t bits = sign | ((e + 112u) << 23) | (mn << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* src/model.c:1277-1286: exponent 0 keeps the sign and nothing else. */
float or_f16_flush(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1f, mn = h & 0x3ff;
    const uint32_t bits = e ? (sign | ((e + 112u) << 23) | (mn << 13)) : sign;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

float or_silu(float v) { return v / (1.0f + expf(-v)); }

float or_situ_pair(float g, float u, float beta, float lbeta)
{
    const float a = beta * tanhf(g / beta) / (1.0f + expf(-g));
    return a * (lbeta > 0.0f ? lbeta * tanhf(u / lbeta) : u);
}

/* ---- formats --------------------------------------------------------------- */

int or_fmt_stages(int fmt)
{
    switch (fmt) {
    case OR_VQ3R: return 3;
    case OR_VQ2R: return 2;
    case OR_VQ4P: return 4;
    case OR_VQ12: return 2;
    }
    return 0;
}

int or_fmt_entries(int fmt)
{
    switch (fmt) {
    case OR_VQ3R: case OR_VQ2R: return 256;
    case OR_VQ4P: return 64;
    case OR_VQ12: return 4096;
    }
    return 0;
}

int or_slot_bytes(int fmt)
{
    switch (fmt) {
    case OR_VQ3R: return 3;
    case OR_VQ2R: return 2;
    case OR_VQ4P: return 3;
    case OR_VQ12: return 3;
    }
    return 0;
}

size_t or_index_bytes(int fmt, int M, int N)
{
    const size_t nb = ((size_t)M + OR_TILE - 1) / OR_TILE;
    return nb * (size_t)(N / 8) * OR_TILE * (size_t)or_slot_bytes(fmt);
}

static void put_slot(int fmt, uint8_t *p, const unsigned *c)
{
    switch (fmt) {
    case OR_VQ3R: p[0] = (uint8_t)c[0]; p[1] = (uint8_t)c[1]; p[2] = (uint8_t)c[2]; break;
    case OR_VQ2R: p[0] = (uint8_t)c[0]; p[1] = (uint8_t)c[1]; break;
    case OR_VQ4P:
        /* docs/FORMAT.md:218-221 */
        p[0] = (uint8_t)((c[0] & 0x3f) | (c[1] << 6));
        p[1] = (uint8_t)(((c[1] & 0x3f) >> 2) | (c[2] << 4));
        p[2] = (uint8_t)(((c[2] & 0x3f) >> 4) | (c[3] << 2));
        break;
    case OR_VQ12: {
        const uint32_t w = (c[0] & 0xfff) | ((c[1] & 0xfff) << 12);
        p[0] = (uint8_t)w; p[1] = (uint8_t)(w >> 8); p[2] = (uint8_t)(w >> 16);
        break;
    }
    }
}

static unsigned get_code(int fmt, const uint8_t *p, int s)
{
    switch (fmt) {
    case OR_VQ3R: case OR_VQ2R: return p[s];
    case OR_VQ4P: {
        /* P6_J0..P6_J3, src/model.c:2131-2134 */
        const unsigned b0 = p[0], b1 = p[1], b2 = p[2];
        switch (s) {
        case 0: return b0 & 0x3f;
        case 1: return ((b0 >> 6) | (b1 << 2)) & 0x3f;
        case 2: return ((b1 >> 4) | (b2 << 4)) & 0x3f;
        default: return (b2 >> 2) & 0x3f;
        }
    }
    case OR_VQ12: {
        const uint32_t w = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16);
        return s == 0 ? (w & 0xfff) : (w >> 12);
    }
    }
    return 0;
}

static const uint8_t *slot_ptr(int fmt, const uint8_t *idx, int N, int r, int v)
{
    const int nv = N / 8, sb = or_slot_bytes(fmt);
    return idx + (((size_t)(r / OR_TILE) * nv + v) * OR_TILE + (size_t)(r % OR_TILE)) * sb;
}

void or_pack_indices(int fmt, const uint16_t *codes, int M, int N, uint8_t *out)
{
    const int nv = N / 8, S = or_fmt_stages(fmt);
    memset(out, 0, or_index_bytes(fmt, M, N));
    for (int r = 0; r < M; r++)
        for (int v = 0; v < nv; v++) {
            unsigned c[4] = {0, 0, 0, 0};
            for (int s = 0; s < S; s++) c[s] = codes[(size_t)s * M * nv + (size_t)r * nv + v];
            put_slot(fmt, (uint8_t *)slot_ptr(fmt, out, N, r, v), c);
        }
}

unsigned or_code_at(int fmt, const uint8_t *idx, int N, int r, int v, int s)
{
    return get_code(fmt, slot_ptr(fmt, idx, N, r, v), s);
}

/* ---- codebooks --------------------------------------------------------------- */

void or_books_decode(const uint16_t *raw, int n_books, int entries, int vec_dim,
                     float *books, float *booksT)
{
    const size_t per = (size_t)entries * vec_dim;
    for (int b = 0; b < n_books; b++)
        for (int c = 0; c < entries; c++)
            for (int d = 0; d < vec_dim; d++) {
                const float f = or_f16_flush(raw[(size_t)b * per + (size_t)c * vec_dim + d]);
                if (books) books[(size_t)b * per + (size_t)c * vec_dim + d] = f;
                if (booksT) booksT[(size_t)b * per + (size_t)d * entries + c] = f;
            }
}

/* ---- the VQ matvec ------------------------------------------------------------ */

void or_decode_weights(int fmt, const uint8_t *idx, const uint16_t *scale,
                       const float *books, int cb_base, int M, int N, float *W)
{
    const int nv = N / 8, S = or_fmt_stages(fmt), E = or_fmt_entries(fmt);
    for (int r = 0; r < M; r++) {
        const float sr = or_f16_keep(scale[r]);
        for (int v = 0; v < nv; v++) {
            const uint8_t *p = slot_ptr(fmt, idx, N, r, v);
            for (int d = 0; d < 8; d++) {
                float t = books[((size_t)(cb_base + 0) * E + get_code(fmt, p, 0)) * 8 + d];
                for (int s = 1; s < S; s++)
                    t += books[((size_t)(cb_base + s) * E + get_code(fmt, p, s)) * 8 + d];
                W[(size_t)r * N + 8 * v + d] = t * sr;
            }
        }
    }
}

void or_lutb_range(int lo, int hi, float *lut, const float *booksT, const float *x,
                   int cb_base, int stages, int entries, int vec_dim, int fused)
{
    const int en = entries, vd = vec_dim, st = stages;
    for (int v = lo; v < hi; v++) {
        const float *xv = x + (size_t)v * vd;
        for (int s = 0; s < st; s++) {
            const float *CT = booksT + (size_t)(cb_base + s) * en * vd;
            float *dst = lut + ((size_t)v * st + s) * en;
            for (int c = 0; c < en; c++) {
                float t = 0.0f;
                if (fused) {
                    /* one fmadd lane per entry, d ascending, from zero; the
                     * scalar tail of those units is contracted the same way */
                    for (int d = 0; d < vd; d++) t = fmaf(xv[d], CT[(size_t)d * en + c], t);
                } else {
                    for (int d = 0; d < vd; d++) t += xv[d] * CT[(size_t)d * en + c];
                }
                dst[c] = t;
            }
        }
    }
}

void or_vq_apply(int fmt, float *y, const uint8_t *idx, const uint16_t *scale,
                 const float *lut, int M, int N)
{
    const int nv = N / 8, S = or_fmt_stages(fmt), E = or_fmt_entries(fmt);
    for (int r = 0; r < M; r++) {
        float acc = 0.0f;
        for (int v = 0; v < nv; v++) {
            const float *blk = lut + (size_t)v * S * E;
            const uint8_t *p = slot_ptr(fmt, idx, N, r, v);
            float t = blk[get_code(fmt, p, 0)];
            for (int s = 1; s < S; s++) t += blk[(size_t)s * E + get_code(fmt, p, s)];
            acc += t;
        }
        y[r] = acc * or_f16_keep(scale[r]);
    }
}

void or_vq_quant_lut(const float *lut, int nv, int st, int en, int8_t *q, float *qs)
{
    const int nblk = (nv + OR_LUT_BLK - 1) / OR_LUT_BLK;
    for (int blk = 0; blk < nblk; blk++) {
        const int v0 = blk * OR_LUT_BLK;
        int v1 = v0 + OR_LUT_BLK;
        if (v1 > nv) v1 = nv;
        const size_t n = (size_t)(v1 - v0) * st * en;
        const float *src = lut + (size_t)v0 * st * en;
        int8_t *dst = q + (size_t)v0 * st * en;
        float mx = 0;
        for (size_t i = 0; i < n; i++) {
            const float f = fabsf(src[i]);
            if (f > mx) mx = f;
        }
        qs[blk] = mx / 127.0f;
        const float inv = mx > 0 ? 127.0f / mx : 0.0f;
        for (size_t i = 0; i < n; i++) {
            int t = (int)lrintf(src[i] * inv);
            if (t > 127) t = 127;
            else if (t < -127) t = -127;
            dst[i] = (int8_t)t;
        }
    }
}

void or_vq_apply_p6(float *y, const uint8_t *idx, const uint16_t *scale,
                    const int8_t *lut8, const float *lscale, int M, int N)
{
    const int nv = N / 8, en = 64;
    for (int r = 0; r < M; r++) {
        float acc = 0.0f;
        for (int v0 = 0; v0 < nv; v0 += OR_LUT_BLK) {
            int v1 = v0 + OR_LUT_BLK;
            if (v1 > nv) v1 = nv;
            int16_t sum = 0;
            for (int v = v0; v < v1; v++) {
                const int8_t *T = lut8 + (size_t)v * 4 * en;
                const uint8_t *p = slot_ptr(OR_VQ4P, idx, N, r, v);
                sum = (int16_t)(sum + T[get_code(OR_VQ4P, p, 0)] + T[en + get_code(OR_VQ4P, p, 1)] +
                                T[2 * en + get_code(OR_VQ4P, p, 2)] + T[3 * en + get_code(OR_VQ4P, p, 3)]);
            }
            acc += lscale[v0 / OR_LUT_BLK] * (float)sum;
        }
        y[r] = acc * or_f16_keep(scale[r]);
    }
}

void or_vq_matvec(int fmt, float *y, const uint8_t *idx, const uint16_t *scale,
                  const float *x, const float *booksT, int cb_base, int M, int N,
                  int fused, float *lut, int8_t *q8, float *qs)
{
    const int S = or_fmt_stages(fmt), E = or_fmt_entries(fmt), nv = N / 8;
    or_lutb_range(0, nv, lut, booksT, x, cb_base, S, E, 8, fused);
    if (fmt == OR_VQ4P) {
        or_vq_quant_lut(lut, nv, S, E, q8, qs);
        or_vq_apply_p6(y, idx, scale, q8, qs, M, N);
    } else {
        or_vq_apply(fmt, y, idx, scale, lut, M, N);
    }
}

/* ---- dense pieces ------------------------------------------------------------- */

float or_dotf(const float *a, const float *b, int n)
{
    float acc = 0;
    for (int i = 0; i < n; i++) acc += a[i] * b[i];
    return acc;
}

/* signed 3-bit code, LSB-first at bit 3*i, biased by +4 (src/simd.h:69-74) */
static int q3_at(const uint8_t *p, long i)
{
    const long off = i * 3;
    const int v = (p[off >> 3] >> (off & 7)) | (p[(off >> 3) + 1] << (8 - (off & 7)));
    return (v & 7) - 4;
}

static void unpack_group(int bits, const int8_t *row, int k, int g, int8_t *unp)
{
    if (bits == 3) {
        for (int i = 0; i < g; i++) unp[i] = (int8_t)q3_at((const uint8_t *)row, (long)k * g + i);
    } else if (bits == 4) {
        const uint8_t *p4 = (const uint8_t *)row + (size_t)k * g / 2;
        for (int i = 0; i < g; i++) {
            const uint8_t byte = p4[i >> 1];
            unp[i] = (int8_t)((i & 1) ? (byte >> 4) - 8 : (byte & 0x0F) - 8);
        }
    } else {
        memcpy(unp, row + (size_t)k * g, (size_t)g);
    }
}

void or_mvq_rows_f32(int b, int e, float *y, const int8_t *W, const uint16_t *ws,
                     const float *x, int in, int ng, int group, int bits,
                     size_t rowbytes, int isa)
{
    const int g = group;
    int8_t *unp = (int8_t *)malloc((size_t)g + 64);
    if (!unp) return;
    for (int o = b; o < e; o++) {
        const int8_t *row = W + (size_t)o * rowbytes;
        const uint16_t *wsr = ws + (size_t)o * ng;
        float acc = 0;
        for (int k = 0; k < ng; k++) {
            unpack_group(bits, row, k, g, unp);
            const float *xx = x + (size_t)k * g;
            const int lim = (k * g + g <= in) ? g : in - k * g;
            if (isa == 0) {
                float part = 0;
                for (int i = 0; i < lim; i++) part += (float)unp[i] * xx[i];
                acc += or_f16_keep(wsr[k]) * part;
            } else {
                /* two vector accumulators of L lanes, fmadd over 2L-wide steps,
                 * then the fixed tree of _mm512_reduce_add_ps / hsum256 */
                const int L = isa == 2 ? 16 : 8;
                float s0[16] = {0}, s1[16] = {0};
                int i = 0;
                for (; i + 2 * L <= lim; i += 2 * L)
                    for (int l = 0; l < L; l++) {
                        s0[l] = fmaf((float)unp[i + l], xx[i + l], s0[l]);
                        s1[l] = fmaf((float)unp[i + L + l], xx[i + L + l], s1[l]);
                    }
                float v[16];
                for (int l = 0; l < L; l++) v[l] = s0[l] + s1[l];
                float t8[8];
                if (L == 16) { for (int l = 0; l < 8; l++) t8[l] = v[8 + l] + v[l]; }
                else { for (int l = 0; l < 8; l++) t8[l] = v[l]; }
                float t4[4];
                for (int l = 0; l < 4; l++) t4[l] = t8[4 + l] + t8[l];
                const float h0 = t4[0] + t4[2], h1 = t4[1] + t4[3];
                float part = h0 + h1;
                /* GCC contracts the scalar tail and the group fold in these
                 * translation units (AVX-512F / FMA enabled, gnu11). */
                for (; i < lim; i++) part = fmaf((float)unp[i], xx[i], part);
                acc = fmaf(or_f16_keep(wsr[k]), part, acc);
            }
        }
        y[o] = acc;
    }
    free(unp);
}

void or_mmq_rows(int b, int e, float *y, const int8_t *W, const uint16_t *ws,
                 const float *x, int in, int ng, int group, int bits, size_t rowbytes)
{
    const int g = group;
    float *row = (float *)malloc((size_t)in * sizeof(float));
    int8_t *unp = (int8_t *)malloc((size_t)g + 64);
    if (!row || !unp) { free(row); free(unp); return; }
    for (int o = b; o < e; o++) {
        const int8_t *q = W + (size_t)o * rowbytes;
        const uint16_t *sc = ws + (size_t)o * ng;
        for (int k = 0; k < ng; k++) {
            const float s = or_f16_keep(sc[k]);
            const int lim = (k * g + g <= in) ? g : in - k * g;
            unpack_group(bits, q, k, g, unp);
            for (int i = 0; i < lim; i++) row[k * g + i] = (float)unp[i] * s;
        }
        y[o] = or_dotf(row, x, in);
    }
    free(row);
    free(unp);
}

/* ---- routing -------------------------------------------------------------------- */

void or_route(const float *logits, const float *bias, int E, int K, int act,
              int renorm, float routed_scale, int *idx, float *w, float *score_out)
{
    float *score = (float *)malloc((size_t)E * sizeof(float));
    if (!score) return;
    if (act == OR_ROUTE_SOFTMAX) {
        float mx = logits[0];
        for (int e = 1; e < E; e++) if (logits[e] > mx) mx = logits[e];
        float s = 0;
        for (int e = 0; e < E; e++) { score[e] = expf(logits[e] - mx); s += score[e]; }
        for (int e = 0; e < E; e++) score[e] = score[e] / s;
    } else {
        for (int e = 0; e < E; e++) score[e] = 1.0f / (1.0f + expf(-logits[e]));
    }
    for (int j = 0; j < K; j++) {
        int best = -1;
        float bv = -1e30f;
        for (int e = 0; e < E; e++) {
            int taken = 0;
            for (int p = 0; p < j; p++) if (idx[p] == e) { taken = 1; break; }
            if (taken) continue;
            const float v = score[e] + (bias ? bias[e] : 0.0f);
            if (v > bv) { bv = v; best = e; }
        }
        idx[j] = best;
        w[j] = score[best];
    }
    if (renorm && K > 1) {
        float s = 0;
        for (int j = 0; j < K; j++) s += w[j];
        for (int j = 0; j < K; j++) w[j] /= (s + 1e-20f);
    }
    for (int j = 0; j < K; j++) w[j] *= routed_scale;
    if (score_out) memcpy(score_out, score, (size_t)E * sizeof(float));
    free(score);
}

/* ---- the layer -------------------------------------------------------------------- */

typedef struct {
    uint32_t magic;
    uint16_t layer, expert_id;
    uint8_t fmt, flags;
    uint16_t codebook_id, lowrank_id, reserved0;
    uint32_t rec_4k_blocks, gate_off, up_off, down_off, chan_corr_off, crc32;
    uint32_t reserved1[2];
} rec_hdr;  /* waste_expert_hdr, src/waste_format.h:98-130 */

static int is_p6(int fmt) { return fmt == OR_VQ4P; }

void or_expert_ffn(const or_layer *L, const uint8_t *rec, const float *lut_gate,
                   const float *lut_up, const int8_t *q_gate, const float *qs_gate,
                   const int8_t *q_up, const float *qs_up, float *acc)
{
    const int fmt = L->fmt, S = or_fmt_stages(fmt), E = or_fmt_entries(fmt);
    const int inter = L->inter, hid = L->hidden;
    const rec_hdr *h = (const rec_hdr *)rec;
    const uint16_t *sc = (const uint16_t *)(rec + h->chan_corr_off);
    float *ga = (float *)malloc((size_t)inter * sizeof(float));
    float *ub = (float *)malloc((size_t)inter * sizeof(float));
    const int nvd = inter / 8;
    float *lut = (float *)malloc((size_t)nvd * S * E * sizeof(float));
    int8_t *q8 = (int8_t *)malloc((size_t)nvd * S * E);
    float *qs = (float *)malloc(((size_t)nvd / OR_LUT_BLK + 2) * sizeof(float));
    if (!ga || !ub || !lut || !q8 || !qs) goto out;
    if (is_p6(fmt)) {
        or_vq_apply_p6(ga, rec + h->gate_off, sc, q_gate, qs_gate, inter, hid);
        or_vq_apply_p6(ub, rec + h->up_off, sc + inter, q_up, qs_up, inter, hid);
    } else {
        or_vq_apply(fmt, ga, rec + h->gate_off, sc, lut_gate, inter, hid);
        or_vq_apply(fmt, ub, rec + h->up_off, sc + inter, lut_up, inter, hid);
    }
    if (L->act_situ)
        for (int i = 0; i < inter; i++) ga[i] = or_situ_pair(ga[i], ub[i], L->situ_beta, L->situ_lbeta);
    else
        for (int i = 0; i < inter; i++) ga[i] = or_silu(ga[i]) * ub[i];
    or_vq_matvec(fmt, acc, rec + h->down_off, sc + 2 * inter, ga, L->booksT,
                 h->codebook_id + 2 * S, hid, inter, L->fused_lutb, lut, q8, qs);
out:
    free(ga); free(ub); free(lut); free(q8); free(qs);
}

/* gate/up tables from x, built with the first record's codebook_id as the
 * reference does (src/model.c:2888-2896). */
static int build_gate_up(const or_layer *L, const uint8_t *rec0, const float *x,
                         float *lut_g, float *lut_u, int8_t *q_g, float *qs_g,
                         int8_t *q_u, float *qs_u)
{
    const int fmt = L->fmt, S = or_fmt_stages(fmt), E = or_fmt_entries(fmt);
    const int nv = L->hidden / 8;
    const rec_hdr *h = (const rec_hdr *)rec0;
    or_lutb_range(0, nv, lut_g, L->booksT, x, h->codebook_id + 0 * S, S, E, 8, L->fused_lutb);
    or_lutb_range(0, nv, lut_u, L->booksT, x, h->codebook_id + 1 * S, S, E, 8, L->fused_lutb);
    if (is_p6(fmt)) {
        or_vq_quant_lut(lut_g, nv, S, E, q_g, qs_g);
        or_vq_quant_lut(lut_u, nv, S, E, q_u, qs_u);
    }
    return 0;
}

/* matvec_t on the router (src/model.c:385-399): an F32 tensor goes through
 * mv_rows -> dotf, a quantised one through the backend's mvq_rows_f32. */
static void router_logits(const or_layer *L, const float *x, float *sc)
{
    const int E = L->n_experts, hid = L->hidden;
    if (L->router) {
        for (int e = 0; e < E; e++) sc[e] = or_dotf(L->router + (size_t)e * hid, x, hid);
    } else {
        const int g = L->router_group, ng = (hid + g - 1) / g;
        or_mvq_rows_f32(0, E, sc, L->router_q, L->router_s, x, hid, ng, g, L->router_bits,
                        L->router_rowbytes, L->mvq_isa);
    }
}

static void shared_ffn(const or_layer *L, const float *in, float *tmp, int batched)
{
    const int hid = L->hidden, si = L->sh_inter, g = L->sh_group;
    float *a = (float *)malloc((size_t)si * sizeof(float));
    float *b = (float *)malloc((size_t)si * sizeof(float));
    if (!a || !b) { free(a); free(b); return; }
    const int ngh = (hid + g - 1) / g, ngi = (si + g - 1) / g;
    if (batched) {
        or_mmq_rows(0, si, a, L->sh_q[0], L->sh_s[0], in, hid, ngh, g, L->sh_bits, L->sh_rowbytes[0]);
        or_mmq_rows(0, si, b, L->sh_q[1], L->sh_s[1], in, hid, ngh, g, L->sh_bits, L->sh_rowbytes[1]);
    } else {
        or_mvq_rows_f32(0, si, a, L->sh_q[0], L->sh_s[0], in, hid, ngh, g, L->sh_bits, L->sh_rowbytes[0], L->mvq_isa);
        or_mvq_rows_f32(0, si, b, L->sh_q[1], L->sh_s[1], in, hid, ngh, g, L->sh_bits, L->sh_rowbytes[1], L->mvq_isa);
    }
    for (int i = 0; i < si; i++)
        a[i] = L->act_situ ? or_situ_pair(a[i], b[i], L->situ_beta, L->situ_lbeta) : or_silu(a[i]) * b[i];
    if (batched)
        or_mmq_rows(0, hid, tmp, L->sh_q[2], L->sh_s[2], a, si, ngi, g, L->sh_bits, L->sh_rowbytes[2]);
    else
        or_mvq_rows_f32(0, hid, tmp, L->sh_q[2], L->sh_s[2], a, si, ngi, g, L->sh_bits, L->sh_rowbytes[2], L->mvq_isa);
    free(a); free(b);
}

void or_rmsnorm(float *o, const float *x, const float *w, int n, float eps)
{
    float s = 0;
    for (int i = 0; i < n; i++) s += x[i] * x[i];
    const float r = 1.0f / sqrtf(s / (float)n + eps);
    for (int i = 0; i < n; i++) o[i] = x[i] * r * w[i];
}

/* The latent projections: matvec_t for one token (mvq_rows_f32,
 * src/model.c:385-399), waste_matmul_t for a chunk (mmq_rows,
 * src/model.c:3366-3398). kind 0: down [latent][hidden], 1: up. */
static void latent_proj(const or_layer *L, int kind, const float *x, float *y, int batched)
{
    const int out = kind == 0 ? L->latent : L->hidden, in = kind == 0 ? L->hidden : L->latent;
    const int g = L->lat_group, ng = (in + g - 1) / g;
    if (batched)
        or_mmq_rows(0, out, y, L->lat_q[kind], L->lat_s[kind], x, in, ng, g, L->lat_bits, L->lat_rowbytes[kind]);
    else
        or_mvq_rows_f32(0, out, y, L->lat_q[kind], L->lat_s[kind], x, in, ng, g, L->lat_bits, L->lat_rowbytes[kind],
                        L->mvq_isa);
}

int or_moe_layer(const or_layer *L, const float *in, float *out, int *idx,
                 float *w, float *logits)
{
    const int E = L->n_experts, K = L->top_k, hid = L->hidden;
    /* the experts' width, and their view of the layer */
    const int lat = L->latent ? L->latent : hid;
    or_layer Le = *L;
    Le.hidden = lat;
    const int S = or_fmt_stages(L->fmt), En = or_fmt_entries(L->fmt), nv = lat / 8;
    float *sc = (float *)malloc((size_t)E * sizeof(float));
    float *acc = (float *)malloc((size_t)lat * sizeof(float));
    float *tmp = (float *)malloc((size_t)hid * sizeof(float));
    float *xl = (float *)malloc((size_t)lat * sizeof(float)), *ys = (float *)malloc((size_t)lat * sizeof(float));
    const size_t lsz = (size_t)nv * S * En;
    float *lg = (float *)malloc(lsz * sizeof(float)), *lu = (float *)malloc(lsz * sizeof(float));
    int8_t *qg = (int8_t *)malloc(lsz), *qu = (int8_t *)malloc(lsz);
    float *qsg = (float *)malloc(((size_t)nv / OR_LUT_BLK + 2) * sizeof(float));
    float *qsu = (float *)malloc(((size_t)nv / OR_LUT_BLK + 2) * sizeof(float));
    int rc = -1;
    if (!sc || !acc || !tmp || !xl || !ys || !lg || !lu || !qg || !qu || !qsg || !qsu) goto out;
    router_logits(L, in, sc);
    if (logits) memcpy(logits, sc, (size_t)E * sizeof(float));
    or_route(sc, L->bias, E, K, L->router_act, L->renorm, L->routed_scale, idx, w, NULL);
    const float *xin = in;
    if (L->latent) {
        latent_proj(L, 0, in, xl, 0);
        xin = xl;
    }
    float *ysum = L->latent ? ys : out;
    memset(ysum, 0, (size_t)lat * sizeof(float));
    for (int j = 0; j < K; j++) {
        const uint8_t *rec = L->recs[idx[j]];
        if (j == 0) build_gate_up(&Le, rec, xin, lg, lu, qg, qsg, qu, qsu);
        or_expert_ffn(&Le, rec, lg, lu, qg, qsg, qu, qsu, acc);
        const float wj = w[j];
        for (int i = 0; i < lat; i++) ysum[i] += wj * acc[i];
    }
    if (L->latent) {
        if (L->lat_norm) or_rmsnorm(ysum, ysum, L->lat_norm, lat, L->eps);
        latent_proj(L, 1, ysum, out, 0);
    }
    if (L->sh_q[0]) {
        shared_ffn(L, in, tmp, 0);
        for (int i = 0; i < hid; i++) out[i] += tmp[i];
    }
    rc = 0;
out:
    free(sc); free(acc); free(tmp); free(xl); free(ys); free(lg); free(lu); free(qg); free(qu); free(qsg); free(qsu);
    return rc;
}

int or_moe_chunk(const or_layer *L, const float *in, float *out, int nT,
                 int *route, float *rw)
{
    const int E = L->n_experts, K = L->top_k, hid = L->hidden;
    const int lat = L->latent ? L->latent : hid;
    or_layer Le = *L;
    Le.hidden = lat;
    const int S = or_fmt_stages(L->fmt), En = or_fmt_entries(L->fmt), nv = lat / 8;
    const size_t lsz = (size_t)nv * S * En, nsc = (size_t)nv / OR_LUT_BLK + 2;
    float *sc = (float *)malloc((size_t)E * sizeof(float));
    float *acc = (float *)malloc((size_t)lat * sizeof(float));
    float *tmp = (float *)malloc((size_t)hid * sizeof(float));
    float *xl = (float *)malloc((size_t)nT * lat * sizeof(float));
    float *ys = (float *)malloc((size_t)nT * lat * sizeof(float));
    float *lgu = (float *)malloc((size_t)nT * 2 * lsz * sizeof(float));
    int8_t *qgu = (int8_t *)malloc((size_t)nT * 2 * lsz);
    float *qsgu = (float *)malloc((size_t)nT * 2 * nsc * sizeof(float));
    int rc = -1;
    if (!sc || !acc || !tmp || !xl || !ys || !lgu || !qgu || !qsgu) goto out;
    for (int t = 0; t < nT; t++) {
        router_logits(L, in + (size_t)t * hid, sc);
        or_route(sc, L->bias, E, K, L->router_act, L->renorm, L->routed_scale,
                 route + (size_t)t * K, rw + (size_t)t * K, NULL);
    }
    const float *xin = in;
    if (L->latent) {
        for (int t = 0; t < nT; t++) latent_proj(L, 0, in + (size_t)t * hid, xl + (size_t)t * lat, 1);
        xin = xl;
    }
    float *ysum = L->latent ? ys : out;
    memset(ysum, 0, (size_t)nT * lat * sizeof(float));
    int lut_ready = 0;
    for (int e = 0; e < E; e++) {               /* distinct experts, ascending */
        int used = 0;
        for (int i = 0; i < nT * K; i++) if (route[i] == e) { used = 1; break; }
        if (!used) continue;
        const uint8_t *rec = L->recs[e];
        if (!lut_ready) {
            for (int t = 0; t < nT; t++)
                build_gate_up(&Le, rec, xin + (size_t)t * lat, lgu + (size_t)(2 * t) * lsz,
                              lgu + (size_t)(2 * t + 1) * lsz, qgu + (size_t)(2 * t) * lsz,
                              qsgu + (size_t)(2 * t) * nsc, qgu + (size_t)(2 * t + 1) * lsz,
                              qsgu + (size_t)(2 * t + 1) * nsc);
            lut_ready = 1;
        }
        for (int t = 0; t < nT; t++) {
            float wj = 0;
            for (int j = 0; j < K; j++)
                if (route[(size_t)t * K + j] == e) { wj = rw[(size_t)t * K + j]; break; }
            if (wj == 0.0f) continue;
            or_expert_ffn(&Le, rec, lgu + (size_t)(2 * t) * lsz, lgu + (size_t)(2 * t + 1) * lsz,
                          qgu + (size_t)(2 * t) * lsz, qsgu + (size_t)(2 * t) * nsc,
                          qgu + (size_t)(2 * t + 1) * lsz, qsgu + (size_t)(2 * t + 1) * nsc, acc);
            float *dst = ysum + (size_t)t * lat;
            for (int i = 0; i < lat; i++) dst[i] += wj * acc[i];
        }
    }
    if (L->latent)
        for (int t = 0; t < nT; t++) {
            float *y = ysum + (size_t)t * lat;
            if (L->lat_norm) or_rmsnorm(y, y, L->lat_norm, lat, L->eps);
            latent_proj(L, 1, y, out + (size_t)t * hid, 1);
        }
    if (L->sh_q[0])
        for (int t = 0; t < nT; t++) {
            shared_ffn(L, in + (size_t)t * hid, tmp, 1);
            float *dst = out + (size_t)t * hid;
            for (int i = 0; i < hid; i++) dst[i] += tmp[i];
        }
    rc = 0;
out:
    free(sc); free(acc); free(tmp); free(xl); free(ys); free(lgu); free(qgu); free(qsgu);
    return rc;
}

/* ---- encoder, checksum, records ------------------------------------------------ */

void or_vq_encode(const float *X, int n, const float *books, int stages,
                  int entries, int dim, uint16_t *out)
{
    float cur[64], nxt[64];
    for (int i = 0; i < n; i++) {
        const float *v = X + (size_t)i * dim;
        for (int d = 0; d < dim; d++) cur[d] = v[d];
        for (int s = 0; s < stages; s++) {
            const float *C = books + (size_t)s * entries * dim;
            int best = 0;
            float bestd = INFINITY;
            for (int c = 0; c < entries; c++) {
                const float *e = C + (size_t)c * dim;
                float d = 0;
                for (int j = 0; j < dim; j++) { const float t = cur[j] - e[j]; d += t * t; }
                if (d < bestd) { bestd = d; best = c; }
            }
            for (int j = 0; j < dim; j++) nxt[j] = cur[j] - C[(size_t)best * dim + j];
            out[(size_t)i * stages + s] = (uint16_t)best;
            for (int d = 0; d < dim; d++) cur[d] = nxt[d];
        }
    }
}

uint32_t or_crc32(const uint8_t *p, size_t n)
{
    uint32_t c = 0xFFFFFFFFu;
    for (size_t i = 0; i < n; i++) {
        c ^= p[i];
        for (int k = 0; k < 8; k++) c = (c >> 1) ^ (0xEDB88320u & (0u - (c & 1u)));
    }
    return c ^ 0xFFFFFFFFu;
}

int or_record_check(const uint8_t *rec, size_t rec_bytes, int layer, int expert,
                    int index_bits, int stages, int n_books, const int expert_m[3], int verify)
{
    const rec_hdr *h = (const rec_hdr *)rec;
    if (rec_bytes < sizeof *h) return 2;
    if (h->magic != 0x50584557u) return 2;
    if (h->layer != (uint16_t)layer || h->expert_id != (uint16_t)expert) return 2;
    if ((size_t)h->rec_4k_blocks * 4096u != rec_bytes) return 2;
    /* VQ4P for 6-bit indices, VQ3R or VQ2R for bytes; the 12-bit extension
     * names its own format code */
    const int want = index_bits == 6 ? OR_VQ4P : index_bits == 12 ? OR_VQ12 : OR_VQ3R;
    if (h->fmt != want && !(index_bits == 8 && h->fmt == OR_VQ2R)) return 2;
    if (h->lowrank_id != 0) return 2;
    if ((long)h->codebook_id + 3L * stages > n_books) return 2;
    if (!(h->gate_off == sizeof *h && h->gate_off < h->up_off && h->up_off < h->down_off &&
          h->down_off < h->chan_corr_off && h->chan_corr_off <= rec_bytes))
        return 2;
    const size_t scales = 2u * (size_t)(expert_m[0] + expert_m[1] + expert_m[2]);
    if (scales > rec_bytes - h->chan_corr_off) return 2;
    if (!verify) return 0;
    const size_t payload = (size_t)h->chan_corr_off + scales - sizeof *h;
    if (or_crc32(rec + sizeof *h, payload) != h->crc32) return 3;
    return 0;
}

/* ---- Kimi Delta Attention step (src/kda.c:19-68) ---------------------------------- */

static float kda_rnorm(const float *x, int n)
{
    float s = 0.0f;
    for (int i = 0; i < n; i++) s += x[i] * x[i];
    return 1.0f / sqrtf(s + 1e-12f);
}

void or_kda_step(int H, int K, int V, const float *q, const float *k, const float *v, const float *g_log,
                 const float *beta, float *S, float *o)
{
    const float qscale = 1.0f / sqrtf((float)K);
    float *u = (float *)malloc((size_t)V * sizeof(float));
    if (!u) return;
    for (int h = 0; h < H; h++) {
        const float *qh = q + (size_t)h * K, *kh = k + (size_t)h * K, *gh = g_log + (size_t)h * K;
        const float *vh = v + (size_t)h * V;
        float *Sh = S + (size_t)h * K * V, *oh = o + (size_t)h * V;
        const float qn = kda_rnorm(qh, K) * qscale, kn = kda_rnorm(kh, K);
        for (int i = 0; i < V; i++) u[i] = 0.0f;
        for (int r = 0; r < K; r++) {               /* decay, u = S^T k */
            const float d = expf(gh[r]), kv = kh[r] * kn;
            for (int i = 0; i < V; i++) {
                Sh[(size_t)r * V + i] *= d;
                u[i] += Sh[(size_t)r * V + i] * kv;
            }
        }
        for (int i = 0; i < V; i++) u[i] = beta[h] * (vh[i] - u[i]);
        for (int i = 0; i < V; i++) oh[i] = 0.0f;
        for (int r = 0; r < K; r++) {               /* S += k d^T, o = S^T q */
            const float kv = kh[r] * kn, qv = qh[r] * qn;
            for (int i = 0; i < V; i++) {
                Sh[(size_t)r * V + i] += u[i] * kv;
                oh[i] += Sh[(size_t)r * V + i] * qv;
            }
        }
    }
    free(u);
}
