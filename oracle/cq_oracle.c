/*
 * CPU oracle, CQ part: a plain-C restatement of go-whistle's internal/cact
 * packed form and internal/cq products. TEST INFRASTRUCTURE ONLY (see
 * oracle.h): the product library never links or calls this file.
 *
 * Reference files followed (paths relative to the go-whistle repository):
 *   internal/cact/half.go:8-40        float16ToFloat32
 *   internal/cact/cq.go:67-169        dequantCQ, unpackLSB, fwht
 *   internal/cact/packed.go:18-40     Packed, Groups, RowBytes, Norm
 *   internal/cq/matrix.go:46-189      New, NewGather, Rows, Row, at
 *   internal/cq/kernel.go:100-393     gemm, GEMMs, gemmScalar, rotate, gather,
 *                                     nibbleTables, lookupNibble,
 *                                     nibbleTables4, lookupNibble4, invSqrt, fwht
 *   internal/cq/lut.go:41-313         lutLayout.blocks, lutSpan, gemmLUT,
 *                                     lutRun, lutTables, lutApply, lutStepOf,
 *                                     lutInv, lutPut, lutTables2/4Generic,
 *                                     lutLookupGeneric
 * The amd64 assembly (lut_amd64.s) equals these Go routines bit for bit
 * (internal/cq/asm_test.go:11-17), so the Go code is the one definition.
 * On a NaN input the two differ (VMAXPS keeps or drops a NaN by its lane
 * and chunk; Go's max and arm64's FMAX keep it): the Go code is followed,
 * so a group holding a NaN or an Inf gives NaN rows.
 *
 * How each part is pinned without running the reference (tests/):
 *   f16 widen     exhaustive against numpy float16 -> float32
 *   unpack / at   brute-force LSB-first bit extraction (numpy unpackbits)
 *   fwht          explicit Sylvester matrix on small integers, exact
 *   Row / CQ      float64 explicit dequantisation (cq_test.go:68-91), cosine
 *   every kernel  float64 product within rotatedBound (+ lutBound for lut),
 *                 cosine (cq_test.go:106-254); row independence, Rows views,
 *                 GEMMs = GEMM (cq_test.go:260-444, parallel_test.go:97-168)
 *   lut tables    closed-form known answers with exact half-way entries
 *                 (round half to even) and the byte-plane split
 *   lut lookup    closed-form known answers: integer sums from hand tables,
 *                 group order of the float32 accumulation
 *   nibble/nibble4 summation order: parity unpinned beyond the float64 bound
 *                 (only running the Go code would pin those last bits)
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* lut.go:31-39 */
enum { LUT_ROWS = 32, LUT_Q = 8191, LUT_BIAS = 64, LUT_MAX_GROUP_BYTES = 256 };

float orc_f16_to_f32(uint16_t h) {
    /* internal/cact/half.go:8-40 */
    uint32_t sign = (uint32_t)(h >> 15) & 1u;
    uint32_t exp = (uint32_t)(h >> 10) & 0x1fu;
    uint32_t frac = (uint32_t)(h & 0x3ffu);
    uint32_t bits;
    if (exp == 0) {
        if (frac == 0) {
            bits = sign << 31;
        } else {
            uint32_t exp32 = 113;
            while ((frac & 0x400u) == 0) {
                frac <<= 1;
                exp32--;
            }
            frac &= 0x3ffu;
            bits = (sign << 31) | (exp32 << 23) | (frac << 13);
        }
    } else if (exp == 0x1f) {
        bits = (sign << 31) | 0x7f800000u | (frac << 13);
    } else {
        bits = (sign << 31) | ((exp + (127 - 15)) << 23) | (frac << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void orc_f16_to_f32_n(float *dst, const uint16_t *h, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_f16_to_f32(h[i]);
}

void orc_unpack_lsb(uint8_t *idx, const uint8_t *packed, int n, int width) {
    /* internal/cact/cq.go:124-137: chunks of 8 indices from width bytes */
    uint64_t mask = ((uint64_t)1 << width) - 1;
    for (int c = 0; c < n / 8; c++) {
        uint64_t word = 0;
        for (int b = 0; b < width; b++) word |= (uint64_t)packed[c * width + b] << (8 * b);
        for (int k = 0; k < 8; k++) idx[8 * c + k] = (uint8_t)((word >> (k * width)) & mask);
    }
}

void orc_fwht(float *x, int n) {
    /* internal/cq/kernel.go:384-393 (= internal/cact/cq.go:160-169) */
    for (int h = 1; h < n; h *= 2)
        for (int i = 0; i < n; i += 2 * h)
            for (int j = i; j < i + h; j++) {
                float a = x[j], b = x[j + h];
                x[j] = a + b;
                x[j + h] = a - b;
            }
}

static float inv_sqrt(int group) { return (float)(1.0 / sqrt((double)group)); } /* kernel.go:377 */

float orc_lut_step(int group) { return (float)(1.0 / ((double)LUT_Q * sqrt((double)group))); } /* lut.go:213-215 */

static float abs32(float v) { return fabsf(v); } /* lut.go:315: clears the sign bit */

/* Go's built-in max for float32 (used as max(m, |v|)): NaN if either is NaN. */
static float gomax(float a, float b) {
    if (a != a || b != b) return NAN;
    if (a == 0 && b == 0) return signbit(a) ? b : a;
    return a > b ? a : b;
}

int orc_cq_dequant(float *w, const orc_packed *p) {
    /* internal/cact/cq.go:67-118 for the 2- and 4-bit records */
    int out = p->out, in = p->in, group = p->group, width = p->width;
    if (group <= 0 || (group & (group - 1)) != 0) return -1;
    int groups = (in + group - 1) / group, in_pad = groups * group;
    int row_bytes = in_pad * width / 8;
    float scale = inv_sqrt(group);
    uint8_t *idx = malloc((size_t)in_pad);
    float *buf = malloc(sizeof(float) * (size_t)group);
    for (int r = 0; r < out; r++) {
        orc_unpack_lsb(idx, p->index + (size_t)r * row_bytes, in_pad, width);
        for (int g = 0; g < groups; g++) {
            const uint8_t *nb = p->norms + 2 * ((size_t)r * groups + g);
            float s = orc_f16_to_f32((uint16_t)(nb[0] | (nb[1] << 8))) * scale;
            for (int k = 0; k < group; k++) buf[k] = p->codebook[idx[g * group + k]] * s;
            orc_fwht(buf, group);
            int col = g * group, hi = col + group < in ? col + group : in;
            memcpy(w + (size_t)r * in + col, buf, sizeof(float) * (size_t)(hi - col));
        }
    }
    free(idx);
    free(buf);
    return 0;
}

/* ---- Matrix ------------------------------------------------------------- */

typedef struct {
    int refs;
    int out;               /* rows of the root matrix */
    uint8_t *index;        /* root rows, row_bytes each */
    float *norms;          /* root [out][groups], widened */
    float cb[16];
    int ncb;
    float cb_max, lut_step;
    /* lutLayout (lut.go:44-55): built once at New */
    uint8_t *bidx;         /* [(b*row_bytes + j)*32 + i] */
    float *bnorm;          /* [(b*groups + g)*32 + i] */
} orc_store;

struct orc_matrix {
    int out, in, group, groups, width, row_bytes, group_bytes;
    int row0;
    orc_store *st;
};

static void set_err(char *err, size_t errlen, const char *msg) {
    if (err && errlen) snprintf(err, errlen, "%s", msg);
}

orc_matrix *orc_new(const orc_packed *p, char *err, size_t errlen) {
    /* internal/cq/matrix.go:46-96; New = NewGather + Prepare (the lut copy
     * is built here at once: the oracle has no lazy state). */
    char msg[256];
    if ((p->bits != 2 && p->bits != 4) || p->width != p->bits) {
        snprintf(msg, sizeof msg, "cq: %d-bit CQ (index width %d) not supported, only 2 and 4", p->bits, p->width);
        set_err(err, errlen, msg);
        return NULL;
    }
    if (p->group < 8 || (p->group & (p->group - 1)) != 0) {
        snprintf(msg, sizeof msg, "cq: group %d is not a power of two >= 8", p->group);
        set_err(err, errlen, msg);
        return NULL;
    }
    if (p->out < 0 || p->in <= 0) {
        snprintf(msg, sizeof msg, "cq: bad shape [%d, %d]", p->out, p->in);
        set_err(err, errlen, msg);
        return NULL;
    }
    if (p->codebook_len != ((size_t)1 << p->bits)) {
        snprintf(msg, sizeof msg, "cq: %zu codebook levels for %d bits", p->codebook_len, p->bits);
        set_err(err, errlen, msg);
        return NULL;
    }
    int groups = (p->in + p->group - 1) / p->group;
    int row_bytes = groups * p->group * p->width / 8;
    if (p->index_len != (size_t)p->out * row_bytes || p->norms_len != 2 * (size_t)p->out * groups) {
        snprintf(msg, sizeof msg, "cq: %zu index and %zu norm bytes for [%d, %d], want %zu and %zu", p->index_len,
                 p->norms_len, p->out, p->in, (size_t)p->out * row_bytes, 2 * (size_t)p->out * groups);
        set_err(err, errlen, msg);
        return NULL;
    }

    orc_matrix *m = calloc(1, sizeof *m);
    orc_store *st = calloc(1, sizeof *st);
    m->out = p->out;
    m->in = p->in;
    m->group = p->group;
    m->groups = groups;
    m->width = p->bits;
    m->row_bytes = row_bytes;
    m->group_bytes = p->group * p->bits / 8;
    m->row0 = 0;
    m->st = st;
    st->refs = 1;
    st->out = p->out;
    st->index = malloc((size_t)p->out * row_bytes + 1);
    memcpy(st->index, p->index, (size_t)p->out * row_bytes);
    st->norms = malloc(sizeof(float) * ((size_t)p->out * groups + 1));
    for (size_t i = 0; i < (size_t)p->out * groups; i++)
        st->norms[i] = orc_f16_to_f32((uint16_t)(p->norms[2 * i] | (p->norms[2 * i + 1] << 8)));
    st->ncb = 1 << p->bits;
    st->cb_max = 0;
    for (int c = 0; c < st->ncb; c++) {
        st->cb[c] = p->codebook[c];
        st->cb_max = gomax(st->cb_max, abs32(st->cb[c]));
    }
    st->lut_step = orc_lut_step(p->group);

    /* lutLayout.blocks (lut.go:58-80) */
    int nb = (p->out + LUT_ROWS - 1) / LUT_ROWS;
    st->bidx = calloc((size_t)nb * row_bytes * LUT_ROWS + 1, 1);
    st->bnorm = calloc((size_t)nb * groups * LUT_ROWS + 1, sizeof(float));
    for (int r = 0; r < p->out; r++) {
        int b = r / LUT_ROWS, i = r % LUT_ROWS;
        for (int j = 0; j < row_bytes; j++)
            st->bidx[((size_t)b * row_bytes + j) * LUT_ROWS + i] = st->index[(size_t)r * row_bytes + j];
        for (int g = 0; g < groups; g++)
            st->bnorm[((size_t)b * groups + g) * LUT_ROWS + i] = st->norms[(size_t)r * groups + g];
    }
    return m;
}

orc_matrix *orc_rows(const orc_matrix *m, int lo, int hi) {
    /* matrix.go:133-145 */
    if (lo < 0 || hi < lo || hi > m->out) return NULL;
    orc_matrix *v = malloc(sizeof *v);
    *v = *m;
    v->out = hi - lo;
    v->row0 = m->row0 + lo;
    v->st->refs++;
    return v;
}

void orc_free(orc_matrix *m) {
    if (!m) return;
    if (--m->st->refs == 0) {
        free(m->st->index);
        free(m->st->norms);
        free(m->st->bidx);
        free(m->st->bnorm);
        free(m->st);
    }
    free(m);
}

int orc_out(const orc_matrix *m) { return m->out; }
int orc_in(const orc_matrix *m) { return m->in; }

static const uint8_t *row_index(const orc_matrix *m, int r) {
    return m->st->index + (size_t)(m->row0 + r) * m->row_bytes;
}
static const float *row_norms(const orc_matrix *m, int r) {
    return m->st->norms + (size_t)(m->row0 + r) * m->groups;
}

/* Matrix.at (matrix.go:185-189) */
static uint8_t at(const orc_matrix *m, const uint8_t *row, int k) {
    int bit = k * m->width;
    return (uint8_t)((row[bit / 8] >> (bit % 8)) & ((1 << m->width) - 1));
}

int orc_row(const orc_matrix *m, float *dst, int r) {
    /* matrix.go:161-181 */
    if (r < 0 || r >= m->out) return -1;
    float *buf = malloc(sizeof(float) * (size_t)m->group);
    const uint8_t *row = row_index(m, r);
    float scale = inv_sqrt(m->group);
    for (int g = 0; g < m->groups; g++) {
        float s = row_norms(m, r)[g] * scale;
        for (int k = 0; k < m->group; k++) buf[k] = m->st->cb[at(m, row, g * m->group + k)] * s;
        orc_fwht(buf, m->group);
        int col = g * m->group, hi = col + m->group < m->in ? col + m->group : m->in;
        memcpy(dst + col, buf, sizeof(float) * (size_t)(hi - col));
    }
    free(buf);
    return 0;
}

/* ---- lut kernel (lut.go) ------------------------------------------------ */

static float lut_inv(float m) { return m > 0 ? (float)LUT_Q / m : 0; } /* lut.go:219-225 */

static void lut_put(uint8_t *t, int c, float e) {
    /* lut.go:229-233: round half to even, two byte planes */
    int32_t v = go_int32_of(rint((double)e)); /* a NaN entry: the integer indefinite */
    t[c] = (uint8_t)(v & 127);
    t[16 + c] = (uint8_t)((v >> 7) + LUT_BIAS);
}

float orc_lut_tables2(uint8_t *tab, const float *x, int n, const float *cb, float cb_max) {
    /* lut.go:239-258 */
    float mx = 0;
    for (int q = 0; q < n; q += 2) mx = gomax(mx, abs32(x[q]) + abs32(x[q + 1]));
    float m = cb_max * mx;
    float inv = lut_inv(m);
    for (int q = 0; q < n / 2; q++) {
        float a = x[2 * q] * inv, b = x[2 * q + 1] * inv;
        uint8_t *t = tab + 32 * q;
        for (int c = 0; c < 16; c++) {
            float lo = cb[c & 3] * a;
            float hi = cb[c >> 2] * b;
            lut_put(t, c, lo + hi);
        }
    }
    return m;
}

float orc_lut_tables4(uint8_t *tab, const float *x, int n, const float *cb, float cb_max) {
    /* lut.go:263-282 */
    float mx = 0;
    for (int q = 0; q < n; q++) mx = gomax(mx, abs32(x[q]));
    float m = cb_max * mx;
    float inv = lut_inv(m);
    for (int q = 0; q < n; q++) {
        float a = x[q] * inv;
        uint8_t *t = tab + 32 * q;
        for (int c = 0; c < 16; c++) lut_put(t, c, cb[c] * a);
    }
    return m;
}

void orc_lut_lookup(float *y, const uint8_t *idx, const uint8_t *tab, const float *norm, const float *steps,
                    int blocks, int groups, int gb) {
    /* lut.go:289-313 */
    int32_t bias = 128 * LUT_BIAS * 2 * gb;
    int row_bytes = groups * gb;
    for (int b = 0; b < blocks; b++) {
        float *yb = y + (size_t)b * LUT_ROWS;
        for (int i = 0; i < LUT_ROWS; i++) yb[i] = 0;
        for (int g = 0; g < groups; g++) {
            float step = steps[g];
            for (int i = 0; i < LUT_ROWS; i++) {
                int32_t lo = 0, hi = 0;
                for (int j = g * gb; j < (g + 1) * gb; j++) {
                    uint8_t v = idx[((size_t)b * row_bytes + j) * LUT_ROWS + i];
                    const uint8_t *t = tab + 64 * (size_t)j;
                    lo += (int32_t)t[v & 15] + (int32_t)t[32 + (v >> 4)];
                    hi += (int32_t)t[16 + (v & 15)] + (int32_t)t[48 + (v >> 4)];
                }
                float coef = norm[((size_t)b * groups + g) * LUT_ROWS + i] * step;
                float prod = (float)(hi * 128 + lo - bias) * coef;
                yb[i] += prod;
            }
        }
    }
}

/* How the lut product runs on this CPU (orc_set_cpu): the generic Go
 * routines or their AVX2 forms (lut_amd64.go:9-61, bit for bit the same),
 * on one thread or split as gemmLUT splits it. Process-wide; set it before
 * the products, not during them. */
static int g_avx2 = 0, g_threads = 1;

int orc_cpu_avx2(void) { return g_avx2; }

int orc_set_cpu(int avx2, int threads) {
    if (avx2 && !orc_have_avx2()) return -1;
    if (threads > 1 && orc_pool_reserve(threads)) return -2;
    g_avx2 = avx2 != 0;
    g_threads = threads < 1 ? 1 : threads;
    return 0;
}

/* tensor.Parallel(n, grain, fn) of algo-tensor v0.4.0 (not vendored with the
 * reference; its call sites are lut.go:109-123, 190-194): [0, n) in
 * contiguous pieces of at least grain items, at most one per worker. The
 * pieces here are equal to within one item. Each output depends on its own
 * inputs only (lut.go:95-101), so any split gives the same bits. */
typedef orc_piece_fn piece_fn;

static void parallel(int n, int grain, piece_fn fn, void *ctx) {
    int pieces = grain > 0 ? n / grain : n;
    if (pieces > g_threads) pieces = g_threads;
    if (pieces < 1) pieces = 1;
    orc_pool_run(n, pieces, fn, ctx); /* piece p: [n*p/pieces, n*(p+1)/pieces) */
}

/* lutPieceBytes (lut.go:88-93) */
enum { LUT_PIECE_BYTES = 1 << 18 };

/* Scratch of one lut product (kernel.go:47-57). */
typedef struct {
    float *xh;
    uint8_t *tab;
    float *steps;
    float *y;
} lut_scratch;

/* lutTables (lut.go:160-178) */
static void lut_tables(const orc_matrix *m, lut_scratch *s, const float *x) {
    int tab_bytes = 64 * m->group_bytes;
    int pad = m->groups * m->group;
    memcpy(s->xh, x, sizeof(float) * (size_t)m->in);
    for (int k = m->in; k < pad; k++) s->xh[k] = 0;
    for (int g = 0; g < m->groups; g++) {
        float *xg = s->xh + (size_t)g * m->group;
        uint8_t *tg = s->tab + (size_t)g * tab_bytes;
        float mm;
        if (g_avx2) { /* the group is at least 8 wide (matrix.go:63-65) */
            orc_fwht_avx2(xg, m->group);
            mm = m->width == 2 ? orc_lut_tables2_avx2(tg, xg, m->group, m->st->cb, m->st->cb_max)
                               : orc_lut_tables4_avx2(tg, xg, m->group, m->st->cb, m->st->cb_max);
        } else {
            orc_fwht(xg, m->group);
            mm = m->width == 2 ? orc_lut_tables2(tg, xg, m->group, m->st->cb, m->st->cb_max)
                               : orc_lut_tables4(tg, xg, m->group, m->st->cb, m->st->cb_max);
        }
        s->steps[g] = mm * m->st->lut_step;
    }
}

typedef struct {
    const orc_matrix *m;
    lut_scratch *s;
    size_t ib, nbk;
    int b0;
} lookup_job;

static void lookup_piece(void *ctx, int lo, int hi) {
    const lookup_job *j = ctx;
    const orc_matrix *m = j->m;
    const uint8_t *idx = m->st->bidx + (size_t)(j->b0 + lo) * j->ib;
    const float *norm = m->st->bnorm + (size_t)(j->b0 + lo) * j->nbk;
    float *y = j->s->y + (size_t)lo * LUT_ROWS;
    if (g_avx2)
        orc_lut_lookup_avx2(y, idx, j->s->tab, norm, j->s->steps, hi - lo, m->groups, m->group_bytes);
    else
        orc_lut_lookup(y, idx, j->s->tab, norm, j->s->steps, hi - lo, m->groups, m->group_bytes);
}

/* lutApply (lut.go:182-201): the blocks split over workers when split. */
static void lut_apply(const orc_matrix *m, lut_scratch *s, float *y, int split) {
    int b0 = m->row0 / LUT_ROWS, b1 = (m->row0 + m->out + LUT_ROWS - 1) / LUT_ROWS;
    lookup_job j = {m, s, (size_t)m->row_bytes * LUT_ROWS, (size_t)m->groups * LUT_ROWS, b0};
    if (split)
        parallel(b1 - b0, (int)((LUT_PIECE_BYTES + j.ib - 1) / j.ib), lookup_piece, &j);
    else
        lookup_piece(&j, 0, b1 - b0);
    int off = m->row0 - b0 * LUT_ROWS;
    memcpy(y, s->y + off, sizeof(float) * (size_t)m->out);
}

typedef struct {
    orc_matrix *const *ms;
    int n, nb;
    float *const *dsts;
    const float *x;
    int split;
} lut_run_job;

/* lutRun (lut.go:128-156) over activations [lo, hi), with its own scratch. */
static void lut_run(void *ctx, int lo, int hi) {
    const lut_run_job *r = ctx;
    const orc_matrix *m0 = r->ms[0];
    lut_scratch s;
    s.xh = malloc(sizeof(float) * (size_t)m0->groups * m0->group);
    s.tab = malloc((size_t)64 * m0->row_bytes);
    s.steps = malloc(sizeof(float) * (size_t)m0->groups);
    s.y = malloc(sizeof(float) * ((size_t)r->nb * LUT_ROWS + 1));
    for (int i = lo; i < hi; i++) {
        lut_tables(m0, &s, r->x + (size_t)i * m0->in);
        for (int k = 0; k < r->n; k++) lut_apply(r->ms[k], &s, r->dsts[k] + (size_t)i * r->ms[k]->out, r->split);
    }
    free(s.xh);
    free(s.tab);
    free(s.steps);
    free(s.y);
}

/* gemmLUT (lut.go:102-126): over the activations when there are several and
 * they outnumber the workers or the product is small, else one activation
 * at a time with each large product's blocks split. */
static void gemm_lut(orc_matrix *const *ms, int n, float *const *dsts, const float *x, int rows) {
    long long per = 0;
    int nb = 0;
    for (int k = 0; k < n; k++) {
        int b0 = ms[k]->row0 / LUT_ROWS, b1 = (ms[k]->row0 + ms[k]->out + LUT_ROWS - 1) / LUT_ROWS;
        if (b1 - b0 > nb) nb = b1 - b0;
        per += (long long)ms[k]->out * ms[k]->row_bytes;
    }
    lut_run_job r = {ms, n, nb, dsts, x, 0};
    if (rows > 1 && (rows >= g_threads || per < 2LL * LUT_PIECE_BYTES)) {
        parallel(rows, (int)((LUT_PIECE_BYTES + per - 1) / per), lut_run, &r);
        return;
    }
    r.split = per >= 2LL * LUT_PIECE_BYTES;
    lut_run(&r, 0, rows);
}

/* ---- scalar kernels (kernel.go:160-374) --------------------------------- */

/* rotate (kernel.go:203-217) */
static void rotate(const orc_matrix *m, float *xh, const float *x) {
    int pad = m->groups * m->group;
    memcpy(xh, x, sizeof(float) * (size_t)m->in);
    for (int k = m->in; k < pad; k++) xh[k] = 0;
    float scale = inv_sqrt(m->group);
    for (int g = 0; g < m->groups; g++) {
        float *xg = xh + (size_t)g * m->group;
        orc_fwht(xg, m->group);
        for (int k = 0; k < m->group; k++) xg[k] *= scale;
    }
}

/* gather (kernel.go:220-237) */
static void gather(const orc_matrix *m, float *y, const float *xh) {
    for (int r = 0; r < m->out; r++) {
        const uint8_t *row = row_index(m, r);
        float acc = 0;
        for (int g = 0; g < m->groups; g++) {
            float dot = 0;
            for (int k = 0; k < m->group; k++) {
                float p = m->st->cb[at(m, row, g * m->group + k)] * xh[g * m->group + k];
                dot += p;
            }
            float p = dot * row_norms(m, r)[g];
            acc += p;
        }
        y[r] = acc;
    }
}

/* nibbleTables (kernel.go:242-265): nib has 2*row_bytes tables of 16. */
static void nibble_tables(const orc_matrix *m, float (*nib)[16], const float *xh) {
    const float *cb = m->st->cb;
    if (m->width == 4) {
        int pad = m->groups * m->group;
        for (int q = 0; q < pad; q++)
            for (int c = 0; c < 16; c++) nib[q][c] = cb[c] * xh[q];
        return;
    }
    int n = 2 * m->row_bytes;
    for (int q = 0; q < n; q++) {
        float a = xh[2 * q], b = xh[2 * q + 1];
        for (int hi = 0; hi < 4; hi++) {
            float hb = cb[hi] * b;
            for (int lo = 0; lo < 4; lo++) {
                float la = cb[lo] * a;
                nib[q][hi << 2 | lo] = la + hb;
            }
        }
    }
}

/* lookupNibble (kernel.go:271-309) */
static void lookup_nibble(const orc_matrix *m, float *y, float (*nib)[16]) {
    int gb = m->group_bytes;
    for (int r = 0; r < m->out; r++) {
        const uint8_t *row = row_index(m, r);
        const float *norms = row_norms(m, r);
        float acc = 0;
        for (int g = 0; g < m->groups; g++) {
            const uint8_t *rg = row + (size_t)g * gb;
            float (*tg)[16] = nib + (size_t)2 * g * gb;
            float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            int j = 0;
            for (; j + 8 <= gb; j += 8) {
                uint64_t w = 0;
                for (int b = 0; b < 8; b++) w |= (uint64_t)rg[j + b] << (8 * b);
                float (*t)[16] = tg + 2 * j;
                for (int k = 0; k < 8; k++) {
                    float pair = t[k][(w >> (4 * k)) & 15] + t[8 + k][(w >> (32 + 4 * k)) & 15];
                    a[k] += pair;
                }
            }
            for (; j < gb; j++) { /* groups under 8 bytes */
                float pair = tg[2 * j][rg[j] & 15] + tg[2 * j + 1][rg[j] >> 4];
                a[0] += pair;
            }
            float t01 = a[0] + a[1], t23 = a[2] + a[3], t45 = a[4] + a[5], t67 = a[6] + a[7];
            float t03 = t01 + t23, t47 = t45 + t67;
            float p = (t03 + t47) * norms[g];
            acc += p;
        }
        y[r] = acc;
    }
}

/* lookupNibble4 with nibbleTables4 folded in: nib4[a] is activation a's
 * nib (kernel.go:314-374); dst is [4][out]. */
static void lookup_nibble4(const orc_matrix *m, float *dst, float (*const nib4[4])[16]) {
    int gb = m->group_bytes;
    for (int r = 0; r < m->out; r++) {
        const uint8_t *row = row_index(m, r);
        const float *norms = row_norms(m, r);
        float c[4] = {0, 0, 0, 0};
        for (int g = 0; g < m->groups; g++) {
            const uint8_t *rg = row + (size_t)g * gb;
            float a[4] = {0, 0, 0, 0}, b[4] = {0, 0, 0, 0};
            for (int j = 0; j < gb; j++) { /* the 8-byte words walk the bytes in order */
                int jj = g * gb + j;
                for (int k = 0; k < 4; k++) {
                    a[k] += nib4[k][2 * jj][rg[j] & 15];
                    b[k] += nib4[k][2 * jj + 1][rg[j] >> 4];
                }
            }
            for (int k = 0; k < 4; k++) {
                float p = (a[k] + b[k]) * norms[g];
                c[k] += p;
            }
        }
        for (int k = 0; k < 4; k++) dst[(size_t)k * m->out + r] = c[k];
    }
}

/* gemmScalar (kernel.go:162-198), serial: the reference splits activations
 * in multiples of four, so nibble4 sees the same groups of four. */
static void gemm_scalar(const orc_matrix *m, int kernel, float *dst, const float *x, int rows) {
    int pad = m->groups * m->group;
    int ntab = 2 * m->row_bytes;
    float *xh = malloc(sizeof(float) * (size_t)pad * 4);
    float (*nib)[16] = malloc(sizeof(float) * 16 * (size_t)ntab * 4);
    int i = 0;
    if (kernel == ORC_NIBBLE4 && rows >= 4) {
        float (*n4[4])[16];
        for (int a = 0; a < 4; a++) n4[a] = nib + (size_t)a * ntab;
        for (; i + 4 <= rows; i += 4) {
            for (int a = 0; a < 4; a++) {
                rotate(m, xh + (size_t)a * pad, x + (size_t)(i + a) * m->in);
                nibble_tables(m, n4[a], xh + (size_t)a * pad);
            }
            lookup_nibble4(m, dst + (size_t)i * m->out, n4);
        }
    }
    for (; i < rows; i++) {
        rotate(m, xh, x + (size_t)i * m->in);
        float *y = dst + (size_t)i * m->out;
        if (kernel == ORC_GATHER) {
            gather(m, y, xh);
            continue;
        }
        nibble_tables(m, nib, xh);
        lookup_nibble(m, y, nib);
    }
    free(xh);
    free(nib);
}

int orc_gemm(const orc_matrix *m, int kernel, float *dst, const float *x, int rows) {
    /* kernel.go:100-125 */
    if (rows < 0) return -1;
    if (rows == 0 || m->out == 0) return 0;
    if (kernel == ORC_LUT) {
        if (m->group_bytes > LUT_MAX_GROUP_BYTES) return -2;
        orc_matrix *one = (orc_matrix *)m;
        gemm_lut(&one, 1, &dst, x, rows);
        return 0;
    }
    gemm_scalar(m, kernel, dst, x, rows);
    return 0;
}

static int shares_tables(const orc_matrix *a, const orc_matrix *b) {
    /* lut.go:206-209 */
    if (a->in != b->in || a->group != b->group || a->width != b->width || a->st->cb_max != b->st->cb_max) return 0;
    for (int c = 0; c < a->st->ncb; c++)
        if (a->st->cb[c] != b->st->cb[c]) return 0;
    return 1;
}

int orc_gemms(orc_matrix *const *ms, int n, int kernel, float *const *dsts, const float *x, int rows) {
    /* kernel.go:134-158 */
    if (rows < 0) return -1;
    int shared = n > 0;
    for (int k = 0; k < n; k++) shared = shared && kernel == ORC_LUT && ms[k]->out > 0 && shares_tables(ms[0], ms[k]);
    if (!shared || rows == 0) {
        for (int k = 0; k < n; k++) {
            int rc = orc_gemm(ms[k], kernel, dsts[k], x, rows);
            if (rc) return rc;
        }
        return 0;
    }
    gemm_lut(ms, n, dsts, x, rows);
    return 0;
}
