/*
 * The synthetic Whistle-shaped decoder's greedy decode, one stream per
 * state, restated in C on the oracle's own pieces: CQ lut GEMMs, int8
 * appends and AttendInt8Spans (int8 query, amd64 exponent), ZCRMSNorm,
 * RoPE, the sigmoid gates, SiLU, argmax, and, where the model has them,
 * the reference's decode-step features:
 *   - causal taps on the raw q/k/v projections with a history of the last
 *     taps - 1 raw rows (Attention.extendTaps / applyTaps,
 *     internal/needle/cache.go:143-154, attention.go:597-613);
 *   - the per-head q/k ZCRMSNorm before RoPE (normRotate,
 *     attention.go:298-330);
 *   - the attention's post-norm and its sigmoid(attn_gate) residual
 *     factor, h += float32(gate * postNorm(a)) (block.go:183-188);
 *   - the cross-attention's per-head q norm (and the memory's k norm,
 *     built by the caller), post norm and residual factor (cross.go:
 *     181-264, QKNormZC and ResSigmoid);
 *   - mHC lanes around every layer: RMSUnit, the three phi products on
 *     int8-quantised input, the heads, the block on u, the lane mix
 *     (mhc.go:182-299), with ExpandLanes / CollapseLanes at the ends
 *     (decoder.go:283-301, mhc.go:137-170).
 * The layer is Block.run with the cross branch as its AfterAttn hook
 * (decoder.go:446-505, block.go:147-215), the FFN being the synthetic
 * model's CQ W2 SiLU(W1 .) in place of the Monarch MLP.
 *
 * A state holds one stream's caches; orc_dec_fork copies them, which the
 * reference's copy-on-append sharing (KVCache.Fork, cache.go:62-67) makes
 * indistinguishable. orc_dec_streams decodes many streams on threads, one
 * stream per thread at a time, as beams run one goroutine each
 * (internal/search/beam.go:508-521).
 *
 * TEST INFRASTRUCTURE ONLY (the checker of the device decoder and the
 * cpu_baseline of bench.py's decode leg).
 */
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

struct orc_dec_state {
    const orc_dec_model *m;
    const orc_dec_memory *mem;
    int pos;
    int8_t **kc, **vc; /* per layer: max_pos rows of dim codes */
    float **ks, **vs;  /* per layer: max_pos rows of heads scales */
    float **hist;      /* per layer: 3 x (taps - 1) raw rows of dim, oldest first; nh rows held */
    int nh;
};

static void *xcalloc(size_t n, size_t sz) {
    void *p = calloc(n ? n : 1, sz ? sz : 1);
    if (!p) abort();
    return p;
}

orc_dec_state *orc_dec_new(const orc_dec_model *m, const orc_dec_memory *mem) {
    orc_dec_state *s = xcalloc(1, sizeof *s);
    const int L = m->layers, hk = m->dim / m->head_dim;
    s->m = m;
    s->mem = mem;
    s->kc = xcalloc((size_t)L, sizeof *s->kc);
    s->vc = xcalloc((size_t)L, sizeof *s->vc);
    s->ks = xcalloc((size_t)L, sizeof *s->ks);
    s->vs = xcalloc((size_t)L, sizeof *s->vs);
    s->hist = xcalloc((size_t)L, sizeof *s->hist);
    for (int l = 0; l < L; l++) {
        s->kc[l] = xcalloc((size_t)m->max_pos * m->dim, 1);
        s->vc[l] = xcalloc((size_t)m->max_pos * m->dim, 1);
        s->ks[l] = xcalloc((size_t)m->max_pos * hk, sizeof(float));
        s->vs[l] = xcalloc((size_t)m->max_pos * hk, sizeof(float));
        if (m->taps > 1) s->hist[l] = xcalloc((size_t)3 * (m->taps - 1) * m->dim, sizeof(float));
    }
    return s;
}

void orc_dec_free(orc_dec_state *s) {
    if (!s) return;
    for (int l = 0; l < s->m->layers; l++) {
        free(s->kc[l]);
        free(s->vc[l]);
        free(s->ks[l]);
        free(s->vs[l]);
        free(s->hist[l]);
    }
    free(s->kc);
    free(s->vc);
    free(s->ks);
    free(s->vs);
    free(s->hist);
    free(s);
}

orc_dec_state *orc_dec_fork(const orc_dec_state *p) {
    const orc_dec_model *m = p->m;
    orc_dec_state *s = orc_dec_new(m, p->mem);
    const int hk = m->dim / m->head_dim;
    s->pos = p->pos;
    s->nh = p->nh;
    for (int l = 0; l < m->layers; l++) {
        memcpy(s->kc[l], p->kc[l], (size_t)p->pos * m->dim);
        memcpy(s->vc[l], p->vc[l], (size_t)p->pos * m->dim);
        memcpy(s->ks[l], p->ks[l], sizeof(float) * (size_t)p->pos * hk);
        memcpy(s->vs[l], p->vs[l], sizeof(float) * (size_t)p->pos * hk);
        if (m->taps > 1) memcpy(s->hist[l], p->hist[l], sizeof(float) * (size_t)3 * (m->taps - 1) * m->dim);
    }
    return s;
}

int orc_dec_len(const orc_dec_state *s) { return s->pos; }

/* The taps of one raw row z (width dim) at the next position against the
 * history rows hist[0 .. nh-1] (oldest first): out = sum_j taps[j] * row(i -
 * j) from 0, j ascending, each product rounded (applyTaps, attention.go:
 * 597-613, on the rows of extendTaps, cache.go:143-154). */
static void taps_row(float *out, const float *z, const float *hist, int nh, const float *w, int taps, int dim) {
    for (int c = 0; c < dim; c++) out[c] = 0.0f;
    for (int j = 0; j < taps; j++) {
        if (j > nh) break; /* positions before the first count as zero */
        const float *src = j == 0 ? z : hist + (size_t)(nh - j) * dim;
        const float *tap = w + (size_t)j * dim;
        for (int c = 0; c < dim; c++) {
            const float p = tap[c] * src[c];
            out[c] = out[c] + p;
        }
    }
}

/* h[i] += float32(s * y[i]) (block.go:186-188; cross.go:258-263 with the
 * hook's add, decoder.go:461-465). */
static void scaled_add(float *h, const float *y, float s, int n) {
    for (int i = 0; i < n; i++) {
        const float p = s * y[i];
        h[i] = h[i] + p;
    }
}

static void vadd(float *h, const float *y, int n) {
    for (int i = 0; i < n; i++) h[i] = h[i] + y[i];
}

/* The decoder block on h (dim values) at position pos, in place:
 * Block.run with the cross branch after the attention (block.go:147-215,
 * decoder.go:461-479). */
static void block(orc_dec_state *st, int l, float *h, float *w) {
    const orc_dec_model *m = st->m;
    const int D = m->dim, H = m->heads, hd = m->head_dim, hk = D / hd, F = m->ffn, pos = st->pos;
    orc_matrix *const *mt = m->mats + (size_t)l * ORC_DEC_NMATS;
    float *n = w, *q = n + D, *k = q + D, *v = k + D, *g = v + D, *a = g + D, *o = a + D, *t = o + D,
          *u = t + 3 * D;
    const float scale = (float)sqrt((double)hd);
    const int32_t p32 = pos;

    orc_zc_rmsnorm(n, h, m->gains + (size_t)(3 * l) * D, 1, D);
    {
        float *d4[4] = {q, k, v, g};
        orc_gemms((orc_matrix **)mt, 4, ORC_LUT, d4, n, 1);
    }
    if (m->taps > 0) { /* extendTaps on q, k, v (cache.go:98-102), then keep the last taps - 1 raw rows */
        const int keep = m->taps - 1;
        float *raw[3] = {q, k, v};
        for (int z = 0; z < 3; z++) {
            float *hist = keep > 0 ? st->hist[l] + (size_t)z * keep * D : NULL;
            taps_row(t, raw[z], hist, st->nh, m->taps_w + ((size_t)(l * 3 + z) * m->taps) * D, m->taps, D);
            if (keep > 0) {
                if (st->nh == keep) memmove(hist, hist + D, sizeof(float) * (size_t)(keep - 1) * D);
                memcpy(hist + (size_t)(st->nh < keep ? st->nh : keep - 1) * D, raw[z], sizeof(float) * (size_t)D);
            }
            memcpy(raw[z], t, sizeof(float) * (size_t)D);
        }
    }
    if (m->qk_norm) { /* normRotate's per-head norms (attention.go:300-303) */
        orc_zc_rmsnorm(q, q, m->qk_gains + (size_t)(l * 4 + 0) * hd, H, hd);
        orc_zc_rmsnorm(k, k, m->qk_gains + (size_t)(l * 4 + 1) * hd, hk, hd);
    }
    orc_rope(q, 1, H, hd, m->rope_cos, m->rope_sin, &p32);
    orc_rope(k, 1, hk, hd, m->rope_cos, m->rope_sin, &p32);
    orc_quantize_rows(st->kc[l] + (size_t)pos * D, st->ks[l] + (size_t)pos * hk, k, 1, D, hd);
    orc_quantize_rows(st->vc[l] + (size_t)pos * D, st->vs[l] + (size_t)pos * hk, v, 1, D, hd);
    {
        const int32_t spans[4] = {0, 0, 0, pos + 1};
        orc_attend_int8_spans(a, q, 1, H, st->kc[l], st->ks[l], D, hd, st->vc[l], st->vs[l], D, hd, pos + 1, spans,
                              scale, 1, 1, NULL);
    }
    orc_sigmoid_gate(a, g, D); /* Attention.output (attention.go:242-260) */
    orc_gemm(mt[4], ORC_LUT, o, a, 1);
    if (m->post_norm) {
        orc_zc_rmsnorm(o, o, m->post_gains + (size_t)(l * 2 + 0) * D, 1, D);
        scaled_add(h, o, m->res_scale[l * 2 + 0], D);
    } else {
        vadd(h, o, D);
    }
    /* the cross branch (cross.go:209-264) */
    orc_zc_rmsnorm(n, h, m->gains + (size_t)(3 * l + 1) * D, 1, D);
    {
        float *d2[2] = {q, g};
        orc_matrix *m2[2] = {mt[5], mt[6]};
        orc_gemms(m2, 2, ORC_LUT, d2, n, 1);
    }
    if (m->cross_norm) orc_zc_rmsnorm(q, q, m->qk_gains + (size_t)(l * 4 + 2) * hd, H, hd);
    {
        const int32_t spans[4] = {0, 0, 0, m->frames};
        orc_attend_int8_spans(a, q, 1, H, st->mem->kq[l], st->mem->ks[l], D, hd, st->mem->vq[l], st->mem->vs[l], D,
                              hd, m->frames, spans, scale, 1, 1, NULL);
    }
    orc_sigmoid_gate(a, g, D);
    orc_gemm(mt[7], ORC_LUT, o, a, 1);
    if (m->cross_norm) {
        orc_zc_rmsnorm(o, o, m->post_gains + (size_t)(l * 2 + 1) * D, 1, D);
        scaled_add(h, o, m->res_scale[l * 2 + 1], D);
    } else {
        vadd(h, o, D);
    }
    /* the FFN: m = W2 SiLU(W1 norm(h)), then m + h */
    orc_zc_rmsnorm(n, h, m->gains + (size_t)(3 * l + 2) * D, 1, D);
    orc_gemm(mt[10], ORC_LUT, u, n, 1);
    orc_silu(u, F);
    orc_gemm(mt[11], ORC_LUT, o, u, 1);
    for (int i = 0; i < D; i++) h[i] = o[i] + h[i];
}

static size_t work_floats(const orc_dec_model *m) {
    const int n = m->lanes > 0 ? m->lanes : 1;
    return (size_t)8 * m->dim + 3 * (size_t)m->dim + (size_t)m->ffn + /* block */
           (size_t)4 * n * m->dim + (size_t)4 * n + (size_t)2 * n * n + (size_t)m->dim; /* mHC */
}

int orc_dec_step(orc_dec_state *st, int token, float *logits) {
    const orc_dec_model *m = st->m;
    const int D = m->dim, n = m->lanes, L = m->layers;
    if (st->pos >= m->max_pos || token < 0 || token >= m->vocab) return -1;
    float *w = xcalloc(work_floats(m), sizeof(float));
    float *x = xcalloc((size_t)D, sizeof(float));
    float *lg = logits ? logits : xcalloc((size_t)m->vocab, sizeof(float));
    orc_row(m->emb, x, token); /* decoder.go:269-275 */
    for (int c = 0; c < D; c++) x[c] = x[c] * m->scale;
    float *blk = w + 8 * (size_t)D + 3 * (size_t)D + m->ffn;
    if (n > 0) {
        float *stream = blk, *nx = stream + (size_t)n * D, *nxq = nx + (size_t)n * D, *mix = nxq + (size_t)n * D;
        float *pl = mix + (size_t)n * D, *ql = pl + n, *hp = ql + n, *hq = hp + n, *rl = hq + n, *hr = rl + n * n;
        float *uu = hr + n * n;
        for (int k = 0; k < n; k++) memcpy(stream + (size_t)k * D, x, sizeof(float) * (size_t)D); /* ExpandLanes */
        for (int l = 0; l < L; l++) {
            orc_matrix *const *mt = m->mats + (size_t)l * ORC_DEC_NMATS;
            orc_rms_unit(nx, stream, 1, n * D);
            orc_fake_quant(nxq, nx, 1, n * D, n * D); /* the phi linears' int8 input (mhc.go:99-106) */
            float *d3[3] = {pl, ql, rl};
            orc_matrix *m3[3] = {mt[12], mt[13], mt[14]};
            orc_gemms(m3, 3, ORC_LUT, d3, nxq, 1);
            orc_mhc_heads(hp, hq, hr, uu, pl, ql, rl, stream, 1, n, D,
                          m->mhc_affine + (size_t)l * (3 + 4 * n + n * n));
            memcpy(x, uu, sizeof(float) * (size_t)D);
            block(st, l, x, w);
            orc_mhc_mix(mix, stream, hr, hq, x, uu, 1, n, D);
            memcpy(stream, mix, sizeof(float) * (size_t)n * D);
        }
        for (int c = 0; c < D; c++) { /* CollapseLanes (mhc.go:153-170) */
            float acc = 0.0f;
            for (int k = 0; k < n; k++) acc = acc + stream[(size_t)k * D + c];
            x[c] = acc / (float)n;
        }
    } else {
        for (int l = 0; l < L; l++) block(st, l, x, w);
    }
    if (m->taps > 1 && st->nh < m->taps - 1) st->nh++;
    st->pos++;
    orc_zc_rmsnorm(x, x, m->gains + (size_t)(3 * L) * D, 1, D); /* logits (decoder.go:507-523) */
    orc_gemm(m->emb, ORC_LUT, lg, x, 1);
    int32_t tok;
    orc_argmax(&tok, lg, 1, m->vocab);
    if (!logits) free(lg);
    free(x);
    free(w);
    return tok;
}

int orc_dec_greedy(orc_dec_state *st, int first, int n, int eos, int32_t *tokens, float *logits, int *stopped) {
    /* GreedyMemory's loop (greedy.go:30-69): feed the token, take the
     * argmax, stop at EOS (left out) or after n tokens. */
    int tok = first, got = 0;
    if (stopped) *stopped = 0;
    for (int i = 0; i < n; i++) {
        tok = orc_dec_step(st, tok, logits ? logits + (size_t)got * st->m->vocab : NULL);
        if (tok < 0) return -1;
        if (eos >= 0 && tok == eos) {
            if (stopped) *stopped = 1;
            break;
        }
        tokens[got++] = tok;
    }
    return got;
}

typedef struct {
    const orc_dec_model *m;
    const orc_dec_memory *mems;
    const int32_t *first;
    int32_t *tokens, *counts;
    int n, streams;
    int next;
    pthread_mutex_t mu;
} streams_job;

static void *stream_worker(void *arg) {
    streams_job *j = arg;
    for (;;) {
        pthread_mutex_lock(&j->mu);
        const int b = j->next++;
        pthread_mutex_unlock(&j->mu);
        if (b >= j->streams) return NULL;
        orc_dec_state *st = orc_dec_new(j->m, j->mems + b);
        j->counts[b] = orc_dec_greedy(st, j->first[b], j->n, -1, j->tokens + (size_t)b * j->n, NULL, NULL);
        orc_dec_free(st);
    }
}

int orc_dec_streams(const orc_dec_model *m, const orc_dec_memory *mems, int streams, const int32_t *first, int n,
                    int threads, int32_t *tokens, int32_t *counts) {
    streams_job j = {m, mems, first, tokens, counts, n, streams, 0, PTHREAD_MUTEX_INITIALIZER};
    if (threads < 1) threads = 1;
    pthread_t *th = xcalloc((size_t)threads, sizeof *th);
    int started = 0;
    for (int t = 0; t < threads; t++)
        if (pthread_create(&th[t], NULL, stream_worker, &j) == 0) started++;
        else break;
    if (started == 0) stream_worker(&j);
    for (int t = 0; t < started; t++) pthread_join(th[t], NULL);
    free(th);
    return 0;
}
