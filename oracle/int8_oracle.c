/*
 * CPU oracle, int8 KV part: a plain-C restatement of go-whistle's
 * internal/needle int8 numerics. TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Reference files followed (paths relative to the go-whistle repository):
 *   internal/needle/int8.go:36-55       QuantizeRow
 *   internal/needle/int8.go:116-141     QuantizeRows, Int8Rows.Append
 *   internal/needle/int8.go:62-88       fakeQuant, quantInput (Linear WithInt8Input)
 *   internal/needle/int8.go:208-300     AttendInt8Spans, int8Logits, dotsF32I8
 *   internal/needle/int8kernel.go:346-368  dotsI8Generic, axpysI8Generic
 *   internal/needle/exp.go:21-31        expSubSumGeneric
 *   internal/needle/exp_amd64.go:13-25  expSubSumF32 (kernel on the multiple-of-8
 *                                       prefix, Go on the tail)
 *   internal/needle/exp_amd64.s:68-124  expSubSumAVX2: Cephes expf (S. L. Moshier's
 *                                       published single-precision exp) with the
 *                                       kernel's FMA steps and 8-lane sum
 *   internal/needle/load.go:125-138     softmaxInPlace
 * With the AVX2 CPU mode (orc_set_cpu) the attention runs the AVX2 forms of
 * dotsI8, axpysI8 and the exp kernel (int8_avx2.c), bit for bit these.
 *
 * How each part is pinned without running the reference (tests/):
 *   QuantizeRow   the reference's hand vectors (int8_test.go:19-34) and its
 *                 invariants s = max|x|/127, |x - s q| <= s/2, no -128
 *   dotsI8        brute force in int64
 *   axpysI8 / dotsF32I8  float64 recompute within the float32 bound
 *   expSubSum     float64 exp within 2 float32 ulps, the flush below
 *                 -87.33, exp(0) = 1 (exp_test.go:21-145)
 *   AttendInt8    float64 recompute on the dequantised codes: probabilities
 *                 within 2e-6, summing to 1 within 1e-5, outputs within 2e-6
 *                 (int8_test.go:212-284)
 *   The summation orders (the 8-lane exp sum, keys in order in axpys) are
 *   restated from the reference; their last bits are parity unpinned beyond
 *   these bounds.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static float gomax(float a, float b) {
    if (a != a || b != b) return NAN;
    if (a == 0 && b == 0) return signbit(a) ? b : a;
    return a > b ? a : b;
}

float orc_quantize_row(int8_t *q, const float *x, int n) {
    /* int8.go:36-55 */
    float m = 0;
    for (int i = 0; i < n; i++) m = gomax(m, fabsf(x[i]));
    float s = 1;
    if (m > 0) s = m / 127.0f;
    for (int i = 0; i < n; i++) {
        float d = x[i] / s;
        double r = rint((double)d);
        /* min(max(r, -128), 127) with Go's NaN-propagating max and min: a
         * NaN stays NaN, and int8 of it is 0 */
        if (r < -128) r = -128;
        if (r > 127) r = 127;
        q[i] = go_int8_of(r);
    }
    return s;
}

void orc_quantize_rows(int8_t *q, float *s, const float *x, int rows, int cols, int width) {
    /* int8.go:116-141: per chunk of width values */
    int chunks = rows * (cols / width);
    for (int c = 0; c < chunks; c++) s[c] = orc_quantize_row(q + (size_t)c * width, x + (size_t)c * width, width);
}

void orc_fake_quant(float *dst, const float *x, long rows, int cols, int width) {
    /* fakeQuant (int8.go:62-75): QuantizeRow per chunk, then float32(q) * s;
     * dst may be x */
    long chunks = rows * (cols / width);
    int8_t *q = malloc((size_t)width + 1);
    for (long c = 0; c < chunks; c++) {
        float s = orc_quantize_row(q, x + c * width, width);
        for (int i = 0; i < width; i++) dst[c * width + i] = (float)q[i] * s;
    }
    free(q);
}

void orc_dots_i8(int32_t *dst, int n, const int8_t *q, int width, const int8_t *k, int stride) {
    /* int8kernel.go:346-357 */
    for (int j = 0; j < n; j++) {
        const int8_t *row = k + (size_t)j * stride;
        int32_t s = 0;
        for (int i = 0; i < width; i++) s += (int32_t)q[i] * (int32_t)row[i];
        dst[j] = s;
    }
}

void orc_axpys_i8(float *out, int width, const float *w, int n, const int8_t *v, int stride) {
    /* int8kernel.go:360-368: keys in order, each product rounded */
    for (int j = 0; j < n; j++) {
        const int8_t *row = v + (size_t)j * stride;
        for (int d = 0; d < width; d++) {
            float p = w[j] * (float)row[d];
            out[d] += p;
        }
    }
}

void orc_dots_f32_i8(float *dst, int n, const float *q, int width, const int8_t *k, int stride) {
    /* int8.go:289-300 */
    for (int j = 0; j < n; j++) {
        const int8_t *row = k + (size_t)j * stride;
        float s = 0;
        for (int i = 0; i < width; i++) {
            float p = q[i] * (float)row[i];
            s += p;
        }
        dst[j] = s;
    }
}

static float exp_sub_sum_generic(float *s, int n, float m) {
    /* exp.go:21-31: float32(math.Exp(float64(v - m))), summed in order */
    float sum = 0;
    for (int i = 0; i < n; i++) {
        float d = s[i] - m;
        float e = (float)exp((double)d);
        s[i] = e;
        sum += e;
    }
    return sum;
}

/* One lane of exp_amd64.s:84-112 (constants exp_amd64.s:7-51). */
float orc_exp_lane(float x) {
    /* exp_amd64.s:7-51, bit for bit */
    const float log2e = 0x1.715476p+0f;  /* 0x3FB8AA3B */
    const float ln2hi = 0x1.63p-1f;      /* 0x3F318000 */
    const float ln2lo = -0x1.bd0106p-13f; /* 0xB95E8083 */
    const float c6 = 0x1.a0d2cep-13f, c5 = 0x1.6e879cp-10f, c4 = 0x1.111210p-7f;
    const float c3 = 0x1.555382p-5f, c2 = 0x1.555554p-3f, c1 = 0x1p-1f;
    const float lo = -0x1.5d51ecp+6f;   /* 0xC2AEA8F6, about -87.33 */
    int lt = x < lo;
    float xc = (x != x) ? x : (lo > x ? lo : x); /* VMAXPS keeps a NaN x */
    float k = rintf(xc * log2e);
    float r = fmaf(-k, ln2hi, xc);
    r = fmaf(-k, ln2lo, r);
    float r2 = r * r;
    float p = c6;
    p = fmaf(p, r, c5);
    p = fmaf(p, r, c4);
    p = fmaf(p, r, c3);
    p = fmaf(p, r, c2);
    p = fmaf(p, r, c1);
    float y = fmaf(p, r2, r);
    y = y + 1.0f;
    int32_t ki = (k != k || k >= 2147483648.0f || k < -2147483648.0f) ? INT32_MIN : (int32_t)k; /* VCVTTPS2DQ */
    uint32_t bits;
    memcpy(&bits, &y, 4);
    bits += (uint32_t)ki << 23;
    memcpy(&y, &bits, 4);
    return lt ? 0.0f : y;
}

static float exp_sub_sum_avx2(float *s, int n8, float m) {
    /* exp_amd64.s:68-124: lane l sums elements l, l+8, ...; then
     * (lo128 + hi128) and two horizontal adds. */
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = 0; i < n8; i += 8)
        for (int l = 0; l < 8; l++) {
            float e = orc_exp_lane(s[i + l] - m);
            s[i + l] = e;
            acc[l] = acc[l] + e;
        }
    float x0 = acc[0] + acc[4], x1 = acc[1] + acc[5], x2 = acc[2] + acc[6], x3 = acc[3] + acc[7];
    float h0 = x0 + x1, h1 = x2 + x3;
    return h0 + h1;
}

float orc_exp_sub_sum(float *s, int n, float m, int variant) {
    if (variant == 0) return exp_sub_sum_generic(s, n, m);
    /* exp_amd64.go:13-25 */
    int n8 = n & ~7;
    if (n8 == 0) return exp_sub_sum_generic(s, n, m);
    float sum = orc_cpu_avx2() ? orc_exp_sub_sum_avx2(s, n8, m) : exp_sub_sum_avx2(s, n8, m);
    if (n8 == n) return sum;
    float tail = exp_sub_sum_generic(s + n8, n - n8, m);
    return sum + tail;
}

void orc_softmax(float *s, int n, int variant) {
    /* load.go:128-138 */
    float m = -INFINITY;
    for (int i = 0; i < n; i++) m = gomax(m, s[i]);
    float sum = orc_exp_sub_sum(s, n, m, variant);
    for (int i = 0; i < n; i++) s[i] /= sum;
}

/* dotsI8Kernel / axpysI8Kernel (int8kernel_amd64.go:13-33): the AVX2 forms
 * for widths that are positive multiples of 16 when the CPU mode asks for
 * them, the generic loops otherwise; the same bits either way. */
static void dots_i8(int32_t *dst, int n, const int8_t *q, int width, const int8_t *k, int stride) {
    if (orc_cpu_avx2() && width > 0 && width % 16 == 0)
        orc_dots_i8_avx2(dst, n, q, width, k, stride);
    else
        orc_dots_i8(dst, n, q, width, k, stride);
}

static void axpys_i8(float *out, int width, const float *w, int n, const int8_t *v, int stride) {
    if (orc_cpu_avx2() && width > 0 && width % 16 == 0)
        orc_axpys_i8_avx2(out, width, w, n, v, stride);
    else
        orc_axpys_i8(out, width, w, n, v, stride);
}

int orc_attend_int8_spans(float *out, const float *q, int t, int heads, const int8_t *kq, const float *ks,
                          int k_cols, int qk, const int8_t *vq, const float *vs, int v_cols, int vd, int nk,
                          const int32_t *spans, float scale, int quant_q, int exp_variant, float *probs) {
    /* int8.go:208-272 */
    int kv_heads = k_cols / qk;
    if (kv_heads <= 0 || heads % kv_heads != 0) return -1;
    memset(out, 0, sizeof(float) * (size_t)t * heads * vd);
    int8_t *q8 = malloc((size_t)qk + 1);
    int32_t *dots = malloc(sizeof(int32_t) * ((size_t)nk + 1));
    float *w = malloc(sizeof(float) * ((size_t)nk + 1));
    for (int h = 0; h < heads; h++) {
        int kv = h / (heads / kv_heads);
        for (int i = 0; i < t; i++) {
            const int32_t *sp = spans + 4 * (size_t)i;
            int len0 = sp[1] - sp[0], len1 = sp[3] - sp[2];
            const float *qi = q + ((size_t)i * heads + h) * qk;
            float *s = w;
            float sq = 0;
            if (quant_q) sq = orc_quantize_row(q8, qi, qk);
            int o = 0;
            for (int p = 0; p < 2; p++) {
                int lo = sp[2 * p], len = p == 0 ? len0 : len1;
                float *sj = s + o;
                o += len;
                if (quant_q) {
                    /* int8Logits (int8.go:278-285) */
                    dots_i8(dots, len, q8, qk, kq + (size_t)lo * k_cols + (size_t)kv * qk, k_cols);
                    for (int j = 0; j < len; j++) {
                        float sc = sq * ks[(size_t)(lo + j) * kv_heads + kv];
                        float a = (float)dots[j] * sc;
                        sj[j] = a / scale;
                    }
                    continue;
                }
                orc_dots_f32_i8(sj, len, qi, qk, kq + (size_t)lo * k_cols + (size_t)kv * qk, k_cols);
                for (int j = 0; j < len; j++) {
                    float a = sj[j] * ks[(size_t)(lo + j) * kv_heads + kv];
                    sj[j] = a / scale;
                }
            }
            orc_softmax(s, len0 + len1, exp_variant);
            o = 0;
            for (int p = 0; p < 2; p++) {
                int lo = sp[2 * p], len = p == 0 ? len0 : len1;
                float *sj = s + o;
                const float *vsp = vs + (size_t)lo * kv_heads;
                if (probs) memcpy(probs + ((size_t)i * heads + h) * nk + lo, sj, sizeof(float) * (size_t)len);
                for (int j = 0; j < len; j++) sj[j] *= vsp[(size_t)j * kv_heads + kv];
                axpys_i8(out + ((size_t)i * heads + h) * vd, vd, sj, len,
                             vq + (size_t)lo * v_cols + (size_t)kv * vd, v_cols);
                o += len;
            }
        }
    }
    free(q8);
    free(dots);
    free(w);
    return 0;
}
