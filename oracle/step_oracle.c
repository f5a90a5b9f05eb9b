/*
 * CPU oracle, decode-step float blocks: plain C restatements of the
 * reference's ZCRMSNorm, RoPE and greedy argmax, and the synthetic decoder's
 * SiLU. TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Reference files followed (paths relative to the go-whistle repository):
 *   internal/needle/norm.go:53-66, 84-109  ZCRMSNorm.Apply, rowRMS, meanSquare
 *   internal/needle/rope.go:17-44, 69-81   NewRope (tables built in Python by
 *                                          the same steps), Rope.apply
 *   internal/decoder/greedy.go:181-191     argmax
 *   internal/needle/attention.go:245-249   Attention.output's gate
 *   internal/needle/load.go:120-123        sigmoid = float32(1/(1 + exp(-float64(x))))
 *   internal/needle/norm.go:68-81          RMSUnit
 *   internal/needle/mhc.go:182-300         MHC.forward's heads, lane sum and mix
 *   internal/needle/mhc.go:301-417         sinkhorn (exp domain in float64; log
 *                                          domain in float32 past its range)
 *
 * Pinned by tests/test_oracle_step.py: ZCRMSNorm against float64 and a
 * closed form (a constant row); RoPE against the float64 rotation and the
 * identity at position 0; argmax against numpy's first-index argmax with
 * planted ties; SiLU against float64 x*sigmoid(x) within a few ulps; the
 * float64 exp against the C library's exp (within 1 ulp, equal in nearly all
 * cases) and exact powers of e; the gate's sigmoid against float32(1/(1 +
 * libm exp(-x))) bit for bit and its closed forms (0 -> 0.5, tails 0 and 1).
 *
 * The reference's sigmoid calls Go's math.Exp (a dependency outside the
 * reference: the Go standard library); exp here is fdlibm's method, whose
 * float64 result is within 1 ulp of Go's, so the float32 sigmoid is the
 * same except where the float64 value lies within 1 ulp of a float32
 * rounding midpoint.
 */
#include <math.h>
#include <stdint.h>

#include "oracle.h"

void orc_zc_rmsnorm(float *dst, const float *x, const float *gain, int rows, int dim) {
    for (int r = 0; r < rows; r++) {
        const float *row = x + (size_t)r * dim;
        float *out = dst + (size_t)r * dim;
        /* meanSquare (norm.go:91-109) */
        double s0 = 0, s1 = 0, s2 = 0, s3 = 0;
        int i = 0;
        for (; i + 3 < dim; i += 4) {
            s0 += (double)row[i] * (double)row[i];
            s1 += (double)row[i + 1] * (double)row[i + 1];
            s2 += (double)row[i + 2] * (double)row[i + 2];
            s3 += (double)row[i + 3] * (double)row[i + 3];
        }
        for (; i < dim; i++) s0 += (double)row[i] * (double)row[i];
        float ms = (float)((s0 + s1 + s2 + s3) / (double)dim);
        /* rowRMS (norm.go:84-86) */
        float e = ms + 1e-6f;
        float rms = (float)sqrt((double)e);
        for (int c = 0; c < dim; c++) {
            float gx = gain[c] * row[c];
            out[c] = gx / rms;
        }
    }
}

void orc_rope(float *x, int rows, int heads, int head_dim, const float *cos_t, const float *sin_t, const int32_t *pos) {
    /* Rope.apply (rope.go:69-81) on every head of every row */
    int h = head_dim / 2;
    for (int r = 0; r < rows; r++) {
        const float *cs = cos_t + (size_t)pos[r] * h, *sn = sin_t + (size_t)pos[r] * h;
        for (int hd = 0; hd < heads; hd++) {
            float *x1 = x + (size_t)r * heads * head_dim + (size_t)hd * head_dim, *x2 = x1 + h;
            for (int i = 0; i < h; i++) {
                float a = x1[i], b = x2[i];
                float ac = a * cs[i], bs = b * sn[i], bc = b * cs[i], as = a * sn[i];
                x1[i] = ac - bs;
                x2[i] = bc + as;
            }
        }
    }
}

void orc_argmax(int32_t *out, const float *v, int rows, int n) {
    /* greedy.go:182-191 */
    for (int r = 0; r < rows; r++) {
        const float *row = v + (size_t)r * n;
        int best = 0;
        for (int i = 0; i < n; i++)
            if (row[i] > row[best]) best = i;
        out[r] = best;
    }
}

void orc_silu(float *x, long n) {
    /* x * sigmoid(x), sigmoid from the exponent lane on non-positive arguments */
    for (long i = 0; i < n; i++) {
        float v = x[i], s;
        if (v >= 0.0f) {
            float e = orc_exp_lane(-v);
            float d = 1.0f + e;
            s = 1.0f / d;
        } else {
            float e = orc_exp_lane(v);
            float d = 1.0f + e;
            s = e / d;
        }
        x[i] = v * s;
    }
}

double orc_exp64(double x) {
    /* fdlibm e_exp.c (Sun Microsystems, 1993), the steps of Go's portable
     * math.Exp: x = k ln2 + r, r = hi - lo, exp(r) = 1 - ((lo - r c/(2 - c)) - hi) */
    const double ln2hi = 6.93147180369123816490e-01, ln2lo = 1.90821492927058770002e-10;
    const double log2e = 1.44269504088896338700e+00;
    const double p1 = 1.66666666666666019037e-01, p2 = -2.77777777770155933842e-03;
    const double p3 = 6.61375632143793436117e-05, p4 = -1.65339022054652515390e-06;
    const double p5 = 4.13813679705723846039e-08;
    if (x != x) return x;
    if (x > 7.09782712893383973096e+02) return HUGE_VAL;
    if (x < -7.45133219101941108420e+02) return 0.0;
    if (x > -3.7252902984619140625e-09 && x < 3.7252902984619140625e-09) return 1.0 + x;
    double kf = x < 0.0 ? log2e * x - 0.5 : log2e * x + 0.5;
    int k = (int)kf;
    double hi = x - (double)k * ln2hi, lo = (double)k * ln2lo;
    double r = hi - lo, t = r * r;
    double c = r - t * (p1 + t * (p2 + t * (p3 + t * (p4 + t * p5))));
    double y = 1.0 - ((lo - (r * c) / (2.0 - c)) - hi);
    return ldexp(y, k);
}

float orc_gate_sigmoid(float x) {
    double e = orc_exp64(-(double)x);
    return (float)(1.0 / (1.0 + e));
}

void orc_sigmoid_gate(float *out, float *gate, long n) {
    /* Attention.output (attention.go:245-249): gate = sigmoid(gate), out *= gate */
    for (long i = 0; i < n; i++) {
        gate[i] = orc_gate_sigmoid(gate[i]);
        out[i] *= gate[i];
    }
}

static float mean_square(const float *row, int dim) {
    /* meanSquare (norm.go:91-109): four float64 partial sums, float32 result */
    double s0 = 0, s1 = 0, s2 = 0, s3 = 0;
    int i = 0;
    for (; i + 3 < dim; i += 4) {
        s0 += (double)row[i] * (double)row[i];
        s1 += (double)row[i + 1] * (double)row[i + 1];
        s2 += (double)row[i + 2] * (double)row[i + 2];
        s3 += (double)row[i + 3] * (double)row[i + 3];
    }
    for (; i < dim; i++) s0 += (double)row[i] * (double)row[i];
    return (float)((s0 + s1 + s2 + s3) / (double)dim);
}

void orc_rms_unit(float *dst, const float *x, int rows, int dim) {
    /* RMSUnit (norm.go:68-81): v * float32(1 / sqrt(float64(ms + eps))) */
    for (int r = 0; r < rows; r++) {
        const float *row = x + (size_t)r * dim;
        float e = mean_square(row, dim) + 1e-6f;
        float inv = (float)(1.0 / sqrt((double)e));
        for (int c = 0; c < dim; c++) dst[(size_t)r * dim + c] = row[c] * inv;
    }
}

/* Go's built-in max and min for float32, and slices.Max / slices.Min: NaN
 * when any operand is NaN. */
static float gomax(float a, float b) {
    if (a != a || b != b) return NAN;
    if (a == 0 && b == 0) return signbit(a) ? b : a;
    return a > b ? a : b;
}
static float gomin(float a, float b) {
    if (a != a || b != b) return NAN;
    if (a == 0 && b == 0) return signbit(a) ? a : b;
    return a < b ? a : b;
}

static float log_sum_exp(const float *k, int off, int stride, int n) {
    /* logSumExp (mhc.go:401-417) */
    float m = -INFINITY;
    for (int i = 0; i < n; i++) m = gomax(m, k[off + i * stride]);
    if (isinf(m)) m = 0.0f;
    float s = 0.0f;
    for (int i = 0; i < n; i++) s += (float)orc_exp64((double)(k[off + i * stride] - m));
    return m + (float)log((double)s);
}

void orc_sinkhorn(float *k, int n, int iters) {
    /* sinkhorn (mhc.go:301-399): the float64 exp domain while the logits'
     * spread allows it, else the float32 log domain */
    float lo = k[0], hi = k[0];
    for (int i = 1; i < n * n; i++) {
        lo = gomin(lo, k[i]);
        hi = gomax(hi, k[i]);
    }
    double spread = (double)hi - (double)lo;
    if (!(isinf(spread) || isnan(spread) || spread + 2.0 * iters * log((double)n) > 700.0)) {
        double e[64];
        for (int i = 0; i < n * n; i++) e[i] = orc_exp64((double)k[i] - (double)hi);
        for (int it = 0; it < iters; it++) {
            for (int r = 0; r < n; r++) {
                double s = 0;
                for (int c = 0; c < n; c++) s += e[r * n + c];
                for (int c = 0; c < n; c++) e[r * n + c] /= s;
            }
            for (int c = 0; c < n; c++) {
                double s = 0;
                for (int r = 0; r < n; r++) s += e[r * n + c];
                for (int r = 0; r < n; r++) e[r * n + c] /= s;
            }
        }
        for (int i = 0; i < n * n; i++) k[i] = (float)e[i];
        return;
    }
    for (int it = 0; it < iters; it++) {
        for (int r = 0; r < n; r++) {
            float l = log_sum_exp(k, r * n, 1, n);
            for (int c = 0; c < n; c++) k[r * n + c] -= l;
        }
        for (int c = 0; c < n; c++) {
            float l = log_sum_exp(k, c, n, n);
            for (int r = 0; r < n; r++) k[r * n + c] -= l;
        }
    }
    for (int i = 0; i < n * n; i++) k[i] = (float)orc_exp64((double)k[i]);
}

void orc_mhc_heads(float *h_pre, float *h_post, float *h_res, float *u, const float *pre_l, const float *post_l,
                   const float *res_l, const float *stream, int rows, int n, int dim, const float *affine) {
    /* MHC.logits' affine maps (mhc.go:246-263; affine = {a_pre, a_post,
     * a_res, b_pre[n], pre_off[n], b_post[n], post_off[n], b_res[n*n]} or
     * NULL for none), then forward's heads and lane sum (mhc.go:204-219):
     * h_pre = sigmoid, u = sum_k h_pre[k] stream[k] (in k order), h_post =
     * 2 sigmoid, h_res = sinkhorn, 20 iterations */
    for (int i = 0; i < rows; i++) {
        for (int k = 0; k < n; k++) {
            float p = pre_l[i * n + k], q = post_l[i * n + k];
            if (affine) {
                float ap = affine[0] * p;
                p = ap + affine[3 + k] + affine[3 + n + k];
                float aq = affine[1] * q;
                q = aq + affine[3 + 2 * n + k] + affine[3 + 3 * n + k];
            }
            h_pre[i * n + k] = orc_gate_sigmoid(p);
            h_post[i * n + k] = 2.0f * orc_gate_sigmoid(q);
        }
        float *ui = u + (size_t)i * dim;
        for (int c = 0; c < dim; c++) ui[c] = 0.0f;
        for (int k = 0; k < n; k++) {
            const float *sk = stream + ((size_t)i * n + k) * dim;
            for (int c = 0; c < dim; c++) ui[c] += h_pre[i * n + k] * sk[c];
        }
        float *hr = h_res + (size_t)i * n * n;
        for (int k = 0; k < n * n; k++) {
            float v = res_l[(size_t)i * n * n + k];
            if (affine) {
                float av = affine[2] * v;
                v = av + affine[3 + 4 * n + k];
            }
            hr[k] = v;
        }
        orc_sinkhorn(hr, n, 20);
    }
}

void orc_mhc_mix(float *out, const float *stream, const float *h_res, const float *h_post, const float *block_out,
                 const float *u, int rows, int n, int dim) {
    /* y = block(u) - u, then mix (mhc.go:229-234, 266-299): out[a] = sum_b
     * h_res[a, b] stream[b] (in b order) + h_post[a] y */
    for (int i = 0; i < rows; i++) {
        for (int a = 0; a < n; a++) {
            float *o = out + ((size_t)i * n + a) * dim;
            for (int c = 0; c < dim; c++) o[c] = 0.0f;
            for (int b = 0; b < n; b++) {
                const float h = h_res[((size_t)i * n + a) * n + b];
                const float *sb = stream + ((size_t)i * n + b) * dim;
                for (int c = 0; c < dim; c++) o[c] += h * sb[c];
            }
            const float hp = h_post[i * n + a];
            for (int c = 0; c < dim; c++) {
                float y = block_out[(size_t)i * dim + c] - u[(size_t)i * dim + c];
                o[c] += hp * y;
            }
        }
    }
}
