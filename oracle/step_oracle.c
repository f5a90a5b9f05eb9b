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
 *
 * Pinned by tests/test_oracle_step.py: ZCRMSNorm against float64 and a
 * closed form (a constant row); RoPE against the float64 rotation and the
 * identity at position 0; argmax against numpy's first-index argmax with
 * planted ties; SiLU against float64 x*sigmoid(x) within a few ulps.
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
