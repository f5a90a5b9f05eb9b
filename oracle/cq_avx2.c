/*
 * CPU oracle, AVX2 form of the lut kernel: the reference's amd64 path
 * (internal/cq/lut_amd64.s, used when the CPU has AVX2, lut_amd64.go:9-61),
 * restated with C intrinsics. TEST INFRASTRUCTURE ONLY (see oracle.h): it
 * serves as the CPU baseline that bench.py times, and tests/ check it against
 * the generic restatement in cq_oracle.c.
 *
 * Every float32 operation is the generic one, on the same operands and in
 * the same order, so the results are equal bit for bit (the reference's
 * internal/cq/asm_test.go requires the same of its assembly):
 *   fwht          fwhtAVX2 (lut_amd64.s:12-75): butterflies at h = 1, 2, 4
 *                 inside 8-float registers by permutes, then 8 floats per
 *                 step for h >= 8; a + b and a - b as in kernel.go:384-393
 *   tables 4-bit  lutTables4AVX2 (lut_amd64.s:199-233): a = x[q] * inv, then
 *                 cb[c] * a for 16 codes, rounded to nearest even by the
 *                 conversion, split into the 7-bit lo plane and the hi plane
 *                 (v >> 7) + 64 (lutPut, lut.go:227-233)
 *   tables 2-bit  lutTables2AVX2 (lut_amd64.s:150-197): float32(cb[c&3] * a)
 *                 + float32(cb[c>>2] * b)
 *   lookup        lutLookupAVX2 (lut_amd64.s:235-378): per 32-row block and
 *                 index byte, one 32-byte load holds the byte of every row;
 *                 byte shuffles look up both nibbles in the lo and hi planes,
 *                 the sums widen into 16-bit lanes, and at the end of each
 *                 group 128 * hi + lo - bias becomes float32 and is added to
 *                 y times norm * step, groups in order from y = 0.
 * The bound M uses the vector maximum, equal to the generic running maximum
 * for inputs without NaN.
 */
#include <immintrin.h>
#include <stdint.h>
#include <string.h>

#include "oracle.h"

enum { ROWS = 32, LUT_Q = 8191, LUT_BIAS = 64 };

int orc_have_avx2(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

#define AVX2 __attribute__((target("avx2")))

AVX2 void orc_fwht_avx2(float *x, int n) {
    /* h = 1, 2, 4 within each 8 floats: the partner of lane j at distance h
     * is one permute away; the lower lane keeps a + b, the upper a - b. */
    for (int i = 0; i < n; i += 8) {
        __m256 v = _mm256_loadu_ps(x + i);
        __m256 p = _mm256_permute_ps(v, 0xB1); /* swap within pairs */
        v = _mm256_blend_ps(_mm256_add_ps(v, p), _mm256_sub_ps(p, v), 0xAA);
        p = _mm256_permute_ps(v, 0x4E); /* swap pairs within 4 */
        v = _mm256_blend_ps(_mm256_add_ps(v, p), _mm256_sub_ps(p, v), 0xCC);
        p = _mm256_permute2f128_ps(v, v, 0x01); /* swap the halves */
        v = _mm256_blend_ps(_mm256_add_ps(v, p), _mm256_sub_ps(p, v), 0xF0);
        _mm256_storeu_ps(x + i, v);
    }
    for (int h = 8; h < n; h *= 2)
        for (int i = 0; i < n; i += 2 * h)
            for (int j = i; j < i + h; j += 8) {
                const __m256 a = _mm256_loadu_ps(x + j), b = _mm256_loadu_ps(x + j + h);
                _mm256_storeu_ps(x + j, _mm256_add_ps(a, b));
                _mm256_storeu_ps(x + j + h, _mm256_sub_ps(a, b));
            }
}

static float lut_inv(float m) { return m > 0 ? (float)LUT_Q / m : 0; } /* lut.go:219-225 */

/* Largest of the eight lanes of v. */
AVX2 static float hmax8(__m256 v) {
    __m128 m = _mm_max_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    m = _mm_max_ps(m, _mm_permute_ps(m, 0x4E));
    m = _mm_max_ps(m, _mm_permute_ps(m, 0xB1));
    return _mm_cvtss_f32(m);
}

/* The 16 entries e0 (codes 0-7) and e1 (codes 8-15), rounded to nearest
 * even, as one 32-byte table: lo plane v & 127, then hi plane (v >> 7) + 64. */
AVX2 static void put_table(uint8_t *t, __m256 e0, __m256 e1) {
    const __m256i v0 = _mm256_cvtps_epi32(e0), v1 = _mm256_cvtps_epi32(e1); /* MXCSR default: nearest even */
    /* |v| <= 8191: the int16 pack is exact; per 128-bit half it interleaves
     * v0 and v1 by fours, the 64-bit permute restores codes 0-15 in order. */
    const __m256i w = _mm256_permute4x64_epi64(_mm256_packs_epi32(v0, v1), 0xD8);
    const __m256i lo = _mm256_and_si256(w, _mm256_set1_epi16(127));
    const __m256i hi = _mm256_add_epi16(_mm256_srai_epi16(w, 7), _mm256_set1_epi16(LUT_BIAS));
    const __m256i bytes = _mm256_permute4x64_epi64(_mm256_packus_epi16(lo, hi), 0xD8);
    _mm256_storeu_si256((__m256i *)t, bytes);
}

AVX2 float orc_lut_tables4_avx2(uint8_t *tab, const float *x, int n, const float *cb, float cb_max) {
    const __m256 absmask = _mm256_castsi256_ps(_mm256_set1_epi32(0x7FFFFFFF));
    __m256 mx = _mm256_setzero_ps();
    for (int q = 0; q < n; q += 8) mx = _mm256_max_ps(mx, _mm256_and_ps(_mm256_loadu_ps(x + q), absmask));
    const float m = cb_max * hmax8(mx);
    const float inv = lut_inv(m);
    const __m256 c0 = _mm256_loadu_ps(cb), c1 = _mm256_loadu_ps(cb + 8);
    for (int q = 0; q < n; q++) {
        const __m256 a = _mm256_set1_ps(x[q] * inv);
        put_table(tab + 32 * q, _mm256_mul_ps(c0, a), _mm256_mul_ps(c1, a));
    }
    return m;
}

AVX2 float orc_lut_tables2_avx2(uint8_t *tab, const float *x, int n, const float *cb, float cb_max) {
    const __m256 absmask = _mm256_castsi256_ps(_mm256_set1_epi32(0x7FFFFFFF));
    __m256 mx = _mm256_setzero_ps();
    for (int q = 0; q < n; q += 8) {
        const __m256 v = _mm256_and_ps(_mm256_loadu_ps(x + q), absmask);
        mx = _mm256_max_ps(mx, _mm256_hadd_ps(v, v)); /* |x[2q]| + |x[2q+1]| */
    }
    const float m = cb_max * hmax8(mx);
    const float inv = lut_inv(m);
    /* codes c = 0-7 and 8-15: cb[c & 3] repeats, cb[c >> 2] is 0,0,0,0,1,1,1,1 / 2,2,2,2,3,3,3,3 */
    const __m256 clo = _mm256_setr_ps(cb[0], cb[1], cb[2], cb[3], cb[0], cb[1], cb[2], cb[3]);
    const __m256 chi0 = _mm256_setr_ps(cb[0], cb[0], cb[0], cb[0], cb[1], cb[1], cb[1], cb[1]);
    const __m256 chi1 = _mm256_setr_ps(cb[2], cb[2], cb[2], cb[2], cb[3], cb[3], cb[3], cb[3]);
    for (int q = 0; q < n / 2; q++) {
        const __m256 a = _mm256_set1_ps(x[2 * q] * inv), b = _mm256_set1_ps(x[2 * q + 1] * inv);
        const __m256 la = _mm256_mul_ps(clo, a);
        put_table(tab + 32 * q, _mm256_add_ps(la, _mm256_mul_ps(chi0, b)), _mm256_add_ps(la, _mm256_mul_ps(chi1, b)));
    }
    return m;
}

/* Rows 0-7 | 16-23 (from the low unpacks) or 8-15 | 24-31 (high unpacks)
 * of one group: 32-bit sums 128 * hi + lo - bias, in row order as two
 * 8-row vectors r0 (rows 0-7 or 8-15) and r1 (rows 16-23 or 24-31). */
AVX2 static void group_sums(__m256i slo, __m256i shi, __m256i bias, __m256i *r0, __m256i *r1) {
    const __m256i z = _mm256_setzero_si256();
    const __m256i a = _mm256_sub_epi32(
        _mm256_add_epi32(_mm256_slli_epi32(_mm256_unpacklo_epi16(shi, z), 7), _mm256_unpacklo_epi16(slo, z)), bias);
    const __m256i b = _mm256_sub_epi32(
        _mm256_add_epi32(_mm256_slli_epi32(_mm256_unpackhi_epi16(shi, z), 7), _mm256_unpackhi_epi16(slo, z)), bias);
    *r0 = _mm256_permute2x128_si256(a, b, 0x20);
    *r1 = _mm256_permute2x128_si256(a, b, 0x31);
}

AVX2 void orc_lut_lookup_avx2(float *y, const uint8_t *idx, const uint8_t *tab, const float *norm, const float *steps,
                              int blocks, int groups, int gb) {
    const __m256i nib = _mm256_set1_epi8(0x0F), z = _mm256_setzero_si256();
    const __m256i bias = _mm256_set1_epi32(128 * LUT_BIAS * 2 * gb);
    const size_t row_bytes = (size_t)groups * gb;
    for (int b = 0; b < blocks; b++) {
        const uint8_t *ib = idx + (size_t)b * row_bytes * ROWS;
        const float *nb = norm + (size_t)b * groups * ROWS;
        __m256 y0 = _mm256_setzero_ps(), y1 = y0, y2 = y0, y3 = y0; /* rows 0-7, 8-15, 16-23, 24-31 */
        for (int g = 0; g < groups; g++) {
            /* uint16 sums: *_l rows 0-7 | 16-23, *_h rows 8-15 | 24-31; a byte
             * sums two plane entries of at most 127, so gb <= 256 bytes fit */
            __m256i lo_l = z, lo_h = z, hi_l = z, hi_h = z;
            for (int j = g * gb; j < (g + 1) * gb; j++) {
                const __m256i v = _mm256_loadu_si256((const __m256i *)(ib + (size_t)j * ROWS));
                const __m256i n0 = _mm256_and_si256(v, nib), n1 = _mm256_and_si256(_mm256_srli_epi16(v, 4), nib);
                const uint8_t *t = tab + 64 * (size_t)j;
                const __m256i tl0 = _mm256_broadcastsi128_si256(_mm_loadu_si128((const __m128i *)t));
                const __m256i th0 = _mm256_broadcastsi128_si256(_mm_loadu_si128((const __m128i *)(t + 16)));
                const __m256i tl1 = _mm256_broadcastsi128_si256(_mm_loadu_si128((const __m128i *)(t + 32)));
                const __m256i th1 = _mm256_broadcastsi128_si256(_mm_loadu_si128((const __m128i *)(t + 48)));
                const __m256i lo = _mm256_add_epi8(_mm256_shuffle_epi8(tl0, n0), _mm256_shuffle_epi8(tl1, n1));
                const __m256i hi = _mm256_add_epi8(_mm256_shuffle_epi8(th0, n0), _mm256_shuffle_epi8(th1, n1));
                lo_l = _mm256_add_epi16(lo_l, _mm256_unpacklo_epi8(lo, z));
                lo_h = _mm256_add_epi16(lo_h, _mm256_unpackhi_epi8(lo, z));
                hi_l = _mm256_add_epi16(hi_l, _mm256_unpacklo_epi8(hi, z));
                hi_h = _mm256_add_epi16(hi_h, _mm256_unpackhi_epi8(hi, z));
            }
            const __m256 step = _mm256_set1_ps(steps[g]);
            const float *ng = nb + (size_t)g * ROWS;
            __m256i s0, s1, s2, s3;
            group_sums(lo_l, hi_l, bias, &s0, &s2);
            group_sums(lo_h, hi_h, bias, &s1, &s3);
            /* y += float32(sum) * (norm * step), as lutLookupGeneric */
            y0 = _mm256_add_ps(y0, _mm256_mul_ps(_mm256_cvtepi32_ps(s0), _mm256_mul_ps(_mm256_loadu_ps(ng), step)));
            y1 = _mm256_add_ps(y1, _mm256_mul_ps(_mm256_cvtepi32_ps(s1), _mm256_mul_ps(_mm256_loadu_ps(ng + 8), step)));
            y2 = _mm256_add_ps(y2, _mm256_mul_ps(_mm256_cvtepi32_ps(s2), _mm256_mul_ps(_mm256_loadu_ps(ng + 16), step)));
            y3 = _mm256_add_ps(y3, _mm256_mul_ps(_mm256_cvtepi32_ps(s3), _mm256_mul_ps(_mm256_loadu_ps(ng + 24), step)));
        }
        float *yb = y + (size_t)b * ROWS;
        _mm256_storeu_ps(yb, y0);
        _mm256_storeu_ps(yb + 8, y1);
        _mm256_storeu_ps(yb + 16, y2);
        _mm256_storeu_ps(yb + 24, y3);
    }
}
