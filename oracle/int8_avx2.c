/*
 * CPU oracle, AVX2 forms of the int8 attention kernels: the reference's
 * amd64 path (internal/needle/int8kernel_amd64.go:9-33 picks them on AVX2
 * CPUs for widths that are multiples of 16; exp_amd64.go:13-25 the exp
 * kernel), restated with C intrinsics. TEST INFRASTRUCTURE ONLY (see
 * oracle.h): the CPU baseline that bench.py times runs them, and tests/
 * hold them to int8_oracle.c bit for bit.
 *   dotsI8    int8kernel_amd64.s dotsI8AVX2: 16 codes at a time widened to
 *             int16, multiplied and added in pairs into eight int32 lanes;
 *             the integer sums are exact in any order
 *   axpysI8   axpysI8AVX2: per 16 outputs, the keys in order, each code
 *             widened and converted, times w[j], then added (no FMA), as
 *             float32(w * c) + out
 *   exp       expSubSumAVX2 (exp_amd64.s:68-124): the Cephes lane of
 *             orc_exp_lane on eight lanes at once with the same fused steps,
 *             lane l summing elements l, l+8, ..., then the halves and two
 *             pairwise adds
 */
#include <immintrin.h>
#include <stdint.h>

#include "oracle.h"

#define AVX2 __attribute__((target("avx2")))
#define AVX2FMA __attribute__((target("avx2,fma")))

AVX2 void orc_dots_i8_avx2(int32_t *dst, int n, const int8_t *q, int width, const int8_t *k, int stride) {
    for (int j = 0; j < n; j++) {
        const int8_t *row = k + (size_t)j * stride;
        __m256i acc = _mm256_setzero_si256();
        for (int i = 0; i < width; i += 16) {
            const __m256i a = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(q + i)));
            const __m256i b = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(row + i)));
            acc = _mm256_add_epi32(acc, _mm256_madd_epi16(a, b));
        }
        __m128i s = _mm_add_epi32(_mm256_castsi256_si128(acc), _mm256_extracti128_si256(acc, 1));
        s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
        s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
        dst[j] = _mm_cvtsi128_si32(s);
    }
}

AVX2 void orc_axpys_i8_avx2(float *out, int width, const float *w, int n, const int8_t *v, int stride) {
    for (int d = 0; d < width; d += 16) {
        __m256 o0 = _mm256_loadu_ps(out + d), o1 = _mm256_loadu_ps(out + d + 8);
        for (int j = 0; j < n; j++) {
            const int8_t *c = v + (size_t)j * stride + d;
            const __m256 wj = _mm256_set1_ps(w[j]);
            const __m256 c0 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)c)));
            const __m256 c1 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)(c + 8))));
            o0 = _mm256_add_ps(o0, _mm256_mul_ps(wj, c0));
            o1 = _mm256_add_ps(o1, _mm256_mul_ps(wj, c1));
        }
        _mm256_storeu_ps(out + d, o0);
        _mm256_storeu_ps(out + d + 8, o1);
    }
}

/* orc_exp_lane on eight lanes (exp_amd64.s:84-112). */
AVX2FMA static __m256 exp8(__m256 x) {
    const __m256 lo = _mm256_set1_ps(-0x1.5d51ecp+6f);
    const __m256 lt = _mm256_cmp_ps(x, lo, _CMP_LT_OQ);
    const __m256 xc = _mm256_max_ps(lo, x); /* the second operand (x) where either is NaN */
    const __m256 k = _mm256_round_ps(_mm256_mul_ps(xc, _mm256_set1_ps(0x1.715476p+0f)),
                                     _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    __m256 r = _mm256_fnmadd_ps(k, _mm256_set1_ps(0x1.63p-1f), xc);
    r = _mm256_fnmadd_ps(k, _mm256_set1_ps(-0x1.bd0106p-13f), r);
    const __m256 r2 = _mm256_mul_ps(r, r);
    __m256 p = _mm256_set1_ps(0x1.a0d2cep-13f);
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0x1.6e879cp-10f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0x1.111210p-7f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0x1.555382p-5f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0x1.555554p-3f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0x1p-1f));
    __m256 y = _mm256_fmadd_ps(p, r2, r);
    y = _mm256_add_ps(y, _mm256_set1_ps(1.0f));
    const __m256i ki = _mm256_cvttps_epi32(k); /* INT32_MIN for NaN or out of range */
    y = _mm256_castsi256_ps(_mm256_add_epi32(_mm256_castps_si256(y), _mm256_slli_epi32(ki, 23)));
    return _mm256_andnot_ps(lt, y);
}

AVX2FMA float orc_exp_sub_sum_avx2(float *s, int n8, float m) {
    const __m256 mv = _mm256_set1_ps(m);
    __m256 acc = _mm256_setzero_ps();
    for (int i = 0; i < n8; i += 8) {
        const __m256 e = exp8(_mm256_sub_ps(_mm256_loadu_ps(s + i), mv));
        _mm256_storeu_ps(s + i, e);
        acc = _mm256_add_ps(acc, e);
    }
    const __m128 x = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    /* (x0 + x1) + (x2 + x3) */
    const float h0 = _mm_cvtss_f32(x) + _mm_cvtss_f32(_mm_shuffle_ps(x, x, 1));
    const float h1 = _mm_cvtss_f32(_mm_shuffle_ps(x, x, 2)) + _mm_cvtss_f32(_mm_shuffle_ps(x, x, 3));
    return h0 + h1;
}
