// Device helpers shared by the kernels, each the reference's arithmetic in
// its order (the library is built with -ffp-contract=off: no fused
// multiply-adds beyond the explicit fmaf of the exponent kernel).
#pragma once

#include <hip/hip_runtime.h>

#include <climits>

namespace cqhip {

// Lane l's value from lane l ^ H of the wavefront, without the LDS
// crossbar where a DPP move reaches: quad permutes for H = 1, 2, row shifts
// within 16 lanes for 4, 8 (lane + H below, lane - H above), a ds_swizzle
// for 16 and ds_bpermute only for 32. The values move unchanged.
template <int H>
__device__ __forceinline__ float xor_lane(float v) {
    const int x = __builtin_bit_cast(int, v);
    if constexpr (H == 1) {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, true));  // quad_perm [1,0,3,2]
    } else if constexpr (H == 2) {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, true));  // quad_perm [2,3,0,1]
    } else if constexpr (H == 4 || H == 8) {
        const int up = __builtin_amdgcn_update_dpp(0, x, 0x100 + H, 0xF, 0xF, true);  // row_shl: lane + H
        const int dn = __builtin_amdgcn_update_dpp(0, x, 0x110 + H, 0xF, 0xF, true);  // row_shr: lane - H
        return __builtin_bit_cast(float, (threadIdx.x & H) ? dn : up);
    } else if constexpr (H == 16) {
        return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(x, 0x401F));  // swizzle(SWAP, 16)
    } else {
        return __shfl_xor(v, H);
    }
}

// The same for h a power of two below 64 (a constant once loops unroll).
__device__ __forceinline__ float xor_lane(float v, int h) {
    switch (h) {
        case 1: return xor_lane<1>(v);
        case 2: return xor_lane<2>(v);
        case 4: return xor_lane<4>(v);
        case 8: return xor_lane<8>(v);
        case 16: return xor_lane<16>(v);
        default: return xor_lane<32>(v);
    }
}

// Go's built-in max of two float32 values, which every max-reduction of the
// reference uses (QuantizeRow's bound, softmaxInPlace's max, the lut tables'
// bound): NaN when either operand is NaN, and -0 below +0. That is IEEE
// 754-2019 maximum, one v_maximum3_f32 on gfx950; fmaxf would drop a NaN.
__device__ __forceinline__ float go_max(float a, float b) { return __builtin_elementwise_maximum(a, b); }
// Go's built-in min (and slices.Min's rule): NaN when either is NaN.
__device__ __forceinline__ float go_min(float a, float b) { return __builtin_elementwise_minimum(a, b); }

// QuantizeRow's code of r = RNE(x / s) (internal/needle/int8.go:50-53):
// int8(min(max(r, -128), 127)) with Go's NaN-propagating min and max, and
// the conversion of a NaN to int8 gives 0 on amd64 (the float64 to integer
// conversion returns the integer indefinite 0x80000000, whose low byte is 0)
// as on arm64 (FCVTZS of a NaN is 0). A +-Inf r clamps to 127 / -128.
__device__ __forceinline__ int go_int8_code(float r) {
    return r != r ? 0 : static_cast<int>(fminf(fmaxf(r, -128.0f), 127.0f));
}

// Workgroup barrier for LDS only: this wavefront's LDS operations complete
// (lgkmcnt 0), then s_barrier. Unlike __syncthreads it does not wait for
// the wavefront's global loads, so loads issued ahead stay in flight across
// it. The empty asm statements keep the compiler from moving memory
// accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// One lane of the amd64 exponent kernel (exp_amd64.s:84-112), constants bit
// for bit (exp_amd64.s:7-51): Cephes expf with the kernel's fused steps.
__device__ __forceinline__ float exp_lane(float x) {
    const float log2e = 0x1.715476p+0f, ln2hi = 0x1.63p-1f, ln2lo = -0x1.bd0106p-13f;
    const float c6 = 0x1.a0d2cep-13f, c5 = 0x1.6e879cp-10f, c4 = 0x1.111210p-7f;
    const float c3 = 0x1.555382p-5f, c2 = 0x1.555554p-3f, c1 = 0x1p-1f;
    const float lo = -0x1.5d51ecp+6f;
    const bool lt = x < lo;
    const float xc = (x != x) ? x : (lo > x ? lo : x);
    const float k = rintf(xc * log2e);
    float r = fmaf(-k, ln2hi, xc);
    r = fmaf(-k, ln2lo, r);
    const float r2 = r * r;
    float p = c6;
    p = fmaf(p, r, c5);
    p = fmaf(p, r, c4);
    p = fmaf(p, r, c3);
    p = fmaf(p, r, c2);
    p = fmaf(p, r, c1);
    float yv = fmaf(p, r2, r);
    yv = yv + 1.0f;
    const int ki = (k != k || k >= 2147483648.0f || k < -2147483648.0f) ? INT_MIN : static_cast<int>(k);
    const float e = __uint_as_float(__float_as_uint(yv) + (static_cast<unsigned>(ki) << 23));
    return lt ? 0.0f : e;
}

// The synthetic decoder's FFN activation: x * sigma(x), sigma built from the
// exponent lane on a non-positive argument (no reference counterpart).
__device__ __forceinline__ float silu_value(float v) {
    float s;
    if (v >= 0.0f) {
        const float e = exp_lane(-v);
        const float d = 1.0f + e;
        s = 1.0f / d;
    } else {
        const float e = exp_lane(v);
        const float d = 1.0f + e;
        s = e / d;
    }
    return v * s;
}

// exp of a float64 by fdlibm's e_exp.c method (Sun Microsystems, 1993; the
// steps of Go's portable math.Exp): k = x log2(e) rounded half away from
// zero, r = hi - lo with hi = x - k ln2_hi and lo = k ln2_lo, exp(r) =
// 1 - ((lo - r c / (2 - c)) - hi) with c = r - r^2 P(r^2) of degree 5, then
// y 2^k. Every operation is an IEEE float64 one, unfused, so the CPU
// restatement returns the same bits; the error is below 1 ulp.
__device__ __forceinline__ double exp_f64(double x) {
    const double ln2hi = 6.93147180369123816490e-01, ln2lo = 1.90821492927058770002e-10;
    const double log2e = 1.44269504088896338700e+00;
    const double p1 = 1.66666666666666019037e-01, p2 = -2.77777777770155933842e-03;
    const double p3 = 6.61375632143793436117e-05, p4 = -1.65339022054652515390e-06;
    const double p5 = 4.13813679705723846039e-08;
    if (x != x) return x;
    if (x > 7.09782712893383973096e+02) return __builtin_huge_val();
    if (x < -7.45133219101941108420e+02) return 0.0;
    if (x > -3.7252902984619140625e-09 && x < 3.7252902984619140625e-09) return 1.0 + x;  // |x| < 2^-28
    const double kf = x < 0.0 ? log2e * x - 0.5 : log2e * x + 0.5;
    const int k = static_cast<int>(kf);  // truncation toward zero
    const double hi = x - static_cast<double>(k) * ln2hi, lo = static_cast<double>(k) * ln2lo;
    const double r = hi - lo, t = r * r;
    const double c = r - t * (p1 + t * (p2 + t * (p3 + t * (p4 + t * p5))));
    const double y = 1.0 - ((lo - (r * c) / (2.0 - c)) - hi);
    return ldexp(y, k);
}

// jax.nn.sigmoid in float32 as the reference computes it,
// float32(1 / (1 + exp(-float64(x)))) (internal/needle/load.go:120-123,
// internal/decoder/cross.go:322-325): the attention's output gate.
__device__ __forceinline__ float gate_sigmoid(float v) {
    const double e = exp_f64(-static_cast<double>(v));
    return static_cast<float>(1.0 / (1.0 + e));
}

// ZCRMSNorm's mean square (norm.go:91-109), partial sum k of four: the
// float64 squares of row[i] for i = k, k+4, ... below dim & ~3, in order,
// and for k = 0 the tail after them.
__device__ __forceinline__ double zc_partial(const float *row, int dim, int k) {
    const int full = dim & ~3;
    double s = 0.0;
    int i = k;
    for (; i + 12 < full; i += 16) {
        const double d0 = row[i], d1 = row[i + 4], d2 = row[i + 8], d3 = row[i + 12];
        s = s + d0 * d0;
        s = s + d1 * d1;
        s = s + d2 * d2;
        s = s + d3 * d3;
    }
    for (; i < full; i += 4) {
        const double d = row[i];
        s = s + d * d;
    }
    if (k == 0)
        for (int t = full; t < dim; ++t) {
            const double d = row[t];
            s = s + d * d;
        }
    return s;
}

// The same partial sum k for a row held in LDS transposed, t[k * stride +
// j] = row[4j + k] for j < q = dim / 4 (dim a multiple of 64): the lane
// reads its q values as float4s, 16 ahead of the adds, so the chain of q
// dependent float64 adds does not wait on each read. Equal to
// zc_partial(row, dim, k) bit for bit (the same squares in the same order).
__device__ __forceinline__ double zc_partial_t(const float *t, int stride, int q, int k) {
    const float4 *r = reinterpret_cast<const float4 *>(t + k * stride);
    const int n4 = q / 4;
    double s = 0.0;
    float4 a0 = r[0], a1 = r[1], a2 = r[2], a3 = r[3];
    for (int j = 0; j < n4; j += 4) {
        float4 b0 = a0, b1 = a1, b2 = a2, b3 = a3;
        if (j + 4 < n4) {
            b0 = r[j + 4];
            b1 = r[j + 5];
            b2 = r[j + 6];
            b3 = r[j + 7];
        }
        const float v[16] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w,
                             a2.x, a2.y, a2.z, a2.w, a3.x, a3.y, a3.z, a3.w};
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const double d = v[e];
            s = s + d * d;
        }
        a0 = b0;
        a1 = b1;
        a2 = b2;
        a3 = b3;
    }
    return s;
}

// ZCRMSNorm's divisor from the four partial sums (norm.go:53-66):
// float32(sqrt(float64(float32(s / dim) + 1e-6))).
__device__ __forceinline__ float zc_rms(double p0, double p1, double p2, double p3, int dim) {
    const double s = ((p0 + p1) + p2) + p3;
    const float ms = static_cast<float>(s / static_cast<double>(dim));
    const float e = ms + 1e-6f;
    return static_cast<float>(sqrt(static_cast<double>(e)));
}

// RoPE of one pair (rope.go:69-81): [a cos - b sin, b cos + a sin], every
// product rounded.
__device__ __forceinline__ void rope_pair(float a, float b, float c, float s, float &o1, float &o2) {
    const float ac = a * c, bs = b * s, bc = b * c, as = a * s;
    o1 = ac - bs;
    o2 = bc + as;
}

// A table entry's bits (the table form): RNE(f) for |f| <= 8191.5 as the
// low bits of f + 1.5 * 2^23 (round to nearest even, exact for |f| < 2^22),
// bits 0-5 the l plane's value and bits 6-13 the h plane's.
constexpr float kRneMagic = 12582912.0f;  // 1.5 * 2^23

__device__ __forceinline__ uint32_t rne_bits(float f) { return __float_as_uint(f + kRneMagic); }

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Four entries' bit patterns -> the l plane's 4 bytes (v & 63) and the h
// plane's 4 bytes ((v >> 6) & 255): the entries' low halfwords are paired,
// shifted right by 6 two at a time (bits 6-13 land in each halfword's low
// byte), and the wanted bytes gathered.
__device__ __forceinline__ void planes4(uint32_t e0, uint32_t e1, uint32_t e2, uint32_t e3, uint32_t &lo,
                                        uint32_t &hi) {
    const uint32_t q01 = __builtin_amdgcn_perm(e1, e0, 0x05040100u);  // e0.lo16 | e1.lo16 << 16
    const uint32_t q23 = __builtin_amdgcn_perm(e3, e2, 0x05040100u);  // e2.lo16 | e3.lo16 << 16
    lo = __builtin_amdgcn_perm(q23, q01, 0x06040200u) & 0x3f3f3f3fu;  // byte 0 of each halfword
    const u16x2 r01 = __builtin_bit_cast(u16x2, q01) >> static_cast<unsigned short>(6);
    const u16x2 r23 = __builtin_bit_cast(u16x2, q23) >> static_cast<unsigned short>(6);
    hi = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, r23), __builtin_bit_cast(uint32_t, r01), 0x06040200u);
}

}  // namespace cqhip
