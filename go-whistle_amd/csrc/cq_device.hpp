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

}  // namespace cqhip
