// gfx950 kernels for go-whistle's int8 KV numerics (internal/needle/int8.go).
//
// quantize_kernel: QuantizeRow (int8.go:36-55) per chunk of `width` values,
//   one wavefront per chunk: s = max|x|/127 (1 for a zero chunk), codes
//   RNE(x/s) clipped to [-128, 127]; the same bits as the reference (the
//   max is exact in any order, the divide is IEEE, the rounding is RNE).
//
// attend_kernel: AttendInt8Spans (int8.go:208-272) for one (stream, query
//   row, head) per workgroup:
//   1. logits, one thread per key: the int8 query's exact int32 dot times
//      (s_q * s_k) / scale (int8Logits, int8.go:278-285), or the float32
//      query against the codes summed in order, * s_k / scale (dotsF32I8,
//      int8.go:289-300);
//   2. softmaxInPlace (load.go:128-138): the max, then expSubSum as amd64
//      runs it (exp_amd64.go:13-25): on the multiple-of-8 prefix the AVX2
//      kernel's Cephes exponent (exp_amd64.s:84-112; S. L. Moshier's
//      published expf, with the kernel's fused steps) summed in eight lanes
//      of stride 8 and reduced as the kernel does; the tail, or the whole row
//      under 8 values, float32 of the float64 exponent summed in order;
//      then every value divided by the sum;
//   3. the weights times the value scales, and axpysI8 (int8kernel.go:
//      360-368): per output, one key after the other, each product rounded
//      before the add. One thread per output carries that chain over LDS
//      chunks of value codes, which the workgroup's other wavefronts stage
//      with 16-byte loads one chunk ahead.
#include "cq_internal.hpp"

#include <algorithm>
#include <climits>

namespace cqhip {
namespace {

__global__ __launch_bounds__(256) void quantize_kernel(int8_t *q, float *s, const float *x, long long chunks,
                                                       int width) {
    const int lane = threadIdx.x & 63;
    const long long c = static_cast<long long>(blockIdx.x) * (blockDim.x / 64) + (threadIdx.x >> 6);
    if (c >= chunks) return;
    const float *xc = x + c * width;
    float m = 0.0f;
    for (int i = lane; i < width; i += 64) m = fmaxf(m, fabsf(xc[i]));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    const float sc = m > 0.0f ? m / 127.0f : 1.0f;
    int8_t *qc = q + c * width;
    for (int i = lane; i < width; i += 64) {
        float r = rintf(xc[i] / sc);
        r = fminf(fmaxf(r, -128.0f), 127.0f);
        qc[i] = static_cast<int8_t>(static_cast<int>(r));
    }
    if (lane == 0) s[c] = sc;
}

// One lane of the amd64 kernel's exponent (exp_amd64.s:84-112), constants
// bit for bit (exp_amd64.s:7-51).
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

__device__ __forceinline__ float exp_generic(float d) { return static_cast<float>(exp(static_cast<double>(d))); }

constexpr int kAttThreads = 256;

__device__ __forceinline__ float block_max(float v, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < kAttThreads / 64; ++w) r = fmaxf(r, red[w]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ int dot4_i8(int a, int b, int acc) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
        acc += static_cast<int>(static_cast<int8_t>(a >> (8 * e))) * static_cast<int>(static_cast<int8_t>(b >> (8 * e)));
    return acc;
}

__global__ __launch_bounds__(kAttThreads) void attend_kernel(AttendArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int h = blockIdx.x, i = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x;
    const int kv_heads = a.k_cols / a.qk;
    const int kv = h / (a.heads / kv_heads);
    const int32_t *sp = a.spans + (static_cast<long long>(b) * a.t + i) * 4;
    const int lo0 = sp[0], len0 = sp[1] - sp[0], lo1 = sp[2], len1 = sp[3] - sp[2];
    const int n = len0 + len1;
    if (lo0 < 0 || len0 < 0 || sp[1] > a.nk_max || lo1 < 0 || len1 < 0 || sp[3] > a.nk_max) return;  // spans off the cache

    float *s = reinterpret_cast<float *>(smem);  // n logits, then weights
    int8_t *vbuf = reinterpret_cast<int8_t *>(s + ((a.nk_max + 3) & ~3));  // value codes: one or two chunks
    __shared__ float red[8];
    __shared__ __align__(16) int8_t q8[256];
    __shared__ float sq_sh, sum_sh;

    const float *qi = a.q + b * a.q_stride + (static_cast<long long>(i) * a.heads + h) * a.qk;
    const int8_t *kq = a.kq + b * a.kv_stride;
    const float *ks = a.ks + b * a.s_stride;
    const int8_t *vq = a.vq + b * a.kv_stride;
    const float *vs = a.vs + b * a.s_stride;
    auto key_of = [&](int j) { return j < len0 ? lo0 + j : lo1 + (j - len0); };

    // QuantizeRow of the query head (int8.go:226-228).
    if (a.quant_q) {
        float m = 0.0f;
        for (int c = tid; c < a.qk; c += kAttThreads) m = fmaxf(m, fabsf(qi[c]));
        m = block_max(m, red);
        const float sc = m > 0.0f ? m / 127.0f : 1.0f;
        for (int c = tid; c < a.qk; c += kAttThreads) {
            float r = rintf(qi[c] / sc);
            r = fminf(fmaxf(r, -128.0f), 127.0f);
            q8[c] = static_cast<int8_t>(static_cast<int>(r));
        }
        if (tid == 0) sq_sh = sc;
        __syncthreads();
    }
    const float sq = a.quant_q ? sq_sh : 0.0f;

    // Value codes: staged into LDS from the start, so their loads overlap
    // the logits and the softmax. All n rows when they fit (vchunk >= n),
    // else chunks of vchunk rows, two buffers, staged one chunk ahead.
    const bool aligned = (a.kv_stride & 15) == 0 && (reinterpret_cast<uintptr_t>(a.kq) & 15) == 0 &&
                         (reinterpret_cast<uintptr_t>(a.vq) & 15) == 0;
    const bool wide = aligned && (a.qk & 15) == 0 && (a.k_cols & 15) == 0;
    const int vchunk = a.vchunk;
    const int nchunks = (n + vchunk - 1) / vchunk;
    const bool wide_v = aligned && (a.vd & 15) == 0 && (a.v_cols & 15) == 0;
    auto stage = [&](int c, int8_t *buf, int t0, int nt) {
        const int j0 = c * vchunk, cnt = min(vchunk, n - j0);
        if (wide_v) {
            // eight 16-byte loads in flight per thread before their LDS stores
            const int per = a.vd / 16, total = cnt * per;
            for (int e0 = t0; e0 < total; e0 += 8 * nt) {
                int4 w[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int e = e0 + u * nt;
                    if (e < total) {
                        const int jj = e / per, part = e - (e / per) * per;
                        w[u] = *reinterpret_cast<const int4 *>(vq + static_cast<long long>(key_of(j0 + jj)) * a.v_cols +
                                                               kv * a.vd + part * 16);
                    }
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int e = e0 + u * nt;
                    if (e < total) {
                        const int jj = e / per, part = e - (e / per) * per;
                        *reinterpret_cast<int4 *>(buf + jj * a.vd + part * 16) = w[u];
                    }
                }
            }
        } else {
            for (int e = t0; e < cnt * a.vd; e += nt) {
                const int jj = e / a.vd, d = e - (e / a.vd) * a.vd;
                buf[jj * a.vd + d] = vq[static_cast<long long>(key_of(j0 + jj)) * a.v_cols + kv * a.vd + d];
            }
        }
    };
    if (nchunks > 0) stage(0, vbuf, tid, kAttThreads);

    // 1. Logits, one thread per key (int8Logits / dotsF32I8), four keys at
    // a time so that their loads are in flight together.
    auto logit = [&](int j) -> float {
        const int key = key_of(j);
        const int8_t *krow = kq + static_cast<long long>(key) * a.k_cols + kv * a.qk;
        const float sk = ks[static_cast<long long>(key) * kv_heads + kv];
        if (a.quant_q) {
            int dot = 0;  // exact in any order
            if (wide) {
                for (int c = 0; c < a.qk; c += 16) {
                    const int4 kw = *reinterpret_cast<const int4 *>(krow + c);
                    const int4 qw = *reinterpret_cast<const int4 *>(q8 + c);
                    dot = dot4_i8(kw.x, qw.x, dot);
                    dot = dot4_i8(kw.y, qw.y, dot);
                    dot = dot4_i8(kw.z, qw.z, dot);
                    dot = dot4_i8(kw.w, qw.w, dot);
                }
            } else {
                for (int c = 0; c < a.qk; c += 4)
                    dot = dot4_i8(*reinterpret_cast<const int *>(krow + c), *reinterpret_cast<const int *>(q8 + c), dot);
            }
            const float scl = sq * sk;
            const float t1 = static_cast<float>(dot) * scl;
            return t1 / a.scale;
        }
        float dot = 0.0f;  // in order
        for (int c = 0; c < a.qk; c += 4) {
            const int w = *reinterpret_cast<const int *>(krow + c);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float pr = qi[c + e] * static_cast<float>(static_cast<int8_t>(w >> (8 * e)));
                dot = dot + pr;
            }
        }
        const float t1 = dot * sk;
        return t1 / a.scale;
    };
    {
        int j = tid;
        for (; j + 3 * kAttThreads < n; j += 4 * kAttThreads) {
            const float l0 = logit(j), l1 = logit(j + kAttThreads), l2 = logit(j + 2 * kAttThreads),
                        l3 = logit(j + 3 * kAttThreads);
            s[j] = l0;
            s[j + kAttThreads] = l1;
            s[j + 2 * kAttThreads] = l2;
            s[j + 3 * kAttThreads] = l3;
        }
        for (; j < n; j += kAttThreads) s[j] = logit(j);
    }
    __syncthreads();

    // 2. softmaxInPlace with amd64's expSubSum.
    float m = -INFINITY;
    for (int j = tid; j < n; j += kAttThreads) m = fmaxf(m, s[j]);
    m = block_max(m, red);
    const int n8 = n & ~7;
    const bool kernel_path = n8 > 0;
    for (int j = tid; j < n; j += kAttThreads) {
        const float d = s[j] - m;
        s[j] = (kernel_path && j < n8) ? exp_lane(d) : exp_generic(d);
    }
    __syncthreads();
    if (tid < 8 && kernel_path) {  // lane tid of the 8-lane sum, elements in order
        float acc = 0.0f;
        int j = tid;
        for (; j + 24 < n8; j += 32) {
            const float e0 = s[j], e1 = s[j + 8], e2 = s[j + 16], e3 = s[j + 24];
            acc = acc + e0;
            acc = acc + e1;
            acc = acc + e2;
            acc = acc + e3;
        }
        for (; j < n8; j += 8) acc = acc + s[j];
        red[tid] = acc;
    }
    __syncthreads();
    if (tid == 0) {
        float sum;
        if (kernel_path) {
            const float x0 = red[0] + red[4], x1 = red[1] + red[5], x2 = red[2] + red[6], x3 = red[3] + red[7];
            const float h0 = x0 + x1, h1 = x2 + x3;
            sum = h0 + h1;
            if (n8 != n) {
                float tail = 0.0f;
                for (int j = n8; j < n; ++j) tail = tail + s[j];
                sum = sum + tail;
            }
        } else {
            sum = 0.0f;
            for (int j = 0; j < n; ++j) sum = sum + s[j];
        }
        sum_sh = sum;
    }
    __syncthreads();
    const float sum = sum_sh;
    for (int j = tid; j < n; j += kAttThreads) {
        const float p = s[j] / sum;
        s[j] = p * vs[static_cast<long long>(key_of(j)) * kv_heads + kv];
    }

    // 3. axpysI8 per output, keys in order: the first ceil(vd/64)
    // wavefronts carry the chains over LDS chunks of value codes; with more
    // than one chunk the other wavefronts stage the next one meanwhile.
    const int chain_threads = ((a.vd + 63) / 64) * 64;
    __syncthreads();
    float acc = 0.0f;
    for (int c = 0; c < nchunks; ++c) {
        int8_t *cur = vbuf + (c & 1) * vchunk * a.vd;
        if (tid < chain_threads) {
            if (tid < a.vd) {
                const int j0 = c * vchunk, cnt = min(vchunk, n - j0);
                int jj = 0;
                for (; jj + 3 < cnt; jj += 4) {
                    const float w0 = s[j0 + jj], w1 = s[j0 + jj + 1], w2 = s[j0 + jj + 2], w3 = s[j0 + jj + 3];
                    const float c0 = static_cast<float>(cur[jj * a.vd + tid]);
                    const float c1 = static_cast<float>(cur[(jj + 1) * a.vd + tid]);
                    const float c2 = static_cast<float>(cur[(jj + 2) * a.vd + tid]);
                    const float c3 = static_cast<float>(cur[(jj + 3) * a.vd + tid]);
                    const float p0 = w0 * c0, p1 = w1 * c1, p2 = w2 * c2, p3 = w3 * c3;
                    acc = acc + p0;
                    acc = acc + p1;
                    acc = acc + p2;
                    acc = acc + p3;
                }
                for (; jj < cnt; ++jj) {
                    const float pr = s[j0 + jj] * static_cast<float>(cur[jj * a.vd + tid]);
                    acc = acc + pr;
                }
            }
        } else if (c + 1 < nchunks) {
            stage(c + 1, vbuf + ((c + 1) & 1) * vchunk * a.vd, tid - chain_threads, kAttThreads - chain_threads);
        }
        if (nchunks > 1) __syncthreads();
    }
    if (tid < a.vd) a.out[b * a.out_stride + (static_cast<long long>(i) * a.heads + h) * a.vd + tid] = acc;
}

}  // namespace

hipError_t launch_quantize_rows(int8_t *q, float *s, const float *x, long long chunks, int width,
                                hipStream_t stream) {
    if (chunks <= 0) return hipSuccess;
    const long long blocks = (chunks + 3) / 4;
    for (long long c0 = 0; c0 < blocks; c0 += 1 << 30) {
        const long long nb = blocks - c0 < (1LL << 30) ? blocks - c0 : (1LL << 30);
        const long long ch0 = c0 * 4;
        hipLaunchKernelGGL(quantize_kernel, dim3(static_cast<unsigned>(nb)), dim3(256), 0, stream, q + ch0 * width,
                           s + ch0, x + ch0 * width, chunks - ch0, width);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_attend_int8(const AttendArgs &a, hipStream_t stream) {
    if (a.t <= 0 || a.heads <= 0 || a.batch <= 0) return hipSuccess;
    const AttendArgs &b = a;
    const bool one_chunk = a.vchunk >= a.nk_max;
    const size_t vbytes = (one_chunk ? 1 : 2) * static_cast<size_t>(a.vchunk) * a.vd;
    const size_t lds = sizeof(float) * static_cast<size_t>((a.nk_max + 3) & ~3) + vbytes;
    static bool attr = false;
    if (!attr) {
        // dynamic LDS beside the kernel's static arrays: 96 KiB of values + up to 8192 logits
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&attend_kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024);
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL(attend_kernel, dim3(a.heads, a.t, a.batch), dim3(kAttThreads), lds, stream, b);
    return hipGetLastError();
}

}  // namespace cqhip
