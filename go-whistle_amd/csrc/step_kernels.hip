// gfx950 kernels for the float blocks between the CQ products of a decode
// step, each bit for bit the reference's arithmetic:
//   zc_rmsnorm_kernel  ZCRMSNorm.Apply (internal/needle/norm.go:53-66, 84-109):
//                      mean(x²) in float64 as four partial sums over i mod 4,
//                      each in order, rounded to float32; rms =
//                      float32(sqrt(float64(ms + 1e-6))); y = (gain·x) / rms.
//   rope_kernel        Rope.apply (internal/needle/rope.go:69-81): per head,
//                      [x1·cos − x2·sin, x2·cos + x1·sin], products rounded.
//   argmax_kernel      argmax (internal/decoder/greedy.go:181-191): the first
//                      index of the largest value (0 when v[0] is NaN).
//   silu_kernel        silu_value (cq_device.hpp): the synthetic decoder's FFN
//                      activation (no reference counterpart; defined so that
//                      CPU and GPU agree bit for bit).
//   add_kernel         x += y (the residual adds, decoder.go / block.go).
//   sigmoid_gate_kernel  Attention.output's gate (internal/needle/attention.go:
//                      245-249): gate = sigmoid(gate), out *= gate, with
//                      sigmoid float32(1 / (1 + exp(-float64(x)))).
//   append_kernel      Int8Rows.Append (internal/needle/int8.go:125-141) of one
//                      row per stream at the stream's position, optionally
//                      after RoPE of each head at that position.
#include "cq_internal.hpp"
#include "cq_device.hpp"

#include <climits>

namespace cqhip {
namespace {

__global__ __launch_bounds__(64) void zc_rmsnorm_kernel(float *dst, const float *x, const float *gain, int dim) {
    extern __shared__ __align__(16) unsigned char smem[];
    double *sq = reinterpret_cast<double *>(smem);  // the row's squares, exact in float64
    const int r = blockIdx.x, lane = threadIdx.x;
    const float *row = x + static_cast<long long>(r) * dim;
    float *out = dst + static_cast<long long>(r) * dim;
    __shared__ double part[4];
    __shared__ float rms_sh;
    for (int i = lane; i < dim; i += 64) {
        const double v = static_cast<double>(row[i]);
        sq[i] = v * v;
    }
    __syncthreads();
    // meanSquare (norm.go:91-109): s_k over i = k, k+4, ... (the full words
    // of four), then the tail into s0, then (s0 + s1 + s2 + s3) / n.
    if (lane < 4) {
        double s = 0.0;
        const int full = dim & ~3;
        int i = lane;
        for (; i + 12 < full; i += 16) {
            const double a0 = sq[i], a1 = sq[i + 4], a2 = sq[i + 8], a3 = sq[i + 12];
            s = s + a0;
            s = s + a1;
            s = s + a2;
            s = s + a3;
        }
        for (; i < full; i += 4) s = s + sq[i];
        if (lane == 0)
            for (int t = full; t < dim; ++t) s = s + sq[t];
        part[lane] = s;
    }
    __syncthreads();
    if (lane == 0) {
        const double s = ((part[0] + part[1]) + part[2]) + part[3];
        const float ms = static_cast<float>(s / static_cast<double>(dim));
        const float e = ms + 1e-6f;
        rms_sh = static_cast<float>(sqrt(static_cast<double>(e)));
    }
    __syncthreads();
    const float rms = rms_sh;
    for (int c = lane; c < dim; c += 64) {
        const float gx = gain[c] * row[c];
        out[c] = gx / rms;
    }
}

__global__ __launch_bounds__(256) void rope_kernel(float *x, int heads, int head_dim, const float *cos_t,
                                                   const float *sin_t, int positions, const int32_t *pos,
                                                   int rows_per_pos) {
    const int r = blockIdx.x;
    const int half = head_dim / 2;
    const int p = pos[r / rows_per_pos];
    if (p < 0 || p >= positions) return;  // a position past the tables: the row is left as it is
    const float *cs = cos_t + static_cast<long long>(p) * half, *sn = sin_t + static_cast<long long>(p) * half;
    float *row = x + static_cast<long long>(r) * heads * head_dim;
    for (int e = threadIdx.x; e < heads * half; e += blockDim.x) {
        const int h = e / half, i = e % half;
        float *xh = row + h * head_dim;
        const float a = xh[i], b = xh[i + half];
        const float ac = a * cs[i], bs = b * sn[i], bc = b * cs[i], as = a * sn[i];
        xh[i] = ac - bs;
        xh[i + half] = bc + as;
    }
}

// greedy.go's argmax keeps best = 0 and moves to i when v[i] > v[best]: the
// answer is 0 when v[0] is NaN, else the first index of the largest value
// that is not NaN (NaN never compares greater; +0 and -0 tie). Each thread
// takes its values in index order (16-byte loads, sixteen in flight), NaN
// never a candidate; candidates combine larger value first, then smaller
// index, across the wavefront (lane exchanges) and the workgroup (LDS).
struct ArgmaxCand {
    float v;
    int i;  // INT_MAX: none
};

__device__ __forceinline__ ArgmaxCand argmax_pick(ArgmaxCand a, ArgmaxCand b) {
    if (b.i == INT_MAX) return a;
    if (a.i == INT_MAX || b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
    return a;
}

// With pos: the decode step's position advance rides on the argmax, pos[r]
// += 1 and the row's self-attention key bound span_hi[r * span_stride] =
// the new position + 1 (the keys the next step's query sees after its
// append), so a step needs no separate launches for them.
__global__ __launch_bounds__(256) void argmax_kernel(int32_t *out, const float *v, int n, int32_t *pos,
                                                     int32_t *span_hi, int span_stride, int32_t *done, int eos) {
    const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // A stream that has stopped keeps its token (the stop token) and its
    // position: the steps it still runs in the batch change nothing it
    // reports (the flag is read with the row, and checked before any store).
    const int stopped = tid == 0 && done ? done[r] : 0;
    const float *row = v + static_cast<long long>(r) * n;
    // the scalar operands of the end, loaded with the row rather than after it
    const float v0 = tid == 0 && n > 0 ? row[0] : 0.0f;
    const int p0 = tid == 0 && pos ? pos[r] : 0;
    ArgmaxCand c{0.0f, INT_MAX};
    auto take = [&](float x, int i) {
        if (x == x && (c.i == INT_MAX || x > c.v)) c = ArgmaxCand{x, i};
    };
    if ((n & 3) == 0 && (reinterpret_cast<uintptr_t>(row) & 15) == 0) {
        const int n4 = n >> 2;
        const float4 *row4 = reinterpret_cast<const float4 *>(row);
        for (int base = 0; base < n4; base += 16 * 256) {  // a 16384-entry row in one round of loads
            float4 f[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const int i4 = base + k * 256 + tid;
                if (i4 < n4) f[k] = row4[i4];
            }
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const int i4 = base + k * 256 + tid;
                if (i4 < n4) {
                    take(f[k].x, 4 * i4);
                    take(f[k].y, 4 * i4 + 1);
                    take(f[k].z, 4 * i4 + 2);
                    take(f[k].w, 4 * i4 + 3);
                }
            }
        }
    } else {
        for (int i = tid; i < n; i += 256) take(row[i], i);
    }
#pragma unroll
    for (int h = 32; h > 0; h >>= 1) {
        ArgmaxCand o;
        o.v = __shfl_xor(c.v, h);
        o.i = __shfl_xor(c.i, h);
        c = argmax_pick(c, o);
    }
    __shared__ float sv[4];
    __shared__ int si[4];
    if (lane == 0) {
        sv[wave] = c.v;
        si[wave] = c.i;
    }
    __syncthreads();
    if (tid == 0 && !stopped) {
        for (int w = 1; w < 4; ++w) c = argmax_pick(c, ArgmaxCand{sv[w], si[w]});
        const bool nan0 = n > 0 && v0 != v0;
        const int tok = (n == 0 || nan0 || c.i == INT_MAX) ? 0 : c.i;
        out[r] = tok;
        if (pos) {
            const int p = p0 + 1;
            pos[r] = p;
            span_hi[static_cast<long long>(r) * span_stride] = p + 1;
        }
        if (done && tok == eos) done[r] = 1;  // greedy.go:55-59: the stream stops at EOS
    }
}

__global__ __launch_bounds__(256) void silu_kernel(float *x, long long n) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    x[i] = silu_value(x[i]);
}

__global__ __launch_bounds__(256) void add_kernel(float *x, const float *y, long long n) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) x[i] = x[i] + y[i];
}

__global__ __launch_bounds__(256) void sigmoid_gate_kernel(float *out, float *gate, long long n) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float g = gate_sigmoid(gate[i]);
    gate[i] = g;
    out[i] = out[i] * g;
}

// Int8Rows.Append of stream b's row at its position pos[b]: QuantizeRow
// per chunk of width (int8.go:36-55), one wavefront per chunk. With cos_t,
// each chunk (a head) is first rotated by RoPE at pos[b] (rope.go:69-81):
// value i < width/2 pairs with i + width/2.
__global__ __launch_bounds__(256) void append_kernel(int8_t *q, float *s, const float *x, int cols, int width,
                                                     long long q_stride, long long s_stride, const int32_t *pos,
                                                     int cap, const float *cos_t, const float *sin_t) {
    const int b = blockIdx.y, lane = threadIdx.x & 63;
    const int c = blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
    const int chunks = cols / width;
    const int p = pos[b];
    if (c >= chunks || p < 0 || p >= cap) return;
    const float *xc = x + static_cast<long long>(b) * cols + static_cast<long long>(c) * width;
    float v[4];  // width <= 256
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int i = lane + 64 * k;
        v[k] = i < width ? xc[i] : 0.0f;
    }
    if (cos_t) {
        const int half = width / 2;
        const float *cs = cos_t + static_cast<long long>(p) * half, *sn = sin_t + static_cast<long long>(p) * half;
        float rv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = lane + 64 * k;
            rv[k] = v[k];
            if (i < width) {
                const int j = i < half ? i : i - half;
                const float a = xc[j], bb = xc[j + half];
                float o1, o2;
                rope_pair(a, bb, cs[j], sn[j], o1, o2);
                rv[k] = i < half ? o1 : o2;
            }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = rv[k];
    }
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (lane + 64 * k < width) m = go_max(m, fabsf(v[k]));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = go_max(m, __shfl_xor(m, off));
    const float sc = m > 0.0f ? m / 127.0f : 1.0f;
    int8_t *qc = q + b * q_stride + static_cast<long long>(p) * cols + static_cast<long long>(c) * width;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int i = lane + 64 * k;
        if (i < width) qc[i] = static_cast<int8_t>(go_int8_code(rintf(v[k] / sc)));
    }
    if (lane == 0) s[b * s_stride + static_cast<long long>(p) * chunks + c] = sc;
}

unsigned blocks_for(long long n, int t) { return static_cast<unsigned>((n + t - 1) / t); }

}  // namespace

hipError_t launch_zc_rmsnorm(float *dst, const float *x, const float *gain, int rows, int dim, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(zc_rmsnorm_kernel, dim3(rows), dim3(64), sizeof(double) * dim, s, dst, x, gain, dim);
    return hipGetLastError();
}

hipError_t launch_rope(float *x, int rows, int heads, int head_dim, const float *cos_t, const float *sin_t,
                       int positions, const int32_t *pos, int rows_per_pos, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(rope_kernel, dim3(rows), dim3(256), 0, s, x, heads, head_dim, cos_t, sin_t, positions, pos,
                       rows_per_pos);
    return hipGetLastError();
}

hipError_t launch_argmax(int32_t *out, const float *v, int rows, int n, int32_t *pos, int32_t *span_hi,
                         int span_stride, int32_t *done, int eos, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(256), 0, s, out, v, n, pos, span_hi, span_stride, done, eos);
    return hipGetLastError();
}

hipError_t launch_silu(float *x, long long n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(silu_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, x, n);
    return hipGetLastError();
}

hipError_t launch_add(float *x, const float *y, long long n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(add_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, x, y, n);
    return hipGetLastError();
}

hipError_t launch_sigmoid_gate(float *out, float *gate, long long n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(sigmoid_gate_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, out, gate, n);
    return hipGetLastError();
}

hipError_t launch_append(int8_t *q, float *sc, const float *x, int batch, int cols, int width, long long q_stride,
                         long long s_stride, const int32_t *pos, int cap, const float *cos_t, const float *sin_t,
                         hipStream_t s) {
    if (batch <= 0) return hipSuccess;
    const int chunks = cols / width;
    hipLaunchKernelGGL(append_kernel, dim3(blocks_for(chunks, 4), batch), dim3(256), 0, s, q, sc, x, cols, width,
                       q_stride, s_stride, pos, cap, cos_t, sin_t);
    return hipGetLastError();
}

}  // namespace cqhip
