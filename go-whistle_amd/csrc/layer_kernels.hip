// gfx950 kernels for the reference decode step's features around the CQ
// products, each bit for bit the reference's arithmetic:
//   qkv_prep_kernel     after the q/k/v projections of one token per stream:
//                       the causal taps over the raw rows of the last taps - 1
//                       positions (applyTaps on extendTaps' rows,
//                       internal/needle/attention.go:597-613, cache.go:143-154),
//                       the per-head q/k ZCRMSNorm (normRotate,
//                       attention.go:298-330), RoPE of k, and Int8Rows.Append
//                       of k and v (int8.go:36-55, 125-141) through the
//                       streams' page tables; q is left normed for the
//                       attention, which rotates it.
//   norm_scaled_add_kernel  h += float32(s * ZCRMSNorm(y)): the attention's
//                       post norm and residual factor (block.go:183-188) and
//                       the cross branch's (cross.go:255-263, decoder.go:461-465).
//   expand_lanes_kernel / collapse_lanes_kernel  ExpandLanes / CollapseLanes
//                       (mhc.go:137-170): the mHC stream from the embedding
//                       row and the lane mean before the head.
//   page_copy_kernel    whole pages of an int8 cache (codes and scales), for
//                       the copy-on-write of a forked stream's last page.
//   gather_rows_kernel  float rows by index (a fork's tap history).
#include "cq_internal.hpp"
#include "cq_device.hpp"

namespace cqhip {
namespace {

// One (stream, projection) per workgroup, one 64-value head per wavefront
// (lane = value): z = 0 q, 1 k, 2 v.
__global__ __launch_bounds__(1024) void qkv_prep_kernel(PrepArgs a) {
    const int b = blockIdx.x, z = blockIdx.y, hh = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int D = a.dim, hk = D >> 6, c = hh * 64 + lane;
    __shared__ float rowbuf[16][64];
    __shared__ float rms_sh[16];
    const int p = a.pos[b];
    const float *src = z == 0 ? a.q : (z == 1 ? a.k : a.v);
    const float raw = src[static_cast<long long>(b) * D + c];
    float val = raw;
    if (a.taps > 0) {
        // The history is a ring of `taps` slots, row of position r at slot r
        // mod taps: the step at p reads slots of p - 1 .. p - taps + 1 and
        // writes slot p, which none of them is, so running a position again
        // (a graph's capture run, a stopped stream) reads the same rows.
        const float *w = a.taps_w + static_cast<long long>(z) * a.taps * D + c;
        const int T = a.taps;
        float *hz = T > 1 ? a.hist + static_cast<long long>(b) * T * 3 * D + static_cast<long long>(z) * D + c : nullptr;
        float acc = 0.0f;
        const float p0 = w[0] * raw;
        acc = acc + p0;
        for (int j = 1; j < T && j <= p; ++j) {  // positions before the first count as zero
            const int slot = (p - j) % T;
            const float pj = w[static_cast<long long>(j) * D] * hz[static_cast<long long>(slot) * 3 * D];
            acc = acc + pj;
        }
        if (T > 1 && p >= 0) hz[static_cast<long long>(p % T) * 3 * D] = raw;
        val = acc;
    }
    const float *gain = z == 0 ? a.qg : (z == 1 ? a.kg : nullptr);
    if (gain) {  // ZCRMSNorm over the head (norm.go:53-109)
        rowbuf[hh][lane] = val;
        __syncthreads();
        double part = 0.0;
        if (lane < 4) part = zc_partial(rowbuf[hh], 64, lane);
        const double p1 = __shfl(part, 1), p2 = __shfl(part, 2), p3 = __shfl(part, 3);
        if (lane == 0) rms_sh[hh] = zc_rms(part, p1, p2, p3, 64);
        __syncthreads();
        const float gx = gain[lane] * val;
        val = gx / rms_sh[hh];
    }
    if (z == 1 && a.cos_t && p >= 0 && p < a.positions) {  // RoPE (rope.go:69-81): i < 32 pairs with i + 32
        const float o = __shfl_xor(val, 32);
        const int jj = lane & 31;
        const float x1 = lane < 32 ? val : o, x2 = lane < 32 ? o : val;
        float o1, o2;
        rope_pair(x1, x2, a.cos_t[p * 32 + jj], a.sin_t[p * 32 + jj], o1, o2);
        val = lane < 32 ? o1 : o2;
    }
    if (z == 0) {
        a.q[static_cast<long long>(b) * D + c] = val;
        return;
    }
    // QuantizeRow of the head (int8.go:36-55), appended at row p.
    float m = fabsf(val);
#pragma unroll
    for (int h = 32; h > 0; h >>= 1) m = go_max(m, __shfl_xor(m, h));
    if (p < 0 || p >= a.cap) return;
    const float sc = m > 0.0f ? m / 127.0f : 1.0f;
    const long long pg = a.pages[static_cast<long long>(b) * a.page_stride + (p >> a.page_shift)];
    if (pg < 0 || pg >= a.pool_pages) return;
    const long long row = (pg << a.page_shift) + (p & ((1 << a.page_shift) - 1));
    int8_t *q8 = z == 1 ? a.kq : a.vq;
    float *s8 = z == 1 ? a.ks : a.vs;
    q8[row * D + c] = static_cast<int8_t>(go_int8_code(rintf(val / sc)));
    if (lane == 0) s8[row * hk + hh] = sc;
}

// A row of dim values (a multiple of 256, at most 4096) by 256 threads:
// thread t holds values t, t + 256, ... in registers and stores them in LDS
// transposed for the mean square's four in-order partial sums
// (zc_partial_t), which lanes 0-3 of wavefront 0 add. Returns the
// partials' sum of squares in float64 to every thread through LDS
// (norm.go:91-109).
constexpr int kRowMax = 4096;

__device__ __forceinline__ double row_square_sum(const float *row, int dim, float (&v)[kRowMax / 256], float *t,
                                                 double *sum_sh) {
    const int tid = threadIdx.x;
    const int V = dim >> 8, q = dim >> 2, stride = q + 4;
#pragma unroll
    for (int e = 0; e < kRowMax / 256; ++e)
        if (e < V) {
            const int i = tid + 256 * e;
            v[e] = row[i];
            t[(i & 3) * stride + (i >> 2)] = v[e];
        }
    __syncthreads();
    double part = 0.0;
    if (tid < 4) part = zc_partial_t(t, stride, q, tid);
    const double p1 = __shfl(part, 1), p2 = __shfl(part, 2), p3 = __shfl(part, 3);
    if (tid == 0) *sum_sh = ((part + p1) + p2) + p3;
    __syncthreads();
    return *sum_sh;
}

// h = resid + float32(s * ZCRMSNorm(y)) per row (resid may be h).
__global__ __launch_bounds__(256) void norm_scaled_add_kernel(float *h, const float *resid, const float *y,
                                                              const float *gain, float s, int dim) {
    __shared__ __align__(16) float t[4 * (kRowMax / 4 + 4)];
    __shared__ double sum_sh;
    const int r = blockIdx.x, tid = threadIdx.x;
    float v[kRowMax / 256];
    const double sum = row_square_sum(y + static_cast<long long>(r) * dim, dim, v, t, &sum_sh);
    // zc_rms: float32(sqrt(float64(float32(s / dim) + 1e-6)))
    const float ms = static_cast<float>(sum / static_cast<double>(dim));
    const float e = ms + 1e-6f;
    const float rms = static_cast<float>(sqrt(static_cast<double>(e)));
    const float *rr = resid + static_cast<long long>(r) * dim;
    float *hr = h + static_cast<long long>(r) * dim;
#pragma unroll
    for (int k = 0; k < kRowMax / 256; ++k)
        if (k < (dim >> 8)) {
            const int c = tid + 256 * k;
            const float gx = gain[c] * v[k];
            const float nv = gx / rms;
            const float sv = s * nv;
            hr[c] = rr[c] + sv;
        }
}

// RMSUnit (norm.go:68-81) of each row, x * float32(1 / sqrt(float64(ms +
// 1e-6))); with quant, then the fakeQuant of the whole row (int8.go:57-75,
// one chunk of dim): the mHC phi products' int8 input (mhc.go:99-106,
// linear.go:80-87).
__global__ __launch_bounds__(256) void rms_unit_row_kernel(float *dst, const float *x, int dim, int quant) {
    __shared__ __align__(16) float t[4 * (kRowMax / 4 + 4)];
    __shared__ double sum_sh;
    __shared__ float red[4];
    const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int V = dim >> 8;
    float v[kRowMax / 256];
    const double sum = row_square_sum(x + static_cast<long long>(r) * dim, dim, v, t, &sum_sh);
    const float ms = static_cast<float>(sum / static_cast<double>(dim));
    const float e = ms + 1e-6f;
    const float inv = static_cast<float>(1.0 / sqrt(static_cast<double>(e)));
#pragma unroll
    for (int k = 0; k < kRowMax / 256; ++k)
        if (k < V) v[k] = v[k] * inv;
    if (quant) {  // QuantizeRow's bound with Go's NaN-keeping max, then code * scale
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < kRowMax / 256; ++k)
            if (k < V) m = go_max(m, fabsf(v[k]));
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = go_max(m, __shfl_xor(m, off));
        if (lane == 0) red[wave] = m;
        __syncthreads();
        m = go_max(go_max(red[0], red[1]), go_max(red[2], red[3]));
        const float sc = m > 0.0f ? m / 127.0f : 1.0f;
#pragma unroll
        for (int k = 0; k < kRowMax / 256; ++k)
            if (k < V) v[k] = static_cast<float>(go_int8_code(rintf(v[k] / sc))) * sc;
    }
    float *out = dst + static_cast<long long>(r) * dim;
#pragma unroll
    for (int k = 0; k < kRowMax / 256; ++k)
        if (k < V) out[tid + 256 * k] = v[k];
}

__global__ __launch_bounds__(256) void expand_lanes_kernel(float *stream, const float *x, int lanes, int dim,
                                                           long long n) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;  // n = rows * lanes * dim
    const long long r = i / (static_cast<long long>(lanes) * dim);
    const int c = static_cast<int>(i % dim);
    stream[i] = x[r * dim + c];
}

__global__ __launch_bounds__(256) void collapse_lanes_kernel(float *x, const float *stream, int lanes, int dim,
                                                             long long n) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;  // n = rows * dim
    const long long r = i / dim;
    const int c = static_cast<int>(i % dim);
    const float *sr = stream + r * lanes * dim + c;
    float acc = 0.0f;
    for (int k = 0; k < lanes; ++k) acc = acc + sr[static_cast<long long>(k) * dim];
    x[i] = acc / static_cast<float>(lanes);
}

// Pair j: page dst[j] of the cache becomes a copy of page src[j] (rows of
// cols codes and heads scales).
__global__ __launch_bounds__(256) void page_copy_kernel(int8_t *q, float *s, const int32_t *src, const int32_t *dst,
                                                        int page_rows, int cols, int heads, int pool_pages) {
    const int j = blockIdx.x;
    const long long from = src[j], to = dst[j];
    if (from < 0 || from >= pool_pages || to < 0 || to >= pool_pages) return;  // outside the pool: no copy
    const long long qb = static_cast<long long>(page_rows) * cols, sb = static_cast<long long>(page_rows) * heads;
    const int8_t *qs = q + from * qb;
    int8_t *qd = q + to * qb;
    if ((qb & 15) == 0) {
        const int4 *s4 = reinterpret_cast<const int4 *>(qs);
        int4 *d4 = reinterpret_cast<int4 *>(qd);
        for (long long i = threadIdx.x; i < qb / 16; i += blockDim.x) d4[i] = s4[i];
    } else {
        for (long long i = threadIdx.x; i < qb; i += blockDim.x) qd[i] = qs[i];
    }
    for (long long i = threadIdx.x; i < sb; i += blockDim.x) s[to * sb + i] = s[from * sb + i];
}

__global__ __launch_bounds__(256) void gather_float_rows_kernel(float *dst, const float *src, const int32_t *idx,
                                                                long long width) {
    const int r = blockIdx.y;
    const long long from = idx ? idx[r] : r;
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < width) dst[r * width + i] = src[from * width + i];
}

unsigned blocks_of(long long n, int t) { return static_cast<unsigned>((n + t - 1) / t); }

}  // namespace

hipError_t launch_qkv_prep(const PrepArgs &a, int batch, hipStream_t s) {
    if (batch <= 0) return hipSuccess;
    hipLaunchKernelGGL(qkv_prep_kernel, dim3(batch, 3), dim3(a.dim), 0, s, a);
    return hipGetLastError();
}

bool row_kernel_dim(int dim) { return dim > 0 && dim % 256 == 0 && dim <= kRowMax; }

hipError_t launch_norm_scaled_add(float *h, const float *resid, const float *y, const float *gain, float sc, int rows,
                                  int dim, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(norm_scaled_add_kernel, dim3(rows), dim3(256), 0, s, h, resid, y, gain, sc, dim);
    return hipGetLastError();
}

hipError_t launch_rms_unit_row(float *dst, const float *x, int rows, int dim, int quant, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(rms_unit_row_kernel, dim3(rows), dim3(256), 0, s, dst, x, dim, quant);
    return hipGetLastError();
}

hipError_t launch_expand_lanes(float *stream, const float *x, int rows, int lanes, int dim, hipStream_t s) {
    const long long n = static_cast<long long>(rows) * lanes * dim;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(expand_lanes_kernel, dim3(blocks_of(n, 256)), dim3(256), 0, s, stream, x, lanes, dim, n);
    return hipGetLastError();
}

hipError_t launch_collapse_lanes(float *x, const float *stream, int rows, int lanes, int dim, hipStream_t s) {
    const long long n = static_cast<long long>(rows) * dim;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(collapse_lanes_kernel, dim3(blocks_of(n, 256)), dim3(256), 0, s, x, stream, lanes, dim, n);
    return hipGetLastError();
}

hipError_t launch_page_copy(int8_t *q, float *sc, const int32_t *src, const int32_t *dst, int n, int page_rows,
                            int cols, int heads, int pool_pages, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(page_copy_kernel, dim3(n), dim3(256), 0, s, q, sc, src, dst, page_rows, cols, heads,
                       pool_pages);
    return hipGetLastError();
}

hipError_t launch_gather_float_rows(float *dst, const float *src, const int32_t *idx, int rows, long long width,
                                    hipStream_t s) {
    if (rows <= 0 || width <= 0) return hipSuccess;
    hipLaunchKernelGGL(gather_float_rows_kernel, dim3(blocks_of(width, 256), rows), dim3(256), 0, s, dst, src, idx,
                       width);
    return hipGetLastError();
}

}  // namespace cqhip
