// gfx950 manifold hyper-connections around a block (internal/needle/mhc.go),
// the pieces on either side of the φ products (which are CQ GEMMs of
// In = lanes * dim): RMSUnit of the lane stream (norm.go:68-81), the heads
// h_pre = sigmoid, h_post = 2 sigmoid and h_res = sinkhorn of their logits
// with the block input u = sum_k h_pre[k] stream[k] (mhc.go:204-219), and
// the mix out[a] = sum_b h_res[a, b] stream[b] + h_post[a] (block(u) - u)
// (mhc.go:229-299). Each is the reference's float32 arithmetic in its
// order; the Sinkhorn runs in float64 in the exp domain (exp_f64, the
// CPU restatement's operations) while the logits' spread allows it, else
// in float32 in the log domain (mhc.go:301-417).
#include "cq_internal.hpp"
#include "cq_device.hpp"

namespace cqhip {
namespace {

constexpr int kMhcMaxLanes = 8;

__global__ __launch_bounds__(64) void rms_unit_kernel(float *dst, const float *x, int dim) {
    const float *row = x + static_cast<long long>(blockIdx.x) * dim;
    float *out = dst + static_cast<long long>(blockIdx.x) * dim;
    const int lane = threadIdx.x;
    const double part = lane < 4 ? zc_partial(row, dim, lane) : 0.0;
    const double p0 = __shfl(part, 0), p1 = __shfl(part, 1), p2 = __shfl(part, 2), p3 = __shfl(part, 3);
    const double s = ((p0 + p1) + p2) + p3;
    const float ms = static_cast<float>(s / static_cast<double>(dim));
    const float e = ms + 1e-6f;
    const float inv = static_cast<float>(1.0 / sqrt(static_cast<double>(e)));
    for (int c = lane; c < dim; c += 64) out[c] = row[c] * inv;
}

// sinkhorn (mhc.go:301-399) of one n x n matrix in k (LDS) by one
// wavefront: lane t < n*n holds entry t = r*n + c. Rows (then columns) are
// independent within a pass, so each lane forms its row's (column's) sum in
// the reference's order from its neighbours' values and divides its own
// entry: the serial routine's operations, n*n of them at a time.
__device__ void sinkhorn_wave(float *k, int n, int iters, int lane) {
    const int nn = n * n;
    const bool act = lane < nn;
    const int r = act ? lane / n : 0, c = act ? lane - r * n : 0;
    float kv = act ? k[lane] : k[0];  // idle lanes repeat entry 0: neutral for min and max
    // slices.Min / slices.Max keep a NaN; min and max are exact in any order
    float lo = kv, hi = kv;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        lo = go_min(lo, __shfl_xor(lo, off));
        hi = go_max(hi, __shfl_xor(hi, off));
    }
    const double spread = static_cast<double>(hi) - static_cast<double>(lo);
    if (!(isinf(spread) || isnan(spread) || spread + 2.0 * iters * log(static_cast<double>(n)) > 700.0)) {
        double e = exp_f64(static_cast<double>(kv) - static_cast<double>(hi));
        for (int it = 0; it < iters; ++it) {
            double s = 0.0;
            for (int j = 0; j < n; ++j) s = s + __shfl(e, r * n + j);
            e = e / s;
            s = 0.0;
            for (int j = 0; j < n; ++j) s = s + __shfl(e, j * n + c);
            e = e / s;
        }
        if (act) k[lane] = static_cast<float>(e);
        return;
    }
    // logSumExp (mhc.go:401-417) of the lane's row (then column), in order
    auto lse = [&](int base, int stride) {
        float m = -INFINITY;
        for (int j = 0; j < n; ++j) m = go_max(m, __shfl(kv, base + j * stride));
        if (isinf(m)) m = 0.0f;
        float s = 0.0f;
        for (int j = 0; j < n; ++j) s = s + static_cast<float>(exp_f64(static_cast<double>(__shfl(kv, base + j * stride) - m)));
        return m + static_cast<float>(log(static_cast<double>(s)));
    };
    for (int it = 0; it < iters; ++it) {
        kv = kv - lse(r * n, 1);
        kv = kv - lse(c, n);
    }
    if (act) k[lane] = static_cast<float>(exp_f64(static_cast<double>(kv)));
}

__global__ __launch_bounds__(256) void mhc_heads_kernel(MhcArgs m) {
    __shared__ float hp[kMhcMaxLanes], kr[kMhcMaxLanes * kMhcMaxLanes];
    const int i = blockIdx.x, tid = threadIdx.x, n = m.lanes, dim = m.dim;
    const float *A = m.affine;  // {a_pre, a_post, a_res, b_pre[n], pre_off[n], b_post[n], post_off[n], b_res[n*n]}
    const long long ps = m.logit_stride ? m.logit_stride : n, rs = m.logit_stride ? m.logit_stride : n * n;
    if (tid < n) {
        float p = m.pre_logits[i * ps + tid], q = m.post_logits[i * ps + tid];
        if (A) {
            const float ap = A[0] * p;
            p = ap + A[3 + tid] + A[3 + n + tid];
            const float aq = A[1] * q;
            q = aq + A[3 + 2 * n + tid] + A[3 + 3 * n + tid];
        }
        const float h = gate_sigmoid(p);
        hp[tid] = h;
        m.h_pre[i * n + tid] = h;
        m.h_post[i * n + tid] = 2.0f * gate_sigmoid(q);
    }
    if (tid < n * n) {
        float v = m.res_logits[i * rs + tid];
        if (A) {
            const float av = A[2] * v;
            v = av + A[3 + 4 * n + tid];
        }
        kr[tid] = v;
    }
    __syncthreads();
    if (tid < 64) sinkhorn_wave(kr, n, 20, tid);
    const float *st = m.stream + static_cast<long long>(i) * n * dim;
    for (int c = tid; c < dim; c += blockDim.x) {  // u = sum_k h_pre[k] stream[k], k in order
        float u = 0.0f;
        for (int k = 0; k < n; ++k) {
            const float pr = hp[k] * st[static_cast<long long>(k) * dim + c];
            u = u + pr;
        }
        m.u[static_cast<long long>(i) * dim + c] = u;
    }
    __syncthreads();
    if (tid < n * n) m.h_res[static_cast<long long>(i) * n * n + tid] = kr[tid];
}

__global__ __launch_bounds__(256) void mhc_mix_kernel(MhcArgs m) {
    const int i = blockIdx.x, a = blockIdx.y, n = m.lanes, dim = m.dim;
    const float *st = m.stream + static_cast<long long>(i) * n * dim;
    const float *hr = m.h_res + (static_cast<long long>(i) * n + a) * n;
    const float hpost = m.h_post[i * n + a];
    float *o = m.out + (static_cast<long long>(i) * n + a) * dim;
    for (int c = threadIdx.x; c < dim; c += blockDim.x) {
        float v = 0.0f;
        for (int b = 0; b < n; ++b) {
            const float pr = hr[b] * st[static_cast<long long>(b) * dim + c];
            v = v + pr;
        }
        const float y = m.block_out[static_cast<long long>(i) * dim + c] - m.u[static_cast<long long>(i) * dim + c];
        const float py = hpost * y;
        o[c] = v + py;
    }
}

}  // namespace

bool mhc_shape_ok(int lanes, int dim) { return lanes > 0 && lanes <= kMhcMaxLanes && dim > 0; }

hipError_t launch_rms_unit(float *dst, const float *x, int rows, int dim, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(rms_unit_kernel, dim3(static_cast<unsigned>(rows)), dim3(64), 0, s, dst, x, dim);
    return hipGetLastError();
}

hipError_t launch_mhc_heads(const MhcArgs &m, int rows, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(mhc_heads_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, s, m);
    return hipGetLastError();
}

hipError_t launch_mhc_mix(const MhcArgs &m, int rows, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(mhc_mix_kernel, dim3(static_cast<unsigned>(rows), static_cast<unsigned>(m.lanes)), dim3(256),
                       0, s, m);
    return hipGetLastError();
}

}  // namespace cqhip
