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
#include "cq_device.hpp"

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
    for (int i = lane; i < width; i += 64) m = go_max(m, fabsf(xc[i]));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = go_max(m, __shfl_xor(m, off));
    const float sc = m > 0.0f ? m / 127.0f : 1.0f;  // a NaN bound fails m > 0: scale 1
    int8_t *qc = q + c * width;
    for (int i = lane; i < width; i += 64) qc[i] = static_cast<int8_t>(go_int8_code(rintf(xc[i] / sc)));
    if (lane == 0) s[c] = sc;
}

// fakeQuant (int8.go:57-75): each chunk of width values through QuantizeRow
// and back, dst = float32(q) * s (the input of a Linear WithInt8Input,
// quantInput, int8.go:81-88). dst may be x: a chunk's reads for its bound
// finish before its writes.
__global__ __launch_bounds__(256) void fake_quant_kernel(float *dst, const float *x, long long chunks, int width) {
    const int lane = threadIdx.x & 63;
    const long long c = static_cast<long long>(blockIdx.x) * (blockDim.x / 64) + (threadIdx.x >> 6);
    if (c >= chunks) return;
    const float *xc = x + c * width;
    float m = 0.0f;
    for (int i = lane; i < width; i += 64) m = go_max(m, fabsf(xc[i]));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = go_max(m, __shfl_xor(m, off));
    const float sc = m > 0.0f ? m / 127.0f : 1.0f;
    float *dc = dst + c * width;
    for (int i = lane; i < width; i += 64)
        dc[i] = static_cast<float>(go_int8_code(rintf(xc[i] / sc))) * sc;  // float32(q): a code of 0 is +0, never -0
}

// Stream b of dst gets rows [0, len[b]) of stream idx[b] of src (idx null:
// of stream b; len clamped to the stream's cap rows; idx outside the streams
// copies nothing), each stream cap rows of row_bytes; 16-byte pieces when
// every row and stream start is 16-byte aligned. Grid: (pieces per
// workgroup chunk, streams).
__global__ __launch_bounds__(256) void gather_rows_kernel(unsigned char *dst, const unsigned char *src,
                                                          const int32_t *idx, const int32_t *len, int streams,
                                                          long long stream_bytes, int row_bytes, int vec) {
    const int b = blockIdx.y;
    const int from = idx ? idx[b] : b;
    const int n = len[b];
    if (from < 0 || from >= streams || n <= 0) return;
    const long long bytes = min(static_cast<long long>(n) * row_bytes, stream_bytes);  // at most the stream's cap rows
    const unsigned char *sp = src + from * stream_bytes;
    unsigned char *dp = dst + b * stream_bytes;
    const long long step = static_cast<long long>(gridDim.x) * blockDim.x;
    if (vec) {
        for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < bytes / 16; i += step)
            reinterpret_cast<uint4 *>(dp)[i] = reinterpret_cast<const uint4 *>(sp)[i];
    } else {
        for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < bytes; i += step)
            dp[i] = sp[i];
    }
}

__device__ __forceinline__ float exp_generic(float d) { return static_cast<float>(exp(static_cast<double>(d))); }

constexpr int kAttThreads = 256;

// Element c of query head qi, after RoPE at table row p when a.rope_cos is
// set (rope.go:69-81; pairs (j, j + qk/2)).
__device__ __forceinline__ float query_value(const AttendArgs &a, const float *qi, int p, int c) {
    if (!a.rope_cos) return qi[c];
    const int half = a.qk / 2;
    const int j = c < half ? c : c - half;
    float o1, o2;
    rope_pair(qi[j], qi[j + half], a.rope_cos[static_cast<long long>(p) * half + j],
              a.rope_sin[static_cast<long long>(p) * half + j], o1, o2);
    return c < half ? o1 : o2;
}

__device__ __forceinline__ float block_max(float v, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = go_max(v, __shfl_xor(v, off));
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < kAttThreads / 64; ++w) r = go_max(r, red[w]);
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
    const long long kb = attend_cache_of(a, b);  // the cache this stream reads
    if (kb < 0 || lo0 < 0 || len0 < 0 || sp[1] > a.nk_max || lo1 < 0 || len1 < 0 || sp[3] > a.nk_max)
        return;  // spans off the cache, or no cache
    attend_stage_pages(a, b, smem);  // paged: the stream's page table into LDS
    const int32_t *pgs = reinterpret_cast<const int32_t *>(smem + a.page_lds);

    float *s = reinterpret_cast<float *>(smem);  // n logits, then weights
    int8_t *vbuf = reinterpret_cast<int8_t *>(s + ((a.nk_max + 3) & ~3));  // value codes: one or two chunks
    __shared__ float red[8];
    __shared__ __align__(16) int8_t q8[256];
    __shared__ float qg[256];
    __shared__ float sq_sh, sum_sh;

    const float *qi = a.q + b * a.q_stride + (static_cast<long long>(i) * a.heads + h) * a.qk;
    const int8_t *kq = a.kq + kb * a.kv_stride;
    const float *ks = a.ks + kb * a.s_stride;
    const int8_t *vq = a.vq + kb * a.kv_stride;
    const float *vs = a.vs + kb * a.s_stride;
    auto key_of = [&](int j) { return j < len0 ? lo0 + j : lo1 + (j - len0); };

    // The query head (after RoPE when asked), then QuantizeRow of it
    // (int8.go:226-228).
    const int qp = a.rope_cos ? a.qpos[static_cast<long long>(b) * a.t + i] : 0;
    for (int c = tid; c < a.qk; c += kAttThreads) qg[c] = query_value(a, qi, qp, c);
    __syncthreads();
    if (a.quant_q) {
        float m = 0.0f;
        for (int c = tid; c < a.qk; c += kAttThreads) m = go_max(m, fabsf(qg[c]));
        m = block_max(m, red);
        const float sc = m > 0.0f ? m / 127.0f : 1.0f;
        for (int c = tid; c < a.qk; c += kAttThreads) q8[c] = static_cast<int8_t>(go_int8_code(rintf(qg[c] / sc)));
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
            // (past the end a load repeats the last piece, so the eight stay
            // in registers; only real pieces are stored)
            const int per = a.vd / 16, total = cnt * per;
            for (int e0 = t0; e0 < total; e0 += 8 * nt) {
                int4 w[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int e = min(e0 + u * nt, total - 1);
                    const int jj = e / per, part = e - (e / per) * per;
                    w[u] = *reinterpret_cast<const int4 *>(vq + attend_row(a, pgs, key_of(j0 + jj)) * a.v_cols +
                                                           kv * a.vd + part * 16);
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
                buf[jj * a.vd + d] = vq[attend_row(a, pgs, key_of(j0 + jj)) * a.v_cols + kv * a.vd + d];
            }
        }
    };
    if (nchunks > 0) stage(0, vbuf, tid, kAttThreads);

    // 1. Logits, one thread per key (int8Logits / dotsF32I8), four keys at
    // a time so that their loads are in flight together.
    auto logit = [&](int j) -> float {
        const int key = key_of(j);
        const int8_t *krow = kq + attend_row(a, pgs, key) * a.k_cols + kv * a.qk;
        const float sk = ks[attend_row(a, pgs, key) * kv_heads + kv];
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
                const float pr = qg[c + e] * static_cast<float>(static_cast<int8_t>(w >> (8 * e)));
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
    for (int j = tid; j < n; j += kAttThreads) m = go_max(m, s[j]);
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
        s[j] = p * vs[attend_row(a, pgs, key_of(j)) * kv_heads + kv];
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


// s_waitcnt vmcnt(K), every other counter left alone (gfx9 encoding).
template <int K>
__device__ __forceinline__ void wait_vm_const() {
    __builtin_amdgcn_s_waitcnt((K & 15) | ((K >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Wait until at most k of this wavefront's vector-memory loads are in flight
// (loads retire in order). Counts above 24 wait for 24, which is stricter.
__device__ __forceinline__ void wait_vm(int k) {
    switch (k < 0 ? 0 : k) {
#define CQ_WAIT_CASE(K) \
    case K: wait_vm_const<K>(); break;
        CQ_WAIT_CASE(0) CQ_WAIT_CASE(1) CQ_WAIT_CASE(2) CQ_WAIT_CASE(3) CQ_WAIT_CASE(4) CQ_WAIT_CASE(5)
        CQ_WAIT_CASE(6) CQ_WAIT_CASE(7) CQ_WAIT_CASE(8) CQ_WAIT_CASE(9) CQ_WAIT_CASE(10) CQ_WAIT_CASE(11)
        CQ_WAIT_CASE(12) CQ_WAIT_CASE(13) CQ_WAIT_CASE(14) CQ_WAIT_CASE(15) CQ_WAIT_CASE(16) CQ_WAIT_CASE(17)
        CQ_WAIT_CASE(18) CQ_WAIT_CASE(19) CQ_WAIT_CASE(20) CQ_WAIT_CASE(21) CQ_WAIT_CASE(22) CQ_WAIT_CASE(23)
#undef CQ_WAIT_CASE
    default: wait_vm_const<24>(); break;
    }
}

// Byte offset of an LDS location, as M0 and the LDS instructions take it.
__device__ __forceinline__ unsigned lds_offset(const void *p) {
    return static_cast<unsigned>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char *)(p)));
}

// One 16-byte global load per lane straight into LDS: lane l's bytes land
// at lds + 16 * l (global_load_lds_dwordx4, M0 = lds). Issued as inline
// assembly so that the compiler does not wait for it before every later LDS
// read; its completion is the caller's wait_vm before a barrier. The K/V
// rows are read once per call, so the load is non-temporal (nt): streaming
// them does not push the products' weights and inputs out of the caches
// (decode step at batch 256: 1.769 -> 1.686 ms, the cross call ~7% faster
// alone).
__device__ __forceinline__ void dma16(const void *src, unsigned lds) {
    asm volatile("global_load_lds_dwordx4 %0, off nt" ::"v"(src), "{m0}"(lds) : "memory");
}

// Geometry of the streamed attention kernel: value heads of VD codes,
// chunks of JC keys.
template <int VD, int JC>
struct StreamGeo {
    static constexpr int kKpt = JC == 64 ? 6 : 4;       // keys per thread per round of logits
    static constexpr int kCW = VD / 64;                 // chain wavefronts: one output per lane
    static constexpr int kPW = kAttThreads / 64 - kCW;  // product wavefronts
    static constexpr int kJC = JC;                      // keys per chunk
    static constexpr int kPitch = JC + 4;               // floats per product row (16 B times an odd number)
    static constexpr int kSeg = VD / 16;                // 16-byte pieces per value row
    static constexpr int kPieces = JC * kSeg;           // pieces per chunk = product items per chunk
    static constexpr int kDma = kPieces / 64;           // wavefront-wide LDS-DMA loads per chunk
    static_assert(kDma * 64 == kPieces, "a chunk is whole wavefront loads");
    static_assert((kPitch / 4) % 2 == 1, "product rows 16 B times an odd number apart");
};

constexpr int kStreamQk = 64;  // widest key head the streamed kernel holds in registers

// AttendInt8Spans for one (stream, query row, head) per workgroup, value
// heads of VD codes (the launcher uses it for 128), key heads of at most 64
// codes, 16-byte aligned rows. Same arithmetic as attend_kernel; the work is
// ordered for latency:
//   - the query and the first keys of every thread are loaded together,
//     the keys into registers (kKpt keys per thread at a time);
//   - value rows stream from HBM straight into an LDS ring of chunks of JC
//     keys (global_load_lds, issued up to rs chunks ahead, all of the stream
//     when `rs` covers it), laid out [16-byte piece][key]; the first chunks
//     are issued after the logits, under the softmax;
//   - the product wavefronts turn a chunk into float32 products
//     fl(w_j * code_jd), stored [d][key] in one of two LDS buffers;
//   - meanwhile each chain lane d adds the previous chunk's products of its
//     output in key order, four per 16-byte LDS read, a chunk's reads
//     issued at once.
// With `swz`, workgroup w serves stream (w mod 8) + 8 * (w / (8 * heads * t))
// (one stream's heads on one XCD, whose L2 then holds the 128-byte lines
// its heads share); otherwise stream w / (heads * t).
template <int VD, int JC>
__global__ __launch_bounds__(kAttThreads) void attend_stream_kernel(AttendArgs a, int rs, int swz) {
    using G = StreamGeo<VD, JC>;
    extern __shared__ __align__(16) unsigned char smem[];
    const int per = a.heads * a.t;
    const int w = blockIdx.x;
    int b, r;
    if (swz) {
        const int full = (a.batch & ~7) * per;
        if (w < full) {
            b = (w & 7) + 8 * (w / (8 * per));
            r = (w >> 3) % per;
        } else {
            const int w2 = w - full, rem = a.batch & 7;
            b = (a.batch & ~7) + w2 % rem;
            r = w2 / rem;
        }
    } else {
        b = w / per;
        r = w - b * per;
    }
    const int h = r % a.heads, i = r / a.heads;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the DMA's LDS base goes to M0
    const int kv_heads = a.k_cols / a.qk;
    const int kv = h / (a.heads / kv_heads);
    const int32_t *sp = a.spans + (static_cast<long long>(b) * a.t + i) * 4;
    const int lo0 = sp[0], len0 = sp[1] - sp[0], lo1 = sp[2], len1 = sp[3] - sp[2];
    const int n = len0 + len1;
    const long long kb = attend_cache_of(a, b);  // the cache this stream reads
    if (kb < 0 || lo0 < 0 || len0 < 0 || sp[1] > a.nk_max || lo1 < 0 || len1 < 0 || sp[3] > a.nk_max)
        return;  // spans off the cache, or no cache
    float *outp = a.out + b * a.out_stride + (static_cast<long long>(i) * a.heads + h) * VD;
    if (n == 0) {
        if (tid < VD) outp[tid] = 0.0f;
        return;
    }
    attend_stage_pages(a, b, smem);  // paged: the stream's page table into LDS
    const int32_t *pgs = reinterpret_cast<const int32_t *>(smem + a.page_lds);

    const int nk_pad = (a.nk_max + 3) & ~3;
    float *s = reinterpret_cast<float *>(smem);  // logits, exponentials, then weights
    float *vsb = s + nk_pad;                     // value scales of the keys
    float *P = vsb + nk_pad;                     // two product buffers [VD][kPitch]
    int8_t *ring = reinterpret_cast<int8_t *>(P + 2 * VD * G::kPitch);
    __shared__ float red[8];
    __shared__ __align__(16) int8_t q8[kStreamQk];
    __shared__ __align__(16) float qf[kStreamQk];
    __shared__ float sq_sh, sum_sh;

    const float *qi = a.q + b * a.q_stride + (static_cast<long long>(i) * a.heads + h) * a.qk;
    const int8_t *kq = a.kq + kb * a.kv_stride;
    const float *ks = a.ks + kb * a.s_stride;
    const int8_t *vq = a.vq + kb * a.kv_stride;
    const float *vs = a.vs + kb * a.s_stride;
    auto key_of = [&](int j) { return j < len0 ? lo0 + j : lo1 + (j - len0); };

    const int nch = (n + G::kJC - 1) / G::kJC;
    const bool producer = wave >= G::kCW;
    const int pw = wave - G::kCW, ptid = tid - 64 * G::kCW;
    const int lw = producer ? (G::kDma - pw + G::kPW - 1) / G::kPW : 0;  // this wavefront's DMA loads per chunk

    // Chunk c of value rows into ring slot c % rs: piece p = (segment,
    // key) lands at p * 16; keys past the stream's end re-read its first key.
    auto dma = [&](int c) {
        const int j0 = c * G::kJC, cnt = min(G::kJC, n - j0);
        int8_t *slot = ring + (c % rs) * (G::kJC * VD);
        for (int u = pw; u < G::kDma; u += G::kPW) {
            const int p = u * 64 + lane;
            const int seg = p / G::kJC, jj = p - seg * G::kJC;
            const int key = key_of(j0 + (jj < cnt ? jj : 0));
            dma16(vq + attend_row(a, pgs, key) * a.v_cols + kv * VD + seg * 16, lds_offset(slot + u * 64 * 16));
        }
    };

    // 1. The query, then the first four keys of this thread, in flight together.
    const int kpieces = a.qk / 16;
    const int qp = a.rope_cos ? a.qpos[static_cast<long long>(b) * a.t + i] : 0;
    const float qv = tid < a.qk ? query_value(a, qi, qp, tid) : 0.0f;
    constexpr int KPT = G::kKpt;
    int4 kw[KPT][kStreamQk / 16];
    float skr[KPT], vsr[KPT];
    auto kload = [&](int g, int j) {
        const int key = key_of(j);
        const int8_t *krow = kq + attend_row(a, pgs, key) * a.k_cols + kv * a.qk;
#pragma unroll
        for (int p = 0; p < kStreamQk / 16; ++p)
            if (p < kpieces) kw[g][p] = *reinterpret_cast<const int4 *>(krow + 16 * p);
        skr[g] = ks[attend_row(a, pgs, key) * kv_heads + kv];
        vsr[g] = vs[attend_row(a, pgs, key) * kv_heads + kv];
    };
    auto logit = [&](int g) -> float {
        if (a.quant_q) {
            int dot = 0;  // exact in any order
#pragma unroll
            for (int p = 0; p < kStreamQk / 16; ++p)
                if (p < kpieces) {
                    const int4 qw = *reinterpret_cast<const int4 *>(q8 + 16 * p);
                    dot = __builtin_amdgcn_sdot4(kw[g][p].x, qw.x, dot, false);
                    dot = __builtin_amdgcn_sdot4(kw[g][p].y, qw.y, dot, false);
                    dot = __builtin_amdgcn_sdot4(kw[g][p].z, qw.z, dot, false);
                    dot = __builtin_amdgcn_sdot4(kw[g][p].w, qw.w, dot, false);
                }
            const float scl = sq_sh * skr[g];
            const float t1 = static_cast<float>(dot) * scl;
            return t1 / a.scale;
        }
        float dot = 0.0f;  // in order
#pragma unroll
        for (int p = 0; p < kStreamQk / 16; ++p)
            if (p < kpieces) {
                const int cw[4] = {kw[g][p].x, kw[g][p].y, kw[g][p].z, kw[g][p].w};
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const float pr = qf[16 * p + e] * static_cast<float>(static_cast<int8_t>(cw[e >> 2] >> (8 * (e & 3))));
                    dot = dot + pr;
                }
            }
        const float t1 = dot * skr[g];
        return t1 / a.scale;
    };
#pragma unroll
    for (int g = 0; g < KPT; ++g)
        if (tid + g * kAttThreads < n) kload(g, tid + g * kAttThreads);

    // QuantizeRow of the query head (int8.go:226-228).
    if (tid < a.qk) qf[tid] = qv;
    if (a.quant_q) {
        const float m = block_max(tid < a.qk ? fabsf(qv) : 0.0f, red);
        const float sc = m > 0.0f ? m / 127.0f : 1.0f;
        if (tid < a.qk) {
            q8[tid] = static_cast<int8_t>(go_int8_code(rintf(qv / sc)));
        }
        if (tid == 0) sq_sh = sc;
    }
    __syncthreads();

    // Logits (int8Logits / dotsF32I8), KPT keys per thread per round; the
    // keys' value scales go to LDS beside them.
    for (int j0 = 0; j0 < n; j0 += KPT * kAttThreads) {
        if (j0 > 0) {
#pragma unroll
            for (int g = 0; g < KPT; ++g)
                if (j0 + tid + g * kAttThreads < n) kload(g, j0 + tid + g * kAttThreads);
        }
#pragma unroll
        for (int g = 0; g < KPT; ++g) {
            const int j = j0 + tid + g * kAttThreads;
            if (j < n) {
                s[j] = logit(g);
                vsb[j] = vsr[g];
            }
        }
    }
    __syncthreads();

    // The first rs chunks of value rows start streaming now, under the
    // softmax. The compiler's own loads are drained first: loads retire in
    // order, so any wait for one of them issued later would also wait for
    // the value rows queued behind it.
    wait_vm_const<0>();
    if (producer) {
        const int c0 = min(rs, nch);
        for (int c = 0; c < c0; ++c) dma(c);
    }

    // 2. softmaxInPlace with amd64's expSubSum. The eight lane sums read
    // the exponentials from a copy transposed to [lane][index] in the
    // product buffers (free until step 3) when it fits.
    float m = -INFINITY;
    for (int j = tid; j < n; j += kAttThreads) m = go_max(m, s[j]);
    m = block_max(m, red);
    const int n8 = n & ~7;
    const bool kernel_path = n8 > 0;
    const int r8 = ((n8 >> 3) + 3) & ~3;
    const bool transposed = kernel_path && 8 * r8 <= 2 * VD * G::kPitch;
    for (int j = tid; j < n8; j += kAttThreads) {
        const float e = exp_lane(s[j] - m);
        s[j] = e;
        if (transposed) P[(j & 7) * r8 + (j >> 3)] = e;
    }
    for (int j = n8 + tid; j < n; j += kAttThreads) s[j] = exp_generic(s[j] - m);
    __syncthreads();
    if (tid < 8 && kernel_path) {  // lane tid of the 8-lane sum, elements in order
        float acc = 0.0f;
        if (transposed) {
            const float *row = P + tid * r8;
            const int cnt = n8 >> 3;
            int k = 0;
            for (; k + 16 <= cnt; k += 16) {
                const float4 v0 = *reinterpret_cast<const float4 *>(row + k);
                const float4 v1 = *reinterpret_cast<const float4 *>(row + k + 4);
                const float4 v2 = *reinterpret_cast<const float4 *>(row + k + 8);
                const float4 v3 = *reinterpret_cast<const float4 *>(row + k + 12);
                acc = acc + v0.x; acc = acc + v0.y; acc = acc + v0.z; acc = acc + v0.w;
                acc = acc + v1.x; acc = acc + v1.y; acc = acc + v1.z; acc = acc + v1.w;
                acc = acc + v2.x; acc = acc + v2.y; acc = acc + v2.z; acc = acc + v2.w;
                acc = acc + v3.x; acc = acc + v3.y; acc = acc + v3.z; acc = acc + v3.w;
            }
            for (; k < cnt; ++k) acc = acc + row[k];
        } else {
            for (int j = tid; j < n8; j += 8) acc = acc + s[j];
        }
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
        s[j] = p * vsb[j];
    }

    // 3. axpysI8 per output, keys in order, over the chunk pipeline. Before
    // the barrier that opens iteration c, chunk c + 1 has landed in the ring.
    auto produce = [&](int c) {
        const int j0 = c * G::kJC, cnt = min(G::kJC, n - j0);
        const int8_t *slot = ring + (c % rs) * (G::kJC * VD);
        float *pb = P + (c & 1) * (VD * G::kPitch);
        for (int e = ptid; e < G::kPieces; e += 64 * G::kPW) {
            const int seg = e / G::kJC, jj = e - seg * G::kJC;
            if (jj < cnt) {
                const int4 c4 = *reinterpret_cast<const int4 *>(slot + e * 16);
                const float wj = s[j0 + jj];
                float *col = pb + seg * 16 * G::kPitch + jj;
                const int cw[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const float code = static_cast<float>(static_cast<int8_t>(cw[q] >> (8 * k)));
                        col[(4 * q + k) * G::kPitch] = wj * code;
                    }
            }
        }
    };
    const int hi0 = min(rs, nch) - 1;  // the last chunk issued so far
    if (producer) wait_vm(lw * hi0);   // chunk 0 has landed
    __syncthreads();                   // weights in LDS
    if (producer) {
        produce(0);
        if (nch > 1) wait_vm(lw * (hi0 - 1));
    }
    __syncthreads();
    float acc = 0.0f;
    for (int c = 0; c < nch; ++c) {
        if (producer) {
            if (c + rs < nch) dma(c + rs);  // slot c % rs was last read producing chunk c
            if (c + 1 < nch) produce(c + 1);
            if (c + 2 < nch) wait_vm(lw * (min(c + rs, nch - 1) - (c + 2)));
        } else {
            const int cnt = min(G::kJC, n - c * G::kJC);
            const float *row = P + (c & 1) * (VD * G::kPitch) + tid * G::kPitch;
            if (cnt == G::kJC) {  // a full chunk: every read issued, then the adds
                float4 v[G::kJC / 4];
#pragma unroll
                for (int q = 0; q < G::kJC / 4; ++q) v[q] = *reinterpret_cast<const float4 *>(row + 4 * q);
#pragma unroll
                for (int q = 0; q < G::kJC / 4; ++q) {
                    acc = acc + v[q].x;
                    acc = acc + v[q].y;
                    acc = acc + v[q].z;
                    acc = acc + v[q].w;
                }
            } else {  // the last chunk: eight keys per round of reads
                int jj = 0;
                for (; jj + 8 <= cnt; jj += 8) {
                    const float4 v0 = *reinterpret_cast<const float4 *>(row + jj);
                    const float4 v1 = *reinterpret_cast<const float4 *>(row + jj + 4);
                    acc = acc + v0.x;
                    acc = acc + v0.y;
                    acc = acc + v0.z;
                    acc = acc + v0.w;
                    acc = acc + v1.x;
                    acc = acc + v1.y;
                    acc = acc + v1.z;
                    acc = acc + v1.w;
                }
                for (; jj < cnt; ++jj) acc = acc + row[jj];
            }
        }
        __syncthreads();
    }
    if (tid < VD) outp[tid] = acc;
}

// Max over the NW wavefronts of a workgroup.
template <int NW>
__device__ __forceinline__ float block_max_nw(float v, float *red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = go_max(v, __shfl_xor(v, off));
    if constexpr (NW == 1) {
        return __shfl(v, 0);
    } else {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        if (lane == 0) red[wave] = v;
        __syncthreads();
        float r = red[0];
#pragma unroll
        for (int w = 1; w < NW; ++w) r = go_max(r, red[w]);
        __syncthreads();
        return r;
    }
}

// A workgroup barrier, kept for a single wavefront too: it is also what
// orders one lane's LDS writes before another lane's reads for the compiler.
template <int NW>
__device__ __forceinline__ void block_sync() {
    __syncthreads();
}

constexpr int kChainVd = 64;  // value codes per head of the chain kernel: one per lane of wavefront 0
constexpr int kProdKeys = 48;    // keys per step of the resident chain's product pipeline
constexpr int kProdStride = 52;  // floats per output row of a product buffer (48 keys, padded)
constexpr int kProdFloats = kChainVd * kProdStride;  // one product buffer, [output][key]

// AttendInt8Spans for one (stream, query row, head) per workgroup of NW
// wavefronts, value heads of 64 codes, key heads of at most 64 codes,
// 16-byte aligned rows. Same arithmetic as attend_kernel. Lane d of
// wavefront 0 carries output d's in-order chain (axpysI8). Value rows stream
// from HBM straight into LDS (global_load_lds, 16-byte pieces, rows
// [key][64 codes]). With RES (NW = 4) every row of the stream is loaded,
// issued by all wavefronts as the workgroup starts, ahead of the keys (the
// keys' loads retire behind them, so the logits start once the whole stream
// has landed: 0.35 us less per 1500-key call than issuing the rows after the
// logits, whose tail then waited for them), and the
// three other wavefronts form the products fl(w_j * code_jd) a step of 48
// keys ahead of the adds, so the chain costs one add per key. Otherwise
// wavefront 0 forms each product itself (a sign-extending convert of the
// key's code, the rounded multiply by the key's weight, the add) over a ring of
// rs chunks of JC keys that wavefront 0 refills behind the chain. The
// logits and the softmax are spread over the NW wavefronts.
template <int NW, int JC, bool RES>
__global__ __launch_bounds__(64 * NW) void attend_chain_kernel(AttendArgs a, int rs, int swz) {
    constexpr int NT = 64 * NW;
    constexpr int KPT = 6;                  // keys per thread per round of logits
    constexpr int LPC = JC / 16;            // wavefront DMA loads per chunk (16 keys of 64 codes each)
    extern __shared__ __align__(16) unsigned char smem[];
    const int per = a.heads * a.t;
    const int w = blockIdx.x;
    int b, r;
    if (swz) {
        const int full = (a.batch & ~7) * per;
        if (w < full) {
            b = (w & 7) + 8 * (w / (8 * per));
            r = (w >> 3) % per;
        } else {
            const int w2 = w - full, rem = a.batch & 7;
            b = (a.batch & ~7) + w2 % rem;
            r = w2 / rem;
        }
    } else {
        b = w / per;
        r = w - b * per;
    }
    const int h = r % a.heads, i = r / a.heads;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kv_heads = a.k_cols / a.qk;
    const int kv = h / (a.heads / kv_heads);
    const int32_t *sp = a.spans + (static_cast<long long>(b) * a.t + i) * 4;
    const int lo0 = sp[0], len0 = sp[1] - sp[0], lo1 = sp[2], len1 = sp[3] - sp[2];
    const int n = len0 + len1;
    const long long kb = attend_cache_of(a, b);  // the cache this stream reads
    if (kb < 0 || lo0 < 0 || len0 < 0 || sp[1] > a.nk_max || lo1 < 0 || len1 < 0 || sp[3] > a.nk_max)
        return;  // spans off the cache, or no cache
    float *outp = a.out + b * a.out_stride + (static_cast<long long>(i) * a.heads + h) * kChainVd;
    if (n == 0) {
        if (tid < kChainVd) outp[tid] = 0.0f;
        return;
    }
    attend_stage_pages(a, b, smem);  // paged: the stream's page table into LDS
    const int32_t *pgs = reinterpret_cast<const int32_t *>(smem + a.page_lds);

    const int nk_pad = (a.nk_max + 3) & ~3;
    float *s = reinterpret_cast<float *>(smem);   // logits, exponentials, then weights
    float *tt = s + nk_pad;                       // exponentials transposed to [lane][index]
    const int r8max = ((a.nk_max >> 3) + 3) & ~3;
    int8_t *ring = reinterpret_cast<int8_t *>(tt + 8 * r8max);
    __shared__ float red[8];
    __shared__ __align__(16) int8_t q8[kStreamQk];
    __shared__ __align__(16) float qf[kStreamQk];
    __shared__ float sq_sh, sum_sh;

    const float *qi = a.q + b * a.q_stride + (static_cast<long long>(i) * a.heads + h) * a.qk;
    const int8_t *kq = a.kq + kb * a.kv_stride;
    const float *ks = a.ks + kb * a.s_stride;
    const int8_t *vq = a.vq + kb * a.kv_stride;
    const float *vs = a.vs + kb * a.s_stride;
    auto key_of = [&](int j) { return j < len0 ? lo0 + j : lo1 + (j - len0); };
    const int nch = (n + JC - 1) / JC;

    // Wavefront-wide DMA load u (16 keys) of chunk c into ring slot c % rs.
    auto dma = [&](int c, int u) {
        const int j0 = c * JC, cnt = min(JC, n - j0);
        int8_t *slot = ring + (c % rs) * (JC * kChainVd);
        const int p = u * 64 + lane;
        const int jj = p >> 2, seg = p & 3;
        const int key = key_of(j0 + (jj < cnt ? jj : 0));
        dma16(vq + attend_row(a, pgs, key) * a.v_cols + kv * kChainVd + seg * 16, lds_offset(slot + u * 64 * 16));
    };

    if constexpr (RES) {
        for (int u = wave; u < nch * LPC; u += NW) dma(u / LPC, u % LPC);
    }

    // 1. The query, then each thread's first KPT keys, in flight together.
    const int kpieces = a.qk / 16;
    const int qp = a.rope_cos ? a.qpos[static_cast<long long>(b) * a.t + i] : 0;
    const float qv = tid < a.qk ? query_value(a, qi, qp, tid) : 0.0f;
    int4 kw[KPT][kStreamQk / 16];
    float skr[KPT], svr[KPT];  // key scales; value scales (kept when one round covers every key)
    auto kload = [&](int g, int j) {
        const int key = key_of(j);
        const int8_t *krow = kq + attend_row(a, pgs, key) * a.k_cols + kv * a.qk;
#pragma unroll
        for (int p = 0; p < kStreamQk / 16; ++p)
            if (p < kpieces) kw[g][p] = *reinterpret_cast<const int4 *>(krow + 16 * p);
        skr[g] = ks[attend_row(a, pgs, key) * kv_heads + kv];
        svr[g] = vs[attend_row(a, pgs, key) * kv_heads + kv];
    };
    auto logit = [&](int g) -> float {
        if (a.quant_q) {
            int dot = 0;  // exact in any order
#pragma unroll
            for (int p = 0; p < kStreamQk / 16; ++p)
                if (p < kpieces) {
                    const int4 qw = *reinterpret_cast<const int4 *>(q8 + 16 * p);
                    dot = __builtin_amdgcn_sdot4(kw[g][p].x, qw.x, dot, false);
                    dot = __builtin_amdgcn_sdot4(kw[g][p].y, qw.y, dot, false);
                    dot = __builtin_amdgcn_sdot4(kw[g][p].z, qw.z, dot, false);
                    dot = __builtin_amdgcn_sdot4(kw[g][p].w, qw.w, dot, false);
                }
            const float scl = sq_sh * skr[g];
            const float t1 = static_cast<float>(dot) * scl;
            return t1 / a.scale;
        }
        float dot = 0.0f;  // in order
#pragma unroll
        for (int p = 0; p < kStreamQk / 16; ++p)
            if (p < kpieces) {
                const int cw[4] = {kw[g][p].x, kw[g][p].y, kw[g][p].z, kw[g][p].w};
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const float pr = qf[16 * p + e] * static_cast<float>(static_cast<int8_t>(cw[e >> 2] >> (8 * (e & 3))));
                    dot = dot + pr;
                }
            }
        const float t1 = dot * skr[g];
        return t1 / a.scale;
    };
#pragma unroll
    for (int g = 0; g < KPT; ++g)
        if (tid + g * NT < n) kload(g, tid + g * NT);

    // QuantizeRow of the query head (int8.go:226-228); qk <= 64 <= NT.
    if (tid < a.qk) qf[tid] = qv;
    if (a.quant_q) {
        const float m = block_max_nw<NW>(tid < a.qk ? fabsf(qv) : 0.0f, red);
        const float sc = m > 0.0f ? m / 127.0f : 1.0f;
        if (tid < a.qk) {
            q8[tid] = static_cast<int8_t>(go_int8_code(rintf(qv / sc)));
        }
        if (tid == 0) sq_sh = sc;
    }
    __syncthreads();

    // Logits (int8Logits / dotsF32I8), KPT keys per thread per round.
    for (int j0 = 0; j0 < n; j0 += KPT * NT) {
        if (j0 > 0) {
#pragma unroll
            for (int g = 0; g < KPT; ++g)
                if (j0 + tid + g * NT < n) kload(g, j0 + tid + g * NT);
        }
#pragma unroll
        for (int g = 0; g < KPT; ++g) {
            const int j = j0 + tid + g * NT;
            if (j < n) s[j] = logit(g);
        }
    }

    // The ring's first value chunks start streaming now (the compiler's own
    // loads drained first: loads retire in order).
    if constexpr (!RES) {
        wait_vm_const<0>();
        const int c0 = min(rs, nch);
        for (int c = 0; c < c0; ++c)
            for (int u = 0; u < LPC; ++u) dma(c, u);
    }
    __syncthreads();

    // 2. softmaxInPlace with amd64's expSubSum; the eight lane sums read a
    // copy transposed to [lane][index].
    float m0 = -INFINITY;
    for (int j = tid; j < n; j += NT) m0 = go_max(m0, s[j]);
    const float m = block_max_nw<NW>(m0, red);
    const int n8 = n & ~7;
    const bool kernel_path = n8 > 0;
    const int r8 = ((n8 >> 3) + 3) & ~3;
    for (int j = tid; j < n8; j += NT) {
        const float e = exp_lane(s[j] - m);
        s[j] = e;
        tt[(j & 7) * r8 + (j >> 3)] = e;
    }
    for (int j = n8 + tid; j < n; j += NT) s[j] = exp_generic(s[j] - m);
    block_sync<NW>();
    if (tid < 8 && kernel_path) {  // lane tid of the 8-lane sum, elements in order
        float acc = 0.0f;
        const float *row = tt + tid * r8;
        const int cnt = n8 >> 3;
        int k = 0;
        for (; k + 16 <= cnt; k += 16) {
            const float4 v0 = *reinterpret_cast<const float4 *>(row + k);
            const float4 v1 = *reinterpret_cast<const float4 *>(row + k + 4);
            const float4 v2 = *reinterpret_cast<const float4 *>(row + k + 8);
            const float4 v3 = *reinterpret_cast<const float4 *>(row + k + 12);
            acc = acc + v0.x; acc = acc + v0.y; acc = acc + v0.z; acc = acc + v0.w;
            acc = acc + v1.x; acc = acc + v1.y; acc = acc + v1.z; acc = acc + v1.w;
            acc = acc + v2.x; acc = acc + v2.y; acc = acc + v2.z; acc = acc + v2.w;
            acc = acc + v3.x; acc = acc + v3.y; acc = acc + v3.z; acc = acc + v3.w;
        }
        for (; k < cnt; ++k) acc = acc + row[k];
        red[tid] = acc;
    }
    block_sync<NW>();
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
    block_sync<NW>();
    const float sum = sum_sh;
    if (n <= KPT * NT) {  // the value scales came with the keys
#pragma unroll
        for (int g = 0; g < KPT; ++g) {
            const int j = tid + g * NT;
            if (j < n) {
                const float p = s[j] / sum;
                s[j] = p * svr[g];
            }
        }
    } else {
        for (int j = tid; j < n; j += NT) {
            const float p = s[j] / sum;
            s[j] = p * vs[attend_row(a, pgs, key_of(j)) * kv_heads + kv];
        }
    }
    if constexpr (RES) {
        static_assert(NW == 4, "the resident chain runs one adding and three multiplying wavefronts");
        wait_vm_const<0>();  // this wavefront's value rows have landed
        __syncthreads();     // weights and every value row in LDS
        // 3. axpysI8 (int8kernel.go:360-368), pipelined over steps of 48
        // keys: wavefronts 1-3 form the step's products fl(w_j * code_jd)
        // into a product buffer [output d][key], while lane d of wavefront 0
        // adds the previous step's row d in key order, so the in-order
        // chain costs one add per key. Two buffers alternate; a barrier
        // ends each step. Key j's codes sit at ring + 64 j.
        float *prod = reinterpret_cast<float *>(ring + rs * (JC * kChainVd));
        const int steps = (n + kProdKeys - 1) / kProdKeys;
        // A multiplying lane's task: codes 4m..4m+3 of keys 4jq..4jq+3 of
        // the step (16 lanes of one write cover 16 distinct bank quads).
        const int m = (lane & 3) + 4 * (lane >> 4), jq = 4 * (wave - 1) + ((lane >> 2) & 3);
        auto produce = [&](int t) {
            const int j = t * kProdKeys + 4 * jq;
            if (j >= n) return;
            const uint32_t *row = reinterpret_cast<const uint32_t *>(ring + static_cast<long long>(j) * kChainVd) + m;
            const uint32_t c0 = row[0], c1 = row[16], c2 = row[32], c3 = row[48];
            const float4 wv = *reinterpret_cast<const float4 *>(s + j);
            float *dst = prod + (t & 1) * kProdFloats + 4 * m * kProdStride + 4 * jq;
            auto code = [](uint32_t cw, int k) { return static_cast<float>(static_cast<int8_t>(cw >> (8 * k))); };
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float4 pv;
                pv.x = wv.x * code(c0, e);
                pv.y = wv.y * code(c1, e);
                pv.z = wv.z * code(c2, e);
                pv.w = wv.w * code(c3, e);
                *reinterpret_cast<float4 *>(dst + e * kProdStride) = pv;
            }
        };
        if (wave != 0) produce(0);
        __syncthreads();
        float acc = 0.0f;
        // Step t: wavefront 0 reads step t's row into ld, then adds step
        // t-1's (all 48 keys: only the last step is partial) from ad under
        // the reads' latency; two register sets alternate.
        auto step = [&](int t, float4 (&ld)[kProdKeys / 4], const float4 (&ad)[kProdKeys / 4]) {
            if (wave == 0) {
                const float4 *src = reinterpret_cast<const float4 *>(prod + (t & 1) * kProdFloats + lane * kProdStride);
#pragma unroll
                for (int q = 0; q < kProdKeys / 4; ++q) ld[q] = src[q];
                if (t > 0) {
#pragma unroll
                    for (int q = 0; q < kProdKeys / 4; ++q) {
                        acc = acc + ad[q].x;
                        acc = acc + ad[q].y;
                        acc = acc + ad[q].z;
                        acc = acc + ad[q].w;
                    }
                }
            } else if (t + 1 < steps) {
                produce(t + 1);
            }
            __syncthreads();
        };
        float4 ra[kProdKeys / 4], rb[kProdKeys / 4];
        for (int t = 0; t < steps; t += 2) {
            step(t, ra, rb);
            if (t + 1 < steps) step(t + 1, rb, ra);
        }
        if (wave != 0) return;
        const int cnt = n - (steps - 1) * kProdKeys;  // keys of the last step, 1..48
        auto tail = [&](const float4 (&ad)[kProdKeys / 4]) {
#pragma unroll
            for (int q = 0; q < kProdKeys / 4; ++q) {
                if (4 * q < cnt) acc = acc + ad[q].x;
                if (4 * q + 1 < cnt) acc = acc + ad[q].y;
                if (4 * q + 2 < cnt) acc = acc + ad[q].z;
                if (4 * q + 3 < cnt) acc = acc + ad[q].w;
            }
        };
        if ((steps - 1) & 1)
            tail(rb);
        else
            tail(ra);
        outp[lane] = acc;
        return;
    }
    __syncthreads();  // weights in LDS
    if (wave != 0) return;

    // 3. axpysI8 (int8kernel.go:360-368): lane d adds fl(w_j * code_jd) in
    // key order, forming each product itself.
    float acc = 0.0f;
    for (int c = 0; c < nch; ++c) {
        wait_vm(LPC * (min(c + rs, nch) - 1 - c));  // chunk c has landed
        const int j0 = c * JC, cnt = min(JC, n - j0);
        const int8_t *slot = ring + (c % rs) * (JC * kChainVd) + lane;
        const float *wj = s + j0;
        int jj = 0;
        // Blocks of 32 keys: every code and weight read issued, then the
        // products and the adds in key order.
        for (; jj + 32 <= cnt; jj += 32) {
            float cd[32];
            float4 wv[8];
#pragma unroll
            for (int k = 0; k < 32; ++k) cd[k] = static_cast<float>(slot[(jj + k) * kChainVd]);
#pragma unroll
            for (int q = 0; q < 8; ++q) wv[q] = *reinterpret_cast<const float4 *>(wj + jj + 4 * q);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float p0 = wv[q].x * cd[4 * q], p1 = wv[q].y * cd[4 * q + 1];
                const float p2 = wv[q].z * cd[4 * q + 2], p3 = wv[q].w * cd[4 * q + 3];
                acc = acc + p0;
                acc = acc + p1;
                acc = acc + p2;
                acc = acc + p3;
            }
        }
        for (; jj + 8 <= cnt; jj += 8) {
            const float4 w0 = *reinterpret_cast<const float4 *>(wj + jj);
            const float4 w1 = *reinterpret_cast<const float4 *>(wj + jj + 4);
            float cd[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) cd[k] = static_cast<float>(slot[(jj + k) * kChainVd]);
            const float p0 = w0.x * cd[0], p1 = w0.y * cd[1], p2 = w0.z * cd[2], p3 = w0.w * cd[3];
            const float p4 = w1.x * cd[4], p5 = w1.y * cd[5], p6 = w1.z * cd[6], p7 = w1.w * cd[7];
            acc = acc + p0;
            acc = acc + p1;
            acc = acc + p2;
            acc = acc + p3;
            acc = acc + p4;
            acc = acc + p5;
            acc = acc + p6;
            acc = acc + p7;
        }
        for (; jj < cnt; ++jj) {
            const float pr = wj[jj] * static_cast<float>(slot[jj * kChainVd]);
            acc = acc + pr;
        }
        if (c + rs < nch) {
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this chunk's slot reads are done
            for (int u = 0; u < LPC; ++u) dma(c + rs, u);
        }
    }
    if (lane < kChainVd) outp[lane] = acc;
}

// One 4-byte global load per active lane straight into LDS: lane l's word
// lands at lds + 4 * l (global_load_lds_dword, M0 = lds); lanes off in EXEC
// neither load nor write. (Plain: the scales of 32 keys share one line,
// which non-temporal loads fetched again.)
__device__ __forceinline__ void dma4(const void *src, unsigned lds) {
    asm volatile("global_load_lds_dword %0, off" ::"v"(src), "{m0}"(lds) : "memory");
}

constexpr int kRingJc = 32;                     // keys per ring chunk
constexpr int kRingSlot = kRingJc * 64 + kRingJc * 4;  // 64 codes per key, then the keys' scales

// AttendInt8Spans for one (stream, query row, head) per single-wavefront
// workgroup, key and value heads of 64 codes, 16-byte aligned rows: the
// many-stream form. Key chunks, then value chunks, of 32 keys stream through
// one LDS ring of RS slots (global_load_lds, refilled behind the reads); a
// slot holds the chunk's rows [key][64 codes] and the 32 keys' scales, so no
// load of the kernel waits on its own: every wavefront keeps RS chunks of
// HBM reads in flight.
//   1. the query; the logits chunk by chunk, two lanes per key (exact int32
//      dots, or the float32 query in order);
//   2. the softmax (amd64's expSubSum) with the eight lane sums read at
//      stride 8;
//   3. per value chunk the keys' weights p_j * vscale_j, then lane d's
//      in-order chain of fl(w_j * code_jd).
// Same arithmetic as attend_kernel.
template <int RS>
__global__ __launch_bounds__(64) void attend_ring_kernel(AttendArgs a, int swz) {
    constexpr int JC = kRingJc, ROW = 64;
    constexpr int LPC = JC * ROW / 1024 + 1;  // wavefront DMA loads per chunk: 2 of rows, 1 of scales
    extern __shared__ __align__(16) unsigned char smem[];
    const int per = a.heads * a.t;
    const int w = blockIdx.x;
    int b, r;
    if (swz) {
        const int full = (a.batch & ~7) * per;
        if (w < full) {
            b = (w & 7) + 8 * (w / (8 * per));
            r = (w >> 3) % per;
        } else {
            const int w2 = w - full, rem = a.batch & 7;
            b = (a.batch & ~7) + w2 % rem;
            r = w2 / rem;
        }
    } else {
        b = w / per;
        r = w - b * per;
    }
    const int h = r % a.heads, i = r / a.heads;
    const int lane = threadIdx.x;
    const int kv_heads = a.k_cols / a.qk;
    const int kv = h / (a.heads / kv_heads);
    const int32_t *sp = a.spans + (static_cast<long long>(b) * a.t + i) * 4;
    const int lo0 = sp[0], len0 = sp[1] - sp[0], lo1 = sp[2], len1 = sp[3] - sp[2];
    const int n = len0 + len1;
    const long long kb = attend_cache_of(a, b);  // the cache this stream reads
    if (kb < 0 || lo0 < 0 || len0 < 0 || sp[1] > a.nk_max || lo1 < 0 || len1 < 0 || sp[3] > a.nk_max)
        return;  // spans off the cache, or no cache
    float *outp = a.out + b * a.out_stride + (static_cast<long long>(i) * a.heads + h) * ROW;
    if (n == 0) {
        outp[lane] = 0.0f;
        return;
    }
    attend_stage_pages(a, b, smem);  // paged: the stream's page table into LDS
    const int32_t *pgs = reinterpret_cast<const int32_t *>(smem + a.page_lds);
    const int nk_pad = (a.nk_max + 3) & ~3;
    float *s = reinterpret_cast<float *>(smem);  // logits, exponentials, then weights
    int8_t *ring = reinterpret_cast<int8_t *>(s + nk_pad);
    __shared__ float qf[ROW];
    __shared__ float red[8];

    const float *qi = a.q + b * a.q_stride + (static_cast<long long>(i) * a.heads + h) * ROW;
    const int8_t *kq = a.kq + kb * a.kv_stride;
    const float *ks = a.ks + kb * a.s_stride;
    const int8_t *vq = a.vq + kb * a.kv_stride;
    const float *vs = a.vs + kb * a.s_stride;
    auto key_of = [&](int j) { return j < len0 ? lo0 + j : lo1 + (j - len0); };
    const int nch = (n + JC - 1) / JC, total = 2 * nch;  // key chunks, then value chunks

    // Ring chunk g (g < nch: key chunk g, else value chunk g - nch) into
    // slot g % RS: rows as 16-byte pieces, then the scales (lanes < 32).
    auto dma = [&](int g) {
        const bool keys = g < nch;
        const int c = keys ? g : g - nch;
        const int j0 = c * JC, cnt = min(JC, n - j0);
        int8_t *slot = ring + (g % RS) * kRingSlot;
        const int8_t *base = keys ? kq + kv * ROW : vq + kv * ROW;
        const long long cols = keys ? a.k_cols : a.v_cols;
#pragma unroll
        for (int u = 0; u < LPC - 1; ++u) {
            const int p = u * 64 + lane;
            const int jj = p >> 2, seg = p & 3;
            const int key = key_of(j0 + (jj < cnt ? jj : 0));
            dma16(base + attend_row(a, pgs, key) * cols + seg * 16, lds_offset(slot + u * 64 * 16));
        }
        const float *sc = keys ? ks : vs;
        const int key = key_of(j0 + (lane < cnt ? lane : 0));
        if (lane < JC) dma4(sc + attend_row(a, pgs, key) * kv_heads + kv, lds_offset(slot + JC * ROW));
    };
    // Chunk g has landed: at most the chunks issued after it are in flight.
    auto wait_chunk = [&](int g) {
        if (g + RS - 1 < total) wait_vm_const<LPC * (RS - 1)>();
        else wait_vm(LPC * (total - 1 - g));
    };
    auto refill = [&](int g) {  // after chunk g's reads: chunk g + RS into its slot
        if (g + RS < total) {
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the slot's reads are done
            dma(g + RS);
        }
    };

    // 1. The query (the compiler's loads drained before the ring starts:
    // loads retire in order).
    const int qp = a.rope_cos ? a.qpos[static_cast<long long>(b) * a.t + i] : 0;
    const float qv = query_value(a, qi, qp, lane);
    wait_vm_const<0>();
    for (int g = 0; g < min(RS, total); ++g) dma(g);
    qf[lane] = qv;
    float sq = 0.0f;
    int4 q4[2];  // this lane's half of the int8 query (32 codes)
    const int half = lane >> 5;
    if (a.quant_q) {
        float m = fabsf(qv);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = go_max(m, __shfl_xor(m, off));
        const float sc = m > 0.0f ? m / 127.0f : 1.0f;
        const int code = go_int8_code(rintf(qv / sc)) & 255;
        // gather this lane's 32 query codes (lanes 32*half ..) into 8 words
        int words[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int c0 = __shfl(code, 32 * half + 4 * k), c1 = __shfl(code, 32 * half + 4 * k + 1);
            const int c2 = __shfl(code, 32 * half + 4 * k + 2), c3 = __shfl(code, 32 * half + 4 * k + 3);
            words[k] = c0 | (c1 << 8) | (c2 << 16) | (c3 << 24);
        }
        q4[0] = make_int4(words[0], words[1], words[2], words[3]);
        q4[1] = make_int4(words[4], words[5], words[6], words[7]);
        sq = sc;
    }
    __syncthreads();

    // Logits: lane (key jj = lane % 32, half) dots its 32 codes; the halves
    // add up exactly (int32), the float query sums in order on half 0.
    for (int g = 0; g < nch; ++g) {
        wait_chunk(g);
        const int j0 = g * JC, cnt = min(JC, n - j0);
        const int jj = lane & 31;
        const int8_t *slot = ring + (g % RS) * kRingSlot;
        const int8_t *row = slot + jj * ROW;
        const float kscale = reinterpret_cast<const float *>(slot + JC * ROW)[jj];
        float lg = 0.0f;
        if (a.quant_q) {
            const int4 k0 = *reinterpret_cast<const int4 *>(row + 32 * half);
            const int4 k1 = *reinterpret_cast<const int4 *>(row + 32 * half + 16);
            int dot = 0;
            dot = __builtin_amdgcn_sdot4(k0.x, q4[0].x, dot, false);
            dot = __builtin_amdgcn_sdot4(k0.y, q4[0].y, dot, false);
            dot = __builtin_amdgcn_sdot4(k0.z, q4[0].z, dot, false);
            dot = __builtin_amdgcn_sdot4(k0.w, q4[0].w, dot, false);
            dot = __builtin_amdgcn_sdot4(k1.x, q4[1].x, dot, false);
            dot = __builtin_amdgcn_sdot4(k1.y, q4[1].y, dot, false);
            dot = __builtin_amdgcn_sdot4(k1.z, q4[1].z, dot, false);
            dot = __builtin_amdgcn_sdot4(k1.w, q4[1].w, dot, false);
            dot += __shfl_xor(dot, 32);
            if (half == 0 && jj < cnt) {
                const float scl = sq * kscale;
                const float t1 = static_cast<float>(dot) * scl;
                lg = t1 / a.scale;
            }
        } else if (half == 0 && jj < cnt) {
            float dot = 0.0f;  // in order
            for (int c = 0; c < ROW; c += 4) {
                const int wd = *reinterpret_cast<const int *>(row + c);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float pr = qf[c + e] * static_cast<float>(static_cast<int8_t>(wd >> (8 * e)));
                    dot = dot + pr;
                }
            }
            const float t1 = dot * kscale;
            lg = t1 / a.scale;
        }
        if (half == 0 && jj < cnt) s[j0 + jj] = lg;
        refill(g);
    }
    __syncthreads();

    // 2. softmaxInPlace with amd64's expSubSum.
    float m = -INFINITY;
    for (int j = lane; j < n; j += 64) m = go_max(m, s[j]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = go_max(m, __shfl_xor(m, off));
    const int n8 = n & ~7;
    const bool kernel_path = n8 > 0;
    for (int j = lane; j < n8; j += 64) s[j] = exp_lane(s[j] - m);
    for (int j = n8 + lane; j < n; j += 64) s[j] = exp_generic(s[j] - m);
    __syncthreads();
    if (lane < 8 && kernel_path) {  // lane k of the 8-lane sum, elements in order
        float acc = 0.0f;
        int j = lane;
        for (; j + 56 < n8; j += 64) {
            float e[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) e[k] = s[j + 8 * k];
#pragma unroll
            for (int k = 0; k < 8; ++k) acc = acc + e[k];
        }
        for (; j < n8; j += 8) acc = acc + s[j];
        red[lane] = acc;
    }
    __syncthreads();
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
    __syncthreads();

    // 3. axpysI8 (int8kernel.go:360-368): the chunk's weights, then lane d's
    // products in key order.
    float acc = 0.0f;
    for (int g = nch; g < total; ++g) {
        wait_chunk(g);
        const int j0 = (g - nch) * JC, cnt = min(JC, n - j0);
        const int8_t *sl = ring + (g % RS) * kRingSlot;
        if (lane < cnt) {
            const float p = s[j0 + lane] / sum;
            s[j0 + lane] = p * reinterpret_cast<const float *>(sl + JC * ROW)[lane];
        }
        __syncthreads();
        const int8_t *slot = sl + lane;
        const float *wj = s + j0;
        if (cnt == JC) {
            // Every code and weight read of the chunk goes out before the
            // first product: left to itself the compiler reused 8 registers
            // for the codes and waited on each 8 reads in turn (batch-256
            // cross call 89.5 -> 86.8 us, bit for bit the same).
            int ci[JC];
            float4 wv[JC / 4];
#pragma unroll
            for (int k = 0; k < JC; ++k) ci[k] = slot[k * ROW];
#pragma unroll
            for (int q = 0; q < JC / 4; ++q) wv[q] = *reinterpret_cast<const float4 *>(wj + 4 * q);
            __builtin_amdgcn_sched_barrier(0);
            float cd[JC];
#pragma unroll
            for (int k = 0; k < JC; ++k) cd[k] = static_cast<float>(ci[k]);
#pragma unroll
            for (int q = 0; q < JC / 4; ++q) {
                const float p0 = wv[q].x * cd[4 * q], p1 = wv[q].y * cd[4 * q + 1];
                const float p2 = wv[q].z * cd[4 * q + 2], p3 = wv[q].w * cd[4 * q + 3];
                acc = acc + p0;
                acc = acc + p1;
                acc = acc + p2;
                acc = acc + p3;
            }
        } else {
            for (int jj = 0; jj < cnt; ++jj) {
                const float pr = wj[jj] * static_cast<float>(slot[jj * ROW]);
                acc = acc + pr;
            }
        }
        refill(g);
    }
    outp[lane] = acc;
}

}  // namespace

hipError_t launch_gather_rows(void *dst, const void *src, const int32_t *idx, const int32_t *len, int streams,
                              int cap, int row_bytes, hipStream_t stream) {
    if (streams <= 0 || cap <= 0 || row_bytes <= 0) return hipSuccess;
    const long long stream_bytes = static_cast<long long>(cap) * row_bytes;
    const int vec = (row_bytes % 16 == 0 && reinterpret_cast<uintptr_t>(dst) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(src) % 16 == 0) ? 1 : 0;
    const long long pieces = vec ? stream_bytes / 16 : stream_bytes;
    const unsigned gx = static_cast<unsigned>(std::min<long long>(64, (pieces + 255) / 256));
    hipLaunchKernelGGL(gather_rows_kernel, dim3(gx, static_cast<unsigned>(streams)), dim3(256), 0, stream,
                       static_cast<unsigned char *>(dst), static_cast<const unsigned char *>(src), idx, len, streams,
                       stream_bytes, row_bytes, vec);
    return hipGetLastError();
}

hipError_t launch_fake_quant(float *dst, const float *x, long long chunks, int width, hipStream_t stream) {
    if (chunks <= 0) return hipSuccess;
    const long long blocks = (chunks + 3) / 4;
    for (long long c0 = 0; c0 < blocks; c0 += 1 << 30) {
        const long long nb = blocks - c0 < (1LL << 30) ? blocks - c0 : (1LL << 30);
        const long long ch0 = c0 * 4;
        hipLaunchKernelGGL(fake_quant_kernel, dim3(static_cast<unsigned>(nb)), dim3(256), 0, stream, dst + ch0 * width,
                           x + ch0 * width, chunks - ch0, width);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

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

template <int VD, int JC>
hipError_t launch_attend_stream(const AttendArgs &a, int rs, size_t lds, hipStream_t stream) {
    static std::atomic<unsigned long long> attr{0};
    if (hipError_t e = lds_limit_once(reinterpret_cast<const void *>(&attend_stream_kernel<VD, JC>), 152 * 1024, attr)) return e;
    const long long wgs = static_cast<long long>(a.heads) * a.t * a.batch;
    hipLaunchKernelGGL((attend_stream_kernel<VD, JC>), dim3(static_cast<unsigned>(wgs)), dim3(kAttThreads), lds,
                       stream, a, rs, a.batch >= 8 ? 1 : 0);
    return hipGetLastError();
}

// Ring slots and LDS bytes of the streamed kernel: every value row of a
// stream when the launch is small and they fit, else a ring within ~50 KiB
// (three workgroups per CU).
template <int VD, int JC>
bool stream_plan(const AttendArgs &a, bool resident, int &rs, size_t &lds) {
    using G = StreamGeo<VD, JC>;
    const size_t nk_pad = (static_cast<size_t>(a.nk_max) + 3) & ~size_t(3);
    const size_t fixed = 8 * nk_pad + 2 * sizeof(float) * VD * G::kPitch;
    const size_t slot = static_cast<size_t>(JC) * VD;
    const int nch_max = (a.nk_max + JC - 1) / JC;
    if (resident) {
        rs = std::max(nch_max, 2);
        lds = fixed + slot * rs;
        return lds <= 150 * 1024;
    }
    const long long room = 50 * 1024 - static_cast<long long>(fixed);
    rs = static_cast<int>(std::min(8LL, std::max(2LL, room / static_cast<long long>(slot))));
    lds = fixed + slot * rs;
    return lds <= 150 * 1024;
}

template <int NW, int JC, bool RES>
hipError_t launch_attend_chain(const AttendArgs &a, int rs, size_t lds, hipStream_t stream) {
    static std::atomic<unsigned long long> attr{0};
    if (hipError_t e = lds_limit_once(reinterpret_cast<const void *>(&attend_chain_kernel<NW, JC, RES>), 152 * 1024, attr)) return e;
    const long long wgs = static_cast<long long>(a.heads) * a.t * a.batch;
    hipLaunchKernelGGL((attend_chain_kernel<NW, JC, RES>), dim3(static_cast<unsigned>(wgs)), dim3(64 * NW), lds,
                       stream, a, rs, a.batch >= 8 ? 1 : 0);
    return hipGetLastError();
}

template <int RS>
hipError_t launch_attend_ring(const AttendArgs &a, size_t lds, hipStream_t stream) {
    static std::atomic<unsigned long long> attr{0};
    if (hipError_t e = lds_limit_once(reinterpret_cast<const void *>(&attend_ring_kernel<RS>), 152 * 1024, attr)) return e;
    const long long wgs = static_cast<long long>(a.heads) * a.t * a.batch;
    hipLaunchKernelGGL((attend_ring_kernel<RS>), dim3(static_cast<unsigned>(wgs)), dim3(64), lds, stream, a,
                       a.batch >= 8 ? 1 : 0);
    return hipGetLastError();
}

// LDS of the chain kernel: logits, their transposed copy, and rs chunks of
// JC value rows.
size_t chain_lds(const AttendArgs &a, int jc, int rs) {
    const size_t nk_pad = (static_cast<size_t>(a.nk_max) + 3) & ~size_t(3);
    const size_t r8 = ((static_cast<size_t>(a.nk_max) >> 3) + 3) & ~size_t(3);
    return 4 * nk_pad + 4 * 8 * r8 + static_cast<size_t>(rs) * jc * kChainVd;
}

// The resident form also holds the two product buffers behind the rows.
size_t chain_res_lds(const AttendArgs &a, int rs) { return chain_lds(a, 64, rs) + 2 * sizeof(float) * kProdFloats; }

hipError_t launch_attend_int8(const AttendArgs &args, hipStream_t stream) {
    AttendArgs a = args;
    if (a.t <= 0 || a.heads <= 0 || a.batch <= 0) return hipSuccess;
    // A paged launch keeps the stream's page table behind the kernel's own
    // dynamic LDS (with_pages gives the total and sets its offset).
    const size_t pb = a.pages ? ((static_cast<size_t>((a.nk_max + (1 << a.page_shift) - 1) >> a.page_shift) * 4 + 15) &
                                 ~size_t(15))
                              : 0;
    auto with_pages = [&](size_t lds) {
        a.page_lds = static_cast<int>((lds + 15) & ~size_t(15));
        return static_cast<size_t>(a.page_lds) + pb;
    };
    const bool aligned = (a.kv_stride & 15) == 0 && (reinterpret_cast<uintptr_t>(a.kq) & 15) == 0 &&
                         (reinterpret_cast<uintptr_t>(a.vq) & 15) == 0;
    const bool stream_ok = aligned && (a.qk & 15) == 0 && a.qk <= kStreamQk && (a.k_cols & 15) == 0 &&
                           (a.v_cols & 15) == 0;
    if (stream_ok && a.vd == kChainVd) {
        if (a.resident) {
            const int rs = std::max(1, (a.nk_max + 63) / 64);
            const size_t lds = with_pages(chain_res_lds(a, rs));
            if (lds <= 150 * 1024) return launch_attend_chain<4, 64, true>(a, rs, lds, stream);
        }
        if (a.qk == kChainVd) {
            // many streams: key and value chunks through a ring of 6 slots
            // (eight workgroups per CU at 1500 keys)
            constexpr int rs = 6;
            const size_t lds = with_pages(4 * ((static_cast<size_t>(a.nk_max) + 3) & ~size_t(3)) +
                                          static_cast<size_t>(rs) * kRingSlot);
            if (lds <= 150 * 1024) return launch_attend_ring<rs>(a, lds, stream);
        }
        const int rs = 4;
        const size_t lds = with_pages(chain_lds(a, 32, rs));
        if (lds <= 150 * 1024) return launch_attend_chain<1, 32, false>(a, rs, lds, stream);
    }
    // (64-code value heads the chain kernel does not fit need more LDS than
    // the streamed kernel has: they take the general kernel)
    int rs = 0;
    size_t slds = 0;
    if (stream_ok && a.vd == 128) {
        if (a.resident && stream_plan<128, 64>(a, true, rs, slds) && with_pages(slds) <= 150 * 1024)
            return launch_attend_stream<128, 64>(a, rs, with_pages(slds), stream);
        if (stream_plan<128, 32>(a, false, rs, slds) && with_pages(slds) <= 150 * 1024)
            return launch_attend_stream<128, 32>(a, rs, with_pages(slds), stream);
    }
    const bool one_chunk = a.vchunk >= a.nk_max;
    const size_t vbytes = (one_chunk ? 1 : 2) * static_cast<size_t>(a.vchunk) * a.vd;
    const size_t lds = with_pages(sizeof(float) * static_cast<size_t>((a.nk_max + 3) & ~3) + vbytes);
    // dynamic LDS beside the kernel's static arrays: 96 KiB of values + up to 8192 logits
    static std::atomic<unsigned long long> attr{0};
    if (hipError_t e = lds_limit_once(reinterpret_cast<const void *>(&attend_kernel), 132 * 1024, attr)) return e;
    hipLaunchKernelGGL(attend_kernel, dim3(a.heads, a.t, a.batch), dim3(kAttThreads), lds, stream, a);
    return hipGetLastError();
}

}  // namespace cqhip
