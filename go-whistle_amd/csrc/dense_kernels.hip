// gfx950 dense fp32 MFMA form of a CQ product, for Dense views: the
// reference's Exact semantics (internal/cq/kernel.go:160-374) as a dense
// contraction on dequantized fp32 tiles, for many activations at once.
//
// Exact's product of row r and activation t is
//   y[t][r] = sum_g norm[r][g] * sum_{k in g} codebook[idx(r, k)] * xh[t][k]
// with xh the activation rotated per group (rotate, kernel.go:203-217:
// zero-padded to groups * G, the plain FWHT in stage order h = 1, 2, ...,
// G/2, times 1/sqrt(G) rounded once). Written densely it is Y = Xh * W^T
// with W[r][k] = norm[r][k / G] * codebook[idx(r, k)], which this form
// computes in two launches (three where K is split):
//   1. dense_rotate_kernel writes Xh [activation][kpad] fp32 into a
//      workspace, bit for bit rotate's values (the FWHT in registers, a
//      wavefront per group); columns past groups * G (up to a multiple of
//      64) and activation rows past the last are zero;
//   2. dense_mfma_kernel: a workgroup of 4 wavefronts owns 128 activations
//      x 128 weight rows (two 64-row blocks of the device layout) and a run
//      of K in chunks of 64 coordinates. Per chunk every thread holds one
//      row's 32 index codes (16 bytes at 4 bits, 8 at 2), looks their levels
//      up a byte at a time in a 256-entry LDS table (a byte's 2 or 4
//      codebook levels), scales them by the row's FP16 norm into the LDS
//      weight tile, and stores 8 float4 of the Xh tile; wavefront w runs
//      v_mfma_f32_32x32x2_f32 over its 64 activations x 64 rows (2 x 2
//      output blocks, 64 accumulators a lane). The next chunk's global loads
//      are in flight while the current chunk's MFMAs run; two workgroups
//      share a CU (72 KB of LDS each), so one's barriers and table stores
//      overlap the other's MFMAs;
//   3. where 128 x 128 tiles leave CUs idle, K is split over workgroups:
//      each writes its run's partial sums, and dense_fold_kernel adds them
//      in run order (so results do not depend on scheduling).
// The sums run in the MFMA's order, not the nibble kernels' (and each W
// element is one rounded product of norm and level), so outputs match Exact
// within float32 rounding of the dot products, not bit for bit.
//
// MFMA roles: A = Xh (rows = activations), B = W (columns = weight rows), so
// a lane's result column is one weight row and 32 lanes store 128
// contiguous bytes of y. In a 32x32x2 step lane l gives A[l % 32][l / 32]
// and B[l / 32][l % 32]; the K pair of MFMA s in a step of 8 coordinates is
// (kk + s, kk + 4 + s), so each lane reads one float4 of its row per step.
#include "cq_internal.hpp"
#include "cq_device.hpp"

#include <hip/hip_fp16.h>

#include <algorithm>

namespace cqhip {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kDM = 128;        // weight rows per workgroup (two 64-row blocks)
constexpr int kDN = 128;        // activations per workgroup
constexpr int kDK = 64;         // coordinates per chunk
constexpr int kDP = kDK + 4;    // LDS row pitch in floats: 8 lanes' float4 reads hit distinct banks
constexpr int kDenseThreads = 256;
constexpr size_t kDenseTileFloats = static_cast<size_t>(kDN + kDM) * kDP;
// the tiles and the byte table (256 entries of 4 levels at 2 bits, 2 at 4)
constexpr size_t kDenseLds = (kDenseTileFloats + 256 * 4) * sizeof(float);

// rotate (kernel.go:203-217) in registers: a wavefront per (activation,
// group) for G >= 64, lane l holding indices e * 64 + l; for G = 32 a
// wavefront per (activation, two groups), lane l index l % 32 of group
// l / 32. Stage h pairs index i (bit h clear) with i + h into u + v and
// u - v: across lanes (lane ^ h) for h < 64, within a lane (value e ^ h/64)
// above. Rows past the activations and columns past groups * G are zero.
template <int G>
__global__ __launch_bounds__(kDenseThreads) void dense_rotate_kernel(DenseRotArgs a) {
    constexpr int E = G >= 64 ? G / 64 : 1, GPW = G >= 64 ? 1 : 64 / G;
    const int lane = threadIdx.x & 63;
    const int gsets = (a.groups + GPW - 1) / GPW;
    const long long wv = static_cast<long long>(blockIdx.x) * (kDenseThreads / 64) + (threadIdx.x >> 6);
    if (wv >= static_cast<long long>(a.rows_pad) * gsets) return;  // the whole wavefront
    const int act = static_cast<int>(wv / gsets), gs = static_cast<int>(wv % gsets);
    const int g = gs * GPW + (G >= 64 ? 0 : lane / G), i0 = G >= 64 ? lane : lane % G;
    const bool live = act < a.rows && g < a.groups;
    const float *x = a.x + static_cast<long long>(live ? act : 0) * a.x_stride;
    float v[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int col = g * G + e * 64 + i0;
        v[e] = live && col < a.in ? x[col] : 0.0f;
    }
#pragma unroll
    for (int h = 1; h < G; h <<= 1) {
        if (h < 64) {
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const float o = xor_lane(v[e], h);
                v[e] = (i0 & h) ? o - v[e] : v[e] + o;
            }
        } else {
            const int he = h / 64;
#pragma unroll
            for (int e = 0; e < E; ++e)
                if (!(e & he)) {
                    const float u = v[e], w = v[e + he];
                    v[e] = u + w;
                    v[e + he] = u - w;
                }
        }
    }
    float *o = a.xh + static_cast<long long>(act) * a.kpad;
    if (g < a.groups)
#pragma unroll
        for (int e = 0; e < E; ++e) o[g * G + e * 64 + i0] = v[e] * a.inv_sqrt;
    if (gs == gsets - 1 && lane < a.kpad - a.groups * G) o[a.groups * G + lane] = 0.0f;
}

// One thread's global loads of a chunk: its row's index codes and norm, and
// its 8 float4 of the activation tile.
template <int BITS>
struct DenseStage {
    static constexpr int LB = 32 * BITS / 8;  // index bytes
    uint32_t iw[LB / 4];
    float nv;
    f32x4 xv[8];

    __device__ __forceinline__ void load(const DenseArgs &a, const float *xt, long long blk, bool wlive, int hf,
                                         int lane, int tid, int c) {
        const int k0 = c * kDK + hf * 32;
        if (wlive && k0 < a.kin) {
            const int bo = k0 * BITS / 8, u = bo / a.U, ub = bo % a.U;
            const uint8_t *p = a.idx + ((blk * a.units + u) * 64 + lane) * a.U + ub;
            if constexpr (BITS == 4) {
                const u32x4 v = *reinterpret_cast<const u32x4 *>(p);
                iw[0] = v.x, iw[1] = v.y, iw[2] = v.z, iw[3] = v.w;
            } else {
                const u32x2 v = *reinterpret_cast<const u32x2 *>(p);
                iw[0] = v.x, iw[1] = v.y;
            }
            nv = __half2float(__ushort_as_half(a.norm[(blk * a.groups + k0 / a.G) * 64 + lane]));
        } else {
#pragma unroll
            for (int i = 0; i < LB / 4; ++i) iw[i] = 0;
            nv = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int f = tid + kDenseThreads * i, r = f >> 4, c4 = f & 15;
            xv[i] = *reinterpret_cast<const f32x4 *>(xt + static_cast<long long>(r) * a.kpad + c * kDK + c4 * 4);
        }
    }

    // Into the LDS tiles: the activations as loaded, the weights as
    // norm * level, byte b's codes LSB first (cact/packed.go:24-27).
    __device__ __forceinline__ void store(float *sa, float *sw, const float *ptab, int wrow, int hf, int tid) const {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int f = tid + kDenseThreads * i, r = f >> 4, c4 = f & 15;
            *reinterpret_cast<f32x4 *>(sa + r * kDP + c4 * 4) = xv[i];
        }
        float *dst = sw + wrow * kDP + hf * 32;
        if constexpr (BITS == 4) {
            f32x2 e[16];
#pragma unroll
            for (int b = 0; b < 16; ++b)
                e[b] = reinterpret_cast<const f32x2 *>(ptab)[(iw[b >> 2] >> (8 * (b & 3))) & 255u];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const f32x4 v = {nv * e[2 * j].x, nv * e[2 * j].y, nv * e[2 * j + 1].x, nv * e[2 * j + 1].y};
                *reinterpret_cast<f32x4 *>(dst + 4 * j) = v;
            }
        } else {
            f32x4 e[8];
#pragma unroll
            for (int b = 0; b < 8; ++b)
                e[b] = reinterpret_cast<const f32x4 *>(ptab)[(iw[b >> 2] >> (8 * (b & 3))) & 255u];
#pragma unroll
            for (int j = 0; j < 8; ++j) *reinterpret_cast<f32x4 *>(dst + 4 * j) = nv * e[j];
        }
    }
};

template <int BITS>
__global__ __launch_bounds__(kDenseThreads, 2) void dense_mfma_kernel(DenseArgs a) {
    extern __shared__ __align__(16) float sm[];
    float *sa = sm, *sw = sm + kDN * kDP, *ptab = sm + kDenseTileFloats;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l32 = lane & 31, hl = lane >> 5;

    // Workgroup L runs on XCD L % 8 as its (L / 8)-th there. The items
    // (activation tile, row tile, K run), K runs innermost, are cut into 8
    // runs of equal size but for one item, one per XCD: the workgroups that
    // read one activation tile run on one XCD, close in time, and share its
    // L2.
    const int total = a.tiles_m * a.tiles_n * a.ksplit, q = total >> 3, rem = total & 7;
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    const int item = (xcd < rem ? xcd * (q + 1) : rem * (q + 1) + (xcd - rem) * q) + slot;
    const int kz = item % a.ksplit, tmn = item / a.ksplit;
    const int tn = tmn / a.tiles_m, tm = tmn % a.tiles_m;
    const int nch = a.kpad / kDK, c0 = kz * a.kchunks, c1 = min(nch, c0 + a.kchunks);

    {  // the byte table: a byte's codes' levels, LSB first
        const int b = tid;
        if constexpr (BITS == 4) {
            const f32x2 v = {a.cb[b & 15], a.cb[b >> 4]};
            reinterpret_cast<f32x2 *>(ptab)[b] = v;
        } else {
            const f32x4 v = {a.cb[b & 3], a.cb[(b >> 2) & 3], a.cb[(b >> 4) & 3], a.cb[b >> 6]};
            reinterpret_cast<f32x4 *>(ptab)[b] = v;
        }
    }

    // This thread's loads: weight row wrow of the tile (block wb, lane lane)
    // at coordinates hf * 32 .. hf * 32 + 31 of each chunk, and Xh vectors
    // tid + 256 * i of the 128 x 64 activation chunk.
    const int wb = w & 1, hf = w >> 1, wrow = wb * 64 + lane;
    const bool wlive = tm * 2 + wb < a.nblk;  // a block of the view (the last tile may have one)
    const long long blk = static_cast<long long>(a.blk0) + tm * 2 + wb;
    const float *xt = a.xh + static_cast<long long>(tn) * kDN * a.kpad;

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    DenseStage<BITS> st;
    st.load(a, xt, blk, wlive, hf, lane, tid, c0);
    // Wavefront w's MFMA operands: activations ar.., weight rows wr.. (block wb).
    const float *pa = sa + ((w >> 1) * 64 + l32) * kDP + 4 * hl;
    const float *pw = sw + (wb * 64 + l32) * kDP + 4 * hl;
    for (int c = c0; c < c1; ++c) {
        __syncthreads();  // the previous chunk's MFMAs have read the tiles (and the table is written)
        st.store(sa, sw, ptab, wrow, hf, tid);
        __syncthreads();
        if (c + 1 < c1) st.load(a, xt, blk, wlive, hf, lane, tid, c + 1);
        f32x4 av[2], bv[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) av[i] = *reinterpret_cast<const f32x4 *>(pa + i * 32 * kDP);
#pragma unroll
        for (int j = 0; j < 2; ++j) bv[j] = *reinterpret_cast<const f32x4 *>(pw + j * 32 * kDP);
#pragma unroll
        for (int kk = 0; kk < kDK; kk += 8) {
            f32x4 an[2], bn[2];
            if (kk + 8 < kDK) {
#pragma unroll
                for (int i = 0; i < 2; ++i) an[i] = *reinterpret_cast<const f32x4 *>(pa + i * 32 * kDP + kk + 8);
#pragma unroll
                for (int j = 0; j < 2; ++j) bn[j] = *reinterpret_cast<const f32x4 *>(pw + j * 32 * kDP + kk + 8);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].x, bv[j].x, acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].y, bv[j].y, acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].z, bv[j].z, acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].w, bv[j].w, acc[i][j], 0, 0, 0);
            if (kk + 8 < kDK) {
#pragma unroll
                for (int i = 0; i < 2; ++i) av[i] = an[i], bv[i] = bn[i];
            }
        }
    }

    // Result v of block (i, j) in lane l: activation 8 (v / 4) + 4 (l / 32) +
    // v % 4 of the block, weight row l % 32; the wavefront's weight rows are
    // block wb's, the rows it dequantized. One K run writes y; several write
    // their partial sums [run][activation][view row] for the fold.
    float *out = a.y;
    long long stride = a.y_stride;
    if (a.ksplit > 1) {
        out = a.part + static_cast<long long>(kz) * a.rows * a.out;
        stride = a.out;
    }
    const int ar = (w >> 1) * 64;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const long long vr = blk * 64 + j * 32 + l32 - a.row0;  // view row
        if (!wlive || vr < 0 || vr >= a.out) continue;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int t = tn * kDN + ar + i * 32 + (v >> 2) * 8 + hl * 4 + (v & 3);
                if (t < a.rows) out[static_cast<long long>(t) * stride + vr] = acc[i][j][v];
            }
    }
}

// y = the K runs' partial sums added in run order from the first.
__global__ __launch_bounds__(kDenseThreads) void dense_fold_kernel(DenseArgs a) {
    const long long n = static_cast<long long>(a.rows) * a.out;
    for (long long e = static_cast<long long>(blockIdx.x) * kDenseThreads + threadIdx.x; e < n;
         e += static_cast<long long>(gridDim.x) * kDenseThreads) {
        float s = a.part[e];
        for (int k = 1; k < a.ksplit; ++k) s = s + a.part[k * n + e];
        a.y[(e / a.out) * a.y_stride + e % a.out] = s;
    }
}

}  // namespace

bool dense_geometry_supported(int bits, int group) {
    return (bits == 4 || bits == 2) && group >= 32 && (group & (group - 1)) == 0 && group <= 1024;
}

int dense_tile_rows() { return kDM; }
int dense_tile_activations() { return kDN; }

hipError_t launch_dense_rotate(const DenseRotArgs &r, hipStream_t s) {
    const int gpw = r.G >= 64 ? 1 : 64 / r.G;
    const long long waves = static_cast<long long>(r.rows_pad) * ((r.groups + gpw - 1) / gpw);
    const dim3 grid(static_cast<unsigned>((waves + kDenseThreads / 64 - 1) / (kDenseThreads / 64)));
    switch (r.G) {
        case 32: hipLaunchKernelGGL(dense_rotate_kernel<32>, grid, dim3(kDenseThreads), 0, s, r); break;
        case 64: hipLaunchKernelGGL(dense_rotate_kernel<64>, grid, dim3(kDenseThreads), 0, s, r); break;
        case 128: hipLaunchKernelGGL(dense_rotate_kernel<128>, grid, dim3(kDenseThreads), 0, s, r); break;
        case 256: hipLaunchKernelGGL(dense_rotate_kernel<256>, grid, dim3(kDenseThreads), 0, s, r); break;
        case 512: hipLaunchKernelGGL(dense_rotate_kernel<512>, grid, dim3(kDenseThreads), 0, s, r); break;
        case 1024: hipLaunchKernelGGL(dense_rotate_kernel<1024>, grid, dim3(kDenseThreads), 0, s, r); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_dense(const DenseArgs &a, int bits, hipStream_t s) {
    const void *fn = bits == 4 ? reinterpret_cast<const void *>(&dense_mfma_kernel<4>)
                               : reinterpret_cast<const void *>(&dense_mfma_kernel<2>);
    static std::atomic<unsigned long long> attr[2] = {{0}, {0}};
    hipError_t e = lds_limit_once(fn, static_cast<int>(kDenseLds), attr[bits == 4]);
    if (e != hipSuccess) return e;
    const dim3 grid(a.tiles_m * a.tiles_n * a.ksplit);
    if (bits == 4)
        hipLaunchKernelGGL(dense_mfma_kernel<4>, grid, dim3(kDenseThreads), kDenseLds, s, a);
    else
        hipLaunchKernelGGL(dense_mfma_kernel<2>, grid, dim3(kDenseThreads), kDenseLds, s, a);
    e = hipGetLastError();
    if (e != hipSuccess || a.ksplit == 1) return e;
    const long long n = static_cast<long long>(a.rows) * a.out;
    const int blocks = static_cast<int>(std::min<long long>((n + kDenseThreads - 1) / kDenseThreads, 4096));
    hipLaunchKernelGGL(dense_fold_kernel, dim3(blocks), dim3(kDenseThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace cqhip
