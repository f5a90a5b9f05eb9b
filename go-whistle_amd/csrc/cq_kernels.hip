// gfx950 kernels for go-whistle's CQ products (internal/cq).
//
// product_kernel runs both of the reference's numerics on one skeleton:
//   kModeLut   the lut kernel (internal/cq/lut.go:12-29, 158-313): per
//              activation group the plain FWHT, the bound M, integer tables
//              v = RNE(entry * 8191/M) and per row and group the exact int32
//              sum of the looked-up v, times norm * (M * lutStep), added to y
//              in group order. Bit for bit lutLookupGeneric's result: the
//              integer sums are exact in any order, every float op is the
//              reference's, unfused (-ffp-contract=off), in its order.
//   kModeExact the nibble kernels of Exact views (internal/cq/kernel.go:
//              200-374): x̂ = FWHT(x)/√G, float tables, and per row and
//              group the float sums in nibble4's order (a per low nibble,
//              b per high nibble, bytes in order) or, for the leftover
//              activations of a GEMM, lookupNibble's eight partial sums and
//              tree; bit for bit the reference's.
//
// Work split. A workgroup (4 wavefronts) owns a tile of up to 4 blocks of
// 64 rows for one activation; each lane owns one row. Per chunk of groups
// that fits LDS it rotates the activation, builds that chunk's tables in
// LDS, and each wavefront takes (block, group) items: it streams the
// block's index units of that group with coalesced 16-byte loads (a
// wavefront reads 1 KiB contiguous per load) and looks every nibble up in
// the LDS tables. All 64 lanes read the same 16-entry table at a time, so
// the lookups are free of bank conflicts. The per-group partial results
// meet in LDS and the lane that owns the row folds them into y in group
// order.
#include "cq_internal.hpp"
#include "cq_device.hpp"

#include <hip/hip_fp16.h>

namespace cqhip {
namespace {

template <int BITS, int GB>
struct Geo {
    static constexpr int G = GB * 8 / BITS;   // weights per group
    static constexpr int U = GB < 16 ? GB : 16;  // index bytes per lane load
    static constexpr int UPG = GB / U;        // loads per group
    static constexpr int NT = 2 * GB;         // 16-entry tables per group (one per nibble)
};

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int U>
__device__ __forceinline__ void load_unit(const uint8_t *p, uint32_t w[4]) {
    if constexpr (U == 16) {
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (U == 8) {
        const uint2 v = *reinterpret_cast<const uint2 *>(p);
        w[0] = v.x; w[1] = v.y; w[2] = 0; w[3] = 0;
    } else if constexpr (U == 4) {
        w[0] = *reinterpret_cast<const uint32_t *>(p); w[1] = 0; w[2] = 0; w[3] = 0;
    } else if constexpr (U == 2) {
        w[0] = *reinterpret_cast<const uint16_t *>(p); w[1] = 0; w[2] = 0; w[3] = 0;
    } else {
        w[0] = *p; w[1] = 0; w[2] = 0; w[3] = 0;
    }
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}

__device__ __forceinline__ int rne_int(float e) { return static_cast<int>(rintf(e)); }

template <typename TabT, int BITS, int GB>
__device__ __forceinline__ size_t tab_bytes_per_group() {
    return sizeof(TabT) * 16 * Geo<BITS, GB>::NT;
}

template <int BITS, int GB, int MODE>
__global__ __launch_bounds__(kThreads) void product_kernel(ProdArgs a) {
    using Gm = Geo<BITS, GB>;
    constexpr int G = Gm::G, U = Gm::U, UPG = Gm::UPG, NT = Gm::NT;
    using TabT = typename std::conditional<MODE == kModeLut, short, float>::type;

    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int act = blockIdx.y;
    const int tile = blockIdx.x;

    // The matrix this tile belongs to (uniform: scalar selects).
    const uint8_t *idx = a.mats[0].idx;
    const uint16_t *nrm = a.mats[0].norm;
    float *y = a.mats[0].y;
    long long ys = a.mats[0].y_stride;
    int row0 = a.mats[0].row0, out = a.mats[0].out, blk0 = a.mats[0].blk0, tile0 = 0;
#pragma unroll
    for (int k = 1; k < kMaxMatrices; ++k) {
        if (k < a.nmats && tile >= a.mats[k].tile0) {
            idx = a.mats[k].idx; nrm = a.mats[k].norm; y = a.mats[k].y; ys = a.mats[k].y_stride;
            row0 = a.mats[k].row0; out = a.mats[k].out; blk0 = a.mats[k].blk0; tile0 = a.mats[k].tile0;
        }
    }

    const int tb = a.tb, gc = a.gc, groups = a.groups;
    const int blkA = blk0 + (tile - tile0) * tb;
    const int blkEnd = (row0 + out + kBlockRows - 1) / kBlockRows;
    const int tbh = min(tb, blkEnd - blkA);
    const int units = a.row_bytes / U;
    const float *x = a.x + static_cast<long long>(act) * a.x_stride;
    const bool nib4 = MODE == kModeExact && act < a.nib4_rows;
    const int tr = tb * kBlockRows;  // partial-result row stride

    TabT *tab = reinterpret_cast<TabT *>(smem);
    const size_t tab_bytes = static_cast<size_t>(gc) * NT * 16 * sizeof(TabT);
    float *xh = reinterpret_cast<float *>(smem + tab_bytes);
    const int xh_floats = max(gc * G, gc * tr);
    float *st_inv = xh + xh_floats;
    float *st_step = st_inv + gc;
    int *pi = reinterpret_cast<int *>(xh);
    float *pf = xh;

    float acc = 0.0f;

    for (int g0 = 0; g0 < groups; g0 += gc) {
        const int gch = min(gc, groups - g0);

        // Activation chunk, zero-padded past In (lut.go:163-165; kernel.go:204-205).
        for (int e = tid; e < gch * G; e += kThreads) {
            const int col = g0 * G + e;
            xh[e] = col < a.in ? x[col] : 0.0f;
        }
        __syncthreads();

        // Plain FWHT per group, stages h = 1, 2, ..., G/2 (kernel.go:384-393).
        for (int lh = 0; (1 << lh) < G; ++lh) {
            const int h = 1 << lh;
            for (int b = tid; b < gch * (G / 2); b += kThreads) {
                const int gi = b / (G / 2), bb = b % (G / 2);
                const int i = ((bb >> lh) << (lh + 1)) | (bb & (h - 1));
                float *xg = xh + gi * G;
                const float u = xg[i], v = xg[i + h];
                xg[i] = u + v;
                xg[i + h] = u - v;
            }
            __syncthreads();
        }

        if constexpr (MODE == kModeLut) {
            // Group bound M and steps (lut.go:239-282, 171-177, 213-225).
            for (int gi = wave; gi < gch; gi += kThreads / 64) {
                const float *xg = xh + gi * G;
                float mx = 0.0f;
                if constexpr (BITS == 4) {
                    for (int k = lane; k < G; k += 64) mx = go_max(mx, fabsf(xg[k]));
                } else {
                    for (int k = lane; k < G / 2; k += 64) {
                        const float s2 = fabsf(xg[2 * k]) + fabsf(xg[2 * k + 1]);
                        mx = go_max(mx, s2);
                    }
                }
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) mx = go_max(mx, __shfl_xor(mx, off));
                if (lane == 0) {
                    const float m = a.cb_max * mx;
                    st_inv[gi] = m > 0.0f ? static_cast<float>(kLutQ) / m : 0.0f;
                    st_step[gi] = m * a.lut_step;
                }
            }
        } else {
            // rotate's 1/√G (kernel.go:207-216).
            for (int e = tid; e < gch * G; e += kThreads) xh[e] = xh[e] * a.inv_sqrt;
        }
        __syncthreads();

        // Tables.
        if constexpr (MODE == kModeLut) {
            if constexpr (BITS == 4) {  // lutTables4Generic (lut.go:263-282)
                for (int p = tid; p < gch * G; p += kThreads) {
                    const float av = xh[p] * st_inv[p / G];
                    uint32_t w[8];
#pragma unroll
                    for (int c = 0; c < 16; c += 2) {
                        const int v0 = rne_int(a.cb[c] * av), v1 = rne_int(a.cb[c + 1] * av);
                        w[c / 2] = (static_cast<uint32_t>(v0) & 0xffffu) | (static_cast<uint32_t>(v1) << 16);
                    }
                    uint4 *dst = reinterpret_cast<uint4 *>(tab + static_cast<size_t>(p) * 16);
                    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
                    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
                }
            } else {  // lutTables2Generic (lut.go:239-258)
                for (int p = tid; p < gch * (G / 2); p += kThreads) {
                    const float inv = st_inv[p / (G / 2)];
                    const float av = xh[2 * p] * inv, bv = xh[2 * p + 1] * inv;
                    uint32_t w[8];
#pragma unroll
                    for (int c = 0; c < 16; c += 2) {
                        const float l0 = a.cb[c & 3] * av, h0 = a.cb[c >> 2] * bv;
                        const float l1 = a.cb[(c + 1) & 3] * av, h1 = a.cb[(c + 1) >> 2] * bv;
                        const int v0 = rne_int(l0 + h0), v1 = rne_int(l1 + h1);
                        w[c / 2] = (static_cast<uint32_t>(v0) & 0xffffu) | (static_cast<uint32_t>(v1) << 16);
                    }
                    uint4 *dst = reinterpret_cast<uint4 *>(tab + static_cast<size_t>(p) * 16);
                    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
                    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
                }
            }
        } else {
            if constexpr (BITS == 4) {  // nibbleTables, 4 bits (kernel.go:243-250)
                for (int p = tid; p < gch * G; p += kThreads) {
                    const float v = xh[p];
                    float w[16];
#pragma unroll
                    for (int c = 0; c < 16; ++c) w[c] = a.cb[c] * v;
                    float4 *dst = reinterpret_cast<float4 *>(tab + static_cast<size_t>(p) * 16);
#pragma unroll
                    for (int q = 0; q < 4; ++q) dst[q] = make_float4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]);
                }
            } else {  // nibbleTables, 2 bits (kernel.go:254-264)
                for (int p = tid; p < gch * (G / 2); p += kThreads) {
                    const float av = xh[2 * p], bv = xh[2 * p + 1];
                    float w[16];
#pragma unroll
                    for (int hi = 0; hi < 4; ++hi) {
                        const float hb = a.cb[hi] * bv;
#pragma unroll
                        for (int lo = 0; lo < 4; ++lo) {
                            const float la = a.cb[lo] * av;
                            w[hi << 2 | lo] = la + hb;
                        }
                    }
                    float4 *dst = reinterpret_cast<float4 *>(tab + static_cast<size_t>(p) * 16);
#pragma unroll
                    for (int q = 0; q < 4; ++q) dst[q] = make_float4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]);
                }
            }
        }
        __syncthreads();

        // Lookups: one (block, group) item per wavefront at a time.
        const int items = tbh * gch;
        for (int it = wave; it < items; it += kThreads / 64) {
            const int bi = it / gch, gi = it % gch;
            const int blk = blkA + bi, g = g0 + gi;
            const uint8_t *up = idx + (static_cast<size_t>(blk) * units + static_cast<size_t>(g) * UPG) * 64 * U +
                                static_cast<size_t>(lane) * U;
            const TabT *tg = tab + static_cast<size_t>(gi) * NT * 16;
            if constexpr (MODE == kModeLut) {
                int s = 0;
#pragma unroll 2
                for (int u = 0; u < UPG; ++u) {
                    uint32_t w[4];
                    load_unit<U>(up + static_cast<size_t>(u) * 64 * U, w);
                    const short *tu = tg + static_cast<size_t>(u) * 2 * U * 16;
#pragma unroll
                    for (int k = 0; k < U; ++k) {
                        const uint32_t byte = (w[k >> 2] >> ((k & 3) * 8)) & 0xffu;
                        s += static_cast<int>(tu[(2 * k) * 16 + (byte & 15u)]) +
                             static_cast<int>(tu[(2 * k + 1) * 16 + (byte >> 4)]);
                    }
                }
                pi[gi * tr + bi * 64 + lane] = s;
            } else {
                const float n = half_bits_to_float(nrm[(static_cast<size_t>(blk) * groups + g) * 64 + lane]);
                if (nib4) {  // lookupNibble4 (kernel.go:330-374)
                    float fa = 0.0f, fb = 0.0f;
#pragma unroll 2
                    for (int u = 0; u < UPG; ++u) {
                        uint32_t w[4];
                        load_unit<U>(up + static_cast<size_t>(u) * 64 * U, w);
                        const float *tu = tg + static_cast<size_t>(u) * 2 * U * 16;
#pragma unroll
                        for (int k = 0; k < U; ++k) {
                            const uint32_t byte = (w[k >> 2] >> ((k & 3) * 8)) & 0xffu;
                            fa = fa + tu[(2 * k) * 16 + (byte & 15u)];
                            fb = fb + tu[(2 * k + 1) * 16 + (byte >> 4)];
                        }
                    }
                    const float ab = fa + fb;
                    pf[gi * tr + bi * 64 + lane] = ab * n;
                } else {  // lookupNibble (kernel.go:271-309)
                    float pa[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
                    if constexpr (GB >= 8) {
#pragma unroll 2
                        for (int u = 0; u < UPG; ++u) {
                            uint32_t w[4];
                            load_unit<U>(up + static_cast<size_t>(u) * 64 * U, w);
                            const float *tu = tg + static_cast<size_t>(u) * 2 * U * 16;
#pragma unroll
                            for (int wd = 0; wd < U / 8; ++wd) {
                                const uint32_t wl = w[2 * wd], wh = w[2 * wd + 1];
                                const float *tw = tu + static_cast<size_t>(wd) * 16 * 16;  // tables 2j.. for the word's bytes
#pragma unroll
                                for (int k = 0; k < 8; ++k) {
                                    const float pair = tw[k * 16 + ((wl >> (4 * k)) & 15u)] +
                                                       tw[(k + 8) * 16 + ((wh >> (4 * k)) & 15u)];
                                    pa[k] = pa[k] + pair;
                                }
                            }
                        }
                    } else {
                        uint32_t w[4];
                        load_unit<U>(up, w);
#pragma unroll
                        for (int k = 0; k < U; ++k) {
                            const uint32_t byte = (w[k >> 2] >> ((k & 3) * 8)) & 0xffu;
                            const float pair = tg[(2 * k) * 16 + (byte & 15u)] + tg[(2 * k + 1) * 16 + (byte >> 4)];
                            pa[0] = pa[0] + pair;
                        }
                    }
                    const float t01 = pa[0] + pa[1], t23 = pa[2] + pa[3], t45 = pa[4] + pa[5], t67 = pa[6] + pa[7];
                    const float t03 = t01 + t23, t47 = t45 + t67;
                    const float tt = t03 + t47;
                    pf[gi * tr + bi * 64 + lane] = tt * n;
                }
            }
        }
        __syncthreads();

        // Fold this chunk's groups into the row's y, in group order
        // (lut.go:297-310; kernel.go:304, 366-369).
        if (tid < tbh * kBlockRows) {
            const int blk = blkA + (tid >> 6);
            for (int gi = 0; gi < gch; ++gi) {
                if constexpr (MODE == kModeLut) {
                    const float n = half_bits_to_float(nrm[(static_cast<size_t>(blk) * groups + g0 + gi) * 64 + (tid & 63)]);
                    const float coef = n * st_step[gi];
                    const float prod = static_cast<float>(pi[gi * tr + tid]) * coef;
                    acc = acc + prod;
                } else {
                    acc = acc + pf[gi * tr + tid];
                }
            }
        }
        __syncthreads();
    }

    if (tid < tbh * kBlockRows) {
        const int r = blkA * kBlockRows + tid;
        if (r >= row0 && r < row0 + out) y[static_cast<long long>(act) * ys + (r - row0)] = acc;
    }
}

template <int BITS, int GB, int MODE>
hipError_t launch_one(const ProdArgs &a, size_t lds, hipStream_t stream) {
    static std::atomic<unsigned long long> attr{0};
    if (hipError_t e = lds_limit_once(reinterpret_cast<const void *>(&product_kernel<BITS, GB, MODE>), 160 * 1024, attr))
        return e;
    for (int r0 = 0; r0 < a.rows; r0 += 65535) {
        ProdArgs b = a;
        b.rows = min(65535, a.rows - r0);
        b.x = a.x + static_cast<long long>(r0) * a.x_stride;
        b.nib4_rows = a.nib4_rows - r0;
        for (int k = 0; k < a.nmats; ++k) b.mats[k].y = a.mats[k].y + static_cast<long long>(r0) * a.mats[k].y_stride;
        dim3 grid(a.tiles, b.rows);
        hipLaunchKernelGGL((product_kernel<BITS, GB, MODE>), grid, dim3(kThreads), lds, stream, b);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

template <int MODE>
hipError_t dispatch(const ProdArgs &a, int bits, int gb, size_t lds, hipStream_t s) {
    if (bits == 4) {
        switch (gb) {
            case 4: return launch_one<4, 4, MODE>(a, lds, s);
            case 8: return launch_one<4, 8, MODE>(a, lds, s);
            case 16: return launch_one<4, 16, MODE>(a, lds, s);
            case 32: return launch_one<4, 32, MODE>(a, lds, s);
            case 64: return launch_one<4, 64, MODE>(a, lds, s);
            case 128: return launch_one<4, 128, MODE>(a, lds, s);
            case 256: return launch_one<4, 256, MODE>(a, lds, s);
            case 512: if (MODE == kModeExact) return launch_one<4, 512, MODE>(a, lds, s); break;
        }
    } else if (bits == 2) {
        switch (gb) {
            case 2: return launch_one<2, 2, MODE>(a, lds, s);
            case 4: return launch_one<2, 4, MODE>(a, lds, s);
            case 8: return launch_one<2, 8, MODE>(a, lds, s);
            case 16: return launch_one<2, 16, MODE>(a, lds, s);
            case 32: return launch_one<2, 32, MODE>(a, lds, s);
            case 64: return launch_one<2, 64, MODE>(a, lds, s);
            case 128: return launch_one<2, 128, MODE>(a, lds, s);
            case 256: return launch_one<2, 256, MODE>(a, lds, s);
            case 512: if (MODE == kModeExact) return launch_one<2, 512, MODE>(a, lds, s); break;
        }
    }
    return hipErrorInvalidValue;
}

// Row (internal/cq/matrix.go:161-181): one workgroup per (row, group).
__global__ __launch_bounds__(kThreads) void rows_kernel(RowArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    float *buf = reinterpret_cast<float *>(smem);
    const int g = blockIdx.x, i = blockIdx.y;
    const int r = a.rows ? a.rows[i] : a.r0 + i;
    float *dst = a.dst + static_cast<size_t>(i) * a.in;
    if (r < 0 || r >= a.nrows) {  // a listed row outside the matrix: zeros, no read
        for (int k = threadIdx.x; k < a.group; k += blockDim.x) {
            const int col = g * a.group + k;
            if (col < a.in) dst[col] = 0.0f;
        }
        return;
    }
    const int blk = r / kBlockRows, lane = r % kBlockRows;
    const float s = half_bits_to_float(a.norm[(static_cast<size_t>(blk) * a.groups + g) * 64 + lane]) * a.inv_sqrt;
    const int G = a.group, mask = (1 << a.width) - 1;
    for (int k = threadIdx.x; k < G; k += blockDim.x) {
        const int bit = (g * G + k) * a.width;
        const int j = bit >> 3;  // row byte
        const int u = j / a.unit_bytes, ku = j % a.unit_bytes;
        const uint8_t byte =
            a.idx[((static_cast<size_t>(blk) * a.units + u) * 64 + lane) * a.unit_bytes + ku];
        const int c = (byte >> (bit & 7)) & mask;
        buf[k] = a.cb[c] * s;
    }
    __syncthreads();
    for (int h = 1; h < G; h <<= 1) {
        for (int b = threadIdx.x; b < G / 2; b += blockDim.x) {
            const int ii = (b / h) * 2 * h + (b % h);
            const float u = buf[ii], v = buf[ii + h];
            buf[ii] = u + v;
            buf[ii + h] = u - v;
        }
        __syncthreads();
    }
    for (int k = threadIdx.x; k < G; k += blockDim.x) {
        const int col = g * G + k;
        if (col < a.in) dst[col] = buf[k] * a.scale;  // x1 is exact; the embedding's scale (decoder.go:269-275)
    }
}

}  // namespace

size_t product_lds_bytes(int bits, int group_bytes, int mode, int gc, int tb) {
    const int G = group_bytes * 8 / bits;
    const size_t tab = static_cast<size_t>(gc) * 2 * group_bytes * 16 * (mode == kModeLut ? 2 : 4);
    const size_t xh = static_cast<size_t>(max(gc * G, gc * tb * kBlockRows)) * 4;
    return tab + xh + static_cast<size_t>(gc) * 8;
}

hipError_t launch_product(const ProdArgs &a, int bits, int group_bytes, int mode, size_t lds, hipStream_t stream) {
    if (a.rows <= 0 || a.tiles <= 0) return hipSuccess;
    return mode == kModeLut ? dispatch<kModeLut>(a, bits, group_bytes, lds, stream)
                            : dispatch<kModeExact>(a, bits, group_bytes, lds, stream);
}

hipError_t launch_rows(const RowArgs &a, hipStream_t stream) {
    if (a.n <= 0) return hipSuccess;
    for (int i0 = 0; i0 < a.n; i0 += 65535) {
        RowArgs b = a;
        b.n = min(65535, a.n - i0);
        b.dst = a.dst + static_cast<size_t>(i0) * a.in;
        if (a.rows) b.rows = a.rows + i0; else b.r0 = a.r0 + i0;
        const int threads = min(kThreads, a.group);
        hipLaunchKernelGGL(rows_kernel, dim3(a.groups, b.n), dim3(threads), sizeof(float) * a.group, stream, b);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace cqhip
