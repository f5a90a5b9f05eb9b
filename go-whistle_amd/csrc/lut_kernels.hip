// gfx950 lut kernel: go-whistle's default CQ product (internal/cq/lut.go),
// bit for bit, for one or many jobs per launch.
//
// Per activation group (lut.go:158-178, 235-282): the plain FWHT of the
// group, the bound M (cbMax * max|x̂|, or * max(|x̂_2q| + |x̂_2q+1|) for two
// bits), the integer tables v = RNE(entry * 8191/M) and the step M *
// lutStep. Per row and group (lut.go:289-313): the exact int32 sum of the
// looked-up v over the group's index bytes, then y += float32(sum) * (norm *
// step) in group order from y = 0. Every float operation is the
// reference's, unfused (-ffp-contract=off) and in its order; the integer
// sums are exact in any order. The int16 tables hold v itself: the
// reference's two byte planes (a VPSHUFB/TBL artefact) sum to the same
// integers (lut.go:16-27).
//
// Work split. A workgroup of W wavefronts owns one activation of a range of
// 64-row blocks of one job.
// The groups go in chunks of gc, so LDS holds one chunk's tables whatever
// the input width; per chunk:
//  1. Wavefront w rotates the chunk's groups w, w+W, ... in registers (a
//     group of G values is G/64 registers per lane; butterflies below 64
//     exchange lanes with shuffles, the others stay in a lane), reduces M
//     across the wavefront and writes the group's tables (NT tables of 16
//     int16) to LDS. Meanwhile the chunk's first index loads are in flight.
//  2. After one barrier the (group, block) items of each tile of blocks go
//     round-robin to the wavefronts. An item is 64 rows' index bytes of one
//     group: each lane streams its row's bytes with 16-byte loads (a
//     wavefront load is 1 KiB contiguous in the device layout), double
//     buffered across items, and looks each nibble up in the LDS tables; all
//     lanes read the same 16-entry table at once, so the lookups are free of
//     bank conflicts. The int32 sums meet in LDS.
//  3. The thread that owns a row folds the chunk's groups into the row's y
//     (in LDS) in group order; y goes out after the last chunk.
#include "cq_internal.hpp"
#include "cq_device.hpp"

#include <hip/hip_fp16.h>

namespace cqhip {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int BITS, int GB>
struct LutGeo {
    static constexpr int G = GB * 8 / BITS;      // weights per group
    static constexpr int U = GB < 16 ? GB : 16;  // index bytes per lane load
    static constexpr int UPG = GB / U;           // loads per group
    static constexpr int NT = 2 * GB;            // 16-entry tables per group
    static constexpr int E = G >= 64 ? G / 64 : 1;  // rotated values per lane
};

template <int U>
__device__ __forceinline__ void load_unit(const uint8_t *p, uint32_t (&w)[4]) {
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

typedef __attribute__((address_space(3))) const short lds_short;

__device__ __forceinline__ int lds_read_i16(uint32_t addr) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wint-to-pointer-cast"
    return *(lds_short *)addr;  // LDS pointers are 32-bit
#pragma clang diagnostic pop
}

// LDS byte address of a shared-memory pointer.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

// Sum of the 2*U looked-up entries of one unit: the low nibble of byte k
// reads table 2k, the high nibble table 2k+1 (lut.go:301-306). base is the
// LDS address of the unit's first table, 32-byte aligned, so an entry's
// address is base | 2*nibble, plus the table's immediate offset 32*(2k or
// 2k+1).
// base | byte B of t, in one VALU op (an SDWA byte select).
template <int B>
__device__ __forceinline__ uint32_t or_byte(uint32_t base, uint32_t t) {
    uint32_t r;
    if constexpr (B == 0)
        asm("v_or_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
            : "=v"(r) : "v"(base), "v"(t));
    else if constexpr (B == 1)
        asm("v_or_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
            : "=v"(r) : "v"(base), "v"(t));
    else if constexpr (B == 2)
        asm("v_or_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
            : "=v"(r) : "v"(base), "v"(t));
    else
        asm("v_or_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
            : "=v"(r) : "v"(base), "v"(t));
    return r;
}

template <int U, int Q>
__device__ __forceinline__ int lookup_word(uint32_t wd, uint32_t base) {
    // 2 * low and 2 * high nibble of each of the word's bytes: each entry
    // address is then one byte-select OR with the table base.
    const uint32_t te = (wd << 1) & 0x1e1e1e1eu, to = (wd >> 3) & 0x1e1e1e1eu;
    int s = 0;
    constexpr int k0 = 4 * Q;
    s += lds_read_i16(or_byte<0>(base, te) + 64 * (k0 + 0)) + lds_read_i16(or_byte<0>(base, to) + 64 * (k0 + 0) + 32);
    if constexpr (k0 + 1 < U)
        s += lds_read_i16(or_byte<1>(base, te) + 64 * (k0 + 1)) + lds_read_i16(or_byte<1>(base, to) + 64 * (k0 + 1) + 32);
    if constexpr (k0 + 2 < U)
        s += lds_read_i16(or_byte<2>(base, te) + 64 * (k0 + 2)) + lds_read_i16(or_byte<2>(base, to) + 64 * (k0 + 2) + 32);
    if constexpr (k0 + 3 < U)
        s += lds_read_i16(or_byte<3>(base, te) + 64 * (k0 + 3)) + lds_read_i16(or_byte<3>(base, to) + 64 * (k0 + 3) + 32);
    return s;
}

template <int U>
__device__ __forceinline__ int lookup_unit(const uint32_t (&w)[4], uint32_t base) {
    int s = lookup_word<U, 0>(w[0], base);
    if constexpr (U > 4) s += lookup_word<U, 1>(w[1], base);
    if constexpr (U > 8) {
        s += lookup_word<U, 2>(w[2], base);
        s += lookup_word<U, 3>(w[3], base);
    }
    return s;
}

__device__ __forceinline__ int rne_int(float e) { return static_cast<int>(rintf(e)); }

__device__ __forceinline__ uint32_t pack16(int lo, int hi) {
    return (static_cast<uint32_t>(lo) & 0xffffu) | (static_cast<uint32_t>(hi) << 16);
}

template <int BITS, int GB, bool DEV>
__global__ __launch_bounds__(1024) void lut_kernel(LutLaunch a) {
    using Gm = LutGeo<BITS, GB>;
    constexpr int G = Gm::G, U = Gm::U, UPG = Gm::UPG, NT = Gm::NT, E = Gm::E;

    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int W = blockDim.x >> 6;

    const JobDesc *J;
    int b0, bc, act;
    if constexpr (DEV) {
        const WorkUnit u = a.dunits[blockIdx.x];
        J = a.djobs + u.job;
        b0 = u.blk;
        bc = u.nb;
        act = u.act;
    } else {
        int j = 0;
#pragma unroll
        for (int k = 1; k < kKernargJobs; ++k)
            if (k < a.njobs && static_cast<int>(blockIdx.x) >= a.wg0[k]) j = k;
        J = &a.jobs[j];
        b0 = (static_cast<int>(blockIdx.x) - a.wg0[j]) * a.bpw;
        bc = min(a.bpw, J->nblk - b0);
        act = blockIdx.y;
    }
    const int groups = J->groups, units = J->units, blk0 = J->blk0 + b0;
    const uint8_t *idx = J->idx;
    const float *x = J->x + static_cast<long long>(act) * J->x_stride;

    // Fused ZCRMSNorm of the activation row (norm.go:53-109): its divisor,
    // from four float64 partial sums on lanes 0-3 of every wavefront.
    float rms = 1.0f;
    if (J->ngain) {
        const double part = lane < 4 ? zc_partial(x, J->in, lane) : 0.0;
        const double p0 = __shfl(part, 0), p1 = __shfl(part, 1), p2 = __shfl(part, 2), p3 = __shfl(part, 3);
        rms = zc_rms(p0, p1, p2, p3, J->in);
    }

    // LDS: tables of a chunk of gc groups, the chunk's int32 sums of a tile,
    // the chunk's steps, and y of the workgroup's rows (folded chunk by chunk).
    const int gc = a.gc, tb = a.tb;
    short *tab = reinterpret_cast<short *>(smem);
    int *part = reinterpret_cast<int *>(smem + static_cast<size_t>(gc) * NT * 16 * sizeof(short));
    float *steps = reinterpret_cast<float *>(part + static_cast<size_t>(gc) * tb * 64);
    float *yacc = steps + gc;

    // Items of a tile within a chunk: k -> chunk group k / nbt, block
    // k % nbt; wavefront w takes k = w, w + W, ...
    auto item_ptr = [&](int g0, int t0, int nbt, int k) -> const uint8_t * {
        const int gi = k / nbt, bb = k - (k / nbt) * nbt;
        return idx + (static_cast<size_t>(blk0 + t0 + bb) * units + static_cast<size_t>(g0 + gi) * UPG) * 64 * U +
               static_cast<size_t>(lane) * U;
    };
    uint32_t bufA[UPG][4], bufB[UPG][4];
    auto load_item = [&](const uint8_t *p, uint32_t (&buf)[UPG][4]) {
#pragma unroll
        for (int u = 0; u < UPG; ++u) load_unit<U>(p + static_cast<size_t>(u) * 64 * U, buf[u]);
    };
    auto compute_item = [&](int nbt, int k, const uint32_t (&buf)[UPG][4]) {
        const int gi = k / nbt, bb = k - (k / nbt) * nbt;
        const uint32_t tg = lds_addr(tab + static_cast<size_t>(gi) * NT * 16);
        int s = 0;
#pragma unroll
        for (int u = 0; u < UPG; ++u) s += lookup_unit<U>(buf[u], tg + u * 2 * U * 16 * 2);
        part[(gi * tb + bb) * 64 + lane] = s;
    };

    for (int t = tid; t < bc * 64; t += blockDim.x) yacc[t] = 0.0f;

    for (int g0 = 0; g0 < groups; g0 += gc) {
        const int gch = min(gc, groups - g0);
        // The chunk's first item is in flight while its tables are built.
        const int nbt0 = min(tb, bc);
        if (w < gch * nbt0) load_item(item_ptr(g0, 0, nbt0, w), bufA);

        // 1. Rotation, bound and tables of the chunk's groups w, w+W, ...
        for (int gi = w; gi < gch; gi += W) {
            const int g = g0 + gi;
            float v[E];
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const int i = G >= 64 ? e * 64 + lane : lane;
                const int col = g * G + i;
                float xv = (i < G && col < J->in) ? x[col] : 0.0f;  // zero-padded past In (lut.go:163-165)
                if (J->ngain && i < G && col < J->in) {
                    const float gx = J->ngain[col] * xv;
                    xv = gx / rms;
                }
                v[e] = xv;
            }
#pragma unroll
            for (int h = 1; h < G; h <<= 1) {  // stages h = 1, 2, ..., G/2 (kernel.go:384-393)
                if (h < 64) {
#pragma unroll
                    for (int e = 0; e < E; ++e) {
                        const float p = __shfl_xor(v[e], h);
                        v[e] = (lane & h) ? p - v[e] : v[e] + p;  // a - b on the upper lane, a + b on the lower
                    }
                } else {
                    const int d = h / 64;
#pragma unroll
                    for (int e = 0; e < E; ++e)
                        if (!(e & d)) {
                            const float p = v[e], q = v[e + d];
                            v[e] = p + q;
                            v[e + d] = p - q;
                        }
                }
            }
            float mx = 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                if constexpr (BITS == 4) {
                    mx = fmaxf(mx, fabsf(v[e]));
                } else {
                    const float p = __shfl_xor(v[e], 1);
                    const float s2 = fabsf(v[e]) + fabsf(p);  // |x̂_2q| + |x̂_2q+1| (lut.go:241-243)
                    mx = fmaxf(mx, s2);
                }
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
            const float m = J->cb_max * mx;
            const float inv = m > 0.0f ? static_cast<float>(kLutQ) / m : 0.0f;  // lutInv (lut.go:219-225)
            if (lane == 0) steps[gi] = m * J->lut_step;
            short *tg = tab + static_cast<size_t>(gi) * NT * 16;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const int i = G >= 64 ? e * 64 + lane : lane;
                if constexpr (BITS == 4) {  // lutTables4Generic (lut.go:263-282)
                    if (i < G) {
                        const float av = v[e] * inv;
                        uint32_t q[8];
#pragma unroll
                        for (int c = 0; c < 16; c += 2)
                            q[c / 2] = pack16(rne_int(J->cb[c] * av), rne_int(J->cb[c + 1] * av));
                        uint4 *dst = reinterpret_cast<uint4 *>(tg + static_cast<size_t>(i) * 16);
                        dst[0] = make_uint4(q[0], q[1], q[2], q[3]);
                        dst[1] = make_uint4(q[4], q[5], q[6], q[7]);
                    }
                } else {  // lutTables2Generic (lut.go:239-258): the even lane writes codes 0-7, the odd 8-15
                    const float p = __shfl_xor(v[e], 1);
                    if (i < G) {
                        const bool odd = lane & 1;
                        const float av = (odd ? p : v[e]) * inv, bv = (odd ? v[e] : p) * inv;
                        const int c0 = odd ? 8 : 0;
                        uint32_t q[4];
#pragma unroll
                        for (int cc = 0; cc < 8; cc += 2) {
                            const int c = c0 + cc;
                            const float l0 = J->cb[c & 3] * av, h0 = J->cb[c >> 2] * bv;
                            const float l1 = J->cb[(c + 1) & 3] * av, h1 = J->cb[(c + 1) >> 2] * bv;
                            q[cc / 2] = pack16(rne_int(l0 + h0), rne_int(l1 + h1));
                        }
                        *reinterpret_cast<uint4 *>(tg + static_cast<size_t>(i / 2) * 16 + c0) =
                            make_uint4(q[0], q[1], q[2], q[3]);
                    }
                }
            }
        }
        __syncthreads();

        // 2./3. Tiles of tb blocks: lookups, then the chunk's groups folded
        // into y in group order.
        for (int t0 = 0; t0 < bc; t0 += tb) {
            const int nbt = min(tb, bc - t0);
            const int items = gch * nbt;
            if (t0 > 0 && w < items) load_item(item_ptr(g0, t0, nbt, w), bufA);
            for (int k = w; k < items; k += 2 * W) {
                const int k1 = k + W, k2 = k + 2 * W;
                if (k1 < items) load_item(item_ptr(g0, t0, nbt, k1), bufB);
                compute_item(nbt, k, bufA);
                if (k1 < items) {
                    if (k2 < items) load_item(item_ptr(g0, t0, nbt, k2), bufA);
                    compute_item(nbt, k1, bufB);
                }
            }
            __syncthreads();
            for (int t = tid; t < nbt * 64; t += blockDim.x) {
                const int blk = blk0 + t0 + (t >> 6), ln = t & 63;
                float acc = yacc[t0 * 64 + t];
                for (int gi = 0; gi < gch; ++gi) {
                    const float n =
                        __half2float(__ushort_as_half(J->norm[(static_cast<size_t>(blk) * groups + g0 + gi) * 64 + ln]));
                    const float coef = n * steps[gi];
                    const float prod = static_cast<float>(part[(gi * tb + (t >> 6)) * 64 + ln]) * coef;
                    acc = acc + prod;
                }
                yacc[t0 * 64 + t] = acc;
            }
            __syncthreads();
        }
    }

    for (int t = tid; t < bc * 64; t += blockDim.x) {
        const int r = blk0 * 64 + t;
        if (r >= J->row0 && r < J->row0 + J->out) {
            float out = yacc[t];
            if (J->resid)
                out = J->resid[static_cast<long long>(act) * J->resid_stride + (r - J->row0)] + out;
            else if (J->act == 1)
                out = silu_value(out);
            J->y[static_cast<long long>(act) * J->y_stride + (r - J->row0)] = out;
        }
    }
}

template <int BITS, int GB>
hipError_t launch_t(const LutLaunch &a, int waves, int gx, int gy, size_t lds, hipStream_t s) {
    const bool dev = a.dunits != nullptr;
    const void *fn = dev ? reinterpret_cast<const void *>(&lut_kernel<BITS, GB, true>)
                         : reinterpret_cast<const void *>(&lut_kernel<BITS, GB, false>);
    static bool attr[2] = {false, false};  // idempotent attribute write; a race is benign
    if (!attr[dev]) {
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return e;
        attr[dev] = true;
    }
    if (dev)
        hipLaunchKernelGGL((lut_kernel<BITS, GB, true>), dim3(gx), dim3(64 * waves), lds, s, a);
    else
        hipLaunchKernelGGL((lut_kernel<BITS, GB, false>), dim3(gx, gy), dim3(64 * waves), lds, s, a);
    return hipGetLastError();
}

}  // namespace

size_t lut_lds_bytes(int bits, int group_bytes, int gc, int tb, int bpw) {
    (void)bits;
    return static_cast<size_t>(gc) * (2 * group_bytes * 16 * sizeof(short) + static_cast<size_t>(tb) * 64 * 4 + 4) +
           static_cast<size_t>(bpw) * 64 * 4;
}

bool lut_geometry_supported(int bits, int gb) {
    if (bits == 4) return gb == 4 || gb == 8 || gb == 16 || gb == 32 || gb == 64 || gb == 128 || gb == 256;
    if (bits == 2) return gb == 2 || gb == 4 || gb == 8 || gb == 16 || gb == 32 || gb == 64 || gb == 128 || gb == 256;
    return false;
}

hipError_t launch_lut(const LutLaunch &a, int bits, int gb, int waves, int gx, int gy, size_t lds, hipStream_t s) {
    if (gx <= 0 || gy <= 0) return hipSuccess;
    if (bits == 4) {
        switch (gb) {
            case 4: return launch_t<4, 4>(a, waves, gx, gy, lds, s);
            case 8: return launch_t<4, 8>(a, waves, gx, gy, lds, s);
            case 16: return launch_t<4, 16>(a, waves, gx, gy, lds, s);
            case 32: return launch_t<4, 32>(a, waves, gx, gy, lds, s);
            case 64: return launch_t<4, 64>(a, waves, gx, gy, lds, s);
            case 128: return launch_t<4, 128>(a, waves, gx, gy, lds, s);
            case 256: return launch_t<4, 256>(a, waves, gx, gy, lds, s);
        }
    } else if (bits == 2) {
        switch (gb) {
            case 2: return launch_t<2, 2>(a, waves, gx, gy, lds, s);
            case 4: return launch_t<2, 4>(a, waves, gx, gy, lds, s);
            case 8: return launch_t<2, 8>(a, waves, gx, gy, lds, s);
            case 16: return launch_t<2, 16>(a, waves, gx, gy, lds, s);
            case 32: return launch_t<2, 32>(a, waves, gx, gy, lds, s);
            case 64: return launch_t<2, 64>(a, waves, gx, gy, lds, s);
            case 128: return launch_t<2, 128>(a, waves, gx, gy, lds, s);
            case 256: return launch_t<2, 256>(a, waves, gx, gy, lds, s);
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace cqhip
