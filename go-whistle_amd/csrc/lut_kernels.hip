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
// 64-row blocks of one job. The groups go in chunks of gc, so LDS holds one
// chunk's tables whatever the input width; per chunk:
//  1. Wavefront w rotates the chunk's groups w, w+W, ... in registers (a
//     group of G values is G/64 registers per lane; butterflies below 64
//     exchange lanes with shuffles, the others stay in a lane), reduces M
//     across the wavefront and writes the group's tables (NT tables of 16
//     int16) to LDS. Meanwhile the wavefront's first index loads are in
//     flight.
//  2. After one barrier each wavefront streams its items, a few groups of
//     16-byte loads ahead (a wavefront load is 1 KiB contiguous in the
//     device layout): an item is one group of 64 rows of one block, each
//     lane its row's index bytes, each nibble looked up in the LDS tables
//     (all lanes read the same 16-entry table at once, free of bank
//     conflicts). With at least W blocks a wavefront owns whole blocks and
//     folds y = y + float32(sum) * (norm * step) in a register in group
//     order; with fewer, wavefronts split a block's groups and one pass
//     folds their terms from LDS in group order.
// y goes out after the last chunk (with the fused residual add or SiLU).
#include "cq_internal.hpp"
#include "cq_device.hpp"

#include <hip/hip_fp16.h>

#include <cstddef>

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

// Global-memory views of pointers the kernel reads from its job table: as
// generic pointers their loads would be flat loads, which also count as LDS
// operations, so every LDS wait would wait for the index stream too.
// (The host pass of hipcc only parses device code: there the qualifier is
// left out.)
#if defined(__HIP_DEVICE_COMPILE__)
#define CQ_GLOBAL __attribute__((address_space(1)))
#else
#define CQ_GLOBAL
#endif
template <class T>
__device__ __forceinline__ const CQ_GLOBAL T *gptr(const T *p) {
    return (const CQ_GLOBAL T *)p;
}
template <class T>
__device__ __forceinline__ CQ_GLOBAL T *gptr_w(T *p) {
    return (CQ_GLOBAL T *)p;
}

constexpr int kCpolNt = 2;  // a buffer load's cache policy: non-temporal (nt)

// An index unit of U bytes. NTL: a non-temporal load, for launches that
// stream more index bytes than the caches hold; the decode step's
// matrices, read again every step, are loaded plainly and stay in the
// caches (decode at batch 1: 0.554 -> 0.525 ms per step).
template <int U, bool NTL>
__device__ __forceinline__ void load_unit(const CQ_GLOBAL uint8_t *p, uint32_t (&w)[4]) {
    if constexpr (U == 16) {
        u32x4 v;
        if constexpr (NTL)
            v = __builtin_nontemporal_load(reinterpret_cast<const CQ_GLOBAL u32x4 *>(p));
        else
            v = *reinterpret_cast<const CQ_GLOBAL u32x4 *>(p);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (U == 8) {
        const uint2 v = *reinterpret_cast<const CQ_GLOBAL uint2 *>(p);
        w[0] = v.x; w[1] = v.y; w[2] = 0; w[3] = 0;
    } else if constexpr (U == 4) {
        w[0] = *reinterpret_cast<const CQ_GLOBAL uint32_t *>(p); w[1] = 0; w[2] = 0; w[3] = 0;
    } else if constexpr (U == 2) {
        w[0] = *reinterpret_cast<const CQ_GLOBAL uint16_t *>(p); w[1] = 0; w[2] = 0; w[3] = 0;
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

// Two table entries RNE(a), RNE(b) as int16 halves of one word. For |e| <
// 2^22, e + 1.5 * 2^23 lands where float32 spacing is 1, so the add rounds
// e to the nearest integer, ties to even, exactly as rintf, and the sum's
// low 16 bits are that integer in two's complement (|v| <= 8191 here). One
// byte permute then joins the two low halves.
constexpr float kRneMagic = 12582912.0f;  // 1.5 * 2^23

__device__ __forceinline__ uint32_t rne_pair(float a, float b) {
    const uint32_t ea = __float_as_uint(a + kRneMagic), eb = __float_as_uint(b + kRneMagic);
    return __builtin_amdgcn_perm(eb, ea, 0x05040100u);  // ea.lo16 | eb.lo16 << 16
}

// This lane's raw inputs of group g: the activation values (zero past In,
// lut.go:163-165) and, where given, the norm gains and the gate values.
template <int BITS, int GB>
__device__ __forceinline__ void group_inputs(const CQ_GLOBAL float *x, int in, int g, const CQ_GLOBAL float *ngain,
                                             const CQ_GLOBAL float *xg, float (&xv)[LutGeo<BITS, GB>::E],
                                             float (&gv)[LutGeo<BITS, GB>::E], float (&hv)[LutGeo<BITS, GB>::E],
                                             int lane) {
    using Gm = LutGeo<BITS, GB>;
    constexpr int G = Gm::G, E = Gm::E;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int i = G >= 64 ? e * 64 + lane : lane;
        const int col = g * G + i;
        const bool ok = i < G && col < in;
        xv[e] = ok ? x[col] : 0.0f;
        gv[e] = ngain && ok ? ngain[col] : 0.0f;
        hv[e] = xg && ok ? xg[col] : 0.0f;
    }
}

// Rotation, bound, tables and step of group g of the activation row x
// (lut.go:158-178, 235-282) by one wavefront, from the lane's raw inputs
// (group_inputs): the plain FWHT of the group in registers (a group of G
// values is G/64 registers per lane; butterflies below 64 exchange lanes
// with shuffles, the others stay in a lane), M reduced across the
// wavefront, the NT tables of 16 int16 to tg and the step to *step (lane
// 0). With ngain the row is ZCRMSNorm'ed first (divisor rms); with xg each
// value is first gated, x * sigmoid(xg) (Attention.output,
// internal/needle/attention.go:245-249).
template <int BITS, int GB>
__device__ __forceinline__ void group_tables(const float (&xin)[LutGeo<BITS, GB>::E],
                                             const float (&gin)[LutGeo<BITS, GB>::E],
                                             const float (&hin)[LutGeo<BITS, GB>::E], int in, int g,
                                             const float (&cbv)[16], float cb_max, float lut_step, bool ngain,
                                             float rms, bool xg, short *tg, float *step, int lane) {
    using Gm = LutGeo<BITS, GB>;
    constexpr int G = Gm::G, E = Gm::E;
    float v[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int i = G >= 64 ? e * 64 + lane : lane;
        const int col = g * G + i;
        float xv = xin[e];
        if (ngain && i < G && col < in) {
            const float gx = gin[e] * xv;
            xv = gx / rms;
        }
        if (xg && i < G && col < in) xv = xv * gate_sigmoid(hin[e]);
        v[e] = xv;
    }
#pragma unroll
    for (int h = 1; h < G; h <<= 1) {  // stages h = 1, 2, ..., G/2 (kernel.go:384-393)
        if (h < 64) {
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const float p = xor_lane(v[e], h);
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
            mx = go_max(mx, fabsf(v[e]));
        } else {
            const float p = xor_lane<1>(v[e]);
            const float s2 = fabsf(v[e]) + fabsf(p);  // |x̂_2q| + |x̂_2q+1| (lut.go:241-243)
            mx = go_max(mx, s2);
        }
    }
    // Go's max keeps a NaN (lut.go:241-243, 266-268): a group holding one
    // has M = NaN, inv = 0 and step NaN, so every row's y is NaN, as the
    // generic Go and the arm64 kernel (FMAX) give.
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = go_max(mx, xor_lane(mx, off));
    const float m = cb_max * mx;
    const float inv = m > 0.0f ? static_cast<float>(kLutQ) / m : 0.0f;  // lutInv (lut.go:219-225)
    if (lane == 0) *step = m * lut_step;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int i = G >= 64 ? e * 64 + lane : lane;
        if constexpr (BITS == 4) {  // lutTables4Generic (lut.go:263-282)
            if (i < G) {
                const float av = v[e] * inv;
                uint32_t q[8];
#pragma unroll
                for (int c = 0; c < 16; c += 2)
                    q[c / 2] = rne_pair(cbv[c] * av, cbv[c + 1] * av);
                uint4 *dst = reinterpret_cast<uint4 *>(tg + static_cast<size_t>(i) * 16);
                dst[0] = make_uint4(q[0], q[1], q[2], q[3]);
                dst[1] = make_uint4(q[4], q[5], q[6], q[7]);
            }
        } else {  // lutTables2Generic (lut.go:239-258): the even lane writes codes 0-7, the odd 8-15
            const float p = xor_lane<1>(v[e]);
            if (i < G) {
                const bool odd = lane & 1;
                const float av = (odd ? p : v[e]) * inv, bv = (odd ? v[e] : p) * inv;
                const int c0 = odd ? 8 : 0;
                const float hlo = odd ? cbv[2] : cbv[0], hhi = odd ? cbv[3] : cbv[1];
                uint32_t q[4];
#pragma unroll
                for (int cc = 0; cc < 8; cc += 2) {
                    // code c = c0 + cc: c & 3 = cc & 3, c >> 2 = (odd ? 2 : 0) + (cc >> 2)
                    const float l0 = cbv[cc & 3] * av, h0 = ((cc >> 2) ? hhi : hlo) * bv;
                    const float l1 = cbv[(cc + 1) & 3] * av, h1 = (((cc + 1) >> 2) ? hhi : hlo) * bv;
                    q[cc / 2] = rne_pair(l0 + h0, l1 + h1);
                }
                *reinterpret_cast<uint4 *>(tg + static_cast<size_t>(i / 2) * 16 + c0) =
                    make_uint4(q[0], q[1], q[2], q[3]);
            }
        }
    }
}

// Groups of index loads a wavefront keeps in flight, and wavefronts per
// SIMD the kernel is built for (its registers fit that many). Eight 16-byte
// loads ahead (DG = 8 / loads per group) at four or five wavefronts per
// SIMD; 32-byte groups of 2-bit indices instead keep four loads ahead at six
// wavefronts per SIMD (measured: a 2-bit sweep launch 53 -> 49 us, where
// 4-bit groups lose with fewer loads ahead).
template <int BITS, int GB>
constexpr int lut_loads_ahead() {
    constexpr int UPG = LutGeo<BITS, GB>::UPG;
    if (BITS == 2 && GB == 32) return 2;
    return UPG >= 8 ? 1 : 8 / UPG;
}
template <int BITS, int GB>
constexpr int lut_waves_per_simd() {
    return GB >= 256 ? 2 : (BITS == 2 && GB == 32) ? 6 : 4;
}

// A JobDesc held one dword per lane (lane i: dword i), fetched by one vector
// load: the wavefront pays a single memory round trip for every field of
// its job. Scalar loads of the same fields went out in three or four
// dependent rounds (the compiler spreads them to spare scalar registers),
// each about a microsecond at batch 1 where a product takes a few.
static_assert(sizeof(JobDesc) <= 256, "a JobDesc must fit one dword per lane");
struct JobRegs {
    uint32_t d;
    template <class T>
    __device__ __forceinline__ T get(size_t off) const {
        const uint32_t lo = __builtin_amdgcn_readlane(d, static_cast<int>(off / 4));
        if constexpr (sizeof(T) == 8) {
            const uint32_t hi = __builtin_amdgcn_readlane(d, static_cast<int>(off / 4 + 1));
            return __builtin_bit_cast(T, static_cast<uint64_t>(lo) | static_cast<uint64_t>(hi) << 32);
        } else {
            return __builtin_bit_cast(T, lo);
        }
    }
};
__device__ __forceinline__ JobRegs job_regs(const JobDesc *J, int lane) {
    const CQ_GLOBAL uint32_t *w = gptr(reinterpret_cast<const uint32_t *>(J));
    return JobRegs{lane * 4 < static_cast<int>(sizeof(JobDesc)) ? w[lane] : 0u};
}
// The same fields by scalar loads through a pointer: the batch plans' job
// table, which lives in device memory behind the unit table (measured
// faster there than the vector fetch).
struct JobPtr {
    const JobDesc *J;
    template <class T>
    __device__ __forceinline__ T get(size_t off) const {
        return *reinterpret_cast<const T *>(reinterpret_cast<const char *>(J) + off);
    }
};
#define JOB(jr, T, field) ((jr).template get<T>(offsetof(JobDesc, field)))

// One work unit: blocks [b0, b0 + bc) of job jr (counted from its blk0) for
// activation act.
// V = 2 (wide launches of one-block units): two wavefronts share each group
// of the block, one half of its index units each; their exact int32 sums
// meet in LDS before the float term.
// The next product's tables from a finished output row (TabOut): the
// table form's pre-pass (lut_tables_kernel) for one activation t, fused
// into the producer's epilogue, op for op the same. yo holds the row (in
// floats), wsp the LDS work area of lut_tout_lds_bytes(in). The whole
// workgroup (W wavefronts) comes here and leaves together.
//   1. ZCRMSNorm's divisor (norm.go:53-109): the squares d * d (exact in
//      float64) go to LDS as [i mod 4][i / 4], lanes 0-3 add each partial in
//      order;
//   2. wavefront w takes groups w, w + W, ...: the gain and divisor, the
//      plain FWHT in the reference's stage order (kernel.go:384-393), the
//      bound M and the step M * lutStep, the values scaled by 8191 / M
//      (lut.go:158-178, 219-225);
//   3. every thread builds items (one position's 16 entries, both planes,
//      lut.go:239-282) and writes them in the A-operand order
//      [tile][group][pair][plane][half][32][16].
template <int TB>
__device__ __forceinline__ void next_tables(const TabOut &o, const float *yo, unsigned char *wsp, int t, int tid,
                                            int lane, int w, int W) {
    constexpr int G = 128, NJ = G * TB / 4, NP = NJ / 2, AP = G + 1;
    const int in = o.in, groups = o.groups, qn = in >> 2, qs = qn + 2;
    double *sq = reinterpret_cast<double *>(wsp + static_cast<size_t>(in) * 4);
    float *av = reinterpret_cast<float *>(wsp + static_cast<size_t>(in) * 12 + 64);
    float *zm = av + ((groups * AP + 3) & ~3);
    const CQ_GLOBAL float *ng = gptr(o.ngain);
    float rms = 1.0f;
    if (ng) {
        for (int i = tid; i < in; i += 64 * W) {
            const double d = yo[i];
            sq[(i & 3) * qs + (i >> 2)] = d * d;
        }
        __syncthreads();
        double part = 0.0;
        if (tid < 4) {
            const double *row = sq + tid * qs;
            int m = 0;
            for (; m + 16 <= qn; m += 16) {
                double v[16];
#pragma unroll
                for (int k = 0; k < 16; ++k) v[k] = row[m + k];
#pragma unroll
                for (int k = 0; k < 16; ++k) part = part + v[k];
            }
            for (; m < qn; ++m) part = part + row[m];
        }
        if (w == 0) {
            const double p0 = __shfl(part, 0), p1 = __shfl(part, 1), p2 = __shfl(part, 2), p3 = __shfl(part, 3);
            if (lane == 0) zm[0] = zc_rms(p0, p1, p2, p3, in);
        }
        __syncthreads();
        rms = zm[0];
    }
    CQ_GLOBAL float *stp = gptr_w(o.stp);
    for (int g = w; g < groups; g += W) {
        float v[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int col = g * G + e * 64 + lane;
            v[e] = yo[col];
            if (ng) {
                const float gx = ng[col] * v[e];
                v[e] = gx / rms;
            }
        }
#pragma unroll
        for (int h = 1; h < 64; h <<= 1)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const float p = xor_lane(v[e], h);
                v[e] = (lane & h) ? p - v[e] : v[e] + p;
            }
        {
            const float p = v[0], q = v[1];
            v[0] = p + q;
            v[1] = p - q;
        }
        float mx = 0.0f;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            if constexpr (TB == 4) {
                mx = go_max(mx, fabsf(v[e]));
            } else {
                const float p = xor_lane<1>(v[e]);
                const float s2 = fabsf(v[e]) + fabsf(p);  // |x̂_2q| + |x̂_2q+1| (lut.go:241-243)
                mx = go_max(mx, s2);
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) mx = go_max(mx, xor_lane(mx, off));
        const float m = o.cb_max * mx;
        const float inv = m > 0.0f ? static_cast<float>(kLutQ) / m : 0.0f;  // lutInv (lut.go:219-225)
#pragma unroll
        for (int e = 0; e < 2; ++e) av[g * AP + e * 64 + lane] = v[e] * inv;
        if (lane == 0) stp[(static_cast<size_t>(t >> 5) * groups + g) * 32 + (t & 31)] = m * o.lut_step;
    }
    __syncthreads();
    float cbv[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) cbv[q] = o.cb[q];
    CQ_GLOBAL int8_t *tab = gptr_w(o.tab) + (static_cast<size_t>(t >> 5) * groups) * NP * 2048 + (t & 31) * 16;
    for (int it = tid; it < groups * NJ; it += 64 * W) {
        const int g = it / NJ, j = it - g * NJ;
        float x0, x1 = 0.0f;
        if constexpr (TB == 4) {
            x0 = av[g * AP + j];
        } else {
            x0 = av[g * AP + 2 * j];
            x1 = av[g * AP + 2 * j + 1];
        }
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            uint32_t b[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int code = 4 * qd + q;
                if constexpr (TB == 4) {
                    b[q] = rne_bits(cbv[code] * x0);
                } else {  // code = hi << 2 | lo
                    const float l = cbv[code & 3] * x0, h = cbv[code >> 2] * x1;
                    const float sm = l + h;
                    b[q] = rne_bits(sm);
                }
            }
            planes4(b[0], b[1], b[2], b[3], lo[qd], hi[qd]);
        }
        CQ_GLOBAL int8_t *dst = tab + static_cast<size_t>(g) * NP * 2048 + (j >> 1) * 2048 + (j & 1) * 512;
        *reinterpret_cast<CQ_GLOBAL uint4 *>(dst) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        *reinterpret_cast<CQ_GLOBAL uint4 *>(dst + 1024) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    }
}

template <int BITS, int GB, class JS, int V = 1, bool PRE = false, bool NTL = false, int TB = 0>
__device__ __forceinline__ void lut_unit(const LutLaunch &a, const JS &jr, int b0, int bc, int act, int W) {
    using Gm = LutGeo<BITS, GB>;
    constexpr int U = Gm::U, UPG = Gm::UPG, NT = Gm::NT;
    static_assert(UPG % V == 0, "a group's units split evenly");
    constexpr int UPGV = UPG / V;  // index units per item of one wavefront
    constexpr int DG = lut_loads_ahead<BITS, GB>();  // groups of index loads in flight per wavefront

    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);

    // The job's fields, taken once before any store.
    const int j_in = JOB(jr, int, in), j_row0 = JOB(jr, int, row0), j_out = JOB(jr, int, out);
    const int j_act = JOB(jr, int, act);
    const CQ_GLOBAL uint16_t *j_norm = gptr(JOB(jr, const uint16_t *, norm));
    CQ_GLOBAL float *j_y = gptr_w(JOB(jr, float *, y));
    const long long j_ystride = JOB(jr, long long, y_stride), j_rstride = JOB(jr, long long, resid_stride);
    const CQ_GLOBAL float *j_ngain = gptr(JOB(jr, const float *, ngain)), *j_resid = gptr(JOB(jr, const float *, resid));
    const float j_cbmax = JOB(jr, float, cb_max), j_step = JOB(jr, float, lut_step);
    float cbv[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) cbv[c] = jr.template get<float>(offsetof(JobDesc, cb) + 4 * c);
    const int groups = JOB(jr, int, groups), units = JOB(jr, int, units), blk0 = JOB(jr, int, blk0) + b0;
    const CQ_GLOBAL uint8_t *idx = gptr(JOB(jr, const uint8_t *, idx));
    // 16-byte units are buffer loads off the matrix's index array: a 32-bit
    // offset per lane instead of a 64-bit address (cq_new keeps the array
    // under 2 GiB)
    const __amdgpu_buffer_rsrc_t irs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(JOB(jr, const uint8_t *, idx)), 0, 0x7fffffff,
                                          0x00020000);
    const long long j_xstride = JOB(jr, long long, x_stride);
    const CQ_GLOBAL float *x = gptr(JOB(jr, const float *, x)) + static_cast<long long>(act) * j_xstride;
    const float *j_xgate = JOB(jr, const float *, xgate);
    const CQ_GLOBAL float *xg = j_xgate ? gptr(j_xgate) + static_cast<long long>(act) * j_xstride : nullptr;

    // LDS: tables of a chunk of gc groups, the chunk's steps, y of the
    // workgroup's rows between chunks, the chunk's float terms of up to tc
    // blocks (when wavefronts share a block), and the row's norm divisor.
    const int gc = a.gc, tc = a.tb;
    short *tab = reinterpret_cast<short *>(smem);
    float *steps = reinterpret_cast<float *>(smem + static_cast<size_t>(gc) * NT * 16 * sizeof(short));
    float *yacc = steps + gc;
    float *term = yacc + static_cast<size_t>(a.bpw_max) * 64;
    float *misc = term + static_cast<size_t>(gc) * tc * 64;
    // With TB: the output row (the next tables' input) and their work area
    // past misc's 16 bytes, 16-byte aligned.
    unsigned char *tob = nullptr;
    float *tyo = nullptr;
    if constexpr (TB != 0) {
        tob = smem + ((reinterpret_cast<unsigned char *>(misc + 4) - smem + 15) & ~static_cast<ptrdiff_t>(15));
        tyo = reinterpret_cast<float *>(tob);
    }

    // Fused ZCRMSNorm of the activation row (norm.go:53-109): the row goes
    // through LDS in pieces (one coalesced read each), lanes 0-3 of
    // wavefront 0 keep the four float64 partial sums in the reference's
    // order (lane k: elements i = k mod 4 below In & ~3, lane 0 then the
    // tail), and the divisor is shared through LDS. With PRE (the
    // latency-bound launches) it runs after the first chunk's index loads
    // are issued, with them in flight.
    float rms = 1.0f;
    auto row_norm = [&]() {
        float *xs = reinterpret_cast<float *>(smem);
        const int cap = static_cast<int>(misc - xs) & ~63;
        const int dim = j_in, full = dim & ~3;
        double part = 0.0;
        for (int p0 = 0; p0 < dim; p0 += cap) {
            const int pn = min(cap, dim - p0);
#pragma unroll 4
            for (int t = tid; t < pn; t += 64 * W) xs[t] = x[p0 + t];
            __syncthreads();
            if (tid < 4) {
                const int lim = min(p0 + pn, full);
                int i = p0 + tid;
                for (; i + 60 < lim; i += 64) {
                    float v[16];
#pragma unroll
                    for (int k = 0; k < 16; ++k) v[k] = xs[i - p0 + 4 * k];
#pragma unroll
                    for (int k = 0; k < 16; ++k) {
                        const double d = v[k];
                        part = part + d * d;
                    }
                }
                for (; i < lim; i += 4) {
                    const double d = xs[i - p0];
                    part = part + d * d;
                }
                if (tid == 0)
                    for (int t = max(full, p0); t < p0 + pn; ++t) {
                        const double d = xs[t - p0];
                        part = part + d * d;
                    }
            }
            __syncthreads();
        }
        if (w == 0) {
            const double p0 = __shfl(part, 0), p1 = __shfl(part, 1), p2 = __shfl(part, 2), p3 = __shfl(part, 3);
            if (lane == 0) misc[0] = zc_rms(p0, p1, p2, p3, dim);
        }
        __syncthreads();
        rms = misc[0];
    };

    if (!PRE && j_ngain) row_norm();

    // With PRE, this wavefront's first group's raw inputs and, for the
    // fold's first wavefront, its row's residual are loaded together with
    // the first index loads, so that no global read waits behind the norm or
    // the lookups (more registers: the launches of many units go without).
    using GmI = LutGeo<BITS, GB>;
    float pxv[GmI::E], pgv[GmI::E], phv[GmI::E];
    float rpre = 0.0f;
    auto preload = [&]() {
        if (w < min(a.gc, groups)) group_inputs<BITS, GB>(x, j_in, w, j_ngain, xg, pxv, pgv, phv, lane);
        const int r = blk0 * 64 + tid;
        if (j_resid && tid < 64 && r >= j_row0 && r < j_row0 + j_out)
            rpre = j_resid[static_cast<long long>(act) * j_rstride + (r - j_row0)];
    };

    // The same norm from the row as the wavefronts hold it (with PRE, one
    // chunk of at most W groups, In a multiple of 4): each lane's squares
    // d * d go to LDS as [k][i / 4] for k = i mod 4, so that lanes 0-3 only
    // add, in the reference's order, with no second read of the row.
    auto row_norm_held = [&]() {
        constexpr int Gh = LutGeo<BITS, GB>::G, Eh = LutGeo<BITS, GB>::E;
        const int qn = j_in >> 2, qs = qn + 2;  // row length, padded stride (16-byte rows)
        double *sq = reinterpret_cast<double *>(smem);
        if (w < groups) {
#pragma unroll
            for (int e = 0; e < Eh; ++e) {
                const int i = Gh >= 64 ? e * 64 + lane : lane;
                const int col = w * Gh + i;
                if (i < Gh && col < j_in) {
                    const double d = pxv[e];
                    sq[(col & 3) * qs + (col >> 2)] = d * d;
                }
            }
        }
        __syncthreads();
        double part = 0.0;
        if (tid < 4) {
            const double *row = sq + tid * qs;
            int m = 0;
            for (; m + 16 <= qn; m += 16) {
                double v[16];
#pragma unroll
                for (int k = 0; k < 16; ++k) v[k] = row[m + k];
#pragma unroll
                for (int k = 0; k < 16; ++k) part = part + v[k];
            }
            for (; m < qn; ++m) part = part + row[m];
        }
        if (w == 0) {
            const double p0 = __shfl(part, 0), p1 = __shfl(part, 1), p2 = __shfl(part, 2), p3 = __shfl(part, 3);
            if (lane == 0) misc[0] = zc_rms(p0, p1, p2, p3, j_in);
        }
        __syncthreads();
        rms = misc[0];
    };

    // The fused int8 append of a finished block: the whole wavefront holds
    // its 64 values (lane = row), one head of the cache row. Int8Rows.Append
    // (int8.go:36-55) with RoPE first (rope.go:69-81: value i < 32 pairs
    // with i + 32), bit for bit the separate append kernel.
    int8_t *const j_aq = JOB(jr, int8_t *, app_q);
    float *const j_as = JOB(jr, float *, app_s);
    const long long j_aqs = JOB(jr, long long, app_q_stride), j_ass = JOB(jr, long long, app_s_stride);
    // The row's cache position, a global load whose value is first needed
    // at the write: with PRE it is issued with the first index loads. An
    // opaque per-lane zero in its address keeps the value in a vector
    // register, where the compiler would otherwise move it to a scalar one
    // at once and wait for every load issued so far.
    int j_apos = -1;
    auto load_apos = [&]() {
        int vz;
        asm volatile("v_mov_b32 %0, 0" : "=v"(vz));
        if (j_aq) j_apos = *gptr(JOB(jr, const int32_t *, app_pos) + act + vz);
    };
    if (!PRE) load_apos();
    const int j_acap = JOB(jr, int, app_cap);
    const CQ_GLOBAL float *j_acos = gptr(JOB(jr, const float *, app_cos)), *j_asin = gptr(JOB(jr, const float *, app_sin));
    float pcos = 0.0f, psin = 0.0f;  // with PRE: wavefront 0's RoPE pair at that position, loaded early
    auto append_block = [&](int bb, int ln, float v, int j_apos) {
        const int r0 = (blk0 + bb) * 64 - j_row0;  // view row of the head's first value
        if (j_acos) {
            const float o = xor_lane<32>(v);
            const int jj = ln & 31;
            const float a = ln < 32 ? v : o, b = ln < 32 ? o : v;
            const float cs = PRE && ln == tid ? pcos : j_acos[j_apos * 32 + jj];
            const float sn = PRE && ln == tid ? psin : j_asin[j_apos * 32 + jj];
            float o1, o2;
            rope_pair(a, b, cs, sn, o1, o2);
            v = ln < 32 ? o1 : o2;
        }
        float m = fabsf(v);
#pragma unroll
        for (int h = 32; h > 0; h >>= 1) m = go_max(m, xor_lane(m, h));
        const float sc = m > 0.0f ? m / 127.0f : 1.0f;
        CQ_GLOBAL int8_t *qp = gptr_w(j_aq) + static_cast<long long>(act) * j_aqs + static_cast<long long>(j_apos) * j_out;
        qp[r0 + ln] = static_cast<int8_t>(go_int8_code(rintf(v / sc)));
        if (ln == 0)
            gptr_w(j_as)[static_cast<long long>(act) * j_ass + static_cast<long long>(j_apos) * (j_out >> 6) + (r0 >> 6)] = sc;
    };

    auto write_out = [&](int bb, int ln, float v) {
        if (j_aq) {
            int ap = j_apos;
            asm volatile("" : "+v"(ap));  // the position's wait stays here
            if (ap >= 0 && ap < j_acap) append_block(bb, ln, v, ap);
        }
        const int r = (blk0 + bb) * 64 + ln;
        if (r >= j_row0 && r < j_row0 + j_out) {
            float out = v;
            if (j_resid)
                out = (PRE && bb == 0 && ln == tid ? rpre : j_resid[static_cast<long long>(act) * j_rstride + (r - j_row0)]) + out;
            else if (j_act == 1)
                out = silu_value(out);
            j_y[static_cast<long long>(act) * j_ystride + (r - j_row0)] = out;
            if constexpr (TB != 0) tyo[r - j_row0] = out;
        }
    };

    // Wavefront roles. With at least as many blocks as wavefronts, wavefront
    // w owns blocks w, w + W, ... and every group of them, and folds each
    // row in a register in group order. With fewer, S wavefronts share a
    // block (groups gs, gs + S, ...), their terms meet in LDS and one pass
    // folds them in group order.
    int S = 1;
    if constexpr (V == 1) {
        while (S * 2 * bc <= W) S *= 2;
    } else {
        S = W / V;  // one block: wavefront w takes half w % V of groups w / V, w / V + S, ...
    }
    const int vp = V == 1 ? 0 : w % V;  // this wavefront's half of each group's units

    // One chunk of groups from g0. With PRE and a single chunk it runs
    // outside any loop: in a loop the compiler's wait analysis carries
    // loads across the back edge and waits for the first index loads before
    // the preloads go out.
    auto chunk = [&](int g0) {
        const int gch = min(gc, groups - g0);
        const bool last = g0 + gch >= groups;
        const int wv = w / V;  // V = 1: w
        const int bbs = wv / S, gs = wv - (wv / S) * S;
        int Q;
        if (S == 1)
            Q = w < bc ? ((bc - w + W - 1) / W) * gch : 0;
        else
            Q = (bbs < bc && gs < gch) ? (gch - gs + S - 1) / S : 0;
        // The wavefront's items in order: (block bb, chunk group gi); with
        // S = 1 the groups of block w, then of block w + W, ...; with S > 1
        // groups gs, gs + S, ... of block bbs.
        struct Pos {
            int bb, gi;
        };
        auto next = [&](Pos &p) {
            if (S == 1) {
                if (++p.gi == gch) {
                    p.gi = 0;
                    p.bb += W;
                }
            } else {
                p.gi += S;
            }
        };
        const Pos first = S == 1 ? Pos{w, 0} : Pos{bbs, gs};
        uint32_t buf[DG][UPGV][4];
        uint32_t nv[DG];
        // Loads past the wavefront's last item read one 16-byte line again
        // (the index array's first, or of the activation row for narrower
        // units; kept in L2): the stream issues the same loads every turn, so
        // each of its waits is a fixed count, and no index byte is fetched
        // twice.
        const CQ_GLOBAL uint8_t *spare =
            U == 16 ? idx : (const CQ_GLOBAL uint8_t *)(reinterpret_cast<uintptr_t>(x) & ~uintptr_t(15));
        auto load_group = [&](const Pos &p, bool real, uint32_t (&bf)[UPGV][4], uint32_t &nrm) {
            const CQ_GLOBAL uint8_t *ip =
                real ? idx + (static_cast<size_t>(blk0 + p.bb) * units + static_cast<size_t>(g0 + p.gi) * UPG +
                              static_cast<size_t>(vp) * UPGV) * 64 * U +
                           static_cast<size_t>(lane) * U
                     : spare;
            const size_t ustride = real ? static_cast<size_t>(64) * U : 0;
            if constexpr (U == 16) {
                const unsigned off = static_cast<unsigned>(ip - idx);
#pragma unroll
                for (int u = 0; u < UPGV; ++u) {
                    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(irs, off + u * static_cast<unsigned>(ustride),
                                                                          0, NTL ? kCpolNt : 0);
                    bf[u][0] = v.x; bf[u][1] = v.y; bf[u][2] = v.z; bf[u][3] = v.w;
                }
            } else {
#pragma unroll
                for (int u = 0; u < UPGV; ++u) load_unit<U, NTL>(ip + u * ustride, bf[u]);
            }
            // The row norm as the aligned 32-bit word holding it (this
            // lane's half: lane & 1), the norm table's own first word on a
            // spare turn: a merge of 32-bit loads needs no extension where
            // the branches meet, so nothing waits for the load here.
            const CQ_GLOBAL uint32_t *np32 =
                real ? reinterpret_cast<const CQ_GLOBAL uint32_t *>(
                           j_norm + (static_cast<size_t>(blk0 + p.bb) * groups + g0 + p.gi) * 64) + (lane >> 1)
                     : reinterpret_cast<const CQ_GLOBAL uint32_t *>(j_norm);
            nrm = *np32;
        };
        // The first items are in flight while the tables are built.
        Pos lp = first;
        int lq = 0;  // items loaded
        auto refill = [&](uint32_t (&bf)[UPGV][4], uint32_t &nrm) {
            load_group(lp, lq < Q, bf, nrm);
            if (lq < Q) next(lp);
            ++lq;
        };
        if (Q > 0) {
#pragma unroll
            for (int d = 0; d < DG; ++d) refill(buf[d], nv[d]);
        }

        if (PRE && g0 == 0) {
            preload();
            load_apos();
        }
        if (PRE && g0 == 0 && j_ngain) {
            if (gch == groups && groups <= W && (j_in & 3) == 0 &&
                2 * (j_in + 8) <= (static_cast<int>(misc - reinterpret_cast<float *>(smem)) & ~63))
                row_norm_held();
            else
                row_norm();
        }
        if (PRE && g0 == 0 && j_acos && tid < 64 && j_aq) {
            int ap = j_apos;
            asm volatile("" : "+v"(ap));  // the position's wait stays here, behind the norm
            if (ap >= 0 && ap < j_acap) {
                pcos = j_acos[ap * 32 + (lane & 31)];
                psin = j_asin[ap * 32 + (lane & 31)];
            }
        }

        // 1. Rotation, bound and tables of the chunk's groups w, w+W, ...
        for (int gi = w; gi < gch; gi += W) {
            float xv[GmI::E], gv[GmI::E], hv[GmI::E];
            if (PRE && g0 == 0 && gi == w) {
#pragma unroll
                for (int e = 0; e < GmI::E; ++e) {
                    xv[e] = pxv[e];
                    gv[e] = pgv[e];
                    hv[e] = phv[e];
                }
            } else {
                group_inputs<BITS, GB>(x, j_in, g0 + gi, j_ngain, xg, xv, gv, hv, lane);
            }
            group_tables<BITS, GB>(xv, gv, hv, j_in, g0 + gi, cbv, j_cbmax, j_step, j_ngain != nullptr, rms,
                                   xg != nullptr, tab + static_cast<size_t>(gi) * NT * 16, &steps[gi], lane);
        }
        __syncthreads();

        // 2. The wavefront's items in order, DG groups of loads ahead: the
        // lookups' exact int32 sum, the term float32(sum) * (norm * step),
        // folded into the row (or parked for the shared fold).
        float acc = 0.0f;
        Pos cp = first;
        for (int q0 = 0; q0 < Q; q0 += DG) {
            // Longest remaining work first. A CU's SIMDs issue their oldest
            // wavefront first, so the workgroups of a CU finished in age
            // order and the end of a launch ran on ever fewer wavefronts;
            // priorities by the items a wavefront has left (s_setprio)
            // keep the long units ahead and the CU full to the end. On
            // MI355X: the GEMV sweep's 4-bit launch 70.4 -> 69.8 us,
            // 64 x 16384x512 CQ4 54.7 -> 52.3 us, the 2-bit launch 38.8 ->
            // 35.7 us (bit for bit the same results).
            if constexpr (V == 1 && !PRE) {
                const int nch = (groups + gc - 1) / gc;
                const int left = (nch - g0 / gc) * Q - q0;
                if (left > 12) __builtin_amdgcn_s_setprio(3);
                else if (left > 8) __builtin_amdgcn_s_setprio(2);
                else if (left > 4) __builtin_amdgcn_s_setprio(1);
                else __builtin_amdgcn_s_setprio(0);
            }
#pragma unroll
            for (int d = 0; d < DG; ++d) {
                if (q0 + d < Q) {
                    const int bb = cp.bb, gi = cp.gi;
                    const uint32_t tg = lds_addr(tab + static_cast<size_t>(gi) * NT * 16);
                    int s = 0;
#pragma unroll
                    for (int u = 0; u < UPGV; ++u)
                        s += lookup_unit<U>(buf[d][u], tg + (vp * UPGV + u) * 2 * U * 16 * 2);
                    const float n = __half2float(__ushort_as_half(static_cast<unsigned short>(nv[d] >> (16 * (lane & 1)))));
                    const float coef = n * steps[gi];
                    if constexpr (V > 1) {  // [gi][half][lane] int32 sums, then [gi][lane] coefficients
                        int *termi = reinterpret_cast<int *>(term);
                        termi[(gi * V + vp) * 64 + lane] = s;
                        if (vp == 0) term[gc * V * 64 + gi * 64 + lane] = coef;
                        next(cp);
                        refill(buf[d], nv[d]);
                        continue;
                    }
                    const float t = static_cast<float>(s) * coef;
                    if (S == 1) {
                        if (gi == 0) acc = g0 == 0 ? 0.0f : yacc[bb * 64 + lane];
                        acc = acc + t;
                        if (gi == gch - 1) {
                            if (last)
                                write_out(bb, lane, acc);
                            else
                                yacc[bb * 64 + lane] = acc;
                        }
                    } else {
                        term[(static_cast<size_t>(gi) * tc + bb) * 64 + lane] = t;
                    }
                    next(cp);
                }
                refill(buf[d], nv[d]);
            }
        }
        if (V > 1) {  // one block: the halves' sums added (exact), then the unfused fold in group order
            __syncthreads();
            if (tid < 64) {
                const int *termi = reinterpret_cast<const int *>(term);
                float y = g0 == 0 ? 0.0f : yacc[tid];
                for (int gi = 0; gi < gch; ++gi) {
                    int sum = 0;
#pragma unroll
                    for (int h = 0; h < V; ++h) sum += termi[(gi * V + h) * 64 + tid];
                    const float t = static_cast<float>(sum) * term[gc * V * 64 + gi * 64 + tid];
                    y = y + t;
                }
                if (last)
                    write_out(0, tid, y);
                else
                    yacc[tid] = y;
            }
        } else if (S > 1) {
            __syncthreads();
            for (int t = tid; t < bc * 64; t += 64 * W) {
                const int bb = t >> 6, ln = t & 63;
                float y = g0 == 0 ? 0.0f : yacc[t];
                for (int gi = 0; gi < gch; ++gi) y = y + term[(static_cast<size_t>(gi) * tc + bb) * 64 + ln];
                if (last)
                    write_out(bb, ln, y);
                else
                    yacc[t] = y;
            }
        }
        if (!last) __syncthreads();  // tables, steps and terms are rewritten by the next chunk
    };
    if (PRE && gc >= groups)
        chunk(0);
    else
        for (int g0 = 0; g0 < groups; g0 += gc) chunk(g0);
    if constexpr (TB != 0) {  // the workgroup wrote all of the row (host: one workgroup per activation)
        __syncthreads();
        next_tables<TB>(a.tout, tyo, tob, act, tid, lane, w, W);
    }
}

template <int BITS, int GB, bool DEV>
__global__ __launch_bounds__(256, (lut_waves_per_simd<BITS, GB>())) void lut_kernel(LutLaunch a) {
    const int lane = threadIdx.x & 63;
    if constexpr (DEV) {  // a batch plan: one unit per workgroup
        // Batch plans stream many matrices once (the GEMV sweep: 4-bit 68
        // against 74 us with plain loads; its 2-bit launch is the other way
        // round, 37.5 against 39.5 us, and loads plainly).
        const WorkUnit u = a.dunits[blockIdx.x];
        lut_unit<BITS, GB, JobPtr, 1, false, BITS == 4>(a, JobPtr{a.djobs + u.job}, u.blk, u.nb, u.act,
                                                        blockDim.x >> 6);
    } else {  // job blockIdx.z: its address needs no load first
        const JobRegs jr = job_regs(&a.jobs[blockIdx.z], lane);
        const int bpw = a.bpw, gc = a.gc, tb = a.tb, bpw_max = a.bpw_max;
        // the job and the launch's fields arrive in one round
        asm volatile("" ::"v"(jr.d), "s"(bpw), "s"(gc), "s"(tb), "s"(bpw_max));
        const int b0 = static_cast<int>(blockIdx.x) * bpw, nblk = JOB(jr, int, nblk);
        if (b0 >= nblk) return;  // a shorter job's surplus workgroups, before any barrier
        // kLutWaves wavefronts (blockDim.x would be one more kernel-argument load)
        lut_unit<BITS, GB>(a, jr, b0, min(bpw, nblk - b0), blockIdx.y, kLutWaves);
    }
}

// Latency-bound launches (the decode step at batch 1, and grids of at most
// one workgroup per CU): a.waves wavefronts per workgroup. V = 1: with one
// block, a wavefront per group; with a.bpw blocks, wavefronts w take block
// w / S and groups w % S, w % S + S, ... (S the largest power of two with
// S * blocks <= waves). V = 2 (one
// block): two per group, each on half its index units, so that each
// wavefront's chain of table lookups is shorter.
//
// TB (2 or 4): the launch is one workgroup per activation over all rows of
// its one job, and each builds the next product's TB-bit tables from its
// output row (next_tables, a.tout).
template <int BITS, int GB, int V, int TB>
__global__ __launch_bounds__(1024) void lut_kernel_wide(LutLaunch a) {
    const int lane = threadIdx.x & 63;
    const JobRegs jr = job_regs(&a.jobs[blockIdx.z], lane);
    const int bpw = a.bpw, gc = a.gc, tb = a.tb, bpw_max = a.bpw_max, waves = a.waves;
    asm volatile("" ::"v"(jr.d), "s"(bpw), "s"(gc), "s"(tb), "s"(bpw_max), "s"(waves));
    const int b0 = static_cast<int>(blockIdx.x) * bpw, nblk = JOB(jr, int, nblk);
    if (b0 >= nblk) return;
    int act = blockIdx.y;
    if constexpr (TB != 0) {
        // 256 workgroups, activation (y mod 8) * 32 + y / 8: workgroup y runs
        // on XCD y mod 8 (dispatch goes round the XCDs), so the 32
        // activations of a table tile share one L2, where their 16-byte
        // pieces of each line meet before the line is written back
        // (measured on MI355X: the batch-256 decode step 1.591 -> 1.561 ms)
        act = (blockIdx.y & 7) * 32 + (blockIdx.y >> 3);
        if (act >= JOB(jr, int, rows)) return;  // the whole workgroup, before any barrier
    }
    lut_unit<BITS, GB, JobRegs, V, true, false, TB>(a, jr, b0, min(bpw, nblk - b0), act, waves);
}

template <int BITS, int GB, int V, int TB = 0>
hipError_t launch_wide(const LutLaunch &a, int gx, int gy, size_t lds, hipStream_t s) {
    static std::atomic<unsigned long long> attr{0};
    if (hipError_t e =
            lds_limit_once(reinterpret_cast<const void *>(&lut_kernel_wide<BITS, GB, V, TB>), 160 * 1024, attr))
        return e;
    hipLaunchKernelGGL((lut_kernel_wide<BITS, GB, V, TB>), dim3(gx, gy, a.njobs), dim3(64 * a.waves), lds, s, a);
    return hipGetLastError();
}

template <int BITS, int GB>
hipError_t launch_t(const LutLaunch &a, int waves, int gx, int gy, size_t lds, hipStream_t s) {
    if constexpr (GB == 32 || GB == 64) {
        if (a.dunits == nullptr && a.waves > kLutWaves) {
            // a.tb blocks' terms fit in LDS: the wavefronts sharing a block park them there
            if (a.waves != waves || a.waves > 16 || a.bpw > a.tb || (a.vsplit == 2 && a.bpw != 1))
                return hipErrorInvalidValue;
            if (a.tout.tab) {
                // one workgroup per activation over all of one job's rows, 128-weight groups both sides
                if (gx != 1 || gy != 256 || a.njobs != 1 || a.vsplit != 1 || a.bpw < a.jobs[0].nblk ||
                    a.tout.in != a.jobs[0].out || a.tout.groups * 128 != a.tout.in || a.tout.groups > 8 ||
                    a.jobs[0].rows > 256 || a.jobs[0].rows > a.tout.tiles * 32)
                    return hipErrorInvalidValue;
                if constexpr (GB == BITS * 16) {
                    if (a.tout.bits == 4) return launch_wide<BITS, GB, 1, 4>(a, gx, gy, lds, s);
                    if (a.tout.bits == 2) return launch_wide<BITS, GB, 1, 2>(a, gx, gy, lds, s);
                }
                return hipErrorInvalidValue;
            }
            return a.vsplit == 2 ? launch_wide<BITS, GB, 2>(a, gx, gy, lds, s) : launch_wide<BITS, GB, 1>(a, gx, gy, lds, s);
        }
    }
    if (a.tout.tab) return hipErrorInvalidValue;  // only the wide form builds tables
    if (a.dunits == nullptr && waves != kLutWaves) return hipErrorInvalidValue;  // that path assumes kLutWaves
    const bool dev = a.dunits != nullptr;
    const void *fn = dev ? reinterpret_cast<const void *>(&lut_kernel<BITS, GB, true>)
                         : reinterpret_cast<const void *>(&lut_kernel<BITS, GB, false>);
    static std::atomic<unsigned long long> attr[2] = {{0}, {0}};
    if (hipError_t e = lds_limit_once(fn, 160 * 1024, attr[dev])) return e;
    if (dev)
        hipLaunchKernelGGL((lut_kernel<BITS, GB, true>), dim3(gx), dim3(64 * waves), lds, s, a);
    else
        hipLaunchKernelGGL((lut_kernel<BITS, GB, false>), dim3(gx, gy, a.njobs), dim3(64 * waves), lds, s, a);
    return hipGetLastError();
}

}  // namespace

size_t lut_lds_bytes(int bits, int group_bytes, int gc, int tb, int bpw) {
    (void)bits;
    return static_cast<size_t>(gc) * (2 * group_bytes * 16 * sizeof(short) + static_cast<size_t>(tb) * 64 * 4 + 4) +
           static_cast<size_t>(bpw) * 64 * 4 + 16;
}

size_t lut_tout_lds_bytes(int in) {
    const size_t groups = static_cast<size_t>(in) / 128;
    return 16 + static_cast<size_t>(in) * 12 + 64 + ((groups * 129 + 3) & ~static_cast<size_t>(3)) * 4 + 16;
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
