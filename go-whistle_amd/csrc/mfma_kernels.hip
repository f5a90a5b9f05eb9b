// gfx950 MFMA form of go-whistle's lut product (internal/cq/lut.go) for
// many activations at once, bit for bit the lut kernel's result.
//
// For one group g of an activation t, the lut product of row r is the exact
// integer S = sum_j v_t[j][idx(r, j)] over the group's nibble positions j
// (4-bit: one index per position, 128 positions; 2-bit: one pair of indices
// per position, 64 positions), with v the int14 table entries
// RNE(entry * 8191/M) (lut.go:235-282). Written with a one-hot expansion of
// the indices, S is an integer matrix product over K = (position, code):
//
//   S[t][r] = sum_{j, c} V[t][(j, c)] * OneHot[(j, c)][r],   OneHot = [idx(r, j) == c]
//
// V does not fit int8, so it is split: v = 64 * h + l with l = v & 63 in
// [0, 63] and h = v >> 6 in [-128, 127]. Per position the K dimension holds
// both planes, l's 16 codes then h's 16 codes, and the one-hot holds 1 in
// the l half and 64 in the h half, so one v_mfma_i32_32x32x32_i8 per
// position sums 64 * h + l = v exactly in int32. The float fold is the lut
// kernel's: y += float32(S) * (norm * step), groups in order from y = 0,
// unfused.
//
// A table entry is RNE(f) for |f| <= 8191.5; f + 1.5 * 2^23 rounds to that
// integer (round to nearest even, exact for |f| < 2^22), and its bit pattern
// is 0x4B400000 + RNE(f), whose bits 0-5 are l and bits 6-13 are h.
//
// Work split: a workgroup of 8 wavefronts owns TA activations (64, or 32
// when 64 would leave CUs idle) and 512 weight rows (one 64-row block per
// wavefront, two 32-row MFMA tiles, TA / 32 activation tiles). Per group:
//   1. the activations' groups are rotated (the plain FWHT in the lut
//      kernel's stage order) and scaled by 8191/M into LDS, TA / 8 per
//      wavefront;
//   2. per chunk of 16 positions, every thread builds two tables' two int8
//      planes in LDS [position][plane][activation][16 codes] (the next chunk
//      while the MFMAs run on the current one);
//   3. each wavefront streams its rows' index bytes (16-byte loads in the
//      lut layout), turns each nibble into a 16-byte one-hot in registers and
//      runs 2 * TA / 32 MFMAs per position (activation tiles x 2 row tiles);
//   4. the int32 sums are folded into float32 y in registers.
// MFMA roles: A = table planes (rows = activations), B = one-hot (columns =
// weight rows), so a result row of 32 weight rows is 128 contiguous bytes
// of y.
#include "cq_internal.hpp"
#include "cq_device.hpp"

#include <hip/hip_fp16.h>

namespace cqhip {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

template <int BITS>
struct MfmaGeo {
    static constexpr int G = 128;           // weights per group
    static constexpr int GB = G * BITS / 8;  // index bytes per row and group: 64 or 32
    static constexpr int NJ = 2 * GB;        // nibble positions (tables) per group: 128 or 64
    static constexpr int KS = GB;            // K-steps per group: 2 positions x 16 codes each
    static constexpr int CK = 16;            // positions per LDS chunk of tables
    static constexpr int CW = CK / 8;        // index words per row and chunk (8 positions each)
    static constexpr int NCH = NJ / CK;      // chunks per group
    static constexpr int UPG = GB / 16;      // 16-byte index loads per row and group
    static constexpr int AP = G + 1;         // LDS pitch of an activation's scaled group (odd: no bank conflicts)
};

constexpr int kMfmaWaves = 8;
constexpr int kMfmaThreads = 64 * kMfmaWaves;
constexpr float kRneMagic = 12582912.0f;  // 1.5 * 2^23

__device__ __forceinline__ uint32_t rne_bits(float f) { return __float_as_uint(f + kRneMagic); }

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Four entries' bit patterns -> the l plane's 4 bytes (v & 63) and the h
// plane's 4 bytes ((v >> 6) & 255): the entries' low halfwords are paired,
// shifted right by 6 two at a time (bits 6-13 land in each halfword's low
// byte), and the wanted bytes gathered.
__device__ __forceinline__ void planes4(uint32_t e0, uint32_t e1, uint32_t e2, uint32_t e3, uint32_t &lo,
                                        uint32_t &hi) {
    const uint32_t q01 = __builtin_amdgcn_perm(e1, e0, 0x05040100u);  // e0.lo16 | e1.lo16 << 16
    const uint32_t q23 = __builtin_amdgcn_perm(e3, e2, 0x05040100u);  // e2.lo16 | e3.lo16 << 16
    lo = __builtin_amdgcn_perm(q23, q01, 0x06040200u) & 0x3f3f3f3fu;  // byte 0 of each halfword
    const u16x2 r01 = __builtin_bit_cast(u16x2, q01) >> static_cast<unsigned short>(6);
    const u16x2 r23 = __builtin_bit_cast(u16x2, q23) >> static_cast<unsigned short>(6);
    hi = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, r23), __builtin_bit_cast(uint32_t, r01), 0x06040200u);
}

// 16-byte one-hot of a nibble n holding `val` (1 or 64) at byte n.
__device__ __forceinline__ i32x4 one_hot(uint32_t n, unsigned long long val) {
    const unsigned long long one = val << ((n & 7u) << 3);
    const bool low = n < 8u;
    const unsigned long long lo = low ? one : 0ull, hi = low ? 0ull : one;
    i32x4 r;
    r.x = static_cast<int>(lo);
    r.y = static_cast<int>(lo >> 32);
    r.z = static_cast<int>(hi);
    r.w = static_cast<int>(hi >> 32);
    return r;
}

template <int BITS, int TA>
__global__ __launch_bounds__(kMfmaThreads) void lut_mfma_kernel(LutLaunch a) {
    using M = MfmaGeo<BITS>;
    constexpr int G = M::G, AP = M::AP, CK = M::CK;
    constexpr int AT = TA / 32;  // activation tiles per wavefront
    extern __shared__ __align__(16) unsigned char smem[];
    float *av = reinterpret_cast<float *>(smem);                    // [TA][AP] scaled rotated groups
    float *stp = av + TA * AP;                                       // [TA] steps of the group
    int8_t *tab = reinterpret_cast<int8_t *>(stp + TA);              // [2][CK][2][TA][16] table planes
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, half = lane >> 5, l32 = lane & 31;

    int jb = 0;
#pragma unroll
    for (int k = 1; k < kKernargJobs; ++k)
        if (k < a.njobs && static_cast<int>(blockIdx.x) >= a.wg0[k]) jb = k;
    const JobDesc &J = a.jobs[jb];
    const int blk = (static_cast<int>(blockIdx.x) - a.wg0[jb]) * kMfmaWaves + w;  // this wavefront's block
    const bool rows_here = blk < J.nblk;
    const int gblk = J.blk0 + blk;
    const int t0 = blockIdx.y * TA;
    const int groups = J.groups;

    // Fused ZCRMSNorm of the activation rows (norm.go:53-109): divisors of
    // the workgroup's activations, four float64 partial sums each.
    __shared__ double zpart[4 * TA];
    __shared__ float zrms[TA];
    if (J.ngain) {
        for (int e = tid; e < 4 * TA; e += kMfmaThreads) {
            const int t = t0 + e / 4;
            zpart[e] = t < J.rows ? zc_partial(J.x + static_cast<long long>(t) * J.x_stride, J.in, e % 4) : 0.0;
        }
        __syncthreads();
        for (int e = tid; e < TA; e += kMfmaThreads)
            zrms[e] = zc_rms(zpart[4 * e], zpart[4 * e + 1], zpart[4 * e + 2], zpart[4 * e + 3], J.in);
        __syncthreads();
    }

    i32x16 acc[AT][2];     // [activation tile][row tile]
    float yv[AT][2][16];   // [activation tile][row tile][element]
#pragma unroll
    for (int at = 0; at < AT; ++at)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int i = 0; i < 16; ++i) yv[at][rt][i] = 0.0f;

    auto build = [&](int c, int buf) {
        for (int e = tid; e < TA * CK; e += kMfmaThreads) {
            const int t = e % TA, jc = e / TA;
            const int j = c * CK + jc;
            uint32_t b[16];
            if constexpr (BITS == 4) {  // lutTables4Generic (lut.go:263-282)
                const float x = av[t * AP + j];
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const float f = J.cb[q] * x;
                    b[q] = rne_bits(f);
                }
            } else {  // lutTables2Generic (lut.go:239-258): code q = hi << 2 | lo
                const float x0 = av[t * AP + 2 * j], x1 = av[t * AP + 2 * j + 1];
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const float l = J.cb[q & 3] * x0, h = J.cb[q >> 2] * x1;
                    const float s = l + h;
                    b[q] = rne_bits(s);
                }
            }
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) planes4(b[4 * q], b[4 * q + 1], b[4 * q + 2], b[4 * q + 3], lo[q], hi[q]);
            int8_t *dst = tab + ((static_cast<size_t>(buf) * CK + jc) * 2 * TA + t) * 16;
            *reinterpret_cast<uint4 *>(dst) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            *reinterpret_cast<uint4 *>(dst + TA * 16) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        }
    };

    // The wavefront's rows' index bytes of group g, unit u (lut layout:
    // 16-byte units of a 64-row block side by side); word q of a unit holds
    // the index bytes of chunk 4u + q.
    auto load_unit = [&](int g, int u, uint32_t (&d)[2][4]) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            if (rows_here) {
                const uint4 v = *reinterpret_cast<const uint4 *>(
                    J.idx + ((static_cast<size_t>(gblk) * J.units + g * M::UPG + u) * 64 + rt * 32 + l32) * 16);
                d[rt][0] = v.x; d[rt][1] = v.y; d[rt][2] = v.z; d[rt][3] = v.w;
            } else {
                d[rt][0] = d[rt][1] = d[rt][2] = d[rt][3] = 0u;
            }
        }
    };

    // A wavefront's activations' values of group g (TA / 8 of them, two per
    // lane each): group 0 loaded here, group g + 1 while group g streams.
    constexpr int PW = TA / kMfmaWaves;  // activations per wavefront
    float xg[PW][2];
    auto load_x = [&](int g) {
#pragma unroll
        for (int k = 0; k < PW; ++k) {
            const int t = t0 + w + k * kMfmaWaves;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int col = g * G + e * 64 + lane;
                float xv = (t < J.rows && col < J.in) ? J.x[static_cast<long long>(t) * J.x_stride + col] : 0.0f;
                if (J.xgate && t < J.rows && col < J.in)  // Attention.output's gate (attention.go:245-249)
                    xv = xv * gate_sigmoid(J.xgate[static_cast<long long>(t) * J.x_stride + col]);
                xg[k][e] = xv;
            }
        }
    };
    load_x(0);
    for (int g = 0; g < groups; ++g) {
        uint32_t cur[2][4], nxt[2][4];
        load_unit(g, 0, nxt);
        float nrm[2];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
            nrm[rt] = rows_here ? __half2float(__ushort_as_half(
                                      J.norm[(static_cast<size_t>(gblk) * groups + g) * 64 + rt * 32 + l32]))
                                : 0.0f;

        // 1. Rotation and bound of the group of each activation (lut.go:158-178):
        // a wavefront's TA / 8 activations together, their butterflies
        // interleaved.
        {
            float v[PW][2];
#pragma unroll
            for (int k = 0; k < PW; ++k)
#pragma unroll
                for (int e = 0; e < 2; ++e) v[k][e] = xg[k][e];
            if (J.ngain) {
#pragma unroll
                for (int k = 0; k < PW; ++k) {
                    const int tt = w + k * kMfmaWaves, t = t0 + tt;
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const int col = g * G + e * 64 + lane;
                        if (t < J.rows && col < J.in) {
                            const float gx = J.ngain[col] * v[k][e];
                            v[k][e] = gx / zrms[tt];
                        }
                    }
                }
            }
#pragma unroll
            for (int h = 1; h < 64; h <<= 1) {  // stages h = 1 .. 32 across lanes (kernel.go:384-393)
#pragma unroll
                for (int k = 0; k < PW; ++k)
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const float p = xor_lane(v[k][e], h);
                        v[k][e] = (lane & h) ? p - v[k][e] : v[k][e] + p;
                    }
            }
#pragma unroll
            for (int k = 0; k < PW; ++k) {  // stage h = 64 within the lane
                const float p = v[k][0], q = v[k][1];
                v[k][0] = p + q;
                v[k][1] = p - q;
            }
            float mx[PW];
#pragma unroll
            for (int k = 0; k < PW; ++k) {
                mx[k] = 0.0f;
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    if constexpr (BITS == 4) {
                        mx[k] = go_max(mx[k], fabsf(v[k][e]));
                    } else {
                        const float p = xor_lane<1>(v[k][e]);
                        const float s2 = fabsf(v[k][e]) + fabsf(p);  // |x̂_2q| + |x̂_2q+1| (lut.go:241-243)
                        mx[k] = go_max(mx[k], s2);
                    }
                }
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1)
#pragma unroll
                for (int k = 0; k < PW; ++k) mx[k] = go_max(mx[k], xor_lane(mx[k], off));
#pragma unroll
            for (int k = 0; k < PW; ++k) {
                const int tt = w + k * kMfmaWaves;
                const float m = J.cb_max * mx[k];
                const float inv = m > 0.0f ? static_cast<float>(kLutQ) / m : 0.0f;  // lutInv (lut.go:219-225)
#pragma unroll
                for (int e = 0; e < 2; ++e) av[tt * AP + e * 64 + lane] = v[k][e] * inv;
                if (lane == 0) stp[tt] = m * J.lut_step;
            }
        }
        lds_barrier();
        build(0, 0);
#pragma unroll
        for (int at = 0; at < AT; ++at)
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) acc[at][rt] = i32x16{};
        lds_barrier();

        if (g + 1 < groups) load_x(g + 1);

        // 2./3. Chunks of CK positions (CW index words per row): the next
        // chunk's tables are built while this chunk's MFMAs run.
        const unsigned long long val = half ? 64ull : 1ull;
        constexpr int CW = M::CW;
        for (int u = 0; u < M::UPG; ++u) {
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                for (int q = 0; q < 4; ++q) cur[rt][q] = nxt[rt][q];
            if (u + 1 < M::UPG) load_unit(g, u + 1, nxt);
#pragma unroll
            for (int q = 0; q < 4 / CW; ++q) {
                const int c = (4 / CW) * u + q;
                if (c + 1 < M::NCH) build(c + 1, (c + 1) & 1);
                if (rows_here) {
                    // lane half 0 reads a position's l plane, half 1 its h plane
                    const int8_t *tb = tab + (static_cast<size_t>(c & 1) * CK * 2 + half) * TA * 16;
                    i32x4 A[2][AT];  // [position parity][activation tile]
#pragma unroll
                    for (int at = 0; at < AT; ++at)
                        A[0][at] = *reinterpret_cast<const i32x4 *>(tb + (at * 32 + l32) * 16);
#pragma unroll
                    for (int jc = 0; jc < CK; ++jc) {
                        if (jc + 1 < CK) {
#pragma unroll
                            for (int at = 0; at < AT; ++at)
                                A[(jc + 1) & 1][at] = *reinterpret_cast<const i32x4 *>(
                                    tb + (static_cast<size_t>(jc + 1) * 2 * TA + at * 32 + l32) * 16);
                        }
#pragma unroll
                        for (int rt = 0; rt < 2; ++rt) {
                            // position jc: word jc / 8 of the chunk, byte (jc % 8) / 2, nibble jc % 2
                            const uint32_t n = (cur[rt][q * CW + jc / 8] >> (4 * (jc % 8))) & 15u;
                            const i32x4 B = one_hot(n, val);
#pragma unroll
                            for (int at = 0; at < AT; ++at)
                                acc[at][rt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[jc & 1][at], B, acc[at][rt], 0, 0, 0);
                        }
                    }
                }
                lds_barrier();
            }
        }

        // 4. Fold group g into y, in group order (lut.go:297-310).
        if (rows_here) {
#pragma unroll
            for (int at = 0; at < AT; ++at)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int tt = at * 32 + (i >> 2) * 8 + half * 4 + (i & 3);
                    const float step = stp[tt];
#pragma unroll
                    for (int rt = 0; rt < 2; ++rt) {
                        const int s = acc[at][rt][i];
                        const float coef = nrm[rt] * step;
                        const float prod = static_cast<float>(s) * coef;
                        yv[at][rt][i] = yv[at][rt][i] + prod;
                    }
                }
        }
        lds_barrier();  // av and stp are rewritten by the next group
    }

    if (rows_here) {
#pragma unroll
        for (int at = 0; at < AT; ++at)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int t = t0 + at * 32 + (i >> 2) * 8 + half * 4 + (i & 3);
                if (t >= J.rows) continue;
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    const int r = gblk * 64 + rt * 32 + l32;
                    if (r >= J.row0 && r < J.row0 + J.out) {
                        float out = yv[at][rt][i];
                        if (J.resid)
                            out = J.resid[static_cast<long long>(t) * J.resid_stride + (r - J.row0)] + out;
                        else if (J.act == 1)
                            out = silu_value(out);
                        J.y[static_cast<long long>(t) * J.y_stride + (r - J.row0)] = out;
                    }
                }
            }
    }
}

template <int BITS, int TA>
size_t mfma_lds_bytes() {
    using M = MfmaGeo<BITS>;
    return sizeof(float) * (TA * M::AP + TA) + static_cast<size_t>(2) * M::CK * 2 * TA * 16;
}

template <int BITS, int TA>
hipError_t launch_mfma_t(const LutLaunch &a, int wg, int act_tiles, hipStream_t s) {
    static bool attr = false;  // idempotent attribute write; a race is benign
    const size_t lds = mfma_lds_bytes<BITS, TA>();
    if (!attr) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&lut_mfma_kernel<BITS, TA>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL((lut_mfma_kernel<BITS, TA>), dim3(wg, act_tiles), dim3(kMfmaThreads), lds, s, a);
    return hipGetLastError();
}

// ---- The split form: one group per workgroup, then a fold in group order ----
//
// For products whose 512-row workgroups would leave most CUs idle (the
// decode step's products at a few hundred activations, the encoder's 375
// frames): a workgroup of 4 wavefronts owns 256 weight rows (a 64-row block
// per wavefront), 32 activations and ONE group g. It rotates the group,
// builds the group's tables in LDS and runs the MFMAs, then writes the
// group's float terms float32(S) * (norm * step) (the lut kernel's term,
// rounded the same way) to the workspace, [g][activation][row].
// mfma_fold_kernel then adds an output's terms in group order from 0
// (lut.go:297-310) and applies the fused epilogue: bit for bit the lut
// kernel's result.
//
// Operands of v_mfma_i32_32x32x32_i8 (lane 32h + c holds K = 16h .. 16h + 15
// of row or column c): one K step is a position pair (2p, 2p + 1), lane half
// h carrying position 2p + h. B (columns = weight rows) is the one-hot of
// the row's code at that position, 1 at byte code; A (rows = activations)
// is one plane of the position's 16 entries (l = v & 63 or h = v >> 6). Two
// MFMAs per pair and row tile, one per plane, into two accumulators, so one
// one-hot serves both planes and S = S_l + 64 * S_h exactly.
//
// Grid: one dimension, 8-aligned tiles (256 rows x 32 activations) times
// groups, the groups of a tile 8 workgroups apart.
constexpr int kSplitWaves = 4;
constexpr int kSplitThreads = 64 * kSplitWaves;
constexpr int kSplitTa = 32;  // activations per workgroup: one 32-wide MFMA tile

// 16-byte one-hot: 1 at byte c (c < 16), as two 64-bit shifts.
__device__ __forceinline__ i32x4 one_hot1(uint32_t c) {
    const uint32_t sh = (c & 7u) << 3;
    const uint32_t up = c >> 3;  // 1: the byte is in the upper eight
    const unsigned long long lo = static_cast<unsigned long long>(up ^ 1u) << sh;
    const unsigned long long hi = static_cast<unsigned long long>(up) << sh;
    i32x4 r;
    r.x = static_cast<int>(lo);
    r.y = static_cast<int>(lo >> 32);
    r.z = static_cast<int>(hi);
    r.w = static_cast<int>(hi >> 32);
    return r;
}

// The lut kernel's epilogue for one activation t and one 64-row block (lane
// = row): the int8 append of the block as a head (Int8Rows.Append,
// int8.go:36-55, after RoPE at the stream's position, rope.go:69-81), and
// y, with the residual add or SiLU, for the view's rows.
__device__ __forceinline__ void fold_epilogue(const JobDesc &J, int t, int blk, int lane, float y) {
    const int row = (J.blk0 + blk) * 64;  // root row of lane 0
    if (J.app_q) {
        const int p = J.app_pos[t];
        if (p >= 0 && p < J.app_cap) {
            float v = y;
            if (J.app_cos) {
                const float o = xor_lane<32>(v);
                const int jj = lane & 31;
                const float x1 = lane < 32 ? v : o, x2 = lane < 32 ? o : v;
                float o1, o2;
                rope_pair(x1, x2, J.app_cos[p * 32 + jj], J.app_sin[p * 32 + jj], o1, o2);
                v = lane < 32 ? o1 : o2;
            }
            float m = fabsf(v);
#pragma unroll
            for (int h = 32; h > 0; h >>= 1) m = go_max(m, xor_lane(m, h));
            const float sc = m > 0.0f ? m / 127.0f : 1.0f;
            const int r0 = row - J.row0;  // view row of the head's first value
            int8_t *qp = J.app_q + static_cast<long long>(t) * J.app_q_stride + static_cast<long long>(p) * J.out;
            qp[r0 + lane] = static_cast<int8_t>(go_int8_code(rintf(v / sc)));
            if (lane == 0)
                J.app_s[static_cast<long long>(t) * J.app_s_stride + static_cast<long long>(p) * (J.out >> 6) +
                        (r0 >> 6)] = sc;
        }
    }
    const int r = row + lane;
    if (r >= J.row0 && r < J.row0 + J.out) {
        float out = y;
        if (J.resid)
            out = J.resid[static_cast<long long>(t) * J.resid_stride + (r - J.row0)] + out;
        else if (J.act == 1)
            out = silu_value(out);
        J.y[static_cast<long long>(t) * J.y_stride + (r - J.row0)] = out;
    }
}

template <int BITS>
__global__ __launch_bounds__(kSplitThreads) void lut_mfma_split_kernel(LutLaunch a) {
    using M = MfmaGeo<BITS>;
    constexpr int G = M::G, AP = M::AP, CK = M::CK, TA = kSplitTa;
    constexpr int CPP = CK / 2;          // position pairs per chunk
    constexpr int PLANE = 2 * TA * 16;   // one plane of a pair: 2 positions x TA activations x 16 codes
    constexpr int PAIR = 2 * PLANE;      // both planes
    constexpr int BUF = CPP * PAIR;      // a chunk's tables
    extern __shared__ __align__(16) unsigned char smem[];
    float *av = reinterpret_cast<float *>(smem);                    // [TA][AP] scaled rotated group
    float *stp = av + TA * AP;                                       // [TA] steps of the group
    int8_t *tab = reinterpret_cast<int8_t *>(stp + TA);              // [2][CPP][plane][half][TA][16]
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, half = lane >> 5, l32 = lane & 31;

    const int groups = a.jobs[0].groups;  // one geometry per launch
    const int L = blockIdx.x;
    const int rest = L >> 3;
    const int g = rest % groups;
    const int tile = (rest / groups) * 8 + (L & 7);
    if (tile >= a.split_tiles) return;
    const int rg = tile / a.split_at;  // row group over the jobs' 256-row groups
    const int t0 = (tile % a.split_at) * TA;
    int jb = 0;
#pragma unroll
    for (int k = 1; k < kKernargJobs; ++k)
        if (k < a.njobs && rg >= a.wg0[k]) jb = k;
    const JobDesc &J = a.jobs[jb];
    const int blk = (rg - a.wg0[jb]) * kSplitWaves + w;  // this wavefront's block
    const bool rows_here = blk < J.nblk;
    const int gblk = J.blk0 + blk;
    const int rows = J.rows, in = J.in, units = J.units;
    const long long xs = J.x_stride;
    const float *X = J.x, *XG = J.xgate, *NG = J.ngain;
    const uint8_t *IDX = J.idx;
    const uint16_t *NRM = J.norm;

    // Every first load at once, without branches (rows past the view and
    // activations past the rows read a clamped address and go unused): the
    // group's index bytes of the wavefront's rows (UPG 16-byte units), their
    // norms, and the wavefront's activations' values of the group (TA / 4
    // activations, two per lane).
    const size_t bk = static_cast<size_t>(J.blk0 + min(blk, J.nblk - 1));
    uint32_t idx[M::UPG][2][4];
#pragma unroll
    for (int u = 0; u < M::UPG; ++u)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const uint4 v = *reinterpret_cast<const uint4 *>(
                IDX + ((bk * units + g * M::UPG + u) * 64 + rt * 32 + l32) * 16);
            idx[u][rt][0] = v.x; idx[u][rt][1] = v.y; idx[u][rt][2] = v.z; idx[u][rt][3] = v.w;
        }
    unsigned short nrm16[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) nrm16[rt] = NRM[(bk * groups + g) * 64 + rt * 32 + l32];
    constexpr int PW = TA / kSplitWaves;
    float v[PW][2], gv[PW][2];
#pragma unroll
    for (int k = 0; k < PW; ++k) {
        const long long rowoff = static_cast<long long>(min(t0 + w + k * kSplitWaves, rows - 1)) * xs;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int col = min(g * G + e * 64 + lane, in - 1);
            v[k][e] = X[rowoff + col];
            gv[k][e] = XG ? XG[rowoff + col] : 0.0f;
        }
    }
#pragma unroll
    for (int k = 0; k < PW; ++k)
#pragma unroll
        for (int e = 0; e < 2; ++e)
            if (!(t0 + w + k * kSplitWaves < rows && g * G + e * 64 + lane < in)) v[k][e] = 0.0f;

    // Fused ZCRMSNorm of the activation rows (norm.go:53-109): the tile's
    // activations' divisors over their whole rows, the reference's four
    // float64 partial sums (i mod 4, each in order), the rows staged through
    // LDS 256 columns at a time.
    __shared__ double zpart[4 * TA];
    __shared__ float zrms[TA];
    if (NG) {
        float *stage = reinterpret_cast<float *>(tab);  // [TA][256]
        const int full = in & ~3;
        const int ct = tid >> 2, ck = tid & 3;         // chain thread (tid < 4 * TA): activation, partial
        double s = 0.0;
        for (int p0 = 0; p0 < full; p0 += 256) {
            float st[TA * 256 / kSplitThreads];
#pragma unroll
            for (int r = 0; r < TA * 256 / kSplitThreads; ++r) {
                const int e = tid + r * kSplitThreads;
                const int tt = e >> 8, col = p0 + (e & 255);
                st[r] = X[static_cast<long long>(min(t0 + tt, rows - 1)) * xs + min(col, full - 1)];
            }
#pragma unroll
            for (int r = 0; r < TA * 256 / kSplitThreads; ++r) {
                const int e = tid + r * kSplitThreads;
                if (!(t0 + (e >> 8) < rows && p0 + (e & 255) < full)) st[r] = 0.0f;
            }
#pragma unroll
            for (int r = 0; r < TA * 256 / kSplitThreads; ++r) stage[tid + r * kSplitThreads] = st[r];
            __syncthreads();
            if (tid < 4 * TA) {
                const int n = min(256, full - p0);
                for (int i = ck; i < n; i += 4) {
                    const double d = stage[ct * 256 + i];
                    s = s + d * d;
                }
            }
            __syncthreads();
        }
        if (tid < 4 * TA) {
            if (ck == 0 && t0 + ct < rows)
                for (int c = full; c < in; ++c) {
                    const double d = X[static_cast<long long>(t0 + ct) * xs + c];
                    s = s + d * d;
                }
            zpart[tid] = s;
        }
        __syncthreads();
        if (tid < TA) zrms[tid] = zc_rms(zpart[4 * tid], zpart[4 * tid + 1], zpart[4 * tid + 2], zpart[4 * tid + 3], in);
        __syncthreads();
    }

    // 1. Rotation and bound of group g of each activation (lut.go:158-178),
    // the wavefront's TA / 4 activations together, their butterflies
    // interleaved; first Attention.output's gate (attention.go:245-249) and
    // the norm.
#pragma unroll
    for (int k = 0; k < PW; ++k) {
        const int tt = w + k * kSplitWaves, t = t0 + tt;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int col = g * G + e * 64 + lane;
            if (t < rows && col < in) {
                if (XG) v[k][e] = v[k][e] * gate_sigmoid(gv[k][e]);
                if (NG) {
                    const float gx = NG[col] * v[k][e];
                    v[k][e] = gx / zrms[tt];
                }
            }
        }
    }
#pragma unroll
    for (int h = 1; h < 64; h <<= 1) {  // stages h = 1 .. 32 across lanes (kernel.go:384-393)
#pragma unroll
        for (int k = 0; k < PW; ++k)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const float p = xor_lane(v[k][e], h);
                v[k][e] = (lane & h) ? p - v[k][e] : v[k][e] + p;
            }
    }
#pragma unroll
    for (int k = 0; k < PW; ++k) {  // stage h = 64 within the lane
        const float p = v[k][0], q = v[k][1];
        v[k][0] = p + q;
        v[k][1] = p - q;
    }
    {
        float mx[PW];
#pragma unroll
        for (int k = 0; k < PW; ++k) {
            mx[k] = 0.0f;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                if constexpr (BITS == 4) {
                    mx[k] = go_max(mx[k], fabsf(v[k][e]));
                } else {
                    const float p = xor_lane<1>(v[k][e]);
                    const float s2 = fabsf(v[k][e]) + fabsf(p);  // |x̂_2q| + |x̂_2q+1| (lut.go:241-243)
                    mx[k] = go_max(mx[k], s2);
                }
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
#pragma unroll
            for (int k = 0; k < PW; ++k) mx[k] = go_max(mx[k], xor_lane(mx[k], off));
#pragma unroll
        for (int k = 0; k < PW; ++k) {
            const int tt = w + k * kSplitWaves;
            const float m = J.cb_max * mx[k];
            const float inv = m > 0.0f ? static_cast<float>(kLutQ) / m : 0.0f;  // lutInv (lut.go:219-225)
#pragma unroll
            for (int e = 0; e < 2; ++e) av[tt * AP + e * 64 + lane] = v[k][e] * inv;
            if (lane == 0) stp[tt] = m * J.lut_step;
        }
    }

    // 2. Table items: this thread's are activation tid % TA at positions
    // jc0 and jc0 + 8 of every chunk, both planes to [buf][jc / 2][plane]
    // [jc % 2][activation] (as lut_mfma_kernel's build). An item is built a
    // quarter (four entries) at a time, so that the building spreads over
    // the previous chunk's MFMAs.
    float cbv[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) cbv[q] = J.cb[q];
    const int tA = tid & (TA - 1), jc0 = tid / TA;
    float ix[2][2];           // [item][input]: the item's rotated value(s)
    uint32_t blo[4], bhi[4];  // the item under construction
    auto item_inputs = [&](int c) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int j = c * CK + jc0 + 8 * k;
            if constexpr (BITS == 4) {
                ix[k][0] = av[tA * AP + j];
            } else {
                ix[k][0] = av[tA * AP + 2 * j];
                ix[k][1] = av[tA * AP + 2 * j + 1];
            }
        }
    };
    auto item_quarter = [&](int c, int s) {  // quarter s & 3 of item s >> 2 of chunk c
        const int k = s >> 2, qd = s & 3;
        uint32_t b[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int code = 4 * qd + q;
            if constexpr (BITS == 4) {  // lutTables4Generic (lut.go:263-282)
                b[q] = rne_bits(cbv[code] * ix[k][0]);
            } else {  // lutTables2Generic (lut.go:239-258): code = hi << 2 | lo
                const float l = cbv[code & 3] * ix[k][0], h = cbv[code >> 2] * ix[k][1];
                const float sm = l + h;
                b[q] = rne_bits(sm);
            }
        }
        planes4(b[0], b[1], b[2], b[3], blo[qd], bhi[qd]);
        if (qd == 3) {
            const int jc = jc0 + 8 * k;
            int8_t *dst = tab + ((c & 1) * CPP + (jc >> 1)) * PAIR + ((jc & 1) * TA + tA) * 16;
            *reinterpret_cast<uint4 *>(dst) = make_uint4(blo[0], blo[1], blo[2], blo[3]);
            *reinterpret_cast<uint4 *>(dst + PLANE) = make_uint4(bhi[0], bhi[1], bhi[2], bhi[3]);
        }
    };
    lds_barrier();
    item_inputs(0);
#pragma unroll
    for (int s = 0; s < 8; ++s) item_quarter(0, s);
    lds_barrier();

    // 3. Per chunk of CK positions: its MFMAs, and between them the next
    // chunk's items, a quarter per position pair.
    i32x16 accl[2] = {i32x16{}, i32x16{}}, acch[2] = {i32x16{}, i32x16{}};
    const uint32_t hs = 4u * static_cast<uint32_t>(half);  // a lane half takes the odd nibbles
#pragma unroll
    for (int c = 0; c < M::NCH; ++c) {
        const bool more = c + 1 < M::NCH;
        if (more) item_inputs(c + 1);
        uint32_t wv[2][2];  // [row tile][word]: 4 position pairs a word, this half's nibbles at 8k
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int q = 0; q < 2; ++q) wv[rt][q] = idx[c >> 1][rt][(c & 1) * 2 + q] >> hs;
        const int8_t *tb = tab + (c & 1) * BUF + (half * TA + l32) * 16;
        // A of pair pp in slot pp % 3 (read two pairs ahead), B of pair pp in
        // slot pp % 2 (built one pair ahead)
        i32x4 Al[3], Ah[3], B[2][2];
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
            Al[pp] = *reinterpret_cast<const i32x4 *>(tb + pp * PAIR);
            Ah[pp] = *reinterpret_cast<const i32x4 *>(tb + pp * PAIR + PLANE);
        }
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) B[0][rt] = one_hot1(wv[rt][0] & 15u);
#pragma unroll
        for (int pp = 0; pp < CPP; ++pp) {
            const int sa = pp % 3, sb = pp & 1;
            if (pp + 2 < CPP) {
                const int8_t *nb = tb + (pp + 2) * PAIR;
                Al[(pp + 2) % 3] = *reinterpret_cast<const i32x4 *>(nb);
                Ah[(pp + 2) % 3] = *reinterpret_cast<const i32x4 *>(nb + PLANE);
            }
            __builtin_amdgcn_sched_barrier(0);  // the reads go out here, two pairs before their use
            if (pp + 1 < CPP) {
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
                    B[sb ^ 1][rt] = one_hot1((wv[rt][(pp + 1) >> 2] >> (8 * ((pp + 1) & 3))) & 15u);
            }
            if (more) item_quarter(c + 1, pp);
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
                accl[rt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(Al[sa], B[sb][rt], accl[rt], 0, 0, 0);
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
                acch[rt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(Ah[sa], B[sb][rt], acch[rt], 0, 0, 0);
            // one MFMA and a share of the VALU work, four times
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 7, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        lds_barrier();  // the next chunk's tables are whole; this chunk's buffer is free again
    }

    // 4. The group's terms float32(S) * (norm * step) (lut.go:297-310), to
    // the workspace: [g][activation][64 * nblk rows] of this job.
    const long long rs = static_cast<long long>(J.nblk) * 64;
    if (rows_here) {
        float *tg = a.term[jb] + static_cast<long long>(g) * rows * rs;
        float nrm[2];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) nrm[rt] = __half2float(__ushort_as_half(nrm16[rt]));
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int tt = (i >> 2) * 8 + half * 4 + (i & 3), t = t0 + tt;
            if (t >= rows) continue;
            const float step = stp[tt];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                const int sum = accl[rt][i] + 64 * acch[rt][i];
                const float coef = nrm[rt] * step;
                tg[static_cast<long long>(t) * rs + blk * 64 + rt * 32 + l32] = static_cast<float>(sum) * coef;
            }
        }
    }
}

// The fold of the split form: one wavefront per (activation, 64-row block),
// lane = row: y = 0, then y = y + term[g] for g in order (lut.go:297-310),
// then the lut kernel's epilogue.
__global__ __launch_bounds__(256) void mfma_fold_kernel(LutLaunch a) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int jb = 0;
#pragma unroll
    for (int k = 1; k < kKernargJobs; ++k)
        if (k < a.njobs && static_cast<int>(blockIdx.x) >= a.fold0[k]) jb = k;
    const JobDesc &J = a.jobs[jb];
    const int blk = static_cast<int>(blockIdx.x) - a.fold0[jb];
    const int t = blockIdx.y * 4 + w;
    if (blk >= J.nblk || t >= J.rows) return;
    const long long rs = static_cast<long long>(J.nblk) * 64;
    const float *tp = a.term[jb] + static_cast<long long>(t) * rs + blk * 64 + lane;
    float y = 0.0f;
    for (int g = 0; g < J.groups; ++g) y = y + tp[static_cast<long long>(g) * J.rows * rs];
    fold_epilogue(J, t, blk, lane, y);
}

template <int BITS>
hipError_t launch_split_t(const LutLaunch &a, int grid, hipStream_t s) {
    const size_t lds = mfma_lds_bytes<BITS, kSplitTa>();
    hipLaunchKernelGGL((lut_mfma_split_kernel<BITS>), dim3(grid), dim3(kSplitThreads), lds, s, a);
    return hipGetLastError();
}

}  // namespace

int mfma_split_rows_per_workgroup() { return 64 * kSplitWaves; }
int mfma_split_activations() { return kSplitTa; }

hipError_t launch_lut_mfma_split(const LutLaunch &a, int bits, int fold_blocks, hipStream_t s) {
    if (a.split_tiles <= 0 || a.njobs <= 0) return hipSuccess;
    const int grid = (a.split_tiles + 7) / 8 * 8 * a.jobs[0].groups;
    hipError_t e = bits == 4 ? launch_split_t<4>(a, grid, s) : bits == 2 ? launch_split_t<2>(a, grid, s)
                                                                          : hipErrorInvalidValue;
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(mfma_fold_kernel, dim3(fold_blocks, (a.jobs[0].rows + 3) / 4), dim3(256), 0, s, a);
    return hipGetLastError();
}

bool mfma_geometry_supported(int bits, int group) { return group == 128 && (bits == 2 || bits == 4); }

int mfma_rows_per_workgroup() { return 64 * kMfmaWaves; }

hipError_t launch_lut_mfma(const LutLaunch &a, int bits, int ta, int wg, int act_tiles, hipStream_t s) {
    if (wg <= 0 || act_tiles <= 0) return hipSuccess;
    if (ta == 64) {
        if (bits == 4) return launch_mfma_t<4, 64>(a, wg, act_tiles, s);
        if (bits == 2) return launch_mfma_t<2, 64>(a, wg, act_tiles, s);
    } else if (ta == 32) {
        if (bits == 4) return launch_mfma_t<4, 32>(a, wg, act_tiles, s);
        if (bits == 2) return launch_mfma_t<2, 32>(a, wg, act_tiles, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace cqhip
