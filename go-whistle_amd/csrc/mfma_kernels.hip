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

#include <type_traits>

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
// m & byte B of t, in one VALU op (an SDWA byte select).
template <int B>
__device__ __forceinline__ uint32_t and_byte(uint32_t m, uint32_t t) {
    uint32_t r;
    if constexpr (B == 0)
        asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
            : "=v"(r) : "v"(m), "v"(t));
    else if constexpr (B == 1)
        asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
            : "=v"(r) : "v"(m), "v"(t));
    else if constexpr (B == 2)
        asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
            : "=v"(r) : "v"(m), "v"(t));
    else
        asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
            : "=v"(r) : "v"(m), "v"(t));
    return r;
}

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

template <int BITS, int TA>
__global__ __launch_bounds__(kMfmaThreads) void lut_mfma_kernel(LutLaunch a) {
    using M = MfmaGeo<BITS>;
    constexpr int G = M::G, AP = M::AP, CK = M::CK, NCH = M::NCH;
    constexpr int AT = TA / 32;  // activation tiles per wavefront
    constexpr int NI = TA * CK / kMfmaThreads;  // table items per thread and chunk: 2 or 1
    constexpr int CPP = CK / 2;                 // position pairs per chunk
    constexpr int PLANE = 2 * TA * 16, PAIR = 2 * PLANE, BUF = CPP * PAIR;
    constexpr int PW = TA / kMfmaWaves;         // activations a wavefront rotates per group
    constexpr int APS = TA == 64 ? 2 : 1;       // activations of a rotation slice
    constexpr int NS = PW / APS;                // slices per group
    constexpr int NA = NCH - 1;                 // chunks of a group that rotate the next one
    constexpr int MAXS = NS > NA ? NS - NA + 1 : 1;  // most slices in one chunk
    extern __shared__ __align__(16) unsigned char smem[];
    float *av = reinterpret_cast<float *>(smem);          // [2][TA][AP] scaled rotated groups (by group parity)
    float *stp = av + 2 * TA * AP;                         // [2][TA] their steps
    int8_t *tab = reinterpret_cast<int8_t *>(stp + 2 * TA);  // [2][CPP][plane][half][TA][16] table planes
    int8_t *ohot = tab + 2 * BUF;                              // [16][16]: entry c is the one-hot of code c
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, half = lane >> 5, l32 = lane & 31;
    if (tid < 16) {
        const uint32_t one = 1u << (8 * (tid & 3)), d = tid >> 2;
        *reinterpret_cast<uint4 *>(ohot + tid * 16) =
            make_uint4(d == 0 ? one : 0u, d == 1 ? one : 0u, d == 2 ? one : 0u, d == 3 ? one : 0u);
    }

    int jb = 0;
#pragma unroll
    for (int k = 1; k < kKernargJobs; ++k)
        if (k < a.njobs && static_cast<int>(blockIdx.x) >= a.wg0[k]) jb = k;
    const JobDesc &J = a.jobs[jb];
    const int blk = (static_cast<int>(blockIdx.x) - a.wg0[jb]) * kMfmaWaves + w;  // this wavefront's block
    const bool rows_here = blk < J.nblk;
    const int gblk = J.blk0 + blk;
    const size_t bk = static_cast<size_t>(J.blk0 + min(blk, J.nblk - 1));  // clamped: loads need no branch
    const int t0 = blockIdx.y * TA;
    const int groups = J.groups, rows = J.rows, in = J.in, units = J.units;
    const long long xs = J.x_stride;
    const float *X = J.x, *XG = J.xgate, *NG = J.ngain;

    // Fused ZCRMSNorm of the activation rows (norm.go:53-109): divisors of
    // the workgroup's activations, four float64 partial sums each.
    __shared__ double zpart[4 * TA];
    __shared__ float zrms[TA];
    if (NG) {
        for (int e = tid; e < 4 * TA; e += kMfmaThreads) {
            const int t = t0 + e / 4;
            zpart[e] = t < rows ? zc_partial(X + static_cast<long long>(t) * xs, in, e % 4) : 0.0;
        }
        __syncthreads();
        for (int e = tid; e < TA; e += kMfmaThreads)
            zrms[e] = zc_rms(zpart[4 * e], zpart[4 * e + 1], zpart[4 * e + 2], zpart[4 * e + 3], in);
        __syncthreads();
    }

    // The wavefront's rows' index bytes, one 16-byte unit (2 chunks of 16
    // positions per 4-bit unit, 4 per 2-bit unit) a load, read one unit
    // ahead in a sequence that runs on across groups; the rows' norms of a
    // group, read one group ahead.
    auto load_unit = [&](int un, uint32_t (&d)[2][4]) {  // unit un of the row's units (group un / UPG)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const uint4 v = *reinterpret_cast<const uint4 *>(J.idx + ((bk * units + un) * 64 + rt * 32 + l32) * 16);
            d[rt][0] = v.x; d[rt][1] = v.y; d[rt][2] = v.z; d[rt][3] = v.w;
        }
    };
    auto load_norm = [&](int g, unsigned short (&d)[2]) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) d[rt] = J.norm[(bk * groups + g) * 64 + rt * 32 + l32];
    };
    // Values of group g of the wavefront's activations k0 .. k0 + n - 1 (of
    // its PW; two per lane each), with Attention.output's gate
    // (attention.go:245-249).
    auto load_x = [&](int g, int k0, auto n_c, float (&d)[decltype(n_c)::value][2]) {
        constexpr int NA = decltype(n_c)::value;
#pragma unroll
        for (int k = 0; k < NA; ++k) {
            const int t = t0 + w + (k0 + k) * kMfmaWaves;
            const long long ro = static_cast<long long>(min(t, rows - 1)) * xs;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int col = min(g * G + e * 64 + lane, in - 1);
                float xv = X[ro + col];
                if (XG) xv = xv * gate_sigmoid(XG[ro + col]);
                d[k][e] = (t < rows && g * G + e * 64 + lane < in) ? xv : 0.0f;
            }
        }
    };
    // Rotation and bound of group g of activations [k0, k0 + n) of the
    // wavefront's (lut.go:158-178): the norm, the plain FWHT in the
    // reference's stage order, lutInv; to av / stp of the group's parity.
    auto rotate = [&](int g, int k0, auto n_c, const float (&xv)[decltype(n_c)::value][2]) {
        constexpr int NA = decltype(n_c)::value;
        float v[NA][2];
#pragma unroll
        for (int k = 0; k < NA; ++k) {
            const int tt = w + (k0 + k) * kMfmaWaves, t = t0 + tt;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int col = g * G + e * 64 + lane;
                v[k][e] = xv[k][e];
                if (NG && t < rows && col < in) {
                    const float gx = NG[col] * v[k][e];
                    v[k][e] = gx / zrms[tt];
                }
            }
        }
#pragma unroll
        for (int h = 1; h < 64; h <<= 1) {  // stages h = 1 .. 32 across lanes (kernel.go:384-393)
#pragma unroll
            for (int k = 0; k < NA; ++k)
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const float p = xor_lane(v[k][e], h);
                    v[k][e] = (lane & h) ? p - v[k][e] : v[k][e] + p;
                }
        }
#pragma unroll
        for (int k = 0; k < NA; ++k) {  // stage h = 64 within the lane
            const float p = v[k][0], q = v[k][1];
            v[k][0] = p + q;
            v[k][1] = p - q;
        }
        float mx[NA];
#pragma unroll
        for (int k = 0; k < NA; ++k) {
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
            for (int k = 0; k < NA; ++k) mx[k] = go_max(mx[k], xor_lane(mx[k], off));
        float *avg = av + (g & 1) * TA * AP;
#pragma unroll
        for (int k = 0; k < NA; ++k) {
            const int tt = w + (k0 + k) * kMfmaWaves;
            const float m = J.cb_max * mx[k];
            const float inv = m > 0.0f ? static_cast<float>(kLutQ) / m : 0.0f;  // lutInv (lut.go:219-225)
#pragma unroll
            for (int e = 0; e < 2; ++e) avg[tt * AP + e * 64 + lane] = v[k][e] * inv;
            if (lane == 0) stp[(g & 1) * TA + tt] = m * J.lut_step;
        }
    };

    // Table items: this thread's are activation tid % TA at positions
    // jc0 + k * (kMfmaThreads / TA) of every chunk (NI per thread), both
    // planes to [buf][jc / 2][plane][jc % 2][activation], built a quarter
    // (four entries) at a time between the previous chunk's MFMAs.
    float cbv[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) cbv[q] = J.cb[q];
    const int tA = tid % TA, jc0 = tid / TA;
    float ix[NI][2];
    uint32_t blo[4], bhi[4];
    auto item_inputs = [&](int g, int c) {
        const float *avg = av + (g & 1) * TA * AP;
#pragma unroll
        for (int k = 0; k < NI; ++k) {
            const int j = c * CK + jc0 + k * (kMfmaThreads / TA);
            if constexpr (BITS == 4) {
                ix[k][0] = avg[tA * AP + j];
            } else {
                ix[k][0] = avg[tA * AP + 2 * j];
                ix[k][1] = avg[tA * AP + 2 * j + 1];
            }
        }
    };
    auto item_quarter = [&](int buf, int s) {  // quarter s & 3 of item s >> 2, into table buffer buf
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
            const int jc = jc0 + k * (kMfmaThreads / TA);
            int8_t *dst = tab + (buf * CPP + (jc >> 1)) * PAIR + ((jc & 1) * TA + tA) * 16;
            *reinterpret_cast<uint4 *>(dst) = make_uint4(blo[0], blo[1], blo[2], blo[3]);
            *reinterpret_cast<uint4 *>(dst + PLANE) = make_uint4(bhi[0], bhi[1], bhi[2], bhi[3]);
        }
    };

    // Prologue: group 0 rotated, its first chunk's tables built; group 1's
    // values, the first index unit and the norms on their way.
    uint32_t cur[2][4], nxt[2][4];
    unsigned short nrm16[2], nrm16n[2];
    load_unit(0, nxt);
    load_norm(0, nrm16);
    {
        float x0[PW][2];
        load_x(0, 0, std::integral_constant<int, PW>{}, x0);
        rotate(0, 0, std::integral_constant<int, PW>{}, x0);
    }
    if (groups > 1) load_norm(1, nrm16n);
    lds_barrier();
    item_inputs(0, 0);
#pragma unroll
    for (int s4 = 0; s4 < 4 * NI; ++s4) item_quarter(0, s4);
    lds_barrier();

    i32x16 acc[AT][2];     // [activation tile][row tile]
    float yv[AT][2][16];   // [activation tile][row tile][element]
#pragma unroll
    for (int at = 0; at < AT; ++at)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            acc[at][rt] = i32x16{};
#pragma unroll
            for (int i = 0; i < 16; ++i) yv[at][rt][i] = 0.0f;
        }

    // Chunks of CK positions, one sequence over all groups. Chunk q's
    // MFMAs, with chunk q + 1's items built between them and, in the first
    // NR chunks of group g, group g + 1 rotated APS activations a chunk. One
    // K step is a position pair (lane half h: position 2p + h); per pair and
    // row tile one one-hot B (1 at the code's byte) for the l plane and
    // B << 6 (64) for the h plane, into one accumulator. After a group's
    // last chunk its sums are folded into y, groups in order (lut.go:
    // 297-310).
    constexpr int CW = M::CW;      // index words per row and chunk
    constexpr int CPU = 4 / CW;    // chunks per unit
    const uint32_t hs = 4u * static_cast<uint32_t>(half);  // a lane half takes the odd nibbles
    const int nq = groups * NCH;
    for (int qq = 0; qq < nq; qq += CPU) {
        const int g = qq / NCH;
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int e = 0; e < 4; ++e) cur[rt][e] = nxt[rt][e];
        if (qq + CPU < nq) load_unit(qq / CPU + 1, nxt);  // units run on across groups: unit u is chunks CPU*u..
#pragma unroll
        for (int q = 0; q < CPU; ++q) {
            const int c = qq % NCH + q;  // chunk within group g
            // The slices of group g + 1 this chunk rotates after its MFMAs:
            // slice c, and in chunk NA - 1 also the slices past NA - 1. Their
            // values are read now, under the MFMAs.
            const bool rot = g + 1 < groups && c < (NS < NA ? NS : NA);
            float xr[MAXS][APS][2];
            if (rot) {
#pragma unroll
                for (int m = 0; m < MAXS; ++m) {
                    const int sl = m == 0 ? c : NA - 1 + m;
                    if (m == 0 || (c == NA - 1 && sl < NS))
                        load_x(g + 1, sl * APS, std::integral_constant<int, APS>{}, xr[m]);
                }
            }
            item_inputs((qq + q + 1) / NCH, (qq + q + 1) % NCH);
            // this half's nibble of pair k in the high nibble of byte k: an
            // entry's offset in the one-hot table is one SDWA and
            uint32_t wv[2][CW];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                for (int e = 0; e < CW; ++e) wv[rt][e] = (cur[rt][q * CW + e] >> hs) << 4;
            auto onehot_of = [&](int rt, int pp) -> i32x4 {
                const uint32_t w4 = wv[rt][pp >> 2];
                uint32_t off;
                switch (pp & 3) {
                    case 0: off = and_byte<0>(0xf0u, w4); break;
                    case 1: off = and_byte<1>(0xf0u, w4); break;
                    case 2: off = and_byte<2>(0xf0u, w4); break;
                    default: off = and_byte<3>(0xf0u, w4); break;
                }
                return *reinterpret_cast<const i32x4 *>(ohot + off);
            };
            const int buf = (qq + q) & 1;
            const int8_t *tb = tab + buf * BUF + (half * TA + l32) * 16;
            i32x4 Al[2][AT], Ah[2][AT], Bl[2][2];
#pragma unroll
            for (int at = 0; at < AT; ++at) {
                Al[0][at] = *reinterpret_cast<const i32x4 *>(tb + at * 512);
                Ah[0][at] = *reinterpret_cast<const i32x4 *>(tb + PLANE + at * 512);
            }
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) Bl[0][rt] = onehot_of(rt, 0);
#pragma unroll
            for (int pp = 0; pp < CPP; ++pp) {
                const int sl = pp & 1;
                if (pp + 1 < CPP) {
                    const int8_t *nb = tb + (pp + 1) * PAIR;
#pragma unroll
                    for (int at = 0; at < AT; ++at) {
                        Al[sl ^ 1][at] = *reinterpret_cast<const i32x4 *>(nb + at * 512);
                        Ah[sl ^ 1][at] = *reinterpret_cast<const i32x4 *>(nb + PLANE + at * 512);
                    }
#pragma unroll
                    for (int rt = 0; rt < 2; ++rt) Bl[sl ^ 1][rt] = onehot_of(rt, pp + 1);
                }
                __builtin_amdgcn_sched_barrier(0);  // the next pair's reads go out here
                // (past the last chunk the items land in the spare buffer and
                // go unread; a wavefront past the view's rows multiplies its
                // clamped rows and stores nothing)
                if (pp < 4 * NI) item_quarter(buf ^ 1, pp);
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    const i32x4 bh = Bl[sl][rt] << 6;  // 64 at the code's byte: the h plane's weight
#pragma unroll
                    for (int at = 0; at < AT; ++at) {
                        acc[at][rt] =
                            __builtin_amdgcn_mfma_i32_32x32x32_i8(Al[sl][at], Bl[sl][rt], acc[at][rt], 0, 0, 0);
                        acc[at][rt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(Ah[sl][at], bh, acc[at][rt], 0, 0, 0);
                    }
                }
#pragma unroll
                for (int m = 0; m < 4 * AT; ++m) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }

            if (rot) {
#pragma unroll
                for (int m = 0; m < MAXS; ++m) {
                    const int sl = m == 0 ? c : NA - 1 + m;
                    if (m == 0 || (c == NA - 1 && sl < NS))
                        rotate(g + 1, sl * APS, std::integral_constant<int, APS>{}, xr[m]);
                }
            }
            lds_barrier();
            if (c == NCH - 1) {
                // fold group g into y (lut.go:297-310); the next group's norms become current
                if (rows_here) {
                    const float *sg = stp + (g & 1) * TA;
                    float nrm[2];
#pragma unroll
                    for (int rt = 0; rt < 2; ++rt) nrm[rt] = __half2float(__ushort_as_half(nrm16[rt]));
#pragma unroll
                    for (int at = 0; at < AT; ++at)
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            const float step = sg[at * 32 + (i >> 2) * 8 + half * 4 + (i & 3)];
#pragma unroll
                            for (int rt = 0; rt < 2; ++rt) {
                                const int sum = acc[at][rt][i];
                                const float coef = nrm[rt] * step;
                                const float prod = static_cast<float>(sum) * coef;
                                yv[at][rt][i] = yv[at][rt][i] + prod;
                            }
                        }
                }
#pragma unroll
                for (int at = 0; at < AT; ++at)
#pragma unroll
                    for (int rt = 0; rt < 2; ++rt) acc[at][rt] = i32x16{};
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) nrm16[rt] = nrm16n[rt];
                if (g + 2 < groups) load_norm(g + 2, nrm16n);
            }
        }
    }

    if (rows_here) {
#pragma unroll
        for (int at = 0; at < AT; ++at)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int t = t0 + at * 32 + (i >> 2) * 8 + half * 4 + (i & 3);
                if (t >= rows) continue;
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

// The MFMA form holds two groups' rotated values and steps (the next one is
// rotated while the current one streams).
template <int BITS, int TA>
size_t mfma_lds_bytes2() {
    using M = MfmaGeo<BITS>;
    return sizeof(float) * 2 * (TA * M::AP + TA) + static_cast<size_t>(2) * M::CK * 2 * TA * 16 + 16 * 16;
}

template <int BITS, int TA>
hipError_t launch_mfma_t(const LutLaunch &a, int wg, int act_tiles, hipStream_t s) {
    static std::atomic<unsigned long long> attr{0};
    const size_t lds = mfma_lds_bytes2<BITS, TA>();
    if (hipError_t e = lds_limit_once(reinterpret_cast<const void *>(&lut_mfma_kernel<BITS, TA>), static_cast<int>(lds),
                                      attr))
        return e;
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


// A job's epilogue fields, read from the kernel arguments once (each use of
// a JobDesc field indexed by a run-time job is a scalar load and a wait).
struct Epilogue {
    int8_t *app_q;
    float *app_s;
    long long app_q_stride, app_s_stride;
    const int32_t *app_pos;
    const float *app_cos, *app_sin;
    int app_cap;
    const float *resid;
    long long resid_stride;
    float *y;
    long long y_stride;
    int act, row0, out, blk0;
    __device__ explicit Epilogue(const JobDesc &J)
        : app_q(J.app_q), app_s(J.app_s), app_q_stride(J.app_q_stride), app_s_stride(J.app_s_stride),
          app_pos(J.app_pos), app_cos(J.app_cos), app_sin(J.app_sin), app_cap(J.app_cap), resid(J.resid),
          resid_stride(J.resid_stride), y(J.y), y_stride(J.y_stride), act(J.act), row0(J.row0), out(J.out),
          blk0(J.blk0) {}
};

// The lut kernel's epilogue for activations t0 .. t0 + nt - 1 of one 64-row
// block (lane = row), FA of them computed together so that their lane
// reductions and divides overlap: the int8 append of the block as a head
// (Int8Rows.Append, int8.go:36-55, after RoPE at the stream's position,
// rope.go:69-81), and y, with the residual add or SiLU, for the view's rows.
// The memory operands come preloaded: p the streams' positions (app_q), c
// and s the RoPE rows' cosine and sine of the lane's pair (app_cos), rv the
// residuals (resid).
template <int FA>
__device__ __forceinline__ void fold_epilogue(const Epilogue &J, int t0, int nt, int blk, int lane, const float *y,
                                              const int *p, const float *c, const float *s, const float *rv) {
    const int row = (J.blk0 + blk) * 64;  // root row of lane 0
    if (J.app_q) {
        float v[FA], m[FA];
#pragma unroll
        for (int k = 0; k < FA; ++k) {
            v[k] = y[k];
            if (J.app_cos) {
                const float o = xor_lane<32>(v[k]);
                const float x1 = lane < 32 ? v[k] : o, x2 = lane < 32 ? o : v[k];
                float o1, o2;
                rope_pair(x1, x2, c[k], s[k], o1, o2);
                v[k] = lane < 32 ? o1 : o2;
            }
            m[k] = fabsf(v[k]);
        }
#pragma unroll
        for (int h = 32; h > 0; h >>= 1)
#pragma unroll
            for (int k = 0; k < FA; ++k) m[k] = go_max(m[k], xor_lane(m[k], h));
        const int r0 = row - J.row0;  // view row of the head's first value
#pragma unroll
        for (int k = 0; k < FA; ++k) {
            const float sc = m[k] > 0.0f ? m[k] / 127.0f : 1.0f;
            const int8_t code = static_cast<int8_t>(go_int8_code(rintf(v[k] / sc)));
            const int t = t0 + k;
            if (k < nt && p[k] >= 0 && p[k] < J.app_cap) {
                J.app_q[static_cast<long long>(t) * J.app_q_stride + static_cast<long long>(p[k]) * J.out + r0 + lane] =
                    code;
                if (lane == 0)
                    J.app_s[static_cast<long long>(t) * J.app_s_stride + static_cast<long long>(p[k]) * (J.out >> 6) +
                            (r0 >> 6)] = sc;
            }
        }
    }
    const int r = row + lane;
    if (r >= J.row0 && r < J.row0 + J.out) {
#pragma unroll
        for (int k = 0; k < FA; ++k) {
            if (k >= nt) break;
            float out = y[k];
            if (J.resid)
                out = rv[k] + out;
            else if (J.act == 1)
                out = silu_value(out);
            J.y[static_cast<long long>(t0 + k) * J.y_stride + (r - J.row0)] = out;
        }
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

// The fold of the split form: a wavefront per (activation, 256 rows), four
// rows per lane (16 lanes a 64-row block), the terms read as 16-byte
// vectors: y = 0, then y = y + term[g] for g in order (lut.go:297-310),
// then the lut kernel's epilogue: the int8 append of each block as a head
// (Int8Rows.Append, int8.go:36-55, after RoPE at the stream's position,
// rope.go:69-81; row i < 32 pairs with i + 32, lane q with lane q + 8), and
// y, with the residual add or SiLU, for the view's rows.
__global__ __launch_bounds__(256) void mfma_fold_kernel(LutLaunch a) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int jb = 0;
#pragma unroll
    for (int k = 1; k < kKernargJobs; ++k)
        if (k < a.njobs && static_cast<int>(blockIdx.x) >= a.fold0[k]) jb = k;
    const JobDesc &J = a.jobs[jb];
    const int q = lane & 15;
    const int blk = (static_cast<int>(blockIdx.x) - a.fold0[jb]) * 4 + (lane >> 4);
    const int t = blockIdx.y * 4 + w;
    if (blk >= J.nblk || t >= J.rows) return;  // whole 16-lane blocks leave together
    const long long rs = static_cast<long long>(J.nblk) * 64, gs = static_cast<long long>(J.rows) * rs;
    const float *tp = a.term[jb] + static_cast<long long>(t) * rs + blk * 64 + 4 * q;
    float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int g = 0; g < J.groups; ++g) {
        const float4 v = *reinterpret_cast<const float4 *>(tp + g * gs);
        y[0] = y[0] + v.x;
        y[1] = y[1] + v.y;
        y[2] = y[2] + v.z;
        y[3] = y[3] + v.w;
    }

    const int row = (J.blk0 + blk) * 64;  // root row of the block's first value
    if (J.app_q) {
        const int p = J.app_pos[t];
        if (p >= 0 && p < J.app_cap) {
            float v[4] = {y[0], y[1], y[2], y[3]};
            if (J.app_cos) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float o = xor_lane<8>(v[e]);
                    const int jj = (4 * q + e) & 31;
                    const float x1 = q < 8 ? v[e] : o, x2 = q < 8 ? o : v[e];
                    float o1, o2;
                    rope_pair(x1, x2, J.app_cos[p * 32 + jj], J.app_sin[p * 32 + jj], o1, o2);
                    v[e] = q < 8 ? o1 : o2;
                }
            }
            float m = go_max(go_max(fabsf(v[0]), fabsf(v[1])), go_max(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
            for (int h = 8; h > 0; h >>= 1) m = go_max(m, xor_lane(m, h));
            const float sc = m > 0.0f ? m / 127.0f : 1.0f;
            const int r0 = row - J.row0;  // view row of the head's first value
            int8_t *qp = J.app_q + static_cast<long long>(t) * J.app_q_stride + static_cast<long long>(p) * J.out + r0;
#pragma unroll
            for (int e = 0; e < 4; ++e) qp[4 * q + e] = static_cast<int8_t>(go_int8_code(rintf(v[e] / sc)));
            if (q == 0)
                J.app_s[static_cast<long long>(t) * J.app_s_stride + static_cast<long long>(p) * (J.out >> 6) +
                        (r0 >> 6)] = sc;
        }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int r = row + 4 * q + e;
        if (r >= J.row0 && r < J.row0 + J.out) {
            float out = y[e];
            if (J.resid)
                out = J.resid[static_cast<long long>(t) * J.resid_stride + (r - J.row0)] + out;
            else if (J.act == 1)
                out = silu_value(out);
            J.y[static_cast<long long>(t) * J.y_stride + (r - J.row0)] = out;
        }
    }
}

template <int BITS>
hipError_t launch_split_t(const LutLaunch &a, int grid, hipStream_t s) {
    const size_t lds = mfma_lds_bytes<BITS, kSplitTa>();
    hipLaunchKernelGGL((lut_mfma_split_kernel<BITS>), dim3(grid), dim3(kSplitThreads), lds, s, a);
    return hipGetLastError();
}

// ---- The table form: tables built once per activation, MFMAs over them ----
//
// At some hundred activations (the decode step's batch) the MFMA forms
// rebuild an activation tile's tables in every row tile's workgroup, and the
// lut kernel looks every entry up once per activation. The table form
// builds each activation's tables once: lut_tables_kernel rotates and
// bounds each (activation, group) and writes the int8 planes of its 16-entry
// tables, in the A-operand order of v_mfma_i32_32x32x32_i8, and the group's
// step; lut_mfma_tab_kernel streams them into the MFMAs of every row tile,
// 64 rows x 32 activations a workgroup, its four wavefronts taking the
// groups in turn. The arithmetic is the split form's, so the result is bit
// for bit the lut kernel's.
constexpr int kTabWaves = 4;      // wavefronts per workgroup of the product
constexpr int kTabDepth = 4;      // position pairs of A operands in flight per wavefront
constexpr int kTabMaxGroups = 16;  // groups whose terms the product's LDS holds
constexpr int kTabPre4Rows = 3072;  // activations up to which the pre-pass takes 4 a workgroup

// The pre-pass: a workgroup per TT activations (4 or 8) and one group g.
// Wavefront w rotates activations w, w + 4, ... (two values per lane), then
// every thread builds items (an activation's 16 entries at one position,
// both planes): threads TT j .. TT j + TT - 1 take position j (and j + 256 /
// TT, ...) of the TT activations, so each plane write of TT threads is 16 TT
// contiguous bytes. Measured on MI355X: 4 activations a workgroup (twice
// the workgroups) make the batch-256 decode step's table-form products 1-1.5
// us faster each (the norm's in-order float64 chains run on twice the CUs)
// and lose at 12,000 activations (2048x512 CQ4 376 -> 392 us).
template <int BITS, int TT>
__global__ __launch_bounds__(256) void lut_tables_kernel(TabArgs a) {
    using M = MfmaGeo<BITS>;
    constexpr int G = M::G, AP = M::AP, NJ = M::NJ, NP = NJ / 2, PW = TT / 4, PS = 256 / TT;
    static_assert(TT % 4 == 0 && NJ % PS == 0, "positions per pass");
    __shared__ float av[TT * AP];      // scaled rotated groups
    __shared__ double stage[TT * 512];  // the norm's squares, 512 columns at a time
    __shared__ double zpart[4 * TT];
    __shared__ float zrms[TT];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = blockIdx.y, t0 = blockIdx.x * TT;
    const int rows = a.rows, in = a.in;
    const long long xs = a.x_stride;
    const float *X = a.x, *XG = a.xgate, *NG = a.ngain;

    // first loads without branches: rows past the activations and columns
    // past the row read clamped addresses and go unused; with no gate the
    // gate loads read x
    const float *GP = XG ? XG : X;
    float v[PW][2], gv[PW][2];
#pragma unroll
    for (int k = 0; k < PW; ++k) {
        const long long rowoff = static_cast<long long>(min(t0 + w + 4 * k, rows - 1)) * xs;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int col = min(g * G + e * 64 + lane, in - 1);
            v[k][e] = X[rowoff + col];
            gv[k][e] = GP[rowoff + col];
        }
    }
#pragma unroll
    for (int k = 0; k < PW; ++k)
#pragma unroll
        for (int e = 0; e < 2; ++e)
            if (!(t0 + w + 4 * k < rows && g * G + e * 64 + lane < in)) v[k][e] = 0.0f;

    // ZCRMSNorm divisors of the 8 activations over their whole rows
    // (norm.go:53-109): four float64 partial sums over i mod 4, each in
    // order. A round of 512 columns: every thread squares its columns
    // (float64 of a float squared is exact) into LDS by partial, then a
    // thread per (activation, partial) adds its 128 squares in order.
    if (NG) {
        const int full = in & ~3;
        const int ct = tid >> 2, ck = tid & 3;  // chain thread (tid < 4 * TT): activation, partial
        double s = 0.0;
        for (int p0 = 0; p0 < full; p0 += 512) {
            float st[2][TT];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < TT; ++r)
                    st[h][r] = X[static_cast<long long>(min(t0 + r, rows - 1)) * xs + min(p0 + h * 256 + tid, full - 1)];
            // column p0 + 256h + tid is value 64h + tid / 4 of partial tid mod 4: [r][partial][128]
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < TT; ++r) {
                    const double d = st[h][r];
                    stage[r * 512 + (tid & 3) * 128 + h * 64 + (tid >> 2)] = d * d;
                }
            __syncthreads();
            if (tid < 4 * TT) {
                const int n4 = min(512, full - p0) >> 2;  // the partial's values this round, in order
                const double2 *sp = reinterpret_cast<const double2 *>(stage + ct * 512 + ck * 128);
                if (n4 == 128) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        double2 dd[16];
#pragma unroll
                        for (int i = 0; i < 16; ++i) dd[i] = sp[q * 16 + i];
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            s = s + dd[i].x;
                            s = s + dd[i].y;
                        }
                    }
                } else {
                    for (int i = 0; i < n4; ++i) s = s + stage[ct * 512 + ck * 128 + i];
                }
            }
            __syncthreads();
        }
        if (tid < 4 * TT) {
            if (ck == 0 && t0 + ct < rows)
                for (int c = full; c < in; ++c) {
                    const double d = X[static_cast<long long>(t0 + ct) * xs + c];
                    s = s + d * d;
                }
            zpart[tid] = s;
        }
        __syncthreads();
        if (tid < TT) zrms[tid] = zc_rms(zpart[4 * tid], zpart[4 * tid + 1], zpart[4 * tid + 2], zpart[4 * tid + 3], in);
        __syncthreads();
    }

    // Gate, norm, rotation and bound (lut.go:158-178, 219-225), as the
    // split form.
#pragma unroll
    for (int k = 0; k < PW; ++k) {
        const int tt = w + 4 * k, t = t0 + tt;
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
            const int tt = w + 4 * k, t = t0 + tt;
            const float m = a.cb_max * mx[k];
            const float inv = m > 0.0f ? static_cast<float>(kLutQ) / m : 0.0f;  // lutInv (lut.go:219-225)
#pragma unroll
            for (int e = 0; e < 2; ++e) av[tt * AP + e * 64 + lane] = v[k][e] * inv;
            if (lane == 0) a.stp[(static_cast<size_t>(t >> 5) * a.groups + g) * 32 + (t & 31)] = m * a.lut_step;
        }
    }
    __syncthreads();

    // Items (lutTables4Generic / lutTables2Generic, lut.go:239-282).
    float cbv[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) cbv[q] = a.cb[q];
    const int tt = tid % TT, jb = tid / TT, t = t0 + tt;
    int8_t *base = a.tab + (static_cast<size_t>(t >> 5) * a.groups + g) * NP * 2048 + (t & 31) * 16;
#pragma unroll
    for (int k = 0; k < NJ / PS; ++k) {
        const int j = jb + PS * k;
        float x0, x1 = 0.0f;
        if constexpr (BITS == 4) {
            x0 = av[tt * AP + j];
        } else {
            x0 = av[tt * AP + 2 * j];
            x1 = av[tt * AP + 2 * j + 1];
        }
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            uint32_t b[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int code = 4 * qd + q;
                if constexpr (BITS == 4) {
                    b[q] = rne_bits(cbv[code] * x0);
                } else {  // code = hi << 2 | lo
                    const float l = cbv[code & 3] * x0, h = cbv[code >> 2] * x1;
                    const float sm = l + h;
                    b[q] = rne_bits(sm);
                }
            }
            planes4(b[0], b[1], b[2], b[3], lo[qd], hi[qd]);
        }
        int8_t *dst = base + (j >> 1) * 2048 + (j & 1) * 512;  // [pair][plane][half][32][16]
        *reinterpret_cast<uint4 *>(dst) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        *reinterpret_cast<uint4 *>(dst + 1024) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    }
}

// The product: a workgroup per (64-row block, 32-activation tile), a
// tile's workgroups on one XCD (or two), which shares their tables in its L2.
// Wavefront w takes groups w, w + 4, ...: per position pair it reads the
// pair's two A planes (1 KiB each, kTabDepth pairs ahead), builds the
// one-hots of its two 32-row tiles and runs 4 MFMAs; at the group's end its
// terms float32(S) * (norm * step) go to LDS [group][activation][row]. Then
// wavefront w folds activations 8w .. 8w + 7 (lane = row) in group order
// from 0 (lut.go:297-310) and runs the lut kernel's epilogue.
template <int BITS>
__global__ __launch_bounds__(64 * kTabWaves) void lut_mfma_tab_kernel(LutLaunch a) {
    using M = MfmaGeo<BITS>;
    constexpr int NP = M::NJ / 2, D = kTabDepth, TP = 64;
    extern __shared__ __align__(16) unsigned char smem[];
    float *terms = reinterpret_cast<float *>(smem);  // [groups][32][TP]
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, half = lane >> 5, l32 = lane & 31;
    const int nat = a.tab_at;
    const int L = blockIdx.x;
    // workgroup L runs on XCD L % 8 (dispatch goes round the XCDs), as its
    // (L / 8)-th there. The (tile, row block) items, tile by tile, are cut
    // into 8 equal runs, one per XCD: an XCD's workgroups take the row blocks
    // of one tile one after the other, so that its tables stay in that L2
    // while they run, and every XCD has the same share of the work
    const int nb = a.tab_nb, total = nat * nb, per = (total + 7) / 8;
    const int k8 = L >> 3, item = (L & 7) * per + k8;
    if (k8 >= per || item >= total) return;  // the whole workgroup
    const int at = item / nb, rb = item % nb;
    int jb = 0;
#pragma unroll
    for (int k = 1; k < kKernargJobs; ++k)
        if (k < a.njobs && rb >= a.wg0[k]) jb = k;
    const JobDesc &J = a.jobs[jb];
    const int blk = rb - a.wg0[jb];
    if (blk >= J.nblk) return;  // the whole workgroup
    const int groups = J.groups, units = J.units;
    int8_t *ohot = reinterpret_cast<int8_t *>(terms + groups * 32 * TP);  // [16][16]: entry c is the one-hot of c
    if (tid < 16) {
        const uint32_t one = 1u << (8 * (tid & 3)), d = tid >> 2;
        *reinterpret_cast<uint4 *>(ohot + tid * 16) =
            make_uint4(d == 0 ? one : 0u, d == 1 ? one : 0u, d == 2 ? one : 0u, d == 3 ? one : 0u);
    }
    const size_t bk = static_cast<size_t>(J.blk0 + blk);
    const uint8_t *IDX = J.idx;
    const uint32_t hs = 4u * static_cast<uint32_t>(half);  // a lane half takes the odd nibbles
    bool first = true;
    // the epilogue's operands for the wavefront's fold activations (t0 + k,
    // clamped to the activations), loaded now so that they are in registers
    // by the fold: positions and residuals here, the RoPE rows after the
    // products
    constexpr int FA = 32 / kTabWaves;
    const Epilogue E(J);
    const int t0 = at * 32 + w * FA, nt = min(FA, J.rows - t0);
    const int rview = min(max((E.blk0 + blk) * 64 + lane - E.row0, 0), E.out - 1);  // the lane's view row, clamped
    int pk[FA];
    float rv[FA], cv[FA], sv[FA];
#pragma unroll
    for (int k = 0; k < FA; ++k) {
        const long long tk = min(t0 + k, J.rows - 1);
        pk[k] = E.app_q ? E.app_pos[tk] : -1;
        rv[k] = E.resid ? E.resid[tk * E.resid_stride + rview] : 0.0f;
    }

    for (int g = w; g < groups; g += kTabWaves) {
        const int8_t *A = a.tab + (static_cast<size_t>(at) * groups + g) * NP * 2048 + lane * 16;
        i32x4 Al[D], Ah[D];
#pragma unroll
        for (int p = 0; p < D; ++p) {
            Al[p] = *reinterpret_cast<const i32x4 *>(A + p * 2048);
            Ah[p] = *reinterpret_cast<const i32x4 *>(A + p * 2048 + 1024);
        }
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
        for (int rt = 0; rt < 2; ++rt) nrm16[rt] = J.norm[(bk * groups + g) * 64 + rt * 32 + l32];
        // the steps of the lane's 16 accumulator activations (used at the
        // group's end)
        float st[16];
        const float *SP = a.tstp + (static_cast<size_t>(at) * groups + g) * 32 + half * 4;
#pragma unroll
        for (int i = 0; i < 16; ++i) st[i] = SP[(i >> 2) * 8 + (i & 3)];
        __builtin_amdgcn_sched_barrier(0);
        if (first) {
            lds_barrier();  // the one-hot table is whole
            first = false;
        }
        // this half's nibble of pair k in the high nibble of byte k: a
        // one-hot's offset in the table is one SDWA and
#pragma unroll
        for (int u = 0; u < M::UPG; ++u)
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                for (int e = 0; e < 4; ++e) idx[u][rt][e] = (idx[u][rt][e] >> hs) << 4;
        auto onehot = [&](int rt, int pp) -> i32x4 {
            const uint32_t w4 = idx[pp >> 4][rt][(pp >> 2) & 3];
            uint32_t off;
            switch (pp & 3) {
                case 0: off = and_byte<0>(0xf0u, w4); break;
                case 1: off = and_byte<1>(0xf0u, w4); break;
                case 2: off = and_byte<2>(0xf0u, w4); break;
                default: off = and_byte<3>(0xf0u, w4); break;
            }
            return *reinterpret_cast<const i32x4 *>(ohot + off);
        };
        i32x4 B[2][2];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) B[0][rt] = onehot(rt, 0);
        i32x16 accl[2] = {i32x16{}, i32x16{}}, acch[2] = {i32x16{}, i32x16{}};
#pragma unroll
        for (int pp = 0; pp < NP; ++pp) {
            const int s = pp % D, sb = pp & 1;
            if (pp + 1 < NP) {
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) B[sb ^ 1][rt] = onehot(rt, pp + 1);
            }
            __builtin_amdgcn_sched_barrier(0);  // the next pair's one-hot reads go out before these MFMAs
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
                accl[rt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(Al[s], B[sb][rt], accl[rt], 0, 0, 0);
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
                acch[rt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(Ah[s], B[sb][rt], acch[rt], 0, 0, 0);
            // the slot's next pair goes out here, kTabDepth pairs before its
            // use (the compiler would otherwise move the loads next to it)
            __builtin_amdgcn_sched_barrier(0);
            if (pp + D < NP) {
                Al[s] = *reinterpret_cast<const i32x4 *>(A + (pp + D) * 2048);
                Ah[s] = *reinterpret_cast<const i32x4 *>(A + (pp + D) * 2048 + 1024);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        float nrm[2];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) nrm[rt] = __half2float(__ushort_as_half(nrm16[rt]));
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int tt = (i >> 2) * 8 + half * 4 + (i & 3);
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                const int sum = accl[rt][i] + 64 * acch[rt][i];
                const float coef = nrm[rt] * st[i];
                terms[(g * 32 + tt) * TP + rt * 32 + l32] = static_cast<float>(sum) * coef;
            }
        }
    }
    if (first) lds_barrier();  // a wavefront without groups still meets the table barrier
#pragma unroll
    for (int k = 0; k < FA; ++k) {
        cv[k] = sv[k] = 0.0f;
        if (E.app_cos) {
            const int pc = pk[k] >= 0 && pk[k] < E.app_cap ? pk[k] : 0;
            cv[k] = E.app_cos[pc * 32 + (lane & 31)];
            sv[k] = E.app_sin[pc * 32 + (lane & 31)];
        }
    }
    __syncthreads();

    // The fold: wavefront w's 8 activations together, lane = row.
    float y[FA];
#pragma unroll
    for (int k = 0; k < FA; ++k) y[k] = 0.0f;
    for (int g = 0; g < groups; ++g) {
        const float *tp = terms + (g * 32 + w * FA) * TP + lane;
        float v[FA];
#pragma unroll
        for (int k = 0; k < FA; ++k) v[k] = tp[k * TP];
#pragma unroll
        for (int k = 0; k < FA; ++k) y[k] = y[k] + v[k];
    }
    fold_epilogue<FA>(E, t0, nt, blk, lane, y, pk, cv, sv, rv);
}

// The table form at large grids: a workgroup per (slab of kSaBlocks row
// blocks, 32-activation tile), wavefront w on block w of the slab, every
// group in turn. The tile's A operands (its tables, contiguous [group][pair]
// [plane][1 KiB]) stream once per workgroup through an LDS ring of kSaSlots
// slots of kSaPairs pairs (global_load_lds, two slots ahead) and all four
// wavefronts read them there: a quarter of lut_mfma_tab_kernel's L2 -> CU
// traffic, where every wavefront streams its own. The block's index units,
// norms and the group's steps also come by DMA, a group ahead, so that no
// load the compiler tracks is in flight in the loop (it would wait for the
// DMAs behind it). Each wavefront folds its rows' terms in registers in
// group order from 0 (lut.go:297-310), then runs the lut kernel's epilogue
// on its block.
constexpr int kSaPairs = 8;   // position pairs per ring slot (16 KiB)
constexpr int kSaSlots = 3;   // ring slots: kSaSlots - 1 in flight while one is read
constexpr int kSaAhead = kSaSlots - 1;
constexpr int kSaBlocks = 4;  // row blocks per workgroup, one per wavefront
constexpr int kSaSlot = kSaPairs * 2048;
constexpr int kSaDma = kSaSlot / 4096;  // a wavefront's 16-byte DMA loads per slot

// LDS byte offset of a shared-memory pointer (M0 and the DS instructions take it).
__device__ __forceinline__ unsigned sa_lds(const void *p) {
    return static_cast<unsigned>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char *)(p)));
}
// One 16-byte (or 4-byte) global load per active lane straight into LDS:
// lane l's bytes land at m0 + 16 l (4 l). Plain loads: the tables are read
// again by the tile's other slabs.
__device__ __forceinline__ void sa_dma16(const void *src, unsigned m0) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}
__device__ __forceinline__ void sa_dma4(const void *src, unsigned m0) {
    asm volatile("global_load_lds_dword %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}
// s_waitcnt vmcnt(n), n <= 15 (gfx9 encoding; lgkm and exp counts untouched).
__device__ __forceinline__ void sa_wait_vm(int n) {
    switch (n) {
#define CQ_SA_WAIT(K) \
    case K: __builtin_amdgcn_s_waitcnt((K) | (7 << 4) | (15 << 8)); break;
        CQ_SA_WAIT(0) CQ_SA_WAIT(1) CQ_SA_WAIT(2) CQ_SA_WAIT(3) CQ_SA_WAIT(4) CQ_SA_WAIT(5) CQ_SA_WAIT(6)
        CQ_SA_WAIT(7) CQ_SA_WAIT(8) CQ_SA_WAIT(9) CQ_SA_WAIT(10) CQ_SA_WAIT(11) CQ_SA_WAIT(12) CQ_SA_WAIT(13)
        CQ_SA_WAIT(14) CQ_SA_WAIT(15)
#undef CQ_SA_WAIT
        default: __builtin_amdgcn_s_waitcnt((0) | (7 << 4) | (15 << 8)); break;
    }
}

template <int BITS>
constexpr size_t sa_lds_bytes() {
    return static_cast<size_t>(kSaSlots) * kSaSlot + kSaBlocks * MfmaGeo<BITS>::UPG * 1024 + kSaBlocks * 128 +
           kSaBlocks * 128 + 256;
}

template <int BITS>
__global__ __launch_bounds__(64 * kSaBlocks, 2) void lut_mfma_tabs_kernel(LutLaunch a) {
    using M = MfmaGeo<BITS>;
    constexpr int NP = M::NJ / 2, SPG = NP / kSaPairs, UPG = M::UPG, AUX = UPG + 2;
    // a group's aux loads go out at its second step and must be older than
    // the next group's first slot
    static_assert(NP % kSaPairs == 0 && SPG >= kSaAhead + 2, "a group's steps");
    static_assert(kSaDma * (kSaAhead - 1) + AUX <= 15, "the wait counts fit sa_wait_vm");
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned char *ring = smem;                                            // [slot][pair][plane][64][16]
    unsigned char *idxl = ring + kSaSlots * kSaSlot;                       // [wave][unit][64 rows][16]
    unsigned char *nrml = idxl + kSaBlocks * UPG * 1024;                   // [wave][64 fp16 norms]
    unsigned char *stpl = nrml + kSaBlocks * 128;                          // [wave][32 steps]
    int8_t *ohot = reinterpret_cast<int8_t *>(stpl + kSaBlocks * 128);     // [16][16]: entry c is the one-hot of c
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, half = lane >> 5, l32 = lane & 31;
    const int nat = a.tab_at, L = blockIdx.x;
    // workgroup L on XCD L % 8 as its (L / 8)-th; the (tile, slab) items,
    // tile by tile, in 8 equal runs, one per XCD (as lut_mfma_tab_kernel)
    const int nb = a.tab_nb, total = nat * nb, per = (total + 7) / 8;
    const int k8 = L >> 3, item = (L & 7) * per + k8;
    if (k8 >= per || item >= total) return;  // the whole workgroup
    const int at = item / nb, rb = item % nb;
    int jb = 0;
#pragma unroll
    for (int k = 1; k < kKernargJobs; ++k)
        if (k < a.njobs && rb >= a.wg0[k]) jb = k;
    const JobDesc &J = a.jobs[jb];
    const int blkS = (rb - a.wg0[jb]) * kSaBlocks;  // the slab's first block (job-relative)
    if (blkS >= J.nblk) return;                     // the whole workgroup
    const int nbh = min(kSaBlocks, J.nblk - blkS);
    const bool mine = w < nbh;                       // a wavefront past the job's blocks reads block nbh - 1, unused
    const int blk = blkS + (mine ? w : nbh - 1);
    const size_t bk = static_cast<size_t>(J.blk0 + blk);
    const int groups = J.groups, units = J.units, nsteps = groups * SPG;
    if (tid < 16) {
        const uint32_t one = 1u << (8 * (tid & 3)), d = tid >> 2;
        *reinterpret_cast<uint4 *>(ohot + tid * 16) =
            make_uint4(d == 0 ? one : 0u, d == 1 ? one : 0u, d == 2 ? one : 0u, d == 3 ? one : 0u);
    }
    const int8_t *T = a.tab + static_cast<size_t>(at) * groups * NP * 2048;  // the tile's A operands
    const uint8_t *IDX = J.idx;
    // the ring's step k: kSaSlot bytes of T into slot k % kSaSlots, 1 KiB a wavefront load
    auto dma_step = [&](int k) {
        const int8_t *src = T + static_cast<size_t>(k) * kSaSlot + w * 1024 + lane * 16;
        const unsigned m0 = sa_lds(ring + (k % kSaSlots) * kSaSlot + w * 1024);
#pragma unroll
        for (int r = 0; r < kSaDma; ++r) sa_dma16(src + r * 4096, m0 + r * 4096);
    };
    // group g's index units, norms and steps for this wavefront's block (AUX loads)
    auto dma_aux = [&](int g) {
#pragma unroll
        for (int u = 0; u < UPG; ++u)
            sa_dma16(IDX + ((bk * units + static_cast<size_t>(g) * UPG + u) * 64 + lane) * 16,
                     sa_lds(idxl + (w * UPG + u) * 1024));
        if (lane < 32) {
            sa_dma4(reinterpret_cast<const char *>(J.norm + (bk * groups + g) * 64) + lane * 4, sa_lds(nrml + w * 128));
            sa_dma4(a.tstp + (static_cast<size_t>(at) * groups + g) * 32 + lane, sa_lds(stpl + w * 128));
        }
    };
    dma_aux(0);
    for (int k = 0; k < kSaAhead && k < nsteps; ++k) dma_step(k);

    const uint32_t hs = 4u * static_cast<uint32_t>(half);  // a lane half takes the odd nibbles
    float y[2][16];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int i = 0; i < 16; ++i) y[rt][i] = 0.0f;
    for (int g = 0; g < groups; ++g) {
        uint32_t idx[UPG][2][4];
        unsigned short nrm16[2];
        float st[16];
        i32x16 accl[2] = {i32x16{}, i32x16{}}, acch[2] = {i32x16{}, i32x16{}};
        const bool aux_next = g + 1 < groups;
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            const int k = g * SPG + s;
            // step k's slot (and, at s = 0, the group's aux loads, older) has
            // landed once only the loads issued after it are in flight: steps
            // k + 1 .. k + kSaAhead - 1, and the next group's aux loads (issued
            // at s = 1, behind step 1 + kSaAhead's) until step 1 + kSaAhead
            sa_wait_vm(kSaDma * min(kSaAhead - 1, nsteps - 1 - k) +
                       (s >= 2 && s <= kSaAhead + 1 && aux_next ? AUX : 0));
            lds_barrier();  // every wavefront's share has landed; slot (k - 1) % kSaSlots is read out
            if (k + kSaAhead < nsteps) dma_step(k + kSaAhead);
            if (s == 0) {
#pragma unroll
                for (int u = 0; u < UPG; ++u)
#pragma unroll
                    for (int rt = 0; rt < 2; ++rt) {
                        const uint4 v = *reinterpret_cast<const uint4 *>(idxl + (w * UPG + u) * 1024 + (rt * 32 + l32) * 16);
                        idx[u][rt][0] = (v.x >> hs) << 4;
                        idx[u][rt][1] = (v.y >> hs) << 4;
                        idx[u][rt][2] = (v.z >> hs) << 4;
                        idx[u][rt][3] = (v.w >> hs) << 4;
                    }
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
                    nrm16[rt] = reinterpret_cast<const unsigned short *>(nrml + w * 128)[rt * 32 + l32];
                const float *sp = reinterpret_cast<const float *>(stpl + w * 128) + half * 4;
#pragma unroll
                for (int i = 0; i < 16; ++i) st[i] = sp[(i >> 2) * 8 + (i & 3)];
            }
            if (s == 1 && aux_next) dma_aux(g + 1);  // the buffers were read out at s = 0 (barrier between)
            // this half's nibble of pair pp in the high nibble of byte pp: a
            // one-hot's offset in the table is one SDWA and
            auto onehot = [&](int rt, int pp) -> i32x4 {
                const uint32_t w4 = idx[pp >> 4][rt][(pp >> 2) & 3];
                uint32_t off;
                switch (pp & 3) {
                    case 0: off = and_byte<0>(0xf0u, w4); break;
                    case 1: off = and_byte<1>(0xf0u, w4); break;
                    case 2: off = and_byte<2>(0xf0u, w4); break;
                    default: off = and_byte<3>(0xf0u, w4); break;
                }
                return *reinterpret_cast<const i32x4 *>(ohot + off);
            };
            const unsigned char *sl = ring + (k % kSaSlots) * kSaSlot + lane * 16;
            i32x4 Al[2], Ah[2], B[2][2];
            Al[0] = *reinterpret_cast<const i32x4 *>(sl);
            Ah[0] = *reinterpret_cast<const i32x4 *>(sl + 1024);
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) B[0][rt] = onehot(rt, s * kSaPairs);
#pragma unroll
            for (int p = 0; p < kSaPairs; ++p) {
                const int c = p & 1;
                if (p + 1 < kSaPairs) {
                    Al[c ^ 1] = *reinterpret_cast<const i32x4 *>(sl + (p + 1) * 2048);
                    Ah[c ^ 1] = *reinterpret_cast<const i32x4 *>(sl + (p + 1) * 2048 + 1024);
#pragma unroll
                    for (int rt = 0; rt < 2; ++rt) B[c ^ 1][rt] = onehot(rt, s * kSaPairs + p + 1);
                }
                __builtin_amdgcn_sched_barrier(0);  // the next pair's reads go out before these MFMAs
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
                    accl[rt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(Al[c], B[c][rt], accl[rt], 0, 0, 0);
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
                    acch[rt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(Ah[c], B[c][rt], acch[rt], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // the group's terms float32(S) * (norm * step), folded in group order
        float nrm[2];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) nrm[rt] = __half2float(__ushort_as_half(nrm16[rt]));
#pragma unroll
        for (int i = 0; i < 16; ++i)
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                const int sum = accl[rt][i] + 64 * acch[rt][i];
                const float coef = nrm[rt] * st[i];
                const float t = static_cast<float>(sum) * coef;
                y[rt][i] = y[rt][i] + t;
            }
    }
    // y to lane = row through LDS (the ring, read out by every wavefront)
    __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
    float *tr = reinterpret_cast<float *>(ring) + w * 32 * 64;  // [activation][row]
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int tt = (i >> 2) * 8 + half * 4 + (i & 3);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) tr[tt * 64 + rt * 32 + l32] = y[rt][i];
    }
    if (!mine) return;  // after the last barrier
    const Epilogue E(J);
    const int rview = min(max((E.blk0 + blk) * 64 + lane - E.row0, 0), E.out - 1);  // the lane's view row, clamped
#pragma unroll 1
    for (int j = 0; j < 4; ++j) {
        constexpr int FA = 8;
        const int t0 = at * 32 + j * FA, nt = min(FA, J.rows - t0);
        if (nt <= 0) break;
        float yy[FA], rv[FA], cv[FA], sv[FA];
        int pk[FA];
#pragma unroll
        for (int q = 0; q < FA; ++q) {
            yy[q] = tr[(j * FA + q) * 64 + lane];
            const long long tk = min(t0 + q, J.rows - 1);
            pk[q] = E.app_q ? E.app_pos[tk] : -1;
            rv[q] = E.resid ? E.resid[tk * E.resid_stride + rview] : 0.0f;
            cv[q] = sv[q] = 0.0f;
            if (E.app_cos) {
                const int pc = pk[q] >= 0 && pk[q] < E.app_cap ? pk[q] : 0;
                cv[q] = E.app_cos[pc * 32 + (lane & 31)];
                sv[q] = E.app_sin[pc * 32 + (lane & 31)];
            }
        }
        fold_epilogue<FA>(E, t0, nt, blk, lane, yy, pk, cv, sv, rv);
    }
}

template <int BITS>
size_t tab_lds_bytes(int groups) {
    return sizeof(float) * static_cast<size_t>(groups) * 32 * 64 + 16 * 16;
}

template <int BITS>
hipError_t launch_tab_t(const TabArgs &t, const LutLaunch &a, int blocks, hipStream_t s, bool pre) {
    hipError_t e;
    if (pre) {
        if (t.rows <= kTabPre4Rows)
            hipLaunchKernelGGL((lut_tables_kernel<BITS, 4>), dim3(t.tiles * 32 / 4, t.groups), dim3(256), 0, s, t);
        else
            hipLaunchKernelGGL((lut_tables_kernel<BITS, 8>), dim3(t.tiles * 32 / 8, t.groups), dim3(256), 0, s, t);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    const dim3 grid(8 * ((a.tab_at * blocks + 7) / 8));  // blocks: slabs of a.tab_rb row blocks
    static std::atomic<unsigned long long> attr[2] = {{0}, {0}};
    if (a.tab_rb == kSaBlocks) {
        e = lds_limit_once(reinterpret_cast<const void *>(&lut_mfma_tabs_kernel<BITS>),
                           static_cast<int>(sa_lds_bytes<BITS>()), attr[1]);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((lut_mfma_tabs_kernel<BITS>), grid, dim3(64 * kSaBlocks), sa_lds_bytes<BITS>(), s, a);
    } else {
        e = lds_limit_once(reinterpret_cast<const void *>(&lut_mfma_tab_kernel<BITS>),
                           static_cast<int>(tab_lds_bytes<BITS>(kTabMaxGroups)), attr[0]);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((lut_mfma_tab_kernel<BITS>), grid, dim3(64 * kTabWaves), tab_lds_bytes<BITS>(t.groups), s,
                           a);
    }
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

size_t tab_table_bytes(int bits, int groups, int tiles) {
    const int np = bits == 4 ? MfmaGeo<4>::NJ / 2 : MfmaGeo<2>::NJ / 2;
    return static_cast<size_t>(tiles) * groups * np * 2048;
}

size_t tab_step_bytes(int groups, int tiles) { return static_cast<size_t>(tiles) * groups * 32 * sizeof(float); }

int tab_max_groups() { return kTabMaxGroups; }

hipError_t launch_lut_tab(const TabArgs &t, const LutLaunch &a, int bits, int blocks, hipStream_t s, bool pre) {
    if (blocks <= 0 || a.tab_at <= 0 || a.njobs <= 0) return hipSuccess;
    if (t.groups > kTabMaxGroups || t.tiles != a.tab_at || a.tab_nb != blocks) return hipErrorInvalidValue;
    if (a.tab_rb != 1 && a.tab_rb != kSaBlocks) return hipErrorInvalidValue;
    if (bits == 4) return launch_tab_t<4>(t, a, blocks, s, pre);
    if (bits == 2) return launch_tab_t<2>(t, a, blocks, s, pre);
    return hipErrorInvalidValue;
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
