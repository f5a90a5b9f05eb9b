// Internal interfaces between the C-ABI host code (cq_api.cpp) and the
// gfx950 kernels (cq_kernels.hip, int8_kernels.hip).
//
// Device layout of a CQ matrix (built once at construction, never changed):
//   rows are padded to blocks of 64 (one wavefront, one row per lane);
//   index: per block, per unit of U = min(16, groupBytes) bytes, the 64 rows'
//          units side by side: idx[((blk * units + u) * 64 + lane) * U + k]
//          is index byte u*U + k of row blk*64 + lane, the packed LSB-first
//          bytes of cact.Packed.Index unchanged (internal/cact/packed.go:24-27);
//          a wavefront's load of one unit is 64*U contiguous bytes;
//   norms: FP16 as stored, norm[(blk * groups + g) * 64 + lane].
// Padding rows hold zero bytes and zero norms and are never written out.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace cqhip {

// A kernel's dynamic-LDS limit, set once per device (the attribute belongs to
// the function on the current device; `done` holds one bit per device
// ordinal below 64, higher ordinals set it on every launch). Concurrent
// first launches both set it: the write is idempotent.
inline hipError_t lds_limit_once(const void *fn, int bytes, std::atomic<unsigned long long> &done) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const unsigned long long bit = dev >= 0 && dev < 64 ? 1ULL << dev : 0;
    if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_release);
    return e;
}

constexpr int kBlockRows = 64;   // rows per block: one per lane of a wavefront
constexpr int kThreads = 256;    // threads per workgroup: four wavefronts
constexpr int kLutQ = 8191;      // internal/cq/lut.go:33
constexpr int kLutMaxGroupBytes = 256;  // internal/cq/lut.go:38
constexpr int kMaxMatrices = 8;  // matrices per shared-table launch

enum Mode { kModeLut = 0, kModeExact = 1 };

// One matrix (or Rows view) of a product launch.
struct MatDesc {
    const uint8_t *idx;    // device layout above
    const uint16_t *norm;  // device layout above
    float *y;              // output rows of this matrix, y_stride floats apart
    long long y_stride;
    int row0, out;         // view: root rows [row0, row0 + out)
    int blk0;              // row0 / 64
    int tile0;             // first tile of this matrix in the launch's tile list
};

struct ProdArgs {
    MatDesc mats[kMaxMatrices];
    int nmats;
    int tiles;             // total tiles over all matrices
    const float *x;        // activations, x_stride floats apart
    long long x_stride;
    int in, groups, row_bytes;
    int tb;                // 64-row blocks per tile
    int gc;                // groups per LDS chunk
    int rows;              // activations
    int nib4_rows;         // Exact: activations [0, nib4_rows) use nibble4's order
    float cb[16];
    float cb_max, lut_step, inv_sqrt;
};

// Launches the product (one matrix or several sharing their tables).
// bits, group_bytes select the template; mode is kModeLut or kModeExact.
hipError_t launch_product(const ProdArgs &a, int bits, int group_bytes, int mode, size_t lds_bytes,
                          hipStream_t stream);
// LDS bytes per group of a chunk, and the fixed part, for choosing gc.
size_t product_lds_bytes(int bits, int group_bytes, int mode, int gc, int tb);

// ---- the lut kernel (lut_kernels.hip) ----

// One product job: a matrix view, its activations and its output.
struct JobDesc {
    const uint8_t *idx;
    const uint16_t *norm;
    const float *x;        // activations, x_stride floats apart
    float *y;              // outputs, y_stride floats apart
    long long x_stride, y_stride;
    int row0, out;         // view: root rows [row0, row0 + out)
    int blk0, nblk;        // first 64-row block of the view and the blocks covering it
    int in, groups, units; // geometry; units = row bytes / unit bytes
    int rows;              // activations
    float cb[16];
    float cb_max, lut_step;
    // Fused prologue and epilogue (null / 0: none). ngain: each activation
    // row is first ZCRMSNorm'ed with this gain (length in). resid: y = resid
    // + product, resid rows resid_stride floats apart (may be y itself).
    // act 1: y = silu(product). xgate: the product is of x * sigmoid(xgate)
    // elementwise (the gated attention output; rows x_stride apart, as x).
    const float *ngain;
    const float *resid;
    long long resid_stride;
    int act;
    const float *xgate;
    // Fused int8 append (app_q null: none; the view's rows and width are
    // whole 64-row blocks): activation b's output row, each 64-wide block
    // a head, is quantized into row app_pos[b] of stream b's cache
    // (codes app_q + b*app_q_stride + p*out, scales app_s + b*app_s_stride
    // + p*(out/64)) unless that position is outside [0, app_cap); with
    // app_cos, each head is first rotated by RoPE at that position.
    int8_t *app_q;
    float *app_s;
    long long app_q_stride, app_s_stride;
    const int32_t *app_pos;
    const float *app_cos, *app_sin;
    int app_cap;
};

// A workgroup's share of a job: blocks [blk, blk + nb) (counted from the
// job's blk0) for activations [act, act + nact).
struct WorkUnit {
    int job, blk, nb, act;
};

constexpr int kKernargJobs = 8;
constexpr int kLutWaves = 4;  // wavefronts per workgroup of the lut kernel

// The next product's tables, built in a producer's epilogue (the table
// form's pre-pass, fused): when a workgroup holds all of its activation's
// output row y, it writes the tables and steps of ZCRMSNorm(y; ngain)
// (ngain null: y itself) for a product over `in` = the producer's out
// inputs, as TabArgs describes them (tab, stp for `tiles` tiles of 32
// activations; slots past the activations are not written).
struct TabOut {
    int8_t *tab;  // null: none
    float *stp;
    const float *ngain;
    int in, groups, bits, tiles;
    float cb[16];
    float cb_max, lut_step;
};

struct LutLaunch {
    JobDesc jobs[kKernargJobs];  // kernel-argument jobs (when dunits is null)
    int njobs;
    int bpw;                     // kernel-argument path: blocks per workgroup
    int wg0[kKernargJobs];       // kernel-argument path: first workgroup of each job
    const JobDesc *djobs;        // device path: job table
    const WorkUnit *dunits;      //              one unit per workgroup
    int tb;                      // blocks of the lut kernel's term buffer: at least a workgroup's blocks
                                 // when its wavefronts share blocks
    int gc;                      // groups per LDS chunk
    int bpw_max;                 // LDS sizing: most blocks of any workgroup
    int waves;                   // kernel-argument path: wavefronts per workgroup (> kLutWaves: the wide form)
    int vsplit;                  // wide form: wavefronts per group (1 or 2)
    // The MFMA form split over groups: job k's float terms [group][activation]
    // [64 * nblk rows] in the workspace; the tiles (256-row groups over the
    // jobs, wg0, times split_at activation tiles) and one counter per tile,
    // zero between launches.
    float *term[kKernargJobs];
    int fold0[kKernargJobs];  // the job's first 256-row group in the fold's grid
    int split_tiles, split_at;
    // The table form: the activations' table planes and steps as
    // lut_tables_kernel wrote them, for tab_at tiles of 32 activations over
    // tab_nb 64-row blocks (all jobs).
    const int8_t *tab;
    const float *tstp;
    int tab_at, tab_nb;
    int tab_rb;  // row blocks per workgroup of the product: 1, or 4 sharing the A operands (tab_nb, wg0 count slabs)
    // The lut kernel's wide form, one workgroup per activation over all of
    // one job's rows: the next product's tables (tout.tab null: none).
    TabOut tout;
};

// The table pre-pass of the table form (mfma_kernels.hip): per activation
// and group, the prologue (gate, ZCRMSNorm), the rotation, the bound and the
// int8 planes of the 16-entry tables, written for tiles of 32 activations
// [tile][group][position pair][plane][half][32][16 codes] (a wavefront's
// MFMA A operand of one plane and pair is 1 KiB contiguous), and the
// groups' steps [tile][group][32]. Activations past rows get zero tables.
struct TabArgs {
    const float *x;
    long long x_stride;
    const float *xgate;  // product of x * sigmoid(xgate) (null: none)
    const float *ngain;  // ZCRMSNorm gain (null: none)
    int rows, in, groups, tiles;
    float cb[16];
    float cb_max, lut_step;
    int8_t *tab;
    float *stp;
};
// Bytes of the tables and of the steps for `tiles` tiles of 32 activations.
size_t tab_table_bytes(int bits, int groups, int tiles);
size_t tab_step_bytes(int groups, int tiles);
// Groups the product kernel's LDS holds terms for.
int tab_max_groups();
// The pre-pass, then the product: grid over the jobs' 64-row blocks (wg0)
// times a.tab_at activation tiles. On stream s.
// pre false: the tables are already there (a producer built them), only the
// product runs.
hipError_t launch_lut_tab(const TabArgs &t, const LutLaunch &a, int bits, int blocks, hipStream_t s, bool pre = true);

size_t lut_lds_bytes(int bits, int group_bytes, int gc, int tb, int bpw);
// LDS bytes the wide form adds for a TabOut over `in` inputs.
size_t lut_tout_lds_bytes(int in);
// grid_y = activations on the kernel-argument path, 1 on the device path.
hipError_t launch_lut(const LutLaunch &a, int bits, int group_bytes, int waves, int grid_x, int grid_y, size_t lds,
                      hipStream_t stream);
bool lut_geometry_supported(int bits, int group_bytes);

// MFMA form of the lut product for many activations (mfma_kernels.hip):
// one launch for up to kKernargJobs views of one geometry; grid x covers
// the jobs' 512-row tiles (wg0), grid y the tiles of ta activations (64 or
// 32).
bool mfma_geometry_supported(int bits, int group);
int mfma_rows_per_workgroup();
hipError_t launch_lut_mfma(const LutLaunch &a, int bits, int ta, int wg, int act_tiles, hipStream_t s);
// The MFMA form split over groups (mfma_kernels.hip), for products whose
// 512-row workgroups would leave most CUs idle: a workgroup per (tile,
// group), a tile being 256 rows (wg0 counts the jobs' row groups) by 32
// activations; each writes its group's float terms to a.term. Then the
// fold, grid x over the jobs' 256-row groups (fold0), y over the activations
// in fours, adds them in group order and applies the epilogue. On stream s.
int mfma_split_rows_per_workgroup();
int mfma_split_activations();
hipError_t launch_lut_mfma_split(const LutLaunch &a, int bits, int fold_blocks, hipStream_t s);

// Dense fp32 MFMA form of Exact's product (dense_kernels.hip), groups of 32
// to 1024. The rotation writes xh [rows_pad][kpad], each activation rotated
// as Exact rotates it (zero rows past rows, zero columns past groups * G).
struct DenseRotArgs {
    const float *x;
    long long x_stride;
    float *xh;
    int rows, rows_pad, in, G, groups, kpad;
    float inv_sqrt;
};
// The product of one view: tiles of dense_tile_rows() weight rows (from
// block blk0, nblk blocks) by dense_tile_activations() activations, K in
// ksplit runs of kchunks chunks of 64 coordinates (more than one: partial
// sums in part [ksplit][rows][out], then the fold into y).
struct DenseArgs {
    const uint8_t *idx;
    const uint16_t *norm;
    const float *xh;
    float *y;
    float *part;
    long long y_stride;
    int row0, out, blk0, nblk;
    int rows, kpad, kin, groups, G, units, U;
    int tiles_m, tiles_n, ksplit, kchunks;
    float cb[16];
};
bool dense_geometry_supported(int bits, int group);
int dense_tile_rows();
int dense_tile_activations();
hipError_t launch_dense_rotate(const DenseRotArgs &r, hipStream_t s);
hipError_t launch_dense(const DenseArgs &a, int bits, hipStream_t s);

struct RowArgs {
    const uint8_t *idx;
    const uint16_t *norm;
    float *dst;            // n rows of `in` floats
    const int32_t *rows;   // device row list (root rows), or nullptr: rows r0 .. r0+n-1
    int r0, n;
    int nrows;             // root rows: listed rows outside [0, nrows) give zeros
    int in, group, groups, row_bytes, width, units, unit_bytes;
    float cb[16];
    float inv_sqrt;
    float scale;           // dst = scale * Row (1 for Row itself)
};
hipError_t launch_rows(const RowArgs &a, hipStream_t stream);

// int8 numerics
hipError_t launch_fake_quant(float *dst, const float *x, long long chunks, int width, hipStream_t stream);
// Stream b of dst (cap rows of row_bytes each) <- rows [0, len[b]) of
// stream idx[b] of src (idx null: stream b); idx, len device int32 arrays.
hipError_t launch_gather_rows(void *dst, const void *src, const int32_t *idx, const int32_t *len, int streams,
                              int cap, int row_bytes, hipStream_t stream);
hipError_t launch_quantize_rows(int8_t *q, float *s, const float *x, long long chunks, int width,
                                hipStream_t stream);

struct AttendArgs {
    float *out; long long out_stride;
    const float *q; long long q_stride;
    int t, heads;
    const int8_t *kq; const float *ks; int k_cols, qk;
    const int8_t *vq; const float *vs; int v_cols, vd;
    long long kv_stride, s_stride;
    const int32_t *spans;
    int nk_max;            // key rows each stream's arrays hold; spans must lie in [0, nk_max)
    int vchunk;            // value rows per LDS chunk (general kernel)
    int resident;          // 1: few workgroups, keep every value row of a stream in LDS
    float scale;
    int quant_q;
    int batch;
    // RoPE of the query heads before they are quantised (null: none): row
    // qpos[b * t + i] of the tables, pairs (j, j + qk/2).
    const float *rope_cos, *rope_sin;
    const int32_t *qpos;
    // Shared caches (null: stream b reads cache b): stream b reads the keys
    // and values of cache kv_index[b], one of kv_streams caches kv_stride /
    // s_stride apart; an index outside [0, kv_streams) leaves its output
    // untouched.
    const int32_t *kv_index;
    int kv_streams;
    // Paged caches (null: none; kv_stride and s_stride are then 0): key j of
    // stream b is row pages[b * page_stride + (j >> page_shift)] *
    // 2^page_shift + (j & (2^page_shift - 1)) of the arrays, which are one
    // pool of pool_pages pages shared by every stream (a forked stream reads
    // its parent's full pages through its own table). An entry outside the
    // pool reads page 0.
    const int32_t *pages;
    int page_stride, page_shift, pool_pages;
    int page_lds;  // set by the launcher: the byte offset of the LDS copy of the page table
};
hipError_t launch_attend_int8(const AttendArgs &a, hipStream_t stream);
constexpr int kAttendMaxPages = 1024;  // a paged launch's pages per stream

// The cache stream a workgroup of stream b reads (kv_index, or b itself),
// or -1 when the index is outside the caches.
__device__ __forceinline__ long long attend_cache_of(const AttendArgs &a, int b) {
    if (!a.kv_index) return b;
    const int c = a.kv_index[b];
    return (c >= 0 && c < a.kv_streams) ? c : -1;
}

// A paged launch copies stream b's page table into LDS at page_lds (its
// entries outside the pool read page 0) before any key is read: key rows are
// then addressed without a global load each, which would also hold up the
// kernels' counted waits on their streamed rows. Every thread of the
// workgroup calls it.
__device__ __forceinline__ void attend_stage_pages(const AttendArgs &a, int b, unsigned char *smem) {
    if (!a.pages) return;
    int32_t *pw = reinterpret_cast<int32_t *>(smem + a.page_lds);
    const int np = (a.nk_max + (1 << a.page_shift) - 1) >> a.page_shift;
    for (int i = threadIdx.x; i < np; i += blockDim.x) {
        const int pg = a.pages[static_cast<long long>(b) * a.page_stride + i];
        pw[i] = (pg >= 0 && pg < a.pool_pages) ? pg : 0;
    }
    __syncthreads();
}

// The array row that holds key `key` of the workgroup's stream: through its
// page table in LDS, or row `key` of the stream's own cache.
__device__ __forceinline__ long long attend_row(const AttendArgs &a, const int32_t *pgs, int key) {
    if (!a.pages) return key;
    return (static_cast<long long>(pgs[key >> a.page_shift]) << a.page_shift) + (key & ((1 << a.page_shift) - 1));
}

// HadamardMLP, Whistle's Monarch FFN (hadamard_kernels.hip): rows of dim
// values in x and out, n = na * nb >= dim, factors row-major (na x na,
// nb x nb), cond_v dim x rank, cond_u rank x n, permutations p1, p2 of n.
struct HadaArgs {
    float *out;
    const float *x;
    int dim, na, nb, rank;
    const float *d1, *d2, *b2, *d3, *d4;
    const float *w1a, *w1b, *w2a, *w2b, *w3a, *w3b;
    const float *cond_v, *cond_u;
    const int32_t *p1, *p2;
};
hipError_t launch_hadamard_mlp(const HadaArgs &h, int rows, hipStream_t s);
bool hadamard_shape_ok(int na, int nb, int dim, int rank);

// Manifold hyper-connections around a block (mhc_kernels.hip): streams of
// rows x lanes x dim, heads rows x lanes (h_res rows x lanes x lanes),
// u / block_out rows x dim.
struct MhcArgs {
    float *h_pre, *h_post, *h_res, *u, *out;
    const float *pre_logits, *post_logits, *res_logits, *stream, *block_out, *affine;
    int lanes, dim;
    int logit_stride;  // floats from one row's logits to the next: 0 for the three separate arrays (lanes, lanes, lanes^2)
};
bool mhc_shape_ok(int lanes, int dim);
hipError_t launch_rms_unit(float *dst, const float *x, int rows, int dim, hipStream_t s);
hipError_t launch_mhc_heads(const MhcArgs &m, int rows, hipStream_t s);
hipError_t launch_mhc_mix(const MhcArgs &m, int rows, hipStream_t s);

// decode-step float blocks (step_kernels.hip)
hipError_t launch_zc_rmsnorm(float *dst, const float *x, const float *gain, int rows, int dim, hipStream_t s);
hipError_t launch_rope(float *x, int rows, int heads, int head_dim, const float *cos_t, const float *sin_t,
                       int positions, const int32_t *pos, int rows_per_pos, hipStream_t s);
hipError_t launch_argmax(int32_t *out, const float *v, int rows, int n, int32_t *pos, int32_t *span_hi,
                         int span_stride, int32_t *done, int eos, hipStream_t s);
hipError_t launch_silu(float *x, long long n, hipStream_t s);
hipError_t launch_add(float *x, const float *y, long long n, hipStream_t s);
hipError_t launch_sigmoid_gate(float *out, float *gate, long long n, hipStream_t s);
hipError_t launch_append(int8_t *q, float *sc, const float *x, int batch, int cols, int width, long long q_stride,
                         long long s_stride, const int32_t *pos, int cap, const float *cos_t, const float *sin_t,
                         hipStream_t s);

// The decode step's features around the products (layer_kernels.hip).
// qkv_prep: for each stream b, the q, k, v rows of one token (dim values,
// heads of 64) at position pos[b]: the causal taps (taps_w [3][taps][dim]
// over hist [batch][taps][3][dim], the raw rows by position mod taps),
// the per-head ZCRMSNorm of q and k (gains qg, kg of 64; null: none), RoPE
// of k at pos[b] (tables of 32 per row, `positions` rows; null: none), and
// the int8 appends of k and v at row pos[b] (< cap) of each stream's pages
// (pages[b * page_stride + pos >> page_shift], pages of 2^page_shift rows of
// dim codes and dim/64 scales; an entry outside [0, pool_pages) skips the
// append). q is written back in place.
struct PrepArgs {
    float *q;
    const float *k, *v;
    float *hist;
    const float *taps_w;
    int taps;
    const float *qg, *kg;
    const float *cos_t, *sin_t;
    int positions;
    const int32_t *pos;
    int cap;
    int8_t *kq, *vq;
    float *ks, *vs;
    const int32_t *pages;
    int page_stride, page_shift, pool_pages;
    int dim;
};
hipError_t launch_qkv_prep(const PrepArgs &a, int batch, hipStream_t s);
// Row kernels of 256 threads (dim a multiple of 256, at most 4096): h =
// resid + float32(sc * ZCRMSNorm(y)); RMSUnit, with quant then fakeQuant of
// the whole row.
bool row_kernel_dim(int dim);
hipError_t launch_norm_scaled_add(float *h, const float *resid, const float *y, const float *gain, float sc, int rows,
                                  int dim, hipStream_t s);
hipError_t launch_rms_unit_row(float *dst, const float *x, int rows, int dim, int quant, hipStream_t s);
hipError_t launch_expand_lanes(float *stream, const float *x, int rows, int lanes, int dim, hipStream_t s);
hipError_t launch_collapse_lanes(float *x, const float *stream, int rows, int lanes, int dim, hipStream_t s);
hipError_t launch_page_copy(int8_t *q, float *sc, const int32_t *src, const int32_t *dst, int n, int page_rows,
                            int cols, int heads, int pool_pages, hipStream_t s);
hipError_t launch_gather_float_rows(float *dst, const float *src, const int32_t *idx, int rows, long long width,
                                    hipStream_t s);

}  // namespace cqhip
